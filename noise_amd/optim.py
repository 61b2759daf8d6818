"""Adam on the HIP kernel, with torch.optim.AdamW's interface and semantics for weight_decay = 0
(the optimizer EGGROLL uses, train/val/eggroll.py:205)."""
import math

import torch

from . import _lib


class Adam(torch.optim.Optimizer):
    """AdamW(lr, betas, eps, weight_decay=0) whose update runs in libnoise_hip.so (noise_adam).

    State per parameter matches torch.optim.AdamW: 'step', 'exp_avg', 'exp_avg_sq'. `lr` is read from
    the param group at every step, so schedules that rewrite group['lr'] (train/val/eggroll.py:208-212)
    work unchanged."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0):
        if weight_decay != 0.0:
            raise ValueError('only weight_decay = 0 is supported (EGGROLL uses plain Adam)')
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))

    @torch.no_grad()
    def step(self, closure=None):
        """One step of every parameter with a gradient: each param group's tensors in one noise_adam_batch launch."""
        loss = closure() if closure is not None else None
        stream = torch.cuda.current_stream().cuda_stream
        for group in self.param_groups:
            b1, b2 = group['betas']
            items, keep = [], []
            for p in group['params']:
                if p.grad is None:
                    continue
                if p.device.type != 'cuda' or p.dtype != torch.float32 or not p.is_contiguous():
                    raise ValueError('Adam (HIP) needs contiguous fp32 CUDA parameters')
                grad = p.grad.contiguous()
                keep.append(grad)
                st = self.state[p]
                if not st:
                    st['step'] = 0
                    st['exp_avg'] = torch.zeros_like(p)
                    st['exp_avg_sq'] = torch.zeros_like(p)
                st['step'] += 1
                t = st['step']
                items.append((p.data_ptr(), grad.data_ptr(), st['exp_avg'].data_ptr(), st['exp_avg_sq'].data_ptr(),
                              p.numel(), group['lr'] / (1 - b1 ** t), math.sqrt(1 - b2 ** t)))
            if items:
                ptr, count, _arr = _lib.adam_tensors(items)
                _lib.call('noise_adam_batch', ptr, count, b1, b2, group['eps'], stream)
        return loss
