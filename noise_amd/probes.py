"""Readout-probe forward differences on the HIP kernel: drop-ins for `cycle_derivatives` and
`row_derivatives` (train/val/run.py:154-185; train/speedrun/run.py:90-103).

Same arguments and results as the reference's compiled functions: base (n, V) = W x of the clean streams, C (P, V)
with row j = W D_j, y (n,) targets (-1 = none), steps (n, 1) or (n,), sq (n, 1) or (n,) = |x|^2, dots the x . D of
the probed directions, dir_sq their |D|^2; the result is (n, P) or (n, K) fp32. All inputs are CUDA tensors;
width is the stream width the head's RMS is taken over (WIDTH of the reference, 512 at the model's shape).
"""
import torch

from . import _lib


def _f32(t, name, shape=None):
    if t.device.type != 'cuda':
        raise ValueError(f'{name} must be a CUDA tensor (no CPU path)')
    t = t.float().contiguous()
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f'{name} must be {tuple(shape)}, got {tuple(t.shape)}')
    return t


def _run(base, C, rows, y, steps, sq, dots, dir_sq, width, per_token):
    n, V = base.shape
    P = C.shape[0]
    K = rows.shape[1] if rows is not None else P
    base = _f32(base, 'base', (n, V))
    C = _f32(C, 'C', (P, V))
    steps = _f32(steps.reshape(n), 'steps')
    sq = _f32(sq.reshape(n), 'sq')
    dots = _f32(dots, 'dots', (n, K))
    dir_sq = _f32(dir_sq, 'dir_sq', (n, K) if per_token else (P,))
    y = y.to(torch.int64).contiguous()
    if y.shape != (n,) or y.device.type != 'cuda':
        raise ValueError(f'y must be a CUDA tensor of shape ({n},)')
    if rows is not None:
        if tuple(rows.shape) != (n, K) or rows.device.type != 'cuda':
            raise ValueError(f'rows must be a CUDA tensor of shape ({n}, {K})')
        rows = rows.to(torch.int64).contiguous()
    out = torch.empty(n, K, device=base.device, dtype=torch.float32)
    _lib.call('noise_readout_probes', base.data_ptr(), V, C.data_ptr(), V, 0 if rows is None else rows.data_ptr(), K,
              y.data_ptr(), steps.data_ptr(), sq.data_ptr(), dots.data_ptr(), K, dir_sq.data_ptr(), int(per_token),
              n, V, P, width, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return out


def cycle_derivatives(base, C, y, steps, sq, dots, dir_sq, width=512):
    """Forward differences of each token's readout loss along every direction of the cycle: (n, P)
    (train/val/run.py:154-167)."""
    return _run(base, C, None, y, steps, sq, dots, dir_sq, width, False)


def row_derivatives(base, C, rows, y, steps, sq, dots, dir_sq, width=512):
    """Forward differences along each token's own directions rows (n, K): (n, K) (train/val/run.py:169-181)."""
    return _run(base, C, rows, y, steps, sq, dots, dir_sq, width, True)
