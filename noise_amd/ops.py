"""torch-facing wrappers of the C ABI (device memory and streams come from PyTorch-ROCm).

Each op validates shapes and dtypes on the host, allocates its outputs and workspace with torch, and
enqueues the HIP kernels on torch's current stream. Inputs must already be CUDA tensors: there is no
CPU path.
"""
import torch

from . import _lib


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _need(t, dtype, shape=None, name='tensor'):
    if t.device.type != 'cuda':
        raise ValueError(f'{name} must be a CUDA tensor (no CPU path)')
    if t.dtype != dtype:
        raise TypeError(f'{name} must be {dtype}, got {t.dtype}')
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f'{name} must have shape {tuple(shape)}, got {tuple(t.shape)}')
    if not t.is_contiguous():
        raise ValueError(f'{name} must be contiguous')


def _rows(x, members, T):
    """(ld, member stride) of a bf16 activation [members, T, in] or a shared [T, in]."""
    if x.dim() == 2:
        return x.stride(0), 0
    if x.shape[0] != members or x.shape[1] != T:
        raise ValueError(f'activation must be [members={members}, T={T}, in], got {tuple(x.shape)}')
    return x.stride(1), x.stride(0)


def _dirs(a, members, pair_shift):
    need = (members + (1 << pair_shift) - 1) >> pair_shift
    if a.shape[0] < need:
        raise ValueError(f'need {need} perturbation rows, got {a.shape[0]}')


def lowrank_linear(x, weight, a, b, sign, T=None, pair_shift=0, out=None, accumulate=False, out_dtype=torch.float32):
    """x [members, T, in] (or shared [T, in]) bf16 through weight [out, in] bf16 + sign_p a_p b_p^T.

    Returns fp32 (or bf16) [members, T, out]; with accumulate=True adds into `out` (fp32) in place."""
    members = sign.shape[0]
    T = T or x.shape[-2]
    d_out, d_in = weight.shape
    _need(x, torch.bfloat16, name='x')
    _need(weight, torch.bfloat16, name='weight')
    _need(a, torch.float32, name='a')
    _need(b, torch.float32, name='b')
    _need(sign, torch.float32, name='sign')
    if a.shape[1] != d_out or b.shape[1] != d_in or x.shape[-1] != d_in:
        raise ValueError('rank-1 vectors or activation do not match the weight')
    _dirs(a, members, pair_shift)
    _dirs(b, members, pair_shift)
    ld, mstride = _rows(x, members, T)
    if accumulate:
        if out is None or out.dtype != torch.float32:
            raise ValueError('accumulate needs an fp32 out tensor')
        y32, y16 = out, None
    else:
        y = out if out is not None else torch.empty(members, T, d_out, device=x.device, dtype=out_dtype)
        y32, y16 = (y, None) if y.dtype == torch.float32 else (None, y)
        out = y
    ws_bytes = _lib.size_query('noise_lowrank_linear_workspace_size', members, T)
    ws = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    _lib.call('noise_lowrank_linear', _ptr(x), ld, mstride, _ptr(weight), d_in, d_out, _ptr(a), _ptr(b), _ptr(sign),
              members, T, pair_shift, _ptr(y32), _ptr(y16), int(accumulate), _ptr(ws), ws_bytes, _stream())
    return out


def lowrank_mlp(x, w_fc, w_proj, a_fc, b_fc, a_proj, b_proj, sign, T=None, pair_shift=0, out=None,
                accumulate=False, out_dtype=torch.float32, workspace=None):
    """relu^2 MLP with rank-1 perturbations on both matrices (train/val/eggroll.py:93), per member.

    x: bf16 [members, T, d] or shared [T, d]; w_fc [f, d], w_proj [d, f] bf16 (nn.Linear orientation)."""
    members = sign.shape[0]
    T = T or x.shape[-2]
    f, d = w_fc.shape
    for t, n in ((x, 'x'), (w_fc, 'w_fc'), (w_proj, 'w_proj')):
        _need(t, torch.bfloat16, name=n)
    for t, n in ((a_fc, 'a_fc'), (b_fc, 'b_fc'), (a_proj, 'a_proj'), (b_proj, 'b_proj'), (sign, 'sign')):
        _need(t, torch.float32, name=n)
    if tuple(w_proj.shape) != (d, f) or a_fc.shape[1] != f or b_fc.shape[1] != d or a_proj.shape[1] != d \
            or b_proj.shape[1] != f:
        raise ValueError('MLP weights / rank-1 vectors have inconsistent shapes')
    for t in (a_fc, b_fc, a_proj, b_proj):
        _dirs(t, members, pair_shift)
    ld, mstride = _rows(x, members, T)
    if accumulate:
        if out is None or out.dtype != torch.float32:
            raise ValueError('accumulate needs an fp32 out tensor')
        y32, y16 = out, None
    else:
        y = out if out is not None else torch.empty(members, T, d, device=x.device, dtype=out_dtype)
        y32, y16 = (y, None) if y.dtype == torch.float32 else (None, y)
        out = y
    ws_bytes = _lib.size_query('noise_lowrank_mlp_workspace_size', members, T, d, f)
    if workspace is None or workspace.numel() < ws_bytes:
        workspace = torch.empty(ws_bytes, device=x.device, dtype=torch.uint8)
    _lib.call('noise_lowrank_mlp', _ptr(x), ld, mstride, _ptr(w_fc), _ptr(w_proj), d, f, _ptr(a_fc), _ptr(b_fc),
              _ptr(a_proj), _ptr(b_proj), _ptr(sign), members, T, pair_shift, _ptr(y32), _ptr(y16), int(accumulate),
              _ptr(workspace), ws_bytes, _stream())
    return out


def mlp_workspace_bytes(members, T, d=512, f=2048):
    return _lib.size_query('noise_lowrank_mlp_workspace_size', members, T, d, f)
