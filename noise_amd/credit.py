"""Credit scoring around batched attention reruns on the HIP kernels: drop-ins for the compiled helpers
`moved_heads`, `head_scores` and `code_estimate` (train/val/run.py:186-211) that `query_key_errors`
(:594-634) composes, and `attention` (utils/model.py:24-31) for the reruns themselves.

Shapes follow the reference: heads of 64 dims, raw [b, t, h, 64], draws a [n, b, t, h, 64] (bf16), attention
tensors [batch, token, head, 64]. Every input is a CUDA tensor; the arithmetic runs in libnoise_hip.so.
"""
import torch

from . import _lib

HD = 64


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _cuda(t, name):
    if t.device.type != 'cuda':
        raise ValueError(f'{name} must be a CUDA tensor (no CPU path)')
    return t


def _tables(t, T):
    """cos / sin as fp32 [T, 32] from the reference's [1, >= T, 1, 32] (or [>= T, 32]) tables."""
    if t.shape[-1] != 32 or t.numel() // 32 < T:
        raise ValueError(f'rotary tables must hold at least {T} rows of 32 (got shape {tuple(t.shape)})')
    _cuda(t, 'rotary table')
    t = t.reshape(-1, 32)[:T]
    return t.float().contiguous()


def moved_heads(raw, a, sigma, cos, sin):
    """norm(rotary(raw + sigma a)) per draw, flattened over (draw, batch): [n * b, t, h, 64] in a's dtype
    (bf16) (train/val/run.py:186-189)."""
    _cuda(raw, 'raw'), _cuda(a, 'a')
    n, b, T, H, hd = a.shape
    if hd != HD or tuple(raw.shape) != (b, T, H, HD):
        raise ValueError(f'raw must be [{b}, {T}, {H}, {HD}] and a [n, b, t, h, {HD}]')
    if a.dtype != torch.bfloat16:
        raise TypeError('a must be bfloat16 (the draws are stored in the model dtype)')
    cos, sin = _tables(cos, T), _tables(sin, T)
    raw = raw.float().contiguous()
    a = a.contiguous()
    out = torch.empty(n * b, T, H, HD, device=a.device, dtype=torch.bfloat16)
    _lib.call('noise_moved_heads', raw.data_ptr(), a.data_ptr(), float(sigma), cos.data_ptr(), sin.data_ptr(), n, b,
              T, H, out.data_ptr(), H * HD, _stream())
    return out


def head_scores(out, baseline, hub):
    """score[b, h, t, j] = sum_d (out[j, b, t, h, d] - baseline[b, t, h, d]) hub[b, t, h, d]: [b, h, t, n] fp32
    (train/val/run.py:192-195). out [n, b, t, h, 64] bf16."""
    _cuda(out, 'out')
    n, b, T, H, hd = out.shape
    if hd != HD or tuple(baseline.shape) != (b, T, H, HD) or tuple(hub.shape) != (b, T, H, HD):
        raise ValueError('baseline and hub must be [b, t, h, 64] like one draw of out')
    if out.dtype != torch.bfloat16:
        raise TypeError('out must be bfloat16 (the attention output of the reruns)')
    out = out.contiguous()
    base, hub = baseline.float().contiguous(), hub.float().contiguous()
    score = torch.empty(b, H, T, n, device=out.device, dtype=torch.float32)
    _lib.call('noise_head_scores', out.data_ptr(), H * HD, base.data_ptr(), hub.data_ptr(), n, b, T, H,
              score.data_ptr(), _stream())
    return score


def code_estimate(credited, a):
    """est[b, t, h, d] = sum_j credited[b, h, t, j] a[j, b, t, h, d]: [b, t, h, 64] fp32
    (train/val/run.py:208-210)."""
    _cuda(credited, 'credited'), _cuda(a, 'a')
    n, b, T, H, hd = a.shape
    if hd != HD or tuple(credited.shape) != (b, H, T, n):
        raise ValueError(f'credited must be [{b}, {H}, {T}, {n}] for a of shape {tuple(a.shape)}')
    if a.dtype != torch.bfloat16:
        raise TypeError('a must be bfloat16')
    cr, a = credited.float().contiguous(), a.contiguous()
    est = torch.empty(b, T, H, HD, device=a.device, dtype=torch.float32)
    _lib.call('noise_code_estimate', cr.data_ptr(), a.data_ptr(), n, b, T, H, est.data_ptr(), _stream())
    return est


def key_scores(filt, score):
    """The key scores of `query_key_errors` (train/val/run.py:622-623): (K.to(bf16) @ score.to(bf16)).float() per
    (b, h), K [b, h, t, t] (the matched filter), score [b, h, t, n] -> [b, h, t, n] fp32 holding bf16 values."""
    _cuda(filt, 'key filter'), _cuda(score, 'score')
    b, H, T, n = score.shape
    if tuple(filt.shape) != (b, H, T, T):
        raise ValueError(f'the key filter must be [{b}, {H}, {T}, {T}] for scores of shape {tuple(score.shape)}')
    if T % 64:
        raise ValueError(f'the key filter kernel runs whole 64-token blocks: t = {T} is not a multiple of 64')
    filt = filt.to(torch.bfloat16).contiguous()
    score = score.float().contiguous()
    out = torch.empty(b, H, T, n, device=score.device, dtype=torch.float32)
    _lib.call('noise_key_filter', filt.data_ptr(), score.data_ptr(), b, H, T, n, out.data_ptr(), _stream())
    return out


def attention(q, k, v, window, qk_norm=False):
    """Causal attention with a left window on [batch, token, head, 64] tensors (utils/model.py:24-31) on the
    attention kernel: q and k bf16, v the bf16-rounded value in fp16 (the kernel's operand format), P in fp16,
    bf16 output. 8 heads; token count a multiple of 128. qk_norm declares RMS-normalised q, k rows (the
    credit reruns' processed heads), which lets the softmax skip its running maximum. fp16 holds every bf16
    value of magnitude 2^-14 .. 65504 exactly; smaller ones lose low bits (absolute error < 2^-25) and larger
    ones overflow, far outside the activations of this model."""
    B, T, H, hd = q.shape
    if hd != HD or H != 8 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError('q, k, v must be [batch, token, 8, 64] of one shape')
    if T % 128:
        raise ValueError(f'the attention kernel runs whole 128-token blocks: token count {T} is not a multiple of 128')
    for t, nm in ((q, 'q'), (k, 'k'), (v, 'v')):
        _cuda(t, nm)
    qkv = torch.empty(B * T, 3 * H * HD, device=q.device, dtype=torch.bfloat16)
    qkv[:, :H * HD] = q.reshape(B * T, H * HD).to(torch.bfloat16)
    qkv[:, H * HD:2 * H * HD] = k.reshape(B * T, H * HD).to(torch.bfloat16)
    qkv[:, 2 * H * HD:] = v.reshape(B * T, H * HD).to(torch.bfloat16).half().view(torch.bfloat16)
    y = torch.empty(B * T, H * HD, device=q.device, dtype=torch.bfloat16)
    _lib.call('noise_attention', qkv.data_ptr(), B, T, int(window), int(bool(qk_norm)), _lib.QK_BF16, None, 0,
              y.data_ptr(), None, None, None, 0, _stream())
    return y.view(B, T, H, HD)


def rerun(kind, raw, a, sigma, cos, sin, fixed, values, window):
    """The attention reruns of one chunk of draws in `query_key_errors` (train/val/run.py:618-622): the moved
    heads of `kind` ('q' or 'k') are written straight into their slot of the q | k | v rows the attention kernel
    reads, beside the other processed head `fixed` and `values` (both [b, t, h, 64], shared by every draw).
    Returns the attention output [n, b, t, h, 64] bf16. Both head slots hold RMS-normalised rows, so the kernel
    runs with bounded scores (no running maximum)."""
    if kind not in ('q', 'k'):
        raise ValueError("kind must be 'q' or 'k'")
    n, b, T, H, hd = a.shape
    if hd != HD or H != 8 or tuple(raw.shape) != (b, T, H, HD):
        raise ValueError('a must be [n, b, t, 8, 64] and raw [b, t, 8, 64]')
    if tuple(fixed.shape) != (b, T, H, HD) or tuple(values.shape) != (b, T, H, HD):
        raise ValueError('fixed and values must be [b, t, 8, 64]')
    if T % 128:
        raise ValueError(f'the attention kernel runs whole 128-token blocks: t = {T} is not a multiple of 128')
    if a.dtype != torch.bfloat16:
        raise TypeError('a must be bfloat16')
    if window < 0:
        raise ValueError('window must be >= 0')
    cos, sin = _tables(cos, T), _tables(sin, T)
    _cuda(raw, 'raw'), _cuda(a, 'a'), _cuda(fixed, 'fixed'), _cuda(values, 'values')
    W = H * HD
    moved_slot, fixed_slot = (0, W) if kind == 'q' else (W, 0)
    qkv = torch.empty(n, b * T, 3 * W, device=a.device, dtype=torch.bfloat16)
    qkv[:, :, fixed_slot:fixed_slot + W] = fixed.reshape(1, b * T, W).to(torch.bfloat16)
    qkv[:, :, 2 * W:] = values.reshape(1, b * T, W).to(torch.bfloat16).half().view(torch.bfloat16)
    rawf, a = raw.float().contiguous(), a.contiguous()
    stream = _stream()
    _lib.call('noise_moved_heads', rawf.data_ptr(), a.data_ptr(), float(sigma), cos.data_ptr(), sin.data_ptr(), n, b,
              T, H, qkv.data_ptr() + 2 * moved_slot, 3 * W, stream)
    y = torch.empty(n * b * T, W, device=a.device, dtype=torch.bfloat16)
    _lib.call('noise_attention', qkv.data_ptr(), n * b, T, int(window), 1, _lib.QK_BF16, None, 0, y.data_ptr(), None,
              None, None, 0, stream)
    return y.view(n, b, T, H, HD)


def credit_chunk(kind, raw, a, sigma, cos, sin, fixed, values, window, baseline, target, key_filter=None):
    """One chunk's contribution to the estimate of `query_key_errors` (train/val/run.py:617-625): rerun, score
    each query's output change against its target, for keys carry the scores back through the matched filter
    key_filter [b, h, t, t] (bf16 MFMA product, as the reference's bf16 matmul), then weight the draws:
    [b, t, h, 64] fp32."""
    n, b, T, H, _ = a.shape
    if kind == 'k' and (key_filter is None or tuple(key_filter.shape) != (b, H, T, T)):
        raise ValueError(f'key credit needs the matched filter key_filter [{b}, {H}, {T}, {T}]')
    out = rerun(kind, raw, a, sigma, cos, sin, fixed, values, window)
    score = head_scores(out, baseline, target)
    if kind == 'k':
        score = key_scores(key_filter, score)
    return code_estimate(score, a)
