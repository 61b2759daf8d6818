"""The allocation-free attention entry point (noise_attention_noalloc: moment partials in the library's own device
array) against noise_attention with a caller workspace, through the C ABI: two calls in a row, the second smaller,
each equal bit for bit in y, the c_proj partials and the moments (the same kernels; every partial is written before
it is read, so the array's leftovers from the first call cannot leak into the second)."""
import pytest
import torch

from noise_amd import _lib
from tests._util import log_case

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def _inputs(P, T, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q, k, v = (torch.randn(P, T, 8, 64, device=DEV, generator=g) for _ in range(3))
    q, k = (t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + 2 ** -23) for t in (q, k))
    qkv = torch.cat([t.half().reshape(P * T, 512).view(torch.bfloat16) for t in (q, k, v)], 1).contiguous()
    bp = torch.randn(P, 512, device=DEV, generator=g)
    return qkv, bp


def _run(entry, qkv, bp, P, T, window):
    y = torch.full((P * T, 512), float('nan'), device=DEV, dtype=torch.bfloat16)
    up = torch.full((P * T, 8), float('nan'), device=DEV)
    mom = torch.full((P, 8, 2, 64), float('nan'), device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    if entry == 'noalloc':
        _lib.call('noise_attention_noalloc', qkv.data_ptr(), P, T, window, 1, 1, bp.data_ptr(), 0, y.data_ptr(),
                  up.data_ptr(), mom.data_ptr(), s)
    else:
        ws = torch.empty(_lib.size_query('noise_attention_workspace_size', P, T), device=DEV, dtype=torch.uint8)
        _lib.call('noise_attention', qkv.data_ptr(), P, T, window, 1, 1, bp.data_ptr(), 0, y.data_ptr(), up.data_ptr(),
                  mom.data_ptr(), ws.data_ptr(), ws.numel(), s)
    torch.cuda.synchronize()
    return y.cpu(), up.cpu(), mom.cpu()


def test_attention_noalloc_equals_workspace_entry_on_two_calls():
    # the largest problem the array holds (256 members at 2048 tokens = 4 Mi partials), then a smaller one
    for P, T, window, seed in ((256, 2048, 1024, 1), (6, 384, 2048, 2)):
        log_case(f'attention_noalloc P={P} T={T} window={window}')
        qkv, bp = _inputs(P, T, seed)
        got = _run('noalloc', qkv, bp, P, T, window)
        ref = _run('workspace', qkv, bp, P, T, window)
        for a, b in zip(got, ref):
            assert torch.isfinite(a.float()).all()
            assert torch.equal(a, b)


def test_attention_noalloc_refuses_sizes_beyond_its_array():
    """257 members at 2048 tokens need more moment partials than the array holds. Every buffer is a real device
    allocation of the full requested size, so even a regressed size guard would only launch in-bounds work."""
    log_case('attention_noalloc size limit')
    P, T = 257, 2048
    qkv = torch.zeros(P * T, 1536, device=DEV, dtype=torch.bfloat16)
    y = torch.empty(P * T, 512, device=DEV, dtype=torch.bfloat16)
    mom = torch.empty(P, 8, 2, 64, device=DEV)
    rc = _lib.load().noise_attention_noalloc(qkv.data_ptr(), P, T, 2048, 1, 1, None, 0, y.data_ptr(), None,
                                             mom.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == -2  # NOISE_ENOSPC
