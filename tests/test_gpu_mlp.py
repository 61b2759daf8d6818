"""GPU parity of the low-rank GEMM paths against the CPU oracle (bf16 rounding-point mode).

Tolerance (north star): <= 1e-2 relative error on bf16 activations. The kernels keep the reference's
autocast rounding points, so the observed error is accumulation-order noise (~1e-3)."""
import pytest
import torch

from oracle import model as om
from tests._util import log_case, rel_err

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def _mlp_inputs(P, T, shared_x, sigma, seed=0, d=512, f=2048):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g) if shared_x else torch.randn(P, T, d, generator=g)
    w1 = (torch.randn(f, d, generator=g) * d ** -0.5).bfloat16()
    w2 = (torch.randn(d, f, generator=g) * f ** -0.5).bfloat16()
    pairs = P // 2
    a1, b1 = torch.randn(pairs, f, generator=g), torch.randn(pairs, d, generator=g)
    a2, b2 = torch.randn(pairs, d, generator=g), torch.randn(pairs, f, generator=g)
    sign = torch.tensor([sigma, -sigma]).repeat(pairs)
    return x.bfloat16(), w1, w2, a1, b1, a2, b2, sign


def _oracle_members(x, w1, w2, a1, b1, a2, b2, sign, members):
    rep = lambda t: t.repeat_interleave(2, 0)[members]  # noqa: E731
    xs = x.float() if x.dim() == 2 else x.float()[members]
    return om.mlp_population(xs, w1.float(), w2.float(), rep(a1), rep(b1), rep(a2), rep(b2), sign[members], 'bf16')


@pytest.mark.parametrize('shared_x,sigma', [(False, 1e-3), (True, 1e-3), (False, 5e-2)])
def test_mlp_small_matches_oracle(shared_x, sigma):
    from noise_amd import ops
    P, T = 4, 256
    log_case(f'mlp small P={P} T={T} shared_x={shared_x} sigma={sigma}')
    args = _mlp_inputs(P, T, shared_x, sigma)
    dev = [t.to(DEV) for t in args]
    y = ops.lowrank_mlp(*dev, T=T, pair_shift=1)
    torch.cuda.synchronize()
    ref = _oracle_members(*args, list(range(P)))
    y = y.cpu()
    assert rel_err(y, ref) < 1e-2
    assert rel_err(y, ref) < 4e-3  # accumulation-order noise only
    # the antithetic difference (the ES signal) survives: compare pair differences
    d_gpu, d_ref = y[0::2] - y[1::2], ref[0::2] - ref[1::2]
    assert rel_err(d_gpu, d_ref) < 5e-2, rel_err(d_gpu, d_ref)


def test_mlp_bf16_output_and_residual_accumulate():
    from noise_amd import ops
    P, T = 2, 128
    log_case(f'mlp bf16 out / accumulate P={P} T={T}')
    args = _mlp_inputs(P, T, False, 1e-2, seed=1)
    dev = [t.to(DEV) for t in args]
    y16 = ops.lowrank_mlp(*dev, T=T, pair_shift=1, out_dtype=torch.bfloat16)
    resid = torch.randn(P, T, 512, generator=torch.Generator().manual_seed(3))
    r = resid.to(DEV)
    ops.lowrank_mlp(*dev, T=T, pair_shift=1, out=r, accumulate=True)
    torch.cuda.synchronize()
    ref = _oracle_members(*args, list(range(P)))
    assert y16.dtype == torch.bfloat16
    assert rel_err(y16.cpu().float(), ref) < 1e-2
    assert rel_err(r.cpu() - resid, ref) < 4e-3


def test_lowrank_linear_matches_oracle():
    from noise_amd import ops
    g = torch.Generator().manual_seed(4)
    P, T, din, dout = 4, 256, 512, 1536
    log_case(f'lowrank_linear P={P} T={T} {din}->{dout}')
    x = torch.randn(P, T, din, generator=g).bfloat16()
    w = (torch.randn(dout, din, generator=g) / 20).bfloat16()
    a, b = torch.randn(P, dout, generator=g), torch.randn(P, din, generator=g)
    sign = torch.tensor([1e-3, -1e-3, 2e-3, -2e-3])
    y = ops.lowrank_linear(x.to(DEV), w.to(DEV), a.to(DEV), b.to(DEV), sign.to(DEV))
    torch.cuda.synchronize()
    ref = om.lowrank(x.float(), w.float(), a, b, sign, 'bf16')
    # same rounding points: the bf16 dense part is exact up to accumulation order
    assert rel_err(y.cpu(), ref) < 1e-3
    assert (y.cpu() - ref).abs().max() < 2e-2


@pytest.mark.parametrize('T', [64, 200])
def test_lowrank_linear_ragged_rows(T):
    """M = members * T not a multiple of the 128-row tile (tail rows clamped / masked)."""
    from noise_amd import ops
    g = torch.Generator().manual_seed(5)
    P, din, dout = 3, 512, 512
    log_case(f'lowrank_linear ragged P={P} T={T}')
    x = torch.randn(P, T, din, generator=g).bfloat16()
    w = (torch.randn(dout, din, generator=g) / 20).bfloat16()
    a, b = torch.randn(P, dout, generator=g), torch.randn(P, din, generator=g)
    sign = torch.tensor([1e-2, -1e-2, 0.0])
    y = ops.lowrank_linear(x.to(DEV), w.to(DEV), a.to(DEV), b.to(DEV), sign.to(DEV))
    torch.cuda.synchronize()
    ref = om.lowrank(x.float(), w.float(), a, b, sign, 'bf16')
    assert rel_err(y.cpu(), ref) < 1e-3


@pytest.mark.parametrize('dout', [384, 640])
def test_lowrank_linear_narrow_tiles(dout):
    """Output widths that are a multiple of 128 but not of 256 run the tile GEMM's 256 x 128 configuration."""
    from noise_amd import ops
    g = torch.Generator().manual_seed(6)
    P, T, din = 4, 128, 512
    log_case(f'lowrank_linear narrow tiles P={P} T={T} {din}->{dout}')
    x = torch.randn(P, T, din, generator=g).bfloat16()
    w = (torch.randn(dout, din, generator=g) / 20).bfloat16()
    a, b = torch.randn(P, dout, generator=g), torch.randn(P, din, generator=g)
    sign = torch.tensor([1e-2, -1e-2, 3e-2, -3e-2])
    y = ops.lowrank_linear(x.to(DEV), w.to(DEV), a.to(DEV), b.to(DEV), sign.to(DEV))
    torch.cuda.synchronize()
    ref = om.lowrank(x.float(), w.float(), a, b, sign, 'bf16')
    assert rel_err(y.cpu(), ref) < 1e-3
    assert (y.cpu() - ref).abs().max() < 2e-2


@pytest.mark.parametrize('dout,din', [(384, 2048), (640, 1024)])
def test_dense_wtile_weight_on_narrow_tiles(dout, din):
    """The dense c_proj product with a WTILE weight on the 256 x 128 tile configuration (output widths a multiple of
    128, not of 256) returns exactly the row-major weight's result, and bf16(x W^T) within one bf16 step."""
    from noise_amd import _lib
    g = torch.Generator().manual_seed(8)
    P, T = 2, 128
    M = P * T
    log_case(f'dense WTILE narrow tiles M={M} {din}->{dout}')
    x = torch.randn(M, din, generator=g).bfloat16()
    w = (torch.randn(dout, din, generator=g) * din ** -0.5).bfloat16()
    xd, wd = x.to(DEV), w.to(DEV)
    wt = torch.empty_like(wd)
    s = torch.cuda.current_stream().cuda_stream
    _lib.call('noise_weight_tiles', wd.data_ptr(), dout, din, wt.data_ptr(), s)
    ys = []
    for layout, ww in ((_lib.LAYOUT_ROWS, wd), (_lib.LAYOUT_WTILE, wt)):
        y = torch.empty(M, dout, device=DEV, dtype=torch.bfloat16)
        _lib.call('noise_dense_bf16', xd.data_ptr(), _lib.LAYOUT_ROWS, din, dout, ww.data_ptr(), layout, P, T,
                  y.data_ptr(), s)
        ys.append(y)
    torch.cuda.synchronize()
    assert torch.equal(ys[1].cpu(), ys[0].cpu())
    ref = (x.float() @ w.float().t()).bfloat16().float()
    assert ((ys[0].cpu().float() - ref).abs() <= ref.abs() * 2 ** -7 + 1e-6).all()


@pytest.mark.parametrize('P', [28, 36, 44])
def test_mlp_block_counts_around_the_steady_loop(P):
    """The c_fc kernel runs an iteration from its steady loop when all earlier stores and later loads are outstanding
    (blocks 3 .. nb - 4 of a workgroup's nb). At T = 256 on a 256-CU part each workgroup gets P / 4 blocks: 7, 9 and
    11 put the first and last steady pairs at different block indices. Sampled members match the oracle at the
    small-case bound."""
    from noise_amd import ops
    T = 256
    log_case(f'mlp steady-loop block counts P={P} T={T}')
    args = _mlp_inputs(P, T, False, 1e-2, seed=9)
    dev = [t.to(DEV) for t in args]
    y = ops.lowrank_mlp(*dev, T=T, pair_shift=1)
    torch.cuda.synchronize()
    members = [0, 1, P // 2, P - 1]
    ref = _oracle_members(*args, members)
    got = y[members].cpu()
    assert rel_err(got, ref) < 4e-3, rel_err(got, ref)


@pytest.mark.parametrize('P', [112, 144, 176])
def test_dense_block_counts_around_the_steady_loop(P):
    """The attention c_proj product (K = N = 512, the weight-resident kernel's dense mode) at 7, 9 and 11 blocks per
    workgroup on a 256-CU part (two 256-column slices, 16 row streams per XCD, T = 256): bf16(x W^T) within one
    bf16 step everywhere."""
    from noise_amd import _lib
    T, D = 256, 512
    M = P * T
    log_case(f'dense steady-loop block counts P={P} T={T}')
    g = torch.Generator().manual_seed(10)
    x = torch.randn(M, D, generator=g).bfloat16()
    w = (torch.randn(D, D, generator=g) * D ** -0.5).bfloat16()
    xd, wd = x.to(DEV), w.to(DEV)  # held: a temporary's memory could be reused before the kernel reads it
    y = torch.empty(M, D, device=DEV, dtype=torch.bfloat16)
    _lib.call('noise_dense_bf16', xd.data_ptr(), _lib.LAYOUT_ROWS, D, D, wd.data_ptr(), _lib.LAYOUT_ROWS, P, T,
              y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = (x.float() @ w.float().t()).bfloat16().float()
    assert ((y.cpu().float() - ref).abs() <= ref.abs() * 2 ** -7 + 1e-6).all()


@pytest.mark.parametrize('din', [128, 192, 256, 320, 1536])
def test_dense_tile_gemm_depths_around_the_steady_loop(din):
    """The tile GEMM's dense product runs k stages 1 .. KT - 4 (KT = din / 32) from its steady loop in pairs: none at
    KT = 4 or 6, one pair at 8, one at 10 (an odd count left for the general loop), 22 at 48. bf16(x W^T) within one
    bf16 step everywhere."""
    from noise_amd import _lib
    P, T, dout = 4, 256, 512
    M = P * T
    log_case(f'dense tile GEMM depth M={M} {din}->{dout}')
    g = torch.Generator().manual_seed(11)
    x = torch.randn(M, din, generator=g).bfloat16()
    w = (torch.randn(dout, din, generator=g) * din ** -0.5).bfloat16()
    xd, wd = x.to(DEV), w.to(DEV)  # held: a temporary's memory could be reused before the kernel reads it
    y = torch.empty(M, dout, device=DEV, dtype=torch.bfloat16)
    _lib.call('noise_dense_bf16', xd.data_ptr(), _lib.LAYOUT_ROWS, din, dout, wd.data_ptr(), _lib.LAYOUT_ROWS, P, T,
              y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = (x.float() @ w.float().t()).bfloat16().float()
    assert ((y.cpu().float() - ref).abs() <= ref.abs() * 2 ** -7 + 1e-6).all()


def test_mlp_config1_full_size_sampled_members():
    """Config 1 at its real shape (P = 256, T = 2048, shared x); three members checked in full."""
    from noise_amd import ops
    P, T = 256, 2048
    log_case(f'mlp config1 P={P} T={T}')
    args = _mlp_inputs(P, T, True, 1e-3, seed=2)
    dev = [t.to(DEV) for t in args]
    y = ops.lowrank_mlp(*dev, T=T, pair_shift=1, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    members = [0, 1, 255]
    ref = _oracle_members(*args, members)
    got = y[members].cpu().float()
    assert rel_err(got, ref) < 1e-2
