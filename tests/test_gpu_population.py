"""GPU parity of the population forward and of the EGGROLL update kernels against the CPU oracle.

Tolerances (north star): <= 1e-2 relative error on bf16 activations, <= 1e-4 absolute error on
per-member fp32 losses. The oracle runs in its bf16 rounding-point mode (the reference under CUDA
autocast) with the fp32 head; the kernels keep those rounding points.

The 1e-4 loss bar is applied at the reference's own initialisation (make_model seed 0), where the
bf16 path's sensitivity to summation order is ~4e-5. At trained-scale weights (`trained_like`) the
same path is chaotic at the 1e-3 level: the oracle itself moves by ~1.5e-3 when its GEMMs accumulate
in fp64 instead of fp32. There the bound is twice that measured floor (plus 1e-4), computed in the
test from two oracle runs."""
import math

import pytest
import torch

from noise_amd import _lib
from noise_amd.model import make_model
from noise_amd.synthetic import antithetic_signs, population_noise, trained_like, zipf_tokens
from oracle import eggroll as oe
from oracle import model as om
from tests._util import log_case, rel_err, tile16_index, wtile_index

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def _dev(noise):
    return {n: tuple(t.to(DEV) for t in v) if isinstance(v, tuple) else v.to(DEV) for n, v in noise.items()}


@pytest.fixture(scope='module')
def trained():
    torch.manual_seed(0)
    model = trained_like(make_model('cpu', 0))
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    return model, params


def _gpu_model(model):
    m = make_model('cpu', 0)
    m.load_state_dict(model.state_dict())
    return m.to(DEV)


# ---------------------------------------------------------------- stage kernels

def test_embed_norm_matches_oracle():
    g = torch.Generator().manual_seed(1)
    V, T, m = 4096, 128, 4
    w = torch.randn(V, 512, generator=g)
    a, b = torch.randn(2, V, generator=g), torch.randn(2, 512, generator=g)
    sign = antithetic_signs(m, 1e-2)
    idx, _ = zipf_tokens(T, seed=3)
    log_case(f'embed_norm m={m} T={T}')
    x0 = torch.empty(m * T, 512, device=DEV)
    d = [t.to(DEV) for t in (w, a, b, sign, idx)]  # device copies stay referenced until the kernel ran
    _lib.call('noise_embed_norm', d[0].data_ptr(), V, d[1].data_ptr(), d[2].data_ptr(), d[3].data_ptr(),
              d[4].data_ptr(), m, T, 1, x0.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    rep = lambda t: t.repeat_interleave(2, 0)  # noqa: E731
    ref = om.norm(om.lowrank_embed(w, rep(a), rep(b), idx, sign)).reshape(m * T, 512)
    assert (x0.cpu() - ref).abs().max() < 2e-5

    # a block entry that recomputes x0 from the embedding (x0 and, at block 0, x_in null) equals one that
    # reads the stored x0, bit for bit
    log_case(f'block_entry with recomputed x0 m={m} T={T}')
    s = torch.cuda.current_stream().cuda_stream
    bq, bk, bv = (torch.randn(2, 512, generator=g).to(DEV) for _ in range(3))
    lr, l0 = torch.tensor([0.9], device=DEV), torch.tensor([0.2], device=DEV)
    er, e0 = torch.randn(2, 8, generator=g).to(DEV), torch.randn(2, 8, generator=g).to(DEV)
    out = {}
    emb, emb_ptr = _lib.embed(d[0].data_ptr(), V, d[1].data_ptr(), d[2].data_ptr(), d[4].data_ptr())
    for mode in ('stored', 'recomputed'):
        xo, h = torch.empty(m * T, 512, device=DEV), torch.empty(m * T, 512, device=DEV, dtype=torch.bfloat16)
        u = torch.empty(m * T, 4, device=DEV)
        stored = mode == 'stored'
        _lib.call('noise_block_entry', x0.data_ptr() if stored else None, x0.data_ptr() if stored else None,
                  xo.data_ptr(), h.data_ptr(), u.data_ptr(), bq.data_ptr(), bk.data_ptr(), bv.data_ptr(), lr.data_ptr(),
                  l0.data_ptr(), er.data_ptr(), e0.data_ptr(), 8, 0, 0, 0, 0, d[3].data_ptr(), m, T, 1, None, 0,
                  None if stored else emb_ptr, s)
        torch.cuda.synchronize()
        out[mode] = (xo.cpu(), h.cpu(), u.cpu())
    for a_, b_ in zip(out['stored'], out['recomputed']):
        assert torch.equal(a_, b_)


def test_block_entry_and_qkv_match_oracle():
    """Block entry (mix, norm, q/k/v dots, value gate) and the QKV GEMM epilogue (segment rank-1,
    rotary, QK-norm, gated value embedding) against the oracle ops at sigma = 0.05."""
    g = torch.Generator().manual_seed(8)
    m, T, V = 4, 128, 4096
    sign = antithetic_signs(m, 0.05)
    x = torch.randn(m, T, 512, generator=g) * 2
    x0 = torch.randn(m, T, 512, generator=g)
    lam_r, lam_0 = torch.tensor([0.9]), torch.tensor([0.15])
    eps = torch.randn(m, 8, generator=g), torch.randn(m, 8, generator=g)
    wq, wk, wv = (torch.randn(512, 512, generator=g) / 22 for _ in range(3))
    (aq, bq), (ak, bk), (av, bv) = ((torch.randn(m, 512, generator=g), torch.randn(m, 512, generator=g))
                                    for _ in range(3))
    gw = torch.randn(8, 32, generator=g) * 0.2
    ga, gb = torch.randn(m, 8, generator=g), torch.randn(m, 32, generator=g)
    vw = torch.randn(V, 512, generator=g) * 0.1
    va, vb = torch.randn(m, V, generator=g), torch.randn(m, 512, generator=g)
    idx, _ = zipf_tokens(T, seed=9)
    cos, sin = om.rotary_tables()
    d = {k: t.to(DEV) for k, t in dict(x=x, x0=x0, lr=lam_r, l0=lam_0, er=eps[0], e0=eps[1], bq=bq, bk=bk, bv=bv,
                                        aq=aq, ak=ak, av=av, gw=gw, ga=ga, gb=gb, vw=vw, va=va, vb=vb, idx=idx,
                                        sign=sign, cos=cos.contiguous(), sin=sin.contiguous()).items()}
    wqkv = torch.cat([wq, wk, wv]).to(DEV)
    wqkv16 = torch.empty(1536, 512, device=DEV, dtype=torch.bfloat16)
    M = m * T
    xo, h = torch.empty(M, 512, device=DEV), torch.empty(M, 512, device=DEV, dtype=torch.bfloat16)
    u, gate = torch.empty(M, 4, device=DEV), torch.empty(M, 8, device=DEV)
    qkv = torch.empty(M, 1536, device=DEV, dtype=torch.bfloat16)
    s = torch.cuda.current_stream().cuda_stream
    log_case(f'block_entry + qkv m={m} T={T}')
    _lib.call('noise_cast_bf16', wqkv.data_ptr(), wqkv16.data_ptr(), wqkv.numel(), 0, s)
    _lib.call('noise_block_entry', d['x'].data_ptr(), d['x0'].data_ptr(), xo.data_ptr(), h.data_ptr(), u.data_ptr(),
              d['bq'].data_ptr(), d['bk'].data_ptr(), d['bv'].data_ptr(), d['lr'].data_ptr(), d['l0'].data_ptr(),
              d['er'].data_ptr() + 4 * 3, d['e0'].data_ptr() + 4 * 3, 8, d['gw'].data_ptr(), d['ga'].data_ptr(),
              d['gb'].data_ptr(), gate.data_ptr(), d['sign'].data_ptr(), m, T, 0, None, 0, None, s)
    _lib.call('noise_qkv', h.data_ptr(), wqkv16.data_ptr(), d['aq'].data_ptr(), d['ak'].data_ptr(), d['av'].data_ptr(),
              u.data_ptr(), d['sign'].data_ptr(), m, T, 0, d['cos'].data_ptr(), d['sin'].data_ptr(), gate.data_ptr(),
              d['vw'].data_ptr(), V, d['va'].data_ptr(), d['vb'].data_ptr(), d['idx'].data_ptr(), 0, qkv.data_ptr(), s)
    torch.cuda.synchronize()
    sg = sign[:, None, None]
    xr = (lam_r + sg * eps[0][:, 3, None, None]) * x + (lam_0 + sg * eps[1][:, 3, None, None]) * x0
    assert (xo.cpu().view(m, T, 512) - xr).abs().max() < 1e-5
    hr = om.norm(xr)
    assert (h.cpu().float().view(m, T, 512) - om.bf(hr)).abs().max() <= 2 ** -7 * hr.abs().max()
    for k, bb in enumerate((bq, bk, bv)):
        ur = om.bf(om.bf(hr) @ om.bf(bb).unsqueeze(-1))[..., 0]
        assert torch.allclose(u.cpu()[:, k].view(m, T), ur, atol=2e-2, rtol=1e-2)
    # column 3 carries the member's sign for the QKV epilogue
    assert torch.equal(u.cpu()[:, 3].view(m, T), sign[:, None].expand(m, T))
    gr = 2 * torch.sigmoid(om.lowrank(hr[..., :32], gw, ga, gb, sign, 'bf16'))
    assert torch.allclose(gate.cpu().view(m, T, 8), gr, atol=2e-3)
    # q | k | v from the GPU's own h, u and gate (isolates the GEMM epilogue)
    hg = h.cpu().float().view(m, T, 512)
    ug = u.cpu().view(m, T, 4)

    def lin(w, a, k):
        return om.bf(hg @ om.bf(w).t()) + sg * ug[..., k:k + 1] * a[:, None, :]
    q, kk_, vv = lin(wq, aq, 0), lin(wk, ak, 1), lin(wv, av, 2)
    ve = om.lowrank_embed(vw, va, vb, idx, sign)
    vv = vv.view(m, T, 8, 64) + gate.cpu().view(m, T, 8).unsqueeze(-1) * ve.view(m, T, 8, 64)
    c, sn = cos[:T], sin[:T]
    qr = om.norm(om.apply_rotary(q.view(m, T, 8, 64), c, sn))
    kr = om.norm(om.apply_rotary(kk_.view(m, T, 8, 64), c, sn))
    # q, k and v are written as fp16 of the fp32 values (11-bit significand), q multiplied by log2(e) / 8 first:
    # the error is fp16 rounding plus the dense product's bf16 rounding, which a different fp32 summation order
    # can move by one bf16 step
    got = qkv.cpu().view(torch.float16).float().view(m, T, 3, 8, 64)
    got[:, :, 0] /= math.log2(math.e) / 8
    for k, ref in enumerate((qr, kr, vv)):
        assert rel_err(got[:, :, k], ref) < 2e-3, k
        assert (got[:, :, k] - ref).abs().max() <= 2 ** -7 * ref.abs().max() + 1e-3, k
    # fp16, not bf16: rounding the fp32 result to fp16 changes it by at most 2^-11 relative, and the GPU's
    # values agree with that rounding far better than bf16 rounding would allow
    assert rel_err(got[:, :, 1], kr.half().float()) < rel_err(om.bf(kr), kr)
    # a block without value embedding (gate null): the same q | k, v = lowrank only
    log_case(f'qkv without value embedding m={m} T={T}')
    qkv2 = torch.empty_like(qkv)
    _lib.call('noise_qkv', h.data_ptr(), wqkv16.data_ptr(), d['aq'].data_ptr(), d['ak'].data_ptr(), d['av'].data_ptr(),
              u.data_ptr(), d['sign'].data_ptr(), m, T, 0, d['cos'].data_ptr(), d['sin'].data_ptr(), None,
              None, V, None, None, None, 0, qkv2.data_ptr(), s)
    torch.cuda.synchronize()
    assert torch.equal(qkv2[:, :1024].cpu(), qkv[:, :1024].cpu())
    v2 = qkv2[:, 1024:].cpu().view(torch.float16).float().view(m, T, 512)
    vref = lin(wv, av, 2)
    assert rel_err(v2, vref) < 2e-3
    assert (v2 - vref).abs().max() <= 2 ** -7 * vref.abs().max() + 1e-3


def test_qkv_tile_gemm_path_for_token_counts_not_a_multiple_of_32():
    """noise_qkv at T = 48 (not a multiple of the weight-resident kernel's 32-row blocks) runs q | k | v, with the
    gated value embedding, on the tile GEMM's QKV epilogue: the same formats (fp16, q times log2(e) / 8) and the
    same arithmetic, checked against the oracle ops from the GPU's own h, u and gate."""
    g = torch.Generator().manual_seed(33)
    m, T, V = 4, 48, 4096
    M = m * T
    sign = antithetic_signs(m, 0.05)
    h = torch.randn(M, 512, generator=g).bfloat16()
    wq, wk, wv = (torch.randn(512, 512, generator=g) / 22 for _ in range(3))
    aq, ak, av = (torch.randn(m // 2, 512, generator=g) for _ in range(3))
    u = torch.randn(M, 4, generator=g)
    u[:, 3] = sign.repeat_interleave(T)
    gate = 2 * torch.sigmoid(torch.randn(M, 8, generator=g))
    vw = torch.randn(V, 512, generator=g) * 0.1
    va, vb = torch.randn(m // 2, V, generator=g), torch.randn(m // 2, 512, generator=g)
    idx, _ = zipf_tokens(T, seed=34)
    cos, sin = om.rotary_tables()
    d = {k: t.to(DEV).contiguous() for k, t in dict(h=h, u=u, gate=gate, vw=vw, va=va, vb=vb, idx=idx, sign=sign,
                                                    aq=aq, ak=ak, av=av, cos=cos, sin=sin).items()}
    w16 = torch.cat([wq, wk, wv]).bfloat16().to(DEV)
    qkv = torch.empty(M, 1536, device=DEV, dtype=torch.bfloat16)
    log_case(f'qkv tile-GEMM path m={m} T={T}')
    _lib.call('noise_qkv', d['h'].data_ptr(), w16.data_ptr(), d['aq'].data_ptr(), d['ak'].data_ptr(),
              d['av'].data_ptr(), d['u'].data_ptr(), d['sign'].data_ptr(), m, T, 1, d['cos'].data_ptr(),
              d['sin'].data_ptr(), d['gate'].data_ptr(), d['vw'].data_ptr(), V, d['va'].data_ptr(), d['vb'].data_ptr(),
              d['idx'].data_ptr(), 0, qkv.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    member = torch.arange(M) // T
    dirn, srow = member // 2, sign[member][:, None]
    hf = h.float()

    def lin(w, a, col):
        return om.bf(hf @ om.bf(w).t()) + (srow * om.bf(u[:, col:col + 1])) * a[dirn]
    q, k, v = lin(wq, aq, 0), lin(wk, ak, 1), lin(wv, av, 2)
    tok = idx.repeat(m)
    v = v + gate.repeat_interleave(64, 1) * (vw[tok] + (srow * va[dirn, tok][:, None]) * vb[dirn])
    c, sn = cos[:T], sin[:T]
    qr = om.norm(om.apply_rotary(q.view(m, T, 8, 64), c, sn)).reshape(M, 512)
    kr = om.norm(om.apply_rotary(k.view(m, T, 8, 64), c, sn)).reshape(M, 512)
    got = qkv.cpu().view(torch.float16).float()
    got[:, :512] /= math.log2(math.e) / 8
    for sl, ref in ((slice(0, 512), qr), (slice(512, 1024), kr), (slice(1024, 1536), v)):
        assert rel_err(got[:, sl], ref) < 2e-3, sl
        assert (got[:, sl] - ref).abs().max() <= 2 ** -7 * ref.abs().max() + 1e-3, sl


@pytest.mark.parametrize('m,T', [(64, 512), (36, 256)])
def test_value_embedding_v_many_blocks_per_workgroup(m, T):
    """v with the gated value embedding (train/val/eggroll.py:84-89) at sizes where every workgroup of the
    weight-resident kernel walks several 32-row blocks (its ring of x blocks, gathered embedding rows and
    next-block token ids in steady state, odd and even block counts), one token sequence per member (four
    distinct sequences) and antithetic pairs sharing a direction: v = bf16(h W_v^T) + s bf16(u_v) a_v +
    gate (W[idx] + s a[idx] b), within fp16 rounding and one bf16 step of the dense product."""
    g = torch.Generator().manual_seed(31)
    V, M, dirs = 4096, m * T, m // 2
    sign = antithetic_signs(m, 0.05)
    h = torch.randn(M, 512, generator=g).bfloat16()
    wqkv = torch.randn(1536, 512, generator=g) / 22
    a = [torch.randn(dirs, 512, generator=g) for _ in range(3)]
    u = torch.randn(M, 4, generator=g)
    u[:, 3] = sign.repeat_interleave(T)
    gate = 2 * torch.sigmoid(torch.randn(M, 8, generator=g))
    vw = torch.randn(V, 512, generator=g) * 0.1
    va, vb = torch.randn(dirs, V, generator=g), torch.randn(dirs, 512, generator=g)
    seqs = torch.stack([zipf_tokens(T, seed=40 + j)[0] for j in range(4)])
    idx = seqs[torch.arange(m) % 4]                         # [m, T]: member p reads sequence p % 4
    cos, sin = om.rotary_tables()
    d = {k: t.to(DEV).contiguous() for k, t in dict(h=h, u=u, gate=gate, vw=vw, va=va, vb=vb, idx=idx, sign=sign,
                                                    aq=a[0], ak=a[1], av=a[2], cos=cos, sin=sin).items()}
    w16 = wqkv.bfloat16().to(DEV)
    s = torch.cuda.current_stream().cuda_stream
    out = {}
    for ve in (True, False):
        log_case(f'qkv value embedding={ve} m={m} T={T} (per-member tokens, pair_shift 1)')
        qkv = torch.empty(M, 1536, device=DEV, dtype=torch.bfloat16)
        _lib.call('noise_qkv', d['h'].data_ptr(), w16.data_ptr(), d['aq'].data_ptr(), d['ak'].data_ptr(),
                  d['av'].data_ptr(), d['u'].data_ptr(), d['sign'].data_ptr(), m, T, 1, d['cos'].data_ptr(),
                  d['sin'].data_ptr(), d['gate'].data_ptr() if ve else None, d['vw'].data_ptr() if ve else None, V,
                  d['va'].data_ptr() if ve else None, d['vb'].data_ptr() if ve else None,
                  d['idx'].data_ptr() if ve else None, T, qkv.data_ptr(), s)
        torch.cuda.synchronize()
        out[ve] = qkv.cpu()
    # q | k do not depend on the value embedding
    assert torch.equal(out[True][:, :1024], out[False][:, :1024])
    member = torch.arange(M) // T
    dirn, srow = member // 2, sign[member][:, None]
    tok = idx.reshape(-1)
    dense = om.bf(h.float() @ om.bf(wqkv[1024:]).t())
    v0 = dense + (srow * om.bf(u[:, 2:3])) * a[2][dirn]
    ve_rows = vw[tok] + (srow * va[dirn, tok][:, None]) * vb[dirn]
    v1 = v0 + gate.repeat_interleave(64, 1) * ve_rows
    for ve, ref in ((False, v0), (True, v1)):
        got = out[ve][:, 1024:].view(torch.float16).float()
        assert rel_err(got, ref) < 2e-3, ve
        assert (got - ref).abs().max() <= 2 ** -7 * ref.abs().max() + 1e-3, ve
        # v leaves as fp16 of the fp32 value: closer to ref than the bf16 rounding of ref
        assert rel_err(got, ref.half().float()) < rel_err(om.bf(ref), ref), ve



def test_deferred_residuals_match_eager_lowrank():
    """Two c_proj outputs deferred into the block entry and one into the MLP entry equal the eager
    `x = x + lowrank(...)` of train/val/eggroll.py:92-93: dense bf16 product plus s bf16(sum of the input-side
    partials) a, added in order in fp32 (partials row-major for the attention, part-major for the MLP)."""
    g = torch.Generator().manual_seed(12)
    m, T, D = 4, 64, 512
    M = m * T
    x, x0 = torch.randn(M, D, generator=g) * 3, torch.randn(M, D, generator=g)
    y1, y2 = (torch.randn(M, D, generator=g).bfloat16() for _ in range(2))
    u1 = torch.randn(M, 8, generator=g)           # row-major partials [rows, 8]
    u2 = torch.randn(8, M, generator=g)           # part-major partials [8, rows]
    a1, a2 = torch.randn(m // 2, D, generator=g), torch.randn(m // 2, D, generator=g)
    sign = torch.tensor([0.05, -0.05, 0.02, -0.02])
    lr, l0 = torch.tensor([0.9]), torch.tensor([0.3])
    er, e0 = torch.randn(m // 2, 8, generator=g), torch.randn(m // 2, 8, generator=g)
    bq, bk, bv = (torch.randn(m // 2, D, generator=g) for _ in range(3))
    dev = {k: v.to(DEV) for k, v in dict(x=x, x0=x0, y1=y1, y2=y2, u1=u1, u2=u2, a1=a1, a2=a2, sign=sign, lr=lr, l0=l0,
                                          er=er, e0=e0, bq=bq, bk=bk, bv=bv).items()}
    log_case(f'deferred residuals m={m} T={T}')
    s = torch.cuda.current_stream().cuda_stream
    p1 = (dev['y1'].data_ptr(), dev['u1'].data_ptr(), 8, 8, 1, dev['a1'].data_ptr())
    p2 = (dev['y2'].data_ptr(), dev['u2'].data_ptr(), 8, 1, M, dev['a2'].data_ptr())
    xo = torch.empty(M, D, device=DEV)
    h = torch.empty(M, D, device=DEV, dtype=torch.bfloat16)
    u = torch.empty(M, 4, device=DEV)
    pend, npend = _lib.pending(p1, p2)
    _lib.call('noise_block_entry', dev['x'].data_ptr(), dev['x0'].data_ptr(), xo.data_ptr(), h.data_ptr(), u.data_ptr(),
              dev['bq'].data_ptr(), dev['bk'].data_ptr(), dev['bv'].data_ptr(), dev['lr'].data_ptr(), dev['l0'].data_ptr(),
              dev['er'].data_ptr() + 4 * 3, dev['e0'].data_ptr() + 4 * 3, 8, 0, 0, 0, 0, dev['sign'].data_ptr(), m, T, 1,
              pend, npend, None, s)
    hn = torch.empty(M, D, device=DEV, dtype=torch.bfloat16)
    un = torch.empty(M, device=DEV)
    pend1, n1 = _lib.pending(p1)
    _lib.call('noise_norm_dot', dev['x'].data_ptr(), hn.data_ptr(), dev['bq'].data_ptr(), un.data_ptr(),
              dev['sign'].data_ptr(), m, T, 1, pend1, n1, s)
    torch.cuda.synchronize()
    rows = torch.arange(M)
    member = rows // T
    srow = sign[member][:, None]
    dirs = member // 2

    def lowrank_out(y, usum, a):
        return y.float() + (srow * om.bf(usum)[:, None]) * a[dirs]
    def seqsum(parts):  # q = 0, 1, ... in fp32, the kernel's order (bf16 rounding of the sum is order-sensitive)
        acc = parts[0].clone()
        for q in range(1, parts.shape[0]):
            acc = acc + parts[q]
        return acc
    v1 = lowrank_out(y1, seqsum(u1.t()), a1)
    v2 = lowrank_out(y2, seqsum(u2), a2)
    mixed = ((x + v1) + v2)
    lam_r = lr + srow * er[dirs][:, 3:4]
    lam_0 = l0 + srow * e0[dirs][:, 3:4]
    ref_x = lam_r * mixed + lam_0 * x0
    assert torch.allclose(xo.cpu(), ref_x, rtol=1e-5, atol=1e-5)
    assert rel_err(h.cpu().float(), om.bf(om.norm(ref_x))) < 5e-3
    ref_h1 = om.norm(x + v1)
    assert rel_err(hn.cpu().float(), om.bf(ref_h1)) < 5e-3
    # x itself is not written by the MLP entry
    assert torch.equal(dev['x'].cpu(), x)


def test_block_entry_grouped_and_per_row_instances_agree_bit_for_bit():
    """The block entry at T = 96 (workgroups of a few rows of one member, the member's vectors staged in LDS) and the
    same rows cut into T = 6 members (one row per wave, vectors read per row) write the same x, h, dots and gates,
    bit for bit: with deferred residuals, the value-embedding gate and x0 both stored and recomputed, and as block 0
    (no incoming stream, no deferred residuals, x0 recomputed: the first-block instances)."""
    g = torch.Generator().manual_seed(21)
    m, T, D, V, R = 4, 96, 512, 4096, 16  # R: members of the cut layout per member
    M = m * T
    x, x0 = torch.randn(M, D, generator=g) * 3, torch.randn(M, D, generator=g)
    y1, y2 = (torch.randn(M, D, generator=g).bfloat16() for _ in range(2))
    u1, u2 = torch.randn(M, 8, generator=g), torch.randn(8, M, generator=g)
    sign = antithetic_signs(m, 0.05)
    lr, l0 = torch.tensor([0.9]), torch.tensor([0.3])
    # per-direction vectors of the grouped layout (pair_shift 1: m // 2 directions)
    vec = dict(a1=torch.randn(m // 2, D, generator=g), a2=torch.randn(m // 2, D, generator=g),
               er=torch.randn(m // 2, 8, generator=g), e0=torch.randn(m // 2, 8, generator=g),
               bq=torch.randn(m // 2, D, generator=g), bk=torch.randn(m // 2, D, generator=g),
               bv=torch.randn(m // 2, D, generator=g), ga=torch.randn(m // 2, 8, generator=g),
               gb=torch.randn(m // 2, 32, generator=g), eb=torch.randn(m // 2, D, generator=g))
    gw = torch.randn(8, 32, generator=g) * 0.2
    w, ea = torch.randn(V, D, generator=g), torch.randn(m // 2, V, generator=g)
    idx, _ = zipf_tokens(T, seed=5)
    idx = idx.repeat(m)  # a sequence per member: member p reads idx[p T .. p T + T)
    s = torch.cuda.current_stream().cuda_stream
    common = {k: t.to(DEV) for k, t in dict(x=x, x0=x0, y1=y1, y2=y2, u1=u1, u2=u2, lr=lr, l0=l0, gw=gw, w=w,
                                             idx=idx).items()}
    out = {}
    for layout, (mm, TT, ps, rep) in dict(grouped=(m, T, 1, 1), per_row=(m * R, T // R, 0, 2 * R)).items():
        # the cut layout's member p' = R p + j is its own direction (pair_shift 0) carrying direction p // 2's vectors
        d = {k: v.repeat_interleave(rep, 0).to(DEV) for k, v in vec.items()}
        d['ea'] = ea.repeat_interleave(rep, 0).to(DEV)
        d['sign'] = sign.repeat_interleave(R if layout == 'per_row' else 1).to(DEV)
        p1 = (common['y1'].data_ptr(), common['u1'].data_ptr(), 8, 8, 1, d['a1'].data_ptr())
        p2 = (common['y2'].data_ptr(), common['u2'].data_ptr(), 8, 1, M, d['a2'].data_ptr())
        pend, npend = _lib.pending(p1, p2)
        emb, emb_ptr = _lib.embed(common['w'].data_ptr(), V, d['ea'].data_ptr(), d['eb'].data_ptr(),
                                  common['idx'].data_ptr(), TT)
        for x0_mode in ('stored', 'recomputed', 'first'):
            log_case(f'block_entry {layout} m={mm} T={TT} x0 {x0_mode}')
            stored, first = x0_mode == 'stored', x0_mode == 'first'
            xo, h = torch.empty(M, D, device=DEV), torch.empty(M, D, device=DEV, dtype=torch.bfloat16)
            u, gate = torch.empty(M, 4, device=DEV), torch.empty(M, 8, device=DEV)
            _lib.call('noise_block_entry', None if first else common['x'].data_ptr(),
                      common['x0'].data_ptr() if stored else None,
                      xo.data_ptr(), h.data_ptr(), u.data_ptr(), d['bq'].data_ptr(), d['bk'].data_ptr(),
                      d['bv'].data_ptr(), common['lr'].data_ptr(), common['l0'].data_ptr(), d['er'].data_ptr() + 4 * 3,
                      d['e0'].data_ptr() + 4 * 3, 8, common['gw'].data_ptr(), d['ga'].data_ptr(), d['gb'].data_ptr(),
                      gate.data_ptr(), d['sign'].data_ptr(), mm, TT, ps, None if first else pend, 0 if first else npend,
                      None if stored else emb_ptr, s)
            torch.cuda.synchronize()
            out[layout, x0_mode] = (xo.cpu(), h.cpu(), u.cpu(), gate.cpu())
    for x0_mode in ('stored', 'recomputed', 'first'):
        for a_, b_ in zip(out['grouped', x0_mode], out['per_row', x0_mode]):
            assert torch.equal(a_, b_), x0_mode
    # the recomputed x0 is a different x0 from the stored one: the two modes must differ
    assert not torch.equal(out['grouped', 'stored'][0], out['grouped', 'recomputed'][0])

def test_mlp_hidden_tile16_matches_rows():
    """noise_mlp_fc writes the same hidden (bit for bit, up to the layout) and the same partials in TILE16 as in
    ROWS, and noise_dense_bf16 on the TILE16 hidden returns exactly its result on the row-major one, with the
    weight row-major or in the WTILE copy noise_weight_tiles makes (itself checked element by element)."""
    g = torch.Generator().manual_seed(13)
    m, T, D, F = 4, 64, 512, 2048
    M = m * T
    h = torch.randn(M, D, generator=g).bfloat16()
    wfc = (torch.randn(F, D, generator=g) * D ** -0.5).bfloat16()
    wpj = (torch.randn(D, F, generator=g) * F ** -0.5).bfloat16()
    afc, bpj = torch.randn(m // 2, F, generator=g), torch.randn(m // 2, F, generator=g)
    u = torch.randn(M, generator=g)
    sign = torch.tensor([0.05, -0.05, 0.02, -0.02])
    d = {k: v.to(DEV) for k, v in dict(h=h, wfc=wfc, wpj=wpj, afc=afc, bpj=bpj, u=u, sign=sign).items()}
    log_case(f'mlp hidden TILE16 vs ROWS m={m} T={T}')
    s = torch.cuda.current_stream().cuda_stream
    parts = _lib.value('noise_mlp_fc_parts', F)
    wt = torch.empty_like(d['wpj'])
    _lib.call('noise_weight_tiles', d['wpj'].data_ptr(), D, F, wt.data_ptr(), s)
    torch.cuda.synchronize()
    assert torch.equal(wt.cpu().flatten()[wtile_index(D, F)], wpj)
    out = {}
    for layout in (_lib.LAYOUT_ROWS, _lib.LAYOUT_TILE16):
        hid = torch.empty(M, F, device=DEV, dtype=torch.bfloat16)
        up = torch.empty(parts, M, device=DEV)
        _lib.call('noise_mlp_fc', d['h'].data_ptr(), d['wfc'].data_ptr(), D, F, d['afc'].data_ptr(), d['u'].data_ptr(),
                  d['bpj'].data_ptr(), d['sign'].data_ptr(), m, T, 1, hid.data_ptr(), layout, up.data_ptr(), s)
        ys = []
        for wl, w in ((_lib.LAYOUT_ROWS, d['wpj']), (_lib.LAYOUT_WTILE, wt)):
            y = torch.empty(M, D, device=DEV, dtype=torch.bfloat16)
            _lib.call('noise_dense_bf16', hid.data_ptr(), layout, F, D, w.data_ptr(), wl, m, T, y.data_ptr(), s)
            ys.append(y)
        torch.cuda.synchronize()
        out[layout] = (hid.cpu(), up.cpu(), ys[0].cpu(), ys[1].cpu())
    rows_h, rows_u, rows_y, rows_yw = out[_lib.LAYOUT_ROWS]
    tile_h, tile_u, tile_y, tile_yw = out[_lib.LAYOUT_TILE16]
    assert torch.equal(tile_h.flatten()[tile16_index(M, F)], rows_h)
    assert torch.equal(tile_u, rows_u)
    assert torch.equal(tile_y, rows_y)
    assert torch.equal(rows_yw, rows_y)
    assert torch.equal(tile_yw, rows_y)
    # and the dense product itself: bf16(hidden W^T) with fp32 accumulation
    ref = (rows_h.float() @ wpj.float().t()).bfloat16().float()
    assert rel_err(rows_y.float(), ref) < 5e-3
    # K = 512 (the attention c_proj shape: the weight-resident kernel) against the same reference
    log_case(f'dense K=512 m={m} T={T}')
    wap = (torch.randn(D, D, generator=g) * D ** -0.5).bfloat16()
    wapd = wap.to(DEV)
    wapt = torch.empty_like(wapd)
    _lib.call('noise_weight_tiles', wapd.data_ptr(), D, D, wapt.data_ptr(), s)
    ya, yat = (torch.empty(M, D, device=DEV, dtype=torch.bfloat16) for _ in range(2))
    _lib.call('noise_dense_bf16', d['h'].data_ptr(), _lib.LAYOUT_ROWS, D, D, wapd.data_ptr(), _lib.LAYOUT_ROWS, m, T,
              ya.data_ptr(), s)
    _lib.call('noise_dense_bf16', d['h'].data_ptr(), _lib.LAYOUT_ROWS, D, D, wapt.data_ptr(), _lib.LAYOUT_WTILE, m, T,
              yat.data_ptr(), s)
    torch.cuda.synchronize()
    assert torch.equal(yat.cpu(), ya.cpu())
    refa = (h.float() @ wap.float().t()).bfloat16().float()
    assert rel_err(ya.cpu().float(), refa) < 5e-3
    # one bf16 ulp at most: only the fp32 summation order differs
    assert ((ya.cpu().float() - refa).abs() <= refa.abs() * 2 ** -7 + 1e-6).all()


@pytest.mark.parametrize('qk_norm,qk_format', [(0, 0), (1, 0), (1, 1), (0, 1), (1, 2), (1, 3)])
def test_attention_matches_oracle_and_moments(qk_norm, qk_format):
    """qk_norm = 0: any q, k (running-maximum softmax); qk_norm = 1: q, k RMS-normalised per head as the
    model's QK-norm leaves them (bounded scores, no running maximum), including rows scaled to the bound.
    qk_format 0: q and k bf16 (the credit reruns'), 1: fp16, 2: fp16 with q pre-multiplied by log2(e) / 8 (the
    population forward's, as noise_qkv writes it); v fp16. qk_format 3: q, k and v bf16 with bf16 probabilities
    (the autocast clean forward's), against the oracle's bf16 attention."""
    g = torch.Generator().manual_seed(2)
    m, T = 2, 256
    dt = torch.float16 if qk_format in (1, 2) else torch.bfloat16
    for window in (T, 100):
        log_case(f'attention m={m} T={T} window={window} qk_norm={qk_norm} qk_format={qk_format}')
        q, k, v = (torch.randn(m, T, 8, 64, generator=g) for _ in range(3))
        if qk_norm:
            q, k = om.norm(q), om.norm(k)
            # extreme case: every key of the first head equal to its query direction (scores at the bound)
            k[:, :, 0] = q[:, :, 0]
        q, k, v = q.to(dt), k.to(dt), (v.bfloat16() if qk_format == 3 else v.half())
        q_in = (q.float() * (math.log2(math.e) / 8)).half() if qk_format == 2 else q
        if qk_format == 2:
            q = q_in.float() / (math.log2(math.e) / 8)  # the q the kernel sees, back in score units (fp32)
        qkv = torch.cat([q_in.reshape(m * T, 512).view(torch.bfloat16), k.reshape(m * T, 512).view(torch.bfloat16),
                         v.reshape(m * T, 512).view(torch.bfloat16)], 1).to(DEV)
        y = torch.empty(m * T, 512, device=DEV, dtype=torch.bfloat16)
        bp = torch.randn(m, 512, generator=g)
        bpd = bp.to(DEV)
        up = torch.empty(m * T, 8, device=DEV)
        mom = torch.empty(m, 8, 2, 64, device=DEV)
        ws = torch.empty(_lib.size_query('noise_attention_workspace_size', m, T), device=DEV, dtype=torch.uint8)
        _lib.call('noise_attention', qkv.data_ptr(), m, T, window, qk_norm, qk_format, bpd.data_ptr(), 0, y.data_ptr(),
                  up.data_ptr(), mom.data_ptr(), ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        if qk_format == 3:
            ref = om.attention_bf16(q.float(), k.float(), v.float(), window)
        else:
            ref = om.bf(om.attention(q.float(), k.float(), v.float(), window))  # [m, T, 8, 64]
        got = y.cpu().float().view(m, T, 8, 64)
        assert rel_err(got, ref) < 1e-2
        assert (got - ref).abs().max() < 2e-2
        # c_proj dot partials: sum over heads equals y . bf16(b_proj)
        dot = (got.reshape(m, T, 512) * om.bf(bp)[:, None, :]).reshape(m, T, 8, 64).sum(-1)
        assert torch.allclose(up.cpu().view(m, T, 8), dot, atol=1e-3, rtol=1e-3)
        # credit moments over tokens of the bf16 output
        m1, m2 = om.attention_moments(got.permute(0, 2, 1, 3))
        assert torch.allclose(mom.cpu()[:, :, 0], m1, atol=1e-5)
        assert torch.allclose(mom.cpu()[:, :, 1], m2, atol=1e-5)


def _head_weight(W, fmt, s):
    """The head weight on the device in noise_head_ce's format fmt (NOISE_HEAD_*): fp32 itself, the bf16 split
    [W_hi | W_lo | W_hi], or bf16."""
    Wd = W.contiguous().to(DEV)
    if fmt == _lib.HEAD_FP32:
        return Wd
    wd = torch.empty(W.shape[0], 1536 if fmt == _lib.HEAD_FP32_SPLIT else 512, device=DEV, dtype=torch.bfloat16)
    _lib.call('noise_cast_bf16', Wd.data_ptr(), wd.data_ptr(), W.numel(), 512 if fmt == _lib.HEAD_FP32_SPLIT else 0, s)
    torch.cuda.synchronize()
    return wd


HEAD_FORMATS = (_lib.HEAD_FP32, _lib.HEAD_FP32_SPLIT, _lib.HEAD_BF16)


def test_head_ce_matches_oracle_fp32_and_bf16_heads():
    g = torch.Generator().manual_seed(4)
    m, T, V = 4, 256, 4096
    x = torch.randn(m * T, 512, generator=g) * 3
    W = torch.randn(V, 512, generator=g) * 512 ** -0.5 * 2
    a, b = torch.randn(m, V, generator=g), torch.randn(m, 512, generator=g)
    sign = torch.tensor([1e-2, -1e-2, 5e-2, -5e-2])
    _, targets = zipf_tokens(T, seed=5)
    s = torch.cuda.current_stream().cuda_stream
    h = om.norm(x.view(m, T, 512))
    xd, ad, bd, sd, td = (t.to(DEV) for t in (x, a, b, sign, targets))
    for fp32 in HEAD_FORMATS:
        log_case(f'head_ce m={m} T={T} fp32_head={fp32}')
        wd = _head_weight(W, fp32, s)
        loss = torch.empty(m, device=DEV)
        ws = torch.empty(_lib.size_query('noise_head_ce_workspace_size', m, T, V, fp32), device=DEV,
                         dtype=torch.uint8)
        _lib.call('noise_head_ce', xd.data_ptr(), 0, 0, wd.data_ptr(), V, fp32, ad.data_ptr(), bd.data_ptr(),
                  sd.data_ptr(), td.data_ptr(), 0, m, T, 0, _lib.CE_MEMBER_MEAN, loss.data_ptr(), None, ws.data_ptr(),
                  ws.numel(), None, 0, s)
        torch.cuda.synchronize()
        if fp32:
            ref = om.head_loss(h, W, a, b, sign, targets, 'fp32', 'fp32')
            assert (loss.cpu() - ref).abs().max() < 1e-4, (loss.cpu(), ref)
        else:
            ref = om.head_loss(h, W, a, b, sign, targets, 'bf16', 'bf16')
            assert (loss.cpu() - ref).abs().max() < 2e-4, (loss.cpu(), ref)


@pytest.mark.parametrize('fp32,T', [(f, t) for t in (96, 90) for f in HEAD_FORMATS])
def test_head_ce_other_vocab_and_partial_row_tile(fp32, T):
    """A 768-entry vocabulary (3 column tiles, 12 CE partials per row) and token counts that leave the last
    256-row tile partial: 96 (the normalised operand in TILE16) and 90 (not a multiple of 16: row-major)."""
    g = torch.Generator().manual_seed(14)
    m, V = 4, 768
    x = torch.randn(m * T, 512, generator=g) * 3
    W = torch.randn(V, 512, generator=g) * 512 ** -0.5 * 2
    a, b = torch.randn(m, V, generator=g), torch.randn(m, 512, generator=g)
    sign = torch.tensor([1e-2, -1e-2, 5e-2, -5e-2])
    targets = torch.randint(0, V, (T,), generator=g)
    s = torch.cuda.current_stream().cuda_stream
    h = om.norm(x.view(m, T, 512))
    xd, ad, bd, sd, td = (t.to(DEV) for t in (x, a, b, sign, targets))
    log_case(f'head_ce m={m} T={T} V={V} fp32_head={fp32}')
    wd = _head_weight(W, fp32, s)
    loss = torch.empty(m, device=DEV)
    ws = torch.empty(_lib.size_query('noise_head_ce_workspace_size', m, T, V, fp32), device=DEV, dtype=torch.uint8)
    _lib.call('noise_head_ce', xd.data_ptr(), 0, 0, wd.data_ptr(), V, fp32, ad.data_ptr(), bd.data_ptr(),
              sd.data_ptr(), td.data_ptr(), 0, m, T, 0, _lib.CE_MEMBER_MEAN, loss.data_ptr(), None, ws.data_ptr(),
              ws.numel(), None, 0, s)
    torch.cuda.synchronize()
    if fp32:
        ref = om.head_loss(h, W, a, b, sign, targets, 'fp32', 'fp32')
        assert (loss.cpu() - ref).abs().max() < 1e-4, (loss.cpu(), ref)
    else:
        ref = om.head_loss(h, W, a, b, sign, targets, 'bf16', 'bf16')
        assert (loss.cpu() - ref).abs().max() < 2e-4, (loss.cpu(), ref)


@pytest.mark.parametrize('fp32', HEAD_FORMATS)
def test_head_ce_tiled_and_row_major_operands_agree_bit_for_bit(fp32):
    """The head's whole-line path (operand rows in TILE16, weight in WTILE: rows in whole 16-row groups) and its
    row-major path (taken when T is not a multiple of 16) on the same 384 rows: 4 members x 96 tokens against 48
    members x 8 tokens whose per-member vectors repeat the original member's. Both stage the same LDS contents and
    contract in the same order, so the per-token losses are equal bit for bit."""
    g = torch.Generator().manual_seed(21)
    m, T, V, rep = 4, 96, 768, 12
    x = torch.randn(m * T, 512, generator=g) * 3
    W = torch.randn(V, 512, generator=g) * 512 ** -0.5 * 2
    a, b = torch.randn(m, V, generator=g), torch.randn(m, 512, generator=g)
    sign = torch.tensor([1e-2, -1e-2, 5e-2, -5e-2])
    tok = torch.randint(0, V, (m * T,), generator=g)
    s = torch.cuda.current_stream().cuda_stream
    xd, td = x.to(DEV), tok.to(DEV)
    wd = _head_weight(W, fp32, s)

    def run(members, t, a_, b_, sign_):
        log_case(f'head_ce members={members} T={t} fp32_head={fp32} per-token losses')
        ad, bd, sd = (v.contiguous().to(DEV) for v in (a_, b_, sign_))
        loss = torch.empty(members * t, device=DEV)
        ws = torch.empty(_lib.size_query('noise_head_ce_workspace_size', members, t, V, fp32), device=DEV,
                         dtype=torch.uint8)
        _lib.call('noise_head_ce', xd.data_ptr(), 0, 0, wd.data_ptr(), V, fp32, ad.data_ptr(), bd.data_ptr(),
                  sd.data_ptr(), td.data_ptr(), t, members, t, 0, _lib.CE_NONE, loss.data_ptr(), None, ws.data_ptr(),
                  ws.numel(), None, 0, s)
        torch.cuda.synchronize()
        return loss.cpu()

    tiled = run(m, T, a, b, sign)
    rows = run(m * rep, T // rep, a.repeat_interleave(rep, 0), b.repeat_interleave(rep, 0), sign.repeat_interleave(rep))
    assert torch.isfinite(tiled).all()
    assert torch.equal(tiled, rows), (tiled - rows).abs().max()


@pytest.mark.parametrize('fmt', [_lib.HEAD_FP32, _lib.HEAD_FP32_SPLIT])
def test_head_ce_config3_bf16_input_with_gain(fmt):
    """Config 3: bf16 hidden states, RMSNorm gain ~ U(0.9, 1.1), fp32 head with rank-1 perturbation."""
    g = torch.Generator().manual_seed(12)
    m, T, V = 4, 256, 4096
    h = torch.randn(m, T, 512, generator=g).bfloat16()
    gain = 0.9 + 0.2 * torch.rand(512, generator=g)
    W = torch.randn(V, 512, generator=g) * 512 ** -0.5
    a, b = torch.randn(m // 2, V, generator=g), torch.randn(m // 2, 512, generator=g)
    sign = antithetic_signs(m, 1e-3)
    _, targets = zipf_tokens(T, seed=13)
    s = torch.cuda.current_stream().cuda_stream
    hd, gd, ad, bd, sd, td = (t.to(DEV) for t in (h, gain, a, b, sign, targets))
    log_case(f'head_ce config3 m={m} T={T} fp32_head={fmt}')
    wd = _head_weight(W, fmt, s)
    loss = torch.empty(m, device=DEV)
    ws = torch.empty(_lib.size_query('noise_head_ce_workspace_size', m, T, V, fmt), device=DEV, dtype=torch.uint8)
    _lib.call('noise_head_ce', hd.data_ptr(), 1, gd.data_ptr(), wd.data_ptr(), V, fmt, ad.data_ptr(), bd.data_ptr(),
              sd.data_ptr(), td.data_ptr(), 0, m, T, 1, _lib.CE_MEMBER_MEAN, loss.data_ptr(), None, ws.data_ptr(),
              ws.numel(), None, 0, s)
    torch.cuda.synchronize()
    rep = lambda t: t.repeat_interleave(2, 0)  # noqa: E731
    ref = om.norm_head_ce(h.float(), gain, W, rep(a), rep(b), sign, targets)
    assert (loss.cpu() - ref).abs().max() < 1e-4, (loss.cpu(), ref)


def test_head_ce_fp32_format_logit_error_bound():
    """NOISE_HEAD_FP32 rounds h once to fp16 (relative error <= 2^-12 per element) and carries each weight row times
    a power of two as fp16 hi + lo (~22 significant bits), accumulating in fp32. Each capped logit then lies within
    2^-11 sum_i |h_i g_i W_vi| (plus a 1e-5 floor for the hardware exp and reciprocal of the cap) of the fp32 oracle's,
    whatever the row's magnitude: here rows scaled by 10^-7 .. 10^1 (the reference init's lm_head is ~1e-6; the
    largest rows push logits far past the cap), a gain, and per-member rank-1 terms. A token's loss
    logsumexp(z') - z'_target then moves by at most twice its largest logit error, which bounds each member's mean.
    (At model-scale weights the members agree within 1e-4: the other head tests.)"""
    g = torch.Generator().manual_seed(31)
    m, T, V = 4, 64, 1024
    x = torch.randn(m * T, 512, generator=g) * 3
    gain = 0.5 + 1.5 * torch.rand(512, generator=g)
    rows = 10.0 ** (-7 + 8 * torch.rand(V, 1, generator=g))
    # the scale's edge cases: an all-zero row (scale 1), a 1e-30 row (the largest scale), a 1e20 row (logits far past
    # the cap: z' = +-15)
    rows[0], rows[1], rows[2] = 0.0, 1e-30, 1e20
    W = torch.randn(V, 512, generator=g) * 512 ** -0.5 * 2 * rows
    a, b = torch.randn(m, V, generator=g), torch.randn(m, 512, generator=g)
    sign = torch.tensor([1e-2, -1e-2, 5e-2, -5e-2])
    targets = torch.randint(0, V, (T,), generator=g)
    s = torch.cuda.current_stream().cuda_stream
    xd, gd, ad, bd, sd, td = (t.to(DEV) for t in (x, gain, a, b, sign, targets))
    wd = _head_weight(W, _lib.HEAD_FP32, s)
    log_case(f'head_ce fp32 format logits m={m} T={T} V={V}')
    loss, logits = torch.empty(m, device=DEV), torch.empty(m * T, V, device=DEV)
    ws = torch.empty(_lib.size_query('noise_head_ce_workspace_size', m, T, V, _lib.HEAD_FP32), device=DEV,
                     dtype=torch.uint8)
    _lib.call('noise_head_ce', xd.data_ptr(), 0, gd.data_ptr(), wd.data_ptr(), V, _lib.HEAD_FP32, ad.data_ptr(),
              bd.data_ptr(), sd.data_ptr(), td.data_ptr(), 0, m, T, 0, _lib.CE_MEMBER_MEAN, loss.data_ptr(),
              logits.data_ptr(), ws.data_ptr(), ws.numel(), None, 0, s)
    torch.cuda.synchronize()
    hn = om.norm(x.view(m, T, 512)) * gain
    z = om.lowrank(hn, W, a, b, sign, 'fp32')
    ref = 15 * torch.tanh(z / 15)
    bound = 2.0 ** -11 * (hn.abs() @ W.abs().t()) + 1e-5 + 1e-5 * z.abs()
    got = logits.cpu().view(m, T, V)
    assert torch.isfinite(got).all()
    err = (got - ref).abs()
    assert (err <= bound).all(), (err - bound).max()
    # the 1e20 row saturates the cap (15 log2(e) ln(2) in fp32: within an ulp of 15)
    assert ((got[..., 2].abs() - 15.0).abs() < 1e-5).all()
    # the bound is not vacuous: the largest rows' logits are O(1) and their errors well above the fp32 floor
    assert ref.abs().max() > 1 and err.max() > 1e-6
    ref_loss = om.head_loss(om.norm(x.view(m, T, 512)) * gain, W, a, b, sign, targets, 'fp32', 'fp32')
    loss_bound = 2 * bound.amax(-1).mean(-1) + 1e-6
    assert ((loss.cpu() - ref_loss).abs() <= loss_bound).all(), (loss.cpu() - ref_loss, loss_bound)


# ---------------------------------------------------------------- whole population forward

def _population_case(model, params, P, T, sigma, seed, head='fp32'):
    from noise_amd.population import Population
    shapes = {n: tuple(t.shape) for n, t in params.items()}
    noise = population_noise(shapes, P // 2, seed=seed)
    sign = antithetic_signs(P, sigma)
    idx, tgt = zipf_tokens(T, seed=seed + 1)
    gm = _gpu_model(model)
    gp = dict(gm.named_parameters())
    pop = Population(gm, chunk=P, head=head)
    got = pop.loss(gp, _dev(noise), sign.to(DEV), idx.to(DEV), tgt.to(DEV)).cpu()
    return got, noise, sign, idx, tgt


def _oracle_with_floor(params, noise, sign, idx, tgt, return_alts=False, head='fp32'):
    """bf16-mode oracle losses, and how far they move under three equally valid changes of rounding: every
    GEMM accumulating in fp64 instead of fp32, attention computed in fp64, and attention at TF32-class
    precision (q, k, v and the probabilities rounded to fp16, the reference's TF32 flex attention's
    significand). The largest move (per loss and per antithetic difference) is the floor: at trained-scale
    weights the bf16 path is chaotic, and one alternative alone under-samples how far valid roundings diverge
    (the CPU oracle's own results also shift with the host's summation order)."""
    ref = om.population_loss(params, noise, sign, idx, tgt, mode='bf16', head=head)
    orig_attn = om.attention

    def attention_p16(q, k, v, window, dtype=torch.float32):
        # q, k, v and the probabilities rounded to fp16 (11-bit significand, the precision class of the
        # reference's TF32 flex attention); normalised by the sum of the rounded probabilities
        B, T, H, D = q.shape
        qh, kh, vh = (t.transpose(1, 2).half().float() for t in (q, k, v))
        scores = qh @ kh.transpose(-1, -2) / math.sqrt(D)
        pos = torch.arange(T)
        mask = (pos[:, None] >= pos[None, :]) & (pos[:, None] - pos[None, :] <= window)
        scores = scores.masked_fill(~mask, float('-inf'))
        p = torch.exp(scores - scores.amax(-1, keepdim=True)).half().float()
        return ((p @ vh) / p.sum(-1, keepdim=True)).transpose(1, 2).to(q.dtype)

    alts = []
    for variant in (lambda q, k, v, window, dtype=torch.float32: orig_attn(q, k, v, window, torch.float64),
                    attention_p16):
        om.attention = variant
        try:
            alts.append(om.population_loss(params, noise, sign, idx, tgt, mode='bf16', head=head))
        finally:
            om.attention = orig_attn
    orig = om.lowrank

    def lowrank64(x, weight, a, b, s, mode='fp32'):
        if mode == 'fp32':
            return orig(x, weight, a, b, s, mode)
        u = om.bf((om.bf(x).double() @ om.bf(b).double().unsqueeze(-1)).float())
        dense = om.bf((om.bf(x).double() @ om.bf(weight).double().t()).float())
        return dense + s[:, None, None] * u * a[:, None, :]

    om.lowrank = lowrank64
    try:
        alt = om.population_loss(params, noise, sign, idx, tgt, mode='bf16', head=head)
    finally:
        om.lowrank = orig
    floor = max(float((a - ref).abs().max()) for a in (alt, *alts))
    pair_floor = max(float(((a[1::2] - a[0::2]) - (ref[1::2] - ref[0::2])).abs().max()) for a in (alt, *alts))
    if return_alts:
        return ref, floor, pair_floor, [alt, *alts]
    return ref, floor, pair_floor


@pytest.mark.parametrize('head', ['fp32', 'bf16'])
def test_population_loss_config0_at_reference_init(head):
    """Config 0 (P = 8, T = 256, sigma = 1e-3) on the reference's seed-0 weights: losses and the
    antithetic differences within 1e-4 of the bf16-mode oracle, with the fp32 head and with the reference's
    autocast (bf16) head that `bench.py --head bf16` times."""
    model = make_model('cpu', 0)
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    P, T = 8, 256
    log_case(f'population_loss P={P} T={T} reference init head={head}')
    got, noise, sign, idx, tgt = _population_case(model, params, P, T, 1e-3, seed=11, head=head)
    ref = om.population_loss(params, noise, sign, idx, tgt, mode='bf16', head=head)
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max() < 1e-4, (got, ref)
    dg, dr = got[1::2] - got[0::2], ref[1::2] - ref[0::2]
    assert (dg - dr).abs().max() < 1e-4, (dg, dr)


def test_population_loss_config4_full_size_sampled_members():
    """Config 4 at its real shape: 3072 members (1536 antithetic pairs, per-pair noise rows) on one 2048-token
    Zipf sequence at the reference's initialisation, in 1024-member passes. Every loss is finite and near
    ln 4096 (the init's head is N(0, 1e-6)); four members (both ends of the population, both signs) match
    the bf16-mode oracle within the 1e-4 loss bar, and so do their antithetic differences."""
    from noise_amd.population import Population
    model = make_model('cpu', 0)
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    pairs, T = 1536, 2048
    P = 2 * pairs
    log_case(f'population_loss config4 P={P} T={T} (1024-member passes)')
    shapes = {n: tuple(t.shape) for n, t in params.items()}
    noise = population_noise(shapes, pairs, seed=71, per_member=False)
    sign = antithetic_signs(P, 1e-3)
    idx, tgt = zipf_tokens(T, seed=72)
    gm = _gpu_model(model)
    got = Population(gm, chunk=1024).loss(dict(gm.named_parameters()), _dev(noise), sign.to(DEV), idx.to(DEV),
                                          tgt.to(DEV), pair_shift=1).cpu()
    assert got.shape == (P,) and torch.isfinite(got).all()
    assert (got - math.log(4096)).abs().max() < 0.05
    members = [0, 1, P - 2, P - 1]
    rows = [m // 2 for m in members]
    sub = {n: tuple(t[rows] for t in v) if isinstance(v, tuple) else v[rows] for n, v in noise.items()}
    ref = om.population_loss(params, sub, sign[members], idx, tgt, mode='bf16', head='fp32')
    assert (got[members] - ref).abs().max() < 1e-4, (got[members], ref)
    dg, dr = got[members][1::2] - got[members][0::2], ref[1::2] - ref[0::2]
    assert (dg - dr).abs().max() < 1e-4, (dg, dr)


@pytest.mark.parametrize('head', ['fp32', 'bf16'])
def test_population_loss_trained_weights_within_rounding_floor(trained, head):
    """Trained-scale weights, with the fp32 head and with the autocast (bf16) head: within twice the oracle's
    rounding floor (measured in the test) plus 1e-4."""
    model, params = trained
    P, T = 8, 256
    log_case(f'population_loss P={P} T={T} trained-scale weights head={head}')
    got, noise, sign, idx, tgt = _population_case(model, params, P, T, 1e-3, seed=11, head=head)
    ref, floor, pair_floor = _oracle_with_floor(params, noise, sign, idx, tgt, head=head)
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max() <= 2 * floor + 1e-4, (got, ref, floor)
    dg, dr = got[1::2] - got[0::2], ref[1::2] - ref[0::2]
    assert (dg - dr).abs().max() <= 2 * pair_floor + 1e-4, (dg, dr, pair_floor)


def test_population_loss_large_sigma_and_chunking(trained):
    """sigma = 0.05 makes every rank-1 term matter; two chunks exercise the chunk slicing."""
    from noise_amd.population import Population
    model, params = trained
    P, T = 8, 128
    log_case(f'population_loss P={P} T={T} sigma=0.05 chunked')
    shapes = {n: tuple(t.shape) for n, t in params.items()}
    noise = population_noise(shapes, P // 2, seed=21)
    sign = antithetic_signs(P, 0.05)
    idx, tgt = zipf_tokens(T, seed=22)
    gm = _gpu_model(model)
    pop = Population(gm, chunk=4)
    got = pop.loss(dict(gm.named_parameters()), _dev(noise), sign.to(DEV), idx.to(DEV), tgt.to(DEV)).cpu()
    ref, floor, _ = _oracle_with_floor(params, noise, sign, idx, tgt)
    # one alternative summation order samples the chaotic spread once; at sigma = 0.05 allow 3x
    assert (got - ref).abs().max() <= 3 * floor + 1e-4, (got, ref, floor)
    assert (got[0] - got[1]).abs() > 1e-3


def test_population_loss_pair_shift_equals_per_member(trained):
    """Per-direction noise with pair_shift = 1 gives the same losses as the repeated per-member noise."""
    from noise_amd.population import Population
    model, params = trained
    P, T = 8, 128
    log_case(f'population_loss pair_shift P={P} T={T}')
    shapes = {n: tuple(t.shape) for n, t in params.items()}
    per_dir = population_noise(shapes, P // 2, seed=31, per_member=False)
    per_mem = {n: tuple(t.repeat_interleave(2, 0) for t in v) if isinstance(v, tuple) else v.repeat_interleave(2, 0)
               for n, v in per_dir.items()}
    sign = antithetic_signs(P, 1e-3).to(DEV)
    idx, tgt = (t.to(DEV) for t in zipf_tokens(T, seed=32))
    gm = _gpu_model(model)
    gp = dict(gm.named_parameters())
    pop = Population(gm, chunk=P)
    a = pop.loss(gp, _dev(per_dir), sign, idx, tgt, pair_shift=1)
    b = pop.loss(gp, _dev(per_mem), sign, idx, tgt, pair_shift=0)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), b.cpu())


def test_population_loss_golden_reference_fp32(golden):
    """The kernels against the reference's own fp32 CPU losses (tests/golden) at trained-scale weights: the
    difference is the bf16 rounding of the autocast GEMMs. Bound: twice the gap between the bf16 rounding class
    and those fp32 losses, plus 1e-4. The gap is measured here as the largest distance from the golden losses of
    the bf16-mode oracle (fp32 attention operands, as the reference) and of its three alternative roundings
    (2.0e-3 .. 2.5e-3 on losses, 1.8e-3 .. 2.2e-3 on antithetic differences on the build host; the CPU's own
    summation order moves each by ~1e-3)."""
    model = trained_like(make_model('cpu', 0))
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    P, T = 2 * golden['pairs'], golden['T']
    log_case(f'population_loss vs golden P={P} T={T}')
    shapes = {n: tuple(t.shape) for n, t in params.items()}
    noise = population_noise(shapes, golden['pairs'])
    sign = antithetic_signs(P, golden['sigma'])
    idx, tgt = zipf_tokens(T)
    gm = _gpu_model(model)
    from noise_amd.population import Population
    got = Population(gm, chunk=P).loss(dict(gm.named_parameters()), _dev(noise), sign.to(DEV), idx.to(DEV),
                                       tgt.to(DEV)).cpu()
    ref = torch.tensor(golden['losses_trained'])
    b16, _, _, alts = _oracle_with_floor(params, noise, sign, idx, tgt, return_alts=True)
    dg, dr = got[1::2] - got[0::2], ref[1::2] - ref[0::2]
    gap = max(float((x - ref).abs().max()) for x in (b16, *alts))
    pair_gap = max(float(((x[1::2] - x[0::2]) - dr).abs().max()) for x in (b16, *alts))
    assert gap < 5e-3 and pair_gap < 5e-3, (gap, pair_gap)
    assert (got - ref).abs().max() <= 2 * gap + 1e-4, (got, ref, gap)
    assert (dg - dr).abs().max() <= 2 * pair_gap + 1e-4, (dg, dr, pair_gap)


def _spearman(a, b):
    ra = torch.argsort(torch.argsort(a)).double()
    rb = torch.argsort(torch.argsort(b)).double()
    ra, rb = ra - ra.mean(), rb - rb.mean()
    return float((ra @ rb) / (ra.norm() * rb.norm()))


@pytest.mark.timeout(600)
def test_es_signal_survives_at_trained_scale(trained):
    """At trained-scale weights a 1e-4 bar on losses cannot hold (equally valid roundings move them by ~3e-3), so
    this checks what the update consumes (train/val/eggroll.py:151-163): 64 antithetic pairs at T = 256.
    - The pair differences L(theta - sE) - L(theta + sE) rank like the oracle's: 1 - Spearman(GPU, oracle) at
      most 1.5x the oracle's own disagreement with its alternative roundings (fp64 GEMM accumulation; TF32-class
      fp16 attention).
    - Every pair whose oracle difference exceeds twice the pair floor has the same sign on the GPU.
    - The update -sum_j w_j a_j b_j^T / n built on the GPU (z-score fitness + grouped outer products) from the GPU
      losses points where the oracle's does from the oracle losses: cosine >= 0.99 for lm_head and a c_fc."""
    from noise_amd.population import Population
    from oracle import eggroll as oe_
    model, params = trained
    pairs, T = 64, 256
    P = 2 * pairs
    log_case(f'ES signal pairs={pairs} T={T} trained-scale weights')
    shapes = {n: tuple(t.shape) for n, t in params.items()}
    per_dir = population_noise(shapes, pairs, seed=41, per_member=False)
    per_mem = {n: tuple(t.repeat_interleave(2, 0) for t in v) if isinstance(v, tuple) else v.repeat_interleave(2, 0)
               for n, v in per_dir.items()}
    sign = antithetic_signs(P, 1e-3)
    idx, tgt = zipf_tokens(T, seed=42)
    gm = _gpu_model(model)
    dnoise = _dev(per_dir)
    got = Population(gm, chunk=P).loss(dict(gm.named_parameters()), dnoise, sign.to(DEV), idx.to(DEV),
                                       tgt.to(DEV), pair_shift=1)
    s = torch.cuda.current_stream().cuda_stream
    fit = torch.empty(pairs, device=DEV)
    w = torch.empty(pairs, device=DEV)
    _lib.call('noise_fitness', got.data_ptr(), P, pairs, _lib.FITNESS_ZSCORE, fit.data_ptr(), w.data_ptr(), s)
    names = ['lm_head.weight', 'transformer.h.3.mlp.c_fc.weight']
    upd = {}
    for n in names:
        a, b = dnoise[n]
        upd[n] = torch.empty(a.shape[1], b.shape[1], device=DEV)
        _lib.call('noise_outer_update', a.data_ptr(), a.shape[1], b.data_ptr(), b.shape[1], w.data_ptr(), pairs,
                  a.shape[1], b.shape[1], -1.0 / pairs, upd[n].data_ptr(), s)
    torch.cuda.synchronize()
    got = got.cpu()
    log_case('ES signal: oracle and its alternative roundings')
    ref, _, pair_floor, alts = _oracle_with_floor(params, per_mem, sign, idx, tgt, return_alts=True)
    dg, dr = got[1::2] - got[0::2], ref[1::2] - ref[0::2]
    rho = _spearman(dg, dr)
    rho_alt = [_spearman(a[1::2] - a[0::2], dr) for a in alts]
    assert 1 - rho <= 1.5 * max(1 - r for r in rho_alt) + 1e-4, (rho, rho_alt)
    big = dr.abs() > 2 * pair_floor
    assert int(big.sum()) >= pairs // 2, (int(big.sum()), pair_floor)
    assert torch.equal(torch.sign(dg[big]), torch.sign(dr[big]))
    _, w_ref = oe_.fitness(ref, pairs)
    ref_upd = oe_.update(w_ref, {n: per_dir[n] for n in names}, pairs)
    for n in names:
        a_, b_ = upd[n].cpu().flatten(), ref_upd[n].flatten()
        cos = float(a_ @ b_ / (a_.norm() * b_.norm()))
        assert cos >= 0.99, (n, cos)


# ---------------------------------------------------------------- update path

def test_noise_gather_rows_equal_buffer_slices():
    """Eggroll.noise on the library's grouped gather equals the reference's indexing of the buffer
    (train/val/eggroll.py:122-128, restated in oracle.eggroll.gather_noise) bit for bit, for every parameter,
    repeated and unordered directions included; a direction outside [0, pairs) yields NaN rows."""
    from noise_amd.eggroll import Eggroll
    model = make_model(DEV, 0)
    pairs = 6
    es = Eggroll(model, pairs, chunk=4, noise_len=1 << 20, chunk_pairs=1)
    offs = es.offsets(3)
    dirs = torch.tensor([0, 5, 2, 2, 4], device=DEV)
    log_case('noise gather rows')
    got = es.noise(offs, dirs)
    shapes = {n: tuple(p.shape) for n, p in es.params.items()}
    ref = oe.gather_noise(es.buffer.cpu(), {n: o.cpu() for n, o in offs.items()}, shapes, dirs.cpu())
    torch.cuda.synchronize()
    for n, shape in shapes.items():
        if len(shape) == 2:
            assert torch.equal(got[n][0].cpu(), ref[n][0]) and torch.equal(got[n][1].cpu(), ref[n][1]), n
        else:
            assert torch.equal(got[n].cpu(), ref[n]), n
    bad = es.noise(offs, torch.tensor([pairs, -1], device=DEV))
    torch.cuda.synchronize()
    assert torch.isnan(bad['lm_head.weight'][0]).all() and torch.isnan(bad['resid_lambdas']).all()


def test_fitness_update_adam_match_oracle():
    g = torch.Generator().manual_seed(7)
    pairs, nl = 6, 24
    losses = torch.randn(nl, generator=g) * 0.01 + 5
    s = torch.cuda.current_stream().cuda_stream
    log_case(f'fitness n={nl} pairs={pairs}')
    fit = torch.empty(nl // 2, device=DEV)
    w = torch.empty(pairs, device=DEV)
    ld = losses.to(DEV)
    _lib.call('noise_fitness', ld.data_ptr(), nl, pairs, 0, fit.data_ptr(), w.data_ptr(), s)
    f_ref, w_ref = oe.fitness(losses, pairs)
    torch.cuda.synchronize()
    assert torch.allclose(fit.cpu(), f_ref, atol=1e-5)
    assert torch.allclose(w.cpu(), w_ref, atol=1e-5)
    # rank mode: a permutation of centred ranks
    _lib.call('noise_fitness', ld.data_ptr(), nl, pairs, 1, fit.data_ptr(), w.data_ptr(), s)
    torch.cuda.synchronize()
    fr, wr = oe.rank_fitness(losses, pairs)
    assert torch.allclose(fit.cpu(), fr, atol=1e-6)
    assert torch.allclose(w.cpu(), wr, atol=1e-6)

    log_case('outer_update')
    out_d, in_d = 70, 130
    a, b = torch.randn(pairs, out_d, generator=g), torch.randn(pairs, in_d, generator=g)
    eps = torch.randn(pairs, 8, generator=g)
    grad = torch.empty(out_d, in_d, device=DEV)
    ad, bd, wd, ed = (t.to(DEV) for t in (a, b, w_ref, eps))
    _lib.call('noise_outer_update', ad.data_ptr(), out_d, bd.data_ptr(), in_d, wd.data_ptr(), pairs, out_d, in_d,
              -1.0 / (nl // 2), grad.data_ptr(), s)
    gl = torch.empty(1, 8, device=DEV)
    _lib.call('noise_outer_update', 0, 0, ed.data_ptr(), 8, wd.data_ptr(), pairs, 1, 8, -1.0 / (nl // 2),
              gl.data_ptr(), s)
    ref = oe.update(w_ref, {'m': (a, b), 'l': eps}, nl // 2)
    torch.cuda.synchronize()
    assert torch.allclose(grad.cpu(), ref['m'], atol=1e-5)
    assert torch.allclose(gl.cpu()[0], ref['l'], atol=1e-6)

    log_case('outer_update_batch')
    # several matrices in one launch, including partial 64 x 64 tiles, a multi-chunk direction count and the
    # scalar (a null) form: each equals the single-matrix result bit for bit and the oracle's update
    nd = 75
    wb = torch.randn(nd, generator=g)
    shapes = [(70, 130), (64, 64), (1, 8), (200, 33), (512, 512)]
    host = {}
    for k, (o, i) in enumerate(shapes):
        host[k] = (None if o == 1 else torch.randn(nd, o, generator=g), torch.randn(nd, i, generator=g))
    dev_ = {k: (None if a_ is None else a_.to(DEV), b_.to(DEV)) for k, (a_, b_) in host.items()}
    wbd = wb.to(DEV)
    grads_b = {k: torch.empty(o, i, device=DEV) for k, (o, i) in enumerate(shapes)}
    grads_s = {k: torch.empty(o, i, device=DEV) for k, (o, i) in enumerate(shapes)}
    mats = []
    for k, (o, i) in enumerate(shapes):
        a_, b_ = dev_[k]
        mats.append((0 if a_ is None else a_.data_ptr(), 0 if a_ is None else o, b_.data_ptr(), i, o, i,
                     grads_b[k].data_ptr()))
        _lib.call('noise_outer_update', 0 if a_ is None else a_.data_ptr(), 0 if a_ is None else o, b_.data_ptr(), i,
                  wbd.data_ptr(), nd, o, i, -0.5, grads_s[k].data_ptr(), s)
    ptr, count, _keep = _lib.outer_mats(mats)
    _lib.call('noise_outer_update_batch', ptr, count, wbd.data_ptr(), nd, -0.5, s)
    torch.cuda.synchronize()
    for k, (o, i) in enumerate(shapes):
        assert torch.equal(grads_b[k].cpu(), grads_s[k].cpu())
        a_, b_ = host[k]
        ref_k = oe.update(wb, {'m': (a_, b_) if a_ is not None else b_}, 2)['m']
        ref_k = ref_k.reshape(o, i)
        assert torch.allclose(grads_b[k].cpu(), ref_k, atol=1e-4, rtol=1e-5), k

    log_case('adam')
    p0 = torch.randn(1000, generator=g)
    param, m_, v_ = p0.clone().to(DEV), torch.zeros(1000, device=DEV), torch.zeros(1000, device=DEV)
    ref_p = p0.clone()
    opt = torch.optim.AdamW([ref_p], lr=1e-3, betas=(0.5, 0.95), eps=1e-8, weight_decay=0.0)
    for step in range(1, 4):
        gr = torch.randn(1000, generator=g)
        ref_p.grad = gr.clone()
        opt.step()
        grd = gr.to(DEV)
        _lib.call('noise_adam', param.data_ptr(), grd.data_ptr(), m_.data_ptr(), v_.data_ptr(), 1000,
                  1e-3 / (1 - 0.5 ** step), 0.5, 0.95, 1e-8, math.sqrt(1 - 0.95 ** step), s)
        torch.cuda.synchronize()
    assert torch.allclose(param.cpu(), ref_p, atol=1e-6, rtol=1e-6)

    log_case('adam_batch')
    # several tensors (one above the 64-tensor launch limit, ragged sizes) in one call equal noise_adam per tensor
    sizes = [1000, 1, 257, 4096 * 3 + 5] + [33] * 62
    ps = [torch.randn(n, generator=g) for n in sizes]
    gs = [torch.randn(n, generator=g) for n in sizes]
    single = [(p_.clone().to(DEV), torch.zeros(n, device=DEV), torch.zeros(n, device=DEV)) for p_, n in zip(ps, sizes)]
    batch = [(p_.clone().to(DEV), torch.zeros(n, device=DEV), torch.zeros(n, device=DEV)) for p_, n in zip(ps, sizes)]
    gd = [g_.to(DEV) for g_ in gs]
    for step in range(1, 3):
        ss, bc = 1e-3 / (1 - 0.5 ** step), math.sqrt(1 - 0.95 ** step)
        for (pp, mm, vv), g_, n in zip(single, gd, sizes):
            _lib.call('noise_adam', pp.data_ptr(), g_.data_ptr(), mm.data_ptr(), vv.data_ptr(), n, ss, 0.5, 0.95, 1e-8,
                      bc, s)
        ptr, count, _keep = _lib.adam_tensors([(pp.data_ptr(), g_.data_ptr(), mm.data_ptr(), vv.data_ptr(), n, ss, bc)
                                               for (pp, mm, vv), g_, n in zip(batch, gd, sizes)])
        _lib.call('noise_adam_batch', ptr, count, 0.5, 0.95, 1e-8, s)
    torch.cuda.synchronize()
    for a_, b_ in zip(single, batch):
        for x_, y_ in zip(a_, b_):
            assert torch.equal(x_.cpu(), y_.cpu())


def test_fitness_at_the_reference_population():
    """noise_fitness at the reference's population (131,072 pairs, train/val/eggroll.py:30): rank mode (spread over
    the GPU) equals the oracle's centred ranks bit for bit, with many ties (losses on a coarse grid); z-score mode
    matches the oracle's within fp32 summation order."""
    from oracle import eggroll as oe_
    pairs = 131072
    g = torch.Generator().manual_seed(17)
    losses = 5 + torch.randint(0, 2000, (2 * pairs,), generator=g).float() * 1e-3  # a 1e-3 grid: ties
    ld = losses.to(DEV)
    s = torch.cuda.current_stream().cuda_stream
    fit = torch.empty(pairs, device=DEV)
    w = torch.empty(pairs, device=DEV)
    log_case(f'rank fitness pairs={pairs}')
    _lib.call('noise_fitness', ld.data_ptr(), 2 * pairs, pairs, _lib.FITNESS_RANK, fit.data_ptr(), w.data_ptr(), s)
    torch.cuda.synchronize()
    fr, wr = oe_.rank_fitness(losses, pairs)
    assert torch.equal(fit.cpu(), fr)
    assert torch.equal(w.cpu(), wr)
    log_case(f'zscore fitness pairs={pairs}, folded onto {pairs // 4} directions')
    w4 = torch.empty(pairs // 4, device=DEV)
    _lib.call('noise_fitness', ld.data_ptr(), 2 * pairs, pairs // 4, _lib.FITNESS_ZSCORE, fit.data_ptr(),
              w4.data_ptr(), s)
    torch.cuda.synchronize()
    fz, wz = oe_.fitness(losses, pairs // 4)
    assert torch.allclose(fit.cpu(), fz, rtol=1e-5, atol=1e-6)
    assert torch.allclose(w4.cpu(), wz, rtol=1e-5, atol=1e-5)


def test_eggroll_step_eight_sequences_reference_chunk_layout():
    """Eggroll.step with BATCH = 8 sequences (train/val/eggroll.py:28) and the reference's chunk layout scaled
    down: 24 pairs, CHUNK = 4 pairs, so per_seq = 6 members and the chunks of 8 members start at 0, 8, ..., 40 and
    run on sequences 0, 1, 2, 4, 5, 6 (:139-145), as 1536 pairs in chunks of 256 do at full size. Kernel passes of
    16 members (each gathering only its own directions' noise) cut across those chunks. Every member's loss within
    1e-4 of the bf16-mode oracle on its chunk's sequence and the reference's noise slices; the gradient estimate
    from those losses against the oracle's."""
    from noise_amd.eggroll import Eggroll
    from noise_amd.optim import Adam
    pairs, batch, cp, T, step = 24, 8, 4, 256, 5
    model = make_model(DEV, 0)
    before = {n: p.detach().cpu().clone() for n, p in model.named_parameters()}
    shapes = {n: tuple(p.shape) for n, p in before.items()}
    seqs = [zipf_tokens(T, seed=40 + i) for i in range(batch)]
    x = torch.stack([s_[0] for s_ in seqs]).to(DEV)
    y = torch.stack([s_[1] for s_ in seqs]).to(DEV)
    es = Eggroll(model, pairs, chunk=16, noise_len=1 << 20, sigma=oe.SIGMA, chunk_pairs=cp)
    opt = Adam(model.parameters(), lr=oe.LR, betas=oe.BETAS, eps=oe.ADAM_EPS)
    log_case(f'Eggroll.step pairs={pairs} sequences={batch} chunk_pairs={cp} T={T}')
    es.step(x, y, opt, step)
    torch.cuda.synchronize()
    losses = es.last_losses.cpu()
    members = 2 * pairs
    seq_of = oe.chunk_sequences(members, members // batch, cp)
    assert sorted(set(seq_of.tolist())) == [0, 1, 2, 4, 5, 6]
    buf = es.buffer.cpu()
    offs = {n: o.cpu() for n, o in es.offsets(step).items()}
    for start in range(0, members, 2 * cp):
        sq = int(seq_of[start])
        dirs = oe.member_directions(start, cp, pairs)
        g_ = oe.gather_noise(buf, offs, shapes, dirs)
        noise = {n: tuple(t.repeat_interleave(2, 0) for t in v) if isinstance(v, tuple) else v.repeat_interleave(2, 0)
                 for n, v in g_.items()}
        sign = torch.tensor([oe.SIGMA, -oe.SIGMA]).repeat(cp)
        ref = om.population_loss(before, noise, sign, seqs[sq][0], seqs[sq][1], mode='bf16', head='fp32')
        got = losses[start:start + 2 * cp]
        assert (got - ref).abs().max() < 1e-4, (start, sq, got, ref)
    f, w = oe.fitness(losses, pairs)
    grads = oe.update(w, oe.gather_noise(buf, offs, shapes, torch.arange(pairs)), len(f))
    for n, p in model.named_parameters():
        g_ref = grads[n].reshape(p.shape)
        assert torch.allclose(p.grad.detach().cpu(), g_ref, atol=1e-6 * float(g_ref.abs().max()) + 1e-12,
                              rtol=1e-4), n


@pytest.mark.timeout(900)
def test_eggroll_step_at_the_reference_population():
    """One whole Eggroll.step at the reference's own population (train/val/eggroll.py:28-34): PAIRS = 131,072 antithetic
    pairs (262,144 members), BATCH = 8 sequences, CHUNK = 256, the full 2^28 noise buffer, at T = 128 tokens (the
    population machinery is what this exercises; T only scales the forward). 16 kernel passes of 16,384 members, each
    gathering its own noise rows; the update walks the directions 256 at a time. Checks: every loss finite and near
    ln 4096 at the reference init; sampled members of several chunks and sequences within 1e-4 of the oracle on their
    chunk's sequence; the z-score fitness of all 131,072 pairs and the gradients of the mixing scalars and of one
    ve_gate weight against the oracle's composition from the same losses and noise."""
    from noise_amd.eggroll import Eggroll, PAIRS, BATCH, CHUNK
    from noise_amd.optim import Adam
    pairs, T, step = PAIRS, 128, 7
    model = make_model(DEV, 0)
    before = {n: p.detach().cpu().clone() for n, p in model.named_parameters()}
    shapes = {n: tuple(p.shape) for n, p in before.items()}
    seqs = [zipf_tokens(T, seed=60 + i) for i in range(BATCH)]
    x = torch.stack([s_[0] for s_ in seqs]).to(DEV)
    y = torch.stack([s_[1] for s_ in seqs]).to(DEV)
    es = Eggroll(model, pairs, chunk=16384, sigma=oe.SIGMA)
    opt = Adam(model.parameters(), lr=oe.LR, betas=oe.BETAS, eps=oe.ADAM_EPS)
    log_case(f'Eggroll.step pairs={pairs} sequences={BATCH} T={T} (reference population)')
    es.step(x, y, opt, step)
    torch.cuda.synchronize()
    losses = es.last_losses.cpu()
    members = 2 * pairs
    assert losses.shape == (members,) and torch.isfinite(losses).all()
    # the init's head keeps every member near ln 4096 (262,144 draws reach ~0.08 away at sigma = 2e-3)
    assert (losses - math.log(4096)).abs().max() < 0.25
    seq_of = oe.chunk_sequences(members, members // BATCH, CHUNK)
    offs = {n: o.cpu() for n, o in es.offsets(step).items()}
    log_case('reference population: oracle on sampled members')
    buf = es.buffer.cpu()
    for m in (0, 1, 2 * CHUNK + 6, members // 2 + 3, members - 2):
        m0 = m - m % 2
        dirs = oe.member_directions(m0, 1, pairs)
        g_ = oe.gather_noise(buf, offs, shapes, dirs)
        noise = {n: tuple(t.repeat_interleave(2, 0) for t in v) if isinstance(v, tuple) else v.repeat_interleave(2, 0)
                 for n, v in g_.items()}
        sq = int(seq_of[m0])
        ref = om.population_loss(before, noise, torch.tensor([oe.SIGMA, -oe.SIGMA]), seqs[sq][0], seqs[sq][1],
                                 mode='bf16', head='fp32')
        assert (losses[m0:m0 + 2] - ref).abs().max() < 1e-4, (m0, sq, losses[m0:m0 + 2], ref)
    f, w = oe.fitness(losses, pairs)
    small = {n: s_ for n, s_ in shapes.items() if n in ('resid_lambdas', 'x0_lambdas', 'transformer.h.1.attn.ve_gate.weight')}
    grads = oe.update(w, oe.gather_noise(buf, {n: offs[n] for n in small}, small, torch.arange(pairs)), len(f))
    params = dict(model.named_parameters())
    for n in small:
        g_ref = grads[n].reshape(params[n].shape)
        g_got = params[n].grad.detach().cpu()
        assert torch.allclose(g_got, g_ref, atol=1e-4 * float(g_ref.abs().max()) + 1e-9, rtol=1e-3), n
    del es
    torch.cuda.empty_cache()


def test_eggroll_step_two_sequences_matches_oracle():
    """One whole `Eggroll.step` on the GPU (train/val/eggroll.py:130-168) with two sequences of 256 tokens and
    4 antithetic pairs (8 members, 4 per sequence, all in one pass through per-member token rows) at the
    reference's initialisation: member losses within 1e-4 of the bf16-mode oracle on the reference's noise
    slices; then fitness, update and Adam from those losses against the oracle's composition
    (torch.optim.AdamW semantics, weight decay 0)."""
    from noise_amd.eggroll import Eggroll
    from noise_amd.optim import Adam
    pairs, T, step = 4, 256, 3
    model = make_model(DEV, 0)
    before = {n: p.detach().cpu().clone() for n, p in model.named_parameters()}
    shapes = {n: tuple(p.shape) for n, p in before.items()}
    seqs = [zipf_tokens(T, seed=21), zipf_tokens(T, seed=22)]
    x = torch.stack([s_[0] for s_ in seqs]).to(DEV)
    y = torch.stack([s_[1] for s_ in seqs]).to(DEV)
    es = Eggroll(model, pairs, chunk=8, noise_len=1 << 20, sigma=oe.SIGMA, chunk_pairs=2)
    opt = Adam(model.parameters(), lr=oe.LR, betas=oe.BETAS, eps=oe.ADAM_EPS)
    log_case(f'Eggroll.step pairs={pairs} sequences=2 T={T}')
    es.step(x, y, opt, step)
    torch.cuda.synchronize()
    losses = es.last_losses.cpu()
    buf = es.buffer.cpu()
    # the step's offsets come from the device generator (train/val/eggroll.py:117-120): taken as given
    offs = {n: o.cpu() for n, o in es.offsets(step).items()}
    per_seq = 2 * pairs // 2  # members per sequence
    for s_ in range(2):
        dirs = oe.member_directions(s_ * per_seq, per_seq // 2, pairs)
        g_ = oe.gather_noise(buf, offs, shapes, dirs)
        noise = {n: tuple(t.repeat_interleave(2, 0) for t in v) if isinstance(v, tuple) else v.repeat_interleave(2, 0)
                 for n, v in g_.items()}
        sign = torch.tensor([oe.SIGMA, -oe.SIGMA]).repeat(per_seq // 2)
        ref = om.population_loss(before, noise, sign, seqs[s_][0], seqs[s_][1], mode='bf16', head='fp32')
        got = losses[s_ * per_seq:(s_ + 1) * per_seq]
        assert (got - ref).abs().max() < 1e-4, (s_, got, ref)
    f, w = oe.fitness(losses, pairs)
    grads = oe.update(w, oe.gather_noise(buf, offs, shapes, torch.arange(pairs)), len(f))
    for n, p in model.named_parameters():
        g_ref = grads[n].reshape(p.shape)
        g_got = p.grad.detach().cpu()
        assert torch.allclose(g_got, g_ref, atol=1e-6 * float(g_ref.abs().max()) + 1e-12, rtol=1e-4), n
        # Adam's first step moves every element by about lr sign(grad): a gradient within rounding of zero may
        # take the other sign, so the parameters are compared element-wise on all but a few such elements
        ref_p = oe.adam_step(before[n].clone(), g_ref, torch.zeros_like(g_ref), torch.zeros_like(g_ref), 1, oe.LR)
        d = (p.detach().cpu() - ref_p).abs()
        assert float((d <= 1e-6 + 1e-5 * ref_p.abs()).float().mean()) > 0.999, n
        assert float(d.max()) <= 2.5 * oe.LR, n
