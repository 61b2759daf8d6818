"""Credit scoring around attention reruns on the HIP kernels (train/val/run.py:186-211, composed by
query_key_errors :594-634) against the CPU oracle on the same seeded inputs."""
import pytest
import torch

from noise_amd import credit
from oracle import credit as oc
from oracle import model as om
from tests._util import log_case, rel_err

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def _tables(T):
    cos, sin = om.rotary_tables()
    return cos[:T].float(), sin[:T].float()


def _heads(g, n, b, T, h=8):
    raw = torch.randn(b, T, h, 64, generator=g) * 2
    a = torch.randn(n, b, T, h, 64, generator=g).bfloat16()
    return raw, a


def test_moved_heads_match_oracle_within_one_bf16_step():
    g = torch.Generator().manual_seed(21)
    n, b, T = 4, 2, 256
    log_case(f'moved_heads n={n} b={b} T={T}')
    raw, a = _heads(g, n, b, T)
    cos, sin = _tables(T)
    got = credit.moved_heads(raw.to(DEV), a.to(DEV), 0.1, cos.to(DEV), sin.to(DEV))
    torch.cuda.synchronize()
    ref = oc.moved_heads(raw, a, 0.1, cos, sin)
    got = got.cpu().float()
    assert got.shape == ref.shape
    # fp32 arithmetic in a different order (fused multiply-adds on the GPU): a result may round to the
    # neighbouring bf16 value; near-cancelling rotations (|y| far below the row RMS of 1) carry the fp32
    # error of the unit-size terms, 1e-6 absolute
    diff = (got - ref.float()).abs()
    bound = ref.float().abs() * 2.0 ** -7 + 1e-6
    worst = int((diff - bound).flatten().argmax())
    print(f'moved_heads: exact {float((diff == 0).float().mean()):.5f}, worst got {float(got.flatten()[worst]):.6e} '
          f'ref {float(ref.float().flatten()[worst]):.6e}', flush=True)
    assert (diff <= bound).all()
    assert float((diff == 0).float().mean()) > 0.99


def test_head_scores_and_code_estimate_match_oracle():
    g = torch.Generator().manual_seed(22)
    n, b, T, h = 6, 2, 128, 8
    log_case(f'head_scores / code_estimate n={n} b={b} T={T}')
    out = torch.randn(n, b, T, h, 64, generator=g).bfloat16()
    base, hub = torch.randn(b, T, h, 64, generator=g), torch.randn(b, T, h, 64, generator=g)
    score = credit.head_scores(out.to(DEV), base.to(DEV), hub.to(DEV))
    cr = torch.randn(b, h, T, n, generator=g)
    a = torch.randn(n, b, T, h, 64, generator=g).bfloat16()
    est = credit.code_estimate(cr.to(DEV), a.to(DEV))
    torch.cuda.synchronize()
    ref_s, ref_e = oc.head_scores(out, base, hub), oc.code_estimate(cr, a)
    print(f'head_scores max diff {float((score.cpu() - ref_s).abs().max()):.3e}, code_estimate max diff '
          f'{float((est.cpu() - ref_e).abs().max()):.3e}', flush=True)
    assert torch.allclose(score.cpu(), ref_s, rtol=1e-5, atol=1e-4)
    assert torch.allclose(est.cpu(), ref_e, rtol=1e-5, atol=1e-5)


def test_attention_wrapper_matches_oracle():
    g = torch.Generator().manual_seed(23)
    b, T, window = 2, 256, 100
    log_case(f'credit.attention b={b} T={T} window={window}')
    q, k, v = (torch.randn(b, T, 8, 64, generator=g).bfloat16() for _ in range(3))
    got = credit.attention(q.to(DEV), k.to(DEV), v.to(DEV), window).cpu().float()
    ref = om.bf(om.attention(q.float(), k.float(), v.float(), window))
    assert rel_err(got, ref) < 1e-2
    assert (got - ref).abs().max() < 2e-2


def _key_bound(filt, score):
    """The exact product of the bf16 operands and the error allowed to the kernel's: its bf16 rounding (one step,
    2^-8 relative) plus fp32 accumulation over T terms (T 2^-24 of the absolute terms' sum: mixed-sign scores can
    cancel, leaving a result far below the terms, where the summation order alone moves it)."""
    K, s = filt.double(), score.bfloat16().double()
    exact = K @ s
    return exact, 2 ** -8 * exact.abs() + filt.shape[-1] * 2 ** -24 * (K.abs() @ s.abs()) + 1e-6


@pytest.mark.parametrize('n', [24, 70])
def test_key_scores_match_the_bf16_product(n):
    """The key scores (train/val/run.py:622-623) on the HIP kernel: bf16(K) @ bf16(score) with fp32 accumulation,
    rounded to bf16; within one bf16 step plus the fp32 accumulation error of the exact product of the same bf16
    operands, for draw counts that are not multiples of the kernel's 64-column blocks."""
    g = torch.Generator().manual_seed(27)
    b, h, T = 2, 8, 256
    filt = torch.rand(b, h, T, T, generator=g).tril().bfloat16()
    score = torch.randn(b, h, T, n, generator=g)
    log_case(f'key_scores b={b} h={h} T={T} n={n}')
    got = credit.key_scores(filt.to(DEV), score.to(DEV)).cpu()
    exact, bound = _key_bound(filt, score)
    assert torch.equal(got, got.bfloat16().float())  # bf16 values
    assert ((got.double() - exact).abs() <= bound).all()


def test_key_scores_wide_grid():
    """A grid of at least two workgroups per CU (4 x 8 heads, 512 tokens, 130 draws: 768 workgroups of 64 draws), which
    takes the kernel's 64-draw blocks; the tests above take its 32-draw ones. Within the same bound, ragged last block
    included."""
    g = torch.Generator().manual_seed(29)
    b, h, T, n = 4, 8, 512, 130
    filt = torch.rand(b, h, T, T, generator=g).tril().bfloat16()
    score = torch.randn(b, h, T, n, generator=g)
    log_case(f'key_scores b={b} h={h} T={T} n={n} (64-draw blocks)')
    got = credit.key_scores(filt.to(DEV), score.to(DEV)).cpu()
    exact, bound = _key_bound(filt, score)
    assert torch.equal(got, got.bfloat16().float())
    assert ((got.double() - exact).abs() <= bound).all()


@pytest.mark.parametrize('window', [256, 96])
def test_key_scores_through_an_attention_map_filter(window):
    """The matched filter as the reference builds it (train/val/run.py:572-592): the clean attention map A of
    RMS-normalised rotary q, k under the causal window, K[t, s] = A[s, t] / max_t' A[s, t'] in bf16 (upper
    triangular and banded: t <= s <= t + window, the opposite side of the diagonal from the test above). The key
    scores through it within the same bound."""
    g = torch.Generator().manual_seed(28)
    b, h, T, n = 1, 8, 256, 24
    log_case(f'key_scores attention-map filter T={T} window={window} n={n}')
    cos, sin = _tables(T)
    q, k = (om.norm(om.apply_rotary(torch.randn(b, T, h, 64, generator=g), cos, sin)) for _ in range(2))
    logits = q.transpose(1, 2) @ k.transpose(1, 2).transpose(-1, -2) / 8.0
    lag = torch.arange(T)[:, None] - torch.arange(T)[None, :]
    A = logits.masked_fill(~((lag >= 0) & (lag <= window)), float('-inf')).softmax(-1)
    filt = (A / A.amax(-1, keepdim=True)).transpose(-1, -2).bfloat16().contiguous()
    assert torch.equal(filt.float().tril(-1), torch.zeros_like(filt.float()))  # nothing below the diagonal
    score = torch.randn(b, h, T, n, generator=g)
    got = credit.key_scores(filt.to(DEV), score.to(DEV)).cpu()
    exact, bound = _key_bound(filt, score)
    assert torch.equal(got, got.bfloat16().float())
    assert ((got.double() - exact).abs() <= bound).all()


@pytest.mark.parametrize('kind', ['q', 'k'])
def test_credit_chunk_matches_oracle(kind):
    """One chunk of query / key credit: GPU estimate within twice the oracle's own bf16-output floor (oracle
    with the attention output rounded to bf16, as the reference's, against the unrounded oracle) plus 1e-3."""
    g = torch.Generator().manual_seed(24 if kind == 'q' else 25)
    n, b, T, window, sigma = 8, 2, 256, 128, 0.1
    log_case(f'credit_chunk kind={kind} n={n} b={b} T={T} window={window}')
    raw, a = _heads(g, n, b, T)
    cos, sin = _tables(T)
    other = om.norm(om.apply_rotary(torch.randn(b, T, 8, 64, generator=g), cos, sin)).bfloat16()
    values = torch.randn(b, T, 8, 64, generator=g).bfloat16()
    processed = om.norm(om.apply_rotary(raw, cos, sin)).bfloat16()
    qp, kp = (processed, other) if kind == 'q' else (other, processed)
    baseline = om.bf(om.attention(qp.float(), kp.float(), values.float(), window))
    target = torch.randn(b, T, 8, 64, generator=g)
    kf = torch.rand(b, 8, T, T, generator=g).tril().bfloat16() if kind == 'k' else None
    fixed = other
    args = lambda d: [t.to(d) if isinstance(t, torch.Tensor) else t for t in  # noqa: E731
                      (raw, a, sigma, cos, sin, fixed, values, window, baseline, target, kf)]
    got = credit.credit_chunk(kind, *args(DEV)).cpu()
    ref32 = oc.credit_chunk(kind, *args('cpu'), round_out=False)
    ref16 = oc.credit_chunk(kind, *args('cpu'), round_out=True)
    floor = rel_err(ref16, ref32)
    log_case(f'credit_chunk kind={kind}: gpu {rel_err(got, ref32):.3e} floor {floor:.3e}')
    assert rel_err(got, ref32) <= 2 * floor + 1e-3


def test_query_credit_full_length_sampled_positions():
    """The model's 2048-token sequence, 16 draws, the short window 1024: the query estimate at sampled
    positions (first and last tokens, both sides of the window edge) against a per-position oracle: each
    query's output depends on its own moved query only (train/val/run.py:617-625). GPU error within twice the
    oracle's bf16-output floor plus 1e-3, as for the small chunk."""
    g = torch.Generator().manual_seed(26)
    n, b, T, window, sigma = 16, 2, 2048, 1024, 0.1
    log_case(f'credit_chunk kind=q n={n} b={b} T={T} window={window}')
    raw, a = _heads(g, n, b, T)
    cos, sin = _tables(T)
    kp = om.norm(om.apply_rotary(torch.randn(b, T, 8, 64, generator=g), cos, sin)).bfloat16()
    values = torch.randn(b, T, 8, 64, generator=g).bfloat16()
    target = torch.randn(b, T, 8, 64, generator=g)
    qp = om.norm(om.apply_rotary(raw, cos, sin)).bfloat16()
    base = credit.attention(qp.to(DEV), kp.to(DEV), values.to(DEV), window)
    est = credit.credit_chunk('q', raw.to(DEV), a.to(DEV), sigma, cos.to(DEV), sin.to(DEV), kp.to(DEV),
                              values.to(DEV), window, base, target.to(DEV)).cpu()
    base = base.cpu().float()
    got, ref16, ref32 = [], [], []
    for bb, t in [(0, 0), (0, 1), (0, 1023), (0, 1024), (0, 1025), (0, 2047), (1, 7), (1, 1500), (1, 2047)]:
        lo = max(0, t - window)
        K, V = kp[bb, lo:t + 1].float(), values[bb, lo:t + 1].float()
        mq = oc.moved_heads(raw[bb:bb + 1, t:t + 1], a[:, bb:bb + 1, t:t + 1], sigma, cos[t:t + 1],
                            sin[t:t + 1]).float()[:, 0]                               # [n, 8, 64]
        p = (torch.einsum('nhd,whd->nhw', mq, K) / 8).softmax(-1)
        out = torch.einsum('nhw,whd->nhd', p, V)
        for rnd, acc in ((True, ref16), (False, ref32)):
            o = out.bfloat16().float() if rnd else out
            score = ((o - base[bb, t]) * target[bb, t]).sum(-1)                          # [n, 8]
            acc.append(torch.einsum('nh,nhd->hd', score, a[:, bb, t].float()))
        got.append(est[bb, t])
    got, ref16, ref32 = torch.stack(got), torch.stack(ref16), torch.stack(ref32)
    floor = rel_err(ref16, ref32)
    log_case(f'full-length query credit: gpu {rel_err(got, ref32):.3e} floor {floor:.3e}')
    assert rel_err(got, ref32) <= 2 * floor + 1e-3


def test_vector_and_scalar_credit_kernels_agree():
    """moved_heads, head_scores and code_estimate take vector accesses when pointers and strides allow and scalar
    ones otherwise (an odd output stride, an offset pointer). On the same inputs: the estimate bit for bit, the moved
    heads within one bf16 step (the norm's sum runs in another order), the scores within fp32 rounding."""
    from noise_amd import _lib
    g = torch.Generator().manual_seed(23)
    n, b, T, H = 4, 2, 128, 8
    log_case(f'credit vector / scalar paths n={n} b={b} T={T}')
    raw, a = (t.to(DEV) for t in _heads(g, n, b, T, H))
    cos, sin = (t.to(DEV).contiguous() for t in _tables(T))
    s = torch.cuda.current_stream().cuda_stream
    W = H * 64
    heads = {}
    for ld in (W, W + 1):  # W + 1: odd stride, the scalar kernel
        o = torch.zeros(n * b * T * ld, device=DEV, dtype=torch.bfloat16)
        _lib.call('noise_moved_heads', raw.data_ptr(), a.data_ptr(), 0.1, cos.data_ptr(), sin.data_ptr(), n, b, T, H,
                  o.data_ptr(), ld, s)
        heads[ld] = o.view(n * b * T, ld)[:, :W].float().cpu()
    vec, sca = heads[W], heads[W + 1]
    assert ((vec - sca).abs() <= sca.abs() * 2.0 ** -7 + 1e-6).all()
    assert float((vec == sca).float().mean()) > 0.999
    base, hub = torch.randn(b, T, H, 64, generator=g).to(DEV), torch.randn(b, T, H, 64, generator=g).to(DEV)
    out = torch.randn(n * b * T, W, generator=g).bfloat16().to(DEV)
    out_odd = torch.zeros(n * b * T, W + 1, device=DEV, dtype=torch.bfloat16)
    out_odd[:, :W] = out
    scores = []
    for o, ld in ((out, W), (out_odd, W + 1)):
        sc = torch.empty(b, H, T, n, device=DEV)
        _lib.call('noise_head_scores', o.data_ptr(), ld, base.data_ptr(), hub.data_ptr(), n, b, T, H, sc.data_ptr(), s)
        scores.append(sc.cpu())
    assert torch.allclose(scores[0], scores[1], rtol=1e-5, atol=1e-5)
    cr = torch.randn(b, H, T, n, generator=g).to(DEV)
    est_buf = torch.empty(b * T * H * 64 + 1, device=DEV)
    ests = []
    for off in (0, 1):  # offset 1: a misaligned output, the scalar kernel
        _lib.call('noise_code_estimate', cr.data_ptr(), a.data_ptr(), n, b, T, H, est_buf.data_ptr() + 4 * off, s)
        ests.append(est_buf[off:off + b * T * H * 64].cpu().clone())
    torch.cuda.synchronize()
    assert torch.equal(ests[0], ests[1])
