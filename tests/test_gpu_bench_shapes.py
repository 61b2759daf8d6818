"""GPU parity at the exact shapes bench.py times and BASELINE.json names (configs 2, 3 and 4), against the CPU
oracle on sampled members.

- Config 4: all 3072 members (1536 antithetic pairs) of the 37.7M model on one 2048-token Zipf sequence in ONE
  kernel pass (M = 6,291,456 rows per launch, bench.py's default), at the reference's seed-0 init (losses and
  antithetic differences within 1e-4) and at trained-scale weights (within twice the oracle's own rounding
  floor, measured in the test, plus 1e-4).
- Config 2: windowed causal attention + credit moments on [256 members, 8 heads, 2048 tokens, 64], windows 2048
  and 1024, with N(0, 1) bf16 q/k (running-maximum softmax) and with RMS-normalised fp16 q/k, q pre-scaled (the population
  forward's bounded-score softmax).
- Config 3: RMSNorm with gain -> fp32 head with rank-1 perturbation -> soft cap -> CE on [512, 2048, 512] bf16.
"""
import math

import pytest
import torch

from noise_amd import _lib
from noise_amd.model import make_model
from noise_amd.synthetic import antithetic_signs, population_noise, trained_like, zipf_tokens
from oracle import model as om
from tests._util import log_case, rel_err
from tests.test_gpu_population import _dev, _gpu_model, _oracle_with_floor

pytestmark = pytest.mark.gpu
DEV = 'cuda'

PAIRS4, T4 = 1536, 2048
# sampled members: both ends and the middle of the population, both signs of each pair
MEMBERS4 = [0, 1, 2, 3, 1534, 1535, 3068, 3069, 3070, 3071]


def _config4_single_pass(model, seed):
    from noise_amd.population import Population
    params = {n: p.detach().clone() for n, p in model.named_parameters()}
    P = 2 * PAIRS4
    shapes = {n: tuple(t.shape) for n, t in params.items()}
    noise = population_noise(shapes, PAIRS4, seed=seed, per_member=False)
    sign = antithetic_signs(P, 1e-3)
    idx, tgt = zipf_tokens(T4, seed=seed + 1)
    gm = _gpu_model(model)
    pop = Population(gm, chunk=P)  # one pass over every member: bench.py's launch shapes
    got = pop.loss(dict(gm.named_parameters()), _dev(noise), sign.to(DEV), idx.to(DEV), tgt.to(DEV),
                   pair_shift=1).cpu()
    del pop, gm
    torch.cuda.empty_cache()
    rows = [m // 2 for m in MEMBERS4]
    sub = {n: tuple(t[rows] for t in v) if isinstance(v, tuple) else v[rows] for n, v in noise.items()}
    return params, got, sub, sign[MEMBERS4], idx, tgt


@pytest.mark.timeout(600)
def test_config4_one_pass_at_reference_init():
    log_case(f'config4 one pass P={2 * PAIRS4} T={T4} reference init')
    params, got, sub, sgn, idx, tgt = _config4_single_pass(make_model('cpu', 0), seed=81)
    assert got.shape == (2 * PAIRS4,) and torch.isfinite(got).all()
    log_case(f'config4 oracle on members {MEMBERS4}')
    ref = om.population_loss(params, sub, sgn, idx, tgt, mode='bf16', head='fp32')
    g = got[MEMBERS4]
    assert (g - ref).abs().max() < 1e-4, (g, ref)
    dg, dr = g[1::2] - g[0::2], ref[1::2] - ref[0::2]
    assert (dg - dr).abs().max() < 1e-4, (dg, dr)


@pytest.mark.timeout(900)
def test_config4_one_pass_at_trained_scale():
    torch.manual_seed(0)
    log_case(f'config4 one pass P={2 * PAIRS4} T={T4} trained-scale weights')
    params, got, sub, sgn, idx, tgt = _config4_single_pass(trained_like(make_model('cpu', 0)), seed=83)
    assert torch.isfinite(got).all()
    # trained-scale losses spread well beyond the init's ln 4096 band
    assert float(got.std()) > 1e-3
    log_case(f'config4 oracle + rounding floor on members {MEMBERS4}')
    ref, floor, pair_floor = _oracle_with_floor(params, sub, sgn, idx, tgt)
    g = got[MEMBERS4]
    assert (g - ref).abs().max() <= 2 * floor + 1e-4, (g, ref, floor)
    dg, dr = g[1::2] - g[0::2], ref[1::2] - ref[0::2]
    assert (dg - dr).abs().max() <= 2 * pair_floor + 1e-4, (dg, dr, pair_floor)


def _attention_case(P, T, qk_norm, qk_format, seed):
    """q, k, v and their q | k | v rows; with qk_format 2 the rows hold q * log2(e) / 8 (noise_qkv's format) and
    the returned q is that fp16 value back in score units (fp32)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    dt = torch.float16 if qk_format else torch.bfloat16
    q, k, v = (torch.randn(P, T, 8, 64, device=DEV, generator=g) for _ in range(3))
    if qk_norm:
        q, k = (t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + 2 ** -23) for t in (q, k))
    q_in = (q * (math.log2(math.e) / 8)).to(dt) if qk_format == 2 else q.to(dt)
    q = q_in.float() / (math.log2(math.e) / 8) if qk_format == 2 else q_in
    k, v = k.to(dt), v.bfloat16().half()
    qkv = torch.cat([t.reshape(P * T, 512).view(torch.bfloat16) for t in (q_in, k, v)], 1)
    return q, k, v, qkv


@pytest.mark.timeout(600)
@pytest.mark.parametrize('qk_norm,qk_format', [(0, 0), (1, 2)])
def test_config2_attention_moments_full_size(qk_norm, qk_format):
    """P = 256, 8 heads, T = 2048, windows 2048 and 1024, one launch each. Sampled members' outputs within 1e-2
    relative of the fp32 oracle on the same 16-bit inputs; every member's moments within 1e-5 of the moments of
    the kernel's own bf16 output (the reduction), the sampled members' within the bf16 output rounding of the
    oracle's moments."""
    P, T = 256, 2048
    q, k, v, qkv = _attention_case(P, T, qk_norm, qk_format, seed=5 + qk_norm)
    s = torch.cuda.current_stream().cuda_stream
    sample = [0, 1, 131, 255]
    bp = torch.randn(P, 512, device=DEV, generator=torch.Generator(device=DEV).manual_seed(9))
    ws = torch.empty(_lib.size_query('noise_attention_workspace_size', P, T), device=DEV, dtype=torch.uint8)
    for window in (2048, 1024):
        log_case(f'config2 attention P={P} T={T} window={window} qk_norm={qk_norm} qk_format={qk_format}')
        y = torch.empty(P * T, 512, device=DEV, dtype=torch.bfloat16)
        up = torch.empty(P * T, 8, device=DEV)
        mom = torch.empty(P, 8, 2, 64, device=DEV)
        _lib.call('noise_attention', qkv.data_ptr(), P, T, window, qk_norm, qk_format, bp.data_ptr(), 0, y.data_ptr(),
                  up.data_ptr(), mom.data_ptr(), ws.data_ptr(), ws.numel(), s)
        torch.cuda.synchronize()
        yv = y.view(P, T, 8, 64)
        # every member: the moments are the per-head token means of y and y^2 of the kernel's own output
        yf = yv.float().permute(0, 2, 1, 3)
        m1, m2 = yf.mean(2), yf.pow(2).mean(2)
        assert (mom[:, :, 0] - m1).abs().max().item() < 1e-5
        assert (mom[:, :, 1] - m2).abs().max().item() < 1e-5
        del yf, m1, m2
        for p in sample:
            ref = om.attention(q[p:p + 1].float().cpu(), k[p:p + 1].float().cpu(), v[p:p + 1].float().cpu(), window)
            got = yv[p:p + 1].float().cpu()
            assert rel_err(got, ref) < 1e-2, p
            assert (got - ref).abs().max() < 2e-2, p
            r1, r2 = om.attention_moments(ref.permute(0, 2, 1, 3))
            # the kernel's moments are of its bf16 output: within bf16 rounding (2^-8 relative) of the oracle's
            assert ((mom[p, :, 0].cpu() - r1[0]).abs() <= 2 ** -8 * ref.abs().mean() + 1e-5).all(), p
            assert ((mom[p, :, 1].cpu() - r2[0]).abs() <= 2 ** -7 * r2[0] + 1e-5).all(), p
            # c_proj input-side partials of the sampled member: y . bf16(b_proj) per head
            dot = (got.reshape(T, 512) * om.bf(bp[p].cpu())).reshape(T, 8, 64).sum(-1)
            assert torch.allclose(up.view(P, T, 8)[p].cpu(), dot, atol=1e-3, rtol=1e-3), p


@pytest.mark.timeout(600)
@pytest.mark.parametrize('fmt', [_lib.HEAD_FP32, _lib.HEAD_FP32_SPLIT])
def test_config3_norm_head_ce_full_size_with_gain(fmt):
    """P = 512, T = 2048: bf16 h [512, 2048, 512], gain ~ U(0.9, 1.1), fp32 head [4096, 512] ~ N(0, 1/512) with
    per-pair rank-1 perturbation, sigma = 1e-3, Zipf targets, in both fp32 head formats. Sampled members within
    1e-4 of the fp32 oracle."""
    P, T, V = 512, 2048, 4096
    g = torch.Generator().manual_seed(31)
    gd = torch.Generator(device=DEV).manual_seed(32)
    h = torch.randn(P, T, 512, device=DEV, generator=gd).bfloat16()
    gain = 0.9 + 0.2 * torch.rand(512, generator=g)
    W = torch.randn(V, 512, generator=g) * 512 ** -0.5
    a, b = torch.randn(P // 2, V, generator=g), torch.randn(P // 2, 512, generator=g)
    sign = antithetic_signs(P, 1e-3)
    _, targets = zipf_tokens(T, seed=33)
    s = torch.cuda.current_stream().cuda_stream
    gdv, Wd, ad, bd, sd, td = (t.to(DEV) for t in (gain, W, a, b, sign, targets))
    log_case(f'config3 head_ce P={P} T={T} fp32_head={fmt}')
    if fmt == _lib.HEAD_FP32:
        wd = Wd
    else:
        wd = torch.empty(V, 1536, device=DEV, dtype=torch.bfloat16)
        _lib.call('noise_cast_bf16', Wd.data_ptr(), wd.data_ptr(), W.numel(), 512, s)
    loss = torch.empty(P, device=DEV)
    ws = torch.empty(_lib.size_query('noise_head_ce_workspace_size', P, T, V, fmt), device=DEV, dtype=torch.uint8)
    _lib.call('noise_head_ce', h.data_ptr(), 1, gdv.data_ptr(), wd.data_ptr(), V, fmt, ad.data_ptr(), bd.data_ptr(),
              sd.data_ptr(), td.data_ptr(), 0, P, T, 1, _lib.CE_MEMBER_MEAN, loss.data_ptr(), None, ws.data_ptr(),
              ws.numel(), None, 0, s)
    torch.cuda.synchronize()
    got = loss.cpu()
    assert torch.isfinite(got).all()
    sample = [0, 1, 256, 257, 510, 511]
    rows = [m // 2 for m in sample]
    ref = om.norm_head_ce(h[sample].float().cpu(), gain, W, a[rows], b[rows], sign[sample], targets)
    assert (got[sample] - ref).abs().max() < 1e-4, (got[sample], ref)
    # the soft-capped CE of an N(0, 1/512) head on unit-RMS rows sits near ln V
    assert (got - math.log(V)).abs().max() < 1.0
