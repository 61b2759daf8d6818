"""Pins of the CPU oracle against closed forms, library routines and brute force (CPU only).

Each check is chosen so that a plausible slip in the oracle (a dropped term, a swapped a/b, a wrong
window edge, a missing square) fails it; none re-types the oracle's own formula.
"""
import math

import pytest
import torch
from torch.nn import functional as F

from oracle import eggroll as oe
from oracle import model as om

torch.set_num_threads(8)


def test_norm_matches_library_rms_norm():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 7, 512, generator=g) * 3
    assert torch.equal(om.norm(x), F.rms_norm(x, (512,)))
    xb = x.bfloat16()
    assert torch.equal(om.norm(xb), F.rms_norm(xb, (512,)))
    q = torch.randn(2, 3, 8, 64, generator=g)
    assert torch.equal(om.norm(q), F.rms_norm(q, (64,)))


def test_rotary_is_complex_rotation():
    g = torch.Generator().manual_seed(1)
    cos, sin = om.rotary_tables(64)
    x = torch.randn(2, 64, 3, 64, generator=g)
    out = om.apply_rotary(x, cos, sin)
    z = torch.complex(x[..., :32].double(), x[..., 32:].double())
    theta = torch.complex(cos.double(), -sin.double())[None, :, None, :]
    r = z * theta
    assert torch.allclose(out[..., :32].double(), r.real, atol=1e-6)
    assert torch.allclose(out[..., 32:].double(), r.imag, atol=1e-6)
    # position 0 is the identity; the tables are bf16 values of cos/sin(t * 10000^(-2i/64))
    assert torch.equal(out[:, 0], x[:, 0])
    t, i = 37, 5
    assert float(cos[t, i]) == float(torch.tensor(math.cos(t * 10000 ** (-2 * i / 64))).bfloat16())


def test_window_sizes_follow_sequence_len():
    assert om.window_sizes() == [1024, 1024, 1024, 2048, 1024, 1024, 1024, 2048]
    assert om.window_sizes(256) == [128, 128, 128, 256, 128, 128, 128, 256]


@pytest.mark.parametrize('window', [3, 7, 100])
def test_attention_matches_fp64_loops(window):
    g = torch.Generator().manual_seed(2)
    B, T, H, D = 2, 9, 2, 8
    q, k, v = (torch.randn(B, T, H, D, generator=g) for _ in range(3))
    out = om.attention(q, k, v, window)
    ref = torch.zeros(B, T, H, D, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            for s in range(T):
                keys = [j for j in range(T) if j <= s and s - j <= window]
                logits = torch.tensor([float(q[b, s, h].double() @ k[b, j, h].double()) / math.sqrt(D) for j in keys])
                w = torch.exp(logits - logits.max())
                w = w / w.sum()
                ref[b, s, h] = sum(w[n] * v[b, j, h].double() for n, j in enumerate(keys))
    assert torch.allclose(out.double(), ref, atol=1e-5)


def _perturbation(g, m, out_dim, in_dim):
    return torch.randn(m, out_dim, generator=g), torch.randn(m, in_dim, generator=g)


def test_lowrank_equals_materialised_perturbed_weight():
    g = torch.Generator().manual_seed(3)
    m, T, din, dout = 4, 5, 16, 12
    x = torch.randn(m, T, din, generator=g)
    W = torch.randn(dout, din, generator=g)
    a, b = _perturbation(g, m, dout, din)
    sign = torch.tensor([0.3, -0.3, 0.1, -0.1])
    y = om.lowrank(x, W, a, b, sign)
    for p in range(m):
        Wp = W.double() + sign[p].double() * torch.outer(a[p].double(), b[p].double())
        assert torch.allclose(y[p].double(), x[p].double() @ Wp.t(), atol=1e-5)
    # an antithetic pair (same input, same a/b, opposite signs) averages to the clean output
    xs = x[:1].expand(2, -1, -1)
    pair = om.lowrank(xs, W, a[:1].expand(2, -1), b[:1].expand(2, -1), torch.tensor([0.3, -0.3]))
    assert torch.allclose((pair[0] + pair[1]) / 2, x[0] @ W.t(), atol=1e-5)


def test_lowrank_bf16_mode_rounding_points():
    g = torch.Generator().manual_seed(4)
    m, T, din, dout = 2, 8, 64, 32
    x = torch.randn(m, T, din, generator=g)
    W = torch.randn(dout, din, generator=g) / 8
    a, b = _perturbation(g, m, dout, din)
    sign = torch.tensor([1e-3, -1e-3])
    y = om.lowrank(x, W, a, b, sign, 'bf16')
    dense = (x.bfloat16().double() @ W.bfloat16().double().t()).float().bfloat16().float()
    u = (x.bfloat16().double() @ b.bfloat16().double().unsqueeze(-1)).float().bfloat16().float()
    assert torch.allclose(y, dense + sign[:, None, None] * u * a[:, None, :], atol=1e-6)
    # the fp32 correction survives on top of the bf16 dense part (it is below bf16 resolution)
    assert not torch.equal(y[0], y[0].bfloat16().float())


def test_lowrank_embed_equals_gathered_perturbed_table():
    g = torch.Generator().manual_seed(5)
    V, d, m = 50, 16, 4
    W = torch.randn(V, d, generator=g)
    a, b = _perturbation(g, m, V, d)
    sign = torch.tensor([0.2, -0.2, 0.5, -0.5])
    idx = torch.randint(0, V, (11,), generator=g)
    out = om.lowrank_embed(W, a, b, idx, sign)
    for p in range(m):
        table = W + sign[p] * torch.outer(a[p], b[p])
        assert torch.allclose(out[p], table[idx], atol=1e-6)


def _tiny_model(seed=0):
    from noise_amd.model import make_model
    from noise_amd.synthetic import trained_like
    model = trained_like(make_model('cpu', seed))
    return {n: p.detach().clone() for n, p in model.named_parameters()}


def test_population_loss_equals_clean_forward_on_perturbed_weights():
    """Member p of the population is the fixed model at theta + s_p E_p (brute force, tiny T)."""
    from noise_amd.synthetic import antithetic_signs, population_noise, zipf_tokens
    p = _tiny_model()
    shapes = {n: tuple(t.shape) for n, t in p.items()}
    noise = population_noise(shapes, 2, seed=7)
    sign = antithetic_signs(4, 0.05)  # large sigma so a dropped perturbation term is visible
    idx, tgt = zipf_tokens(24, seed=8)
    losses = om.population_loss(p, noise, sign, idx, tgt)
    for m in range(4):
        pm = om.perturbed_params(p, noise, sign, m)
        ref = om.gpt_forward(pm, idx[None], tgt[None])
        assert abs(float(losses[m]) - float(ref)) < 2e-5, m
    assert float((losses[0] - losses[1]).abs()) > 1e-3


def test_population_loss_sigma_zero_is_clean_loss():
    from noise_amd.synthetic import antithetic_signs, population_noise, zipf_tokens
    p = _tiny_model()
    noise = population_noise({n: tuple(t.shape) for n, t in p.items()}, 2, seed=7)
    idx, tgt = zipf_tokens(16, seed=9)
    losses = om.population_loss(p, noise, antithetic_signs(4, 0.0), idx, tgt)
    clean = om.gpt_forward(p, idx[None], tgt[None])
    assert torch.allclose(losses, clean.expand(4), atol=1e-6)


def test_head_loss_is_capped_cross_entropy_with_stable_lse():
    g = torch.Generator().manual_seed(6)
    m, T, D, V = 2, 3, 8, om.VOCAB
    h = torch.randn(m, T, D, generator=g)
    W = torch.randn(V, D, generator=g) * 100  # logits far beyond the cap
    a, b = _perturbation(g, m, V, D)
    sign = torch.tensor([0.0, 0.0])
    tgt = torch.tensor([0, 5, V - 1])
    out = om.head_loss(h, W, a, b, sign, tgt)
    z = 15 * torch.tanh((h.double() @ W.double().t()) / 15)
    lse = torch.logsumexp(z, -1)
    ce = lse - z.gather(-1, tgt.expand(m, T)[..., None])[..., 0]
    assert torch.allclose(out.double(), ce.mean(-1), atol=1e-4)
    assert torch.isfinite(out).all()


def test_moments_match_fp64_brute_force():
    g = torch.Generator().manual_seed(7)
    o = torch.randn(2, 3, 10, 4, generator=g)
    m1, m2 = om.attention_moments(o)
    for p in range(2):
        for h in range(3):
            for d in range(4):
                col = [float(o[p, h, t, d]) for t in range(10)]
                assert abs(float(m1[p, h, d]) - sum(col) / 10) < 1e-6
                assert abs(float(m2[p, h, d]) - sum(c * c for c in col) / 10) < 1e-6


def test_fitness_closed_form():
    losses = torch.tensor([1.0, 3.0, 2.0, 1.0, 5.0, 5.5])
    f, w = oe.fitness(losses, 3)
    raw = [3.0 - 1.0, 1.0 - 2.0, 5.5 - 5.0]  # odd minus even, no centering
    mean = sum(raw) / 3
    std = math.sqrt(sum((r - mean) ** 2 for r in raw) / 2)  # unbiased
    assert torch.allclose(f, torch.tensor([r / (std + 1e-8) for r in raw]), atol=1e-6)
    assert torch.allclose(w, f)
    _, w2 = oe.fitness(losses, 2)  # folding: direction j collects pairs j, j+2, ...
    assert torch.allclose(w2, torch.tensor([f[0] + f[2], f[1]]), atol=1e-6)


def test_update_is_weighted_sum_of_outer_products():
    g = torch.Generator().manual_seed(8)
    n, out_d, in_d = 5, 4, 3
    a, b = torch.randn(n, out_d, generator=g), torch.randn(n, in_d, generator=g)
    eps = torch.randn(n, 8, generator=g)
    w = torch.randn(n, generator=g)
    grads = oe.update(w, {'m': (a, b), 'l': eps}, 10)
    ref = -sum(w[j] * torch.outer(a[j], b[j]) for j in range(n)) / 10
    assert torch.allclose(grads['m'], ref, atol=1e-6)
    assert torch.allclose(grads['l'], -sum(w[j] * eps[j] for j in range(n)) / 10, atol=1e-6)


def test_adam_matches_torch_adamw():
    g = torch.Generator().manual_seed(9)
    p0 = torch.randn(6, 5, generator=g)
    ref = p0.clone().requires_grad_(False)
    opt = torch.optim.AdamW([ref], lr=1e-3, betas=oe.BETAS, eps=1e-8, weight_decay=0.0)
    mine, m, v = p0.clone(), torch.zeros_like(p0), torch.zeros_like(p0)
    for step in range(1, 4):
        grad = torch.randn(6, 5, generator=g)
        ref.grad = grad.clone()
        opt.step()
        oe.adam_step(mine, grad, m, v, step, 1e-3)
        assert torch.allclose(mine, ref, atol=1e-7, rtol=1e-6)


def test_learning_rate_warmdown():
    assert oe.learning_rate(1, 10) == pytest.approx(1e-3)
    assert oe.learning_rate(10, 10) == pytest.approx(1e-3 * 0.1 / 0.3)
    assert oe.learning_rate(8, 10) == pytest.approx(1e-3)


def test_member_directions():
    d = oe.member_directions(0, 4, 4)
    assert d.tolist() == [0, 1, 2, 3]
    assert oe.member_directions(8, 4, 4).tolist() == [0, 1, 2, 3]


def test_chunk_sequences_hand_worked_layout():
    """pairs = 1536 on BATCH = 8 sequences: 3072 members, per_seq = 384, chunks of 2 * 256 = 512 members start at
    0, 512, ..., 2560 and run on sequences 0 // 384 = 0, 1, 2, 4, 5, 6 (3 and 7 host no member)."""
    seq = oe.chunk_sequences(3072, 384, 256)
    want = torch.tensor([0, 1, 2, 4, 5, 6]).repeat_interleave(512)
    assert torch.equal(seq, want)
    # when per_seq is a multiple of 2 * CHUNK every sequence hosts exactly per_seq members
    seq = oe.chunk_sequences(8 * 1024, 1024, 256)
    assert torch.equal(seq, torch.arange(8).repeat_interleave(1024))
    # two ranks: each walks its own half from rank * per_rank
    seq = oe.chunk_sequences(24, 12, 2, world=2)
    assert seq.tolist() == [0] * 12 + [1] * 12


def test_rank_fitness_hand_ranked_with_ties():
    # pair differences: [2, -1, 2, 0.5] -> ranks with ties by index: -1 -> 0, 0.5 -> 1, 2 (j=0) -> 2, 2 (j=2) -> 3
    losses = torch.tensor([1.0, 3.0, 2.0, 1.0, 0.0, 2.0, 4.0, 4.5])
    f, w = oe.rank_fitness(losses, 4)
    assert torch.allclose(f, torch.tensor([2 / 3, 0.0, 1.0, 1 / 3]) - 0.5)
    assert torch.allclose(w, f)
    _, w2 = oe.rank_fitness(losses, 2)
    assert torch.allclose(w2, torch.tensor([f[0] + f[2], f[1] + f[3]]))


def test_mlp_population_equals_materialised_weights():
    g = torch.Generator().manual_seed(10)
    m, T, d, f = 2, 5, 16, 24
    x = torch.randn(m, T, d, generator=g)
    w1, w2 = torch.randn(f, d, generator=g), torch.randn(d, f, generator=g)
    a1, b1 = torch.randn(m, f, generator=g), torch.randn(m, d, generator=g)
    a2, b2 = torch.randn(m, d, generator=g), torch.randn(m, f, generator=g)
    sign = torch.tensor([0.1, -0.1])
    y = om.mlp_population(x, w1, w2, a1, b1, a2, b2, sign, 'fp32')
    for p in range(m):
        W1 = w1 + sign[p] * torch.outer(a1[p], b1[p])
        W2 = w2 + sign[p] * torch.outer(a2[p], b2[p])
        ref = torch.relu(x[p].double() @ W1.double().t()) ** 2 @ W2.double().t()
        assert torch.allclose(y[p].double(), ref, rtol=1e-5, atol=1e-4)


def test_norm_head_ce_with_gain_is_capped_cross_entropy():
    g = torch.Generator().manual_seed(11)
    m, T, D, V = 2, 4, 8, om.VOCAB
    h = torch.randn(m, T, D, generator=g)
    gain = 0.9 + 0.2 * torch.rand(D, generator=g)
    W = torch.randn(V, D, generator=g)
    a, b = torch.randn(m, V, generator=g), torch.randn(m, D, generator=g)
    sign = torch.tensor([0.05, -0.05])
    tgt = torch.tensor([3, 0, V - 1, 17])
    out = om.norm_head_ce(h, gain, W, a, b, sign, tgt)
    for p in range(m):
        hn = h[p].double() * torch.rsqrt(h[p].double().pow(2).mean(-1, keepdim=True) + 2 ** -23) * gain.double()
        z = hn @ (W.double() + float(sign[p]) * torch.outer(a[p].double(), b[p].double())).t()
        z = 15 * torch.tanh(z / 15)
        ce = torch.logsumexp(z, -1) - z.gather(-1, tgt[:, None])[:, 0]
        assert abs(float(out[p]) - float(ce.mean())) < 1e-4
    # gain = 1 reproduces the reference head path
    ones = om.norm_head_ce(h, torch.ones(D), W, a, b, sign, tgt)
    assert torch.allclose(ones, om.head_loss(om.norm(h), W, a, b, sign, tgt), atol=1e-6)


def test_readout_probes_equal_moved_stream_brute_force():
    """cycle_derivatives / row_derivatives (train/val/run.py:154-185) against moving the stream itself:
    norm(x + s D_j) through the head, capped, cross-entropy; the RMS-from-dots algebra and C = W D are what
    the brute force does not assume. float64; a target of -1 gives 0."""
    from oracle import probes as op
    g = torch.Generator().manual_seed(5)
    n, width, V, P, K = 4, 16, 32, 6, 3
    x = torch.randn(n, width, generator=g, dtype=torch.float64) * 2
    W = torch.randn(V, width, generator=g, dtype=torch.float64)
    D = torch.randn(width, P, generator=g, dtype=torch.float64)
    y = torch.tensor([3, -1, 31, 0])
    steps = torch.tensor([[1e-2], [3e-2], [5e-3], [2e-2]], dtype=torch.float64)
    base, C = x @ W.T, (W @ D).T
    sq, dots, dir_sq = x.square().sum(-1, keepdim=True), x @ D, D.square().sum(0)
    got = op.cycle_derivatives(base, C, y, steps, sq, dots, dir_sq, width=width)
    moved, clean = op.moved_stream_losses(x, W, D, y, steps)
    ref = (moved - clean[:, None]) / steps * (y >= 0)[:, None]
    assert torch.allclose(got, ref, rtol=1e-9, atol=1e-9)
    assert torch.all(got[1] == 0) and got.abs().sum() > 0
    rows = torch.randint(0, P, (n, K), generator=g)
    got_r = op.row_derivatives(base, C, rows, y, steps, sq, dots.gather(1, rows), dir_sq[rows], width=width)
    assert torch.allclose(got_r, ref.gather(1, rows), rtol=1e-9, atol=1e-9)


def test_credit_helpers_equal_index_loops():
    """moved_heads / head_scores / code_estimate (train/val/run.py:186-211) against per-element loops: the
    rotation as a complex product, the RMS as an explicit mean, the sums over their named indices."""
    from oracle import credit as oc
    g = torch.Generator().manual_seed(11)
    n, b, t, h = 3, 2, 4, 2
    raw = torch.randn(b, t, h, 64, generator=g).double()
    a = torch.randn(n, b, t, h, 64, generator=g).double()
    ang = torch.rand(t, 32, generator=g).double() * 6
    cos, sin, sigma = ang.cos(), ang.sin(), 0.3
    got = oc.moved_heads(raw, a, sigma, cos, sin).view(n, b, t, h, 64)
    for j in range(n):
        for bb in range(b):
            for tt in range(t):
                for hh in range(h):
                    x = raw[bb, tt, hh] + sigma * a[j, bb, tt, hh]
                    z = torch.complex(x[:32], x[32:]) * torch.complex(cos[tt], -sin[tt])
                    y = torch.cat([z.real, z.imag])
                    y = y / math.sqrt(float((y * y).sum()) / 64 + torch.finfo(torch.float32).eps)
                    assert torch.allclose(got[j, bb, tt, hh], y, rtol=1e-6, atol=1e-6)
    out = torch.randn(n, b, t, h, 64, generator=g).double()
    base, hub = torch.randn(b, t, h, 64, generator=g).double(), torch.randn(b, t, h, 64, generator=g).double()
    score = oc.head_scores(out, base, hub)
    assert score.shape == (b, h, t, n)
    cr = torch.randn(b, h, t, n, generator=g).double()
    est = oc.code_estimate(cr, a)
    for bb in range(b):
        for hh in range(h):
            for tt in range(t):
                for j in range(n):
                    want = sum(float((out[j, bb, tt, hh, d] - base[bb, tt, hh, d]) * hub[bb, tt, hh, d])
                               for d in range(64))
                    assert abs(float(score[bb, hh, tt, j]) - want) < 1e-5 * (1 + abs(want))  # fp32 sums
                for d in (0, 17, 63):
                    want = sum(float(cr[bb, hh, tt, j] * a[j, bb, tt, hh, d]) for j in range(n))
                    assert abs(float(est[bb, tt, hh, d]) - want) < 1e-5 * (1 + abs(want))


def test_query_credit_with_basis_draws_is_the_gradient():
    """With the 64 draws a_j = e_j at every (b, t, h) and a small sigma, the query estimate of one chunk
    (train/val/run.py:617-625) divided by sigma is the gradient of sum(target * attention output) with respect
    to the raw queries (each query's output depends on its own query only): fp64 autograd through
    norm(rotary(.)) and a dense masked softmax."""
    from oracle import credit as oc
    g = torch.Generator().manual_seed(12)
    b, t, h, window, sigma = 1, 6, 2, 3, 1e-3
    raw = torch.randn(b, t, h, 64, generator=g, dtype=torch.float64)
    kp = om.norm(torch.randn(b, t, h, 64, generator=g, dtype=torch.float64))
    v = torch.randn(b, t, h, 64, generator=g, dtype=torch.float64)
    hub = torch.randn(b, t, h, 64, generator=g, dtype=torch.float64)
    ang = torch.rand(t, 32, generator=g, dtype=torch.float64) * 6
    cos, sin = ang.cos(), ang.sin()
    a = torch.eye(64, dtype=torch.float64)[:, None, None, None, :].expand(64, b, t, h, 64).contiguous()

    def out_of(q_raw):
        x1, x2 = q_raw[..., :32], q_raw[..., 32:]
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        y = torch.cat([x1 * c + x2 * s, -x1 * s + x2 * c], -1)
        y = y * torch.rsqrt((y * y).mean(-1, keepdim=True) + torch.finfo(torch.float32).eps)
        return om.attention(y, kp, v, window, dtype=torch.float64)

    q = raw.clone().requires_grad_(True)
    (out_of(q) * hub).sum().backward()
    baseline = out_of(raw)
    est = oc.credit_chunk('q', raw, a, sigma, cos, sin, kp, v, window, baseline, hub, round_out=False)
    assert torch.allclose(est.double() / sigma, q.grad, rtol=2e-2, atol=2e-3 * float(q.grad.abs().max()))


def test_key_credit_through_a_permutation_filter_sums_key_gradients():
    """Keys (train/val/run.py:617-625): with the 64 draws a_j = e_j at every (b, t, h), every key of the sequence
    moves by the same draw, so query u's score for draw j is sigma * sum_s d(target_u . out_u) / d raw_k[s, j]. A
    matched filter that is a cyclic shift of the positions (t <- t + 1, not symmetric) carries query t + 1's score to
    key position t, so the estimate / sigma at t is sum_s d(target_{t+1} . out_{t+1}) / d raw_k[s]: fp64 autograd one
    query at a time. A transposed filter product would land on t - 1 instead."""
    from oracle import credit as oc
    g = torch.Generator().manual_seed(13)
    b, t, h, window, sigma = 1, 6, 2, 3, 1e-3
    raw = torch.randn(b, t, h, 64, generator=g, dtype=torch.float64)
    qp = om.norm(torch.randn(b, t, h, 64, generator=g, dtype=torch.float64))
    v = torch.randn(b, t, h, 64, generator=g, dtype=torch.float64)
    hub = torch.randn(b, t, h, 64, generator=g, dtype=torch.float64)
    ang = torch.rand(t, 32, generator=g, dtype=torch.float64) * 6
    cos, sin = ang.cos(), ang.sin()
    a = torch.eye(64, dtype=torch.float64)[:, None, None, None, :].expand(64, b, t, h, 64).contiguous()

    def out_of(k_raw):
        x1, x2 = k_raw[..., :32], k_raw[..., 32:]
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        y = torch.cat([x1 * c + x2 * s, -x1 * s + x2 * c], -1)
        y = y * torch.rsqrt((y * y).mean(-1, keepdim=True) + torch.finfo(torch.float32).eps)
        return om.attention(qp, y, v, window, dtype=torch.float64)

    shift = torch.zeros(t, t, dtype=torch.float64)
    for u in range(t):
        shift[u, (u + 1) % t] = 1.0   # key row u reads query (u + 1) % t
    filt = shift[None, None].expand(b, h, t, t).contiguous()
    est = oc.credit_chunk('k', raw, a, sigma, cos, sin, qp, v, window, out_of(raw), hub, key_filter=filt,
                          round_out=False)
    ref = torch.zeros(b, t, h, 64, dtype=torch.float64)
    for u in range(t):
        k = raw.clone().requires_grad_(True)
        (out_of(k)[:, (u + 1) % t] * hub[:, (u + 1) % t]).sum().backward()
        ref[:, u] = k.grad.sum(1)
    assert torch.allclose(est.double() / sigma, ref, rtol=2e-2, atol=2e-3 * float(ref.abs().max()))


def test_autocast_helpers_equal_torch_bf16_arithmetic():
    """The autocast oracle's elementwise rounding rules against torch's own bf16 arithmetic on the CPU, which torch
    2.10's CUDA autocast reproduces bit for bit (checked on the MI355X box for the mix, rotary and value gate): a
    lambda left in fp32, a dropped rounding of a product or a sum, or an eps of 2^-7 fails here."""
    g = torch.Generator().manual_seed(31)
    x = (torch.randn(3, 16, 512, generator=g) * 0.7).bfloat16()
    x0 = torch.randn(3, 16, 512, generator=g).bfloat16()
    lam = torch.tensor([0.913, 0.1, 0.37])
    assert torch.equal(om.ac_mix(lam[0], lam[2], x.float(), x0.float()), (lam[0] * x + lam[2] * x0).float())
    # norm of a bf16 input: torch's rms_norm (fp32 compute, fp32 epsilon) -- including rows small enough for the
    # epsilon to matter
    small = (torch.randn(4, 512, generator=g) * 3e-4).bfloat16()
    for t in (x, small):
        assert torch.equal(om.ac_norm(t.float()), F.rms_norm(t, (t.shape[-1],)).float())
    cos, sin = om.rotary_tables(16)
    q = (torch.randn(3, 16, 8, 64, generator=g)).bfloat16()
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    ref = torch.cat([q[..., :32] * c + q[..., 32:] * s, q[..., :32] * -s + q[..., 32:] * c], 3)
    assert torch.equal(om.ac_rotary(q.float(), cos, sin), ref.float())
    v = torch.randn(3, 16, 8, 64, generator=g).bfloat16()
    z = torch.randn(3, 16, 8, generator=g).bfloat16()
    ve = torch.randn(3, 16, 8, 64, generator=g).bfloat16()
    ref = v + (2 * torch.sigmoid(z)).unsqueeze(-1) * ve
    assert torch.equal(om.ac_value_gate(v.float(), z.float(), ve.float()), ref.float())


@pytest.mark.parametrize('window', [3, 100])
def test_bf16_attention_is_the_fp64_softmax_within_bf16_rounding(window):
    """attention_bf16 = the fp64 masked softmax of the same bf16 q, k, v up to the bf16 probabilities and the bf16
    output: within a few bf16 steps of the exact result, and exactly the bf16 rounding of it when the rounded
    probabilities carry no error (one visible key per query)."""
    g = torch.Generator().manual_seed(32)
    B, T, H, D = 2, 9, 2, 8
    q, k, v = (torch.randn(B, T, H, D, generator=g).bfloat16().float() for _ in range(3))
    out = om.attention_bf16(q, k, v, window)
    ref = om.attention(q.double(), k.double(), v.double(), window, dtype=torch.float64)
    assert (out.double() - ref).abs().max() <= 4 * 2 ** -8 * ref.abs().max()
    assert torch.equal(out[:, 0], om.bf(v[:, 0]))  # the first query sees only itself


def test_autocast_forward_is_the_fp32_forward_within_bf16_rounding():
    """The whole autocast forward against the golden-pinned fp32 forward: equal within the bf16 class at the
    reference init (lm_head ~ N(0, 1e-6) keeps the losses near ln 4096) and at trained-scale weights, and really
    rounded (not the fp32 forward itself)."""
    from noise_amd.model import make_model
    from noise_amd.synthetic import trained_like, zipf_tokens
    torch.manual_seed(0)
    idx, tgt = zipf_tokens(128, seed=33)
    for model in (make_model('cpu', 0), trained_like(make_model('cpu', 0))):
        p = {n: t.detach() for n, t in model.named_parameters()}
        a = om.autocast_forward(p, idx[None], tgt[None], 'none')
        b = om.gpt_forward(p, idx[None], tgt[None], 'none')
        # per token the bf16 stream moves a trained-scale loss by up to ~0.1; the mean over tokens by ~1e-3
        assert 0 < (a - b).abs().max() < 0.25, float((a - b).abs().max())
        assert abs(float(a.mean() - b.mean())) < 5e-3
    logits = om.autocast_forward(p, idx[None])
    assert logits.dtype == torch.float32 and logits.abs().max() <= 15.0
