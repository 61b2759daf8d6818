"""CPU restatement of the fixed model and of the population-perturbed forward (TEST INFRASTRUCTURE ONLY).

Follows `utils/model.py:14-210` (norm, rotary, windows, attention, clean forward) and
`train/val/eggroll.py:56-103` (lowrank, lowrank_embed, population_loss). Plain PyTorch on the CPU.

Two rounding modes:

* ``mode='fp32'`` -- every op in float32. This is what the reference itself computes on a CPU, where
  `torch.autocast('cuda')` (`train/val/eggroll.py:144`) is inactive; the golden fixtures in
  `tests/golden/` were produced that way.
* ``mode='bf16'`` -- the rounding points of the reference under CUDA bf16 autocast
  (`train/val/eggroll.py:144`): every GEMM (including the rank-1 GEMV ``x @ b``) rounds both operands
  to bf16, accumulates in fp32 and rounds its output to bf16; the rank-1 correction and the residual
  stream stay fp32. q, k and v stay fp32 into attention, as in the reference (flex attention is not
  covered by autocast); the attention output y is rounded to bf16 where the c_proj GEMM casts it.

``head='fp32'`` evaluates the lm_head GEMM in float32 (the north star's fp32 head); ``head='bf16'`` is
the reference's autocast head.

``autocast_forward`` restates the clean GPT.forward at the rounding points of the speedrun's scorer
(utils/eval.py:44-45: bf16 autocast with bf16 embedding tables), where the whole residual stream is bf16.

Parity pins (tests/test_oracle.py): norm against F.rms_norm; rotary against the complex-rotation
closed form; attention against an fp64 loop over (query, key) on tiny T; lowrank / lowrank_embed
against the materialised perturbed weight W + s a b^T; population_loss against (i) the golden
per-member losses written by importing the reference in the build container and (ii) the clean
forward on materialised perturbed weights; moments against an fp64 brute force.
"""
import math

import torch
from torch.nn import functional as F

VOCAB = 4096
N_EMBD = 512
N_LAYER = 8
N_HEAD = 8
HEAD_DIM = 64
SEQUENCE_LEN = 2048
EPS = torch.finfo(torch.float32).eps  # F.rms_norm with eps=None on fp32 compute (utils/model.py:46-47)
SOFTCAP = 15.0                         # utils/model.py:204, train/val/eggroll.py:100


def bf(t):
    """Round to bfloat16 (round-to-nearest-even) and return float32."""
    return t.to(torch.bfloat16).to(torch.float32)


def has_ve(layer, n_layer=N_LAYER):
    """Value embeddings on every other block counting back from the last (utils/model.py:50-52)."""
    return layer % 2 == (n_layer - 1) % 2


def window_sizes(sequence_len=SEQUENCE_LEN, n_layer=N_LAYER, pattern='SSSL'):
    """Left window per layer (utils/model.py:185-191): S = sequence_len // 2, L = sequence_len, last is L.

    Derived from the configured sequence length, never from the runtime T."""
    long_w, short_w = sequence_len, sequence_len // 2
    sizes = [long_w if pattern.upper()[i % len(pattern)] == 'L' else short_w for i in range(n_layer)]
    sizes[-1] = long_w
    return sizes


def rotary_tables(seq_len=SEQUENCE_LEN * 10, head_dim=HEAD_DIM, base=10000):
    """bf16 cos/sin tables [seq_len, head_dim/2] (utils/model.py:177-183, 144)."""
    inv_freq = 1.0 / base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim)
    t = torch.arange(seq_len, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return freqs.cos().bfloat16(), freqs.sin().bfloat16()


def norm(x):
    """RMSNorm without gain, fp32 compute, eps = 2^-23 (utils/model.py:46-47)."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)).to(x.dtype)


def apply_rotary(x, cos, sin):
    """Half-split rotary on [B, T, H, D] with bf16 tables [T, D/2] (utils/model.py:55-58)."""
    d = x.shape[3] // 2
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    x1, x2 = x[..., :d], x[..., d:]
    return torch.cat([x1 * c + x2 * s, x1 * -s + x2 * c], 3)


def attention(q, k, v, window, dtype=torch.float32):
    """Dense masked softmax(q k^T / sqrt(D)) v on [B, T, H, D]; key k visible to query s iff
    s >= k and s - k <= window (utils/model.py:17-31, flex default scale 1/sqrt(D))."""
    B, T, H, D = q.shape
    qh, kh, vh = (t.transpose(1, 2).to(dtype) for t in (q, k, v))
    scores = qh @ kh.transpose(-1, -2) / math.sqrt(D)
    pos = torch.arange(T)
    mask = (pos[:, None] >= pos[None, :]) & (pos[:, None] - pos[None, :] <= window)
    scores = scores.masked_fill(~mask, float('-inf'))
    return (torch.softmax(scores, -1) @ vh).transpose(1, 2).to(q.dtype)


def matmul_nt(x, w, mode):
    """x [..., in] @ w[out, in]^T under the given rounding mode."""
    if mode == 'fp32':
        return x @ w.t()
    return bf(bf(x) @ bf(w).t())


def lowrank(x, weight, a, b, sign, mode='fp32'):
    """x [m, T, in] through W [out, in] + sign * a b^T per member (train/val/eggroll.py:56-58)."""
    if mode == 'fp32':
        u = x @ b.unsqueeze(-1)
    else:
        u = bf(bf(x) @ bf(b).unsqueeze(-1))
    return matmul_nt(x, weight, mode) + sign[:, None, None] * u * a[:, None, :]


def lowrank_embed(weight, a, b, idx, sign):
    """Rows W[idx] + sign * a[:, idx] b^T for token ids idx [T] (train/val/eggroll.py:61-63)."""
    return weight[idx].unsqueeze(0) + sign[:, None, None] * a[:, idx].unsqueeze(-1) * b[:, None, :]


def head_loss(h, weight, a, b, sign, targets, mode='fp32', head='fp32', slice_members=32):
    """Per-member mean soft-capped CE of the head (train/val/eggroll.py:94-103).

    h: [m, T, D] fp32 (already normalised); weight [V, D]; targets [T] int64."""
    m, length = h.shape[0], h.shape[1]
    out = []
    for c in range(0, m, slice_members):  # 32-member slices as the reference (:96)
        part = slice(c, c + slice_members)
        logits = lowrank(h[part], weight, a[part], b[part], sign[part], head if mode == 'bf16' else 'fp32')
        logits = logits[..., :VOCAB].float()
        logits = SOFTCAP * torch.tanh(logits / SOFTCAP)
        ce = F.cross_entropy(logits.flatten(0, 1), targets.repeat(logits.shape[0]), reduction='none')
        out.append(ce.view(-1, length).mean(-1))
    return torch.cat(out)


def population_loss(p, noise, sign, idx, targets, mode='fp32', head='fp32', cos=None, sin=None,
                    windows=None, return_hidden=False):
    """Mean CE [m] of m perturbed models on one sequence (train/val/eggroll.py:66-103).

    p: name -> parameter (reference state-dict names); noise: name -> (a [m, out], b [m, in]) for
    matrices and embeddings, eps [m, L] for resid_lambdas / x0_lambdas; sign [m] = +-sigma."""
    if cos is None:
        cos, sin = rotary_tables()
    if windows is None:
        windows = window_sizes()
    m, length = sign.shape[0], idx.shape[0]
    cos, sin = cos[:length], sin[:length]
    s = sign[:, None, None]
    x = x0 = norm(lowrank_embed(p['transformer.wte.weight'], *noise['transformer.wte.weight'], idx, sign))
    for i in range(N_LAYER):
        pre = f'transformer.h.{i}.'
        resid = p['resid_lambdas'][i] + s * noise['resid_lambdas'][:, i, None, None]
        mix = p['x0_lambdas'][i] + s * noise['x0_lambdas'][:, i, None, None]
        x = resid * x + mix * x0

        def linear(name, inp):
            return lowrank(inp, p[pre + name], *noise[pre + name], sign, mode)

        h = norm(x)
        q = linear('attn.c_q.weight', h).view(m, length, N_HEAD, HEAD_DIM)
        k = linear('attn.c_k.weight', h).view(m, length, N_HEAD, HEAD_DIM)
        v = linear('attn.c_v.weight', h).view(m, length, N_HEAD, HEAD_DIM)
        if has_ve(i):
            name = f'value_embeds.{i}.weight'
            ve = lowrank_embed(p[name], *noise[name], idx, sign).view(m, length, N_HEAD, HEAD_DIM)
            gate = 2 * torch.sigmoid(linear('attn.ve_gate.weight', h[..., :32]))
            v = v + gate.unsqueeze(-1) * ve
        q, k = norm(apply_rotary(q, cos, sin)), norm(apply_rotary(k, cos, sin))
        # q, k, v reach attention in fp32 (the fp32 rank-1 term promotes lowrank's output; flex runs on fp32
        # operands at TF32 under set_float32_matmul_precision('high'), train/val/eggroll.py:58, :90-91, :184)
        y = attention(q, k, v, windows[i]).reshape(m, length, -1)
        if mode == 'bf16':
            y = bf(y)
        x = x + linear('attn.c_proj.weight', y)
        hid = F.relu(linear('mlp.c_fc.weight', norm(x))).square()
        x = x + linear('mlp.c_proj.weight', hid)
    h = norm(x)
    losses = head_loss(h, p['lm_head.weight'], *noise['lm_head.weight'], sign, targets, mode, head)
    return (losses, h) if return_hidden else losses


def gpt_forward(p, idx, targets=None, loss_reduction='mean', cos=None, sin=None, windows=None):
    """Clean fp32 forward of the fixed model on [B, T] token ids (utils/model.py:193-210)."""
    if cos is None:
        cos, sin = rotary_tables()
    if windows is None:
        windows = window_sizes()
    B, T = idx.shape
    cos, sin = cos[:T], sin[:T]
    x = x0 = norm(p['transformer.wte.weight'][idx])
    for i in range(N_LAYER):
        pre = f'transformer.h.{i}.'
        x = p['resid_lambdas'][i] * x + p['x0_lambdas'][i] * x0
        h = norm(x)
        q = (h @ p[pre + 'attn.c_q.weight'].t()).view(B, T, N_HEAD, HEAD_DIM)
        k = (h @ p[pre + 'attn.c_k.weight'].t()).view(B, T, N_HEAD, HEAD_DIM)
        v = (h @ p[pre + 'attn.c_v.weight'].t()).view(B, T, N_HEAD, HEAD_DIM)
        if has_ve(i):
            ve = p[f'value_embeds.{i}.weight'][idx].view(B, T, N_HEAD, HEAD_DIM)
            gate = 2 * torch.sigmoid(h[..., :32] @ p[pre + 'attn.ve_gate.weight'].t())
            v = v + gate.unsqueeze(-1) * ve
        q, k = norm(apply_rotary(q, cos, sin)), norm(apply_rotary(k, cos, sin))
        y = attention(q, k, v, windows[i]).reshape(B, T, -1)
        x = x + y @ p[pre + 'attn.c_proj.weight'].t()
        h = norm(x)
        x = x + F.relu(h @ p[pre + 'mlp.c_fc.weight'].t()).square() @ p[pre + 'mlp.c_proj.weight'].t()
    x = norm(x)
    logits = (x @ p['lm_head.weight'].t())[..., :VOCAB].float()
    logits = SOFTCAP * torch.tanh(logits / SOFTCAP)
    if targets is None:
        return logits
    return F.cross_entropy(logits.view(-1, logits.size(-1)), targets.view(-1), ignore_index=-1,
                           reduction=loss_reduction)


def attention_bf16(q, k, v, window):
    """torch's attention on bf16 q, k, v [B, T, H, D] (flex, utils/model.py:31, as GPT.forward runs it under autocast):
    fp32 scores of the bf16 operands scaled by 1/sqrt(D), softmax probabilities exp(s - rowmax) rounded to bf16 for
    P V with fp32 accumulation, the normaliser summed from the unrounded probabilities, bf16 output. (The flex
    kernel's running maximum and block order are not restated: parity unpinned below that rounding class.)"""
    B, T, H, D = q.shape
    qh, kh, vh = (t.transpose(1, 2).double() for t in (q, k, v))
    scores = (qh @ kh.transpose(-1, -2) / math.sqrt(D)).float()
    pos = torch.arange(T)
    mask = (pos[:, None] >= pos[None, :]) & (pos[:, None] - pos[None, :] <= window)
    scores = scores.masked_fill(~mask, float('-inf'))
    pr = torch.exp(scores - scores.amax(-1, keepdim=True))
    y = (bf(pr).double() @ vh) / pr.double().sum(-1, keepdim=True)
    return bf(y.float()).transpose(1, 2)


def ac_norm(x):
    """norm of a bf16 tensor under autocast: fp32 mean of squares, eps 2^-23, bf16 result (utils/model.py:46-47;
    torch 2.10's rms_norm computes a bf16 input in fp32 with the fp32 epsilon)."""
    return bf(x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + EPS))


def ac_mix(lam_r, lam_0, x, x0):
    """lambda_r * x + lambda_0 * x0 with 0-d fp32 lambdas on the bf16 stream (utils/model.py:199): type promotion
    casts the lambdas to bf16; the products and the sum round to bf16."""
    return bf(bf(bf(lam_r) * x) + bf(bf(lam_0) * x0))


def ac_rotary(x, cos, sin):
    """apply_rotary_emb (utils/model.py:55-58) on bf16 x [B, T, H, D] and bf16 tables [T, D/2]: every product and
    every sum rounds to bf16."""
    d = x.shape[3] // 2
    c, s = cos.float()[None, :, None, :], sin.float()[None, :, None, :]
    x1, x2 = x[..., :d], x[..., d:]
    return torch.cat([bf(bf(x1 * c) + bf(x2 * s)), bf(bf(x1 * -s) + bf(x2 * c))], 3)


def ac_value_gate(v, gate_logit, ve):
    """v + 2 sigmoid(gate_logit) * ve (utils/model.py:89-90) on bf16 v [B, T, H, D], the bf16 gate logits [B, T, H]
    and the bf16 value embedding: sigmoid rounds to bf16, the doubling is exact, the product and the sum round."""
    gate = 2 * bf(torch.sigmoid(gate_logit))
    return bf(v + bf(gate.unsqueeze(-1) * ve))


def autocast_forward(p, idx, targets=None, loss_reduction='mean', cos=None, sin=None, windows=None,
                     accumulate=torch.float32):
    """GPT.forward (utils/model.py:193-210) as the speedrun's scorer runs it: under CUDA bf16 autocast
    (utils/eval.py:44-45) with the token and value embeddings stored in bf16 (utils/model.py:171-175). Every tensor
    of the stream is bf16 and every op rounds its result to bf16 (torch computes elementwise ops in fp32):

    * norm of a bf16 input (ac_norm; :196, :94, :118-119, :202);
    * the lambda mix (ac_mix, :199);
    * every nn.Linear: bf16 operands, accumulation in `accumulate` (fp32, as the GPU's GEMMs; fp64 gives an equally
      valid rounding for measuring this mode's floor), bf16 output (autocast);
    * the value gate (ac_value_gate, :89-90) and rotary (ac_rotary, :93);
    * attention on bf16 q, k, v (attention_bf16, :95);
    * residual adds rounded; relu(bf16).square() is an exact fp32 square (pow autocasts to fp32), rounded by the
      c_proj's input cast (:107, :118-119);
    * the head's bf16 logits are widened to fp32 before the cap and the cross-entropy (:203-209).

    The dtype rules were checked on the MI355X box against torch 2.10's CUDA autocast: bf16 results for the mix,
    norm, linear and sigmoid; fp32 for relu.square; the mix equals ac_mix; the mix, rotary and value-gate results
    equal torch's CPU bf16 arithmetic bit for bit (which tests/test_oracle.py compares these helpers with)."""
    if cos is None:
        cos, sin = rotary_tables()
    if windows is None:
        windows = window_sizes()
    B, T = idx.shape
    cos, sin = cos[:T], sin[:T]

    def lin(name, x):
        return bf((bf(x).to(accumulate) @ bf(p[name]).to(accumulate).t()).float())

    x = x0 = ac_norm(bf(p['transformer.wte.weight'])[idx])
    for i in range(N_LAYER):
        pre = f'transformer.h.{i}.'
        x = ac_mix(p['resid_lambdas'][i], p['x0_lambdas'][i], x, x0)
        h = ac_norm(x)
        q = lin(pre + 'attn.c_q.weight', h).view(B, T, N_HEAD, HEAD_DIM)
        k = lin(pre + 'attn.c_k.weight', h).view(B, T, N_HEAD, HEAD_DIM)
        v = lin(pre + 'attn.c_v.weight', h).view(B, T, N_HEAD, HEAD_DIM)
        if has_ve(i):
            ve = bf(p[f'value_embeds.{i}.weight'])[idx].view(B, T, N_HEAD, HEAD_DIM)
            v = ac_value_gate(v, lin(pre + 'attn.ve_gate.weight', h[..., :32]), ve)
        q, k = ac_norm(ac_rotary(q, cos, sin)), ac_norm(ac_rotary(k, cos, sin))
        y = attention_bf16(q, k, v, windows[i]).reshape(B, T, -1)
        x = bf(x + lin(pre + 'attn.c_proj.weight', y))
        m = F.relu(lin(pre + 'mlp.c_fc.weight', ac_norm(x))).square()
        x = bf(x + lin(pre + 'mlp.c_proj.weight', m))
    logits = lin('lm_head.weight', ac_norm(x))[..., :VOCAB]
    logits = SOFTCAP * torch.tanh(logits / SOFTCAP)
    if targets is None:
        return logits
    return F.cross_entropy(logits.reshape(-1, logits.size(-1)), targets.reshape(-1), ignore_index=-1,
                           reduction=loss_reduction)


def perturbed_params(p, noise, sign, member):
    """theta + s_p E_p for one member, materialised (test helper for the brute-force pin).

    2-D params: W + s a b^T with a on the output side (train/val/eggroll.py:57); embeddings
    W + s a b^T gathered by row (:63); lambdas: lambda + s eps (:77-78)."""
    out = {}
    s = sign[member]
    for name, w in p.items():
        n = noise[name]
        if isinstance(n, tuple):
            a, b = n[0][member], n[1][member]
            out[name] = w + s * torch.outer(a, b)
        else:
            out[name] = w + s * n[member]
    return out


def mlp_population(x, w1, w2, a1, b1, a2, b2, sign, mode='bf16'):
    """Config-1 fused relu^2 MLP in the reference orientation: W1 = c_fc [F, D], W2 = c_proj [D, F];
    y_p = relu^2(x W1^T + s (x.b1) a1^T) W2^T + s (h.b2) a2^T per member (train/val/eggroll.py:93)."""
    if x.dim() == 2:
        x = x.unsqueeze(0).expand(sign.shape[0], -1, -1)
    hid = F.relu(lowrank(x, w1, a1, b1, sign, mode)).square()
    return lowrank(hid, w2, a2, b2, sign, mode)


def attention_moments(o):
    """Credit moments of an attention output o [P, H, T, D]: per (member, head, dim) mean over tokens of
    o and o^2, fp32 (config-2 definition; no reference function -- closest: head_scores,
    train/val/run.py:192-195)."""
    of = o.float()
    return of.mean(2), of.pow(2).mean(2)


def norm_head_ce(h, gain, weight, a, b, sign, targets):
    """Config-3: RMSNorm with gain (gain = 1 reproduces utils/model.py:46-47) -> fp32 head with rank-1
    perturbation -> soft cap -> CE -> per-member mean. h [P, T, D]; weight [V, D]."""
    hn = norm(h.float()) * gain
    return head_loss(hn, weight, a, b, sign, targets, 'fp32', 'fp32')
