"""Population-perturbed forward of the fixed 37.7M GPT on the gfx950 kernels (the drop-in for
`population_loss`, train/val/eggroll.py:66-103).

The host side only orders kernel launches and owns device buffers (torch tensors); every op of the
forward runs in libnoise_hip.so. Members are evaluated in chunks so activations stay bounded: a chunk
of m members at T tokens holds about m * T * 13 KiB of activations (fp32 residual stream, bf16 q|k|v,
attention output and the 2048-wide MLP hidden; x0 is recomputed, never stored).
"""
import torch

from . import _lib
from .model import GPTConfig, has_ve, window_sizes

D, H, HD, F = 512, 8, 64, 2048
# Head formats: 'fp32' = NOISE_HEAD_FP32 (h rounded once to fp16 against a 22-bit weight, two fp16 MFMA passes),
# 'fp32_split' = NOISE_HEAD_FP32_SPLIT (bf16 hi / lo, three bf16 passes, ~2^-16), 'bf16' = the autocast head.
HEAD_MODES = ('fp32', 'fp32_split', 'bf16')
HEAD_FORMAT = {'fp32': _lib.HEAD_FP32, 'fp32_split': _lib.HEAD_FP32_SPLIT, 'bf16': _lib.HEAD_BF16}


def _p(t):
    return 0 if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _need_cuda(t, dtype, name):
    if t.device.type != 'cuda':
        raise ValueError(f'{name} must be a CUDA tensor (no CPU path)')
    if t.dtype != dtype:
        raise TypeError(f'{name} must be {dtype}, got {t.dtype}')
    if not t.is_contiguous():
        raise ValueError(f'{name} must be contiguous')


class Weights:
    """Per-step device copies of the shared weights in the kernels' formats: bf16 GEMM operands (the
    autocast cast the reference performs inside every matmul, done once per step; the MLP c_proj weight in
    the tile GEMM's WTILE layout) and the head weight in its format (the fp32 parameter itself for 'fp32', whose
    operand the head call derives; the bf16 split for 'fp32_split'). Built from `p` = name -> fp32 parameter
    (train/val/eggroll.py:113)."""

    def __init__(self, p, config=None, head='fp32'):
        if head not in HEAD_MODES:
            raise ValueError(f'head must be one of {HEAD_MODES}')
        self.config = config or GPTConfig()
        self.head = head
        self.p = p
        dev = p['transformer.wte.weight'].device
        s = _stream()
        L = self.config.n_layer
        self.qkv = torch.empty(L, 3 * D, D, device=dev, dtype=torch.bfloat16)
        self.proj = torch.empty(L, D, D, device=dev, dtype=torch.bfloat16)
        self.fc = torch.empty(L, F, D, device=dev, dtype=torch.bfloat16)
        self.mproj = torch.empty(L, D, F, device=dev, dtype=torch.bfloat16)
        # the MLP c_proj weight (K = 2048, the tile GEMM's operand) is kept in the library's WTILE layout
        rows = torch.empty(D, F, device=dev, dtype=torch.bfloat16)
        for i in range(L):
            pre = f'transformer.h.{i}.'
            for k, name in enumerate(('attn.c_q.weight', 'attn.c_k.weight', 'attn.c_v.weight')):
                self._cast(p[pre + name], self.qkv[i, k * D:(k + 1) * D], s)
            self._cast(p[pre + 'attn.c_proj.weight'], self.proj[i], s)
            self._cast(p[pre + 'mlp.c_fc.weight'], self.fc[i], s)
            self._cast(p[pre + 'mlp.c_proj.weight'], rows, s)
            _lib.call('noise_weight_tiles', rows.data_ptr(), D, F, self.mproj[i].data_ptr(), s)
        w_head = p['lm_head.weight']
        V = w_head.shape[0]
        if head == 'fp32':
            _need_cuda(w_head, torch.float32, 'lm_head.weight')
            self.head_w = w_head
        elif head == 'fp32_split':
            self.head_w = torch.empty(V, 3 * D, device=dev, dtype=torch.bfloat16)
            _need_cuda(w_head, torch.float32, 'lm_head.weight')
            _lib.call('noise_cast_bf16', w_head.data_ptr(), self.head_w.data_ptr(), w_head.numel(), D, s)
        else:
            self.head_w = torch.empty(V, D, device=dev, dtype=torch.bfloat16)
            self._cast(w_head, self.head_w, s)

    @staticmethod
    def _cast(src, dst, s):
        _need_cuda(src, torch.float32, 'weight')
        if src.shape != dst.shape:
            raise ValueError(f'weight shape {tuple(src.shape)} != {tuple(dst.shape)}')
        _lib.call('noise_cast_bf16', src.data_ptr(), dst.data_ptr(), src.numel(), 0, s)


class Buffers:
    """Activation buffers for one chunk of `members` members at `T` tokens (reused across chunks)."""

    def __init__(self, members, T, device, head='fp32', vocab=4096):
        M = members * T
        self.members, self.T = members, T
        f32, b16 = torch.float32, torch.bfloat16
        self.x = torch.empty(M, D, device=device, dtype=f32)
        self.h = torch.empty(M, D, device=device, dtype=b16)
        self.u_qkv = torch.empty(M, 4, device=device, dtype=f32)
        self.gate = torch.empty(M, H, device=device, dtype=f32)
        self.qkv = torch.empty(M, 3 * D, device=device, dtype=b16)
        self.y = torch.empty(M, D, device=device, dtype=b16)
        self.u_attn = torch.empty(M, H, device=device, dtype=f32)
        # dense products of the two c_proj GEMMs (their rank-1 terms and residual adds are deferred)
        self.y_ap = torch.empty(M, D, device=device, dtype=b16)
        self.y_mp = torch.empty(M, D, device=device, dtype=b16)
        self.u_fc = torch.empty(M, device=device, dtype=f32)
        self.parts = _lib.value('noise_mlp_fc_parts', F)
        self.hidden = torch.empty(M, F, device=device, dtype=b16)
        self.u_mlp = torch.empty(self.parts, M, device=device, dtype=f32)  # part-major
        ws = _lib.size_query('noise_head_ce_workspace_size', members, T, vocab, HEAD_FORMAT[head])
        self.head_ws = torch.empty(ws, device=device, dtype=torch.uint8)

    def fits(self, members, T):
        return members <= self.members and T == self.T


def _noise_rows(noise, name, lo, hi):
    """Rows lo..hi of a (a, b) pair or of an eps matrix, as contiguous device tensors."""
    n = noise[name]
    if isinstance(n, tuple):
        return tuple(t[lo:hi] for t in n)
    return n[lo:hi]


class StageTimer:
    """Optional per-stage timing of forward_chunk: HIP events recorded on the launch stream around each
    stage (embed, entry, qkv, attention, attn_proj, mlp, head); `ms` accumulates milliseconds per
    stage once `collect()` has synchronised."""

    def __init__(self):
        self.pending = []
        self.ms = {}
        self.count = {}

    def mark(self, stage):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(torch.cuda.current_stream())
        return stage, ev

    def close(self, opened):
        stage, ev0 = opened
        ev1 = torch.cuda.Event(enable_timing=True)
        ev1.record(torch.cuda.current_stream())
        self.pending.append((stage, ev0, ev1))

    def collect(self):
        torch.cuda.synchronize()
        for stage, e0, e1 in self.pending:
            self.ms[stage] = self.ms.get(stage, 0.0) + e0.elapsed_time(e1)
            self.count[stage] = self.count.get(stage, 0) + 1
        self.pending = []
        return self.ms


class _NoTimer:
    def mark(self, stage):
        return None

    def close(self, opened):
        pass


TIMER = _NoTimer()


# q and k reach attention RMS-normalised (noise_qkv applies the QK-norm), so its bounded-score softmax applies
QK_NORM = True


def forward_chunk(W, buf, noise, sign, idx, targets, pair_shift, out, cos, sin, windows, tok_mstride=0,
                  reduction=_lib.CE_MEMBER_MEAN, logits=None):
    """Losses of members 0..m-1 of `sign` (m = len(sign)) into `out` (per member, or reduced as
    `reduction` says); noise rows are indexed by p >> pair_shift. Member p reads the token ids and targets
    at p * tok_mstride (0: one shared sequence). When `logits` is given, the capped logits are written there
    too (targets and out may then be None). Follows train/val/eggroll.py:72-103 op for op."""
    tm = TIMER
    cfg = W.config
    p = W.p
    m, T = sign.shape[0], idx.shape[-1]
    # every launch below sizes its grid from (m, T): refuse anything the buffers or token ids do not cover
    if not buf.fits(m, T):
        raise ValueError(f'buffers hold {buf.members} members x {buf.T} tokens, not {m} x {T}')
    ntok = T if tok_mstride == 0 else (m - 1) * tok_mstride + T
    for name, t in (('idx', idx), ('targets', targets)):
        if t is not None and (not t.is_contiguous() or t.numel() < ntok):
            raise ValueError(f'{name} must be contiguous with >= {ntok} ids for {m} members x {T} tokens')
    if logits is not None and (not logits.is_contiguous() or logits.numel() < m * T * W.head_w.shape[0]):
        raise ValueError(f'logits must be contiguous [{m}, {T}, {W.head_w.shape[0]}]')
    if out is not None:
        nout = m * T if reduction == _lib.CE_NONE else m if reduction == _lib.CE_MEMBER_MEAN else 1
        if out.numel() < nout:
            raise ValueError(f'out must hold {nout} losses')
    s = _stream()
    ps = pair_shift
    a, b = noise['transformer.wte.weight']
    V = p['transformer.wte.weight'].shape[0]
    # x0 = norm(lowrank_embed(wte)) (train/val/eggroll.py:74) is never stored: every block entry recomputes its
    # rows from the L2-resident table (the same arithmetic as noise_embed_norm), which saves reading a 4 KiB
    # per member-token fp32 stream from HBM at each of the n_layer blocks
    emb, emb_ptr = _lib.embed(_p(p['transformer.wte.weight']), V, _p(a), _p(b), _p(idx), tok_mstride)
    eps_r, eps_0 = noise['resid_lambdas'], noise['x0_lambdas']
    lam_r, lam_0 = p['resid_lambdas'], p['x0_lambdas']
    # Deferred residuals. `x = x + lowrank(c_proj, ...)` (train/val/eggroll.py:92-93) is split: the c_proj GEMM
    # writes only its bf16 dense product, and the next kernel that reads the residual stream adds the rank-1
    # term and the residual with the same fp32 operations, in the same order (the MLP entry for the attention
    # output; the next block entry, or the head, for both outputs of a block).
    pend_prev = []
    for i in range(cfg.n_layer):
        pre = f'transformer.h.{i}.'
        aq, bq = noise[pre + 'attn.c_q.weight']
        ak, bk = noise[pre + 'attn.c_k.weight']
        av, bv = noise[pre + 'attn.c_v.weight']
        ve = has_ve(i, cfg.n_layer)
        if ve:
            gw = p[pre + 'attn.ve_gate.weight']
            ga, gb = noise[pre + 'attn.ve_gate.weight']
            vw = p[f'value_embeds.{i}.weight']
            va, vb = noise[f'value_embeds.{i}.weight']
        x_in = None if i == 0 else _p(buf.x)
        t0 = tm.mark('entry')
        pend, npend = _lib.pending(*pend_prev)
        _lib.call('noise_block_entry', x_in, None, _p(buf.x), _p(buf.h), _p(buf.u_qkv), _p(bq), _p(bk),
                  _p(bv), lam_r.data_ptr() + 4 * i, lam_0.data_ptr() + 4 * i, eps_r.data_ptr() + 4 * i,
                  eps_0.data_ptr() + 4 * i, eps_r.stride(0), _p(gw) if ve else 0, _p(ga) if ve else 0,
                  _p(gb) if ve else 0, _p(buf.gate) if ve else 0, _p(sign), m, T, ps, pend, npend, emb_ptr, s)
        tm.close(t0)
        t0 = tm.mark('qkv')
        _lib.call('noise_qkv', _p(buf.h), _p(W.qkv[i]), _p(aq), _p(ak), _p(av), _p(buf.u_qkv), _p(sign), m, T, ps,
                  _p(cos), _p(sin), _p(buf.gate) if ve else 0, _p(vw) if ve else 0, V, _p(va) if ve else 0,
                  _p(vb) if ve else 0, _p(idx), tok_mstride, _p(buf.qkv), s)
        tm.close(t0)
        ap, bp = noise[pre + 'attn.c_proj.weight']
        t0 = tm.mark('attention')
        # q and k come out of noise_qkv RMS-normalised
        _lib.call('noise_attention', _p(buf.qkv), m, T, windows[i], int(QK_NORM), _lib.QK_F16_Q_LOG2, _p(bp), ps,
                  _p(buf.y), _p(buf.u_attn), 0, 0, 0, s)
        tm.close(t0)
        t0 = tm.mark('attn_proj')
        _lib.call('noise_dense_bf16', _p(buf.y), _lib.LAYOUT_ROWS, D, D, _p(W.proj[i]), _lib.LAYOUT_ROWS, m, T,
                  _p(buf.y_ap), s)
        tm.close(t0)
        attn_out = (_p(buf.y_ap), _p(buf.u_attn), H, H, 1, _p(ap))
        af, bf_ = noise[pre + 'mlp.c_fc.weight']
        am, bm = noise[pre + 'mlp.c_proj.weight']
        t0 = tm.mark('mlp_entry')
        pend, npend = _lib.pending(attn_out)
        _lib.call('noise_norm_dot', _p(buf.x), _p(buf.h), _p(bf_), _p(buf.u_fc), _p(sign), m, T, ps, pend, npend, s)
        tm.close(t0)
        t0 = tm.mark('mlp')
        # the hidden stays in the library's TILE16 layout between the two MLP GEMMs
        _lib.call('noise_mlp_fc', _p(buf.h), _p(W.fc[i]), D, F, _p(af), _p(buf.u_fc), _p(bm), _p(sign), m, T, ps,
                  _p(buf.hidden), _lib.LAYOUT_TILE16, _p(buf.u_mlp), s)
        _lib.call('noise_dense_bf16', _p(buf.hidden), _lib.LAYOUT_TILE16, F, D, _p(W.mproj[i]), _lib.LAYOUT_WTILE, m,
                  T, _p(buf.y_mp), s)
        tm.close(t0)
        # the fc partials are part-major with stride m * T (this chunk's rows)
        mlp_out = (_p(buf.y_mp), _p(buf.u_mlp), buf.parts, 1, m * T, _p(am))
        pend_prev = [attn_out, mlp_out]
    ah, bh = noise['lm_head.weight']
    Vh = W.head_w.shape[0]
    t0 = tm.mark('head')
    pend, npend = _lib.pending(*pend_prev)
    _lib.call('noise_head_ce', _p(buf.x), 0, 0, _p(W.head_w), Vh, HEAD_FORMAT[W.head], _p(ah), _p(bh), _p(sign),
              _p(targets), tok_mstride, m, T, ps, reduction, _p(out), _p(logits), _p(buf.head_ws), buf.head_ws.numel(),
              pend, npend, s)
    tm.close(t0)


def check_noise(noise, shapes, rows):
    for name, shape in shapes.items():
        n = noise[name]
        if len(shape) == 2:
            a, b = n
            _need_cuda(a, torch.float32, f'noise[{name}][0]')
            _need_cuda(b, torch.float32, f'noise[{name}][1]')
            if a.shape[0] < rows or b.shape[0] < rows or a.shape[1] != shape[0] or b.shape[1] != shape[1]:
                raise ValueError(f'noise[{name}] must be ([>= {rows}, {shape[0]}], [>= {rows}, {shape[1]}])')
        else:
            _need_cuda(n, torch.float32, f'noise[{name}]')
            if n.shape[0] < rows or n.shape[1] != shape[0]:
                raise ValueError(f'noise[{name}] must be [>= {rows}, {shape[0]}]')


class Population:
    """Evaluates populations of one model: keeps the kernels' weight formats and activation buffers.

    chunk -- members per forward pass (activation memory ~ chunk * T * 17 KiB);
    head  -- 'fp32' (fp32-accurate head) or 'bf16' (the reference's autocast head)."""

    def __init__(self, model, chunk=256, head='fp32'):
        self.model = model
        self.config = model.config
        self.chunk, self.head = chunk, head
        self.windows = [w for w, _ in model.window_sizes]
        self._buf = None
        self._cos_sin = None

    def tables(self, T):
        cos = self.model.cos[0, :, 0, :]
        sin = self.model.sin[0, :, 0, :]
        if cos.shape[0] < T:
            raise ValueError(f'rotary tables cover {cos.shape[0]} positions < T = {T}')
        if self._cos_sin is None or self._cos_sin[0].device != cos.device:
            self._cos_sin = (cos.to(torch.bfloat16).contiguous(), sin.to(torch.bfloat16).contiguous())
        return self._cos_sin

    def buffers(self, members, T, device):
        if self._buf is None or not self._buf.fits(members, T):
            self._buf = None
            self._buf = Buffers(members, T, device, self.head, self.model.lm_head.weight.shape[0])
        return self._buf

    def loss(self, p, noise, sign, idx, targets, pair_shift=0, weights=None):
        """Per-member mean CE [m] fp32 (train/val/eggroll.py:66-103). noise rows are per member
        (pair_shift 0, as population_loss receives them) or per antithetic pair (pair_shift 1). idx and
        targets are one sequence [T] shared by every member, or one row per member [m, T] (the members of
        several sequences in one pass, as `Eggroll.step` spreads them, train/val/eggroll.py:133-143)."""
        m, T = sign.shape[0], idx.shape[-1]
        dev = sign.device
        per_member = idx.dim() == 2
        if idx.dim() not in (1, 2) or targets.shape != idx.shape or (per_member and idx.shape[0] != m):
            raise ValueError(f'idx and targets must both be [T] or both [{m}, T]')
        _need_cuda(sign, torch.float32, 'sign')
        _need_cuda(idx, torch.int64, 'idx')
        _need_cuda(targets, torch.int64, 'targets')
        idx, targets = idx.contiguous(), targets.contiguous()
        if T % 128:
            raise ValueError(f'T = {T} must be a multiple of 128 (attention query blocks)')
        V = p['transformer.wte.weight'].shape[0]
        lo = torch.minimum(idx.min(), targets.min()).item()
        hi = torch.maximum(idx.max(), targets.max()).item()
        if lo < 0 or hi >= V:
            raise IndexError(f'token ids must lie in [0, {V}), got [{lo}, {hi}]')
        rows = (m + (1 << pair_shift) - 1) >> pair_shift
        check_noise(noise, {n: tuple(t.shape) for n, t in p.items()}, rows)
        W = weights or Weights(p, self.config, self.head)
        cos, sin = self.tables(T)
        out = torch.empty(m, device=dev, dtype=torch.float32)
        step = self.chunk if pair_shift == 0 else self.chunk - self.chunk % 2
        buf = self.buffers(min(step, m), T, dev)
        for c0 in range(0, m, step):
            c1 = min(m, c0 + step)
            r0, r1 = c0 >> pair_shift, (c1 + (1 << pair_shift) - 1) >> pair_shift
            chunk_noise = {n: _noise_rows(noise, n, r0, r1) for n in p}
            ci, ct = (idx[c0:c1], targets[c0:c1]) if per_member else (idx, targets)
            forward_chunk(W, buf, chunk_noise, sign[c0:c1], ci, ct, pair_shift, out[c0:c1], cos, sin,
                          self.windows, tok_mstride=T if per_member else 0)
        return out


def population_loss(model, p, noise, sign, idx, targets, head='fp32', chunk=256):
    """Drop-in for `population_loss(model, p, noise, sign, idx, targets)` (train/val/eggroll.py:66-103):
    mean cross-entropy [m] of m perturbed models on one sequence, evaluated by the HIP kernels."""
    return Population(model, chunk=chunk, head=head).loss(p, noise, sign, idx, targets)


REDUCTIONS = {'mean': _lib.CE_MEAN, 'sum': _lib.CE_SUM, 'none': _lib.CE_NONE}
ROUNDINGS = ('population', 'autocast')


def _check_clean_inputs(model, idx, targets, loss_reduction):
    if loss_reduction not in REDUCTIONS:
        raise ValueError(f"loss_reduction must be one of {tuple(REDUCTIONS)}, got {loss_reduction!r}")
    _need_cuda(idx, torch.int64, 'idx')
    if idx.dim() != 2:
        raise ValueError(f'idx must be [B, T], got {tuple(idx.shape)}')
    B, T = idx.shape
    if T % 128:
        raise ValueError(f'T = {T} must be a multiple of 128 (attention query blocks)')
    V = model.transformer.wte.weight.shape[0]
    if idx.min().item() < 0 or idx.max().item() >= V:
        raise IndexError(f'token ids must lie in [0, {V})')
    if targets is not None:
        _need_cuda(targets, torch.int64, 'targets')
        if targets.shape != idx.shape:
            raise ValueError(f'targets must be {tuple(idx.shape)}, got {tuple(targets.shape)}')
        valid = targets != -1
        if ((targets < 0) & valid).any().item() or (targets >= V).any().item():
            raise IndexError(f'targets must lie in [0, {V}) or be -1 (ignored)')
    return B, T, V


def autocast_forward(model, idx, targets=None, loss_reduction='mean', weights=None):
    """GPT.forward (utils/model.py:193-210) on the HIP kernels at the rounding points the speedrun's scorer gives it:
    torch's bf16 autocast with the token and value embeddings stored in bf16 (utils/eval.py:44-45,
    utils/model.py:171-175). The residual stream is bf16 and every op rounds to bf16: noise_ac_stream (embedding
    norm, residual adds, lambda mix, norms, value gate), noise_dense_bf16 (every nn.Linear: bf16 operands, fp32
    accumulation, bf16 output), noise_ac_qkv (rotary and QK norm in bf16, value embedding), noise_attention on bf16
    q, k, v with bf16 probabilities, noise_mlp_fc at sigma = 0 (relu(bf16)^2 rounded to bf16 where c_proj casts it)
    and the bf16 head with the fp32 cap and cross-entropy (noise_head_ce). Same returns as clean_forward. The
    embedding tables are read as bf16 (fp32 tensors holding bf16 values, as noise_amd.eval.load_model keeps them)."""
    B, T, V = _check_clean_inputs(model, idx, targets, loss_reduction)
    cfg = model.config
    p = dict(model.named_parameters())
    dev = idx.device
    W = weights or Weights(p, cfg, 'bf16')
    if W.head != 'bf16':
        raise ValueError("the autocast forward needs bf16 head weights (Weights(p, config, 'bf16'))")
    s = _stream()
    M = B * T
    b16 = torch.bfloat16
    x, h, xf = (torch.empty(M, D, device=dev, dtype=b16) for _ in range(3))
    y, y_ap, y_mp = (torch.empty(M, D, device=dev, dtype=b16) for _ in range(3))
    qkv = torch.empty(M, 3 * D, device=dev, dtype=b16)
    hidden = torch.empty(M, F, device=dev, dtype=b16)
    gate = torch.empty(M, H, device=dev)
    parts = _lib.value('noise_mlp_fc_parts', F)
    upart = torch.empty(parts, M, device=dev)
    # sigma = 0: zero rank-1 vectors and signs, so noise_mlp_fc and the head add exactly nothing
    zf, zb, zu, zsign = (torch.zeros(B, F, device=dev), torch.zeros(B, F, device=dev), torch.zeros(M, device=dev),
                         torch.zeros(B, device=dev))
    za, zbh = torch.zeros(B, W.head_w.shape[0], device=dev), torch.zeros(B, D, device=dev)
    pop = Population(model, chunk=B, head='bf16')
    cos, sin = pop.tables(T)
    idx = idx.contiguous()
    wte = p['transformer.wte.weight']
    lam_r, lam_0 = p['resid_lambdas'], p['x0_lambdas']
    for i in range(cfg.n_layer):
        pre = f'transformer.h.{i}.'
        ve = has_ve(i, cfg.n_layer)
        first = i == 0
        _lib.call('noise_ac_stream', None if first else _p(x), _p(wte), V, _p(idx), T, None if first else _p(y_ap),
                  None if first else _p(y_mp), lam_r.data_ptr() + 4 * i, lam_0.data_ptr() + 4 * i, _p(x), _p(h),
                  _p(p[pre + 'attn.ve_gate.weight']) if ve else None, _p(gate) if ve else None, M, T, s)
        _lib.call('noise_dense_bf16', _p(h), _lib.LAYOUT_ROWS, D, 3 * D, _p(W.qkv[i]), _lib.LAYOUT_ROWS, B, T, _p(qkv), s)
        vw = p[f'value_embeds.{i}.weight'] if ve else None
        _lib.call('noise_ac_qkv', _p(qkv), _p(cos), _p(sin), _p(gate) if ve else None, _p(vw), V if ve else 0,
                  _p(idx), T, M, T, s)
        _lib.call('noise_attention', _p(qkv), B, T, pop.windows[i], 1, _lib.QK_BF16_V_BF16, None, 0, _p(y), None, None,
                  None, 0, s)
        _lib.call('noise_dense_bf16', _p(y), _lib.LAYOUT_ROWS, D, D, _p(W.proj[i]), _lib.LAYOUT_ROWS, B, T, _p(y_ap), s)
        _lib.call('noise_ac_stream', _p(x), None, 0, None, 0, _p(y_ap), None, None, None, None, _p(h), None, None, M, T,
                  s)
        _lib.call('noise_mlp_fc', _p(h), _p(W.fc[i]), D, F, _p(zf), _p(zu), _p(zb), _p(zsign), B, T, 0, _p(hidden),
                  _lib.LAYOUT_TILE16, _p(upart), s)
        _lib.call('noise_dense_bf16', _p(hidden), _lib.LAYOUT_TILE16, F, D, _p(W.mproj[i]), _lib.LAYOUT_WTILE, B, T,
                  _p(y_mp), s)
    _lib.call('noise_ac_stream', _p(x), None, 0, None, 0, _p(y_ap), _p(y_mp), None, None, _p(xf), None, None, None, M, T,
              s)
    Vh = W.head_w.shape[0]
    ws = torch.empty(_lib.size_query('noise_head_ce_workspace_size', B, T, Vh, 0), device=dev, dtype=torch.uint8)
    if targets is None:
        logits = torch.empty(B, T, Vh, device=dev)
        _lib.call('noise_head_ce', _p(xf), 1, None, _p(W.head_w), Vh, 0, _p(za), _p(zbh), _p(zsign), None, T, B, T, 0,
                  _lib.CE_MEMBER_MEAN, None, _p(logits), _p(ws), ws.numel(), None, 0, s)
        return logits
    red = REDUCTIONS[loss_reduction]
    out = torch.empty(M if red == _lib.CE_NONE else 1, device=dev)
    _lib.call('noise_head_ce', _p(xf), 1, None, _p(W.head_w), Vh, 0, _p(za), _p(zbh), _p(zsign),
              _p(targets.contiguous()), T, B, T, 0, red, _p(out), None, _p(ws), ws.numel(), None, 0, s)
    return out if red == _lib.CE_NONE else out[0]


def clean_forward(model, idx, targets=None, loss_reduction='mean', head='fp32', weights=None):
    """GPT.forward (utils/model.py:193-210) on the HIP kernels.

    The clean model is the population forward at sigma = 0: the B batch rows run as B members in one pass,
    member b reading its own sequence (token stride T), with zero signs, so every rank-1 term and every
    lambda perturbation vanishes exactly. With targets, the loss is F.cross_entropy of the capped logits with
    ignore_index = -1 and `loss_reduction` 'mean' / 'sum' (0-dim) or 'none' ([B * T]); without, the capped
    fp32 logits [B, T, vocab] are returned. The kernels keep the rounding points of the population path (fp32
    residual stream and norms, bf16 GEMMs, fp16 attention operands), not the all-bf16 stream GPT.forward has under
    autocast with bf16 embeddings; head='fp32' keeps the head fp32-accurate, 'bf16' rounds it as autocast does."""
    B, T, V = _check_clean_inputs(model, idx, targets, loss_reduction)
    p = dict(model.named_parameters())
    dev = idx.device
    # sigma = 0: zero signs and zero noise rows (finite, so s * (x . b) * a is exactly zero)
    noise = {n: (torch.zeros(B, t.shape[0], device=dev), torch.zeros(B, t.shape[1], device=dev)) if t.dim() == 2
             else torch.zeros(B, t.shape[0], device=dev) for n, t in p.items()}
    sign = torch.zeros(B, device=dev)
    pop = Population(model, chunk=B, head=head)
    W = weights or Weights(p, model.config, head)
    cos, sin = pop.tables(T)
    buf = pop.buffers(B, T, dev)
    if targets is None:
        logits = torch.empty(B, T, W.head_w.shape[0], device=dev, dtype=torch.float32)
        forward_chunk(W, buf, noise, sign, idx, None, 0, None, cos, sin, pop.windows, tok_mstride=T, logits=logits)
        return logits
    red = REDUCTIONS[loss_reduction]
    out = torch.empty(B * T if red == _lib.CE_NONE else 1, device=dev, dtype=torch.float32)
    forward_chunk(W, buf, noise, sign, idx, targets, 0, out, cos, sin, pop.windows, tok_mstride=T, reduction=red)
    return out if red == _lib.CE_NONE else out[0]
