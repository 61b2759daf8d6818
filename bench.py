"""Benchmark of the population-perturbed forward + EGGROLL update on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload step|mlp] [--no-cpu-baseline]

Default workload (the full population step on one GPU's share): the 37.7M
model (8 layers, d 512, vocab 4096) with bf16 GEMM weights and an fp32 head, 3072 members = 1536
antithetic pairs of rank-1 perturbations on every matrix and embedding (Gaussian on the 16 mixing
scalars), sigma = 1e-3, one 2048-token Zipf(1.1) sequence; then the rank-normalised fitness, the
fitness-weighted sum of the perturbation outer products and an Adam step on all 37,749,776 weights.
One step = all of that (Eggroll.step). All 3072 members run as one pass of the kernels (`--chunk`, about
105 GB of activations in HBM; smaller chunks run the same kernels on fewer rows per launch). Weights are the reference's seed-0 initialisation, data is
synthetic and resident in HBM before the timed region.

`--workload mlp` times BASELINE config 1 alone (the rank-1-perturbed relu^2 MLP, P = 256, T = 2048,
shared x); `--workload attention` config 2 (windowed causal attention + per-head moments, P = 256,
8 heads, T = 2048); `--workload head` config 3 (RMSNorm with gain + fp32 head + soft-capped CE,
P = 512, T = 2048). `--workload stream` measures the HBM ceilings of the row kernels' read / write mixes with the
library's own streaming kernel; `--workload library` times the vendor GEMM on the fused MLP's shapes (a reference
point); `--workload copy` calibrates the PMC traffic counters; `--workload probes` and `--workload credit` time the
readout probes (row f3) and the credit kernels of one rerun chunk (row f4). Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = 'perturbed member-tokens/sec on 1 GPU; fused-MLP MFMA % of bf16 peak'
PEAK_BF16_TFLOPS = 2500.0         # MI355X dense bf16 MFMA
D, F, T, V, L = 512, 2048, 2048, 4096, 8
SIGMA = 1e-3
# how each head format (noise_amd.population.HEAD_FORMAT: noise_head_ce's NOISE_HEAD_*) runs
HEAD_DESC = {'fp32': 'fp32 (fp16 h x fp16 hi/lo weight: 2 MFMA passes)',
             'fp32_split': 'fp32 (bf16 hi/lo split: 3 MFMA passes)', 'bf16': 'bf16 (autocast rounding)'}
MLP_FLOP_PER_MEMBER_TOKEN = 2 * (2 * D * F)  # both MLP GEMMs, counted per member
# per member-token algorithmic FLOPs of the forward: dense GEMMs (q, k, v, proj, fc, mlp proj per layer,
# ve_gate, head) and window-aware attention at T = 2048 (QK^T and PV over the visible keys)
DENSE_FLOP = L * 2 * (4 * D * D + 2 * D * F) + 4 * 2 * 32 * 8 + 2 * D * V


def attention_flop_per_token(T, windows, H=8, hd=64):
    pairs = sum(sum(min(q, w) + 1 for q in range(T)) for w in windows)
    return 4 * hd * H * pairs / T


def roofline_traffic(chunk):
    """HBM bytes of one MLP launch pair, from the PMC passes recorded in profiles/mlp_traffic.json (measured
    at its `chunk_members`; every kernel of the pair streams per row, so another chunk scales the bytes by
    the ratio of rows)."""
    path = ROOT / 'profiles' / 'mlp_traffic.json'
    if not path.exists():
        return None
    rec = json.loads(path.read_text())
    b, c = rec.get('hbm_bytes_per_launch'), rec.get('chunk_members')
    if b is None or not c:
        return None
    return b if c == chunk else b * chunk / c


def cpu_baseline_step(budget_s=15.0):
    """The CPU oracle (fp32 port of population_loss: what the reference computes on a CPU) on a bounded
    sample of the config-4 workload: antithetic pairs of members on the same 2048-token sequence, as
    many as fit the time budget (at least one pair)."""
    from oracle import model as om
    from noise_amd.model import make_model
    from noise_amd.synthetic import antithetic_signs, population_noise, zipf_tokens
    threads = min(int(os.environ.get('OMP_NUM_THREADS', os.cpu_count() or 1)), os.cpu_count() or 1)
    torch.set_num_threads(threads)
    model = make_model('cpu', 0)
    params = {n: p.detach() for n, p in model.named_parameters()}
    shapes = {n: tuple(p.shape) for n, p in params.items()}
    idx, tgt = zipf_tokens(T, seed=1)
    done, t0 = 0, time.perf_counter()
    while done == 0 or time.perf_counter() - t0 < budget_s:
        noise = population_noise(shapes, 1, seed=2 + done)
        om.population_loss(params, noise, antithetic_signs(2, SIGMA), idx, tgt, mode='fp32', head='fp32')
        done += 2
        if done >= 64:
            break
    dt = time.perf_counter() - t0
    return {'value': done * T / dt, 'unit': 'member-tokens/s', 'cores': threads, 'kind': 'port',
            'sample': f'{done} members ({done // 2} antithetic pairs) x {T} tokens of the config-4 forward through '
                      f'oracle.model.population_loss (torch CPU fp32, dense masked attention), {dt:.1f} s'}


def cpu_baseline_mlp(budget_s=12.0):
    """The CPU oracle of the config-1 MLP (bf16 rounding points emulated in fp32) on whole 2048-token
    members of one antithetic pair, repeated for the time budget."""
    from oracle import model as om
    threads = min(int(os.environ.get('OMP_NUM_THREADS', os.cpu_count() or 1)), os.cpu_count() or 1)
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, D, generator=g).bfloat16().float()
    w1 = (torch.randn(F, D, generator=g) * D ** -0.5).bfloat16().float()
    w2 = (torch.randn(D, F, generator=g) * F ** -0.5).bfloat16().float()
    a1, b1, a2, b2 = (torch.randn(2, n, generator=g) for n in (F, D, D, F))
    sign = torch.tensor([SIGMA, -SIGMA])
    done, t0 = 0, time.perf_counter()
    while done == 0 or time.perf_counter() - t0 < budget_s:
        om.mlp_population(x, w1, w2, a1, b1, a2, b2, sign, 'bf16')
        done += 2
    dt = time.perf_counter() - t0
    return {'value': done * T / dt, 'unit': 'member-tokens/s', 'cores': threads, 'kind': 'port',
            'sample': f'{done} members x {T} tokens of config 1 through oracle.model.mlp_population '
                      f'(torch CPU, bf16 rounding points emulated in fp32), {dt:.1f} s'}


def run_step(args):
    from noise_amd import population
    from noise_amd.eggroll import Eggroll, LR, BETAS
    from noise_amd.model import make_model
    from noise_amd.optim import Adam
    from noise_amd.synthetic import trained_like, zipf_tokens

    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    pairs = args.pairs
    P = 2 * pairs
    model = make_model(dev, 0)
    if args.weights == 'trained':
        # lm_head, ve_gate and the lambdas at trained-model scale (the seed-0 init leaves them degenerate: the MFMA
        # clock depends on the operand data, so both step times are recorded)
        trained_like(model)
    es = Eggroll(model, pairs, chunk=args.chunk, head=args.head, fitness=args.fitness, sigma=SIGMA)
    opt = Adam(model.parameters(), lr=LR, betas=BETAS, eps=1e-8)
    idx, tgt = zipf_tokens(T, seed=1)
    x, y = idx[None].to(dev), tgt[None].to(dev)
    for w in range(args.warmup):
        es.step(x, y, opt, w + 1)
    torch.cuda.synchronize()
    timer = population.StageTimer()
    population.TIMER = timer
    t0 = time.perf_counter()
    for k in range(args.steps):
        loss = es.step(x, y, opt, args.warmup + k + 1)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    population.TIMER = population._NoTimer()
    stages = timer.collect()
    ms_step = wall * 1e3 / args.steps
    windows = [w for w, _ in model.window_sizes]
    flop_tok = DENSE_FLOP + attention_flop_per_token(T, windows)
    # the fused MLP (c_fc relu^2 GEMM + c_proj GEMM) of every layer and chunk, timed with HIP events on the
    # launch stream inside the timed steps
    mlp_launches = timer.count['mlp']
    mlp_ms = stages['mlp'] / mlp_launches
    mlp_flop = MLP_FLOP_PER_MEMBER_TOKEN * (P * T) * L * args.steps / mlp_launches  # per launch (one layer, one chunk)
    achieved = mlp_flop / (mlp_ms * 1e-3) / 1e12
    result = {
        'metric': METRIC,
        'value': P * T / (ms_step * 1e-3),
        'unit': 'member-tokens/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': ms_step,
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16',
        'data': 'synthetic (Zipf(1.1) tokens, ' + ('seed-0 reference init' if args.weights == 'init' else
                                                   'seed-0 init with trained-scale lm_head, ve_gate and lambdas') +
                ', N(0,1) noise buffer)',
        'config': {'workload': 'config4_population_step', 'members': P, 'pairs': pairs, 'tokens': T,
                   'layers': 8, 'd_model': 512, 'vocab': 4096,
                   'head': HEAD_DESC[args.head],
                   'sigma': SIGMA, 'fitness': args.fitness, 'optimizer': 'Adam (HIP)', 'chunk_members': args.chunk,
                   'gpus': 1},
        'roofline': {'bound': 'mfma', 'achieved': achieved, 'peak': PEAK_BF16_TFLOPS, 'unit': 'TFLOP/s',
                     'frac': achieved / PEAK_BF16_TFLOPS, 'traffic': roofline_traffic(args.chunk),
                     'kernel': 'fused relu^2 MLP: xs_relu2_kernel (c_fc, weight-resident) + lowrank_gemm<EPI_DENSE> (c_proj)',
                     'flop_per_launch': mlp_flop, 'ms_per_launch': mlp_ms},
        'forward_tflops': flop_tok * P * T / (sum(v for k, v in stages.items()) / args.steps * 1e-3) / 1e12,
        'stage_ms_per_step': {k: v / args.steps for k, v in stages.items()},
        'mean_population_loss': loss,
    }
    return result


def run_mlp(args):
    from noise_amd import ops
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    P = 256
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, D, generator=g).bfloat16()
    w1 = (torch.randn(F, D, generator=g) * D ** -0.5).bfloat16()
    w2 = (torch.randn(D, F, generator=g) * F ** -0.5).bfloat16()
    pairs = P // 2
    a1, b1 = torch.randn(pairs, F, generator=g), torch.randn(pairs, D, generator=g)
    a2, b2 = torch.randn(pairs, D, generator=g), torch.randn(pairs, F, generator=g)
    sign = torch.tensor([SIGMA, -SIGMA]).repeat(pairs)
    x, w1, w2, a1, b1, a2, b2, sign = (t.to(dev) for t in (x, w1, w2, a1, b1, a2, b2, sign))
    y = torch.empty(P, T, D, device=dev, dtype=torch.bfloat16)
    ws = torch.empty(ops.mlp_workspace_bytes(P, T, D, F), device=dev, dtype=torch.uint8)

    def step():
        ops.lowrank_mlp(x, w1, w2, a1, b1, a2, b2, sign, T=T, pair_shift=1, out=y, workspace=ws)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    ms_launch = ev0.elapsed_time(ev1) / args.steps
    flop = MLP_FLOP_PER_MEMBER_TOKEN * P * T
    achieved = flop / (ms_launch * 1e-3) / 1e12
    return {
        'metric': METRIC, 'value': P * T / (ms_step * 1e-3), 'unit': 'member-tokens/s', 'n_gpus': 1,
        'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': ms_step, 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16', 'data': 'synthetic',
        'config': {'workload': 'config1_fused_relu2_mlp_rank1', 'members': P, 'pairs': pairs, 'tokens': T,
                   'd_model': D, 'd_hidden': F, 'sigma': SIGMA, 'x': 'shared [2048, 512]', 'output': 'bf16',
                   'gpus': 1},
        'roofline': {'bound': 'mfma', 'achieved': achieved, 'peak': PEAK_BF16_TFLOPS, 'unit': 'TFLOP/s',
                     'frac': achieved / PEAK_BF16_TFLOPS, 'traffic': None,
                     'kernel': 'noise_lowrank_mlp (rowdot + xs_relu2_kernel + lowrank_gemm<EPI_STORE> proj)',
                     'flop_per_launch': flop, 'ms_per_launch': ms_launch},
    }


def _timed(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        fn()
    ev1.record(stream)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps, ev0.elapsed_time(ev1) / steps


def _common(args, value, ms_step, config, roofline):
    return {'metric': METRIC, 'value': value, 'unit': 'member-tokens/s', 'n_gpus': 1, 'steps': args.steps,
            'warmup': args.warmup, 'ms_per_step': ms_step, 'higher_is_better': True, 'scaling': 'weak',
            'vs_baseline': None, 'dtype': 'bf16', 'data': 'synthetic', 'config': config, 'roofline': roofline}


def run_attention(args):
    """Config 2: windowed causal attention + credit moments on q | k | v rows (P = 256, H = 8, T = 2048)."""
    from noise_amd import _lib
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    P, window = 256, args.window
    g = torch.Generator(device=dev).manual_seed(0)
    qkv = torch.randn(P * T, 3 * D, device=dev, generator=g)
    if args.qk_norm:
        # q and k rows RMS-normalised per head, as the model's QK-norm leaves them (utils/model.py:46-47)
        qk = qkv[:, :2 * D].view(P * T, 16, 64)
        qkv[:, :2 * D] = (qk * torch.rsqrt(qk.pow(2).mean(-1, keepdim=True) + 2 ** -23)).view(P * T, 2 * D)
    qkv16 = qkv.to(torch.bfloat16)
    # config 2's bf16 q, k (NOISE_QK_BF16 below); v travels as fp16 (here holding the bf16 value exactly)
    qkv16[:, 2 * D:] = qkv16[:, 2 * D:].half().view(torch.bfloat16)
    qkv = qkv16
    y = torch.empty(P * T, D, device=dev, dtype=torch.bfloat16)
    up = torch.empty(P * T, 8, device=dev)
    bp = torch.randn(P, D, device=dev, generator=g)
    mom = torch.empty(P, 8, 2, 64, device=dev)
    ws = torch.empty(_lib.size_query('noise_attention_workspace_size', P, T), device=dev, dtype=torch.uint8)
    s = torch.cuda.current_stream().cuda_stream

    def step():
        _lib.call('noise_attention', qkv.data_ptr(), P, T, window, int(args.qk_norm), 0, bp.data_ptr(), 0, y.data_ptr(),
                  up.data_ptr(), mom.data_ptr(), ws.data_ptr(), ws.numel(), s)
    ms_step, ms_launch = _timed(step, args.steps, args.warmup)
    pairs = sum(min(q, window) + 1 for q in range(T))
    flop = 4 * 64 * 8 * P * pairs
    achieved = flop / (ms_launch * 1e-3) / 1e12
    return _common(args, P * T / (ms_step * 1e-3), ms_step,
                   {'workload': 'config2_attention_moments', 'members': P, 'heads': 8, 'tokens': T, 'head_dim': 64,
                    'window': window, 'q_k': 'RMS-normalised rows (QK-norm)' if args.qk_norm else 'N(0,1)',
                    'outputs': 'y bf16, c_proj dot partials, per-head mean of y and y^2',
                    'gpus': 1},
                   {'bound': 'mfma', 'achieved': achieved, 'peak': PEAK_BF16_TFLOPS, 'unit': 'TFLOP/s',
                    'frac': achieved / PEAK_BF16_TFLOPS, 'traffic': None, 'kernel': 'attention_kernel + moments_reduce',
                    'flop_per_launch': flop, 'ms_per_launch': ms_launch})


def run_head(args):
    """Config 3: RMSNorm (gain ~ U(0.9, 1.1)) + fp32 head (rank-1 perturbed) + soft-capped CE, P = 512."""
    from noise_amd import _lib
    from noise_amd.synthetic import antithetic_signs, zipf_tokens
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    P = 512
    g = torch.Generator(device=dev).manual_seed(0)
    h = torch.randn(P * T, D, device=dev, generator=g).to(torch.bfloat16)
    gain = 0.9 + 0.2 * torch.rand(D, device=dev, generator=g)
    W = torch.randn(V, D, device=dev, generator=g) * D ** -0.5
    a, b = torch.randn(P // 2, V, device=dev, generator=g), torch.randn(P // 2, D, device=dev, generator=g)
    sign = antithetic_signs(P, SIGMA).to(dev)
    tgt = zipf_tokens(T, seed=1)[1].to(dev)
    from noise_amd.population import HEAD_FORMAT
    s = torch.cuda.current_stream().cuda_stream
    fmt = HEAD_FORMAT[args.head]
    if fmt == _lib.HEAD_FP32:
        w_op = W  # the call derives its fp16 operand from the fp32 weight
    else:
        w_op = torch.empty(V, 3 * D if fmt == _lib.HEAD_FP32_SPLIT else D, device=dev, dtype=torch.bfloat16)
        _lib.call('noise_cast_bf16', W.data_ptr(), w_op.data_ptr(), W.numel(), D if fmt == _lib.HEAD_FP32_SPLIT else 0, s)
    loss = torch.empty(P, device=dev)
    ws = torch.empty(_lib.size_query('noise_head_ce_workspace_size', P, T, V, fmt), device=dev, dtype=torch.uint8)

    def step():
        _lib.call('noise_head_ce', h.data_ptr(), 1, gain.data_ptr(), w_op.data_ptr(), V, fmt, a.data_ptr(),
                  b.data_ptr(), sign.data_ptr(), tgt.data_ptr(), 0, P, T, 1, _lib.CE_MEMBER_MEAN, loss.data_ptr(), None,
                  ws.data_ptr(), ws.numel(), None, 0, s)
    ms_step, ms_launch = _timed(step, args.steps, args.warmup)
    flop = 2 * D * V * P * T  # algorithmic fp32 head FLOPs (run as 2 fp16 or 3 bf16 MFMA passes)
    achieved = flop / (ms_launch * 1e-3) / 1e12
    return _common(args, P * T / (ms_step * 1e-3), ms_step,
                   {'workload': 'config3_norm_head_ce', 'members': P, 'tokens': T, 'd_model': D, 'vocab': V,
                    'head': HEAD_DESC[args.head], 'sigma': SIGMA, 'gpus': 1},
                   {'bound': 'mfma', 'achieved': achieved, 'peak': PEAK_BF16_TFLOPS, 'unit': 'TFLOP/s',
                    'frac': achieved / PEAK_BF16_TFLOPS, 'traffic': None,
                    'kernel': 'head_norm + lowrank_gemm<EPI_CE%s> + ce_finalize' % ('_F16' if fmt == _lib.HEAD_FP32 else ''),
                    'flop_per_launch': flop,
                    'ms_per_launch': ms_launch})


def run_copy(args):
    """A plain 1 GiB device-to-device copy: the known-size kernel that calibrates the FETCH_SIZE and
    WRITE_SIZE counters (read 1 GiB, write 1 GiB per launch) and a check of the HBM roofline."""
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    n = 1 << 29
    src = torch.ones(n, device=dev, dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    ms_step, ms_launch = _timed(lambda: dst.copy_(src), args.steps, args.warmup)
    nbytes = 2 * 2 * n
    achieved = nbytes / (ms_launch * 1e-3) / 1e9
    return {'metric': 'device copy bandwidth (counter calibration)', 'value': achieved, 'unit': 'GB/s', 'n_gpus': 1,
            'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': ms_step, 'higher_is_better': True,
            'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16', 'data': 'synthetic',
            'config': {'workload': 'copy_1GiB', 'bytes_read': 2 * n, 'bytes_written': 2 * n},
            'roofline': {'bound': 'hbm', 'achieved': achieved, 'peak': 8000.0, 'unit': 'GB/s',
                         'frac': achieved / 8000.0, 'traffic': nbytes, 'kernel': 'torch copy_'}}


def run_stream(args):
    """HBM ceilings of the row kernels' read / write mixes, measured with the library's own streaming kernel
    (noise_hbm_stream: one wave per row, 16-byte vector accesses) over the config-4 row count (3072 x 2048 rows):
    block entry (4 KiB read, 3 KiB written per row), MLP entry (3 / 1), a copy (2 / 2), read-heavy (2 / 1) and
    write-heavy (1 / 2). value = the block-entry mix."""
    from noise_amd import _lib
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    rows = 3072 * T
    src = torch.zeros(rows * 4096 // 4, device=dev, dtype=torch.int32)
    dst = torch.empty(rows * 3072 // 4, device=dev, dtype=torch.int32)
    s = torch.cuda.current_stream().cuda_stream
    mixes = {'block_entry_4r_3w': (4, 3), 'mlp_entry_3r_1w': (3, 1), 'copy_2r_2w': (2, 2), 'read_heavy_2r_1w': (2, 1),
             'write_heavy_1r_2w': (1, 2)}
    out = {}
    for name, (ri, wo) in mixes.items():
        ms_step, ms_launch = _timed(lambda: _lib.call('noise_hbm_stream', src.data_ptr(), ri, dst.data_ptr(), wo, rows, s),
                                    args.steps, args.warmup)
        out[name] = {'ms': ms_launch, 'TB/s': (ri + wo) * 1024 * rows / (ms_launch * 1e-3) / 1e12}
    be = out['block_entry_4r_3w']
    return {'metric': 'HBM streaming ceiling of the row-kernel mixes', 'value': be['TB/s'] * 1e3, 'unit': 'GB/s',
            'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': be['ms'], 'higher_is_better': True,
            'scaling': 'weak', 'vs_baseline': None, 'dtype': 'u32', 'data': 'synthetic',
            'config': {'workload': 'hbm_stream', 'rows': rows, 'mixes': out},
            'roofline': {'bound': 'hbm', 'achieved': be['TB/s'] * 1e3, 'peak': 8000.0, 'unit': 'GB/s',
                         'frac': be['TB/s'] * 1e3 / 8000.0, 'traffic': 7 * 1024 * rows, 'kernel': 'hbm_stream_kernel'}}


def run_library(args):
    """The vendor library (torch.matmul -> hipBLASLt / rocBLAS) on plain bf16 GEMMs of the fused MLP's shapes at
    config 4 (M = 3072 x 2048 rows: c_fc [M, 512] x [512, 2048], c_proj [M, 2048] x [2048, 512]) and on an 8192^3 GEMM:
    a reference point for the MLP pair's fraction of the nominal 2.5 PFLOP/s (plain products, no rank-1 terms, relu^2
    or dot partials). value = the pair's TFLOP/s."""
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    M = 3072 * T
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(M, D, device=dev, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(F, D, device=dev, generator=g) * D ** -0.5).to(torch.bfloat16)
    w2 = (torch.randn(D, F, device=dev, generator=g) * F ** -0.5).to(torch.bfloat16)
    h = torch.empty(M, F, device=dev, dtype=torch.bfloat16)
    y = torch.empty(M, D, device=dev, dtype=torch.bfloat16)
    _, t_fc = _timed(lambda: torch.matmul(x, w1.t(), out=h), args.steps, args.warmup)
    _, t_proj = _timed(lambda: torch.matmul(h, w2.t(), out=y), args.steps, args.warmup)
    del x, h, y
    a = torch.randn(8192, 8192, device=dev, generator=g).to(torch.bfloat16)
    b = torch.randn(8192, 8192, device=dev, generator=g).to(torch.bfloat16)
    _, t_sq = _timed(lambda: a @ b, args.steps, args.warmup)
    f_mlp = 2 * M * D * F
    tf = lambda f, ms: f / (ms * 1e-3) / 1e12  # noqa: E731
    pair = tf(2 * f_mlp, t_fc + t_proj)
    return {'metric': 'vendor bf16 GEMM on the fused-MLP shapes (reference point)', 'value': pair, 'unit': 'TFLOP/s',
            'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': t_fc + t_proj,
            'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16', 'data': 'synthetic',
            'config': {'workload': 'library_gemm', 'M': M,
                       'c_fc': {'ms': t_fc, 'TFLOP/s': tf(f_mlp, t_fc), 'frac': tf(f_mlp, t_fc) / PEAK_BF16_TFLOPS},
                       'c_proj': {'ms': t_proj, 'TFLOP/s': tf(f_mlp, t_proj), 'frac': tf(f_mlp, t_proj) / PEAK_BF16_TFLOPS},
                       'square_8192': {'ms': t_sq, 'TFLOP/s': tf(2 * 8192 ** 3, t_sq),
                                       'frac': tf(2 * 8192 ** 3, t_sq) / PEAK_BF16_TFLOPS}},
            'roofline': {'bound': 'mfma', 'achieved': pair, 'peak': PEAK_BF16_TFLOPS, 'unit': 'TFLOP/s',
                         'frac': pair / PEAK_BF16_TFLOPS, 'traffic': None, 'kernel': 'torch.matmul (vendor library)'}}


def run_probes(args):
    """Row f3: the readout-probe forward differences (noise_readout_probes, `cycle_derivatives`,
    train/val/run.py:154-167) of 1024 tokens along 512 directions over a 4096 vocabulary. value = (token, direction,
    vocabulary entry) terms per second; each costs two exp2, one reciprocal and ~6 other VALU operations."""
    from noise_amd.probes import cycle_derivatives
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    n, P, Vv = 1024, 512, V
    g = torch.Generator(device=dev).manual_seed(0)
    base = torch.randn(n, Vv, device=dev, generator=g) * 3
    C = torch.randn(P, Vv, device=dev, generator=g) * 0.5
    y = torch.randint(0, Vv, (n,), device=dev, generator=g)
    steps = 1e-2 * (1 + torch.rand(n, device=dev, generator=g))
    sq = D * (1 + 0.1 * torch.rand(n, device=dev, generator=g))
    dots = torch.randn(n, P, device=dev, generator=g)
    dir_sq = D * (1 + 0.1 * torch.rand(P, device=dev, generator=g))
    ms_step, ms_launch = _timed(lambda: cycle_derivatives(base, C, y, steps, sq, dots, dir_sq), args.steps, args.warmup)
    entries = n * P * Vv
    return {'metric': 'readout-probe terms per second (row f3)', 'value': entries / (ms_launch * 1e-3), 'unit': 'terms/s',
            'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': ms_step, 'higher_is_better': True,
            'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f32', 'data': 'synthetic',
            'config': {'workload': 'readout_probes', 'tokens': n, 'directions': P, 'vocab': Vv, 'ms_per_launch': ms_launch},
            'roofline': None}


def run_credit(args):
    """Row f4: the credit kernels of one rerun chunk at the reference's shapes (`query_key_errors`,
    train/val/run.py:594-634: 64 draws, batch 1, 2048 tokens, 8 heads of 64): moved heads, head scores, the code
    estimate (HBM streams of the bf16 draws and outputs) and the key filter (bf16 MFMA). value = the moved heads'
    algorithmic HBM rate."""
    from noise_amd import _lib
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    n, b, H = 64, 1, 8
    g = torch.Generator(device=dev).manual_seed(0)
    raw = torch.randn(b, T, H, 64, device=dev, generator=g)
    a = torch.randn(n, b, T, H, 64, device=dev, generator=g).to(torch.bfloat16)
    cos, sin = torch.rand(T, 32, device=dev, generator=g), torch.rand(T, 32, device=dev, generator=g)
    out = torch.empty(n * b * T, H * 64, device=dev, dtype=torch.bfloat16)
    base, hub = torch.randn(b, T, H, 64, device=dev, generator=g), torch.randn(b, T, H, 64, device=dev, generator=g)
    score = torch.empty(b, H, T, n, device=dev)
    cred = torch.randn(b, H, T, n, device=dev, generator=g)
    est = torch.empty(b, T, H, 64, device=dev)
    filt = torch.randn(b, H, T, T, device=dev, generator=g).to(torch.bfloat16)
    kout = torch.empty(b, H, T, n, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    kernels = {
        'moved_heads': (lambda: _lib.call('noise_moved_heads', raw.data_ptr(), a.data_ptr(), 0.1, cos.data_ptr(),
                                          sin.data_ptr(), n, b, T, H, out.data_ptr(), H * 64, s),
                        raw.numel() * 4 + a.numel() * 2 * 2 + cos.numel() * 8),
        'head_scores': (lambda: _lib.call('noise_head_scores', out.data_ptr(), H * 64, base.data_ptr(), hub.data_ptr(),
                                          n, b, T, H, score.data_ptr(), s),
                        out.numel() * 2 + base.numel() * 8 + score.numel() * 4),
        'code_estimate': (lambda: _lib.call('noise_code_estimate', cred.data_ptr(), a.data_ptr(), n, b, T, H,
                                            est.data_ptr(), s),
                          cred.numel() * 4 + a.numel() * 2 + est.numel() * 4),
        'key_filter': (lambda: _lib.call('noise_key_filter', filt.data_ptr(), cred.data_ptr(), b, H, T, n,
                                         kout.data_ptr(), s),
                       filt.numel() * 2 + cred.numel() * 4 + kout.numel() * 4),
    }
    res = {}
    for name, (fn, nbytes) in kernels.items():
        _, ms = _timed(fn, args.steps, args.warmup)
        res[name] = {'us': ms * 1e3, 'bytes': nbytes, 'TB/s': nbytes / (ms * 1e-3) / 1e12}
    res['key_filter']['TFLOP/s'] = 2 * b * H * T * T * n / (res['key_filter']['us'] * 1e-6) / 1e12
    mh = res['moved_heads']
    return {'metric': 'credit kernels, algorithmic HBM rate (row f4)', 'value': mh['TB/s'] * 1e3, 'unit': 'GB/s',
            'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': mh['us'] * 1e-3,
            'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'bf16', 'data': 'synthetic',
            'config': {'workload': 'credit_chunk', 'draws': n, 'batch': b, 'tokens': T, 'heads': H, 'kernels': res},
            'roofline': {'bound': 'hbm', 'achieved': mh['TB/s'] * 1e3, 'peak': 8000.0, 'unit': 'GB/s',
                         'frac': mh['TB/s'] * 1e3 / 8000.0, 'traffic': mh['bytes'], 'kernel': 'moved_heads_vec_kernel'}}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=10)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--workload', choices=('step', 'mlp', 'attention', 'head', 'copy', 'stream', 'library', 'probes',
                                           'credit'),
                    default='step')
    ap.add_argument('--window', type=int, default=2048, help='attention window (config 2)')
    ap.add_argument('--qk-norm', action='store_true', help='config 2 with RMS-normalised q, k rows (the model case)')
    ap.add_argument('--pairs', type=int, default=1536)
    ap.add_argument('--chunk', type=int, default=3072,
                    help='members per kernel pass (default: the whole population in one pass, ~105 GB of activations)')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--fitness', choices=('rank', 'zscore'), default='rank',
                    help="config 4 names rank-normalised fitness; 'zscore' is the reference's (train/val/eggroll.py:151-152)")
    ap.add_argument('--weights', choices=('init', 'trained'), default='init',
                    help="config 4 weights: the reference's seed-0 init, or with trained-scale lm_head, ve_gate and "
                         "lambdas (noise_amd.synthetic.trained_like)")
    ap.add_argument('--head', choices=tuple(HEAD_DESC), default='fp32',
                    help="configs 3 and 4 name an fp32 head: 'fp32' (fp16 h against a 22-bit fp16 hi/lo weight) or "
                         "'fp32_split' (bf16 hi/lo, ~2^-16); 'bf16' is the reference's autocast head "
                         "(train/val/eggroll.py:99 under :144), for comparison")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f'bench.py measures one GPU only: every box in this build has a single MI355X; --gpus {args.gpus} '
              f'is not supported (the population would shard by members across GPUs, one loss all-gather per '
              f'step; that path is not built here).', file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print('bench.py needs a GPU', file=sys.stderr)
        sys.exit(2)
    result = {'step': run_step, 'mlp': run_mlp, 'attention': run_attention, 'head': run_head, 'probes': run_probes,
              'credit': run_credit,
              'copy': run_copy, 'stream': run_stream, 'library': run_library}[args.workload](args)
    if not args.no_cpu_baseline and args.workload not in ('copy', 'stream', 'library', 'probes', 'credit'):
        result['cpu_baseline'] = cpu_baseline_mlp() if args.workload == 'mlp' else cpu_baseline_step()
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
