"""Benchmark of the population-perturbed fused relu^2 MLP on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

One step = one pass of the low-rank relu^2 MLP (noise_lowrank_mlp) over the whole population:
P = 256 members (128 antithetic pairs, sigma = 1e-3) of y_p = relu^2(x W1_p^T) W2_p^T with
W_p = W + s_p a_p b_p^T, x [2048 tokens, 512] shared, W1 [2048, 512], W2 [512, 2048], bf16 operands with
fp32 accumulation, bf16 output [256, 2048, 512]. Inputs are synthetic and resident in HBM before the
timed region. Prints one JSON line (rank 0).
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
PEAK_HBM_GBS = 8000.0
P, T, D, F = 256, 2048, 512, 2048
SIGMA = 1e-3
FLOP_PER_MEMBER_TOKEN = 2 * (2 * D * F)  # both GEMMs, counted per member


def make_inputs(device, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, D, generator=g).bfloat16()
    w1 = (torch.randn(F, D, generator=g) * D ** -0.5).bfloat16()
    w2 = (torch.randn(D, F, generator=g) * F ** -0.5).bfloat16()
    pairs = P // 2
    a1, b1 = torch.randn(pairs, F, generator=g), torch.randn(pairs, D, generator=g)
    a2, b2 = torch.randn(pairs, D, generator=g), torch.randn(pairs, F, generator=g)
    sign = torch.tensor([SIGMA, -SIGMA]).repeat(pairs)
    return [t.to(device) for t in (x, w1, w2, a1, b1, a2, b2, sign)]


def cpu_baseline(budget_s=12.0):
    """The CPU oracle (port of the reference MLP sublayer, bf16 rounding-point mode) on a bounded
    sample: whole 2048-token members, as many as fit the time budget."""
    from oracle import model as om
    threads = int(os.environ.get('OMP_NUM_THREADS', os.cpu_count() or 1))
    threads = min(threads, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    x, w1, w2, a1, b1, a2, b2, sign = make_inputs('cpu')
    xf, w1f, w2f = x.float(), w1.float(), w2.float()
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s and done < P:
        m = [done, done + 1]
        om.mlp_population(xf, w1f, w2f, a1[[done // 2] * 2], b1[[done // 2] * 2], a2[[done // 2] * 2],
                          b2[[done // 2] * 2], sign[m], 'bf16')
        done += 2
    dt = time.perf_counter() - t0
    return {'value': done * T / dt, 'unit': 'member-tokens/s', 'cores': threads, 'kind': 'port',
            'sample': f'{done} members x {T} tokens of config 1 through oracle.model.mlp_population '
                      f'(torch CPU, bf16 rounding points emulated in fp32), {dt:.1f} s'}


def load_traffic():
    path = ROOT / 'profiles' / 'traffic_mlp.json'
    if path.exists():
        return json.loads(path.read_text()).get('hbm_bytes_per_launch')
    return None


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    args = ap.parse_args()
    if args.gpus != 1:
        print(f'bench.py measures one GPU only: every box in this build has a single MI355X; '
              f'--gpus {args.gpus} is not supported (the member dimension shards across GPUs by design, '
              f'see DESIGN.md).', file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print('bench.py needs a GPU', file=sys.stderr)
        sys.exit(2)
    from noise_amd import ops

    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    x, w1, w2, a1, b1, a2, b2, sign = make_inputs(dev)
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
    flop = FLOP_PER_MEMBER_TOKEN * P * T
    achieved = flop / (ms_launch * 1e-3) / 1e12
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
        'data': 'synthetic',
        'config': {'workload': 'config1_fused_relu2_mlp_rank1', 'members': P, 'pairs': P // 2, 'tokens': T,
                   'd_model': D, 'd_hidden': F, 'sigma': SIGMA, 'x': 'shared [2048, 512]', 'output': 'bf16',
                   'parallelism': 'single GPU'},
        'roofline': {'bound': 'mfma', 'achieved': achieved, 'peak': PEAK_BF16_TFLOPS, 'unit': 'TFLOP/s',
                     'frac': achieved / PEAK_BF16_TFLOPS, 'traffic': load_traffic(),
                     'kernel': 'noise_lowrank_mlp (rowdot + relu2 GEMM + proj GEMM)',
                     'flop_per_launch': flop, 'ms_per_launch': ms_launch},
    }
    if not args.no_cpu_baseline:
        result['cpu_baseline'] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == '__main__':
    main()
