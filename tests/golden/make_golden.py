"""Write the golden vectors for the population path by running the reference on the CPU.

Run in the build container only (the reference is not present on the GPU box):

    python tests/golden/make_golden.py [--reference /root/reference]

It imports `utils/model.py` and `train/val/eggroll.py` from the reference checkout and records, for the
functions that only the reference's own composition pins:

* sha256 of every tensor of `make_model('cpu', 0)` (train/val/eggroll.py:38-53);
* per-member losses of `population_loss` (train/val/eggroll.py:66-103) on seeded synthetic inputs at
  config-0 shape (P = 8, T = 256, sigma = 1e-3), at the reference init and with `trained_like` weights;
* the clean `GPT.forward` loss (utils/model.py:193-210) on the same tokens;
* `Eggroll.offsets` / `noise` streams and two whole `Eggroll.step` updates (train/val/eggroll.py:106-168)
  with CHUNK = 4 and NOISE = 2**20 so that a 4-pair population fits.

On the CPU `torch.autocast('cuda')` is inactive, so every number here is the reference in float32.
Inputs come from `noise_amd.synthetic`; their sha256 is stored so a drift in the generators is caught.
Output: tests/golden/config0.json (data only: inputs' hashes, expected outputs).
"""
import argparse
import hashlib
import json
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from noise_amd.synthetic import antithetic_signs, population_noise, trained_like, zipf_tokens  # noqa: E402

SIGMA = 1e-3
PAIRS = 4
T = 256


def sha(t):
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return hashlib.sha256(t.numpy().tobytes()).hexdigest()


def noise_sha(noise):
    h = hashlib.sha256()
    for name, n in noise.items():
        for t in (n if isinstance(n, tuple) else (n,)):
            h.update(name.encode())
            h.update(t.contiguous().numpy().tobytes())
    return h.hexdigest()


def floats(t):
    return [float(v) for v in t.detach().flatten().tolist()]


def sample_idx(shape, count=16, seed=5):
    g = torch.Generator().manual_seed(seed)
    return [[int(torch.randint(0, s, (1,), generator=g)) for s in shape] for _ in range(count)]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--reference', default='/root/reference')
    ap.add_argument('--out', default=str(ROOT / 'tests' / 'golden' / 'config0.json'))
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    import utils.model as ref_model          # noqa: E402
    import train.val.eggroll as ref_egg      # noqa: E402

    torch.set_num_threads(8)
    out = {'sigma': SIGMA, 'pairs': PAIRS, 'T': T, 'torch': torch.__version__}
    t0 = time.time()
    model = ref_egg.make_model(torch.device('cpu'), 0)
    out['weights_sha256'] = {n: sha(p) for n, p in model.state_dict().items()}
    out['rotary_sha256'] = {'cos': sha(model.cos), 'sin': sha(model.sin)}
    out['window_sizes'] = [w for w, _ in model.window_sizes]

    idx, targets = zipf_tokens(T)
    out['tokens_sha256'] = {'idx': sha(idx), 'targets': sha(targets)}
    params = dict(model.named_parameters())
    shapes = {n: tuple(p.shape) for n, p in params.items()}
    noise = population_noise(shapes, PAIRS)
    out['noise_sha256'] = noise_sha(noise)
    sign = antithetic_signs(2 * PAIRS, SIGMA)

    with torch.no_grad():
        out['losses_init'] = floats(ref_egg.population_loss(model, params, noise, sign, idx, targets))
        out['clean_loss_init'] = float(model(idx[None], targets[None]))
        print('init done', time.time() - t0, out['losses_init'], flush=True)

        trained_like(model)
        out['trained_weights_sha256'] = {n: sha(p) for n, p in model.state_dict().items()
                                         if n in ('lm_head.weight', 'resid_lambdas', 'x0_lambdas')}
        out['losses_trained'] = floats(ref_egg.population_loss(model, params, noise, sign, idx, targets))
        out['clean_loss_trained'] = float(model(idx[None], targets[None]))
        out['clean_token_losses_trained'] = floats(model(idx[None], targets[None], loss_reduction='none'))
        print('trained done', time.time() - t0, out['losses_trained'], flush=True)

    # Eggroll.step with a reduced chunk and buffer so a 4-pair population is one chunk.
    ref_egg.CHUNK = PAIRS
    ref_egg.NOISE = 2 ** 20
    step_t = 64
    sx, sy = zipf_tokens(step_t, seed=4)
    es = ref_egg.Eggroll(model, PAIRS)
    recorded = []
    compiled = es.loss
    es.loss = lambda *a: recorded.append(compiled(*a)) or recorded[-1]
    opt = torch.optim.AdamW(model.parameters(), lr=ref_egg.LR, betas=ref_egg.BETAS, eps=1e-8, weight_decay=0.0)
    step_out = {'chunk': PAIRS, 'noise_len': 2 ** 20, 'T': step_t, 'seq_seed': 4,
                'buffer_sha256': sha(es.buffer), 'steps': []}
    for step in (1, 2):
        offs = es.offsets(step)
        before = {n: p.detach().clone() for n, p in params.items()}
        mean = es.step(sx[None], sy[None], opt, step)
        rec = {'step': step, 'mean_loss': mean, 'member_losses': floats(recorded[-1]),
               'offsets': {n: [int(v) for v in o] for n, o in offs.items()}, 'grads': {}, 'deltas': {}}
        for n, p in params.items():
            g, d = p.grad, p.detach() - before[n]
            if p.numel() <= 256:
                rec['grads'][n] = floats(g)
                rec['deltas'][n] = floats(d)
            else:
                pos = sample_idx(p.shape)
                rec['grads'][n] = {'idx': pos, 'val': [float(g[tuple(i)]) for i in pos],
                                   'sum': float(g.double().sum()), 'abs_sum': float(g.double().abs().sum())}
                rec['deltas'][n] = {'idx': pos, 'val': [float(d[tuple(i)]) for i in pos],
                                    'abs_sum': float(d.double().abs().sum())}
        step_out['steps'].append(rec)
        print('step', step, 'done', time.time() - t0, mean, flush=True)
    out['eggroll_step'] = step_out
    Path(args.out).write_text(json.dumps(out, indent=1) + '\n')
    print('wrote', args.out, time.time() - t0)


if __name__ == '__main__':
    main()
