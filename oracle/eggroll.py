"""CPU restatement of EGGROLL's perturbation bookkeeping, fitness, update and Adam (TEST INFRASTRUCTURE
ONLY). Follows `train/val/eggroll.py:106-168` and `:205`, `:208-212`.

Parity pins (tests/test_oracle.py, tests/test_golden.py): chunk_sequences against the hand-worked layout of
pairs = 1536 on 8 sequences (chunks of 512 members on sequences 0, 1, 2, 4, 5, 6); offsets / gathered noise against golden streams
written by importing the reference in the build container; fitness against a hand-computed closed form
(unbiased std, no centering); rank_fitness (no reference function) against hand-ranked vectors with ties; update against the explicit sum_j w_j a_j b_j^T; Adam against
torch.optim.AdamW (library routine); a whole reference step (losses, new weights) against the golden
fixture of `Eggroll.step` with CHUNK and NOISE reduced.
"""
import torch

SEED = 0
SIGMA = 0.002
LR, BETAS, ADAM_EPS = 0.001, (0.5, 0.95), 1e-8
WARMDOWN = 0.3
CHUNK = 256
NOISE = 2 ** 28


def noise_buffer(length=NOISE, seed=SEED):
    """The fixed N(0, 1) buffer every perturbation is sliced from (train/val/eggroll.py:114)."""
    return torch.randn(length, generator=torch.Generator().manual_seed(seed))


def offsets(shapes, pairs, step, length=NOISE, seed=SEED):
    """name -> int64 [pairs] slice starts, drawn in parameter order (train/val/eggroll.py:117-120)."""
    g = torch.Generator().manual_seed(1_000_003 * seed + step)
    return {name: torch.randint(0, length - sum(shape), (pairs,), generator=g) for name, shape in shapes.items()}


def gather_noise(buffer, offs, shapes, directions):
    """name -> (a [n, out], b [n, in]) for matrices and embeddings, eps [n, L] for 1-D params
    (train/val/eggroll.py:122-128)."""
    out = {}
    for name, shape in shapes.items():
        rows = buffer[offs[name][directions, None] + torch.arange(sum(shape))]
        out[name] = rows.split(list(shape), dim=1) if len(shape) == 2 else rows
    return out


def member_directions(start, chunk, pairs):
    """Directions of the members start .. start+2*chunk (train/val/eggroll.py:140): members 2j, 2j+1 share
    direction j (mod pairs); member 2j has +sigma and 2j+1 has -sigma (:138)."""
    return torch.arange(start, start + 2 * chunk, 2) % (2 * pairs) // 2


def chunk_sequences(members, per_seq, chunk, world=1):
    """Sequence of every member of the population, as the reference's loop assigns them: each rank walks its
    members in chunks of 2 * chunk starting at rank * per_rank, and a whole chunk runs on sequence
    start // per_seq (train/val/eggroll.py:137-145)."""
    per_rank = members // world
    seq = torch.full((members,), -1, dtype=torch.int64)
    for rank in range(world):
        for start in range(rank * per_rank, (rank + 1) * per_rank, 2 * chunk):
            seq[start:start + 2 * chunk] = start // per_seq
    return seq


def fitness(losses, pairs):
    """Pair fitness z-scored without centering, folded onto directions (train/val/eggroll.py:151-154)."""
    f = losses[1::2] - losses[0::2]
    f = f / (f.std() + 1e-8)
    weight = torch.zeros(pairs).index_add_(0, torch.arange(len(f)) % pairs, f)
    return f, weight


def rank_fitness(losses, pairs):
    """Config-4 option: pair fitness f_j = L[2j+1] - L[2j] replaced by centred ranks
    rank_j / (n - 1) - 0.5 (ties broken by index), folded onto directions like `fitness`. No reference
    function: the reference z-scores (train/val/eggroll.py:151-152)."""
    f = losses[1::2] - losses[0::2]
    n = len(f)
    order = torch.argsort(f, stable=True)
    ranks = torch.empty(n, dtype=torch.float32)
    ranks[order] = torch.arange(n, dtype=torch.float32)
    f = ranks / (n - 1) - 0.5 if n > 1 else torch.zeros(n)
    weight = torch.zeros(pairs).index_add_(0, torch.arange(n) % pairs, f)
    return f, weight


def update(weight, noise_dirs, n_fitness):
    """Gradient estimate per param, -sum_j w_j a_j b_j^T / n (2-D) or -w @ eps / n (1-D)
    (train/val/eggroll.py:155-166). noise_dirs: name -> gathered noise for all directions in order."""
    grads = {}
    for name, n in noise_dirs.items():
        if isinstance(n, tuple):
            g = -((weight[:, None] * n[0]).t() @ n[1])
        else:
            g = -(weight @ n)
        grads[name] = g / n_fitness
    return grads


def learning_rate(step, steps, lr=LR, warmdown=WARMDOWN):
    """Linear warmdown over the last `warmdown` fraction of the epoch (train/val/eggroll.py:208-212)."""
    left = (steps - step + 1) / steps
    return lr * min(1.0, left / warmdown)


def adam_step(param, grad, exp_avg, exp_avg_sq, step, lr, betas=BETAS, eps=ADAM_EPS):
    """One AdamW step with weight_decay = 0 (train/val/eggroll.py:205), in place; `step` counts from 1."""
    b1, b2 = betas
    exp_avg.mul_(b1).add_(grad, alpha=1 - b1)
    exp_avg_sq.mul_(b2).addcmul_(grad, grad, value=1 - b2)
    bc1, bc2 = 1 - b1 ** step, 1 - b2 ** step
    denom = (exp_avg_sq.sqrt() / bc2 ** 0.5).add_(eps)
    param.addcdiv_(exp_avg, denom, value=-lr / bc1)
    return param
