"""EGGROLL population step on the HIP kernels: the drop-in for `Eggroll` (train/val/eggroll.py:106-168).

Perturbation bookkeeping (the fixed N(0, 1) buffer, per-step offsets, the member -> direction and
member -> sequence layout) follows the reference exactly; the population forward, the fitness, the
gradient estimate and (with noise_amd.optim.Adam) the optimizer step run in libnoise_hip.so.

Noise rows are gathered per kernel pass (the members one forward pass evaluates), never for the whole
population at once: a pass of m members holds m / 2 directions x 101,552 floats (624 MB at m = 3072),
whatever the population size.
"""
import torch

from . import _lib
from .population import Population, Weights

BATCH = 8            # sequences per update (train/val/eggroll.py:28)
SEED = 0
PAIRS = 131072
SIGMA = 0.002
LR, BETAS = 0.001, (0.5, 0.95)
WARMDOWN = 0.3
CHUNK = 256          # pairs per batched forward in the reference; members per kernel pass here is `chunk`
NOISE = 2 ** 28

FITNESS = {'zscore': _lib.FITNESS_ZSCORE, 'rank': _lib.FITNESS_RANK}


def gather_losses(losses, world):
    """Every member's loss in member order, from each rank's contiguous share (rank r evaluates members
    r * per_rank .. (r + 1) * per_rank - 1): the `all_gather` of train/val/eggroll.py:147-150. One rank: the
    losses themselves."""
    if world == 1:
        return losses
    gathered = [torch.empty_like(losses) for _ in range(world)]
    torch.distributed.all_gather(gathered, losses)
    return torch.cat(gathered)


def member_sequences(lo, hi, per_seq, chunk_pairs=CHUNK, device=None):
    """Sequence index of members lo .. hi - 1. The reference walks a rank's members in chunks of 2 * CHUNK and
    evaluates each whole chunk on sequence start // per_seq (train/val/eggroll.py:139-145): when per_seq is not a
    multiple of 2 * CHUNK, a chunk runs on the sequence its first member falls in and some sequences host no
    member at all."""
    j = torch.arange(lo, hi, device=device)
    return (j // (2 * chunk_pairs)) * (2 * chunk_pairs) // per_seq


class Eggroll:
    """Perturbation bookkeeping + the population step (train/val/eggroll.py:106-168).

    chunk       -- members per forward pass of the kernels (a multiple of 2; bounded by activation memory); the
                   noise rows are gathered per pass;
    chunk_pairs -- the reference's CHUNK (pairs per batched forward, :34): it fixes which sequence each member
                   is evaluated on and that every rank hosts whole chunks (:139-145, the check of :187-188);
    head        -- 'fp32' or 'bf16' head (see noise_amd.population.Population);
    fitness     -- 'zscore' (the reference, :151-152) or 'rank' (centred ranks);
    sigma, noise_len -- SIGMA and NOISE of the reference by default."""

    def __init__(self, model, pairs, rank=0, world=1, chunk=512, head='fp32', fitness='zscore', sigma=SIGMA,
                 noise_len=NOISE, chunk_pairs=CHUNK):
        if chunk % 2:
            raise ValueError('chunk must be even (antithetic pairs stay together)')
        if chunk_pairs <= 0:
            raise ValueError('chunk_pairs must be positive')
        self.chunk_pairs = chunk_pairs
        self.model, self.pairs, self.rank, self.world = model, pairs, rank, world
        self.device = next(model.parameters()).device
        self.params = dict(model.named_parameters())
        self.sigma, self.noise_len = sigma, noise_len
        self.fitness_mode = FITNESS[fitness]
        self.buffer = torch.randn(noise_len, device=self.device,
                                  generator=torch.Generator(self.device).manual_seed(SEED))
        self.pop = Population(model, chunk=chunk, head=head)
        self.last_losses = None

    def offsets(self, step):
        """name -> int64 [pairs] slice starts (train/val/eggroll.py:117-120)."""
        g = torch.Generator(self.device).manual_seed(1_000_003 * SEED + step)
        return {name: torch.randint(0, self.noise_len - sum(p.shape), (self.pairs,), device=self.device, generator=g)
                for name, p in self.params.items()}

    def noise(self, offsets, directions):
        """name -> (a [n, out], b [n, in]) for matrices and embeddings, eps [n, L] for the mixing scalars
        (train/val/eggroll.py:122-128), as contiguous tensors: every parameter's rows gathered from the buffer
        by one noise_gather_rows launch."""
        directions = directions.to(device=self.device, dtype=torch.int64).contiguous()
        n = directions.numel()
        out, items = {}, []
        for name, p in self.params.items():
            off = offsets[name]
            if p.dim() == 2:
                a = torch.empty(n, p.shape[0], device=self.device)
                b = torch.empty(n, p.shape[1], device=self.device)
                out[name] = (a, b)
                items.append((off.data_ptr(), a.data_ptr(), b.data_ptr(), p.shape[0], p.shape[1]))
            else:
                e = torch.empty(n, p.shape[0], device=self.device)
                out[name] = e
                items.append((off.data_ptr(), e.data_ptr(), None, p.shape[0], 0))
        if n:
            ptr, count, _keep = _lib.gather_params(items)
            _lib.call('noise_gather_rows', self.buffer.data_ptr(), self.buffer.numel(), ptr, count,
                      directions.data_ptr(), n, self.pairs, torch.cuda.current_stream().cuda_stream)
        return out

    @torch.no_grad()
    def step(self, x, y, optimizer, step):
        """Evaluate this rank's share of the population, gather the losses, rebuild the update
        (train/val/eggroll.py:130-168). Returns the mean population loss."""
        pairs, cp = self.pairs, self.chunk_pairs
        members = max(2 * pairs, 2 * len(x))
        per_seq, per_rank = members // len(x), members // self.world
        if members % self.world or per_rank % (2 * cp):
            # the reference's own requirement: every rank evaluates whole chunks of 2 * CHUNK members (:187-188)
            raise ValueError(f'each rank must evaluate whole chunks of {2 * cp} members (chunk_pairs = {cp})')
        offsets = self.offsets(step)
        losses = torch.empty(per_rank, device=self.device)
        weights = Weights(self.params, self.model.config, self.pop.head)
        lo, hi = self.rank * per_rank, (self.rank + 1) * per_rank
        sign = torch.tensor([self.sigma, -self.sigma], device=self.device).repeat(self.pop.chunk // 2)
        # one kernel pass per `chunk` members, each with only its own directions' noise rows; the members of a
        # pass may span several of the reference's chunks and so several sequences (per-member token rows)
        for c0 in range(lo, hi, self.pop.chunk):
            c1 = min(hi, c0 + self.pop.chunk)
            directions = torch.arange(c0, c1, 2, device=self.device) % (2 * pairs) // 2
            noise = self.noise(offsets, directions)
            seq = member_sequences(c0, c1, per_seq, cp, device=self.device)
            first, last = (c0 // (2 * cp)) * (2 * cp) // per_seq, ((c1 - 1) // (2 * cp)) * (2 * cp) // per_seq
            if first == last:
                seq_x, seq_y = x[first], y[first]
            else:
                seq_x, seq_y = x[seq], y[seq]
            losses[c0 - lo:c1 - lo] = self.pop.loss(self.params, noise, sign[:c1 - c0], seq_x, seq_y, pair_shift=1,
                                                    weights=weights)
            del noise
        losses = gather_losses(losses, self.world)
        self.last_losses = losses
        nfit = len(losses) // 2
        fit = torch.empty(nfit, device=self.device)
        weight = torch.empty(pairs, device=self.device)
        s = torch.cuda.current_stream().cuda_stream
        _lib.call('noise_fitness', losses.data_ptr(), len(losses), pairs, self.fitness_mode, fit.data_ptr(),
                  weight.data_ptr(), s)
        grads = {name: torch.empty_like(p) for name, p in self.params.items()}
        for d0 in range(0, pairs, CHUNK if pairs > 8 * CHUNK else pairs):
            d1 = min(pairs, d0 + (CHUNK if pairs > 8 * CHUNK else pairs))
            dirs = torch.arange(d0, d1, device=self.device)
            w = weight[d0:d1].contiguous()
            noise = self.noise(offsets, dirs)
            tmps, mats = {}, []
            for name, n in noise.items():
                p = self.params[name]
                tmps[name] = tmp = grads[name] if d0 == 0 else torch.empty_like(p)
                if isinstance(n, tuple):
                    a, b = n
                    mats.append((a.data_ptr(), a.shape[1], b.data_ptr(), b.shape[1], p.shape[0], p.shape[1],
                                 tmp.data_ptr()))
                else:
                    mats.append((0, 0, n.data_ptr(), n.shape[1], 1, p.shape[0], tmp.data_ptr()))
            # every parameter's outer-product sum in one launch
            ptr, count, _keep = _lib.outer_mats(mats)
            _lib.call('noise_outer_update_batch', ptr, count, w.data_ptr(), d1 - d0, -1.0 / nfit, s)
            if d0 != 0:
                for name, tmp in tmps.items():
                    grads[name] += tmp
        optimizer.zero_grad(set_to_none=True)
        for name, p in self.params.items():
            p.grad = grads[name]
        optimizer.step()
        return losses.mean().item()
