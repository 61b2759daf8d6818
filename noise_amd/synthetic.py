"""Seeded synthetic inputs for the population path (host-side, torch CPU generators).

Seeds: weights 0 (make_model), tokens 1, perturbations 2. Inputs are generated on the CPU and moved,
so every device sees identical bytes.
"""
import torch

ZIPF_S = 1.1


def zipf_tokens(length, vocab=4096, s=ZIPF_S, seed=1):
    """length + 1 token ids with p(id = r - 1) ~ r^-s, r = 1..vocab; returns (idx, targets) [length]
    int64 as `train/val/eggroll.py:218` splits a row."""
    p = torch.arange(1, vocab + 1, dtype=torch.float64).pow(-s)
    seq = torch.multinomial(p.float(), length + 1, replacement=True,
                            generator=torch.Generator().manual_seed(seed))
    return seq[:-1].contiguous(), seq[1:].contiguous()


def antithetic_signs(members, sigma):
    """[+sigma, -sigma] repeated: member 2j is +sigma E_j, 2j+1 is -sigma E_j (train/val/eggroll.py:138)."""
    return torch.tensor([sigma, -sigma], dtype=torch.float32).repeat(members // 2)


def population_noise(shapes, pairs, seed=2, per_member=True):
    """name -> (a [n, out], b [n, in]) ~ N(0, 1) for 2-D params and eps [n, L] for 1-D params, one draw per
    antithetic pair in parameter order; with per_member the rows are repeated so both members of a
    pair share them (train/val/eggroll.py:141)."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, shape in shapes.items():
        if len(shape) == 2:
            a = torch.randn(pairs, shape[0], generator=g)
            b = torch.randn(pairs, shape[1], generator=g)
            out[name] = (a.repeat_interleave(2, 0), b.repeat_interleave(2, 0)) if per_member else (a, b)
        else:
            e = torch.randn(pairs, shape[0], generator=g)
            out[name] = e.repeat_interleave(2, 0) if per_member else e
    return out


def trained_like(model, seed=3):
    """Overwrite the weights that the reference init leaves degenerate for loss checks (lm_head ~
    N(0, 1e-6), zero ve_gate, constant lambdas) with seeded values of trained-model scale, in place."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name == 'lm_head.weight':
                p.copy_(torch.randn(p.shape, generator=g) * p.shape[1] ** -0.5 * 2.0)
            elif name.endswith('ve_gate.weight'):
                p.copy_(torch.randn(p.shape, generator=g) * 0.2)
            elif name == 'resid_lambdas':
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            elif name == 'x0_lambdas':
                p.copy_(0.1 + 0.05 * torch.randn(p.shape, generator=g))
    return model
