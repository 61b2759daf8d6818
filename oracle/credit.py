"""CPU restatement of the credit-scoring helpers around attention reruns (TEST INFRASTRUCTURE ONLY).

Follows train/val/run.py:186-211: `moved_heads` (:186-189), `head_scores` (:192-195), `code_estimate`
(:208-210); the reruns use `oracle.model.attention` (utils/model.py:14-31). Pinned in tests/test_oracle.py
against per-element loops: the rotation as a complex multiplication, the norm as an explicit mean, the sums as
Python loops over their indices.
"""
import torch

from .model import apply_rotary, attention, norm


def moved_heads(raw, a, sigma, cos, sin):
    """raw [b, t, h, 64] fp32, a [n, b, t, h, 64], cos / sin [t, 32] -> [n * b, t, h, 64] in a's dtype."""
    moved = (raw.unsqueeze(0) + sigma * a.float()).flatten(0, 1)
    return norm(apply_rotary(moved, cos, sin)).to(a.dtype)


def head_scores(out, baseline, hub):
    """out [n, b, t, h, 64] -> [b, h, t, n]."""
    change = out.float() - baseline.float().unsqueeze(0)
    return (change * hub.float().unsqueeze(0)).sum(-1).permute(1, 3, 2, 0)


def code_estimate(credited, a):
    """credited [b, h, t, n], a [n, b, t, h, 64] -> [b, t, h, 64]."""
    return (credited.permute(3, 0, 2, 1).unsqueeze(-1) * a.float()).sum(0)


def credit_chunk(kind, raw, a, sigma, cos, sin, fixed, values, window, baseline, target, key_filter=None,
                 round_out=True):
    """One chunk of `query_key_errors` (train/val/run.py:617-625) with the attention in fp32 (output rounded to
    bf16 when round_out, as the reference's bf16 attention returns it)."""
    n, b, t, h, hd = a.shape
    rep = lambda z: z.to(a.dtype).unsqueeze(0).expand(n, -1, -1, -1, -1).reshape(n * b, t, h, hd)
    moved = moved_heads(raw, a, sigma, cos, sin)
    fx, vals = rep(fixed), rep(values)
    qa, ka = (moved, fx) if kind == 'q' else (fx, moved)
    out = attention(qa.float(), ka.float(), vals.float(), window)
    if round_out:
        out = out.to(torch.bfloat16)
    score = head_scores(out.view(n, b, t, h, hd), baseline, target)
    if kind == 'k':
        score = (key_filter.to(torch.bfloat16).float() @ score.to(torch.bfloat16).float()).to(torch.bfloat16).float()
    return code_estimate(score, a)
