"""CPU restatement of the readout-probe forward differences (TEST INFRASTRUCTURE ONLY).

Follows `cycle_derivatives` and `row_derivatives` of train/val/run.py:154-185 (identical copies in
train/speedrun/run.py:90-103): for a token with clean stream x (|x|^2 = sq), readout logits base = W x,
target y and step s, and a direction D_j with W D_j = C[j], x . D_j = dots and |D_j|^2 = dir_sq, the soft-capped
cross-entropy of the head applied to norm(x + s D_j) minus that of norm(x), divided by s. The moved stream's RMS
comes from sq + 2 s dots + s^2 dir_sq, so the head's norm is exact at every probe; a target of -1 gives 0.

Pins (tests/test_oracle.py): against a brute force that moves the stream itself (x + s D_j), normalises it,
applies the head, caps and takes the cross-entropy with F.cross_entropy; in float64.
"""
import torch

SOFTCAP = 15.0
EPS = torch.finfo(torch.float32).eps  # train/val/run.py:58


def _capped_loss(z, target_z):
    """logsumexp_v(15 tanh(z_v / 15)) - 15 tanh(target_z / 15) over the last axis of z."""
    return torch.exp(SOFTCAP * torch.tanh(z / SOFTCAP)).sum(-1).log() - SOFTCAP * torch.tanh(target_z / SOFTCAP)


def cycle_derivatives(base, C, y, steps, sq, dots, dir_sq, width=512):
    """base (n, V), C (P, V), y (n,) int64, steps (n, 1), sq (n, 1), dots (n, P), dir_sq (P,) -> (n, P)
    (train/val/run.py:154-167)."""
    target = y.clamp(min=0)
    base_y = base.gather(1, target[:, None])
    dirs_y = C.T[target]
    inv0 = torch.rsqrt(sq / width + EPS)
    clean = _capped_loss(base * inv0, (base_y * inv0).squeeze(-1))[:, None]
    inv = torch.rsqrt((sq + 2 * steps * dots + steps * steps * dir_sq) / width + EPS)
    z = (base[:, None, :] + steps[:, :, None] * C[None]) * inv[:, :, None]
    moved = _capped_loss(z, (base_y + steps * dirs_y) * inv)
    return (moved - clean) / steps * (y >= 0)[:, None]


def row_derivatives(base, C, rows, y, steps, sq, dots, dir_sq, width=512):
    """The same along each token's own directions: rows (n, K) into C, dots and dir_sq (n, K) -> (n, K)
    (train/val/run.py:169-181)."""
    target = y.clamp(min=0)
    dirs = C[rows]
    base_y = base.gather(1, target[:, None])
    dirs_y = dirs.gather(2, target[:, None, None].expand(-1, rows.shape[1], 1)).squeeze(-1)
    inv0 = torch.rsqrt(sq / width + EPS)
    clean = _capped_loss(base * inv0, (base_y * inv0).squeeze(-1))[:, None]
    inv = torch.rsqrt((sq + 2 * steps * dots + steps * steps * dir_sq) / width + EPS)
    z = (base[:, None, :] + steps[:, :, None] * dirs) * inv[:, :, None]
    moved = _capped_loss(z, (base_y + steps * dirs_y) * inv)
    return (moved - clean) / steps * (y >= 0)[:, None]


def moved_stream_losses(x, W, D, y, steps):
    """Brute force for the pins: the capped cross-entropy of the head on norm(x + s D_j) for every token and
    direction (x (n, width), W (V, width), D (width, P), y (n,), steps (n, 1)) -> (n, P), and on norm(x) -> (n,)."""
    width = x.shape[1]
    t = y.clamp(min=0)

    def loss(stream):  # stream (..., width) -> (...,) against the token's target
        h = stream * torch.rsqrt(stream.square().sum(-1, keepdim=True) / width + EPS)
        z = SOFTCAP * torch.tanh((h @ W.T) / SOFTCAP)
        idx = t.view(-1, *([1] * (z.dim() - 1))).expand(*z.shape[:-1], 1)
        return torch.logsumexp(z, -1) - z.gather(-1, idx).squeeze(-1)

    return loss(x[:, None, :] + steps[:, :, None] * D.T[None]), loss(x)
