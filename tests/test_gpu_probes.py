"""GPU parity of the readout-probe forward differences (train/val/run.py:154-185) against the CPU oracle
(oracle/probes.py, pinned by a moved-stream brute force) evaluated in float64 on the same fp32 inputs.

Tolerance: the output is (L_moved - L_clean) / step, so fp32 rounding of the two log-sum-exps (each a sum of
4096 terms) is divided by the step; each element is bounded by 64 ulp of fp32 of |L_moved| + |L_clean| over
its step (the reference's own fp32 evaluation carries noise of the same order)."""
import pytest
import torch

from noise_amd import probes
from oracle import probes as op
from tests._util import log_case

pytestmark = pytest.mark.gpu
DEV = 'cuda'


def _case(n, width, V, P, sigma, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, width, generator=g) * 1.5
    W = torch.randn(V, width, generator=g) * (2.0 / width ** 0.5)
    D, _ = torch.linalg.qr(torch.randn(width, P, generator=g))    # orthonormal directions
    y = torch.randint(0, V, (n,), generator=g)
    y[::7] = -1
    steps = sigma * x.square().mean(-1, keepdim=True).sqrt()
    base, C = x @ W.T, (W @ D).T.contiguous()
    sq, dots, dir_sq = x.square().sum(-1, keepdim=True), x @ D, D.square().sum(0)
    return base, C, y, steps, sq, dots, dir_sq


def _bound(base, C, y, steps, sq, dots, dir_sq, width, rows=None):
    """64 fp32 ulp of |L_moved| + |L_clean| over the step, per element."""
    b64 = lambda t: t.double()  # noqa: E731
    inv0 = torch.rsqrt(b64(sq) / width + op.EPS)
    lclean = torch.logsumexp(op.SOFTCAP * torch.tanh(b64(base) * inv0 / op.SOFTCAP), -1, keepdim=True).abs()
    # |L_moved| <= log V + 15 (capped logits lie in [-15, 15])
    lmax = torch.log(torch.tensor(float(base.shape[1]), dtype=torch.float64)) + 2 * op.SOFTCAP
    return 64 * 2.0 ** -24 * (lclean + lmax) / b64(steps)


@pytest.mark.parametrize('sigma', [5e-2, 2e-1])
def test_cycle_derivatives_match_oracle(sigma):
    n, width, V, P = 48, 512, 4096, 512
    log_case(f'cycle_derivatives n={n} V={V} P={P} sigma={sigma}')
    args = _case(n, width, V, P, sigma, seed=3)
    got = probes.cycle_derivatives(*(t.to(DEV) for t in args), width=width).cpu()
    ref = op.cycle_derivatives(*(t.double() if t.is_floating_point() else t for t in args), width=width)
    assert got.shape == (n, P) and torch.isfinite(got).all()
    assert torch.all(got[args[2] < 0] == 0)
    err = (got.double() - ref).abs()
    bound = _bound(*args, width)
    assert (err <= bound).all(), (float(err.max()), float(bound.min()))
    assert float(ref.abs().mean()) > 10 * float(bound.mean())   # the derivatives carry signal well above the bound


def test_row_derivatives_equal_cycle_entries():
    """Each token's own K directions: the same kernel arithmetic on gathered dots and |D|^2, so the entries
    equal the full cycle's bit for bit; the oracle agrees within the bound."""
    n, width, V, P, K = 32, 512, 4096, 512, 24
    log_case(f'row_derivatives n={n} K={K}')
    base, C, y, steps, sq, dots, dir_sq = _case(n, width, V, P, 5e-2, seed=4)
    rows = torch.randint(0, P, (n, K), generator=torch.Generator().manual_seed(9))
    full = probes.cycle_derivatives(*(t.to(DEV) for t in (base, C, y, steps, sq, dots, dir_sq)), width=width)
    got = probes.row_derivatives(base.to(DEV), C.to(DEV), rows.to(DEV), y.to(DEV), steps.to(DEV), sq.to(DEV),
                                 dots.gather(1, rows).to(DEV), dir_sq[rows].to(DEV), width=width)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), full.cpu().gather(1, rows))
    ref = op.row_derivatives(base.double(), C.double(), rows, y, steps.double(), sq.double(),
                             dots.gather(1, rows).double(), dir_sq[rows].double(), width=width)
    assert ((got.cpu().double() - ref).abs() <= _bound(base, C, y, steps, sq, dots, dir_sq, width)).all()


def test_probes_runtime_vocab_odd_counts_and_invalid_rows():
    """A vocabulary other than the model's 4096 (the kernel instance that reads the chunk count at run time), odd
    direction counts (the unpaired last direction of the kernel's two-direction steps), and row lists holding
    invalid rows (-1 and past P): NaN at those entries, every other entry bit for bit the full cycle's, and the
    cycle within the bound of the oracle."""
    n, width, V, P, K = 20, 512, 768, 33, 7
    log_case(f'probes n={n} V={V} P={P} K={K} invalid rows')
    args = _case(n, width, V, P, 5e-2, seed=5)
    base, C, y, steps, sq, dots, dir_sq = args
    full = probes.cycle_derivatives(*(t.to(DEV) for t in args), width=width).cpu()
    ref = op.cycle_derivatives(*(t.double() if t.is_floating_point() else t for t in args), width=width)
    assert ((full.double() - ref).abs() <= _bound(*args, width)).all()
    rows = torch.randint(0, P, (n, K), generator=torch.Generator().manual_seed(11))
    rows[::3, 0] = -1
    rows[1::4, K - 1] = P + 3
    valid = (rows >= 0) & (rows < P)
    rc = rows.clamp(0, P - 1)
    got = probes.row_derivatives(base.to(DEV), C.to(DEV), rows.to(DEV), y.to(DEV), steps.to(DEV), sq.to(DEV),
                                 dots.gather(1, rc).to(DEV), dir_sq[rc].to(DEV), width=width).cpu()
    assert torch.isnan(got[~valid]).all()
    assert torch.equal(got[valid], full.gather(1, rc)[valid])
    for k in (1, 2):  # one direction (no prefetch at all) and two (the first and the last, no loop trip)
        rk = rows[:, :k].clamp(0, P - 1).contiguous()
        gk = probes.row_derivatives(base.to(DEV), C.to(DEV), rk.to(DEV), y.to(DEV), steps.to(DEV), sq.to(DEV),
                                    dots.gather(1, rk).to(DEV), dir_sq[rk].to(DEV), width=width).cpu()
        assert torch.equal(gk, full.gather(1, rk)), k

