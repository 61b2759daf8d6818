"""Host-side guards of the forward: a shape the activation buffers or token ids do not cover is refused
before any kernel is launched (CPU only; the library is never called)."""
import types

import pytest
import torch

from noise_amd import _lib, population


class _Buf:
    def __init__(self, members, T):
        self.members, self.T = members, T

    def fits(self, members, T):
        return members <= self.members and T == self.T


def _weights():
    return types.SimpleNamespace(config=None, p={}, head_w=torch.empty(4096, 1))


@pytest.fixture
def no_launch(monkeypatch):
    def refuse(*a, **k):
        raise AssertionError('a kernel was launched')
    monkeypatch.setattr(_lib, 'call', refuse)
    monkeypatch.setattr(_lib, 'embed', refuse)


def _run(buf, sign, idx, targets=None, out=None, tok_mstride=0, reduction=_lib.CE_MEMBER_MEAN, logits=None):
    population.forward_chunk(_weights(), buf, {}, sign, idx, targets, 0, out, None, None, [], tok_mstride=tok_mstride,
                             reduction=reduction, logits=logits)


def test_flattened_batch_ids_are_refused(no_launch):
    """[B * T] ids read as one sequence of B * T tokens would size every grid three times too large."""
    B, T = 3, 256
    with pytest.raises(ValueError, match='buffers hold'):
        _run(_Buf(B, T), torch.zeros(B), torch.zeros(B * T, dtype=torch.int64), tok_mstride=T)


def test_short_token_ids_and_outputs_are_refused(no_launch):
    B, T = 3, 256
    buf = _Buf(B, T)
    with pytest.raises(ValueError, match='idx must'):
        _run(buf, torch.zeros(B), torch.zeros(2, T, dtype=torch.int64), tok_mstride=T)
    with pytest.raises(ValueError, match='targets must'):
        _run(buf, torch.zeros(B), torch.zeros(B, T, dtype=torch.int64), torch.zeros(T, dtype=torch.int64),
             tok_mstride=T)
    with pytest.raises(ValueError, match='out must'):
        _run(buf, torch.zeros(B), torch.zeros(B, T, dtype=torch.int64), torch.zeros(B, T, dtype=torch.int64),
             out=torch.zeros(B), tok_mstride=T, reduction=_lib.CE_NONE)
    with pytest.raises(ValueError, match='logits must'):
        _run(buf, torch.zeros(B), torch.zeros(B, T, dtype=torch.int64), tok_mstride=T,
             logits=torch.zeros(B, T, 100))
    with pytest.raises(ValueError, match='buffers hold'):
        _run(buf, torch.zeros(B + 1), torch.zeros(T, dtype=torch.int64))


def test_credit_wrappers_reject_bad_shapes_before_any_launch():
    from noise_amd import credit
    bf = torch.bfloat16
    raw, fixed = torch.zeros(1, 100, 8, 64), torch.zeros(1, 100, 8, 64)
    a = torch.zeros(2, 1, 100, 8, 64, dtype=bf)
    with pytest.raises(ValueError, match="'q' or 'k'"):
        credit.rerun('v', raw, a, 0.1, None, None, fixed, fixed, 50)
    with pytest.raises(ValueError, match='multiple of 128'):
        credit.rerun('q', raw, a, 0.1, None, None, fixed, fixed, 50)
    with pytest.raises(ValueError, match='multiple of 128'):
        credit.attention(raw, raw, raw, 50)
    raw, a = torch.zeros(1, 128, 8, 64), torch.zeros(2, 1, 128, 8, 64, dtype=bf)
    with pytest.raises(ValueError, match='fixed and values'):
        credit.rerun('k', raw, a, 0.1, None, None, raw[:, :64], raw, 50)
    with pytest.raises(ValueError, match='matched filter'):
        credit.credit_chunk('k', raw, a, 0.1, None, None, raw, raw, 50, raw, raw, torch.zeros(1, 8, 128, 64))
    with pytest.raises(ValueError, match='window'):
        credit.rerun('q', raw, a, 0.1, None, None, raw, raw, -1)
    with pytest.raises(ValueError, match='at least 128 rows'):
        credit.rerun('q', raw, a, 0.1, torch.zeros(1, 100, 1, 32), torch.zeros(1, 100, 1, 32), raw, raw, 50)
    with pytest.raises(ValueError, match='CUDA'):
        credit.rerun('q', raw, a, 0.1, torch.zeros(1, 128, 1, 32), torch.zeros(1, 128, 1, 32), raw, raw, 50)


def test_probe_rows_must_be_cuda():
    from noise_amd import probes
    z = torch.zeros
    with pytest.raises(ValueError, match='CUDA'):
        probes.row_derivatives(z(4, 256), z(8, 256), z(4, 2, dtype=torch.int64), z(4, dtype=torch.int64), z(4), z(4),
                               z(4, 2), z(4, 2))


def test_population_loss_rejects_mismatched_token_rows():
    """idx / targets are one shared [T] sequence or one [m, T] row per member; anything else is refused
    before any launch."""
    pop = population.Population.__new__(population.Population)
    sign = torch.zeros(4)
    i64 = torch.int64
    for idx, tgt in ((torch.zeros(3, 128, dtype=i64), torch.zeros(3, 128, dtype=i64)),   # 3 rows for 4 members
                     (torch.zeros(4, 128, dtype=i64), torch.zeros(128, dtype=i64)),      # shapes differ
                     (torch.zeros(1, 4, 128, dtype=i64), torch.zeros(1, 4, 128, dtype=i64))):
        with pytest.raises(ValueError, match=r'both be \[T\]'):
            pop.loss({}, {}, sign, idx, tgt)
