"""Host-side bookkeeping of noise_amd.eggroll against the oracle's restatement of the reference's loop (CPU)."""
import socket

import pytest
import torch
import torch.multiprocessing as mp

from noise_amd.eggroll import gather_losses, member_sequences
from oracle import eggroll as oe


@pytest.mark.parametrize('pairs,batch,chunk,world', [(1536, 8, 256, 1), (131072, 8, 256, 1), (4096, 8, 256, 2),
                                                     (24, 8, 4, 1), (4, 2, 2, 1), (512, 8, 256, 1)])
def test_member_sequences_follow_the_reference_chunks(pairs, batch, chunk, world):
    members = max(2 * pairs, 2 * batch)
    per_seq, per_rank = members // batch, members // world
    want = oe.chunk_sequences(members, per_seq, chunk, world)
    for rank in range(world):
        lo, hi = rank * per_rank, (rank + 1) * per_rank
        got = member_sequences(lo, hi, per_seq, chunk)
        assert torch.equal(got, want[lo:hi]), rank
        # any split of the rank's members into kernel passes sees the same mapping
        for c0 in range(lo, hi, 6):
            assert torch.equal(member_sequences(c0, min(hi, c0 + 6), per_seq, chunk), want[c0:min(hi, c0 + 6)])


def _gather_rank(rank, world, port, per_rank, out):
    torch.distributed.init_process_group('gloo', init_method=f'tcp://127.0.0.1:{port}', rank=rank,
                                         world_size=world)
    try:
        # rank r's share: the losses of members r * per_rank .. (r + 1) * per_rank - 1 (CPU tensors on gloo)
        share = torch.arange(rank * per_rank, (rank + 1) * per_rank, dtype=torch.float32) * 0.5 + 3.0
        got = gather_losses(share, world)
        out[rank] = got.tolist()
    finally:
        torch.distributed.destroy_process_group()


@pytest.mark.parametrize('world', [2, 3])
def test_gather_losses_puts_every_rank_share_in_member_order(world):
    """The multi-rank loss gather (train/val/eggroll.py:147-150) on gloo with CPU tensors, one process per rank:
    every rank ends with the whole population in member order, so the fitness and update it rebuilds are the same
    on every rank and equal to the one-rank run."""
    with socket.socket() as s:
        s.bind(('127.0.0.1', 0))
        port = s.getsockname()[1]
    per_rank = 6
    out = mp.Manager().dict()
    mp.spawn(_gather_rank, args=(world, port, per_rank, out), nprocs=world, join=True)
    want = (torch.arange(world * per_rank, dtype=torch.float32) * 0.5 + 3.0).tolist()
    for rank in range(world):
        assert out[rank] == want, rank
    # one rank: the losses themselves
    one = torch.arange(4.0)
    assert gather_losses(one, 1) is one



def test_head_formats_map_to_the_library_and_unknown_ones_are_refused():
    """The host's head names map onto noise_head_ce's NOISE_HEAD_* values, and an unknown name is refused before any
    tensor is touched (no CPU path)."""
    from noise_amd import _lib
    from noise_amd.population import HEAD_FORMAT, HEAD_MODES, Weights
    assert set(HEAD_FORMAT) == set(HEAD_MODES)
    assert HEAD_FORMAT == {'fp32': _lib.HEAD_FP32, 'fp32_split': _lib.HEAD_FP32_SPLIT, 'bf16': _lib.HEAD_BF16}
    with pytest.raises(ValueError, match='head must be one of'):
        Weights({}, head='fp16')
