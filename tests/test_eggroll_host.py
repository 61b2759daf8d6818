"""Host-side bookkeeping of noise_amd.eggroll against the oracle's restatement of the reference's loop (CPU)."""
import pytest
import torch

from noise_amd.eggroll import member_sequences
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
