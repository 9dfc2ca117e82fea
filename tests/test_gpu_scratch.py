"""The restore's bounded scratch and its exact fallback.

A restore keeps a bounded share of candidate words per diff sub-range
(continued in spill space shared by a tile's sub-ranges), a bounded override
region per graph and no ragged-word sources.  An archive that needs more -- differences too
dense for the regions and the spill space, or params that are not whole aligned
words -- makes the restore run again with what it lacked before any result
is read, and the archive keeps that layout.  Every output must equal the
oracle's either way, the second restore included."""
import pytest

from foundry_amd import synth
from tests.parity import assert_restore_parity, gpu_and_oracle

pytestmark = pytest.mark.gpu

FULL, RAGGED = 0x2, 0x4  # scratch level 2 (full capacity); ragged-word sources held


def _check(p, want_scratch):
    print(f"[case] graphs={p.num_graphs} nodes={p.nodes_per_graph} diff={p.diff_lo}-{p.diff_hi} "
          f"ragged={p.ragged} seed={p.seed:#x}", flush=True)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s, threads=8)
    assert arch.info()["scratch"] == want_scratch
    assert_restore_parity(arch, ref)
    arch.restore()  # the archive's later restores use the layout it settled on
    assert arch.info()["scratch"] == want_scratch
    assert_restore_parity(arch, ref)
    arch.close()


def test_sparse_differences_fit_the_compact_scratch(cuda):
    _check(synth.preset(2, num_graphs=24, num_groups=2, seed=0x5C01), 0)


def test_dense_differences_overflow_to_full_scratch(cuda):
    # Half the words of every member differ: more than levels 0 and 1 hold
    # (in a sub-range's region and its slot's spill space, and in a graph's
    # record region).
    _check(synth.preset(2, num_graphs=24, num_groups=2, diff_lo=0.5, diff_hi=0.5, seed=0x5C02), FULL)


def test_clustered_differences_spill(cuda):
    # Runs of 64-256 differing bytes at 10% (the MoE-style shape): some
    # sub-ranges hold more candidates than their regions, and the rest go to
    # their slot's spill space.
    _check(synth.preset(3, num_graphs=16, num_groups=2, nodes_per_graph=600, seed=0x5C03), 0)


def test_ragged_params_restore_again_with_sources(cuda):
    _check(synth.preset(2, num_graphs=12, num_groups=2, ragged=1, seed=0x5C04), RAGGED)
