"""HIP restore vs the oracle at the workloads' full sizes.

The decode-style (256 graphs x 1200 nodes, 40k intervals) and MoE-style
(256 graphs x ~3000 nodes, memset/memcpy nodes, 16 groups) archives are
compared output for output with the oracle's restore of the same images.
The 1024-graph archive (8 GB of params) is restored whole on the GPU and
checked on a sample: the oracle restores only the sampled graphs (each
group's template among them), and every per-graph output must equal the
GPU's for the same graph -- a graph's restore depends on its template and
the interval table alone, not on which other graphs are open.
"""
import numpy as np
import pytest

import oracle
from foundry_amd import synth
from foundry_amd.restore import Archive
from oracle import Restore
from tests.parity import assert_restore_parity, gpu_and_oracle

pytestmark = pytest.mark.gpu


def _case(name, p):
    print(f"[case] {name}: graphs={p.num_graphs} nodes={p.nodes_per_graph} groups={p.num_groups} "
          f"intervals={p.num_intervals} seed={p.seed:#x}", flush=True)


@pytest.mark.parametrize("preset", [2, 3])
def test_full_size_parity(cuda, preset):
    p = synth.preset(preset)
    _case(f"preset{preset}-full", p)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s, threads=16)
    assert_restore_parity(arch, ref)
    assert len(set(arch.groups().tolist())) == p.num_groups
    arch.close()


@pytest.fixture(scope="module")
def c5(cuda):
    """The 1024-graph archive, restored whole on the GPU (shared by the
    sampled restore check and the switch sequence)."""
    p = synth.preset(5)
    _case("preset5-full", p)
    s = synth.SynthArchive(p)
    lo, hi, new_lo = s.intervals()
    arch = Archive.from_synth(s)
    arch.set_relocation(lo, hi, new_lo)
    arch.restore()
    yield p, s, arch, (lo, hi, new_lo)
    arch.close()


def test_1024_graph_archive_sampled(c5):
    p, s, arch, (lo, hi, new_lo) = c5
    groups = arch.groups()
    assert len(set(groups.tolist())) == p.num_groups
    rng = np.random.default_rng(5)
    templates = sorted(set(groups.tolist()))
    chosen = set()
    for t in rng.choice(templates, size=6, replace=False).tolist():
        members = np.flatnonzero(groups == t).tolist()
        chosen.add(t)
        chosen.update(rng.choice([m for m in members if m != t], size=2, replace=False).tolist())
    sample = sorted(chosen)
    print(f"[case] sampled graphs {sample}", flush=True)
    ref = Restore([s.image(g) for g in sample], (lo, hi, new_lo), threads=16)
    sub_groups = ref.groups()
    for i, g in enumerate(sample):
        assert sample[sub_groups[i]] == groups[g], f"template of graph {g}"
        np.testing.assert_array_equal(arch.node_flags(g), ref.node_flags(i), err_msg=f"node flags g={g}")
        np.testing.assert_array_equal(arch.node_words(g), ref.node_words(i), err_msg=f"node words g={g}")
        np.testing.assert_array_equal(arch.param_image(g), ref.param_image(i), err_msg=f"param image g={g}")
        np.testing.assert_array_equal(arch.node_pointers(g), ref.node_pointers(i), err_msg=f"node pointers g={g}")
        np.testing.assert_array_equal(arch.overrides(g), ref.overrides(i), err_msg=f"overrides g={g}")
    np.testing.assert_array_equal(arch.digests()[sample], ref.digests(), err_msg="digests")


def test_1024_graph_archive_switch_sequence(c5):
    """The 10,000 seeded switches of the 1024-graph workload, then every
    group's live state against the oracle's: the live image depends only on
    the last graph switched to in the group (the switch end state of
    csrc/CUDAGraph.cpp:340-461), so the oracle restores each template with
    that graph alone and switches once."""
    p, s, arch, (lo, hi, new_lo) = c5
    groups = arch.groups()
    seq = synth.switch_sequence(p.seed, s.num_graphs, 10_000)
    print(f"[case] preset5-full: {len(seq)} seeded switches", flush=True)
    # The first half one call each, the second half in one sequence call
    # (switches of different groups batched into shared launches).
    for g in seq[:5000]:
        arch.switch(int(g))
    arch.switch_sequence(seq[5000:])
    last = {int(t): int(t) for t in set(groups.tolist())}
    for g in seq:
        last[int(groups[g])] = int(g)
    assert len(last) == p.num_groups
    for t, g in sorted(last.items()):
        w, src, cur = arch.live(t)
        assert cur == g, f"group {t}"
        pair = [t] if g == t else [t, g]
        ref = Restore([s.image(x) for x in pair], (lo, hi, new_lo), template_of=[0] * len(pair), threads=16)
        if g != t:
            ref.switch(1)
        w2, src2, cur2 = ref.live(0)
        np.testing.assert_array_equal(w, w2, err_msg=f"live words of group {t} (last graph {g})")
        np.testing.assert_array_equal(src, np.array(pair, dtype=np.uint32)[src2], err_msg=f"node sources of group {t}")


@pytest.mark.parametrize("spins", [0, 1])
def test_1024_graph_grouping_when_keys_are_hashed_by_waiters(c5, spins):
    """The grouping scan's fallback: a workgroup that finds a lower graph's
    key hash unpublished hashes that key itself after `spins` rounds of
    sleep (0: at once, so nearly every lookup takes the fallback).  Graphs
    above 512 scan the lower graphs in more than one step.  Groups and
    digests must equal the oracle's key grouping of all 1024 graphs and the
    default restore's digests; runs after the switch sequence, and leaves
    the default wait behind."""
    p, s, arch, _ = c5
    print(f"[case] preset5-full: grouping with a wait of {spins} spins", flush=True)
    keys = [oracle.topology_key_saved(s.image(g)) for g in range(s.num_graphs)]
    want = oracle.group_by_keys(keys)
    digests = arch.digests()
    arch.set_group_wait(spins)
    try:
        arch.restore()
        np.testing.assert_array_equal(arch.groups(), want, err_msg="template_of")
        np.testing.assert_array_equal(arch.digests(), digests, err_msg="digests")
    finally:
        arch.set_group_wait(1 << 14)
        arch.restore()
    np.testing.assert_array_equal(arch.groups(), want, err_msg="template_of (default wait)")


def test_decode_style_grouping_when_keys_are_hashed_by_waiters(cuda):
    p = synth.preset(2)
    _case("preset2-full, grouping wait 0", p)
    s = synth.SynthArchive(p)
    lo, hi, new_lo = s.intervals()
    arch = Archive.from_synth(s)
    arch.set_relocation(lo, hi, new_lo)
    arch.set_group_wait(0)
    arch.restore()
    ref = Restore(s.images(), (lo, hi, new_lo), threads=16)
    assert_restore_parity(arch, ref, graphs=range(0, s.num_graphs, 17))
    arch.close()
