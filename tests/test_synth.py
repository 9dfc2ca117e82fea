"""The synthetic-archive generator: seeded and deterministic, and its
archives read back through the independent reader."""
import numpy as np

from foundry_amd import synth
from tests import cugraph_reader as R


def test_same_seed_same_bytes():
    p = synth.preset(2, num_graphs=6, nodes_per_graph=50, num_intervals=300)
    a, b = synth.SynthArchive(p, threads=1), synth.SynthArchive(p, threads=4)
    assert a.images() == b.images()
    for x, y in zip(a.intervals(), b.intervals()):
        np.testing.assert_array_equal(x, y)


def test_other_seed_other_bytes():
    p = synth.preset(2, num_graphs=4, nodes_per_graph=50, num_intervals=300)
    q = synth.preset(2, num_graphs=4, nodes_per_graph=50, num_intervals=300, seed=p.seed + 1)
    assert synth.SynthArchive(p).images() != synth.SynthArchive(q).images()


def test_archives_parse_and_intervals_tile():
    p = synth.preset(2, num_graphs=5, nodes_per_graph=60, num_intervals=500)
    s = synth.SynthArchive(p)
    for img in s.images():
        arc = R.read(img)
        assert len(arc.nodes) == 60
        assert all(n.type == 0 for n in arc.nodes)
    lo, hi, nlo = s.intervals()
    assert len(lo) == 500 and (lo < hi).all() and (hi[:-1] <= lo[1:]).all()
    # the intervals tile the region exactly
    assert lo[0] == p.region_base and hi[-1] == p.region_base + p.region_size
    assert (hi[:-1] == lo[1:]).all()


def test_decode_preset_shape():
    p = synth.preset(2)
    assert (p.num_graphs, p.num_groups, p.nodes_per_graph, p.num_intervals) == (256, 4, 1200, 40000)
    assert p.region_size == 64 << 30 and abs(p.pointer_frac - 0.25) < 1e-9


def test_sink_mode_names_one_kernel_and_keeps_groups_apart():
    import oracle

    p = synth.preset(5, num_graphs=16, num_groups=8, nodes_per_graph=40, num_intervals=200)
    p.sink_hash = 0xFEEDFACE12345678
    s = synth.SynthArchive(p)
    imgs = s.images()
    for img in imgs:
        arc = R.read(img)
        for n in arc.nodes:
            if n.type == 0:
                assert n.kernel.name == b"fdy_sink" and n.kernel.binary_hash == p.sink_hash
                assert n.kernel.kna_flags == 0  # no cluster dims
    ref = oracle.Restore(imgs, s.intervals())
    assert len(set(int(t) for t in ref.groups())) == 8


def test_differences_confined_to_a_few_nodes():
    """diff_node_pct=10: the members' differing words fall in about a tenth
    of the kernel nodes, the same ones in every member, and the overall
    fraction of differing words stays about that of the unconfined archive."""
    from oracle import Restore

    def node_sets(pct):
        p = synth.preset(2, num_graphs=12, num_groups=1, nodes_per_graph=400, num_intervals=500)
        p.diff_node_pct = pct
        s = synth.SynthArchive(p)
        ref = Restore([s.image(g) for g in range(12)], s.intervals(), threads=4)
        sets = []
        for g in range(1, 12):
            nodes = set(ref.overrides(g)["node"].tolist())
            nodes |= set(np.flatnonzero(ref.node_flags(g)).tolist())
            sets.append(nodes)
        records = sum(len(ref.overrides(g)["node"]) for g in range(1, 12))
        return sets, records

    wide, r_wide = node_sets(0)
    few, r_few = node_sets(10)
    union = set().union(*few)
    assert 15 <= len(union) <= 70, len(union)  # about 40 of 400
    assert min(len(x) for x in wide) > 200
    assert 0.5 < r_few / r_wide < 2.0, (r_few, r_wide)
