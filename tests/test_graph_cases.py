"""The group-graph test archives, checked on the CPU: the independent reader
sees the nodes and id-named dependencies that were written, and the oracle
restores exactly the params, pointers, flags and override sets the GPU tests
expect before they launch anything."""
import numpy as np

import cugraph_reader as R
import graph_cases as GC
import oracle

BHASH = 0x0123456789ABCDEF
BASE = 0x7E5500000000  # stands in for the device buffer address


def _restore():
    iv = ([GC.SAVED], [GC.SAVED + GC.BUF_BYTES], [BASE])
    return oracle.Restore(GC.images(BHASH), iv)


def test_reader_sees_written_nodes_and_id_named_edges():
    arc = R.read(GC.image_of(GC.Spec(), BHASH))
    assert [n.type for n in arc.nodes] == [0, 0, 0, 0, 1, 2, 3, 4, 5, 0, 0]
    assert [n.node_id for n in arc.nodes] == list(range(100, 111))
    assert arc.deps == [(100 + a, 100 + b) for a, b in GC.EDGES]
    assert arc.nodes[2].kernel.params == [("ARG", 0, 24)]
    assert arc.nodes[1].kernel.name == b"probe_blob"


def test_groups_and_relocated_images():
    ref = _restore()
    assert list(ref.groups()) == [0, 0, 0, 0, 0, 5]
    for g, s in enumerate(GC.SPECS):
        assert list(ref.param_image(g)) == GC.expected_image(s, BHASH, BASE), g
        assert list(ref.node_pointers(g)) == GC.expected_pointers(s, BASE), g
    # Every saved pointer landed inside the relocated buffer.
    img = ref.param_image(0)
    assert int(img[0]) == BASE


def test_flags_and_override_nodes():
    ref = _restore()
    t = GC.SPECS[0]
    expect_override_nodes = {1: {0, 1, 3}, 2: set(), 3: {0}, 4: {2}}
    for g in GC.GROUP_A[1:]:
        s = GC.SPECS[g]
        fl = ref.node_flags(g)
        own = {n for n in range(len(fl)) if fl[n] & 0x03}
        assert own == GC.own_nodes(s, t), g
        layout = {n for n in range(len(fl)) if fl[n] & 0x01}
        assert layout == ({1} if s.layout_mix else set()), g
        assert set(int(x) for x in ref.overrides(g)["node"]) == expect_override_nodes[g], g


def test_expected_results_are_self_consistent():
    s = GC.SPECS[1]
    slots, fill, copy = GC.expected_buffer(s)
    assert slots[10] == GC.mix(GC.mix(slots[0], 9), 10)
    assert slots[3] == 5 * 4 * 64
    assert len(fill) == 4 * s.fill_words and copy == fill[:256]
    assert np.uint64(GC.mix(0, 0)) == 0
