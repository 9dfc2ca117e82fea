"""The oracle against the hand-assembled fixtures in tests/golden/ (see
make_fixtures.py: every expected value there is written out by hand), and
its digests against the bit-serial CRC of streams read by the independent
reader (tests/cugraph_reader.py)."""
import json
import os
import struct

import numpy as np
import pytest

import oracle
from tests import cugraph_reader as R
from tests.refcrc import crc64_xz

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
EXP = json.load(open(os.path.join(GOLDEN, "expected.json")))
NAMES = ("tiny_a", "tiny_b", "tiny_c", "tiny_d")
LAYOUT, DESC, RAGGED, TEMPLATE = 1, 2, 4, 8


def img(name):
    with open(os.path.join(GOLDEN, name + ".cugraph"), "rb") as f:
        return f.read()


def intervals():
    iv = np.array(EXP["relocation"]["intervals"], dtype=np.uint64)
    return iv[:, 0].copy(), iv[:, 1].copy(), iv[:, 2].copy()


@pytest.mark.parametrize("name", ["tiny_a", "tiny_c", "tiny_d"])
def test_keys(name):
    e = EXP[name]
    assert oracle.topology_key_saved(img(name)).decode() == e["saved_key"]
    assert oracle.topology_key_recomputed(img(name)).decode() == e["recomputed_key"]


@pytest.mark.parametrize("name", ["tiny_a", "tiny_c"])
def test_param_extraction(name):
    for node, hx in EXP[name]["params"].items():
        assert oracle.extract_node_params(img(name), int(node)).hex() == hx


def test_fixture_words_follow_params():
    assert EXP["check"]["words_a_from_params"] == EXP["tiny_a"]["words"]


def test_restore_a_b_without_relocation():
    r = oracle.Restore([img("tiny_a"), img("tiny_b")])
    assert r.groups().tolist() == EXP["a_b_group"]["template_of"]
    assert r.param_image(0).tolist() == EXP["tiny_a"]["words"]
    assert r.param_image(1).tolist() == EXP["tiny_b"]["words"]
    assert np.diff(r.node_words(0)).tolist() == EXP["tiny_a"]["node_words"]
    assert len(r.overrides(0)) == 0
    o = r.overrides(1)
    assert [[int(x["word"]), int(x["node"]), int(x["value"])] for x in o] == EXP["a_b_group"]["overrides_b"]
    assert r.override_offsets().tolist() == [0, 0, 2]
    fa, fb = r.node_flags(0), r.node_flags(1)
    for n in EXP["tiny_a"]["ragged_nodes"]:
        assert fa[n] & RAGGED and fb[n] & RAGGED
    assert (fa & TEMPLATE).all() and not (fb & TEMPLATE).any()
    assert not (fb & (LAYOUT | DESC)).any()  # same descriptors, params differ only in words
    assert r.status().tolist() == [0, 0]


def test_restore_with_relocation():
    r = oracle.Restore([img("tiny_a"), img("tiny_b"), img("tiny_c")], intervals())
    e = EXP["relocation"]
    assert r.param_image(0).tolist() == e["words_a"]
    assert r.node_pointers(0)[2 * 1] == e["memset_dst_a"]
    ptr_c = r.node_pointers(2)
    assert ptr_c[2 * 2] == e["memcpy_dst_c"] and ptr_c[2 * 2 + 1] == e["memcpy_src_c"]
    assert r.param_image(2).tolist() == [e["words_a"][0] + 0x3000, EXP["tiny_c"]["words"][1]]
    # Relocated space: pointer words equal in a and b give no records.
    assert [[int(x["word"]), int(x["node"]), int(x["value"])] for x in r.overrides(1)] == EXP["a_b_group"]["overrides_b"]


def test_grouping_of_fixtures():
    # a and b share a key, c has its own, d's saved key is empty.
    r = oracle.Restore([img(n) for n in NAMES])
    assert r.groups().tolist() == [0, 0, 2, 3]


def _digests_from_reader(data: bytes):
    arc = R.read(data)
    d_key = crc64_xz(arc.key())
    d_edge = crc64_xz(arc.section("DEP")[: 8 * len(arc.deps)])
    types, kents = b"", b""
    for n, node in enumerate(arc.nodes):
        c = R.load_rule_cluster(arc, n) if node.type == 0 else (0, 0, 0)
        types += struct.pack("<B3xIII", node.type, *c)
        if node.type == 0:
            kents += struct.pack("<QQ", node.kernel.binary_hash, crc64_xz(node.kernel.name))
        else:
            kents += b"\0" * 16
    return [d_key, d_edge, crc64_xz(types), crc64_xz(kents)]


def test_digests_are_crcs_of_the_defined_streams():
    images = [img(n) for n in NAMES]
    r = oracle.Restore(images)
    d = r.digests()
    for i, data in enumerate(images):
        assert d[i].tolist() == _digests_from_reader(data), NAMES[i]


# ---- launch-attribute merge (attr_t / attr_m) ---------------------------

ATTR = EXP["attrs"]


def _attr_fixture_disagreements():
    """Which hand-derived attribute values the oracle (as currently built or
    mutated) does not reproduce: effective attributes, DESC flags, status."""
    t, m = img("attr_t"), img("attr_m")
    bad = []
    for n, want in enumerate(ATTR["effective_t"]):
        if oracle.effective_attrs(t, n) != want:
            bad.append(("effective_t", n))
    for n, want in enumerate(ATTR["effective_m"]):
        if oracle.effective_attrs(m, n) != want:
            bad.append(("effective_m", n))
    r = oracle.Restore([t, m])
    desc = ((r.node_flags(1) & DESC) != 0).astype(int).tolist()
    if desc != ATTR["desc_m"]:
        bad.append(("desc_m", desc))
    return bad, r


def test_attribute_merge_matches_the_hand_derived_values():
    bad, r = _attr_fixture_disagreements()
    assert bad == []
    assert r.groups().tolist() == ATTR["template_of"]
    assert r.status().tolist() == ATTR["status"]
    assert r.param_image(0).tolist() == ATTR["words_t"]
    assert r.param_image(1).tolist() == ATTR["words_m"]
    o = r.overrides(1)
    assert [[int(x["word"]), int(x["node"]), int(x["value"])] for x in o] == ATTR["overrides_m"]
    assert oracle.topology_key_recomputed(img("attr_t")).decode() == ATTR["recomputed_key_t"]
    assert oracle.topology_key_recomputed(img("attr_m")).decode() == ATTR["recomputed_key_m"]


@pytest.mark.parametrize("mutation", [1, 2, 3, 4, 5, 6])
def test_every_planted_merge_mistake_is_caught(mutation):
    """A mistake planted in the oracle's merge (common over per-node,
    negative values overriding, the required cluster ignored, per-node attrs
    replacing common ones, common attrs ignored, zero required dims kept)
    disagrees with the hand-derived values on at least one node."""
    oracle.set_mutation(mutation)
    try:
        bad, _ = _attr_fixture_disagreements()
    finally:
        oracle.set_mutation(0)
    assert bad, f"mutation {mutation} went unnoticed"


def test_planted_swap_changes_a_desc_flag():
    """The swapped merge order (common attrs over per-node ones) shows up in
    the DESC flags themselves, the output the GPU test compares."""
    oracle.set_mutation(1)
    try:
        bad, _ = _attr_fixture_disagreements()
    finally:
        oracle.set_mutation(0)
    assert any(k == "desc_m" for k, _ in bad)


# ---- unaligned param-index offsets, a node past 16 params (tiny_e / tiny_f) ----

UNAL = EXP["unaligned_pidx"]


def test_unaligned_param_index_offsets():
    r = oracle.Restore([img("tiny_e"), img("tiny_f")])
    assert r.groups().tolist() == UNAL["template_of"]
    assert np.diff(r.node_words(0)).tolist() == UNAL["node_words"]
    assert r.param_image(0).tolist() == UNAL["words_e"]
    assert r.param_image(1).tolist() == UNAL["words_f"]
    o = r.overrides(1)
    assert [[int(x["word"]), int(x["node"]), int(x["value"])] for x in o] == UNAL["overrides_f"]
    fe = r.node_flags(0)
    assert [n for n in range(4) if fe[n] & RAGGED] == UNAL["ragged_nodes"]
    r2 = oracle.Restore([img("tiny_e"), img("tiny_f")], intervals())
    assert r2.param_image(0).tolist() == UNAL["words_e_relocated"]
