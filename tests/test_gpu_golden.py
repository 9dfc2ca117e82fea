"""The HIP restore on the hand-assembled fixtures of tests/golden/ (read from
disk through fdy_archive_open), against the hand-derived values of
expected.json and the oracle."""
import json
import os

import numpy as np
import pytest

import oracle
from foundry_amd.restore import Archive
from tests.parity import assert_restore_parity

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
EXP = json.load(open(os.path.join(GOLDEN, "expected.json")))
NAMES = ("tiny_a", "tiny_b", "tiny_c", "tiny_d")


def test_golden_fixtures(cuda):
    print("[case] golden fixtures tiny_a..tiny_d", flush=True)
    paths = [os.path.join(GOLDEN, n + ".cugraph") for n in NAMES]
    images = [open(p, "rb").read() for p in paths]
    iv = np.array(EXP["relocation"]["intervals"], dtype=np.uint64)
    lo, hi, nlo = iv[:, 0].copy(), iv[:, 1].copy(), iv[:, 2].copy()
    arch = Archive.open(paths)
    try:
        arch.restore()
        assert arch.groups().tolist() == [0, 0, 2, 3]
        assert arch.param_image(0).tolist() == EXP["tiny_a"]["words"]
        assert arch.param_image(1).tolist() == EXP["tiny_b"]["words"]
        o = arch.overrides(1)
        assert [[int(x["word"]), int(x["node"]), int(x["value"])] for x in o] == EXP["a_b_group"]["overrides_b"]
        assert_restore_parity(arch, oracle.Restore(images))

        arch.set_relocation(lo, hi, nlo)
        arch.restore()
        e = EXP["relocation"]
        assert arch.param_image(0).tolist() == e["words_a"]
        assert int(arch.node_pointers(0)[2]) == e["memset_dst_a"]
        ptr_c = arch.node_pointers(2)
        assert int(ptr_c[4]) == e["memcpy_dst_c"] and int(ptr_c[5]) == e["memcpy_src_c"]
        assert_restore_parity(arch, oracle.Restore(images, (lo, hi, nlo)))
    finally:
        arch.close()


def test_attribute_merge_fixtures(cuda):
    """Conflicting common, per-node and required-cluster launch attributes:
    the GPU's DESC flags, groups and status against the hand-derived values,
    then every output against the oracle."""
    print("[case] golden fixtures attr_t, attr_m", flush=True)
    e = EXP["attrs"]
    paths = [os.path.join(GOLDEN, n + ".cugraph") for n in ("attr_t", "attr_m")]
    images = [open(p, "rb").read() for p in paths]
    arch = Archive.open(paths)
    try:
        arch.restore()
        assert arch.groups().tolist() == e["template_of"]
        assert arch.status().tolist() == e["status"]
        desc = ((arch.node_flags(1) & 2) != 0).astype(int).tolist()
        assert desc == e["desc_m"]
        assert not (arch.node_flags(1) & 1).any()  # same layout everywhere
        assert arch.param_image(0).tolist() == e["words_t"]
        assert arch.param_image(1).tolist() == e["words_m"]
        o = arch.overrides(1)
        assert [[int(x["word"]), int(x["node"]), int(x["value"])] for x in o] == e["overrides_m"]
        assert_restore_parity(arch, oracle.Restore(images))
    finally:
        arch.close()


def test_digest_collision_groups_by_exact_key_bytes(cuda):
    """Keys with equal CRC-64/XZ and length but other bytes (forged, see
    tests/refcrc.forge_collision) form separate groups, as the reference's
    exact-string partition does; the graphs that met a colliding key are
    flagged.  Then switches within both groups."""
    import collision_cases as CC
    from parity import assert_live_matches

    print("[case] forged CRC-64/XZ key collision, 5 graphs", flush=True)
    images = CC.images()
    arch = Archive.from_images(images)
    try:
        arch.restore()
        assert arch.groups().tolist() == CC.TEMPLATE_OF
        assert arch.status().tolist() == CC.STATUS
        ref = oracle.Restore(images)
        assert_restore_parity(arch, ref)
        for g in (3, 2, 1):
            arch.switch(g)
            ref.switch(g)
        assert_live_matches(arch, ref, 0)
        assert_live_matches(arch, ref, 1)
    finally:
        arch.close()


def test_unaligned_param_index_and_many_params(cuda):
    """Param-index offsets 4, 21 and 29 (entries read at any byte offset) and
    a node of 18 params (two past those kept field-major): hand-derived
    words and overrides, then every output against the oracle, with and
    without relocation."""
    print("[case] golden fixtures tiny_e, tiny_f", flush=True)
    e = EXP["unaligned_pidx"]
    paths = [os.path.join(GOLDEN, n + ".cugraph") for n in ("tiny_e", "tiny_f")]
    images = [open(p, "rb").read() for p in paths]
    iv = np.array(EXP["relocation"]["intervals"], dtype=np.uint64)
    lo, hi, nlo = iv[:, 0].copy(), iv[:, 1].copy(), iv[:, 2].copy()
    arch = Archive.open(paths)
    try:
        arch.restore()
        assert arch.groups().tolist() == e["template_of"]
        assert np.diff(arch.node_words(0)).tolist() == e["node_words"]
        assert arch.param_image(0).tolist() == e["words_e"]
        assert arch.param_image(1).tolist() == e["words_f"]
        o = arch.overrides(1)
        assert [[int(x["word"]), int(x["node"]), int(x["value"])] for x in o] == e["overrides_f"]
        assert_restore_parity(arch, oracle.Restore(images))
        arch.set_relocation(lo, hi, nlo)
        arch.restore()
        assert arch.param_image(0).tolist() == e["words_e_relocated"]
        assert_restore_parity(arch, oracle.Restore(images, (lo, hi, nlo)))
    finally:
        arch.close()
