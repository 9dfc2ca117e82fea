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
