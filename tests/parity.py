"""Shared checks: the HIP restore (through the C ABI) against the oracle."""
from __future__ import annotations

import numpy as np

import oracle
from foundry_amd.restore import Archive


def gpu_and_oracle(synth, policy=0, relocate=True, template_of=None, threads=4):
    iv = synth.intervals() if relocate else None
    arch = Archive.from_synth(synth)
    if iv is not None:
        arch.set_relocation(*iv, policy=policy)
    if template_of is not None:
        arch.set_groups(template_of)
    arch.restore()
    ref = oracle.Restore(synth.images(), iv, policy=policy, template_of=template_of, threads=threads)
    return arch, ref


def assert_restore_parity(arch, ref, graphs=None):
    """Every output of the restore, bit for bit."""
    G = ref.n
    np.testing.assert_array_equal(arch.groups(), ref.groups(), err_msg="template_of")
    np.testing.assert_array_equal(arch.digests(), ref.digests(), err_msg="digests (key, edge, type, kernel-entry)")
    np.testing.assert_array_equal(arch.status(), ref.status(), err_msg="graph status")
    np.testing.assert_array_equal(arch.override_offsets(), ref.override_offsets(), err_msg="override offsets")
    pb = arch.param_bytes()
    assert int(pb.sum()) == ref.total_param_bytes()
    for g in graphs if graphs is not None else range(G):
        np.testing.assert_array_equal(arch.node_flags(g), ref.node_flags(g), err_msg=f"node flags g={g}")
        np.testing.assert_array_equal(arch.node_words(g), ref.node_words(g), err_msg=f"node words g={g}")
        np.testing.assert_array_equal(arch.param_image(g), ref.param_image(g), err_msg=f"param image g={g}")
        np.testing.assert_array_equal(arch.node_pointers(g), ref.node_pointers(g), err_msg=f"node pointers g={g}")
        a, b = arch.overrides(g), ref.overrides(g)
        assert a.shape == b.shape, f"override count g={g}: {a.shape} vs {b.shape}"
        np.testing.assert_array_equal(a, b, err_msg=f"overrides g={g}")


def assert_live_matches(arch, ref, template):
    w1, s1, c1 = arch.live(template)
    w2, s2, c2 = ref.live(template)
    assert c1 == c2
    np.testing.assert_array_equal(s1, s2, err_msg="live node sources")
    np.testing.assert_array_equal(w1, w2, err_msg="live words")
