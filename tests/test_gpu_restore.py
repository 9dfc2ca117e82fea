"""HIP restore vs the oracle, bit for bit, through the C ABI.

Every test builds a seeded synthetic archive with the product's generator,
runs the GPU restore (hash, group, node pass, fused diff + relocate) and the
oracle's CPU restore on the same images and interval table, and compares
every output.
"""
import numpy as np
import pytest

from foundry_amd import synth
from foundry_amd._lib import NODE_DESC, NODE_LAYOUT, RELOC_INCLUSIVE
from tests.parity import assert_live_matches, assert_restore_parity, gpu_and_oracle

pytestmark = pytest.mark.gpu


def _print_case(name, p):
    print(f"[case] {name}: graphs={p.num_graphs} nodes={p.nodes_per_graph} groups={p.num_groups} "
          f"intervals={p.num_intervals} seed={p.seed:#x}", flush=True)


def test_preset1_full(cuda):
    p = synth.preset(1)
    _print_case("preset1", p)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    assert_restore_parity(arch, ref)
    assert len(set(arch.groups().tolist())) == 1
    assert arch.override_offsets()[-1] > 0


def test_preset2_reduced(cuda):
    # Decode-style archive at reduced size: the full 40k-interval table, 4 groups.
    p = synth.preset(2, num_graphs=24, nodes_per_graph=300)
    _print_case("preset2-reduced", p)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    assert_restore_parity(arch, ref)
    assert len(set(arch.groups().tolist())) == 4


def test_mixed_nodes_ragged_params(cuda):
    # Memset/memcpy/event nodes, extra-style arg buffers, odd-sized params and
    # batch-size-dependent layouts: every branch of the node pass.
    p = synth.preset(
        2, num_graphs=12, nodes_per_graph=400, num_groups=3, ragged=1, extra_style_pct=10,
        memset_pct=8, memcpy_pct=6, event_pct=6, layout_var_pct=10, num_intervals=3000,
        seed=0xABCDEF,
    )
    _print_case("mixed-ragged", p)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    assert_restore_parity(arch, ref)
    flags = np.concatenate([ref.node_flags(g) for g in range(s.num_graphs)])
    assert (flags & NODE_LAYOUT).any() and (flags & NODE_DESC).any() and (flags & 0x04).any()


def test_inclusive_policy_and_no_relocation(cuda):
    p = synth.preset(1, num_graphs=8)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s, policy=RELOC_INCLUSIVE)
    assert_restore_parity(arch, ref)
    arch2, ref2 = gpu_and_oracle(s, relocate=False)
    assert_restore_parity(arch2, ref2)


def test_explicit_groups(cuda):
    # Manifest-style grouping: every graph its own template, then pairs.
    p = synth.preset(1, num_graphs=6)
    s = synth.SynthArchive(p)
    tmpl = np.array([0, 0, 2, 2, 4, 4], dtype=np.uint32)
    arch, ref = gpu_and_oracle(s, template_of=tmpl)
    assert_restore_parity(arch, ref)


def test_restore_twice_is_identical(cuda):
    p = synth.preset(2, num_graphs=8, nodes_per_graph=200, num_groups=2)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    first = [arch.overrides(g) for g in range(s.num_graphs)]
    arch.restore()
    for g in range(s.num_graphs):
        np.testing.assert_array_equal(arch.overrides(g), first[g])
    assert_restore_parity(arch, ref)


def test_switch_sequence(cuda):
    p = synth.preset(2, num_graphs=16, nodes_per_graph=250, num_groups=2, layout_var_pct=5)
    _print_case("switch", p)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    seq = synth.switch_sequence(0x5EED, s.num_graphs, 200)
    templates = sorted(set(ref.groups().tolist()))
    for i, g in enumerate(seq.tolist()):
        arch.switch(g)
        ref.switch(g)
        if i % 25 == 0:
            for t in templates:
                assert_live_matches(arch, ref, t)
    for t in templates:
        assert_live_matches(arch, ref, t)
    # End state: the live image equals R_g on every node without a layout change.
    for t in templates:
        words, src, cur = arch.live(t)
        img = ref.param_image(cur)
        flags = ref.node_flags(cur)
        tw, gw = ref.node_words(t), ref.node_words(cur)
        for n in np.nonzero((flags & NODE_LAYOUT) == 0)[0]:
            np.testing.assert_array_equal(words[tw[n]:tw[n + 1]], img[gw[n]:gw[n + 1]])


def test_graph_longer_than_the_chunk_shift_table(cuda):
    # 66,000 nodes = 258 chunks of 256: the first two chunks of each graph are
    # shifted past the node-type and kernel-entry streams without the table.
    p = synth.preset(1, num_graphs=3, nodes_per_graph=66000)
    _print_case("long-graphs", p)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    assert_restore_parity(arch, ref)
