"""HIP restore vs the oracle, bit for bit, through the C ABI.

Every test builds a seeded synthetic archive with the product's generator,
runs the GPU restore (hash, group, node pass, fused diff + relocate) and the
oracle's CPU restore on the same images and interval table, and compares
every output.
"""
import numpy as np
import pytest

import oracle
from foundry_amd._lib import FoundryError, check, restore_lib
from foundry_amd.restore import Archive

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


def test_explicit_template_of_another_length(cuda):
    # Graphs of 300 and 520 nodes grouped across lengths: a template's node n
    # sits at another lane of the field-major node table than the member's
    # node n, and a member longer than its template has nodes without one.
    a = synth.SynthArchive(synth.preset(1, num_graphs=2, nodes_per_graph=300, seed=11))
    b = synth.SynthArchive(synth.preset(1, num_graphs=2, nodes_per_graph=520, seed=12))
    images = a.images() + b.images()
    iv = a.intervals()
    tmpl = np.array([0, 2, 2, 0], dtype=np.uint32)
    print("[case] cross-length groups 300/520 nodes", flush=True)
    arch = Archive.from_images(images)
    arch.set_relocation(*iv)
    arch.set_groups(tmpl)
    arch.restore()
    ref = oracle.Restore(images, iv, template_of=tmpl)
    assert_restore_parity(arch, ref)
    arch.close()


def test_explicit_template_with_other_kernels(cuda):
    # Same length, different kernels (other seeds): grouped explicitly, every
    # node is compared against a template node of another name, function
    # hash and params.
    a = synth.SynthArchive(synth.preset(2, num_graphs=2, nodes_per_graph=400, num_groups=1, seed=21))
    b = synth.SynthArchive(synth.preset(2, num_graphs=2, nodes_per_graph=400, num_groups=1, seed=22))
    images = a.images() + b.images()
    iv = a.intervals()
    tmpl = np.array([0, 2, 2, 0], dtype=np.uint32)
    print("[case] explicit groups across kernels, 400 nodes", flush=True)
    arch = Archive.from_images(images)
    arch.set_relocation(*iv)
    arch.set_groups(tmpl)
    arch.restore()
    ref = oracle.Restore(images, iv, template_of=tmpl)
    assert_restore_parity(arch, ref)
    arch.close()


def test_restore_twice_is_identical(cuda):
    p = synth.preset(2, num_graphs=8, nodes_per_graph=200, num_groups=2)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    first = [arch.overrides(g) for g in range(s.num_graphs)]
    arch.restore()
    for g in range(s.num_graphs):
        np.testing.assert_array_equal(arch.overrides(g), first[g])
    assert_restore_parity(arch, ref)


def test_timed_restores(cuda):
    """Restores timed after every kernel, or only at the two phases'
    boundaries, give the same results; each mode's fields add up."""
    p = synth.preset(2, num_graphs=8, nodes_per_graph=200, num_groups=2)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    with pytest.raises(FoundryError):
        arch.timing()  # no timed restore yet
    with pytest.raises(FoundryError):
        check(restore_lib().fdy_set_timing(arch._h, 3))
    arch.set_timing(True)
    arch.restore()
    t = arch.timing()
    kernels = ("group_ms", "node_ms", "tmpl_ms", "diff_ms", "search_ms")
    assert all(t[k] > 0 for k in kernels)
    assert t["prepare_ms"] == pytest.approx(t["group_ms"] + t["node_ms"], abs=1e-3)
    assert t["diff_phase_ms"] == pytest.approx(t["tmpl_ms"] + t["diff_ms"] + t["search_ms"], abs=1e-3)
    arch.set_timing(True, phases_only=True)
    arch.restore()
    t = arch.timing()
    assert all(t[k] == -1.0 for k in kernels)
    assert t["prepare_ms"] > 0 and t["diff_phase_ms"] > 0
    assert t["total_ms"] == pytest.approx(t["prepare_ms"] + t["diff_phase_ms"], abs=1e-3)
    arch.set_timing(False)
    arch.restore()
    assert_restore_parity(arch, ref)


def test_per_graph_arrays_of_another_length_are_refused(cuda):
    """fdy_archive_set_groups and fdy_archive_set_manifest read one entry
    per graph: the binding refuses other lengths before the call, and the
    archive still restores as before."""
    p = synth.preset(1, num_graphs=6)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    with pytest.raises(ValueError):
        arch.set_groups(np.zeros(5, np.uint32))
    with pytest.raises(ValueError):
        arch.set_groups(np.zeros((6, 1), np.uint32))
    with pytest.raises(ValueError):
        arch.set_manifest("{}", [f"g{i}.json" for i in range(7)])
    arch.restore()
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


def test_switch_sequence_in_one_call(cuda):
    # The same seeded targets through fdy_switch_sequence, in chunks (so the
    # sequence continues from a live state left by an earlier call), against
    # the oracle after every chunk; a bad target anywhere refuses the whole
    # call and enqueues nothing.
    p = synth.preset(2, num_graphs=16, nodes_per_graph=250, num_groups=2, layout_var_pct=5)
    _print_case("switch-sequence", p)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    seq = synth.switch_sequence(0x5EED, s.num_graphs, 200)
    templates = sorted(set(ref.groups().tolist()))
    for k in range(0, 200, 50):
        chunk = seq[k:k + 50]
        arch.switch_sequence(chunk)
        for g in chunk.tolist():
            ref.switch(g)
        for t in templates:
            assert_live_matches(arch, ref, t)
    before = {t: arch.live(t) for t in templates}
    with pytest.raises(FoundryError):
        arch.switch_sequence([int(seq[0]), s.num_graphs])
    for t in templates:
        w, src, cur = arch.live(t)
        assert cur == before[t][2]
        np.testing.assert_array_equal(w, before[t][0])
    arch.switch_sequence([])  # nothing to do


def test_graph_longer_than_the_chunk_shift_table(cuda):
    # 66,000 nodes = 258 chunks of 256: the first two chunks of each graph are
    # shifted past the node-type and kernel-entry streams without the table.
    p = synth.preset(1, num_graphs=3, nodes_per_graph=66000)
    _print_case("long-graphs", p)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    assert_restore_parity(arch, ref)


def test_more_graphs_than_a_scan_block(cuda):
    # 1100 graphs: the override offsets are scanned 1024 graphs at a time, the
    # second batch continuing from the first one's total.
    p = synth.preset(1, num_graphs=1100, nodes_per_graph=6, num_groups=5)
    _print_case("many-graphs", p)
    s = synth.SynthArchive(p)
    arch, ref = gpu_and_oracle(s)
    assert_restore_parity(arch, ref)
    assert int(np.asarray(arch.override_offsets())[-1]) > 0


def _two_node_graph(values, overlap: bool) -> bytes:
    """Node 0: four 64-byte params; node 1: ten 64-byte params.  With
    `overlap`, node 1's ten entries all cover the same 64 bytes (the
    param-data section holds only those), so the param image (112 words)
    exceeds the capacity the sections allow (56 words) and the graph is
    flagged OVERFLOW; node 0's 32 words lie within the capacity."""
    import struct

    import cugraph_writer as W

    p0 = [b"".join(W.le(v) for v in values[8 * i:8 * i + 8]) for i in range(4)]
    p1 = [b"".join(W.le(v) for v in values[32 + 8 * i:40 + 8 * i]) for i in range(10)]
    if overlap:
        p1 = [p1[0]] + [b""] * 9
    img = bytearray(W.write([W.Kernel("k0", 0x1234, params=p0), W.Kernel("k1", 0x1234, params=p1)]))
    if overlap:
        pidx_off = struct.unpack_from("<Q", img, 64 + 24 * 3 + 8)[0]
        for j in range(10):
            struct.pack_into("<II", img, pidx_off + 8 * (4 + j), 256, 64)
    return bytes(img)


def test_members_of_an_overflowed_template(cuda):
    # The template's image overflows its capacity (OVERFLOW): it keeps no
    # image, its node past the capacity is not compared (its members keep no
    # records there, and switches to them are refused), and its node within
    # the capacity is compared against template words the member pass
    # relocates itself -- those records must equal the oracle's.
    print("[case] overflowed template with two members", flush=True)
    base, size = 0x7F0000000000, 1 << 32
    rng = np.random.default_rng(7)
    tvals = [int(base + 16 * rng.integers(0, size // 16)) if i % 3 == 0 else int(rng.integers(0, 1 << 62))
             for i in range(112)]
    images = [_two_node_graph(tvals, True)]
    for m in range(2):
        vals = list(tvals[:32]) + list(tvals[32:40]) * 10  # what the template's params read
        for i in range(0, 112, 5 + m):  # some words differ, some of them pointers
            vals[i] = int(base + 16 * rng.integers(0, size // 16)) if i % 2 else int(rng.integers(0, 1 << 62))
        images.append(_two_node_graph(vals, False))
    lo = np.array([base, base + (1 << 31)], dtype=np.uint64)
    hi = np.array([base + (1 << 31), base + size], dtype=np.uint64)
    nlo = np.array([0x7E0000000000, 0x7D0000000000], dtype=np.uint64)
    arch = Archive.from_images(images)
    arch.set_relocation(lo, hi, nlo)
    arch.restore()
    ref = oracle.Restore(images, (lo, hi, nlo))
    status = arch.status()
    assert status[0] & 0x20 and status[0] & 0x02, status  # OVERFLOW, reported as BAD_PARAMS
    assert not (status[1] & 0x22) and not (status[2] & 0x22), status
    assert arch.groups().tolist() == [0, 0, 0]
    assert arch.param_image(0).size == 0
    for g in (1, 2):
        np.testing.assert_array_equal(arch.param_image(g), ref.param_image(g), err_msg=f"param image g={g}")
        a, b = arch.overrides(g), ref.overrides(g)
        b0 = b[b["node"] == 0]
        assert len(b0) > 0 and len(b) > len(b0)
        np.testing.assert_array_equal(a, b0, err_msg=f"node-0 overrides g={g}")
        with pytest.raises(FoundryError):
            arch.switch(g)


def _reorder_param_index(img: bytes, order) -> bytes:
    """The archive with its param-index entries regrouped node by node in
    `order` (every kernel node's entries kept together and in their own
    order; each entry's param-index offset updated): the same params, laid
    out other than in node order, which the format allows."""
    import struct

    img = bytearray(img)
    sec = lambda i: struct.unpack_from("<QQ", img, 64 + 24 * i + 8)  # (offset, size)
    nodes_off, _ = sec(1)
    pidx_off, pidx_size = sec(3)
    n_nodes = struct.unpack_from("<I", img, 16)[0]
    old = bytes(img[pidx_off:pidx_off + pidx_size])
    at = 0
    for n in order:
        e = nodes_off + 168 * n
        if img[e + 4] != 0:
            continue
        pio, np_ = struct.unpack_from("<II", img, e + 128)
        img[pidx_off + at:pidx_off + at + 8 * np_] = old[pio:pio + 8 * np_]
        struct.pack_into("<I", img, e + 128, at)
        at += 8 * np_
    assert at == pidx_size and n_nodes > max(order)
    return bytes(img)


def test_param_entries_out_of_node_order(cuda):
    # Param-index entries laid out in reverse node order: a member chunk's
    # first nodes then hold the highest offsets, so the param entries it
    # compares start below the range its first loads suggest.  Members differ
    # from their template in param data, and two of them in the param entries
    # of one node (two params' offsets swapped) below and inside that range;
    # every output must equal the oracle's.
    import struct

    import cugraph_writer as W

    print("[case] param entries in reverse node order: 300 kernel nodes, template + 3 members", flush=True)
    N, base, size = 300, 0x7F0000000000, 1 << 32
    rng = np.random.default_rng(11)

    def words(k):
        return [int(base + 16 * rng.integers(0, size // 16)) if rng.random() < 0.4 else int(rng.integers(0, 1 << 62))
                for _ in range(k)]

    tvals = [words(4) for _ in range(N)]

    def graph(vals, swap_node=None):
        nodes = [W.Kernel(f"k{n % 7}", 0x1234 + n % 3, params=[W.le(v) for v in vals[n]]) for n in range(N)]
        img = _reorder_param_index(W.write(nodes), list(range(N - 1, -1, -1)))
        if swap_node is not None:  # the node's first two params read each other's bytes
            img = bytearray(img)
            nodes_off = struct.unpack_from("<Q", img, 64 + 24 * 1 + 8)[0]
            pidx_off = struct.unpack_from("<Q", img, 64 + 24 * 3 + 8)[0]
            pio = struct.unpack_from("<I", img, nodes_off + 168 * swap_node + 128)[0]
            a, b = struct.unpack_from("<8s8s", img, pidx_off + pio)
            struct.pack_into("<8s8s", img, pidx_off + pio, b, a)
            img = bytes(img)
        return img

    images = [graph(tvals)]
    for swap in (250, 100, None):
        vals = [list(v) for v in tvals]
        for n in range(0, N, 7):
            vals[n][n % 4] = words(1)[0]
        images.append(graph(vals, swap))
    lo = np.array([base], dtype=np.uint64)
    hi = np.array([base + size], dtype=np.uint64)
    nlo = np.array([0x7E0000000000], dtype=np.uint64)
    arch = Archive.from_images(images)
    arch.set_relocation(lo, hi, nlo)
    arch.restore()
    ref = oracle.Restore(images, (lo, hi, nlo))
    assert ref.groups().tolist() == [0, 0, 0, 0]
    # The swapped entries change what those nodes' first two params read.
    for g, n in ((1, 250), (2, 100)):
        assert (ref.overrides(g)["node"] == n).any(), (g, n)
    assert_restore_parity(arch, ref)


def test_graphs_without_nodes(cuda):
    # Two graphs without nodes (one the other's template) among two kernel
    # graphs, the last image of the archive empty: every output must equal
    # the oracle's, and nothing is read past an image.
    import cugraph_writer as W

    print("[case] two graphs without nodes among two 40-node graphs, the last image empty", flush=True)
    rng = np.random.default_rng(3)

    def kern(n):
        return W.Kernel(f"k{n % 3}", 0x99, params=[W.le(int(rng.integers(0, 1 << 62))) for _ in range(3)])

    images = [W.write([kern(n) for n in range(40)]), W.write([]), W.write([kern(n) for n in range(40)]), W.write([])]
    arch = Archive.from_images(images)
    arch.restore()
    ref = oracle.Restore(images, None)
    assert ref.groups().tolist() == [0, 1, 0, 1]
    assert_restore_parity(arch, ref)
