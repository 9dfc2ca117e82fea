"""Group graphs on the GPU: build one hipGraph per topology group from the
restored template, switch it between member graphs, and check what the
graphs compute against the values the graphs' params determine.

Before the first launch, the restored param images and node pointers are
compared with the values graph_cases restates, so every pointer a kernel,
fill or copy node dereferences is known to lie inside the test's buffer."""
import ctypes
import random
import struct

import numpy as np
import pytest
import torch

import graph_cases as GC
import refcrc
from foundry_amd import _lib
from foundry_amd.graph import GroupGraph, Registry, code_object_hash, code_object_kernels
from foundry_amd.restore import Archive

pytestmark = pytest.mark.gpu

_hip = None


def _hip_memcpy(dst: int, src: int, n: int, kind: int) -> None:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert _hip.hipMemcpy(dst, src, n, kind) == 0


class Env:
    def __init__(self, packed_dir: str | None = None):
        torch.cuda.set_device(0)
        self.stream = torch.cuda.current_stream()
        self.reg = Registry()
        data = open(GC.PROBE_CO, "rb").read()
        if packed_dir is None:
            self.bhash = self.reg.add_file(GC.PROBE_CO)
        else:  # the code object comes back from a packed pair
            assert self.reg.load_packed(packed_dir) == 1
            self.bhash = code_object_hash(data)
        assert self.bhash == refcrc.crc64_xz(data) == code_object_hash(data)
        self.slots, nbytes = self.reg.global_address(self.bhash, "probe_slots")
        assert nbytes == 256 * 8
        self.buf = torch.zeros(GC.BUF_BYTES // 8, dtype=torch.int64, device="cuda")
        self.base = self.buf.data_ptr()
        self.arch = Archive.from_images(GC.images(self.bhash))
        self.arch.set_relocation([GC.SAVED], [GC.SAVED + GC.BUF_BYTES], [self.base])
        self.arch.restore(self.stream)
        self.check_restored()

    def check_restored(self):
        assert list(self.arch.groups(self.stream)) == [0, 0, 0, 0, 0, 5]
        for g, s in enumerate(GC.SPECS):
            img = [int(x) for x in self.arch.param_image(g, self.stream)]
            assert img == GC.expected_image(s, self.bhash, self.base), f"graph {g}: restored params"
            ptrs = [int(x) for x in self.arch.node_pointers(g, self.stream)]
            assert ptrs == GC.expected_pointers(s, self.base), f"graph {g}: restored node pointers"

    def poison_slot2(self):
        v = np.array([0xDEADDEADDEADDEAD], dtype=np.uint64)
        _hip_memcpy(self.slots + 16, v.ctypes.data, 8, 1)

    def read_slot2(self) -> int:
        v = np.zeros(1, dtype=np.uint64)
        _hip_memcpy(v.ctypes.data, self.slots + 16, 8, 2)
        return int(v[0])

    def run(self, gg: GroupGraph, g: int) -> dict:
        """Zero the buffer, replay graph g, and check every result."""
        torch.cuda.synchronize()
        self.buf.zero_()
        self.poison_slot2()
        torch.cuda.synchronize()
        st = gg.replay(g, self.stream)
        torch.cuda.synchronize()
        self.check(g)
        return st

    def check(self, g: int):
        s = GC.SPECS[g]
        raw = self.buf.cpu().numpy().view(np.uint64)
        slots, fill, copy = GC.expected_buffer(s)
        for i in range(GC.CAP):
            assert int(raw[i]) == slots.get(i, 0), f"graph {g}: result slot {i}"
        b = raw.tobytes()
        assert b[GC.FILL_OFF:GC.FILL_OFF + len(fill)] == fill, f"graph {g}: fill node"
        assert b[GC.FILL_OFF + len(fill):GC.COPY_OFF] == bytes(GC.COPY_OFF - GC.FILL_OFF - len(fill))
        assert b[GC.COPY_OFF:GC.COPY_OFF + len(copy)] == copy, f"graph {g}: copy node"
        assert b[GC.COPY_OFF + len(copy):] == bytes(GC.BUF_BYTES - GC.COPY_OFF - len(copy))
        assert self.read_slot2() == GC.expected_slot2(s), f"graph {g}: extra-style node"

    def expected_resets(self, prev: int, new: int) -> int:
        def nodes(g):
            o = {int(x) for x in self.arch.overrides(g, self.stream)["node"]}
            fl = self.arch.node_flags(g, self.stream)
            return o | {n for n in range(len(fl)) if fl[n] & (_lib.NODE_LAYOUT | _lib.NODE_DESC)}
        return len(nodes(prev) | nodes(new))


@pytest.fixture(scope="module")
def env():
    e = Env()
    yield e


def test_registry_lookup_and_errors(env):
    assert env.reg.lookup(env.bhash, "probe_mix") != 0
    with pytest.raises(_lib.FoundryError, match="FDY_E_NOT_FOUND"):
        env.reg.lookup(env.bhash, "no_such_kernel")
    with pytest.raises(_lib.FoundryError, match="FDY_E_NOT_FOUND"):
        env.reg.lookup(env.bhash ^ 1, "probe_mix")
    # Adding the same bytes again keeps one module.
    assert env.reg.add(open(GC.PROBE_CO, "rb").read()) == env.bhash


def _pack_probe(dirpath) -> tuple[int, bytes]:
    src = Registry()
    h = src.add_file(GC.PROBE_CO)
    assert src.pack(str(dirpath)) == 1
    src.close()
    return h, open(GC.PROBE_CO, "rb").read()


def test_packed_code_objects_reload_and_launch(tmp_path):
    """pack_fatbins_to_folder's pair (csrc/hook.cpp:1589-1700): the image
    holds {binary_hash, size, bytes}, the index the hash, the loader line and
    the kernel names; a fresh registry loaded from the pair (3787-3830)
    resolves the graphs' kernels, which then run."""
    h, data = _pack_probe(tmp_path)
    assert (tmp_path / "fatbin_image_packed.img").read_bytes() == struct.pack("<QQ", h, len(data)) + data
    names = code_object_kernels(data)
    assert (tmp_path / "fatbin_entrypoint_packed.txt").read_text().splitlines() == \
        [f"{h:016x}", "hipModuleLoadData,binary_flags=0", str(len(names)), *names, "---"]
    e = Env(packed_dir=str(tmp_path))
    for n in names:
        assert e.reg.lookup(e.bhash, n) != 0
    with GroupGraph(e.arch, 0, e.reg, e.stream) as gg:
        for g in [0, 3, 1]:
            e.run(gg, g)


def test_packed_pair_damage_is_refused(tmp_path):
    h, data = _pack_probe(tmp_path)
    img = tmp_path / "fatbin_image_packed.img"
    txt = tmp_path / "fatbin_entrypoint_packed.txt"
    good_img, good_txt = img.read_bytes(), txt.read_text()
    cases = [
        (good_img[:-1], good_txt, "truncated"),
        (good_img[:100] + bytes([good_img[100] ^ 1]) + good_img[101:], good_txt, "hash to its binary_hash"),
        (good_img, good_txt.replace(f"{h:016x}", f"{h ^ 1:016x}"), "another binary_hash"),
        (good_img, good_txt.replace("probe_mix\n", "probe_nothing\n"), "lacks"),
        (good_img, good_txt.replace("---\n", ""), "without ---"),
        (good_img + good_img, good_txt, "fewer records"),
    ]
    for b, t, msg in cases:
        img.write_bytes(b)
        txt.write_text(t)
        reg = Registry()
        with pytest.raises(_lib.FoundryError, match=msg):
            reg.load_packed(str(tmp_path))
        reg.close()
    img.unlink()
    reg = Registry()
    with pytest.raises(_lib.FoundryError, match="FDY_E_IO"):
        reg.load_packed(str(tmp_path))
    reg.close()


def test_build_shape(env):
    with GroupGraph(env.arch, 0, env.reg, env.stream) as gg:
        info = gg.info()
        assert info["num_nodes"] == 11
        assert info["num_kernel_nodes"] == 6
        assert info["num_fill_nodes"] == 1
        assert info["num_memcpy_nodes"] == 1
        assert info["num_event_nodes"] == 2
        assert info["num_deps"] == len(GC.EDGES)
        assert info["num_events"] == 1
        assert info["current_graph"] == 0


def test_each_member_runs_its_own_params(env):
    with GroupGraph(env.arch, 0, env.reg, env.stream) as gg:
        for g in GC.GROUP_A:
            env.run(gg, g)
        env.run(gg, 0)


def test_only_changed_nodes_are_reset(env):
    """With one exec (the reference's shape), every switch updates it: only
    the nodes that differ between the two graphs are re-set."""
    with GroupGraph(env.arch, 0, env.reg, env.stream) as gg:
        gg.set_exec_cache(1)
        prev = 0
        for g in [1, 2, 3, 4, 1, 0, 4, 3, 2]:
            st = env.run(gg, g)
            assert st["nodes_reset"] == env.expected_resets(prev, g), (prev, g)
            prev = g
        assert gg.select(prev, env.stream)["nodes_reset"] == 0  # already current


@pytest.mark.parametrize("execs", [1, 2, 4])
def test_exec_cache(env, execs):
    """Up to `execs` execs hold recently selected graphs.  A graph one of
    them holds becomes current with nothing re-set.  Otherwise the least
    recently selected exec (or a new one, which starts from the template's
    params) takes the graph: the re-set nodes are those whose params differ
    among the live image's graph (the previous selection), the exec's graph
    and the new one.  Every launch runs the selected graph's params,
    whatever exec holds them."""
    def own(g):
        o = {int(x) for x in env.arch.overrides(g, env.stream)["node"]}
        fl = env.arch.node_flags(g, env.stream)
        return o | {n for n in range(len(fl)) if fl[n] & (_lib.NODE_LAYOUT | _lib.NODE_DESC)}

    order = [1, 2, 1, 3, 2, 4, 0, 1, 4, 4, 3, 0, 2, 1]
    with GroupGraph(env.arch, 0, env.reg, env.stream) as gg:
        gg.set_exec_cache(execs)
        slots = [[0, 0]]  # per exec: [graph, tick of its last selection]
        prev = 0
        for tick, g in enumerate(order, start=1):
            st = env.run(gg, g)
            hit = [x for x in slots if x[0] == g]
            if hit:
                assert st["cache_hit"] == 1 and st["nodes_reset"] == 0, (tick, g, slots)
                hit[0][1] = tick
            else:
                if len(slots) < execs:
                    slots.append([0, 0])
                    x = slots[-1]
                else:
                    x = min(slots, key=lambda y: y[1])
                h = x[0]
                want = own(h) | own(g) | (own(prev) if prev != h else set())
                assert st["cache_hit"] == 0 and st["nodes_reset"] == len(want), (tick, g, h, prev)
                x[:] = [g, tick]
            assert gg.info()["num_execs"] == len(slots)
            prev = g
        gg.set_exec_cache(1)  # the current exec stays
        assert gg.info()["num_execs"] == 1 and gg.info()["current_graph"] == prev
        env.run(gg, prev)
        env.run(gg, 3)


def test_seeded_switch_sequence(env):
    rng = random.Random(0x5EED)
    with GroupGraph(env.arch, 0, env.reg, env.stream) as gg:
        for _ in range(24):
            env.run(gg, rng.choice(GC.GROUP_A))


def test_switch_sequence_with_a_bound_group_keeps_its_order(env):
    # A switch sequence that touches a group held by a group graph keeps the
    # sequence's order (no layering) and selects each target through the
    # group graph: afterwards the exec runs the last target's params.
    rng = random.Random(0x5EED + 7)
    seq = [rng.choice(GC.GROUP_A) for _ in range(12)]
    with GroupGraph(env.arch, 0, env.reg, env.stream) as gg:
        env.arch.switch_sequence(seq, env.stream)
        torch.cuda.synchronize()
        assert gg.info()["current_graph"] == seq[-1]
        torch.cuda.synchronize()
        env.buf.zero_()
        env.poison_slot2()
        torch.cuda.synchronize()
        gg.launch(env.stream)
        torch.cuda.synchronize()
        env.check(seq[-1])


def test_archive_switch_goes_through_the_group_graph(env):
    with GroupGraph(env.arch, 0, env.reg, env.stream) as gg:
        for g in (3, 1, 0):
            env.arch.switch(g, env.stream)
            torch.cuda.synchronize()
            env.buf.zero_()
            env.poison_slot2()
            torch.cuda.synchronize()
            gg.launch(env.stream)
            torch.cuda.synchronize()
            env.check(g)
            assert gg.info()["current_graph"] == g


def test_second_group_and_misuse(env):
    with GroupGraph(env.arch, 0, env.reg, env.stream) as gg:
        with pytest.raises(_lib.FoundryError, match="FDY_E_INVALID"):
            gg.select(5, env.stream)  # graph of another group
        with pytest.raises(_lib.FoundryError, match="FDY_E_STATE"):
            GroupGraph(env.arch, 0, env.reg, env.stream)  # one group graph per template
        with pytest.raises(_lib.FoundryError, match="FDY_E_STATE"):
            env.arch.restore(env.stream)  # restored params are in use
        with GroupGraph(env.arch, 5, env.reg, env.stream) as gb:
            assert gb.info()["num_nodes"] == 12
    with pytest.raises(_lib.FoundryError, match="FDY_E_INVALID"):
        GroupGraph(env.arch, 1, env.reg, env.stream)  # not a template


def test_unresolvable_templates_are_refused_before_launch(env):
    import cugraph_writer as W
    from cugraph_writer import le

    out = le(GC.SAVED)
    cases = [
        ([W.Kernel("no_such_kernel", env.bhash, params=[out])], "FDY_E_NOT_FOUND"),
        ([W.Kernel("probe_mix", env.bhash ^ 0xFF, params=[out])], "FDY_E_NOT_FOUND"),
        ([W.Kernel("probe_mix", env.bhash, cluster=(2, 1, 1),
                   params=[out, le(0, 4), le(1, 4), le(0), le(0)])], "FDY_E_UNSUPPORTED"),
        ([W.Memcpy(dst=GC.SAVED, src=0x1000, width_bytes=8, src_type=1)], "FDY_E_UNSUPPORTED"),
        ([W.Memset(dst=GC.SAVED, value=0, width=4, element_size=3)], "FDY_E_FORMAT"),
    ]
    for nodes, code in cases:
        arch = Archive.from_images([W.write(nodes)])
        arch.set_relocation([GC.SAVED], [GC.SAVED + GC.BUF_BYTES], [env.base])
        arch.restore(env.stream)
        with pytest.raises(_lib.FoundryError, match=code):
            GroupGraph(arch, 0, env.reg, env.stream)
        arch.close()


@pytest.mark.parametrize("diff_node_pct", [0, 10])
def test_synthetic_groups_build_and_switch_without_launch(env, diff_node_pct):
    """Group graphs of a synthetic decode-style archive whose kernels all
    resolve to the probe's sink kernel (built and switched, never launched:
    the saved pointers are synthetic).  Every switch re-sets exactly the
    nodes the override sets and flags name; with the differences confined to
    10% of the kernel nodes, a switch re-sets only those."""
    from foundry_amd import synth

    p = synth.preset(2, num_graphs=24, num_groups=3, nodes_per_graph=300, num_intervals=2000)
    p.sink_hash = env.bhash
    p.diff_node_pct = diff_node_pct
    s = synth.SynthArchive(p)
    arch = Archive.from_synth(s)
    arch.set_relocation(*s.intervals())
    arch.restore(env.stream)
    groups = arch.groups(env.stream)
    temps = sorted(set(int(t) for t in groups))
    assert len(temps) == 3
    ggs = {t: GroupGraph(arch, t, env.reg, env.stream) for t in temps}
    for gg in ggs.values():
        gg.set_exec_cache(1)  # one exec per group: every switch updates it

    def touched(g):
        o = {int(x) for x in arch.overrides(g, env.stream)["node"]}
        fl = arch.node_flags(g, env.stream)
        return o | {n for n in range(len(fl)) if fl[n] & (_lib.NODE_LAYOUT | _lib.NODE_DESC)}

    current = {t: t for t in temps}
    rng = random.Random(7)
    for _ in range(30):
        g = rng.randrange(s.num_graphs)
        t = int(groups[g])
        st = ggs[t].select(g, env.stream)
        want = 0 if current[t] == g else len(touched(current[t]) | touched(g))
        assert st["nodes_reset"] == want, (current[t], g)
        if diff_node_pct:
            assert want <= 75, want  # about 30 of 300 nodes may differ
        current[t] = g
    full = ggs[temps[0]].reset_all(env.stream)
    assert full["nodes_reset"] == 300
    _, _, cur = arch.live(temps[0], env.stream)
    assert cur == current[temps[0]]
    for gg in ggs.values():
        gg.close()
    arch.close()
