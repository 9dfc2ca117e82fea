"""The allocation region on the GPU: real VMM reservations and mappings
(hipMemAddressReserve / hipMemCreate / hipMemMap / hipMemSetAccess), the
replay of one region's allocator events into a second region placed
elsewhere, and graphs saved against the first region run in the second after
relocation by the replay's interval table.

Every pointer a launched kernel dereferences is checked on the host first:
the relocated param images must name the second region's allocation."""
import ctypes

import numpy as np
import pytest
import torch

import cugraph_writer as W
import graph_cases as GC
from cugraph_writer import le
from foundry_amd import _lib
from foundry_amd.graph import GroupGraph, Registry
from foundry_amd.region import MiB, Region
from foundry_amd.restore import Archive, RelocPlan

pytestmark = pytest.mark.gpu

BASE = 0x200000000000  # a base the MI355X can map (FDY_REGION_DEFAULT_BASE)
REF_BASE = 0x500000000000  # the reference's default base: granted by hipMemAddressReserve, not mappable
SIZE = 1 << 30

_hip = None


def _memcpy(dst: int, src: int, n: int, kind: int) -> None:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert _hip.hipMemcpy(dst, src, n, kind) == 0


def _write(dev: int, arr: np.ndarray) -> None:
    _memcpy(dev, arr.ctypes.data, arr.nbytes, 1)


def _read(dev: int, n_words: int) -> np.ndarray:
    out = np.zeros(n_words, dtype=np.uint64)
    _memcpy(out.ctypes.data, dev, out.nbytes, 2)
    return out


@pytest.fixture(scope="module")
def dev():
    torch.cuda.set_device(0)
    torch.cuda.synchronize()
    return torch.cuda.current_stream()


def test_mapped_memory_is_usable_by_copies_and_kernels(dev):
    with Region(BASE, SIZE) as r:
        info = r.info()
        assert info["size"] == SIZE and info["base"] % (2 * MiB) == 0
        a = r.alloc(3 * MiB + 123)
        b = r.alloc(5 * MiB)
        assert b - a == 4 * MiB
        n = (3 * MiB) // 8
        src = np.arange(n, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)
        _write(a, src)
        np.testing.assert_array_equal(_read(a, n), src)
        # A kernel of this library reads one mapping and writes the other
        # (relocation with no intervals passes words through).
        plan = RelocPlan([], [], [])
        plan.relocate(a, b, n, dev)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_read(b, n), src)
        plan.close()
        r.free(a)
        assert r.info()["live_allocations"] == 1


def test_unmappable_base_moves_or_fails(dev):
    with Region(REF_BASE, SIZE) as r:
        assert r.base != REF_BASE and r.info()["saved_base"] == REF_BASE
        p = r.alloc(MiB)
        v = np.arange(16, dtype=np.uint64)
        _write(p, v)
        np.testing.assert_array_equal(_read(p, 16), v)
        lo, hi, nlo = r.intervals()
        assert (int(lo[0]), int(hi[0]), int(nlo[0])) == (REF_BASE, REF_BASE + SIZE, r.base)
    with pytest.raises(_lib.FoundryError, match="FDY_E_STATE"):
        Region(REF_BASE, SIZE, exact=True)


def test_preallocation_serves_allocations_without_new_mappings(dev):
    with Region(BASE, SIZE) as r:
        r.preallocate(64 * MiB)
        p = r.alloc(10 * MiB)
        q = r.alloc(20 * MiB)
        assert r.info()["mapped_bytes"] == 64 * MiB
        v = np.full(1024, 0xABCDEF, dtype=np.uint64)
        _write(q + 20 * MiB - 8192, v)
        np.testing.assert_array_equal(_read(q + 20 * MiB - 8192, 1024), v)
        with pytest.raises(_lib.FoundryError, match="FDY_E_NOMEM"):
            r.alloc(44 * MiB)  # would start inside at 30 MiB and run past the end
        t = r.alloc(34 * MiB)  # fills the rest exactly
        u = r.alloc(MiB)       # past the preallocation: its own mapping
        assert t - r.base == 30 * MiB and u - r.base == 64 * MiB
        assert r.info()["mapped_bytes"] == 64 * MiB + MiB
        w = np.arange(4096, dtype=np.uint64)
        _write(t + 34 * MiB - 32768, w)
        _write(u, w)
        np.testing.assert_array_equal(_read(t + 34 * MiB - 32768, 4096), w)
        np.testing.assert_array_equal(_read(u, 4096), w)
        r.free(p)
        r.free(q)
        r.free(t)
        r.free(u)
        r.free_preallocated()
        assert r.info()["mapped_bytes"] == 0


def test_second_region_replays_the_first_elsewhere(dev):
    with Region(BASE, SIZE) as r1:
        r1.alloc(9 * MiB)
        r1.record(True)
        x = r1.alloc(4096)
        y = r1.reserve(8 * MiB, 4 * MiB)
        z = r1.alloc(12 * MiB)
        text = r1.events_json()
        with pytest.raises(_lib.FoundryError, match="FDY_E_STATE"):
            Region(r1.base, SIZE, exact=True)  # the reference's rule: the saved base must be free
        with Region(r1.base, SIZE, align=64 * MiB) as r2:
            assert r2.base != r1.base and r2.info()["saved_base"] == r1.base
            r2.alloc(9 * MiB)
            r2.replay(text)
            lo, hi, nlo = r2.intervals(per_allocation=True)
            rows = [tuple(int(v) for v in t) for t in zip(lo, hi, nlo)]
            shift = r2.base - r1.base
            assert rows[1:] == [(x, x + 4096, x + shift), (y, y + 8 * MiB, y + shift), (z, z + 12 * MiB, z + shift)]
            # the replayed allocation is real memory
            v = np.arange(512, dtype=np.uint64)
            _write(z + shift, v)
            np.testing.assert_array_equal(_read(z + shift, 512), v)


def test_graph_saved_in_one_region_runs_in_another(dev):
    reg = Registry()
    bhash = reg.add_file(GC.PROBE_CO)
    with Region(BASE, SIZE) as r1:
        r1.record(True)
        out1 = r1.alloc(GC.BUF_BYTES)
        text = r1.events_json()
        with Region(r1.base, SIZE) as r2:
            r2.replay(text)
            out2 = out1 - r1.base + r2.base
            assert r2.base != r1.base
            # A graph saved against region 1: results go to out1.
            nodes = [
                W.Kernel("probe_mix", bhash, grid=(2, 1, 1), block=(64, 1, 1),
                         params=[le(out1), le(0, 4), le(GC.CAP, 4), le(5), le(6)]),
                W.Memset(dst=out1 + GC.FILL_OFF, value=0x11223344, width=32, element_size=4),
                W.Memcpy(dst=out1 + GC.COPY_OFF, src=out1 + GC.FILL_OFF, width_bytes=128),
                W.Kernel("probe_chain", bhash, params=[le(out1), le(1, 4), le(GC.CAP, 4), le(0, 4)]),
            ]
            arch = Archive.from_images([W.write(nodes, [(1, 2), (0, 3)])])
            arch.set_relocation(*r2.intervals(per_allocation=True))
            arch.restore(dev)
            img = [int(v) for v in arch.param_image(0, dev)]
            ptrs = [int(v) for v in arch.node_pointers(0, dev)]
            assert img[0] == out2 and img[5] == out2, "kernel pointers must name region 2"
            assert ptrs[2] == out2 + GC.FILL_OFF and ptrs[4] == out2 + GC.COPY_OFF and ptrs[5] == out2 + GC.FILL_OFF
            _write(out2, np.zeros(GC.BUF_BYTES // 8, dtype=np.uint64))
            _write(out1, np.zeros(GC.BUF_BYTES // 8, dtype=np.uint64))
            with GroupGraph(arch, 0, reg, dev) as gg:
                gg.launch(dev)
                torch.cuda.synchronize()
            got = _read(out2, GC.BUF_BYTES // 8)
            r0 = GC.mix_expect(5, 6, 2, 64)
            assert int(got[0]) == r0 and int(got[1]) == GC.mix(r0, 1)
            b = got.tobytes()
            assert b[GC.FILL_OFF:GC.FILL_OFF + 128] == le(0x11223344, 4) * 32
            assert b[GC.COPY_OFF:GC.COPY_OFF + 128] == le(0x11223344, 4) * 32
            assert not _read(out1, GC.BUF_BYTES // 8).any(), "region 1 must be untouched"
            arch.close()
    reg.close()
