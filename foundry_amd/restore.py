"""Python view of the restore C ABI (include/foundry_restore.h).

Every method is a thin wrapper over one `fdy_*` entry point; results come
back as numpy arrays.  `stream` arguments accept a torch.cuda.Stream, a raw
hipStream_t integer, or None for the null stream.
"""
from __future__ import annotations

import ctypes as C
import sys
from typing import Sequence

import numpy as np

from . import _lib
from ._lib import ArchiveInfo, Override, RestoreTiming, check, restore_lib

OVERRIDE_DTYPE = np.dtype([("word", "<u4"), ("node", "<u4"), ("value", "<u8")])


def _stream(s) -> C.c_void_p:
    if s is None:
        return C.c_void_p(0)
    if isinstance(s, int):
        return C.c_void_p(s)
    return C.c_void_p(int(s.cuda_stream))


def _u64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint64))


def _table(lo, hi, new_lo):
    """An interval table as three contiguous u64 arrays of one length (the
    library reads n entries of each)."""
    lo, hi, new_lo = _u64(lo), _u64(hi), _u64(new_lo)
    if not (lo.ndim == hi.ndim == new_lo.ndim == 1 and len(lo) == len(hi) == len(new_lo)):
        raise ValueError("lo, hi and new_lo must be 1-D with one entry per interval")
    return lo, hi, new_lo


class Archive:
    """A set of `.cugraph` archives resident in HBM, and their restore state."""

    def __init__(self, handle: C.c_void_p, keepalive=None):
        self._h = handle
        self._keep = keepalive
        self._graphs = None

    def _graph_count(self) -> int:
        """The archive's graph count (fixed when it is opened): the length of
        the per-graph arrays the library reads without a length argument."""
        if self._graphs is None:
            self._graphs = int(self.info()["num_graphs"])
        return self._graphs

    # ---- opening ---------------------------------------------------------
    @classmethod
    def open(cls, paths: Sequence[str], num_threads: int = 4) -> "Archive":
        arr = (C.c_char_p * len(paths))(*[p.encode() for p in paths])
        h = C.c_void_p()
        check(restore_lib().fdy_archive_open(arr, len(paths), num_threads, C.byref(h)))
        return cls(h)

    @classmethod
    def from_images(cls, images: Sequence[bytes]) -> "Archive":
        bufs = [C.create_string_buffer(b, len(b)) if len(b) else C.create_string_buffer(1) for b in images]
        ptrs = (_lib.u8p * len(images))(*[C.cast(b, _lib.u8p) for b in bufs])
        sizes = (C.c_uint64 * len(images))(*[len(b) for b in images])
        h = C.c_void_p()
        check(restore_lib().fdy_archive_open_images(ptrs, sizes, len(images), C.byref(h)))
        return cls(h)

    @classmethod
    def from_synth(cls, synth) -> "Archive":
        n = synth.num_graphs
        addrs = [synth.image_ptr(i) for i in range(n)]
        ptrs = (_lib.u8p * n)(*[C.cast(C.c_void_p(a), _lib.u8p) for a, _ in addrs])
        sizes = (C.c_uint64 * n)(*[s for _, s in addrs])
        h = C.c_void_p()
        check(restore_lib().fdy_archive_open_images(ptrs, sizes, n, C.byref(h)))
        return cls(h)

    def close(self) -> None:
        if self._h:
            check(restore_lib().fdy_archive_close(self._h))
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- configuration ---------------------------------------------------
    def set_relocation(self, lo, hi, new_lo, policy: int = _lib.RELOC_HALF_OPEN) -> None:
        lo, hi, new_lo = _table(lo, hi, new_lo)
        self._reloc_keep = (lo, hi, new_lo)
        check(
            restore_lib().fdy_archive_set_relocation(
                self._h,
                lo.ctypes.data_as(_lib.u64p),
                hi.ctypes.data_as(_lib.u64p),
                new_lo.ctypes.data_as(_lib.u64p),
                len(lo),
                policy,
            )
        )

    def set_groups(self, template_of) -> None:
        if template_of is None:
            check(restore_lib().fdy_archive_set_groups(self._h, None))
            return
        t = np.ascontiguousarray(np.asarray(template_of, dtype=np.uint32))
        if t.ndim != 1 or len(t) != self._graph_count():
            raise ValueError(f"template_of needs one entry per graph ({self._graph_count()})")
        check(restore_lib().fdy_archive_set_groups(self._h, t.ctypes.data_as(_lib.u32p)))

    def set_manifest(self, text, names: Sequence[str]) -> bool:
        """Group by a graph_manifest.json text; False if the reference would
        ignore it (and group by keys)."""
        data = text.encode() if isinstance(text, str) else bytes(text)
        if len(names) != self._graph_count():
            raise ValueError(f"set_manifest needs one name per graph ({self._graph_count()})")
        arr = (C.c_char_p * len(names))(*[n.encode() for n in names])
        used = C.c_int()
        check(restore_lib().fdy_archive_set_manifest(self._h, data, len(data), arr, C.byref(used)))
        return bool(used.value)

    def set_timing(self, enabled: bool = True, phases_only: bool = False) -> None:
        """Time the following restores with HIP events after every kernel,
        or (phases_only) only around the grouping + node passes and the diff
        phase, which leaves the kernels within each phase back to back."""
        check(restore_lib().fdy_set_timing(self._h, (2 if phases_only else 1) if enabled else 0))

    def set_group_wait(self, spins: int) -> None:
        """Rounds of s_sleep the grouping step waits for a lower graph's
        unpublished key hash before hashing that key itself (0: at once)."""
        check(restore_lib().fdy_set_group_wait(self._h, int(spins)))

    # ---- the restore -----------------------------------------------------
    def restore(self, stream=None) -> None:
        check(restore_lib().fdy_restore(self._h, _stream(stream)))

    def timing(self) -> dict:
        t = RestoreTiming()
        check(restore_lib().fdy_restore_timing_get(self._h, C.byref(t)))
        return {k: getattr(t, k) for k, _ in RestoreTiming._fields_}

    def info(self) -> dict:
        i = ArchiveInfo()
        check(restore_lib().fdy_archive_info_get(self._h, C.byref(i)))
        return {k: getattr(i, k) for k, _ in ArchiveInfo._fields_}

    @property
    def num_graphs(self) -> int:
        return self.info()["num_graphs"]

    def digests(self, stream=None) -> np.ndarray:
        out = np.zeros((self.num_graphs, 4), dtype=np.uint64)
        check(restore_lib().fdy_get_digests(self._h, _stream(stream), out.ctypes.data_as(_lib.u64p)))
        return out

    def groups(self, stream=None) -> np.ndarray:
        out = np.zeros(self.num_graphs, dtype=np.uint32)
        check(restore_lib().fdy_get_groups(self._h, _stream(stream), out.ctypes.data_as(_lib.u32p)))
        return out

    def status(self, stream=None) -> np.ndarray:
        out = np.zeros(self.num_graphs, dtype=np.uint32)
        check(restore_lib().fdy_get_graph_status(self._h, _stream(stream), out.ctypes.data_as(_lib.u32p)))
        return out

    def override_offsets(self, stream=None) -> np.ndarray:
        out = np.zeros(self.num_graphs + 1, dtype=np.uint64)
        check(restore_lib().fdy_get_override_offsets(self._h, _stream(stream), out.ctypes.data_as(_lib.u64p)))
        return out

    def param_bytes(self, stream=None) -> np.ndarray:
        out = np.zeros(self.num_graphs, dtype=np.uint64)
        check(restore_lib().fdy_get_param_bytes(self._h, _stream(stream), out.ctypes.data_as(_lib.u64p)))
        return out

    def _sized(self, fn, g: int, dtype, stream, mult: int = 1):
        n = C.c_uint64()
        check(fn(self._h, _stream(stream), g, None, 0, C.byref(n)))
        out = np.zeros(n.value, dtype=dtype)
        ptr = out.ctypes.data_as(C.POINTER(np.ctypeslib.as_ctypes_type(dtype))) if n.value else None
        check(fn(self._h, _stream(stream), g, ptr, n.value, C.byref(n)))
        return out

    def overrides(self, g: int, stream=None) -> np.ndarray:
        n = C.c_uint64()
        lib = restore_lib()
        check(lib.fdy_get_overrides(self._h, _stream(stream), g, None, 0, C.byref(n)))
        out = np.zeros(n.value, dtype=OVERRIDE_DTYPE)
        if n.value:
            check(
                lib.fdy_get_overrides(
                    self._h, _stream(stream), g, out.ctypes.data_as(C.POINTER(Override)), n.value, C.byref(n)
                )
            )
        return out

    def node_flags(self, g: int, stream=None) -> np.ndarray:
        return self._sized(restore_lib().fdy_get_node_flags, g, np.uint8, stream)

    def node_words(self, g: int, stream=None) -> np.ndarray:
        return self._sized(restore_lib().fdy_get_node_words, g, np.uint32, stream)

    def param_image(self, g: int, stream=None) -> np.ndarray:
        return self._sized(restore_lib().fdy_get_param_image, g, np.uint64, stream)

    def node_pointers(self, g: int, stream=None) -> np.ndarray:
        return self._sized(restore_lib().fdy_get_node_pointers, g, np.uint64, stream)

    def section(self, g: int, section: int) -> bytes:
        """Raw bytes of one section of graph g's archive."""
        n = C.c_uint64()
        check(restore_lib().fdy_get_section(self._h, g, section, None, 0, C.byref(n)))
        buf = (C.c_uint8 * max(1, n.value))()
        if n.value:
            check(restore_lib().fdy_get_section(self._h, g, section, buf, n.value, C.byref(n)))
        return bytes(buf)[: n.value]

    # ---- switching -------------------------------------------------------
    def switch(self, g: int, stream=None) -> None:
        check(restore_lib().fdy_switch(self._h, g, _stream(stream)))

    def switch_sequence(self, targets, stream=None) -> None:
        """fdy_switch for each target in order, checked and enqueued in one call."""
        t = np.ascontiguousarray(np.asarray(targets, dtype=np.uint32))
        check(restore_lib().fdy_switch_sequence(self._h, t.ctypes.data_as(_lib.u32p), t.size, _stream(stream)))

    def live(self, template: int, stream=None) -> tuple[np.ndarray, np.ndarray, int]:
        words = self.param_image(template, stream).size
        nodes = self.node_flags(template, stream).size
        w = np.zeros(words, dtype=np.uint64)
        src = np.zeros(nodes, dtype=np.uint32)
        cur = C.c_uint32()
        check(
            restore_lib().fdy_get_live(
                self._h,
                _stream(stream),
                template,
                w.ctypes.data_as(_lib.u64p) if words else None,
                words,
                src.ctypes.data_as(_lib.u32p) if nodes else None,
                nodes,
                C.byref(cur),
            )
        )
        return w, src, cur.value


class RelocPlan:
    """Interval search structure for fdy_relocate_words."""

    def __init__(self, lo, hi, new_lo, policy: int = _lib.RELOC_HALF_OPEN):
        self._h = C.c_void_p()
        lo, hi, new_lo = _table(lo, hi, new_lo)
        h = C.c_void_p()
        check(
            restore_lib().fdy_reloc_plan_create(
                lo.ctypes.data_as(_lib.u64p),
                hi.ctypes.data_as(_lib.u64p),
                new_lo.ctypes.data_as(_lib.u64p),
                len(lo),
                policy,
                C.byref(h),
            )
        )
        self._h = h

    def relocate(self, d_in: int, d_out: int, n_words: int, stream=None) -> None:
        """Relocate n_words u64 words at device address d_in into d_out."""
        check(restore_lib().fdy_relocate_words(self._h, C.c_void_p(d_in), C.c_void_p(d_out), n_words, _stream(stream)))

    def lines(self) -> np.ndarray:
        """The plan's interval index: one row of eight u64 words per 64-byte line."""
        n = C.c_uint64()
        check(restore_lib().fdy_reloc_plan_lines(self._h, None, 0, C.byref(n)))
        out = np.zeros((n.value, 8), dtype=np.uint64)
        check(restore_lib().fdy_reloc_plan_lines(self._h, out.ctypes.data_as(C.c_void_p), n.value, C.byref(n)))
        return out

    def close(self) -> None:
        if self._h:
            check(restore_lib().fdy_reloc_plan_destroy(self._h))
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def relocate_words_static(lo, hi, new_lo, d_in: int, d_out: int, n_words: int, policy: int = _lib.RELOC_HALF_OPEN,
                          stream=None) -> None:
    """fdy_relocate_words_static: relocate device words by the table (lo, hi,
    new_lo) with no device allocation (the index lives in the library's
    static per-GPU array)."""
    lo, hi, new_lo = _table(lo, hi, new_lo)
    check(restore_lib().fdy_relocate_words_static(lo.ctypes.data_as(_lib.u64p), hi.ctypes.data_as(_lib.u64p),
                                                  new_lo.ctypes.data_as(_lib.u64p), len(lo), policy, d_in, d_out,
                                                  n_words, _stream(stream)))


def version() -> str:
    return restore_lib().fdy_version().decode()


def cugraph_from_json(text) -> bytes:
    """The .cugraph archive CUDAGraph::save_binary writes for one graph's JSON
    document (csrc/BinaryGraphIO.cpp:15-371); no device needed."""
    data = text.encode() if isinstance(text, str) else bytes(text)
    n = C.c_uint64()
    rc = restore_lib().fdy_cugraph_from_json(data, len(data), None, 0, C.byref(n))
    if rc != -8:  # FDY_E_CAPACITY: the size is known
        check(rc)
    buf = (C.c_uint8 * max(1, n.value))()
    check(restore_lib().fdy_cugraph_from_json(data, len(data), buf, n.value, C.byref(n)))
    return bytes(buf)[: n.value]


def load_topology_key(text) -> bytes:
    """The key the LOAD path groups a graph read from its JSON document by
    (csrc/CUDAGraphParallel.cpp:1791-1841); no device needed."""
    data = text.encode() if isinstance(text, str) else bytes(text)
    n = C.c_uint64()
    rc = restore_lib().fdy_load_topology_key(data, len(data), None, 0, C.byref(n))
    if rc != -8:  # FDY_E_CAPACITY: the size is known
        check(rc)
    buf = C.create_string_buffer(max(1, n.value))
    check(restore_lib().fdy_load_topology_key(data, len(data), buf, n.value, C.byref(n)))
    return buf.raw[: n.value]


def cugraph_path(json_path: str) -> str:
    """The archive path CUDAGraph::save writes beside a graph's JSON
    (csrc/CUDAGraph.cpp:1494-1500): ".json" replaced, else ".cugraph" appended."""
    return json_path[:-5] + ".cugraph" if json_path.endswith(".json") else json_path + ".cugraph"


def save_binary(bin_path: str, text) -> None:
    """CUDAGraph::save_binary (csrc/BinaryGraphIO.cpp:15-371): write the archive
    of one graph's JSON document to bin_path.  As there, a file that cannot
    be written prints a warning and returns; a document that cannot be
    serialised raises."""
    data = text.encode() if isinstance(text, str) else bytes(text)
    rc = restore_lib().fdy_cugraph_save_binary(bin_path.encode(), data, len(data))
    if rc == -2:  # FDY_E_IO
        print(f"[foundry] WARNING: Failed to write binary graph: {bin_path}", file=sys.stderr)
        return
    check(rc)


def manifest_groups(text, names: Sequence[str]):
    """template_of from a graph_manifest.json text (no device), or None when
    the reference would ignore the manifest."""
    data = text.encode() if isinstance(text, str) else bytes(text)
    arr = (C.c_char_p * max(1, len(names)))(*[n.encode() for n in names])
    out = np.zeros(max(1, len(names)), dtype=np.uint32)
    used = C.c_int()
    check(restore_lib().fdy_manifest_groups(data, len(data), arr, len(names), out.ctypes.data_as(_lib.u32p),
                                            C.byref(used)))
    return out[: len(names)] if used.value else None
