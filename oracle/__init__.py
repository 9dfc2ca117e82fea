"""Python handle on the oracle (oracle.cpp): the CPU restatement of the
reference's graph-restore path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
the cpu_baseline leg of bench.py, as the checker -- never by the product.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(_HERE, "_build", "liboracle.so")

u8p = C.POINTER(C.c_uint8)
u32p = C.POINTER(C.c_uint32)
u64p = C.POINTER(C.c_uint64)
OVERRIDE_DTYPE = np.dtype([("word", "<u4"), ("node", "<u4"), ("value", "<u8")])

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        vp = C.c_void_p
        sigs = {
            "orc_last_error": (C.c_char_p, []),
            "orc_crc64": (C.c_uint64, [C.c_char_p, C.c_uint64]),
            "orc_topology_key_saved": (C.c_int64, [C.c_char_p, C.c_uint64, C.c_char_p, C.c_uint64]),
            "orc_topology_key_recomputed": (C.c_int64, [C.c_char_p, C.c_uint64, C.c_char_p, C.c_uint64]),
            "orc_group_by_keys": (C.c_int, [C.POINTER(C.c_char_p), u64p, C.c_uint32, u32p]),
            "orc_group_manifest": (C.c_int, [C.c_char_p, C.c_uint64, C.POINTER(C.c_char_p), C.c_uint32, u32p]),
            "orc_extract_node_params": (C.c_int64, [C.c_char_p, C.c_uint64, C.c_uint32, u8p, C.c_uint64]),
            "orc_effective_attrs": (C.c_int, [C.c_char_p, C.c_uint64, C.c_uint32, C.POINTER(C.c_int32)]),
            "orc_set_mutation": (None, [C.c_int]),
            "orc_restore": (
                C.c_int,
                [C.POINTER(u8p), u64p, C.c_uint32, u64p, u64p, u64p, C.c_uint64, C.c_uint32, u32p, C.c_uint32,
                 C.POINTER(vp)],
            ),
            "orc_free": (None, [vp]),
            "orc_digests": (C.c_int, [vp, u64p]),
            "orc_groups": (C.c_int, [vp, u32p]),
            "orc_status": (C.c_int, [vp, u32p]),
            "orc_override_offsets": (C.c_int, [vp, u64p]),
            "orc_overrides": (C.c_int64, [vp, C.c_uint32, vp, C.c_uint64]),
            "orc_node_flags": (C.c_int64, [vp, C.c_uint32, u8p, C.c_uint64]),
            "orc_node_words": (C.c_int64, [vp, C.c_uint32, u32p, C.c_uint64]),
            "orc_param_image": (C.c_int64, [vp, C.c_uint32, u64p, C.c_uint64]),
            "orc_node_pointers": (C.c_int64, [vp, C.c_uint32, u64p, C.c_uint64]),
            "orc_total_param_bytes": (C.c_uint64, [vp]),
            "orc_switch": (C.c_int, [vp, C.c_uint32]),
            "orc_live": (C.c_int64, [vp, C.c_uint32, u64p, C.c_uint64, u32p, C.c_uint64, u32p]),
            "orc_relocate_word": (C.c_uint64, [C.c_uint64, u64p, u64p, u64p, C.c_uint64, C.c_uint32]),
            "orc_relocate_words": (C.c_int, [u64p, u64p, C.c_uint64, u64p, u64p, u64p, C.c_uint64, C.c_uint32, C.c_uint32]),
            "orc_reference_load_ms": (C.c_double, [C.POINTER(C.c_char_p), C.c_uint32, C.c_uint32, C.c_uint32, u64p]),
            "orc_region_replay": (C.c_int64, [C.c_char_p, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, u64p, u64p,
                                              C.c_uint64]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _err() -> str:
    return lib().orc_last_error().decode(errors="replace")


def region_replay(events: str, saved_base: int, base: int, size: int, cursor: int):
    """Replay one graph's allocator events: (placements as (saved lo, saved hi,
    new lo) rows, new cursor), or (error code, cursor) with -1 parse, -2
    mismatch, -3 region too small."""
    data = events.encode()
    cur = C.c_uint64(cursor)
    n = lib().orc_region_replay(data, len(data), saved_base, base, size, C.byref(cur), None, 0)
    if n < 0:
        return int(n), cursor
    out = np.zeros(3 * max(1, n), dtype=np.uint64)
    cur = C.c_uint64(cursor)
    lib().orc_region_replay(data, len(data), saved_base, base, size, C.byref(cur), out.ctypes.data_as(u64p), n)
    return out[: 3 * n].reshape(n, 3), cur.value


def crc64(data: bytes) -> int:
    return lib().orc_crc64(data, len(data))


def topology_key_saved(image: bytes) -> bytes:
    n = lib().orc_topology_key_saved(image, len(image), None, 0)
    if n < 0:
        raise ValueError(_err())
    buf = C.create_string_buffer(max(1, n))
    lib().orc_topology_key_saved(image, len(image), buf, n)
    return buf.raw[:n]


def topology_key_recomputed(image: bytes) -> bytes:
    n = lib().orc_topology_key_recomputed(image, len(image), None, 0)
    if n < 0:
        raise ValueError(_err())
    buf = C.create_string_buffer(max(1, n))
    lib().orc_topology_key_recomputed(image, len(image), buf, n)
    return buf.raw[:n]


def group_by_keys(keys: Sequence[bytes]) -> np.ndarray:
    arr = (C.c_char_p * len(keys))(*keys)
    lens = np.array([len(k) for k in keys], dtype=np.uint64)
    out = np.zeros(len(keys), dtype=np.uint32)
    lib().orc_group_by_keys(arr, lens.ctypes.data_as(u64p), len(keys), out.ctypes.data_as(u32p))
    return out


def group_manifest(manifest: bytes, names: Sequence[str]) -> np.ndarray | None:
    arr = (C.c_char_p * len(names))(*[n.encode() for n in names])
    out = np.zeros(len(names), dtype=np.uint32)
    rc = lib().orc_group_manifest(manifest, len(manifest), arr, len(names), out.ctypes.data_as(u32p))
    return None if rc else out


def extract_node_params(image: bytes, node: int, cap: int = 1 << 20) -> bytes:
    buf = (C.c_uint8 * cap)()
    n = lib().orc_extract_node_params(image, len(image), node, buf, cap)
    if n < 0:
        raise ValueError("bounds error")
    return bytes(buf[:n])


def effective_attrs(image: bytes, node: int) -> list[int]:
    """The 17 merged launch-attribute fields of kernel node `node`."""
    out = (C.c_int32 * 17)()
    if lib().orc_effective_attrs(image, len(image), node, out):
        raise ValueError("not a kernel node")
    return list(out)


def set_mutation(m: int) -> None:
    """Plant mistake m in the oracle's attribute merge (0 removes it); test use only."""
    lib().orc_set_mutation(m)


def relocate_word(w: int, lo, hi, new_lo, policy: int = 0) -> int:
    lo, hi, new_lo = (np.ascontiguousarray(np.asarray(x, dtype=np.uint64)) for x in (lo, hi, new_lo))
    return lib().orc_relocate_word(
        w, lo.ctypes.data_as(u64p), hi.ctypes.data_as(u64p), new_lo.ctypes.data_as(u64p), len(lo), policy
    )


def relocate_words(words, lo, hi, new_lo, policy: int = 0, threads: int = 1) -> np.ndarray:
    words = np.ascontiguousarray(np.asarray(words, dtype=np.uint64))
    lo, hi, new_lo = (np.ascontiguousarray(np.asarray(x, dtype=np.uint64)) for x in (lo, hi, new_lo))
    out = np.empty_like(words)
    lib().orc_relocate_words(
        words.ctypes.data_as(u64p), out.ctypes.data_as(u64p), len(words), lo.ctypes.data_as(u64p),
        hi.ctypes.data_as(u64p), new_lo.ctypes.data_as(u64p), len(lo), policy, threads,
    )
    return out


def reference_load_ms(paths: Sequence[str], threads: int, reps: int = 5) -> tuple[float, int]:
    arr = (C.c_char_p * len(paths))(*[p.encode() for p in paths])
    calls = C.c_uint64()
    ms = lib().orc_reference_load_ms(arr, len(paths), threads, reps, C.byref(calls))
    if ms < 0:
        raise RuntimeError(f"reference load path failed ({ms})")
    return ms, calls.value


class Restore:
    """The CPU restore of a list of archive images."""

    def __init__(self, images: Sequence[bytes], intervals=None, policy: int = 0, template_of=None,
                 threads: int = 1):
        self._bufs = [C.create_string_buffer(b, max(1, len(b))) for b in images]
        ptrs = (u8p * len(images))(*[C.cast(b, u8p) for b in self._bufs])
        sizes = np.array([len(b) for b in images], dtype=np.uint64)
        if intervals is None:
            lo = hi = nlo = np.zeros(0, dtype=np.uint64)
        else:
            lo, hi, nlo = (np.ascontiguousarray(np.asarray(x, dtype=np.uint64)) for x in intervals)
        self._iv = (lo, hi, nlo)
        t = None
        if template_of is not None:
            self._tmpl = np.ascontiguousarray(np.asarray(template_of, dtype=np.uint32))
            t = self._tmpl.ctypes.data_as(u32p)
        h = C.c_void_p()
        rc = lib().orc_restore(
            ptrs, sizes.ctypes.data_as(u64p), len(images), lo.ctypes.data_as(u64p), hi.ctypes.data_as(u64p),
            nlo.ctypes.data_as(u64p), len(lo), policy, t, threads, C.byref(h),
        )
        if rc:
            raise ValueError("oracle restore failed: " + _err())
        self._h = h
        self.n = len(images)

    def __del__(self):
        # At interpreter exit the module's globals may already be gone.
        if getattr(self, "_h", None) and _lib is not None:
            _lib.orc_free(self._h)
            self._h = None

    def digests(self) -> np.ndarray:
        out = np.zeros((self.n, 4), dtype=np.uint64)
        lib().orc_digests(self._h, out.ctypes.data_as(u64p))
        return out

    def groups(self) -> np.ndarray:
        out = np.zeros(self.n, dtype=np.uint32)
        lib().orc_groups(self._h, out.ctypes.data_as(u32p))
        return out

    def status(self) -> np.ndarray:
        out = np.zeros(self.n, dtype=np.uint32)
        lib().orc_status(self._h, out.ctypes.data_as(u32p))
        return out

    def override_offsets(self) -> np.ndarray:
        out = np.zeros(self.n + 1, dtype=np.uint64)
        lib().orc_override_offsets(self._h, out.ctypes.data_as(u64p))
        return out

    def overrides(self, g: int) -> np.ndarray:
        n = lib().orc_overrides(self._h, g, None, 0)
        out = np.zeros(n, dtype=OVERRIDE_DTYPE)
        if n:
            lib().orc_overrides(self._h, g, out.ctypes.data, n)
        return out

    def _arr(self, fn, g, dtype, ctype):
        n = fn(self._h, g, None, 0)
        out = np.zeros(n, dtype=dtype)
        if n:
            fn(self._h, g, out.ctypes.data_as(ctype), n)
        return out

    def node_flags(self, g: int) -> np.ndarray:
        return self._arr(lib().orc_node_flags, g, np.uint8, u8p)

    def node_words(self, g: int) -> np.ndarray:
        return self._arr(lib().orc_node_words, g, np.uint32, u32p)

    def param_image(self, g: int) -> np.ndarray:
        return self._arr(lib().orc_param_image, g, np.uint64, u64p)

    def node_pointers(self, g: int) -> np.ndarray:
        return self._arr(lib().orc_node_pointers, g, np.uint64, u64p)

    def total_param_bytes(self) -> int:
        return lib().orc_total_param_bytes(self._h)

    def switch(self, g: int) -> None:
        if lib().orc_switch(self._h, g):
            raise ValueError(_err())

    def live(self, template: int) -> tuple[np.ndarray, np.ndarray, int]:
        n = lib().orc_live(self._h, template, None, 0, None, 0, None)
        if n < 0:
            raise ValueError("not a template")
        words = np.zeros(n, dtype=np.uint64)
        nodes = len(self.node_flags(template))
        src = np.zeros(nodes, dtype=np.uint32)
        cur = C.c_uint32()
        lib().orc_live(self._h, template, words.ctypes.data_as(u64p), n, src.ctypes.data_as(u32p), nodes,
                       C.byref(cur))
        return words, src, cur.value
