"""Seeded synthetic `.cugraph` archives (include/fdy_synth.h)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import SynthParams, check_synth, synth_lib


def preset(n: int, **overrides) -> SynthParams:
    p = SynthParams()
    check_synth(synth_lib().fdy_synth_preset(n, C.byref(p)))
    for k, v in overrides.items():
        if not hasattr(p, k):
            raise AttributeError(f"unknown synthetic-archive field {k!r}")
        setattr(p, k, v)
    return p


class SynthArchive:
    """An in-memory synthetic archive: graph images, the allocation
    intervals (old lo, hi, new lo) and, for preset 4, packed words."""

    def __init__(self, params: SynthParams, threads: int = 0):
        self.params = params
        h = C.c_void_p()
        check_synth(synth_lib().fdy_synth_create(C.byref(params), threads, C.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h:
            synth_lib().fdy_synth_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def num_graphs(self) -> int:
        return synth_lib().fdy_synth_num_graphs(self._h)

    def image_ptr(self, i: int) -> tuple[int, int]:
        p = _lib.u8p()
        n = C.c_uint64()
        check_synth(synth_lib().fdy_synth_image(self._h, i, C.byref(p), C.byref(n)))
        return C.cast(p, C.c_void_p).value or 0, n.value

    def image(self, i: int) -> bytes:
        addr, n = self.image_ptr(i)
        return C.string_at(addr, n)

    def images(self) -> list[bytes]:
        return [self.image(i) for i in range(self.num_graphs)]

    def batch_size(self, i: int) -> int:
        v = C.c_uint32()
        check_synth(synth_lib().fdy_synth_batch_size(self._h, i, C.byref(v)))
        return v.value

    def intervals(self) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        lo, hi, nlo = _lib.u64p(), _lib.u64p(), _lib.u64p()
        n = C.c_uint64()
        check_synth(synth_lib().fdy_synth_intervals(self._h, C.byref(lo), C.byref(hi), C.byref(nlo), C.byref(n)))
        k = n.value
        return (
            np.ctypeslib.as_array(lo, (k,)).copy(),
            np.ctypeslib.as_array(hi, (k,)).copy(),
            np.ctypeslib.as_array(nlo, (k,)).copy(),
        )

    def words(self) -> np.ndarray:
        w = _lib.u64p()
        n = C.c_uint64()
        check_synth(synth_lib().fdy_synth_words(self._h, C.byref(w), C.byref(n)))
        if n.value == 0:
            return np.zeros(0, dtype=np.uint64)
        return np.ctypeslib.as_array(w, (n.value,))  # view; valid while the archive lives

    def write_dir(self, path: str) -> list[str]:
        check_synth(synth_lib().fdy_synth_write_dir(self._h, path.encode()))
        return [f"{path}/graph_{i}.cugraph" for i in range(self.num_graphs)]


def switch_sequence(seed: int, num_graphs: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.uint32)
    check_synth(
        synth_lib().fdy_synth_switch_sequence(seed, num_graphs, n, out.ctypes.data_as(_lib.u32p))
    )
    return out
