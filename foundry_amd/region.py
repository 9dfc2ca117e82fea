"""Python view of the allocation-region C ABI (include/foundry_region.h).

A `Region` is a virtual-address range whose allocations are placed by the
reference's cursor rule (csrc/hook.cpp:2246-2441), with the allocator-event
record and replay of csrc/hook.cpp:3354-3492.  After replaying an archive's
events, `intervals()` is the relocation table for `Archive.set_relocation`.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import RegionInfo, check, restore_lib

MiB = 1 << 20


class Region:
    def __init__(self, base: int, size: int, align: int = 0, exact: bool = False, _handle=None):
        if _handle is not None:
            self._h = _handle
            return
        h = C.c_void_p()
        check(restore_lib().fdy_region_create(base, size, align, _lib.REGION_EXACT_BASE if exact else 0, C.byref(h)))
        self._h = h

    @classmethod
    def plan(cls, saved_base: int, base: int, size: int, granularity: int = 0) -> "Region":
        """Placement arithmetic only (no device): saved at saved_base, placed from base."""
        h = C.c_void_p()
        check(restore_lib().fdy_region_create_plan(saved_base, base, size, granularity, C.byref(h)))
        return cls(0, 0, _handle=h)

    def info(self) -> dict:
        i = RegionInfo()
        check(restore_lib().fdy_region_info_get(self._h, C.byref(i)))
        return {k: getattr(i, k) for k, _ in RegionInfo._fields_}

    @property
    def base(self) -> int:
        return self.info()["base"]

    def alloc(self, nbytes: int) -> int:
        p = C.c_uint64()
        check(restore_lib().fdy_region_alloc(self._h, nbytes, C.byref(p)))
        return p.value

    def free(self, ptr: int) -> None:
        check(restore_lib().fdy_region_free(self._h, ptr))

    def reserve(self, size: int, alignment: int) -> int:
        p = C.c_uint64()
        check(restore_lib().fdy_region_reserve(self._h, size, alignment, C.byref(p)))
        return p.value

    def preallocate(self, size: int) -> None:
        check(restore_lib().fdy_region_preallocate(self._h, size))

    def free_preallocated(self) -> None:
        check(restore_lib().fdy_region_free_preallocated(self._h))

    @property
    def offset(self) -> int:
        v = C.c_uint64()
        check(restore_lib().fdy_region_get_offset(self._h, C.byref(v)))
        return v.value

    @offset.setter
    def offset(self, value: int) -> None:
        check(restore_lib().fdy_region_set_offset(self._h, value))

    def record(self, enabled: bool = True) -> None:
        check(restore_lib().fdy_region_record(self._h, 1 if enabled else 0))

    def clear_events(self) -> None:
        check(restore_lib().fdy_region_clear_events(self._h))

    def events_json(self) -> str:
        n = C.c_uint64()
        check(restore_lib().fdy_region_events_json(self._h, None, 0, C.byref(n)))
        buf = C.create_string_buffer(max(1, n.value))
        check(restore_lib().fdy_region_events_json(self._h, buf, n.value, C.byref(n)))
        return buf.raw[: n.value].decode()

    def replay(self, events) -> None:
        data = events.encode() if isinstance(events, str) else bytes(events)
        check(restore_lib().fdy_region_replay(self._h, data, len(data)))

    def intervals(self, per_allocation: bool = False):
        mode = _lib.REGION_IV_ALLOCATIONS if per_allocation else _lib.REGION_IV_REGION
        n = C.c_uint64()
        check(restore_lib().fdy_region_intervals(self._h, mode, None, None, None, 0, C.byref(n)))
        lo, hi, nlo = (np.zeros(n.value, dtype=np.uint64) for _ in range(3))
        if n.value:
            check(
                restore_lib().fdy_region_intervals(
                    self._h, mode, lo.ctypes.data_as(_lib.u64p), hi.ctypes.data_as(_lib.u64p),
                    nlo.ctypes.data_as(_lib.u64p), n.value, C.byref(n),
                )
            )
        return lo, hi, nlo

    def close(self) -> None:
        if self._h:
            check(restore_lib().fdy_region_destroy(self._h))
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
