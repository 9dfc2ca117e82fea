"""Python view of the group-graph C ABI (include/foundry_graph.h).

`Registry` holds gfx950 code objects under their CRC-64/XZ identity (the
`binary_hash` a `.cugraph` kernel node names, csrc/hook.cpp:315-321).
`GroupGraph` is one hipGraph + exec per topology group, built from a
restored `Archive`; `select(g)` makes it run graph g by re-setting only the
nodes that differ from the graph it held, and `replay(g)` is select + launch,
the on-demand replay of csrc/CUDAGraph.cpp:330-483.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from ._lib import GroupGraphInfo, SelectStats, check, restore_lib
from .restore import Archive, _stream


def code_object_hash(data: bytes) -> int:
    """CRC-64/XZ of a code object's bytes (no device needed)."""
    return int(restore_lib().fdy_code_object_hash(data, len(data)))


def code_object_kernels(data: bytes) -> list[str]:
    """Kernel names of a code object (its `name.kd` symbols), sorted (no
    device needed)."""
    n = C.c_uint64()
    rc = restore_lib().fdy_code_object_kernels(data, len(data), None, 0, C.byref(n))
    if rc != -8:  # FDY_E_CAPACITY: the size query
        check(rc)
    buf = C.create_string_buffer(max(1, n.value))
    check(restore_lib().fdy_code_object_kernels(data, len(data), buf, n.value, C.byref(n)))
    return buf.raw[: n.value].decode().splitlines()


class Registry:
    """Loaded code objects, looked up by (binary_hash, kernel name)."""

    def __init__(self):
        h = C.c_void_p()
        check(restore_lib().fdy_registry_create(C.byref(h)))
        self._h = h

    def add(self, data: bytes) -> int:
        out = C.c_uint64()
        check(restore_lib().fdy_registry_add(self._h, data, len(data), C.byref(out)))
        return out.value

    def add_file(self, path: str) -> int:
        out = C.c_uint64()
        check(restore_lib().fdy_registry_add_file(self._h, path.encode(), C.byref(out)))
        return out.value

    def pack(self, directory: str) -> int:
        """Write every registered code object into the packed pair in
        `directory` (fdy_registry_pack); returns the number written."""
        n = C.c_uint32()
        check(restore_lib().fdy_registry_pack(self._h, directory.encode(), C.byref(n)))
        return n.value

    def load_packed(self, directory: str) -> int:
        """Register the code objects of the packed pair in `directory`
        (fdy_registry_load_packed); returns the number read."""
        n = C.c_uint32()
        check(restore_lib().fdy_registry_load_packed(self._h, directory.encode(), C.byref(n)))
        return n.value

    def lookup(self, binary_hash: int, name: str) -> int:
        fn = C.c_void_p()
        check(restore_lib().fdy_registry_lookup(self._h, binary_hash, name.encode(), C.byref(fn)))
        return int(fn.value or 0)

    def global_address(self, binary_hash: int, name: str) -> tuple[int, int]:
        """(device address, bytes) of a global variable of a code object."""
        p, n = C.c_void_p(), C.c_uint64()
        check(restore_lib().fdy_registry_global(self._h, binary_hash, name.encode(), C.byref(p), C.byref(n)))
        return int(p.value or 0), n.value

    def close(self) -> None:
        if self._h:
            check(restore_lib().fdy_registry_destroy(self._h))
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GroupGraph:
    """The executable graph of one topology group of a restored archive."""

    def __init__(self, archive: Archive, template: int, registry: Registry, stream=None):
        h = C.c_void_p()
        check(restore_lib().fdy_group_graph_create(archive._h, template, registry._h, _stream(stream), C.byref(h)))
        self._h = h
        self.archive = archive  # the archive refuses close/restore while this exists
        self.registry = registry

    def select(self, graph: int, stream=None) -> dict:
        st = SelectStats()
        check(restore_lib().fdy_group_graph_select(self._h, graph, _stream(stream), C.byref(st)))
        return {k: getattr(st, k) for k, _ in SelectStats._fields_ if k != "pad_"}

    def set_exec_cache(self, max_execs: int) -> None:
        """Execs kept for recently selected graphs (at least 1; default 4)."""
        check(restore_lib().fdy_group_graph_set_exec_cache(self._h, int(max_execs)))

    def reset_all(self, stream=None) -> dict:
        st = SelectStats()
        check(restore_lib().fdy_group_graph_reset_all(self._h, _stream(stream), C.byref(st)))
        return {k: getattr(st, k) for k, _ in SelectStats._fields_ if k != "pad_"}

    def launch(self, stream=None) -> None:
        check(restore_lib().fdy_group_graph_launch(self._h, _stream(stream)))

    def replay(self, graph: int, stream=None) -> dict:
        st = self.select(graph, stream)
        self.launch(stream)
        return st

    def handles(self) -> tuple[int, int]:
        """(hipGraph_t, hipGraphExec_t) as integers; owned by this group graph."""
        g, e = C.c_void_p(), C.c_void_p()
        check(restore_lib().fdy_group_graph_handles(self._h, C.byref(g), C.byref(e)))
        return g.value or 0, e.value or 0

    def debug_dot(self, path: str) -> None:
        """hipGraphDebugDotPrint (verbose) of the group's graph to `path`."""
        check(restore_lib().fdy_group_graph_debug_dot(self._h, path.encode()))

    def info(self) -> dict:
        i = GroupGraphInfo()
        check(restore_lib().fdy_group_graph_info_get(self._h, C.byref(i)))
        return {k: getattr(i, k) for k, _ in GroupGraphInfo._fields_ if k != "pad_"}

    def close(self) -> None:
        if self._h:
            check(restore_lib().fdy_group_graph_destroy(self._h))
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


__all__ = ["Registry", "GroupGraph", "code_object_hash", "code_object_kernels", "_lib"]
