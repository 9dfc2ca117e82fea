"""ctypes bindings for libfoundry_restore.so and libfdy_synth.so.

The restore library is the product: every call goes through its C ABI
(include/foundry_restore.h).  There is no Python or CPU fallback -- if the
library is missing, loading raises.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
BUILD_DIR = os.path.join(_HERE, "_build")
RESTORE_LIB = os.path.join(BUILD_DIR, "libfoundry_restore.so")
SYNTH_LIB = os.path.join(BUILD_DIR, "libfdy_synth.so")

u8p = C.POINTER(C.c_uint8)
u32p = C.POINTER(C.c_uint32)
u64p = C.POINTER(C.c_uint64)

FDY_OK = 0
ERRORS = {
    -1: "FDY_E_INVALID",
    -2: "FDY_E_IO",
    -3: "FDY_E_FORMAT",
    -4: "FDY_E_HIP",
    -5: "FDY_E_NOMEM",
    -6: "FDY_E_RANGE",
    -7: "FDY_E_STATE",
    -8: "FDY_E_CAPACITY",
    -9: "FDY_E_MISMATCH",
    -10: "FDY_E_NOT_FOUND",
    -11: "FDY_E_UNSUPPORTED",
}

NODE_LAYOUT, NODE_DESC, NODE_RAGGED, NODE_TEMPLATE = 0x01, 0x02, 0x04, 0x08
GRAPH_TYPE_MISMATCH, GRAPH_BAD_PARAMS, GRAPH_COLLISION = 0x01, 0x02, 0x08
GRAPH_NODE_COUNT, GRAPH_OVERFLOW = 0x10, 0x20
RELOC_HALF_OPEN, RELOC_INCLUSIVE = 0, 1


class FoundryError(RuntimeError):
    def __init__(self, code: int, message: str):
        self.code = code
        super().__init__(f"{ERRORS.get(code, code)}: {message}")


class Override(C.Structure):
    _fields_ = [("word", C.c_uint32), ("node", C.c_uint32), ("value", C.c_uint64)]


class ArchiveInfo(C.Structure):
    _fields_ = [
        ("num_graphs", C.c_uint32),
        ("num_groups", C.c_uint32),
        ("total_nodes", C.c_uint64),
        ("total_param_bytes", C.c_uint64),
        ("total_words", C.c_uint64),
        ("total_overrides", C.c_uint64),
        ("file_bytes", C.c_uint64),
        ("num_intervals", C.c_uint64),
        ("device_bytes", C.c_uint64),
        ("serving_layout", C.c_uint32),
        ("scratch", C.c_uint32),
    ]


class RestoreTiming(C.Structure):
    _fields_ = [
        ("group_ms", C.c_float),
        ("node_ms", C.c_float),
        ("tmpl_ms", C.c_float),
        ("diff_ms", C.c_float),
        ("search_ms", C.c_float),
        ("total_ms", C.c_float),
        ("prepare_ms", C.c_float),
        ("diff_phase_ms", C.c_float),
    ]


class GroupGraphInfo(C.Structure):
    _fields_ = [
        ("template_graph", C.c_uint32),
        ("current_graph", C.c_uint32),
        ("num_nodes", C.c_uint32),
        ("num_kernel_nodes", C.c_uint32),
        ("num_fill_nodes", C.c_uint32),
        ("num_memcpy_nodes", C.c_uint32),
        ("num_event_nodes", C.c_uint32),
        ("num_deps", C.c_uint32),
        ("num_events", C.c_uint32),
        ("num_execs", C.c_uint32),
        ("build_ms", C.c_double),
        ("instantiate_ms", C.c_double),
    ]


class SelectStats(C.Structure):
    _fields_ = [
        ("nodes_reset", C.c_uint32),
        ("kernel_nodes_reset", C.c_uint32),
        ("words_scattered", C.c_uint64),
        ("host_us", C.c_double),
        ("reset_us", C.c_double),
        ("instantiate_us", C.c_double),
        ("cache_hit", C.c_uint32),
        ("pad_", C.c_uint32),
    ]


class RegionInfo(C.Structure):
    _fields_ = [
        ("saved_base", C.c_uint64),
        ("base", C.c_uint64),
        ("size", C.c_uint64),
        ("offset", C.c_uint64),
        ("granularity", C.c_uint64),
        ("mapped_bytes", C.c_uint64),
        ("live_allocations", C.c_uint64),
        ("prealloc_begin", C.c_uint64),
        ("prealloc_end", C.c_uint64),
        ("num_events", C.c_uint64),
        ("recording", C.c_uint32),
        ("flags", C.c_uint32),
    ]


class SynthParams(C.Structure):
    _fields_ = [
        ("preset", C.c_uint32),
        ("num_graphs", C.c_uint32),
        ("num_groups", C.c_uint32),
        ("nodes_per_graph", C.c_uint32),
        ("min_blob_bytes", C.c_uint32),
        ("max_blob_bytes", C.c_uint32),
        ("max_params", C.c_uint32),
        ("ragged", C.c_uint32),
        ("extra_style_pct", C.c_uint32),
        ("memset_pct", C.c_uint32),
        ("memcpy_pct", C.c_uint32),
        ("event_pct", C.c_uint32),
        ("grid_bs_pct", C.c_uint32),
        ("layout_var_pct", C.c_uint32),
        ("run_min_bytes", C.c_uint32),
        ("run_max_bytes", C.c_uint32),
        ("pointer_frac", C.c_double),
        ("diff_lo", C.c_double),
        ("diff_hi", C.c_double),
        ("seed", C.c_uint64),
        ("region_base", C.c_uint64),
        ("region_size", C.c_uint64),
        ("new_base", C.c_uint64),
        ("num_intervals", C.c_uint32),
        ("interval_granule", C.c_uint32),
        ("interval_min", C.c_uint64),
        ("interval_max", C.c_uint64),
        ("num_words", C.c_uint64),
        ("boundary_frac", C.c_double),
        ("sink_hash", C.c_uint64),
        ("diff_node_pct", C.c_uint32),
        ("pad_", C.c_uint32),
    ]


_vp = C.c_void_p
_SIGS = {
    "fdy_last_error": (C.c_char_p, []),
    "fdy_version": (C.c_char_p, []),
    "fdy_archive_open": (C.c_int, [C.POINTER(C.c_char_p), C.c_uint32, C.c_uint32, C.POINTER(_vp)]),
    "fdy_archive_open_images": (C.c_int, [C.POINTER(u8p), u64p, C.c_uint32, C.POINTER(_vp)]),
    "fdy_archive_close": (C.c_int, [_vp]),
    "fdy_archive_info_get": (C.c_int, [_vp, C.POINTER(ArchiveInfo)]),
    "fdy_archive_set_relocation": (C.c_int, [_vp, u64p, u64p, u64p, C.c_uint64, C.c_uint32]),
    "fdy_archive_set_groups": (C.c_int, [_vp, u32p]),
    "fdy_manifest_groups": (C.c_int, [C.c_char_p, C.c_uint64, C.POINTER(C.c_char_p), C.c_uint32, u32p,
                                      C.POINTER(C.c_int)]),
    "fdy_archive_set_manifest": (C.c_int, [_vp, C.c_char_p, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(C.c_int)]),
    "fdy_restore": (C.c_int, [_vp, _vp]),
    "fdy_get_digests": (C.c_int, [_vp, _vp, u64p]),
    "fdy_get_groups": (C.c_int, [_vp, _vp, u32p]),
    "fdy_get_graph_status": (C.c_int, [_vp, _vp, u32p]),
    "fdy_get_override_offsets": (C.c_int, [_vp, _vp, u64p]),
    "fdy_get_param_bytes": (C.c_int, [_vp, _vp, u64p]),
    "fdy_get_overrides": (C.c_int, [_vp, _vp, C.c_uint32, C.POINTER(Override), C.c_uint64, u64p]),
    "fdy_get_node_flags": (C.c_int, [_vp, _vp, C.c_uint32, u8p, C.c_uint64, u64p]),
    "fdy_get_node_words": (C.c_int, [_vp, _vp, C.c_uint32, u32p, C.c_uint64, u64p]),
    "fdy_get_param_image": (C.c_int, [_vp, _vp, C.c_uint32, u64p, C.c_uint64, u64p]),
    "fdy_get_node_pointers": (C.c_int, [_vp, _vp, C.c_uint32, u64p, C.c_uint64, u64p]),
    "fdy_get_section": (C.c_int, [_vp, C.c_uint32, C.c_uint32, u8p, C.c_uint64, u64p]),
    "fdy_cugraph_from_json": (C.c_int, [C.c_char_p, C.c_uint64, u8p, C.c_uint64, u64p]),
    "fdy_load_topology_key": (C.c_int, [C.c_char_p, C.c_uint64, C.c_char_p, C.c_uint64, u64p]),
    "fdy_dlpack_view": (_vp, [C.c_uint64, C.c_int32, C.c_int32, C.c_int32, C.POINTER(C.c_int64),
                              C.POINTER(C.c_int64), C.c_uint8, C.c_uint8]),
    "fdy_cugraph_save_binary": (C.c_int, [C.c_char_p, C.c_char_p, C.c_uint64]),
    "fdy_switch": (C.c_int, [_vp, C.c_uint32, _vp]),
    "fdy_switch_sequence": (C.c_int, [_vp, u32p, C.c_uint64, _vp]),
    "fdy_get_live": (C.c_int, [_vp, _vp, C.c_uint32, u64p, C.c_uint64, u32p, C.c_uint64, u32p]),
    "fdy_reloc_plan_create": (C.c_int, [u64p, u64p, u64p, C.c_uint64, C.c_uint32, C.POINTER(_vp)]),
    "fdy_reloc_plan_destroy": (C.c_int, [_vp]),
    "fdy_reloc_plan_lines": (C.c_int, [_vp, _vp, C.c_uint64, C.POINTER(C.c_uint64)]),
    "fdy_relocate_words": (C.c_int, [_vp, _vp, _vp, C.c_uint64, _vp]),
    "fdy_relocate_words_static": (C.c_int, [u64p, u64p, u64p, C.c_uint64, C.c_uint32, _vp, _vp, C.c_uint64, _vp]),
    "fdy_restore_timing_get": (C.c_int, [_vp, C.POINTER(RestoreTiming)]),
    "fdy_set_timing": (C.c_int, [_vp, C.c_int]),
    "fdy_set_group_wait": (C.c_int, [_vp, C.c_uint32]),
}

_GRAPH_SIGS = {
    "fdy_code_object_hash": (C.c_uint64, [_vp, C.c_uint64]),
    "fdy_registry_create": (C.c_int, [C.POINTER(_vp)]),
    "fdy_registry_destroy": (C.c_int, [_vp]),
    "fdy_registry_add": (C.c_int, [_vp, _vp, C.c_uint64, u64p]),
    "fdy_registry_add_file": (C.c_int, [_vp, C.c_char_p, u64p]),
    "fdy_code_object_kernels": (C.c_int, [_vp, C.c_uint64, C.c_char_p, C.c_uint64, u64p]),
    "fdy_registry_pack": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_uint32)]),
    "fdy_registry_load_packed": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_uint32)]),
    "fdy_registry_lookup": (C.c_int, [_vp, C.c_uint64, C.c_char_p, C.POINTER(_vp)]),
    "fdy_registry_global": (C.c_int, [_vp, C.c_uint64, C.c_char_p, C.POINTER(_vp), u64p]),
    "fdy_group_graph_create": (C.c_int, [_vp, C.c_uint32, _vp, _vp, C.POINTER(_vp)]),
    "fdy_group_graph_destroy": (C.c_int, [_vp]),
    "fdy_group_graph_select": (C.c_int, [_vp, C.c_uint32, _vp, C.POINTER(SelectStats)]),
    "fdy_group_graph_reset_all": (C.c_int, [_vp, _vp, C.POINTER(SelectStats)]),
    "fdy_group_graph_set_exec_cache": (C.c_int, [_vp, C.c_uint32]),
    "fdy_group_graph_launch": (C.c_int, [_vp, _vp]),
    "fdy_group_graph_info_get": (C.c_int, [_vp, C.POINTER(GroupGraphInfo)]),
    "fdy_group_graph_handles": (C.c_int, [_vp, C.POINTER(_vp), C.POINTER(_vp)]),
    "fdy_group_graph_debug_dot": (C.c_int, [_vp, C.c_char_p]),
}
_SIGS.update(_GRAPH_SIGS)

_REGION_SIGS = {
    "fdy_region_create": (C.c_int, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32, C.POINTER(_vp)]),
    "fdy_region_create_plan": (C.c_int, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.POINTER(_vp)]),
    "fdy_region_destroy": (C.c_int, [_vp]),
    "fdy_region_info_get": (C.c_int, [_vp, C.POINTER(RegionInfo)]),
    "fdy_region_alloc": (C.c_int, [_vp, C.c_uint64, u64p]),
    "fdy_region_free": (C.c_int, [_vp, C.c_uint64]),
    "fdy_region_reserve": (C.c_int, [_vp, C.c_uint64, C.c_uint64, u64p]),
    "fdy_region_preallocate": (C.c_int, [_vp, C.c_uint64]),
    "fdy_region_free_preallocated": (C.c_int, [_vp]),
    "fdy_region_get_offset": (C.c_int, [_vp, u64p]),
    "fdy_region_set_offset": (C.c_int, [_vp, C.c_uint64]),
    "fdy_region_record": (C.c_int, [_vp, C.c_int]),
    "fdy_region_clear_events": (C.c_int, [_vp]),
    "fdy_region_events_json": (C.c_int, [_vp, C.c_char_p, C.c_uint64, u64p]),
    "fdy_region_replay": (C.c_int, [_vp, C.c_char_p, C.c_uint64]),
    "fdy_region_intervals": (C.c_int, [_vp, C.c_uint32, u64p, u64p, u64p, C.c_uint64, u64p]),
}
_SIGS.update(_REGION_SIGS)
REGION_EXACT_BASE = 0x1
REGION_IV_REGION, REGION_IV_ALLOCATIONS = 0, 1

_SYNTH_SIGS = {
    "fdy_synth_preset": (C.c_int, [C.c_uint32, C.POINTER(SynthParams)]),
    "fdy_synth_create": (C.c_int, [C.POINTER(SynthParams), C.c_uint32, C.POINTER(_vp)]),
    "fdy_synth_destroy": (C.c_int, [_vp]),
    "fdy_synth_num_graphs": (C.c_uint32, [_vp]),
    "fdy_synth_image": (C.c_int, [_vp, C.c_uint32, C.POINTER(u8p), u64p]),
    "fdy_synth_batch_size": (C.c_int, [_vp, C.c_uint32, u32p]),
    "fdy_synth_intervals": (C.c_int, [_vp, C.POINTER(u64p), C.POINTER(u64p), C.POINTER(u64p), u64p]),
    "fdy_synth_words": (C.c_int, [_vp, C.POINTER(u64p), u64p]),
    "fdy_synth_write_dir": (C.c_int, [_vp, C.c_char_p]),
    "fdy_synth_switch_sequence": (C.c_int, [C.c_uint64, C.c_uint32, C.c_uint32, u32p]),
    "fdy_synth_last_error": (C.c_char_p, []),
}

_restore = None
_synth = None


def _bind(path: str, sigs: dict) -> C.CDLL:
    if not os.path.exists(path):
        raise FoundryError(
            -7, f"{path} is not built; run __graft_entry__.build() (make -C foundry_amd/csrc) first"
        )
    lib = C.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def restore_lib() -> C.CDLL:
    global _restore
    if _restore is None:
        # One HIP runtime per process: torch bundles its own libamdhip64 under
        # the same soname as the system's, and whichever loads first serves
        # both.  Loading torch first makes it torch's, so device memory and
        # streams from torch and the library's calls meet in one runtime (the
        # library loaded first ran a second runtime that found no device).
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        _restore = _bind(RESTORE_LIB, _SIGS)
    return _restore


def synth_lib() -> C.CDLL:
    global _synth
    if _synth is None:
        _synth = _bind(SYNTH_LIB, _SYNTH_SIGS)
    return _synth


def check(rc: int) -> None:
    if rc != FDY_OK:
        raise FoundryError(rc, restore_lib().fdy_last_error().decode(errors="replace"))


def check_synth(rc: int) -> None:
    if rc != 0:
        raise RuntimeError("synthetic archive: " + synth_lib().fdy_synth_last_error().decode(errors="replace"))


def exported_symbols() -> list[str]:
    return [k for k in _SIGS if k not in _GRAPH_SIGS and k not in _REGION_SIGS]


def region_symbols() -> list[str]:
    return list(_REGION_SIGS)


def graph_symbols() -> list[str]:
    return list(_GRAPH_SIGS)
