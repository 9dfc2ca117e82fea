"""The reference's `foundry` names on this build (python/foundry/__init__.py,
pinned by the reference's tests/test_imports.py:41-69), its size parser, and
save_graph_manifest's output -- all without a GPU."""
import json
import os

import pytest

import cugraph_writer as W
import foundry_amd
from foundry_amd import _lib, api

PUBLIC_NAMES_FROM_FOUNDRY = [
    "CUDAGraph", "allocation_region", "free_preallocated_region", "get_current_alloc_offset", "graph",
    "parse_size", "preallocate_region", "resume_allocation_region", "save_graph_manifest",
    "set_current_alloc_offset", "set_allocation_region", "stop_allocation_region",
]


def test_re_exports_present():
    missing = [n for n in PUBLIC_NAMES_FROM_FOUNDRY if not hasattr(foundry_amd, n)]
    assert not missing
    ops = __import__("foundry_amd.ops", fromlist=["CUDAGraph"])
    for name in ("start_graph_builds", "finish_graph_loads", "finish_one_graph_load", "load", "replay"):
        assert hasattr(ops.CUDAGraph, name)


@pytest.mark.parametrize("text,value", [
    (4096, 4096), ("1GB", 1 << 30), ("16MB", 16 << 20), ("24KB", 24 << 10), (" 2tb ", 2 << 40), ("1.5GB", 3 << 29),
    ("512", 512), ("7 b", 7),
])
def test_parse_size(text, value):
    assert api.parse_size(text) == value


@pytest.mark.parametrize("bad", ["", "GB", "1XB", "-1GB", "1,5GB"])
def test_parse_size_rejects(bad):
    with pytest.raises(ValueError):
        api.parse_size(bad)


def test_capture_is_refused_clearly():
    g = api.CUDAGraph()
    with pytest.raises(NotImplementedError):
        g.capture_begin()
    with pytest.raises(NotImplementedError):
        with api.graph(g):
            pass


def _kern(name):
    return W.Kernel(name, 0x1234, params=[W.le(0)])


def test_save_graph_manifest_groups_by_key_in_capture_order(tmp_path):
    a = [_kern("k"), W.Empty()]
    b = [_kern("k"), _kern("k")]
    specs = {0: a, 1: b, 2: a, 3: b, 10: a}
    for i, nodes in specs.items():
        (tmp_path / f"graph_{i}_bs{i}.cugraph").write_bytes(W.write(nodes))
    # one graph also has its JSON, whose dependencies are stripped (not a template)
    (tmp_path / "graph_2_bs2.json").write_text(json.dumps({"topology_key": W.saved_key(a).decode(),
                                                           "dependencies": [{"from": 0, "to": 1}]}))
    api.save_graph_manifest(str(tmp_path))
    text = (tmp_path / "graph_manifest.json").read_text()
    key_a, key_b = W.saved_key(a).decode(), W.saved_key(b).decode()
    expect = {"topology_groups": [
        {"topology_key": key_a, "template": "graph_0_bs0.json",
         "members": ["graph_0_bs0.json", "graph_2_bs2.json", "graph_10_bs10.json"]},
        {"topology_key": key_b, "template": "graph_1_bs1.json", "members": ["graph_1_bs1.json", "graph_3_bs3.json"]},
    ]}
    assert text == json.dumps(expect, indent=2)  # the reference writes with json.dump(indent=2)
    assert "dependencies" not in json.loads((tmp_path / "graph_2_bs2.json").read_text())


def test_save_graph_manifest_needs_every_key(tmp_path):
    (tmp_path / "graph_0.json").write_text(json.dumps({"topology_key": ""}))
    api.save_graph_manifest(str(tmp_path))
    assert not os.path.exists(tmp_path / "graph_manifest.json")


# python/foundry/__init__.py names, and those tests/test_imports.py:41-54 pins.
REFERENCE_PUBLIC_NAMES = ["CUDAGraph", "allocation_region", "free_preallocated_region", "get_current_alloc_offset",
                          "graph", "parse_size", "preallocate_region", "resume_allocation_region",
                          "save_graph_manifest", "set_current_alloc_offset", "set_allocation_region",
                          "stop_allocation_region"]
# csrc/binding.cpp:14-90 module functions.
REFERENCE_OPS_FUNCTIONS = ["graph_pool_handle", "get_graph_ptr", "set_allocation_region", "stop_allocation_region",
                           "resume_allocation_region", "preallocate_region", "free_preallocated_region",
                           "get_current_alloc_offset", "set_current_alloc_offset", "set_pack_fatbins_on_exit",
                           "set_skip_fatbin_processing", "set_nvshmem_auto_init", "init_nvshmem_for_loaded_modules",
                           "pack_fatbins_to_folder", "load_cuda_modules_and_libraries",
                           "preallocate_cublas_workspaces"]
REFERENCE_CUDAGRAPH_METHODS = ["capture_begin", "capture_end", "register_generator_state", "replay", "reset", "pool",
                               "debug_dump", "enable_debug_mode", "raw_cuda_graph", "raw_cuda_graph_exec", "save",
                               "load", "start_graph_builds", "finish_graph_loads", "finish_one_graph_load"]


def test_ops_surface_complete():
    from foundry_amd import ops

    assert sorted(set(REFERENCE_OPS_FUNCTIONS) - set(ops.__all__)) == []
    for name in REFERENCE_OPS_FUNCTIONS:
        assert callable(getattr(ops, name)), name
    for name in REFERENCE_CUDAGRAPH_METHODS:
        assert callable(getattr(ops.CUDAGraph, name)), name
    assert ops.init_nvshmem_for_loaded_modules() == 0
    ops.set_skip_fatbin_processing(True)
    ops.set_pack_fatbins_on_exit(False)
    ops.set_nvshmem_auto_init(False)
    g = ops.CUDAGraph()
    with pytest.raises(RuntimeError, match="keep_graph"):
        g.raw_cuda_graph()
    with pytest.raises(RuntimeError):
        g.pool()


def test_load_modules_needs_code_objects(tmp_path):
    """Neither the packed pair nor a loose code object: an error, as the
    reference aborts when the packed files are missing."""
    from foundry_amd import ops

    (tmp_path / "notes.txt").write_text("no code objects here")
    with pytest.raises(RuntimeError, match="no packed code objects"):
        ops.load_cuda_modules_and_libraries(str(tmp_path))


def test_code_object_kernels():
    """Kernel names come from the code object's `.kd` symbols (no device)."""
    import graph_cases as GC
    from foundry_amd.graph import code_object_kernels

    data = open(GC.PROBE_CO, "rb").read()
    names = code_object_kernels(data)
    assert {"probe_mix", "probe_chain"} <= set(names) and names == sorted(names)
    assert all(not n.endswith(".kd") for n in names)
    with pytest.raises(_lib.FoundryError, match="FDY_E_FORMAT"):
        code_object_kernels(b"\x7fELF" + bytes(60))
    with pytest.raises(_lib.FoundryError, match="FDY_E_FORMAT"):
        code_object_kernels(data[:100])


def test_install_as_foundry():
    import importlib
    import sys

    from foundry_amd import api, ops

    saved = {k: sys.modules.pop(k) for k in list(sys.modules) if k == "foundry" or k.startswith("foundry.")}
    try:
        api.install_as_foundry()
        foundry = importlib.import_module("foundry")
        assert [n for n in REFERENCE_PUBLIC_NAMES if not hasattr(foundry, n)] == []
        from foundry.graph import CUDAGraph as GraphCUDAGraph
        from foundry.ops import set_skip_fatbin_processing

        assert GraphCUDAGraph is api.CUDAGraph
        assert foundry.CUDAGraph is ops.CUDAGraph  # the star import of foundry.ops comes last
        assert set_skip_fatbin_processing is ops.set_skip_fatbin_processing
        assert foundry.graph is api.graph  # the class shadows the submodule, as in the reference
        region = importlib.import_module("foundry.allocation_region")
        assert region.parse_size("16MB") == 16 << 20
        api.install_as_foundry()  # idempotent
    finally:
        for k in [k for k in sys.modules if k == "foundry" or k.startswith("foundry.")]:
            del sys.modules[k]
        sys.modules.update(saved)


def test_generator_registry_and_section_rows():
    """get_state_from_id makes a state of the saved seed and offset 0 once per
    id (csrc/CUDAGraph.cpp:147-160); GENERATORS rows are (id, seed,
    wholegraph_increment) u64 triples (include/BinaryGraphFormat.h:214-219)."""
    import struct

    from foundry_amd import ops

    reg = ops.GeneratorStateRegistry()
    a = reg.get_state_from_id(3, 0xFFFF_FFFF_FFFF_FFF0)
    assert a.seed == 0xFFFF_FFFF_FFFF_FFF0 and a.philox_offset_per_thread == 0
    assert reg.get_state_from_id(3, 1) is a and a.seed == 0xFFFF_FFFF_FFFF_FFF0
    assert reg.get_state_from_id(4, 1) is not a
    rows = ops.generators_of(struct.pack("<6Q", 1, 2, 3, 4, 5, 6))
    assert rows == [(1, 2, 3), (4, 5, 6)]
    assert ops.generators_of(b"") == []
    assert ops._as_i64(0xFFFF_FFFF_FFFF_FFF0) == -16 and ops._as_i64(5) == 5


def test_dlpack_view_of_host_memory():
    """fdy_dlpack_view's struct layout and deleter, checked on host memory
    (DLPack device type 1, kDLCPU) with torch's importer: shape, strides,
    dtype and aliasing, and views that die before and after the memory's
    owner is read again."""
    import ctypes as C

    import numpy as np
    import torch

    from foundry_amd import _lib, ops

    a = np.arange(24, dtype=np.int64)
    shape = (C.c_int64 * 2)(4, 3)
    strides = (C.c_int64 * 2)(6, 2)
    view = _lib.restore_lib().fdy_dlpack_view(a.ctypes.data, 1, 0, 2, shape, strides, 1, 64)
    t = torch.from_dlpack(ops._PyCapsule_New(view, b"dltensor", None)).view(torch.int64)
    assert t.shape == (4, 3) and t.stride() == (6, 2)
    assert t.tolist() == [[0, 2, 4], [6, 8, 10], [12, 14, 16], [18, 20, 22]]
    t[1, 1] = -5
    assert a[8] == -5
    del t
    for _ in range(100):  # many views made and freed
        v = _lib.restore_lib().fdy_dlpack_view(a.ctypes.data, 1, 0, 1, (C.c_int64 * 1)(24), (C.c_int64 * 1)(1), 1, 64)
        assert int(torch.from_dlpack(ops._PyCapsule_New(v, b"dltensor", None)).sum()) == int(a.sum())
