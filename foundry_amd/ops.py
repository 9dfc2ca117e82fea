"""The reference's `foundry.ops` LOAD surface, on the MI355X restore path.

Mirrors the names, arguments and error behaviour of the compiled module the
reference binds in csrc/binding.cpp:13-338 for the LOAD side:

  allocation region   set_allocation_region / stop_ / resume_allocation_region,
                      preallocate_region / free_preallocated_region,
                      get_ / set_current_alloc_offset        (csrc/binding.cpp:16-69)
  code objects        load_cuda_modules_and_libraries(dir)   (csrc/binding.cpp:81-86)
  graphs              CUDAGraph.load / start_graph_builds / finish_graph_loads /
                      finish_one_graph_load, CUDAGraph.replay / reset / pool /
                      debug_dump / raw_cuda_graph(_exec)     (csrc/binding.cpp:118-338)
  the rest            graph_pool_handle, get_graph_ptr, preallocate_cublas_workspaces,
                      and the fatbin / NVSHMEM switches, which have nothing to act
                      on for gfx950 code objects              (csrc/binding.cpp:14-90)

Underneath: the archives are opened and restored on the GPU in one pass
(`Archive`), each topology group gets one hipGraph exec (`GroupGraph`), and a
graph's replay switches its group's exec to it and launches.  When the
allocation region could not sit at its saved base, the restore relocates
every saved pointer by the region's interval, and output tensors are views at
the relocated addresses.

Capture and SAVE (capture_begin / capture_end / save) are not part of this
build: they raise NotImplementedError.
"""
from __future__ import annotations

import atexit
import concurrent.futures
import ctypes as C
import json
import os
import threading
import warnings
from typing import Sequence

import numpy as np
import torch

from . import _lib
from .graph import GroupGraph, Registry
from .region import Region
from .restore import Archive

MiB = 1 << 20
SEC_GENERATORS, SEC_ALLOC_EVENTS, SEC_OUTPUT_TENSORS = 7, 8, 9

# ---- allocation region (per thread, as the reference's TLS state, csrc/hook.cpp:218-251) ----

_tls = threading.local()


def _region() -> Region | None:
    return getattr(_tls, "region", None)


def set_allocation_region(base: int, size: int) -> None:
    """Reserve the region (csrc/hook.cpp:3088-3142).  The base is rounded up to
    2 MiB as the reference does; when the device cannot hold the region there,
    it is placed elsewhere and graphs restored later are relocated."""
    old = _region()
    if old is not None:
        old.close()
    base = (int(base) + 2 * MiB - 1) // (2 * MiB) * (2 * MiB)
    size = (int(size) + 2 * MiB - 1) // (2 * MiB) * (2 * MiB)
    _tls.region = Region(base, size)
    _tls.enabled = True


def release_allocation_region() -> None:
    """Unmap and unreserve this thread's region (no counterpart in the
    reference, whose region lives as long as the process).  Views into it
    must be dropped first."""
    r = _region()
    if r is not None:
        r.close()
    _tls.region = None
    _tls.enabled = False


def stop_allocation_region() -> None:
    _tls.enabled = False


def resume_allocation_region() -> None:
    _tls.enabled = True


def allocation_region_enabled() -> bool:
    return _region() is not None and getattr(_tls, "enabled", False)


def preallocate_region(size: int) -> bool:
    """csrc/hook.cpp:3161-3275: False (not an exception) when it cannot."""
    r = _region()
    if r is None:
        return False
    try:
        r.preallocate(int(size))
    except _lib.FoundryError:
        return False
    return True


def free_preallocated_region() -> None:
    r = _region()
    if r is not None:
        r.free_preallocated()


def get_current_alloc_offset() -> int:
    r = _region()
    return r.offset if r is not None else 0


def set_current_alloc_offset(offset: int) -> None:
    r = _region()
    if r is None:
        raise RuntimeError("set_current_alloc_offset: no allocation region is set")
    r.offset = int(offset)


def region_alloc(nbytes: int) -> int:
    """An allocation placed by the region's cursor rule (what the reference's
    cuMemAlloc_v2 interposer does for every driver allocation)."""
    r = _region()
    if r is None or not allocation_region_enabled():
        raise RuntimeError("no enabled allocation region")
    return r.alloc(int(nbytes))


def region_free(ptr: int) -> None:
    r = _region()
    if r is None:
        raise RuntimeError("no allocation region")
    r.free(int(ptr))


def graph_pool_handle():
    return torch.cuda.graph_pool_handle()


def get_graph_ptr(graph) -> int:
    """csrc/binding.cpp:16-19: an integer naming the graph object for hook
    integration (here the Python object's identity)."""
    return id(graph)


# ---- code-object packing and the reference's NVSHMEM switches --------------
# csrc/binding.cpp:54-81.  Packing writes the process registry's gfx950 code
# objects into the packed pair (csrc/hook.cpp:1589-1707); the fatbin
# interception that skip_fatbin_processing turns off and the NVSHMEM module
# initialisation have no gfx950 counterpart: those setters record the value
# and change nothing, and initialisation finds no modules to initialise.

_flags = {"pack_fatbins_on_exit": False, "skip_fatbin_processing": False, "nvshmem_auto_init": True}
PACK_ON_EXIT_DIR = "hook_archive"  # where the reference packs at exit (csrc/hook.cpp:1702-1707)


def _pack_on_exit() -> None:
    if _flags["pack_fatbins_on_exit"] and _registry is not None:
        _registry.pack(PACK_ON_EXIT_DIR)


def set_pack_fatbins_on_exit(enabled: bool) -> None:
    """Pack the registry into ./hook_archive when the process exits."""
    _flags["pack_fatbins_on_exit"] = bool(enabled)


def set_skip_fatbin_processing(enabled: bool) -> None:
    _flags["skip_fatbin_processing"] = bool(enabled)


def set_nvshmem_auto_init(enabled: bool) -> None:
    _flags["nvshmem_auto_init"] = bool(enabled)


def init_nvshmem_for_loaded_modules() -> int:
    """Modules initialised for NVSHMEM: none among gfx950 code objects."""
    return 0


def pack_fatbins_to_folder(folder_path: str) -> None:
    """Write every code object of the process registry into
    folder_path/fatbin_image_packed.img + fatbin_entrypoint_packed.txt
    (csrc/hook.cpp:1589-1700), which load_cuda_modules_and_libraries reads."""
    registry().pack(str(folder_path))


def preallocate_cublas_workspaces() -> None:
    """csrc/binding.cpp:88-90: create the BLAS handle and workspace of the
    current stream before graphs that use them are loaded (hipBLAS/hipBLASLt
    through torch: one small product on the current stream)."""
    torch.cuda.current_blas_handle()
    a = torch.ones((8, 8), device="cuda", dtype=torch.bfloat16)
    (a @ a).sum().item()


# ---- code objects -----------------------------------------------------------

_registry: Registry | None = None
_registry_lock = threading.Lock()


def registry() -> Registry:
    global _registry
    with _registry_lock:
        if _registry is None:
            _registry = Registry()
            atexit.register(_pack_on_exit)
        return _registry


def load_cuda_modules_and_libraries(directory: str) -> int:
    """Register the code objects of `directory` in the process registry;
    kernels then resolve by CRC-64/XZ of the code object and name
    (csrc/hook.cpp:3514-3551).  The packed pair pack_fatbins_to_folder writes
    is read when present (csrc/hook.cpp:3787-3830); otherwise every loose
    gfx950 code object (*.co, *.hsaco).  A directory with neither is an
    error, as the reference's missing packed files are.  Returns the number
    of code objects registered."""
    if all(os.path.exists(os.path.join(directory, f))
           for f in ("fatbin_image_packed.img", "fatbin_entrypoint_packed.txt")):
        return registry().load_packed(directory)
    n = 0
    for name in sorted(os.listdir(directory)):
        if name.endswith((".co", ".hsaco")):
            registry().add_file(os.path.join(directory, name))
            n += 1
    if n == 0:
        raise RuntimeError(f"no packed code objects (fatbin_image_packed.img + fatbin_entrypoint_packed.txt) "
                           f"and no *.co / *.hsaco in {directory}")
    return n


# ---- output tensors ---------------------------------------------------------

# c10::ScalarType numbering, as the reference saves `dtype` (csrc/CUDAGraph.cpp:961).
_SCALAR_TYPES = {
    0: torch.uint8, 1: torch.int8, 2: torch.int16, 3: torch.int32, 4: torch.int64, 5: torch.float16,
    6: torch.float32, 7: torch.float64, 9: torch.complex64, 10: torch.complex128, 11: torch.bool,
    15: torch.bfloat16, 23: torch.float8_e5m2, 24: torch.float8_e4m3fn, 25: torch.float8_e5m2fnuz,
    26: torch.float8_e4m3fnuz,
}


_PyCapsule_New = C.pythonapi.PyCapsule_New
_PyCapsule_New.restype = C.py_object
_PyCapsule_New.argtypes = [C.c_void_p, C.c_char_p, C.c_void_p]
_kDLROCM = 10


def tensor_at(ptr: int, sizes: Sequence[int], strides: Sequence[int], dtype: torch.dtype, device_index: int = 0,
              requires_grad: bool = False) -> torch.Tensor:
    """A non-owning view of device memory at `ptr` (at::from_blob,
    csrc/CUDAGraph.cpp:996): a DLPack view made by the library (whose deleter
    frees only its own block, no Python involved), imported as unsigned
    integers of the element size and viewed as `dtype`."""
    esize = torch.empty((), dtype=dtype).element_size()
    nd = len(sizes)
    shape = (C.c_int64 * max(1, nd))(*sizes)
    strd = (C.c_int64 * max(1, nd))(*strides)
    view = _lib.restore_lib().fdy_dlpack_view(int(ptr), _kDLROCM, int(device_index), nd, shape, strd, 1, 8 * esize)
    if not view:
        raise RuntimeError(_lib.restore_lib().fdy_last_error().decode(errors="replace"))
    t = torch.from_dlpack(_PyCapsule_New(view, b"dltensor", None)).view(dtype)
    if requires_grad:
        t.requires_grad_(True)
    return t


def _relocate(ptr: int, intervals) -> int:
    lo, hi, nlo = intervals
    if not len(lo):
        return ptr
    i = int(np.searchsorted(lo, np.uint64(ptr), side="right")) - 1
    if i >= 0 and ptr < int(hi[i]):
        return (ptr - int(lo[i]) + int(nlo[i])) & ((1 << 64) - 1)
    return ptr


def _outputs_from(text: bytes, intervals):
    """OUTPUT_TENSORS metadata -> None, a tensor, or a list/tuple of tensors
    (csrc/CUDAGraph.cpp:971-999, csrc/CUDAGraphParallel.cpp:2077-2095)."""
    if not text:
        return None
    obj = json.loads(text)
    kind = int(obj.get("type", 0))
    metas = obj.get("tensors", [])

    def one(m):
        dt = _SCALAR_TYPES.get(int(m["dtype"]))
        if dt is None:
            raise RuntimeError(f"output tensor of unsupported scalar type {m['dtype']}")
        return tensor_at(_relocate(int(m["data_ptr"]), intervals), [int(s) for s in m["sizes"]],
                         [int(s) for s in m["strides"]], dt, int(m.get("device_index", 0) or 0),
                         bool(m.get("requires_grad", False)))

    if kind == 1 and len(metas) == 1:
        return one(metas[0])
    if kind in (2, 3):
        ts = [one(m) for m in metas]
        return tuple(ts) if kind == 3 else ts
    return None


# ---- generator state (csrc/CUDAGraph.cpp:35-97, 133-160, 185-194) -----------

_I64 = 1 << 63


def _as_i64(v: int) -> int:
    """int64_t(v) for a uint64 value, as the reference's fill_ receives it."""
    v &= (1 << 64) - 1
    return v - (1 << 64) if v >= _I64 else v


class GeneratorState:
    """The state a captured graph's random-number kernels read: the graph-safe
    Philox seed and offset words (at::CUDAGeneratorState as the reference
    overrides it, csrc/CUDAGraph.cpp:35-97).

    The two words are allocated when the first graph registers (register_graph,
    35-46): as two one-element int64 tensors, which torch's caching allocator
    places 512 bytes apart in a fresh small-block segment of 2 MiB.  With an
    allocation region enabled on this thread the segment is one region
    allocation of 2 MiB at the cursor (what the reference's cuMemAlloc_v2
    interposer does with that segment), seed at +0 and offset at +512; the
    reference registers before replaying the graph's allocator events, so the
    words land where they were at SAVE.  Without a region, a torch tensor of
    the same layout.  replay_prologue (79-86) writes both words on the
    current stream and advances the offset by the graph's increment rounded
    up to a multiple of 4 (increase, 60-77)."""

    SEGMENT = 2 * MiB
    OFFSET_AT = 512

    def __init__(self, seed: int, philox_offset_per_thread: int = 0):
        self.seed = int(seed) & ((1 << 64) - 1)
        self.philox_offset_per_thread = int(philox_offset_per_thread)
        self._graphs: set[int] = set()
        self._buf = None      # torch tensor keeping the words alive (no region)
        self._region_ptr = 0  # region allocation holding them
        self.seed_ptr = 0
        self.offset_ptr = 0

    def register_graph(self, graph) -> None:
        if not self._graphs:
            r = _region()
            if r is not None and allocation_region_enabled():
                self._region_ptr = r.alloc(self.SEGMENT)
                self.seed_ptr = self._region_ptr
            else:
                self._buf = torch.empty(self.SEGMENT // 8, dtype=torch.int64, device="cuda")
                self.seed_ptr = self._buf.data_ptr()
            self.offset_ptr = self.seed_ptr + self.OFFSET_AT
            dev = torch.cuda.current_device()
            self._seed = tensor_at(self.seed_ptr, [1], [1], torch.int64, dev)
            self._offset = tensor_at(self.offset_ptr, [1], [1], torch.int64, dev)
        self._graphs.add(id(graph))

    def unregister_graph(self, graph) -> None:
        self._graphs.discard(id(graph))

    def replay_prologue(self, wholegraph_increment: int) -> None:
        if wholegraph_increment:
            self._seed.fill_(_as_i64(self.seed))
            self._offset.fill_(_as_i64(self.philox_offset_per_thread))
            self.philox_offset_per_thread += (int(wholegraph_increment) + 3) // 4 * 4


class GeneratorStateRegistry:
    """Generator states by the id a graph saved them under; a new id makes a
    state of the saved seed and offset 0 (get_state_from_id,
    csrc/CUDAGraph.cpp:147-160)."""

    def __init__(self):
        self._states: dict[int, GeneratorState] = {}
        self._lock = threading.Lock()

    def get_state_from_id(self, state_id: int, seed: int) -> GeneratorState:
        with self._lock:
            st = self._states.get(int(state_id))
            if st is None:
                st = GeneratorState(seed, 0)
                self._states[int(state_id)] = st
            return st


global_generator_state_registry = GeneratorStateRegistry()


def generators_of(section: bytes) -> list[tuple[int, int, int]]:
    """(id, seed, wholegraph_increment) rows of a GENERATORS section
    (BinGenerator, include/BinaryGraphFormat.h:214-219)."""
    n = len(section) // 24
    a = np.frombuffer(section[: 24 * n], dtype="<u8").reshape(n, 3)
    return [(int(r[0]), int(r[1]), int(r[2])) for r in a]


# ---- graphs -----------------------------------------------------------------


class PendingGraphLoads:
    """The split-load state (include/CUDAGraphInternal.h:13-28): one CUDAGraph
    shell per graph at once, and, once the background build is complete, the
    restored archive and one group graph per topology group.

    start_graph_builds returns while a worker thread opens the archives,
    restores them on the GPU and builds the group graphs (the reference's
    detached Phase 2 thread, csrc/CUDAGraphParallel.cpp:1861-2017, which also
    overlaps the caller's own initialisation).  `build_complete` is that
    work's future; the finish calls, `archive`, `template_of`,
    `used_manifest` and `group_graphs` wait for it and raise the worker's
    error, every time they are asked (the reference's finish_graph_loads uses
    get(), which rethrows; its finish_one_graph_load only waits)."""

    def __init__(self, json_paths: Sequence[str], num_threads: int, pool=None):
        self.pool = pool if pool is not None else (0, 0)
        self.json_paths = list(json_paths)
        self.names = [os.path.basename(p) for p in self.json_paths]
        self.num_threads = max(1, int(num_threads))
        self.graphs = [CUDAGraph._restored(self, i) for i in range(len(self.json_paths))]
        self.finished = [False] * len(self.json_paths)
        self.outputs: list = [None] * len(self.json_paths)
        # The allocation region is per thread: its intervals are read here,
        # on the caller's thread, for the worker.
        r = _region()
        self.intervals = (np.zeros(0, np.uint64),) * 3
        if r is not None:
            info = r.info()
            if info["base"] != info["saved_base"]:
                self.intervals = r.intervals()
        self.device = torch.cuda.current_device()
        self._archive: Archive | None = None
        self._template_of = None
        self._used_manifest = False
        self._group_graphs: dict[int, GroupGraph] = {}
        self.build_complete: concurrent.futures.Future = concurrent.futures.Future()
        self._worker = threading.Thread(target=self._build, name="foundry-graph-build", daemon=False)
        self._worker.start()

    def _build(self) -> None:
        """The worker: open, restore and build on a stream of its own (the
        reference's bg thread makes the context current first, 1895-1897)."""
        archive, ggs = None, {}
        try:
            torch.cuda.set_device(self.device)
            stream = torch.cuda.Stream(device=self.device)
            archive = Archive.open(self.json_paths, self.num_threads)
            used = False
            manifest = os.path.join(os.path.dirname(self.json_paths[0]) or ".", "graph_manifest.json")
            if os.path.exists(manifest):
                with open(manifest, "rb") as f:
                    used = archive.set_manifest(f.read(), self.names)
            if len(self.intervals[0]):
                archive.set_relocation(*self.intervals)
            archive.restore(stream)
            template_of = archive.groups(stream)
            for t in sorted(set(int(x) for x in template_of)):
                ggs[t] = GroupGraph(archive, t, registry(), stream)
            stream.synchronize()
        except BaseException as e:  # handed to the finish calls
            for gg in ggs.values():
                gg.close()
            if archive is not None:
                archive.close()
            self.build_complete.set_exception(e)
            return
        self._archive, self._template_of, self._used_manifest, self._group_graphs = archive, template_of, used, ggs
        self.build_complete.set_result(None)

    def wait(self) -> None:
        """Wait for the background build; raises its error."""
        self.build_complete.result()

    @property
    def archive(self) -> Archive:
        self.wait()
        return self._archive

    @property
    def template_of(self) -> np.ndarray:
        self.wait()
        return self._template_of

    @property
    def used_manifest(self) -> bool:
        self.wait()
        return self._used_manifest

    @property
    def group_graphs(self) -> dict:
        self.wait()
        return self._group_graphs

    def group_graph(self, index: int) -> GroupGraph:
        return self.group_graphs[int(self.template_of[index])]

    def close(self) -> None:
        self._worker.join()
        for gg in self._group_graphs.values():
            gg.close()
        self._group_graphs = {}
        if self._archive is not None:
            self._archive.close()
            self._archive = None


class CUDAGraph:
    """A restored graph (csrc/CUDAGraph.cpp).  Graphs of one topology group
    share their group's exec; replay() makes it run this graph's params."""

    def __init__(self, keep_graph: bool = False):
        self.keep_graph = keep_graph
        self._pending: PendingGraphLoads | None = None
        self._index = -1
        # generator state -> wholegraph increment (captured_generator_states_)
        self._generators: dict[GeneratorState, int] = {}

    @classmethod
    def _restored(cls, pending: PendingGraphLoads, index: int) -> "CUDAGraph":
        g = cls()
        g._pending = pending
        g._index = index
        return g

    # capture and SAVE are out of scope
    def capture_begin(self, pool=None, capture_error_mode: str = "global") -> None:
        raise NotImplementedError("graph capture is not part of this build (LOAD path only)")

    def capture_end(self) -> None:
        raise NotImplementedError("graph capture is not part of this build (LOAD path only)")

    def save(self, json_path: str, output_tensors=None) -> None:
        raise NotImplementedError("SAVE is not part of this build (LOAD path only)")

    def replay(self) -> None:
        """csrc/CUDAGraph.cpp:330-483: switch the group's exec to this graph
        (only the nodes that differ are re-set), then launch on the current
        stream."""
        if self._pending is None:
            raise RuntimeError("replay: this CUDAGraph holds no restored graph")
        gg = self._pending.group_graph(self._index)
        stream = torch.cuda.current_stream()
        gg.select(self._index, stream)
        for state, increment in self._generators.items():  # 469-472
            state.replay_prologue(increment)
        gg.launch(stream)

    def reset(self) -> None:
        for state in self._generators:
            state.unregister_graph(self)
        self._generators = {}
        self._pending = None
        self._index = -1

    def register_generator_state(self, state, wholegraph_increment: int = 0) -> None:
        """csrc/CUDAGraph.cpp:185-194: run `state`'s replay prologue with this
        increment before every replay.  A torch.Generator (the capture-side
        overload) is refused: capture is not part of this build."""
        if not isinstance(state, GeneratorState):
            raise NotImplementedError("registering a torch generator is part of capture, which this build "
                                      "does not provide (LOAD path only)")
        state.register_graph(self)
        self._generators[state] = int(wholegraph_increment)

    def _group(self) -> GroupGraph:
        if self._pending is None:
            raise RuntimeError("this CUDAGraph holds no restored graph")
        return self._pending.group_graph(self._index)

    def pool(self):
        """csrc/CUDAGraph.cpp:611-614: the graph's memory pool id.  Restored
        graphs allocate nothing through a pool of their own, so this is the
        pool the load was given (or the default (0, 0))."""
        if self._pending is None:
            raise RuntimeError("Called CUDAGraph::pool() without a preceding successful capture.")
        return self._pending.pool

    def enable_debug_mode(self) -> None:
        self._debug = True

    def debug_dump(self, debug_path: str) -> None:
        """csrc/CUDAGraph.cpp:515-532: write the graph as DOT (the group's
        hipGraph, which this graph's params are selected into first) when
        debug mode or keep_graph is on; otherwise warn, as the reference does."""
        if not (getattr(self, "_debug", False) or self.keep_graph):
            warnings.warn("CUDA Graphs debug not enabled, set with [graph].enable_debug_mode()")
            return
        gg = self._group()
        gg.select(self._index, torch.cuda.current_stream())
        gg.debug_dot(debug_path)

    def raw_cuda_graph(self) -> int:
        """csrc/CUDAGraph.cpp:537-544: the hipGraph_t (the topology group's, shared
        by its members) as an integer; like the reference, only with keep_graph."""
        if not self.keep_graph:
            raise RuntimeError("You cannot access the raw cudaGraph_t instance unless CUDAGraph was initialized "
                               "with keep_graph=true")
        return self._group().handles()[0]

    def raw_cuda_graph_exec(self) -> int:
        """csrc/CUDAGraph.cpp:546-551: the hipGraphExec_t (the topology group's,
        shared by its members; replay() selects this graph's params into it)."""
        return self._group().handles()[1]

    @property
    def index(self) -> int:
        return self._index

    # ---- split load -------------------------------------------------------
    @staticmethod
    def start_graph_builds(json_paths: Sequence[str], pool=None, num_threads: int = 4) -> PendingGraphLoads:
        """Start opening and restoring every archive on the GPU and building
        one exec per topology group (csrc/CUDAGraphParallel.cpp:1543-2015),
        and return while that runs on a worker thread: the caller goes on
        with its own initialisation, and the finish calls wait for the
        build.  A graph_manifest.json beside the first path groups the
        graphs; without it, graphs group by their saved topology keys.  Open,
        restore and build errors are raised by the finish calls."""
        if not json_paths:
            raise RuntimeError("start_graph_builds: no graphs given")
        torch.cuda.synchronize()
        return PendingGraphLoads(json_paths, num_threads, pool)

    @staticmethod
    def finish_one_graph_load(pending: PendingGraphLoads, index: int):
        """csrc/CUDAGraphParallel.cpp:2034-2069: register graph `index`'s
        saved generator states, replay its allocator events into the region
        (in SAVE order), then rebuild its output tensors.  Raises IndexError
        out of range, as the reference's std::out_of_range does through
        pybind."""
        pending.wait()
        if index < 0 or index >= len(pending.graphs):
            raise IndexError(f"finish_one_graph_load: index {index} out of range "
                             f"(num_graphs={len(pending.graphs)})")
        if not pending.finished[index]:
            # Deferred generators first, so that their words land where SAVE
            # put them (2048-2059).
            graph = pending.graphs[index]
            for state_id, seed, increment in generators_of(pending.archive.section(index, SEC_GENERATORS)):
                graph.register_generator_state(global_generator_state_registry.get_state_from_id(state_id, seed),
                                               increment)
            events = pending.archive.section(index, SEC_ALLOC_EVENTS)
            r = _region()
            if events and r is not None:
                r.replay(events)
            pending.outputs[index] = _outputs_from(pending.archive.section(index, SEC_OUTPUT_TENSORS),
                                                   pending.intervals)
            pending.finished[index] = True
        return pending.graphs[index], pending.outputs[index]

    @staticmethod
    def finish_graph_loads(pending: PendingGraphLoads):
        """csrc/CUDAGraphParallel.cpp:2071-2099: wait for the background
        build (raising its error), then finish every graph in index order."""
        pending.wait()
        return [CUDAGraph.finish_one_graph_load(pending, i) for i in range(len(pending.graphs))]

    @staticmethod
    def load(json_path: str, pool=None):
        """One graph: (graph, outputs or None) (csrc/CUDAGraph.cpp:1520-1560)."""
        pending = CUDAGraph.start_graph_builds([json_path], pool, 1)
        return CUDAGraph.finish_one_graph_load(pending, 0)


# The names csrc/binding.cpp binds (a star import of this module gives these).
__all__ = [
    "CUDAGraph",
    "GeneratorState",
    "GeneratorStateRegistry",
    "PendingGraphLoads",
    "free_preallocated_region",
    "get_current_alloc_offset",
    "get_graph_ptr",
    "graph_pool_handle",
    "init_nvshmem_for_loaded_modules",
    "load_cuda_modules_and_libraries",
    "pack_fatbins_to_folder",
    "preallocate_cublas_workspaces",
    "preallocate_region",
    "resume_allocation_region",
    "set_allocation_region",
    "set_current_alloc_offset",
    "set_nvshmem_auto_init",
    "set_pack_fatbins_on_exit",
    "set_skip_fatbin_processing",
    "stop_allocation_region",
]
