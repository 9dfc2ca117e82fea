"""The reference's `foundry` package names (python/foundry/__init__.py:3-32)
over the MI355X restore path: CUDAGraph with its static LOAD methods, the
allocation-region helpers, and save_graph_manifest."""
from __future__ import annotations

import json
import os
import re
import struct
import sys
from contextlib import contextmanager

from . import ops
from .ops import (  # noqa: F401  (re-exported)
    free_preallocated_region,
    get_current_alloc_offset,
    load_cuda_modules_and_libraries,
    preallocate_region,
    resume_allocation_region,
    set_allocation_region,
    set_current_alloc_offset,
    stop_allocation_region,
)


class CUDAGraph(ops.CUDAGraph):
    """python/foundry/graph.py:19-123: load() returns the graph alone when it
    has no saved outputs, else (graph, outputs)."""

    @staticmethod
    def load(json_path: str, pool=None):
        g, out = ops.CUDAGraph.load(json_path, pool)
        return g if out is None else (g, out)


class graph:
    """The capture context manager (python/foundry/graph.py:126-167).  Capture
    is not part of this build; entering raises NotImplementedError."""

    default_capture_stream = None

    def __init__(self, cuda_graph, pool=None, stream=None, capture_error_mode: str = "global"):
        self.cuda_graph = cuda_graph

    def __enter__(self):
        raise NotImplementedError("graph capture is not part of this build (LOAD path only)")

    def __exit__(self, *args):
        return False


def parse_size(size) -> int:
    """python/foundry/allocation_region.py:30-58: int, or '<n>[B|KB|MB|GB|TB]'."""
    if isinstance(size, int):
        return size
    m = re.match(r"^(\d+(?:\.\d+)?)\s*(B|KB|MB|GB|TB)?$", size.strip().upper())
    if not m:
        raise ValueError(f"Invalid size format: {size}. Expected format like '1GB', '16MB', '24KB', or integer bytes")
    mult = {"B": 1, "KB": 1 << 10, "MB": 1 << 20, "GB": 1 << 30, "TB": 1 << 40}[m.group(2) or "B"]
    return int(float(m.group(1)) * mult)


@contextmanager
def allocation_region(base, size, prealloc_size=None):
    """python/foundry/allocation_region.py:66-109."""
    base_addr = (int(base, 16) if base.lower().startswith("0x") else int(base)) if isinstance(base, str) else base
    set_allocation_region(base_addr, parse_size(size))
    try:
        if prealloc_size is not None:
            n = parse_size(prealloc_size)
            if not preallocate_region(n):
                raise RuntimeError(f"Failed to preallocate {n} bytes")
        yield
    finally:
        if prealloc_size is not None:
            free_preallocated_region()
        stop_allocation_region()


_GRAPH_FILE = re.compile(r"^graph_(\d+)(?:_.*)?\.(json|cugraph)$")


def _cugraph_key(path: str) -> str:
    """The TOPOLOGY_KEY section of a .cugraph archive (include/BinaryGraphFormat.h:274-278)."""
    with open(path, "rb") as f:
        head = f.read(64 + 11 * 24)
        if len(head) < 64 or head[:8] != b"CUGRAPH\0":
            raise ValueError(f"{path}: not a .cugraph archive")
        num_sections = struct.unpack_from("<I", head, 28)[0]
        for i in range(min(num_sections, 11)):
            sid, _pad, off, size = struct.unpack_from("<IIQQ", head, 64 + 24 * i)
            if sid == 10:
                f.seek(off)
                return f.read(size).decode()
    return ""


def save_graph_manifest(archive_dir: str) -> None:
    """python/foundry/graph.py:170-242: group the saved graphs by topology
    key in capture order, the first of each group as its template, write
    graph_manifest.json, and strip `dependencies` from the JSON of graphs
    that are not templates.  Graphs are graph_<n>[_...].json files, or
    .cugraph archives (whose key section supplies the key); manifest entries
    name the .json file either way, as LOAD looks graphs up by that name."""
    stems = {}
    for f in os.listdir(archive_dir):
        m = _GRAPH_FILE.match(f)
        if m:
            stems.setdefault(f.rsplit(".", 1)[0], int(m.group(1)))
    if not stems:
        return
    order = sorted(stems, key=lambda s: stems[s])
    keys: dict[str, list[str]] = {}
    for stem in order:
        jpath = os.path.join(archive_dir, stem + ".json")
        if os.path.exists(jpath):
            with open(jpath) as f:
                key = json.load(f).get("topology_key", "")
        else:
            key = _cugraph_key(os.path.join(archive_dir, stem + ".cugraph"))
        if not key:
            return  # as the reference: no manifest without every key
        keys.setdefault(key, []).append(stem + ".json")
    groups, templates = [], set()
    for key, names in keys.items():
        groups.append({"topology_key": key, "template": names[0], "members": names})
        templates.add(names[0])
    with open(os.path.join(archive_dir, "graph_manifest.json"), "w") as f:
        json.dump({"topology_groups": groups}, f, indent=2)
    stripped = 0
    for stem in order:
        name = stem + ".json"
        jpath = os.path.join(archive_dir, name)
        if name in templates or not os.path.exists(jpath):
            continue
        with open(jpath) as f:
            data = json.load(f)
        if "dependencies" in data:
            del data["dependencies"]
            with open(jpath, "w") as f:
                json.dump(data, f)
            stripped += 1
    on_demand = sum(len(g["members"]) - 1 for g in groups)
    print(f"[foundry] Saved graph_manifest.json: {len(groups)} topology groups ({len(groups)} templates, "
          f"{on_demand} on-demand, {stripped} stripped)", file=sys.stderr)


def install_as_foundry() -> None:
    """Register this build under the reference's module names, so code that
    imports `foundry`, `foundry.graph`, `foundry.ops` or
    `foundry.allocation_region` (the vLLM and SGLang integrations do:
    python/foundry/integration/vllm/graph_ops.py:36) runs on it unchanged.

    `foundry` is assembled as python/foundry/__init__.py:3-17 assembles it:
    the allocation-region helpers, then CUDAGraph / graph /
    save_graph_manifest from `foundry.graph`, then every name of `foundry.ops`
    -- which, coming last, leaves `foundry.CUDAGraph` naming the ops class
    while `foundry.graph.CUDAGraph` is the subclass whose load() returns the
    graph alone when it has no outputs.  Refused if another `foundry` is
    already imported."""
    import types

    current = sys.modules.get("foundry")
    if current is not None and not getattr(current, "__foundry_amd__", False):
        raise RuntimeError("a different `foundry` package is already imported")
    region = types.ModuleType("foundry.allocation_region")
    for name in ("allocation_region", "free_preallocated_region", "get_current_alloc_offset", "parse_size",
                 "preallocate_region", "resume_allocation_region", "set_current_alloc_offset",
                 "set_allocation_region", "stop_allocation_region"):
        setattr(region, name, globals()[name])
    gmod = types.ModuleType("foundry.graph")
    for name in ("CUDAGraph", "graph", "save_graph_manifest"):
        setattr(gmod, name, globals()[name])
    pkg = types.ModuleType("foundry", "The reference's `foundry` package names, on the MI355X restore path.")
    pkg.__path__ = []
    pkg.__foundry_amd__ = True
    for mod in (region, gmod):
        for name, value in vars(mod).items():
            if not name.startswith("_"):
                setattr(pkg, name, value)
    for name in ops.__all__:
        setattr(pkg, name, getattr(ops, name))
    pkg.__all__ = ["CUDAGraph", "allocation_region", "free_preallocated_region", "get_current_alloc_offset",
                   "graph", "parse_size", "preallocate_region", "resume_allocation_region", "save_graph_manifest",
                   "set_current_alloc_offset"]
    pkg.ops = ops
    sys.modules.update({"foundry": pkg, "foundry.graph": gmod, "foundry.ops": ops,
                        "foundry.allocation_region": region})


__all__ = [
    "CUDAGraph",
    "allocation_region",
    "free_preallocated_region",
    "get_current_alloc_offset",
    "graph",
    "install_as_foundry",
    "load_cuda_modules_and_libraries",
    "parse_size",
    "preallocate_region",
    "resume_allocation_region",
    "save_graph_manifest",
    "set_allocation_region",
    "set_current_alloc_offset",
    "stop_allocation_region",
]
