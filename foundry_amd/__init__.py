"""MI355X-native graph-restore (LOAD) data path.

The product is libfoundry_restore.so (hand-written HIP kernels for gfx950
behind the C ABI in include/foundry_restore.h, foundry_graph.h and
foundry_region.h).  This package binds it:

  foundry_amd.restore  Archive / RelocPlan: one method per restore entry point
  foundry_amd.graph    Registry / GroupGraph: code objects, one hipGraph per topology group
  foundry_amd.region   Region: the deterministic VMM allocation region
  foundry_amd.ops      the reference's foundry.ops LOAD surface (CUDAGraph.start_graph_builds /
                       finish_graph_loads / finish_one_graph_load / load / replay, region functions)
  foundry_amd.api      the reference's `foundry` package names, also reachable from here
  foundry_amd.synth    seeded synthetic .cugraph archives

The `foundry` names (CUDAGraph, allocation_region, save_graph_manifest, ...)
load torch on first use.
"""
from ._lib import FoundryError  # noqa: F401

_API_NAMES = {
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
}


def __getattr__(name):
    if name in _API_NAMES:
        from . import api

        return getattr(api, name)
    raise AttributeError(f"module 'foundry_amd' has no attribute {name!r}")


__all__ = ["FoundryError", *sorted(_API_NAMES)]
