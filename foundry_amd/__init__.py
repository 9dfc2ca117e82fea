"""MI355X-native graph-restore (LOAD) data path.

The product is libfoundry_restore.so (hand-written HIP kernels for gfx950
behind the C ABI in include/foundry_restore.h).  This package binds it:

  foundry_amd.restore  Archive / RelocPlan: one method per C entry point
  foundry_amd.ops      the reference's foundry.ops CUDAGraph surface
                       (start_graph_builds / finish_graph_loads /
                       finish_one_graph_load / replay) on top of it
  foundry_amd.synth    seeded synthetic .cugraph archives
"""
from ._lib import FoundryError  # noqa: F401

__all__ = ["FoundryError"]
