// foundry/CUDAGraph.h -- the C++ LOAD surface of the reference's CUDAGraph
// (include/CUDAGraph.h:43-247, include/CUDAGraphInternal.h:13-28,
// include/hook.h:27-50) for MI355X, built against PyTorch's C++ headers over
// this library's C-ABI (foundry_restore.h, foundry_graph.h, foundry_region.h).
//
//   GraphLoadResult, OutputTensors, OutputTensorType   as in the reference
//   CUDAGraph::start_graph_builds / finish_graph_loads / finish_one_graph_load / load
//   CUDAGraph::replay / reset / pool / debug_dump / raw_cuda_graph(_exec)
//   the per-thread allocation region and the code-object registry
//
// Loading restores every archive on the GPU in one pass, builds one hipGraph
// exec per topology group, and shares it among the group's graphs (the
// reference's SharedGraphExec); replay() switches the exec to the graph and
// launches it on the current HIP stream.  start_graph_builds returns while a
// worker thread does that work; the finish calls wait for it.  Capture and
// SAVE are not part of this library.  Errors throw c10::Error (TORCH_CHECK),
// an index out of range std::out_of_range, as in the reference.
#pragma once

#include <ATen/Tensor.h>
#include <ATen/core/Generator.h>
#include <ATen/hip/HIPGeneratorImpl.h>  // at::CUDAGeneratorState (the ROCm build's header for it)
#include <c10/core/Allocator.h>
#include <c10/util/intrusive_ptr.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <future>
#include <memory>
#include <string>
#include <utility>
#include <variant>
#include <vector>

namespace foundry {

using MempoolId_t = c10::MempoolId_t;

enum class OutputTensorType { None, Single, List, Tuple };

using OutputTensors = std::variant<std::monostate, at::Tensor, std::vector<at::Tensor>>;

struct CUDAGraph;
struct PendingGraphLoads;

struct GraphLoadResult {
  std::shared_ptr<CUDAGraph> graph;
  OutputTensors outputs;
  OutputTensorType output_type;
};

// A fresh pool id (the reference's graph_pool_handle): restored graphs
// allocate nothing through it; it is carried for the caller.
MempoolId_t graph_pool_handle();

// ---- allocation region, per thread (csrc/hook.cpp:3088-3275) ----------------
// Reserve the region at `base` (rounded up to 2 MiB, as is `size`).  Where
// the device cannot map it there it is placed elsewhere, and graphs loaded
// afterwards are relocated by the move.
void set_allocation_region(uint64_t base, uint64_t size);
void stop_allocation_region();
void resume_allocation_region();
bool preallocate_region(uint64_t size);
void free_preallocated_region();
uint64_t get_current_alloc_offset();
void set_current_alloc_offset(uint64_t offset);
// Not in the reference (whose region lives as long as the process and whose
// interposed cuMemAlloc places every allocation): an allocation placed by
// the region's cursor rule, and the release of this thread's region.
uint64_t region_alloc(uint64_t bytes);
void release_allocation_region();

// ---- code objects (csrc/hook.cpp:1589-1700, 3787-3830) ----------------------
// Register the packed pair in `dir` (or, without one, every loose *.co /
// *.hsaco) in the process registry; returns the number registered.
int load_cuda_modules_and_libraries(const std::string& dir);
// Write the registry's code objects into the packed pair in `dir`.
void pack_fatbins_to_folder(const std::string& dir);

// ---- BLAS handles (csrc/CUDAGraph.cpp:165-174) --------------------------------
// Create the current stream's hipBLAS and hipBLASLt handles and the hipBLASLt
// workspace (through torch) before graphs that use them are loaded, so that
// they are not allocated inside the graphs' region later.
void preallocate_cublas_workspaces();

// ---- generator state (csrc/CUDAGraph.cpp:35-97, 133-160) ---------------------
// A restored graph's random kernels read torch's graph-safe Philox seed and
// offset words, seed_extragraph_ and offset_extragraph_ of an
// at::CUDAGeneratorState.  When the first graph registers a state, the two
// words are one 2 MiB segment (an allocation of this thread's region when one
// is enabled, else a torch tensor), seed at +0 and offset at +512, where
// torch's caching allocator puts two one-element tensors in a fresh segment;
// they are released when the last graph unregisters.
struct CUDAGeneratorStateRegistry {
  // The id a state is known under: the id get_state_from_id made it for, else
  // a new one (query_state_id, csrc/CUDAGraph.cpp:133-145).
  uint64_t query_state_id(at::CUDAGeneratorState* state);
  // The state saved under `id`; a new id makes one of `seed` and offset 0
  // (get_state_from_id, csrc/CUDAGraph.cpp:147-160).
  c10::intrusive_ptr<at::CUDAGeneratorState> get_state_from_id(uint64_t id, uint64_t seed);
  struct Impl;
  std::shared_ptr<Impl> impl_;
};

CUDAGeneratorStateRegistry& global_generator_state_registry();

namespace detail {
struct Group;  // one topology group's hipGraph exec, shared by its graphs
}

struct CUDAGraph {
  explicit CUDAGraph(bool keep_graph = false);
  ~CUDAGraph();

  // Run `state`'s replay prologue with this increment before every replay:
  // seed and offset written on the current stream, then the offset advanced
  // by the increment rounded up to a multiple of 4 (csrc/CUDAGraph.cpp:
  // 60-86, 185-194).  The one-argument form registers with increment 0.
  void register_generator_state(c10::intrusive_ptr<at::CUDAGeneratorState> state, uint64_t wholegraph_increment);
  void register_generator_state(c10::intrusive_ptr<at::CUDAGeneratorState> state);
  // A torch generator is registered while capturing (csrc/CUDAGraph.cpp:
  // 180-183); capture is not part of this library, so this throws.
  void register_generator_state(const at::Generator& generator);
  // Switch the group's exec to this graph (only nodes that differ are
  // re-set), run the generator prologues, launch on the current stream
  // (csrc/CUDAGraph.cpp:330-483).
  void replay();
  void reset();
  MempoolId_t pool();
  void enable_debug_mode();
  void debug_dump(const std::string& debug_path);
  hipGraph_t raw_cuda_graph();
  hipGraphExec_t raw_cuda_graph_exec();
  // Index of this graph in the load that made it (-1 if none).
  int64_t index() const { return index_; }

  static GraphLoadResult load(const std::string& json_path, MempoolId_t pool = {0, 0});
  static std::shared_ptr<PendingGraphLoads> start_graph_builds(const std::vector<std::string>& json_paths,
                                                               MempoolId_t pool = {0, 0}, int num_threads = 4);
  static std::vector<GraphLoadResult> finish_graph_loads(std::shared_ptr<PendingGraphLoads> pending);
  static GraphLoadResult finish_one_graph_load(std::shared_ptr<PendingGraphLoads> pending, size_t index);

 private:
  friend struct PendingGraphLoads;
  bool keep_graph_ = false;
  bool debug_ = false;
  int64_t index_ = -1;
  MempoolId_t pool_{0, 0};
  std::shared_ptr<detail::Group> group_;
  std::vector<std::pair<c10::intrusive_ptr<at::CUDAGeneratorState>, uint64_t>> generators_;
};

// The split-load state (include/CUDAGraphInternal.h:13-28).  The graphs exist
// when start_graph_builds returns; the rest is filled in by the worker thread,
// whose completion (or error) build_complete_ carries.
struct PendingGraphLoads {
  std::vector<std::shared_ptr<CUDAGraph>> graphs;
  MempoolId_t pool{0, 0};
  c10::DeviceIndex dev = 0;
  CUDAGeneratorStateRegistry* registry = nullptr;  // for the deferred generator registration
  std::shared_future<void> build_complete_;
  // Valid once build_complete_ is ready (after a finish call has returned).
  std::vector<uint32_t> template_of;  // per graph: its topology group's template
  bool used_manifest = false;
  struct Impl;
  std::shared_ptr<Impl> impl;
  ~PendingGraphLoads();  // waits for the worker
};

}  // namespace foundry
