// cudagraph.cpp -- include/foundry/CUDAGraph.h over the C-ABI: the
// reference's C++ LOAD surface (include/CUDAGraph.h:43-247,
// include/CUDAGraphInternal.h:13-28; csrc/CUDAGraphParallel.cpp:1543-2099,
// csrc/CUDAGraph.cpp:330-483) for MI355X.
//
// Ownership follows the reference's: the caller holds PendingGraphLoads and
// the graphs as shared_ptr; a topology group's exec (detail::Group, the
// reference's SharedGraphExec) is owned jointly by its graphs and the
// pending loads, and holds the archive, which is closed after the last
// group is destroyed.
#include "../../include/foundry/CUDAGraph.h"

#include <ATen/ATen.h>
#include <ATen/hip/HIPContextLight.h>
#include <c10/hip/HIPStream.h>
#include <c10/util/Exception.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <map>
#include <mutex>
#include <set>
#include <sstream>
#include <stdexcept>
#include <thread>

#include "../../include/fdy_format.h"
#include "../../include/foundry_graph.h"
#include "../../include/foundry_region.h"
#include "../../include/foundry_restore.h"
#include "json_min.h"

namespace foundry {
namespace {

constexpr uint64_t kMiB = 1ull << 20;
constexpr uint64_t kRegionAlign = 2 * kMiB;

void check(int rc, const char* what) {
  TORCH_CHECK(rc == FDY_OK, what, ": ", fdy_last_error());
}

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// Regions alive in this process: memory placed in a region for a generator
// state is freed by its tensor's deleter only while the region exists.
std::mutex g_live_mu;
std::set<fdy_region*> g_live_regions;

void destroy_region(fdy_region* r) {
  {
    std::lock_guard<std::mutex> lk(g_live_mu);
    g_live_regions.erase(r);
  }
  fdy_region_destroy(r);
}

void free_in_region(fdy_region* r, uint64_t p) {
  std::lock_guard<std::mutex> lk(g_live_mu);
  if (g_live_regions.count(r)) (void)fdy_region_free(r, p);
}

// The allocation region of this thread (the reference keeps it per thread,
// csrc/hook.cpp:218-251).
struct RegionState {
  fdy_region* r = nullptr;
  bool enabled = false;
  ~RegionState() {
    if (r) destroy_region(r);
  }
};
thread_local RegionState t_region;

bool region_enabled() { return t_region.r && t_region.enabled; }

fdy_region_info region_info() {
  fdy_region_info i{};
  check(fdy_region_info_get(t_region.r, &i), "fdy_region_info_get");
  return i;
}

// The process code-object registry, created on first use on the current device.
std::mutex g_registry_mu;
fdy_registry* g_registry = nullptr;

fdy_registry* registry() {
  std::lock_guard<std::mutex> lk(g_registry_mu);
  if (!g_registry) check(fdy_registry_create(&g_registry), "fdy_registry_create");
  return g_registry;
}

hipStream_t current_stream() { return c10::hip::getCurrentHIPStream().stream(); }

std::string basename_of(const std::string& p) {
  const size_t s = p.find_last_of('/');
  return s == std::string::npos ? p : p.substr(s + 1);
}

std::string dirname_of(const std::string& p) {
  const size_t s = p.find_last_of('/');
  return s == std::string::npos ? std::string(".") : p.substr(0, s);
}

bool read_file(const std::string& path, std::string* out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::ostringstream ss;
  ss << f.rdbuf();
  *out = ss.str();
  return true;
}

uint64_t json_u64(const fdy::json::Value* v, const char* what) {
  TORCH_CHECK(v && v->kind == fdy::json::Value::Number && v->num != fdy::json::Value::Double, "output_tensors: ",
              what, " is not an integer");
  return v->num == fdy::json::Value::Uint ? v->u : (uint64_t)v->i;
}

int64_t json_i64(const fdy::json::Value* v, const char* what) {
  TORCH_CHECK(v && v->kind == fdy::json::Value::Number && v->num == fdy::json::Value::Int, "output_tensors: ",
              what, " is not a signed 64-bit integer");
  return v->i;
}

}  // namespace

namespace detail {

// The archive of one load, closed once the last group using it is gone.
struct Archive {
  fdy_archive* a = nullptr;
  ~Archive() {
    if (a) fdy_archive_close(a);
  }
};

struct Group {
  std::shared_ptr<Archive> archive;
  fdy_group_graph* gg = nullptr;
  ~Group() {
    if (gg) fdy_group_graph_destroy(gg);
  }
};

}  // namespace detail

struct PendingGraphLoads::Impl {
  std::shared_ptr<detail::Archive> archive;
  std::map<uint32_t, std::shared_ptr<detail::Group>> groups;  // by template index
  std::vector<uint64_t> iv_lo, iv_hi, iv_new;  // relocation intervals (empty: none)
  std::vector<bool> finished;
  std::vector<GraphLoadResult> results;
  std::thread worker;  // the background build; joined by ~PendingGraphLoads

  // Point each graph at its group's exec (the reference's
  // link_on_demand_shared_exec, csrc/CUDAGraphParallel.cpp:1998-2004).
  static void link(PendingGraphLoads* p, const std::vector<uint32_t>& template_of) {
    for (size_t i = 0; i < template_of.size(); ++i) p->graphs[i]->group_ = p->impl->groups.at(template_of[i]);
  }

  std::string section(uint32_t g, uint32_t sec) {
    uint64_t n = 0;
    int rc = fdy_get_section(archive->a, g, sec, nullptr, 0, &n);
    if (rc != FDY_OK && rc != FDY_E_CAPACITY) check(rc, "fdy_get_section");
    std::string s(n, '\0');
    if (n) check(fdy_get_section(archive->a, g, sec, reinterpret_cast<uint8_t*>(&s[0]), n, &n), "fdy_get_section");
    s.resize(n);
    return s;
  }

  uint64_t relocate(uint64_t p) const {
    auto it = std::upper_bound(iv_lo.begin(), iv_lo.end(), p);
    if (it == iv_lo.begin()) return p;
    const size_t i = (size_t)(it - iv_lo.begin()) - 1;
    return p < iv_hi[i] ? p - iv_lo[i] + iv_new[i] : p;
  }
};

// ---- pool, region, code objects ------------------------------------------------

MempoolId_t graph_pool_handle() {
  static std::atomic<uint64_t> next{1};
  return {0, next.fetch_add(1)};
}

void set_allocation_region(uint64_t base, uint64_t size) {
  if (t_region.r) {
    destroy_region(t_region.r);
    t_region.r = nullptr;
  }
  fdy_region* r = nullptr;
  check(fdy_region_create(align_up(base, kRegionAlign), align_up(size, kRegionAlign), 0, 0, &r),
        "set_allocation_region");
  {
    std::lock_guard<std::mutex> lk(g_live_mu);
    g_live_regions.insert(r);
  }
  t_region.r = r;
  t_region.enabled = true;
}

void release_allocation_region() {
  if (t_region.r) destroy_region(t_region.r);
  t_region.r = nullptr;
  t_region.enabled = false;
}

void stop_allocation_region() { t_region.enabled = false; }
void resume_allocation_region() { t_region.enabled = true; }

bool preallocate_region(uint64_t size) {
  return t_region.r && fdy_region_preallocate(t_region.r, size) == FDY_OK;
}

void free_preallocated_region() {
  if (t_region.r) check(fdy_region_free_preallocated(t_region.r), "free_preallocated_region");
}

uint64_t get_current_alloc_offset() {
  uint64_t off = 0;
  if (t_region.r) check(fdy_region_get_offset(t_region.r, &off), "get_current_alloc_offset");
  return off;
}

void set_current_alloc_offset(uint64_t offset) {
  TORCH_CHECK(t_region.r, "set_current_alloc_offset: no allocation region is set");
  check(fdy_region_set_offset(t_region.r, offset), "set_current_alloc_offset");
}

uint64_t region_alloc(uint64_t bytes) {
  TORCH_CHECK(region_enabled(), "region_alloc: no enabled allocation region");
  uint64_t p = 0;
  check(fdy_region_alloc(t_region.r, bytes, &p), "region_alloc");
  return p;
}

int load_cuda_modules_and_libraries(const std::string& dir) {
  namespace fs = std::filesystem;
  uint32_t n = 0;
  std::error_code ec;
  if (fs::exists(fs::path(dir) / "fatbin_image_packed.img", ec) &&
      fs::exists(fs::path(dir) / "fatbin_entrypoint_packed.txt", ec)) {
    check(fdy_registry_load_packed(registry(), dir.c_str(), &n), "load_cuda_modules_and_libraries");
    return (int)n;
  }
  // Loose code objects, in name order.
  std::vector<std::string> names;
  for (fs::directory_iterator it(dir, ec), end; !ec && it != end; it.increment(ec)) {
    if (!it->is_regular_file(ec)) continue;
    const std::string nm = it->path().filename().string();
    auto ends = [&](const char* suf) {
      const size_t k = std::strlen(suf);
      return nm.size() > k && nm.compare(nm.size() - k, k, suf) == 0;
    };
    if (ends(".co") || ends(".hsaco")) names.push_back(nm);
  }
  std::sort(names.begin(), names.end());
  TORCH_CHECK(!names.empty(), "no packed code objects (fatbin_image_packed.img + fatbin_entrypoint_packed.txt) and no ",
              "*.co / *.hsaco in ", dir);
  for (const auto& nm : names) {
    uint64_t h = 0;
    check(fdy_registry_add_file(registry(), (dir + "/" + nm).c_str(), &h), "load_cuda_modules_and_libraries");
  }
  return (int)names.size();
}

void pack_fatbins_to_folder(const std::string& dir) {
  uint32_t n = 0;
  check(fdy_registry_pack(registry(), dir.c_str(), &n), "pack_fatbins_to_folder");
}

void preallocate_cublas_workspaces() {
  at::globalContext().lazyInitDevice(at::kCUDA);  // torch's device allocator, as its tensor factories do first
  TORCH_CHECK(at::cuda::getCurrentCUDABlasHandle() != nullptr, "Failed to get the hipBLAS handle");
  TORCH_CHECK(at::cuda::getCurrentCUDABlasLtHandle() != nullptr, "Failed to get the hipBLASLt handle");
  TORCH_CHECK(at::cuda::getCUDABlasLtWorkspace() != nullptr, "Failed to allocate the hipBLASLt workspace");
}

// ---- generator state -------------------------------------------------------------

namespace {

constexpr uint64_t kGenSegment = 2 * kMiB;
constexpr int64_t kGenOffsetWord = 512 / 8;

// A graph registers `st` (at::CUDAGeneratorState::register_graph as the
// reference overrides it, csrc/CUDAGraph.cpp:35-47): the first registration
// allocates the seed and offset words.
void attach_words(at::CUDAGeneratorState& st, CUDAGraph* graph) {
  if (!st.seed_extragraph_.defined()) {
    const auto opts = at::TensorOptions().dtype(at::kLong).device(at::kCUDA);
    at::Tensor seg;
    if (region_enabled()) {
      const uint64_t p = region_alloc(kGenSegment);
      fdy_region* r = t_region.r;
      seg = at::from_blob(reinterpret_cast<void*>(p), {(int64_t)(kGenSegment / 8)},
                          [r](void* q) { free_in_region(r, reinterpret_cast<uint64_t>(q)); }, opts);
    } else {
      seg = at::empty({(int64_t)(kGenSegment / 8)}, opts);
    }
    st.seed_extragraph_ = seg.narrow(0, 0, 1);
    st.offset_extragraph_ = seg.narrow(0, kGenOffsetWord, 1);
  }
  st.registered_graphs_.insert(reinterpret_cast<at::cuda::CUDAGraph*>(graph));
}

// unregister_graph (csrc/CUDAGraph.cpp:49-59): the last graph releases the words.
void detach_words(at::CUDAGeneratorState& st, CUDAGraph* graph) {
  st.registered_graphs_.erase(reinterpret_cast<at::cuda::CUDAGraph*>(graph));
  if (st.registered_graphs_.empty()) {
    st.seed_extragraph_.reset();
    st.offset_extragraph_.reset();
  }
}

// replay_prologue and increase (csrc/CUDAGraph.cpp:60-86).
void replay_prologue(at::CUDAGeneratorState& st, uint64_t increment) {
  if (!increment) return;
  TORCH_CHECK(st.seed_extragraph_.defined(), "replay_prologue: the generator state is registered with no graph");
  at::Tensor(st.seed_extragraph_).fill_((int64_t)st.seed_);
  at::Tensor(st.offset_extragraph_).fill_((int64_t)st.philox_offset_per_thread_);
  st.philox_offset_per_thread_ += (increment + 3) / 4 * 4;
}

}  // namespace

struct CUDAGeneratorStateRegistry::Impl {
  std::mutex mu;
  uint64_t next_id = 0;
  std::map<at::CUDAGeneratorState*, uint64_t> ids;
  std::map<uint64_t, c10::intrusive_ptr<at::CUDAGeneratorState>> states;
};

uint64_t CUDAGeneratorStateRegistry::query_state_id(at::CUDAGeneratorState* state) {
  if (!impl_) impl_ = std::make_shared<Impl>();
  std::lock_guard<std::mutex> lk(impl_->mu);
  auto it = impl_->ids.find(state);
  if (it != impl_->ids.end()) return it->second;
  const uint64_t id = impl_->next_id++;
  impl_->ids.emplace(state, id);
  return id;
}

c10::intrusive_ptr<at::CUDAGeneratorState> CUDAGeneratorStateRegistry::get_state_from_id(uint64_t id, uint64_t seed) {
  if (!impl_) impl_ = std::make_shared<Impl>();
  std::lock_guard<std::mutex> lk(impl_->mu);
  auto& st = impl_->states[id];
  if (!st) {
    st = c10::make_intrusive<at::CUDAGeneratorState>(seed, 0, 0);
    impl_->ids.emplace(st.get(), id);
  }
  return st;
}

CUDAGeneratorStateRegistry& global_generator_state_registry() {
  static CUDAGeneratorStateRegistry r;
  static std::once_flag once;
  std::call_once(once, [] { r.impl_ = std::make_shared<CUDAGeneratorStateRegistry::Impl>(); });
  return r;
}

// ---- graphs ------------------------------------------------------------------------

CUDAGraph::CUDAGraph(bool keep_graph) : keep_graph_(keep_graph) {}
CUDAGraph::~CUDAGraph() { reset(); }

void CUDAGraph::register_generator_state(c10::intrusive_ptr<at::CUDAGeneratorState> state, uint64_t increment) {
  TORCH_CHECK(state, "register_generator_state: null state");
  attach_words(*state, this);
  for (auto& g : generators_)
    if (g.first == state) {
      g.second = increment;
      return;
    }
  generators_.emplace_back(std::move(state), increment);
}

void CUDAGraph::register_generator_state(c10::intrusive_ptr<at::CUDAGeneratorState> state) {
  TORCH_CHECK(state, "register_generator_state: null state");
  global_generator_state_registry().query_state_id(state.get());
  register_generator_state(std::move(state), 0);
}

void CUDAGraph::register_generator_state(const at::Generator&) {
  TORCH_CHECK(false, "register_generator_state(Generator) registers a generator during capture, which this ",
              "library does not provide (LOAD path only)");
}

void CUDAGraph::replay() {
  TORCH_CHECK(group_, "replay: this CUDAGraph holds no restored graph");
  hipStream_t s = current_stream();
  check(fdy_group_graph_select(group_->gg, (uint32_t)index_, s, nullptr), "replay (select)");
  for (auto& g : generators_) replay_prologue(*g.first, g.second);  // csrc/CUDAGraph.cpp:469-472
  check(fdy_group_graph_launch(group_->gg, s), "replay (launch)");
}

void CUDAGraph::reset() {
  for (auto& g : generators_) detach_words(*g.first, this);
  generators_.clear();
  group_.reset();
  index_ = -1;
}

MempoolId_t CUDAGraph::pool() {
  TORCH_CHECK(group_, "Called CUDAGraph::pool() without a preceding successful capture.");
  return pool_;
}

void CUDAGraph::enable_debug_mode() { debug_ = true; }

void CUDAGraph::debug_dump(const std::string& path) {
  if (!(debug_ || keep_graph_)) {
    TORCH_WARN("CUDA Graphs debug not enabled, set with [graph].enable_debug_mode()");
    return;
  }
  TORCH_CHECK(group_, "debug_dump: this CUDAGraph holds no restored graph");
  check(fdy_group_graph_select(group_->gg, (uint32_t)index_, current_stream(), nullptr), "debug_dump (select)");
  check(fdy_group_graph_debug_dot(group_->gg, path.c_str()), "debug_dump");
}

hipGraph_t CUDAGraph::raw_cuda_graph() {
  TORCH_CHECK(keep_graph_, "You cannot access the raw cudaGraph_t instance unless CUDAGraph was initialized with ",
              "keep_graph=true");
  TORCH_CHECK(group_, "raw_cuda_graph: this CUDAGraph holds no restored graph");
  void *g = nullptr, *e = nullptr;
  check(fdy_group_graph_handles(group_->gg, &g, &e), "raw_cuda_graph");
  return static_cast<hipGraph_t>(g);
}

hipGraphExec_t CUDAGraph::raw_cuda_graph_exec() {
  TORCH_CHECK(group_, "raw_cuda_graph_exec: this CUDAGraph holds no restored graph");
  void *g = nullptr, *e = nullptr;
  check(fdy_group_graph_handles(group_->gg, &g, &e), "raw_cuda_graph_exec");
  return static_cast<hipGraphExec_t>(e);
}

PendingGraphLoads::~PendingGraphLoads() {
  if (impl && impl->worker.joinable()) impl->worker.join();
}

namespace {

// A HIP stream of the worker's own, at the default priority.
struct OwnStream {
  hipStream_t s = nullptr;
  OwnStream() {
    TORCH_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess, "start_graph_builds: ",
                "cannot create a stream");
  }
  ~OwnStream() {
    if (s) (void)hipStreamDestroy(s);
  }
};

// The background build (the reference's Phase 2 thread,
// csrc/CUDAGraphParallel.cpp:1887-2017, with its Phase 1 reads): open the
// archives, group them, restore them on the GPU and build one exec per
// topology group.  Runs on the worker thread; `p` outlives it.
void build_graphs(PendingGraphLoads* p, const std::vector<std::string>& json_paths, int num_threads) {
  auto& impl = *p->impl;
  TORCH_CHECK(hipSetDevice(p->dev) == hipSuccess, "start_graph_builds: cannot make device ", (int)p->dev,
              " current");
  OwnStream stream;
  hipStream_t s = stream.s;
  std::vector<const char*> cpaths;
  for (const auto& path : json_paths) cpaths.push_back(path.c_str());
  check(fdy_archive_open(cpaths.data(), (uint32_t)cpaths.size(), (uint32_t)std::max(1, num_threads),
                         &impl.archive->a),
        "start_graph_builds (open)");
  fdy_archive* a = impl.archive->a;
  const uint32_t G = (uint32_t)json_paths.size();

  // A graph_manifest.json beside the first path groups the graphs
  // (csrc/CUDAGraphParallel.cpp:1720-1786); otherwise the saved keys do.
  std::string manifest;
  bool used_manifest = false;
  if (read_file(dirname_of(json_paths[0]) + "/graph_manifest.json", &manifest)) {
    std::vector<std::string> names;
    for (const auto& path : json_paths) names.push_back(basename_of(path));
    std::vector<const char*> cnames;
    for (const auto& n : names) cnames.push_back(n.c_str());
    int used = 0;
    check(fdy_archive_set_manifest(a, manifest.data(), manifest.size(), cnames.data(), &used),
          "start_graph_builds (manifest)");
    used_manifest = used != 0;
  }
  if (!impl.iv_lo.empty())
    check(fdy_archive_set_relocation(a, impl.iv_lo.data(), impl.iv_hi.data(), impl.iv_new.data(), impl.iv_lo.size(),
                                     FDY_RELOC_HALF_OPEN),
          "start_graph_builds (relocation)");
  check(fdy_restore(a, s), "start_graph_builds (restore)");
  std::vector<uint32_t> template_of(G);
  check(fdy_get_groups(a, s, template_of.data()), "start_graph_builds (groups)");
  for (uint32_t t : template_of) {
    if (impl.groups.count(t)) continue;
    auto grp = std::make_shared<detail::Group>();
    grp->archive = impl.archive;
    check(fdy_group_graph_create(a, t, registry(), s, &grp->gg), "start_graph_builds (group graph)");
    impl.groups.emplace(t, std::move(grp));
  }
  TORCH_CHECK(hipStreamSynchronize(s) == hipSuccess, "start_graph_builds: the restore stream failed");
  PendingGraphLoads::Impl::link(p, template_of);
  p->template_of = std::move(template_of);
  p->used_manifest = used_manifest;
}

}  // namespace

std::shared_ptr<PendingGraphLoads> CUDAGraph::start_graph_builds(const std::vector<std::string>& json_paths,
                                                                 MempoolId_t pool, int num_threads) {
  TORCH_CHECK(!json_paths.empty(), "start_graph_builds: no graphs given");
  TORCH_CHECK(hipDeviceSynchronize() == hipSuccess, "start_graph_builds: device synchronization failed");
  int dev = 0;
  TORCH_CHECK(hipGetDevice(&dev) == hipSuccess, "start_graph_builds: no current device");
  auto pending = std::make_shared<PendingGraphLoads>();
  pending->pool = pool;
  pending->dev = (c10::DeviceIndex)dev;
  pending->registry = &global_generator_state_registry();
  auto impl = std::make_shared<PendingGraphLoads::Impl>();
  pending->impl = impl;
  impl->archive = std::make_shared<detail::Archive>();
  const uint32_t G = (uint32_t)json_paths.size();
  // The graph shells exist at once (Phase 1b, csrc/CUDAGraphParallel.cpp:1622-1718).
  for (uint32_t i = 0; i < G; ++i) {
    auto g = std::make_shared<CUDAGraph>();
    g->index_ = i;
    g->pool_ = pool;
    pending->graphs.push_back(std::move(g));
  }
  impl->finished.assign(G, false);
  impl->results.resize(G);
  // A region placed away from its saved base relocates every saved pointer.
  // The region is this thread's: its interval is read here, for the worker.
  if (t_region.r) {
    const fdy_region_info info = region_info();
    if (info.base != info.saved_base) {
      uint64_t n = 0;
      check(fdy_region_intervals(t_region.r, FDY_REGION_IV_REGION, nullptr, nullptr, nullptr, 0, &n),
            "start_graph_builds (intervals)");
      impl->iv_lo.resize(n);
      impl->iv_hi.resize(n);
      impl->iv_new.resize(n);
      if (n)
        check(fdy_region_intervals(t_region.r, FDY_REGION_IV_REGION, impl->iv_lo.data(), impl->iv_hi.data(),
                                   impl->iv_new.data(), n, &n),
              "start_graph_builds (intervals)");
    }
  }
  // Everything else runs on a worker thread; its error reaches the finish
  // calls through build_complete_ (2010-2015).
  auto done = std::make_shared<std::promise<void>>();
  pending->build_complete_ = done->get_future().share();
  PendingGraphLoads* p = pending.get();
  impl->worker = std::thread([p, json_paths, num_threads, done]() {
    try {
      build_graphs(p, json_paths, num_threads);
      done->set_value();
    } catch (...) {
      done->set_exception(std::current_exception());
    }
  });
  return pending;
}

GraphLoadResult CUDAGraph::finish_one_graph_load(std::shared_ptr<PendingGraphLoads> pending, size_t index) {
  TORCH_CHECK(pending && pending->impl, "finish_one_graph_load: no pending loads");
  auto& impl = *pending->impl;
  // Wait for the background build, and raise its error (2034-2038 waits
  // without raising; get() keeps the error).
  if (pending->build_complete_.valid()) pending->build_complete_.get();
  if (index >= pending->graphs.size())
    throw std::out_of_range("finish_one_graph_load: index " + std::to_string(index) +
                            " out of range (num_graphs=" + std::to_string(pending->graphs.size()) + ")");
  if (impl.finished[index]) return impl.results[index];
  const uint32_t g = (uint32_t)index;
  auto& graph = pending->graphs[index];
  // Deferred generators first, so that their words land where SAVE put them
  // (csrc/CUDAGraphParallel.cpp:2048-2059).
  const std::string gens = impl.section(g, FDY_SEC_GENERATORS);
  for (size_t k = 0; k + 24 <= gens.size(); k += 24) {
    uint64_t row[3];
    std::memcpy(row, gens.data() + k, 24);
    CUDAGeneratorStateRegistry& reg = pending->registry ? *pending->registry : global_generator_state_registry();
    graph->register_generator_state(reg.get_state_from_id(row[0], row[1]), row[2]);
  }
  // Allocator events in SAVE order (2060-2064).
  const std::string events = impl.section(g, FDY_SEC_ALLOC_EVENTS);
  if (!events.empty() && t_region.r)
    check(fdy_region_replay(t_region.r, events.data(), events.size()), "finish_one_graph_load (allocator events)");
  // Output tensors: non-owning views at the relocated addresses
  // (csrc/CUDAGraph.cpp:971-999, csrc/CUDAGraphParallel.cpp:2077-2095).
  GraphLoadResult res{graph, std::monostate{}, OutputTensorType::None};
  const std::string text = impl.section(g, FDY_SEC_OUTPUT_TENSORS);
  if (!text.empty()) {
    fdy::json::Value doc;
    std::string error;
    TORCH_CHECK(fdy::json::Reader(text.data(), text.size()).parse(doc, error), "output_tensors: ", error);
    TORCH_CHECK(doc.kind == fdy::json::Value::Object, "output_tensors: not an object");
    const int64_t kind = doc.get("type") ? json_i64(doc.get("type"), "type") : 0;
    std::vector<at::Tensor> ts;
    if (const fdy::json::Value* arr = doc.get("tensors")) {
      TORCH_CHECK(arr->kind == fdy::json::Value::Array, "output_tensors: tensors is not an array");
      for (const auto& m : arr->items) {
        const int64_t dt = json_i64(m.get("dtype"), "dtype");
        TORCH_CHECK(dt >= 0 && dt < (int64_t)c10::ScalarType::NumOptions, "output tensor of unsupported scalar type ",
                    dt);
        std::vector<int64_t> sizes, strides;
        for (const auto& v : m.get("sizes") ? m.get("sizes")->items : std::vector<fdy::json::Value>{})
          sizes.push_back(json_i64(&v, "sizes"));
        for (const auto& v : m.get("strides") ? m.get("strides")->items : std::vector<fdy::json::Value>{})
          strides.push_back(json_i64(&v, "strides"));
        TORCH_CHECK(sizes.size() == strides.size(), "output_tensors: sizes and strides differ in rank");
        const fdy::json::Value* dev = m.get("device_index");
        const int64_t device = dev && dev->kind == fdy::json::Value::Number ? json_i64(dev, "device_index") : 0;
        const fdy::json::Value* rg = m.get("requires_grad");
        const uint64_t ptr = impl.relocate(json_u64(m.get("data_ptr"), "data_ptr"));
        auto t = at::from_blob(reinterpret_cast<void*>(ptr), sizes, strides,
                               at::TensorOptions()
                                   .dtype(static_cast<c10::ScalarType>(dt))
                                   .device(at::Device(at::kCUDA, (c10::DeviceIndex)device)));
        if (rg && rg->kind == fdy::json::Value::Bool && rg->b) t.requires_grad_(true);
        ts.push_back(std::move(t));
      }
    }
    if (kind == 1 && ts.size() == 1) {
      res.outputs = ts[0];
      res.output_type = OutputTensorType::Single;
    } else if (kind == 2 || kind == 3) {
      res.outputs = std::move(ts);
      res.output_type = kind == 3 ? OutputTensorType::Tuple : OutputTensorType::List;
    }
  }
  impl.results[index] = res;
  impl.finished[index] = true;
  return res;
}

std::vector<GraphLoadResult> CUDAGraph::finish_graph_loads(std::shared_ptr<PendingGraphLoads> pending) {
  TORCH_CHECK(pending, "finish_graph_loads: no pending loads");
  if (pending->build_complete_.valid()) pending->build_complete_.get();  // 2079-2088
  std::vector<GraphLoadResult> out;
  for (size_t i = 0; i < pending->graphs.size(); ++i) out.push_back(finish_one_graph_load(pending, i));
  return out;
}

GraphLoadResult CUDAGraph::load(const std::string& json_path, MempoolId_t pool) {
  return finish_one_graph_load(start_graph_builds({json_path}, pool, 1), 0);
}

}  // namespace foundry
