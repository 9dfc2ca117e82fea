// graph.hip -- host side of include/foundry_graph.h: the code-object registry
// and the group graphs (one hipGraph + hipGraphExec per topology group).
//
// The params a graph's nodes take come from the restore: the template's
// relocated param image R_t when the group graph is built, and afterwards
// the group's live image, which the device override scatter keeps equal to
// the selected graph's R_g.  The scatter marks each node it touches as
// dirty (device memory), and k_mirror then copies the dirty nodes' words
// into device-visible host memory (h_live) as whole lines, so that a switch
// re-sets exactly the nodes whose params changed, plus the nodes whose
// descriptor or layout is the current or the new graph's own.
#include <hip/hip_runtime.h>

#include <elf.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <memory>
#include <set>
#include <sstream>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/fdy_format.h"
#include "../../include/foundry_graph.h"
#include "../../include/foundry_restore.h"
#include "archive.h"
#include "crc64.h"
#include "kernels.h"

using fdy::err;

struct fdy_registry {
  int device = 0;
  struct Code {
    uint64_t hash = 0;
    std::vector<uint8_t> bytes;  // kept for the module's lifetime
    hipModule_t mod = nullptr;
  };
  std::vector<std::unique_ptr<Code>> codes;
  std::unordered_map<uint64_t, Code*> by_hash;
  std::unordered_map<std::string, hipFunction_t> fns;  // key: 8 hash bytes + name
  std::mutex mu;

  ~fdy_registry() {
    if (!codes.empty()) (void)hipSetDevice(device);
    for (auto& c : codes)
      if (c->mod) (void)hipModuleUnload(c->mod);
  }
};

namespace fdy {
namespace {

using Clock = std::chrono::steady_clock;
double us_since(Clock::time_point t0) { return std::chrono::duration<double, std::micro>(Clock::now() - t0).count(); }

const SliceTables& slice_tables() {
  static const SliceTables t = make_slice_tables();
  return t;
}

uint64_t crc64_xz(const uint8_t* p, uint64_t n) {
  const SliceTables& t = slice_tables();
  uint64_t c = ~0ull;
  uint64_t i = 0;
  for (; i + 8 <= n; i += 8) {
    uint64_t w;
    std::memcpy(&w, p + i, 8);
    c = crc_slice8(t.t, c, w);
  }
  for (; i < n; ++i) c = crc_byte(t.t[0], c, p[i]);
  return ~c;
}

int registry_lookup(fdy_registry* r, uint64_t hash, const char* name, size_t name_len, hipFunction_t* out) {
  std::string key(reinterpret_cast<const char*>(&hash), 8);
  key.append(name, name_len);
  std::lock_guard<std::mutex> lk(r->mu);
  auto f = r->fns.find(key);
  if (f != r->fns.end()) {
    *out = f->second;
    return FDY_OK;
  }
  char hex[20];
  std::snprintf(hex, sizeof hex, "%016llx", (unsigned long long)hash);
  auto c = r->by_hash.find(hash);
  if (c == r->by_hash.end())
    return err(FDY_E_NOT_FOUND, std::string("no code object with binary_hash 0x") + hex + " is registered (kernel '" +
                                    std::string(name, name_len) + "')");
  hipFunction_t fn = nullptr;
  const std::string nm(name, name_len);
  hipError_t e = hipModuleGetFunction(&fn, c->second->mod, nm.c_str());
  if (e != hipSuccess || !fn) {
    (void)hipGetLastError();
    return err(FDY_E_NOT_FOUND, "code object 0x" + std::string(hex) + " has no kernel '" + nm + "'");
  }
  r->fns.emplace(std::move(key), fn);
  *out = fn;
  return FDY_OK;
}

// Host copies of one graph's sections and restore results.  `flags` is
// always present.  The node table, strings, param index and common attrs
// come with `desc_loaded` (the template, and members with nodes whose
// descriptor or layout is their own); node descriptors and the param image
// R_g with `layout_loaded` (members with layout changes, and the template);
// relocated memset/memcpy pointers with `ptrs_loaded`.
struct HostGraph {
  uint32_t g = 0;
  bool desc_loaded = false, layout_loaded = false, ptrs_loaded = false;
  std::vector<uint8_t> flags;
  std::vector<fdy_node> nodes;
  std::vector<uint8_t> strings, pidx;
  std::vector<fdy_dep> deps;
  bool has_common = false;
  fdy_common_attrs common{};
  std::vector<NodeDesc> desc;
  std::vector<uint64_t> ptrs;   // relocated memset dst / memcpy dst, src: 2 per node
  std::vector<uint64_t> words;  // R_g
};

template <typename T>
int fetch(const void* dev, uint64_t count, std::vector<T>& out) {
  out.resize(count);
  if (count) FDY_HIP(hipMemcpy(out.data(), dev, count * sizeof(T), hipMemcpyDeviceToHost));
  return FDY_OK;
}

int fetch_section(fdy_archive* a, uint32_t g, int sec, std::vector<uint8_t>& out) {
  return fetch(a->img.as<uint8_t>() + a->graphs[g].sec_off[sec], a->graphs[g].sec_size[sec], out);
}

int fetch_flags(fdy_archive* a, uint32_t g, HostGraph& h) {
  h.g = g;
  return fetch(a->nflags.as<uint8_t>() + a->graphs[g].node_base, a->graphs[g].num_nodes, h.flags);
}

int fetch_desc(fdy_archive* a, uint32_t g, HostGraph& h) {
  const DevGraph& d = a->graphs[g];
  std::vector<uint8_t> raw;
  int rc = fetch_section(a, g, FDY_SEC_NODES, raw);
  if (rc) return rc;
  if (raw.size() < (uint64_t)d.num_nodes * sizeof(fdy_node)) return err(FDY_E_FORMAT, "node section too short");
  h.nodes.resize(d.num_nodes);
  if (d.num_nodes) std::memcpy(h.nodes.data(), raw.data(), (uint64_t)d.num_nodes * sizeof(fdy_node));
  if (!rc) rc = fetch_section(a, g, FDY_SEC_STRINGS, h.strings);
  if (!rc) rc = fetch_section(a, g, FDY_SEC_PARAM_INDEX, h.pidx);
  if (!rc) rc = fetch_section(a, g, FDY_SEC_DEPS, raw);
  if (rc) return rc;
  const uint64_t ndeps = (d.flags & FDY_HAS_DEPS) ? d.num_deps : 0;
  if (raw.size() < ndeps * sizeof(fdy_dep)) return err(FDY_E_FORMAT, "dependency section too short");
  h.deps.resize(ndeps);
  if (ndeps) std::memcpy(h.deps.data(), raw.data(), ndeps * sizeof(fdy_dep));
  h.has_common = false;
  if (d.flags & FDY_HAS_COMMON_ATTRS) {
    rc = fetch_section(a, g, FDY_SEC_COMMON_ATTRS, raw);
    if (rc) return rc;
    if (raw.size() >= sizeof(fdy_common_attrs)) {
      std::memcpy(&h.common, raw.data(), sizeof(fdy_common_attrs));
      h.has_common = true;
    }
  }
  h.desc_loaded = true;
  return FDY_OK;
}

int fetch_layout(fdy_archive* a, uint32_t g, HostGraph& h) {
  const DevGraph& d = a->graphs[g];
  int rc = fetch(a->ndesc.as<NodeDesc>() + d.node_base, d.num_nodes, h.desc);
  if (!rc) rc = fetch(a->image.as<uint64_t>() + r_base(a, g), a->h_gwords[g], h.words);
  if (!rc) h.layout_loaded = true;
  return rc;
}

int fetch_ptrs(fdy_archive* a, uint32_t g, HostGraph& h) {
  int rc = fetch(a->nptrs.as<uint64_t>() + 2 * a->graphs[g].node_base, 2ull * a->graphs[g].num_nodes, h.ptrs);
  if (!rc) h.ptrs_loaded = true;
  return rc;
}

// Cluster dims and cooperative flag of kernel node n: common attrs, then the
// node's own attrs where set, then required cluster dims from the function
// attrs (csrc/CUDAGraphParallel.cpp:1345-1389).
struct LaunchAttrs {
  uint32_t cx = 0, cy = 0, cz = 0;
  int32_t coop = -1;
};

void read_attrs(const uint8_t* b, LaunchAttrs& a, bool merge) {
  uint32_t f;
  std::memcpy(&f, b, 4);
  if (f & FDY_KNA_CLUSTER_DIM) {
    std::memcpy(&a.cx, b + 4, 4);
    std::memcpy(&a.cy, b + 8, 4);
    std::memcpy(&a.cz, b + 12, 4);
  }
  if (f & FDY_KNA_COOPERATIVE) {
    int32_t v;
    std::memcpy(&v, b + 32, 4);
    if (!merge || v >= 0) a.coop = v;
  }
}

LaunchAttrs launch_attrs(const HostGraph& h, uint32_t n) {
  LaunchAttrs a;
  const uint8_t* e = reinterpret_cast<const uint8_t*>(&h.nodes[n]);
  if (h.has_common) read_attrs(reinterpret_cast<const uint8_t*>(&h.common), a, false);
  uint32_t kf;
  std::memcpy(&kf, e + FDY_KOFF_KNA_FLAGS, 4);
  if (kf) read_attrs(e + FDY_KOFF_KNA_FLAGS, a, true);
  const fdy_kernel_body& k = h.nodes[n].u.kernel;
  if (k.required_cluster[0] > 0 || k.required_cluster[1] > 0 || k.required_cluster[2] > 0) {
    a.cx = k.required_cluster[0] > 0 ? k.required_cluster[0] : 1;
    a.cy = k.required_cluster[1] > 0 ? k.required_cluster[1] : 1;
    a.cz = k.required_cluster[2] > 0 ? k.required_cluster[2] : 1;
  }
  return a;
}

std::string node_name(uint32_t g, uint32_t n) { return "graph " + std::to_string(g) + " node " + std::to_string(n); }

// Everything one exec node needs to be added or re-set, computed once: for
// every node of the template when the group graph is built, and for each
// member graph's own-descriptor nodes when that graph is first selected.
// Kernel params point into `words` (the node's words of an image laid out
// param by param, each padded to 8 bytes) through the owner's pointer array
// (pfirst, pcount), so an update is a single exec call.
struct NodeUpdate {
  uint8_t type = 0;
  bool copy3d = false;
  int32_t coop = -1;
  hipFunction_t fn = nullptr;
  dim3 grid, block;
  uint32_t shmem = 0;
  bool extra = false;
  size_t arg_size = 0;
  void* extra_cfg[5] = {};
  uint32_t pfirst = 0, pcount = 0;
  FillArgs fill{};
  hipEvent_t event = nullptr;
  // memcpy
  void* dst = nullptr;
  const void* src = nullptr;
  size_t bytes = 0;
  hipMemcpy3DParms p3{};

  NodeUpdate() = default;
  NodeUpdate(const NodeUpdate&) = delete;  // extra_cfg points at arg_size
  NodeUpdate& operator=(const NodeUpdate&) = delete;
};

// The updates of one graph's nodes and the param pointer array they index.
struct UpdateSet {
  std::vector<std::unique_ptr<NodeUpdate>> u;
  std::vector<void*> params;
};

hipKernelNodeParams kernel_params(const NodeUpdate& u, void** params) {
  hipKernelNodeParams p{};
  p.func = reinterpret_cast<void*>(u.fn);
  p.gridDim = u.grid;
  p.blockDim = u.block;
  p.sharedMemBytes = u.shmem;
  if (u.extra) p.extra = const_cast<void**>(u.extra_cfg);
  else p.kernelParams = u.pcount ? params + u.pfirst : nullptr;
  return p;
}

hipKernelNodeParams fill_params(NodeUpdate& u) {
  hipKernelNodeParams p{};
  p.func = fill_kernel();
  p.gridDim = fill_grid(u.fill);
  p.blockDim = dim3(kFillThreads);
  // HIP copies the argument when the node is added or set.
  static thread_local void* arg[1];
  arg[0] = &u.fill;
  p.kernelParams = arg;
  return p;
}

int kernel_update(fdy_registry* r, const HostGraph& h, uint32_t n, uint64_t* words, uint32_t nwords, NodeUpdate& k,
                  std::vector<void*>& params) {
  const fdy_kernel_body& b = h.nodes[n].u.kernel;
  if ((uint64_t)b.name_offset + b.name_length > h.strings.size())
    return err(FDY_E_FORMAT, node_name(h.g, n) + ": kernel name outside the string section");
  size_t len = b.name_length;
  const char* name = reinterpret_cast<const char*>(h.strings.data()) + b.name_offset;
  while (len && name[len - 1] == '\0') --len;
  int rc = registry_lookup(r, b.binary_hash, name, len, &k.fn);
  if (rc) return rc;
  const LaunchAttrs at = launch_attrs(h, n);
  if (at.cx > 1 || at.cy > 1 || at.cz > 1)
    return err(FDY_E_UNSUPPORTED, node_name(h.g, n) + ": cluster dims " + std::to_string(at.cx) + "x" +
                                      std::to_string(at.cy) + "x" + std::to_string(at.cz) +
                                      " (gfx950 has no thread-block clusters)");
  k.coop = at.coop;
  k.grid = dim3(b.grid[0], b.grid[1], b.grid[2]);
  k.block = dim3(b.block[0], b.block[1], b.block[2]);
  k.shmem = b.shared_mem_bytes;
  uint64_t used = 0;
  if (b.arg_offset != FDY_NO_ARG_BUFFER) {
    k.extra = true;
    k.arg_size = b.arg_size;
    used = (b.arg_size + 7) / 8;
    k.extra_cfg[0] = HIP_LAUNCH_PARAM_BUFFER_POINTER;
    k.extra_cfg[1] = words;
    k.extra_cfg[2] = HIP_LAUNCH_PARAM_BUFFER_SIZE;
    k.extra_cfg[3] = &k.arg_size;
    k.extra_cfg[4] = HIP_LAUNCH_PARAM_END;
  } else {
    k.extra = false;
    if ((uint64_t)b.param_index_offset + 8ull * b.num_params > h.pidx.size())
      return err(FDY_E_FORMAT, node_name(h.g, n) + ": param entries outside the param-index section");
    k.pfirst = (uint32_t)params.size();
    k.pcount = b.num_params;
    for (uint32_t j = 0; j < b.num_params; ++j) {
      fdy_param pe;
      std::memcpy(&pe, h.pidx.data() + b.param_index_offset + 8ull * j, sizeof pe);
      params.push_back(words + used);
      used += (pe.size + 7) / 8;
    }
  }
  if (used != nwords)
    return err(FDY_E_FORMAT, node_name(h.g, n) + ": params take " + std::to_string(used) +
                                 " image words, the restore laid out " + std::to_string(nwords));
  return FDY_OK;
}

int fill_args(const HostGraph& h, uint32_t n, FillArgs& f) {
  const fdy_memset_body& m = h.nodes[n].u.memset;
  const uint32_t es = m.element_size;
  if (es != 1 && es != 2 && es != 4)
    return err(FDY_E_FORMAT, node_name(h.g, n) + ": memset element size " + std::to_string(es));
  f.dst = reinterpret_cast<uint8_t*>(h.ptrs[2ull * n]);
  f.row_bytes = m.width * es;
  f.height = m.height;
  f.pitch = m.pitch;
  f.pattern = es == 1 ? (m.value & 0xFFu) * 0x01010101u : es == 2 ? (m.value & 0xFFFFu) * 0x00010001u : m.value;
  f.pad_ = 0;
  if (f.height > 1 && f.pitch < f.row_bytes)
    return err(FDY_E_FORMAT, node_name(h.g, n) + ": memset pitch below the row width");
  return FDY_OK;
}

struct CopyDesc {
  bool is3d = false;
  void* dst = nullptr;
  const void* src = nullptr;
  size_t bytes = 0;
  hipMemcpy3DParms p3{};
};

int copy_desc(const HostGraph& h, uint32_t n, CopyDesc& c) {
  const fdy_memcpy_body& m = h.nodes[n].u.memcpy;
  auto device_side = [](int32_t t) { return t == FDY_MEMTYPE_DEVICE || t == FDY_MEMTYPE_UNIFIED; };
  if (!device_side(m.dst_mem_type) || !device_side(m.src_mem_type))
    return err(FDY_E_UNSUPPORTED, node_name(h.g, n) + ": memcpy with a host or array endpoint (types " +
                                      std::to_string(m.src_mem_type) + " -> " + std::to_string(m.dst_mem_type) +
                                      ") has no address valid in another process");
  const uint64_t dst = h.ptrs[2ull * n], src = h.ptrs[2ull * n + 1];
  if (m.height <= 1 && m.depth <= 1) {
    c.is3d = false;
    c.dst = reinterpret_cast<void*>(dst + m.dst_x_bytes + m.dst_y * m.dst_pitch + m.dst_z * m.dst_pitch * m.dst_height);
    c.src = reinterpret_cast<const void*>(src + m.src_x_bytes + m.src_y * m.src_pitch +
                                          m.src_z * m.src_pitch * m.src_height);
    c.bytes = m.width_bytes;
    return FDY_OK;
  }
  if (m.src_pitch < m.width_bytes || m.dst_pitch < m.width_bytes ||
      (m.depth > 1 && (m.src_height < m.height || m.dst_height < m.height)))
    return err(FDY_E_FORMAT, node_name(h.g, n) + ": memcpy pitch or height below the copied extent");
  c.is3d = true;
  c.p3 = hipMemcpy3DParms{};
  c.p3.srcPtr = make_hipPitchedPtr(reinterpret_cast<void*>(src), m.src_pitch, m.width_bytes, m.src_height);
  c.p3.srcPos = make_hipPos(m.src_x_bytes, m.src_y, m.src_z);
  c.p3.dstPtr = make_hipPitchedPtr(reinterpret_cast<void*>(dst), m.dst_pitch, m.width_bytes, m.dst_height);
  c.p3.dstPos = make_hipPos(m.dst_x_bytes, m.dst_y, m.dst_z);
  c.p3.extent = make_hipExtent(m.width_bytes, m.height, m.depth);
  c.p3.kind = hipMemcpyDeviceToDevice;
  return FDY_OK;
}

struct GNode {
  hipGraphNode_t h = nullptr;
  uint8_t type = 0;
  bool copy3d = false;
  int32_t coop = -1;
  uint32_t tword = 0, nwords = 0;  // the node's words in the template's image
};

// A member graph: its host copies, and the updates of its own-descriptor
// nodes (own[n] indexes `set`, or -1).
struct Member {
  HostGraph h;
  std::vector<int32_t> own;
  UpdateSet set;
};

}  // namespace
}  // namespace fdy

using namespace fdy;

// One instantiated exec of a group graph, holding one graph's params.
struct ExecSlot {
  hipGraphExec_t exec = nullptr;
  uint32_t graph = 0;          // graph whose params the exec holds
  uint64_t used = 0;           // selection tick of its last selection
  hipEvent_t done = nullptr;   // recorded after each launch
  bool launched = false;
  bool stale = false;          // an update failed part-way: re-set every node next time
};

// Execs a group graph keeps by default (fdy_group_graph_set_exec_cache).
constexpr uint32_t kDefaultExecs = 4;

struct fdy_group_graph {
  fdy_archive* a = nullptr;
  fdy_registry* reg = nullptr;
  uint32_t t = 0;
  uint32_t N = 0;
  hipGraph_t graph = nullptr;
  // Execs of recently selected graphs: selecting a graph that holds one
  // makes it current with no node update; otherwise the least recently
  // selected exec (or a new one, below max_execs) is updated to the graph.
  std::vector<ExecSlot> slots;
  uint32_t cur = 0;            // the current exec (launched by fdy_group_graph_launch)
  uint32_t max_execs = kDefaultExecs;
  uint64_t tick = 0;
  std::vector<GNode> nodes;
  HostGraph th;                                 // the template
  UpdateSet tset;                               // the template's updates, one per node
  std::unordered_map<uint32_t, std::unique_ptr<Member>> members;
  std::unordered_map<int32_t, hipEvent_t> events;  // saved event id -> event
  uint64_t* h_live = nullptr;                   // host mirror of the group's live image
  uint8_t* h_dirty = nullptr;                   // per node
  uint64_t* d_live = nullptr;                   // device addresses of the two
  uint8_t* d_dirty = nullptr;
  DevBuf dirty;                                 // per node, device memory: the scatter's marks
  fdy_group_graph_info info{};

  ~fdy_group_graph() {
    (void)hipSetDevice(a ? a->device : 0);
    for (ExecSlot& x : slots) {
      if (x.done && x.launched) (void)hipEventSynchronize(x.done);
      if (x.exec) (void)hipGraphExecDestroy(x.exec);
      if (x.done) (void)hipEventDestroy(x.done);
    }
    if (graph) (void)hipGraphDestroy(graph);
    for (auto& e : events) (void)hipEventDestroy(e.second);
    if (h_live) (void)hipHostFree(h_live);
    if (h_dirty) (void)hipHostFree(h_dirty);
  }
};

namespace fdy {
namespace {

int event_for(fdy_group_graph* gg, int32_t id, hipEvent_t* out) {
  auto it = gg->events.find(id);
  if (it == gg->events.end()) {
    hipEvent_t e = nullptr;
    FDY_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    it = gg->events.emplace(id, e).first;
  }
  *out = it->second;
  return FDY_OK;
}

// The update of node n of graph h: params from `words` (nwords of them).
int make_update(fdy_group_graph* gg, const HostGraph& h, uint32_t n, uint64_t* words, uint32_t nwords, NodeUpdate& u,
                std::vector<void*>& params) {
  u.type = h.nodes[n].type;
  switch (u.type) {
    case FDY_NODE_KERNEL:
      return kernel_update(gg->reg, h, n, words, nwords, u, params);
    case FDY_NODE_MEMSET:
      return fill_args(h, n, u.fill);
    case FDY_NODE_MEMCPY: {
      CopyDesc c;
      int rc = copy_desc(h, n, c);
      if (rc) return rc;
      u.copy3d = c.is3d;
      u.dst = c.dst;
      u.src = c.src;
      u.bytes = c.bytes;
      u.p3 = c.p3;
      return FDY_OK;
    }
    case FDY_NODE_EVENT_RECORD:
    case FDY_NODE_EVENT_WAIT:
      return event_for(gg, h.nodes[n].u.event.event_id, &u.event);
    case FDY_NODE_EMPTY:
      return FDY_OK;
    default:
      return err(FDY_E_FORMAT, node_name(h.g, n) + ": unknown node type " + std::to_string(u.type));
  }
}

int apply_update(hipGraphExec_t exec, const GNode& x, NodeUpdate& u, void** params) {
  switch (x.type) {
    case FDY_NODE_KERNEL: {
      hipKernelNodeParams p = kernel_params(u, params);
      FDY_HIP(hipGraphExecKernelNodeSetParams(exec, x.h, &p));
      return FDY_OK;
    }
    case FDY_NODE_MEMSET: {
      hipKernelNodeParams p = fill_params(u);
      FDY_HIP(hipGraphExecKernelNodeSetParams(exec, x.h, &p));
      return FDY_OK;
    }
    case FDY_NODE_MEMCPY:
      if (u.copy3d) FDY_HIP(hipGraphExecMemcpyNodeSetParams(exec, x.h, &u.p3));
      else FDY_HIP(hipGraphExecMemcpyNodeSetParams1D(exec, x.h, u.dst, u.src, u.bytes, hipMemcpyDeviceToDevice));
      return FDY_OK;
    case FDY_NODE_EVENT_RECORD:
      FDY_HIP(hipGraphExecEventRecordNodeSetEvent(exec, x.h, u.event));
      return FDY_OK;
    case FDY_NODE_EVENT_WAIT:
      FDY_HIP(hipGraphExecEventWaitNodeSetEvent(exec, x.h, u.event));
      return FDY_OK;
    default:
      return FDY_OK;
  }
}

// Member g's host state, fetched and prepared on its first use.
Member* member(fdy_group_graph* gg, uint32_t g, int* rc) {
  auto it = gg->members.find(g);
  if (it != gg->members.end()) return it->second.get();
  auto m = std::make_unique<Member>();
  HostGraph& h = m->h;
  *rc = fetch_flags(gg->a, g, h);
  if (*rc) return nullptr;
  const uint32_t N = (uint32_t)h.flags.size();
  m->own.assign(N, -1);
  uint32_t n_own = 0;
  bool layout = false, ptr_nodes = false;
  for (uint32_t n = 0; n < N; ++n) {
    const uint8_t f = h.flags[n];
    if (!(f & (FDY_NODE_LAYOUT | FDY_NODE_DESC))) continue;
    ++n_own;
    layout |= (f & FDY_NODE_LAYOUT) != 0;
    const uint8_t ty = gg->nodes[n].type;
    ptr_nodes |= ty == FDY_NODE_MEMSET || ty == FDY_NODE_MEMCPY;
  }
  if (n_own) {
    *rc = fetch_desc(gg->a, g, h);
    if (!*rc && layout) *rc = fetch_layout(gg->a, g, h);
    if (!*rc && ptr_nodes) *rc = fetch_ptrs(gg->a, g, h);
    if (*rc) return nullptr;
    m->set.u.reserve(n_own);
    for (uint32_t n = 0; n < N; ++n) {
      const uint8_t f = h.flags[n];
      if (!(f & (FDY_NODE_LAYOUT | FDY_NODE_DESC))) continue;
      const GNode& x = gg->nodes[n];
      uint64_t* words = gg->h_live + x.tword;
      uint32_t nw = x.nwords;
      if (f & FDY_NODE_LAYOUT) {
        words = h.words.data() + h.desc[n].gword;
        nw = h.desc[n].nwords;
      }
      auto u = std::make_unique<NodeUpdate>();
      *rc = make_update(gg, h, n, words, nw, *u, m->set.params);
      if (*rc) return nullptr;
      if (u->type != x.type) {
        *rc = err(FDY_E_MISMATCH, node_name(g, n) + ": node type differs from the template's");
        return nullptr;
      }
      if (u->type == FDY_NODE_KERNEL && (u->coop > 0) != (x.coop > 0)) {
        *rc = err(FDY_E_UNSUPPORTED, node_name(g, n) + ": cooperative attribute differs from the template's");
        return nullptr;
      }
      if (u->type == FDY_NODE_MEMCPY && u->copy3d != x.copy3d) {
        *rc = err(FDY_E_UNSUPPORTED, node_name(g, n) + ": memcpy changes between 1-D and 3-D form");
        return nullptr;
      }
      m->own[n] = (int32_t)m->set.u.size();
      m->set.u.push_back(std::move(u));
    }
  }
  Member* p = m.get();
  gg->members.emplace(g, std::move(m));
  return p;
}

// A new exec of the group's graph (which holds the template's params).
int add_exec(fdy_group_graph* gg) {
  ExecSlot x;
  x.graph = gg->t;
  FDY_HIP(hipGraphInstantiate(&x.exec, gg->graph, nullptr, nullptr, 0));
  const hipError_t e = hipEventCreateWithFlags(&x.done, hipEventDisableTiming);
  if (e != hipSuccess) {
    (void)hipGraphExecDestroy(x.exec);
    FDY_HIP(e);
  }
  gg->slots.push_back(x);
  gg->info.num_execs = (uint32_t)gg->slots.size();
  return FDY_OK;
}

int build(fdy_group_graph* gg) {
  const auto t0 = Clock::now();
  fdy_archive* a = gg->a;
  const uint32_t t = gg->t;
  HostGraph& th = gg->th;
  th.g = t;
  int rc = fetch_flags(a, t, th);
  if (!rc) rc = fetch_desc(a, t, th);
  if (!rc) rc = fetch_layout(a, t, th);
  if (!rc) rc = fetch_ptrs(a, t, th);
  if (rc) return rc;
  const uint32_t N = gg->N = a->graphs[t].num_nodes;
  gg->nodes.assign(N, GNode{});

  // Mirror of the live image (the template's R_t) and the dirty marks, in
  // host memory k_mirror writes through.
  const uint64_t cap = std::max<uint64_t>(a->graphs[t].word_cap, 1);
  FDY_HIP(hipHostMalloc(reinterpret_cast<void**>(&gg->h_live), 8 * cap, hipHostMallocMapped | hipHostMallocCoherent));
  FDY_HIP(hipHostMalloc(reinterpret_cast<void**>(&gg->h_dirty), std::max<uint32_t>(N, 1),
                        hipHostMallocMapped | hipHostMallocCoherent));
  FDY_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&gg->d_live), gg->h_live, 0));
  FDY_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&gg->d_dirty), gg->h_dirty, 0));
  std::memset(gg->h_live, 0, 8 * cap);
  std::memset(gg->h_dirty, 0, std::max<uint32_t>(N, 1));
  if (!th.words.empty()) std::memcpy(gg->h_live, th.words.data(), 8 * th.words.size());
  rc = dev_alloc(gg->dirty, std::max<uint32_t>(N, 1), "group graph dirty marks");
  if (rc) return rc;
  FDY_HIP(hipMemset(gg->dirty.p, 0, std::max<uint32_t>(N, 1)));

  FDY_HIP(hipGraphCreate(&gg->graph, 0));
  fdy_group_graph_info& info = gg->info;
  gg->tset.u.reserve(N);
  for (uint32_t n = 0; n < N; ++n) {
    GNode& x = gg->nodes[n];
    x.type = th.nodes[n].type;
    x.tword = th.desc[n].gword;
    x.nwords = th.desc[n].nwords;
    if ((uint64_t)x.tword + x.nwords > cap) return err(FDY_E_FORMAT, node_name(t, n) + ": words beyond the image");
    auto up = std::make_unique<NodeUpdate>();
    NodeUpdate& u = *up;
    rc = make_update(gg, th, n, gg->h_live + x.tword, x.nwords, u, gg->tset.params);
    if (rc) return rc;
    x.coop = u.coop;
    x.copy3d = u.copy3d;
    gg->tset.u.push_back(std::move(up));
  }
  for (uint32_t n = 0; n < N; ++n) {
    GNode& x = gg->nodes[n];
    NodeUpdate& u = *gg->tset.u[n];
    switch (x.type) {
      case FDY_NODE_KERNEL: {
        hipKernelNodeParams p = kernel_params(u, gg->tset.params.data());
        FDY_HIP(hipGraphAddKernelNode(&x.h, gg->graph, nullptr, 0, &p));
        if (u.coop > 0) {
          hipKernelNodeAttrValue v{};
          v.cooperative = 1;
          FDY_HIP(hipGraphKernelNodeSetAttribute(x.h, hipLaunchAttributeCooperative, &v));
        }
        ++info.num_kernel_nodes;
        break;
      }
      case FDY_NODE_MEMSET: {
        hipKernelNodeParams p = fill_params(u);
        FDY_HIP(hipGraphAddKernelNode(&x.h, gg->graph, nullptr, 0, &p));
        ++info.num_fill_nodes;
        break;
      }
      case FDY_NODE_MEMCPY:
        if (u.copy3d) FDY_HIP(hipGraphAddMemcpyNode(&x.h, gg->graph, nullptr, 0, &u.p3));
        else FDY_HIP(hipGraphAddMemcpyNode1D(&x.h, gg->graph, nullptr, 0, u.dst, u.src, u.bytes, hipMemcpyDeviceToDevice));
        ++info.num_memcpy_nodes;
        break;
      case FDY_NODE_EVENT_RECORD:
        FDY_HIP(hipGraphAddEventRecordNode(&x.h, gg->graph, nullptr, 0, u.event));
        ++info.num_event_nodes;
        break;
      case FDY_NODE_EVENT_WAIT:
        FDY_HIP(hipGraphAddEventWaitNode(&x.h, gg->graph, nullptr, 0, u.event));
        ++info.num_event_nodes;
        break;
      default:
        FDY_HIP(hipGraphAddEmptyNode(&x.h, gg->graph, nullptr, 0));
        break;
    }
  }

  // Dependencies name node ids (csrc/CUDAGraphParallel.cpp:774-800).
  std::unordered_map<uint32_t, uint32_t> index_of;
  index_of.reserve(N * 2 + 1);
  for (uint32_t n = 0; n < N; ++n)
    if (!index_of.emplace(th.nodes[n].node_id, n).second)
      return err(FDY_E_FORMAT, node_name(t, n) + ": node id " + std::to_string(th.nodes[n].node_id) + " repeats");
  if (!th.deps.empty()) {
    std::vector<hipGraphNode_t> from(th.deps.size()), to(th.deps.size());
    for (size_t i = 0; i < th.deps.size(); ++i) {
      auto f = index_of.find(th.deps[i].from), d = index_of.find(th.deps[i].to);
      if (f == index_of.end() || d == index_of.end())
        return err(FDY_E_FORMAT, "graph " + std::to_string(t) + " dependency " + std::to_string(i) +
                                     " names a node id that does not exist");
      from[i] = gg->nodes[f->second].h;
      to[i] = gg->nodes[d->second].h;
    }
    FDY_HIP(hipGraphAddDependencies(gg->graph, from.data(), to.data(), from.size()));
  }
  const auto ti = Clock::now();
  rc = add_exec(gg);
  if (rc) return rc;
  info.instantiate_ms = us_since(ti) / 1000.0;
  info.template_graph = t;
  info.current_graph = t;
  info.num_nodes = N;
  info.num_deps = (uint32_t)th.deps.size();
  info.num_events = (uint32_t)gg->events.size();
  info.build_ms = us_since(t0) / 1000.0;
  return FDY_OK;
}

}  // namespace

int group_graph_select(fdy_group_graph* gg, uint32_t g, hipStream_t s, void* stats_v) {
  const auto t0 = Clock::now();
  fdy_select_stats st{};
  fdy_archive* a = gg->a;
  int rc = check_graph(a, g);
  if (!rc) rc = ensure_cache(a, s);
  uint32_t t = 0;
  if (!rc) rc = check_switchable(a, g, &t);
  if (rc) return rc;
  if (t != gg->t)
    return err(FDY_E_INVALID, "graph " + std::to_string(g) + " belongs to the group of template " + std::to_string(t) +
                                  ", not " + std::to_string(gg->t));
  if (a->h_status[g] & FDY_GRAPH_TYPE_MISMATCH)
    return err(FDY_E_MISMATCH, "graph " + std::to_string(g) + " has node types other than its template's");
  if (a->h_status[g] & FDY_GRAPH_BAD_PARAMS)
    return err(FDY_E_FORMAT, "graph " + std::to_string(g) + " has ranges outside its sections");
  const uint32_t c = a->h_current[t];  // the live image's graph
  ++gg->tick;
  // An exec that holds g already: it becomes current, with no node update;
  // the live image follows (the scatter, enqueued on `s`, marks nothing).
  for (uint32_t i = 0; i < gg->slots.size(); ++i) {
    ExecSlot& x = gg->slots[i];
    if (x.graph != g || x.stale) continue;
    if (c != g) {
      FDY_HIP(hipSetDevice(a->device));
      st.words_scattered = (a->h_ovr_off[c + 1] - a->h_ovr_off[c]) + (a->h_ovr_off[g + 1] - a->h_ovr_off[g]);
      rc = enqueue_switch(a, g, s, nullptr);
      if (rc) return rc;
    }
    x.used = gg->tick;
    gg->cur = i;
    gg->info.current_graph = g;
    st.cache_hit = 1;
    st.host_us = us_since(t0);
    if (stats_v) *static_cast<fdy_select_stats*>(stats_v) = st;
    return FDY_OK;
  }
  Member* m = nullptr;
  if (g != gg->t) {
    m = member(gg, g, &rc);
    if (!m) return rc;
  }
  FDY_HIP(hipSetDevice(a->device));
  // The exec to update: a new one while there are fewer than max_execs,
  // else the least recently selected.
  uint32_t v = 0;
  if (gg->slots.size() < gg->max_execs) {
    const auto ti = Clock::now();
    rc = add_exec(gg);
    if (rc) return rc;
    st.instantiate_us = us_since(ti);
    v = (uint32_t)gg->slots.size() - 1;
  } else {
    for (uint32_t i = 1; i < gg->slots.size(); ++i)
      if (gg->slots[i].used < gg->slots[v].used) v = i;
  }
  ExecSlot& x = gg->slots[v];
  if (x.launched) FDY_HIP(hipEventSynchronize(x.done));
  // The nodes whose params differ between the exec's graph h and g are
  // those of O_h, O_g and the two graphs' own descriptors and layouts: the
  // live image moves to h first when h is not its graph (c), so that the
  // scatters' marks cover all of them (and O_c's, which take g's params
  // too).
  const uint32_t h = x.graph;
  st.words_scattered = (a->h_ovr_off[c + 1] - a->h_ovr_off[c]) + (a->h_ovr_off[g + 1] - a->h_ovr_off[g]);
  if (h != c && h != g) {
    st.words_scattered += 2 * (a->h_ovr_off[h + 1] - a->h_ovr_off[h]);
    rc = enqueue_switch(a, h, s, gg->dirty.as<uint8_t>());
    if (rc) return rc;
  }
  rc = enqueue_switch(a, g, s, gg->dirty.as<uint8_t>());
  if (rc) return rc;
  const bool all = x.stale;
  MirrorArgs mr{};
  mr.live = a->live.as<uint64_t>() + live_base(a, t);
  mr.desc = a->ndesc.as<NodeDesc>() + a->graphs[t].node_base;
  mr.dirty = gg->dirty.as<uint8_t>();
  mr.h_live = gg->d_live;
  mr.h_dirty = gg->d_dirty;
  mr.num_nodes = gg->N;
  mr.all = all ? 1 : 0;
  FDY_HIP(launch_mirror(mr, s));
  FDY_HIP(hipStreamSynchronize(s));
  const auto tr = Clock::now();
  x.stale = true;  // until every node below is set
  gg->cur = v;
  for (uint32_t n = 0; n < gg->N; ++n) {
    if (!gg->h_dirty[n]) continue;
    gg->h_dirty[n] = 0;
    const int32_t k = m ? m->own[n] : -1;
    if (k >= 0) rc = apply_update(x.exec, gg->nodes[n], *m->set.u[k], m->set.params.data());
    else rc = apply_update(x.exec, gg->nodes[n], *gg->tset.u[n], gg->tset.params.data());
    if (rc) return rc;
    ++st.nodes_reset;
    st.kernel_nodes_reset += gg->nodes[n].type == FDY_NODE_KERNEL;
  }
  x.stale = false;
  x.graph = g;
  x.used = gg->tick;
  gg->info.current_graph = g;
  st.reset_us = us_since(tr);
  st.host_us = us_since(t0);
  if (stats_v) *static_cast<fdy_select_stats*>(stats_v) = st;
  return FDY_OK;
}

}  // namespace fdy

extern "C" {

uint64_t fdy_code_object_hash(const void* bytes, uint64_t size) {
  return crc64_xz(static_cast<const uint8_t*>(bytes), bytes ? size : 0);
}

int fdy_registry_create(fdy_registry** out) {
  if (!out) return err(FDY_E_INVALID, "null output pointer");
  auto r = std::make_unique<fdy_registry>();
  FDY_HIP(hipGetDevice(&r->device));
  *out = r.release();
  return FDY_OK;
}

int fdy_registry_destroy(fdy_registry* r) {
  delete r;
  return FDY_OK;
}

int fdy_registry_add(fdy_registry* r, const void* code_object, uint64_t size, uint64_t* hash_out) {
  if (!r || !code_object || size == 0) return err(FDY_E_INVALID, "need a registry and a non-empty code object");
  const uint64_t h = crc64_xz(static_cast<const uint8_t*>(code_object), size);
  if (hash_out) *hash_out = h;
  std::lock_guard<std::mutex> lk(r->mu);
  if (r->by_hash.count(h)) return FDY_OK;
  auto c = std::make_unique<fdy_registry::Code>();
  c->hash = h;
  c->bytes.assign(static_cast<const uint8_t*>(code_object), static_cast<const uint8_t*>(code_object) + size);
  FDY_HIP(hipSetDevice(r->device));
  hipError_t e = hipModuleLoadData(&c->mod, c->bytes.data());
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return err(FDY_E_FORMAT, std::string("hipModuleLoadData failed: ") + hipGetErrorString(e) +
                                 " (not a code object for this device?)");
  }
  r->by_hash.emplace(h, c.get());
  r->codes.push_back(std::move(c));
  return FDY_OK;
}

int fdy_registry_add_file(fdy_registry* r, const char* path, uint64_t* hash_out) {
  if (!r || !path) return err(FDY_E_INVALID, "need a registry and a path");
  FILE* f = std::fopen(path, "rb");
  if (!f) return err(FDY_E_IO, std::string("cannot open ") + path);
  std::vector<uint8_t> b;
  uint8_t buf[1 << 16];
  size_t got;
  while ((got = std::fread(buf, 1, sizeof buf, f)) > 0) b.insert(b.end(), buf, buf + got);
  const bool bad = std::ferror(f) != 0;
  std::fclose(f);
  if (bad) return err(FDY_E_IO, std::string("read error on ") + path);
  return fdy_registry_add(r, b.data(), b.size(), hash_out);
}

namespace {

// Kernel names of a code object: symbols "name.kd" (kernel descriptors)
// of the .symtab and .dynsym of its ELF64 image, every offset
// bounds-checked.  A clang offload bundle (what `hipcc --genco` writes:
// magic, entry count, then {offset, size, triple length, triple} per entry)
// is opened at its amdgcn entry.
constexpr char kBundleMagic[] = "__CLANG_OFFLOAD_BUNDLE__";

int code_object_kernels(const uint8_t* p, uint64_t n, std::vector<std::string>* out) {
  auto bad = [](const char* why) { return err(FDY_E_FORMAT, std::string("code object: ") + why); };
  constexpr uint64_t kMagic = sizeof(kBundleMagic) - 1;
  if (n >= kMagic + 8 && std::memcmp(p, kBundleMagic, kMagic) == 0) {
    uint64_t entries, at = kMagic;
    std::memcpy(&entries, p + at, 8);
    at += 8;
    for (uint64_t e = 0; e < entries; ++e) {
      if (n - at < 24) return bad("offload bundle entry out of bounds");
      uint64_t off, size, tlen;
      std::memcpy(&off, p + at, 8);
      std::memcpy(&size, p + at + 8, 8);
      std::memcpy(&tlen, p + at + 16, 8);
      at += 24;
      if (tlen > n - at) return bad("offload bundle triple out of bounds");
      const std::string triple(reinterpret_cast<const char*>(p + at), tlen);
      at += tlen;
      if (triple.find("amdgcn") == std::string::npos) continue;
      if (off > n || size > n - off) return bad("offload bundle image out of bounds");
      return code_object_kernels(p + off, size, out);
    }
    return bad("offload bundle without an amdgcn image");
  }
  if (n < sizeof(Elf64_Ehdr) || std::memcmp(p, ELFMAG, SELFMAG) != 0 || p[EI_CLASS] != ELFCLASS64)
    return bad("neither an ELF64 image nor an uncompressed offload bundle");
  Elf64_Ehdr eh;
  std::memcpy(&eh, p, sizeof eh);
  if (eh.e_shentsize != sizeof(Elf64_Shdr) || eh.e_shoff > n ||
      (uint64_t)eh.e_shnum * sizeof(Elf64_Shdr) > n - eh.e_shoff)
    return bad("section headers out of bounds");
  auto shdr = [&](uint32_t i) {
    Elf64_Shdr h;
    std::memcpy(&h, p + eh.e_shoff + (uint64_t)i * sizeof(Elf64_Shdr), sizeof h);
    return h;
  };
  std::set<std::string> names;
  for (uint32_t i = 0; i < eh.e_shnum; ++i) {
    const Elf64_Shdr sh = shdr(i);
    if (sh.sh_type != SHT_SYMTAB && sh.sh_type != SHT_DYNSYM) continue;
    if (sh.sh_link >= eh.e_shnum || sh.sh_entsize != sizeof(Elf64_Sym) || sh.sh_offset > n ||
        sh.sh_size > n - sh.sh_offset)
      return bad("symbol table out of bounds");
    const Elf64_Shdr st = shdr(sh.sh_link);
    if (st.sh_offset > n || st.sh_size > n - st.sh_offset) return bad("string table out of bounds");
    const char* strs = reinterpret_cast<const char*>(p + st.sh_offset);
    for (uint64_t k = 0; k < sh.sh_size / sizeof(Elf64_Sym); ++k) {
      Elf64_Sym sym;
      std::memcpy(&sym, p + sh.sh_offset + k * sizeof(Elf64_Sym), sizeof sym);
      if (sym.st_name >= st.sh_size) continue;
      const size_t len = strnlen(strs + sym.st_name, st.sh_size - sym.st_name);
      if (len == st.sh_size - sym.st_name) return bad("unterminated symbol name");
      const std::string nm(strs + sym.st_name, len);
      if (nm.size() > 3 && nm.compare(nm.size() - 3, 3, ".kd") == 0) names.insert(nm.substr(0, nm.size() - 3));
    }
  }
  out->assign(names.begin(), names.end());
  return FDY_OK;
}

constexpr const char* kPackedImage = "fatbin_image_packed.img";
constexpr const char* kPackedIndex = "fatbin_entrypoint_packed.txt";
constexpr const char* kPackedLoader = "hipModuleLoadData,binary_flags=0";

}  // namespace

int fdy_code_object_kernels(const void* bytes, uint64_t size, char* buf, uint64_t cap, uint64_t* len) {
  if (!bytes || !len) return err(FDY_E_INVALID, "need a code object and a length output");
  std::vector<std::string> names;
  int rc = code_object_kernels(static_cast<const uint8_t*>(bytes), size, &names);
  if (rc) return rc;
  std::string text;
  for (const auto& nm : names) text += nm + "\n";
  *len = text.size();
  if (!buf || cap < text.size()) return err(FDY_E_CAPACITY, "kernel-name buffer too small");
  std::memcpy(buf, text.data(), text.size());
  return FDY_OK;
}

int fdy_registry_pack(fdy_registry* r, const char* dir, uint32_t* n_out) {
  if (!r || !dir) return err(FDY_E_INVALID, "need a registry and a directory");
  std::error_code ec;
  std::filesystem::create_directories(dir, ec);
  if (ec) return err(FDY_E_IO, std::string("cannot create ") + dir + ": " + ec.message());
  const std::filesystem::path d(dir);
  std::ofstream img(d / kPackedImage, std::ios::binary | std::ios::trunc);
  std::ofstream txt(d / kPackedIndex, std::ios::trunc);
  if (!img || !txt) return err(FDY_E_IO, std::string("cannot write the packed pair in ") + dir);
  std::lock_guard<std::mutex> lk(r->mu);
  for (const auto& c : r->codes) {
    std::vector<std::string> names;
    int rc = code_object_kernels(c->bytes.data(), c->bytes.size(), &names);
    if (rc) return rc;
    const uint64_t hdr[2] = {c->hash, (uint64_t)c->bytes.size()};
    img.write(reinterpret_cast<const char*>(hdr), sizeof hdr);
    img.write(reinterpret_cast<const char*>(c->bytes.data()), (std::streamsize)c->bytes.size());
    char hex[20];
    std::snprintf(hex, sizeof hex, "%016llx", (unsigned long long)c->hash);
    txt << hex << "\n" << kPackedLoader << "\n" << names.size() << "\n";
    for (const auto& nm : names) txt << nm << "\n";
    txt << "---\n";
  }
  img.flush();
  txt.flush();
  if (!img || !txt) return err(FDY_E_IO, std::string("write error in ") + dir);
  if (n_out) *n_out = (uint32_t)r->codes.size();
  return FDY_OK;
}

int fdy_registry_load_packed(fdy_registry* r, const char* dir, uint32_t* n_out) {
  if (!r || !dir) return err(FDY_E_INVALID, "need a registry and a directory");
  const std::filesystem::path d(dir);
  std::ifstream img(d / kPackedImage, std::ios::binary);
  std::ifstream txt(d / kPackedIndex);
  if (!img || !txt)
    return err(FDY_E_IO, std::string("packed code objects not found in ") + dir + " (" + kPackedImage + ", " +
                             kPackedIndex + ")");
  struct Rec {
    uint64_t hash = 0;
    std::vector<uint8_t> bytes;
    std::vector<std::string> names;
  };
  std::vector<Rec> recs;
  for (;;) {
    uint64_t hdr[2];
    img.read(reinterpret_cast<char*>(hdr), sizeof hdr);
    if (img.gcount() == 0 && img.eof()) break;
    if (img.gcount() != (std::streamsize)sizeof hdr) return err(FDY_E_FORMAT, "packed image: truncated record header");
    Rec rec;
    rec.hash = hdr[0];
    if (hdr[1] == 0) return err(FDY_E_FORMAT, "packed image: empty record (link segments have no gfx950 form)");
    std::error_code ec;
    const uint64_t file_size = std::filesystem::file_size(d / kPackedImage, ec);
    if (ec || hdr[1] > file_size) return err(FDY_E_FORMAT, "packed image: record larger than the file");
    rec.bytes.resize(hdr[1]);
    img.read(reinterpret_cast<char*>(rec.bytes.data()), (std::streamsize)hdr[1]);
    if (img.gcount() != (std::streamsize)hdr[1]) return err(FDY_E_FORMAT, "packed image: truncated record");
    if (crc64_xz(rec.bytes.data(), rec.bytes.size()) != rec.hash)
      return err(FDY_E_FORMAT, "packed image: a record's bytes do not hash to its binary_hash");
    recs.push_back(std::move(rec));
  }
  // The index: hash, loader line, name count, names, "---" per record.
  std::string line;
  size_t k = 0;
  while (std::getline(txt, line)) {
    if (k >= recs.size()) return err(FDY_E_FORMAT, "packed index lists more records than the image holds");
    char* end = nullptr;
    const uint64_t h = std::strtoull(line.c_str(), &end, 16);
    if (line.size() != 16 || *end || h != recs[k].hash)
      return err(FDY_E_FORMAT, "packed index: record " + std::to_string(k) + " names another binary_hash");
    std::string loader, count;
    if (!std::getline(txt, loader) || loader.rfind("hipModuleLoadData", 0) != 0)
      return err(FDY_E_FORMAT, "packed index: record " + std::to_string(k) + " has no hipModuleLoadData line");
    if (!std::getline(txt, count) || count.empty() || count.find_first_not_of("0123456789") != std::string::npos)
      return err(FDY_E_FORMAT, "packed index: record " + std::to_string(k) + " has no name count");
    const unsigned long nn = std::stoul(count);
    for (unsigned long q = 0; q < nn; ++q) {
      if (!std::getline(txt, line)) return err(FDY_E_FORMAT, "packed index: truncated name list");
      recs[k].names.push_back(line);
    }
    if (!std::getline(txt, line) || line != "---") return err(FDY_E_FORMAT, "packed index: record without ---");
    ++k;
  }
  if (k != recs.size()) return err(FDY_E_FORMAT, "packed index lists fewer records than the image holds");
  for (const auto& rec : recs) {
    uint64_t h = 0;
    int rc = fdy_registry_add(r, rec.bytes.data(), rec.bytes.size(), &h);
    if (rc) return rc;
    for (const auto& nm : rec.names) {
      hipFunction_t fn = nullptr;
      rc = registry_lookup(r, h, nm.c_str(), nm.size(), &fn);
      if (rc) return err(FDY_E_FORMAT, "packed index names kernel '" + nm + "', which its code object lacks");
    }
  }
  if (n_out) *n_out = (uint32_t)recs.size();
  return FDY_OK;
}

int fdy_registry_lookup(fdy_registry* r, uint64_t hash, const char* name, void** fn) {
  if (!r || !name || !fn) return err(FDY_E_INVALID, "need a registry, a name and an output pointer");
  hipFunction_t f = nullptr;
  int rc = registry_lookup(r, hash, name, std::strlen(name), &f);
  if (rc) return rc;
  *fn = reinterpret_cast<void*>(f);
  return FDY_OK;
}

int fdy_registry_global(fdy_registry* r, uint64_t hash, const char* name, void** dptr, uint64_t* bytes) {
  if (!r || !name || !dptr) return err(FDY_E_INVALID, "need a registry, a name and an output pointer");
  std::lock_guard<std::mutex> lk(r->mu);
  auto c = r->by_hash.find(hash);
  if (c == r->by_hash.end()) return err(FDY_E_NOT_FOUND, "no code object with that binary_hash is registered");
  hipDeviceptr_t p = nullptr;
  size_t sz = 0;
  FDY_HIP(hipSetDevice(r->device));
  hipError_t e = hipModuleGetGlobal(&p, &sz, c->second->mod, name);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return err(FDY_E_NOT_FOUND, std::string("the code object has no global '") + name + "'");
  }
  *dptr = p;
  if (bytes) *bytes = sz;
  return FDY_OK;
}

int fdy_group_graph_create(fdy_archive* a, uint32_t t, fdy_registry* r, void* stream, fdy_group_graph** out) {
  if (!a || !r || !out) return err(FDY_E_INVALID, "need an archive, a registry and an output pointer");
  *out = nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = check_graph(a, t);
  if (!rc) rc = ensure_cache(a, s);
  if (rc) return rc;
  if (a->h_tmpl[t] != t) return err(FDY_E_INVALID, "graph " + std::to_string(t) + " is not a template");
  if (a->h_status[t] & (FDY_GRAPH_BAD_PARAMS | FDY_GRAPH_OVERFLOW))
    return err(FDY_E_FORMAT, "template " + std::to_string(t) + " has ranges outside its sections");
  if (a->bound.size() != a->G) a->bound.assign(a->G, nullptr);
  if (a->bound[t]) return err(FDY_E_STATE, "template " + std::to_string(t) + " already has a group graph");
  FDY_HIP(hipSetDevice(a->device));
  // Serving from here on: overrides packed, template live images only.
  rc = compact_for_serving(a, s);
  if (rc) return rc;
  // The exec starts from the template's params: move the live image back first.
  rc = enqueue_switch(a, t, s, nullptr);
  if (rc) return rc;
  FDY_HIP(hipStreamSynchronize(s));
  auto gg = std::make_unique<fdy_group_graph>();
  gg->a = a;
  gg->reg = r;
  gg->t = t;
  rc = build(gg.get());
  if (rc) return rc;
  a->bound[t] = gg.get();
  ++a->num_bound;
  *out = gg.release();
  return FDY_OK;
}

int fdy_group_graph_destroy(fdy_group_graph* gg) {
  if (!gg) return FDY_OK;
  fdy_archive* a = gg->a;
  if (a && a->bound.size() == a->G && a->bound[gg->t] == gg) {
    a->bound[gg->t] = nullptr;
    --a->num_bound;
  }
  delete gg;
  return FDY_OK;
}

int fdy_group_graph_select(fdy_group_graph* gg, uint32_t graph, void* stream, fdy_select_stats* stats) {
  if (!gg) return err(FDY_E_INVALID, "null group graph");
  return group_graph_select(gg, graph, static_cast<hipStream_t>(stream), stats);
}

int fdy_group_graph_reset_all(fdy_group_graph* gg, void* stream, fdy_select_stats* stats) {
  if (!gg) return err(FDY_E_INVALID, "null group graph");
  // The current exec re-set from its graph, every node (the other execs stay).
  ExecSlot& x = gg->slots[gg->cur];
  x.stale = true;
  x.used = 0;  // the least recently selected: the update below takes it
  for (ExecSlot& y : gg->slots)
    if (&y != &x) y.used = std::max<uint64_t>(y.used, 1);
  const uint32_t keep = gg->max_execs;
  gg->max_execs = (uint32_t)gg->slots.size();  // no new exec for this
  const int rc = group_graph_select(gg, x.graph, static_cast<hipStream_t>(stream), stats);
  gg->max_execs = keep;
  return rc;
}

int fdy_group_graph_set_exec_cache(fdy_group_graph* gg, uint32_t max_execs) {
  if (!gg) return err(FDY_E_INVALID, "null group graph");
  if (max_execs == 0) return err(FDY_E_INVALID, "a group graph keeps at least one exec");
  FDY_HIP(hipSetDevice(gg->a->device));
  // Execs past the new limit go, least recently selected first; the current one stays.
  while (gg->slots.size() > max_execs) {
    uint32_t v = gg->cur == 0 ? 1 : 0;
    for (uint32_t i = 0; i < gg->slots.size(); ++i)
      if (i != gg->cur && gg->slots[i].used < gg->slots[v].used) v = i;
    ExecSlot& x = gg->slots[v];
    if (x.launched) FDY_HIP(hipEventSynchronize(x.done));
    FDY_HIP(hipGraphExecDestroy(x.exec));
    FDY_HIP(hipEventDestroy(x.done));
    gg->slots.erase(gg->slots.begin() + v);
    if (gg->cur > v) --gg->cur;
  }
  gg->max_execs = max_execs;
  gg->info.num_execs = (uint32_t)gg->slots.size();
  return FDY_OK;
}

int fdy_group_graph_launch(fdy_group_graph* gg, void* stream) {
  if (!gg) return err(FDY_E_INVALID, "null group graph");
  ExecSlot& x = gg->slots[gg->cur];
  if (x.stale) return err(FDY_E_STATE, "the last select failed part-way; select a graph again before launching");
  hipStream_t s = static_cast<hipStream_t>(stream);
  FDY_HIP(hipSetDevice(gg->a->device));
  FDY_HIP(hipGraphLaunch(x.exec, s));
  FDY_HIP(hipEventRecord(x.done, s));
  x.launched = true;
  return FDY_OK;
}

int fdy_group_graph_handles(fdy_group_graph* gg, void** graph, void** exec) {
  if (!gg) return err(FDY_E_INVALID, "null group graph");
  if (graph) *graph = gg->graph;
  if (exec) *exec = gg->slots[gg->cur].exec;
  return FDY_OK;
}

int fdy_group_graph_debug_dot(fdy_group_graph* gg, const char* path) {
  if (!gg || !path) return err(FDY_E_INVALID, "need a group graph and a path");
  FDY_HIP(hipSetDevice(gg->a->device));
  FDY_HIP(hipGraphDebugDotPrint(gg->graph, path, hipGraphDebugDotFlagsVerbose));
  return FDY_OK;
}

int fdy_group_graph_info_get(fdy_group_graph* gg, fdy_group_graph_info* out) {
  if (!gg || !out) return err(FDY_E_INVALID, "need a group graph and an output pointer");
  *out = gg->info;
  return FDY_OK;
}

}  // extern "C"
