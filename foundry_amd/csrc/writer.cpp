// writer.cpp -- the .cugraph v1 archive of one graph's JSON document.
//
// The document is the object a graph is saved as (csrc/CUDAGraph.cpp:
// 1389-1491: nodes, dependencies, generators, allocator_events,
// output_tensors, topology_key, common_kernel_node_attrs), and the archive
// is the one CUDAGraph::save_binary writes for it (csrc/BinaryGraphIO.cpp:
// 15-371), byte for byte:
//   - function names interned in first-use order, each NUL-terminated
//     (24-36); num_strings counts distinct names (336);
//   - one 168-B entry per node in document order, zero-filled, with the
//     fields of its type (149-264); an unknown type string leaves an entry
//     of type 0 (kernel) with a zero body;
//   - kernel params: a value_hex param is hex-decoded into the param-data
//     section, two characters per byte through strtoul (48-53), with size
//     = half the string length; a param without value_hex keeps its
//     offset/size (197-201); a non-empty extra_argBuffer_hex goes to the
//     arg section, else the arg offset is 0xFFFFFFFF (205-216);
//   - kernel_node_attrs and common_kernel_node_attrs set a flag bit per
//     attribute present (55-137);
//   - allocator_events / output_tensors are the serialised JSON of those
//     members (compact, members in document order), empty when absent
//     (283-287);
//   - sections in id order, each 8-byte aligned after the 64-B header and the
//     11-entry directory (289-315); header flags for common attrs, non-empty
//     dependencies, events, outputs and generators (325-336).
// Errors the reference raises as exceptions (a missing member, a value of
// the wrong type or out of range for its field, a hex pair strtoul cannot
// read) fail with FDY_E_FORMAT here.  Two things the reference never meets
// in documents it writes are refused rather than guessed: duplicate object
// keys, and non-integer numbers inside the two serialised members.
#include "writer.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <unordered_map>

#include "../../include/fdy_format.h"
#include "../../include/foundry_restore.h"
#include "json_min.h"

namespace fdy {
namespace {

using json::Value;

struct Fail {
  int code;
  std::string what;
};

[[noreturn]] void fail(const std::string& what, int code = FDY_E_FORMAT) { throw Fail{code, what}; }

const Value& at(const Value& o, const char* key, const char* where) {
  if (o.kind != Value::Object) fail(std::string(where) + " is not an object");
  const Value* v = o.get(key);
  if (!v) fail(std::string(where) + " has no \"" + key + "\"");
  return *v;
}

bool has(const Value& o, const char* key) { return o.kind == Value::Object && o.get(key) != nullptr; }

const std::string& as_string(const Value& v, const char* what) {
  if (v.kind != Value::String) fail(std::string(what) + " is not a string");
  return v.s;
}

const std::vector<Value>& as_array(const Value& v, const char* what) {
  if (v.kind != Value::Array) fail(std::string(what) + " is not an array");
  return v.items;
}

// The value as integer type T when it holds that integer exactly: a signed
// or unsigned integer in T's range, or a whole double in range.
template <typename T>
T to_num(const Value& v, const char* what) {
  if (v.kind != Value::Number) fail(std::string(what) + " is not a number");
  using L = std::numeric_limits<T>;
  switch (v.num) {
    case Value::Int:
      if (v.i < 0 ? (!L::is_signed || v.i < (int64_t)L::min()) : (uint64_t)v.i > (uint64_t)L::max())
        fail(std::string(what) + " is out of range");
      return (T)v.i;
    case Value::Uint:
      if (v.u > (uint64_t)L::max()) fail(std::string(what) + " is out of range");
      return (T)v.u;
    default: {
      const double d = std::strtod(v.s.c_str(), nullptr);
      const double hi = std::ldexp(1.0, L::digits);  // 2^bits (exclusive)
      const double lo = L::is_signed ? -hi : 0.0;
      if (!std::isfinite(d) || d != std::trunc(d) || d < lo || d >= hi) fail(std::string(what) + " is not exact");
      return (T)d;
    }
  }
}

bool as_bool(const Value& v, const char* what) {
  if (v.kind != Value::Bool) fail(std::string(what) + " is not a bool");
  return v.b;
}

// Duplicate keys have no single meaning; documents written by a graph save
// never hold them.
void check_unique_keys(const Value& v, int depth = 0) {
  if (v.kind == Value::Object) {
    std::unordered_map<std::string, int> seen;
    for (const auto& m : v.members) {
      if (!seen.emplace(m.first, 0).second) fail("duplicate key \"" + m.first + "\"");
      check_unique_keys(m.second, depth + 1);
    }
  } else if (v.kind == Value::Array) {
    for (const auto& x : v.items) check_unique_keys(x, depth + 1);
  }
}

void serialize_string(const std::string& str, std::string& out) {
  static const char hex[] = "0123456789abcdef";
  out.push_back('"');
  for (unsigned char c : str) {
    if (c == '"') out += "\\\"";
    else if (c == '\\') out += "\\\\";
    else if (c == '\b') out += "\\b";
    else if (c == '\t') out += "\\t";
    else if (c == '\n') out += "\\n";
    else if (c == '\f') out += "\\f";
    else if (c == '\r') out += "\\r";
    else if (c < 0x20) {
      out += "\\u00";
      out.push_back(hex[c >> 4]);
      out.push_back(hex[c & 15]);
    } else {
      out.push_back((char)c);
    }
  }
  out.push_back('"');
}

// Compact serialisation: no whitespace, members in document order, '"' and
// '\' escaped, control characters as \b \t \n \f \r or \u00xx (lower-case
// hex), all other bytes as they are; integers in decimal.
void serialize(const Value& v, std::string& out) {
  switch (v.kind) {
    case Value::Null: out += "null"; return;
    case Value::Bool: out += v.b ? "true" : "false"; return;
    case Value::Number:
      if (v.num == Value::Int) out += std::to_string(v.i);
      else if (v.num == Value::Uint) out += std::to_string(v.u);
      else fail("a non-integer number in a serialised member (" + v.s + ")", FDY_E_UNSUPPORTED);
      return;
    case Value::String:
      serialize_string(v.s, out);
      return;
    case Value::Array:
      out.push_back('[');
      for (size_t i = 0; i < v.items.size(); ++i) {
        if (i) out.push_back(',');
        serialize(v.items[i], out);
      }
      out.push_back(']');
      return;
    case Value::Object:
      out.push_back('{');
      for (size_t i = 0; i < v.members.size(); ++i) {
        if (i) out.push_back(',');
        serialize_string(v.members[i].first, out);
        out.push_back(':');
        serialize(v.members[i].second, out);
      }
      out.push_back('}');
      return;
  }
}

// Two hex characters per byte, each pair read as strtoul reads it (a final
// odd character alone); a pair it cannot read is an error.
void hex_decode(const std::string& hex, std::vector<uint8_t>& out) {
  for (size_t j = 0; j < hex.size(); j += 2) {
    char buf[3] = {hex[j], j + 1 < hex.size() ? hex[j + 1] : '\0', '\0'};
    char* end = nullptr;
    const unsigned long x = std::strtoul(buf, &end, 16);
    if (end == buf) fail("value_hex holds an unreadable pair \"" + std::string(buf) + "\"");
    out.push_back((uint8_t)x);
  }
}

// The launch attributes present in `o` (a kernel_node_attrs or
// common_kernel_node_attrs object), into a kernel body's kna fields.
void parse_kna(const Value& o, fdy_kernel_body& k) {
  if (o.kind != Value::Object) fail("kernel node attrs are not an object");
  k.kna_flags = 0;
  if (has(o, "attrQueryAvailable")) {
    k.kna_flags |= FDY_KNA_ATTR_QUERY_AVAILABLE;
    k.kna_attr_query_available = as_bool(at(o, "attrQueryAvailable", "attrs"), "attrQueryAvailable") ? 1 : 0;
  }
  if (has(o, "clusterDimX")) {
    k.kna_flags |= FDY_KNA_CLUSTER_DIM;
    k.kna_cluster[0] = to_num<uint32_t>(at(o, "clusterDimX", "attrs"), "clusterDimX");
    k.kna_cluster[1] = to_num<uint32_t>(at(o, "clusterDimY", "attrs"), "clusterDimY");
    k.kna_cluster[2] = to_num<uint32_t>(at(o, "clusterDimZ", "attrs"), "clusterDimZ");
  }
  if (has(o, "preferredClusterDimX")) {
    k.kna_flags |= FDY_KNA_PREFERRED_CLUSTER_DIM;
    k.kna_preferred_cluster[0] = to_num<uint32_t>(at(o, "preferredClusterDimX", "attrs"), "preferredClusterDimX");
    k.kna_preferred_cluster[1] = to_num<uint32_t>(at(o, "preferredClusterDimY", "attrs"), "preferredClusterDimY");
    k.kna_preferred_cluster[2] = to_num<uint32_t>(at(o, "preferredClusterDimZ", "attrs"), "preferredClusterDimZ");
  }
  if (has(o, "clusterSchedulingPolicyPreference")) {
    k.kna_flags |= FDY_KNA_CLUSTER_SCHEDULING;
    k.kna_cluster_sched = to_num<int32_t>(at(o, "clusterSchedulingPolicyPreference", "attrs"), "clusterSchedulingPolicyPreference");
  }
  if (has(o, "cooperative")) {
    k.kna_flags |= FDY_KNA_COOPERATIVE;
    k.kna_cooperative = to_num<int32_t>(at(o, "cooperative", "attrs"), "cooperative");
  }
  if (has(o, "priority")) {
    k.kna_flags |= FDY_KNA_PRIORITY;
    k.kna_priority = to_num<int32_t>(at(o, "priority", "attrs"), "priority");
  }
  if (has(o, "memSyncDomain")) {
    k.kna_flags |= FDY_KNA_MEM_SYNC_DOMAIN;
    k.kna_mem_sync_domain = to_num<int32_t>(at(o, "memSyncDomain", "attrs"), "memSyncDomain");
  }
  if (has(o, "memSyncDomainMapDefault")) {
    k.kna_flags |= FDY_KNA_MEM_SYNC_DOMAIN_MAP;
    k.kna_mem_sync_map_default = (uint8_t)to_num<int32_t>(at(o, "memSyncDomainMapDefault", "attrs"), "memSyncDomainMapDefault");
    k.kna_mem_sync_map_remote = (uint8_t)to_num<int32_t>(at(o, "memSyncDomainMapRemote", "attrs"), "memSyncDomainMapRemote");
  }
  if (has(o, "preferredSharedMemCarveout")) {
    k.kna_flags |= FDY_KNA_SHARED_MEM_CARVEOUT;
    k.kna_preferred_carveout = to_num<uint32_t>(at(o, "preferredSharedMemCarveout", "attrs"), "preferredSharedMemCarveout");
  }
}

template <typename T>
void put(std::vector<uint8_t>& out, const T& x) {
  const auto* p = reinterpret_cast<const uint8_t*>(&x);
  out.insert(out.end(), p, p + sizeof(T));
}

// The key the LOAD path groups a graph read from its JSON document by
// (csrc/CUDAGraphParallel.cpp:1791-1841): its topology_key when that is a
// non-empty string, else the key recomputed from its nodes -- each node's
// type string, and for a KernelNode ":C<x>_<y>_<z>" (or ":0" when all are 0)
// with the cluster dims taken from the node's kernel_node_attrs when they
// hold clusterDimX, else from common_kernel_node_attrs when x is still 0,
// else, when x is still 0, from whichever required_cluster_* fields the
// node's func_attrs hold.  Values are read as unsigned 32-bit integers.
std::string load_key(const Value& root) {
  if (root.kind != Value::Object) fail("the graph document is not an object");
  if (has(root, "topology_key")) {
    const std::string& k = as_string(at(root, "topology_key", "graph"), "topology_key");
    if (!k.empty()) return k;
  }
  const auto& nodes = as_array(at(root, "nodes", "graph"), "nodes");
  std::string key;
  key.reserve(nodes.size() * 14);
  auto dims = [](const Value& o, uint32_t c[3]) {
    c[0] = to_num<uint32_t>(at(o, "clusterDimX", "attrs"), "clusterDimX");
    c[1] = to_num<uint32_t>(at(o, "clusterDimY", "attrs"), "clusterDimY");
    c[2] = to_num<uint32_t>(at(o, "clusterDimZ", "attrs"), "clusterDimZ");
  };
  for (size_t n = 0; n < nodes.size(); ++n) {
    if (n) key += ',';
    const Value& no = nodes[n];
    const std::string& type = as_string(at(no, "type", "node"), "node type");
    key += type;
    if (type != "KernelNode") continue;
    uint32_t c[3] = {0, 0, 0};
    const Value& p = at(no, "params", "node");
    if (p.kind != Value::Object) fail("kernel params are not an object");
    if (has(p, "kernel_node_attrs")) {
      const Value& kna = at(p, "kernel_node_attrs", "params");
      if (kna.kind != Value::Object) fail("kernel_node_attrs is not an object");
      if (has(kna, "clusterDimX")) dims(kna, c);
    }
    if (c[0] == 0 && has(root, "common_kernel_node_attrs")) {
      const Value& ck = at(root, "common_kernel_node_attrs", "graph");
      if (ck.kind != Value::Object) fail("common_kernel_node_attrs is not an object");
      if (has(ck, "clusterDimX")) dims(ck, c);
    }
    if (c[0] == 0 && has(p, "func_attrs")) {
      const Value& fa = at(p, "func_attrs", "params");
      if (fa.kind != Value::Object) fail("func_attrs is not an object");
      if (has(fa, "required_cluster_width"))
        c[0] = to_num<uint32_t>(at(fa, "required_cluster_width", "func_attrs"), "required_cluster_width");
      if (has(fa, "required_cluster_height"))
        c[1] = to_num<uint32_t>(at(fa, "required_cluster_height", "func_attrs"), "required_cluster_height");
      if (has(fa, "required_cluster_depth"))
        c[2] = to_num<uint32_t>(at(fa, "required_cluster_depth", "func_attrs"), "required_cluster_depth");
    }
    if (c[0] || c[1] || c[2])
      key += ":C" + std::to_string(c[0]) + "_" + std::to_string(c[1]) + "_" + std::to_string(c[2]);
    else
      key += ":0";
  }
  return key;
}

// key_override: the TOPOLOGY_KEY section's bytes instead of topology_key.
void build(const Value& root, std::vector<uint8_t>& out, const std::string* key_override) {
  if (root.kind != Value::Object) fail("the graph document is not an object");
  check_unique_keys(root);
  const auto& nodes = as_array(at(root, "nodes", "graph"), "nodes");
  static const std::vector<Value> kNone;
  const auto& deps = has(root, "dependencies") ? as_array(at(root, "dependencies", "graph"), "dependencies") : kNone;
  const auto& gens = as_array(at(root, "generators", "graph"), "generators");

  std::vector<uint8_t> strings;
  std::unordered_map<std::string, uint32_t> interned;
  auto intern = [&](const std::string& s) -> uint32_t {
    auto it = interned.find(s);
    if (it != interned.end()) return it->second;
    const uint32_t off = (uint32_t)strings.size();
    strings.insert(strings.end(), s.begin(), s.end());
    strings.push_back(0);
    interned.emplace(s, off);
    return off;
  };
  const std::string key = key_override ? *key_override
                         : has(root, "topology_key") ? as_string(at(root, "topology_key", "graph"), "topology_key")
                                                     : "";

  const bool has_common = has(root, "common_kernel_node_attrs");
  fdy_common_attrs common{};
  if (has_common) {
    fdy_kernel_body tmp{};
    parse_kna(at(root, "common_kernel_node_attrs", "graph"), tmp);
    common.flags = tmp.kna_flags;
    std::memcpy(common.cluster, tmp.kna_cluster, sizeof common.cluster);
    std::memcpy(common.preferred_cluster, tmp.kna_preferred_cluster, sizeof common.preferred_cluster);
    common.cluster_sched = tmp.kna_cluster_sched;
    common.cooperative = tmp.kna_cooperative;
    common.priority = tmp.kna_priority;
    common.mem_sync_domain = tmp.kna_mem_sync_domain;
    common.mem_sync_map_default = tmp.kna_mem_sync_map_default;
    common.mem_sync_map_remote = tmp.kna_mem_sync_map_remote;
    common.attr_query_available = tmp.kna_attr_query_available;
    common.preferred_carveout = tmp.kna_preferred_carveout;
  }

  std::vector<fdy_node> entries;
  std::vector<fdy_param> pindex;
  std::vector<uint8_t> pdata, adata;
  entries.reserve(nodes.size());
  for (const Value& no : nodes) {
    fdy_node e;
    std::memset(&e, 0, sizeof e);
    e.node_id = to_num<uint32_t>(at(no, "id", "node"), "node id");
    const std::string& type = as_string(at(no, "type", "node"), "node type");
    if (type == "KernelNode") {
      e.type = FDY_NODE_KERNEL;
      const Value& p = at(no, "params", "node");
      if (p.kind != Value::Object) fail("kernel params are not an object");
      fdy_kernel_body& k = e.u.kernel;
      k.block[0] = to_num<uint32_t>(at(p, "blockDimX", "params"), "blockDimX");
      k.block[1] = to_num<uint32_t>(at(p, "blockDimY", "params"), "blockDimY");
      k.block[2] = to_num<uint32_t>(at(p, "blockDimZ", "params"), "blockDimZ");
      k.grid[0] = to_num<uint32_t>(at(p, "gridDimX", "params"), "gridDimX");
      k.grid[1] = to_num<uint32_t>(at(p, "gridDimY", "params"), "gridDimY");
      k.grid[2] = to_num<uint32_t>(at(p, "gridDimZ", "params"), "gridDimZ");
      k.shared_mem_bytes = to_num<uint32_t>(at(p, "sharedMemBytes", "params"), "sharedMemBytes");
      const std::string& fn = as_string(at(p, "function_name", "params"), "function_name");
      k.name_offset = intern(fn);
      k.name_length = (uint32_t)fn.size();
      k.binary_hash = to_num<uint64_t>(at(p, "kernel_source_binary_hash", "params"), "kernel_source_binary_hash");
      if (has(p, "func_attrs")) {
        const Value& fa = at(p, "func_attrs", "params");
        k.max_dynamic_shared = to_num<int32_t>(at(fa, "max_dynamic_shared_size_bytes", "func_attrs"), "max_dynamic_shared_size_bytes");
        k.preferred_carveout = to_num<int32_t>(at(fa, "preferred_shared_memory_carveout", "func_attrs"), "preferred_shared_memory_carveout");
        auto opt = [&](const char* name) -> int32_t { return has(fa, name) ? to_num<int32_t>(at(fa, name, "func_attrs"), name) : 0; };
        k.cluster_sched_pref = opt("cluster_scheduling_policy_preference");
        k.required_cluster[0] = opt("required_cluster_width");
        k.required_cluster[1] = opt("required_cluster_height");
        k.required_cluster[2] = opt("required_cluster_depth");
      }
      if (has(p, "kernel_node_attrs")) parse_kna(at(p, "kernel_node_attrs", "params"), k);
      k.param_index_offset = (uint32_t)(pindex.size() * sizeof(fdy_param));
      const auto& kps = as_array(at(p, "kernelParams", "params"), "kernelParams");
      k.num_params = (uint32_t)kps.size();
      for (const Value& kp : kps) {
        if (kp.kind != Value::Object) fail("a kernel param is not an object");
        fdy_param pe{};
        if (has(kp, "value_hex")) {
          const std::string& hex = as_string(at(kp, "value_hex", "param"), "value_hex");
          pe.data_offset = (uint32_t)pdata.size();
          pe.size = (uint32_t)(hex.size() / 2);
          hex_decode(hex, pdata);
        } else {
          pe.data_offset = to_num<uint32_t>(at(kp, "offset", "param"), "param offset");
          pe.size = to_num<uint32_t>(at(kp, "size", "param"), "param size");
        }
        pindex.push_back(pe);
      }
      const std::string extra =
          has(p, "extra_argBuffer_hex") ? as_string(at(p, "extra_argBuffer_hex", "params"), "extra_argBuffer_hex") : "";
      if (!extra.empty()) {
        k.arg_offset = (uint32_t)adata.size();
        k.arg_size = (uint32_t)(extra.size() / 2);
        hex_decode(extra, adata);
      } else {
        k.arg_offset = FDY_NO_ARG_BUFFER;
        k.arg_size = 0;
      }
    } else if (type == "MemcpyNode") {
      e.type = FDY_NODE_MEMCPY;
      const Value& p = at(no, "params", "node");
      fdy_memcpy_body& m = e.u.memcpy;
      auto u64 = [&](const char* name) { return to_num<uint64_t>(at(p, name, "params"), name); };
      m.depth = u64("Depth");
      m.height = u64("Height");
      m.width_bytes = u64("WidthInBytes");
      m.dst = u64("dstDevice");
      m.dst_height = u64("dstHeight");
      m.dst_lod = u64("dstLOD");
      m.dst_mem_type = to_num<int32_t>(at(p, "dstMemoryType", "params"), "dstMemoryType");
      m.dst_pitch = u64("dstPitch");
      m.dst_x_bytes = u64("dstXInBytes");
      m.dst_y = u64("dstY");
      m.dst_z = u64("dstZ");
      m.src = u64("srcDevice");
      m.src_height = u64("srcHeight");
      m.src_lod = u64("srcLOD");
      m.src_mem_type = to_num<int32_t>(at(p, "srcMemoryType", "params"), "srcMemoryType");
      m.src_pitch = u64("srcPitch");
      m.src_x_bytes = u64("srcXInBytes");
      m.src_y = u64("srcY");
      m.src_z = u64("srcZ");
    } else if (type == "MemsetNode") {
      e.type = FDY_NODE_MEMSET;
      const Value& p = at(no, "params", "node");
      fdy_memset_body& m = e.u.memset;
      m.dst = to_num<uint64_t>(at(p, "dst", "params"), "dst");
      m.element_size = to_num<uint32_t>(at(p, "elementSize", "params"), "elementSize");
      m.height = to_num<uint64_t>(at(p, "height", "params"), "height");
      m.pitch = to_num<uint64_t>(at(p, "pitch", "params"), "pitch");
      m.value = to_num<uint32_t>(at(p, "value", "params"), "value");
      m.width = to_num<uint64_t>(at(p, "width", "params"), "width");
    } else if (type == "EventRecordNode" || type == "EventWaitNode") {
      e.type = type == "EventRecordNode" ? FDY_NODE_EVENT_RECORD : FDY_NODE_EVENT_WAIT;
      e.u.event.event_id = to_num<int32_t>(at(at(no, "params", "node"), "event_id", "params"), "event_id");
    } else if (type == "EmptyNode") {
      e.type = FDY_NODE_EMPTY;
    }
    entries.push_back(e);
  }

  std::vector<fdy_dep> dv;
  dv.reserve(deps.size());
  for (const Value& d : deps) dv.push_back({to_num<uint32_t>(at(d, "from", "dependency"), "from"), to_num<uint32_t>(at(d, "to", "dependency"), "to")});
  std::vector<fdy_generator> gv;
  gv.reserve(gens.size());
  for (const Value& g : gens)
    gv.push_back({to_num<uint64_t>(at(g, "id", "generator"), "generator id"), to_num<uint64_t>(at(g, "seed", "generator"), "seed"),
                  to_num<uint64_t>(at(g, "wholegraph_increment", "generator"), "wholegraph_increment")});

  std::string events, outputs;
  if (has(root, "allocator_events")) serialize(at(root, "allocator_events", "graph"), events);
  if (has(root, "output_tensors")) serialize(at(root, "output_tensors", "graph"), outputs);

  struct Part {
    const void* p;
    uint64_t n;
  };
  const Part parts[FDY_SEC_COUNT] = {
      {strings.data(), strings.size()},
      {entries.data(), entries.size() * sizeof(fdy_node)},
      {dv.data(), dv.size() * sizeof(fdy_dep)},
      {pindex.data(), pindex.size() * sizeof(fdy_param)},
      {pdata.data(), pdata.size()},
      {adata.data(), adata.size()},
      {&common, has_common ? (uint64_t)sizeof(fdy_common_attrs) : 0},
      {gv.data(), gv.size() * sizeof(fdy_generator)},
      {events.data(), events.size()},
      {outputs.data(), outputs.size()},
      {key.data(), key.size()},
  };
  fdy_section dir[FDY_SEC_COUNT];
  std::memset(dir, 0, sizeof dir);
  uint64_t off = sizeof(fdy_file_header) + sizeof dir;
  for (uint32_t s = 0; s < FDY_SEC_COUNT; ++s) {
    dir[s].id = s;
    dir[s].offset = off;
    dir[s].size = parts[s].n;
    off = (off + parts[s].n + 7) & ~7ull;
  }
  fdy_file_header h;
  std::memset(&h, 0, sizeof h);
  std::memcpy(h.magic, "CUGRAPH", 8);
  h.version = FDY_FORMAT_VERSION;
  h.flags = (has_common ? FDY_HAS_COMMON_ATTRS : 0u) | (!dv.empty() ? FDY_HAS_DEPS : 0u) |
            (!events.empty() ? FDY_HAS_ALLOC_EVENTS : 0u) | (!outputs.empty() ? FDY_HAS_OUTPUT_TENSORS : 0u) |
            (!gv.empty() ? FDY_HAS_GENERATORS : 0u);
  h.num_nodes = (uint32_t)entries.size();
  h.num_deps = (uint32_t)dv.size();
  h.num_generators = (uint32_t)gv.size();
  h.num_sections = FDY_SEC_COUNT;
  h.num_strings = (uint32_t)interned.size();

  out.clear();
  out.reserve(off);
  put(out, h);
  put(out, dir);
  for (uint32_t s = 0; s < FDY_SEC_COUNT; ++s) {
    const auto* p = static_cast<const uint8_t*>(parts[s].p);
    if (parts[s].n) out.insert(out.end(), p, p + parts[s].n);
    out.resize((out.size() + 7) & ~(size_t)7, 0);
  }
}

}  // namespace

namespace {

// Parse `text` and run f(root); errors as FDY_E_* codes.
template <typename F>
int with_document(const char* text, size_t len, std::string& error, F&& fn) {
  json::Value root;
  json::Reader rd(text, len);
  if (!rd.parse(root, error)) {
    error = "graph document: " + error;
    return FDY_E_FORMAT;
  }
  try {
    fn(root);
  } catch (const Fail& f) {
    error = "graph document: " + f.what;
    return f.code;
  } catch (const std::bad_alloc&) {
    error = "graph document: out of host memory";
    return FDY_E_NOMEM;
  }
  return 0;
}

}  // namespace

int cugraph_from_json(const char* text, size_t len, std::vector<uint8_t>& out, std::string& error) {
  return with_document(text, len, error, [&](const Value& root) { build(root, out, nullptr); });
}

int load_topology_key(const char* text, size_t len, std::string& key, std::string& error) {
  return with_document(text, len, error, [&](const Value& root) { key = load_key(root); });
}

int cugraph_for_load(const char* text, size_t len, std::vector<uint8_t>& out, std::string& error) {
  return with_document(text, len, error, [&](const Value& root) {
    const std::string key = load_key(root);
    build(root, out, &key);
  });
}

}  // namespace fdy
