// cugraph.cpp -- `.cugraph` v1 writer, validator and topology-key rule.
#include "cugraph.h"

#include <cstring>
#include <unordered_map>

namespace fdy {

namespace {

constexpr uint8_t kMagic[8] = {'C', 'U', 'G', 'R', 'A', 'P', 'H', '\0'};

uint64_t align8(uint64_t v) { return (v + 7) & ~uint64_t(7); }

template <typename T>
void append_bytes(std::vector<uint8_t>& out, const T* p, size_t n) {
  const uint8_t* b = reinterpret_cast<const uint8_t*>(p);
  out.insert(out.end(), b, b + n * sizeof(T));
}

}  // namespace

const char* node_type_name(uint8_t type) {
  switch (type) {
    case FDY_NODE_KERNEL: return "KernelNode";
    case FDY_NODE_MEMSET: return "MemsetNode";
    case FDY_NODE_MEMCPY: return "MemcpyNode";
    case FDY_NODE_EVENT_RECORD: return "EventRecordNode";
    case FDY_NODE_EVENT_WAIT: return "EventWaitNode";
    case FDY_NODE_EMPTY: return "EmptyNode";
    default: return "";
  }
}

std::string topology_key_save_rule(const GraphSpec& g) {
  std::string key;
  key.reserve(g.nodes.size() * 16);
  for (size_t n = 0; n < g.nodes.size(); ++n) {
    if (n) key += ',';
    const NodeSpec& s = g.nodes[n];
    key += node_type_name(s.type);
    if (s.type != FDY_NODE_KERNEL) continue;
    uint32_t c[3] = {0, 0, 0};
    if (s.kernel.kna_flags & FDY_KNA_CLUSTER_DIM) {
      c[0] = s.kernel.kna_cluster[0];
      c[1] = s.kernel.kna_cluster[1];
      c[2] = s.kernel.kna_cluster[2];
    }
    // The SAVE side always records func_attrs, so a zero x dimension falls
    // through to the function's required cluster size (all three fields).
    if (c[0] == 0) {
      c[0] = static_cast<uint32_t>(s.kernel.required_cluster[0]);
      c[1] = static_cast<uint32_t>(s.kernel.required_cluster[1]);
      c[2] = static_cast<uint32_t>(s.kernel.required_cluster[2]);
    }
    if (c[0] || c[1] || c[2]) {
      key += ":C" + std::to_string(c[0]) + "_" + std::to_string(c[1]) + "_" + std::to_string(c[2]);
    } else {
      key += ":0";
    }
  }
  return key;
}

std::vector<uint8_t> write_cugraph(const GraphSpec& g) {
  std::vector<char> strings;
  std::unordered_map<std::string, uint32_t> interned;
  std::vector<fdy_node> nodes(g.nodes.size());
  std::vector<fdy_param> index;
  std::vector<uint8_t> pdata;
  std::vector<uint8_t> adata;

  for (size_t n = 0; n < g.nodes.size(); ++n) {
    const NodeSpec& s = g.nodes[n];
    fdy_node e;
    std::memset(&e, 0, sizeof(e));
    e.node_id = static_cast<uint32_t>(n);
    e.type = s.type;
    switch (s.type) {
      case FDY_NODE_KERNEL: {
        fdy_kernel_body k = s.kernel;
        auto it = interned.find(s.name);
        if (it == interned.end()) {
          uint32_t off = static_cast<uint32_t>(strings.size());
          strings.insert(strings.end(), s.name.begin(), s.name.end());
          strings.push_back('\0');
          it = interned.emplace(s.name, off).first;
        }
        k.name_offset = it->second;
        k.name_length = static_cast<uint32_t>(s.name.size());
        k.param_index_offset = static_cast<uint32_t>(index.size() * sizeof(fdy_param));
        if (s.extra_style) {
          k.num_params = static_cast<uint32_t>(s.extra_params.size());
          index.insert(index.end(), s.extra_params.begin(), s.extra_params.end());
        } else {
          k.num_params = static_cast<uint32_t>(s.param_sizes.size());
          uint64_t at = 0;
          for (uint32_t sz : s.param_sizes) {
            fdy_param p;
            p.data_offset = static_cast<uint32_t>(pdata.size());
            p.size = sz;
            index.push_back(p);
            pdata.insert(pdata.end(), s.param_bytes.begin() + at, s.param_bytes.begin() + at + sz);
            at += sz;
          }
        }
        if (s.extra_style && !s.arg_buffer.empty()) {
          k.arg_offset = static_cast<uint32_t>(adata.size());
          k.arg_size = static_cast<uint32_t>(s.arg_buffer.size());
          adata.insert(adata.end(), s.arg_buffer.begin(), s.arg_buffer.end());
        } else {
          k.arg_offset = FDY_NO_ARG_BUFFER;
          k.arg_size = 0;
        }
        e.u.kernel = k;
        break;
      }
      case FDY_NODE_MEMSET: e.u.memset = s.memset_body; break;
      case FDY_NODE_MEMCPY: e.u.memcpy = s.memcpy_body; break;
      case FDY_NODE_EVENT_RECORD:
      case FDY_NODE_EVENT_WAIT: e.u.event.event_id = s.event_id; break;
      default: break;
    }
    nodes[n] = e;
  }

  uint64_t sizes[FDY_SEC_COUNT] = {
      strings.size(),
      nodes.size() * sizeof(fdy_node),
      g.deps.size() * sizeof(fdy_dep),
      index.size() * sizeof(fdy_param),
      pdata.size(),
      adata.size(),
      g.has_common ? sizeof(fdy_common_attrs) : 0,
      g.generators.size() * sizeof(fdy_generator),
      g.alloc_events.size(),
      g.output_tensors.size(),
      g.topology_key.size(),
  };
  fdy_section sec[FDY_SEC_COUNT];
  std::memset(sec, 0, sizeof(sec));
  uint64_t cursor = sizeof(fdy_file_header) + FDY_SEC_COUNT * sizeof(fdy_section);
  for (int i = 0; i < FDY_SEC_COUNT; ++i) {
    sec[i].id = static_cast<uint32_t>(i);
    sec[i].offset = cursor;
    sec[i].size = sizes[i];
    cursor = align8(cursor + sizes[i]);
  }

  fdy_file_header h;
  std::memset(&h, 0, sizeof(h));
  std::memcpy(h.magic, kMagic, 8);
  h.version = FDY_FORMAT_VERSION;
  if (g.has_common) h.flags |= FDY_HAS_COMMON_ATTRS;
  if (!g.deps.empty()) h.flags |= FDY_HAS_DEPS;
  if (!g.alloc_events.empty()) h.flags |= FDY_HAS_ALLOC_EVENTS;
  if (!g.output_tensors.empty()) h.flags |= FDY_HAS_OUTPUT_TENSORS;
  if (!g.generators.empty()) h.flags |= FDY_HAS_GENERATORS;
  h.num_nodes = static_cast<uint32_t>(nodes.size());
  h.num_deps = static_cast<uint32_t>(g.deps.size());
  h.num_generators = static_cast<uint32_t>(g.generators.size());
  h.num_sections = FDY_SEC_COUNT;
  h.num_strings = static_cast<uint32_t>(interned.size());

  std::vector<uint8_t> out;
  out.reserve(cursor);
  append_bytes(out, &h, 1);
  append_bytes(out, sec, FDY_SEC_COUNT);
  auto put = [&](const void* p, uint64_t n) {
    if (n) append_bytes(out, static_cast<const uint8_t*>(p), n);
    out.resize(align8(out.size()), 0);
  };
  put(strings.data(), strings.size());
  put(nodes.data(), sizes[FDY_SEC_NODES]);
  put(g.deps.data(), sizes[FDY_SEC_DEPS]);
  put(index.data(), sizes[FDY_SEC_PARAM_INDEX]);
  put(pdata.data(), pdata.size());
  put(adata.data(), adata.size());
  if (g.has_common) put(&g.common, sizeof(fdy_common_attrs));
  put(g.generators.data(), sizes[FDY_SEC_GENERATORS]);
  put(g.alloc_events.data(), g.alloc_events.size());
  put(g.output_tensors.data(), g.output_tensors.size());
  put(g.topology_key.data(), g.topology_key.size());
  return out;
}

std::string validate_image(const uint8_t* data, uint64_t size, GraphView* out) {
  if (size < sizeof(fdy_file_header)) return "file shorter than the 64-byte header";
  fdy_file_header h;
  std::memcpy(&h, data, sizeof(h));
  if (std::memcmp(h.magic, kMagic, 8) != 0) return "bad magic (not a .cugraph file)";
  if (h.version != FDY_FORMAT_VERSION) return "unsupported .cugraph version " + std::to_string(h.version);
  if (h.num_sections < FDY_SEC_COUNT) return "section directory holds fewer than 11 sections";
  uint64_t dir_end = sizeof(fdy_file_header) + uint64_t(h.num_sections) * sizeof(fdy_section);
  if (dir_end > size) return "section directory runs past the end of the file";
  out->data = data;
  out->size = size;
  out->hdr = h;
  std::memcpy(out->sec, data + sizeof(fdy_file_header), sizeof(out->sec));
  for (int i = 0; i < FDY_SEC_COUNT; ++i) {
    const fdy_section& s = out->sec[i];
    if (s.offset > size || s.size > size - s.offset)
      return "section " + std::to_string(i) + " lies outside the file";
    if (s.size && (s.offset & 7)) return "section " + std::to_string(i) + " is not 8-byte aligned";
  }
  if (out->sec[FDY_SEC_NODES].size < uint64_t(h.num_nodes) * sizeof(fdy_node))
    return "node table shorter than num_nodes entries";
  if (out->sec[FDY_SEC_DEPS].size < uint64_t(h.num_deps) * sizeof(fdy_dep))
    return "dependency table shorter than num_dependencies entries";
  if (out->sec[FDY_SEC_GENERATORS].size < uint64_t(h.num_generators) * sizeof(fdy_generator))
    return "generator table shorter than num_generators entries";
  if ((h.flags & FDY_HAS_COMMON_ATTRS) && out->sec[FDY_SEC_COMMON_ATTRS].size < sizeof(fdy_common_attrs))
    return "common-attrs flag set but the section is short";
  return std::string();
}

}  // namespace fdy
