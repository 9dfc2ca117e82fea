// cugraph.h -- host-side model of one `.cugraph` v1 archive: a validated
// read-only view, and a writer that lays out sections exactly as the
// reference's SAVE path does (csrc/BinaryGraphIO.cpp:15-371).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "../../include/fdy_format.h"

namespace fdy {

// A node as the SAVE side knows it, before section offsets exist.
struct NodeSpec {
  uint8_t type = FDY_NODE_EMPTY;
  fdy_kernel_body kernel{};            // name/param/arg offsets are assigned by the writer
  std::string name;                    // kernel function name
  std::vector<uint32_t> param_sizes;   // per-param style: sizes, in order
  std::vector<uint8_t> param_bytes;    // per-param style: the params back-to-back
  bool extra_style = false;            // params travel in one arg buffer
  std::vector<fdy_param> extra_params; // extra style: (in-kernel offset, size) descriptors
  std::vector<uint8_t> arg_buffer;
  fdy_memset_body memset_body{};
  fdy_memcpy_body memcpy_body{};
  int32_t event_id = 0;
};

struct GraphSpec {
  std::vector<NodeSpec> nodes;
  std::vector<fdy_dep> deps;
  std::vector<fdy_generator> generators;
  bool has_common = false;
  fdy_common_attrs common{};
  std::string alloc_events;    // JSON text, stored verbatim
  std::string output_tensors;  // JSON text, stored verbatim
  std::string topology_key;    // stored verbatim (see topology_key_save_rule)
};

// Serialise a graph in the reference's section order with 8-byte section
// alignment and its header flags (csrc/BinaryGraphIO.cpp:291-368).
std::vector<uint8_t> write_cugraph(const GraphSpec& g);

// The topology key as CUDAGraph::save computes it from per-node attributes
// (csrc/CUDAGraph.cpp:1347-1385): "Type[:0|:Cx_y_z]" joined by ','.
std::string topology_key_save_rule(const GraphSpec& g);

// Type name used in topology keys (csrc/BinaryGraphIO.cpp:494-615).
const char* node_type_name(uint8_t type);

// Read-only view of one archive image with every section bounds-checked.
struct GraphView {
  const uint8_t* data = nullptr;
  uint64_t size = 0;
  fdy_file_header hdr{};
  fdy_section sec[FDY_SEC_COUNT]{};

  const uint8_t* section(int id) const { return data + sec[id].offset; }
  uint64_t section_size(int id) const { return sec[id].size; }
  const fdy_node* nodes() const { return reinterpret_cast<const fdy_node*>(section(FDY_SEC_NODES)); }
};

// Validate header and section directory.  Stricter than the reference's
// validate_header (include/BinaryGraphFormat.h:233-235): every section must
// lie inside the image and start 8-byte aligned, and the node, dependency
// and generator tables must hold their header counts, so device code can
// index them without further checks.  Returns an empty string when valid.
std::string validate_image(const uint8_t* data, uint64_t size, GraphView* out);

}  // namespace fdy
