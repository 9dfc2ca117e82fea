// restore_dev.h -- device-side data structures and helpers shared by the
// restore kernels (restore_kernels.hip) and the host glue (restore.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fdy_format.h"
#include "crc64.h"

namespace fdy {

// Words of the param image handled by one diff tile, and its thread count.
constexpr uint32_t kDiffThreads = 512;
constexpr uint32_t kDiffWordsPerThread = 8;
constexpr uint32_t kTileWords = kDiffThreads * kDiffWordsPerThread;  // 4096
constexpr uint32_t kDiffWindow = 512;    // node descriptors staged in LDS per tile
constexpr uint32_t kRelocFanout = 16;    // keys per interval-search node
constexpr uint32_t kRelocLdsKeys = 4096; // top search level kept in LDS (32 KB)
constexpr uint32_t kNoTile = 0xFFFFFFFFu;

// Internal node flag bits beyond the public FDY_NODE_* bits (0x0F).
constexpr uint32_t kNodeRaggedT = 0x10;  // template's node n is ragged
constexpr uint32_t kNodeCompare = 0x20;  // compare words against the template
constexpr uint32_t kNodeBad = 0x40;      // a range of this node lies outside its section

// Graph status bits beyond the public FDY_GRAPH_* bits.
constexpr uint32_t kGraphNodeCount = 0x10;  // node count differs from the template
constexpr uint32_t kGraphOverflow = 0x20;   // param image larger than its capacity

// Per-graph metadata, computed on the host at open and uploaded once.
struct DevGraph {
  uint64_t sec_off[FDY_SEC_COUNT];   // absolute byte offsets into the device file image
  uint64_t sec_size[FDY_SEC_COUNT];
  uint32_t num_nodes;
  uint32_t num_deps;
  uint32_t flags;        // header flags
  uint32_t word_cap;     // param-image capacity in words
  uint64_t node_base;    // global index of node 0
  uint64_t word_base;    // global index of word 0 in R / live / aux
  uint32_t tile_base;    // first diff-tile slot
  uint32_t tile_cap;     // number of diff-tile slots
};

// Per-node work description written by the node pass for the diff pass.
struct NodeDesc {
  uint32_t gword;   // first word of this node in its graph's image
  uint32_t nwords;
  uint32_t tword;   // first word of node n in the template's image
  uint32_t flags;   // FDY_NODE_* | kNode*
  uint64_t src_g;   // absolute byte offset of the blob in the file image (aligned nodes)
  uint64_t src_t;   // same for the template's node n
};
static_assert(sizeof(NodeDesc) == 32, "NodeDesc is 32 B");

// Interval search structure (see restore.hip: RelocPlanHost).
struct RelocDev {
  const uint64_t* level[8];  // level[0] = lo (padded); level[k] = every 16th key of level[k-1]
  const uint64_t* hi;
  const uint64_t* delta;     // new_lo - lo
  uint64_t n;                // intervals; 0 = relocation off
  uint64_t lo_min;
  uint64_t hi_max;
  uint32_t n_levels;         // global levels below the LDS top (level[n_levels] is the top)
  uint32_t n_top;
  uint32_t policy;
  uint32_t pad;
};

__device__ inline uint32_t ld_u32(const uint8_t* p) {
  if ((reinterpret_cast<uintptr_t>(p) & 3) == 0) return *reinterpret_cast<const uint32_t*>(p);
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

__device__ inline uint64_t ld_u64(const uint8_t* p) {
  if ((reinterpret_cast<uintptr_t>(p) & 7) == 0) return *reinterpret_cast<const uint64_t*>(p);
  return (uint64_t)ld_u32(p) | ((uint64_t)ld_u32(p + 4) << 32);
}

// Relocate one word.  `top` is the top search level (LDS or global).
__device__ inline uint64_t reloc_word(const RelocDev& r, const uint64_t* top, uint64_t w) {
  if (r.n == 0 || w < r.lo_min) return w;
  if (r.policy ? (w > r.hi_max) : (w >= r.hi_max)) return w;
  // Top level: last j with top[j] <= w (top[0] == lo_min <= w).
  uint32_t lo = 0, len = r.n_top;
  while (len > 1) {
    uint32_t half = len >> 1;
    if (top[lo + half] <= w) lo += half;
    len -= half;
  }
  uint64_t j = lo;
  for (int k = (int)r.n_levels - 1; k >= 0; --k) {
    const uint64_t* node = r.level[k] + j * kRelocFanout;
    uint32_t cnt = 0;
#pragma unroll
    for (uint32_t q = 0; q < kRelocFanout; ++q) cnt += node[q] <= w;
    j = j * kRelocFanout + cnt - 1;
  }
  uint64_t hi = r.hi[j];
  bool inside = r.policy ? (w <= hi) : (w < hi);
  return inside ? w + r.delta[j] : w;
}

}  // namespace fdy
