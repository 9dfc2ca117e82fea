// restore_dev.h -- device-side data structures and helpers shared by the
// restore kernels (restore_kernels.hip) and the host glue (restore.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fdy_format.h"
#include "crc64.h"

namespace fdy {

// Words of the param image handled by one diff tile, and its thread count.
constexpr uint32_t kDiffThreads = 256;
constexpr uint32_t kDiffWordsPerThread = 16;
constexpr uint32_t kTileWords = kDiffThreads * kDiffWordsPerThread;  // 4096
constexpr uint32_t kDiffWindow = 512;    // node descriptors staged in LDS per tile
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
  uint64_t crc_fin[4];   // CRC-64/XZ finishing terms of the key, edge, type, kernel-entry streams
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

// End and shift of one saved allocation interval (its lo is implied by the search).
struct RelocRec {
  uint64_t hi;
  uint64_t delta;  // new_lo - lo (mod 2^64)
};
static_assert(sizeof(RelocRec) == 16, "RelocRec is 16 B");

// One 64-byte line of the bucket index.  Bucket b covers addresses
// [lo_min + b*2^shift, lo_min + (b+1)*2^shift).  `first` is the last
// interval whose lo is <= the bucket's first address; intervals first+1 ..
// first+count start inside the bucket, and off[k] holds lo - bucket start
// of interval first+1+k for the first min(count, 14) of them.
constexpr uint32_t kBucketOffsets = 14;
struct RelocBucket {
  uint32_t first;
  uint32_t count;
  uint32_t off[kBucketOffsets];
};
static_assert(sizeof(RelocBucket) == 64, "RelocBucket is one 64-byte line");

struct RelocDev {
  const RelocBucket* bucket;
  const RelocRec* rec;
  const uint64_t* lo;  // every interval's lo (for buckets with > 14 starts)
  uint64_t n;          // intervals; 0 = relocation off
  uint64_t lo_min;
  uint64_t hi_max;
  uint32_t shift;      // <= 32, so offsets inside a bucket fit in 32 bits
  uint32_t policy;
};

__device__ inline uint32_t ld_u32(const uint8_t* p) {
  if ((reinterpret_cast<uintptr_t>(p) & 3) == 0) return *reinterpret_cast<const uint32_t*>(p);
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

__device__ inline uint64_t ld_u64(const uint8_t* p) {
  if ((reinterpret_cast<uintptr_t>(p) & 7) == 0) return *reinterpret_cast<const uint64_t*>(p);
  return (uint64_t)ld_u32(p) | ((uint64_t)ld_u32(p + 4) << 32);
}

// Relocate one word: the last interval with lo <= w moves w if w < hi
// (w <= hi under the inclusive policy).
__device__ inline uint64_t reloc_word(const RelocDev& r, uint64_t w) {
  if (r.n == 0 || w < r.lo_min) return w;
  if (r.policy ? (w > r.hi_max) : (w >= r.hi_max)) return w;
  const uint64_t rel = w - r.lo_min;
  const uint64_t b = rel >> r.shift;
  const uint32_t x = (uint32_t)(rel - (b << r.shift));
  // The first 16 bytes carry `first`, `count` and two offsets, which is the
  // whole bucket most of the time; the other 48 are read only when needed.
  const uint4* line = reinterpret_cast<const uint4*>(r.bucket + b);
  const uint4 q0 = line[0];
  const uint32_t count = q0.y;
  uint32_t c = (count > 0 && q0.z <= x) + (count > 1 && q0.w <= x);
  if (count > 2) {
    const uint4 q1 = line[1], q2 = line[2], q3 = line[3];
    const uint32_t m = count < kBucketOffsets ? count : kBucketOffsets;
    const uint32_t off[kBucketOffsets - 2] = {q1.x, q1.y, q1.z, q1.w, q2.x, q2.y,
                                              q2.z, q2.w, q3.x, q3.y, q3.z, q3.w};
#pragma unroll
    for (uint32_t k = 0; k < kBucketOffsets - 2; ++k) c += (k + 2 < m) & (off[k] <= x);
  }
  uint32_t i = q0.x + c;
  if (count > kBucketOffsets && c == kBucketOffsets) {
    // More starts than the line holds: binary search the rest of the bucket.
    uint32_t lo = i, hi = q0.x + count;
    while (hi > lo) {
      const uint32_t mid = (lo + hi + 1) >> 1;
      if (r.lo[mid] <= w) lo = mid;
      else hi = mid - 1;
    }
    i = lo;
  }
  const RelocRec iv = r.rec[i];
  const bool inside = r.policy ? (w <= iv.hi) : (w < iv.hi);
  return inside ? w + iv.delta : w;
}

}  // namespace fdy
