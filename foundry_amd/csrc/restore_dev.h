// restore_dev.h -- device-side data structures and helpers shared by the
// restore kernels (restore_kernels.hip) and the host glue (restore.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fdy_format.h"
#include "crc64.h"

namespace fdy {

// Words of the param image handled by one diff tile (one slot); words per
// lane in the member diff; and the sub-ranges (one wave each) whose override
// records are compacted independently.
constexpr uint32_t kTileWords = 4096;
constexpr uint32_t kMWords = 4;
constexpr uint32_t kSubWords = 64 * kMWords;
constexpr uint32_t kSubsPerSlot = kTileWords / kSubWords;
constexpr uint32_t kDiffWindow = 384;    // node descriptors staged in LDS per tile (12 KB: as much as the
                                         // member pass's candidate staging needs; 512 held its workgroups
                                         // to five waves per SIMD, 83.8 against 81.6 us)
constexpr uint32_t kNoTile = 0xFFFFFFFFu;

// The restore's flag word (RestoreArgs::restore_flags), read by the host
// before any result is.
constexpr uint32_t kFlagGaps = 1;      // a slot made fewer records than its bound: close the gaps (k_repack)
constexpr uint32_t kFlagNeedAux = 2;   // a ragged node found no ragged-word sources: restore again with them
constexpr uint32_t kFlagOverflow = 4;  // a slot's candidate spill space or a graph's record region ran out:
                                       // restore again with the next scratch level

// Scratch levels.  Each sub-range has a region of candidates, each slot spill
// space its sub-ranges continue their lists in, and each graph one override
// record per 2^rec_shift capacity words.  A restore that overflows a level
// runs again at the next; the last (full) holds a candidate and a record per
// word, so it cannot overflow.
struct ScratchLevel {
  uint32_t cand_cap;   // candidates per sub-range region
  uint32_t spill_cap;  // spill candidates per slot
  uint32_t rec_shift;
};
constexpr ScratchLevel kScratchLevels[] = {
    {kSubWords / 8, kTileWords / 16, 3},  // 768 candidates per 4096 words, a record per 8 words
    {kSubWords / 4, kTileWords / 4, 2},   // 2048 candidates per 4096 words, a record per 4 words
    {kSubWords, 0, 0},                    // full capacity
};
constexpr uint32_t kScratchFull = 2;

// Internal node flag bits beyond the public FDY_NODE_* bits (0x0F).
constexpr uint32_t kNodeRaggedT = 0x10;  // template's node n is ragged
constexpr uint32_t kNodeCompare = 0x20;  // compare words against the template
constexpr uint32_t kNodeBad = 0x40;      // a range of this node lies outside its section
constexpr uint32_t kNodeExtra = 0x80;    // kernel node whose params travel in an arg buffer
constexpr uint32_t kNodeClean = 0x100;   // entry and param entries equal the template node's: the
                                         // second node pass completes it from the template's results

// Graph status bits beyond the public FDY_GRAPH_* bits.
constexpr uint32_t kGraphNodeCount = 0x10;    // node count differs from the template
constexpr uint32_t kGraphOverflow = 0x20;     // param image larger than its capacity

// A 4 KB unit of the CRC digests: a node chunk's records, or a slice of a
// saved key or dependency table.
constexpr uint32_t kSliceBytes = 4096;

// Per-graph metadata, computed on the host at open and uploaded once.
struct DevGraph {
  uint64_t sec_off[FDY_SEC_COUNT];   // absolute byte offsets into the device file image
  uint64_t sec_size[FDY_SEC_COUNT];
  uint32_t num_nodes;
  uint32_t num_deps;
  uint32_t flags;        // header flags
  uint32_t word_cap;     // param-image capacity in words
  uint64_t node_base;    // global index of node 0
  uint64_t word_base;    // global index of word 0 in R and aux (the override records: word_base >> rec_shift)
  uint32_t tile_base;    // first diff-tile slot
  uint32_t tile_cap;     // number of diff-tile slots
  uint64_t crc_fin[4];   // CRC-64/XZ finishing terms of the key, edge, type, kernel-entry streams
  uint32_t chunk_base;   // first node chunk (kNodeChunk nodes each)
  uint32_t pad_;
};

// One unit of the key and dependency digests: a 4 KB slice of one graph's
// saved key or dependency table, built on the host at open.
struct DigestUnit {
  uint64_t src;   // byte offset of the stream in the file image (8-byte aligned)
  uint64_t len;   // stream bytes
  uint32_t back;  // the slice ends 4096 * back bytes before the stream's end
  uint32_t dst;   // digest word: 4 * graph + 0 (key) or 1 (dependency table)
  uint64_t pad_;
};
static_assert(sizeof(DigestUnit) == 32, "DigestUnit is 32 B");

// Nodes per chunk of the node pass (a graph has at least one chunk), and
// what a chunk reports to its graph.
constexpr uint32_t kNodeChunk = 256;
constexpr uint32_t kChunkDiff = 1;  // records are the XOR of the graph's and its template's
struct NodeChunk {
  uint64_t crc_type, crc_kent;  // raw CRCs (zero initial value) of the chunk's node-type and kernel-entry
                                // records (kChunkDiff: of the XOR of the graph's and the template's records)
  uint64_t pbytes;              // param bytes of the chunk's nodes handled in the chunk (not the clean ones)
  uint32_t status;              // FDY_GRAPH_* bits found in the chunk
  uint32_t mode;                // kChunkDiff or 0
};
static_assert(sizeof(NodeChunk) == 32, "NodeChunk is 32 B");

// Per-slot work description written by the node pass for the diff pass.
constexpr uint32_t kSlotFlat = 1;      // every word of the tile sits at kg + 8w (and kt + 8w)
constexpr uint32_t kSlotCompare = 2;   // flat tile whose words are compared with the template
constexpr uint32_t kSlotTemplate = 4;  // tile of a template graph
constexpr uint32_t kSlotFirst = 8;     // the graph's first slot
constexpr uint32_t kSlotLast = 16;     // the graph's last slot
struct SlotDesc {
  uint64_t kg;           // flat: byte offset of image word 0 of the graph in the file image
  uint64_t kt;           // flat + compare: the same for the template
  uint64_t word_base;    // the graph's first word in R and aux
  uint64_t t_word_base;  // the template's first word in R
  uint32_t wbeg, wend;   // graph-local word range of the tile (empty: inactive slot)
  uint32_t graph;
  uint32_t tmpl;         // the graph's template
  uint32_t flags;        // kSlot*
  uint32_t t_cap;        // the template's image capacity in words
  uint32_t node_base;    // the graph's node 0 in the node arrays (an archive holds fewer than 2^32 nodes)
  uint32_t num_nodes;    // the graph's node count
};
static_assert(sizeof(SlotDesc) == 64, "SlotDesc is one 64-byte line");

// A word the member pass leaves to k_diff_s: a whole word to relocate
// (kCandReloc), possibly differing from the template's (kCandCompare).
constexpr uint32_t kCandReloc = 1;
constexpr uint32_t kCandCompare = 2;
struct Candidate {
  uint32_t word;   // graph-local word index
  uint32_t flags;  // kCand*
  uint64_t raw;    // the graph's raw word
  uint64_t tval;   // the template's relocated word (kCandCompare)
};
static_assert(sizeof(Candidate) == 24, "Candidate is 24 B");
static_assert(sizeof(Candidate) >= 16, "a region of candidates holds as many 16-byte records");

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

// The interval index: 64-byte lines, each answering every search inside
// its address range from that one line or naming the line that does.  Root
// line b covers addresses [lo_min + b*2^shift, lo_min + (b+1)*2^shift)
// (shift <= 31, so offsets inside a line fit in 31 bits).
//   A leaf line with first address B holds four 16-byte slots: slot 0 the
// last interval whose lo is at or before B (it moves the line's addresses
// below the first start inside it), slots 1-3 the intervals starting inside
// the line, in order.  A slot holds lo - B (slot 0: the line's kind, zero
// for a leaf), hi - B + 1 clamped into [0, 2^32 - 1], and new_lo - lo;
// unused slots have lo - B = 2^32 - 1.  A word at offset x of a leaf moves
// by the delta of the last slot whose lo - B is <= x, if x + 1 < that
// slot's end (x + 1 <= end under the inclusive policy).
//   A line whose range holds more than four intervals is a fence line
// (kind kLineFence): up to 14 fences, the lo - B of intervals starting
// inside it, in order (unused: 2^32 - 1), cut it into up to 15 child lines
// first, first + 1, ... (first in slot 0's end field); child c starts at
// fence c - 1 (child 0 at B) and is itself a leaf or a fence line, so a
// search reads one line per level: one for a leaf root, two for up to 60
// intervals under one root, three for up to 900.
constexpr uint32_t kLineSlots = 4;
constexpr uint32_t kLineFence = 0x80000000u;
constexpr uint32_t kLineFences = 14;
constexpr uint32_t kLineNone = 0xFFFFFFFFu;  // lo - B of an unused slot, an unused fence
constexpr uint32_t kMaxLineShift = 31;
struct RelocSlot {
  uint32_t lo;     // lo - B (slot 0: the line's kind)
  uint32_t end;    // hi - B + 1, clamped into [0, 2^32 - 1] (fence line, slot 0: first child)
  uint64_t delta;  // new_lo - lo (mod 2^64)
};
struct RelocLine {
  RelocSlot s[kLineSlots];
};
static_assert(sizeof(RelocLine) == 64, "RelocLine is one 64-byte line");
// Fence f of a fence line: its 32-bit word 2 + f.
__host__ __device__ inline uint32_t* line_fences(RelocLine& L) { return reinterpret_cast<uint32_t*>(&L) + 2; }

struct RelocDev {
  const RelocLine* line;
  uint64_t n;           // intervals; 0 = relocation off
  uint64_t lo_min;
  uint64_t hi_max;
  uint32_t shift;       // <= kMaxLineShift
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

// The 8 bytes at p (any alignment) from the two aligned words covering
// them, loaded unconditionally so that a run of these issues together.
// Reads up to 15 bytes past p: callers keep p inside the archive-image
// buffer, whose 4 KB zero tail covers the overrun.
__device__ __forceinline__ uint64_t ld_u64_any(const uint8_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint64_t* q = reinterpret_cast<const uint64_t*>(a & ~(uintptr_t)7);
  const uint32_t sh = (uint32_t)(a & 7) * 8;
  const uint64_t w0 = q[0], w1 = q[1];
  return sh ? (w0 >> sh) | (w1 << (64 - sh)) : w0;
}

// Fields of a node entry, its kernel-attribute block or the common attrs:
// these start 8-byte aligned (sections are validated 8-byte aligned and an
// entry is 168 = 8 * 21 bytes), so every 4-byte field is 4-byte aligned and
// its load needs no run-time alignment branch (which would keep the
// compiler from issuing a node's loads together).
__device__ __forceinline__ uint32_t f32(const uint8_t* e, uint32_t off) {
  return *reinterpret_cast<const uint32_t*>(e + off);
}
__device__ __forceinline__ uint64_t f64(const uint8_t* e, uint32_t off) {
  return (uint64_t)f32(e, off) | ((uint64_t)f32(e, off + 4) << 32);
}

// Relocate K words at once (the words whose bit is set in `mask`; the others
// pass through): the interval containing w (the last one with lo <= w)
// moves w if w < hi (w <= hi under the inclusive policy).  The K searches
// advance in lockstep, so each step issues its K line reads before waiting
// for any of them.
template <int K>
__host__ __device__ inline void reloc_batch(const RelocDev& r, const uint64_t* w, uint64_t* out, uint32_t mask) {
  if (r.n == 0) {  // relocation off (uniform)
#pragma unroll
    for (int k = 0; k < K; ++k) out[k] = w[k];
    return;
  }
  bool ok[K];
  uint32_t x[K];
  uint4 q[K][kLineSlots];
  // Every search's root line is loaded without a branch (line 0 stands in
  // for words outside the table and is masked off): a load behind a
  // per-word branch is followed by its own wait, and the K searches would
  // go one after another instead of together.
#pragma unroll
  for (int k = 0; k < K; ++k) {
    ok[k] = ((mask >> k) & 1) && w[k] >= r.lo_min && (r.policy ? w[k] <= r.hi_max : w[k] < r.hi_max);
    const uint64_t rel = w[k] - r.lo_min;
    const uint64_t b = ok[k] ? rel >> r.shift : 0;
    x[k] = ok[k] ? (uint32_t)(rel - (b << r.shift)) : 0u;
    const uint4* p = reinterpret_cast<const uint4*>(r.line + b);
#pragma unroll
    for (uint32_t j = 0; j < kLineSlots; ++j) q[k][j] = p[j];
  }
  // Descend through fence lines to the leaves: the child after the last
  // fence at or before x (fences are in order; unused ones are 2^32 - 1 > x).
  for (;;) {
    bool any = false;
#pragma unroll
    for (int k = 0; k < K; ++k) any |= ok[k] && (q[k][0].x & kLineFence);
    if (!any) break;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (ok[k] && (q[k][0].x & kLineFence)) {
        const uint32_t f[kLineFences] = {q[k][0].z, q[k][0].w, q[k][1].x, q[k][1].y, q[k][1].z,
                                         q[k][1].w, q[k][2].x, q[k][2].y, q[k][2].z, q[k][2].w,
                                         q[k][3].x, q[k][3].y, q[k][3].z, q[k][3].w};
        uint32_t c = 0, at = 0;
#pragma unroll
        for (uint32_t e = 0; e < kLineFences; ++e) {
          const bool le = f[e] <= x[k];
          c += le;
          at = le ? f[e] : at;
        }
        x[k] -= at;
        const uint4* p = reinterpret_cast<const uint4*>(r.line + q[k][0].y + c);
#pragma unroll
        for (uint32_t j = 0; j < kLineSlots; ++j) q[k][j] = p[j];
      }
    }
  }
  // The last slot starting at or before x (slots are in lo order; unused
  // ones start at 2^32 - 1 > x).
#pragma unroll
  for (int k = 0; k < K; ++k) {
    uint32_t end = q[k][0].y;
    uint64_t delta = (uint64_t)q[k][0].z | ((uint64_t)q[k][0].w << 32);
#pragma unroll
    for (uint32_t j = 1; j < kLineSlots; ++j) {
      const bool at = q[k][j].x <= x[k];
      end = at ? q[k][j].y : end;
      delta = at ? ((uint64_t)q[k][j].z | ((uint64_t)q[k][j].w << 32)) : delta;
    }
    const bool inside = ok[k] && (r.policy ? x[k] + 1 <= end : x[k] + 1 < end);
    out[k] = inside ? w[k] + delta : w[k];
  }
}

__host__ __device__ inline uint64_t reloc_word(const RelocDev& r, uint64_t w) {
  uint64_t o;
  reloc_batch<1>(r, &w, &o, 1u);
  return o;
}

}  // namespace fdy
