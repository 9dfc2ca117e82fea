// kernels.h -- launch wrappers for the restore kernels (kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/foundry_restore.h"
#include "restore_dev.h"

namespace fdy {

// Default RestoreArgs::hash_wait_spins: about 1 ms of s_sleep.
constexpr uint32_t kHashWaitSpins = 1u << 14;

// Everything the restore kernels read or write for one archive.
struct RestoreArgs {
  const uint8_t* img;         // .cugraph images, each 256-B aligned
  const DevGraph* graphs;
  const CrcConsts* cc;
  uint32_t num_graphs;
  uint32_t num_slots;
  uint32_t num_chunks;        // node chunks over all graphs
  uint2* chunk_gt;            // per node chunk: {graph, template} (the grouping pass writes both)
  uint32_t num_units;         // digest units (4 KB slices of keys and dependency tables) over all graphs
  const DigestUnit* units;
  NodeChunk* chunks;          // per node chunk
  uint64_t* digests;          // 4 per graph
  const uint32_t* explicit_template;  // or null
  uint64_t* key_hash;                 // per graph: the grouping pass's published key hash (epoch-tagged)
  uint32_t epoch;                     // this restore's tag for published key hashes (1..65535)
  uint32_t hash_wait_spins;           // s_sleep rounds the grouping scan waits for an unpublished hash
                                      // before hashing that key itself (0: at once)
  uint32_t* template_of;
  uint32_t* status;
  uint32_t* gwords;
  uint64_t* pbytes;           // param bytes per graph
  uint8_t* node_flags;
  NodeDesc* node_desc;
  uint64_t* node_ptrs;        // 2 per node
  uint32_t* tile_node;        // per slot
  SlotDesc* tslot_desc;       // descriptors of the template graphs' slots holding words (capacity: num_slots)
  uint32_t* tslot_count;      // entries of tslot_desc
  SlotDesc* slot_desc;        // per slot
  uint64_t* aux;              // ragged-word sources (per word), or null until a restore finds a ragged node
  uint64_t* image;            // relocated param images R
  uint32_t* live_src;         // per node
  uint32_t* live_cur;         // per graph
  fdy_override* ovr;          // override records: graph g's in canonical order from index word_base(g) >> rec_shift,
                              // at most ((word_base + word_cap) >> rec_shift) - (word_base >> rec_shift) of them
  uint32_t rec_shift;         // 0: a record per capacity word; kCompactShift: one per 2^kCompactShift
  uint32_t cand_cap;          // candidates in a sub-range's own region (kSubWords, or fewer with spill space)
  uint32_t spill_cap;         // candidates a slot's sub-ranges can spill past their own regions (0: none)
  Candidate* cand;            // per slot: kSubsPerSlot regions of cand_cap candidates, then spill_cap more
  uint32_t* slot_spill;       // per slot: spill entries taken by this restore
  uint32_t* sub_off;          // per (slot, sub-range): first entry of its candidate list in the slot's area
  uint32_t* sub_count;        // per (slot, sub-range): candidates | compared candidates << 16
  uint32_t* slot_rec;         // records per slot
  uint32_t* restore_flags;    // kFlag* raised by this restore
  uint64_t* node_pbytes;      // param bytes per node (nodes the first node pass handles itself)
  RelocDev reloc;
};

hipError_t launch_group(const RestoreArgs& a, hipStream_t s);
hipError_t launch_node(const RestoreArgs& a, hipStream_t s);
hipError_t launch_diff_templates(const RestoreArgs& a, hipStream_t s);
hipError_t launch_diff_members(const RestoreArgs& a, hipStream_t s);
hipError_t launch_diff_search(const RestoreArgs& a, hipStream_t s);

// Closing the gaps in override arrays (k_repack).
struct RepackArgs {
  const DevGraph* graphs;
  const uint32_t* sub_count;
  const uint32_t* slot_rec;
  fdy_override* ovr;
  uint32_t num_graphs;
  uint32_t rec_shift;
};
hipError_t launch_repack(const RepackArgs& a, hipStream_t s);

struct SwitchArgs {
  const fdy_override* ovr_cur;  // current graph's overrides
  uint64_t n_cur;
  const fdy_override* ovr_new;  // target graph's overrides
  uint64_t n_new;
  const uint64_t* tmpl_image;   // R of the template
  uint64_t* live;               // live image of the template
  const uint8_t* flags_cur;     // node flags of the current graph
  const uint8_t* flags_new;     // node flags of the target
  uint32_t* live_src;           // node sources of the template's group
  uint8_t* dirty;               // or null: per node, set to 1 when the node must be re-set
  uint32_t num_nodes;           // template's node count
  uint32_t target;
  uint32_t tmpl;
};
hipError_t launch_switch(const SwitchArgs& a, hipStream_t s);

// Up to kSwitchBatch switches of different groups in one launch.
constexpr uint32_t kSwitchBatch = 16;
struct SwitchBatch {
  SwitchArgs sw[kSwitchBatch];
  uint32_t end[kSwitchBatch];  // running block counts
  uint32_t n;
};
static_assert(sizeof(SwitchBatch) <= 2048, "a switch batch travels as kernel arguments");
// Blocks of one switch's scatter (the same split as launch_switch's).
uint32_t switch_blocks(const SwitchArgs& a);
hipError_t launch_switch_many(const SwitchBatch& b, hipStream_t s);

// Copy of the dirty nodes' live words (or of every node's) into the host
// mirror of a group graph, with the dirty marks; clears the device marks.
struct MirrorArgs {
  const uint64_t* live;   // the group's live image
  const NodeDesc* desc;   // the template's node descriptors (gword, nwords)
  uint8_t* dirty;         // per node (device memory)
  uint64_t* h_live;       // device-visible host memory, same indexing as live
  uint8_t* h_dirty;       // device-visible host memory, per node
  uint32_t num_nodes;
  uint32_t all;           // 1: copy every node and mark it dirty
};
constexpr uint32_t kMirrorNodes = 64;  // nodes per block
hipError_t launch_mirror(const MirrorArgs& a, hipStream_t s);

hipError_t launch_reloc_words(const RelocDev& r, const uint64_t* in, uint64_t* out, uint64_t n, hipStream_t s);

// The interval index built on the device (the builder of reloc_index.h, one
// thread per root line): launch_index_count writes each workgroup's first
// line below its roots into block_sum (one per kIndexThreads root lines) and
// the index's line count into *total; launch_index_place then writes the
// lines (line holds *total of them).
constexpr uint32_t kIndexThreads = 64;  // one wave: 24 KB of LDS for the subtree counts
struct IndexArgs {
  const uint64_t* lo;   // the table, on the device
  const uint64_t* hi;
  const uint64_t* nlo;
  uint64_t n;           // intervals (> 0)
  uint64_t nb;          // root lines
  uint32_t shift;       // root line width: 2^shift bytes
  uint32_t pad_;
  uint64_t* block_sum;  // ceil(nb / kIndexThreads) entries
  uint64_t* total;
  RelocLine* line;
};
hipError_t launch_index_count(const IndexArgs& a, hipStream_t s);
hipError_t launch_index_place(const IndexArgs& a, hipStream_t s);

// A memset node of a restored graph, run as a kernel node: `height` rows of
// `row_bytes` bytes, `pitch` bytes apart, each byte k of a row taking byte
// k % 4 of `pattern` (the value replicated to 32 bits).
struct FillArgs {
  uint8_t* dst;
  uint64_t pitch;
  uint64_t row_bytes;
  uint64_t height;
  uint32_t pattern;
  uint32_t pad_;
};
constexpr uint32_t kFillThreads = 256;
// Host handle of the fill kernel, for hipKernelNodeParams::func.
void* fill_kernel();
dim3 fill_grid(const FillArgs& f);

}  // namespace fdy
