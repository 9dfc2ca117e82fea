// archive.h -- the archive object shared by the two host halves of the C ABI:
// restore.hip (open, restore, results, switch) and graph.hip (code-object
// registry and group graphs).  Internal to libfoundry_restore.so.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "../../include/foundry_restore.h"
#include "kernels.h"

struct fdy_group_graph;

namespace fdy {

// Message of the calling thread's last error (fdy_last_error).
extern thread_local std::string g_err;

inline int err(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

#define FDY_HIP(call)                                                                                 \
  do {                                                                                                \
    hipError_t e_ = (call);                                                                           \
    if (e_ != hipSuccess)                                                                             \
      return ::fdy::err(FDY_E_HIP, std::string(#call) + " failed: " + hipGetErrorString(e_) +         \
                                       " (hipError_t " + std::to_string((int)e_) + ")");              \
  } while (0)

// Device allocation owned by one archive, plan or group graph.
struct DevBuf {
  void* p = nullptr;
  size_t bytes = 0;
  bool owned = true;  // false: a part of another buffer (an arena), not freed here
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() {
    if (p && owned) (void)hipFree(p);
  }
  template <typename T>
  T* as() const {
    return static_cast<T*>(p);
  }
  void swap(DevBuf& o) {
    std::swap(p, o.p);
    std::swap(bytes, o.bytes);
    std::swap(owned, o.owned);
  }
  void release() {
    if (p && owned) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
    owned = true;
  }
};

int dev_alloc(DevBuf& b, size_t bytes, const char* what);

// The interval search structure: an index of 64-byte lines, one to two
// root lines per interval, each answering the searches inside it or naming
// the lines that do (see RelocLine).
struct RelocPlan {
  DevBuf line;
  RelocDev dev{};
};

}  // namespace fdy

struct fdy_archive {
  int device = 0;
  uint32_t G = 0;
  std::vector<fdy::DevGraph> graphs;
  uint64_t img_bytes = 0;
  uint64_t total_nodes = 0;
  uint64_t total_cap = 0;
  uint32_t num_slots = 0;
  uint32_t num_chunks = 0;
  uint32_t num_units = 0;

  // `arena` holds every open-time buffer other than the images, R and the
  // restore's scratch, as parts (one allocation instead of some twenty).
  fdy::DevBuf arena;
  fdy::DevBuf img, dgraphs, cc, digests, tmpl, explicit_tmpl, status, gwords, pbytes;
  fdy::DevBuf nflags, ndesc, nptrs, live_src, tile_node, chunk_gt, units, chunks, slot_desc, live_cur, tslot_desc;
  fdy::DevBuf tslot_count;
  fdy::DevBuf aux, image, live, ovr, cand, sub_count, slot_rec, restore_flags, node_pbytes, key_hash;
  fdy::DevBuf slot_spill, sub_off;

  fdy::RelocPlan reloc;
  // Restoring layout: R_g at word_base(g); graph g's override records from
  // word_base(g) >> rec_shift; the scratch (candidate regions and spill
  // space, ragged-word sources once a restore has found a ragged node) at
  // the archive's scratch level.  Live images exist for the templates only (template t's
  // from h_live_base[t]), filled from R_t when results are first read after
  // a restore.
  //   Serving layout, taken when the first group graph is bound (no restore
  // can run until the last is destroyed): override records packed in
  // canonical order (graph g's from h_ovr_off[g]), each R_g packed to its
  // words (from h_r_base[g]), and the restore's scratch freed.
  bool compact = false;
  uint32_t scratch_level = 0;  // kScratchLevels index: raised by a restore that overflowed, kept from then on
  bool need_aux = false;       // a restore found a ragged node: ragged-word sources from then on
  uint32_t rec_shift = 0, cand_cap = 0, spill_cap = 0;
  bool live_ready = false;    // live images filled from this restore's R
  std::vector<uint64_t> h_live_base, h_r_base;  // h_r_base[g]: first word of R_g, packed to its words
  bool use_explicit = false;
  bool restored = false;
  hipStream_t last_stream = nullptr;

  // Host copies taken after a restore (one synchronisation, then reused).
  bool cached = false;
  std::vector<uint32_t> h_tmpl, h_status, h_gwords;
  std::vector<uint64_t> h_ovr_off, h_pbytes;  // h_ovr_off: prefix of the per-graph record counts
  std::vector<uint32_t> h_current;

  // Group graph bound to each template (null if none); while any is bound the
  // archive refuses a new restore and close, and switches of a bound group go
  // through its group graph so that the exec follows the live image.
  std::vector<fdy_group_graph*> bound;
  uint32_t num_bound = 0;

  int timing = 0;  // fdy_set_timing: 0 off, 1 every kernel, 2 the two phases only
  uint32_t epoch = 0;  // tag of the last restore's published key hashes (1..65535)
  uint32_t hash_wait_spins = fdy::kHashWaitSpins;  // fdy_set_group_wait
  int timed = 0;  // the mode the last restore was timed in
  hipEvent_t ev[6] = {};

  ~fdy_archive() {
    for (hipEvent_t& e : ev)
      if (e) (void)hipEventDestroy(e);
  }
};

namespace fdy {

// Host copies of the per-graph results; the first call after a restore
// synchronizes `s`.
int ensure_cache(fdy_archive* a, hipStream_t s);
int check_graph(const fdy_archive* a, uint32_t g);
// Whether graph g may take its group's live image; *t receives its template.
int check_switchable(fdy_archive* a, uint32_t g, uint32_t* t);
// Enqueue the override scatter that moves the live image of g's group from
// its current graph to g, and record g as current.  With `dirty` (device
// memory, one byte per node of the group) the scatter also marks the nodes
// whose params, descriptor or layout change.
int enqueue_switch(fdy_archive* a, uint32_t g, hipStream_t s, uint8_t* dirty, bool set_device = true);
// Switch of a group that has a bound group graph (graph.hip).
int group_graph_select(fdy_group_graph* gg, uint32_t g, hipStream_t s, void* stats);

// First override record of graph g, first live word of template t, and
// first word of R_g, in the current layout.
inline uint64_t ovr_base(const fdy_archive* a, uint32_t g) {
  return a->compact ? a->h_ovr_off[g] : a->graphs[g].word_base >> a->rec_shift;
}
inline uint64_t live_base(const fdy_archive* a, uint32_t t) { return a->h_live_base[t]; }
inline uint64_t r_base(const fdy_archive* a, uint32_t g) {
  return a->compact ? a->h_r_base[g] : a->graphs[g].word_base;
}
// Take the serving layout (after a restore, before the first group graph is
// bound); synchronizes `s`.
int compact_for_serving(fdy_archive* a, hipStream_t s);
// The restore's override records and scratch at the archive's scratch
// level, with ragged-word sources when need_aux.
int alloc_restore_buffers(fdy_archive* a);
// Enqueue the restore kernels on `s` (fdy_restore after its checks).
int enqueue_restore(fdy_archive* a, hipStream_t s);
// Device bytes the archive holds.
uint64_t held_bytes(const fdy_archive* a);

}  // namespace fdy
