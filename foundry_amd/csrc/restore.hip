// restore.hip -- host side of the C ABI in include/foundry_restore.h.
//
// Host work is limited to what cannot run on the device: reading files,
// validating section bounds (so device code never indexes outside an image),
// sizing buffers, and enqueueing the kernels of kernels.hip.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/foundry_restore.h"
#include "archive.h"
#include "cugraph.h"
#include "json_min.h"
#include "kernels.h"
#include "reloc_index.h"
#include "writer.h"

namespace fdy {

thread_local std::string g_err;

int dev_alloc(DevBuf& b, size_t bytes, const char* what) {
  if (bytes == 0) bytes = 256;
  hipError_t e = hipMalloc(&b.p, bytes);
  if (e != hipSuccess) {
    b.p = nullptr;
    return err(FDY_E_NOMEM, std::string("hipMalloc(") + std::to_string(bytes) + ") for " + what +
                                " failed: " + hipGetErrorString(e));
  }
  b.bytes = bytes;
  return FDY_OK;
}

namespace {

template <typename F>
void parallel_for(uint32_t n, uint32_t threads, F&& f) {
  threads = std::max(1u, std::min(threads ? threads : 1u, std::max(1u, n)));
  if (threads == 1) {
    for (uint32_t i = 0; i < n; ++i) f(i);
    return;
  }
  std::atomic<uint32_t> next{0};
  std::vector<std::thread> pool;
  for (uint32_t t = 0; t < threads; ++t)
    pool.emplace_back([&] {
      for (uint32_t i; (i = next.fetch_add(1)) < n;) f(i);
    });
  for (auto& t : pool) t.join();
}

uint32_t default_threads() { return std::max(1u, std::min(16u, std::thread::hardware_concurrency())); }

// The upload of archive images to HBM.  Bytes reach the device through a
// ring of pinned host slots that the process allocates once and every open
// reuses (pinning and unpinning an image-sized buffer per open cost more than
// the copy itself): each upload thread owns two slots and a stream, fills
// one slot (pread from the file, or memcpy from memory) while the other's
// copy is in flight, and waits for a slot's previous copy before refilling
// it.  One upload uses the ring at a time.
constexpr uint64_t kUploadSlot = 8ull << 20;
constexpr uint32_t kUploadThreads = 8;

struct UploadRing {
  std::mutex mu;
  uint8_t* host = nullptr;  // 2 * kUploadThreads slots, pinned
  bool pinned = false;
};
UploadRing g_ring;

// A stretch of the device image: `len` bytes at `dst`, read from file
// descriptor `fd` at `foff`, or copied from `src`; `zero` bytes of zeros
// follow (padding to the next graph).
struct UploadPiece {
  uint64_t dst, len, zero;
  int fd;
  uint64_t foff;
  const uint8_t* src;
};

// Split graph i's bytes (and its padding) into pieces of at most one slot.
void add_pieces(std::vector<UploadPiece>& out, uint64_t dst, uint64_t len, uint64_t pad, int fd, const uint8_t* src) {
  if (len == 0 && pad == 0) return;
  uint64_t at = 0;
  do {
    const uint64_t n = std::min(len - at, kUploadSlot);
    const uint64_t z = at + n == len ? std::min(pad, kUploadSlot - n) : 0;
    out.push_back({dst + at, n, z, fd, at, src ? src + at : nullptr});
    if (at + n == len && pad > z) out.push_back({dst + len + z, 0, pad - z, -1, 0, nullptr});
    at += n;
  } while (at < len);
}

int upload(uint8_t* dev, const std::vector<UploadPiece>& pieces, uint32_t threads) {
  std::lock_guard<std::mutex> lk(g_ring.mu);
  if (!g_ring.host) {
    void* p = nullptr;
    if (hipHostMalloc(&p, 2 * kUploadThreads * kUploadSlot, hipHostMallocPortable) == hipSuccess) {
      g_ring.pinned = true;
    } else {
      (void)hipGetLastError();
      p = std::malloc(2 * kUploadThreads * kUploadSlot);
      if (!p) return err(FDY_E_NOMEM, "upload ring of " + std::to_string(2 * kUploadThreads * kUploadSlot) + " bytes");
    }
    g_ring.host = static_cast<uint8_t*>(p);
  }
  int dev_id = 0;
  FDY_HIP(hipGetDevice(&dev_id));
  threads = std::max(1u, std::min({threads, kUploadThreads, (uint32_t)pieces.size()}));
  std::atomic<size_t> next{0};
  std::vector<std::string> errs(threads);
  std::vector<int> codes(threads, FDY_OK);
  auto work = [&](uint32_t t) {
    auto fail = [&](int code, const std::string& m) {
      if (codes[t] == FDY_OK) {
        codes[t] = code;
        errs[t] = m;
      }
    };
    if (hipSetDevice(dev_id) != hipSuccess) return fail(FDY_E_HIP, "hipSetDevice failed on an upload thread");
    hipStream_t st = nullptr;
    hipEvent_t ev[2] = {nullptr, nullptr};
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&ev[0], hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ev[1], hipEventDisableTiming) != hipSuccess) {
      fail(FDY_E_HIP, "cannot create an upload stream or event");
    }
    bool used[2] = {false, false};
    for (uint32_t k = 0; codes[t] == FDY_OK;) {
      const size_t i = next.fetch_add(1);
      if (i >= pieces.size()) break;
      const UploadPiece& pc = pieces[i];
      const uint32_t b = k++ & 1;
      uint8_t* slot = g_ring.host + (2ull * t + b) * kUploadSlot;
      if (used[b] && hipEventSynchronize(ev[b]) != hipSuccess) {
        fail(FDY_E_HIP, "upload copy failed");
        break;
      }
      if (pc.src) {
        std::memcpy(slot, pc.src, pc.len);
      } else if (pc.len) {
        uint64_t got = 0;
        while (got < pc.len) {
          const ssize_t r = pread(pc.fd, slot + got, pc.len - got, (off_t)(pc.foff + got));
          if (r <= 0) break;
          got += (uint64_t)r;
        }
        if (got != pc.len) {
          fail(FDY_E_IO, "short read");
          break;
        }
      }
      std::memset(slot + pc.len, 0, pc.zero);
      if (hipMemcpyAsync(dev + pc.dst, slot, pc.len + pc.zero, hipMemcpyHostToDevice, st) != hipSuccess ||
          hipEventRecord(ev[b], st) != hipSuccess) {
        fail(FDY_E_HIP, "upload copy failed");
        break;
      }
      used[b] = true;
    }
    if (st && hipStreamSynchronize(st) != hipSuccess) fail(FDY_E_HIP, "upload copy failed");
    for (hipEvent_t e : ev)
      if (e) (void)hipEventDestroy(e);
    if (st) (void)hipStreamDestroy(st);
  };
  std::vector<std::thread> pool;
  for (uint32_t t = 1; t < threads; ++t) pool.emplace_back(work, t);
  work(0);
  for (auto& th : pool) th.join();
  for (uint32_t t = 0; t < threads; ++t)
    if (codes[t] != FDY_OK) {
      (void)hipGetLastError();
      return err(codes[t], "uploading the archive images: " + errs[t]);
    }
  return FDY_OK;
}

int build_reloc_index(const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo, uint64_t n, uint32_t policy,
                      HostIndex* out, uint64_t root_lines_per_interval = kRootLinesPerInterval) {
  std::string why;
  const int rc = build_reloc_index(lo, hi, nlo, n, policy, out, &why, root_lines_per_interval);
  return rc ? err(rc, why) : FDY_OK;
}

// A table's index on the device: checked and shaped on the host, its lines
// counted, placed and written on the device (one thread per root line,
// kernels.hip), so only the table travels over PCIe.  Synchronizes.
int build_reloc_plan(const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo, uint64_t n, uint32_t policy,
                     RelocPlan* out, uint64_t root_lines_per_interval = kRootLinesPerInterval) {
  std::memset(&out->dev, 0, sizeof(out->dev));
  out->line.release();
  std::string why;
  IndexShape sh;
  int rc = index_shape(lo, hi, nlo, n, policy, root_lines_per_interval, &sh, &why);
  if (rc) return err(rc, why);
  out->dev.policy = policy;
  if (n == 0) return FDY_OK;
  const uint64_t nblocks = (sh.nb + kIndexThreads - 1) / kIndexThreads;
  DevBuf table, sums;
  rc = dev_alloc(table, 24 * n, "interval table");
  if (!rc) rc = dev_alloc(sums, 8 * (nblocks + 1), "interval index counts");
  if (rc) return rc;
  uint64_t* t = table.as<uint64_t>();
  FDY_HIP(hipMemcpy(t, lo, 8 * n, hipMemcpyHostToDevice));
  FDY_HIP(hipMemcpy(t + n, hi, 8 * n, hipMemcpyHostToDevice));
  FDY_HIP(hipMemcpy(t + 2 * n, nlo, 8 * n, hipMemcpyHostToDevice));
  IndexArgs ia{};
  ia.lo = t;
  ia.hi = t + n;
  ia.nlo = t + 2 * n;
  ia.n = n;
  ia.nb = sh.nb;
  ia.shift = sh.shift;
  ia.block_sum = sums.as<uint64_t>();
  ia.total = sums.as<uint64_t>() + nblocks;
  FDY_HIP(launch_index_count(ia, nullptr));
  uint64_t total = 0;
  FDY_HIP(hipMemcpy(&total, ia.total, 8, hipMemcpyDeviceToHost));
  if (total > kMaxIndexLines) return err(FDY_E_INVALID, "interval index too large");
  rc = dev_alloc(out->line, total * sizeof(RelocLine), "interval index lines");
  if (rc) return rc;
  ia.line = out->line.as<RelocLine>();
  FDY_HIP(launch_index_place(ia, nullptr));
  FDY_HIP(hipStreamSynchronize(nullptr));  // before the table and counts are freed
  out->dev.line = out->line.as<RelocLine>();
  out->dev.n = n;
  out->dev.lo_min = lo[0];
  out->dev.hi_max = hi[n - 1];
  out->dev.shift = sh.shift;
  return FDY_OK;
}

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

}  // namespace
}  // namespace fdy

using namespace fdy;

struct fdy_reloc_plan {
  int device = 0;
  RelocPlan plan;
};

namespace {

// Bytes of a graph's file the host reads before its upload: the header and
// the section directory, all that validation and the layout need.
constexpr uint64_t kHeadBytes = sizeof(fdy_file_header) + FDY_SEC_COUNT * sizeof(fdy_section);

// heads[i]: the first min(sizes[i], kHeadBytes) bytes of graph i.  The
// images themselves reach HBM through `pieces` (the upload ring).
int finish_open(fdy_archive* a, const std::vector<std::vector<uint8_t>>& heads, const std::vector<uint64_t>& off,
                const std::vector<uint64_t>& sizes, const std::vector<std::string>& names,
                const std::vector<UploadPiece>& pieces, uint32_t threads) {
  const uint32_t G = a->G;
  a->graphs.resize(G);
  std::vector<std::string> errs(G);
  const X2nTable x2n = make_x2n_table();
  parallel_for(G, default_threads(), [&](uint32_t i) {
    GraphView v;
    errs[i] = validate_image(heads[i].data(), sizes[i], &v);
    if (!errs[i].empty()) return;
    DevGraph& d = a->graphs[i];
    std::memset(&d, 0, sizeof(d));
    for (int s = 0; s < FDY_SEC_COUNT; ++s) {
      d.sec_off[s] = off[i] + v.sec[s].offset;
      d.sec_size[s] = v.sec[s].size;
    }
    d.num_nodes = v.hdr.num_nodes;
    d.num_deps = v.hdr.num_deps;
    d.flags = v.hdr.flags;
    // Digest streams: key bytes, dependency entries, 16-byte records per node (twice).
    d.crc_fin[0] = crc_finish_term(x2n.v, v.sec[FDY_SEC_TOPOLOGY_KEY].size);
    d.crc_fin[1] = crc_finish_term(x2n.v, 8ull * v.hdr.num_deps);
    d.crc_fin[2] = d.crc_fin[3] = crc_finish_term(x2n.v, 16ull * v.hdr.num_nodes);
    // Capacity of the param image: every param rounds up to whole words, and
    // an extra-style node's arg buffer can end in a partial word.
    uint64_t cap = (v.sec[FDY_SEC_PARAM_DATA].size + 7) / 8 + v.sec[FDY_SEC_PARAM_INDEX].size / 8 +
                   (v.sec[FDY_SEC_ARG_DATA].size + 7) / 8 + v.hdr.num_nodes;
    if (cap > 0xFFFFFFF0ull) {
      errs[i] = "param image of more than 2^32 words";
      return;
    }
    d.word_cap = (uint32_t)cap;
  });
  for (uint32_t i = 0; i < G; ++i)
    if (!errs[i].empty()) return err(FDY_E_FORMAT, names[i] + ": " + errs[i]);

  uint64_t nodes = 0, words = 0, slots = 0, chunks = 0;
  for (uint32_t i = 0; i < G; ++i) {
    DevGraph& d = a->graphs[i];
    d.node_base = nodes;
    d.word_base = words;
    d.tile_base = (uint32_t)slots;
    d.tile_cap = (uint32_t)std::max<uint64_t>(1, (d.word_cap + kTileWords - 1) / kTileWords);
    d.chunk_base = (uint32_t)chunks;
    nodes += d.num_nodes;
    words += d.word_cap;
    slots += d.tile_cap;
    chunks += std::max<uint64_t>(1, (d.num_nodes + kNodeChunk - 1) / kNodeChunk);  // at least one per graph
  }
  if (nodes >= (1ull << 32)) return err(FDY_E_FORMAT, "archive too large (2^32 nodes or more)");
  // The member pass launches 1024 threads per tile, and a launch holds fewer than 2^32 threads.
  if (slots >= (1ull << 22)) return err(FDY_E_FORMAT, "archive too large (more than 2^22 diff tiles, 128 GiB of params)");
  a->total_nodes = nodes;
  a->total_cap = words;
  a->num_slots = (uint32_t)slots;
  a->num_chunks = (uint32_t)chunks;

  // The digest units: every 4 KB slice of every key and dependency table.
  std::vector<DigestUnit> units;
  for (uint32_t i = 0; i < G; ++i) {
    const DevGraph& d = a->graphs[i];
    const uint64_t src[2] = {d.sec_off[FDY_SEC_TOPOLOGY_KEY], d.sec_off[FDY_SEC_DEPS]};
    const uint64_t len[2] = {d.sec_size[FDY_SEC_TOPOLOGY_KEY], 8ull * d.num_deps};
    for (uint32_t k = 0; k < 2; ++k)
      for (uint64_t b = 0; b * kSliceBytes < len[k]; ++b) units.push_back({src[k], len[k], (uint32_t)b, 4 * i + k, 0});
  }
  if (units.size() >= (1ull << 31)) return err(FDY_E_FORMAT, "archive too large (keys and dependency tables past 8 TB)");
  a->num_units = (uint32_t)units.size();
  if (units.empty()) units.push_back({0, 0, 0, 0, 0});  // never read (no unit workgroups)

  // The tables: parts of one arena allocation, each 256-byte aligned.
  const std::pair<DevBuf*, uint64_t> parts[] = {
      {&a->dgraphs, G * sizeof(DevGraph)},  {&a->cc, sizeof(CrcConsts)},
      {&a->digests, 32ull * G},             {&a->tmpl, 4ull * G},
      {&a->explicit_tmpl, 4ull * G},        {&a->status, 4ull * G},
      {&a->gwords, 4ull * G},               {&a->pbytes, 8ull * G},
      {&a->live_cur, 4ull * G},             {&a->nflags, nodes},
      {&a->ndesc, nodes * sizeof(NodeDesc)}, {&a->nptrs, 16 * nodes},
      {&a->live_src, 4 * nodes},            {&a->tile_node, 4 * slots},
      {&a->chunk_gt, 8 * chunks},          {&a->node_pbytes, 8 * nodes},
      {&a->units, sizeof(DigestUnit) * units.size()},
      {&a->key_hash, 8ull * G},             {&a->chunks, sizeof(NodeChunk) * chunks},
      {&a->slot_desc, sizeof(SlotDesc) * slots}, {&a->tslot_desc, sizeof(SlotDesc) * slots}, {&a->tslot_count, 4},
      {&a->sub_count, 4 * slots * kSubsPerSlot}, {&a->slot_rec, 4 * slots},
      {&a->restore_flags, 4},               {&a->slot_spill, 4 * slots},
      {&a->sub_off, 4 * slots * kSubsPerSlot},
  };
  uint64_t arena_bytes = 0;
  for (const auto& pt : parts) arena_bytes += (pt.second + 255) / 256 * 256;
  int rc = dev_alloc(a->arena, arena_bytes, "archive tables");
  if (!rc) {
    uint64_t at = 0;
    for (const auto& pt : parts) {
      pt.first->p = static_cast<uint8_t*>(a->arena.p) + at;
      pt.first->bytes = pt.second;
      pt.first->owned = false;
      at += (pt.second + 255) / 256 * 256;
    }
  }
  if (!rc) rc = dev_alloc(a->img, a->img_bytes + 4096, "archive images");
  if (!rc) rc = dev_alloc(a->image, 8 * words, "param images");
  if (!rc) rc = alloc_restore_buffers(a);
  if (rc) return rc;

  rc = upload(static_cast<uint8_t*>(a->img.p), pieces, threads);
  if (rc) return rc;
  FDY_HIP(hipMemset(static_cast<uint8_t*>(a->img.p) + a->img_bytes, 0, 4096));
  FDY_HIP(hipMemcpy(a->dgraphs.p, a->graphs.data(), G * sizeof(DevGraph), hipMemcpyHostToDevice));
  auto consts = std::make_unique<CrcConsts>();
  make_crc_consts(consts.get());
  FDY_HIP(hipMemcpy(a->cc.p, consts.get(), sizeof(CrcConsts), hipMemcpyHostToDevice));
  // No key hash is published yet (the grouping pass tags its hashes with the
  // restore's epoch, never 0).
  FDY_HIP(hipMemset(a->key_hash.p, 0, 8ull * G));
  FDY_HIP(hipMemcpy(a->units.p, units.data(), sizeof(DigestUnit) * units.size(), hipMemcpyHostToDevice));
  return FDY_OK;
}

}  // namespace

namespace fdy {

int alloc_restore_buffers(fdy_archive* a) {
  const uint64_t words = a->total_cap;
  const ScratchLevel& L = kScratchLevels[a->scratch_level];
  a->ovr.release();
  a->cand.release();
  a->aux.release();
  a->rec_shift = L.rec_shift;
  a->cand_cap = L.cand_cap;
  a->spill_cap = L.spill_cap;
  int rc = dev_alloc(a->cand, sizeof(Candidate) * ((uint64_t)a->cand_cap * kSubsPerSlot + a->spill_cap) * a->num_slots,
                     "candidate regions");
  if (!rc && a->need_aux) rc = dev_alloc(a->aux, 8 * words, "ragged word sources");
  if (!rc) rc = dev_alloc(a->ovr, sizeof(fdy_override) * std::max<uint64_t>(1, words >> a->rec_shift), "override records");
  if (!rc) a->compact = false;
  return rc;
}

// The templates' live images, filled from R (after a restore, once its
// results are settled).
int fill_live(fdy_archive* a, hipStream_t s) {
  const uint32_t G = a->G;
  std::vector<uint64_t> lbase(G, 0);
  uint64_t live_words = 0;
  for (uint32_t g = 0; g < G; ++g)
    if (a->h_tmpl[g] == g) {
      lbase[g] = live_words;
      live_words += a->graphs[g].word_cap;
    }
  const uint64_t bytes = 8 * std::max<uint64_t>(1, live_words);
  if (a->live.bytes != bytes) {
    a->live.release();
    int rc = dev_alloc(a->live, bytes, "template live images");
    if (rc) return rc;
  }
  for (uint32_t g = 0; g < G; ++g)
    if (a->h_tmpl[g] == g && a->h_gwords[g])
      FDY_HIP(hipMemcpyAsync(a->live.as<uint64_t>() + lbase[g], a->image.as<uint64_t>() + r_base(a, g),
                             8ull * a->h_gwords[g], hipMemcpyDeviceToDevice, s));
  FDY_HIP(hipStreamSynchronize(s));
  a->h_live_base = std::move(lbase);
  a->live_ready = true;
  return FDY_OK;
}

int compact_for_serving(fdy_archive* a, hipStream_t s) {
  if (a->compact) return FDY_OK;
  int rc = ensure_cache(a, s);
  if (rc) return rc;
  const uint32_t G = a->G;
  std::vector<uint64_t> rbase(G, 0);
  uint64_t r_words = 0;
  for (uint32_t g = 0; g < G; ++g) {
    rbase[g] = r_words;
    r_words += a->h_gwords[g];
  }
  DevBuf ovr, image;
  rc = dev_alloc(ovr, sizeof(fdy_override) * std::max<uint64_t>(1, a->h_ovr_off[G]), "packed override records");
  if (!rc) rc = dev_alloc(image, 8 * std::max<uint64_t>(1, r_words), "packed param images");
  if (rc) return rc;
  FDY_HIP(hipSetDevice(a->device));
  for (uint32_t g = 0; g < G; ++g) {
    const uint64_t n = a->h_ovr_off[g + 1] - a->h_ovr_off[g];
    if (n)
      FDY_HIP(hipMemcpyAsync(ovr.as<fdy_override>() + a->h_ovr_off[g], a->ovr.as<fdy_override>() + ovr_base(a, g),
                             sizeof(fdy_override) * n, hipMemcpyDeviceToDevice, s));
    if (a->h_gwords[g])
      FDY_HIP(hipMemcpyAsync(image.as<uint64_t>() + rbase[g], a->image.as<uint64_t>() + a->graphs[g].word_base,
                             8ull * a->h_gwords[g], hipMemcpyDeviceToDevice, s));
  }
  FDY_HIP(hipStreamSynchronize(s));
  a->ovr.swap(ovr);
  a->image.swap(image);
  a->cand.release();
  a->aux.release();
  a->h_r_base = std::move(rbase);
  a->compact = true;
  return FDY_OK;
}

uint64_t held_bytes(const fdy_archive* a) {
  const DevBuf* bufs[] = {&a->arena, &a->img, &a->image, &a->aux, &a->live, &a->ovr, &a->cand,
                          &a->reloc.line};
  uint64_t n = 0;
  for (const DevBuf* b : bufs) n += b->bytes;
  return n;
}

int ensure_cache(fdy_archive* a, hipStream_t s) {
  if (!a->restored) return err(FDY_E_STATE, "call fdy_restore first");
  if (a->cached) return FDY_OK;
  FDY_HIP(hipStreamSynchronize(s));
  const uint32_t G = a->G;
  uint32_t flags = 0;
  FDY_HIP(hipMemcpy(&flags, a->restore_flags.p, 4, hipMemcpyDeviceToHost));
  while (flags & (kFlagNeedAux | kFlagOverflow)) {
    // The restore found a ragged node without ragged-word sources, or ran
    // out of scratch: its results are discarded, and it runs again with what
    // it lacked (kept for every later restore of this archive).
    if (flags & kFlagNeedAux) {
      if (a->need_aux) return err(FDY_E_STATE, "the restore asked again for ragged-word sources it had");
      a->need_aux = true;
    }
    if (flags & kFlagOverflow) {
      if (a->scratch_level == kScratchFull) return err(FDY_E_STATE, "the restore overflowed full-capacity scratch");
      ++a->scratch_level;
    }
    int rc = alloc_restore_buffers(a);
    if (!rc) rc = enqueue_restore(a, s);
    if (rc) return rc;
    FDY_HIP(hipStreamSynchronize(s));
    FDY_HIP(hipMemcpy(&flags, a->restore_flags.p, 4, hipMemcpyDeviceToHost));
  }
  a->h_tmpl.resize(G);
  a->h_status.resize(G);
  a->h_gwords.resize(G);
  a->h_pbytes.resize(G);
  a->h_ovr_off.resize(G + 1);
  // A compared word equal to the template's only once relocated makes no
  // record and leaves a gap where the search pass placed its slot's records
  // by their bounds: such override arrays are closed up before anything
  // reads them (rare; never in archives without such words).
  if (flags & kFlagGaps) {
    RepackArgs rp{a->dgraphs.as<DevGraph>(), a->sub_count.as<uint32_t>(), a->slot_rec.as<uint32_t>(),
                  a->ovr.as<fdy_override>(), G, a->rec_shift};
    FDY_HIP(launch_repack(rp, s));
    FDY_HIP(hipStreamSynchronize(s));
  }
  std::vector<uint32_t> slot_rec(a->num_slots);
  FDY_HIP(hipMemcpy(a->h_tmpl.data(), a->tmpl.p, 4ull * G, hipMemcpyDeviceToHost));
  FDY_HIP(hipMemcpy(a->h_status.data(), a->status.p, 4ull * G, hipMemcpyDeviceToHost));
  FDY_HIP(hipMemcpy(a->h_gwords.data(), a->gwords.p, 4ull * G, hipMemcpyDeviceToHost));
  FDY_HIP(hipMemcpy(a->h_pbytes.data(), a->pbytes.p, 8ull * G, hipMemcpyDeviceToHost));
  FDY_HIP(hipMemcpy(slot_rec.data(), a->slot_rec.p, 4ull * a->num_slots, hipMemcpyDeviceToHost));
  // Offsets of each graph's records in canonical order over all graphs (the
  // device keeps graph g's records from index word_base(g) instead): the
  // sums of its slots' record counts.
  a->h_ovr_off[0] = 0;
  for (uint32_t i = 0; i < G; ++i) {
    uint64_t n = 0;
    for (uint32_t k = 0; k < a->graphs[i].tile_cap; ++k) n += slot_rec[a->graphs[i].tile_base + k];
    a->h_ovr_off[i + 1] = a->h_ovr_off[i] + n;
  }
  a->h_current.resize(G);
  for (uint32_t i = 0; i < G; ++i) a->h_current[i] = i;
  int rc = fill_live(a, s);
  if (rc) return rc;
  a->cached = true;
  return FDY_OK;
}

int check_graph(const fdy_archive* a, uint32_t g) {
  if (!a) return err(FDY_E_INVALID, "null archive");
  if (g >= a->G) return err(FDY_E_RANGE, "graph " + std::to_string(g) + " out of range (num_graphs=" +
                                             std::to_string(a->G) + ")");
  return FDY_OK;
}

int check_switchable(fdy_archive* a, uint32_t g, uint32_t* t_out) {
  const uint32_t t = a->h_tmpl[g];
  if (a->h_status[g] & FDY_GRAPH_NODE_COUNT)
    return err(FDY_E_MISMATCH, "graph " + std::to_string(g) + " has " + std::to_string(a->graphs[g].num_nodes) +
                                   " nodes but its template " + std::to_string(t) + " has " +
                                   std::to_string(a->graphs[t].num_nodes));
  if (a->h_status[g] & FDY_GRAPH_OVERFLOW)
    return err(FDY_E_MISMATCH, "graph " + std::to_string(g) + " has a param image larger than its sections allow");
  if (a->h_status[t] & FDY_GRAPH_OVERFLOW)
    return err(FDY_E_MISMATCH, "the template " + std::to_string(t) + " of graph " + std::to_string(g) +
                                   " has a param image larger than its sections allow");
  *t_out = t;
  return FDY_OK;
}

// The scatter that moves the live image of g's group from its current graph
// to g.
// The switch of g's group from its graph c to g.
SwitchArgs switch_args(const fdy_archive* a, uint32_t g, uint8_t* dirty, uint32_t c) {
  const uint32_t t = a->h_tmpl[g];
  SwitchArgs w{};
  w.ovr_cur = a->ovr.as<fdy_override>() + ovr_base(a, c);
  w.n_cur = a->h_ovr_off[c + 1] - a->h_ovr_off[c];
  w.ovr_new = a->ovr.as<fdy_override>() + ovr_base(a, g);
  w.n_new = a->h_ovr_off[g + 1] - a->h_ovr_off[g];
  w.tmpl_image = a->image.as<uint64_t>() + r_base(a, t);
  w.live = a->live.as<uint64_t>() + live_base(a, t);
  w.flags_cur = a->nflags.as<uint8_t>() + a->graphs[c].node_base;
  w.flags_new = a->nflags.as<uint8_t>() + a->graphs[g].node_base;
  w.live_src = a->live_src.as<uint32_t>() + a->graphs[t].node_base;
  w.dirty = dirty;
  w.num_nodes = a->graphs[t].num_nodes;
  w.target = g;
  w.tmpl = t;
  return w;
}
SwitchArgs switch_args(const fdy_archive* a, uint32_t g, uint8_t* dirty) {
  return switch_args(a, g, dirty, a->h_current[a->h_tmpl[g]]);
}

int enqueue_switch(fdy_archive* a, uint32_t g, hipStream_t s, uint8_t* dirty, bool set_device) {
  const uint32_t t = a->h_tmpl[g];
  if (a->h_current[t] == g) return FDY_OK;
  if (set_device) FDY_HIP(hipSetDevice(a->device));
  const SwitchArgs w = switch_args(a, g, dirty);
  FDY_HIP(launch_switch(w, s));
  a->h_current[t] = g;
  return FDY_OK;
}

}  // namespace fdy

namespace {

template <typename T>
int copy_out(const void* dev, uint64_t n, T* out, uint64_t cap, uint64_t* n_out) {
  if (n_out) *n_out = n;
  if (!out) return FDY_OK;
  if (cap < n) return err(FDY_E_CAPACITY, "output array holds " + std::to_string(cap) + ", needs " + std::to_string(n));
  if (n) FDY_HIP(hipMemcpy(out, dev, n * sizeof(T), hipMemcpyDeviceToHost));
  return FDY_OK;
}

}  // namespace

namespace fdy {

int enqueue_restore(fdy_archive* a, hipStream_t s) {
  RestoreArgs r{};
  r.img = a->img.as<uint8_t>();
  r.graphs = a->dgraphs.as<DevGraph>();
  r.cc = a->cc.as<CrcConsts>();
  r.num_graphs = a->G;
  r.num_slots = a->num_slots;
  r.num_chunks = a->num_chunks;
  r.chunk_gt = a->chunk_gt.as<uint2>();
  r.num_units = a->num_units;
  r.units = a->units.as<DigestUnit>();
  r.chunks = a->chunks.as<NodeChunk>();
  r.digests = a->digests.as<uint64_t>();
  r.explicit_template = a->use_explicit ? a->explicit_tmpl.as<uint32_t>() : nullptr;
  r.key_hash = a->key_hash.as<uint64_t>();
  a->epoch = a->epoch % 65535 + 1;
  r.epoch = a->epoch;
  r.hash_wait_spins = a->hash_wait_spins;
  r.template_of = a->tmpl.as<uint32_t>();
  r.status = a->status.as<uint32_t>();
  r.gwords = a->gwords.as<uint32_t>();
  r.pbytes = a->pbytes.as<uint64_t>();
  r.node_flags = a->nflags.as<uint8_t>();
  r.node_desc = a->ndesc.as<NodeDesc>();
  r.node_ptrs = a->nptrs.as<uint64_t>();
  r.tile_node = a->tile_node.as<uint32_t>();
  r.tslot_desc = a->tslot_desc.as<SlotDesc>();
  r.tslot_count = a->tslot_count.as<uint32_t>();
  r.slot_desc = a->slot_desc.as<SlotDesc>();
  r.aux = a->aux.as<uint64_t>();
  r.image = a->image.as<uint64_t>();
  r.live_src = a->live_src.as<uint32_t>();
  r.live_cur = a->live_cur.as<uint32_t>();
  r.ovr = a->ovr.as<fdy_override>();
  r.rec_shift = a->rec_shift;
  r.cand_cap = a->cand_cap;
  r.spill_cap = a->spill_cap;
  r.cand = a->cand.as<Candidate>();
  r.slot_spill = a->slot_spill.as<uint32_t>();
  r.sub_off = a->sub_off.as<uint32_t>();
  r.sub_count = a->sub_count.as<uint32_t>();
  r.slot_rec = a->slot_rec.as<uint32_t>();
  r.restore_flags = a->restore_flags.as<uint32_t>();
  r.node_pbytes = a->node_pbytes.as<uint64_t>();
  r.reloc = a->reloc.dev;
  if (a->timing) {
    for (hipEvent_t& e : a->ev)
      if (!e) FDY_HIP(hipEventCreate(&e));
    FDY_HIP(hipEventRecord(a->ev[0], s));
  }
  // Grouping first (the key and dependency digests run beside the second
  // node pass).
  FDY_HIP(launch_group(r, s));
  // Phase timing records no event inside a phase: each event waits for the
  // kernel before it to drain, which adds 1-3 us between kernels.
  const bool per_kernel = a->timing == 1;
  if (per_kernel) FDY_HIP(hipEventRecord(a->ev[1], s));
  FDY_HIP(launch_node(r, s));
  if (a->timing) FDY_HIP(hipEventRecord(a->ev[2], s));
  FDY_HIP(launch_diff_templates(r, s));
  if (per_kernel) FDY_HIP(hipEventRecord(a->ev[3], s));
  FDY_HIP(launch_diff_members(r, s));
  if (per_kernel) FDY_HIP(hipEventRecord(a->ev[4], s));
  FDY_HIP(launch_diff_search(r, s));
  if (a->timing) FDY_HIP(hipEventRecord(a->ev[5], s));
  a->timed = a->timing;
  a->restored = true;
  a->cached = false;
  a->live_ready = false;
  a->last_stream = s;
  return FDY_OK;
}

}  // namespace fdy

extern "C" {

const char* fdy_last_error(void) { return g_err.c_str(); }
const char* fdy_version(void) { return "foundry-mi355x restore 0.1 (gfx950)"; }

int fdy_archive_open(const char* const* paths, uint32_t n, uint32_t num_threads, fdy_archive** out) {
  if (!paths || !out || n == 0) return err(FDY_E_INVALID, "need at least one path and an output pointer");
  *out = nullptr;
  const uint32_t threads = std::min(num_threads ? num_threads : 4u, n);
  std::vector<std::string> names(n);
  std::vector<uint64_t> sizes(n), off(n);
  std::vector<std::vector<uint8_t>> converted(n);  // graphs read from their JSON document
  std::vector<std::vector<uint8_t>> heads(n);      // header and section directory of each graph
  std::vector<int> fds(n, -1);
  struct Fds {
    std::vector<int>& v;
    ~Fds() {
      for (int fd : v)
        if (fd >= 0) ::close(fd);
    }
  } close_fds{fds};
  std::vector<std::string> errs(n);
  std::vector<int> codes(n, FDY_OK);
  // Which file holds each graph: the .cugraph if it opens with a v1 header
  // (csrc/BinaryGraphIO.cpp:710-737), else the JSON document at the path
  // (csrc/CUDAGraphParallel.cpp:1606-1617), converted as save_binary would.
  // Phase 1a's reads (csrc/CUDAGraphParallel.cpp:1583-1620) are split: the
  // header and section directory here, the rest streamed to HBM below.
  parallel_for(n, threads, [&](uint32_t i) {
    const std::string path = paths[i] ? paths[i] : "";
    std::string p = path;
    if (p.size() >= 5 && p.compare(p.size() - 5, 5, ".json") == 0) p = p.substr(0, p.size() - 5) + ".cugraph";
    heads[i].assign(kHeadBytes, 0);
    struct stat st;
    const int fd = p.empty() ? -1 : ::open(p.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd >= 0 && fstat(fd, &st) == 0 && S_ISREG(st.st_mode) && (uint64_t)st.st_size >= sizeof(fdy_file_header)) {
      const uint64_t want = std::min<uint64_t>((uint64_t)st.st_size, kHeadBytes);
      uint64_t got = 0;
      while (got < want) {
        const ssize_t r = pread(fd, heads[i].data() + got, want - got, (off_t)got);
        if (r <= 0) break;
        got += (uint64_t)r;
      }
      fdy_file_header h;
      std::memcpy(&h, heads[i].data(), sizeof h);
      if (got == want && std::memcmp(h.magic, "CUGRAPH", 8) == 0 && h.version == FDY_FORMAT_VERSION) {
        names[i] = p;
        sizes[i] = (uint64_t)st.st_size;
        fds[i] = fd;
        return;
      }
    }
    if (fd >= 0) ::close(fd);
    names[i] = path;
    std::string text;
    FILE* f = path.empty() ? nullptr : std::fopen(path.c_str(), "rb");
    if (!f) {
      codes[i] = FDY_E_IO;
      errs[i] = "cannot open " + (p.empty() ? std::string("<null path>") : p) + (p == path ? "" : " or " + path);
      return;
    }
    char buf[1 << 16];
    size_t got;
    while ((got = std::fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, got);
    std::fclose(f);
    codes[i] = fdy::cugraph_for_load(text.data(), text.size(), converted[i], errs[i]);
    if (codes[i] == FDY_OK) {
      sizes[i] = converted[i].size();
      std::memcpy(heads[i].data(), converted[i].data(), std::min<uint64_t>(sizes[i], kHeadBytes));
    } else {
      errs[i] = path + ": " + errs[i];
    }
  });
  for (uint32_t i = 0; i < n; ++i)
    if (codes[i] != FDY_OK) return err(codes[i], errs[i]);
  uint64_t at = 0;
  std::vector<UploadPiece> pieces;
  for (uint32_t i = 0; i < n; ++i) {
    off[i] = at;
    const uint64_t end = align_up(at + sizes[i], 256);
    add_pieces(pieces, at, sizes[i], end - at - sizes[i], fds[i], converted[i].empty() ? nullptr : converted[i].data());
    at = end;
  }
  auto a = std::make_unique<fdy_archive>();
  (void)hipGetDevice(&a->device);
  a->G = n;
  a->img_bytes = at;
  const int rc = finish_open(a.get(), heads, off, sizes, names, pieces, std::max(threads, default_threads()));
  if (rc) return rc;
  *out = a.release();
  return FDY_OK;
}

int fdy_archive_open_images(const uint8_t* const* images, const uint64_t* sizes_in, uint32_t n, fdy_archive** out) {
  if (!images || !sizes_in || !out || n == 0) return err(FDY_E_INVALID, "need at least one image and an output pointer");
  *out = nullptr;
  std::vector<std::string> names(n);
  std::vector<uint64_t> sizes(sizes_in, sizes_in + n), off(n);
  std::vector<std::vector<uint8_t>> heads(n);
  std::vector<UploadPiece> pieces;
  uint64_t at = 0;
  for (uint32_t i = 0; i < n; ++i) {
    if (!images[i] && sizes[i]) return err(FDY_E_INVALID, "null image " + std::to_string(i));
    names[i] = "image " + std::to_string(i);
    heads[i].assign(kHeadBytes, 0);
    if (sizes[i]) std::memcpy(heads[i].data(), images[i], std::min<uint64_t>(sizes[i], kHeadBytes));
    off[i] = at;
    const uint64_t end = align_up(at + sizes[i], 256);
    add_pieces(pieces, at, sizes[i], end - at - sizes[i], -1, images[i]);
    at = end;
  }
  auto a = std::make_unique<fdy_archive>();
  (void)hipGetDevice(&a->device);
  a->G = n;
  a->img_bytes = at;
  const int rc = finish_open(a.get(), heads, off, sizes, names, pieces, default_threads());
  if (rc) return rc;
  *out = a.release();
  return FDY_OK;
}

int fdy_archive_close(fdy_archive* a) {
  if (!a) return FDY_OK;
  if (a->num_bound)
    return err(FDY_E_STATE, std::to_string(a->num_bound) + " group graph(s) still use this archive; destroy them first");
  (void)hipSetDevice(a->device);
  (void)hipDeviceSynchronize();
  delete a;
  return FDY_OK;
}

int fdy_archive_info_get(fdy_archive* a, fdy_archive_info* o) {
  if (!a || !o) return err(FDY_E_INVALID, "null argument");
  std::memset(o, 0, sizeof(*o));
  o->num_graphs = a->G;
  o->total_nodes = a->total_nodes;
  o->file_bytes = a->img_bytes;
  o->num_intervals = a->reloc.dev.n;
  if (a->restored) {
    int rc = ensure_cache(a, a->last_stream);  // settles the restore (a second run if it lacked scratch)
    if (rc) return rc;
    for (uint32_t i = 0; i < a->G; ++i) {
      o->num_groups += a->h_tmpl[i] == i;
      o->total_words += a->h_gwords[i];
      o->total_param_bytes += a->h_pbytes[i];
    }
    o->total_overrides = a->h_ovr_off[a->G];
  }
  o->device_bytes = held_bytes(a);
  o->serving_layout = a->compact ? 1u : 0u;
  o->scratch = a->scratch_level | (a->need_aux ? FDY_SCRATCH_RAGGED : 0u);
  return FDY_OK;
}

int fdy_archive_set_relocation(fdy_archive* a, const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo,
                               uint64_t n, uint32_t policy) {
  if (!a) return err(FDY_E_INVALID, "null archive");
  FDY_HIP(hipSetDevice(a->device));
  FDY_HIP(hipDeviceSynchronize());  // kernels in flight may still read the old table
  a->reloc.~RelocPlan();
  new (&a->reloc) RelocPlan();
  return build_reloc_plan(lo, hi, nlo, n, policy, &a->reloc);
}

int fdy_archive_set_groups(fdy_archive* a, const uint32_t* template_of) {
  if (!a) return err(FDY_E_INVALID, "null archive");
  if (!template_of) {
    a->use_explicit = false;
    return FDY_OK;
  }
  for (uint32_t i = 0; i < a->G; ++i) {
    const uint32_t t = template_of[i];
    if (t >= a->G) return err(FDY_E_RANGE, "template_of[" + std::to_string(i) + "] out of range");
    if (template_of[t] != t)
      return err(FDY_E_INVALID, "template_of[" + std::to_string(i) + "] = " + std::to_string(t) +
                                    " is not a template itself");
  }
  FDY_HIP(hipSetDevice(a->device));
  FDY_HIP(hipMemcpy(a->explicit_tmpl.p, template_of, 4ull * a->G, hipMemcpyHostToDevice));
  a->use_explicit = true;
  return FDY_OK;
}

int fdy_cugraph_from_json(const char* json, uint64_t len, uint8_t* out, uint64_t cap, uint64_t* size_out) {
  if (!json && len) return err(FDY_E_INVALID, "null document");
  if (!size_out) return err(FDY_E_INVALID, "need size_out");
  std::vector<uint8_t> img;
  std::string why;
  const int rc = fdy::cugraph_from_json(json ? json : "", len, img, why);
  if (rc) return err(rc, why);
  *size_out = img.size();
  if (!out || cap < img.size())
    return err(FDY_E_CAPACITY, "archive needs " + std::to_string(img.size()) + " bytes, buffer holds " + std::to_string(out ? cap : 0));
  std::memcpy(out, img.data(), img.size());
  return FDY_OK;
}

int fdy_load_topology_key(const char* json, uint64_t len, char* out, uint64_t cap, uint64_t* size_out) {
  if (!json && len) return err(FDY_E_INVALID, "null document");
  if (!size_out) return err(FDY_E_INVALID, "need size_out");
  std::string key, why;
  const int rc = fdy::load_topology_key(json ? json : "", len, key, why);
  if (rc) return err(rc, why);
  *size_out = key.size();
  if (!out || cap < key.size())
    return err(FDY_E_CAPACITY, "key needs " + std::to_string(key.size()) + " bytes, buffer holds " +
                                   std::to_string(out ? cap : 0));
  std::memcpy(out, key.data(), key.size());
  return FDY_OK;
}

int fdy_cugraph_save_binary(const char* bin_path, const char* json, uint64_t len) {
  if (!bin_path) return err(FDY_E_INVALID, "null path");
  if (!json && len) return err(FDY_E_INVALID, "null document");
  std::vector<uint8_t> img;
  std::string why;
  const int rc = fdy::cugraph_from_json(json ? json : "", len, img, why);
  if (rc) return err(rc, why);
  FILE* f = std::fopen(bin_path, "wb");
  if (!f) return err(FDY_E_IO, std::string("Failed to write binary graph: ") + bin_path);
  const bool ok = std::fwrite(img.data(), 1, img.size(), f) == img.size();
  if (std::fclose(f) != 0 || !ok) return err(FDY_E_IO, std::string("Failed to write binary graph: ") + bin_path);
  return FDY_OK;
}

int fdy_manifest_groups(const char* text, uint64_t len, const char* const* names, uint32_t n, uint32_t* template_of,
                        int* used) {
  if ((!text && len) || (!names && n) || (!template_of && n) || !used)
    return err(FDY_E_INVALID, "need the manifest text, the names, the output array and the used flag");
  *used = 0;
  std::unordered_map<std::string, uint32_t> index;
  for (uint32_t i = 0; i < n; ++i) {
    if (!names[i]) return err(FDY_E_INVALID, "null name " + std::to_string(i));
    index[names[i]] = i;  // a repeated name resolves to its last graph (filename_to_idx[fname] = i, 1728-1732)
  }
  json::Value doc;
  std::string perr;
  json::Reader reader(text ? text : "", len);
  // Any shape the reference's parse would throw on means "no manifest" (1776-1783).
  if (!reader.parse(doc, perr) || doc.kind != json::Value::Object) return FDY_OK;
  const json::Value* groups = doc.get("topology_groups");
  if (!groups || groups->kind != json::Value::Array) return FDY_OK;
  std::vector<uint32_t> res(n, UINT32_MAX);
  for (const json::Value& g : groups->items) {
    if (g.kind != json::Value::Object) return FDY_OK;
    const json::Value* t = g.get("template");
    if (!t || t->kind != json::Value::String) return FDY_OK;
    auto ti = index.find(t->s);
    if (ti == index.end()) continue;  // members of a skipped group are not read (1754-1755)
    const json::Value* m = g.get("members");
    if (!m || m->kind != json::Value::Array) return FDY_OK;
    for (const json::Value& mem : m->items) {
      if (mem.kind != json::Value::String) return FDY_OK;
      if (mem.s == t->s) continue;
      auto mi = index.find(mem.s);
      if (mi == index.end()) continue;
      res[mi->second] = ti->second;
    }
  }
  for (uint32_t i = 0; i < n; ++i) {
    const uint32_t t = res[i];
    if (t != UINT32_MAX && res[t] != UINT32_MAX)
      return err(FDY_E_INVALID, std::string("manifest: ") + names[i] + " has template " + names[t] +
                                    ", which is itself a member of another group");
  }
  for (uint32_t i = 0; i < n; ++i) template_of[i] = res[i] == UINT32_MAX ? i : res[i];
  *used = 1;
  return FDY_OK;
}

int fdy_archive_set_manifest(fdy_archive* a, const char* text, uint64_t len, const char* const* names, int* used) {
  if (!a || !used) return err(FDY_E_INVALID, "need an archive and the used flag");
  std::vector<uint32_t> t(a->G);
  int rc = fdy_manifest_groups(text, len, names, a->G, t.data(), used);
  if (rc) return rc;
  return *used ? fdy_archive_set_groups(a, t.data()) : fdy_archive_set_groups(a, nullptr);
}

int fdy_restore(fdy_archive* a, void* stream) {
  if (!a) return err(FDY_E_INVALID, "null archive");
  if (a->num_bound)
    return err(FDY_E_STATE, "group graphs hold the restored params; destroy them before restoring again");
  hipStream_t s = static_cast<hipStream_t>(stream);
  FDY_HIP(hipSetDevice(a->device));
  if (a->compact) {  // group graphs were bound and are gone: back to the restore's layout
    a->image.release();
    int rc = dev_alloc(a->image, 8 * a->total_cap, "param images");
    if (!rc) rc = alloc_restore_buffers(a);
    if (rc) return rc;
  }
  return enqueue_restore(a, s);
}

int fdy_set_timing(fdy_archive* a, int enabled) {
  if (!a) return err(FDY_E_INVALID, "null archive");
  if (enabled < 0 || enabled > 2) return err(FDY_E_INVALID, "timing mode is 0 (off), 1 (every kernel) or 2 (phases)");
  a->timing = enabled;
  return FDY_OK;
}

int fdy_set_group_wait(fdy_archive* a, uint32_t spins) {
  if (!a) return err(FDY_E_INVALID, "null archive");
  a->hash_wait_spins = spins;
  return FDY_OK;
}

int fdy_restore_timing_get(fdy_archive* a, fdy_restore_timing* o) {
  if (!a || !o) return err(FDY_E_INVALID, "null argument");
  if (!a->timed) return err(FDY_E_STATE, "enable timing with fdy_set_timing before fdy_restore");
  FDY_HIP(hipEventSynchronize(a->ev[5]));
  o->group_ms = o->node_ms = o->tmpl_ms = o->diff_ms = o->search_ms = -1.0f;
  if (a->timed == 1) {
    FDY_HIP(hipEventElapsedTime(&o->group_ms, a->ev[0], a->ev[1]));
    FDY_HIP(hipEventElapsedTime(&o->node_ms, a->ev[1], a->ev[2]));
    FDY_HIP(hipEventElapsedTime(&o->tmpl_ms, a->ev[2], a->ev[3]));
    FDY_HIP(hipEventElapsedTime(&o->diff_ms, a->ev[3], a->ev[4]));
    FDY_HIP(hipEventElapsedTime(&o->search_ms, a->ev[4], a->ev[5]));
  }
  FDY_HIP(hipEventElapsedTime(&o->total_ms, a->ev[0], a->ev[5]));
  FDY_HIP(hipEventElapsedTime(&o->prepare_ms, a->ev[0], a->ev[2]));
  FDY_HIP(hipEventElapsedTime(&o->diff_phase_ms, a->ev[2], a->ev[5]));
  return FDY_OK;
}

int fdy_get_digests(fdy_archive* a, void* stream, uint64_t* out) {
  if (!a || !out) return err(FDY_E_INVALID, "null argument");
  int rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  FDY_HIP(hipMemcpy(out, a->digests.p, 32ull * a->G, hipMemcpyDeviceToHost));
  return FDY_OK;
}

int fdy_get_groups(fdy_archive* a, void* stream, uint32_t* out) {
  if (!a || !out) return err(FDY_E_INVALID, "null argument");
  int rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  std::memcpy(out, a->h_tmpl.data(), 4ull * a->G);
  return FDY_OK;
}

int fdy_get_graph_status(fdy_archive* a, void* stream, uint32_t* out) {
  if (!a || !out) return err(FDY_E_INVALID, "null argument");
  int rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  // TYPE_MISMATCH is set by the diff pass after the cache may have been taken.
  FDY_HIP(hipMemcpy(a->h_status.data(), a->status.p, 4ull * a->G, hipMemcpyDeviceToHost));
  std::memcpy(out, a->h_status.data(), 4ull * a->G);
  return FDY_OK;
}

int fdy_get_override_offsets(fdy_archive* a, void* stream, uint64_t* out) {
  if (!a || !out) return err(FDY_E_INVALID, "null argument");
  int rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  std::memcpy(out, a->h_ovr_off.data(), 8ull * (a->G + 1));
  return FDY_OK;
}

int fdy_get_param_bytes(fdy_archive* a, void* stream, uint64_t* out) {
  if (!a || !out) return err(FDY_E_INVALID, "null argument");
  int rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  std::memcpy(out, a->h_pbytes.data(), 8ull * a->G);
  return FDY_OK;
}

int fdy_get_overrides(fdy_archive* a, void* stream, uint32_t g, fdy_override* out, uint64_t cap, uint64_t* n_out) {
  int rc = check_graph(a, g);
  if (!rc) rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  const uint64_t n = a->h_ovr_off[g + 1] - a->h_ovr_off[g];
  return copy_out(a->ovr.as<fdy_override>() + ovr_base(a, g), n, out, cap, n_out);
}

int fdy_get_node_flags(fdy_archive* a, void* stream, uint32_t g, uint8_t* out, uint64_t cap, uint64_t* n_out) {
  int rc = check_graph(a, g);
  if (!rc) rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  return copy_out(a->nflags.as<uint8_t>() + a->graphs[g].node_base, a->graphs[g].num_nodes, out, cap, n_out);
}

int fdy_get_node_words(fdy_archive* a, void* stream, uint32_t g, uint32_t* out, uint64_t cap, uint64_t* n_out) {
  int rc = check_graph(a, g);
  if (!rc) rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  const uint32_t N = a->graphs[g].num_nodes;
  if (n_out) *n_out = N + 1ull;
  if (!out) return FDY_OK;
  if (cap < N + 1ull) return err(FDY_E_CAPACITY, "output array too small for N+1 word offsets");
  std::vector<NodeDesc> d(N);
  if (N) FDY_HIP(hipMemcpy(d.data(), a->ndesc.as<NodeDesc>() + a->graphs[g].node_base, N * sizeof(NodeDesc),
                           hipMemcpyDeviceToHost));
  for (uint32_t i = 0; i < N; ++i) out[i] = d[i].gword;
  out[N] = a->h_gwords[g];
  return FDY_OK;
}

int fdy_get_param_image(fdy_archive* a, void* stream, uint32_t g, uint64_t* out, uint64_t cap, uint64_t* n_out) {
  int rc = check_graph(a, g);
  if (!rc) rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  return copy_out(a->image.as<uint64_t>() + r_base(a, g), a->h_gwords[g], out, cap, n_out);
}

int fdy_get_node_pointers(fdy_archive* a, void* stream, uint32_t g, uint64_t* out, uint64_t cap, uint64_t* n_out) {
  int rc = check_graph(a, g);
  if (!rc) rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  return copy_out(a->nptrs.as<uint64_t>() + 2 * a->graphs[g].node_base, 2ull * a->graphs[g].num_nodes, out, cap,
                  n_out);
}

int fdy_get_section(fdy_archive* a, uint32_t g, uint32_t sec, uint8_t* out, uint64_t cap, uint64_t* n_out) {
  int rc = check_graph(a, g);
  if (rc) return rc;
  if (sec >= FDY_SEC_COUNT) return err(FDY_E_RANGE, "section " + std::to_string(sec) + " out of range");
  FDY_HIP(hipSetDevice(a->device));
  return copy_out(a->img.as<uint8_t>() + a->graphs[g].sec_off[sec], a->graphs[g].sec_size[sec], out, cap, n_out);
}

int fdy_switch(fdy_archive* a, uint32_t g, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = check_graph(a, g);
  if (!rc) rc = ensure_cache(a, s);
  uint32_t t = 0;
  if (!rc) rc = check_switchable(a, g, &t);
  if (rc) return rc;
  if (a->bound.size() == a->G && a->bound[t]) return group_graph_select(a->bound[t], g, s, nullptr);
  return enqueue_switch(a, g, s, nullptr, true);
}

int fdy_switch_sequence(fdy_archive* a, const uint32_t* targets, uint64_t n, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!a) return err(FDY_E_INVALID, "null archive");
  if (n && !targets) return err(FDY_E_INVALID, "null target list");
  int rc = ensure_cache(a, s);
  if (rc) return rc;
  for (uint64_t i = 0; i < n; ++i) {
    uint32_t t = 0;
    rc = check_graph(a, targets[i]);
    if (!rc) rc = check_switchable(a, targets[i], &t);
    if (rc) return rc;
  }
  const bool bound = a->bound.size() == a->G;
  // Every switch's launch size depends on the group's current graph at that
  // point of the sequence: follow the sequence on a copy first, so that a
  // switch too large for one launch refuses the whole sequence before
  // anything is enqueued.
  {
    std::vector<uint32_t> cur = a->h_current;
    for (uint64_t i = 0; i < n; ++i) {
      const uint32_t g = targets[i], t = a->h_tmpl[g];
      if ((bound && a->bound[t]) || cur[t] == g) continue;
      if (switch_blocks(switch_args(a, g, nullptr, cur[t])) >= 0x7FFFFFFFull)
        return err(FDY_E_CAPACITY, "override sets too large for one switch launch (target " +
                                       std::to_string(g) + ")");
      cur[t] = g;
    }
  }
  FDY_HIP(hipSetDevice(a->device));
  // Switches of different groups touch disjoint live images and node
  // sources, so only each group's own switches need their order.  Unless a
  // group graph holds one of the groups involved, the sequence runs in
  // layers: layer k holds every group's k-th switch (no-op switches, to the
  // group's current graph, left out), up to kSwitchBatch per launch, and
  // the layers launch in order.  A group's state after the sequence, and
  // after each of its own switches, is the same as in sequence order; where
  // consecutive switches often hit one group (32 groups, uniform targets:
  // about 7 in a row before a repeat) a launch holds up to kSwitchBatch
  // instead of those 7.
  bool layered = true;
  if (bound)
    for (uint64_t i = 0; i < n && layered; ++i) layered = !a->bound[a->h_tmpl[targets[i]]];
  if (layered) {
    std::vector<uint32_t> cur = a->h_current, depth(a->G, 0);
    std::vector<std::vector<std::pair<uint32_t, uint32_t>>> layers;  // {target, its group's graph before it}
    for (uint64_t i = 0; i < n; ++i) {
      const uint32_t g = targets[i], t = a->h_tmpl[g];
      if (cur[t] == g) continue;
      const uint32_t k = depth[t]++;
      if (k == layers.size()) layers.emplace_back();
      layers[k].push_back({g, cur[t]});
      cur[t] = g;
    }
    // A launch's switches are recorded as their groups' current graphs once
    // it is enqueued.
    SwitchBatch lb{};
    auto launch = [&]() -> int {
      if (lb.n) FDY_HIP(launch_switch_many(lb, s));
      for (uint32_t k = 0; k < lb.n; ++k) a->h_current[lb.sw[k].tmpl] = lb.sw[k].target;
      lb.n = 0;
      return FDY_OK;
    };
    for (const auto& layer : layers) {
      for (const auto& gc : layer) {
        const SwitchArgs w = switch_args(a, gc.first, nullptr, gc.second);
        const uint32_t blocks = (uint32_t)switch_blocks(w);  // below 2^31: checked above
        if (lb.n == kSwitchBatch || (lb.n && lb.end[lb.n - 1] + (uint64_t)blocks >= 0x7FFFFFFFull)) {
          rc = launch();
          if (rc) return rc;
        }
        lb.sw[lb.n] = w;
        lb.end[lb.n] = (lb.n ? lb.end[lb.n - 1] : 0u) + blocks;
        ++lb.n;
      }
      rc = launch();  // the next layer's switches follow this layer's in their groups
      if (rc) return rc;
    }
    return FDY_OK;
  }
  // With a group graph involved: consecutive switches of different groups,
  // up to kSwitchBatch, share one launch.  A switch of a group already in
  // the batch, or of a group whose live image a group graph holds, first
  // launches the batch so far (stream order keeps the sequence's order where
  // it matters).  A group's current graph is recorded once its switch is
  // enqueued.
  SwitchBatch b{};
  uint32_t batch_t[kSwitchBatch], batch_g[kSwitchBatch];
  auto flush = [&]() -> int {
    if (b.n) FDY_HIP(launch_switch_many(b, s));
    for (uint32_t k = 0; k < b.n; ++k) a->h_current[batch_t[k]] = batch_g[k];
    b.n = 0;
    return FDY_OK;
  };
  for (uint64_t i = 0; i < n; ++i) {
    const uint32_t g = targets[i];
    const uint32_t t = a->h_tmpl[g];
    if (bound && a->bound[t]) {
      rc = flush();
      if (!rc) rc = group_graph_select(a->bound[t], g, s, nullptr);
      if (rc) return rc;
      continue;
    }
    if (std::find(batch_t, batch_t + b.n, t) != batch_t + b.n) {
      rc = flush();
      if (rc) return rc;
    }
    if (a->h_current[t] == g) continue;
    if (b.n == kSwitchBatch) {
      rc = flush();
      if (rc) return rc;
    }
    const SwitchArgs w = switch_args(a, g, nullptr);
    const uint32_t blocks = (uint32_t)switch_blocks(w);  // below 2^31: checked above
    if (b.n && b.end[b.n - 1] + (uint64_t)blocks >= 0x7FFFFFFFull) {
      rc = flush();
      if (rc) return rc;
    }
    b.sw[b.n] = w;
    b.end[b.n] = (b.n ? b.end[b.n - 1] : 0u) + blocks;
    batch_t[b.n] = t;
    batch_g[b.n] = g;
    ++b.n;
  }
  return flush();
}

int fdy_get_live(fdy_archive* a, void* stream, uint32_t t, uint64_t* words, uint64_t cap, uint32_t* node_src,
                 uint64_t node_cap, uint32_t* current) {
  int rc = check_graph(a, t);
  if (!rc) rc = ensure_cache(a, static_cast<hipStream_t>(stream));
  if (rc) return rc;
  if (a->h_tmpl[t] != t) return err(FDY_E_INVALID, "graph " + std::to_string(t) + " is not a template");
  FDY_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  rc = copy_out(a->live.as<uint64_t>() + live_base(a, t), a->h_gwords[t], words, cap, nullptr);
  if (!rc) rc = copy_out(a->live_src.as<uint32_t>() + a->graphs[t].node_base, a->graphs[t].num_nodes, node_src,
                         node_cap, nullptr);
  if (rc) return rc;
  if (current) *current = a->h_current[t];
  return FDY_OK;
}

// DLPack's managed tensor (dlpack.h v0.8 layout): a non-owning view whose
// deleter frees only this block.
namespace {
struct DLDevice_ {
  int32_t device_type, device_id;
};
struct DLDataType_ {
  uint8_t code, bits;
  uint16_t lanes;
};
struct DLTensor_ {
  void* data;
  DLDevice_ device;
  int32_t ndim;
  DLDataType_ dtype;
  int64_t* shape;
  int64_t* strides;
  uint64_t byte_offset;
};
struct DLManagedTensor_ {
  DLTensor_ dl_tensor;
  void* manager_ctx;
  void (*deleter)(DLManagedTensor_*);
};
void free_view(DLManagedTensor_* t) { std::free(t); }
}  // namespace

void* fdy_dlpack_view(uint64_t ptr, int32_t device_type, int32_t device_id, int32_t ndim, const int64_t* shape,
                      const int64_t* strides, uint8_t code, uint8_t bits) {
  if (ndim < 0 || ndim > 64 || (ndim && (!shape || !strides))) {
    err(FDY_E_INVALID, "fdy_dlpack_view: bad shape");
    return nullptr;
  }
  const size_t bytes = sizeof(DLManagedTensor_) + 2 * sizeof(int64_t) * (size_t)ndim;
  auto* t = static_cast<DLManagedTensor_*>(std::malloc(bytes));
  if (!t) {
    err(FDY_E_NOMEM, "fdy_dlpack_view: out of host memory");
    return nullptr;
  }
  int64_t* dims = reinterpret_cast<int64_t*>(t + 1);
  for (int32_t i = 0; i < ndim; ++i) {
    dims[i] = shape[i];
    dims[ndim + i] = strides[i];
  }
  t->dl_tensor.data = reinterpret_cast<void*>(ptr);
  t->dl_tensor.device = DLDevice_{device_type, device_id};
  t->dl_tensor.ndim = ndim;
  t->dl_tensor.dtype = DLDataType_{code, bits, 1};
  t->dl_tensor.shape = dims;
  t->dl_tensor.strides = dims + ndim;
  t->dl_tensor.byte_offset = 0;
  t->manager_ctx = nullptr;
  t->deleter = free_view;
  return t;
}

// ---- relocation without device allocation --------------------------------

namespace {

// The interval index of fdy_relocate_words_static.  Each GPU the library
// runs on holds its own copy until the process ends.  In host code the
// array's name is not a device address: it is only ever passed to
// hipGetSymbolAddress, and the address that returns is what kernels,
// copies and fills receive.
static __device__ __align__(256) uint8_t scratch[FDY_STATIC_INDEX_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// The table whose index each device's array holds, so that a call with the
// same table uses it as it stands: no host build, no copy, no wait.
struct StaticTable {
  bool valid = false;
  uint32_t policy = 0;
  std::vector<uint64_t> lo, hi, nlo;
  RelocDev dev{};
};
StaticTable g_static_table[kMaxDevices];

bool same_table(const StaticTable& t, const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo, uint64_t n,
                uint32_t policy) {
  if (!t.valid || t.policy != policy || t.lo.size() != n) return false;
  const size_t b = 8 * n;
  return !n || (!std::memcmp(t.lo.data(), lo, b) && !std::memcmp(t.hi.data(), hi, b) && !std::memcmp(t.nlo.data(), nlo, b));
}

// The device address of `scratch` on device `dev` (current), looked up on
// the first call on that device.
int scratch_on(int dev, uint8_t** out) {
  if (dev < 0 || dev >= kMaxDevices) return err(FDY_E_RANGE, "device " + std::to_string(dev) + " out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return err(FDY_E_HIP, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = static_cast<uint8_t*>(g_scratch[dev]);
  return FDY_OK;
}

}  // namespace

int fdy_relocate_words_static(const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo, uint64_t n_iv,
                              uint32_t policy, const uint64_t* in, uint64_t* out, uint64_t n, void* stream) {
  if ((!in && n) || (!out && n)) return err(FDY_E_INVALID, "null word array");
  if (((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 7) != 0)
    return err(FDY_E_INVALID, "word arrays must be 8-byte aligned");
  if (n_iv && (!lo || !hi || !nlo)) return err(FDY_E_INVALID, "null interval array");
  int dev = 0;
  const hipError_t ge = hipGetDevice(&dev);
  bool same = false;
  if (ge == hipSuccess && dev >= 0 && dev < kMaxDevices) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    same = same_table(g_static_table[dev], lo, hi, nlo, n_iv, policy);
  }
  // A new table: its index is built and checked against the array's size
  // (on the host, so an oversized table is refused with or without a GPU).
  HostIndex x;
  if (!same) {
    int rc = build_reloc_index(lo, hi, nlo, n_iv, policy, &x);
    if (rc) return rc;
    const uint64_t total = x.line.size() * sizeof(RelocLine);
    if (total > FDY_STATIC_INDEX_BYTES)
      return err(FDY_E_CAPACITY, "the index of " + std::to_string(n_iv) + " intervals takes " + std::to_string(total) +
                                     " bytes; the static index holds " + std::to_string(FDY_STATIC_INDEX_BYTES));
  }
  FDY_HIP(ge);
  uint8_t* base = nullptr;
  int rc = scratch_on(dev, &base);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  RelocDev d{};
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    StaticTable& st = g_static_table[dev];
    if (!same_table(st, lo, hi, nlo, n_iv, policy)) {
      if (same) {  // another thread replaced the table meanwhile
        rc = build_reloc_index(lo, hi, nlo, n_iv, policy, &x);
        if (rc) return rc;
        if (x.line.size() * sizeof(RelocLine) > FDY_STATIC_INDEX_BYTES)
          return err(FDY_E_CAPACITY, "the static index cannot hold this table");
      }
      st.valid = false;
      d = x.dev;
      if (n_iv) {
        // In stream order, so after any earlier call's kernel on this
        // stream; then wait for the copy, after which the host index may go.
        FDY_HIP(hipMemcpyAsync(base, x.line.data(), x.line.size() * sizeof(RelocLine), hipMemcpyHostToDevice, s));
        FDY_HIP(hipStreamSynchronize(s));
        d.line = reinterpret_cast<const RelocLine*>(base);
      }
      st.lo.assign(lo, lo + n_iv);
      st.hi.assign(hi, hi + n_iv);
      st.nlo.assign(nlo, nlo + n_iv);
      st.policy = policy;
      st.dev = d;
      st.valid = true;
    }
    d = st.dev;
  }
  FDY_HIP(launch_reloc_words(d, in, out, n, s));
  return FDY_OK;
}

int fdy_reloc_plan_create(const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo, uint64_t n, uint32_t policy,
                          fdy_reloc_plan** out) {
  if (!out) return err(FDY_E_INVALID, "null output");
  auto p = std::make_unique<fdy_reloc_plan>();
  (void)hipGetDevice(&p->device);
  int rc = build_reloc_plan(lo, hi, nlo, n, policy, &p->plan, kPlanRootLinesPerInterval);
  if (rc) return rc;
  *out = p.release();
  return FDY_OK;
}

int fdy_reloc_plan_lines(const fdy_reloc_plan* p, void* lines, uint64_t cap, uint64_t* n_lines) {
  if (!p) return err(FDY_E_INVALID, "null plan");
  const uint64_t n = p->plan.dev.n ? p->plan.line.bytes / sizeof(RelocLine) : 0;
  if (n_lines) *n_lines = n;
  if (!lines) return FDY_OK;
  if (cap < n) return err(FDY_E_CAPACITY, "output holds " + std::to_string(cap) + " lines, the index has " +
                                              std::to_string(n));
  FDY_HIP(hipSetDevice(p->device));
  if (n) FDY_HIP(hipMemcpy(lines, p->plan.line.p, n * sizeof(RelocLine), hipMemcpyDeviceToHost));
  return FDY_OK;
}

int fdy_reloc_plan_destroy(fdy_reloc_plan* p) {
  if (p) {
    (void)hipSetDevice(p->device);
    (void)hipDeviceSynchronize();
  }
  delete p;
  return FDY_OK;
}

int fdy_relocate_words(const fdy_reloc_plan* p, const uint64_t* in, uint64_t* out, uint64_t n, void* stream) {
  if (!p || (!in && n) || (!out && n)) return err(FDY_E_INVALID, "null argument");
  if (((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 7) != 0)
    return err(FDY_E_INVALID, "word arrays must be 8-byte aligned");
  FDY_HIP(launch_reloc_words(p->plan.dev, in, out, n, static_cast<hipStream_t>(stream)));
  return FDY_OK;
}

}  // extern "C"
