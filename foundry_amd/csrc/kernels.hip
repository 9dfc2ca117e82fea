// kernels.hip -- the restore kernels for gfx950 (wave64, 160 KB LDS per CU).
//
//   k_group   per graph: a word hash of its saved key, published with an
//             atomic store; template_of[g] = lowest graph with the same key
//             bytes (by the published hashes, then a byte compare).
//   k_node_a  one workgroup per 256-node chunk of a graph: for a
//             member, a coalesced compare of the chunk's node entries and
//             param entries with its template's; the per-node path (param
//             layout, compare against the template's node, memset/memcpy
//             pointer relocation, node-type and kernel-entry records) for
//             every node that differs or has nothing to compare with.
//   k_node_b  one workgroup per graph: clean nodes completed from the
//             template's results, chunk CRCs joined into the node-type and
//             kernel-entry digests, word offsets by block scans, the
//             diff-tile -> first-node table, ragged-word sources, slot
//             descriptors; beside them, one wave per 4 KB slice of every key
//             and dependency table: their CRC-64/XZ digests.
//   k_diff_t  the template graphs' words, relocated through the line-indexed
//             interval search into R and the live image (1024-word units);
//             the key-digest collision report.
//   k_diff_m  eight workgroups per 4096-word tile of every other graph: coalesced
//             8-byte loads of the graph's and the template's words, the
//             template's relocated word reused where the raw words are equal,
//             the relocated image store, and per-wave ballot compaction of
//             the words left to search or compare into candidate regions.
//   k_diff_s  one wave per tile: the candidates' interval searches, and the
//             differing words as completed override records, written at
//             their place in the graph's dense override array.
//   k_repack  per graph, only when flagged (before results are read): the
//             gaps that compared words equal after relocation leave in a
//             graph's override array closed.
//   k_switch  override scatter for one graph switch.
//   k_mirror  dirty nodes' live words -> a group graph's host mirror.
//   k_fill    memset node of a restored graph, as a kernel node.
//   k_reloc   streaming relocation of packed words.
//   k_index_count, k_index_scan, k_index_place
//             the interval index of a relocation table, one thread per root
//             line (the builder of reloc_index.h).
#include <type_traits>

#include "kernels.h"
#include "reloc_index.h"

namespace fdy {
namespace {

// A graph record read through the constant address space (scalar loads).
typedef __attribute__((address_space(4))) const DevGraph ConstGraph;

// Memory that no workgroup writes during the kernel at hand (the records,
// or what an earlier pass of the restore wrote), read through the constant
// address space: a wave-uniform address becomes a scalar load, which
// neither waits for the vector loads in flight nor is repeated after a
// barrier's fence.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* readonly(const T* p) {
  return (const __attribute__((address_space(4))) T*)p;
}

constexpr uint32_t kNodeThreads = 512;
constexpr uint32_t kRelocThreads = 256;
constexpr uint32_t kRelocPairs = 4;  // 16-byte word pairs per thread per iteration

__device__ inline uint64_t shfl_down64(uint64_t v, int d) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl_down(lo, (unsigned)d, 64);
  hi = __shfl_down(hi, (unsigned)d, 64);
  return ((uint64_t)hi << 32) | lo;
}

__device__ inline uint32_t shfl_up32(uint32_t v, int d) { return __shfl_up(v, (unsigned)d, 64); }
__device__ inline uint64_t shfl_up64(uint64_t v, int d) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl_up(lo, (unsigned)d, 64);
  hi = __shfl_up(hi, (unsigned)d, 64);
  return ((uint64_t)hi << 32) | lo;
}

// Word qi (bytes [8 qi, 8 qi + 8)) of the L-byte stream at p (8-aligned,
// inside the archive-image buffer), with bytes outside [0, L) read as zero.
// The load is unconditional, from the nearest word of the stream (word 0
// of an empty stream: the buffer ends in 4 KB of zero padding, so that load
// stays inside it), so a run of calls issues its loads together instead of
// one branch and wait per word.
__device__ __forceinline__ uint64_t stream_word(const uint8_t* p, uint64_t L, int64_t qi) {
  const int64_t last = L ? (int64_t)((L - 1) >> 3) : 0;
  const int64_t qc = qi < 0 ? 0 : (qi > last ? last : qi);
  uint64_t v = *reinterpret_cast<const uint64_t*>(p + 8 * qc);
  const uint64_t rem = L - 8 * (uint64_t)qc;
  if (rem < 8) v &= (1ull << (8 * rem)) - 1;
  return qi == qc ? v : 0;
}

// The 8 bytes [b0, b0+8) of the L-byte stream at p (8-aligned), with bytes
// outside [0, L) read as zero.
__device__ __forceinline__ uint64_t stream_window(const uint8_t* p, uint64_t L, int64_t b0) {
  const int64_t q = b0 >> 3;
  const uint32_t sh = (uint32_t)(b0 & 7);
  const uint64_t w0 = stream_word(p, L, q), w1 = stream_word(p, L, q + 1);
  return sh ? (w0 >> (8 * sh)) | (w1 << (64 - 8 * sh)) : w0;
}

static_assert(kSliceBytes == 16 * kPosRecords, "a slice is as long as a chunk's records");

// Shift a raw CRC z past k 4 KB units (a chunk's records, or a stream
// slice): lane i holds x^(8 * 4096 * k) * x^i and keeps it where z has x^i
// (bit 63 - i); the caller XORs over the wave.  Past the table, one lane
// multiplies.
__device__ __noinline__ uint64_t far_shift(const CrcConsts* cc, uint64_t z, uint32_t k) {
  return gf2_mulmod(x2n_mod(cc->x2n.v, (uint64_t)kSliceBytes * k, 3), z);
}
__device__ __forceinline__ uint64_t shift_share(const CrcConsts* cc, uint64_t z, uint32_t k, uint32_t lane) {
  if (k < (uint32_t)kChunkShifts) return ((z >> (63 - lane)) & 1) ? cc->chunk_shift[k][lane] : 0ull;
  return lane == 0 ? gf2_mulmod(x2n_mod(cc->x2n.v, (uint64_t)kSliceBytes * k, 3), z) : 0ull;
}

// Per graph, one workgroup: template_of[i] = the lowest j <= i whose saved
// key has the same bytes (the reference partitions graphs by exact key
// string, csrc/CUDAGraphParallel.cpp:1788-1851).
//   - The workgroup hashes its own key (key_term over its words, kHashBatch
//     loads per thread issued together) and publishes the hash with one
//     64-bit atomic store, tagged with the restore's epoch in its low 16
//     bits.  Nothing else is shared, so no fence is needed: only atomics
//     touch the published hashes.
//   - The workgroup then scans the lower graphs' hashes, one per thread per
//     step, with atomic loads; a hash not yet published this restore is
//     waited for a bounded time (RestoreArgs::hash_wait_spins sleeps) and
//     then computed by the wave itself, so no workgroup depends on another's
//     progress.  The lowest j with i's hash and key length is confirmed byte
//     for byte by the workgroup; on a difference scanning goes on past j.
// The restore's first kernel: it also resets the counters later kernels
// accumulate into and starts the key and dependency digests from their
// finishing terms (the node pass's digest units XOR every slice's share in).
constexpr uint32_t kGroupThreads = 512;
constexpr uint32_t kHashBatch = 8;

// A 64-bit hash of a key for finding grouping candidates (not a digest the
// restore reports): the XOR over the key's 8-byte words w_k (the last one
// zero-padded) of the SplitMix64 finaliser (Steele, Lea and Flood 2014) of
// w_k + (k + 1) * golden ratio.  Word terms are independent, so every lane
// hashes its own words; equal keys hash equal, and a hash match is always
// confirmed byte for byte.
__device__ __forceinline__ uint64_t key_term(uint64_t w, uint64_t k) {
  uint64_t z = w + (k + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// This thread's share of the hash of the L-byte key at p (threads
// `first`, `first + stride`, ... take its words).
__device__ __forceinline__ uint64_t key_share(const uint8_t* p, uint64_t L, uint32_t first, uint32_t stride) {
  const uint64_t nw = (L + 7) / 8;
  uint64_t x = 0;
  for (uint64_t k0 = first; k0 < nw; k0 += (uint64_t)kHashBatch * stride) {
    uint64_t w[kHashBatch];
#pragma unroll
    for (uint32_t m = 0; m < kHashBatch; ++m) w[m] = stream_word(p, L, (int64_t)(k0 + (uint64_t)m * stride));
#pragma unroll
    for (uint32_t m = 0; m < kHashBatch; ++m) {
      const uint64_t k = k0 + (uint64_t)m * stride;
      x ^= k < nw ? key_term(w[m], k) : 0ull;
    }
  }
  return x;
}

// The published form of a key hash: its upper 48 bits, and the epoch.
__device__ __forceinline__ uint64_t tag_hash(uint64_t h, uint32_t epoch) { return (h & ~0xFFFFull) | epoch; }

__global__ __launch_bounds__(kGroupThreads) void k_group(RestoreArgs a) {
  __shared__ uint64_t s_x[kGroupThreads / 64];
  __shared__ uint32_t s_found, s_differs;
  const uint32_t i = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (i == 0 && tid == 0) {
    *a.tslot_count = 0;  // the node pass lists template slots here
    *a.restore_flags = 0;  // kFlag* raised by the later passes
  }
  const ConstGraph& Gi = *readonly(a.graphs + i);
  if (tid < 2) a.digests[4ull * i + tid] = Gi.crc_fin[tid];
  // The node pass reads {graph, template} per node chunk.
  const uint32_t nch = Gi.num_nodes ? (Gi.num_nodes + kNodeChunk - 1) / kNodeChunk : 1;
  if (a.explicit_template) {
    const uint32_t t = a.explicit_template[i];
    if (tid == 0) a.template_of[i] = t;
    for (uint32_t c = tid; c < nch; c += kGroupThreads) a.chunk_gt[Gi.chunk_base + c] = make_uint2(i, t);
    return;
  }
  const uint64_t L = Gi.sec_size[FDY_SEC_TOPOLOGY_KEY];
  const uint8_t* pi = a.img + Gi.sec_off[FDY_SEC_TOPOLOGY_KEY];
  uint64_t x = key_share(pi, L, tid, kGroupThreads);
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) x ^= shfl_down64(x, d);
  if (lane == 0) s_x[wave] = x;
  __syncthreads();
  for (uint32_t w = 0; w < kGroupThreads / 64; ++w)
    if (w != wave) x ^= s_x[w];  // lane 0 of every wave holds the whole hash
  const uint64_t hi = tag_hash(x, a.epoch);
  if (tid == 0) __hip_atomic_store(a.key_hash + i, hi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  uint32_t from = 0, tmpl = i;
  const uint64_t hiw = ((uint64_t)__shfl((uint32_t)(hi >> 32), 0, 64) << 32) | __shfl((uint32_t)hi, 0, 64);
  for (;;) {
    // Every thread takes one lower graph per step (kGroupThreads per step);
    // the lowest match wins.
    if (tid == 0) {
      s_found = i;
      s_differs = 0;
    }
    __syncthreads();
    uint32_t found = i;
    for (uint32_t base = from; base < i; base += kGroupThreads) {
      const uint32_t j = base + tid;
      const bool in = j < i;
      uint64_t hj = in ? __hip_atomic_load(a.key_hash + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
      const uint64_t Lj = in ? a.graphs[j].sec_size[FDY_SEC_TOPOLOGY_KEY] : ~0ull;
      // Hashes of this restore carry its epoch; wait (bounded) for the rest.
      for (uint32_t spin = 0; __ballot(in && (hj & 0xFFFF) != a.epoch) && spin < a.hash_wait_spins; ++spin) {
        __builtin_amdgcn_s_sleep(2);
        if (in && (hj & 0xFFFF) != a.epoch)
          hj = __hip_atomic_load(a.key_hash + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      // Still missing: the wave hashes those keys itself, one at a time.
      uint64_t miss = __ballot(in && (hj & 0xFFFF) != a.epoch);
      while (miss) {
        const uint32_t l = (uint32_t)__ffsll((long long)miss) - 1;
        miss &= miss - 1;
        const ConstGraph& Gj = *readonly(a.graphs + base + (tid & ~63u) + l);
        uint64_t y = key_share(a.img + Gj.sec_off[FDY_SEC_TOPOLOGY_KEY], Gj.sec_size[FDY_SEC_TOPOLOGY_KEY], lane, 64);
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) y ^= shfl_down64(y, d);
        const uint64_t yl = ((uint64_t)__shfl((uint32_t)(y >> 32), 0, 64) << 32) | __shfl((uint32_t)y, 0, 64);
        if (lane == l) hj = tag_hash(yl, a.epoch);
      }
      const bool m = in && (hj >> 16) == (hiw >> 16) && Lj == L;
      const uint64_t mk = __ballot(m);
      if (mk && lane == 0) atomicMin(&s_found, base + (tid & ~63u) + (uint32_t)__ffsll((long long)mk) - 1);
      __syncthreads();
      found = s_found;
      // Every wave holds this step's minimum before any wave of the next
      // step can lower s_found again.
      __syncthreads();
      if (found != i) break;  // uniform over the workgroup
    }
    const uint32_t j = found;
    if (j == i) break;  // uniform over the workgroup
    const uint8_t* pj = a.img + a.graphs[j].sec_off[FDY_SEC_TOPOLOGY_KEY];
    // Both keys start 8-byte aligned: compare whole words, kHashBatch per
    // side per thread in flight.
    bool d = false;
    const uint64_t nw = (L + 7) / 8;
    for (uint64_t q0 = tid; q0 < nw; q0 += kHashBatch * kGroupThreads) {
      uint64_t vi[kHashBatch], vj[kHashBatch];
#pragma unroll
      for (uint32_t m = 0; m < kHashBatch; ++m) {
        vi[m] = stream_word(pi, L, (int64_t)(q0 + m * kGroupThreads));
        vj[m] = stream_word(pj, L, (int64_t)(q0 + m * kGroupThreads));
      }
#pragma unroll
      for (uint32_t m = 0; m < kHashBatch; ++m) d |= vi[m] != vj[m];
    }
    if (d) s_differs = 1;
    __syncthreads();
    if (!s_differs) {
      tmpl = j;
      break;
    }
    from = j + 1;
    __syncthreads();  // every thread has read s_found and s_differs
  }
  if (tid == 0) a.template_of[i] = tmpl;
  for (uint32_t c = tid; c < nch; c += kGroupThreads) a.chunk_gt[Gi.chunk_base + c] = make_uint2(i, tmpl);
}

// ---- node pass ----------------------------------------------------------

// A kernel node's params: layout, bounds and sizes.
struct Side {
  uint32_t words;
  uint32_t num_params;
  uint32_t arg_size;
  bool bad, extra, ragged;
  uint64_t src;        // absolute byte offset of the blob
  uint64_t pbytes;     // param bytes (0 when bad)
  const uint8_t* pidx; // param entries (per-param style)
};

// A node entry's fields (byte offsets, multiples of 4), read in place (the
// image in global memory; every field of an entry is 4-byte aligned).
struct RawEntry {
  const uint8_t* e;
  __device__ explicit RawEntry(const uint8_t* p) : e(p) {}
  __device__ uint32_t u32(uint32_t off) const { return f32(e, off); }
  __device__ uint64_t u64(uint32_t off) const { return f64(e, off); }
  __device__ uint8_t type() const { return e[FDY_NODE_OFF_TYPE]; }
};

// A node entry whose type and kernel fields (bytes 4-7, 36-51, 64-91 and
// 128-143: type, binary hash, name, required and per-node cluster dims, KNA
// flags, param and arg-buffer references) are loaded together up front, so
// that the per-node path waits for them once, where reading each field at
// its first use (behind the branches on the type and flags) waited once per
// group of fields.  Other fields are read in place.
struct PreEntry {
  const uint8_t* e;
  uint32_t w1, k36[4], k64[7], k128[4];
  __device__ explicit PreEntry(const uint8_t* p) : e(p) {
    w1 = f32(p, 4);
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) k36[i] = f32(p, 36 + 4 * i);
#pragma unroll
    for (uint32_t i = 0; i < 7; ++i) k64[i] = f32(p, 64 + 4 * i);
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) k128[i] = f32(p, 128 + 4 * i);
  }
  // Offsets are compile-time constants at every use, so the selection folds away.
  __device__ uint32_t u32(uint32_t off) const {
    if (off == 4) return w1;
    if (off >= 36 && off < 52) return k36[(off - 36) / 4];
    if (off >= 64 && off < 92) return k64[(off - 64) / 4];
    if (off >= 128 && off < 144) return k128[(off - 128) / 4];
    return f32(e, off);
  }
  __device__ uint64_t u64(uint32_t off) const { return (uint64_t)u32(off) | ((uint64_t)u32(off + 4) << 32); }
  __device__ uint8_t type() const { return (uint8_t)w1; }
};
static_assert(FDY_NODE_OFF_TYPE == 4, "the type is the low byte of entry bytes 4-7");

// The param references of kernel node entry e: the name, param-index and
// arg-buffer bounds; an extra-style node's blob.  Per-param nodes are
// completed by scan_params.
template <class E, class GR>
__device__ __forceinline__ void side_header(const uint8_t* img, const GR& G, const E& e, Side& s) {
  s = Side{};
  const uint32_t pio = e.u32(FDY_KOFF_PARAM_INDEX), np = e.u32(FDY_KOFF_NUM_PARAMS);
  const uint32_t ao = e.u32(FDY_KOFF_ARG_OFFSET), as = e.u32(FDY_KOFF_ARG_SIZE);
  const uint32_t no = e.u32(FDY_KOFF_NAME_OFFSET), nl = e.u32(FDY_KOFF_NAME_LENGTH);
  s.bad = (uint64_t)no + nl > G.sec_size[FDY_SEC_STRINGS] ||
          (uint64_t)pio + 8ull * np > G.sec_size[FDY_SEC_PARAM_INDEX];
  s.extra = ao != FDY_NO_ARG_BUFFER;
  s.num_params = np;
  s.arg_size = as;
  s.pidx = img + G.sec_off[FDY_SEC_PARAM_INDEX] + pio;
  if (!s.bad && s.extra) {
    s.bad = (uint64_t)ao + as > G.sec_size[FDY_SEC_ARG_DATA];
    s.words = (as + 7) / 8;
    s.src = G.sec_off[FDY_SEC_ARG_DATA] + ao;
    s.ragged = (ao & 7) || (as & 7);
    s.pbytes = as;
  }
  if (s.bad) {
    s.words = 0;
    s.ragged = false;
    s.pbytes = 0;
  }
}

// Param entry j ({u32 offset, u32 size}) into a side's running totals.
template <class GR>
__device__ inline void side_param(const GR& G, Side& s, uint32_t j, uint64_t entry, uint64_t& prev,
                                  uint64_t& words) {
  const uint32_t o = (uint32_t)entry, sz = (uint32_t)(entry >> 32);
  if ((uint64_t)o + sz > G.sec_size[FDY_SEC_PARAM_DATA]) {
    s.bad = true;
    return;
  }
  if (j == 0) {
    s.src = G.sec_off[FDY_SEC_PARAM_DATA] + o;
    prev = o;
  }
  if ((sz & 7) || (o & 7) || o != prev) s.ragged = true;
  prev = (uint64_t)o + sz;
  words += (sz + 7) / 8;
  s.pbytes += sz;
}

// The per-param entries of a kernel node (with_g) and of its template's node
// (with_t), walked together in batches of kParamBatch entries per side whose
// loads are all issued before any is used.  *same_sizes: equal param counts
// and sizes.
constexpr uint32_t kParamBatch = 8;

template <class GA, class GB>
__device__ __forceinline__ void scan_params(const uint8_t* img, const GA& Gg, Side& g, bool with_g,
                                            const GB& Gt, Side& t, bool with_t, bool* same_sizes) {
  const bool wg = with_g && !g.bad && !g.extra;
  const bool wt = with_t && !t.bad && !t.extra;
  const uint32_t ng = wg ? g.num_params : 0, nt = wt ? t.num_params : 0;
  uint64_t prev_g = 0, prev_t = 0, words_g = 0, words_t = 0;
  bool same = ng == nt;
  // A side's entries may sit at any alignment.  The loads are unconditional
  // (past a side's count, its entry 0, or the image start for a side with
  // none), so a batch's loads issue together instead of one branch and
  // wait per entry.
  const uint8_t* bg = ng ? g.pidx : img;
  const uint8_t* bt = nt ? t.pidx : img;
  // Entries 8-byte aligned in every lane (the usual case): one load each.
  const bool aligned = __all(((reinterpret_cast<uintptr_t>(bg) | reinterpret_cast<uintptr_t>(bt)) & 7) == 0);
  for (uint32_t jb = 0; jb < max(ng, nt); jb += kParamBatch) {
    uint64_t eg[kParamBatch], et[kParamBatch];
    if (aligned) {
#pragma unroll
      for (uint32_t k = 0; k < kParamBatch; ++k) {
        const uint32_t j = jb + k;
        eg[k] = *reinterpret_cast<const uint64_t*>(bg + 8ull * (j < ng ? j : 0));
        et[k] = *reinterpret_cast<const uint64_t*>(bt + 8ull * (j < nt ? j : 0));
      }
    } else {
#pragma unroll
      for (uint32_t k = 0; k < kParamBatch; ++k) {
        const uint32_t j = jb + k;
        eg[k] = ld_u64_any(bg + 8ull * (j < ng ? j : 0));
        et[k] = ld_u64_any(bt + 8ull * (j < nt ? j : 0));
      }
    }
#pragma unroll
    for (uint32_t k = 0; k < kParamBatch; ++k) {
      const uint32_t j = jb + k;
      if (j < ng && !g.bad) side_param(Gg, g, j, eg[k], prev_g, words_g);
      if (j < nt && !t.bad) side_param(Gt, t, j, et[k], prev_t, words_t);
      if (j < ng && j < nt) same &= (eg[k] >> 32) == (et[k] >> 32);
    }
  }
  auto finish = [](Side& s, bool walked, uint64_t words) {
    if (walked) s.words = words > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)words;
    if (s.bad) {
      s.words = 0;
      s.ragged = false;
      s.pbytes = 0;
    }
  };
  if (with_g) finish(g, wg, words_g);
  if (with_t) finish(t, wt, words_t);
  *same_sizes = same;
}

__device__ __forceinline__ bool same_layout(const Side& a, const Side& b, bool same_sizes) {
  if (a.bad || b.bad || a.extra != b.extra) return false;
  if (a.extra) return a.arg_size == b.arg_size;
  return same_sizes;
}

// Effective launch attributes (csrc/CUDAGraphParallel.cpp:1211-1389): common
// attrs, then per-node attrs when any are present, then required cluster dims.
struct Attrs {
  int32_t has_cluster, cx, cy, cz, has_pref, px, py, pz, sched, coop, prio, msd, has_map, map_def, map_remote,
      has_carve, carve;
};

template <class E>
__device__ inline void attrs_from(const E& b, uint32_t base, Attrs& a, bool merge) {
  const uint32_t f = b.u32(base);
  if (f & FDY_KNA_CLUSTER_DIM) {
    a.has_cluster = 1;
    a.cx = (int32_t)b.u32(base + 4);
    a.cy = (int32_t)b.u32(base + 8);
    a.cz = (int32_t)b.u32(base + 12);
  }
  if (f & FDY_KNA_PREFERRED_CLUSTER_DIM) {
    a.has_pref = 1;
    a.px = (int32_t)b.u32(base + 16);
    a.py = (int32_t)b.u32(base + 20);
    a.pz = (int32_t)b.u32(base + 24);
  }
  // When merging per-node attrs over common ones, a negative value does not override.
  auto take = [&](uint32_t flag, uint32_t off, int32_t& dst) {
    if (!(f & flag)) return;
    int32_t v = (int32_t)b.u32(base + off);
    if (!merge || v >= 0) dst = v;
  };
  take(FDY_KNA_CLUSTER_SCHEDULING, 28, a.sched);
  take(FDY_KNA_COOPERATIVE, 32, a.coop);
  take(FDY_KNA_PRIORITY, 36, a.prio);
  take(FDY_KNA_MEM_SYNC_DOMAIN, 40, a.msd);
  if (f & FDY_KNA_MEM_SYNC_DOMAIN_MAP) {
    a.has_map = 1;
    a.map_def = b.u32(base + 44) & 0xFF;
    a.map_remote = (b.u32(base + 44) >> 8) & 0xFF;
  }
  if (f & FDY_KNA_SHARED_MEM_CARVEOUT) {
    a.has_carve = 1;
    a.carve = (int32_t)b.u32(base + 48);
  }
}

// `common`: the graph's common kernel attrs, or null.
template <class E>
__device__ __forceinline__ Attrs effective_attrs(const uint8_t* common, const E& e) {
  Attrs a{0, 0, 0, 0, 0, 0, 0, 0, -1, -1, -1, -1, 0, 0, 0, 0, 0};
  if (common) attrs_from(RawEntry{common}, 0, a, false);
  if (e.u32(FDY_KOFF_KNA_FLAGS) != 0) attrs_from(e, FDY_KOFF_KNA_FLAGS, a, true);
  const int32_t w = (int32_t)e.u32(64), h = (int32_t)e.u32(68), d = (int32_t)e.u32(72);
  if (w > 0 || h > 0 || d > 0) {
    a.has_cluster = 1;
    a.cx = w > 0 ? w : 1;
    a.cy = h > 0 ? h : 1;
    a.cz = d > 0 ? d : 1;
  }
  return a;
}

__device__ __forceinline__ bool attrs_equal(const Attrs& a, const Attrs& b) {
  const int32_t* x = &a.has_cluster;
  const int32_t* y = &b.has_cluster;
  bool eq = true;
  for (int i = 0; i < 17; ++i) eq &= x[i] == y[i];
  return eq;
}

// A graph's string section (8-byte aligned start), in LDS or in the image.
struct Strings {
  const uint8_t* p;
  uint64_t size;
};

// Equal kernel names, compared through 8-byte windows.
template <class EA, class EB>
__device__ __forceinline__ bool names_equal(const Strings& A, const EA& ea, const Strings& B, const EB& eb) {
  const uint32_t ao = ea.u32(FDY_KOFF_NAME_OFFSET), al = ea.u32(FDY_KOFF_NAME_LENGTH);
  const uint32_t bo = eb.u32(FDY_KOFF_NAME_OFFSET), bl = eb.u32(FDY_KOFF_NAME_LENGTH);
  if (al != bl) return false;
  if ((uint64_t)ao + al > A.size || (uint64_t)bo + bl > B.size) return false;
  bool eq = true;
  for (uint32_t i = 0; i < al && eq; i += 8) {
    const uint32_t n = min(8u, al - i);
    const uint64_t m = n == 8 ? ~0ull : (1ull << (8 * n)) - 1;
    eq = ((stream_window(A.p, A.size, (int64_t)ao + i) ^ stream_window(B.p, B.size, (int64_t)bo + i)) & m) == 0;
  }
  return eq;
}

// CRC-64/XZ of a kernel's name.
template <class E>
__device__ __forceinline__ uint64_t name_crc(const Strings& S, const E& e, const uint64_t (*slice)[256]) {
  const uint32_t no = e.u32(FDY_KOFF_NAME_OFFSET), nl = e.u32(FDY_KOFF_NAME_LENGTH);
  if ((uint64_t)no + nl > S.size) return 0;
  uint64_t c = ~0ull;
  uint32_t i = 0;
  for (; i + 8 <= nl; i += 8) c = crc_slice8(slice, c, stream_window(S.p, S.size, (int64_t)no + i));
  if (i < nl) {
    uint64_t tail = stream_window(S.p, S.size, (int64_t)no + i);
    for (; i < nl; ++i, tail >>= 8) c = crc_byte(slice[0], c, (uint8_t)tail);
  }
  return ~c;
}

// Relocated memset dst / memcpy dst, src of node entry e (0 when not a pointer node).
template <class E>
__device__ __forceinline__ void node_pointers(const E& e, const RelocDev& r, uint64_t* p0, uint64_t* p1) {
  const uint8_t type = e.type();
  *p0 = 0;
  *p1 = 0;
  if (type == FDY_NODE_MEMSET) {
    *p0 = reloc_word(r, e.u64(FDY_MSOFF_DST));
  } else if (type == FDY_NODE_MEMCPY) {
    const uint64_t dst = e.u64(FDY_MCOFF_DST), src = e.u64(FDY_MCOFF_SRC);
    const int32_t dt = (int32_t)e.u32(FDY_MCOFF_DST_MEMTYPE), st = (int32_t)e.u32(FDY_MCOFF_SRC_MEMTYPE);
    *p0 = (dt == FDY_MEMTYPE_DEVICE || dt == FDY_MEMTYPE_UNIFIED) ? reloc_word(r, dst) : dst;
    *p1 = (st == FDY_MEMTYPE_DEVICE || st == FDY_MEMTYPE_UNIFIED) ? reloc_word(r, src) : src;
  }
}

template <class EA, class EB>
__device__ __forceinline__ bool u64_range_differs(const EA& a, const EB& b, uint32_t off, uint32_t n) {
  bool d = false;
  for (uint32_t i = 0; i < n; i += 8) d |= a.u64(off + i) != b.u64(off + i);
  return d;
}

// Does node entry ea (strings A, common attrs ca) differ in its descriptor
// from eb (strings B, common attrs cb)?  pa/pb: relocated pointers.
// same_ctx: both graphs have byte-identical string sections and common
// attrs, so equal entry bytes [8, 128) (launch config, function hash, name
// offset and length, function attrs, per-node attrs) mean equal descriptors.
template <class EA, class EB>
__device__ __forceinline__ bool desc_differs(const Strings& A, const uint8_t* ca, const EA& ea, const Strings& B,
                                             const uint8_t* cb, const EB& eb, uint64_t pa0, uint64_t pa1,
                                             uint64_t pb0, uint64_t pb1, bool same_ctx) {
  const uint8_t ta = ea.type(), tb = eb.type();
  if (ta != tb) return true;
  switch (ta) {
    case FDY_NODE_KERNEL: {
      if (same_ctx && !u64_range_differs(ea, eb, 8, 120)) return false;
      bool d = false;
      for (uint32_t off = 8; off < 44; off += 4) d |= ea.u32(off) != eb.u32(off);
      for (uint32_t off = 52; off < 76; off += 4) d |= ea.u32(off) != eb.u32(off);
      if (d) return true;
      if (!names_equal(A, ea, B, eb)) return true;
      return !attrs_equal(effective_attrs(ca, ea), effective_attrs(cb, eb));
    }
    case FDY_NODE_MEMSET:
      return pa0 != pb0 || ea.u32(16) != eb.u32(16) || u64_range_differs(ea, eb, 24, 16) ||
             ea.u32(40) != eb.u32(40) || ea.u64(48) != eb.u64(48);
    case FDY_NODE_MEMCPY:
      return pa0 != pb0 || pa1 != pb1 || u64_range_differs(ea, eb, 8, 24) || u64_range_differs(ea, eb, 40, 48) ||
             ea.u32(88) != eb.u32(88) || u64_range_differs(ea, eb, 104, 48) ||
             ea.u32(152) != eb.u32(152);
    case FDY_NODE_EVENT_RECORD:
    case FDY_NODE_EVENT_WAIT:
      return ea.u32(FDY_EVOFF_ID) != eb.u32(FDY_EVOFF_ID);
    default:
      return false;
  }
}

// A workgroup barrier ordering LDS accesses only: unlike __syncthreads it
// does not first wait for the workgroup's outstanding global stores, which
// no thread of the workgroup reads back.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Exclusive block-wide prefix sums of two u32 values per thread (over
// blockDim.x <= 1024 threads); tot[0..1] get the sums.  The workgroup's two
// barriers order its LDS only.
__device__ void block_excl_scan2(const uint32_t v[2], uint32_t (*s_tmp)[16], uint32_t out[2], uint32_t tot[2]) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x[2] = {v[0], v[1]};
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t y = shfl_up32(x[k], d);
      if (lane >= (uint32_t)d) x[k] += y;
    }
  }
  if (lane == 63) {
    s_tmp[0][wave] = x[0];
    s_tmp[1][wave] = x[1];
  }
  lds_barrier();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    uint32_t before = 0, sum = 0;
    for (uint32_t w = 0; w < blockDim.x / 64; ++w) {
      const uint32_t t = s_tmp[k][w];
      if (w < wave) before += t;
      sum += t;
    }
    out[k] = before + x[k] - v[k];
    tot[k] = sum;
  }
  lds_barrier();
}

template <class GR>
__device__ void write_aux(const uint8_t* img, const GR& G, const uint8_t* e, const Side& s, uint64_t* aux,
                          uint32_t gword) {
  uint32_t idx = 0;
  auto put = [&](uint64_t byte, uint32_t size) {
    for (uint32_t m = 0; m < size; m += 8, ++idx) {
      if ((uint64_t)gword + idx >= G.word_cap) return;
      const uint32_t width = min(8u, size - m);
      aux[G.word_base + gword + idx] = ((byte + m) << 4) | width;
    }
  };
  if (s.extra) {
    put(s.src, s.arg_size);
  } else {
    for (uint32_t j = 0; j < s.num_params; ++j)
      put(G.sec_off[FDY_SEC_PARAM_DATA] + ld_u32(s.pidx + 8ull * j), ld_u32(s.pidx + 8ull * j + 4));
  }
  (void)img;
  (void)e;
}

// The node pass runs in two parts.
//
// Part A, k_node_a: one workgroup of kNodeChunk threads per chunk of a
// graph's nodes (a graph's chunks end at its last node, so its first chunk
// is padded at the front; a graph without nodes has one empty chunk).
//   - A member whose node count, section sizes and common attrs match its
//     template's compares the chunk's node entries with the template's
//     (8-byte words, coalesced) and the union of its clean kernel nodes'
//     param entries likewise.  Nodes whose bytes all agree are "clean":
//     every output of theirs equals the template node's (the string
//     sections and common attrs being identical), so part B copies them.
//     The chunk's records are then the XOR of the graph's and the
//     template's (zero at clean nodes; CRCs are linear, so part B adds the
//     template chunk's CRC).
//   - Every other node (all of a template's, and those that differ) takes
//     the per-node path, compacted into the first lanes: type, params and
//     their bounds, layout and descriptor against the template's node,
//     relocated memset/memcpy pointers, the node-type and kernel-entry
//     records.
// Part B, k_node_b: one workgroup per graph: clean nodes completed from the
// template's results, the chunk CRCs shifted to their place, word offsets
// by block scans, the tile -> first-node table, ragged-word sources,
// flatness, status, digests and the slot descriptors of the diff pass.

constexpr uint32_t kEntryWords = 168 / 8;  // 8-byte words of a node entry
constexpr uint32_t kStrStage = 2048;       // string sections up to this size are staged in LDS
constexpr uint32_t kChunkCtxDiff = 1, kChunkPidxDiff = 2;

__device__ __forceinline__ uint32_t node_chunks(uint32_t N) { return max(1u, (N + kNodeChunk - 1) / kNodeChunk); }

// The node-type record (type, then the key's cluster dims for a kernel
// node, csrc/CUDAGraphParallel.cpp:1807-1833) and the kernel-entry record
// (binary hash, CRC-64/XZ of the name) of node entry e.
template <class E>
__device__ __forceinline__ void node_records(const E& e, const uint8_t* common, const Strings& str,
                                             const uint64_t (*slice)[256], uint64_t r[4]) {
  const uint8_t type = e.type();
  r[0] = type;
  r[1] = r[2] = r[3] = 0;
  if (type != FDY_NODE_KERNEL) return;
  uint32_t cx = 0, cy = 0, cz = 0;
  if (e.u32(FDY_KOFF_KNA_FLAGS) & FDY_KNA_CLUSTER_DIM) {
    cx = e.u32(80);
    cy = e.u32(84);
    cz = e.u32(88);
  }
  if (cx == 0 && common && (f32(common, 0) & FDY_KNA_CLUSTER_DIM)) {
    cx = f32(common, 4);
    cy = f32(common, 8);
    cz = f32(common, 12);
  }
  if (cx == 0) {
    cx = e.u32(64);
    cy = e.u32(68);
    cz = e.u32(72);
  }
  r[0] |= (uint64_t)cx << 32;
  r[1] = cy | ((uint64_t)cz << 32);
  r[2] = e.u64(FDY_KOFF_BINARY_HASH);
  r[3] = name_crc(str, e, slice);
}

// The per-node path for node n of graph g (template t, is_t when g is its
// own template): everything the node pass reports for the node.
struct NodeOut {
  NodeDesc d;
  uint64_t p0, p1;
  uint64_t pbytes;
  uint64_t rec[4];  // node-type record (2 words), kernel-entry record (2 words)
};

// A template's nodes (is_t) read their entry's kernel fields up front: no
// template side to compare with leaves registers free for them.
template <bool is_t, class GR>
__device__ __forceinline__ void node_full(const RestoreArgs& a, const GR& Gg, const GR& Gt, uint32_t n,
                                          const Strings& sg_str, const Strings& st_str, const uint8_t* common_g,
                                          const uint8_t* common_t, bool same_ctx, bool xor_t,
                                          const uint64_t (*slice)[256], NodeOut& o) {
  const uint8_t* img = a.img;
  const uint32_t NT = Gt.num_nodes;
  using Entry = typename std::conditional<is_t, PreEntry, RawEntry>::type;
  const Entry eg(img + Gg.sec_off[FDY_SEC_NODES] + 168ull * n);
  const bool has_t = !is_t && n < NT;
  const RawEntry et{img + Gt.sec_off[FDY_SEC_NODES] + 168ull * (has_t ? n : 0)};
  uint32_t words_g = 0, words_t = 0, flags = 0;
  uint64_t src_g = 0, src_t = 0, pbytes = 0;
  const uint8_t type = eg.type();
  const uint8_t ttype = has_t ? et.type() : 0xFF;
  node_records(eg, common_g, sg_str, slice, o.rec);
  Side sg{}, st{};
  bool same_sizes = false;
  if (type == FDY_NODE_KERNEL) side_header(img, Gg, eg, sg);
  const bool t_kernel = has_t && ttype == FDY_NODE_KERNEL;
  if (t_kernel) side_header(img, Gt, et, st);
  scan_params(img, Gg, sg, type == FDY_NODE_KERNEL, Gt, st, t_kernel, &same_sizes);
  if (type == FDY_NODE_KERNEL) {
    words_g = sg.words;
    pbytes = sg.pbytes;
    src_g = sg.src;
    if (sg.ragged) flags |= FDY_NODE_RAGGED;
    if (sg.bad) flags |= kNodeBad;
    if (sg.extra) flags |= kNodeExtra;
  }
  // A template's node reads its type from the prefetched fields; a member's
  // reads the entry in place (the fields need not stay live this long).
  if (is_t) node_pointers(eg, a.reloc, &o.p0, &o.p1);
  else node_pointers(RawEntry{eg.e}, a.reloc, &o.p0, &o.p1);
  if (is_t) {
    flags |= FDY_NODE_TEMPLATE;
  } else if (has_t) {
    uint64_t q0, q1;
    node_pointers(et, a.reloc, &q0, &q1);
    bool layout = ttype != type;
    if (t_kernel) {
      words_t = st.words;
      src_t = st.src;
      if (st.ragged) flags |= kNodeRaggedT;
      if (type == FDY_NODE_KERNEL) layout = !same_layout(sg, st, same_sizes);
    }
    if (layout) flags |= FDY_NODE_LAYOUT;
    else if (words_g) flags |= kNodeCompare;
    // Read in place: the prefetched fields need not stay live this long.
    if (desc_differs(sg_str, common_g, RawEntry{eg.e}, st_str, common_t, et, o.p0, o.p1, q0, q1, same_ctx))
      flags |= FDY_NODE_DESC;
    if (xor_t) {
      uint64_t rt[4];
      node_records(et, common_t, st_str, slice, rt);
#pragma unroll
      for (int k = 0; k < 4; ++k) o.rec[k] ^= rt[k];
    }
  } else {
    flags |= FDY_NODE_LAYOUT | FDY_NODE_DESC;
  }
  o.d.gword = 0;        // word offsets are filled in by k_node_b
  o.d.nwords = words_g;
  o.d.tword = words_t;  // the template node's word count until then
  o.d.flags = flags;
  o.d.src_g = src_g;
  o.d.src_t = src_t;
  o.pbytes = pbytes;
}

// Two consecutive 8-byte words as one 16-byte access at 8-byte alignment
// (gfx950 serves a 16-byte global access at any 4-byte alignment).
typedef uint64_t u64x2a8 __attribute__((ext_vector_type(2), aligned(8)));

// Write-once results that no pass of the restore reads back soon (the
// member graphs' relocated images, candidates, override records) are stored
// nontemporally, and streams read once (the member graphs' words) loaded
// so: otherwise they evict from the L2s and the 256 MB MALL the node tables,
// template words and interval lines that the passes read again (measured on
// the decode-style archive: restore 165 -> 158 us; MoE-style 1163 -> 1095 us).
// (Overloads rather than a template: a template parameter would drop the
// pair type's 8-byte alignment.)
__device__ __forceinline__ void st_stream(uint64_t* p, uint64_t v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void st_stream(u64x2a8* p, u64x2a8 v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ uint64_t ld_stream(const uint64_t* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ u64x2a8 ld_stream(const u64x2a8* p) { return __builtin_nontemporal_load(p); }

// The CRC slice tables (16 KB) into LDS by a workgroup of kNodeChunk
// threads: eight loads per thread, all issued before any store.
__device__ __forceinline__ void stage_slice(uint64_t (*dst)[256], const uint64_t (*src)[256]) {
  static_assert(8 * 256 == 8 * kNodeChunk, "eight words per thread");
  uint64_t v[8];
#pragma unroll
  for (uint32_t k = 0; k < 8; ++k) v[k] = src[k][threadIdx.x];
#pragma unroll
  for (uint32_t k = 0; k < 8; ++k) dst[k][threadIdx.x] = v[k];
}

// Five waves per SIMD (registers held to 96 for that; LDS under 32 KB).
__global__ __launch_bounds__(kNodeChunk, 5) void k_node_a(RestoreArgs a) {
  static_assert(kNodeChunk == kPosRecords, "one position multiplier per record of a chunk");
  __shared__ uint64_t s_slice[8][256];
  __shared__ uint64_t s_str[2][kStrStage / 8];
  __shared__ uint64_t s_common[2][7];
  // The chunk's node-type and kernel-entry records, eight to a row; the odd
  // row length keeps a half-wave's reads of eight rows apart in the banks.
  // Before the records, the same rows hold each node's param-index offset
  // and count for the param-entry check.
  __shared__ uint64_t s_rec[2][kNodeChunk / 8][17];
  static_assert(sizeof(s_rec) >= 2 * kNodeChunk * sizeof(uint32_t), "param-entry fields fit the record rows");
  uint32_t* const s_pio = reinterpret_cast<uint32_t*>(&s_rec[0][0][0]);
  uint32_t* const s_np = s_pio + kNodeChunk;
  __shared__ uint8_t s_type[kNodeChunk], s_perparam[kNodeChunk], s_dirty[kNodeChunk], s_launch[kNodeChunk];
  __shared__ uint16_t s_list[kNodeChunk];
  __shared__ uint32_t s_wave_n[kNodeChunk / 64];
  __shared__ uint64_t s_pb[kNodeChunk / 64];
  __shared__ uint32_t s_flags, s_status, s_pmin, s_pmax, s_umin;

  const uint32_t chunk = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // {graph, template}: the grouping pass filled in the template.
  const auto* gt = readonly(reinterpret_cast<const uint32_t*>(a.chunk_gt + chunk));
  const uint32_t g = gt[0], t = gt[1];
  const bool is_t = t == g;
  // A template's chunk takes the per-node path for all of its nodes, the
  // longest chain of the pass: its waves issue first wherever they share a
  // SIMD with member chunks (decode-style node pass 42.0 -> 39.5 us).
  if (is_t) __builtin_amdgcn_s_setprio(3);
  // The records through the constant address space: nothing writes them
  // during the restore, so their fields are scalar loads, which neither
  // wait for the vector loads in flight nor are repeated after a barrier's
  // fence.
  const ConstGraph& Gg = *readonly(a.graphs + g);
  const ConstGraph& Gt = *readonly(a.graphs + t);
  const uint32_t N = Gg.num_nodes;
  const uint32_t c = chunk - Gg.chunk_base;
  const uint8_t* img = a.img;
  const bool common_g_on = (Gg.flags & FDY_HAS_COMMON_ATTRS) && Gg.sec_size[FDY_SEC_COMMON_ATTRS] >= 52;
  const bool common_t_on = (Gt.flags & FDY_HAS_COMMON_ATTRS) && Gt.sec_size[FDY_SEC_COMMON_ATTRS] >= 52;
  // Equal node counts, section sizes (bounds then agree node for node) and
  // common-attr presence: the byte compare may decide nodes.
  // (A graph without nodes has one empty chunk and nothing to compare: its
  // entry pairs, loaded without bounds checks, would read past the section.)
  const bool fast = !is_t && N != 0 && N == Gt.num_nodes && common_g_on == common_t_on &&
                    Gg.sec_size[FDY_SEC_STRINGS] == Gt.sec_size[FDY_SEC_STRINGS] &&
                    Gg.sec_size[FDY_SEC_PARAM_INDEX] == Gt.sec_size[FDY_SEC_PARAM_INDEX] &&
                    Gg.sec_size[FDY_SEC_PARAM_DATA] == Gt.sec_size[FDY_SEC_PARAM_DATA] &&
                    Gg.sec_size[FDY_SEC_ARG_DATA] == Gt.sec_size[FDY_SEC_ARG_DATA];

  // Record fields used past the first barrier, kept in registers: each
  // barrier's fence would have a later use load the field again.
  const uint64_t pidx_size = Gg.sec_size[FDY_SEC_PARAM_INDEX];
  const uint64_t node_base = Gg.node_base;
  const uint64_t* pg = reinterpret_cast<const uint64_t*>(img + Gg.sec_off[FDY_SEC_PARAM_INDEX]);
  const uint64_t* pt = reinterpret_cast<const uint64_t*>(img + Gt.sec_off[FDY_SEC_PARAM_INDEX]);
  const uint32_t pad = (kNodeChunk - N % kNodeChunk) % kNodeChunk;
  const int64_t first = (int64_t)c * kNodeChunk - pad;  // node of thread 0
  // The chunk's entries against the template's: word w of the chunk is word
  // w % 21 of its node w / 21 (168 = 21 * 8), read coalesced, two words
  // (16 bytes) per lane per load: pair p = tid + 256 m holds words 2p, 2p + 1.
  const uint8_t* eg0 = img + Gg.sec_off[FDY_SEC_NODES];
  const uint8_t* et0 = img + Gt.sec_off[FDY_SEC_NODES];
  const int64_t b0 = first * 168;
  static_assert(kEntryWords * kNodeChunk % 2 == 0, "whole pairs");
  constexpr uint32_t kPairs = kEntryWords * kNodeChunk / 2;  // per side
  // Loaded without a branch (a branch per pair made each wait for the one
  // before): a pair wholly before the chunk's first node (its padded front)
  // reads the section's first pair instead, and the one straddling the
  // section start reads the 8 bytes before it, which the file's header and
  // directory precede; take_pair drops the words before the first node.  A
  // chunk's pairs never pass its last node.
  auto pair_off = [&](uint32_t m) -> int64_t { return b0 + 16 * (int64_t)(tid + kNodeChunk * m); };
  auto load_pair = [&](uint32_t m, uint64_t* vg, uint64_t* vt) {
    const int64_t off = pair_off(m);
    const int64_t offl = off < -8 ? 0 : off;
    const u64x2a8 g2 = *reinterpret_cast<const u64x2a8*>(eg0 + offl);
    const u64x2a8 t2 = *reinterpret_cast<const u64x2a8*>(et0 + offl);
    vg[0] = g2.x;
    vg[1] = g2.y;
    vt[0] = t2.x;
    vt[1] = t2.y;
  };
  auto take_word = [&](uint32_t w, uint64_t vg, uint64_t vt) {
    const uint32_t node = w / kEntryWords, k = w % kEntryWords;
    // Words 1-3 and the low half of word 4 of a kernel entry are its
    // launch dimensions and shared memory (bytes 8-36): a difference there
    // alone changes the node's descriptor and nothing else.
    const uint64_t x = vg ^ vt;
    if (x) {
      if ((k >= 1 && k <= 3) || (k == 4 && (x >> 32) == 0)) s_launch[node] = 1;
      else s_dirty[node] = 1;
    }
    // Fields the param-entry check needs: type (word 0), param index
    // offset and count (word 16), arg buffer offset (word 17).
    if (k == 0) s_type[node] = (uint8_t)(vg >> 32);
    if (k == FDY_KOFF_PARAM_INDEX / 8) {
      s_pio[node] = (uint32_t)vg;
      s_np[node] = (uint32_t)(vg >> 32);
    }
    if (k == FDY_KOFF_ARG_OFFSET / 8) s_perparam[node] = (uint32_t)vg == FDY_NO_ARG_BUFFER;
  };
  auto take_pair = [&](uint32_t m, const uint64_t* vg, const uint64_t* vt) {
    const uint32_t w = 2 * (tid + kNodeChunk * m);
    const int64_t off = pair_off(m);
    if (off >= 0) take_word(w, vg[0], vt[0]);
    if (off >= -8) take_word(w + 1, vg[1], vt[1]);
  };
  // Pairs 0-6 in the first round, 7-10 in the second (pair 10 for the first
  // half of the threads).
  constexpr uint32_t kPairs1 = 7, kPairs2 = (kPairs + kNodeChunk - 1) / kNodeChunk - kPairs1;
  static_assert(kPairs2 == 4 && kPairs - (kPairs1 + kPairs2 - 1) * kNodeChunk == kNodeChunk / 2, "pair rounds");
  // The nodes whose param-index field (entry word 16) the first round holds.
  constexpr uint32_t kSpecNodes = (2 * kPairs1 * kNodeChunk - FDY_KOFF_PARAM_INDEX / 8 - 1) / kEntryWords + 1;
  const int64_t ns = first + tid;
  const bool valid = ns >= 0 && ns < (int64_t)N;
  const uint32_t n = valid ? (uint32_t)ns : 0;
  // A member's first round of entry loads goes out before the staging below.
  uint64_t vg0[2 * kPairs1], vt0[2 * kPairs1];
  if (fast) {
#pragma unroll
    for (uint32_t m = 0; m < kPairs1; ++m) load_pair(m, vg0 + 2 * m, vt0 + 2 * m);
  }

  if (tid == 0) {
    s_flags = 0;
    s_status = 0;
    s_pmin = s_umin = 0xFFFFFFFFu;
    s_pmax = 0;
  }
  s_dirty[tid] = 0;
  s_launch[tid] = 0;

  // The (small) string sections and the common attrs in LDS (sections start
  // 8-byte aligned).
  // All of these loads are issued before any LDS store, so the staging costs
  // one round trip, not one per piece.
  Strings sg_str{img + Gg.sec_off[FDY_SEC_STRINGS], Gg.sec_size[FDY_SEC_STRINGS]};
  Strings st_str{img + Gt.sec_off[FDY_SEC_STRINGS], Gt.sec_size[FDY_SEC_STRINGS]};
  const bool str_g = sg_str.size <= kStrStage, str_t = !is_t && st_str.size <= kStrStage;
  static_assert(kStrStage / 8 <= kNodeChunk, "one string word per thread");
  const uint32_t nsg = (uint32_t)((sg_str.size + 7) / 8), nst = (uint32_t)((st_str.size + 7) / 8);
  const bool cm_t = !is_t && common_t_on;
  uint64_t xg = 0, xt = 0, yg = 0, yt = 0;
  if (str_g && tid < nsg) xg = reinterpret_cast<const uint64_t*>(sg_str.p)[tid];
  if (str_t && tid < nst) xt = reinterpret_cast<const uint64_t*>(st_str.p)[tid];
  if (common_g_on && tid < 7) yg = reinterpret_cast<const uint64_t*>(img + Gg.sec_off[FDY_SEC_COMMON_ATTRS])[tid];
  if (cm_t && tid < 7) yt = reinterpret_cast<const uint64_t*>(img + Gt.sec_off[FDY_SEC_COMMON_ATTRS])[tid];
  // Every node of a chunk that is not a member's takes the per-node path: the
  // CRC tables, in LDS.
  uint64_t sl[8];
  if (!fast) {
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) sl[k] = a.cc->slice.t[k][tid];
  }
  if (str_g && tid < nsg) s_str[0][tid] = xg;
  if (str_t && tid < nst) s_str[1][tid] = xt;
  if (common_g_on && tid < 7) s_common[0][tid] = yg;
  if (cm_t && tid < 7) s_common[1][tid] = yt;
  if (!fast) {
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) s_slice[k][tid] = sl[k];
  }
  if (str_g) sg_str.p = reinterpret_cast<const uint8_t*>(s_str[0]);
  if (str_t) st_str.p = reinterpret_cast<const uint8_t*>(s_str[1]);
  if (is_t) st_str = sg_str;
  const uint8_t* common_g = common_g_on ? reinterpret_cast<const uint8_t*>(s_common[0]) : nullptr;
  const uint8_t* common_t = is_t ? common_g : cm_t ? reinterpret_cast<const uint8_t*>(s_common[1]) : nullptr;
  __syncthreads();  // the marks are zero before any thread sets one

  if (fast) {
#pragma unroll
    for (uint32_t m = 0; m < kPairs1; ++m) take_pair(m, vg0 + 2 * m, vt0 + 2 * m);
  }
  lds_barrier();
  if (fast) {
    // The first in-bounds param entry of the kernel nodes whose fields the
    // first round held: where the chunk's param entries most likely start.
    uint32_t umin = 0xFFFFFFFFu;
    if (valid && tid < kSpecNodes && s_type[tid] == FDY_NODE_KERNEL && s_np[tid] &&
        (uint64_t)s_pio[tid] + 8ull * s_np[tid] <= pidx_size)
      umin = s_pio[tid];
#pragma unroll
    for (int dd = 32; dd >= 1; dd >>= 1) umin = min(umin, (uint32_t)__shfl_down(umin, (unsigned)dd, 64));
    if (lane == 0 && umin != 0xFFFFFFFFu) atomicMin(&s_umin, umin);
  }
  __syncthreads();
  // The last entry pairs, and kPidxSpec * kNodeChunk param-entry words from
  // there on both sides (within the section: the sizes are equal and 8-byte
  // aligned), compared once loaded; which of the differing words count is
  // settled once the clean nodes are known.
  constexpr uint32_t kPidxSpec = 9;
  const uint32_t pidx_words = (uint32_t)(pidx_size / 8);
  const uint32_t u0 = s_umin == 0xFFFFFFFFu ? 0 : s_umin / 8;
  const uint32_t u1 = s_umin == 0xFFFFFFFFu ? 0 : min(u0 + kPidxSpec * kNodeChunk, pidx_words);
  uint32_t pdiff = 0;  // bit m: word u0 + tid + m * kNodeChunk differs
  if (fast) {
    uint64_t vg[2 * kPairs2], vt[2 * kPairs2];
#pragma unroll
    for (uint32_t m = 0; m < kPairs2; ++m) {
      vg[2 * m] = vg[2 * m + 1] = vt[2 * m] = vt[2 * m + 1] = 0;
      if (tid + kNodeChunk * (kPairs1 + m) < kPairs) load_pair(kPairs1 + m, vg + 2 * m, vt + 2 * m);
    }
    uint64_t wg[kPidxSpec], wt[kPidxSpec];
    if (u1 > u0) {  // uniform
#pragma unroll
      for (uint32_t m = 0; m < kPidxSpec; ++m) {
        const uint32_t q = u0 + tid + m * kNodeChunk;
        const uint32_t qc = q < u1 ? q : u1 - 1;  // a word inside the range stands in past its end
        wg[m] = pg[qc];
        wt[m] = pt[qc];
      }
    }
#pragma unroll
    for (uint32_t m = 0; m < kPairs2; ++m)
      if (tid + kNodeChunk * (kPairs1 + m) < kPairs) take_pair(kPairs1 + m, vg + 2 * m, vt + 2 * m);
    if (u1 > u0) {
#pragma unroll
      for (uint32_t m = 0; m < kPidxSpec; ++m)
        if (u0 + tid + m * kNodeChunk < u1 && wg[m] != wt[m]) pdiff |= 1u << m;
    }
  }
  __syncthreads();

  if (fast) {
    // Identical string sections and common attrs.
    bool d = false;
    if (tid < 7 && common_g) d |= s_common[0][tid] != s_common[1][tid];
    const uint32_t nw = (uint32_t)((sg_str.size + 7) / 8);
    const uint64_t* ps = reinterpret_cast<const uint64_t*>(sg_str.p);
    const uint64_t* pt = reinterpret_cast<const uint64_t*>(st_str.p);
    for (uint32_t w = tid; w < nw; w += kNodeChunk) d |= ps[w] != pt[w];
    // Launch-dimension differences are such only in kernel entries (the
    // same bytes hold other fields of other node types).
    if (valid && s_launch[tid] && s_type[tid] != FDY_NODE_KERNEL) s_dirty[tid] = 1;
    // The clean per-param kernel nodes' param entries span [pmin, pmax).
    uint32_t pmin = 0xFFFFFFFFu, pmax = 0;
    if (valid && !s_dirty[tid] && s_type[tid] == FDY_NODE_KERNEL && s_perparam[tid] && s_np[tid]) {
      const uint64_t end = (uint64_t)s_pio[tid] + 8ull * s_np[tid];
      if (end > pidx_size) {
        s_dirty[tid] = 1;  // out of bounds: the per-node path reports it
      } else {
        pmin = s_pio[tid];
        pmax = (uint32_t)end;
      }
    }
#pragma unroll
    for (int dd = 32; dd >= 1; dd >>= 1) {
      pmin = min(pmin, (uint32_t)__shfl_down(pmin, (unsigned)dd, 64));
      pmax = max(pmax, (uint32_t)__shfl_down(pmax, (unsigned)dd, 64));
    }
    if (lane == 0 && pmax) {
      atomicMin(&s_pmin, pmin);
      atomicMax(&s_pmax, pmax);
    }
    if (__ballot(d) && lane == 0) atomicOr(&s_flags, kChunkCtxDiff);
  }
  __syncthreads();
  if (fast && s_pmax > s_pmin) {
    // The words covering [pmin, pmax) inside [u0, u1): their compare is in
    // pdiff.
    const uint32_t p0 = s_pmin / 8, q1 = (s_pmax + 7) / 8;
    bool d = false;
#pragma unroll
    for (uint32_t m = 0; m < kPidxSpec; ++m) {
      const uint32_t q = u0 + tid + m * kNodeChunk;
      d |= ((pdiff >> m) & 1) && q >= p0 && q < q1;
    }
    // Words outside the ones compared above (before them, or past them in a
    // chunk with more param entries), kPidxBatch per side in flight per
    // thread.
    constexpr uint32_t kPidxBatch = 8;
    auto compare_words = [&](uint32_t r0, uint32_t r1) {
      for (uint32_t q0 = r0 + tid; q0 < r1; q0 += kPidxBatch * kNodeChunk) {
        uint64_t vg[kPidxBatch], vt[kPidxBatch];
#pragma unroll
        for (uint32_t m = 0; m < kPidxBatch; ++m) {
          const uint32_t q = q0 + m * kNodeChunk;
          const uint32_t qc = q < r1 ? q : r1 - 1;  // a word inside the range stands in past its end
          vg[m] = pg[qc];
          vt[m] = pt[qc];
        }
#pragma unroll
        for (uint32_t m = 0; m < kPidxBatch; ++m) d |= vg[m] != vt[m];
      }
    };
    if (u1 > u0) {
      compare_words(p0, min(q1, u0));
      compare_words(max(p0, u1), q1);
    } else {
      compare_words(p0, q1);
    }
    if (d) atomicOr(&s_flags, kChunkPidxDiff);
  }
  __syncthreads();
  // The record rows are free again: zero them (clean and padding nodes
  // keep zero records).
  s_rec[0][tid >> 3][2 * (tid & 7)] = s_rec[0][tid >> 3][2 * (tid & 7) + 1] = 0;
  s_rec[1][tid >> 3][2 * (tid & 7)] = s_rec[1][tid >> 3][2 * (tid & 7) + 1] = 0;
  const bool same_ctx = fast && !(s_flags & kChunkCtxDiff);
  const bool diff = fast && s_flags == 0;  // records as XORs with the template's; clean nodes skipped
  const bool mine = valid && (!diff || s_dirty[tid]);
  const uint64_t mb = __ballot(mine);
  if (lane == 0) s_wave_n[wave] = (uint32_t)__popcll(mb);
  if (valid && !mine) {
    NodeDesc d{};
    d.flags = kNodeClean | (s_launch[tid] ? FDY_NODE_DESC : 0u);
    a.node_desc[node_base + n] = d;
  }
  lds_barrier();  // the clean nodes' descriptors are not read back here
  uint32_t before = 0, total = 0;
#pragma unroll
  for (uint32_t w = 0; w < kNodeChunk / 64; ++w) {
    before += w < wave ? s_wave_n[w] : 0u;
    total += s_wave_n[w];
  }
  if (mine) s_list[before + (uint32_t)__popcll(mb & ((1ull << lane) - 1))] = (uint16_t)tid;
  if (fast && total) stage_slice(s_slice, a.cc->slice.t);  // uniform
  __syncthreads();

  uint64_t pbytes = 0;
  for (uint32_t k = tid; k < total; k += kNodeChunk) {
    const uint32_t slot = s_list[k];
    const uint32_t nn = (uint32_t)(first + slot);
    NodeOut o;
    if (is_t) node_full<true>(a, Gg, Gt, nn, sg_str, st_str, common_g, common_t, same_ctx, diff, s_slice, o);
    else node_full<false>(a, Gg, Gt, nn, sg_str, st_str, common_g, common_t, same_ctx, diff, s_slice, o);
    const uint64_t gi = node_base + nn;
    a.node_desc[gi] = o.d;
    a.node_flags[gi] = (uint8_t)(o.d.flags & 0x0F);
    a.node_ptrs[2 * gi] = o.p0;
    a.node_ptrs[2 * gi + 1] = o.p1;
    a.node_pbytes[gi] = o.pbytes;
    if (is_t) a.live_src[gi] = g;
    if (o.d.flags & kNodeBad) atomicOr(&s_status, FDY_GRAPH_BAD_PARAMS);
    pbytes += o.pbytes;
    s_rec[0][slot >> 3][2 * (slot & 7)] = o.rec[0];
    s_rec[0][slot >> 3][2 * (slot & 7) + 1] = o.rec[1];
    s_rec[1][slot >> 3][2 * (slot & 7)] = o.rec[2];
    s_rec[1][slot >> 3][2 * (slot & 7) + 1] = o.rec[3];
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) pbytes += shfl_down64(pbytes, d);
  if (lane == 0) s_pb[wave] = pbytes;
  lds_barrier();  // nor are the per-node outputs
  if (tid >= 64) return;
  if (total == 0) {  // every record is zero (clean member chunk, or padding only): so are their CRCs
    if (tid == 0) {
      NodeChunk ch;
      ch.crc_type = ch.crc_kent = 0;
      ch.pbytes = 0;
      for (uint32_t w = 0; w < kNodeChunk / 64; ++w) ch.pbytes += s_pb[w];
      ch.status = s_status;
      ch.mode = diff ? kChunkDiff : 0u;
      a.chunks[chunk] = ch;
    }
    return;
  }
  // Raw CRCs of the two record streams, by the first wave: lane l folds the
  // eight records 8q..8q+7 (q = l % 32) of stream l / 32 into one raw CRC
  // and moves it into place, times x^(8*16*(255-(8q+7))); each half-wave
  // XOR-joins its 32 shares (crc(A || B) = crc(A) * x^(8|B|) xor crc(B)).
  static_assert(kNodeChunk == 8 * 32, "eight records per lane, 32 lanes per stream");
  uint64_t z = 0;
  {
    const uint32_t st = tid >> 5, q = tid & 31;
#pragma unroll
    for (uint32_t r = 0; r < 16; ++r) z = crc_slice8(s_slice, z, s_rec[st][q][r]);
    z = z ? gf2_mulmod(a.cc->pos16[8 * q + 7], z) : 0;
#pragma unroll
    for (int d = 16; d >= 1; d >>= 1) z ^= shfl_down64(z, d);  // lanes 0 and 32 hold their half's XOR
  }
  const uint64_t zk = ((uint64_t)__shfl((uint32_t)(z >> 32), 32, 64) << 32) | __shfl((uint32_t)z, 32, 64);
  if (tid == 0) {
    NodeChunk ch;
    ch.crc_type = z;
    ch.crc_kent = zk;
    ch.pbytes = 0;
    for (uint32_t w = 0; w < kNodeChunk / 64; ++w) ch.pbytes += s_pb[w];
    ch.status = s_status;
    ch.mode = diff ? kChunkDiff : 0u;
    a.chunks[chunk] = ch;
  }
}

__global__ __launch_bounds__(kNodeThreads, 6) void k_node_b(RestoreArgs a) {
  static_assert(kNodeThreads <= 1024, "a scan step holds 16 waves");
  __shared__ uint32_t s_tmp[2][16];
  __shared__ uint64_t s_x[4][kNodeThreads / 64];
  __shared__ unsigned long long s_pb;
  __shared__ uint32_t s_status, s_words, s_flat, s_tbase;
  if (blockIdx.x >= a.num_graphs) {
    // Workgroups past the graphs: the digest units, one per wave (the key
    // and dependency digests are off the grouping chain, so they run beside
    // this pass).  A wave takes the raw CRC of its 4 KB slice (lane l absorbs
    // 64 bytes through the slicing tables and is moved into place by
    // x^(8*64*(63-l))), shifts it past the slices after it and XORs it into
    // the digest (XOR is order-free).  Every load that does not depend on
    // the slice's bytes is issued with them, before the tables are staged.
    __shared__ uint64_t s_slice[8][256];
    static_assert(8 * 256 == 4 * kNodeThreads, "four table words per thread");
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t* tab = &a.cc->slice.t[0][0];
    uint64_t tw[4];
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) tw[k] = tab[threadIdx.x + k * kNodeThreads];
    const uint32_t u = (blockIdx.x - a.num_graphs) * (kNodeThreads / 64) + (threadIdx.x >> 6);
    const bool on = u < a.num_units;
    const DigestUnit du = a.units[on ? u : 0];
    const int64_t b0 = (int64_t)du.len - (int64_t)kSliceBytes * du.back - 64 * (64 - (int64_t)lane);
    const int64_t q0 = b0 >> 3;  // b0 = 8 q0 + (len mod 8) in every lane
    const uint32_t sh = (uint32_t)(du.len & 7);
    const uint8_t* p = a.img + du.src;
    // Words before the stream read as zero.  Past its end only word q0 + 8
    // of the last lane can lie (one word, when len is a multiple of 8, and
    // then unused): inside the image buffer, whose 4 KB zero tail covers it.
    uint64_t w[9];
#pragma unroll
    for (uint32_t k = 0; k < 9; ++k) {
      const int64_t q = q0 + k;
      const uint64_t v = reinterpret_cast<const uint64_t*>(p)[q < 0 ? 0 : q];
      w[k] = q < 0 ? 0 : v;
    }
    uint64_t pm = a.cc->pos64[kPosLanes - 64 + lane];
    const uint64_t cs = a.cc->chunk_shift[min(du.back, (uint32_t)kChunkShifts - 1)][lane];
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) (&s_slice[0][0])[threadIdx.x + k * kNodeThreads] = tw[k];
    __syncthreads();
    if (!on) return;
    // pm opaque from here: otherwise the multiply's 64 per-bit masks of pm
    // are computed before the barrier and spilled.
    asm volatile("" : "+v"(pm));
    uint64_t z = 0;
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) z = crc_slice8(s_slice, z, sh ? (w[k] >> (8 * sh)) | (w[k + 1] << (64 - 8 * sh)) : w[k]);
    z = gf2_mulmod(pm, z);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) z ^= shfl_down64(z, d);
    z = ((uint64_t)__shfl((uint32_t)(z >> 32), 0, 64) << 32) | __shfl((uint32_t)z, 0, 64);  // the slice's raw CRC
    uint64_t share;
    if (du.back == 0) share = lane == 0 ? z : 0;
    else if (du.back < (uint32_t)kChunkShifts) share = ((z >> (63 - lane)) & 1) ? cs : 0;
    else share = lane == 0 ? far_shift(a.cc, z, du.back) : 0;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) share ^= shfl_down64(share, d);
    if (lane == 0 && share) atomicXor(reinterpret_cast<unsigned long long*>(a.digests + du.dst), share);
    return;
  }

  const uint32_t g = blockIdx.x;
  const uint32_t t = *readonly(a.template_of + g);  // written by the grouping pass
  const bool is_t = t == g;
  const DevGraph& Gg = a.graphs[g];
  // The record fields this pass uses, read through the constant address
  // space: nothing writes the records during the restore, so these are
  // scalar loads, which neither wait for the vector loads in flight nor
  // are repeated after a barrier's fence (as loads of a record that might
  // be written would be).
  const ConstGraph* cg = readonly(a.graphs + g);
  const ConstGraph* ct = readonly(a.graphs + t);
  const uint32_t N = cg->num_nodes, NT = ct->num_nodes;
  const uint64_t g_node_base = cg->node_base, t_node_base = ct->node_base;
  const uint32_t g_chunk_base = cg->chunk_base, t_chunk_base = ct->chunk_base;
  const uint64_t g_sec_param = cg->sec_off[FDY_SEC_PARAM_DATA], g_sec_arg = cg->sec_off[FDY_SEC_ARG_DATA];
  const uint64_t t_sec_param = ct->sec_off[FDY_SEC_PARAM_DATA], t_sec_arg = ct->sec_off[FDY_SEC_ARG_DATA];
  const uint32_t g_word_cap = cg->word_cap, t_word_cap = ct->word_cap;
  const uint32_t g_tile_base = cg->tile_base, g_tile_cap = cg->tile_cap;
  const uint64_t g_word_base = cg->word_base, t_word_base = ct->word_base;
  const uint8_t* img = a.img;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // A block of kNodeThreads nodes' inputs: the node's first-pass results
  // and, for a member, its template node's (loaded for every node, not only
  // the clean ones, so that they need not wait for the node's flags), one
  // block ahead of the block being completed.
  struct NodeIn {
    NodeDesc d;
    uint4 th;            // the template node's gword, nwords, tword, flags
    uint64_t ts, q0, q1, tpb;
  };
  auto load_in = [&](uint32_t base, NodeIn& in) {
    const uint32_t n = base + threadIdx.x;
    in.d = NodeDesc{};
    in.th = make_uint4(0, 0, 0, 0);
    in.ts = in.q0 = in.q1 = in.tpb = 0;
    if (n < N) {
      in.d = a.node_desc[g_node_base + n];
      if (!is_t && n < NT) {
        const uint64_t ti = t_node_base + n;
        in.th = *reinterpret_cast<const uint4*>(a.node_desc + ti);
        in.ts = a.node_desc[ti].src_g;
        in.q0 = a.node_ptrs[2 * ti];
        in.q1 = a.node_ptrs[2 * ti + 1];
        in.tpb = a.node_pbytes[ti];
      }
    }
  };
  NodeIn cur;
  load_in(0, cur);

  // Chunk results, one wave per chunk: the node-type and kernel-entry CRCs
  // (of a diff chunk: XORed with the template chunk's) shifted past the
  // chunks after them; param bytes and status bits.  The chunk, its
  // template chunk and the lane's shift multiple load together, before the
  // workgroup's first barrier.
  static_assert(kNodeChunk == kPosRecords, "chunk shift tables are built for kPosRecords records per chunk");
  const uint32_t nch = node_chunks(N), ncht = node_chunks(NT);
  uint64_t x[4] = {0, 0, 0, 0}, pb = 0;
  uint32_t st = 0;
  for (uint32_t c = wave; c < nch; c += kNodeThreads / 64) {
    const uint32_t k = nch - 1 - c;
    const NodeChunk ch = a.chunks[g_chunk_base + c];
    const NodeChunk ctc = a.chunks[t_chunk_base + (c < ncht ? c : 0)];  // used for a diff chunk only
    const uint64_t row = a.cc->chunk_shift[k < (uint32_t)kChunkShifts ? k : 0][lane];
    uint64_t rt = ch.crc_type, rk = ch.crc_kent;
    if (ch.mode & kChunkDiff) {
      rt ^= ctc.crc_type;
      rk ^= ctc.crc_kent;
    }
    if (k < (uint32_t)kChunkShifts) {
      x[2] ^= ((rt >> (63 - lane)) & 1) ? row : 0ull;
      x[3] ^= ((rk >> (63 - lane)) & 1) ? row : 0ull;
    } else {
      x[2] ^= shift_share(a.cc, rt, k, lane);
      x[3] ^= shift_share(a.cc, rk, k, lane);
    }
    if (lane == 0) {
      pb += ch.pbytes;
      st |= ch.status;
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1)
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] ^= shfl_down64(x[k], d);
  if (lane == 0)
#pragma unroll
    for (int k = 0; k < 4; ++k) s_x[k][wave] = x[k];
  if (threadIdx.x == 0) {
    s_status = 0;
    s_pb = 0;
    s_flat = 1;
  }
  lds_barrier();

  // Word offsets of every node in the graph's and in the template's image;
  // clean nodes first take their template node's results (its first pass
  // is done; its second pass, running beside this one, rewrites only the
  // template's word offsets).
  uint32_t gcarry = 0, tcarry = 0;
  for (uint32_t base = 0; base < N; base += kNodeThreads) {
    NodeIn nxt;
    if (base + kNodeThreads < N) load_in(base + kNodeThreads, nxt);  // uniform
    const uint32_t n = base + threadIdx.x;
    const bool valid = n < N;
    const uint64_t gi = g_node_base + n;
    NodeDesc d = cur.d;
    if (valid && (d.flags & kNodeClean)) {
      const uint32_t tw = cur.th.y, tf = cur.th.w;
      const uint64_t ts = cur.ts;
      const uint64_t q0 = cur.q0, q1 = cur.q1;
      pb += cur.tpb;
      uint32_t f = (tf & kNodeExtra) | (d.flags & FDY_NODE_DESC);  // launch dimensions differ: DESC
      if (tf & kNodeBad) {
        f |= FDY_NODE_LAYOUT | kNodeBad;
        st |= FDY_GRAPH_BAD_PARAMS;
      } else {
        if (tf & FDY_NODE_RAGGED) f |= FDY_NODE_RAGGED | kNodeRaggedT;
        if (tw) f |= kNodeCompare;
      }
      const int sec = (tf & kNodeExtra) ? FDY_SEC_ARG_DATA : FDY_SEC_PARAM_DATA;
      d.nwords = tw;
      d.tword = tw;
      d.flags = f;
      d.src_t = ts;
      d.src_g = ts ? ts - (sec == FDY_SEC_ARG_DATA ? t_sec_arg : t_sec_param) +
                         (sec == FDY_SEC_ARG_DATA ? g_sec_arg : g_sec_param)
                   : 0;
      a.node_flags[gi] = (uint8_t)(f & 0x0F);
      a.node_ptrs[2 * gi] = q0;
      a.node_ptrs[2 * gi + 1] = q1;
    }
    const uint32_t words_g = d.nwords, words_t = d.tword;
    uint32_t flags = d.flags;
    const uint32_t wv[2] = {words_g, words_t};
    uint32_t ex[2], tot[2];
    block_excl_scan2(wv, s_tmp, ex, tot);
    const uint32_t gword = gcarry + ex[0], tword = tcarry + ex[1];
    const uint32_t tot_g = tot[0], tot_t = tot[1];
    // A template whose image overflows its capacity (overlapping param
    // ranges) has no usable words past the capacity; never index them.
    if ((flags & kNodeCompare) && (uint64_t)tword + words_t > t_word_cap) flags &= ~kNodeCompare;
    if (valid) {
      // The graph's image is flat when every node with words is aligned and
      // placed canonically (word w of the image at param-data byte 8w), and
      // likewise in the template's image for every compared node.
      if (words_g) {
        const bool ok = !(flags & (FDY_NODE_RAGGED | kNodeRaggedT)) &&
                        d.src_g == g_sec_param + 8ull * gword &&
                        (is_t || ((flags & kNodeCompare) && tword == gword &&
                                  d.src_t == t_sec_param + 8ull * gword));
        if (!ok) s_flat = 0;
      }
      if (is_t) {
        // Only the offsets change: members read this node's other fields.
        a.node_desc[gi].gword = gword;
        a.node_desc[gi].tword = tword;
      } else {
        d.gword = gword;
        d.tword = tword;
        d.flags = flags;
        a.node_desc[gi] = d;
      }
      if (words_g) {
        uint64_t k = ((uint64_t)gword + kTileWords - 1) / kTileWords;
        const uint64_t k_last = ((uint64_t)gword + words_g - 1) / kTileWords;
        for (; k <= k_last && k < g_tile_cap; ++k) a.tile_node[g_tile_base + k] = n;
        if (flags & FDY_NODE_RAGGED) {
          const uint8_t* eg = img + Gg.sec_off[FDY_SEC_NODES] + 168ull * n;
          Side sd_{}, none_{};
          bool same_;
          side_header(img, Gg, RawEntry{eg}, sd_);
          scan_params(img, Gg, sd_, true, Gg, none_, false, &same_);
          if (a.aux) write_aux(img, Gg, eg, sd_, a.aux, gword);
          else atomicOr(a.restore_flags, kFlagNeedAux);  // the host restores again with ragged-word sources
        }
      }
    }
    gcarry += tot_g;
    tcarry += tot_t;
    cur = nxt;
  }
  // One LDS atomic per wave: every thread's own atomic on one address
  // serialised (about 8 us of the pass at 1024 threads).
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    pb += shfl_down64(pb, d);
    st |= __shfl_down(st, (unsigned)d, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    if (pb) atomicAdd(&s_pb, (unsigned long long)pb);
    if (st) atomicOr(&s_status, st);
  }
  lds_barrier();
  if (threadIdx.x == 0) {
    uint64_t acc[4] = {0, 0, 0, 0};
    for (uint32_t w = 0; w < kNodeThreads / 64; ++w)
      for (int k = 0; k < 4; ++k) acc[k] ^= s_x[k][w];
    const bool overflow = gcarry > g_word_cap;
    s_words = overflow ? 0 : gcarry;
    uint32_t stat = s_status;
    if (!is_t && N != NT) stat |= kGraphNodeCount;
    if (overflow) stat |= FDY_GRAPH_BAD_PARAMS | kGraphOverflow;
    a.status[g] = stat;
    a.gwords[g] = s_words;
    a.pbytes[g] = s_pb;
    for (int k = 2; k < 4; ++k) a.digests[4ull * g + k] = acc[k] ^ cg->crc_fin[k];  // 0, 1: the digest units
    if (is_t) {
      a.live_cur[g] = g;
      // List the template's slots that hold words for k_diff_t.
      s_tbase = atomicAdd(a.tslot_count, (s_words + kTileWords - 1) / kTileWords);
    }
  }
  lds_barrier();
  const uint32_t words = s_words;
  const uint32_t first_unused = (words + kTileWords - 1) / kTileWords;
  const uint32_t sflags = (s_flat ? kSlotFlat | (is_t ? 0u : kSlotCompare) : 0u) | (is_t ? kSlotTemplate : 0u);
  for (uint32_t k = threadIdx.x; k < g_tile_cap; k += kNodeThreads) {
    if (k >= first_unused) a.tile_node[g_tile_base + k] = kNoTile;
    SlotDesc sd;
    sd.kg = g_sec_param;
    sd.kt = t_sec_param;
    sd.word_base = g_word_base;
    sd.wbeg = (uint32_t)min((uint64_t)k * kTileWords, (uint64_t)words);
    sd.wend = (uint32_t)min((uint64_t)(k + 1) * kTileWords, (uint64_t)words);
    sd.graph = g;
    sd.tmpl = t;
    sd.flags = sflags | (k == 0 ? kSlotFirst : 0u) | (k + 1 == g_tile_cap ? kSlotLast : 0u);
    sd.t_cap = t_word_cap;
    sd.node_base = (uint32_t)g_node_base;
    sd.num_nodes = N;
    sd.t_word_base = t_word_base;
    a.slot_desc[g_tile_base + k] = sd;
    a.slot_spill[g_tile_base + k] = 0;
    if (is_t && k < first_unused) a.tslot_desc[s_tbase + k] = sd;
  }
}

// ---- diff pass ----------------------------------------------------------

// The `width` bytes at byte offset `byte` of the image (any alignment).
__device__ inline uint64_t load_bytes(const uint8_t* img, uint64_t byte, uint32_t width) {
  const uint64_t a = byte & ~7ull;
  const uint32_t sh = (uint32_t)(byte & 7);
  uint64_t v = *reinterpret_cast<const uint64_t*>(img + a);
  if (sh) {
    v >>= 8 * sh;
    if (sh + width > 8) v |= *reinterpret_cast<const uint64_t*>(img + a + 8) << (64 - 8 * sh);
  }
  return width >= 8 ? v : v & ((1ull << (8 * width)) - 1);
}

// A slot descriptor, loaded whole before any branch (left to itself the
// compiler loads each field at its first use, behind branches, and every
// such load is another serial round trip before the tile's loads can start),
// by scalar loads: the node pass wrote it and nothing writes it here.
__device__ inline SlotDesc load_slot(const SlotDesc* p) {
  const auto* q = readonly(reinterpret_cast<const uint64_t*>(p));  // written by the node pass, read-only here
  SlotDesc d;
  static_assert(sizeof(SlotDesc) == 8 * sizeof(uint64_t), "SlotDesc is eight 8-byte words");
  uint64_t* o = reinterpret_cast<uint64_t*>(&d);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = q[i];
  return d;
}

// The same by vector loads, for a descriptor prefetched across LDS work:
// a scalar load's wait shares its counter with LDS accesses, so every LDS
// wait in between would wait for the prefetch too.
__device__ inline SlotDesc load_slot_v(const SlotDesc* p) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
  const uint4 v0 = q[0], v1 = q[1], v2 = q[2], v3 = q[3];
  asm volatile("" ::"s"(v0.x), "s"(v0.y), "s"(v0.z), "s"(v0.w), "s"(v1.x), "s"(v1.y), "s"(v1.z), "s"(v1.w),
               "s"(v2.x), "s"(v2.y), "s"(v2.z), "s"(v2.w), "s"(v3.x), "s"(v3.y), "s"(v3.z), "s"(v3.w));
  SlotDesc d;
  uint4* o = reinterpret_cast<uint4*>(&d);
  o[0] = v0;
  o[1] = v1;
  o[2] = v2;
  o[3] = v3;
  return d;
}

// Stage the descriptors of the nodes holding slot `slot`'s words in LDS
// (from its first node to the next slot's first node, at most kDiffWindow).
struct NodeWindow {
  const NodeDesc* nd;  // the graph's node descriptors
  uint32_t n0, N, nwin;
};

// The slot descriptor carries the graph's node range, so the window's loads
// wait only for it and the tile -> node table.
__device__ inline NodeWindow stage_window(const RestoreArgs& a, const SlotDesc& sd, uint32_t slot, NodeDesc* s_nd) {
  NodeWindow nw;
  nw.n0 = *readonly(a.tile_node + slot);
  nw.N = sd.num_nodes;
  const uint32_t n_next = (sd.flags & kSlotLast) ? kNoTile : *readonly(a.tile_node + slot + 1);
  const uint32_t n_last = n_next == kNoTile ? nw.N - 1 : n_next;
  nw.nwin = min(kDiffWindow, n_last - nw.n0 + 1);
  nw.nd = a.node_desc + sd.node_base;
  for (uint32_t i = threadIdx.x; i < nw.nwin; i += blockDim.x) s_nd[i] = nw.nd[nw.n0 + i];
  return nw;
}

// The nodes holding graph-local words w[0..J): for each, the last node whose
// first word is <= w[j].  The searches over the LDS window run in lockstep
// (the window size is uniform), so their LDS reads overlap; a word past a
// full window continues in global memory.  Nodes without words never
// match, since the node holding w follows them.
template <uint32_t J>
__device__ inline void find_nodes(const NodeDesc* s_nd, const NodeWindow& nw, const uint64_t* w, uint32_t* node) {
  uint32_t lo[J];
#pragma unroll
  for (uint32_t j = 0; j < J; ++j) lo[j] = 0;
  for (uint32_t len = nw.nwin; len > 1;) {
    const uint32_t half = len >> 1;
#pragma unroll
    for (uint32_t j = 0; j < J; ++j)
      if (s_nd[lo[j] + half].gword <= w[j]) lo[j] += half;
    len -= half;
  }
#pragma unroll
  for (uint32_t j = 0; j < J; ++j) {
    node[j] = nw.n0 + lo[j];
    if (nw.nwin == kDiffWindow && lo[j] == kDiffWindow - 1) {
      const NodeDesc& d = s_nd[lo[j]];
      if (w[j] >= (uint64_t)d.gword + d.nwords) {
        uint32_t l2 = node[j], h2 = nw.N;
        while (h2 - l2 > 1) {
          const uint32_t mid = (l2 + h2) >> 1;
          if (nw.nd[mid].gword <= w[j]) l2 = mid;
          else h2 = mid;
        }
        node[j] = l2;
      }
    }
  }
}

__device__ inline NodeDesc window_desc(const NodeDesc* s_nd, const NodeWindow& nw, uint32_t node) {
  const uint32_t i = node - nw.n0;
  return i < nw.nwin ? s_nd[i] : nw.nd[node];
}

// Raw word w of a graph whose node descriptor is d (general path): ragged
// words through their recorded byte position and width.
template <class GR>
__device__ inline uint64_t load_word(const RestoreArgs& a, const GR& G, const NodeDesc& d, uint64_t w,
                                     bool ragged, uint64_t src, uint32_t* width) {
  if (ragged) {
    if (!a.aux) {  // flagged by the node pass: this restore's results are discarded and it runs again
      *width = 8;
      return 0;
    }
    const uint64_t x = a.aux[G.word_base + w];
    *width = (uint32_t)(x & 15);
    return load_bytes(a.img, x >> 4, *width);
  }
  *width = 8;
  return *reinterpret_cast<const uint64_t*>(a.img + src + 8ull * (w - d.gword));
}

// Template graphs: relocate their words into R and the live image.  The
// template slots listed by the node pass are cut into units of kTUnit words
// (kTWords per thread, so one search batch), spread over the grid.  Four
// words per thread suit small graphs; where graphs average 256K words or
// more, eight (half as many units, each workgroup working through fewer in
// turn) measured 108 -> 97 us on the MoE-style archive, while four keep the
// decode-style pass at 10.9 us (13.0 us with eight).
constexpr uint32_t kTThreads = 256;
constexpr uint64_t kTWideSlotsPerGraph = 64;  // 64 slots of 4096 words: 256K words per graph
template <uint32_t kTWords>
constexpr uint32_t t_units_per_tile() {
  static_assert(kTileWords % (kTThreads * kTWords) == 0, "template units tile a slot");
  return kTileWords / (kTThreads * kTWords);
}

constexpr uint32_t kTSearch = 2;  // searches per lane in one lockstep batch

template <uint32_t kTWords>
__global__ __launch_bounds__(kTThreads) void k_diff_t(RestoreArgs a) {
  constexpr uint32_t kTUnit = kTThreads * kTWords;
  constexpr uint32_t kTUnitsPerTile = t_units_per_tile<kTWords>();
  __shared__ NodeDesc s_nd[kDiffWindow];
  __shared__ uint64_t s_q[kTThreads / 64][64 * kTWords];  // per wave: the words it searches
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint64_t lt = (1ull << lane) - 1;
  const RelocDev& R = a.reloc;
  const uint32_t units = *readonly(a.tslot_count) * kTUnitsPerTile;
  // The next unit's slot descriptor is loaded while this unit is worked on
  // (with eight words per thread: MoE-style 105 -> 97 us).  The node pass
  // lists the template slots' descriptors themselves, so the first one is
  // a single load.
  SlotDesc next{};
  if (blockIdx.x < units) next = load_slot_v(a.tslot_desc + blockIdx.x / kTUnitsPerTile);
  for (uint32_t u = blockIdx.x; u < units; u += gridDim.x) {
    const SlotDesc sd = next;
    if (u + gridDim.x < units) next = load_slot_v(a.tslot_desc + (u + gridDim.x) / kTUnitsPerTile);
    const uint64_t ubeg = (uint64_t)sd.wbeg + (u % kTUnitsPerTile) * kTUnit;
    const uint64_t uend = min((uint64_t)sd.wend, ubeg + kTUnit);
    if (ubeg >= uend) continue;  // uniform over the block
    uint64_t v[kTWords], r[kTWords];
    uint32_t m = 0;
    if (sd.flags & kSlotFlat) {
      const uint8_t* pg = a.img + sd.kg;
#pragma unroll
      for (uint32_t q = 0; q < kTWords; ++q) {
        const uint64_t w = ubeg + q * kTThreads + tid;
        v[q] = 0;
        if (w < uend) {
          v[q] = *reinterpret_cast<const uint64_t*>(pg + 8 * w);
          m |= 1u << q;
        }
      }
    } else {
      const ConstGraph& G = *readonly(a.graphs + sd.graph);
      const uint32_t slot = G.tile_base + sd.wbeg / kTileWords;
      __syncthreads();  // the previous unit's lookups are done with s_nd
      const NodeWindow nw = stage_window(a, sd, slot, s_nd);
      __syncthreads();
      uint64_t wv[kTWords];
      uint32_t node[kTWords];
#pragma unroll
      for (uint32_t q = 0; q < kTWords; ++q) wv[q] = ubeg + q * kTThreads + tid;
      find_nodes<kTWords>(s_nd, nw, wv, node);
#pragma unroll
      for (uint32_t q = 0; q < kTWords; ++q) {
        const uint64_t w = wv[q];
        v[q] = 0;
        if (w < uend) {
          const NodeDesc d = window_desc(s_nd, nw, node[q]);
          uint32_t width;
          v[q] = load_word(a, G, d, w, (d.flags & FDY_NODE_RAGGED) != 0, d.src_g, &width);
          if (width == 8) m |= 1u << q;  // partial words are never relocated
        }
      }
    }
    // The whole words inside the table's range need an interval search:
    // about a quarter of them on the presets (the pointers).  Each wave
    // compacts its words to search in LDS, searches them kTSearch per lane
    // in lockstep, and every lane reads its results back, so no lane holds
    // line registers for words that need no search.
    uint32_t need = 0;
    if (R.n != 0) {
#pragma unroll
      for (uint32_t q = 0; q < kTWords; ++q)
        if (((m >> q) & 1) && v[q] >= R.lo_min && (R.policy ? v[q] <= R.hi_max : v[q] < R.hi_max)) need |= 1u << q;
    }
    uint64_t* sq = s_q[tid >> 6];
    uint32_t rank[kTWords], cnt = 0;
#pragma unroll
    for (uint32_t q = 0; q < kTWords; ++q) {
      const uint64_t mk = __ballot((need >> q) & 1);
      rank[q] = cnt + (uint32_t)__popcll(mk & lt);
      if ((need >> q) & 1) sq[rank[q]] = v[q];
      cnt += (uint32_t)__popcll(mk);
    }
    // The wave's own LDS words: its writes precede its reads in program order.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (uint32_t b = 0; b < cnt; b += 64 * kTSearch) {
      uint64_t x[kTSearch], y[kTSearch];
      uint32_t mm = 0;
#pragma unroll
      for (uint32_t k = 0; k < kTSearch; ++k) {
        const uint32_t i = b + 64 * k + lane;
        x[k] = i < cnt ? sq[i] : 0;
        mm |= (i < cnt ? 1u : 0u) << k;
      }
      reloc_batch<kTSearch>(R, x, y, mm);
#pragma unroll
      for (uint32_t k = 0; k < kTSearch; ++k) {
        const uint32_t i = b + 64 * k + lane;
        if (i < cnt) sq[i] = y[k];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (uint32_t q = 0; q < kTWords; ++q) r[q] = ((need >> q) & 1) ? sq[rank[q]] : v[q];
    uint64_t* img_out = a.image + sd.word_base;
#pragma unroll
    for (uint32_t q = 0; q < kTWords; ++q) {
      const uint64_t w = ubeg + q * kTThreads + tid;
      if (w < uend) img_out[w] = r[q];
    }
  }
  // The collision report, one graph per workgroup in turn, from the last
  // workgroup down (the first ones hold the template units; the digests are
  // final after the node pass): a graph below this graph's template whose
  // key has the same CRC-64/XZ and length.  Its key bytes differ, or it
  // would be the template (grouping is by exact bytes).
  if (a.explicit_template) return;
  for (uint32_t g = gridDim.x - 1 - blockIdx.x; g < a.num_graphs; g += gridDim.x) {
    const uint32_t t = a.template_of[g];
    const uint64_t dg = a.digests[4ull * g];
    const uint64_t Lg = a.graphs[g].sec_size[FDY_SEC_TOPOLOGY_KEY];
    bool coll = false;
    for (uint32_t j = tid; j < t; j += kTThreads)
      coll |= a.digests[4ull * j] == dg && a.graphs[j].sec_size[FDY_SEC_TOPOLOGY_KEY] == Lg;
    if (__ballot(coll) && (tid & 63) == 0) atomicOr(&a.status[g], FDY_GRAPH_COLLISION);
  }
}

// The other graphs: kMSplit workgroups per slot, each of kMThreads / 64
// waves; wave v of the slot (counted over its workgroups) owns the slot's
// sub-range v (kSubWords consecutive words), lane l its words
// v*kSubWords + 128h + 2l and the one after, for h < kMWords / 2.  Small workgroups retire and are
// replaced wave by wave, where one workgroup per slot left its CU idle
// while its last waves finished (measured: 91 us against 100 us for the
// 256-graph decode-style archive).  Relocation is a function of the
// raw word, so where a compared word equals the template's raw word the
// template's relocated word is taken from R and stored at once, as are
// partial words (never relocated).  The words left over (to be searched, or
// possibly differing from the template) become candidates: each wave
// compacts them, in word order, into its sub-range's region and their
// number into sub_count, and k_diff_s settles them.  No wave waits for an
// interval search, and flat tiles need neither LDS nor a barrier.
constexpr uint32_t kMSplit = 8;
constexpr uint32_t kMThreads = kSubsPerSlot * 64 / kMSplit;
static_assert(kSubsPerSlot % kMSplit == 0, "whole sub-ranges per workgroup");
constexpr uint32_t kSlots = 2;  // searches per batch in the overflowed-template path

// Six waves per SIMD: the node window in LDS (12 KB per workgroup) allows
// no more.
__global__ __launch_bounds__(kMThreads, 6) void k_diff_m(RestoreArgs a) {
  constexpr uint32_t J = kMWords;
  static_assert((kMThreads / 64) * kSubWords * sizeof(Candidate) <= kDiffWindow * sizeof(NodeDesc),
                "each wave's candidates fit its part of the node window");
  __shared__ NodeDesc s_nd[kDiffWindow];
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t slot = blockIdx.x / kMSplit, part = blockIdx.x % kMSplit;
  const uint32_t wave = part * (kMThreads / 64) + (tid >> 6);  // sub-range of the slot
  const SlotDesc sd = load_slot(a.slot_desc + slot);
  uint32_t* sub_count = a.sub_count + (uint64_t)slot * kSubsPerSlot;
  if (sd.flags & kSlotTemplate) {  // relocated by k_diff_t; a template has no overrides
    if (lane == 0) sub_count[wave] = 0;
    return;
  }
  const uint32_t g = sd.graph, t = sd.tmpl;
  const uint64_t wbeg = sd.wbeg, wend = sd.wend;
  // Lane l holds words 2l and 2l + 1 of each 128-word half of the sub-range:
  // word j is wb + 128 (j / 2) + j % 2, so a flat tile's pairs load and store
  // as 16-byte accesses (half the address-unit work of one word per lane).
  static_assert(J % 2 == 0 && kSubWords == 64 * J, "pairs of words per lane");
  const uint64_t wb = wbeg + (uint64_t)wave * kSubWords + 2 * lane;
  auto word_of = [&](uint32_t j) -> uint64_t { return wb + 128 * (j >> 1) + (j & 1); };
  const bool flat = (sd.flags & kSlotFlat) != 0;
  const RelocDev& R = a.reloc;
  // Issued ahead of the word loads so that its wait does not follow theirs.
  const uint32_t t_status = *readonly(a.status + t);  // a template's status: final after the node pass
  uint64_t* img_out = a.image + sd.word_base;
  // The template's relocated image (read within the template's capacity;
  // with relocation off it equals the raw image and is not read).  Its
  // words are usable unless the template overflowed its capacity (its image
  // is then empty); that is checked once the loads are in flight.
  const uint64_t* rimg_t = a.image + sd.t_word_base;
  const uint32_t t_last = sd.t_cap ? sd.t_cap - 1 : 0;

  // fg: the graph's raw word; ft: the template's raw word; fr: the
  // template's relocated word.  A flat tile's words all sit at kg + 8w (the
  // template's at kt + 8w, word w of its image) and are all compared.
  uint64_t fg[J], ft[J], fr[J];
  uint32_t valid = 0, cmp = 0, full = 0;
  if (flat) {
    const uint8_t* pg = a.img + sd.kg;
    const uint8_t* pt = a.img + sd.kt;
#pragma unroll
    for (uint32_t q = 0; q < J / 2; ++q) {
      const uint64_t w = word_of(2 * q);
      fg[2 * q] = ft[2 * q] = fr[2 * q] = fg[2 * q + 1] = ft[2 * q + 1] = fr[2 * q + 1] = 0;
      if (w + 1 < wend) {
        valid |= 3u << (2 * q);
        const u64x2a8 g2 = ld_stream(reinterpret_cast<const u64x2a8*>(pg + 8 * w));
        const u64x2a8 t2 = *reinterpret_cast<const u64x2a8*>(pt + 8 * w);
        fg[2 * q] = g2.x;
        fg[2 * q + 1] = g2.y;
        ft[2 * q] = t2.x;
        ft[2 * q + 1] = t2.y;
      } else if (w < wend) {
        valid |= 1u << (2 * q);
        fg[2 * q] = ld_stream(reinterpret_cast<const uint64_t*>(pg + 8 * w));
        ft[2 * q] = *reinterpret_cast<const uint64_t*>(pt + 8 * w);
      }
    }
    if (R.n != 0) {
#pragma unroll
      for (uint32_t q = 0; q < J / 2; ++q) {
        const uint64_t w = word_of(2 * q);
        if (((valid >> (2 * q)) & 3) == 3 && w + 1 <= t_last) {
          const u64x2a8 r2 = *reinterpret_cast<const u64x2a8*>(rimg_t + w);
          fr[2 * q] = r2.x;
          fr[2 * q + 1] = r2.y;
        } else {
          if ((valid >> (2 * q)) & 1) fr[2 * q] = rimg_t[min(w, (uint64_t)t_last)];
          if ((valid >> (2 * q + 1)) & 1) fr[2 * q + 1] = rimg_t[min(w + 1, (uint64_t)t_last)];
        }
      }
    }
    cmp = full = valid;
  }
  if (!flat && wend > wbeg) {  // uniform over the workgroup
    const ConstGraph& G = *readonly(a.graphs + g);
    const ConstGraph& T = *readonly(a.graphs + t);
    const NodeWindow nw = stage_window(a, sd, slot, s_nd);
    __syncthreads();
    uint64_t wv[J];
    uint32_t node[J];
#pragma unroll
    for (uint32_t j = 0; j < J; ++j) wv[j] = word_of(j);
    find_nodes<J>(s_nd, nw, wv, node);
#pragma unroll
    for (uint32_t j = 0; j < J; ++j) {
      const uint64_t w = wv[j];
      fg[j] = ft[j] = fr[j] = 0;
      if (w >= wend) continue;
      valid |= 1u << j;
      const NodeDesc d = window_desc(s_nd, nw, node[j]);
      uint32_t width;
      fg[j] = load_word(a, G, d, w, (d.flags & FDY_NODE_RAGGED) != 0, d.src_g, &width);
      if (width == 8) full |= 1u << j;
      if (d.flags & kNodeCompare) {
        // Compared nodes have equal param sizes, so the template's word has
        // the same width (and was relocated into R iff this one is).
        cmp |= 1u << j;
        const uint64_t tw = d.tword + (w - d.gword);
        uint32_t wt;
        NodeDesc dt = d;
        dt.gword = d.tword;
        ft[j] = load_word(a, T, dt, tw, (d.flags & kNodeRaggedT) != 0, d.src_t, &wt);
        if (R.n != 0) fr[j] = rimg_t[min(tw, (uint64_t)t_last)];
      }
    }
  }
  if (R.n == 0) {
#pragma unroll
    for (uint32_t j = 0; j < J; ++j) fr[j] = ft[j];  // relocation off: R equals the raw image
  } else if (t_status & kGraphOverflow) {
    // The template overflowed its capacity: relocate its compared words here.
#pragma unroll
    for (uint32_t jb = 0; jb < J; jb += kSlots) {
      uint64_t tin[kSlots], tout[kSlots];
#pragma unroll
      for (uint32_t k = 0; k < kSlots; ++k) tin[k] = ft[jb + k];
      reloc_batch<kSlots>(R, tin, tout, ((cmp & full) >> jb) & ((1u << kSlots) - 1));
#pragma unroll
      for (uint32_t k = 0; k < kSlots; ++k) fr[jb + k] = tout[k];
    }
  }

  // Store what is settled; the rest (whole words to relocate, and partial
  // words that differ from the template's) are candidates.  Every valid
  // word is stored, a whole word to relocate as its raw value until
  // k_diff_s writes the relocated one, so each word takes one
  // unconditional store.
  uint32_t cand = 0, creloc = 0;
  uint64_t res[J];
#pragma unroll
  for (uint32_t j = 0; j < J; ++j) res[j] = ((cmp >> j) & 1) && fg[j] == ft[j] ? fr[j] : fg[j];
#pragma unroll
  for (uint32_t q = 0; q < J / 2; ++q) {
    const uint64_t w = word_of(2 * q);
    if (((valid >> (2 * q)) & 3) == 3) {
      u64x2a8 r2;
      r2.x = res[2 * q];
      r2.y = res[2 * q + 1];
      st_stream(reinterpret_cast<u64x2a8*>(img_out + w), r2);
    } else if ((valid >> (2 * q)) & 1) {
      st_stream(img_out + w, res[2 * q]);
    }
  }
#pragma unroll
  for (uint32_t j = 0; j < J; ++j) {
    if (!((valid >> j) & 1)) continue;
    const bool c = (cmp >> j) & 1;
    const bool same = c && fg[j] == ft[j];
    if (same) continue;
    if (!((full >> j) & 1)) {
      if (c && fg[j] != fr[j]) cand |= 1u << j;
    } else {
      cand |= 1u << j;
      creloc |= 1u << j;
    }
  }
  // The candidates are compacted into the wave's part of the node window's
  // LDS (free once the loads are done), then copied out as whole 8-byte
  // words: one or two wide stores per wave where storing each word's
  // candidate directly took two narrow stores per word (measured: 91 -> 86 us
  // for the 256-graph decode-style archive).
  const uint64_t lt = (1ull << lane) - 1;
  if (!flat) __syncthreads();  // every wave of the workgroup is done with the node window
  Candidate* stage = reinterpret_cast<Candidate*>(s_nd) + (tid >> 6) * kSubWords;
  // In word order: within a 128-word half, lane l's two words follow the
  // candidates of the lanes below it.
  uint32_t run = 0, ncmp = 0;
#pragma unroll
  for (uint32_t q = 0; q < J / 2; ++q) {
    const uint64_t m0 = __ballot((cand >> (2 * q)) & 1), m1 = __ballot((cand >> (2 * q + 1)) & 1);
    ncmp += (uint32_t)__popcll(__ballot(((cand & cmp) >> (2 * q)) & 1)) +
            (uint32_t)__popcll(__ballot(((cand & cmp) >> (2 * q + 1)) & 1));
    const uint32_t below = (uint32_t)__popcll(m0 & lt) + (uint32_t)__popcll(m1 & lt);
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
      const uint32_t j = 2 * q + h;
      if ((cand >> j) & 1) {
        Candidate c;
        c.word = (uint32_t)word_of(j);
        c.flags = (((creloc >> j) & 1) ? kCandReloc : 0u) | (((cmp >> j) & 1) ? kCandCompare : 0u);
        c.raw = fg[j];
        c.tval = fr[j];
        stage[run + below + (h ? (uint32_t)((m0 >> lane) & 1) : 0u)] = c;
      }
    }
    run += (uint32_t)__popcll(m0) + (uint32_t)__popcll(m1);
  }
  // The first cand_cap candidates go to the sub-range's own region, the
  // rest to the slot's spill space (taken with one atomic, by the few waves
  // whose sub-range has that many; never with the full layout, whose
  // regions hold a whole sub-range).  Spill space that runs out raises the
  // overflow flag and keeps the region's share, so every later read stays
  // in bounds.
  const uint32_t C = a.cand_cap;
  uint32_t keep = run, spill = 0;
  if (run > C) {  // uniform over the wave
    uint32_t at = 0;
    if (lane == 0) at = atomicAdd(a.slot_spill + slot, run - C);
    at = __shfl(at, 0, 64);
    if (at + (run - C) <= a.spill_cap) {
      spill = kSubsPerSlot * C + at;
    } else {
      keep = C;
      if (lane == 0) atomicOr(a.restore_flags, kFlagOverflow);
    }
  }
  {
    static_assert(sizeof(Candidate) % 8 == 0, "candidates copy as 8-byte words");
    constexpr uint32_t kCandWords = sizeof(Candidate) / 8;
    const uint64_t* src = reinterpret_cast<const uint64_t*>(stage);
    uint64_t* area = reinterpret_cast<uint64_t*>(a.cand + (uint64_t)slot * (kSubsPerSlot * C + a.spill_cap));
    for (uint32_t i = lane; i < keep * kCandWords; i += 64)
      st_stream(area + (i < C * kCandWords ? wave * C * kCandWords + i : (spill - C) * kCandWords + i), src[i]);
  }
  // Candidates in the low half, compared candidates (a bound on the
  // records they make) in the high half: the search pass places a slot's
  // records after the bounds of its graph's earlier slots.
  if (lane == 0) {
    sub_count[wave] = keep | (ncmp << 16);
    if (keep > C) a.sub_off[(uint64_t)slot * kSubsPerSlot + wave] = spill;  // where the rest went
  }
  if (tid == 0 && part == 0 && (sd.flags & kSlotFirst)) {
    if (a.digests[4ull * g + 2] != a.digests[4ull * t + 2]) atomicOr(&a.status[g], FDY_GRAPH_TYPE_MISMATCH);
  }
}

// Candidates of the member pass, one wave per slot: the slot's sub-range
// lists are taken as one list in word order, kSBatch / 64 candidates per
// lane searched in one lockstep batch.  The relocated word goes to R, and
// the words whose value differs from the template's become override
// records, written straight to their place in the graph's override array
// (which starts at the graph's word base: a graph has at most one record
// per word).  A slot's place is the sum of its graph's earlier slots'
// compared-candidate counts (the member pass's bound on their records, in
// the high halves of the sub-range counts), so no pass over the slots'
// actual counts has to come first, and records keep the canonical order.
// Each record is completed here: the node holding its word (searched in the
// slot's node window, staged in LDS) and the word's index in the template's
// image.  A compared candidate whose relocated value equals the template's
// makes no record and leaves a gap at the end of its slot's range: the slot
// raises the archive's gap flag, and k_repack closes the gaps before any
// result is read.  The slot's record count goes to slot_rec.
constexpr uint32_t kSThreads = 256;  // four slots per workgroup
constexpr uint32_t kSBatch = 128;  // two per lane: three or four per lane measured 1.8 and 4.4 times slower

// The last node of the window (whose first word is <= w), or past a full
// window the last such node of the graph.
__device__ __forceinline__ void window_node(const uint2* s_gt, uint32_t nwin, uint32_t n0, const NodeDesc* nd,
                                            uint32_t N, uint64_t w, uint32_t* node, uint32_t* gw, uint32_t* tw) {
  uint32_t lo = 0;
  for (uint32_t len = nwin; len > 1;) {
    const uint32_t half = len >> 1;
    if (s_gt[lo + half].x <= w) lo += half;
    len -= half;
  }
  *node = n0 + lo;
  *gw = s_gt[lo].x;
  *tw = s_gt[lo].y;
  if (nwin == kDiffWindow && lo == kDiffWindow - 1 && w >= (uint64_t)nd[*node].gword + nd[*node].nwords) {
    uint32_t l2 = *node, h2 = N;
    while (h2 - l2 > 1) {
      const uint32_t mid = (l2 + h2) >> 1;
      if (nd[mid].gword <= w) l2 = mid;
      else h2 = mid;
    }
    *node = l2;
    *gw = nd[l2].gword;
    *tw = nd[l2].tword;
  }
}

// Six waves per SIMD (78 VGPRs, no spills): a batch's candidates are loaded
// at its start rather than during the previous batch's searches, which most
// slots (one batch) never used and which took the registers of the sixth
// wave (search pass 26.5 -> 25.5 us on the decode-style archive, 272 -> 260
// us on the MoE-style one).
__global__ __launch_bounds__(kSThreads, 6) void k_diff_s(RestoreArgs a) {
  constexpr uint32_t K = kSBatch / 64;
  static_assert(kSubsPerSlot <= 64, "one lane per sub-range count");
  // Per wave: {first graph word, first template word} of its window's nodes.
  __shared__ uint2 s_win[kSThreads / 64][kDiffWindow];
  __shared__ uint32_t s_off[kSThreads / 64][kSubsPerSlot];
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t slot = blockIdx.x * (kSThreads / 64) + (threadIdx.x >> 6);
  if (slot >= a.num_slots) return;  // per wave: this kernel has no barrier
  uint2* const s_gt = s_win[threadIdx.x >> 6];
  uint32_t* counts = a.sub_count + (uint64_t)slot * kSubsPerSlot;
  // What depends on the slot alone is loaded first.
  const uint32_t cnt = lane < kSubsPerSlot ? counts[lane] : 0;
  // A sub-range's list is its own region, continued in the slot's spill
  // space where the member pass recorded (only for lists longer than the
  // region).
  const uint32_t C = a.cand_cap;
  const uint32_t so =
      lane < kSubsPerSlot && (cnt & 0xFFFFu) > C ? a.sub_off[(uint64_t)slot * kSubsPerSlot + lane] : 0u;
  const SlotDesc sd = load_slot(a.slot_desc + slot);
  const uint32_t n0 = *readonly(a.tile_node + slot);
  const uint32_t n_after = slot + 1 < a.num_slots ? *readonly(a.tile_node + slot + 1) : kNoTile;
  // Lane q < kSubsPerSlot holds sub-range q's count; inclusive prefix over lanes.
  uint32_t incl = cnt;
#pragma unroll
  for (int d = 1; d < (int)kSubsPerSlot; d <<= 1) {
    const uint32_t y = shfl_up32(incl, d);
    if (lane >= (uint32_t)d) incl += y;
  }
  const uint32_t total = __shfl(incl, kSubsPerSlot - 1, 64) & 0xFFFFu;
  const uint32_t bound = __shfl(incl, kSubsPerSlot - 1, 64) >> 16;
  if (total == 0) {  // an inactive slot, a template's, or no candidates: no records
    if (lane == 0) a.slot_rec[slot] = 0;
    return;
  }
  // Per sub-range: the exclusive prefix of the candidate counts (the same
  // in every lane), and where its list continues in the slot's spill space
  // (in the wave's LDS: a select over sixteen of them per candidate cost
  // spills).
  uint32_t start[kSubsPerSlot];
#pragma unroll
  for (uint32_t q = 0; q < kSubsPerSlot; ++q) start[q] = __builtin_amdgcn_readlane(incl - cnt, q) & 0xFFFFu;
  uint32_t* const s_o = s_off[threadIdx.x >> 6];
  if (lane < kSubsPerSlot) s_o[lane] = so;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // Batch b's K candidates per lane, loaded unconditionally (a list index
  // past the end reads the first candidate and is masked off later) so that
  // they are issued together rather than each behind its own branch.  The
  // first batch is loaded before the bounds and the node window, so its
  // loads wait together with theirs.
  const Candidate* base = a.cand + (uint64_t)slot * (kSubsPerSlot * a.cand_cap + a.spill_cap);
  auto load_batch = [&](uint32_t b, Candidate* cand) {
#pragma unroll
    for (uint32_t kk = 0; kk < K; ++kk) {
      const uint32_t i0 = b + 64 * kk + lane;  // list index
      const uint32_t i = i0 < total ? i0 : 0u;
      uint32_t q = 0;
#pragma unroll
      for (uint32_t s = 1; s < kSubsPerSlot; ++s) q += start[s] <= i;
      uint32_t sq = start[0];
#pragma unroll
      for (uint32_t s = 1; s < kSubsPerSlot; ++s) sq = q == s ? start[s] : sq;
      const uint32_t j = i - sq;
      cand[kk] = base[j < C ? q * C + j : s_o[q] + (j - C)];
    }
  };
  Candidate cur[K];
  load_batch(0, cur);
  // A slot with candidates holds words, so it starts at k * kTileWords: its
  // index in the graph, and the graph's first slot, follow.  The earlier
  // slots' bounds: the high halves of their sub-range counts, four to a
  // 16-byte load.
  const uint32_t k = sd.wbeg / kTileWords;
  const uint4* earlier = reinterpret_cast<const uint4*>(a.sub_count + (uint64_t)(slot - k) * kSubsPerSlot);
  uint32_t before = 0;
  for (uint32_t j = lane; j < k * (kSubsPerSlot / 4); j += 64) {
    const uint4 v = earlier[j];
    before += (v.x >> 16) + (v.y >> 16) + (v.z >> 16) + (v.w >> 16);
  }
  const uint32_t word_cap = readonly(a.graphs + sd.graph)->word_cap;
  const uint32_t N = sd.num_nodes;
  const NodeDesc* nd = a.node_desc + sd.node_base;
  // The graph's last slot, or its last slot holding words (the next one's
  // table entry is kNoTile), ends at its last node.
  const uint32_t n_last = ((sd.flags & kSlotLast) || n_after == kNoTile) ? N - 1 : n_after;
  const uint32_t nwin = min(kDiffWindow, n_last - n0 + 1);
  for (uint32_t i = lane; i < nwin; i += 64) {
    const uint4 v = *reinterpret_cast<const uint4*>(nd + n0 + i);  // gword, nwords, tword, flags
    s_gt[i] = make_uint2(v.x, v.z);
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) before += __shfl_down(before, (unsigned)d, 64);
  before = __shfl(before, 0, 64);
  // The window is this wave's own: its LDS writes precede its reads in
  // program order.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  uint64_t* img_out = a.image + sd.word_base;
  // The graph's record region: in the compact layout it can be smaller than
  // the records' bound, and then nothing is written and the restore runs
  // again with full-capacity scratch.
  const uint64_t rb = sd.word_base >> a.rec_shift;
  const uint64_t rcap = ((sd.word_base + word_cap) >> a.rec_shift) - rb;
  if ((uint64_t)before + bound > rcap) {  // uniform over the wave
    if (lane == 0) {
      a.slot_rec[slot] = 0;
      atomicOr(a.restore_flags, kFlagOverflow);
    }
    return;
  }
  fdy_override* rec = a.ovr + rb + before;
  const uint64_t lt = (1ull << lane) - 1;
  uint32_t run = 0;
  for (uint32_t b = 0; b < total; b += kSBatch) {
    if (b) load_batch(b, cur);  // uniform over the wave
    uint64_t raw[K], tval[K], res[K];
    uint32_t word[K], fl[K], m = 0;
#pragma unroll
    for (uint32_t kk = 0; kk < K; ++kk) {
      const bool in = b + 64 * kk + lane < total;
      raw[kk] = in ? cur[kk].raw : 0;
      tval[kk] = in ? cur[kk].tval : 0;
      word[kk] = in ? cur[kk].word : 0;
      fl[kk] = in ? cur[kk].flags : 0;
      if (fl[kk] & kCandReloc) m |= 1u << kk;
    }
    reloc_batch<K>(a.reloc, raw, res, m);
    // The member pass stored each candidate's raw word; only the words the
    // relocation moved are stored again (a scattered 8-byte store costs a
    // partly written line).
#pragma unroll
    for (uint32_t kk = 0; kk < K; ++kk)
      if (((m >> kk) & 1) && res[kk] != raw[kk]) st_stream(img_out + word[kk], res[kk]);
#pragma unroll
    for (uint32_t kk = 0; kk < K; ++kk) {
      const bool d = (fl[kk] & kCandCompare) && res[kk] != tval[kk];
      const uint64_t mk = __ballot(d);
      if (d) {
        uint32_t node, gw, tw;
        window_node(s_gt, nwin, n0, nd, N, word[kk], &node, &gw, &tw);
        // One 16-byte record {word, node, value}.
        static_assert(sizeof(fdy_override) == 16 && __builtin_offsetof(fdy_override, node) == 4 &&
                          __builtin_offsetof(fdy_override, value) == 8,
                      "a record is {u32 word, u32 node, u64 value}");
        u64x2a8 o;
        o.x = (uint64_t)(tw + (word[kk] - gw)) | ((uint64_t)node << 32);
        o.y = res[kk];
        st_stream(reinterpret_cast<u64x2a8*>(rec + run + (uint32_t)__popcll(mk & lt)), o);
      }
      run += (uint32_t)__popcll(mk);
    }
  }
  if (lane == 0) {
    a.slot_rec[slot] = run;
    if (run != bound) atomicOr(a.restore_flags, kFlagGaps);  // rare: a compared word equal once relocated
  }
}

// Closing the gaps (launched before results are read, only when the search
// pass raised the gap flag), one workgroup per graph: a graph whose slots
// made fewer records than their bounds has its slots' records moved down to
// their canonical places, slot by slot in word order.  A batch's records are
// all read before any is written, and records only move to lower indices,
// so nothing is overwritten before it is read.
constexpr uint32_t kRepackThreads = 256;

__global__ __launch_bounds__(kRepackThreads) void k_repack(RepackArgs a) {
  __shared__ uint32_t s_part[kRepackThreads / 64];
  const uint32_t g = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const DevGraph& G = a.graphs[g];
  auto slot_bound = [&](uint32_t slot) {
    uint32_t b = 0;
    for (uint32_t q = 0; q < kSubsPerSlot; ++q) b += a.sub_count[(uint64_t)slot * kSubsPerSlot + q] >> 16;
    return b;
  };
  uint32_t gap = 0;
  for (uint32_t j = tid; j < G.tile_cap; j += kRepackThreads) gap |= slot_bound(G.tile_base + j) != a.slot_rec[G.tile_base + j];
  gap = __ballot(gap != 0) != 0;
  if (lane == 0) s_part[wave] = gap;
  __syncthreads();
  gap = 0;
#pragma unroll
  for (uint32_t w = 0; w < kRepackThreads / 64; ++w) gap |= s_part[w];
  if (!gap) return;  // uniform over the workgroup
  fdy_override* ovr = a.ovr + (G.word_base >> a.rec_shift);
  uint32_t bound_at = 0, rec_at = 0;  // the slot's place by the bounds, and its canonical place
  for (uint32_t k = 0; k < G.tile_cap; ++k) {
    const uint32_t slot = G.tile_base + k;
    const uint32_t c = a.slot_rec[slot];
    if (bound_at != rec_at) {
      for (uint32_t b0 = 0; b0 < c; b0 += kRepackThreads) {
        const uint32_t i = b0 + tid;
        fdy_override o{};
        if (i < c) o = ovr[bound_at + i];
        __syncthreads();
        if (i < c) ovr[rec_at + i] = o;
        __syncthreads();
      }
    }
    bound_at += slot_bound(slot);
    rec_at += c;
  }
}

// ---- switch --------------------------------------------------------------

// The first kSwitchChunkBlocks(n_cur) blocks restore the template's words
// under the current graph's overrides that the target does not override;
// the other blocks write the target's overrides and the node sources.  The
// two sets of words are disjoint, so the parts need no ordering.
//
// A restoring block takes 256 consecutive current records (sorted by word)
// and decides "does the target override this word too?" in LDS: it loads
// every kSwitchSample-th word of the target's records, finds from them the
// index range of target records whose words can fall inside its own word
// range, loads those words, and binary-searches them per record.  That is
// three rounds of loads per block where a binary search of the target's
// records in global memory took one round per step (16 at 40 thousand
// records: 8.6 us per switch on the 1024-graph archive).  Lists too long for
// the LDS arrays search in global memory as before.
constexpr uint32_t kSwitchThreads = 256;
constexpr uint32_t kSwitchSample = 256;   // target records per sample
constexpr uint32_t kSwitchSamples = 1024; // samples held in LDS (targets up to 256 K records)
constexpr uint32_t kSwitchSeg = 2048;     // target words held in LDS per block

__device__ inline uint64_t switch_chunk_blocks(uint64_t n_cur) { return (n_cur + kSwitchThreads - 1) / kSwitchThreads; }

__device__ __forceinline__ void switch_block(const SwitchArgs& a, uint32_t blk, uint32_t nblk, uint32_t* s_sample,
                                             uint32_t* s_seg) {
  const uint32_t tid = threadIdx.x;
  const uint64_t cb = switch_chunk_blocks(a.n_cur);
  if (blk < cb) {
    const uint64_t i = (uint64_t)blk * kSwitchThreads + tid;
    const bool have = i < a.n_cur;
    fdy_override r{};
    if (have) r = a.ovr_cur[i];
    // The template's word, loaded now so that its wait overlaps the search's.
    const uint64_t tv = have ? a.tmpl_image[r.word] : 0;
    const uint64_t ns = (a.n_new + kSwitchSample - 1) / kSwitchSample;
    const bool staged = ns <= kSwitchSamples;
    if (staged)
      for (uint64_t k = tid; k < ns; k += kSwitchThreads) s_sample[k] = a.ovr_new[k * kSwitchSample].word;
    // The block's word range: its first and last records' words.
    const uint64_t last = min(a.n_cur, (uint64_t)(blk + 1) * kSwitchThreads) - 1;
    const uint32_t w_a = a.ovr_cur[(uint64_t)blk * kSwitchThreads].word, w_b = a.ovr_cur[last].word;
    __syncthreads();
    // Target records with words in [w_a, w_b] lie in [beg, end).
    uint64_t beg = 0, end = a.n_new;
    if (staged) {
      uint32_t below = 0, upto = 0;  // samples < w_a, samples <= w_b
      for (uint64_t k = tid; k < ns; k += kSwitchThreads) {
        below += s_sample[k] < w_a;
        upto += s_sample[k] <= w_b;
      }
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) {
        below += __shfl_down(below, (unsigned)d, 64);
        upto += __shfl_down(upto, (unsigned)d, 64);
      }
      __shared__ uint32_t s_cnt[2][kSwitchThreads / 64];
      if ((tid & 63) == 0) {
        s_cnt[0][tid >> 6] = below;
        s_cnt[1][tid >> 6] = upto;
      }
      __syncthreads();
      below = upto = 0;
#pragma unroll
      for (uint32_t w = 0; w < kSwitchThreads / 64; ++w) {
        below += s_cnt[0][w];
        upto += s_cnt[1][w];
      }
      beg = (uint64_t)(below ? below - 1 : 0) * kSwitchSample;
      end = min(a.n_new, (uint64_t)upto * kSwitchSample);
      if (end < beg) end = beg;
    }
    const bool seg = staged && end - beg <= kSwitchSeg;
    if (seg)
      for (uint64_t k = beg + tid; k < end; k += kSwitchThreads) s_seg[k - beg] = a.ovr_new[k].word;
    __syncthreads();
    if (have) {
      bool also;
      if (seg) {
        uint32_t lo = 0, hi = (uint32_t)(end - beg);
        while (lo < hi) {
          const uint32_t mid = (lo + hi) >> 1;
          if (s_seg[mid] < r.word) lo = mid + 1;
          else hi = mid;
        }
        also = lo < end - beg && s_seg[lo] == r.word;
      } else {
        uint64_t lo = beg, hi = end;
        while (lo < hi) {
          const uint64_t mid = (lo + hi) >> 1;
          if (a.ovr_new[mid].word < r.word) lo = mid + 1;
          else hi = mid;
        }
        also = lo < end && a.ovr_new[lo].word == r.word;
      }
      if (!also) a.live[r.word] = tv;
      if (a.dirty) a.dirty[r.node] = 1;
    }
    return;
  }
  const uint64_t lim = a.n_new > a.num_nodes ? a.n_new : a.num_nodes;
  const uint64_t nb = nblk - cb;
  for (uint64_t i = (uint64_t)(blk - cb) * kSwitchThreads + tid; i < lim; i += nb * kSwitchThreads) {
    if (i < a.n_new) {
      const fdy_override r = a.ovr_new[i];
      a.live[r.word] = r.value;
      if (a.dirty) a.dirty[r.node] = 1;
    }
    if (i < a.num_nodes) {
      const uint32_t fn = a.flags_new[i];
      a.live_src[i] = (fn & (FDY_NODE_LAYOUT | FDY_NODE_DESC)) ? a.target : a.tmpl;
      // A node whose descriptor or layout comes from the current or the
      // target graph is re-set even without word changes.
      if (a.dirty && ((fn | a.flags_cur[i]) & (FDY_NODE_LAYOUT | FDY_NODE_DESC))) a.dirty[i] = 1;
    }
  }
}

__global__ __launch_bounds__(kSwitchThreads) void k_switch(SwitchArgs a) {
  __shared__ uint32_t s_sample[kSwitchSamples];
  __shared__ uint32_t s_seg[kSwitchSeg];
  switch_block(a, blockIdx.x, gridDim.x, s_sample, s_seg);
}

// Switches of different groups in one launch (they touch disjoint live
// images and node sources): switch k takes blocks [end[k-1], end[k]).
__global__ __launch_bounds__(kSwitchThreads) void k_switch_many(SwitchBatch b) {
  __shared__ uint32_t s_sample[kSwitchSamples];
  __shared__ uint32_t s_seg[kSwitchSeg];
  uint32_t k = 0;
  while (k + 1 < b.n && b.end[k] <= blockIdx.x) ++k;
  const uint32_t first = k ? b.end[k - 1] : 0u;
  switch_block(b.sw[k], blockIdx.x - first, b.end[k] - first, s_sample, s_seg);
}

// ---- interval index, built on the device ------------------------------

// Exclusive prefix over the workgroup of one u64 per thread (kWaves waves);
// *tot gets the sum.
template <uint32_t kWaves>
__device__ inline uint64_t index_block_scan(uint64_t v, uint64_t* s_part, uint64_t* tot) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint64_t y = shfl_up64(x, d);
    if (lane >= (uint32_t)d) x += y;
  }
  if (lane == 63) s_part[wave] = x;
  __syncthreads();
  uint64_t before = 0, sum = 0;
  for (uint32_t w = 0; w < kWaves; ++w) {
    if (w < wave) before += s_part[w];
    sum += s_part[w];
  }
  __syncthreads();  // s_part is free again
  *tot = sum;
  return before + x - v;
}

// Root line b's range and the lines below it (st: this thread's
// 2 * kSubtreeStack words of LDS).
__device__ inline uint64_t index_root(const IndexArgs& a, uint64_t b, uint64_t* s0, uint64_t* i, uint64_t* j,
                                      uint64_t* st) {
  *s0 = root_start(a.lo[0], a.shift, b);
  root_range(a.lo, a.n, *s0, root_start(a.lo[0], a.shift, b + 1), i, j);
  return subtree_lines(*j - *i + 1, st, st + kSubtreeStack);
}

// Pass 1, one thread per root line: the lines below each workgroup's roots.
__global__ __launch_bounds__(kIndexThreads) void k_index_count(IndexArgs a) {
  __shared__ uint64_t s_part[kIndexThreads / 64];
  __shared__ uint64_t s_st[kIndexThreads][2 * kSubtreeStack];
  const uint64_t b = (uint64_t)blockIdx.x * kIndexThreads + threadIdx.x;
  uint64_t sub = 0;
  if (b < a.nb) {
    uint64_t s0, i, j;
    sub = index_root(a, b, &s0, &i, &j, s_st[threadIdx.x]);
  }
  uint64_t tot;
  (void)index_block_scan<kIndexThreads / 64>(sub, s_part, &tot);
  if (threadIdx.x == 0) a.block_sum[blockIdx.x] = tot;
}

// Pass 2, one workgroup of kIndexScanThreads: each root workgroup's first
// line below its roots (after the nb root lines), and the index's line
// count.  Each thread sums, then rewrites, a contiguous run of the counts.
constexpr uint32_t kIndexScanThreads = 1024;
__global__ __launch_bounds__(kIndexScanThreads) void k_index_scan(IndexArgs a, uint64_t nblocks) {
  __shared__ uint64_t s_part[kIndexScanThreads / 64];
  const uint64_t per = (nblocks + kIndexScanThreads - 1) / kIndexScanThreads;
  const uint64_t k0 = min(nblocks, (uint64_t)threadIdx.x * per), k1 = min(nblocks, k0 + per);
  uint64_t v = 0;
#pragma unroll 8
  for (uint64_t k = k0; k < k1; ++k) v += a.block_sum[k];
  uint64_t tot;
  uint64_t at = a.nb + index_block_scan<kIndexScanThreads / 64>(v, s_part, &tot);
  for (uint64_t k = k0; k < k1; ++k) {
    const uint64_t x = a.block_sum[k];
    a.block_sum[k] = at;
    at += x;
  }
  if (threadIdx.x == 0) *a.total = a.nb + tot;
}

// Pass 3, one thread per root line: the root line and the lines below it.
__global__ __launch_bounds__(kIndexThreads) void k_index_place(IndexArgs a) {
  __shared__ uint64_t s_part[kIndexThreads / 64];
  __shared__ uint64_t s_st[kIndexThreads][2 * kSubtreeStack];
  const uint64_t b = (uint64_t)blockIdx.x * kIndexThreads + threadIdx.x;
  uint64_t sub = 0, s0 = 0, i = 0, j = 0;
  if (b < a.nb) sub = index_root(a, b, &s0, &i, &j, s_st[threadIdx.x]);
  uint64_t tot;
  const uint64_t base = a.block_sum[blockIdx.x] + index_block_scan<kIndexThreads / 64>(sub, s_part, &tot);
  if (b < a.nb) place_root(a.line, b, s0, i, j, a.lo, a.hi, a.nlo, base);
}

// ---- host mirror of a group graph's live image ---------------------------

// Block b covers nodes [64b, 64b + 64): the first wave moves their marks to
// the host as one 64-byte line, then each wave copies whole dirty nodes, so
// the words reach host memory as full lines rather than as single words.
__global__ __launch_bounds__(256) void k_mirror(MirrorArgs a) {
  __shared__ uint8_t s_dirty[kMirrorNodes];
  const uint32_t n0 = blockIdx.x * kMirrorNodes;
  const uint32_t cnt = min(kMirrorNodes, a.num_nodes - n0);
  if (threadIdx.x < cnt) {
    const uint32_t n = n0 + threadIdx.x;
    const uint8_t d = a.all ? 1 : a.dirty[n];
    s_dirty[threadIdx.x] = d;
    a.h_dirty[n] = d;
    if (d) a.dirty[n] = 0;
  }
  __syncthreads();
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (uint32_t i = wave; i < cnt; i += 4) {
    if (!s_dirty[i]) continue;
    const NodeDesc d = a.desc[n0 + i];
    for (uint32_t w = lane; w < d.nwords; w += 64) a.h_live[d.gword + w] = a.live[d.gword + w];
  }
}

// ---- fill (memset nodes of restored graphs) -----------------------------

// Row r starts at dst + r * pitch.  Its bytes up to the first 16-byte
// boundary and after the last one are stored singly; the rest as 16-byte
// vectors of the pattern rotated to the phase of the row offset.
__global__ __launch_bounds__(kFillThreads) void k_fill(FillArgs a) {
  const uint64_t tid = (uint64_t)blockIdx.x * kFillThreads + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * kFillThreads;
  for (uint64_t r = blockIdx.y; r < a.height; r += gridDim.y) {
    uint8_t* row = a.dst + r * a.pitch;
    const uint64_t mis = (16 - ((uintptr_t)row & 15)) & 15;
    const uint64_t head = mis < a.row_bytes ? mis : a.row_bytes;
    const uint64_t nvec = (a.row_bytes - head) >> 4;
    const uint64_t tail = head + (nvec << 4);
    const uint32_t sh = 8 * (uint32_t)(head & 3);
    const uint32_t w = sh ? (a.pattern >> sh) | (a.pattern << (32 - sh)) : a.pattern;
    const uint4 q = make_uint4(w, w, w, w);
    for (uint64_t v = tid; v < nvec; v += stride) *reinterpret_cast<uint4*>(row + head + (v << 4)) = q;
    const uint64_t singles = head + (a.row_bytes - tail);
    for (uint64_t k = tid; k < singles; k += stride) {
      const uint64_t off = k < head ? k : tail + (k - head);
      row[off] = (uint8_t)(a.pattern >> (8 * (off & 3)));
    }
  }
}

// ---- standalone relocation ---------------------------------------------

// `in` and `out` may be the same array: each word is read and then written
// by one thread, so in-place relocation needs no ordering between threads.
// Standalone relocation of packed words.  Each thread owns kRelocPairs
// 16-byte pairs per chunk (coalesced across the workgroup).  The words
// inside the table's range (the pointers: 40% on the relocation-heavy
// workload) are compacted per wave in LDS and searched kRelocSearch per lane
// in lockstep, then read back in place, so no lane holds index lines for
// words that need no search: 90 VGPRs and five waves per SIMD, where
// searching every word in batches of four took 148 VGPRs and three.
constexpr uint32_t kRelocSearch = 2;
static_assert((64 * 2 * kRelocPairs) % (64 * kRelocSearch) == 0, "whole search batches per wave");

__global__ __launch_bounds__(kRelocThreads) void k_reloc(RelocDev R, const uint64_t* in, uint64_t* out, uint64_t n,
                                                         int vec) {
  constexpr uint32_t kW = 2 * kRelocPairs;  // words per lane per chunk
  __shared__ uint64_t s_q[kRelocThreads / 64][64 * kW];
  const uint64_t chunk = (uint64_t)kRelocThreads * kRelocPairs;
  const uint32_t lane = threadIdx.x & 63;
  const uint64_t lt = (1ull << lane) - 1;
  uint64_t* sq = s_q[threadIdx.x >> 6];
  if (vec) {
    const uint64_t pairs = n / 2;
    const ulonglong2* in2 = reinterpret_cast<const ulonglong2*>(in);
    ulonglong2* out2 = reinterpret_cast<ulonglong2*>(out);
    for (uint64_t c = (uint64_t)blockIdx.x * chunk; c < pairs; c += (uint64_t)gridDim.x * chunk) {
      uint64_t w[kW];
#pragma unroll
      for (uint32_t q = 0; q < kRelocPairs; ++q) {
        const uint64_t p = c + q * kRelocThreads + threadIdx.x;
        const ulonglong2 v = p < pairs ? in2[p] : ulonglong2{0, 0};
        w[2 * q] = v.x;
        w[2 * q + 1] = v.y;
      }
      uint32_t need = 0, rank[kW], cnt = 0;
      if (R.n != 0) {
#pragma unroll
        for (uint32_t j = 0; j < kW; ++j)
          if (w[j] >= R.lo_min && (R.policy ? w[j] <= R.hi_max : w[j] < R.hi_max)) need |= 1u << j;
      }
#pragma unroll
      for (uint32_t j = 0; j < kW; ++j) {
        const uint64_t mk = __ballot((need >> j) & 1);
        rank[j] = cnt + (uint32_t)__popcll(mk & lt);
        if ((need >> j) & 1) sq[rank[j]] = w[j];
        cnt += (uint32_t)__popcll(mk);
      }
      // The wave's own LDS words: its writes precede its reads in program order.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      for (uint32_t b = 0; b < cnt; b += 64 * kRelocSearch) {
        uint64_t x[kRelocSearch], y[kRelocSearch];
        uint32_t mm = 0;
#pragma unroll
        for (uint32_t k = 0; k < kRelocSearch; ++k) {
          const uint32_t i = b + 64 * k + lane;
          x[k] = i < cnt ? sq[i] : 0;
          mm |= (i < cnt ? 1u : 0u) << k;
        }
        reloc_batch<kRelocSearch>(R, x, y, mm);
#pragma unroll
        for (uint32_t k = 0; k < kRelocSearch; ++k) {
          const uint32_t i = b + 64 * k + lane;
          if (i < cnt) sq[i] = y[k];
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (uint32_t j = 0; j < kW; ++j)
        if ((need >> j) & 1) w[j] = sq[rank[j]];
#pragma unroll
      for (uint32_t q = 0; q < kRelocPairs; ++q) {
        const uint64_t p = c + q * kRelocThreads + threadIdx.x;
        if (p < pairs) out2[p] = ulonglong2{w[2 * q], w[2 * q + 1]};
      }
      // The next chunk's compaction overwrites this wave's LDS words only
      // after every lane has read its own back (program order in the wave).
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && (n & 1)) out[n - 1] = reloc_word(R, in[n - 1]);
  } else {
    const uint64_t stride = (uint64_t)gridDim.x * kRelocThreads;
    for (uint64_t p = (uint64_t)blockIdx.x * kRelocThreads + threadIdx.x; p < n; p += stride)
      out[p] = reloc_word(R, in[p]);
  }
}

}  // namespace

hipError_t launch_group(const RestoreArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_group, dim3(a.num_graphs), dim3(kGroupThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_node(const RestoreArgs& a, hipStream_t s) {
  if (a.num_chunks) {
    hipLaunchKernelGGL(k_node_a, dim3(a.num_chunks), dim3(kNodeChunk), 0, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const uint32_t unit_blocks = (a.num_units + kNodeThreads / 64 - 1) / (kNodeThreads / 64);
  hipLaunchKernelGGL(k_node_b, dim3(a.num_graphs + unit_blocks), dim3(kNodeThreads), 0, s, a);
  return hipGetLastError();
}

// Templates first: the other graphs read their relocated words.
hipError_t launch_diff_templates(const RestoreArgs& a, hipStream_t s) {
  if ((uint64_t)a.num_slots >= kTWideSlotsPerGraph * a.num_graphs) {
    const uint32_t tgrid = (uint32_t)std::min<uint64_t>((uint64_t)a.num_slots * t_units_per_tile<8>(), 2048);
    hipLaunchKernelGGL(k_diff_t<8>, dim3(tgrid), dim3(kTThreads), 0, s, a);
  } else {
    const uint32_t tgrid = (uint32_t)std::min<uint64_t>((uint64_t)a.num_slots * t_units_per_tile<4>(), 2048);
    hipLaunchKernelGGL(k_diff_t<4>, dim3(tgrid), dim3(kTThreads), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_diff_members(const RestoreArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_diff_m, dim3(a.num_slots * kMSplit), dim3(kMThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_diff_search(const RestoreArgs& a, hipStream_t s) {
  const uint32_t sgrid = (a.num_slots + kSThreads / 64 - 1) / (kSThreads / 64);
  hipLaunchKernelGGL(k_diff_s, dim3(sgrid), dim3(kSThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_repack(const RepackArgs& a, hipStream_t s) {
  if (a.num_graphs == 0) return hipSuccess;
  hipLaunchKernelGGL(k_repack, dim3(a.num_graphs), dim3(kRepackThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_switch(const SwitchArgs& a, hipStream_t s) {
  const uint64_t cb = (a.n_cur + kSwitchThreads - 1) / kSwitchThreads;  // switch_chunk_blocks
  const uint64_t lim = a.n_new > a.num_nodes ? a.n_new : a.num_nodes;
  uint64_t wb = (lim + kSwitchThreads - 1) / kSwitchThreads;
  if (wb > 2048) wb = 2048;
  if (wb == 0) wb = 1;
  if (cb + wb > 0x7FFFFFFFull) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_switch, dim3((uint32_t)(cb + wb)), dim3(kSwitchThreads), 0, s, a);
  return hipGetLastError();
}

uint32_t switch_blocks(const SwitchArgs& a) {
  const uint64_t cb = (a.n_cur + kSwitchThreads - 1) / kSwitchThreads;  // switch_chunk_blocks
  const uint64_t lim = a.n_new > a.num_nodes ? a.n_new : a.num_nodes;
  uint64_t wb = (lim + kSwitchThreads - 1) / kSwitchThreads;
  if (wb > 2048) wb = 2048;
  if (wb == 0) wb = 1;
  return (uint32_t)std::min<uint64_t>(cb + wb, 0x7FFFFFFFull);
}

hipError_t launch_switch_many(const SwitchBatch& b, hipStream_t s) {
  if (b.n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_switch_many, dim3(b.end[b.n - 1]), dim3(kSwitchThreads), 0, s, b);
  return hipGetLastError();
}

hipError_t launch_mirror(const MirrorArgs& a, hipStream_t s) {
  if (a.num_nodes == 0) return hipSuccess;
  hipLaunchKernelGGL(k_mirror, dim3((a.num_nodes + kMirrorNodes - 1) / kMirrorNodes), dim3(256), 0, s, a);
  return hipGetLastError();
}

void* fill_kernel() { return reinterpret_cast<void*>(&k_fill); }

dim3 fill_grid(const FillArgs& f) {
  const uint64_t vec = (f.row_bytes >> 4) + 1;
  const uint64_t x = std::min<uint64_t>((vec + kFillThreads - 1) / kFillThreads, 1024);
  const uint64_t y = std::min<uint64_t>(std::max<uint64_t>(f.height, 1), 65535);
  return dim3((uint32_t)std::max<uint64_t>(x, 1), (uint32_t)y);
}

hipError_t launch_index_count(const IndexArgs& a, hipStream_t s) {
  const uint64_t nblocks = (a.nb + kIndexThreads - 1) / kIndexThreads;
  if (nblocks == 0 || nblocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_index_count, dim3((uint32_t)nblocks), dim3(kIndexThreads), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_index_scan, dim3(1), dim3(kIndexScanThreads), 0, s, a, nblocks);
  return hipGetLastError();
}

hipError_t launch_index_place(const IndexArgs& a, hipStream_t s) {
  const uint64_t nblocks = (a.nb + kIndexThreads - 1) / kIndexThreads;
  if (nblocks == 0 || nblocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_index_place, dim3((uint32_t)nblocks), dim3(kIndexThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_reloc_words(const RelocDev& r, const uint64_t* in, uint64_t* out, uint64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const int vec = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  const uint64_t per_block = (uint64_t)kRelocThreads * (vec ? 2 * kRelocPairs : 1);
  uint64_t blocks = (n + per_block - 1) / per_block;
  if (blocks > 256 * 32) blocks = 256 * 32;
  hipLaunchKernelGGL(k_reloc, dim3((uint32_t)blocks), dim3(kRelocThreads), 0, s, r, in, out, n, vec);
  return hipGetLastError();
}

}  // namespace fdy
