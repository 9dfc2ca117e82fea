// kernels.hip -- the restore kernels for gfx950 (wave64, 160 KB LDS per CU).
//
//   k_hash    one workgroup per graph: CRC-64/XZ of the saved topology key and
//             of the dependency table, as a block-wide segmented CRC (each
//             lane absorbs 64 bytes, lanes are joined by a combine tree whose
//             multipliers are constants applied through nibble tables in LDS).
//   k_group   template_of[g] = lowest graph with the same key bytes (found by
//             key digest and length, then compared byte for byte).
//   k_node_a  one workgroup per 256-node chunk of a graph: per node, the
//             param layout, the compare against the template's node,
//             memset/memcpy pointer relocation, the node-type and kernel-entry
//             records (raw CRC per chunk) and the node descriptor.
//   k_node_b  one workgroup per graph: chunk CRCs joined into the
//             digests, word offsets by block scans, the diff-tile -> first-node
//             table, ragged-word sources, slot descriptors.
//   k_diff_t  the template graphs' words, relocated through a bucket-indexed
//             interval search into R and the live image (1024-word units).
//   k_diff_m  eight workgroups per 4096-word tile of every other graph: coalesced
//             8-byte loads of the graph's and the template's words, the
//             template's relocated word reused where the raw words are equal,
//             lockstep batched searches for the rest, the relocated image
//             store, and per-wave ballot compaction of the differing words
//             into override record regions.
//   k_count   override records per graph.
//   k_compact record regions -> the dense override array in canonical order
//             (offsets from the per-graph record counts),
//             completing each record's node and template word index.
//   k_switch  override scatter for one graph switch.
//   k_mirror  dirty nodes' live words -> a group graph's host mirror.
//   k_fill    memset node of a restored graph, as a kernel node.
//   k_reloc   streaming relocation of packed words.
#include "kernels.h"

namespace fdy {
namespace {

constexpr uint32_t kHashThreads = 1024;
constexpr uint32_t kNodeThreads = 1024;
constexpr uint32_t kGroupSteps = 8;  // 64-candidate steps whose loads are issued together
constexpr uint32_t kRelocThreads = 256;
constexpr uint32_t kRelocPairs = 4;  // 16-byte word pairs per thread per iteration
constexpr uint32_t kRelocBatch = 4;  // words searched in lockstep (8 and 2 measured no faster)
static_assert(kRelocBatch % 2 == 0 && (2 * kRelocPairs) % kRelocBatch == 0, "whole pairs per batch");

__device__ inline uint64_t shfl_down64(uint64_t v, int d) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl_down(lo, (unsigned)d, 64);
  hi = __shfl_down(hi, (unsigned)d, 64);
  return ((uint64_t)hi << 32) | lo;
}

__device__ inline uint32_t shfl_up32(uint32_t v, int d) { return __shfl_up(v, (unsigned)d, 64); }

// The 8 bytes [b0, b0+8) of the L-byte stream at p (8-aligned), with bytes
// outside [0, L) read as zero.
__device__ inline uint64_t stream_window(const uint8_t* p, uint64_t L, int64_t b0) {
  const int64_t q = b0 >> 3;
  const uint32_t sh = (uint32_t)(b0 & 7);
  auto word = [&](int64_t qi) -> uint64_t {
    if (qi < 0 || (uint64_t)qi * 8 >= L) return 0;
    uint64_t v = *reinterpret_cast<const uint64_t*>(p + qi * 8);
    uint64_t rem = L - (uint64_t)qi * 8;
    if (rem < 8) v &= (1ull << (8 * rem)) - 1;
    return v;
  };
  uint64_t w0 = word(q);
  if (sh == 0) return w0;
  return (w0 >> (8 * sh)) | (word(q + 1) << (64 - 8 * sh));
}

// XOR of two values over the block (blockDim.x a multiple of 64); valid in
// thread 0.  s_wave is free again when it returns.
__device__ void block_xor2(uint64_t& x, uint64_t& y, uint64_t (*s_wave)[2]) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    x ^= shfl_down64(x, d);
    y ^= shfl_down64(y, d);
  }
  if (lane == 0) {
    s_wave[wave][0] = x;
    s_wave[wave][1] = y;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    for (uint32_t w = 1; w < nw; ++w) {
      x ^= s_wave[w][0];
      y ^= s_wave[w][1];
    }
  __syncthreads();
}

// One of the two byte streams hashed together by block_crc_bytes2.
struct HashStream {
  const uint8_t* p;
  uint64_t L;
  uint64_t fin;  // the stream's finishing term
};

// CRC-64/XZ of two byte streams at once (their loads in flight together, one
// reduction for both).  Each lane absorbs 64 consecutive bytes of a stream
// (eight slicing steps); lane i's raw CRC times x^(8*64*(1023-i)) is its
// share of the 64 KB chunk's raw CRC (crc(A || B) = crc(A) * x^(8|B|) xor
// crc(B)), XOR-joined over the block; chunks are joined by the 64 KB
// multiplier.  Each stream is front-padded with zeros to whole chunks
// (leading zeros leave a zero-initialised register at zero; `fin` adds the
// effect of the all-ones initial value).  Results in thread 0.
__device__ void block_crc_bytes2(const HashStream& s0, const HashStream& s1, const uint64_t (*slice)[256],
                                 const uint64_t (*chunk_mul)[16], const uint64_t* pos64, uint64_t (*s_wave)[2],
                                 uint64_t* out0, uint64_t* out1) {
  constexpr uint64_t kLane = 64;
  constexpr uint64_t kChunk = kHashThreads * kLane;
  static_assert(kHashThreads == kPosLanes, "one position multiplier per lane");
  const uint64_t pad0 = (kChunk - s0.L % kChunk) % kChunk, pad1 = (kChunk - s1.L % kChunk) % kChunk;
  const uint64_t n0 = (s0.L + pad0) / kChunk, n1 = (s1.L + pad1) / kChunk;
  const uint64_t m = pos64[threadIdx.x];
  uint64_t acc0 = 0, acc1 = 0;
  for (uint64_t c = 0; c < n0 || c < n1; ++c) {
    const int64_t b0 = (int64_t)(c * kChunk + kLane * threadIdx.x) - (int64_t)pad0;
    const int64_t b1 = (int64_t)(c * kChunk + kLane * threadIdx.x) - (int64_t)pad1;
    uint64_t v0[kLane / 8], v1[kLane / 8];
#pragma unroll
    for (uint32_t q = 0; q < kLane / 8; ++q) {
      v0[q] = c < n0 ? stream_window(s0.p, s0.L, b0 + 8 * q) : 0;
      v1[q] = c < n1 ? stream_window(s1.p, s1.L, b1 + 8 * q) : 0;
    }
    uint64_t z0 = 0, z1 = 0;
#pragma unroll
    for (uint32_t q = 0; q < kLane / 8; ++q) {
      z0 = crc_slice8(slice, z0, v0[q]);
      z1 = crc_slice8(slice, z1, v1[q]);
    }
    z0 = z0 ? gf2_mulmod(m, z0) : 0;
    z1 = z1 ? gf2_mulmod(m, z1) : 0;
    block_xor2(z0, z1, s_wave);
    if (threadIdx.x == 0) {
      if (c < n0) acc0 = nibble_mul(chunk_mul, acc0) ^ z0;
      if (c < n1) acc1 = nibble_mul(chunk_mul, acc1) ^ z1;
    }
  }
  *out0 = acc0 ^ s0.fin;
  *out1 = acc1 ^ s1.fin;
}

__global__ __launch_bounds__(kHashThreads) void k_hash(RestoreArgs a) {
  __shared__ uint64_t s_slice[8][256];
  __shared__ uint64_t s_chunk[16][16];  // multiplier x^(8 * 64 KB): joins chunks
  __shared__ uint64_t s_wave[kHashThreads / 64][2];
  stage_words(&s_slice[0][0], &a.cc->slice.t[0][0], 8 * 256);
  stage_words(&s_chunk[0][0], &a.cc->chunk64.t[0][0], 256);
  __syncthreads();
  const uint32_t g = blockIdx.x;
  const DevGraph& G = a.graphs[g];
  const HashStream key{a.img + G.sec_off[FDY_SEC_TOPOLOGY_KEY], G.sec_size[FDY_SEC_TOPOLOGY_KEY], G.crc_fin[0]};
  const HashStream deps{a.img + G.sec_off[FDY_SEC_DEPS], 8ull * G.num_deps, G.crc_fin[1]};
  uint64_t dk, de;
  block_crc_bytes2(key, deps, s_slice, s_chunk, a.cc->pos64, s_wave, &dk, &de);
  if (threadIdx.x == 0) {
    a.digests[4ull * g + 0] = dk;
    a.digests[4ull * g + 1] = de;
  }
}

// template_of[i] = the lowest j <= i whose saved key has the same bytes
// (the reference partitions by exact key string, csrc/CUDAGraphParallel.cpp:
// 1788-1851): one workgroup per graph.  Its first wave finds the lowest
// candidate with an equal key digest and length (64 candidates per step,
// eight steps' loads in flight at once); the workgroup then compares the
// two keys' bytes, and on a digest collision (equal digest and length,
// other bytes) flags the graph and goes on scanning past the candidate.
constexpr uint32_t kGroupThreads = 256;

__global__ __launch_bounds__(kGroupThreads) void k_group(RestoreArgs a) {
  __shared__ uint32_t s_found, s_differs;
  const uint32_t i = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  if (i == 0 && tid == 0) *a.tslot_count = 0;  // the node pass lists template slots here
  if (a.explicit_template) {
    if (tid == 0) {
      a.template_of[i] = a.explicit_template[i];
      a.status[i] = 0;
    }
    return;
  }
  const DevGraph& Gi = a.graphs[i];
  const uint64_t di = a.digests[4ull * i];
  const uint64_t L = Gi.sec_size[FDY_SEC_TOPOLOGY_KEY];
  const uint8_t* pi = a.img + Gi.sec_off[FDY_SEC_TOPOLOGY_KEY];
  uint32_t from = 0, status = 0, tmpl = i;
  for (;;) {
    if (tid < 64) {
      uint32_t found = i;
      for (uint32_t base = from; base < i && found == i; base += 64 * kGroupSteps) {
        bool m[kGroupSteps];
#pragma unroll
        for (uint32_t k = 0; k < kGroupSteps; ++k) {
          const uint32_t j = base + 64 * k + lane;
          m[k] = j < i && a.digests[4ull * j] == di && a.graphs[j].sec_size[FDY_SEC_TOPOLOGY_KEY] == L;
        }
#pragma unroll
        for (uint32_t k = 0; k < kGroupSteps; ++k) {
          const uint64_t mk = __ballot(m[k]);
          if (found == i && mk) found = base + 64 * k + (uint32_t)__ffsll((long long)mk) - 1;
        }
      }
      if (tid == 0) {
        s_found = found;
        s_differs = 0;
      }
    }
    __syncthreads();
    const uint32_t j = s_found;
    if (j == i) break;  // uniform over the workgroup
    const uint8_t* pj = a.img + a.graphs[j].sec_off[FDY_SEC_TOPOLOGY_KEY];
    bool d = false;
    for (uint64_t q = tid; q * 8 < L; q += kGroupThreads)
      d |= stream_window(pi, L, (int64_t)q * 8) != stream_window(pj, L, (int64_t)q * 8);
    if (d) s_differs = 1;
    __syncthreads();
    if (!s_differs) {
      tmpl = j;
      break;
    }
    status = FDY_GRAPH_COLLISION;
    from = j + 1;
    __syncthreads();  // every thread has read s_found and s_differs
  }
  if (tid == 0) {
    a.template_of[i] = tmpl;
    a.status[i] = status;  // completed by the node pass
  }
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
  const uint64_t* pp;  // the first kPlaneParams of them, field-major (stride kNodeChunk), or null
};

// A node entry's fields (byte offsets, multiples of 4).  RawEntry reads the
// 168 saved bytes in place; PlaneEntry reads the field-major copy of the
// node table (dword k of every node of a 256-node chunk in one plane), where
// a wave's read of one field is one coalesced access instead of 64 lines.

struct RawEntry {
  const uint8_t* e;
  __device__ uint32_t u32(uint32_t off) const { return f32(e, off); }
  __device__ uint64_t u64(uint32_t off) const { return f64(e, off); }
  __device__ uint8_t type() const { return e[FDY_NODE_OFF_TYPE]; }
};

struct PlaneEntry {
  const uint32_t* p;  // dword 0 of the node
  __device__ uint32_t u32(uint32_t off) const { return p[(off >> 2) * kNodeChunk]; }
  __device__ uint64_t u64(uint32_t off) const { return (uint64_t)u32(off) | ((uint64_t)u32(off + 4) << 32); }
  __device__ uint8_t type() const { return (uint8_t)(u32(FDY_NODE_OFF_TYPE & ~3u) >> (8 * (FDY_NODE_OFF_TYPE & 3))); }
};

// Node n of graph G in the field-major tables: chunks hold 256 nodes, a
// graph's first chunk padded at the front.
struct PlanePos {
  uint64_t chunk;
  uint32_t lane;
};

__device__ inline PlanePos plane_pos(const DevGraph& G, uint32_t n) {
  const uint32_t pad = (kNodeChunk - G.num_nodes % kNodeChunk) % kNodeChunk;
  const uint32_t pos = pad + n;
  return PlanePos{G.chunk_base + pos / kNodeChunk, pos % kNodeChunk};
}

// The param references of kernel node entry e: the name, param-index and
// arg-buffer bounds; an extra-style node's blob.  Per-param nodes are
// completed by scan_params.
template <class E>
__device__ __forceinline__ void side_header(const uint8_t* img, const DevGraph& G, const E& e, Side& s) {
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
__device__ inline void side_param(const DevGraph& G, Side& s, uint32_t j, uint64_t entry, uint64_t& prev,
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

__device__ __forceinline__ void scan_params(const DevGraph& Gg, Side& g, bool with_g, const DevGraph& Gt, Side& t,
                                            bool with_t, bool* same_sizes) {
  const bool wg = with_g && !g.bad && !g.extra;
  const bool wt = with_t && !t.bad && !t.extra;
  const uint32_t ng = wg ? g.num_params : 0, nt = wt ? t.num_params : 0;
  uint64_t prev_g = 0, prev_t = 0, words_g = 0, words_t = 0;
  bool same = ng == nt;
  // The first kPlaneParams entries come from the field-major copy, the rest
  // in place (byte-safe loads: a side's entries may sit at any alignment).
  for (uint32_t jb = 0; jb < max(ng, nt); jb += kParamBatch) {
    uint64_t eg[kParamBatch], et[kParamBatch];
#pragma unroll
    for (uint32_t k = 0; k < kParamBatch; ++k) {
      const uint32_t j = jb + k;
      eg[k] = j < ng ? (g.pp && j < kPlaneParams ? g.pp[(uint64_t)j * kNodeChunk] : ld_u64(g.pidx + 8ull * j)) : 0;
      et[k] = j < nt ? (t.pp && j < kPlaneParams ? t.pp[(uint64_t)j * kNodeChunk] : ld_u64(t.pidx + 8ull * j)) : 0;
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
template <class E>
__device__ __forceinline__ bool names_equal(const Strings& A, const E& ea, const Strings& B, const E& eb) {
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

template <class E>
__device__ __forceinline__ bool u64_range_differs(const E& a, const E& b, uint32_t off, uint32_t n) {
  bool d = false;
  for (uint32_t i = 0; i < n; i += 8) d |= a.u64(off + i) != b.u64(off + i);
  return d;
}

// Does node entry ea (strings A, common attrs ca) differ in its descriptor
// from eb (strings B, common attrs cb)?  pa/pb: relocated pointers.
// same_ctx: both graphs have byte-identical string sections and common
// attrs, so equal entry bytes [8, 128) (launch config, function hash, name
// offset and length, function attrs, per-node attrs) mean equal descriptors.
template <class E>
__device__ __forceinline__ bool desc_differs(const Strings& A, const uint8_t* ca, const E& ea, const Strings& B,
                             const uint8_t* cb, const E& eb, uint64_t pa0, uint64_t pa1, uint64_t pb0,
                             uint64_t pb1, bool same_ctx) {
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

// Exclusive block-wide prefix sum of 256 u32 values; *total gets the sum.
__device__ uint32_t block_excl_scan(uint32_t v, uint32_t* s_tmp, uint32_t* total) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t y = shfl_up32(x, d);
    if (lane >= (uint32_t)d) x += y;
  }
  if (lane == 63) s_tmp[wave] = x;
  __syncthreads();
  uint32_t before = 0, sum = 0;
  for (uint32_t w = 0; w < blockDim.x / 64; ++w) {
    uint32_t t = s_tmp[w];
    if (w < wave) before += t;
    sum += t;
  }
  __syncthreads();
  *total = sum;
  return before + x - v;
}

__device__ void write_aux(const uint8_t* img, const DevGraph& G, const uint8_t* e, const Side& s, uint64_t* aux,
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

// The field-major node table: thread l of chunk c copies the 42 dwords of
// node (c - chunk_base) * 256 + l - pad of its graph into plane k at
// planes[(c * 42 + k) * 256 + l]; padding lanes write zeros.
__global__ __launch_bounds__(kNodeChunk) void k_planes(const uint8_t* img, const DevGraph* graphs,
                                                       const uint32_t* chunk_graph, uint32_t* planes,
                                                       uint64_t* pplanes) {
  const uint32_t c = blockIdx.x, l = threadIdx.x;
  const DevGraph& G = graphs[chunk_graph[c]];
  const uint32_t N = G.num_nodes;
  const uint32_t pad = (kNodeChunk - N % kNodeChunk) % kNodeChunk;
  const int64_t n = (int64_t)(c - G.chunk_base) * kNodeChunk + l - pad;
  uint32_t v[kEntryDwords];
  if (n >= 0 && n < (int64_t)N) {
    const uint32_t* e = reinterpret_cast<const uint32_t*>(img + G.sec_off[FDY_SEC_NODES] + 168ull * (uint64_t)n);
#pragma unroll
    for (uint32_t k = 0; k < kEntryDwords; ++k) v[k] = e[k];
  } else {
#pragma unroll
    for (uint32_t k = 0; k < kEntryDwords; ++k) v[k] = 0;
  }
  uint32_t* out = planes + (uint64_t)c * kEntryDwords * kNodeChunk + l;
#pragma unroll
  for (uint32_t k = 0; k < kEntryDwords; ++k) out[k * kNodeChunk] = v[k];
  // The first kPlaneParams param entries of a per-param kernel node whose
  // entries lie inside the param-index section (others are never read).
  uint32_t np = 0;
  const uint8_t* pidx = nullptr;
  if (n >= 0 && n < (int64_t)N && (v[FDY_NODE_OFF_TYPE / 4] >> (8 * (FDY_NODE_OFF_TYPE % 4)) & 0xFF) == FDY_NODE_KERNEL) {
    const uint32_t pio = v[FDY_KOFF_PARAM_INDEX / 4], num = v[FDY_KOFF_NUM_PARAMS / 4];
    if (v[FDY_KOFF_ARG_OFFSET / 4] == FDY_NO_ARG_BUFFER && (uint64_t)pio + 8ull * num <= G.sec_size[FDY_SEC_PARAM_INDEX]) {
      np = min(num, kPlaneParams);
      pidx = img + G.sec_off[FDY_SEC_PARAM_INDEX] + pio;
    }
  }
  uint64_t* pout = pplanes + (uint64_t)c * kPlaneParams * kNodeChunk + l;
#pragma unroll
  for (uint32_t j = 0; j < kPlaneParams; ++j) pout[j * kNodeChunk] = j < np ? ld_u64(pidx + 8ull * j) : 0;
}

// The node pass runs in two parts.
//
// Part A, k_node_a: one workgroup of kNodeChunk threads per chunk of a
// graph's nodes, one node per thread.  A graph's chunks end at its last
// node, so its first chunk is padded at the front (leading zero records
// leave a zero-initialised CRC at zero).  Per node: type, params and their
// bounds, layout and descriptor against the template's node, relocated
// memset/memcpy pointers, the node-type and kernel-entry records; written
// to the node descriptor with the node's word counts in place of its word
// offsets.  Per chunk: the raw CRCs of the two record streams, word and
// param-byte totals, status bits.
//
// Part B, k_node_b: one workgroup per graph: the template's key bytes, the
// chunk CRCs shifted to their place, word offsets by block scans, the
// tile -> first-node table, ragged-word sources, flatness, status, digests
// and the slot descriptors of the diff pass.

// Five waves per SIMD: held to 96 VGPRs it spills 12 bytes per lane and
// still beats four waves per SIMD at 99 VGPRs (73 -> 68 us, decode-style).
__global__ __launch_bounds__(kNodeChunk, 5) void k_node_a(RestoreArgs a) {
  constexpr uint32_t kStrStage = 2048; // string sections up to this size are staged in LDS
  static_assert(kNodeChunk == kPosRecords, "one position multiplier per record of a chunk");
  __shared__ uint64_t s_slice[8][256];
  __shared__ uint64_t s_str[2][kStrStage / 8];
  __shared__ uint64_t s_common[2][7];
  // The chunk's node-type and kernel-entry records, eight to a row; the odd
  // row length keeps a half-wave's reads of eight rows apart in the banks.
  __shared__ uint64_t s_rec[2][kNodeChunk / 8][17];
  __shared__ uint32_t s_diff;
  __shared__ uint32_t s_sum[2][kNodeChunk / 64];
  __shared__ uint64_t s_pb[kNodeChunk / 64];
  __shared__ uint32_t s_status;

  const uint32_t chunk = blockIdx.x, tid = threadIdx.x;
  const uint32_t g = a.chunk_graph[chunk];
  const uint32_t t = a.template_of[g];
  const bool is_t = t == g;
  const DevGraph& Gg = a.graphs[g];
  const DevGraph& Gt = a.graphs[t];
  const uint32_t N = Gg.num_nodes, NT = Gt.num_nodes;
  const uint8_t* img = a.img;
  if (tid == 0) s_status = 0;

  // CRC tables, the (small) string sections and the common attrs in LDS;
  // sections start 8-byte aligned.
  auto stage_strings = [&](const DevGraph& G, uint64_t* buf) -> Strings {
    Strings S{img + G.sec_off[FDY_SEC_STRINGS], G.sec_size[FDY_SEC_STRINGS]};
    if (S.size <= kStrStage) {
      stage_words(buf, reinterpret_cast<const uint64_t*>(S.p), (uint32_t)((S.size + 7) / 8));
      S.p = reinterpret_cast<const uint8_t*>(buf);
    }
    return S;
  };
  auto stage_common = [&](const DevGraph& G, uint64_t* buf) -> const uint8_t* {
    if (!(G.flags & FDY_HAS_COMMON_ATTRS) || G.sec_size[FDY_SEC_COMMON_ATTRS] < 52) return nullptr;
    if (tid < 7) buf[tid] = reinterpret_cast<const uint64_t*>(img + G.sec_off[FDY_SEC_COMMON_ATTRS])[tid];
    return reinterpret_cast<const uint8_t*>(buf);
  };
  const Strings sg_str = stage_strings(Gg, s_str[0]);
  const Strings st_str = is_t ? sg_str : stage_strings(Gt, s_str[1]);
  const uint8_t* common_g = stage_common(Gg, s_common[0]);
  const uint8_t* common_t = is_t ? common_g : stage_common(Gt, s_common[1]);
  if (tid == 0) s_diff = 0;
  stage_words(&s_slice[0][0], &a.cc->slice.t[0][0], 8 * 256);
  __syncthreads();
  const uint64_t (*slice)[256] = s_slice;
  // Identical string sections and common attrs (both staged in LDS) let the
  // descriptor compare use the entry bytes alone.
  bool same_ctx = false;
  if (!is_t && sg_str.size == st_str.size && sg_str.size <= kStrStage && (common_g == nullptr) == (common_t == nullptr)) {
    const uint32_t nw = (uint32_t)((sg_str.size + 7) / 8);
    uint32_t d = 0;
    for (uint32_t w = tid; w < nw; w += kNodeChunk) d |= s_str[0][w] != s_str[1][w];
    if (common_g && tid < 7) d |= s_common[0][tid] != s_common[1][tid];
    if (d) atomicOr(&s_diff, 1u);
    __syncthreads();
    same_ctx = s_diff == 0;
  }

  const uint32_t pad = (kNodeChunk - N % kNodeChunk) % kNodeChunk;
  const int64_t first = (int64_t)(chunk - Gg.chunk_base) * kNodeChunk - pad;  // node of thread 0
  const int64_t ns = first + tid;
  const bool valid = ns >= 0 && ns < (int64_t)N;
  const uint32_t n = valid ? (uint32_t)ns : 0;
  uint32_t words_g = 0, words_t = 0, flags = 0;
  uint64_t src_g = 0, src_t = 0, p0 = 0, p1 = 0, pbytes = 0;
  uint64_t tw0 = 0, tw1 = 0, kw0 = 0, kw1 = 0;
  const PlaneEntry eg{a.planes + ((uint64_t)chunk * kEntryDwords) * kNodeChunk + tid};
  const PlanePos tpos = plane_pos(Gt, n < NT ? n : 0);
  const PlaneEntry et{a.planes + (tpos.chunk * kEntryDwords) * kNodeChunk + tpos.lane};
  if (valid) {
    const uint8_t type = eg.type();
    const bool has_t = !is_t && n < NT;
    const uint8_t ttype = has_t ? et.type() : 0xFF;
    tw0 = type;
    Side sg{}, st{};
    bool same_sizes = false;
    if (type == FDY_NODE_KERNEL) {
      // Cluster dims of the recomputed key (csrc/CUDAGraphParallel.cpp:1807-1833).
      uint32_t cx = 0, cy = 0, cz = 0;
      if (eg.u32(FDY_KOFF_KNA_FLAGS) & FDY_KNA_CLUSTER_DIM) {
        cx = eg.u32(80);
        cy = eg.u32(84);
        cz = eg.u32(88);
      }
      if (cx == 0 && common_g && (f32(common_g, 0) & FDY_KNA_CLUSTER_DIM)) {
        cx = f32(common_g, 4);
        cy = f32(common_g, 8);
        cz = f32(common_g, 12);
      }
      if (cx == 0) {
        cx = eg.u32(64);
        cy = eg.u32(68);
        cz = eg.u32(72);
      }
      tw0 |= (uint64_t)cx << 32;
      tw1 = cy | ((uint64_t)cz << 32);
      kw0 = eg.u64(FDY_KOFF_BINARY_HASH);
      kw1 = name_crc(sg_str, eg, slice);
      side_header(img, Gg, eg, sg);
    }
    const bool t_kernel = has_t && ttype == FDY_NODE_KERNEL;
    if (t_kernel) side_header(img, Gt, et, st);
    sg.pp = a.pplanes + ((uint64_t)chunk * kPlaneParams) * kNodeChunk + tid;
    st.pp = a.pplanes + (tpos.chunk * kPlaneParams) * kNodeChunk + tpos.lane;
    scan_params(Gg, sg, type == FDY_NODE_KERNEL, Gt, st, t_kernel, &same_sizes);
    if (type == FDY_NODE_KERNEL) {
      words_g = sg.words;
      pbytes = sg.pbytes;
      src_g = sg.src;
      if (sg.ragged) flags |= FDY_NODE_RAGGED;
      if (sg.bad) flags |= kNodeBad;
    }
    node_pointers(eg, a.reloc, &p0, &p1);
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
      if (desc_differs(sg_str, common_g, eg, st_str, common_t, et, p0, p1, q0, q1, same_ctx)) flags |= FDY_NODE_DESC;
    } else {
      flags |= FDY_NODE_LAYOUT | FDY_NODE_DESC;
    }
    if (flags & kNodeBad) atomicOr(&s_status, FDY_GRAPH_BAD_PARAMS);

    const uint64_t gi = Gg.node_base + n;
    NodeDesc d;
    d.gword = 0;          // word offsets are filled in by k_node_b
    d.nwords = words_g;
    d.tword = words_t;    // the template node's word count until then
    d.flags = flags;
    d.src_g = src_g;
    d.src_t = src_t;
    a.node_desc[gi] = d;
    a.node_flags[gi] = (uint8_t)(flags & 0x0F);
    a.node_ptrs[2 * gi] = p0;
    a.node_ptrs[2 * gi + 1] = p1;
    if (is_t) a.live_src[gi] = g;
  }

  // The records go to LDS (zero for the front padding: leading zero records
  // leave a zero-initialised CRC at zero).
  s_rec[0][tid >> 3][2 * (tid & 7)] = tw0;
  s_rec[0][tid >> 3][2 * (tid & 7) + 1] = tw1;
  s_rec[1][tid >> 3][2 * (tid & 7)] = kw0;
  s_rec[1][tid >> 3][2 * (tid & 7) + 1] = kw1;
  uint32_t sum_g = words_g, sum_t = words_t;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    sum_g += __shfl_down(sum_g, (unsigned)d, 64);
    sum_t += __shfl_down(sum_t, (unsigned)d, 64);
    pbytes += shfl_down64(pbytes, d);
  }
  if ((tid & 63) == 0) {
    s_sum[0][tid >> 6] = sum_g;
    s_sum[1][tid >> 6] = sum_t;
    s_pb[tid >> 6] = pbytes;
  }
  __syncthreads();
  if (tid >= 64) return;
  // Raw CRCs of the two record streams, by the first wave: lane l folds the
  // eight records 8q..8q+7 (q = l % 32) of stream l / 32 into one raw CRC
  // and moves it into place, times x^(8*16*(255-(8q+7))); each half-wave
  // XOR-joins its 32 shares (crc(A || B) = crc(A) * x^(8|B|) xor crc(B)).
  // One position multiply per lane of one wave, where a multiply per record
  // would cost every wave two.
  static_assert(kNodeChunk == 8 * 32, "eight records per lane, 32 lanes per stream");
  uint64_t z = 0;
  {
    const uint32_t st = tid >> 5, q = tid & 31;
#pragma unroll
    for (uint32_t r = 0; r < 16; ++r) z = crc_slice8(slice, z, s_rec[st][q][r]);
    z = z ? gf2_mulmod(a.cc->pos16[8 * q + 7], z) : 0;
#pragma unroll
    for (int d = 16; d >= 1; d >>= 1) z ^= shfl_down64(z, d);  // lanes 0 and 32 hold their half's XOR
  }
  const uint64_t zk = ((uint64_t)__shfl((uint32_t)(z >> 32), 32, 64) << 32) | __shfl((uint32_t)z, 32, 64);
  if (tid == 0) {
    NodeChunk c;
    c.crc_type = z;
    c.crc_kent = zk;
    c.pbytes = 0;
    uint64_t wg = 0, wt = 0;
    for (uint32_t w = 0; w < kNodeChunk / 64; ++w) {
      wg += s_sum[0][w];
      wt += s_sum[1][w];
      c.pbytes += s_pb[w];
    }
    c.words_g = wg > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)wg;
    c.words_t = wt > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)wt;
    c.status = s_status;
    c.pad_ = 0;
    a.chunks[chunk] = c;
  }
}

__global__ __launch_bounds__(kNodeThreads) void k_node_b(RestoreArgs a) {
  __shared__ uint32_t s_tmp[kNodeThreads / 64];
  __shared__ uint64_t s_x[2][kNodeThreads / 64];
  __shared__ unsigned long long s_pb;
  __shared__ uint32_t s_status, s_words, s_flat, s_tbase;

  const uint32_t g = blockIdx.x;
  const uint32_t t = a.template_of[g];
  const bool is_t = t == g;
  const DevGraph& Gg = a.graphs[g];
  const DevGraph& Gt = a.graphs[t];
  const uint32_t N = Gg.num_nodes, NT = Gt.num_nodes;
  const uint8_t* img = a.img;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) {
    s_status = a.status[g];  // the grouping pass's collision bit
    s_pb = 0;
    s_flat = 1;
  }
  __syncthreads();

  // Chunk results: each chunk's raw CRC times x^(8 * bytes after it),
  // XOR-joined; param bytes and status bits.  One wave per chunk: lane i
  // holds the multiplier times x^i and keeps it where the CRC has x^i
  // (bit 63 - i); the wave's XOR is the product.
  static_assert(kNodeChunk == kPosRecords, "chunk shift tables are built for kPosRecords records per chunk");
  const uint32_t nch = (N + kNodeChunk - 1) / kNodeChunk;
  uint64_t xt = 0, xk = 0, pb = 0;
  uint32_t st = 0;
  for (uint32_t c = wave; c < nch; c += kNodeThreads / 64) {
    const NodeChunk ch = a.chunks[Gg.chunk_base + c];
    const uint32_t k = nch - 1 - c;
    if (k < (uint32_t)kChunkShifts) {
      const uint64_t mi = a.cc->chunk_shift[k][lane];
      if ((ch.crc_type >> (63 - lane)) & 1) xt ^= mi;
      if ((ch.crc_kent >> (63 - lane)) & 1) xk ^= mi;
    } else if (lane == 0) {
      const uint64_t m = x2n_mod(a.cc->x2n.v, 16ull * kNodeChunk * k, 3);
      xt ^= gf2_mulmod(m, ch.crc_type);
      xk ^= gf2_mulmod(m, ch.crc_kent);
    }
    if (lane == 0) {
      pb += ch.pbytes;
      st |= ch.status;
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    xt ^= shfl_down64(xt, d);
    xk ^= shfl_down64(xk, d);
  }
  if (lane == 0) {
    s_x[0][wave] = xt;
    s_x[1][wave] = xk;
  }
  if (pb) atomicAdd(&s_pb, (unsigned long long)pb);
  if (st) atomicOr(&s_status, st);

  // Word offsets of every node in the graph's and in the template's image.
  uint32_t gcarry = 0, tcarry = 0;
  for (uint32_t base = 0; base < N; base += kNodeThreads) {
    const uint32_t n = base + threadIdx.x;
    const bool valid = n < N;
    const uint64_t gi = Gg.node_base + n;
    NodeDesc d{};
    if (valid) d = a.node_desc[gi];
    const uint32_t words_g = d.nwords, words_t = d.tword;
    uint32_t flags = d.flags;
    uint32_t tot_g, tot_t;
    const uint32_t gword = gcarry + block_excl_scan(words_g, s_tmp, &tot_g);
    const uint32_t tword = tcarry + block_excl_scan(words_t, s_tmp, &tot_t);
    // A template whose image overflows its capacity (overlapping param
    // ranges) has no usable words past the capacity; never index them.
    if ((flags & kNodeCompare) && (uint64_t)tword + words_t > Gt.word_cap) flags &= ~kNodeCompare;
    if (valid) {
      // The graph's image is flat when every node with words is aligned and
      // placed canonically (word w of the image at param-data byte 8w), and
      // likewise in the template's image for every compared node.
      if (words_g) {
        const bool ok = !(flags & (FDY_NODE_RAGGED | kNodeRaggedT)) &&
                        d.src_g == Gg.sec_off[FDY_SEC_PARAM_DATA] + 8ull * gword &&
                        (is_t || ((flags & kNodeCompare) && tword == gword &&
                                  d.src_t == Gt.sec_off[FDY_SEC_PARAM_DATA] + 8ull * gword));
        if (!ok) s_flat = 0;
      }
      d.gword = gword;
      d.tword = tword;
      d.flags = flags;
      a.node_desc[gi] = d;
      if (words_g) {
        uint64_t k = ((uint64_t)gword + kTileWords - 1) / kTileWords;
        const uint64_t k_last = ((uint64_t)gword + words_g - 1) / kTileWords;
        for (; k <= k_last && k < Gg.tile_cap; ++k) a.tile_node[Gg.tile_base + k] = n;
        if (flags & FDY_NODE_RAGGED) {
          const uint8_t* eg = img + Gg.sec_off[FDY_SEC_NODES] + 168ull * n;
          Side sd_{}, none_{};
          bool same_;
          side_header(img, Gg, RawEntry{eg}, sd_);
          scan_params(Gg, sd_, true, Gg, none_, false, &same_);
          write_aux(img, Gg, eg, sd_, a.aux, gword);
        }
      }
    }
    gcarry += tot_g;
    tcarry += tot_t;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t acc_type = 0, acc_kent = 0;
    for (uint32_t w = 0; w < kNodeThreads / 64; ++w) {
      acc_type ^= s_x[0][w];
      acc_kent ^= s_x[1][w];
    }
    const bool overflow = gcarry > Gg.word_cap;
    s_words = overflow ? 0 : gcarry;
    uint32_t stat = s_status;
    if (!is_t && N != NT) stat |= kGraphNodeCount;
    if (overflow) stat |= FDY_GRAPH_BAD_PARAMS | kGraphOverflow;
    a.status[g] = stat;
    a.gwords[g] = s_words;
    a.pbytes[g] = s_pb;
    a.digests[4ull * g + 2] = acc_type ^ Gg.crc_fin[2];
    a.digests[4ull * g + 3] = acc_kent ^ Gg.crc_fin[3];
    if (is_t) {
      a.live_cur[g] = g;
      // List the template's slots that hold words for k_diff_t.
      s_tbase = atomicAdd(a.tslot_count, (s_words + kTileWords - 1) / kTileWords);
    }
  }
  __syncthreads();
  const uint32_t words = s_words;
  const uint32_t first_unused = (words + kTileWords - 1) / kTileWords;
  const uint32_t sflags = (s_flat ? kSlotFlat | (is_t ? 0u : kSlotCompare) : 0u) | (is_t ? kSlotTemplate : 0u);
  for (uint32_t k = threadIdx.x; k < Gg.tile_cap; k += kNodeThreads) {
    if (k >= first_unused) a.tile_node[Gg.tile_base + k] = kNoTile;
    SlotDesc sd;
    sd.kg = Gg.sec_off[FDY_SEC_PARAM_DATA];
    sd.kt = Gt.sec_off[FDY_SEC_PARAM_DATA];
    sd.word_base = Gg.word_base;
    sd.wbeg = (uint32_t)min((uint64_t)k * kTileWords, (uint64_t)words);
    sd.wend = (uint32_t)min((uint64_t)(k + 1) * kTileWords, (uint64_t)words);
    sd.graph = g;
    sd.tmpl = t;
    sd.flags = sflags | (k == 0 ? kSlotFirst : 0u);
    sd.t_cap = Gt.word_cap;
    sd.pad[0] = sd.pad[1] = 0;
    sd.t_word_base = Gt.word_base;
    a.slot_desc[Gg.tile_base + k] = sd;
    if (is_t && k < first_unused) a.tslots[s_tbase + k] = Gg.tile_base + k;
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

// A slot descriptor, loaded whole before any branch: left to itself the
// compiler loads each field at its first use, behind branches, and every
// such load is another serial round trip before the tile's loads can start.
__device__ inline SlotDesc load_slot(const SlotDesc* p) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
  const uint4 v0 = q[0], v1 = q[1], v2 = q[2], v3 = q[3];
  asm volatile("" ::"s"(v0.x), "s"(v0.y), "s"(v0.z), "s"(v0.w), "s"(v1.x), "s"(v1.y), "s"(v1.z), "s"(v1.w),
               "s"(v2.x), "s"(v2.y), "s"(v2.z), "s"(v2.w), "s"(v3.x), "s"(v3.y), "s"(v3.z), "s"(v3.w));
  SlotDesc d;
  static_assert(sizeof(SlotDesc) == 4 * sizeof(uint4), "SlotDesc is four 16-byte words");
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

__device__ inline NodeWindow stage_window(const RestoreArgs& a, const DevGraph& G, uint32_t slot, NodeDesc* s_nd) {
  NodeWindow nw;
  const uint32_t k = slot - G.tile_base;
  nw.n0 = a.tile_node[slot];
  nw.N = G.num_nodes;
  const uint32_t n_next = k + 1 < G.tile_cap ? a.tile_node[slot + 1] : kNoTile;
  const uint32_t n_last = n_next == kNoTile ? nw.N - 1 : n_next;
  nw.nwin = min(kDiffWindow, n_last - nw.n0 + 1);
  nw.nd = a.node_desc + G.node_base;
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
__device__ inline uint64_t load_word(const RestoreArgs& a, const DevGraph& G, const NodeDesc& d, uint64_t w,
                                     bool ragged, uint64_t src, uint32_t* width) {
  if (ragged) {
    const uint64_t x = a.aux[G.word_base + w];
    *width = (uint32_t)(x & 15);
    return load_bytes(a.img, x >> 4, *width);
  }
  *width = 8;
  return *reinterpret_cast<const uint64_t*>(a.img + src + 8ull * (w - d.gword));
}

// Template graphs: relocate their words into R and the live image.  The
// template slots listed by the node pass are cut into units of kTUnit words
// (kTWords per thread, so one search batch), spread over the grid.
constexpr uint32_t kTThreads = 256;
constexpr uint32_t kTWords = 4;
constexpr uint32_t kTUnit = kTThreads * kTWords;
constexpr uint32_t kTUnitsPerTile = kTileWords / kTUnit;
static_assert(kTileWords % kTUnit == 0, "template units tile a slot");

__global__ __launch_bounds__(kTThreads) void k_diff_t(RestoreArgs a) {
  __shared__ NodeDesc s_nd[kDiffWindow];
  const uint32_t tid = threadIdx.x;
  const uint32_t units = *a.tslot_count * kTUnitsPerTile;
  for (uint32_t u = blockIdx.x; u < units; u += gridDim.x) {
    const uint32_t slot = a.tslots[u / kTUnitsPerTile];
    const SlotDesc sd = load_slot(a.slot_desc + slot);
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
      const DevGraph& G = a.graphs[sd.graph];
      __syncthreads();  // the previous unit's lookups are done with s_nd
      const NodeWindow nw = stage_window(a, G, slot, s_nd);
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
    reloc_batch<kTWords>(a.reloc, v, r, m);
    uint64_t* img_out = a.image + sd.word_base;
    uint64_t* live_out = a.live + sd.word_base;
#pragma unroll
    for (uint32_t q = 0; q < kTWords; ++q) {
      const uint64_t w = ubeg + q * kTThreads + tid;
      if (w < uend) {
        img_out[w] = r[q];
        live_out[w] = r[q];
      }
    }
  }
}

// The other graphs: kMSplit workgroups per slot, each of kMThreads / 64
// waves; wave v of the slot (counted over its workgroups) owns the slot's
// sub-range v (kSubWords consecutive words), lane l its words
// v*kSubWords + j*64 + l for j < kMWords.  Small workgroups retire and are
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

// Five waves per SIMD: the node window in LDS allows no more.
__global__ __launch_bounds__(kMThreads, 5) void k_diff_m(RestoreArgs a) {
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
  const uint64_t w0 = wbeg + (uint64_t)wave * kSubWords + lane;  // word j is w0 + 64j
  const bool flat = (sd.flags & kSlotFlat) != 0;
  const RelocDev& R = a.reloc;
  // Issued ahead of the word loads so that its wait does not follow theirs.
  const uint32_t t_status = a.status[t];
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
    for (uint32_t j = 0; j < J; ++j) {
      const uint64_t w = w0 + 64 * j;
      fg[j] = ft[j] = fr[j] = 0;
      if (w < wend) {
        valid |= 1u << j;
        fg[j] = *reinterpret_cast<const uint64_t*>(pg + 8 * w);
        ft[j] = *reinterpret_cast<const uint64_t*>(pt + 8 * w);
      }
    }
    if (R.n != 0) {
#pragma unroll
      for (uint32_t j = 0; j < J; ++j)
        if ((valid >> j) & 1) fr[j] = rimg_t[min(w0 + 64 * j, (uint64_t)t_last)];
    }
    cmp = full = valid;
  }
  if (!flat && wend > wbeg) {  // uniform over the workgroup
    const DevGraph& G = a.graphs[g];
    const DevGraph& T = a.graphs[t];
    const NodeWindow nw = stage_window(a, G, slot, s_nd);
    __syncthreads();
    uint64_t wv[J];
    uint32_t node[J];
#pragma unroll
    for (uint32_t j = 0; j < J; ++j) wv[j] = w0 + 64 * j;
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
#pragma unroll
  for (uint32_t j = 0; j < J; ++j) {
    if (!((valid >> j) & 1)) continue;
    const uint64_t w = w0 + 64 * j;
    const bool c = (cmp >> j) & 1;
    const bool same = c && fg[j] == ft[j];
    img_out[w] = same ? fr[j] : fg[j];
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
  Candidate* out = a.cand + ((uint64_t)slot * kSubsPerSlot + wave) * kSubWords;
  const uint64_t lt = (1ull << lane) - 1;
  if (!flat) __syncthreads();  // every wave of the workgroup is done with the node window
  Candidate* stage = reinterpret_cast<Candidate*>(s_nd) + (tid >> 6) * kSubWords;
  uint32_t run = 0;
#pragma unroll
  for (uint32_t j = 0; j < J; ++j) {
    const uint64_t mk = __ballot((cand >> j) & 1);
    if ((cand >> j) & 1) {
      Candidate c;
      c.word = (uint32_t)(w0 + 64 * j);
      c.flags = (((creloc >> j) & 1) ? kCandReloc : 0u) | (((cmp >> j) & 1) ? kCandCompare : 0u);
      c.raw = fg[j];
      c.tval = fr[j];
      stage[run + (uint32_t)__popcll(mk & lt)] = c;
    }
    run += (uint32_t)__popcll(mk);
  }
  {
    static_assert(sizeof(Candidate) % 8 == 0, "candidates copy as 8-byte words");
    constexpr uint32_t kCandWords = sizeof(Candidate) / 8;
    const uint64_t* src = reinterpret_cast<const uint64_t*>(stage);
    uint64_t* dst = reinterpret_cast<uint64_t*>(out);
    for (uint32_t i = lane; i < run * kCandWords; i += 64) dst[i] = src[i];
  }
  if (lane == 0) sub_count[wave] = run;
  if (tid == 0 && part == 0 && (sd.flags & kSlotFirst)) {
    if (a.digests[4ull * g + 2] != a.digests[4ull * t + 2]) atomicOr(&a.status[g], FDY_GRAPH_TYPE_MISMATCH);
  }
}

// Candidates of the member pass, one wave per slot: the slot's sub-range
// lists are taken as one list in word order, kSBatch / 64 candidates per
// lane searched in one lockstep batch.  The relocated word goes to R, and
// the words whose value differs from the template's become override records,
// compacted in word order at the start of the slot's region; the slot's
// record count replaces the first sub-range count (the others become 0).
// Writing over the candidates is safe: record r takes bytes [16r, 16r + 16)
// and every candidate at or after list index r lies at or past byte 24r of
// its own sub-range region, hence past them; a batch reads all its
// candidates before writing any record.
constexpr uint32_t kSThreads = 256;  // four slots per workgroup
constexpr uint32_t kSBatch = 128;  // two per lane: 256 measured slower (fewer waves in flight)

__global__ __launch_bounds__(kSThreads) void k_diff_s(RestoreArgs a) {
  constexpr uint32_t K = kSBatch / 64;
  static_assert(kSubsPerSlot <= 64, "one lane per sub-range count");
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t slot = blockIdx.x * (kSThreads / 64) + (threadIdx.x >> 6);
  if (slot >= a.num_slots) return;  // per wave: this kernel has no barrier
  uint32_t* counts = a.sub_count + (uint64_t)slot * kSubsPerSlot;
  // Lane q < kSubsPerSlot holds sub-range q's count; inclusive prefix over lanes.
  const uint32_t cnt = lane < kSubsPerSlot ? counts[lane] : 0;
  uint32_t incl = cnt;
#pragma unroll
  for (int d = 1; d < (int)kSubsPerSlot; d <<= 1) {
    const uint32_t y = shfl_up32(incl, d);
    if (lane >= (uint32_t)d) incl += y;
  }
  const uint32_t total = __shfl(incl, kSubsPerSlot - 1, 64);
  if (total == 0) return;
  uint32_t start[kSubsPerSlot];  // exclusive prefix, the same in every lane
#pragma unroll
  for (uint32_t q = 0; q < kSubsPerSlot; ++q) start[q] = __shfl(incl - cnt, q, 64);
  const uint64_t word_base = a.slot_desc[slot].word_base;
  uint64_t* img_out = a.image + word_base;
  Candidate* base = a.cand + (uint64_t)slot * kSubsPerSlot * kSubWords;
  fdy_override* rec = reinterpret_cast<fdy_override*>(base);
  const uint64_t lt = (1ull << lane) - 1;
  uint32_t run = 0;
  for (uint32_t b = 0; b < total; b += kSBatch) {
    uint64_t raw[K], tval[K], res[K];
    uint32_t word[K], fl[K], m = 0;
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
      const uint32_t i = b + 64 * k + lane;  // list index
      raw[k] = tval[k] = 0;
      word[k] = fl[k] = 0;
      if (i < total) {
        uint32_t q = 0;
#pragma unroll
        for (uint32_t s = 1; s < kSubsPerSlot; ++s) q += start[s] <= i;
        uint32_t sq = start[0];
#pragma unroll
        for (uint32_t s = 1; s < kSubsPerSlot; ++s) sq = q == s ? start[s] : sq;
        const Candidate c = base[(uint64_t)q * kSubWords + (i - sq)];
        raw[k] = c.raw;
        tval[k] = c.tval;
        word[k] = c.word;
        fl[k] = c.flags;
        if (c.flags & kCandReloc) m |= 1u << k;
      }
    }
    reloc_batch<K>(a.reloc, raw, res, m);
    // The member pass stored each candidate's raw word; only the words the
    // relocation moved are stored again (a scattered 8-byte store costs a
    // partly written line).
#pragma unroll
    for (uint32_t k = 0; k < K; ++k)
      if (((m >> k) & 1) && res[k] != raw[k]) img_out[word[k]] = res[k];
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) {
      const bool d = (fl[k] & kCandCompare) && res[k] != tval[k];
      const uint64_t mk = __ballot(d);
      if (d) {
        fdy_override o;
        o.word = word[k];
        o.node = 0;
        o.value = res[k];
        rec[run + (uint32_t)__popcll(mk & lt)] = o;
      }
      run += (uint32_t)__popcll(mk);
    }
  }
  if (lane < kSubsPerSlot) counts[lane] = lane == 0 ? run : 0u;
}

// Records per graph: the sum of its slots' sub-range counts (one workgroup
// per graph; a global atomic per slot instead measured slower).
constexpr uint32_t kCountThreads = 256;

// Exclusive prefix sum of u64 values over the block (blockDim.x a multiple
// of 64, at most 4096); *total gets the sum.
__device__ uint64_t block_excl_scan64(uint64_t v, uint64_t* s_tmp, uint64_t* total) {
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint64_t y = ((uint64_t)shfl_up32((uint32_t)(x >> 32), d) << 32) | shfl_up32((uint32_t)x, d);
    if (lane >= (uint32_t)d) x += y;
  }
  if (lane == 63) s_tmp[wave] = x;
  __syncthreads();
  uint64_t before = 0, sum = 0;
  for (uint32_t w = 0; w < blockDim.x / 64; ++w) {
    const uint64_t t = s_tmp[w];
    if (w < wave) before += t;
    sum += t;
  }
  __syncthreads();
  *total = sum;
  return before + x - v;
}

// Records per graph and each slot's offset among its graph's records (an
// exclusive scan over the graph's slots, one slot per thread), so that the
// compaction reads its base instead of summing every earlier slot's count.
__global__ __launch_bounds__(kCountThreads) void k_count(RestoreArgs a) {
  static_assert(kCountThreads == 256, "block_excl_scan covers 256 values");
  static_assert(kSubsPerSlot % 4 == 0, "a slot's counts are read 16 bytes at a time");
  __shared__ uint32_t s_tmp[kCountThreads / 64];
  const uint32_t g = blockIdx.x, tid = threadIdx.x;
  const DevGraph& G = a.graphs[g];
  uint32_t carry = 0;
  for (uint32_t k0 = 0; k0 < G.tile_cap; k0 += kCountThreads) {
    const uint32_t k = k0 + tid;
    uint32_t n = 0;
    if (k < G.tile_cap) {
      const uint4* c = reinterpret_cast<const uint4*>(a.sub_count + (uint64_t)(G.tile_base + k) * kSubsPerSlot);
#pragma unroll
      for (uint32_t q = 0; q < kSubsPerSlot / 4; ++q) {
        const uint4 v = c[q];
        n += v.x + v.y + v.z + v.w;
      }
    }
    uint32_t tot;
    const uint32_t ex = block_excl_scan(n, s_tmp, &tot);
    if (k < G.tile_cap) a.slot_off[G.tile_base + k] = carry + ex;
    carry += tot;
  }
  if (tid == 0) a.graph_count[g] = carry;
}

// The override offsets: an exclusive scan of the graph counts by one
// workgroup (a separate launch: a last-workgroup scan inside the count pass
// needs device-wide fences, whose L2 write-backs measured slower).
constexpr uint32_t kScanThreads = 1024;

__global__ __launch_bounds__(kScanThreads) void k_scan(RestoreArgs a) {
  __shared__ uint64_t s_tmp[kScanThreads / 64];
  uint64_t base = 0;
  for (uint32_t j0 = 0; j0 < a.num_graphs; j0 += kScanThreads) {
    const uint32_t j = j0 + threadIdx.x;
    uint64_t tot;
    const uint64_t ex = block_excl_scan64(j < a.num_graphs ? a.graph_count[j] : 0, s_tmp, &tot);
    if (j < a.num_graphs) a.ovr_off[j] = base + ex;
    base += tot;
  }
  if (threadIdx.x == 0) a.ovr_off[a.num_graphs] = base;
}

// Move each slot's records to their place in the dense array, completing
// them: the node holding the word (searched in the slot's node window) and
// the word's index in the template's image.  The search pass leaves a slot's
// records at the start of its region in word order, their number in the
// slot's first sub-range count (the others are zero).  A slot's records
// start at its graph's override offset plus the slot's offset among the
// graph's records.  Everything that depends on the slot alone (the count,
// the first records, the window's bounds) is loaded before what depends on
// its graph, to keep the chain of dependent loads short.
// One wave per slot: a slot holds about a hundred records on the presets,
// and more slots in flight per CU beat more lanes per slot (256 threads per
// slot: 0.57 ms on the 1024-graph archive; 128: 0.41; 64: 0.36).
constexpr uint32_t kCompactThreads = 64;
constexpr uint32_t kCompactPre = 4;  // records per thread loaded up front

__global__ __launch_bounds__(kCompactThreads) void k_compact(RestoreArgs a) {
  __shared__ uint2 s_gt[kDiffWindow];  // {first graph word, first template word} of the window's nodes
  const uint32_t slot = blockIdx.x, tid = threadIdx.x;
  const uint32_t total = a.sub_count[(uint64_t)slot * kSubsPerSlot];
  if (total == 0) return;  // uniform over the workgroup
  const fdy_override* recs = reinterpret_cast<const fdy_override*>(a.cand + (uint64_t)slot * kSubsPerSlot * kSubWords);
  fdy_override pre[kCompactPre];
#pragma unroll
  for (uint32_t p = 0; p < kCompactPre; ++p) {
    const uint32_t i = tid + p * kCompactThreads;
    if (i < total) pre[p] = recs[i];
  }
  const SlotDesc sd = load_slot(a.slot_desc + slot);
  const uint32_t n0 = a.tile_node[slot];
  const uint32_t off = a.slot_off[slot];
  const DevGraph& G = a.graphs[sd.graph];
  const uint32_t k = slot - G.tile_base;
  const uint32_t N = G.num_nodes;
  const uint32_t n_next = k + 1 < G.tile_cap ? a.tile_node[slot + 1] : kNoTile;
  const uint32_t n_last = n_next == kNoTile ? N - 1 : n_next;
  const uint32_t nwin = min(kDiffWindow, n_last - n0 + 1);
  const NodeDesc* nd = a.node_desc + G.node_base;
  const uint64_t base = a.ovr_off[sd.graph] + off;
  for (uint32_t i = tid; i < nwin; i += kCompactThreads) {
    const uint4 v = *reinterpret_cast<const uint4*>(nd + n0 + i);  // gword, nwords, tword, flags
    s_gt[i] = make_uint2(v.x, v.z);
  }
  __syncthreads();
  auto finish = [&](fdy_override o, uint32_t i) {
    const uint64_t w = o.word;
    // The last node whose first word is <= w (nodes without words never
    // match: the node holding w follows them); past a full window the
    // search continues in global memory.
    uint32_t lo = 0;
    for (uint32_t len = nwin; len > 1;) {
      const uint32_t half = len >> 1;
      if (s_gt[lo + half].x <= w) lo += half;
      len -= half;
    }
    uint32_t node = n0 + lo, gw = s_gt[lo].x, tw = s_gt[lo].y;
    if (nwin == kDiffWindow && lo == kDiffWindow - 1 && w >= (uint64_t)nd[node].gword + nd[node].nwords) {
      uint32_t l2 = node, h2 = N;
      while (h2 - l2 > 1) {
        const uint32_t mid = (l2 + h2) >> 1;
        if (nd[mid].gword <= w) l2 = mid;
        else h2 = mid;
      }
      node = l2;
      gw = nd[node].gword;
      tw = nd[node].tword;
    }
    o.word = tw + (uint32_t)(w - gw);
    o.node = node;
    a.ovr[base + i] = o;
  };
#pragma unroll
  for (uint32_t p = 0; p < kCompactPre; ++p) {
    const uint32_t i = tid + p * kCompactThreads;
    if (i < total) finish(pre[p], i);
  }
  for (uint32_t i = tid + kCompactPre * kCompactThreads; i < total; i += kCompactThreads) finish(recs[i], i);
}

// ---- switch --------------------------------------------------------------

__global__ __launch_bounds__(256) void k_switch(SwitchArgs a) {
  const uint64_t total = a.n_cur + a.n_new;
  const uint64_t lim = total > a.num_nodes ? total : a.num_nodes;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < lim; i += (uint64_t)gridDim.x * 256) {
    if (i < a.n_cur) {
      const fdy_override r = a.ovr_cur[i];
      uint64_t lo = 0, hi = a.n_new;  // does the target override this word too?
      while (lo < hi) {
        const uint64_t mid = (lo + hi) >> 1;
        if (a.ovr_new[mid].word < r.word) lo = mid + 1;
        else hi = mid;
      }
      if (lo == a.n_new || a.ovr_new[lo].word != r.word) a.live[r.word] = a.tmpl_image[r.word];
      if (a.dirty) a.dirty[r.node] = 1;
    } else if (i < total) {
      const fdy_override r = a.ovr_new[i - a.n_cur];
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
__global__ __launch_bounds__(kRelocThreads) void k_reloc(RelocDev R, const uint64_t* in, uint64_t* out, uint64_t n,
                                                         int vec) {
  // Each thread owns kRelocPairs 16-byte pairs per chunk (coalesced across
  // the workgroup): all loads first, then the searches, then the stores, so
  // the searches of 2 * kRelocPairs words overlap.
  const uint64_t chunk = (uint64_t)kRelocThreads * kRelocPairs;
  if (vec) {
    const uint64_t pairs = n / 2;
    const ulonglong2* in2 = reinterpret_cast<const ulonglong2*>(in);
    ulonglong2* out2 = reinterpret_cast<ulonglong2*>(out);
    for (uint64_t c = (uint64_t)blockIdx.x * chunk; c < pairs; c += (uint64_t)gridDim.x * chunk) {
      ulonglong2 v[kRelocPairs];
#pragma unroll
      for (uint32_t q = 0; q < kRelocPairs; ++q) {
        const uint64_t p = c + q * kRelocThreads + threadIdx.x;
        v[q] = p < pairs ? in2[p] : ulonglong2{0, 0};
      }
#pragma unroll
      for (uint32_t q = 0; q < kRelocPairs; q += kRelocBatch / 2) {
        uint64_t w[kRelocBatch], r[kRelocBatch];
#pragma unroll
        for (uint32_t k = 0; k < kRelocBatch / 2; ++k) {
          w[2 * k] = v[q + k].x;
          w[2 * k + 1] = v[q + k].y;
        }
        reloc_batch<kRelocBatch>(R, w, r, (1u << kRelocBatch) - 1);
#pragma unroll
        for (uint32_t k = 0; k < kRelocBatch / 2; ++k) v[q + k] = ulonglong2{r[2 * k], r[2 * k + 1]};
      }
#pragma unroll
      for (uint32_t q = 0; q < kRelocPairs; ++q) {
        const uint64_t p = c + q * kRelocThreads + threadIdx.x;
        if (p < pairs) out2[p] = v[q];
      }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && (n & 1)) out[n - 1] = reloc_word(R, in[n - 1]);
  } else {
    const uint64_t stride = (uint64_t)gridDim.x * kRelocThreads;
    for (uint64_t p = (uint64_t)blockIdx.x * kRelocThreads + threadIdx.x; p < n; p += stride)
      out[p] = reloc_word(R, in[p]);
  }
}

}  // namespace

hipError_t launch_hash(const RestoreArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_hash, dim3(a.num_graphs), dim3(kHashThreads), 0, s, a);
  return hipGetLastError();
}

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
  hipLaunchKernelGGL(k_node_b, dim3(a.num_graphs), dim3(kNodeThreads), 0, s, a);
  return hipGetLastError();
}

// Templates first: the other graphs read their relocated words.
hipError_t launch_diff_templates(const RestoreArgs& a, hipStream_t s) {
  const uint32_t tgrid = (uint32_t)std::min<uint64_t>((uint64_t)a.num_slots * kTUnitsPerTile, 2048);
  hipLaunchKernelGGL(k_diff_t, dim3(tgrid), dim3(kTThreads), 0, s, a);
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

hipError_t launch_planes(const uint8_t* img, const DevGraph* graphs, const uint32_t* chunk_graph, uint32_t num_chunks,
                         uint32_t* planes, uint64_t* pplanes, hipStream_t s) {
  hipLaunchKernelGGL(k_planes, dim3(num_chunks), dim3(kNodeChunk), 0, s, img, graphs, chunk_graph, planes, pplanes);
  return hipGetLastError();
}

hipError_t launch_compact(const RestoreArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_count, dim3(a.num_graphs), dim3(kCountThreads), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_scan, dim3(1), dim3(kScanThreads), 0, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_compact, dim3(a.num_slots), dim3(kCompactThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_switch(const SwitchArgs& a, hipStream_t s) {
  uint64_t lim = a.n_cur + a.n_new;
  if (a.num_nodes > lim) lim = a.num_nodes;
  if (lim == 0) return hipSuccess;
  uint64_t blocks = (lim + 255) / 256;
  if (blocks > 2048) blocks = 2048;
  hipLaunchKernelGGL(k_switch, dim3((uint32_t)blocks), dim3(256), 0, s, a);
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
