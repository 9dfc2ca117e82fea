// synth.cpp -- seeded synthetic `.cugraph` archives (see include/fdy_synth.h).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "../../include/fdy_synth.h"
#include "cugraph.h"

namespace {

thread_local std::string g_err;

int fail(const std::string& msg) {
  g_err = msg;
  return -1;
}

// SplitMix64 (Steele, Lea, Flood 2014).
struct Rng {
  uint64_t x;
  explicit Rng(uint64_t s) : x(s) {}
  uint64_t next() {
    uint64_t z = (x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  uint64_t below(uint64_t n) { return n ? (uint64_t)(((unsigned __int128)next() * n) >> 64) : 0; }
  double unit() { return (next() >> 11) * (1.0 / 9007199254740992.0); }
  uint64_t range(uint64_t lo, uint64_t hi) { return lo + below(hi - lo + 1); }  // inclusive
};

uint64_t mix(uint64_t a, uint64_t b) {
  Rng r(a ^ (b * 0xD1B54A32D192ED03ull));
  r.next();
  return r.next();
}

enum WordKind : uint8_t { W_PTR = 0, W_U32 = 1, W_F32 = 2 };

struct Intervals {
  std::vector<uint64_t> lo, hi, nlo;
};

// Node layout shared by every graph of a group at one node position.
struct NodeLayout {
  uint8_t type = FDY_NODE_KERNEL;
  std::string name;
  uint64_t binary_hash = 0;
  uint32_t block = 128, grid[3] = {1, 1, 1}, shmem = 0;
  uint32_t cluster_x = 0;  // >0: per-node cluster attribute (distinguishes groups)
  bool grid_bs = false;
  bool extra = false;
  bool layout_var = false;
  bool diff_ok = true;  // differing words may fall in this node
  std::vector<uint32_t> sizes[2];  // [0] base layout, [1] variant used by large batch sizes
  std::vector<uint8_t> kinds[2];   // per 8-byte word of the padded blob
  std::vector<uint64_t> base[2];   // group-base words
  int32_t event_id = 0;
  uint64_t memset_dst = 0, memcpy_src = 0, memcpy_dst = 0;
};

struct Group {
  std::vector<NodeLayout> nodes;
  std::vector<fdy_dep> deps;
};

struct Synth {
  fdy_synth_params p{};
  std::vector<std::vector<uint8_t>> images;
  std::vector<uint32_t> bs;
  Intervals iv;
  std::vector<uint64_t> words;
};

void make_intervals(const fdy_synth_params& p, Rng& r, Intervals& iv) {
  uint32_t n = std::max<uint32_t>(1, p.num_intervals);
  iv.lo.resize(n);
  iv.hi.resize(n);
  iv.nlo.resize(n);
  if (n == 1) {
    iv.lo[0] = p.region_base;
    iv.hi[0] = p.region_base + p.region_size;
    iv.nlo[0] = p.new_base;
    return;
  }
  // Log-uniform sizes, rescaled (largest remainder, >= 1 granule each) so
  // that the intervals tile the region exactly.
  const uint64_t q = std::max<uint32_t>(16, p.interval_granule);
  const uint64_t units = p.region_size / q;
  std::vector<double> raw(n);
  double lmin = std::log((double)std::max<uint64_t>(1, p.interval_min));
  double lmax = std::log((double)std::max<uint64_t>(p.interval_min + 1, p.interval_max));
  double sum = 0;
  for (uint32_t i = 0; i < n; ++i) {
    raw[i] = std::exp(lmin + (lmax - lmin) * r.unit());
    sum += raw[i];
  }
  std::vector<uint64_t> u(n);
  std::vector<std::pair<double, uint32_t>> frac(n);
  uint64_t spare = units - n;  // every interval gets one granule up front
  uint64_t used = 0;
  for (uint32_t i = 0; i < n; ++i) {
    double x = raw[i] / sum * (double)spare;
    u[i] = 1 + (uint64_t)x;
    used += (uint64_t)x;
    frac[i] = {x - std::floor(x), i};
  }
  std::sort(frac.begin(), frac.end(), [](auto& a, auto& b) { return a.first > b.first || (a.first == b.first && a.second < b.second); });
  for (uint64_t k = 0; used < spare; ++k, ++used) u[frac[k % n].second] += 1;
  uint64_t at = p.region_base;
  for (uint32_t i = 0; i < n; ++i) {
    iv.lo[i] = at;
    at += u[i] * q;
    iv.hi[i] = at;
  }
  // New placement: the same intervals in a seeded random order at new_base.
  std::vector<uint32_t> perm(n);
  for (uint32_t i = 0; i < n; ++i) perm[i] = i;
  for (uint32_t i = n - 1; i > 0; --i) std::swap(perm[i], perm[r.below(i + 1)]);
  uint64_t nat = p.new_base;
  for (uint32_t k = 0; k < n; ++k) {
    uint32_t i = perm[k];
    iv.nlo[i] = nat;
    nat += iv.hi[i] - iv.lo[i];
  }
}

uint64_t draw_pointer(Rng& r, const Intervals& iv, double boundary_frac) {
  uint64_t i = r.below(iv.lo.size());
  uint64_t lo = iv.lo[i], hi = iv.hi[i];
  if (boundary_frac > 0 && r.unit() < boundary_frac) {
    switch (r.below(4)) {
      case 0: return lo;
      case 1: return hi - 1;
      case 2: return hi;
      default: return lo - 1;
    }
  }
  uint64_t span = (hi - lo) / 16;
  return lo + 16 * r.below(span ? span : 1);
}

uint64_t draw_word(Rng& r, uint8_t kind, const Intervals& iv) {
  switch (kind) {
    case W_PTR: return draw_pointer(r, iv, 0.0);
    case W_U32: return r.next();
    default: {
      float f = (float)(r.unit() * 20.0 - 10.0);
      uint32_t b;
      std::memcpy(&b, &f, 4);
      return b;
    }
  }
}

// Split `blob` bytes into 1..max_params params.  Sizes are multiples of 8
// unless `ragged`, in which case some become 1..7 bytes shorter or longer.
std::vector<uint32_t> split_blob(Rng& r, uint32_t blob, uint32_t max_params, bool ragged) {
  uint32_t words = blob / 8;
  uint32_t np = 1 + (uint32_t)r.below(std::min<uint32_t>(std::max<uint32_t>(1, max_params), words));
  std::vector<uint32_t> cut;
  for (uint32_t i = 1; i < words; ++i) cut.push_back(i);
  for (uint32_t i = 0; i + 1 < np && i < cut.size(); ++i) std::swap(cut[i], cut[i + r.below(cut.size() - i)]);
  cut.resize(np - 1);
  std::sort(cut.begin(), cut.end());
  std::vector<uint32_t> sizes;
  uint32_t prev = 0;
  for (uint32_t c : cut) {
    sizes.push_back((c - prev) * 8);
    prev = c;
  }
  sizes.push_back((words - prev) * 8);
  if (ragged) {
    for (auto& s : sizes) {
      uint64_t k = r.below(4);
      if (k == 0) s = 4;                       // an int
      else if (k == 1 && s > 8) s -= 1 + (uint32_t)r.below(7);  // odd-sized struct
      else if (k == 2) s = 1 + (uint32_t)r.below(3);            // char / short flags
    }
  }
  return sizes;
}

void make_kinds(Rng& r, const std::vector<uint32_t>& sizes, double pfrac, std::vector<uint8_t>& kinds) {
  kinds.clear();
  for (uint32_t s : sizes) {
    for (uint32_t w = 0; w < (s + 7) / 8; ++w) {
      bool full = (w + 1) * 8 <= s;
      if (full && r.unit() < pfrac) kinds.push_back(W_PTR);
      else kinds.push_back(r.below(2) ? W_U32 : W_F32);
    }
  }
}

std::string kernel_name(uint32_t group, uint32_t pos, uint64_t h) {
  static const char* stems[] = {"rms_norm_kernel", "fused_add_rms_norm", "rotary_embedding_kernel",
                                "paged_attention_v2_kernel", "reshape_and_cache_flash", "act_and_mul_kernel",
                                "cutlass_gemm_sm_bf16_128x128x64", "moe_align_block_size", "topk_softmax",
                                "fused_moe_kernel_grouped", "all_reduce_one_shot", "silu_and_mul"};
  char buf[160];
  std::snprintf(buf, sizeof(buf), "_ZN4vllm%zu%sILi%uELi%uEEvPT_PKS1_i_%016llx",
                std::strlen(stems[pos % 12]), stems[pos % 12], group, pos % 7,
                (unsigned long long)h);
  return buf;
}

Group make_group(const fdy_synth_params& p, uint32_t g, const Intervals& iv) {
  Rng r(mix(p.seed, 0x100000000ull + g));
  Group grp;
  uint32_t N = p.nodes_per_graph;
  grp.nodes.resize(N);
  int32_t next_event = 1 + (int32_t)g * 1000;
  for (uint32_t n = 0; n < N; ++n) {
    NodeLayout& L = grp.nodes[n];
    uint64_t roll = r.below(100);
    if (p.sink_hash && n >= 1 && n <= 6 && n + 1 < N) {
      // The group's key: node n is empty where bit n-1 of the group index is set.
      L.type = ((g >> (n - 1)) & 1) ? FDY_NODE_EMPTY : FDY_NODE_KERNEL;
      if (L.type == FDY_NODE_EMPTY) continue;
    } else if (n > 0 && roll < p.memset_pct) L.type = FDY_NODE_MEMSET;
    else if (n > 0 && roll < p.memset_pct + p.memcpy_pct) L.type = FDY_NODE_MEMCPY;
    else if (n > 0 && n + 1 < N && roll < p.memset_pct + p.memcpy_pct + p.event_pct &&
             grp.nodes[n - 1].type != FDY_NODE_EVENT_RECORD)
      L.type = FDY_NODE_EVENT_RECORD;
    else L.type = FDY_NODE_KERNEL;
    if (n > 0 && grp.nodes[n - 1].type == FDY_NODE_EVENT_RECORD) {
      L.type = FDY_NODE_EVENT_WAIT;
      L.event_id = grp.nodes[n - 1].event_id;
    } else if (L.type == FDY_NODE_EVENT_RECORD) {
      L.event_id = next_event++;
    }
    if (L.type == FDY_NODE_MEMSET) L.memset_dst = draw_pointer(r, iv, 0);
    if (L.type == FDY_NODE_MEMCPY) {
      L.memcpy_src = draw_pointer(r, iv, 0);
      L.memcpy_dst = draw_pointer(r, iv, 0);
    }
    if (L.type != FDY_NODE_KERNEL) continue;
    uint32_t pos = n % 25;
    L.binary_hash = mix(p.seed ^ 0xC0DEull, (uint64_t)g * 4096 + pos);
    L.name = kernel_name(g, pos, L.binary_hash);
    if (p.sink_hash) {
      L.binary_hash = p.sink_hash;
      L.name = "fdy_sink";
    }
    L.block = r.below(2) ? 256 : 128;
    L.grid[0] = 1 + (uint32_t)r.below(512);
    L.grid[1] = 1 + (uint32_t)r.below(4);
    L.shmem = (uint32_t)r.below(3) * 16384;
    L.grid_bs = r.below(100) < p.grid_bs_pct;
    L.extra = r.below(100) < p.extra_style_pct;
    L.layout_var = r.below(100) < p.layout_var_pct;
    if (p.diff_node_pct) {  // no draw when 0: presets unchanged
      L.diff_ok = r.below(100) < p.diff_node_pct;
      L.grid_bs = L.grid_bs && L.diff_ok;  // all batch-size dependence sits in the same nodes
      L.layout_var = L.layout_var && L.diff_ok;
    }
    if (n == 0 && p.num_groups > 1 && !p.sink_hash) L.cluster_x = g + 1;
    uint32_t lo = std::max<uint32_t>(8, p.min_blob_bytes) / 8, hi = std::max<uint32_t>(lo * 8, p.max_blob_bytes) / 8;
    for (int v = 0; v < 2; ++v) {
      uint32_t blob = 8 * (uint32_t)r.range(lo, hi);
      if (L.extra) {
        L.sizes[v].assign(1, blob);  // one arg buffer, params at 8-aligned in-kernel offsets
      } else {
        L.sizes[v] = split_blob(r, blob, p.max_params, p.ragged != 0);
      }
      make_kinds(r, L.sizes[v], p.pointer_frac, L.kinds[v]);
      L.base[v].resize(L.kinds[v].size());
      for (size_t w = 0; w < L.kinds[v].size(); ++w) L.base[v][w] = draw_word(r, L.kinds[v][w], iv);
      if (!L.layout_var) {
        L.sizes[1] = L.sizes[0];
        L.kinds[1] = L.kinds[0];
        L.base[1] = L.base[0];
        break;
      }
    }
  }
  for (uint32_t n = 0; n + 1 < N; ++n) grp.deps.push_back({n, n + 1});
  for (uint32_t n = 2; n < N; n += 10) grp.deps.push_back({n - 2, n});  // fan-in edges
  return grp;
}

void put_word(std::vector<uint8_t>& bytes, uint64_t at, uint32_t n, uint64_t v) {
  for (uint32_t b = 0; b < n; ++b) bytes[at + b] = (uint8_t)(v >> (8 * b));
}

std::vector<uint8_t> make_graph(const fdy_synth_params& p, const Group& grp, uint32_t gidx, uint32_t group,
                                bool is_base, uint32_t bs, const Intervals& iv, uint32_t group_first) {
  Rng r(mix(p.seed, gidx));
  double rate = p.diff_lo + (p.diff_hi - p.diff_lo) * r.unit();
  uint32_t run_lo = p.run_min_bytes / 8, run_hi = std::max(p.run_min_bytes, p.run_max_bytes) / 8;
  double mean_run = run_lo ? 0.5 * (run_lo + run_hi) : 1.0;
  // Differing words concentrated in diff_node_pct % of the kernel nodes keep
  // the graph's overall fraction of differing words.
  const double krate = p.diff_node_pct ? std::min(1.0, rate * 100.0 / p.diff_node_pct) : rate;
  double p_start = krate / mean_run;
  bool large_bs = gidx > group_first && (gidx - group_first) * 2 >= 1;  // every member but the base
  fdy::GraphSpec spec;
  spec.nodes.resize(grp.nodes.size());
  uint32_t run_left = 0;
  for (size_t n = 0; n < grp.nodes.size(); ++n) {
    const NodeLayout& L = grp.nodes[n];
    fdy::NodeSpec& s = spec.nodes[n];
    s.type = L.type;
    if (L.type == FDY_NODE_MEMSET) {
      s.memset_body.dst = L.memset_dst;
      s.memset_body.element_size = 4;
      s.memset_body.height = 1;
      s.memset_body.pitch = 0;
      s.memset_body.value = 0;
      s.memset_body.width = 256ull * bs;
      if (!is_base && r.unit() < rate) s.memset_body.dst = draw_pointer(r, iv, 0);
      continue;
    }
    if (L.type == FDY_NODE_MEMCPY) {
      s.memcpy_body.depth = 1;
      s.memcpy_body.height = 1;
      s.memcpy_body.width_bytes = 1024ull * bs;
      s.memcpy_body.dst = L.memcpy_dst;
      s.memcpy_body.src = L.memcpy_src;
      s.memcpy_body.dst_mem_type = FDY_MEMTYPE_DEVICE;
      s.memcpy_body.src_mem_type = FDY_MEMTYPE_DEVICE;
      continue;
    }
    if (L.type == FDY_NODE_EVENT_RECORD || L.type == FDY_NODE_EVENT_WAIT) {
      s.event_id = L.event_id;
      continue;
    }
    if (L.type != FDY_NODE_KERNEL) continue;
    int v = (L.layout_var && large_bs && (bs & 2)) ? 1 : 0;
    fdy_kernel_body& k = s.kernel;
    k.block[0] = L.block;
    k.block[1] = k.block[2] = 1;
    k.grid[0] = L.grid_bs ? L.grid[0] * ((bs + 15) / 16) : L.grid[0];
    k.grid[1] = L.grid[1];
    k.grid[2] = 1;
    k.shared_mem_bytes = L.shmem;
    k.binary_hash = L.binary_hash;
    k.max_dynamic_shared = (int32_t)L.shmem;
    k.preferred_carveout = -1;
    if (L.cluster_x) {
      k.kna_flags = FDY_KNA_CLUSTER_DIM;
      k.kna_cluster[0] = L.cluster_x;
      k.kna_cluster[1] = 1;
      k.kna_cluster[2] = 1;
    }
    s.name = L.name;
    const auto& sizes = L.sizes[v];
    const auto& kinds = L.kinds[v];
    const auto& base = L.base[v];
    uint64_t total = 0;
    for (uint32_t sz : sizes) total += sz;
    std::vector<uint8_t> bytes(total);
    uint64_t at = 0, w = 0;
    for (uint32_t sz : sizes) {
      for (uint32_t off = 0; off < sz; off += 8, ++w) {
        uint64_t val = base[w];
        if (!is_base && L.diff_ok) {
          bool hit;
          if (run_lo) {
            if (!run_left && r.unit() < p_start) run_left = (uint32_t)r.range(run_lo, run_hi);
            hit = run_left > 0;
            if (run_left) --run_left;
          } else {
            hit = r.unit() < krate;
          }
          if (hit) {
            uint64_t nv = draw_word(r, kinds[w], iv);
            if (nv == val) nv ^= (kinds[w] == W_PTR) ? 16 : 1;
            val = nv;
          }
        }
        put_word(bytes, at + off, std::min<uint32_t>(8, sz - off), val);
      }
      at += sz;
    }
    if (L.extra) {
      s.extra_style = true;
      s.arg_buffer = bytes;
      uint32_t o = 0;
      for (uint32_t q = 0; q < total / 8 && q < 8; ++q) {  // descriptors of the first params
        s.extra_params.push_back({o, 8});
        o += 8;
      }
    } else {
      s.param_sizes = sizes;
      s.param_bytes = std::move(bytes);
    }
  }
  spec.deps = grp.deps;
  (void)group;
  spec.alloc_events = "{\"start_base_addr\":" + std::to_string(p.region_base) +
                      ",\"events\":[{\"type\":\"alloc\",\"size\":1048576,\"ptr\":" +
                      std::to_string(p.region_base) + "}]}";
  spec.topology_key = fdy::topology_key_save_rule(spec);
  return fdy::write_cugraph(spec);
}

template <typename F>
void parallel_for(uint32_t n, uint32_t threads, F&& f) {
  if (threads == 0) threads = std::max(1u, std::thread::hardware_concurrency());
  threads = std::min(threads, std::max(1u, n));
  std::atomic<uint32_t> next{0};
  std::vector<std::thread> pool;
  for (uint32_t t = 0; t < threads; ++t)
    pool.emplace_back([&] {
      for (uint32_t i; (i = next.fetch_add(1)) < n;) f(i);
    });
  for (auto& t : pool) t.join();
}

}  // namespace

struct fdy_synth : Synth {};

extern "C" {

const char* fdy_synth_last_error(void) { return g_err.c_str(); }

int fdy_synth_preset(uint32_t preset, fdy_synth_params* o) {
  if (!o) return fail("null params");
  std::memset(o, 0, sizeof(*o));
  o->preset = preset;
  o->seed = 0x5EED0000ull + preset;
  o->region_base = 0x7f0000000000ull;
  o->new_base = 0x7e0000000000ull;
  o->interval_granule = 512;
  o->max_params = 16;
  switch (preset) {
    case 1:
      o->num_graphs = 64; o->num_groups = 1; o->nodes_per_graph = 120;
      o->min_blob_bytes = 64; o->max_blob_bytes = 512; o->max_params = 8;
      o->pointer_frac = 0.30; o->diff_lo = o->diff_hi = 0.05;
      o->region_size = 4ull << 30; o->num_intervals = 1;
      break;
    case 2:
      o->num_graphs = 256; o->num_groups = 4; o->nodes_per_graph = 1200;
      o->min_blob_bytes = 32; o->max_blob_bytes = 1024; o->max_params = 16;
      o->pointer_frac = 0.25; o->diff_lo = o->diff_hi = 0.03; o->grid_bs_pct = 20;
      o->region_size = 64ull << 30; o->num_intervals = 40000;
      o->interval_min = 512; o->interval_max = 256ull << 20;
      break;
    case 3:
      o->num_graphs = 256; o->num_groups = 16; o->nodes_per_graph = 3000;
      // Up to 40 params per kernel (grouped-GEMM descriptor arrays take many).
      o->min_blob_bytes = 32; o->max_blob_bytes = 4096; o->max_params = 40;
      o->memset_pct = 10; o->memcpy_pct = 5; o->grid_bs_pct = 20;
      o->pointer_frac = 0.25; o->diff_lo = o->diff_hi = 0.10;
      o->run_min_bytes = 64; o->run_max_bytes = 256;
      o->region_size = 64ull << 30; o->num_intervals = 40000;
      o->interval_min = 512; o->interval_max = 256ull << 20;
      break;
    case 4:
      o->num_graphs = 0; o->num_words = (1ull << 30) / 8; o->pointer_frac = 0.40;
      o->boundary_frac = 0.01; o->region_size = 200ull << 30; o->num_intervals = 2000000;
      o->interval_granule = 256; o->interval_min = 256; o->interval_max = 64ull << 20;
      break;
    case 5:
      o->num_graphs = 1024; o->num_groups = 32; o->nodes_per_graph = 5000;
      o->min_blob_bytes = 64; o->max_blob_bytes = 3064; o->max_params = 16;
      o->pointer_frac = 0.25; o->diff_lo = 0.01; o->diff_hi = 0.08; o->grid_bs_pct = 20;
      o->region_size = 64ull << 30; o->num_intervals = 40000;
      o->interval_min = 512; o->interval_max = 256ull << 20;
      break;
    default:
      return fail("unknown preset " + std::to_string(preset));
  }
  return 0;
}

int fdy_synth_create(const fdy_synth_params* p, uint32_t num_threads, fdy_synth** out) {
  if (!p || !out) return fail("null argument");
  if (p->sink_hash && p->num_groups > 64) return fail("sink mode tells at most 64 groups apart");
  if (p->num_groups == 0 && p->num_graphs) return fail("num_groups must be >= 1");
  if (p->num_intervals == 0) return fail("num_intervals must be >= 1");
  if (p->region_size / std::max<uint32_t>(16, p->interval_granule) < p->num_intervals)
    return fail("region too small for the interval count");
  try {
    auto s = std::make_unique<fdy_synth>();
    s->p = *p;
    Rng r(mix(p->seed, 0xFFFFFFFF00000000ull));
    make_intervals(*p, r, s->iv);
    if (p->num_words) {
      s->words.resize(p->num_words);
      const uint64_t chunk = 1 << 20;
      uint32_t nchunks = (uint32_t)((p->num_words + chunk - 1) / chunk);
      parallel_for(nchunks, num_threads, [&](uint32_t c) {
        Rng wr(mix(p->seed ^ 0xAB0DEull, c));
        uint64_t end = std::min<uint64_t>(p->num_words, (uint64_t)(c + 1) * chunk);
        for (uint64_t i = (uint64_t)c * chunk; i < end; ++i) {
          if (wr.unit() < p->pointer_frac) s->words[i] = draw_pointer(wr, s->iv, p->boundary_frac);
          else s->words[i] = draw_word(wr, wr.below(2) ? W_U32 : W_F32, s->iv);
        }
      });
    }
    uint32_t G = p->num_graphs;
    s->bs.resize(G);
    uint32_t step = std::max<uint32_t>(1, 512 / std::max<uint32_t>(1, G));
    for (uint32_t i = 0; i < G; ++i) s->bs[i] = i == 0 ? 1 : i * step;
    std::vector<Group> groups(G ? p->num_groups : 0);
    parallel_for((uint32_t)groups.size(), num_threads, [&](uint32_t k) { groups[k] = make_group(*p, k, s->iv); });
    s->images.resize(G);
    parallel_for(G, num_threads, [&](uint32_t i) {
      uint32_t k = (uint32_t)((uint64_t)i * p->num_groups / G);
      uint32_t first = (uint32_t)(((uint64_t)k * G + p->num_groups - 1) / p->num_groups);
      s->images[i] = make_graph(*p, groups[k], i, k, i == first, s->bs[i], s->iv, first);
    });
    *out = s.release();
    return 0;
  } catch (const std::exception& e) {
    return fail(std::string("synthetic archive: ") + e.what());
  }
}

int fdy_synth_destroy(fdy_synth* s) {
  delete s;
  return 0;
}

uint32_t fdy_synth_num_graphs(const fdy_synth* s) { return s ? (uint32_t)s->images.size() : 0; }

int fdy_synth_image(const fdy_synth* s, uint32_t i, const uint8_t** data, uint64_t* size) {
  if (!s || i >= s->images.size()) return fail("graph index out of range");
  *data = s->images[i].data();
  *size = s->images[i].size();
  return 0;
}

int fdy_synth_batch_size(const fdy_synth* s, uint32_t i, uint32_t* bs) {
  if (!s || i >= s->bs.size()) return fail("graph index out of range");
  *bs = s->bs[i];
  return 0;
}

int fdy_synth_intervals(const fdy_synth* s, const uint64_t** lo, const uint64_t** hi, const uint64_t** nlo,
                        uint64_t* n) {
  if (!s) return fail("null synth");
  *lo = s->iv.lo.data();
  *hi = s->iv.hi.data();
  *nlo = s->iv.nlo.data();
  *n = s->iv.lo.size();
  return 0;
}

int fdy_synth_words(const fdy_synth* s, const uint64_t** words, uint64_t* n) {
  if (!s) return fail("null synth");
  *words = s->words.data();
  *n = s->words.size();
  return 0;
}

int fdy_synth_write_dir(const fdy_synth* s, const char* dir) {
  if (!s || !dir) return fail("null argument");
  for (size_t i = 0; i < s->images.size(); ++i) {
    std::string path = std::string(dir) + "/graph_" + std::to_string(i) + ".cugraph";
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return fail("cannot write " + path);
    size_t w = std::fwrite(s->images[i].data(), 1, s->images[i].size(), f);
    std::fclose(f);
    if (w != s->images[i].size()) return fail("short write " + path);
  }
  return 0;
}

int fdy_synth_switch_sequence(uint64_t seed, uint32_t num_graphs, uint32_t n, uint32_t* out) {
  if (!out || !num_graphs) return fail("bad argument");
  Rng r(seed);
  for (uint32_t i = 0; i < n; ++i) out[i] = (uint32_t)r.below(num_graphs);
  return 0;
}

}  // extern "C"
