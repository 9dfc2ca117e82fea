// oracle.cpp -- CPU restatement of the reference's graph-restore (LOAD) path.
//
// TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
// the cpu_baseline leg of bench.py, never by the product.
//
// What it follows (reference paths relative to the reference root):
//   format, section views      include/BinaryGraphFormat.h:37-284, csrc/BinaryGraphIO.cpp:710-737
//   saved topology key         include/BinaryGraphFormat.h:274-278
//   recomputed key (LOAD rule) csrc/CUDAGraphParallel.cpp:1798-1841 on the JSON twin that
//                              csrc/BinaryGraphIO.cpp:452-651 reconstructs
//   grouping                   csrc/CUDAGraphParallel.cpp:1788-1851 (binary graphs: saved key,
//                              "" when empty, because the shell's node list is empty, 1642-1644)
//   manifest grouping          csrc/CUDAGraphParallel.cpp:1727-1786
//   param extraction           csrc/CUDAGraphParallel.cpp:1391-1409
//   effective launch attrs     csrc/CUDAGraphParallel.cpp:1211-1389
//   switch end state           csrc/CUDAGraph.cpp:340-461 (every node ends with the target's params)
//   CRC-64/XZ                  csrc/hook.cpp:315-321 (Boost crc_optimal<64,0x42F0E1EBA9EA3693,~0,~0,true,true>)
// The diff, the relocation and the digests have no reference counterpart;
// their definitions are the build's and are restated here independently of
// the product code.
//
// How each part is pinned (tests/test_oracle_*.py):
//   crc64            textbook check value crc("123456789") = 0x995DC9BBDF1939FA, and an
//                    independent bit-serial Python CRC on random inputs
//   format / key     hand-assembled byte fixtures (tests/golden/), every offset derived from
//                    the reference header text; hand-written key strings
//   grouping         brute force over tiny archives; manifest cases from the reference's rules
//   extraction       round trip: concatenated params == the param-data slice
//   relocation       brute-force linear scan on small tables; identity at delta 0;
//                    hand cases at lo, hi-1, hi, lo-1 for both policies
//   diff             apply(R_t, O_g) == R_g, minimality, canonical order, O_t == {}
//   switch           live image == R_g after seeded switch sequences
//   digests          same byte streams through the independent Python CRC
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cctype>
#include <exception>
#include <chrono>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <functional>
#include <future>
#include <memory>
#include <mutex>
#include <queue>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

thread_local std::string g_err;

// ---- field access (the entries are packed; read through memcpy) ---------

template <typename T>
T rd(const uint8_t* p, uint64_t off) {
  T v;
  std::memcpy(&v, p + off, sizeof(T));
  return v;
}

constexpr uint64_t kHeader = 64, kSecEntry = 24, kNode = 168, kParam = 8, kDep = 8;
enum { S_STR = 0, S_NODE, S_DEP, S_PIDX, S_PDATA, S_ARG, S_COMMON, S_GEN, S_AE, S_OT, S_KEY, S_COUNT };
enum { N_KERNEL = 0, N_MEMSET, N_MEMCPY, N_EVREC, N_EVWAIT, N_EMPTY };
enum : uint32_t {
  KNA_CLUSTER = 1, KNA_PREF = 2, KNA_SCHED = 4, KNA_COOP = 8, KNA_PRIO = 16,
  KNA_MSD = 32, KNA_MAP = 64, KNA_CARVE = 128
};
constexpr uint32_t HDR_COMMON = 1;

// ---- CRC-64/XZ, byte at a time ------------------------------------------

struct CrcTable {
  uint64_t t[256];
  CrcTable() {
    const uint64_t poly = 0xC96C5795D7870F42ull;  // 0x42F0E1EBA9EA3693 bit-reversed
    for (int i = 0; i < 256; ++i) {
      uint64_t c = (uint64_t)i;
      for (int k = 0; k < 8; ++k) c = (c & 1) ? (c >> 1) ^ poly : c >> 1;
      t[i] = c;
    }
  }
};
const CrcTable& crc_table() {
  static CrcTable t;
  return t;
}
struct Crc {
  uint64_t c = ~0ull;
  void feed(const uint8_t* p, uint64_t n) {
    const uint64_t* t = crc_table().t;
    for (uint64_t i = 0; i < n; ++i) c = t[(c ^ p[i]) & 0xFF] ^ (c >> 8);
  }
  void feed_u32(uint32_t v) {
    uint8_t b[4];
    std::memcpy(b, &v, 4);
    feed(b, 4);
  }
  void feed_u64(uint64_t v) {
    uint8_t b[8];
    std::memcpy(b, &v, 8);
    feed(b, 8);
  }
  uint64_t value() const { return ~c; }
};

// ---- one archive --------------------------------------------------------

struct View {
  const uint8_t* d = nullptr;
  uint64_t size = 0;
  uint32_t flags = 0, num_nodes = 0, num_deps = 0;
  uint64_t off[S_COUNT]{}, sz[S_COUNT]{};
};

bool open_view(const uint8_t* d, uint64_t size, View* v) {
  static const uint8_t magic[8] = {'C', 'U', 'G', 'R', 'A', 'P', 'H', 0};
  if (size < kHeader || std::memcmp(d, magic, 8) != 0 || rd<uint32_t>(d, 8) != 1) {
    g_err = "invalid header";
    return false;
  }
  v->d = d;
  v->size = size;
  v->flags = rd<uint32_t>(d, 12);
  v->num_nodes = rd<uint32_t>(d, 16);
  v->num_deps = rd<uint32_t>(d, 20);
  uint32_t nsec = rd<uint32_t>(d, 28);
  if (nsec < S_COUNT || kHeader + nsec * kSecEntry > size) {
    g_err = "section directory";
    return false;
  }
  for (int i = 0; i < S_COUNT; ++i) {
    v->off[i] = rd<uint64_t>(d, kHeader + i * kSecEntry + 8);
    v->sz[i] = rd<uint64_t>(d, kHeader + i * kSecEntry + 16);
    if (v->off[i] > size || v->sz[i] > size - v->off[i]) {
      g_err = "section out of bounds";
      return false;
    }
  }
  if (v->sz[S_NODE] < (uint64_t)v->num_nodes * kNode || v->sz[S_DEP] < (uint64_t)v->num_deps * kDep) {
    g_err = "short table";
    return false;
  }
  return true;
}

const uint8_t* node_at(const View& v, uint32_t n) { return v.d + v.off[S_NODE] + (uint64_t)n * kNode; }

// Effective launch attributes of a kernel node, merged the way
// prepare_on_demand_graph_binary does (csrc/CUDAGraphParallel.cpp:1211-1389).
struct Attrs {
  int32_t has_cluster = 0, cx = 0, cy = 0, cz = 0;
  int32_t has_pref = 0, px = 0, py = 0, pz = 0;
  int32_t sched = -1, coop = -1, prio = -1, msd = -1;
  int32_t has_map = 0, map_def = 0, map_remote = 0;
  int32_t has_carve = 0, carve = 0;
  bool operator==(const Attrs& o) const { return std::memcmp(this, &o, sizeof(Attrs)) == 0; }
};

// Fields of the kna block (flags at +0, cluster +4.., preferred +16.., sched +28,
// coop +32, prio +36, msd +40, map bytes +44/+45, carveout +48) -- the same
// relative layout in the node's kernel body (from entry offset 76) and in the
// common-attrs section.
Attrs attrs_from_block(const uint8_t* b) {
  Attrs a;
  uint32_t f = rd<uint32_t>(b, 0);
  if (f & KNA_CLUSTER) {
    a.has_cluster = 1;
    a.cx = rd<int32_t>(b, 4);
    a.cy = rd<int32_t>(b, 8);
    a.cz = rd<int32_t>(b, 12);
  }
  if (f & KNA_PREF) {
    a.has_pref = 1;
    a.px = rd<int32_t>(b, 16);
    a.py = rd<int32_t>(b, 20);
    a.pz = rd<int32_t>(b, 24);
  }
  if (f & KNA_SCHED) a.sched = rd<int32_t>(b, 28);
  if (f & KNA_COOP) a.coop = rd<int32_t>(b, 32);
  if (f & KNA_PRIO) a.prio = rd<int32_t>(b, 36);
  if (f & KNA_MSD) a.msd = rd<int32_t>(b, 40);
  if (f & KNA_MAP) {
    a.has_map = 1;
    a.map_def = b[44];
    a.map_remote = b[45];
  }
  if (f & KNA_CARVE) {
    a.has_carve = 1;
    a.carve = rd<int32_t>(b, 48);
  }
  return a;
}

// A planted mistake in the merge below (orc_set_mutation; 0 = none).  Test
// infrastructure for showing that the attribute fixtures pin the merge:
// each mutation must change an effective attribute or a DESC flag they hold.
int g_mutation = 0;

// Per-node attrs p merged over a (csrc/CUDAGraphParallel.cpp:1345-1373):
// dims and the map/carveout when flagged, scalars when not negative.
void merge_over(Attrs& a, const Attrs& p) {
  if (p.has_cluster) { a.has_cluster = 1; a.cx = p.cx; a.cy = p.cy; a.cz = p.cz; }
  if (p.has_pref) { a.has_pref = 1; a.px = p.px; a.py = p.py; a.pz = p.pz; }
  if (p.sched >= 0) a.sched = p.sched;
  if (p.coop >= 0) a.coop = p.coop;
  if (p.prio >= 0) a.prio = p.prio;
  if (p.msd >= 0) a.msd = p.msd;
  if (p.has_map) { a.has_map = 1; a.map_def = p.map_def; a.map_remote = p.map_remote; }
  if (p.has_carve) { a.has_carve = 1; a.carve = p.carve; }
}

Attrs effective_attrs(const View& v, const uint8_t* e) {
  Attrs a;
  const bool has_common = v.flags & HDR_COMMON && v.sz[S_COMMON] >= 52 && g_mutation != 5;  // 5: common ignored
  if (has_common) a = attrs_from_block(v.d + v.off[S_COMMON]);
  if (rd<uint32_t>(e, 76) != 0) {
    Attrs p = attrs_from_block(e + 76);
    if (g_mutation == 1 && has_common) {  // 1: common attrs win over per-node ones
      Attrs c = a;
      a = Attrs();
      merge_over(a, p);
      merge_over(a, c);
    } else if (g_mutation == 4) {  // 4: per-node attrs replace the common ones wholesale
      a = p;
    } else {
      merge_over(a, p);
      if (g_mutation == 2) {  // 2: flagged per-node scalars override even when negative
        const uint32_t f = rd<uint32_t>(e, 76);
        if (f & KNA_SCHED) a.sched = p.sched;
        if (f & KNA_COOP) a.coop = p.coop;
        if (f & KNA_PRIO) a.prio = p.prio;
        if (f & KNA_MSD) a.msd = p.msd;
      }
    }
  }
  // Required cluster dims win over both (1376-1385); zero dims become 1.
  int32_t w = rd<int32_t>(e, 64), h = rd<int32_t>(e, 68), dd = rd<int32_t>(e, 72);
  if ((w > 0 || h > 0 || dd > 0) && g_mutation != 3) {  // 3: required cluster ignored
    a.has_cluster = 1;
    const int32_t one = g_mutation == 6 ? 0 : 1;  // 6: zero dims stay 0
    a.cx = w > 0 ? w : one;
    a.cy = h > 0 ? h : one;
    a.cz = dd > 0 ? dd : one;
  }
  return a;
}

// Cluster dims the LOAD fallback puts in the key (csrc/CUDAGraphParallel.cpp:1807-1833).
void load_rule_dims(const View& v, const uint8_t* e, uint32_t c[3]) {
  c[0] = c[1] = c[2] = 0;
  if (rd<uint32_t>(e, 76) & KNA_CLUSTER) {
    c[0] = rd<uint32_t>(e, 80);
    c[1] = rd<uint32_t>(e, 84);
    c[2] = rd<uint32_t>(e, 88);
  }
  if (c[0] == 0 && (v.flags & HDR_COMMON) && v.sz[S_COMMON] >= 52) {
    const uint8_t* ca = v.d + v.off[S_COMMON];
    if (rd<uint32_t>(ca, 0) & KNA_CLUSTER) {
      c[0] = rd<uint32_t>(ca, 4);
      c[1] = rd<uint32_t>(ca, 8);
      c[2] = rd<uint32_t>(ca, 12);
    }
  }
  if (c[0] == 0) {  // func_attrs always carries the three required_cluster fields
    c[0] = rd<uint32_t>(e, 64);
    c[1] = rd<uint32_t>(e, 68);
    c[2] = rd<uint32_t>(e, 72);
  }
}

const char* type_name(uint8_t t) {
  static const char* names[] = {"KernelNode", "MemsetNode", "MemcpyNode", "EventRecordNode", "EventWaitNode", "EmptyNode"};
  return t < 6 ? names[t] : "";
}

std::string recomputed_key(const View& v) {
  std::string key;
  for (uint32_t n = 0; n < v.num_nodes; ++n) {
    if (n) key += ',';
    const uint8_t* e = node_at(v, n);
    key += type_name(e[4]);
    if (e[4] != N_KERNEL) continue;
    uint32_t c[3];
    load_rule_dims(v, e, c);
    if (c[0] || c[1] || c[2])
      key += ":C" + std::to_string(c[0]) + "_" + std::to_string(c[1]) + "_" + std::to_string(c[2]);
    else
      key += ":0";
  }
  return key;
}

std::string saved_key(const View& v) { return std::string((const char*)v.d + v.off[S_KEY], v.sz[S_KEY]); }

// A kernel node's params: (section-relative source offset, size, section).
struct ParamRef {
  uint64_t off;
  uint32_t size;
  int sec;
};

// Returns false if any referenced range lies outside its section.
bool node_params(const View& v, const uint8_t* e, std::vector<ParamRef>* out, bool* extra) {
  out->clear();
  uint32_t pio = rd<uint32_t>(e, 128), np = rd<uint32_t>(e, 132);
  uint32_t ao = rd<uint32_t>(e, 136), as = rd<uint32_t>(e, 140);
  uint32_t no = rd<uint32_t>(e, 44), nl = rd<uint32_t>(e, 48);
  *extra = ao != 0xFFFFFFFFu;
  bool ok = (uint64_t)no + nl <= v.sz[S_STR];
  if ((uint64_t)pio + (uint64_t)np * kParam > v.sz[S_PIDX]) return false;
  if (*extra) {
    if ((uint64_t)ao + as > v.sz[S_ARG]) return false;
    out->push_back({ao, as, S_ARG});
    return ok;
  }
  const uint8_t* pi = v.d + v.off[S_PIDX] + pio;
  for (uint32_t j = 0; j < np; ++j) {
    uint32_t o = rd<uint32_t>(pi, (uint64_t)j * 8), s = rd<uint32_t>(pi, (uint64_t)j * 8 + 4);
    if ((uint64_t)o + s > v.sz[S_PDATA]) return false;
    out->push_back({o, s, S_PDATA});
  }
  return ok;
}

uint64_t reloc(uint64_t w, const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo, uint64_t n,
               uint32_t policy) {
  if (n == 0) return w;
  const uint64_t* p = std::upper_bound(lo, lo + n, w);  // first lo > w
  if (p == lo) return w;
  uint64_t i = (uint64_t)(p - lo) - 1;
  bool inside = policy == 1 ? w <= hi[i] : w < hi[i];
  return inside ? w - lo[i] + nlo[i] : w;
}

struct Table {
  const uint64_t *lo = nullptr, *hi = nullptr, *nlo = nullptr;
  uint64_t n = 0;
  uint32_t policy = 0;
  uint64_t operator()(uint64_t w) const { return reloc(w, lo, hi, nlo, n, policy); }
};

// Per-node layout signature; nodes compare equal in layout iff these match.
struct Layout {
  uint8_t type = N_EMPTY;
  bool bad = false, extra = false;
  std::vector<uint32_t> sizes;
  bool operator==(const Layout& o) const {
    return !bad && !o.bad && type == o.type && extra == o.extra && sizes == o.sizes;
  }
};

struct Graph {
  View v;
  std::vector<Layout> layout;
  std::vector<uint32_t> words;    // per node
  std::vector<uint32_t> woff;     // N+1
  std::vector<uint64_t> image;    // relocated param image
  std::vector<uint8_t> flags;
  std::vector<uint64_t> ptrs;     // 2N relocated memset/memcpy pointers
  uint64_t dig[4]{};
  uint32_t status = 0;
  uint32_t tmpl = 0;
  uint64_t param_bytes = 0;
  std::vector<orc_override> ovr;
};

constexpr uint8_t F_LAYOUT = 1, F_DESC = 2, F_RAGGED = 4, F_TEMPLATE = 8;
constexpr uint32_t ST_TYPE = 1, ST_BAD = 2, ST_COLLISION = 8, ST_COUNT = 0x10;

// Pass 1 of a graph: layout, relocated image, pointers, digests.
void build_graph(Graph& g, const Table& tab) {
  const View& v = g.v;
  uint32_t N = v.num_nodes;
  g.layout.assign(N, Layout());
  g.words.assign(N, 0);
  g.woff.assign(N + 1, 0);
  g.flags.assign(N, 0);
  g.ptrs.assign(2 * (size_t)N, 0);
  g.image.clear();
  Crc ck, ce, ct, cn;
  ck.feed(v.d + v.off[S_KEY], v.sz[S_KEY]);
  ce.feed(v.d + v.off[S_DEP], (uint64_t)v.num_deps * kDep);
  std::vector<ParamRef> ps;
  for (uint32_t n = 0; n < N; ++n) {
    const uint8_t* e = node_at(v, n);
    uint8_t type = e[4];
    Layout& L = g.layout[n];
    L.type = type;
    uint32_t c[3] = {0, 0, 0};
    uint64_t kent_hash = 0, kent_name = 0;
    if (type == N_KERNEL) {
      load_rule_dims(v, e, c);
      bool extra = false;
      bool ok = node_params(v, e, &ps, &extra);
      L.extra = extra;
      kent_hash = rd<uint64_t>(e, 36);
      uint32_t no = rd<uint32_t>(e, 44), nl = rd<uint32_t>(e, 48);
      if ((uint64_t)no + nl <= v.sz[S_STR]) {
        Crc cname;
        cname.feed(v.d + v.off[S_STR] + no, nl);
        kent_name = cname.value();
      }
      if (!ok) {
        L.bad = true;
        g.status |= ST_BAD;
      } else {
        uint64_t prev_end = ps.empty() ? 0 : ps[0].off;
        bool ragged = false;
        for (const ParamRef& p : ps) {
          L.sizes.push_back(p.size);
          if ((p.size & 7) || (p.off & 7) || p.off != prev_end) ragged = true;
          prev_end = p.off + p.size;
          const uint8_t* src = v.d + v.off[p.sec] + p.off;
          for (uint32_t b = 0; b < p.size; b += 8) {
            uint64_t w = 0;
            uint32_t width = std::min<uint32_t>(8, p.size - b);
            std::memcpy(&w, src + b, width);
            g.image.push_back(width == 8 ? tab(w) : w);
            g.words[n]++;
          }
          g.param_bytes += p.size;
        }
        if (ragged) g.flags[n] |= F_RAGGED;
      }
    } else if (type == N_MEMSET) {
      g.ptrs[2 * n] = tab(rd<uint64_t>(e, 8));
    } else if (type == N_MEMCPY) {
      uint64_t dst = rd<uint64_t>(e, 32), src = rd<uint64_t>(e, 96);
      int32_t dt = rd<int32_t>(e, 88), st = rd<int32_t>(e, 152);
      g.ptrs[2 * n] = (dt == 2 || dt == 4) ? tab(dst) : dst;
      g.ptrs[2 * n + 1] = (st == 2 || st == 4) ? tab(src) : src;
    }
    g.woff[n + 1] = g.woff[n] + g.words[n];
    uint8_t rec[16] = {0};
    rec[0] = type;
    std::memcpy(rec + 4, c, 12);
    ct.feed(rec, 16);
    cn.feed_u64(kent_hash);
    cn.feed_u64(kent_name);
  }
  g.dig[0] = ck.value();
  g.dig[1] = ce.value();
  g.dig[2] = ct.value();
  g.dig[3] = cn.value();
}

bool same_name(const View& a, const uint8_t* ea, const View& b, const uint8_t* eb) {
  uint32_t ao = rd<uint32_t>(ea, 44), al = rd<uint32_t>(ea, 48);
  uint32_t bo = rd<uint32_t>(eb, 44), bl = rd<uint32_t>(eb, 48);
  if (al != bl) return false;
  if ((uint64_t)ao + al > a.sz[S_STR] || (uint64_t)bo + bl > b.sz[S_STR]) return false;
  return std::memcmp(a.d + a.off[S_STR] + ao, b.d + b.off[S_STR] + bo, al) == 0;
}

// Does node n's descriptor differ between g and its template t?
bool desc_differs(const Graph& g, const Graph& t, uint32_t n) {
  const uint8_t* a = node_at(g.v, n);
  const uint8_t* b = node_at(t.v, n);
  if (a[4] != b[4]) return true;
  switch (a[4]) {
    case N_KERNEL:
      if (std::memcmp(a + 8, b + 8, 36) != 0) return true;    // block, grid, shmem, binary_hash
      if (std::memcmp(a + 52, b + 52, 24) != 0) return true;  // func attrs
      if (!same_name(g.v, a, t.v, b)) return true;
      return !(effective_attrs(g.v, a) == effective_attrs(t.v, b));
    case N_MEMSET:
      return g.ptrs[2 * n] != t.ptrs[2 * n] || rd<uint32_t>(a, 16) != rd<uint32_t>(b, 16) ||
             std::memcmp(a + 24, b + 24, 16) != 0 || rd<uint32_t>(a, 40) != rd<uint32_t>(b, 40) ||
             rd<uint64_t>(a, 48) != rd<uint64_t>(b, 48);
    case N_MEMCPY:
      return g.ptrs[2 * n] != t.ptrs[2 * n] || g.ptrs[2 * n + 1] != t.ptrs[2 * n + 1] ||
             std::memcmp(a + 8, b + 8, 24) != 0 || std::memcmp(a + 40, b + 40, 52) != 0 ||
             std::memcmp(a + 104, b + 104, 52) != 0;
    case N_EVREC:
    case N_EVWAIT:
      return rd<int32_t>(a, 8) != rd<int32_t>(b, 8);
    default:
      return false;
  }
}

// Pass 2 of a non-template graph: flags against the template and overrides.
void diff_graph(Graph& g, const Graph& t) {
  uint32_t N = g.v.num_nodes, NT = t.v.num_nodes;
  if (N != NT) g.status |= ST_COUNT;
  if (g.dig[2] != t.dig[2]) g.status |= ST_TYPE;
  for (uint32_t n = 0; n < N; ++n) {
    if (n >= NT) {
      g.flags[n] |= F_LAYOUT | F_DESC;
      continue;
    }
    bool layout = !(g.layout[n] == t.layout[n]);
    if (layout) g.flags[n] |= F_LAYOUT;
    if (desc_differs(g, t, n)) g.flags[n] |= F_DESC;
    if (layout) continue;
    for (uint32_t k = 0; k < g.words[n]; ++k) {
      uint64_t a = g.image[g.woff[n] + k], b = t.image[t.woff[n] + k];
      if (a != b) g.ovr.push_back({t.woff[n] + k, n, a});
    }
  }
}

template <typename F>
void parallel_for(uint32_t n, uint32_t threads, F&& f) {
  threads = std::max(1u, std::min(threads ? threads : 1u, std::max(1u, n)));
  if (threads == 1) {
    for (uint32_t i = 0; i < n; ++i) f(i);
    return;
  }
  std::atomic<uint32_t> next{0};
  std::vector<std::thread> pool;
  for (uint32_t k = 0; k < threads; ++k)
    pool.emplace_back([&] {
      for (uint32_t i; (i = next.fetch_add(1)) < n;) f(i);
    });
  for (auto& th : pool) th.join();
}

// Minimal JSON reader for graph_manifest.json (objects, arrays, strings,
// numbers, literals); enough to walk topology_groups.
struct Json {
  enum K { NUL, BOOL, NUM, STR, ARR, OBJ } k = NUL;
  std::string s;
  std::vector<Json> a;
  std::vector<std::pair<std::string, Json>> o;
  const Json* get(const char* key) const {
    for (auto& kv : o)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const char* p;
  const char* e;
  bool ok = true;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool str(std::string* out) {
    if (p >= e || *p != '"') return false;
    ++p;
    while (p < e && *p != '"') {
      if (*p == '\\') {
        ++p;
        if (p >= e) return false;
        char c = *p;
        if (c == 'n') out->push_back('\n');
        else if (c == 't') out->push_back('\t');
        else if (c == 'u') {
          if (e - p < 5) return false;
          unsigned v = (unsigned)std::stoul(std::string(p + 1, 4), nullptr, 16);
          if (v < 0x80) out->push_back((char)v);
          else if (v < 0x800) { out->push_back((char)(0xC0 | (v >> 6))); out->push_back((char)(0x80 | (v & 0x3F))); }
          else { out->push_back((char)(0xE0 | (v >> 12))); out->push_back((char)(0x80 | ((v >> 6) & 0x3F))); out->push_back((char)(0x80 | (v & 0x3F))); }
          p += 4;
        } else out->push_back(c);
        ++p;
      } else {
        out->push_back(*p++);
      }
    }
    if (p >= e) return false;
    ++p;
    return true;
  }
  bool val(Json* j, int depth) {
    if (depth > 64) return false;
    ws();
    if (p >= e) return false;
    if (*p == '{') {
      j->k = Json::OBJ;
      ++p;
      ws();
      if (p < e && *p == '}') { ++p; return true; }
      for (;;) {
        ws();
        std::string key;
        if (!str(&key)) return false;
        ws();
        if (p >= e || *p != ':') return false;
        ++p;
        Json child;
        if (!val(&child, depth + 1)) return false;
        j->o.emplace_back(std::move(key), std::move(child));
        ws();
        if (p < e && *p == ',') { ++p; continue; }
        if (p < e && *p == '}') { ++p; return true; }
        return false;
      }
    }
    if (*p == '[') {
      j->k = Json::ARR;
      ++p;
      ws();
      if (p < e && *p == ']') { ++p; return true; }
      for (;;) {
        Json child;
        if (!val(&child, depth + 1)) return false;
        j->a.push_back(std::move(child));
        ws();
        if (p < e && *p == ',') { ++p; continue; }
        if (p < e && *p == ']') { ++p; return true; }
        return false;
      }
    }
    if (*p == '"') {
      j->k = Json::STR;
      return str(&j->s);
    }
    const char* st = p;
    while (p < e && (std::isalnum((unsigned char)*p) || *p == '-' || *p == '+' || *p == '.')) ++p;
    if (p == st) return false;
    std::string lit(st, p);
    j->s = lit;
    j->k = (lit == "true" || lit == "false") ? Json::BOOL : lit == "null" ? Json::NUL : Json::NUM;
    return true;
  }
};

}  // namespace

struct orc_result {
  std::vector<Graph> g;
  std::vector<uint32_t> tmpl;
  std::vector<uint64_t> ovr_off;
  // live state per template: words, node sources, current graph
  std::unordered_map<uint32_t, std::vector<uint64_t>> live;
  std::unordered_map<uint32_t, std::vector<uint32_t>> live_src;
  std::unordered_map<uint32_t, uint32_t> current;
};

extern "C" {

const char* orc_last_error(void) { return g_err.c_str(); }

uint64_t orc_crc64(const uint8_t* data, uint64_t n) {
  Crc c;
  c.feed(data, n);
  return c.value();
}

int64_t orc_topology_key_saved(const uint8_t* image, uint64_t size, char* buf, uint64_t cap) {
  View v;
  if (!open_view(image, size, &v)) return -1;
  std::string k = saved_key(v);
  if (buf) std::memcpy(buf, k.data(), std::min<uint64_t>(cap, k.size()));
  return (int64_t)k.size();
}

int64_t orc_topology_key_recomputed(const uint8_t* image, uint64_t size, char* buf, uint64_t cap) {
  View v;
  if (!open_view(image, size, &v)) return -1;
  std::string k = recomputed_key(v);
  if (buf) std::memcpy(buf, k.data(), std::min<uint64_t>(cap, k.size()));
  return (int64_t)k.size();
}

int orc_group_by_keys(const char* const* keys, const uint64_t* lens, uint32_t n, uint32_t* out) {
  std::unordered_map<std::string, std::vector<uint32_t>> groups;
  for (uint32_t i = 0; i < n; ++i) groups[std::string(keys[i], lens[i])].push_back(i);
  for (uint32_t i = 0; i < n; ++i) out[i] = i;
  for (auto& kv : groups)
    for (size_t j = 1; j < kv.second.size(); ++j) out[kv.second[j]] = kv.second[0];
  return 0;
}

int orc_group_manifest(const char* text, uint64_t len, const char* const* names, uint32_t n, uint32_t* out) {
  Json root;
  JsonParser jp{text, text + len};
  try {
    if (!jp.val(&root, 0) || root.k != Json::OBJ) return -1;
  } catch (const std::exception&) {  // a malformed \u escape
    return -1;
  }
  const Json* groups = root.get("topology_groups");
  if (!groups || groups->k != Json::ARR) return -1;
  std::unordered_map<std::string, uint32_t> idx;
  for (uint32_t i = 0; i < n; ++i) idx[names[i]] = i;
  std::vector<uint32_t> res(n, UINT32_MAX);
  for (const Json& grp : groups->a) {
    if (grp.k != Json::OBJ) return -1;
    const Json* t = grp.get("template");
    if (!t || t->k != Json::STR) return -1;
    auto ti = idx.find(t->s);
    // Unknown template: the group is skipped before its members are read
    // (1754-1755), so they are not checked either.
    if (ti == idx.end()) continue;
    const Json* m = grp.get("members");
    if (!m || m->k != Json::ARR) return -1;
    // The template's own entry is left alone (1759, 1771): a template listed
    // as a member of an earlier group stays that group's member.
    for (const Json& mem : m->a) {
      if (mem.k != Json::STR) return -1;
      if (mem.s == t->s) continue;
      auto mi = idx.find(mem.s);
      if (mi == idx.end()) continue;
      res[mi->second] = ti->second;
    }
  }
  std::memcpy(out, res.data(), n * sizeof(uint32_t));
  return 0;
}

void orc_set_mutation(int m) { g_mutation = m; }

int orc_effective_attrs(const uint8_t* image, uint64_t size, uint32_t node, int32_t* out) {
  View v;
  if (!open_view(image, size, &v) || node >= v.num_nodes) return -1;
  const uint8_t* e = node_at(v, node);
  if (e[4] != N_KERNEL) return -1;
  const Attrs a = effective_attrs(v, e);
  static_assert(sizeof(Attrs) == 17 * sizeof(int32_t), "17 attribute fields");
  std::memcpy(out, &a, sizeof(Attrs));
  return 0;
}

int64_t orc_extract_node_params(const uint8_t* image, uint64_t size, uint32_t node, uint8_t* out, uint64_t cap) {
  View v;
  if (!open_view(image, size, &v) || node >= v.num_nodes) return -1;
  const uint8_t* e = node_at(v, node);
  if (e[4] != N_KERNEL) return 0;
  std::vector<ParamRef> ps;
  bool extra;
  if (!node_params(v, e, &ps, &extra)) return -1;
  uint64_t at = 0;
  for (const ParamRef& p : ps) {
    if (at + p.size > cap) return -1;
    std::memcpy(out + at, v.d + v.off[p.sec] + p.off, p.size);
    at += p.size;
  }
  return (int64_t)at;
}

int orc_restore(const uint8_t* const* images, const uint64_t* sizes, uint32_t n, const uint64_t* lo,
                const uint64_t* hi, const uint64_t* nlo, uint64_t n_iv, uint32_t policy,
                const uint32_t* template_of, uint32_t threads, orc_result** out) {
  auto r = std::make_unique<orc_result>();
  r->g.resize(n);
  for (uint32_t i = 0; i < n; ++i)
    if (!open_view(images[i], sizes[i], &r->g[i].v)) return -1;
  Table tab{lo, hi, nlo, n_iv, policy};
  parallel_for(n, threads, [&](uint32_t i) { build_graph(r->g[i], tab); });
  r->tmpl.resize(n);
  if (template_of) {
    std::memcpy(r->tmpl.data(), template_of, n * sizeof(uint32_t));
  } else {
    std::vector<std::string> keys(n);
    std::vector<const char*> kp(n);
    std::vector<uint64_t> kl(n);
    for (uint32_t i = 0; i < n; ++i) {
      keys[i] = saved_key(r->g[i].v);
      kp[i] = keys[i].data();
      kl[i] = keys[i].size();
    }
    orc_group_by_keys(kp.data(), kl.data(), n, r->tmpl.data());
    // Collision bit (a build-defined report, the grouping above is by exact
    // key strings): a graph below i's template whose key has the same
    // CRC-64/XZ and length as i's but other bytes.
    for (uint32_t i = 0; i < n; ++i)
      for (uint32_t j = 0; j < r->tmpl[i]; ++j)
        if (r->g[j].dig[0] == r->g[i].dig[0] && keys[j].size() == keys[i].size() && keys[j] != keys[i])
          r->g[i].status |= ST_COLLISION;
  }
  for (uint32_t i = 0; i < n; ++i) {
    if (r->tmpl[i] >= n) {
      g_err = "template index out of range";
      return -1;
    }
    r->g[i].tmpl = r->tmpl[i];
  }
  parallel_for(n, threads, [&](uint32_t i) {
    Graph& g = r->g[i];
    if (g.tmpl == i) {
      for (auto& f : g.flags) f |= F_TEMPLATE;
    } else {
      diff_graph(g, r->g[g.tmpl]);
    }
  });
  r->ovr_off.assign(n + 1, 0);
  for (uint32_t i = 0; i < n; ++i) r->ovr_off[i + 1] = r->ovr_off[i] + r->g[i].ovr.size();
  for (uint32_t i = 0; i < n; ++i)
    if (r->tmpl[i] == i) {
      r->live[i] = r->g[i].image;
      r->live_src[i].assign(r->g[i].v.num_nodes, i);
      r->current[i] = i;
    }
  *out = r.release();
  return 0;
}

void orc_free(orc_result* r) { delete r; }

int orc_digests(const orc_result* r, uint64_t* out) {
  for (size_t i = 0; i < r->g.size(); ++i) std::memcpy(out + 4 * i, r->g[i].dig, 32);
  return 0;
}
int orc_groups(const orc_result* r, uint32_t* out) {
  std::memcpy(out, r->tmpl.data(), r->tmpl.size() * 4);
  return 0;
}
int orc_status(const orc_result* r, uint32_t* out) {
  for (size_t i = 0; i < r->g.size(); ++i) out[i] = r->g[i].status;
  return 0;
}
int orc_override_offsets(const orc_result* r, uint64_t* out) {
  std::memcpy(out, r->ovr_off.data(), r->ovr_off.size() * 8);
  return 0;
}

}  // extern "C"

template <typename T, typename U>
static int64_t copy_out(const std::vector<T>& v, U* out, uint64_t cap) {
  if (out) std::memcpy(out, v.data(), std::min<uint64_t>(cap, v.size()) * sizeof(T));
  return (int64_t)v.size();
}

extern "C" {

int64_t orc_overrides(const orc_result* r, uint32_t g, orc_override* out, uint64_t cap) {
  return g < r->g.size() ? copy_out(r->g[g].ovr, out, cap) : -1;
}
int64_t orc_node_flags(const orc_result* r, uint32_t g, uint8_t* out, uint64_t cap) {
  return g < r->g.size() ? copy_out(r->g[g].flags, out, cap) : -1;
}
int64_t orc_node_words(const orc_result* r, uint32_t g, uint32_t* out, uint64_t cap) {
  return g < r->g.size() ? copy_out(r->g[g].woff, out, cap) : -1;
}
int64_t orc_param_image(const orc_result* r, uint32_t g, uint64_t* out, uint64_t cap) {
  return g < r->g.size() ? copy_out(r->g[g].image, out, cap) : -1;
}
int64_t orc_node_pointers(const orc_result* r, uint32_t g, uint64_t* out, uint64_t cap) {
  return g < r->g.size() ? copy_out(r->g[g].ptrs, out, cap) : -1;
}
uint64_t orc_total_param_bytes(const orc_result* r) {
  uint64_t s = 0;
  for (auto& g : r->g) s += g.param_bytes;
  return s;
}

int orc_switch(orc_result* r, uint32_t gi) {
  if (gi >= r->g.size()) return -1;
  uint32_t t = r->tmpl[gi];
  uint32_t c = r->current[t];
  if (c == gi) return 0;
  const Graph& g = r->g[gi];
  if (g.status & ST_COUNT) {
    g_err = "node count differs from the template";
    return -1;
  }
  auto& live = r->live[t];
  const auto& rt = r->g[t].image;
  for (const orc_override& o : r->g[c].ovr) live[o.word] = rt[o.word];
  for (const orc_override& o : g.ovr) live[o.word] = o.value;
  auto& src = r->live_src[t];
  for (uint32_t n = 0; n < src.size(); ++n) src[n] = (g.flags[n] & (F_LAYOUT | F_DESC)) ? gi : t;
  r->current[t] = gi;
  return 0;
}

int64_t orc_live(const orc_result* r, uint32_t t, uint64_t* words, uint64_t cap, uint32_t* node_src,
                 uint64_t node_cap, uint32_t* current) {
  auto it = r->live.find(t);
  if (it == r->live.end()) return -1;
  copy_out(it->second, words, cap);
  copy_out(r->live_src.at(t), node_src, node_cap);
  if (current) *current = r->current.at(t);
  return (int64_t)it->second.size();
}

uint64_t orc_relocate_word(uint64_t w, const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo, uint64_t n,
                           uint32_t policy) {
  return reloc(w, lo, hi, nlo, n, policy);
}

int orc_relocate_words(const uint64_t* in, uint64_t* out, uint64_t n_words, const uint64_t* lo, const uint64_t* hi,
                       const uint64_t* nlo, uint64_t n, uint32_t policy, uint32_t threads) {
  const uint64_t chunk = 1 << 16;
  uint32_t nchunks = (uint32_t)((n_words + chunk - 1) / chunk);
  parallel_for(nchunks, threads, [&](uint32_t c) {
    uint64_t end = std::min<uint64_t>(n_words, (uint64_t)(c + 1) * chunk);
    for (uint64_t i = (uint64_t)c * chunk; i < end; ++i) out[i] = reloc(in[i], lo, hi, nlo, n, policy);
  });
  return 0;
}


// Allocator-event replay.  Follows csrc/hook.cpp:
//   3397-3421 start_base_addr: move the cursor forward to it, abort if behind
//   3432-3461 alloc: cuMemAlloc_v2 at the cursor, abort unless at the saved ptr
//   2272-2291, 2424 placement: ptr = align_up(cursor, 2 MiB); cursor = align_up(ptr + size, 2 MiB)
//   3463-3478 reserve: ptr = align_up(cursor, alignment), abort unless saved ptr; cursor = align_up(ptr + size, 2 MiB)
//   3480-3488 free: no placement
int64_t orc_region_replay(const char* json, uint64_t len, uint64_t saved_base, uint64_t base, uint64_t size,
                          uint64_t* cursor, uint64_t* out, uint64_t cap) {
  const uint64_t A = 2ull << 20;
  auto up = [](uint64_t v, uint64_t a) { return (v + a - 1) / a * a; };
  Json doc;
  JsonParser jp{json, json + len};
  if (!jp.val(&doc, 0) || doc.k != Json::OBJ) return -1;
  auto num = [](const Json* j, uint64_t* v) {
    if (!j || j->k != Json::NUM || j->s.empty() || j->s[0] == '-') return false;
    for (char c : j->s)
      if (c < '0' || c > '9') return false;
    *v = std::stoull(j->s);
    return true;
  };
  uint64_t cur = *cursor;
  if (const Json* s0 = doc.get("start_base_addr")) {
    uint64_t st;
    if (!num(s0, &st)) return -1;
    const uint64_t target = base + (st - saved_base);
    if (target < cur) return -2;
    cur = target;
  }
  const Json* evs = doc.get("events");
  if (!evs || evs->k != Json::ARR) return -1;
  int64_t n = 0;
  for (const Json& ev : evs->a) {
    const Json* ty = ev.get("type");
    if (!ty || ty->k != Json::STR) return -1;
    uint64_t ptr, sz, al;
    if (!num(ev.get("ptr"), &ptr)) return -1;
    if (ty->s == "free") continue;
    if (!num(ev.get("size"), &sz)) return -1;
    uint64_t at;
    if (ty->s == "alloc") {
      at = up(cur, A);
    } else if (ty->s == "reserve") {
      if (!num(ev.get("alignment"), &al) || al == 0) return -1;
      at = up(cur, al);
    } else {
      return -1;
    }
    if (at + sz > base + size) return -3;
    if (ptr < saved_base || at - base != ptr - saved_base) return -2;
    cur = up(at + sz, A);
    if ((uint64_t)n < cap && out) {
      out[3 * n] = ptr;
      out[3 * n + 1] = ptr + sz;
      out[3 * n + 2] = at;
    }
    ++n;
  }
  *cursor = cur;
  return n;
}

}  // extern "C"

// ---- the reference's CPU LOAD data work, restated ----------------------

namespace {

// SimpleThreadPool as in csrc/CUDAGraphParallel.cpp:38-89.
class Pool {
 public:
  explicit Pool(size_t n) {
    for (size_t i = 0; i < n; ++i)
      workers_.emplace_back([this] {
        for (;;) {
          std::function<void()> task;
          {
            std::unique_lock<std::mutex> lk(m_);
            cv_.wait(lk, [this] { return stop_ || !q_.empty(); });
            if (stop_ && q_.empty()) return;
            task = std::move(q_.front());
            q_.pop();
          }
          task();
        }
      });
  }
  template <class F>
  std::future<typename std::invoke_result<F>::type> submit(F&& f) {
    using R = typename std::invoke_result<F>::type;
    auto t = std::make_shared<std::packaged_task<R()>>(std::forward<F>(f));
    auto fut = t->get_future();
    {
      std::lock_guard<std::mutex> lk(m_);
      q_.emplace([t] { (*t)(); });
    }
    cv_.notify_one();
    return fut;
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> lk(m_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& w : workers_) w.join();
  }

 private:
  std::vector<std::thread> workers_;
  std::queue<std::function<void()>> q_;
  std::mutex m_;
  std::condition_variable cv_;
  bool stop_ = false;
};

struct NodeUpdate {  // the per-node host state of OnDemandNodeUpdate (include/CUDAGraph.h:110-151)
  int type = 5;
  uint8_t launch[64];
  std::vector<std::vector<uint8_t>> param_data;
  std::vector<void*> param_ptrs;
  std::vector<uint8_t> arg_buffer;
  uint64_t handle = 0;
};

}  // namespace

extern "C" double orc_reference_load_ms(const char* const* paths, uint32_t n, uint32_t num_threads, uint32_t reps,
                                        uint64_t* driver_calls) {
  if (n == 0 || reps == 0) return -1;
  std::vector<double> times;
  uint64_t calls = 0;
  // Synthetic function registry: (binary_hash, name) -> handle, like
  // query_function_handle's map (csrc/hook.cpp:3514-3551).
  std::unordered_map<std::string, uint64_t> registry;
  std::mutex reg_mu;
  for (uint32_t rep = 0; rep < reps + 1; ++rep) {
    auto t0 = std::chrono::steady_clock::now();
    uint32_t threads = std::max(1u, std::min(num_threads, n));
    std::vector<std::vector<uint8_t>> files(n);
    {
      Pool pool(threads);
      std::vector<std::future<std::vector<uint8_t>>> fs;
      for (uint32_t i = 0; i < n; ++i)
        fs.push_back(pool.submit([&, i] {
          std::vector<uint8_t> buf;
          FILE* f = std::fopen(paths[i], "rb");
          if (!f) return buf;
          std::fseek(f, 0, SEEK_END);
          long sz = std::ftell(f);
          std::fseek(f, 0, SEEK_SET);
          buf.resize((size_t)sz);
          if (std::fread(buf.data(), 1, buf.size(), f) != buf.size()) buf.clear();
          std::fclose(f);
          return buf;
        }));
      for (uint32_t i = 0; i < n; ++i) files[i] = fs[i].get();
    }
    std::vector<View> views(n);
    for (uint32_t i = 0; i < n; ++i)
      if (!open_view(files[i].data(), files[i].size(), &views[i])) return -2;
    std::unordered_map<std::string, std::vector<size_t>> groups;
    std::vector<size_t> template_for(n, SIZE_MAX);
    for (uint32_t i = 0; i < n; ++i) groups[saved_key(views[i])].push_back(i);
    for (auto& kv : groups)
      for (size_t j = 1; j < kv.second.size(); ++j) template_for[kv.second[j]] = kv.second[0];
    std::atomic<uint64_t> skipped{0};
    std::vector<std::vector<NodeUpdate>> updates(n);
    {
      Pool pool(threads);
      std::vector<std::future<void>> fs;
      for (uint32_t i = 0; i < n; ++i) {
        if (template_for[i] == SIZE_MAX) continue;
        fs.push_back(pool.submit([&, i] {
          const View& v = views[i];
          auto& ups = updates[i];
          ups.resize(v.num_nodes);
          std::vector<ParamRef> ps;
          for (uint32_t k = 0; k < v.num_nodes; ++k) {
            const uint8_t* e = node_at(v, k);
            NodeUpdate& u = ups[k];
            u.type = e[4];
            if (e[4] == N_KERNEL) {
              std::memset(u.launch, 0, sizeof(u.launch));
              std::memcpy(u.launch, e + 8, 28);
              uint32_t no = rd<uint32_t>(e, 44), nl = rd<uint32_t>(e, 48);
              std::string name((const char*)v.d + v.off[S_STR] + no, nl);
              std::string key = std::to_string(rd<uint64_t>(e, 36)) + ":" + name;
              {
                std::lock_guard<std::mutex> lk(reg_mu);
                auto it = registry.find(key);
                if (it == registry.end()) it = registry.emplace(key, registry.size() + 1).first;
                u.handle = it->second;
              }
              if (rd<int32_t>(e, 52) > 0) skipped++;
              if (rd<int32_t>(e, 56) >= 0) skipped++;
              bool extra;
              node_params(v, e, &ps, &extra);
              if (extra) {
                u.arg_buffer.assign(v.d + v.off[S_ARG] + ps[0].off, v.d + v.off[S_ARG] + ps[0].off + ps[0].size);
              } else {
                u.param_data.resize(ps.size());
                for (size_t j = 0; j < ps.size(); ++j) {
                  u.param_data[j].resize(ps[j].size);
                  std::memcpy(u.param_data[j].data(), v.d + v.off[S_PDATA] + ps[j].off, ps[j].size);
                }
                u.param_ptrs.resize(ps.size());
                for (size_t j = 0; j < ps.size(); ++j) u.param_ptrs[j] = u.param_data[j].data();
              }
            } else if (e[4] == N_EVREC || e[4] == N_EVWAIT) {
              skipped++;  // cuEventCreate
            }
          }
        }));
      }
      for (auto& f : fs) f.get();
    }
    double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    if (rep > 0) times.push_back(ms);  // first run warms the page cache
    calls = skipped.load();
  }
  std::sort(times.begin(), times.end());
  if (driver_calls) *driver_calls = calls;
  return times[times.size() / 2];
}
