// reloc_index.h -- the interval index of the relocation search and its
// builder.  The builder's per-root-line steps are host and device code
// alike: the library builds relocation plans and an archive's index with
// them as kernels (one thread per root line, kernels.hip), the no-allocation
// entry point and the CPU check of the search (tests/native) on the host,
// so both produce the same lines.
#pragma once

#include <stdint.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/foundry_restore.h"
#include "restore_dev.h"

namespace fdy {

// The interval index of a table, built on the host: its lines and the
// search parameters (dev.line is set when the lines are placed on the
// device).
struct HostIndex {
  std::vector<RelocLine> line;
  RelocDev dev{};
};

// Root lines per interval, about (between k/2 and k per interval, a power
// of two in all): a root line whose range holds more than four intervals
// takes a second read, its child.  More root lines mean fewer second reads
// and a larger index (64 B per line): 2 per interval for the index that
// lives beside a restored archive, 16 for a relocation plan, which is built
// once to relocate many words (2M intervals: 1.55 reads per lookup and
// 228 MB, against about 1.3 reads and 2 GB).
constexpr uint64_t kRootLinesPerInterval = 2;
constexpr uint64_t kPlanRootLinesPerInterval = 16;
constexpr uint32_t kLeafIntervals = kLineSlots;  // the interval at or before B, and three starting inside
constexpr uint64_t kMaxIndexLines = 0xFFFFFFF0ull;

// The root lines: 2^shift bytes each from lo_min, nb of them.
struct IndexShape {
  uint32_t shift;
  uint64_t nb;
};

// Checks a table (sorted, non-overlapping, non-empty intervals below 2^64-1
// spanning less than 2^54 bytes, fewer than 2^32 of them) and picks the
// root lines: the line width is the smallest power of two giving at most
// `target` root lines over [lo_min, hi_max], and at most 2^31 so offsets
// inside a line fit in 31 bits (a span of 2^47, a process's whole address
// space, then takes at most 2^16 root lines).
inline int index_shape(const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo, uint64_t n, uint32_t policy,
                       uint64_t root_lines_per_interval, IndexShape* shape, std::string* why) {
  auto err = [why](int code, const std::string& msg) {
    *why = msg;
    return code;
  };
  if (policy > FDY_RELOC_INCLUSIVE) return err(FDY_E_INVALID, "unknown relocation policy");
  shape->shift = 0;
  shape->nb = 0;
  if (n == 0) return FDY_OK;
  if (!lo || !hi || !nlo) return err(FDY_E_INVALID, "null interval array");
  for (uint64_t i = 0; i < n; ++i) {
    if (lo[i] >= hi[i]) return err(FDY_E_INVALID, "interval " + std::to_string(i) + " is empty (lo >= hi)");
    if (hi[i] == UINT64_MAX) return err(FDY_E_INVALID, "interval " + std::to_string(i) + " ends at 2^64-1");
    if (i && hi[i - 1] > lo[i])
      return err(FDY_E_INVALID, "intervals " + std::to_string(i - 1) + " and " + std::to_string(i) +
                                    " overlap or are not sorted by lo");
  }
  if (n > 0xFFFFFFF0ull) return err(FDY_E_INVALID, "more than 2^32 intervals");
  const uint64_t span = hi[n - 1] - lo[0];
  if (span >> 54) return err(FDY_E_INVALID, "intervals span more than 2^54 bytes");
  uint64_t target = 1;
  while (target < root_lines_per_interval * n) target <<= 1;
  uint32_t shift = 0;
  while ((span >> shift) + 1 > target) ++shift;
  if (shift > kMaxLineShift) shift = kMaxLineShift;
  shape->shift = shift;
  shape->nb = (span >> shift) + 1;  // w - lo_min <= span, so (w - lo_min) >> shift < nb
  return FDY_OK;
}

// First address of root line b.
__host__ __device__ inline uint64_t root_start(uint64_t lo0, uint32_t shift, uint64_t b) {
  const uint64_t off = b << shift;  // b <= nb, so no overflow below 2^55
  return off > UINT64_MAX - lo0 ? UINT64_MAX : lo0 + off;
}

// The intervals root line b's range [s0, s1) holds: i, the last with
// lo <= s0 (lo[0] <= s0 always), and i + 1 .. j, those starting inside it.
__host__ __device__ inline void root_range(const uint64_t* lo, uint64_t n, uint64_t s0, uint64_t s1, uint64_t* i,
                                           uint64_t* j) {
  uint64_t a = 0, b = n;  // first lo > s0
  while (a < b) {
    const uint64_t mid = (a + b) >> 1;
    if (lo[mid] <= s0) a = mid + 1;
    else b = mid;
  }
  *i = a ? a - 1 : 0;
  uint64_t c = *i, d = n;  // first lo >= s1
  while (c < d) {
    const uint64_t mid = (c + d) >> 1;
    if (lo[mid] < s1) c = mid + 1;
    else d = mid;
  }
  *j = c ? c - 1 : 0;
  if (*j < *i) *j = *i;
}

// A fence line's children for m intervals (m > kLeafIntervals): up to 15
// leaves; past 60 intervals, the fewest children one level deeper (capacity
// `big`) beside children of capacity `small`, so that most intervals stay
// as shallow as the count allows.  Child c holds size(c) intervals.
struct FenceKids {
  uint32_t kids;
  uint64_t m, small, t, q, r;  // past 60: 15 - t children of `small`, then t of q + 1 (the first r) or q
  __host__ __device__ explicit FenceKids(uint64_t m_) : m(m_), small(0), t(0), q(0), r(0) {
    constexpr uint64_t kKids = kLineFences + 1;
    if (m <= kKids * kLeafIntervals) {
      kids = (uint32_t)((m + kLeafIntervals - 1) / kLeafIntervals);
      return;
    }
    kids = (uint32_t)kKids;
    uint64_t big = kKids * kLeafIntervals;
    small = kLeafIntervals;
    while (kKids * big < m) {
      small = big;
      big *= kKids;
    }
    t = (m - kKids * small + (big - small) - 1) / (big - small);  // 1 .. 15 deeper children
    const uint64_t rest = m - (kKids - t) * small;
    q = rest / t;
    r = rest % t;
  }
  __host__ __device__ uint64_t size(uint32_t c) const {
    if (!small) return c + 1 < kids ? kLeafIntervals : m - (uint64_t)c * kLeafIntervals;
    const uint64_t n_small = kLineFences + 1 - t;
    if (c < n_small) return small;
    return q + (c - n_small < r ? 1 : 0);
  }
};

// Lines below a root line whose range holds m intervals.  A fence line's
// children take at most three sizes, so the count walks a short list of
// {size, multiplicity} pairs (each level adds at most three, and 2^32
// intervals take eight levels): `size` and `mult` hold kSubtreeStack each
// (in LDS on the device, where an array in registers would be private
// memory that the runtime sizes for every lane of the GPU).
constexpr uint32_t kSubtreeStack = 24;
__host__ __device__ inline uint64_t subtree_lines(uint64_t m, uint64_t* size, uint64_t* mult) {
  uint32_t top = 0;
  uint64_t total = 0;
  if (m > kLeafIntervals) {
    size[0] = m;
    mult[0] = 1;
    top = 1;
  }
  while (top) {
    --top;
    const uint64_t k = mult[top];
    const FenceKids f(size[top]);
    total += k * f.kids;
    if (!f.small) continue;  // leaves only
    const uint64_t run_size[3] = {f.small, f.q + 1, f.q};
    const uint64_t run_mult[3] = {kLineFences + 1 - f.t, f.r, f.t - f.r};
    for (uint32_t e = 0; e < 3; ++e)
      if (run_mult[e] && run_size[e] > kLeafIntervals && top < kSubtreeStack) {
        size[top] = run_size[e];
        mult[top] = k * run_mult[e];
        ++top;
      }
  }
  return total;
}

// The line at `at` whose range from s0 holds intervals i (lo[i] <= s0, the
// last such) .. j: a leaf for up to four, else a fence line whose children
// take the next free lines (*next on), each holding until it is placed the
// {s0, i, j} it is to be placed with.
__host__ __device__ inline void place_line(RelocLine* line, uint64_t at, uint64_t s0, uint64_t i, uint64_t j,
                                           const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo,
                                           uint64_t* next) {
  auto end_of = [&](uint64_t k) -> uint32_t {
    if (hi[k] < s0) return 0;
    const uint64_t e = hi[k] - s0 + 1;
    return e > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)e;
  };
  RelocLine L;
  const uint64_t m = j - i + 1;
  if (m <= kLeafIntervals) {
    L.s[0] = RelocSlot{0, end_of(i), nlo[i] - lo[i]};
    for (uint32_t k = 1; k < kLineSlots; ++k) {
      if (i + k <= j) L.s[k] = RelocSlot{(uint32_t)(lo[i + k] - s0), end_of(i + k), nlo[i + k] - lo[i + k]};
      else L.s[k] = RelocSlot{kLineNone, 0, 0};
    }
    line[at] = L;
    return;
  }
  // A fence line, written field by field in place (a fence array indexed
  // at run time would be private memory on the device).
  const FenceKids f(m);
  const uint64_t base = *next;
  *next += f.kids;
  line[at].s[0].lo = kLineFence;
  line[at].s[0].end = (uint32_t)base;
  uint32_t* fence = line_fences(line[at]);
  uint64_t ci = i;
  for (uint32_t c = 0; c < f.kids; ++c) {
    if (c) fence[c - 1] = (uint32_t)(lo[ci] - s0);  // a start inside the line: 0 < lo - s0 < 2^31
    RelocLine P;  // pending: {s0, i, j} of the child
    P.s[0] = RelocSlot{0, 0, c ? lo[ci] : s0};
    P.s[1] = RelocSlot{0, 0, ci};
    P.s[2] = RelocSlot{0, 0, ci + f.size(c) - 1};
    P.s[3] = RelocSlot{0, 0, 0};
    line[base + c] = P;
    ci += f.size(c);
  }
  for (uint32_t e = f.kids - 1; e < kLineFences; ++e) fence[e] = kLineNone;
}

// Root line b and every line below it, its descendants taking lines base ..
// base + subtree_lines(j - i + 1) - 1 breadth first (children of one line
// together), each placed after its parent.
__host__ __device__ inline void place_root(RelocLine* line, uint64_t b, uint64_t s0, uint64_t i, uint64_t j,
                                           const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo,
                                           uint64_t base) {
  uint64_t next = base;
  place_line(line, b, s0, i, j, lo, hi, nlo, &next);
  for (uint64_t at = base; at < next; ++at) {
    const RelocLine P = line[at];  // this thread's own pending line
    place_line(line, at, P.s[0].delta, P.s[1].delta, P.s[2].delta, lo, hi, nlo, &next);
  }
}

// The whole index on the host.
inline int build_reloc_index(const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo, uint64_t n,
                             uint32_t policy, HostIndex* out, std::string* why,
                             uint64_t root_lines_per_interval = kRootLinesPerInterval) {
  std::memset(&out->dev, 0, sizeof(out->dev));
  IndexShape sh;
  const int rc = index_shape(lo, hi, nlo, n, policy, root_lines_per_interval, &sh, why);
  if (rc || n == 0) return rc;
  std::vector<uint64_t> ri(sh.nb), rj(sh.nb), base(sh.nb);
  uint64_t total = sh.nb;
  for (uint64_t b = 0; b < sh.nb; ++b) {
    root_range(lo, n, root_start(lo[0], sh.shift, b), root_start(lo[0], sh.shift, b + 1), &ri[b], &rj[b]);
    base[b] = total;
    uint64_t st_size[kSubtreeStack], st_mult[kSubtreeStack];
    total += subtree_lines(rj[b] - ri[b] + 1, st_size, st_mult);
    if (total > kMaxIndexLines) {
      *why = "interval index too large";
      return FDY_E_INVALID;
    }
  }
  out->line.assign(total, RelocLine{});
  for (uint64_t b = 0; b < sh.nb; ++b)
    place_root(out->line.data(), b, root_start(lo[0], sh.shift, b), ri[b], rj[b], lo, hi, nlo, base[b]);
  out->dev.n = n;
  out->dev.lo_min = lo[0];
  out->dev.hi_max = hi[n - 1];
  out->dev.shift = sh.shift;
  out->dev.policy = policy;
  return FDY_OK;
}

}  // namespace fdy
