// reloc_index.h -- the interval index of the relocation search, built on
// the host (host code only: the library's open and plan calls, and a test
// program that runs the search on the CPU).
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

inline int build_reloc_index(const uint64_t* lo, const uint64_t* hi, const uint64_t* nlo, uint64_t n,
                             uint32_t policy, HostIndex* out, std::string* why,
                             uint64_t root_lines_per_interval = kRootLinesPerInterval) {
  auto err = [why](int code, const std::string& msg) {
    *why = msg;
    return code;
  };
  std::memset(&out->dev, 0, sizeof(out->dev));
  if (policy > FDY_RELOC_INCLUSIVE) return err(FDY_E_INVALID, "unknown relocation policy");
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
  // Line width: the smallest power of two giving at most `target` root lines
  // over [lo_min, hi_max], and at most 2^31 so offsets inside a line fit in
  // 31 bits (a span of 2^47, a process's whole address space, then takes at
  // most 2^16 root lines).
  uint64_t target = 1;
  while (target < root_lines_per_interval * n) target <<= 1;
  uint32_t shift = 0;
  while ((span >> shift) + 1 > target) ++shift;
  if (shift > kMaxLineShift) shift = kMaxLineShift;
  const uint64_t nb = (span >> shift) + 1;  // w - lo_min <= span, so (w - lo_min) >> shift < nb
  auto start = [&](uint64_t b) -> uint64_t {
    const uint64_t off = b << shift;  // b <= nb, so no overflow below 2^55
    return off > UINT64_MAX - lo[0] ? UINT64_MAX : lo[0] + off;
  };
  std::vector<RelocLine>& line = out->line;
  line.assign(nb, RelocLine{});
  auto end_of = [&](uint64_t k, uint64_t s0) -> uint32_t {
    if (hi[k] < s0) return 0;
    const uint64_t e = hi[k] - s0 + 1;
    return e > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)e;
  };
  // The line at s0 whose range holds intervals i (lo[i] <= s0, the last
  // such) .. j (i + 1 .. j start inside it): a leaf for up to four, else a
  // fence line over children of up to 4 * 15^d intervals each.
  struct Pending {
    uint64_t line, s0, i, j;
  };
  std::vector<Pending> todo;
  auto place = [&](uint64_t at, uint64_t s0, uint64_t i, uint64_t j) -> int {
    RelocLine& L = line[at];
    const uint64_t m = j - i + 1;
    if (m <= kLeafIntervals) {
      L.s[0] = RelocSlot{0, end_of(i, s0), nlo[i] - lo[i]};
      for (uint32_t k = 1; k < kLineSlots; ++k) {
        if (i + k <= j) L.s[k] = RelocSlot{(uint32_t)(lo[i + k] - s0), end_of(i + k, s0), nlo[i + k] - lo[i + k]};
        else L.s[k] = RelocSlot{kLineNone, 0, 0};
      }
      return FDY_OK;
    }
    // Children: up to 15 leaves; past 60 intervals, the fewest children one
    // level deeper (capacity `big`) beside children of capacity `small`, so
    // that most intervals stay as shallow as the count allows.
    constexpr uint64_t kKids = kLineFences + 1;
    uint64_t sizes[kKids], kids = 0;
    if (m <= kKids * kLeafIntervals) {
      for (uint64_t left = m; left; left -= std::min(left, (uint64_t)kLeafIntervals))
        sizes[kids++] = std::min(left, (uint64_t)kLeafIntervals);
    } else {
      uint64_t small = kLeafIntervals, big = kKids * kLeafIntervals;
      while (kKids * big < m) {
        small = big;
        big *= kKids;
      }
      const uint64_t t = (m - kKids * small + (big - small) - 1) / (big - small);  // 1 .. 15 deeper children
      for (uint64_t c = 0; c < kKids - t; ++c) sizes[kids++] = small;
      const uint64_t rest = m - (kKids - t) * small;
      for (uint64_t c = 0; c < t; ++c) sizes[kids++] = rest / t + (c < rest % t);
    }
    const uint64_t base = line.size();
    if (base + kids > 0xFFFFFFF0ull) return err(FDY_E_INVALID, "interval index too large");
    L.s[0] = RelocSlot{kLineFence, (uint32_t)base, 0};
    uint32_t* f = line_fences(L);
    uint64_t ci = i;
    for (uint64_t c = 0; c < kids; ++c) {
      if (c) f[c - 1] = (uint32_t)(lo[ci] - s0);  // a start inside the line: 0 < lo - s0 < 2^31
      todo.push_back({base + c, c ? lo[ci] : s0, ci, ci + sizes[c] - 1});
      ci += sizes[c];
    }
    for (uint64_t e = kids - 1; e < kLineFences; ++e) f[e] = kLineNone;
    line.resize(base + kids);  // L is not used past here
    return FDY_OK;
  };
  uint64_t i = 0, j = 0;  // i: last lo <= line start; j: last lo < next line's start
  for (uint64_t b = 0; b < nb; ++b) {
    const uint64_t s0 = start(b), s1 = start(b + 1);
    while (i + 1 < n && lo[i + 1] <= s0) ++i;
    if (j < i) j = i;
    while (j + 1 < n && lo[j + 1] < s1) ++j;
    const int rc = place(b, s0, i, j);
    if (rc) return rc;
    while (!todo.empty()) {
      const Pending p = todo.back();
      todo.pop_back();
      const int rc2 = place(p.line, p.s0, p.i, p.j);
      if (rc2) return rc2;
    }
  }
  out->dev.n = n;
  out->dev.lo_min = lo[0];
  out->dev.hi_max = hi[n - 1];
  out->dev.shift = shift;
  out->dev.policy = policy;
  return FDY_OK;
}

}  // namespace fdy
