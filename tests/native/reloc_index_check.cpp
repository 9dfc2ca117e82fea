// reloc_index_check -- the library's interval index (foundry_amd/csrc/
// reloc_index.h) and its search (reloc_batch in restore_dev.h, the code the
// kernels run) executed on the CPU, so the index can be checked without a
// GPU.
//
//   reloc_index_check TABLE WORDS OUT [ROOT_LINES_PER_INTERVAL [INDEX_OUT]]
//
// TABLE: u64 n, u64 policy, then n lo, n hi, n new_lo (little endian).
// WORDS: u64 words.  INDEX_OUT: the index's 64-byte lines.  OUT: the relocated
// words, then one JSON line on stdout
// with the index's shape (lines, root lines, root shift, fence lines, and
// `bad_refs`: fence lines naming children outside the index or not after
// themselves, or fences out of order) and the line reads the searches took.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../foundry_amd/csrc/reloc_index.h"

using namespace fdy;

static std::vector<uint64_t> read_all(const char* path) {
  std::vector<uint64_t> v;
  FILE* f = std::fopen(path, "rb");
  if (!f) {
    std::perror(path);
    std::exit(2);
  }
  uint64_t x;
  while (std::fread(&x, 8, 1, f) == 1) v.push_back(x);
  std::fclose(f);
  return v;
}

int main(int argc, char** argv) {
  if (argc < 4 || argc > 6) {
    std::fprintf(stderr, "usage: %s TABLE WORDS OUT [ROOT_LINES_PER_INTERVAL [INDEX_OUT]]\n", argv[0]);
    return 2;
  }
  const std::vector<uint64_t> t = read_all(argv[1]);
  if (t.size() < 2 || t.size() != 2 + 3 * t[0]) {
    std::fprintf(stderr, "bad table file\n");
    return 2;
  }
  const uint64_t n = t[0];
  const uint32_t policy = (uint32_t)t[1];
  const uint64_t* lo = t.data() + 2;
  const uint64_t* hi = lo + n;
  const uint64_t* nlo = hi + n;
  const std::vector<uint64_t> w = read_all(argv[2]);

  HostIndex x;
  std::string why;
  const uint64_t per = argc >= 5 ? std::strtoull(argv[4], nullptr, 10) : kRootLinesPerInterval;
  const int rc = build_reloc_index(lo, hi, nlo, n, policy, &x, &why, per);
  if (rc) {
    std::printf("{\"error\": %d}\n", rc);
    std::fprintf(stderr, "%s\n", why.c_str());
    return 0;
  }
  if (argc == 6) {  // the index itself, for comparing with the device build
    FILE* f = std::fopen(argv[5], "wb");
    if (!f || std::fwrite(x.line.data(), sizeof(RelocLine), x.line.size(), f) != x.line.size()) {
      std::perror(argv[5]);
      return 2;
    }
    std::fclose(f);
  }
  RelocDev d = x.dev;
  d.line = x.line.data();

  // Every child a fence line names lies inside the index, after the fence
  // line (so descents end), and its fences are in order.
  uint64_t fences = 0, bad = 0;
  for (size_t l = 0; l < x.line.size(); ++l) {
    RelocLine L = x.line[l];
    if (!(L.s[0].lo & kLineFence)) continue;
    ++fences;
    const uint32_t* f = line_fences(L);
    uint32_t kids = 1;
    while (kids <= kLineFences && f[kids - 1] != kLineNone) ++kids;
    for (uint32_t e = 1; e < kids - 1; ++e) bad += f[e] <= f[e - 1];
    for (uint32_t e = kids; e <= kLineFences; ++e) bad += f[e - 1] != kLineNone;
    bad += kids < 2 || (uint64_t)L.s[0].end <= l || (uint64_t)L.s[0].end + kids > x.line.size();
  }

  // Line reads per search, counted by walking the split lines as the search does.
  uint64_t reads = 0, searched = 0, max_depth = 1;
  std::vector<uint64_t> out(w.size());
  constexpr int K = 4;
  for (size_t i = 0; i < w.size(); i += K) {
    uint64_t in[K] = {0, 0, 0, 0}, res[K];
    uint32_t mask = 0;
    for (int k = 0; k < K && i + k < w.size(); ++k) {
      in[k] = w[i + k];
      mask |= 1u << k;
    }
    reloc_batch<K>(d, in, res, mask);
    for (int k = 0; k < K && i + k < w.size(); ++k) {
      out[i + k] = res[k];
      const uint64_t v = in[k];
      if (n == 0 || v < d.lo_min || (policy ? v > d.hi_max : v >= d.hi_max)) continue;
      const uint64_t rel = v - d.lo_min;
      uint64_t b = rel >> d.shift;
      uint32_t xo = (uint32_t)(rel - (b << d.shift));
      ++searched;
      const uint64_t reads0 = reads++;
      while (x.line[b].s[0].lo & kLineFence) {
        RelocLine L = x.line[b];
        const uint32_t* f = line_fences(L);
        uint32_t c = 0, at = 0;
        for (uint32_t e = 0; e < kLineFences; ++e)
          if (f[e] <= xo) c = e + 1, at = f[e];
        xo -= at;
        b = L.s[0].end + c;
        ++reads;
        max_depth = std::max(max_depth, reads - reads0);
      }
    }
  }
  FILE* f = std::fopen(argv[3], "wb");
  if (!f || std::fwrite(out.data(), 8, out.size(), f) != out.size()) {
    std::perror(argv[3]);
    return 2;
  }
  std::fclose(f);
  std::printf(
      "{\"lines\": %zu, \"root_lines\": %llu, \"shift\": %u, \"fence_lines\": %llu, \"bad_refs\": %llu, "
      "\"searched\": %llu, \"line_reads\": %llu, \"max_reads\": %llu}\n",
      x.line.size(), (unsigned long long)((n ? ((hi[n - 1] - lo[0]) >> d.shift) + 1 : 0)), d.shift,
      (unsigned long long)fences, (unsigned long long)bad, (unsigned long long)searched,
      (unsigned long long)reads, (unsigned long long)max_depth);
  return 0;
}
