// random_reads -- the rate at which the GPU serves independent random reads
// of small blocks from HBM (and from a cache-resident working set): the
// bound of a kernel whose reads are random lines, such as the interval
// search of the standalone relocation.
//
// Each group of S / 16 lanes reads one S-byte block (16 bytes per lane, one
// coalesced access) at a pseudo-random S-aligned offset of a working set,
// eight blocks per lane group in flight per round, 16384 workgroups of 256
// threads, 8 rounds.  Every offset is masked into the working set (a power
// of two), so every access stays inside the buffer.
//
// Usage: random_reads            (prints one line per block size and working set)
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#define CHECK(x)                                                                 \
  do {                                                                           \
    const hipError_t e_ = (x);                                                   \
    if (e_ != hipSuccess) {                                                      \
      std::fprintf(stderr, "%s: %s (line %d)\n", #x, hipGetErrorString(e_), __LINE__); \
      return 1;                                                                  \
    }                                                                            \
  } while (0)

namespace {

constexpr uint32_t kThreads = 256, kGrid = 16384, kRounds = 8, kInFlight = 8;

__device__ inline uint64_t mix64(uint64_t x) {  // a 64-bit finaliser (MurmurHash3's fmix64)
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdull;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ull;
  x ^= x >> 33;
  return x;
}

// kLanes lanes per block: block b is uint4s [b * kLanes, (b + 1) * kLanes).
template <uint32_t kLanes>
__global__ __launch_bounds__(kThreads) void k_random_reads(const uint4* buf, uint64_t block_mask, uint4* sink,
                                                           uint64_t salt) {
  const uint64_t gid = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  const uint64_t grp = gid / kLanes;
  const uint32_t sub = (uint32_t)(gid % kLanes);
  uint4 acc = make_uint4(0, 0, 0, 0);
  for (uint32_t r = 0; r < kRounds; ++r) {
    uint4 v[kInFlight];
#pragma unroll
    for (uint32_t k = 0; k < kInFlight; ++k) {
      const uint64_t b = mix64(grp * 1000003ull + r * kInFlight + k + salt) & block_mask;
      v[k] = buf[b * kLanes + sub];
    }
#pragma unroll
    for (uint32_t k = 0; k < kInFlight; ++k) {
      acc.x ^= v[k].x;
      acc.y += v[k].y;
      acc.z ^= v[k].z;
      acc.w += v[k].w;
    }
  }
  if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u) sink[0] = acc;  // keeps the loads; never true for the fill
}

template <uint32_t kLanes>
int measure(const uint4* buf, uint64_t set_bytes, uint4* sink, hipEvent_t e0, hipEvent_t e1) {
  const uint64_t blocks_in_set = set_bytes / (16ull * kLanes);
  const double blocks = (double)kGrid * kThreads / kLanes * kRounds * kInFlight;
  float best = 1e30f;
  for (int rep = 0; rep < 4; ++rep) {
    CHECK(hipEventRecord(e0));
    hipLaunchKernelGGL(k_random_reads<kLanes>, dim3(kGrid), dim3(kThreads), 0, 0, buf, blocks_in_set - 1, sink,
                       (uint64_t)rep * 0x9E37ull);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    if (rep && ms < best) best = ms;  // the first launch warms up
  }
  std::printf("working set %6llu MiB, block %4u B: %.3f ms, %.1f G blocks/s, %.0f GB/s\n",
              (unsigned long long)(set_bytes >> 20), 16 * kLanes, best, blocks / best / 1e6,
              blocks * 16 * kLanes / best / 1e6);
  return 0;
}

}  // namespace

int main() {
  const uint64_t bytes = 4ull << 30;  // the largest working set; every set is a power of two
  uint4* buf = nullptr;
  uint4* sink = nullptr;
  CHECK(hipMalloc(&buf, bytes));
  CHECK(hipMalloc(&sink, 64));
  CHECK(hipMemset(buf, 1, bytes));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  for (const uint64_t set : {bytes, (uint64_t)256 << 20, (uint64_t)32 << 20}) {
    if (measure<2>(buf, set, sink, e0, e1) || measure<4>(buf, set, sink, e0, e1) ||
        measure<8>(buf, set, sink, e0, e1) || measure<16>(buf, set, sink, e0, e1) ||
        measure<32>(buf, set, sink, e0, e1))
      return 1;
  }
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  CHECK(hipFree(buf));
  CHECK(hipFree(sink));
  return 0;
}
