// Kernels whose graphs the group-graph tests save, restore and run.
//
// Each kernel writes results into out[0, cap): every index is checked
// against cap before the access, so a wrong param can give a wrong value
// but never an access outside the buffer.  Results are functions of the
// params and the launch shape that the tests restate on the host (mix()).
#include <hip/hip_runtime.h>
#include <stdint.h>

struct Blob64 {
  uint64_t w[8];
};

__device__ inline uint64_t mix(uint64_t h, uint64_t v) {
  h ^= v;
  h *= 0x9E3779B97F4A7C15ull;
  return h ^ (h >> 29);
}

__device__ inline bool first_thread() {
  return (blockIdx.x | blockIdx.y | blockIdx.z | threadIdx.x | threadIdx.y | threadIdx.z) == 0;
}

// out[idx] = mix over (a, b, grid.x, block.x).
extern "C" __global__ void probe_mix(uint64_t* out, uint32_t idx, uint32_t cap, uint64_t a, uint64_t b) {
  if (!first_thread() || idx >= cap) return;
  uint64_t h = mix(mix(0x243F6A8885A308D3ull, a), b);
  out[idx] = mix(mix(h, gridDim.x), blockDim.x);
}

// out[idx] = mix over the 8 words of a 64-byte by-value struct.
extern "C" __global__ void probe_blob(uint64_t* out, uint32_t idx, uint32_t cap, Blob64 b) {
  if (!first_thread() || idx >= cap) return;
  uint64_t h = 0x13198A2E03707344ull;
  for (int i = 0; i < 8; ++i) h = mix(h, b.w[i]);
  out[idx] = h;
}

// out[idx] = mix(out[src], idx): reads another node's result, so the result
// depends on the dependency edges being honoured.
extern "C" __global__ void probe_chain(uint64_t* out, uint32_t idx, uint32_t cap, uint32_t src) {
  if (!first_thread() || idx >= cap || src >= cap) return;
  out[idx] = mix(out[src], idx);
}

// Every thread of every block adds v: out[idx] = v * (threads in the grid).
extern "C" __global__ void probe_count(uint64_t* out, uint32_t idx, uint32_t cap, uint64_t v) {
  if (idx >= cap) return;
  atomicAdd(reinterpret_cast<unsigned long long*>(out + idx), (unsigned long long)v);
}

// What a kernel drawing random numbers in a captured graph reads of its
// generator (the graph-safe Philox state): out[idx] = *seed,
// out[idx + 1] = *offset + intragraph (the offset the capture recorded).
extern "C" __global__ void probe_rng(uint64_t* out, uint32_t idx, uint32_t cap, const int64_t* seed,
                                     const int64_t* offset, uint32_t intragraph) {
  if (!first_thread() || idx + 1 >= cap) return;
  out[idx] = (uint64_t)*seed;
  out[idx + 1] = (uint64_t)*offset + intragraph;
}

// Pointer-free variant for the extra-style (packed arg buffer) path: the
// result goes to this code object's own array, indexed below its size.
constexpr uint32_t kProbeSlots = 256;
__device__ uint64_t probe_slots[kProbeSlots];

extern "C" __global__ void probe_mix_slot(uint32_t idx, uint32_t pad, uint64_t a, uint64_t b) {
  if (!first_thread() || idx >= kProbeSlots) return;
  uint64_t h = mix(mix(0x243F6A8885A308D3ull, a), b);
  probe_slots[idx] = mix(mix(h, gridDim.x), blockDim.x) ^ pad;
}

// Stands in for every kernel of a synthetic archive whose group graphs are
// built and switched but not launched: it reads only its first 8 param bytes.
extern "C" __global__ void fdy_sink(uint64_t first_word) {
  if (first_word == 0x5EED5EED5EED5EEDull && first_thread()) probe_slots[0] = first_word;
}
