// crc64.h -- CRC-64/XZ arithmetic for host and device.
//
// CRC-64/XZ is the code-object identity hash of the reference
// (csrc/hook.cpp:315-321: width 64, poly 0x42F0E1EBA9EA3693, reflected in
// and out, init and xorout all ones).  The restore path uses it for every
// per-graph digest so that digests are checkable against any textbook
// CRC-64/XZ implementation.
//
// Reflected representation: bit 63 holds the coefficient of x^0, so a
// right shift multiplies by x.  Segments are combined with
//   crc(A || B) = (crc(A) * x^(8|B|) mod P) xor crc(B)
// (the method of zlib's crc32_combine, Adler 2011), which holds for raw
// register values (init 0, no xorout) and for finished values alike.  For
// fixed-size records the multipliers x^(8*S*2^k) are constants; device code
// multiplies by them through 16 nibble tables per constant.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fdy {

constexpr uint64_t kCrcPolyRefl = 0xC96C5795D7870F42ull;  // 0x42F0E1EBA9EA3693 bit-reversed
constexpr uint64_t kX0 = 0x8000000000000000ull;           // the polynomial "1"

// a * b mod P, reflected; 64 steps, branch-free in b.
__host__ __device__ inline uint64_t gf2_mulmod(uint64_t a, uint64_t b) {
  uint64_t p = 0;
  for (int i = 0; i < 64; ++i) {
    uint64_t bit = (a >> (63 - i)) & 1;
    p ^= b & (0 - bit);
    b = (b >> 1) ^ (kCrcPolyRefl & (0 - (b & 1)));
  }
  return p;
}

// x^(2^k) mod P for k = 0..63.
struct X2nTable {
  uint64_t v[64];
};

inline X2nTable make_x2n_table() {
  X2nTable t;
  uint64_t p = kX0 >> 1;  // x^1
  for (int k = 0; k < 64; ++k) {
    t.v[k] = p;
    p = gf2_mulmod(p, p);
  }
  return t;
}

// x^(n * 2^k) mod P.
__host__ __device__ inline uint64_t x2n_mod(const uint64_t* x2n, uint64_t n, unsigned k) {
  uint64_t p = kX0;
  while (n) {
    if (n & 1) p = gf2_mulmod(x2n[k & 63], p);
    n >>= 1;
    ++k;
  }
  return p;
}

// Slicing-by-8 tables: t[0] is the byte table, t[k][i] = byte i followed by k zero bytes.
struct SliceTables {
  uint64_t t[8][256];
};

inline SliceTables make_slice_tables() {
  SliceTables s;
  for (int i = 0; i < 256; ++i) {
    uint64_t c = (uint64_t)i;
    for (int b = 0; b < 8; ++b) c = (c & 1) ? (c >> 1) ^ kCrcPolyRefl : c >> 1;
    s.t[0][i] = c;
  }
  for (int k = 1; k < 8; ++k)
    for (int i = 0; i < 256; ++i) s.t[k][i] = (s.t[k - 1][i] >> 8) ^ s.t[0][s.t[k - 1][i] & 0xFF];
  return s;
}

// Register after absorbing 8 bytes (little-endian word w) into register c.
__host__ __device__ inline uint64_t crc_slice8(const uint64_t (*t)[256], uint64_t c, uint64_t w) {
  c ^= w;
  return t[7][c & 0xFF] ^ t[6][(c >> 8) & 0xFF] ^ t[5][(c >> 16) & 0xFF] ^ t[4][(c >> 24) & 0xFF] ^
         t[3][(c >> 32) & 0xFF] ^ t[2][(c >> 40) & 0xFF] ^ t[1][(c >> 48) & 0xFF] ^ t[0][c >> 56];
}

__host__ __device__ inline uint64_t crc_byte(const uint64_t* t0, uint64_t c, uint8_t b) {
  return t0[(c ^ b) & 0xFF] ^ (c >> 8);
}

// Nibble tables for multiplying by a fixed constant X:
//   z * X mod P = xor over i of tab[i][(z >> 4i) & 15]
struct NibbleTable {
  uint64_t t[16][16];
};

inline NibbleTable make_nibble_table(uint64_t X) {
  NibbleTable n;
  for (int i = 0; i < 16; ++i)
    for (int v = 0; v < 16; ++v) n.t[i][v] = gf2_mulmod((uint64_t)v << (4 * i), X);
  return n;
}

__host__ __device__ inline uint64_t nibble_mul(const uint64_t (*tab)[16], uint64_t z) {
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) r ^= tab[i][(z >> (4 * i)) & 15];
  return r;
}

// Records per node-pass chunk, and the multiplier of record i's raw CRC in
// its chunk's CRC: x^(8 * 16 * (kPosRecords - 1 - i)) mod P.
constexpr int kPosRecords = 256;

// Lanes of a byte-stream chunk (64 bytes each), and the multiplier of lane
// i's raw CRC in its chunk's CRC: x^(8 * 64 * (kPosLanes - 1 - i)) mod P.
constexpr int kPosLanes = 1024;

// Node-pass chunks a graph's chunk CRCs can be shifted past by table: for
// k < kChunkShifts, chunk_shift[k][i] = x^(8 * 16 * kPosRecords * k) * x^i
// mod P, so one wave forms a chunk's shifted CRC with one multiple per lane
// (lane i takes it when bit x^i of the CRC is set) and an XOR reduction.
constexpr int kChunkShifts = 256;

struct CrcConsts {
  SliceTables slice;
  NibbleTable chunk64;             // x^(8 * 64 * kPosLanes): joins 64 KB byte-stream chunks
  X2nTable x2n;
  uint64_t pos16[kPosRecords];
  uint64_t pos64[kPosLanes];
  uint64_t chunk_shift[kChunkShifts][64];
};

inline void make_crc_consts(CrcConsts* c) {
  c->slice = make_slice_tables();
  c->x2n = make_x2n_table();
  c->chunk64 = make_nibble_table(x2n_mod(c->x2n.v, 64ull * kPosLanes, 3));
  for (int i = 0; i < kPosRecords; ++i) c->pos16[i] = x2n_mod(c->x2n.v, 16ull * (kPosRecords - 1 - i), 3);
  for (int i = 0; i < kPosLanes; ++i) c->pos64[i] = x2n_mod(c->x2n.v, 64ull * (kPosLanes - 1 - i), 3);
  for (int k = 0; k < kChunkShifts; ++k) {
    uint64_t m = x2n_mod(c->x2n.v, 16ull * kPosRecords * k, 3);
    for (int i = 0; i < 64; ++i) {
      c->chunk_shift[k][i] = m;
      m = (m >> 1) ^ (kCrcPolyRefl & (0 - (m & 1)));  // times x
    }
  }
}

// Finish a raw CRC of an L-byte stream: crc = raw ^ (~0 * x^(8L)) ^ ~0.
// The term after `raw` depends on L only; hosts precompute it per stream.
__host__ __device__ inline uint64_t crc_finish_term(const uint64_t* x2n, uint64_t len) {
  return gf2_mulmod(x2n_mod(x2n, len, 3), ~0ull) ^ ~0ull;
}

}  // namespace fdy
