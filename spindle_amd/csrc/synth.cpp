// Seeded synthetic weights in GGUF block layout (counter-based, so any block can be produced
// independently and in parallel, on any host, with identical bytes).
//
// Every 64-bit word is mix(seed, index) (a SplitMix64 finaliser over a Weyl sequence); block
// g of a tensor draws its words from indices [g*32, g*32+32). Field rules (sigma = target
// standard deviation of the dequantised weight):
//   Q4_K: scales/mins (12 B) and codes (128 B) uniform; d = f16(sigma/258.3 * j), dmin =
//         f16(7.5 * d) (zero mean), j in [0.75, 1.25) per block.
//   Q6_K: ql, qh uniform; int8 scales uniform; d = f16(sigma/1365.3 * j) (f16-subnormal range,
//         converted with round-to-nearest-even).
//   Q8_0: codes uniform in [-127, 127]; d = f16(sigma/73.6 * j).
//   Q5_0: low nibbles and high bits uniform; d = f16(sigma/9.23 * j).
//   Q5_K: scales/mins, high bits and codes uniform; d = f16(sigma/533 * j), dmin = f16(15.5 * d).
//   F32:  kind 1: uniform with standard deviation sigma; kind 2: 1 + sigma * U(-1, 1).
#include <string.h>

#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "../../include/spx.h"
#include "internal.h"

namespace {

inline uint64_t mix(uint64_t seed, uint64_t i) {
  uint64_t z = seed * 0xD1B54A32D192ED03ull + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline float unit(uint64_t w) { return (float)(w >> 40) * (1.0f / 16777216.0f); }  // [0, 1)

uint16_t f2h(float f) {  // IEEE binary16, round to nearest even
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000, ax = x & 0x7fffffff;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00 | (ax > 0x7f800000u ? 0x200 : 0));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00);
  if (ax < 0x38800000u) {
    if (ax < 0x33000000u) return (uint16_t)sign;
    const int e = (int)(ax >> 23), s = 126 - e;
    const uint32_t m = (ax & 0x7fffff) | 0x800000;
    uint32_t q = m >> s;
    const uint32_t rem = m & ((1u << s) - 1), half = 1u << (s - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return (uint16_t)(sign | q);
  }
  const uint32_t e = (ax >> 23) - 112, m = ax & 0x7fffff;
  uint32_t q = (e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) q++;
  return (uint16_t)(sign | q);
}

float h2f_host(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16, exp = (h >> 10) & 0x1f, mant = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (mant == 0) bits = sign;
    else {
      uint32_t m = mant;
      int e = 127 - 14;
      while ((m & 0x400) == 0) { m <<= 1; e--; }
      bits = sign | ((uint32_t)e << 23) | ((m & 0x3ff) << 13);
    }
  } else if (exp == 31) bits = sign | 0x7f800000u | (mant << 13);
  else bits = sign | ((exp + 112) << 23) | (mant << 13);
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

void fill_bytes(uint8_t *dst, int n, uint64_t seed, uint64_t idx) {
  for (int i = 0; i < n; i += 8) {
    const uint64_t w = mix(seed, idx + i / 8);
    const int k = n - i < 8 ? n - i : 8;
    memcpy(dst + i, &w, k);
  }
}

void gen_block(int dtype, uint8_t *blk, uint64_t seed, uint64_t g, float sigma) {
  const uint64_t base = g * 32;
  const float j = 0.75f + 0.5f * unit(mix(seed, base + 31));
  switch (dtype) {
  case spx::T_Q4K: {
    fill_bytes(blk + 4, 140, seed, base);
    const uint16_t d = f2h(sigma / 258.3f * j);
    const uint16_t dm = f2h(7.5f * h2f_host(d));
    memcpy(blk, &d, 2);
    memcpy(blk + 2, &dm, 2);
    break;
  }
  case spx::T_Q5K: {
    fill_bytes(blk + 4, 172, seed, base);
    const uint16_t d = f2h(sigma / 533.0f * j);
    const uint16_t dm = f2h(15.5f * h2f_host(d));
    memcpy(blk, &d, 2);
    memcpy(blk + 2, &dm, 2);
    break;
  }
  case spx::T_Q6K: {
    fill_bytes(blk, 208, seed, base);
    const uint16_t d = f2h(sigma / 1365.3f * j);
    memcpy(blk + 208, &d, 2);
    break;
  }
  case spx::T_Q8_0: {
    uint8_t r[32];
    fill_bytes(r, 32, seed, base);
    for (int i = 0; i < 32; i++) blk[2 + i] = (uint8_t)(int8_t)((int)(r[i] % 255) - 127);
    const uint16_t d = f2h(sigma / 73.6f * j);
    memcpy(blk, &d, 2);
    break;
  }
  case spx::T_Q5_0: {
    fill_bytes(blk + 2, 20, seed, base);
    const uint16_t d = f2h(sigma / 9.23f * j);
    memcpy(blk, &d, 2);
    break;
  }
  }
}

}  // namespace

extern "C" {

// Fills `out` (GGUF layout, n_expert slabs of rows x cols) with seeded synthetic values.
// kind 0: quantized weights (dtype Q4_K/Q5_K/Q6_K/Q8_0/Q5_0) with std sigma; kind 1: F32 uniform
// with std sigma; kind 2: F32 1 + sigma*U(-1,1) (norm weights).
int spx_synth_tensor(int dtype, int64_t cols, int64_t rows, int n_expert, uint64_t seed, float sigma, int kind, void *out) {
  const int64_t rb = spx::row_bytes(dtype, cols);
  if (!rb || !out || rows <= 0 || n_expert <= 0) return spx::fail("spx_synth_tensor: bad arguments");
  uint8_t *o = static_cast<uint8_t *>(out);
  const int64_t total_rows = rows * n_expert;
  if (dtype == spx::T_F32) {
    const int64_t n = total_rows * cols;
    const float a = sigma * std::sqrt(3.0f);
    float *f = reinterpret_cast<float *>(o);
    for (int64_t i = 0; i < n; i++) {
      const float u = unit(mix(seed, (uint64_t)i));
      f[i] = kind == 2 ? 1.0f + sigma * (2.0f * u - 1.0f) : a * (2.0f * u - 1.0f);
    }
    return 0;
  }
  const int64_t be = spx::block_elems(dtype), bb = rb / (cols / be);
  const int64_t nblk = total_rows * (cols / be);
  const int nt = (int)std::min<int64_t>(16, std::max<int64_t>(1, nblk / 65536));
  std::vector<std::thread> th;
  for (int t = 0; t < nt; t++)
    th.emplace_back([=] {
      for (int64_t g = nblk * t / nt; g < nblk * (t + 1) / nt; g++) gen_block(dtype, o + g * bb, seed, (uint64_t)g, sigma);
    });
  for (auto &x : th) x.join();
  return 0;
}

}  // extern "C"
