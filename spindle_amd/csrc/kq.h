// Device building blocks of the integer K-quant path (Q4_K / Q6_K weights x Q8_K activations),
// restating rows<B,T> of quant_q8k.rs:163-250 on the gfx950 wavefront.
//
// Row group: 8 lanes own one weight row; lane l is the reference's 32-bit lane l of `sumi`
// (element e of a 256-block lands in lane (e % 32) / 4). Lane l walks the row's blocks in
// order and keeps its own fp32 accumulator acc_l = fma(d*xd_i, float(P_il), acc_l), exactly the
// reference's per-lane chain; the correction integer s_i (the min / -32 offset term) is summed
// over the 8 lanes with DPP (exact), and the row result is hsum(acc) - corr with the
// reference's tree ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)). A row's output is therefore bit
// identical to the reference's for the same Q8_K input, and independent of the batch size.
//
// Weights (device layout, built at upload): planar fields, and inside a Q4_K code record /
// Q6_K ql and qh records the bytes are permuted so that lane l's bytes are contiguous:
//   Q4_K codes: lane l holds qs[32c + 4l .. +4) for c = 0..3 at 16l (one 16-byte load)
//   Q6_K ql:    lane l holds ql[64h + 32mm + 4l .. +4) at 16l + 8h + 4mm
//   Q6_K qh:    lane l holds qh[32h + 4l .. +4) at 8l + 4h
// Activations ("Q8KP", permuted Q8_K): per 256-block, lane l's eight code dwords (elements
// 32k + 4l .. +3, k = 0..7) are contiguous at [blk][l][k]; d per block; and per block the
// pair (bsum_2l, bsum_2l+1) of 16-element code sums as int2 at [blk][l].
#pragma once
#include "common.h"

namespace spx {

// Q8_K activations in the permuted layout; vector v of a buffer with `cols` columns lives at
// q + v*cols/4, d + v*cols/256, bs + v*cols/256*8.
struct Q8KP {
  uint32_t *q;
  float *d;
  int2 *bs;
};

__device__ __forceinline__ uint4 ld16(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ uint2 ld8(const uint8_t *p) { return *reinterpret_cast<const uint2 *>(p); }

// Sum over the 8 lanes of each row group (exact, integer); every lane gets the total.
// row_half_mirror pairs lane i with 7-i, then the quad permutes [2,3,0,1] and [1,0,3,2].
__device__ __forceinline__ int sum8(int v) {
  v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true);
  v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);
  v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);
  return v;
}

// hsum of quant_q8k.rs:151-158 over the row group's 8 lane accumulators; valid in lane 0.
// DPP row shifts (lane j reads lane j + n of its 16-lane row; lanes 0-3 of a group read
// inside their own group): x_l = a_l + a_(l+4), t = x_l + x_(l+2), result t_0 + t_1.
#define SPX_SHLF(v, n) __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x100 + (n), 0xF, 0xF, true))
__device__ __forceinline__ float hsum_rows8(float a) {
  const float x = a + SPX_SHLF(a, 4);   // x_l = a_l + a_{l+4}
  const float t = x + SPX_SHLF(x, 2);   // lane 0: x0 + x2, lane 1: x1 + x3
  return t + SPX_SHLF(t, 1);            // (x0 + x2) + (x1 + x3)
}

// Raw bytes of one block as lane l loads them.
template <int T> struct KQRaw;
template <> struct KQRaw<T_Q4K> {
  uint4 c, h;  // c: this lane's 16 code bytes; h: d, dmin, scales[12]
  __device__ __forceinline__ void load(const Planes &pl, int64_t g, int l) {
    c = ld16(pl.p0 + g * 128 + 16 * l);
    h = ld16(pl.p1 + g * 16);
  }
};
template <> struct KQRaw<T_Q6K> {
  uint4 ql, sc;
  uint2 qh;
  uint32_t d;
  __device__ __forceinline__ void load(const Planes &pl, int64_t g, int l) {
    ql = ld16(pl.p0 + g * 128 + 16 * l);
    qh = ld8(pl.p1 + g * 64 + 8 * l);
    sc = ld16(pl.p2 + g * 16);
    d = *reinterpret_cast<const uint16_t *>(pl.p3 + g * 2);
  }
};

// A block decoded for lane l (shared by all activation vectors).
// The lane's scaled dot P = sum_k sc_k d_k (d_k the 4-code dot of sub-block k) is taken in
// Abel form: t_k = d_0 + .. + d_k accumulates in the dot instruction itself (v_dot4c, no
// zeroing), and P = sum_{k<7} (sc_k - sc_{k+1}) t_k + sc_7 t_7 with the differences computed
// once per block at decode. Same integer, every term exact: |t_k| <= 8 * 4 * 63 * 128 < 2^23
// and |sc_k - sc_{k+1}| <= 255, so the 24-bit multiplies (v_mad_i32_i24, full rate; a 32-bit
// multiply is quarter rate) see in-range operands and the sums stay far inside int32. The min
// correction's operands (mins 0..63 or int8 scales, bsums |.| <= 32 * 128) also fit 24 bits.
template <int T> struct KQDec;

// sum_k cf_k t_k over the running dots t_k of W_k . Y_k (cf: the Abel coefficients)
__device__ __forceinline__ int abel_dot8(const uint32_t (&W)[8], const uint32_t (&Y)[8], const int (&cf)[8]) {
  int t = sdot4((int)W[0], (int)Y[0], 0);
  int p = __mul24(cf[0], t);
#pragma unroll
  for (int k = 1; k < 8; k++) {
    t = sdot4((int)W[k], (int)Y[k], t);
    p += __mul24(cf[k], t);
  }
  return p;
}
__device__ __forceinline__ void abel_coef(int (&cf)[8], const int (&sc)[8]) {
#pragma unroll
  for (int k = 0; k < 7; k++) cf[k] = sc[k] - sc[k + 1];
  cf[7] = sc[7];
}
template <> struct KQDec<T_Q4K> {
  uint32_t w[8];  // sub-block k: lo nibbles of code word k / 2 (k even), hi nibbles (k odd)
  int cf[8], mn;  // Abel coefficients of the sub-block scales
  float d, dm;  // d and dmin
  __device__ __forceinline__ void decode(const KQRaw<T_Q4K> &r, int l) {
    const uint32_t cw[4] = {r.c.x, r.c.y, r.c.z, r.c.w};
#pragma unroll
    for (int c = 0; c < 4; c++) {
      w[2 * c] = cw[c] & 0x0F0F0F0Fu;             // sub-block 2c
      w[2 * c + 1] = (cw[c] >> 4) & 0x0F0F0F0Fu;  // sub-block 2c+1
    }
    // unpack_q4k_scales (q4k_gemv.rs:70-85): bytes 0-3 = S0, 4-7 = S1, 8-11 = S2
    const uint32_t S0 = r.h.y, S1 = r.h.z, S2 = r.h.w;
    int sc[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      sc[k] = (int)((S0 >> (8 * k)) & 63u);
      sc[4 + k] = (int)(((S2 >> (8 * k)) & 15u) | (((S0 >> (8 * k + 6)) & 3u) << 4));
    }
    abel_coef(cf, sc);
    const int k = l & 3;
    mn = l < 4 ? (int)((S1 >> (8 * k)) & 63u) : (int)(((S2 >> (8 * k + 4)) & 15u) | (((S1 >> (8 * k + 6)) & 3u) << 4));
    d = h2f(r.h.x);
    dm = h2f(r.h.x >> 16);
  }
  // P = this lane's scaled dot (lane l of sumi), s = its part of the min correction.
  __device__ __forceinline__ void dot(const uint4 &y0, const uint4 &y1, const int2 &bs, int &P, int &s) const {
    const uint32_t Y[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
    P = abel_dot8(w, Y, cf);
    s = __mul24(mn, bs.x + bs.y);
  }
  // corr += (dmin*xd) * float(s); the caller applies acc = fma(d*xd, float(P), acc)
  __device__ __forceinline__ float corr_term(float xd, int s) const { return (dm * xd) * (float)s; }
};
template <> struct KQDec<T_Q6K> {
  uint32_t q[8];  // k = 4h + m: codes of elements 32k + 4l .. +3 (0..63)
  int cf[8], sa, sb;  // Abel coefficients of the lane's eight scales
  float d, dm;
  __device__ __forceinline__ void decode(const KQRaw<T_Q6K> &r, int l) {
    const uint32_t QL[4] = {r.ql.x, r.ql.y, r.ql.z, r.ql.w};  // [h][mm]
    const uint32_t QH[2] = {r.qh.x, r.qh.y};
    const uint32_t SC[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
    const int hb = (l >> 2) * 8;  // scale of elements 16..31 of each 32 for lanes 4..7
    int sc[8];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int m = 0; m < 4; m++) {
        const uint32_t lo4 = (QL[2 * h + (m & 1)] >> (4 * (m >> 1))) & 0x0F0F0F0Fu;
        const uint32_t hi2 = ((QH[h] >> (2 * m)) & 0x03030303u) << 4;
        q[4 * h + m] = lo4 | hi2;
        // scale index 8h + 2m + (l >> 2): word 2h + (m >> 1), byte 2(m & 1) + (l >> 2)
        sc[4 * h + m] = (int)(int8_t)(SC[2 * h + (m >> 1)] >> (16 * (m & 1) + hb));
      }
    abel_coef(cf, sc);
    // scales 2l and 2l+1 for this lane's share of 32 * sum_g sc_g * bsum_g
    const uint32_t w = l < 4 ? (l < 2 ? SC[0] : SC[1]) : (l < 6 ? SC[2] : SC[3]);
    const int sh = 16 * (l & 1);
    sa = (int)(int8_t)(w >> sh);
    sb = (int)(int8_t)(w >> (sh + 8));
    d = h2f(r.d);
    dm = d;
  }
  __device__ __forceinline__ void dot(const uint4 &y0, const uint4 &y1, const int2 &bs, int &P, int &s) const {
    const uint32_t Y[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
    P = abel_dot8(q, Y, cf);
    s = __mul24(sa, bs.x) + __mul24(sb, bs.y);
  }
  __device__ __forceinline__ float corr_term(float xd, int s) const { return (dm * xd) * (float)(32 * s); }
};

}  // namespace spx
