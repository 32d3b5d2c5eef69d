// Quantized matrix x activation-vector kernels for gfx950 (wave64).
//
// Integer path (Q4_K, Q6_K x Q8_K), restating quant_q8k.rs:163-295 (rows<B,T>/matmul_rows):
//   per block i and vector v the kernel forms the exact int32 quantities of the reference,
//     S_i = sum_e scale(e) * w_e * y_e            (Q4_K: 6-bit scale per 32, codes 0..15;
//                                                  Q6_K: int8 scale per 16, codes 0..63)
//     s_i = Q4_K: sum_j min_j * (bsum_2j + bsum_2j+1);  Q6_K: 32 * sum_g scale_g * bsum_g
//   with v_dot4_i32_i8 (codes are non-negative, so the signed dot is exact), split exactly
//   like the reference's 8 x int32 lanes of sumi (element e in lane (e % 32) / 4), then the
//   reference's fp32 epilogue: eight chains acc_l = fma(d*xd_i, float(P_il), acc_l) in block
//   order, corr = corr + (dmin*xd_i) * float(s_i) (Q6_K: (d*xd_i) * float(32 s)), and
//   out = hsum(acc) - corr with the tree of quant_q8k.rs:151-158. Given the same Q8_K input
//   the output is bit-identical to the reference's rows<B,T>, for every batch size (the
//   property quant_q8k.rs:413-442 tests).
//
// Float path (Q8_0, Q5_0, F32 weights x fp32 activations), restating quant.rs:48-161 and
// quant_multi.rs:168-190: per block s = sum q_e * x_e, acc = fma(d, s, acc); the reduction
// order is this kernel's own (fixed, batch-independent), within 1e-4 of the reference's.
//
// Mapping: a workgroup of 256 threads is 64 quads; quad q owns weight row r0+blockIdx.x*64+q
// and walks that row's blocks in order. Integer path: lane c of the quad takes code bytes
// [32c, 32c+32) of a Q4_K block (scale groups 2c, 2c+1) or the (half c>>1, l-range c&1) slice
// of a Q6_K block; the quad sums its four int32 partials with DPP quad permutes (exact).
// Float path: lane c owns blocks c, c+4, c+8, ... of the row.
#include <algorithm>

#include "common.h"

namespace spx {



template <int MT>
struct VecSet {
  int m;
  int src[MT];
  int dst[MT];
};

// ---------------------------------------------------------------- Q4_K block decode
// The activation slice a lane needs for one block: four 16-byte pieces of Q8_K codes and the
// bsums its sub-blocks use.
struct YSlice {
  uint4 y[4];
  int bs[4];
};

struct Q4KBlock {
  uint32_t lo[8], hi[8];
  int sc0, sc1, mn0, mn1;
  float d, dmin;
  __device__ __forceinline__ void load(const Planes &pl, int64_t g, int c) {
    const uint4 q0 = *reinterpret_cast<const uint4 *>(pl.p0 + g * 128 + c * 32);
    const uint4 q1 = *reinterpret_cast<const uint4 *>(pl.p0 + g * 128 + c * 32 + 16);
    const uint4 hd = *reinterpret_cast<const uint4 *>(pl.p1 + g * 16);
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int t = 0; t < 8; t++) {
      lo[t] = w[t] & 0x0F0F0F0Fu;
      hi[t] = (w[t] >> 4) & 0x0F0F0F0Fu;
    }
    d = h2f(hd.x);
    dmin = h2f(hd.x >> 16);
    // 6-bit scale/min unpack of q4k_gemv.rs:70-85 for sub-blocks 2c and 2c+1.
    const uint32_t S0 = hd.y, S1 = hd.z, S2 = hd.w;
    if (c < 2) {
      const int k0 = 2 * c, k1 = 2 * c + 1;
      sc0 = (S0 >> (8 * k0)) & 63; mn0 = (S1 >> (8 * k0)) & 63;
      sc1 = (S0 >> (8 * k1)) & 63; mn1 = (S1 >> (8 * k1)) & 63;
    } else {
      const int k0 = 2 * c - 4, k1 = 2 * c - 3;
      sc0 = ((S2 >> (8 * k0)) & 0xF) | (((S0 >> (8 * k0 + 6)) & 3) << 4);
      mn0 = ((S2 >> (8 * k0 + 4)) & 0xF) | (((S1 >> (8 * k0 + 6)) & 3) << 4);
      sc1 = ((S2 >> (8 * k1)) & 0xF) | (((S0 >> (8 * k1 + 6)) & 3) << 4);
      mn1 = ((S2 >> (8 * k1 + 4)) & 0xF) | (((S1 >> (8 * k1 + 6)) & 3) << 4);
    }
  }
  // y: the vector's 256 codes of this block; bs: its 16 bsums. Lane c: codes [64c, 64c+64).
  static __device__ __forceinline__ void load_y(const int8_t *y, const int16_t *bs, int c, YSlice &ys) {
    const uint4 *yl = reinterpret_cast<const uint4 *>(y + c * 64);
    ys.y[0] = yl[0]; ys.y[1] = yl[1]; ys.y[2] = yl[2]; ys.y[3] = yl[3];
    const int2 bb = *reinterpret_cast<const int2 *>(bs + 4 * c);
    ys.bs[0] = (int)(int16_t)(bb.x & 0xffff); ys.bs[1] = (int)(int16_t)(bb.x >> 16);
    ys.bs[2] = (int)(int16_t)(bb.y & 0xffff); ys.bs[3] = (int)(int16_t)(bb.y >> 16);
  }
  // Lane c's contribution to the eight 32-bit lanes of the reference's sumi (element e goes to
  // lane (e % 32) / 4): dword t of this lane's codes holds elements 64c + 4t.. (low nibbles, scale
  // 2c) and 64c + 32 + 4t.. (high nibbles, scale 2c+1), both in lane t.
  __device__ __forceinline__ void dot8(const YSlice &ys, int c, int P[8], int &s) const {
    const int ya[8] = {(int)ys.y[0].x, (int)ys.y[0].y, (int)ys.y[0].z, (int)ys.y[0].w, (int)ys.y[1].x, (int)ys.y[1].y, (int)ys.y[1].z, (int)ys.y[1].w};
    const int yb[8] = {(int)ys.y[2].x, (int)ys.y[2].y, (int)ys.y[2].z, (int)ys.y[2].w, (int)ys.y[3].x, (int)ys.y[3].y, (int)ys.y[3].z, (int)ys.y[3].w};
#pragma unroll
    for (int t = 0; t < 8; t++) P[t] = sc0 * sdot4((int)lo[t], ya[t], 0) + sc1 * sdot4((int)hi[t], yb[t], 0);
    s = mn0 * (ys.bs[0] + ys.bs[1]) + mn1 * (ys.bs[2] + ys.bs[3]);
  }
  __device__ __forceinline__ void dot(const YSlice &ys, int c, int &p, int &s) const {
    int P[8];
    dot8(ys, c, P, s);
    p = ((P[0] + P[1]) + (P[2] + P[3])) + ((P[4] + P[5]) + (P[6] + P[7]));
  }
  __device__ __forceinline__ float dm() const { return dmin; }
};

// ---------------------------------------------------------------- Q6_K block decode
struct Q6KBlock {
  uint32_t q[4][4];  // [group m][dword t], codes 0..63
  int sc[4];
  float d;
  __device__ __forceinline__ void load(const Planes &pl, int64_t g, int c) {
    const int h = c >> 1, half = c & 1;
    const uint4 la = *reinterpret_cast<const uint4 *>(pl.p0 + g * 128 + 64 * h + 16 * half);
    const uint4 lb = *reinterpret_cast<const uint4 *>(pl.p0 + g * 128 + 64 * h + 32 + 16 * half);
    const uint4 qh = *reinterpret_cast<const uint4 *>(pl.p1 + g * 64 + 32 * h + 16 * half);
    const uint4 sv = *reinterpret_cast<const uint4 *>(pl.p2 + g * 16);
    d = h2f(*reinterpret_cast<const uint16_t *>(pl.p3 + g * 2));
    const uint32_t A[4] = {la.x, la.y, la.z, la.w}, B[4] = {lb.x, lb.y, lb.z, lb.w}, H[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int t = 0; t < 4; t++) {
      q[0][t] = (A[t] & 0x0F0F0F0Fu) | ((H[t] & 0x03030303u) << 4);
      q[1][t] = (B[t] & 0x0F0F0F0Fu) | (((H[t] >> 2) & 0x03030303u) << 4);
      q[2][t] = ((A[t] >> 4) & 0x0F0F0F0Fu) | (((H[t] >> 4) & 0x03030303u) << 4);
      q[3][t] = ((B[t] >> 4) & 0x0F0F0F0Fu) | (((H[t] >> 6) & 0x03030303u) << 4);
    }
    // scale index of group m: 8h + 2m + half (element 128h + 32m + 16half + j, j < 16)
    const uint32_t w0 = h ? sv.z : sv.x, w1 = h ? sv.w : sv.y;
    sc[0] = (int)(int8_t)(w0 >> (8 * half));
    sc[1] = (int)(int8_t)(w0 >> (8 * (2 + half)));
    sc[2] = (int)(int8_t)(w1 >> (8 * half));
    sc[3] = (int)(int8_t)(w1 >> (8 * (2 + half)));
  }
  // Lane c = (h, half): codes 128h + 32m + 16half + [0, 16) for m = 0..3, bsums 8h + 2m + half.
  static __device__ __forceinline__ void load_y(const int8_t *y, const int16_t *bs, int c, YSlice &ys) {
    const int h = c >> 1, half = c & 1;
#pragma unroll
    for (int m = 0; m < 4; m++) ys.y[m] = *reinterpret_cast<const uint4 *>(y + 128 * h + 32 * m + 16 * half);
    const int4 bb = *reinterpret_cast<const int4 *>(bs + 8 * h);  // bsums 8h .. 8h+7
    const int w[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
    for (int m = 0; m < 4; m++) ys.bs[m] = (int)(int16_t)((w[m] >> (16 * half)) & 0xffff);
  }
  // Lane c = (h, half) holds elements 128h + 32m + 16half + 4t.. for m = 0..3: reference lane
  // 4*half + t (scale per 16 elements, so one scale per (m, half)).
  __device__ __forceinline__ void dot8(const YSlice &ys, int c, int P[8], int &s) const {
    const int half = c & 1;
    int L[4];
    const uint32_t *yw[4] = {&ys.y[0].x, &ys.y[1].x, &ys.y[2].x, &ys.y[3].x};
#pragma unroll
    for (int t = 0; t < 4; t++) {
      int acc = 0;
#pragma unroll
      for (int m = 0; m < 4; m++) acc += sc[m] * sdot4((int)q[m][t], (int)yw[m][t], 0);
      L[t] = acc;
    }
#pragma unroll
    for (int t = 0; t < 4; t++) { P[t] = half ? 0 : L[t]; P[4 + t] = half ? L[t] : 0; }
    s = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) s += sc[m] * ys.bs[m];
  }
  __device__ __forceinline__ void dot(const YSlice &ys, int c, int &p, int &s) const {
    int P[8];
    dot8(ys, c, P, s);
    p = ((P[0] + P[1]) + (P[2] + P[3])) + ((P[4] + P[5]) + (P[6] + P[7]));
  }
  __device__ __forceinline__ float dm() const { return d; }
};

template <int T>
struct KQBlock;
template <> struct KQBlock<T_Q4K> { using type = Q4KBlock; };
template <> struct KQBlock<T_Q6K> { using type = Q6KBlock; };

// The fp32 epilogue of rows<B,T> (quant_q8k.rs:204/:232/:243-247), bit for bit: eight lane
// accumulators acc_l = fma(d*xd, float(P_l), acc_l) over the blocks in order, the correction
// chain corr = corr + (dmin*xd)*float(s) (Q6_K: (d*xd)*float(32 s)), and out =
// hsum(acc) - corr with the tree ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) of quant_q8k.rs:151-158.
template <int T>
__device__ __forceinline__ void kq_accum8(float d, float dm, float xdv, const int *P, int s, float acc[8], float &corr) {
  if (T == T_Q4K) corr = corr + (dm * xdv) * (float)s;
  else corr = corr + (dm * xdv) * (float)(32 * s);
  const float dd = d * xdv;
#pragma unroll
  for (int l = 0; l < 8; l++) acc[l] = fmaf(dd, (float)P[l], acc[l]);
}
__device__ __forceinline__ float hsum8(const float a[8]) {
  const float x0 = a[0] + a[4], x1 = a[1] + a[5], x2 = a[2] + a[6], x3 = a[3] + a[7];
  return (x0 + x2) + (x1 + x3);
}

// Block-parallel integer matvec. A pass covers R = (64/nb)*RR rows: quad q takes block q%nb of
// row group q/nb (RR rows), forms the exact int32 partials for every vector and leaves them in
// LDS; then one thread per (row, vector) runs the fp32 chain over the blocks in order.
template <int T, int MT, int RR, bool GROUPED>
__global__ __launch_bounds__(256) void k_gemv_kq(KQArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  VecSet<MT> vs;
  int expert;
  if (GROUPED) {
    if ((int)blockIdx.y >= *a.njobs) return;
    const Job &J = a.jobs[blockIdx.y];
    expert = J.expert;
    vs.m = J.nvec;
#pragma unroll
    for (int v = 0; v < MT; v++) { vs.src[v] = v < J.nvec ? J.vec[v] : 0; vs.dst[v] = v < J.nvec ? J.out[v] : 0; }
  } else {
    expert = a.expert;
    vs.m = a.m;
#pragma unroll
    for (int v = 0; v < MT; v++) { vs.src[v] = v; vs.dst[v] = v; }
  }
  const int nb = (int)a.w.nb, cols = (int)a.w.cols;
  const int gpp = 64 / nb, R = gpp * RR;            // row groups and rows per pass
  int *sP = reinterpret_cast<int *>(smem);          // [R][nb][MT][8] lane partials
  int *sS = sP + R * nb * MT * 8;                    // [R][nb][MT]
  float *sD = reinterpret_cast<float *>(sS + R * nb * MT);  // [R][nb]
  float *sM = sD + R * nb;                           // [R][nb]
  const int quad = threadIdx.x >> 2, c = threadIdx.x & 3;
  const int grp = quad / nb, blk = quad % nb;
  const bool active = grp < gpp;
  const int64_t rows_per_wg = (int64_t)R * a.passes;
  const int64_t wg_r0 = a.r0 + (int64_t)blockIdx.x * rows_per_wg;
  for (int pass = 0; pass < a.passes; pass++) {
    const int64_t pr0 = wg_r0 + (int64_t)pass * R;
    if (pr0 >= a.r1) break;
    if (active) {
      typename KQBlock<T>::type B[RR];
      bool ok[RR];
#pragma unroll
      for (int rr = 0; rr < RR; rr++) {
        const int64_t row = pr0 + grp * RR + rr;
        ok[rr] = row < a.r1;
        if (ok[rr]) B[rr].load(a.w.pl, ((int64_t)expert * a.w.rows + row) * nb + blk, c);
      }
#pragma unroll
      for (int v = 0; v < MT; v++) {
        if (v < vs.m) {
          YSlice ys;
          KQBlock<T>::type::load_y(a.xq + (int64_t)vs.src[v] * cols + blk * 256, a.xb + ((int64_t)vs.src[v] * nb + blk) * 16, c, ys);
#pragma unroll
          for (int rr = 0; rr < RR; rr++) {
            int P[8] = {0, 0, 0, 0, 0, 0, 0, 0}, s = 0;
            if (ok[rr]) B[rr].dot8(ys, c, P, s);
#pragma unroll
            for (int l = 0; l < 8; l++) P[l] = quad_sum(P[l]);
            s = quad_sum(s);
            if (c == 0) {
              const int o = ((grp * RR + rr) * nb + blk) * MT + v;
              int4 *pp = reinterpret_cast<int4 *>(sP + 8 * o);
              pp[0] = make_int4(P[0], P[1], P[2], P[3]);
              pp[1] = make_int4(P[4], P[5], P[6], P[7]);
              sS[o] = s;
            }
          }
        }
      }
      if (c == 0) {
#pragma unroll
        for (int rr = 0; rr < RR; rr++) {
          sD[(grp * RR + rr) * nb + blk] = ok[rr] ? B[rr].d : 0.0f;
          sM[(grp * RR + rr) * nb + blk] = ok[rr] ? B[rr].dm() : 0.0f;
        }
      }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < R * vs.m; t += 256) {
      const int r = t / vs.m, v = t % vs.m;
      const int64_t row = pr0 + r;
      if (row < a.r1) {
        const float *xd = a.xd + (int64_t)vs.src[v] * nb;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, corr = 0.0f;
        for (int i = 0; i < nb; i++) {
          const int o = (r * nb + i) * MT + v;
          kq_accum8<T>(sD[r * nb + i], sM[r * nb + i], xd[i], sP + 8 * o, sS[o], acc, corr);
        }
        a.out[(int64_t)vs.dst[v] * a.ld_out + row] = hsum8(acc) - corr;
      }
    }
    __syncthreads();
  }
}

// Per-block integer probe for one (row, vector): the same decode and dot as k_gemv_kq.
template <int T>
__global__ __launch_bounds__(64) void k_kq_block_sums(KQArgs a) {
  const int c = threadIdx.x & 3, blk = threadIdx.x >> 2;  // 16 blocks per workgroup
  const int64_t i = (int64_t)blockIdx.x * 16 + blk;
  if (i >= a.w.nb) return;
  const int64_t g = ((int64_t)a.expert * a.w.rows + a.r0) * a.w.nb + i;
  typename KQBlock<T>::type B;
  B.load(a.w.pl, g, c);
  YSlice ys;
  KQBlock<T>::type::load_y(a.xq + i * 256, a.xb + i * 16, c, ys);
  int p, s;
  B.dot(ys, c, p, s);
  p = quad_sum(p);
  s = quad_sum(s);
  if (c == 0) { a.dbg[2 * i] = p; a.dbg[2 * i + 1] = T == T_Q6K ? 32 * s : s; }
}

// ---------------------------------------------------------------- float path


template <int T, int MT, bool GROUPED>
__global__ __launch_bounds__(256) void k_gemv_f(FArgs a) {
  VecSet<MT> vs;
  int expert;
  if (GROUPED) {
    if ((int)blockIdx.y >= *a.njobs) return;
    const Job &J = a.jobs[blockIdx.y];
    expert = J.expert;
    vs.m = J.nvec;
#pragma unroll
    for (int v = 0; v < MT; v++) { vs.src[v] = v < J.nvec ? J.vec[v] : 0; vs.dst[v] = v < J.nvec ? J.out[v] : 0; }
  } else {
    expert = a.expert;
    vs.m = a.m;
#pragma unroll
    for (int v = 0; v < MT; v++) { vs.src[v] = v; vs.dst[v] = v; }
  }
  const int quad = threadIdx.x >> 2, c = threadIdx.x & 3;
  const int64_t r = a.r0 + (int64_t)blockIdx.x * 64 + quad;
  if (r >= a.r1) return;
  const int64_t row = (int64_t)expert * a.w.rows + r;
  float acc[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) acc[v] = 0.0f;
  if (T == T_F32) {
    const float4 *wr = reinterpret_cast<const float4 *>(a.w.pl.p0 + row * a.w.cols * 4);
    const int64_t n4 = a.w.cols / 4;
    float part[MT][4];
#pragma unroll
    for (int v = 0; v < MT; v++) part[v][0] = part[v][1] = part[v][2] = part[v][3] = 0.0f;
    for (int64_t k = c; k < n4; k += 4) {
      const float4 w = wr[k];
#pragma unroll
      for (int v = 0; v < MT; v++) {
        if (v < vs.m) {
          const float4 xv = reinterpret_cast<const float4 *>(a.x + (int64_t)vs.src[v] * a.ld_x)[k];
          part[v][0] = fmaf(w.x, xv.x, part[v][0]);
          part[v][1] = fmaf(w.y, xv.y, part[v][1]);
          part[v][2] = fmaf(w.z, xv.z, part[v][2]);
          part[v][3] = fmaf(w.w, xv.w, part[v][3]);
        }
      }
    }
#pragma unroll
    for (int v = 0; v < MT; v++) acc[v] = (part[v][0] + part[v][1]) + (part[v][2] + part[v][3]);
  } else {
    const int64_t nb = a.w.nb;
    for (int64_t i = c; i < nb; i += 4) {
      const int64_t g = row * nb + i;
      float q[32];
      float d = h2f(*reinterpret_cast<const uint16_t *>(a.w.pl.p3 + g * 2));
      if (T == T_Q8_0) {
        const uint4 c0 = *reinterpret_cast<const uint4 *>(a.w.pl.p0 + g * 32);
        const uint4 c1 = *reinterpret_cast<const uint4 *>(a.w.pl.p0 + g * 32 + 16);
        const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
          for (int j = 0; j < 4; j++) q[4 * k + j] = (float)(int8_t)(cw[k] >> (8 * j));
      } else {  // Q5_0: element j<16 low nibble of qs[j] | bit j; j>=16 high nibble | bit j
        const uint4 qs = *reinterpret_cast<const uint4 *>(a.w.pl.p0 + g * 16);
        const uint32_t qh = *reinterpret_cast<const uint32_t *>(a.w.pl.p1 + g * 4);
        const uint32_t cw[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int e = 4 * k + j;
            const int byte = (cw[k] >> (8 * j)) & 0xff;
            q[e] = (float)((int)((byte & 0xF) | (((qh >> e) & 1u) << 4)) - 16);
            q[e + 16] = (float)((int)((byte >> 4) | (((qh >> (e + 16)) & 1u) << 4)) - 16);
          }
      }
#pragma unroll
      for (int v = 0; v < MT; v++) {
        if (v < vs.m) {
          const float4 *xv = reinterpret_cast<const float4 *>(a.x + (int64_t)vs.src[v] * a.ld_x + i * 32);
          float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
          for (int k = 0; k < 8; k++) {
            const float4 xx = xv[k];
            s0 = fmaf(q[4 * k + 0], xx.x, s0);
            s1 = fmaf(q[4 * k + 1], xx.y, s1);
            s2 = fmaf(q[4 * k + 2], xx.z, s2);
            s3 = fmaf(q[4 * k + 3], xx.w, s3);
          }
          acc[v] = fmaf(d, (s0 + s1) + (s2 + s3), acc[v]);
        }
      }
    }
  }
  // fixed quad tree: (a0 + a1) + (a2 + a3)
#pragma unroll
  for (int v = 0; v < MT; v++) {
    float t = acc[v] + quad_xor1f(acc[v]);
    acc[v] = t + quad_xor2f(t);
  }
  if (c == 0) {
#pragma unroll
    for (int v = 0; v < MT; v++)
      if (v < vs.m) a.out[(int64_t)vs.dst[v] * a.ld_out + r] = acc[v];
  }
}

// ---------------------------------------------------------------- launchers
static inline int mt_bucket(int m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : 16; }

static int kq_rr(int mt) { return mt <= 1 ? 1 : mt <= 4 ? 2 : 4; }

size_t kq_smem_bytes(const TensorView &w, int mt) {
  const int nb = (int)w.nb, R = (64 / nb) * kq_rr(mt);
  return (size_t)R * nb * (9 * mt * 4 + 8);
}

template <int T, int MT, bool G>
static hipError_t launch_kq_mt(KQArgs a, int grid_y, hipStream_t st) {
  constexpr int RR = MT <= 1 ? 1 : MT <= 4 ? 2 : 4;
  const int nb = (int)a.w.nb, R = (64 / nb) * RR;
  const int64_t rows = a.r1 - a.r0, groups = (rows + R - 1) / R;
  // enough passes per workgroup to amortise its set-up, while keeping >= ~2048 workgroups
  const int64_t per_y = std::max<int64_t>(1, 2048 / std::max(1, grid_y));
  a.passes = (int)std::max<int64_t>(1, std::min<int64_t>(16, groups / per_y));
  dim3 grid((unsigned)((groups + a.passes - 1) / a.passes), (unsigned)grid_y);
  const size_t sm = (size_t)R * nb * (9 * MT * 4 + 8);
  hipLaunchKernelGGL((k_gemv_kq<T, MT, RR, G>), grid, dim3(256), sm, st, a);
  return hipGetLastError();
}

template <int T, bool G>
static hipError_t launch_kq_t(const KQArgs &a, int mt, int grid_y, hipStream_t st) {
  switch (mt) {
  case 1: return launch_kq_mt<T, 1, G>(a, grid_y, st);
  case 2: return launch_kq_mt<T, 2, G>(a, grid_y, st);
  case 4: return launch_kq_mt<T, 4, G>(a, grid_y, st);
  case 8: return launch_kq_mt<T, 8, G>(a, grid_y, st);
  default: return launch_kq_mt<T, 16, G>(a, grid_y, st);
  }
}

hipError_t launch_gemv_kq(const KQArgs &a, int mt, bool grouped, int grid_y, hipStream_t st) {
  if (a.w.nb > 64) return hipErrorInvalidValue;
  mt = mt_bucket(mt);
  if (a.w.dtype == T_Q4K) return grouped ? launch_kq_t<T_Q4K, true>(a, mt, grid_y, st) : launch_kq_t<T_Q4K, false>(a, mt, 1, st);
  return grouped ? launch_kq_t<T_Q6K, true>(a, mt, grid_y, st) : launch_kq_t<T_Q6K, false>(a, mt, 1, st);
}

hipError_t launch_kq_block_sums(const KQArgs &a, hipStream_t st) {
  dim3 grid((unsigned)((a.w.nb + 15) / 16));
  if (a.w.dtype == T_Q4K) hipLaunchKernelGGL((k_kq_block_sums<T_Q4K>), grid, dim3(64), 0, st, a);
  else hipLaunchKernelGGL((k_kq_block_sums<T_Q6K>), grid, dim3(64), 0, st, a);
  return hipGetLastError();
}

// F32 weights (MoE routers): one wavefront per row, lane l takes float4 chunks l, l+64, ...;
// the lane partials are reduced with a fixed butterfly and lane 0's sum is written, so the
// order is the same for every batch size (matvec_multi runs F32 per vector, :455-464).
template <int MT, bool GROUPED>
__global__ __launch_bounds__(256) void k_gemv_f32(FArgs a) {
  VecSet<MT> vs;
  int expert;
  if (GROUPED) {
    if ((int)blockIdx.y >= *a.njobs) return;
    const Job &J = a.jobs[blockIdx.y];
    expert = J.expert;
    vs.m = J.nvec;
#pragma unroll
    for (int v = 0; v < MT; v++) { vs.src[v] = v < J.nvec ? J.vec[v] : 0; vs.dst[v] = v < J.nvec ? J.out[v] : 0; }
  } else {
    expert = a.expert;
    vs.m = a.m;
#pragma unroll
    for (int v = 0; v < MT; v++) { vs.src[v] = v; vs.dst[v] = v; }
  }
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t r = a.r0 + (int64_t)blockIdx.x * 4 + wv;
  if (r >= a.r1) return;
  const float4 *wr = reinterpret_cast<const float4 *>(a.w.pl.p0 + ((int64_t)expert * a.w.rows + r) * a.w.cols * 4);
  const int64_t n4 = a.w.cols / 4;
  float part[MT][4];
#pragma unroll
  for (int v = 0; v < MT; v++) part[v][0] = part[v][1] = part[v][2] = part[v][3] = 0.0f;
  for (int64_t k = lane; k < n4; k += 64) {
    const float4 w = wr[k];
#pragma unroll
    for (int v = 0; v < MT; v++) {
      if (v < vs.m) {
        const float4 xv = reinterpret_cast<const float4 *>(a.x + (int64_t)vs.src[v] * a.ld_x)[k];
        part[v][0] = fmaf(w.x, xv.x, part[v][0]);
        part[v][1] = fmaf(w.y, xv.y, part[v][1]);
        part[v][2] = fmaf(w.z, xv.z, part[v][2]);
        part[v][3] = fmaf(w.w, xv.w, part[v][3]);
      }
    }
  }
#pragma unroll
  for (int v = 0; v < MT; v++) {
    float t = (part[v][0] + part[v][1]) + (part[v][2] + part[v][3]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o);
    if (lane == 0 && v < vs.m) a.out[(int64_t)vs.dst[v] * a.ld_out + r] = t;
  }
}

template <bool G>
static hipError_t launch_f32(const FArgs &a, int mt, int grid_y, hipStream_t st) {
  dim3 grid((unsigned)((a.r1 - a.r0 + 3) / 4), (unsigned)grid_y);
  switch (mt) {
  case 1: hipLaunchKernelGGL((k_gemv_f32<1, G>), grid, dim3(256), 0, st, a); break;
  case 2: hipLaunchKernelGGL((k_gemv_f32<2, G>), grid, dim3(256), 0, st, a); break;
  case 4: hipLaunchKernelGGL((k_gemv_f32<4, G>), grid, dim3(256), 0, st, a); break;
  case 8: hipLaunchKernelGGL((k_gemv_f32<8, G>), grid, dim3(256), 0, st, a); break;
  default: hipLaunchKernelGGL((k_gemv_f32<16, G>), grid, dim3(256), 0, st, a); break;
  }
  return hipGetLastError();
}

template <int T, bool G>
static hipError_t launch_f_t(const FArgs &a, int mt, int grid_y, hipStream_t st) {
  const int64_t rows = a.r1 - a.r0;
  dim3 grid((unsigned)((rows + 63) / 64), (unsigned)grid_y);
  switch (mt) {
  case 1: hipLaunchKernelGGL((k_gemv_f<T, 1, G>), grid, dim3(256), 0, st, a); break;
  case 2: hipLaunchKernelGGL((k_gemv_f<T, 2, G>), grid, dim3(256), 0, st, a); break;
  case 4: hipLaunchKernelGGL((k_gemv_f<T, 4, G>), grid, dim3(256), 0, st, a); break;
  case 8: hipLaunchKernelGGL((k_gemv_f<T, 8, G>), grid, dim3(256), 0, st, a); break;
  default: hipLaunchKernelGGL((k_gemv_f<T, 16, G>), grid, dim3(256), 0, st, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_gemv_f(const FArgs &a, int mt, bool grouped, int grid_y, hipStream_t st) {
  mt = mt_bucket(mt);
  const int gy = grouped ? grid_y : 1;
  switch (a.w.dtype) {
  case T_Q8_0: return grouped ? launch_f_t<T_Q8_0, true>(a, mt, gy, st) : launch_f_t<T_Q8_0, false>(a, mt, gy, st);
  case T_Q5_0: return grouped ? launch_f_t<T_Q5_0, true>(a, mt, gy, st) : launch_f_t<T_Q5_0, false>(a, mt, gy, st);
  case T_F32: return grouped ? launch_f32<true>(a, mt, gy, st) : launch_f32<false>(a, mt, gy, st);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace spx
