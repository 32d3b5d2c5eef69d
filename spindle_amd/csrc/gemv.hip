// Quantized matrix x activation-vector kernels for gfx950 (wave64).
//
// Integer path (Q4_K, Q6_K x Q8_K), restating quant_q8k.rs:163-295 (rows<B,T>/matmul_rows):
//   per block i and vector v the kernel forms the exact int32 quantities of the reference,
//     S_i = sum_e scale(e) * w_e * y_e            (Q4_K: 6-bit scale per 32, codes 0..15;
//                                                  Q6_K: int8 scale per 16, codes 0..63)
//     s_i = Q4_K: sum_j min_j * (bsum_2j + bsum_2j+1);  Q6_K: 32 * sum_g scale_g * bsum_g
//   with v_dot4_i32_i8 (codes are non-negative, so the signed dot is exact), then
//     acc = fma(d*xd_i, float(S_i), acc)            (one chain over blocks, block order)
//     corr = corr + (dmin*xd_i) * float(s_i)        (Q6_K: (d*xd_i) * float(32 s); the
//                                                    reference's own expression, :204/:232)
//     out = acc - corr
//   S_i and s_i equal the reference's per-block integers bit for bit; the fp32 result
//   differs from the reference's eight-lane accumulation (:243-247) only in rounding. The
//   same per-vector code runs for every batch size, so a vector's result is bitwise
//   independent of the batch it is in (the property quant_q8k.rs:413-442 tests).
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
#include "common.h"

namespace spx {



template <int MT>
struct VecSet {
  int m;
  int src[MT];
  int dst[MT];
};

// ---------------------------------------------------------------- Q4_K block decode
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
  // y: this vector's 256 codes of the block; bs: its 16 bsums. Returns the lane partials.
  __device__ __forceinline__ void dot(const int8_t *y, const int16_t *bs, int c, int &p, int &s) const {
    const uint4 *yl = reinterpret_cast<const uint4 *>(y + c * 64);
    const uint4 a0 = yl[0], a1 = yl[1], b0 = yl[2], b1 = yl[3];
    const int ya[8] = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
    const int yb[8] = {(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
    int slo = 0, shi = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      slo = sdot4((int)lo[t], ya[t], slo);
      shi = sdot4((int)hi[t], yb[t], shi);
    }
    p = sc0 * slo + sc1 * shi;
    const int2 bb = *reinterpret_cast<const int2 *>(bs + 4 * c);
    const int b0s = (int)(int16_t)(bb.x & 0xffff), b1s = (int)(int16_t)(bb.x >> 16);
    const int b2s = (int)(int16_t)(bb.y & 0xffff), b3s = (int)(int16_t)(bb.y >> 16);
    s = mn0 * (b0s + b1s) + mn1 * (b2s + b3s);
  }
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
  __device__ __forceinline__ void dot(const int8_t *y, const int16_t *bs, int c, int &p, int &s) const {
    const int h = c >> 1, half = c & 1;
    p = 0;
    s = 0;
#pragma unroll
    for (int m = 0; m < 4; m++) {
      const uint4 yv = *reinterpret_cast<const uint4 *>(y + 128 * h + 32 * m + 16 * half);
      int t = sdot4((int)q[m][0], (int)yv.x, 0);
      t = sdot4((int)q[m][1], (int)yv.y, t);
      t = sdot4((int)q[m][2], (int)yv.z, t);
      t = sdot4((int)q[m][3], (int)yv.w, t);
      p += sc[m] * t;
      s += sc[m] * (int)bs[8 * h + 2 * m + half];
    }
  }
};

template <int T>
struct KQBlock;
template <> struct KQBlock<T_Q4K> { using type = Q4KBlock; };
template <> struct KQBlock<T_Q6K> { using type = Q6KBlock; };

// Accumulates one block's exact integers into the fp32 chain (quant_q8k.rs:204/:232/:243).
template <int T>
__device__ __forceinline__ void kq_accum(const typename KQBlock<T>::type &B, float xdv, int p, int s, float &acc, float &corr) {
  if (T == T_Q4K) {
    const Q4KBlock &b = reinterpret_cast<const Q4KBlock &>(B);
    acc = fmaf(b.d * xdv, (float)p, acc);
    corr = corr + (b.dmin * xdv) * (float)s;
  } else {
    const Q6KBlock &b = reinterpret_cast<const Q6KBlock &>(B);
    acc = fmaf(b.d * xdv, (float)p, acc);
    corr = corr + (b.d * xdv) * (float)(32 * s);
  }
}

template <int T, int MT, bool GROUPED>
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
  const int64_t cols = a.w.cols, nb = a.w.nb;
  // LDS holds the job's Q8_K vectors: codes, then scales, then bsums (16-byte aligned parts).
  const int64_t mcap = GROUPED ? MT : a.m;
  int8_t *sy = reinterpret_cast<int8_t *>(smem);
  float *sd = reinterpret_cast<float *>(smem + mcap * cols);
  int16_t *sb = reinterpret_cast<int16_t *>(smem + mcap * cols + ((mcap * nb * 4 + 15) & ~(int64_t)15));
  for (int v = 0; v < vs.m; v++) {
    const int64_t src = vs.src[v];
    const uint4 *s4 = reinterpret_cast<const uint4 *>(a.xq + src * cols);
    uint4 *d4 = reinterpret_cast<uint4 *>(sy + v * cols);
    for (int i = threadIdx.x; i < cols / 16; i += 256) d4[i] = s4[i];
    for (int i = threadIdx.x; i < nb; i += 256) sd[v * nb + i] = a.xd[src * nb + i];
    for (int i = threadIdx.x; i < nb * 16; i += 256) sb[v * nb * 16 + i] = a.xb[src * nb * 16 + i];
  }
  __syncthreads();
  const int quad = threadIdx.x >> 2, c = threadIdx.x & 3;
  const int64_t r = a.r0 + (int64_t)blockIdx.x * 64 + quad;
  if (r >= a.r1) return;
  const int64_t g0 = ((int64_t)expert * a.w.rows + r) * nb;
  float acc[MT], corr[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) { acc[v] = 0.0f; corr[v] = 0.0f; }
  typename KQBlock<T>::type B;
  for (int64_t i = 0; i < nb; i++) {
    B.load(a.w.pl, g0 + i, c);
#pragma unroll
    for (int v = 0; v < MT; v++) {
      if (v < vs.m) {
        int p, s;
        B.dot(sy + v * cols + i * 256, sb + (v * nb + i) * 16, c, p, s);
        p = quad_sum(p);
        s = quad_sum(s);
        kq_accum<T>(B, sd[v * nb + i], p, s, acc[v], corr[v]);
      }
    }
  }
  if (c == 0) {
#pragma unroll
    for (int v = 0; v < MT; v++)
      if (v < vs.m) a.out[(int64_t)vs.dst[v] * a.ld_out + r] = acc[v] - corr[v];
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
  int p, s;
  B.dot(a.xq + i * 256, a.xb + i * 16, c, p, s);
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

size_t kq_smem_bytes(const TensorView &w, int mt) {
  return (size_t)mt * w.cols + (((size_t)mt * w.nb * 4 + 15) & ~(size_t)15) + (size_t)mt * w.nb * 32;
}

template <int T, bool G>
static hipError_t launch_kq_t(const KQArgs &a, int mt, int grid_y, hipStream_t st) {
  const int64_t rows = a.r1 - a.r0;
  dim3 grid((unsigned)((rows + 63) / 64), (unsigned)grid_y);
  const size_t sm = kq_smem_bytes(a.w, G ? mt : a.m);
  switch (mt) {
  case 1: hipLaunchKernelGGL((k_gemv_kq<T, 1, G>), grid, dim3(256), sm, st, a); break;
  case 2: hipLaunchKernelGGL((k_gemv_kq<T, 2, G>), grid, dim3(256), sm, st, a); break;
  case 4: hipLaunchKernelGGL((k_gemv_kq<T, 4, G>), grid, dim3(256), sm, st, a); break;
  case 8: hipLaunchKernelGGL((k_gemv_kq<T, 8, G>), grid, dim3(256), sm, st, a); break;
  default: hipLaunchKernelGGL((k_gemv_kq<T, 16, G>), grid, dim3(256), sm, st, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_gemv_kq(const KQArgs &a, int mt, bool grouped, int grid_y, hipStream_t st) {
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
  case T_F32: return grouped ? launch_f_t<T_F32, true>(a, mt, gy, st) : launch_f_t<T_F32, false>(a, mt, gy, st);
  default: return hipErrorInvalidValue;
  }
}

}  // namespace spx
