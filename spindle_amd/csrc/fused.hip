// Fused decode / verify kernels for gfx950 (wave64). One forward pass of m <= 16 token rows
// is, per layer:
//   q/k/v projections     one launch over the three tensors (segments)
//   attention             q/k norm, RoPE, K/V cache write, split-K attention, last-workgroup
//                         merge (+ Q8_K of the output)
//   attn_output           + the residual add, ffn_norm and Q8_K of the next input, computed
//                         once by the launch's last workgroup ("norm tail")
//   router + routing      F32 router rows, then the last workgroup routes and builds the
//                         grouped job lists (MoE layers)
//   gate/up + SwiGLU      grouped over the selected experts (+ Q8_K of h by the last
//                         workgroup covering each 256-row block)
//   down + combine        grouped, weighted sum in chosen order, + the residual add and the
//                         next layer's attn_norm (or output_norm) as a norm tail
// Decode (m <= 2) runs the integer projections row-parallel: the 8-lane groups of a
// wavefront each take one block of a row, and the reference's per-lane fp32 chain then runs
// over the per-block results in LDS, in block order. Larger passes run eight rows per
// wavefront, each lane walking its row's blocks in order; both give the same bits.
// Positions and row counts come from the device-side step record, so a captured HIP graph
// replays at any position. References are to smollm_chat.rs unless a file is named.
#include <float.h>

#include <type_traits>
#include "fused.h"
#include "decode.h"
#include "dev.h"
#include "attn.h"
#include "decode_dev.h"

namespace spx {

// ------------------------------------------------------------------ norm tail
// Rows [b0, b1) of a NormTail by all NW wavefronts of the workgroup. Wave w takes the
// 256-value blocks w, w+NW, ...; lane j holds values 4j..4j+3 of a block.
template <int NW>
__device__ __forceinline__ void norm_rows(const NormTail &t, int b0, int b1) {
  __shared__ float bsum[NORM_NT];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int dim = t.dim, n4 = dim >> 2, nblk = (n4 + 63) >> 6, nbq = dim >> 8;
  const rsrc_t ra = rsrc_of(t.add ? t.add : t.x);
  const float4 *x4 = reinterpret_cast<const float4 *>(t.x);
  const float4 *w4 = reinterpret_cast<const float4 *>(t.nw);
  float4 wn[NORM_NT / NW];  // the norm weights, loaded once with the first row's inputs
#pragma unroll
  for (int k = 0; k < NORM_NT / NW; k++) {
    const int f = (wave + NW * k) * 64 + lane;
    wn[k] = f < n4 ? w4[f] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int b = b0; b < b1; b++) {
    float4 r[NORM_NT / NW];
#pragma unroll
    for (int k = 0; k < NORM_NT / NW; k++) {
      const int tb = wave + NW * k, f = tb * 64 + lane;
      r[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (tb < nblk) {
        if (f < n4) {
          float4 v = x4[(int64_t)b * n4 + f];
          if (t.add) {
            const f4v a = ld_coh4(ra, (b * n4 + f) * 16);
            v.x = v.x + t.rscale * a.x; v.y = v.y + t.rscale * a.y; v.z = v.z + t.rscale * a.z; v.w = v.w + t.rscale * a.w;
          }
          r[k] = v;
        }
        float p = r[k].x * r[k].x;
        p = fmaf(r[k].y, r[k].y, p);
        p = fmaf(r[k].z, r[k].z, p);
        p = fmaf(r[k].w, r[k].w, p);
        p = wave_sum(p);
        if (lane == 0) bsum[tb] = p;
      }
    }
    __syncthreads();
    float S = 0.0f;
    for (int k = 0; k < nblk; k++) S = S + bsum[k];
    const float inv = inv_rms(S, (float)dim, t.eps);
#pragma unroll
    for (int k = 0; k < NORM_NT / NW; k++) {
      const int tb = wave + NW * k, f = tb * 64 + lane;
      if (tb < nblk) {
        float4 v = r[k];
        if (f < n4) {
          if (t.x_out) reinterpret_cast<float4 *>(t.x_out)[(int64_t)b * n4 + f] = v;
          const float4 w = wn[k];
          v.x = v.x * inv * w.x; v.y = v.y * inv * w.y; v.z = v.z * inv * w.z; v.w = v.w * inv * w.w;
          if (t.xn_out) reinterpret_cast<float4 *>(t.xn_out)[(int64_t)b * n4 + f] = v;
        }
        if (t.q_out.q) {
          const float am = q8k_amax(v);
          const int64_t vb = (int64_t)b * nbq + tb;
          q8k_block_store(v, am, t.q_out.q + vb * 64, t.q_out.d + vb, reinterpret_cast<int *>(t.q_out.bs + vb * 8));
        }
      }
    }
    __syncthreads();
  }
}

// The same RMSNorm of one row (t.x, no residual add) computed by a consumer's workgroup for
// itself: the row and its weights loaded (load), then norm_rows's per-block fma chains and
// wavefront trees, the blocks in order, x * inv * w (finish) into LDS lx (and memory, xn_out).
// The bits are norm_rows's: a producer's residual epilogue plus this prologue replace its tail.
template <int NW>
struct NormRow {
  float4 r[NORM_NT / NW], w[NORM_NT / NW];
  __device__ __forceinline__ void load(const NormTail &t) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, n4 = t.dim >> 2, nblk = (n4 + 63) >> 6;
#pragma unroll
    for (int k = 0; k < NORM_NT / NW; k++) {
      const int tb = wave + NW * k, f = tb * 64 + lane;
      r[k] = w[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (tb < nblk && f < n4) {
        r[k] = reinterpret_cast<const float4 *>(t.x)[f];
        w[k] = reinterpret_cast<const float4 *>(t.nw)[f];
      }
    }
  }
  __device__ __forceinline__ void finish(const NormTail &t, float *lx, float *xn_out) {
    __shared__ float bsum[NORM_NT];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, n4 = t.dim >> 2, nblk = (n4 + 63) >> 6;
#pragma unroll
    for (int k = 0; k < NORM_NT / NW; k++) {
      const int tb = wave + NW * k;
      if (tb < nblk) {
        float p = r[k].x * r[k].x;
        p = fmaf(r[k].y, r[k].y, p);
        p = fmaf(r[k].z, r[k].z, p);
        p = fmaf(r[k].w, r[k].w, p);
        p = wave_sum(p);
        if (lane == 0) bsum[tb] = p;
      }
    }
    __syncthreads();
    float S = 0.0f;
    for (int k = 0; k < nblk; k++) S = S + bsum[k];
    const float inv = inv_rms(S, (float)t.dim, t.eps);
#pragma unroll
    for (int k = 0; k < NORM_NT / NW; k++) {
      const int tb = wave + NW * k, f = tb * 64 + lane;
      if (tb < nblk && f < n4) {
        float4 v = r[k];
        const float4 ww = w[k];
        v.x = v.x * inv * ww.x; v.y = v.y * inv * ww.y; v.z = v.z * inv * ww.z; v.w = v.w * inv * ww.w;
        reinterpret_cast<float4 *>(lx)[f] = v;
        if (xn_out) reinterpret_cast<float4 *>(xn_out)[f] = v;
      }
    }
    __syncthreads();
  }
};

// ------------------------------------------------------------------ activations in LDS
__host__ __device__ inline size_t ldsq_dbytes(int mt, int dim) { return ((size_t)mt * (dim / 256) * 4 + 15) & ~(size_t)15; }
__host__ __device__ inline size_t ldsq_bytes(int mt, int dim) {
  return ((size_t)mt * dim + ldsq_dbytes(mt, dim) + (size_t)mt * (dim / 256) * 64 + 15) & ~(size_t)15;
}
// LDS image of mt permuted Q8_K vectors of dim columns: q [mt][dim/4], d [mt][nb], bs [mt][nb][8].
__device__ __forceinline__ Q8KP ldsq_of(uint8_t *smem, int mt, int dim) {
  Q8KP r;
  r.q = reinterpret_cast<uint32_t *>(smem);
  r.d = reinterpret_cast<float *>(smem + (size_t)mt * dim);
  r.bs = reinterpret_cast<int2 *>(smem + (size_t)mt * dim + ldsq_dbytes(mt, dim));
  return r;
}

typedef __attribute__((address_space(3))) void *lds_ptr;

// Copies permuted Q8_K vectors vsrc(u), u < nv, of `cols` columns from global y into the LDS
// image ly (vector u at slot u) with direct global->LDS loads (lane i's piece lands at
// M0 + size * i) spread over the workgroup's nw waves. Each region (codes, d, bsums) is
// contiguous in LDS across vectors, so a wave's destinations are consecutive.
template <class F>
__device__ __forceinline__ void stage_q8kp(const Q8KP &ly, const Q8KP &y, int cols, int nv, int nw, F vsrc) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nb = cols >> 8;
  const int pq = cols / 16, pb = nb * 4;  // 16-byte pieces per vector: codes, bsums (nb * 64 bytes)
  for (int p0 = wave * 64; p0 < nv * pq; p0 += nw * 64) {
    const int p = p0 + lane, u = p / pq, w = p - u * pq;
    if (p < nv * pq)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t *>(y.q) + (int64_t)vsrc(u) * cols + 16 * w,
                                       (lds_ptr)(reinterpret_cast<uint8_t *>(ly.q) + 16 * p0), 16, 0, 0);
  }
  for (int p0 = wave * 64; p0 < nv * pb; p0 += nw * 64) {
    const int p = p0 + lane, u = p / pb, w = p - u * pb;
    if (p < nv * pb)
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t *>(y.bs + (int64_t)vsrc(u) * nb * 8) + 16 * w,
                                       (lds_ptr)(reinterpret_cast<uint8_t *>(ly.bs) + 16 * p0), 16, 0, 0);
  }
  for (int p0 = wave * 64; p0 < nv * nb; p0 += nw * 64) {
    const int p = p0 + lane, u = p / nb, w = p - u * nb;
    if (p < nv * nb)
      __builtin_amdgcn_global_load_lds(y.d + (int64_t)vsrc(u) * nb + w, (lds_ptr)(reinterpret_cast<uint8_t *>(ly.d) + 4 * p0), 4, 0, 0);
  }
}

// ------------------------------------------------------------------ integer tiles in LDS
// A wavefront's slots (rows) x nb blocks of a K-quant tensor are copied into LDS with direct
// loads, then the blocks are read from LDS. Tile layout, plane by plane, slot-major:
//   Q4_K: codes [ns][nb][128], headers [ns][nb][16]
//   Q6_K: ql [ns][nb][128], qh [ns][nb][64], scales [ns][nb][16], d [ns][nb] as the dword
//         that holds the 2-byte d (the dword at the record's address rounded down to 4)
template <int T> struct KQPlanes;
template <> struct KQPlanes<T_Q4K> {
  static constexpr int NP = 2;
  __host__ __device__ static constexpr int rec(int k) { return k == 0 ? 128 : 16; }
  __host__ __device__ static constexpr int lrec(int k) { return rec(k); }
};
template <> struct KQPlanes<T_Q6K> {
  static constexpr int NP = 4;
  __host__ __device__ static constexpr int rec(int k) { return k == 0 ? 128 : k == 1 ? 64 : k == 2 ? 16 : 2; }
  __host__ __device__ static constexpr int lrec(int k) { return k == 3 ? 4 : rec(k); }
};
__host__ __device__ constexpr int tile_bpb() { return 128 + 64 + 16 + 4; }  // LDS bytes per block, the larger of Q4_K and Q6_K

// src(s) = global row index (expert * rows + row) of slot s < ns, or -1 for an empty slot.
template <int T, class F>
__device__ __forceinline__ void tile_fetch(uint8_t *tile, const Planes &pl, int ns, int nb, F src) {
  const int lane = threadIdx.x & 63;
  const uint8_t *planes[4] = {pl.p0, pl.p1, pl.p2, pl.p3};
  int off = 0;
#pragma unroll
  for (int k = 0; k < KQPlanes<T>::NP; k++) {
    const int R = KQPlanes<T>::rec(k);
    if (R >= 16) {
      const int per = nb * R / 16, total = ns * per;
      for (int p0 = 0; p0 < total; p0 += 64) {
        const int p = p0 + lane, sl = p / per, w = p - sl * per;
        const int64_t grow = p < total ? src(sl) : -1;
        if (grow >= 0) __builtin_amdgcn_global_load_lds(planes[k] + grow * nb * R + 16 * w, (lds_ptr)(tile + off + 16 * p0), 16, 0, 0);
      }
    } else {  // 2-byte records: the dword holding each
      const int total = ns * nb;
      for (int p0 = 0; p0 < total; p0 += 64) {
        const int p = p0 + lane, sl = p / nb, w = p - sl * nb;
        const int64_t grow = p < total ? src(sl) : -1;
        if (grow >= 0) {
          const uintptr_t a = reinterpret_cast<uintptr_t>(planes[k] + (grow * nb + w) * 2) & ~(uintptr_t)3;
          __builtin_amdgcn_global_load_lds(reinterpret_cast<const void *>(a), (lds_ptr)(tile + off + 4 * p0), 4, 0, 0);
        }
      }
    }
    off += ns * nb * KQPlanes<T>::lrec(k);
  }
}

// Block i of slot s as lane l needs it. odd = the block's global index is odd (Q6_K d half).
__device__ __forceinline__ void tile_block(const uint8_t *tile, int ns, int nb, int s, int i, int l, bool odd, KQRaw<T_Q4K> &r) {
  const int rec = s * nb + i;
  r.c = *reinterpret_cast<const uint4 *>(tile + rec * 128 + 16 * l);
  r.h = *reinterpret_cast<const uint4 *>(tile + ns * nb * 128 + rec * 16);
}
__device__ __forceinline__ void tile_block(const uint8_t *tile, int ns, int nb, int s, int i, int l, bool odd, KQRaw<T_Q6K> &r) {
  const int rec = s * nb + i;
  r.ql = *reinterpret_cast<const uint4 *>(tile + rec * 128 + 16 * l);
  r.qh = *reinterpret_cast<const uint2 *>(tile + ns * nb * 128 + rec * 64 + 8 * l);
  r.sc = *reinterpret_cast<const uint4 *>(tile + ns * nb * 192 + rec * 16);
  r.d = (*reinterpret_cast<const uint32_t *>(tile + ns * nb * 208 + rec * 4) >> (odd ? 16 : 0)) & 0xffffu;
}

// One block of one row against one vector (lane l's part): P = the lane's scaled dot,
// s = the correction integer summed over the row group's 8 lanes.
template <int T>
__device__ __forceinline__ void kq_block_dot(const KQDec<T> &dec, const Q8KP &y, int64_t vb, int l, int &P, int &s) {
  const uint4 *yq = reinterpret_cast<const uint4 *>(y.q + vb * 64 + 8 * l);
  dec.dot(yq[0], yq[1], y.bs[vb * 8 + l], P, s);
  s = sum8(s);
}

// Eight-rows-per-wavefront walker: slot s's row (global row index grow) against vectors
// vidx[0..mv) of y, blocks in order, the reference's per-lane chain kept in registers.
template <int T, int MT>
__device__ __forceinline__ void kq_walk_tile(const uint8_t *tile, int ns, int nb, int s, int64_t grow, const Q8KP &y, const int *vidx, int mv,
                                             int l, float *res) {
  float acc[MT], corr[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) { acc[v] = 0.0f; corr[v] = 0.0f; }
  const bool odd0 = ((grow * nb) & 1) != 0;
  for (int i = 0; i < nb; i++) {
    KQRaw<T> r;
    tile_block(tile, ns, nb, s, i, l, odd0 ^ ((i & 1) != 0), r);
    KQDec<T> dec;
    dec.decode(r, l);
#pragma unroll
    for (int v = 0; v < MT; v++) {
      if (v < mv) {
        const int64_t vb = (int64_t)vidx[v] * nb + i;
        int P, sc;
        kq_block_dot<T>(dec, y, vb, l, P, sc);
        const float xd = y.d[vb];
        corr[v] = corr[v] + dec.corr_term(xd, sc);
        acc[v] = fmaf(dec.d * xd, (float)P, acc[v]);
      }
    }
  }
#pragma unroll
  for (int v = 0; v < MT; v++) res[v] = hsum_rows8(acc[v]) - corr[v];
}

// Row-parallel walker: the wavefront's R slots (rows) x G lane groups (G a power of two);
// group gi of row r computes blocks gi, gi+G, ... and leaves, per block and vector, d*xd, the
// 8 lane dots as floats and the correction term in the chain buffer cb (LDS); then, for
// vector v, group v % G of each row runs the reference's chain acc_l = fma(d*xd_i, float(P_il),
// acc_l), corr = corr + term_i over the blocks in order and its lane 0 writes the row's result
// to ov[r * MT + v] (LDS). The caller reads ov after the call.
// cb: [R][nb][MT] x {8 lane dots, d*xd, term} floats.
template <int T, int MT, class GROW, class VID, class MV>
__device__ __forceinline__ void kq_rows_par(const uint8_t *tile, int ns, int nb, int G, int R, GROW grow_of, VID vid, MV mv_of, const Q8KP &y,
                                            float *cb, float *ov) {
  const int lane = threadIdx.x & 63, l = lane & 7, grp = lane >> 3;
  const int r = grp / G, gi = grp - r * G;
  if (r < R) {
    const int64_t grow = grow_of(r);
    const int mv = mv_of(r);
    const bool odd0 = ((grow * nb) & 1) != 0;
    for (int i = gi; i < nb; i += G) {
      KQRaw<T> raw;
      tile_block(tile, ns, nb, r, i, l, odd0 ^ ((i & 1) != 0), raw);
      KQDec<T> dec;
      dec.decode(raw, l);
#pragma unroll 4
      for (int v = 0; v < MT; v++) {
        if (v < mv) {
          const int64_t vb = (int64_t)vid(r, v) * nb + i;
          int P, sc;
          kq_block_dot<T>(dec, y, vb, l, P, sc);
          const float xd = y.d[vb];
          float *e = cb + (((int64_t)r * nb + i) * MT + v) * 10;
          e[l] = (float)P;
          if (l == 0) { e[8] = dec.d * xd; e[9] = dec.corr_term(xd, sc); }
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  if (r < R) {
    const int mvc = mv_of(r);
#pragma unroll
    for (int v = 0; v < MT; v++) {
      if ((v & (G - 1)) == gi && v < mvc) {
        float acc = 0.0f, cr = 0.0f;
#pragma unroll 8
        for (int i = 0; i < nb; i++) {
          const float *e = cb + (((int64_t)r * nb + i) * MT + v) * 10;
          acc = fmaf(e[8], e[l], acc);
          cr = cr + e[9];
        }
        const float res = hsum_rows8(acc) - cr;
        if (l == 0) ov[r * MT + v] = res;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
}

// ------------------------------------------------------------------ float row walker
// Q8_0 / Q5_0 weights x fp32 activations (quant.rs:48-161, quant_multi.rs:168-190): lane l
// of the row group takes blocks l, l+8, ...; per block s = sum q*x in four fixed chains,
// acc = fma(d, s, acc); the row is the 8-lane tree. The order is this kernel's own (fixed
// for every batch size), within 1e-4 of the reference's.
template <int T> struct FRaw;
template <> struct FRaw<T_Q8_0> {
  uint4 c0, c1;
  uint32_t d;
  __device__ __forceinline__ void load(const Planes &pl, int64_t g) {
    c0 = ld16(pl.p0 + g * 32);
    c1 = ld16(pl.p0 + g * 32 + 16);
    d = *reinterpret_cast<const uint16_t *>(pl.p3 + g * 2);
  }
  __device__ __forceinline__ void decode(float q[32]) const {
    const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
    for (int k = 0; k < 8; k++)
#pragma unroll
      for (int j = 0; j < 4; j++) q[4 * k + j] = (float)(int8_t)(cw[k] >> (8 * j));
  }
};
template <> struct FRaw<T_Q5_0> {
  uint4 c;
  uint32_t qh, d;
  __device__ __forceinline__ void load(const Planes &pl, int64_t g) {
    c = ld16(pl.p0 + g * 16);
    qh = *reinterpret_cast<const uint32_t *>(pl.p1 + g * 4);
    d = *reinterpret_cast<const uint16_t *>(pl.p3 + g * 2);
  }
  __device__ __forceinline__ void decode(float q[32]) const {  // j<16: low nibble | bit j; j>=16: high nibble | bit j
    const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int e = 4 * k + j;
        const uint32_t byte = (cw[k] >> (8 * j)) & 0xffu;
        q[e] = (float)((int)((byte & 0xFu) | (((qh >> e) & 1u) << 4)) - 16);
        q[e + 16] = (float)((int)((byte >> 4) | (((qh >> (e + 16)) & 1u) << 4)) - 16);
      }
  }
};

// Q5_K weights x fp32 activations: the reference's float kernel (dot_q5_k_row_avx2_presum,
// quant.rs:1266-1313) lane for lane, lane l of the row group being its lane l: per 32-value
// sub-block j = 2c + h the lane's chain sqx = fma over elements l, 8+l, 16+l, 24+l, then
// acc = fma(d * sc_j, sqx, acc); per block the activation sums of the eight sub-blocks
// (compute_subblock_sums_32 :167-178, the hadd tree over the lanes) give
// total_min += (sum_k mn_k * act_k) * dmin; the row is hadd(acc) - total_min (lane 0).
// Device layout: lane l's code bytes (qs[32c + 8k + l]) at 16l + 4c + k, its high-bit bytes
// (qh[8k + l]) at 4l + k.
__device__ __forceinline__ float hsum_hadd8(float a) {  // valid in lane 0 of the row group
  const float x = a + SPX_SHLF(a, 4);  // x_l = a_l + a_{l+4}
  const float t = x + SPX_SHLF(x, 1);  // lane 0: x0 + x1, lane 2: x2 + x3
  return t + SPX_SHLF(t, 2);           // (x0 + x1) + (x2 + x3)
}
template <int MT>
__device__ __forceinline__ void q5k_walk(const Planes &pl, int64_t grow, int nb, const float *x, int64_t ld_x, const int *vidx, int mv, int l,
                                         float *res) {
  float acc[MT], tmin[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) { acc[v] = 0.0f; tmin[v] = 0.0f; }
  for (int i = 0; i < nb; i++) {
    const int64_t g = grow * nb + i;
    const uint4 qs = ld16(pl.p0 + g * 128 + 16 * l);
    const uint32_t qh = *reinterpret_cast<const uint32_t *>(pl.p1 + g * 32 + 4 * l);
    const uint4 hd = ld16(pl.p2 + g * 16);
    const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
    const uint32_t S0 = hd.y, S1 = hd.z, S2 = hd.w;  // unpack_q4k_scales (q4k_gemv.rs:70-85)
    int sc[8], mn[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      sc[k] = (int)((S0 >> (8 * k)) & 63u);
      mn[k] = (int)((S1 >> (8 * k)) & 63u);
      sc[4 + k] = (int)(((S2 >> (8 * k)) & 15u) | (((S0 >> (8 * k + 6)) & 3u) << 4));
      mn[4 + k] = (int)(((S2 >> (8 * k + 4)) & 15u) | (((S1 >> (8 * k + 6)) & 3u) << 4));
    }
    const uint32_t cw[4] = {qs.x, qs.y, qs.z, qs.w};  // word c: byte k = qs[32c + 8k + l]
#pragma unroll
    for (int v = 0; v < MT; v++) {
      if (v < mv) {
        const float *xb = x + (int64_t)vidx[v] * ld_x + (int64_t)i * 256 + l;
        float xv[32];  // xv[8j + k] = value 32j + 8k + l of the block
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
          for (int k = 0; k < 4; k++) xv[4 * j + k] = xb[32 * j + 8 * k];
        float min_term = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const float p = (xv[4 * j] + xv[4 * j + 1]) + (xv[4 * j + 2] + xv[4 * j + 3]);
          min_term += (float)mn[j] * hsum_hadd8(p);
        }
        tmin[v] += min_term * dmin;
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
          for (int h = 0; h < 2; h++) {
            const int j = 2 * c + h;
            float sq = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
              const uint32_t byte = (cw[c] >> (8 * k)) & 0xffu, nib = h ? byte >> 4 : byte & 15u;
              const uint32_t q = nib | (((qh >> (8 * k + j)) & 1u) << 4);
              sq = fmaf((float)q, xv[4 * j + k], sq);
            }
            acc[v] = fmaf(d * (float)sc[j], sq, acc[v]);
          }
      }
    }
  }
#pragma unroll
  for (int v = 0; v < MT; v++) res[v] = hsum_hadd8(acc[v]) - tmin[v];
}

template <> struct FRaw<T_Q5K> {  // not used: Q5_K rows take q5k_walk
  uint32_t d;
  __device__ __forceinline__ void load(const Planes &, int64_t) {}
  __device__ __forceinline__ void decode(float q[32]) const {}
};

struct NoPre {
  __device__ __forceinline__ void operator()() const {}
};
// pre() runs once the first blocks' loads are issued, before x is read (every thread of the
// workgroup reaches it: it may synchronise the workgroup).
template <int T, int MT, int D, class Pre = NoPre>
__device__ __forceinline__ void f_walk(const Planes &pl, int64_t grow, int nb, const float *x, int64_t ld_x, const int *vidx, int mv, int l,
                                       float *res, Pre pre = Pre{}) {
  if constexpr (T == T_Q5K) {
    pre();
    q5k_walk<MT>(pl, grow, nb, x, ld_x, vidx, mv, l, res);
    return;
  }
  float acc[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) acc[v] = 0.0f;
  const int64_t g0 = grow * nb;
  const int nmine = nb > l ? (nb - l + 7) >> 3 : 0;
  FRaw<T> buf[D];
#pragma unroll
  for (int j = 0; j < D; j++)
    if (j < nmine) buf[j].load(pl, g0 + l + 8 * j);
  pre();
  for (int k0 = 0; k0 < nmine; k0 += D) {
#pragma unroll
    for (int j = 0; j < D; j++) {
      const int k = k0 + j;
      if (k < nmine) {
        const int i = l + 8 * k;
        float q[32];
        buf[j].decode(q);
        const float d = h2f(buf[j].d);
        if (k + D < nmine) buf[j].load(pl, g0 + l + 8 * (k + D));
#pragma unroll
        for (int v = 0; v < MT; v++) {
          if (v < mv) {
            const float4 *xv = reinterpret_cast<const float4 *>(x + (int64_t)vidx[v] * ld_x + (int64_t)i * 32);
            float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
              const float4 xx = xv[kk];
              s0 = fmaf(q[4 * kk + 0], xx.x, s0);
              s1 = fmaf(q[4 * kk + 1], xx.y, s1);
              s2 = fmaf(q[4 * kk + 2], xx.z, s2);
              s3 = fmaf(q[4 * kk + 3], xx.w, s3);
            }
            acc[v] = fmaf(d, (s0 + s1) + (s2 + s3), acc[v]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int v = 0; v < MT; v++) res[v] = hsum_rows8(acc[v]);
}

// F32 weights (quant.rs:1409-1502 semantics): lane l of the row group takes float4 chunks
// l, l+8, ... in one fma chain per vector; the row is the 8-lane tree.
template <int MT>
__device__ __forceinline__ void f32_walk(const Planes &pl, int64_t grow, int64_t cols, const float *x, int64_t ld_x, const int *vidx, int mv,
                                         int l, float *res) {
  float acc[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) acc[v] = 0.0f;
  const float4 *wr = reinterpret_cast<const float4 *>(pl.p0 + grow * cols * 4);
  const int64_t n4 = cols / 4;
  for (int64_t k = l; k < n4; k += 8) {
    const float4 w = wr[k];
#pragma unroll
    for (int v = 0; v < MT; v++) {
      if (v < mv) {
        const float4 xx = reinterpret_cast<const float4 *>(x + (int64_t)vidx[v] * ld_x)[k];
        acc[v] = fmaf(w.x, xx.x, acc[v]);
        acc[v] = fmaf(w.y, xx.y, acc[v]);
        acc[v] = fmaf(w.z, xx.z, acc[v]);
        acc[v] = fmaf(w.w, xx.w, acc[v]);
      }
    }
  }
#pragma unroll
  for (int v = 0; v < MT; v++) res[v] = hsum_rows8(acc[v]);
}

template <int MT>
constexpr int f_depth() { return MT <= 2 ? 4 : 2; }

template <int MT, int NW>
__device__ __forceinline__ void best_flush(const MVArgs &a, unsigned long long (&bestv)[MT], int m) {
  __shared__ unsigned long long sb[NW][MT];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int v = 0; v < MT; v++) {
    const unsigned long long w = wave_max_u64(bestv[v]);
    if (lane == 0) sb[wave][v] = w;
  }
  __syncthreads();
  if (threadIdx.x < MT && (int)threadIdx.x < m) {
    unsigned long long b = 0;
    for (int w = 0; w < NW; w++) b = sb[w][threadIdx.x] > b ? sb[w][threadIdx.x] : b;
    a.best[(int64_t)threadIdx.x * a.nbest + blockIdx.x] = b;
  }
}

// A launch output a norm tail will read is stored coherently.
__device__ __forceinline__ void out_store(float *p, float v, bool coh) {
  if (coh) st_dev(p, v);
  else *p = v;
}

// Segment of workgroup task t and the task's index within it. The index is computed with
// selects and made wave-uniform, so the segment's fields are read from the kernel arguments
// directly (no branchy selection between argument sub-objects).
__device__ __forceinline__ int seg_index(const MVArgs &a, int t, int &wg) {
  const int w0 = a.seg[0].wgs, w1 = a.nseg > 1 ? a.seg[1].wgs : 0;
  const int i = a.nseg > 1 && t >= w0 ? (a.nseg > 2 && t >= w0 + w1 ? 2 : 1) : 0;
  wg = t - (i > 0 ? w0 : 0) - (i > 1 ? w1 : 0);
  return __builtin_amdgcn_readfirstlane(i);
}

// ------------------------------------------------------------------ integer matvec, 8 rows per wavefront
// One wavefront per workgroup, eight rows per task; tasks stride over the grid (the LM head
// runs on a few thousand workgroups). LDS: the activations (staged once), then the tile. No
// norm tail (a pass that needs one runs the row-parallel kernel or a standalone norm).
template <int MT>
__global__ __launch_bounds__(64) void k_mvt(const MVArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int m = st ? st->m : a.m;
  const int lane = threadIdx.x, slot = lane >> 3, l = lane & 7;
  const int cols = (int)a.seg[0].w.cols, nb = cols >> 8;
  constexpr bool ST = MT <= 2;  // activations staged in LDS (small m); else read through the caches
  const Q8KP ly = ST ? ldsq_of(smem, MT, cols) : a.y;
  uint8_t *tile = smem + (ST ? ldsq_bytes(MT, cols) : 0);
  unsigned long long bestv[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) bestv[v] = 0;
  const int total = a.seg[0].wgs + (a.nseg > 1 ? a.seg[1].wgs : 0) + (a.nseg > 2 ? a.seg[2].wgs : 0);
  bool first = true;
  for (int t = blockIdx.x; t < total; t += gridDim.x) {
    int wg;
    const Seg &sg = a.seg[seg_index(a, t, wg)];
    const int64_t ebase = (int64_t)sg.expert * sg.w.rows, rbase = sg.r0 + (int64_t)wg * 8, r1 = sg.r1;
    const bool q4 = sg.w.dtype == T_Q4K;
    auto src = [&](int s) -> int64_t { return rbase + s < r1 ? ebase + rbase + s : -1; };
    if (q4) tile_fetch<T_Q4K>(tile, sg.w.pl, 8, nb, src); else tile_fetch<T_Q6K>(tile, sg.w.pl, 8, nb, src);
    if (ST && first) stage_q8kp(ly, a.y, cols, m, 1, [](int u) { return u; });
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int64_t row = rbase + slot;
    const bool valid = row < r1;
    int vidx[MT];
#pragma unroll
    for (int v = 0; v < MT; v++) vidx[v] = v;
    float res[MT];
    const int64_t grow = ebase + (valid ? row : r1 - 1);
    if (q4) kq_walk_tile<T_Q4K, MT>(tile, 8, nb, slot, grow, ly, vidx, m, l, res);
    else kq_walk_tile<T_Q6K, MT>(tile, 8, nb, slot, grow, ly, vidx, m, l, res);
    if (valid && l == 0) {
#pragma unroll
      for (int v = 0; v < MT; v++)
        if (v < m) {
          sg.out[(int64_t)v * sg.ld_out + row] = res[v];
          if (a.best) { const unsigned long long k = pick_key(res[v], a.lscale, row); bestv[v] = k > bestv[v] ? k : bestv[v]; }
        }
    }
    __syncthreads();  // the tile may be refilled by the next task
    first = false;
  }
  if (a.best) best_flush<MT, 1>(a, bestv, m);
}

// ------------------------------------------------------------------ integer matvec, row-parallel
// Four wavefronts per workgroup, R rows per wavefront, G lane groups per row. m <= 2: the
// activations are staged in LDS; larger m reads them through the caches.
__host__ __device__ inline size_t rp_wave_bytes(int R, int nb, int mt) {
  return ((size_t)R * nb * tile_bpb() + (size_t)R * nb * mt * 10 * 4 + (size_t)R * mt * 4 + 15) & ~(size_t)15;
}
__host__ __device__ inline size_t rp_act_bytes(int mt, int cols) { return mt <= 2 ? ldsq_bytes(mt, cols) : 0; }

template <int MT>
__global__ __launch_bounds__(256) void k_mvr(const MVArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr bool ST = MT <= 2;
  const int m = st ? st->m : a.m;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int cols = (int)a.seg[0].w.cols, nb = cols >> 8, G = a.G, R = a.R;
  const Q8KP ly = ST ? ldsq_of(smem, MT, cols) : a.y;
  uint8_t *tile = smem + rp_act_bytes(MT, cols) + (size_t)wave * rp_wave_bytes(R, nb, MT);
  float *cb = reinterpret_cast<float *>(tile + (size_t)R * nb * tile_bpb());
  float *ov = cb + (size_t)R * nb * MT * 10;
  const bool coh = a.tail.nw != nullptr;
  int wg;
  const Seg &sg = a.seg[seg_index(a, blockIdx.x, wg)];
  const int64_t ebase = (int64_t)sg.expert * sg.w.rows, rbase = sg.r0 + ((int64_t)wg * 4 + wave) * R, r1 = sg.r1;
  const bool q4 = sg.w.dtype == T_Q4K;
  auto src = [&](int s) -> int64_t { return s < R && rbase + s < r1 ? ebase + rbase + s : -1; };
  if (q4) tile_fetch<T_Q4K>(tile, sg.w.pl, R, nb, src); else tile_fetch<T_Q6K>(tile, sg.w.pl, R, nb, src);
  if (ST) stage_q8kp(ly, a.y, cols, m, 4, [](int u) { return u; });
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  auto grow = [&](int r) -> int64_t { return ebase + (rbase + r < r1 ? rbase + r : r1 - 1); };
  auto vid = [](int r, int v) { return v; };
  auto mvf = [&](int r) { return m; };
  if (q4) kq_rows_par<T_Q4K, MT>(tile, R, nb, G, R, grow, vid, mvf, ly, cb, ov);
  else kq_rows_par<T_Q6K, MT>(tile, R, nb, G, R, grow, vid, mvf, ly, cb, ov);
  for (int idx = lane; idx < R * MT; idx += 64) {
    const int r = idx / MT, v = idx - r * MT;
    if (v < m && rbase + r < r1) out_store(sg.out + (int64_t)v * sg.ld_out + rbase + r, ov[idx], coh);
  }
  if (a.best) {  // lane v: the wavefront's best key of vector v, then the workgroup's
    __shared__ unsigned long long sbest[4][MAX_M];
    if (lane < MT) {
      unsigned long long b = 0;
      if (lane < m)
        for (int r = 0; r < R; r++)
          if (rbase + r < r1) {
            const unsigned long long k = pick_key(ov[r * MT + lane], a.lscale, rbase + r);
            b = k > b ? k : b;
          }
      sbest[wave][lane] = b;
    }
    __syncthreads();
    if ((int)threadIdx.x < m) {
      unsigned long long b = sbest[0][threadIdx.x];
      for (int w = 1; w < 4; w++) b = sbest[w][threadIdx.x] > b ? sbest[w][threadIdx.x] : b;
      a.best[(int64_t)threadIdx.x * a.nbest + blockIdx.x] = b;
    }
  }
  if (coh && arrive_last(a.tail.counter, gridDim.x)) norm_rows<4>(a.tail, 0, m);
}

// ------------------------------------------------------------------ float matvec
// Q8_0 / Q5_0 / F32 weights x fp32 activations; four wavefronts per workgroup, eight rows per
// wavefront; tasks stride over the grid.
template <int T, int MT>
__device__ __forceinline__ void mv_f_task(const MVArgs &a, const Seg &sg, int wg, int m, bool coh, unsigned long long (&bestv)[MT]) {
  constexpr int D = MT <= 2 ? 4 : 2;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, slot = lane >> 3, l = lane & 7;
  const int64_t row = sg.r0 + ((int64_t)wg * 4 + wave) * 8 + slot;
  const bool valid = row < sg.r1;
  const int64_t grow = (int64_t)sg.expert * sg.w.rows + (valid ? row : sg.r1 - 1);
  int vidx[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) vidx[v] = v;
  float res[MT];
  if constexpr (T == T_F32) f32_walk<MT>(sg.w.pl, grow, sg.w.cols, a.x, a.ld_x, vidx, m, l, res);
  else f_walk<T, MT, D>(sg.w.pl, grow, (int)sg.w.nb, a.x, a.ld_x, vidx, m, l, res);
  if (valid && l == 0) {
#pragma unroll
    for (int v = 0; v < MT; v++)
      if (v < m) {
        out_store(sg.out + (int64_t)v * sg.ld_out + row, res[v], coh);
        if (a.best) { const unsigned long long k = pick_key(res[v], a.lscale, row); bestv[v] = k > bestv[v] ? k : bestv[v]; }
      }
  }
}

template <int MT>
__global__ __launch_bounds__(256) void k_mv_f(const MVArgs a, const StepRec *st) {
  const int m = st ? st->m : a.m;
  const bool coh = a.tail.nw != nullptr;
  unsigned long long bestv[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) bestv[v] = 0;
  const int total = a.seg[0].wgs + (a.nseg > 1 ? a.seg[1].wgs : 0) + (a.nseg > 2 ? a.seg[2].wgs : 0);
  for (int t = blockIdx.x; t < total; t += gridDim.x) {
    int wg;
    const Seg &sg = a.seg[seg_index(a, t, wg)];
    if (sg.w.dtype == T_Q8_0) mv_f_task<T_Q8_0, MT>(a, sg, wg, m, coh, bestv);
    else if (sg.w.dtype == T_Q5_0) mv_f_task<T_Q5_0, MT>(a, sg, wg, m, coh, bestv);
    else if (sg.w.dtype == T_Q5K) mv_f_task<T_Q5K, MT>(a, sg, wg, m, coh, bestv);
    else mv_f_task<T_F32, MT>(a, sg, wg, m, coh, bestv);
  }
  if (a.best) best_flush<MT, 4>(a, bestv, m);
  if (coh && arrive_last(a.tail.counter, gridDim.x)) norm_rows<4>(a.tail, 0, m);
}

// One-row float matvec over Q8_0 segments (the one-row pass of a Q8_0 model), f_walk's
// arithmetic spread over the wavefront. A task's 32 rows (k_mv_f's tasks) go to S = 8 / RW
// workgroups of four wavefronts, RW rows a wavefront (few tasks: more workgroups); a
// wavefront's RW nb (row, block) items go to its lanes in turn (item i: row i / nb, block
// i % nb; all their loads in flight), each lane forms its blocks' dots as f_walk does (four
// chains over the block's eight float4 of x, (s0 + s1) + (s2 + s3)) and parks (d, dot) in LDS;
// then lane 8 r + l runs row r's chain l over blocks l, l + 8, ... (acc = fma(d, dot, acc)) and
// the 8-lane tree hsum_rows8 forms the row: the bits of k_mv_f<1>. x is staged in LDS once.
// NI = items a lane takes (ceil(RW nb / 64)).
constexpr int MVF1_NW = 4;
template <int NI, int RW>
__global__ __launch_bounds__(MVF1_NW * 64) void k_mv_f1(const MVArgs a, const StepRec *st) {
  constexpr int S = 8 / RW;
  extern __shared__ __align__(16) uint8_t smem[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const bool coh = a.tail.nw != nullptr;
  const int nb = (int)a.seg[0].w.nb, cols = 32 * nb, ni = RW * nb;
  float *lx = reinterpret_cast<float *>(smem);
  float2 *ldd = reinterpret_cast<float2 *>(smem + (size_t)cols * 4) + (size_t)wave * ni;  // (d, dot) [row][block]
  unsigned long long bestv[1] = {0};
  const int total = a.seg[0].wgs + (a.nseg > 1 ? a.seg[1].wgs : 0) + (a.nseg > 2 ? a.seg[2].wgs : 0);
  const int sub = (int)blockIdx.x % S;
  uint4 c0[NI], c1[NI];
  uint32_t dh[NI];
  auto fetch = [&](int t) {  // task t's items (the first task's before x is staged)
    int wg;
    const Seg &sg = a.seg[seg_index(a, min(t, total - 1), wg)];
    const int64_t rbase = sg.r0 + (int64_t)wg * 32 + (sub * MVF1_NW + wave) * RW, ebase = (int64_t)sg.expert * sg.w.rows;
#pragma unroll
    for (int k = 0; k < NI; k++) {
      const int i = min(lane + 64 * k, ni - 1), r = i / nb, b = i - r * nb;
      const int64_t g = (ebase + min(rbase + r, sg.r1 - 1)) * nb + b;
      c0[k] = ld16(sg.w.pl.p0 + g * 32);
      c1[k] = ld16(sg.w.pl.p0 + g * 32 + 16);
      dh[k] = *reinterpret_cast<const uint16_t *>(sg.w.pl.p3 + g * 2);
    }
  };
  if (a.pro.nw) {  // the input row normalised here (a producer's tail otherwise)
    NormRow<MVF1_NW> nr;
    nr.load(a.pro);
    fetch((int)blockIdx.x / S);
    nr.finish(a.pro, lx, blockIdx.x == 0 ? a.pro.xn_out : nullptr);
  } else {
    fetch((int)blockIdx.x / S);
    for (int i = threadIdx.x; i < cols / 4; i += MVF1_NW * 64) reinterpret_cast<float4 *>(lx)[i] = reinterpret_cast<const float4 *>(a.x)[i];
    __syncthreads();
  }
  for (int t = (int)blockIdx.x / S; t < total; t += (int)gridDim.x / S) {
    int wg;
    const Seg &sg = a.seg[seg_index(a, t, wg)];
    const int64_t rbase = sg.r0 + (int64_t)wg * 32 + (sub * MVF1_NW + wave) * RW;
    if (t != (int)blockIdx.x / S) fetch(t);
#pragma unroll
    for (int k = 0; k < NI; k++) {
      const int i = lane + 64 * k;
      if (i < ni) {
        const int b = i % nb;
        const float4 *xv = reinterpret_cast<const float4 *>(lx + 32 * b);
        const uint32_t cw[8] = {c0[k].x, c0[k].y, c0[k].z, c0[k].w, c1[k].x, c1[k].y, c1[k].z, c1[k].w};
        float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
          const float4 xx = xv[kk];
          s0 = fmaf((float)(int8_t)(cw[kk]), xx.x, s0);
          s1 = fmaf((float)(int8_t)(cw[kk] >> 8), xx.y, s1);
          s2 = fmaf((float)(int8_t)(cw[kk] >> 16), xx.z, s2);
          s3 = fmaf((float)(int8_t)(cw[kk] >> 24), xx.w, s3);
        }
        ldd[i] = make_float2(h2f(dh[k]), (s0 + s1) + (s2 + s3));
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the items are parked
    __builtin_amdgcn_wave_barrier();
    const int r = lane >> 3, l = lane & 7;
    float acc = 0.0f;
    if (r < RW)
      for (int b = l; b < nb; b += 8) {
        const float2 e = ldd[r * nb + b];
        acc = fmaf(e.x, e.y, acc);
      }
    const float res = hsum_rows8(acc);
    const int64_t row = rbase + r;
    if (r < RW && l == 0 && row < sg.r1) {
      out_store(sg.out + row, res, coh);
      if (a.res_out) a.res_out[row] = a.res_in[row] + a.rscale * res;
      if (a.best) { const unsigned long long key = pick_key(res, a.lscale, row); bestv[0] = key > bestv[0] ? key : bestv[0]; }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();  // the items' LDS is refilled by the next task
  }
  if (a.best) best_flush<1, MVF1_NW>(a, bestv, 1);
  if (coh && arrive_last(a.tail.counter, gridDim.x)) norm_rows<MVF1_NW>(a.tail, 0, 1);
}

// One wavefront's part of a Q8_0 16-row tile against up to 16 vectors on the fp32 matrix cores:
// the batches of FQ_B 32-column blocks with index = kp mod FQ_KP (all of a batch's loads in flight),
// eight v_mfma_f32_16x16x4f32 per block with A[vector j][kq] = x[j][32b + 8kq + s] and
// B[kq][row j] = code[32b + 8kq + s] * d (an int8 times an f16 scale: exact in fp32), four
// accumulator chains (block b in chain b mod 4) summed (0 + 1) + (2 + 3). cp / dp: row
// lane & 15's codes (+ 8 (lane >> 4)) and scales; xr: vector lane & 15's values (+ 8 (lane >> 4)).
// r[q]: row lane & 15 of vector 4 (lane >> 4) + q.
constexpr int FQ_KP = 8;  // parts a tile's blocks are split into (wavefronts per tile)
constexpr int FQ_B = 4;   // blocks a part loads at once
__device__ __forceinline__ void fq_part(const uint8_t *cp, const uint16_t *dp, const float *xr, bool vin, int nb, int kp, float (&r)[4]) {
  f4v acc[4];
#pragma unroll
  for (int u = 0; u < 4; u++) acc[u] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
  for (int b0 = FQ_B * kp; b0 < nb; b0 += FQ_B * FQ_KP) {
    uint2 c[FQ_B];
    uint32_t dh[FQ_B];
    float4 x0[FQ_B], x1[FQ_B];
#pragma unroll
    for (int u = 0; u < FQ_B; u++) {
      const int b = min(b0 + u, nb - 1);
      c[u] = *reinterpret_cast<const uint2 *>(cp + (int64_t)b * 32);
      dh[u] = dp[b];
      x0[u] = *reinterpret_cast<const float4 *>(xr + (int64_t)b * 32);
      x1[u] = *reinterpret_cast<const float4 *>(xr + (int64_t)b * 32 + 4);
    }
#pragma unroll
    for (int u = 0; u < FQ_B; u++) {
      if (b0 + u < nb) {
        const float d = h2f(dh[u]);
        const float xs[8] = {x0[u].x, x0[u].y, x0[u].z, x0[u].w, x1[u].x, x1[u].y, x1[u].z, x1[u].w};
#pragma unroll
        for (int s2 = 0; s2 < 8; s2++) {
          const float w = (float)(int8_t)((s2 < 4 ? c[u].x : c[u].y) >> (8 * (s2 & 3))) * d;
          acc[u & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vin ? xs[s2] : 0.0f, w, acc[u & 3], 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < 4; q++) r[q] = (acc[0][q] + acc[1][q]) + (acc[2][q] + acc[3][q]);
}

// Float matvec of 2..16 vectors on the fp32 matrix cores (Q8_0 weights): TPW 16-row tiles per
// workgroup, eight wavefronts per tile (tasks stride over the grid as k_mv_f's): wavefront w
// takes tile w / 8 and part w % 8 of its blocks (fq_part); the parts meet in LDS and are summed
// in part order. Every product is the per-lane walk's; the sums run in a fixed order of their
// own, so a row's result does not depend on the pass's other rows, nor on TPW (one tile a
// workgroup for matrices of few rows: twice the workgroups).
template <int TPW>
__global__ __launch_bounds__(512 * TPW) void k_mv_fq(const MVArgs a, const StepRec *st) {
  constexpr int NWV = 8 * TPW;
  const int m = st ? st->m : a.m;
  const bool coh = a.tail.nw != nullptr;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 15, kq = lane >> 4;
  const int tile = wave / FQ_KP, kp = wave % FQ_KP;
  __shared__ unsigned long long sbest[16];
  __shared__ float part[FQ_KP][TPW][4][64];
  if (threadIdx.x < 16) sbest[threadIdx.x] = 0;
  __syncthreads();
  // segments in units of TPW tiles (a segment's wgs counts 32-row tasks)
  const int s0 = a.seg[0].wgs * 2 / TPW, s1 = a.nseg > 1 ? a.seg[1].wgs * 2 / TPW : 0, s2 = a.nseg > 2 ? a.seg[2].wgs * 2 / TPW : 0;
  const int total = s0 + s1 + s2;
  const bool vin = j < m;
  for (int t = blockIdx.x; t < total; t += gridDim.x) {
    const int si = __builtin_amdgcn_readfirstlane(t >= s0 ? (t >= s0 + s1 ? 2 : 1) : 0);
    const int wg = t - (si > 0 ? s0 : 0) - (si > 1 ? s1 : 0);
    const Seg &sg = a.seg[si];
    const int64_t r0 = sg.r0 + ((int64_t)wg * TPW + tile) * 16;
    float r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (r0 < sg.r1) {
      const int64_t grow = (int64_t)sg.expert * sg.w.rows + min(r0 + j, sg.r1 - 1);
      const int nb = (int)sg.w.nb;
      fq_part(sg.w.pl.p0 + grow * nb * 32 + 8 * kq, reinterpret_cast<const uint16_t *>(sg.w.pl.p3) + grow * nb,
              a.x + (int64_t)(vin ? j : 0) * a.ld_x + 8 * kq, vin, nb, kp, r);
    }
#pragma unroll
    for (int q = 0; q < 4; q++) part[kp][tile][q][lane] = r[q];
    __syncthreads();
    if (kp == 0 && r0 < sg.r1) {
      const int64_t row = r0 + j;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int v = 4 * kq + q;
        float res = part[0][tile][q][lane];
#pragma unroll
        for (int p2 = 1; p2 < FQ_KP; p2++) res = res + part[p2][tile][q][lane];
        unsigned long long key = 0;
        if (v < m && row < sg.r1) {
          out_store(sg.out + (int64_t)v * sg.ld_out + row, res, coh);
          key = pick_key(res, a.lscale, row);
        }
        if (a.best) {  // the 16 rows' best key of vector v, then one atomic per vector
#pragma unroll
          for (int o = 1; o < 16; o <<= 1) {
            const unsigned long long k2 = __shfl_xor(key, o, 64);
            key = k2 > key ? k2 : key;
          }
          if (j == 0 && v < m) atomicMax(&sbest[v], key);
        }
      }
    }
    __syncthreads();
  }
  if (a.best) {
    __syncthreads();
    if ((int)threadIdx.x < m) a.best[(int64_t)threadIdx.x * a.nbest + blockIdx.x] = sbest[threadIdx.x];
  }
  if (coh && arrive_last(a.tail.counter, gridDim.x)) norm_rows<NWV>(a.tail, 0, m);
}

// ------------------------------------------------------------------ standalone kernels
// Standalone norm: one workgroup per row.
__global__ __launch_bounds__(256) void k_norm(const NormTail t, const StepRec *st) {
  if ((int)blockIdx.x < st->m) norm_rows<4>(t, blockIdx.x, blockIdx.x + 1);
}

// fp32 rows -> permuted Q8_K, one wavefront per 256-block.
__global__ __launch_bounds__(256) void k_q8kp_quantize(const float *x, int64_t n, int64_t ld_x, int m, Q8KP out) {
  const int lane = threadIdx.x & 63;
  const int64_t nb = n / 256, gb = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gb >= nb * m) return;
  const int64_t v = gb / nb, b = gb % nb;
  const float4 xv = reinterpret_cast<const float4 *>(x + v * ld_x + b * 256)[lane];
  const float am = q8k_amax(xv);
  const int64_t vb = v * nb + b;
  q8k_block_store(xv, am, out.q + vb * 64, out.d + vb, reinterpret_cast<int *>(out.bs + vb * 8));
}

// Reference-layout Q8_K (d, qs, bsums) -> permuted layout.
__global__ __launch_bounds__(64) void k_q8kp_from_ref(const float *d, const int8_t *qs, const int16_t *bs, int64_t n, Q8KP out) {
  const int lane = threadIdx.x;
  const int64_t vb = blockIdx.x;  // (vector, block)
  const uint32_t w = reinterpret_cast<const uint32_t *>(qs + vb * 256)[lane];
  out.q[vb * 64 + (lane & 7) * 8 + (lane >> 3)] = w;
  if (lane < 16) reinterpret_cast<int *>(out.bs + vb * 8)[lane] = (int)bs[vb * 16 + lane];
  if (lane == 0 && d) out.d[vb] = d[vb];
}

// Per-block integers of one row against one vector (probe): sums[2i] = sum over the 8 lanes
// of P (the block's scaled dot), sums[2i+1] = the correction integer (Q6_K: 32 * s).
template <int T>
__global__ __launch_bounds__(64) void k_kq_block_sums(TensorView w, int expert, int64_t row, Q8KP y, int32_t *sums) {
  const int lane = threadIdx.x, l = lane & 7;
  const int64_t i = (int64_t)blockIdx.x * 8 + (lane >> 3);
  const bool ok = i < w.nb;
  const int64_t g = ((int64_t)expert * w.rows + row) * w.nb + (ok ? i : 0);
  KQRaw<T> r;
  r.load(w.pl, g, l);
  KQDec<T> dec;
  dec.decode(r, l);
  const int64_t ib = ok ? i : 0;
  const uint4 *yq = reinterpret_cast<const uint4 *>(y.q + ib * 64 + 8 * l);
  int P, s;
  dec.dot(yq[0], yq[1], y.bs[ib * 8 + l], P, s);
  P = sum8(P);
  s = sum8(s);
  if (ok && l == 0) { sums[2 * i] = P; sums[2 * i + 1] = T == T_Q6K ? 32 * s : s; }
}

// ------------------------------------------------------------------ embedding
// dequant_row (quant.rs:1548-1660) of token rows, times embedding_scale (:3381-3388), into
// t.x; then the row's norm tail (layer 0's attn_norm). One workgroup per row.
__global__ __launch_bounds__(256) void k_embed(TensorView e, const StepRec *st, float escale, const NormTail t) {
  const int b = blockIdx.x;
  if (b >= st->m) return;
  const int64_t tok = st->ids[b];
  const int64_t cols = e.cols;
  float *out = const_cast<float *>(t.x) + b * cols;
  for (int64_t j = threadIdx.x; j < cols; j += 256) {
    float v = 0.0f;
    if (e.dtype == T_F32) {
      v = reinterpret_cast<const float *>(e.pl.p0)[tok * cols + j];
    } else if (e.dtype == T_Q8_0) {
      const int64_t g = tok * e.nb + j / 32;
      const float dd = h2f(*reinterpret_cast<const uint16_t *>(e.pl.p3 + g * 2));
      v = (float)(int8_t)e.pl.p0[g * 32 + j % 32] * dd;
    } else if (e.dtype == T_Q5_0) {
      const int64_t g = tok * e.nb + j / 32;
      const int k = (int)(j % 32), l = k & 15;
      const float dd = h2f(*reinterpret_cast<const uint16_t *>(e.pl.p3 + g * 2));
      const uint32_t qh = *reinterpret_cast<const uint32_t *>(e.pl.p1 + g * 4);
      const int byte = e.pl.p0[g * 16 + l];
      const int nib = k < 16 ? (byte & 0xF) : (byte >> 4);
      const int q = nib | (int)(((qh >> k) & 1u) << 4);
      v = (float)(q - 16) * dd + 0.0f;
    } else if (e.dtype == T_Q4K) {  // element 64c + 32hi + t: byte qs[32c + t] (device offset 16(t/4) + 4c + t%4)
      const int64_t g = tok * e.nb + j / 256;
      const int k = (int)(j % 256), c = k / 64, tt = k % 32, hi = (k % 64) >= 32;
      const uint8_t *hd = e.pl.p1 + g * 16;
      const float dd = h2f(hd[0] | (hd[1] << 8)), dm = h2f(hd[2] | (hd[3] << 8));
      const uint8_t *s = hd + 4;
      const int jj = 2 * c + hi;
      int sc, mn;
      if (jj < 4) { sc = s[jj] & 63; mn = s[jj + 4] & 63; }
      else { sc = (s[jj + 4] & 0xF) | ((s[jj - 4] >> 6) << 4); mn = (s[jj + 4] >> 4) | ((s[jj] >> 6) << 4); }
      const int byte = e.pl.p0[g * 128 + 16 * (tt >> 2) + 4 * c + (tt & 3)];
      const int q = hi ? (byte >> 4) : (byte & 0xF);
      v = dd * (float)sc * (float)q - dm * (float)mn;
    } else if (e.dtype == T_Q5K) {  // element 64c + 32h + t: qs[32c + t] (device 16(t%8) + 4c + t/8), qh[t] bit 2c+h
      const int64_t g = tok * e.nb + j / 256;
      const int k = (int)(j % 256), c = k / 64, tt = k % 32, hi = (k % 64) >= 32;
      const uint8_t *hd = e.pl.p2 + g * 16;
      const float dd = h2f(hd[0] | (hd[1] << 8)), dm = h2f(hd[2] | (hd[3] << 8));
      const uint8_t *s = hd + 4;
      const int jj = 2 * c + hi;
      int sc, mn;
      if (jj < 4) { sc = s[jj] & 63; mn = s[jj + 4] & 63; }
      else { sc = (s[jj + 4] & 0xF) | ((s[jj - 4] >> 6) << 4); mn = (s[jj + 4] >> 4) | ((s[jj] >> 6) << 4); }
      const int byte = e.pl.p0[g * 128 + 16 * (tt & 7) + 4 * c + (tt >> 3)];
      const int qhb = e.pl.p1[g * 32 + 4 * (tt & 7) + (tt >> 3)];
      const int q = (hi ? (byte >> 4) : (byte & 0xF)) | (((qhb >> jj) & 1) << 4);
      v = dd * (float)sc * (float)q - dm * (float)mn;
    } else if (e.dtype == T_Q6K) {  // element 128h + 32mq + t
      const int64_t g = tok * e.nb + j / 256;
      const int k = (int)(j % 256), h = k / 128, r = k % 128, mq = r / 32, tt = r % 32;
      const int lb = 16 * (tt >> 2) + 8 * h + 4 * (mq & 1) + (tt & 3);
      const int hb = 8 * (tt >> 2) + 4 * h + (tt & 3);
      const int qlb = e.pl.p0[g * 128 + lb], qhb = e.pl.p1[g * 64 + hb];
      const int8_t *sc = reinterpret_cast<const int8_t *>(e.pl.p2 + g * 16);
      const float dd = h2f(*reinterpret_cast<const uint16_t *>(e.pl.p3 + g * 2));
      const int q = ((mq >> 1) ? (qlb >> 4) : (qlb & 0xF)) | (((qhb >> (2 * mq)) & 3) << 4);
      v = dd * (float)sc[h * 8 + tt / 16 + 2 * mq] * (float)(q - 32);
    }
    if (escale != 1.0f) v *= escale;
    out[j] = v;
  }
  if (!t.nw) return;  // no norm tail: the consumers normalise the row themselves
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  norm_rows<4>(t, b, b + 1);
}

// One workgroup per (chunk, kv head, query tile) of the pass in the step record.
template <int HD, bool MERGE>
__global__ __launch_bounds__(256) void k_attn(const AttnArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int h = blockIdx.y, c = blockIdx.x, qt = blockIdx.z;
  const int m = st->m, start = st->start, total = start + m;
  if (qt * 16 >= m * (a.n_heads / a.n_kv) || c >= (total + 63) / 64) return;
  uint32_t kr[HD / 8], vr[HD / 8];
  AttnPre pre;
  if constexpr (MERGE) attn_pre_load<HD>(a, m, start, c, h, qt, pre);
  attn_kv_first<HD, MERGE>(a, total, c, h, kr, vr);
  attn_item<HD, MERGE, false>(a, m, start, c, h, qt, smem, kr, vr, &pre);
}

// Attention partials of a prefill pass (rows prepared by k_rows_prep, so every K / V row is in
// the cache): one workgroup per (64-position chunk, kv head, four 16-query tiles). The chunk's
// K / V go to LDS once; then wavefront w takes tile 4 blockIdx.z + w on its own (its LDS
// regions private, no workgroup barrier): the query operand straight from the prepared rows
// (hi + lo f16 in registers), S = Q K^T for the four 16-position blocks, the online softmax of
// each query row over the chunk (lane = position, the chunk's only sub-chunk), O = P V for
// every 16-dim tile. Per element the operations and their order are attn_item's, so each
// (chunk, query) partial has its bits; k_attn_pf_merge merges them as attn_item's mergers do.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_pf(const AttnArgs a, const StepRec *st) {
  using LY = AttnLds<HD>;
  constexpr int KS = LY::KS, VS = LY::VS, PS = LY::PS, SS = LY::SS;
  constexpr int DT = HD / 16, DQ = HD / 4, NU = DQ / 8;
  extern __shared__ __align__(16) uint8_t smem[];
  const int h = blockIdx.y, c = blockIdx.x;
  const int m = st->m, start = st->start, total = start + m;
  const int g = a.n_heads / a.n_kv, NQ = m * g;
  if (blockIdx.z * 64 >= NQ || c >= (total + 63) / 64) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lp = tid >> 2, lq = tid & 3;
  const int ar = lane & 15, kg = (lane >> 4) * 4;
  const int qt = blockIdx.z * 4 + wave, qa = qt * 16;
  const bool act = qa < NQ;
  const int p_lo = c * 64, p_hi = min(p_lo + 64, total);
  _Float16 *ks = reinterpret_cast<_Float16 *>(smem);  // [64][KS]
  _Float16 *vt = ks + 64 * KS;                         // [HD][VS]
  uint8_t *wp = reinterpret_cast<uint8_t *>(vt + HD * VS) + (size_t)wave * (16 * SS * 4 + 2 * 16 * PS * 2 + 16 * 4);
  float *ss = reinterpret_cast<float *>(wp);             // [16][SS]
  _Float16 *ph = reinterpret_cast<_Float16 *>(ss + 16 * SS), *pl = ph + 16 * PS;  // [16][PS]
  float *sa = reinterpret_cast<float *>(pl + 16 * PS);  // [16]
  uint32_t kr[HD / 8], vr[HD / 8];
  attn_kv_first<HD, true>(a, total, c, h, kr, vr);
  // the query operand: row ar of the tile, dims 16 kt + kg .. + 3, as hi + lo f16
  h4v qhi[DT], qlo[DT];
  {
    const int qi = qa + ar;
    const float *src = qi < NQ ? a.q + (int64_t)(qi / g) * a.n_heads * HD + (h * g + qi % g) * HD : nullptr;
    float4 x[DT];
#pragma unroll
    for (int kt = 0; kt < DT; kt++) x[kt] = src ? *reinterpret_cast<const float4 *>(src + kt * 16 + kg) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int kt = 0; kt < DT; kt++) {
      _Float16 hh, ll;
      split_f16(x[kt].x, hh, ll); qhi[kt][0] = hh; qlo[kt][0] = ll;
      split_f16(x[kt].y, hh, ll); qhi[kt][1] = hh; qlo[kt][1] = ll;
      split_f16(x[kt].z, hh, ll); qhi[kt][2] = hh; qlo[kt][2] = ll;
      split_f16(x[kt].w, hh, ll); qhi[kt][3] = hh; qlo[kt][3] = ll;
    }
  }
  // cached rows -> LDS (K row-major, V transposed); rows past the pass are zero
  if (p_lo + lp >= total) {
#pragma unroll
    for (int t = 0; t < 4 * NU; t++) { kr[t] = 0u; vr[t] = 0u; }
  }
  {
    uint16_t *vt16 = reinterpret_cast<uint16_t *>(vt);
#pragma unroll
    for (int u = 0; u < NU; u++) reinterpret_cast<uint4 *>(ks + lp * KS + lq * DQ)[u] = make_uint4(kr[4 * u], kr[4 * u + 1], kr[4 * u + 2], kr[4 * u + 3]);
#pragma unroll
    for (int t = 0; t < 4 * NU; t++) {
      vt16[(lq * DQ + 2 * t) * VS + lp] = (uint16_t)(vr[t] & 0xffffu);
      vt16[(lq * DQ + 2 * t + 1) * VS + lp] = (uint16_t)(vr[t] >> 16);
    }
  }
  __syncthreads();
  if (!act) return;
  // scores S = Q K^T, position blocks pb = 0..3
#pragma unroll
  for (int pb = 0; pb < 4; pb++) {
    f4v sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kt = 0; kt < DT; kt++) {
      const h4v bk = *reinterpret_cast<const h4v *>(ks + (pb * 16 + ar) * KS + kt * 16 + kg);
      sacc = mfma16(qhi[kt], bk, sacc);
      sacc = mfma16(qlo[kt], bk, sacc);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) ss[(kg + r) * SS + pb * 16 + ar] = sacc[r];
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the scores are in LDS
  __builtin_amdgcn_wave_barrier();
  // online softmax of rows r4 * 4 .. r4 * 4 + 3 (lane = position) from the running state
  // (max -inf, sum 0) of a chunk's first sub-chunk
  float rm = -INFINITY, rl = 0.0f;  // lane r: row r's results
#pragma unroll
  for (int r0 = 0; r0 < 16; r0 += 4) {
    float sv[4], mx[4], pv[4], ls[4], mn[4], al[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = r0 + i, qi = qa + row, pos = p_lo + lane;
      sv[i] = qi < NQ && pos < p_hi && pos <= start + qi / g ? ss[row * SS + lane] * a.scale : -INFINITY;
      mx[i] = sv[i];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) mx[i] = wave_max(mx[i]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float m_old = -INFINITY;
      mn[i] = fmaxf(m_old, mx[i]);
      pv[i] = (sv[i] == -INFINITY || mn[i] == -INFINITY) ? 0.0f : expf(sv[i] - mn[i]);
      al[i] = mn[i] == -INFINITY ? 1.0f : (m_old == -INFINITY ? 0.0f : expf(m_old - mn[i]));
      ls[i] = pv[i];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) ls[i] = wave_sum(ls[i]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = r0 + i;
      split_f16(pv[i], ph[row * PS + lane], pl[row * PS + lane]);
      if (lane == row) { rm = mn[i]; rl = 0.0f * al[i] + ls[i]; }
      if (lane == 0) sa[row] = al[i];
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // probabilities and rescales in LDS
  __builtin_amdgcn_wave_barrier();
  const rsrc_t r_ml = rsrc_of(a.part_ml + ((int64_t)h * a.nslot) * ATT_QMAX * 2);
  const rsrc_t r_o = rsrc_of(a.part_o + ((int64_t)h * a.nslot) * ATT_QMAX * HD);
  float sar[4];
#pragma unroll
  for (int r = 0; r < 4; r++) sar[r] = sa[kg + r];
  // O = O * alpha + P V for every 16-dim tile (O starts at zero), then to the partial slot
#pragma unroll
  for (int j = 0; j < DT; j++) {
    f4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < 4; r++) acc[r] *= sar[r];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
      const h4v bv = *reinterpret_cast<const h4v *>(vt + (j * 16 + ar) * VS + kt * 16 + kg);
      const h4v ahi = *reinterpret_cast<const h4v *>(ph + ar * PS + kt * 16 + kg);
      const h4v alo = *reinterpret_cast<const h4v *>(pl + ar * PS + kt * 16 + kg);
      acc = mfma16(ahi, bv, acc);
      acc = mfma16(alo, bv, acc);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int qi = qa + kg + r;
      if (qi < NQ) st_coh1(r_o, ((c * ATT_QMAX + qi) * HD + j * 16 + ar) * 4, acc[r]);  // through the L2 (see k_attn_mt)
    }
  }
  if (lane < 16 && qa + lane < NQ)
    st_coh2(r_ml, (c * ATT_QMAX + qa + lane) * 8, f2v{rm, rl});
}

// The merges of a prefill pass's partials, one workgroup per (kv head, query tile, chunk group):
// the group's chunks in chunk order (with one group: straight to the tile's att rows + Q8_K;
// else to slot nch + group), then the last of the tile's group mergers merges the groups in
// group order: attn_item's merges, operation for operation.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_pf_merge(const AttnArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int h = blockIdx.x, qt = blockIdx.y, grp = blockIdx.z;
  const int m = st->m, total = st->start + m, g = a.n_heads / a.n_kv, NQ = m * g, qa = qt * 16;
  const int nch = (total + 63) / 64, ngrp = (nch + ATT_GRP - 1) / ATT_GRP;
  if (qa >= NQ || grp >= ngrp) return;
  const int gcnt = min(ATT_GRP, nch - grp * ATT_GRP);
  const rsrc_t r_ml = rsrc_of(a.part_ml + ((int64_t)h * a.nslot) * ATT_QMAX * 2);
  const rsrc_t r_o = rsrc_of(a.part_o + ((int64_t)h * a.nslot) * ATT_QMAX * HD);
  float *ol = reinterpret_cast<float *>(smem);  // [16][HD]
  if (ngrp == 1) {
    attn_merge16<HD>(r_ml, r_o, 0, gcnt, qa, NQ, ol, nullptr, nullptr, 0);
  } else {
    attn_merge16<HD>(r_ml, r_o, grp * ATT_GRP, gcnt, qa, NQ, nullptr, &r_ml, &r_o, a.nch + grp);
    int *cnt = a.counter + ((int64_t)h * ATT_QT + qt) * (1 + ATT_GMAX) * CNT_STRIDE;
    if (arrive(cnt) != ngrp - 1) return;
    if (threadIdx.x == 0) *cnt = 0;
    attn_merge16<HD>(r_ml, r_o, a.nch, ngrp, qa, NQ, ol, nullptr, nullptr, 0);
  }
  __syncthreads();
  attn_tile_out<HD>(a, h, qa, NQ, ol);
}

// ------------------------------------------------------------------ prefill attention, chunk loop
// Prefill passes (rows prepared by k_rows_prep: queries in qp, every K / V row in the cache) with
// attention bits of their own: a workgroup of eight wavefronts per (kv head, block of 64 queries,
// split sp of FL_SPLITS over the pass's 64-position chunks). Its two halves (wavefronts 0-3 and
// 4-7, 16 queries a wavefront) walk the split's even and odd chunks with an online softmax: per
// chunk S^T = K Q^T on the matrix cores (queries as hi + lo f16, as the chunk items take them),
// the chunk's max, M' = max(M, m_c), p = exp(s - M'), O = O exp(M - M') + P V,
// L = L exp(M - M') + sum p; then the halves' states meet in LDS (half 0 then half 1) and one
// (M, L, O) partial per query and split goes to memory, which k_attn_fl_merge merges in split
// order (attn_merge16: the chunk merges' arithmetic). The queries are prepared once per
// workgroup, not once per chunk, and the partials are FL_SPLITS a query, not one a chunk. The
// workgroups of one (kv head, split) run on one XCD (workgroup i on XCD i mod 8), so its
// chunks' K / V come from HBM about once for all its query blocks.
constexpr int FL_SPLITS = 4;
// Prepared query qi of kv head h (g queries a row) as hi + lo f16 matrix-core operands: dims
// 16 kt + kg .. + 3 (a query past the pass: zeros)
template <int HD>
__device__ __forceinline__ void fl_queries(const AttnArgs &a, int h, int g, int qi, bool qact, int kg, h4v (&qhi)[HD / 16], h4v (&qlo)[HD / 16]) {
  const int qb_row = qact ? qi / g : 0, qhead = qact ? qi % g : 0;
  const float *src = a.q + (int64_t)qb_row * a.n_heads * HD + (h * g + qhead) * HD + kg;
#pragma unroll
  for (int kt = 0; kt < HD / 16; kt++) {
    const float4 x = *reinterpret_cast<const float4 *>(src + kt * 16);
    const float xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) {
      _Float16 hh, ll;
      split_f16(qact ? xs[s4] : 0.0f, hh, ll);
      qhi[kt][s4] = hh;
      qlo[kt][s4] = ll;
    }
  }
}
template <int HD>
__global__ __launch_bounds__(512) void k_attn_fl(const AttnArgs a, const StepRec *st) {
  constexpr int KS = HD + 8, VS = 64 + 8, DT = HD / 16, DQ = HD / 4, NU = DQ / 8;
  constexpr int HALF_E = 64 * KS + HD * VS;  // f16 elements of one half's K / V tiles
  extern __shared__ __align__(16) uint8_t smem[];
  const int m = st->m, start = st->start, total = start + m;
  const int g = a.n_heads / a.n_kv, NQ = m * g, nqb = (gridDim.x >> 3) / ((a.n_kv * FL_SPLITS + 7) >> 3);
  const int L = blockIdx.x, xcd = L & 7, j = L >> 3, qb = j % nqb, pr = (j / nqb) * 8 + xcd;
  if (pr >= a.n_kv * FL_SPLITS || qb * 64 >= NQ) return;
  const int h = pr / FL_SPLITS, sp = pr - h * FL_SPLITS;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, ar = lane & 15, kq = lane >> 4, kg = 4 * kq;
  const int hf = wave >> 2, t256 = tid & 255;  // half (stream) and the thread's place in it
  _Float16 *ks = reinterpret_cast<_Float16 *>(smem) + hf * HALF_E;  // [64][KS]
  _Float16 *vt = ks + 64 * KS;                                       // [HD][VS] (V transposed)
  const int qa = qb * 64 + (wave & 3) * 16, qi = qa + ar;
  const bool qact = qi < NQ;
  // chunks of this split, up to the last position the workgroup's queries see; half hf takes
  // c0 + hf, c0 + hf + 2, ... (both halves walk the same number of steps: the barriers)
  const int nch = (total + 63) >> 6, b_last = min(NQ, qb * 64 + 64) - 1;
  const int c0 = sp * nch / FL_SPLITS, c1 = min((sp + 1) * nch / FL_SPLITS, (start + b_last / g) / 64 + 1);
  const int nstep = c1 > c0 ? (c1 - c0 + 1) >> 1 : 0;
  const int64_t cache0 = (int64_t)a.layer * a.max_seq * a.kv_dim + (int64_t)h * HD;
  const int lp = t256 >> 2, lq = t256 & 3;  // K / V loader: position lp, dims lq DQ ..
  uint32_t kr[4 * NU], vr[4 * NU];
  auto kv_load = [&](int c) {  // (a step past the split's chunks loads a valid row, never used)
    attn_kv_load<NU>(a, cache0 + (int64_t)min(min(c, nch - 1) * 64 + lp, total - 1) * a.kv_dim + lq * DQ, kr, vr);
  };
  if (nstep > 0) kv_load(c0 + hf);
  // the queries (prepared rows), hi + lo f16 operands: lane holds query ar, dims 16 kt + kg ..
  h4v qhi[DT], qlo[DT];
  fl_queries<HD>(a, h, g, qi, qact, kg, qhi, qlo);
  const int lim = qact ? start + qi / g + 1 : 0;  // positions < lim are visible to query ar
  float Mq = -INFINITY, Lq = 0.0f;                // running max and sum of query ar
  f4v acc[DT];                                    // O: query kg + r, dim 16 dt + ar
#pragma unroll
  for (int dt = 0; dt < DT; dt++) acc[dt] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
  for (int step = 0; step < nstep; step++) {
    const int c = c0 + hf + 2 * step, p_lo = c * 64;
    const bool mine = c < c1;
    __syncthreads();  // the previous chunks' K / V are read
    {  // chunk c's rows to LDS (rows past the pass: zero), then the next chunk's loads in flight
      uint16_t *vt16 = reinterpret_cast<uint16_t *>(vt);
      const bool live = mine && p_lo + lp < total;
#pragma unroll
      for (int u = 0; u < NU; u++)
        reinterpret_cast<uint4 *>(ks + lp * KS + lq * DQ)[u] =
            live ? make_uint4(kr[4 * u], kr[4 * u + 1], kr[4 * u + 2], kr[4 * u + 3]) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int t = 0; t < 4 * NU; t++) {
        const uint32_t w = live ? vr[t] : 0u;
        vt16[(lq * DQ + 2 * t) * VS + lp] = (uint16_t)(w & 0xffffu);
        vt16[(lq * DQ + 2 * t + 1) * VS + lp] = (uint16_t)(w >> 16);
      }
    }
    if (step + 1 < nstep) kv_load(c + 2);
    __syncthreads();
    if (qa >= NQ || !mine) continue;  // (such wavefronts still meet the barriers)
    // scores: sacc[pb][r] = S[query ar][position p_lo + 16 pb + kg + r]
    f4v sacc[4];
#pragma unroll
    for (int pb = 0; pb < 4; pb++) {
      sacc[pb] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kt = 0; kt < DT; kt++) {
        const h4v bk = *reinterpret_cast<const h4v *>(ks + (pb * 16 + ar) * KS + kt * 16 + kg);
        sacc[pb] = mfma16(bk, qhi[kt], sacc[pb]);
        sacc[pb] = mfma16(bk, qlo[kt], sacc[pb]);
      }
    }
    float sv[4][4], mx = -INFINITY;
#pragma unroll
    for (int pb = 0; pb < 4; pb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int pos = p_lo + pb * 16 + kg + r;
        sv[pb][r] = pos < lim ? sacc[pb][r] * a.scale : -INFINITY;
        mx = fmaxf(mx, sv[pb][r]);
      }
    mx = max16(mx);
    mx = max32(mx);
    const float Mn = fmaxf(Mq, mx);
    const float al = Mq == -INFINITY ? 0.0f : expf(Mq - Mn);  // (nothing accumulated yet: O, L are 0)
    float pv[4][4], ls4[4];
#pragma unroll
    for (int pb = 0; pb < 4; pb++) {
#pragma unroll
      for (int r = 0; r < 4; r++) pv[pb][r] = sv[pb][r] == -INFINITY ? 0.0f : expf(sv[pb][r] - Mn);
      ls4[pb] = (pv[pb][0] + pv[pb][1]) + (pv[pb][2] + pv[pb][3]);
      ls4[pb] = add16(ls4[pb]);
      ls4[pb] = add32(ls4[pb]);
    }
    Lq = fmaf(Lq, al, (ls4[0] + ls4[1]) + (ls4[2] + ls4[3]));
    Mq = Mn;
    // O rows are queries kg + r: their factors from lanes kg + r (query ar = kg + r)
    float alr[4];
#pragma unroll
    for (int r = 0; r < 4; r++) alr[r] = __shfl(al, kg + r, 64);
    h4v phv[4], plv[4];
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        _Float16 hh, ll;
        split_f16(pv[kt][r], hh, ll);
        phv[kt][r] = hh;
        plv[kt][r] = ll;
      }
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
      f4v o = acc[dt];
#pragma unroll
      for (int r = 0; r < 4; r++) o[r] = o[r] * alr[r];
#pragma unroll
      for (int kt = 0; kt < 4; kt++) {
        const h4v bv = *reinterpret_cast<const h4v *>(vt + (dt * 16 + ar) * VS + kt * 16 + kg);
        o = mfma16(phv[kt], bv, o);
        o = mfma16(plv[kt], bv, o);
      }
      acc[dt] = o;
    }
  }
  // the halves meet: half 1's states to LDS (over the K / V tiles), half 0 combines (half 0's
  // weight first) and writes the split's partial
  __syncthreads();
  float *xo = reinterpret_cast<float *>(smem);            // [4 waves][DT][4][64]
  float *xm = xo + 4 * DT * 4 * 64;                       // [4 waves][16][2]
  const int w4 = wave & 3;
  if (hf == 1) {
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int r = 0; r < 4; r++) xo[((w4 * DT + dt) * 4 + r) * 64 + lane] = acc[dt][r];
    if (kq == 0) { xm[(w4 * 16 + ar) * 2] = Mq; xm[(w4 * 16 + ar) * 2 + 1] = Lq; }
  }
  __syncthreads();
  if (hf == 1 || qa >= NQ) return;
  const float M1 = xm[(w4 * 16 + ar) * 2], L1 = xm[(w4 * 16 + ar) * 2 + 1];
  const float Mt = fmaxf(Mq, M1);
  const float w0 = Mq == -INFINITY ? 0.0f : expf(Mq - Mt), w1 = M1 == -INFINITY ? 0.0f : expf(M1 - Mt);
  const float Lt = fmaf(L1, w1, Lq * w0);
  float w0r[4], w1r[4];
#pragma unroll
  for (int r = 0; r < 4; r++) { w0r[r] = __shfl(w0, kg + r, 64); w1r[r] = __shfl(w1, kg + r, 64); }
  const rsrc_t r_ml = rsrc_of(a.part_ml + ((int64_t)h * a.nslot) * ATT_QMAX * 2);
  const rsrc_t r_o = rsrc_of(a.part_o + ((int64_t)h * a.nslot) * ATT_QMAX * HD);
  if (kq == 0 && qact) st_coh2(r_ml, (sp * ATT_QMAX + qi) * 8, f2v{Mt, Lt});
#pragma unroll
  for (int dt = 0; dt < DT; dt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int q = qa + kg + r;
      const float o = fmaf(xo[((w4 * DT + dt) * 4 + r) * 64 + lane], w1r[r], acc[dt][r] * w0r[r]);
      if (q < NQ) st_coh1(r_o, ((sp * ATT_QMAX + q) * HD + dt * 16 + ar) * 4, o);
    }
}

// The splits' partials of 16 queries merged in split order (attn_merge16), then the att rows
// and their Q8_K (attn_tile_out): a workgroup per (kv head, 16-query tile).
template <int HD>
__global__ __launch_bounds__(256) void k_attn_fl_merge(const AttnArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int h = blockIdx.x, qa = blockIdx.y * 16, NQ = st->m * (a.n_heads / a.n_kv);
  if (qa >= NQ) return;
  const rsrc_t r_ml = rsrc_of(a.part_ml + ((int64_t)h * a.nslot) * ATT_QMAX * 2);
  const rsrc_t r_o = rsrc_of(a.part_o + ((int64_t)h * a.nslot) * ATT_QMAX * HD);
  float *ol = reinterpret_cast<float *>(smem);  // [16][HD]
  attn_merge16<HD>(r_ml, r_o, 0, FL_SPLITS, qa, NQ, ol, nullptr, nullptr, 0);
  __syncthreads();
  attn_tile_out<HD>(a, h, qa, NQ, ol);
}

// ------------------------------------------------------------------ prefill attention, position slices
// Prefill passes (rows prepared by k_rows_prep) with attention bits of their own and no partials
// in memory: a workgroup of eight wavefronts per (kv head, block of 16 queries). Wavefront w
// takes the 32-position slices w, w + 8, w + 16, ... of the positions its queries see (each
// workgroup starting at its own place in that list) and keeps
// an online softmax over them in registers, with no LDS and no barrier until the end: per slice
// S^T = K Q^T as two 16-position tiles and P V over the 32 positions, on the K = 32 f16 matrix
// cores (v_mfma_f32_16x16x32_f16; queries and probabilities as hi + lo f16, products exact in
// fp32), the slice's max, M' = max(M, m_s), p = exp(s - M'), O = O exp(M - M') + P V,
// L = L exp(M - M') + sum p. The slice's K rows and V columns go from memory straight into the
// operand layouts (the next slice's loads in flight during the softmax and P V): the contraction
// dims are permuted alike in K and Q (lane group kq holds dims 32 u + 8 kq .. + 7 of step u: a
// 16-byte piece of a K row per load), the positions alike in P and V (lane group kq holds
// positions 16 t + 4 kq + r, r < 4, of tile t: the rows of S^T it holds), and P V's output
// columns are dims DT x + t (lane x holds DT consecutive dims of each of its eight V rows: four
// whole 256-byte rows per load). The eight states then meet in LDS (M = max M_w,
// w_w = exp(M_w - M), L = sum L_w w_w, O = sum w_w O_w, wavefronts in order) and O / L goes to
// the att rows (and their Q8_K). Workgroup i runs on XCD i mod 8, and XCD x takes the
// (kv head, block) units x P .. x P + P - 1 (kv head major): a kv head's blocks share one or two
// L2s.
__device__ __forceinline__ uint32_t word_of(const uint4 &v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
__device__ __forceinline__ uint32_t word_of(const uint2 &v, int i) { return i == 0 ? v.x : v.y; }
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f4v mfma32h(h8v a, h8v b, f4v c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
template <int HD>
__global__ __launch_bounds__(512) void k_attn_fs(const AttnArgs a, const StepRec *st) {
  constexpr int DT = HD / 16, NPC = HD / 32;  // output tiles (dims a lane's column holds), K pieces a lane
  using VRow = typename std::conditional<DT == 8, uint4, uint2>::type;  // DT f16 of one V row
  extern __shared__ __align__(16) uint8_t smem[];
  const int m = st->m, start = st->start, total = start + m;
  const int g = a.n_heads / a.n_kv, NQ = m * g, nqb = (NQ + 15) >> 4;
  const int u = (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3);
  if (u >= a.n_kv * nqb) return;
  const int h = u / nqb, qa = (u - h * nqb) * 16;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, ar = lane & 15, kq = lane >> 4, kg = 4 * kq;
  const int qi = qa + ar;
  const bool qact = qi < NQ;
  const int p_end = start + (min(NQ, qa + 16) - 1) / g + 1;  // positions any of the block's queries sees
  const int nsl = (p_end + 31) >> 5, nstep = wave < nsl ? (nsl - wave + 7) >> 3 : 0;
  const __half *kc = a.kc + (int64_t)a.layer * a.max_seq * a.kv_dim + (int64_t)h * HD;
  const __half *vc = a.vc + (int64_t)a.layer * a.max_seq * a.kv_dim + (int64_t)h * HD;
  // slice i's rows as this lane takes them (rows past the pass: the last row, masked)
  uint4 kr[2][NPC];
  VRow vr[2][4];
  auto kv_load = [&](int i) {
    const int p0 = min(i, nsl - 1) * 32;
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const __half *kp = kc + (int64_t)min(p0 + 16 * t + ar, total - 1) * a.kv_dim + 8 * kq;
#pragma unroll
      for (int uu = 0; uu < NPC; uu++) kr[t][uu] = *reinterpret_cast<const uint4 *>(kp + 32 * uu);
    }
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        vr[t][r] = *reinterpret_cast<const VRow *>(vc + (int64_t)min(p0 + 16 * t + kg + r, total - 1) * a.kv_dim + DT * ar);
  };
  // the workgroups of a kv head start their walks at different slices (rot), so the CUs of an
  // XCD read different lines of its K / V at a time
  const int rot = nstep > 0 ? (u - h * nqb) % nstep : 0;
  if (nstep > 0) kv_load(wave + 8 * rot);
  // the queries as hi + lo f16 operands, dims permuted as K's: step uu takes dims 32 uu + 8 kq ..
  // + 7. a.prepped 2: from the raw projections, with head_prep's operations here (bias; RMSNorm,
  // the sum of squares over the lane's 32 dims then the query's four lanes; RoPE, whose pairs
  // (d, d + HD / 2) or (2 i, 2 i + 1) a lane holds both halves of); 1: prepared rows
  h8v qhi[NPC], qlo[NPC];
  {
    const int qb_row = qact ? qi / g : 0, qhead = h * g + (qact ? qi % g : 0);
    const float *src = a.q + (int64_t)qb_row * a.n_heads * HD + qhead * HD + 8 * kq;
    float x[NPC][8];
#pragma unroll
    for (int uu = 0; uu < NPC; uu++) {
      const float4 x0 = *reinterpret_cast<const float4 *>(src + 32 * uu), x1 = *reinterpret_cast<const float4 *>(src + 32 * uu + 4);
      x[uu][0] = x0.x; x[uu][1] = x0.y; x[uu][2] = x0.z; x[uu][3] = x0.w;
      x[uu][4] = x1.x; x[uu][5] = x1.y; x[uu][6] = x1.z; x[uu][7] = x1.w;
    }
    if (a.prepped == 2) {
      if (a.q_bias) {
        const float *bp = a.q_bias + qhead * HD + 8 * kq;
#pragma unroll
        for (int uu = 0; uu < NPC; uu++)
#pragma unroll
          for (int j = 0; j < 8; j++) x[uu][j] += bp[32 * uu + j];
      }
      if (a.q_norm) {
        float ss = 0.0f;
#pragma unroll
        for (int uu = 0; uu < NPC; uu++)
#pragma unroll
          for (int j = 0; j < 8; j++) ss = fmaf(x[uu][j], x[uu][j], ss);
        ss = add16(ss);
        ss = add32(ss);
        const float inv = inv_rms(ss, (float)HD, a.eps);
        const float *nw = a.q_norm + 8 * kq;
#pragma unroll
        for (int uu = 0; uu < NPC; uu++)
#pragma unroll
          for (int j = 0; j < 8; j++) x[uu][j] = x[uu][j] * inv * nw[32 * uu + j];
      }
      const float2 *rp = a.rope + (int64_t)(start + qb_row) * (HD / 2);
      if (a.neox) {
#pragma unroll
        for (int uu = 0; uu < NPC / 2; uu++)
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float2 cs = rp[32 * uu + 8 * kq + j];
            const float x0 = x[uu][j], x1 = x[uu + NPC / 2][j];
            x[uu][j] = x0 * cs.x - x1 * cs.y;
            x[uu + NPC / 2][j] = x0 * cs.y + x1 * cs.x;
          }
      } else {
#pragma unroll
        for (int uu = 0; uu < NPC; uu++)
#pragma unroll
          for (int j = 0; j < 8; j += 2) {
            const float2 cs = rp[16 * uu + 4 * kq + j / 2];
            const float x0 = x[uu][j], x1 = x[uu][j + 1];
            x[uu][j] = x0 * cs.x - x1 * cs.y;
            x[uu][j + 1] = x0 * cs.y + x1 * cs.x;
          }
      }
    }
#pragma unroll
    for (int uu = 0; uu < NPC; uu++)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        _Float16 hh, ll;
        split_f16(qact ? x[uu][j] : 0.0f, hh, ll);
        qhi[uu][j] = hh;
        qlo[uu][j] = ll;
      }
  }
  const int lim = qact ? start + qi / g + 1 : 0;  // positions < lim are visible to query ar
  float Mq = -INFINITY, Lq = 0.0f;                // running max and sum of query ar over the slices
  f4v acc[DT];                                    // O: query kg + r, dim DT ar + dt
#pragma unroll
  for (int dt = 0; dt < DT; dt++) acc[dt] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
  for (int step = 0, sr = rot; step < nstep; step++, sr = sr + 1 == nstep ? 0 : sr + 1) {
    const int i = wave + 8 * sr, p0 = 32 * i;
    // scores: sacc[t][r] = S[query ar][position p0 + 16 t + kg + r]
    f4v sacc[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
      sacc[t] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int uu = 0; uu < NPC; uu++) {
        const h8v bk = __builtin_bit_cast(h8v, kr[t][uu]);
        sacc[t] = mfma32h(bk, qhi[uu], sacc[t]);
        sacc[t] = mfma32h(bk, qlo[uu], sacc[t]);
      }
    }
    // V columns of this lane: vv[dt] element 4 t + r = V[p0 + 16 t + kg + r][DT ar + dt]
    h8v vv[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
      // (v_perm_b32: the low or high halves of two rows' words side by side)
      const uint32_t sel = (dt & 1) ? 0x07060302u : 0x05040100u;
      uint32_t e[4];
#pragma unroll
      for (int j = 0; j < 4; j++)
        e[j] = __builtin_amdgcn_perm(word_of(vr[j >> 1][2 * (j & 1) + 1], dt >> 1), word_of(vr[j >> 1][2 * (j & 1)], dt >> 1), sel);
      vv[dt] = __builtin_bit_cast(h8v, make_uint4(e[0], e[1], e[2], e[3]));
    }
    if (step + 1 < nstep) kv_load(wave + 8 * (sr + 1 == nstep ? 0 : sr + 1));
    float sv[2][4], mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        sv[t][r] = p0 + 16 * t + kg + r < lim ? sacc[t][r] * a.scale : -INFINITY;
        mx = fmaxf(mx, sv[t][r]);
      }
    mx = max16(mx);
    mx = max32(mx);
    const float Mn = fmaxf(Mq, mx);
    const float al = Mq == -INFINITY ? 0.0f : expf(Mq - Mn);  // (nothing accumulated yet: O, L are 0)
    float pv[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) pv[t][r] = sv[t][r] == -INFINITY ? 0.0f : expf(sv[t][r] - Mn);
    float ls = ((pv[0][0] + pv[0][1]) + (pv[0][2] + pv[0][3])) + ((pv[1][0] + pv[1][1]) + (pv[1][2] + pv[1][3]));
    ls = add16(ls);
    ls = add32(ls);
    Lq = fmaf(Lq, al, ls);
    Mq = Mn;
    // O rows are queries kg + r: their factors from lanes kg + r (query ar = kg + r)
    float alr[4];
#pragma unroll
    for (int r = 0; r < 4; r++) alr[r] = __shfl(al, kg + r, 64);
    h8v phv, plv;
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        _Float16 hh, ll;
        split_f16(pv[t][r], hh, ll);
        phv[4 * t + r] = hh;
        plv[4 * t + r] = ll;
      }
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
      f4v o = acc[dt];
#pragma unroll
      for (int r = 0; r < 4; r++) o[r] = o[r] * alr[r];
      o = mfma32h(phv, vv[dt], o);
      o = mfma32h(plv, vv[dt], o);
      acc[dt] = o;
    }
  }
  // the eight states to LDS, merged per (query, dim) in wavefront order
  float *xo = reinterpret_cast<float *>(smem);  // [8 waves][DT][4][64]
  float *xm = xo + 8 * DT * 4 * 64;             // [8 waves][16][2]
  float *ol = xm + 8 * 16 * 2;                  // [16][HD]
#pragma unroll
  for (int dt = 0; dt < DT; dt++)
#pragma unroll
    for (int r = 0; r < 4; r++) xo[((wave * DT + dt) * 4 + r) * 64 + lane] = acc[dt][r];
  if (kq == 0) { xm[(wave * 16 + ar) * 2] = Mq; xm[(wave * 16 + ar) * 2 + 1] = Lq; }
  __syncthreads();
  {
    constexpr int DW = HD / 32;  // 32 threads a query, DW dims each
    const int qq = tid >> 5, d0 = (tid & 31) * DW, src_lane = 16 * (qq >> 2), r = qq & 3;
    float mw[8], ww[8], M = -INFINITY, L = 0.0f;
#pragma unroll
    for (int w = 0; w < 8; w++) { mw[w] = xm[(w * 16 + qq) * 2]; M = fmaxf(M, mw[w]); }
#pragma unroll
    for (int w = 0; w < 8; w++) {
      ww[w] = mw[w] == -INFINITY ? 0.0f : expf(mw[w] - M);
      L = fmaf(xm[(w * 16 + qq) * 2 + 1], ww[w], L);
    }
    const float il = __fdiv_rn(1.0f, fmaxf(L, 1e-30f));
#pragma unroll
    for (int j = 0; j < DW; j++) {
      const int d = d0 + j, dt = d % DT, x = d / DT;  // dim d = DT x + dt: tile dt, column x
      float o = 0.0f;
#pragma unroll
      for (int w = 0; w < 8; w++) o = fmaf(xo[((w * DT + dt) * 4 + r) * 64 + src_lane + x], ww[w], o);
      ol[qq * HD + d] = o * il;
    }
  }
  __syncthreads();
  if (tid < 256) attn_tile_out<HD>(a, h, qa, NQ, ol);
}

// ------------------------------------------------------------------ multi-tile attention
// Passes of up to 16 rows: one workgroup of eight wavefronts per (64-position chunk, kv head,
// eight 16-query tiles). The chunk's K / V rows go to LDS once (the pass's own rows normed and
// rotated on the way, and written to the cache); then wavefront w computes query tile
// 8 blockIdx.z + w alone, in registers, with no further barrier:
//   * its queries prepared in the matrix cores' operand layout (lane: query lane & 15, dims
//     16 kt + 4 (lane >> 4) .. + 3), head_prep's operations with its norm reduction tree
//     restated over that layout (every butterfly node pairs the same two values);
//   * the scores as S^T = K Q^T: a lane then holds positions 16 pb + 4 (lane >> 4) + r of its
//     query, which is the layout P V takes its probabilities in, so they never go to LDS;
//     the products are the ones of Q K^T (f16 x f16, exact in fp32) summed in the same order;
//   * the chunk's max and sum as the 64-lane butterflies of wave_max / wave_sum restated over
//     the positions a lane holds (in-lane for position bits 0, 1, 4, 5; lane ^ 16, lane ^ 32 for
//     bits 2, 3), then P V as attn_item does it.
// Each (chunk, query) partial therefore has attn_item's bits; k_attn_mrg merges them.
template <int HD>
struct MtLds {
  static constexpr int KS = HD + 8, VS = 64 + 8;
  // K [64][KS], V^T [HD][VS] (f16); the query norm weights [HD]; with a query bias the kv
  // group's biases [g][HD]; the rotations of the pass rows the workgroup's queries belong to
  // [rows][HD/2] (float2) at off_rot
  static constexpr size_t OFF_QN = (size_t)64 * KS * 2 + (size_t)HD * VS * 2, OFF_QB = OFF_QN + (size_t)HD * 4;
  __host__ __device__ static size_t off_rot(int g, bool bias) { return OFF_QB + (bias ? (size_t)g * HD * 4 : 0); }
  // pass rows the 128 queries of a workgroup span (g queries a row)
  __host__ __device__ static int rot_rows(int g, int m) { return min(m, (128 + g - 1) / g + 1); }
  static size_t bytes(int g, bool bias, int m) { return off_rot(g, bias) + (size_t)rot_rows(g, m) * HD * 4; }
};

// BIG: prefill passes (up to 128 rows, a workgroup per 128 queries of a (chunk, kv head)); the
// pass's new K / V rows in the chunk (up to 64) are prepared from memory in a loop
template <int HD, bool BIG>
__global__ __launch_bounds__(512) void k_attn_mt(const AttnArgs a, const StepRec *st) {
  using LY = MtLds<HD>;
  constexpr int KS = LY::KS, VS = LY::VS;
  constexpr int DT = HD / 16;              // 16-dim tiles: k steps of K Q^T, output tiles of P V
  constexpr int DQ = HD / 8, NU = DQ / 8;  // K / V loader: 8 threads a position, DQ dims each
  constexpr int half = HD / 2;
  extern __shared__ __align__(16) uint8_t smem[];
  _Float16 *ks = reinterpret_cast<_Float16 *>(smem);  // [64][KS]
  _Float16 *vt = ks + 64 * KS;                        // [HD][VS] (V transposed)
  // BIG: workgroups placed by XCD (workgroup i runs on XCD i mod 8): XCD x takes the
  // (kv head, query block) pairs x P/8 .. x P/8 + P/8 - 1 (P = n_kv x query blocks, kv head
  // major) over all chunks, so a query block's raw rows are fetched by one L2, not eight, and a
  // kv head's chunks by P/8 query blocks' XCDs; the same (chunk, head, block) items as the grid
  int c = blockIdx.x, h = blockIdx.y, zb = blockIdx.z;
  if (BIG && ((gridDim.y * gridDim.z) & 7) == 0) {
    const int L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z), sl = L >> 3;
    const int pr = (L & 7) * ((gridDim.y * gridDim.z) >> 3) + sl / gridDim.x;
    c = sl % gridDim.x;
    h = pr / gridDim.z;
    zb = pr % gridDim.z;
  }
  const int m = st->m, start = st->start, total = start + m;
  const int g = a.n_heads / a.n_kv, NQ = m * g;
  float *qn_s = reinterpret_cast<float *>(smem + LY::OFF_QN), *qb_s = reinterpret_cast<float *>(smem + LY::OFF_QB);
  float *rot_s = reinterpret_cast<float *>(smem + LY::off_rot(g, a.q_bias != nullptr));
  if (zb * 128 >= NQ || c >= (total + 63) / 64) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ar = lane & 15, kq = lane >> 4, kg = 4 * kq;
  const int qa = (zb * 8 + wave) * 16, qi = qa + ar;
  const bool qact = qi < NQ;
  const int p_lo = c * 64, p_hi = min(p_lo + 64, total);
  const int64_t cache0 = (int64_t)a.layer * a.max_seq * a.kv_dim + (int64_t)h * HD;

  // (1) loads in the order their values are needed (they return in issue order): the values
  // every wavefront shares (rotations of the pass's rows, norm weights, biases) for LDS, then
  // this lane's raw query values
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  constexpr int RPT = BIG ? 5 : 1;  // rotation float4s a thread stages (rows <= 65 at g >= 2 for BIG)
  const int rb0 = zb * 128 / g, nrot = min(m - rb0, LY::rot_rows(g, m)), nrv = nrot * (half / 2);
  float4 sh_rot[RPT], sh_qn = z4, sh_qb = z4;
  const bool ld_qn = a.q_norm && tid < HD / 4, ld_qb = a.q_bias && tid < g * HD / 4;
#pragma unroll
  for (int i = 0; i < RPT; i++)
    sh_rot[i] = reinterpret_cast<const float4 *>(a.rope + (int64_t)(start + rb0) * half)[min(tid + 512 * i, nrv - 1)];  // (valid index)
  if (ld_qn) sh_qn = reinterpret_cast<const float4 *>(a.q_norm)[tid];
  if (ld_qb) sh_qb = reinterpret_cast<const float4 *>(a.q_bias + (int64_t)h * g * HD)[tid];
  float4 xq[DT];
  const int qb_row = qact ? qi / g : 0, qhead = qact ? qi % g : 0;  // a lane past the pass reads row 0 and drops it
  {
    const float *src = a.q + (int64_t)qb_row * a.n_heads * HD + (h * g + qhead) * HD + kg;
#pragma unroll
    for (int kt = 0; kt < DT; kt++) xq[kt] = *reinterpret_cast<const float4 *>(src + kt * 16);
  }
  // (2) the pass's new K / V rows in this chunk: rows b = wave, wave + 8 (head_prep's layout;
  // BIG: prepared from memory below)
  const bool act = lane < half;
  const int da = a.neox ? lane : 2 * lane, db = a.neox ? lane + half : 2 * lane + 1;
  float nk0[2], nk1[2], nkb0[2], nkb1[2], nv0[2], nv1[2], nvb0[2], nvb1[2], nkc[2], nks[2], kn0 = 0.0f, kn1 = 0.0f;
  if (a.k_norm && act) { kn0 = a.k_norm[da]; kn1 = a.k_norm[db]; }
#pragma unroll
  for (int j = 0; j < 2 && !BIG; j++) {
    const int b = wave + 8 * j, pos = start + b;
    nk0[j] = nk1[j] = nkb0[j] = nkb1[j] = nv0[j] = nv1[j] = nvb0[j] = nvb1[j] = 0.0f;
    nkc[j] = 1.0f;
    nks[j] = 0.0f;
    if (b < m && pos >= p_lo && pos < p_hi && act) {
      const float *kp = a.k + (int64_t)b * a.kv_dim + h * HD, *vp = a.v + (int64_t)b * a.kv_dim + h * HD;
      nk0[j] = kp[da]; nk1[j] = kp[db];
      nv0[j] = vp[da]; nv1[j] = vp[db];
      if (a.k_bias) { nkb0[j] = a.k_bias[h * HD + da]; nkb1[j] = a.k_bias[h * HD + db]; }
      if (a.v_bias) { nvb0[j] = a.v_bias[h * HD + da]; nvb1[j] = a.v_bias[h * HD + db]; }
      const float2 cs = a.rope[(int64_t)pos * half + lane];
      nkc[j] = cs.x;
      nks[j] = cs.y;
    }
  }
  // (3) the chunk's cached rows
  const int lp = tid >> 3, lq = tid & 7;
  uint32_t kr[4 * NU], vr[4 * NU];
  attn_kv_load<NU>(a, cache0 + (int64_t)min(p_lo + lp, p_hi - 1) * a.kv_dim + lq * DQ, kr, vr);

  // the shared values to LDS (waits for them only)
#pragma unroll
  for (int i = 0; i < RPT; i++)
    if (tid + 512 * i < nrv) reinterpret_cast<float4 *>(rot_s)[tid + 512 * i] = sh_rot[i];
  if (ld_qn) reinterpret_cast<float4 *>(qn_s)[tid] = sh_qn;
  if (ld_qb) reinterpret_cast<float4 *>(qb_s)[tid] = sh_qb;
  __syncthreads();
  // (4) the queries: bias, RMSNorm, rotation (head_prep's operations), as hi + lo f16 operands
  // (waits for (1) only; a wavefront without a tile prepares zeros)
  float x[DT][4];
#pragma unroll
  for (int kt = 0; kt < DT; kt++) {
    x[kt][0] = xq[kt].x; x[kt][1] = xq[kt].y; x[kt][2] = xq[kt].z; x[kt][3] = xq[kt].w;
    if (a.q_bias) {
      const float4 xb = *reinterpret_cast<const float4 *>(qb_s + qhead * HD + kt * 16 + kg);
      x[kt][0] += xb.x; x[kt][1] += xb.y; x[kt][2] += xb.z; x[kt][3] += xb.w;
    }
  }
  if (a.q_norm) {
    // head_prep: wave_sum over lanes L < HD/2 of fmaf(x[da(L)], x[da(L)], x[db(L)]^2) (lanes
    // past HD/2 add zeros); node L ^ 2^i of that butterfly, over the values this lane holds
    float ssq;
    if (a.neox) {  // L = 16kt + 4kq + s (kt < DT/2): bits 0-1 s, 2-3 kq, 4.. kt
      float t4[DT / 2];
#pragma unroll
      for (int kt = 0; kt < DT / 2; kt++) {
        float tt[4];
#pragma unroll
        for (int s = 0; s < 4; s++) tt[s] = fmaf(x[kt][s], x[kt][s], x[kt + DT / 2][s] * x[kt + DT / 2][s]);
        t4[kt] = (tt[0] + tt[1]) + (tt[2] + tt[3]);
        t4[kt] = add16(t4[kt]);
        t4[kt] = add32(t4[kt]);
      }
      if constexpr (DT / 2 == 4) ssq = (t4[0] + t4[1]) + (t4[2] + t4[3]);
      else ssq = t4[0] + t4[1];
    } else {  // L = 8kt + 2kq + s/2: bit 0 s/2, bits 1-2 kq, 3.. kt
      float t2[DT];
#pragma unroll
      for (int kt = 0; kt < DT; kt++) {
        t2[kt] = fmaf(x[kt][0], x[kt][0], x[kt][1] * x[kt][1]) + fmaf(x[kt][2], x[kt][2], x[kt][3] * x[kt][3]);
        t2[kt] = add16(t2[kt]);
        t2[kt] = add32(t2[kt]);
      }
      if constexpr (DT == 8) ssq = ((t2[0] + t2[1]) + (t2[2] + t2[3])) + ((t2[4] + t2[5]) + (t2[6] + t2[7]));
      else ssq = (t2[0] + t2[1]) + (t2[2] + t2[3]);
    }
    const float inv = inv_rms(ssq, (float)HD, a.eps);
#pragma unroll
    for (int kt = 0; kt < DT; kt++) {
      const float4 nq = *reinterpret_cast<const float4 *>(qn_s + kt * 16 + kg);
      x[kt][0] = x[kt][0] * inv * nq.x; x[kt][1] = x[kt][1] * inv * nq.y;
      x[kt][2] = x[kt][2] * inv * nq.z; x[kt][3] = x[kt][3] * inv * nq.w;
    }
  }
  if (a.neox) {
#pragma unroll
    for (int kt = 0; kt < DT / 2; kt++) {
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const float4 r4 = *reinterpret_cast<const float4 *>(rot_s + (qb_row - rb0) * HD + 2 * (kt * 16 + kg) + 4 * (s >> 1));
        const float cv = (s & 1) ? r4.z : r4.x, sn = (s & 1) ? r4.w : r4.y;
        const float x0 = x[kt][s], x1 = x[kt + DT / 2][s];
        x[kt][s] = x0 * cv - x1 * sn;
        x[kt + DT / 2][s] = x0 * sn + x1 * cv;
      }
    }
  } else {
#pragma unroll
    for (int kt = 0; kt < DT; kt++) {
      const float4 r4 = *reinterpret_cast<const float4 *>(rot_s + (qb_row - rb0) * HD + 2 * (kt * 8 + 2 * kq));
#pragma unroll
      for (int p = 0; p < 2; p++) {
        const float cv = p ? r4.z : r4.x, sv = p ? r4.w : r4.y;
        const float x0 = x[kt][2 * p], x1 = x[kt][2 * p + 1];
        x[kt][2 * p] = x0 * cv - x1 * sv;
        x[kt][2 * p + 1] = x0 * sv + x1 * cv;
      }
    }
  }
  h4v qhi[DT], qlo[DT];
#pragma unroll
  for (int kt = 0; kt < DT; kt++)
#pragma unroll
    for (int s = 0; s < 4; s++) {
      _Float16 hh, ll;
      split_f16(qact ? x[kt][s] : 0.0f, hh, ll);
      qhi[kt][s] = hh;
      qlo[kt][s] = ll;
    }
  // (5) LDS
  // cached rows -> LDS (K row-major, V transposed); rows past the pass are zero, the pass's
  // rows come from (2)
  if (p_lo + lp >= total) {
#pragma unroll
    for (int t = 0; t < 4 * NU; t++) { kr[t] = 0u; vr[t] = 0u; }
  }
  if (p_lo + lp < start || p_lo + lp >= total) {
    uint16_t *vt16 = reinterpret_cast<uint16_t *>(vt);
#pragma unroll
    for (int u = 0; u < NU; u++) reinterpret_cast<uint4 *>(ks + lp * KS + lq * DQ)[u] = make_uint4(kr[4 * u], kr[4 * u + 1], kr[4 * u + 2], kr[4 * u + 3]);
#pragma unroll
    for (int t = 0; t < 4 * NU; t++) {
      vt16[(lq * DQ + 2 * t) * VS + lp] = (uint16_t)(vr[t] & 0xffffu);
      vt16[(lq * DQ + 2 * t + 1) * VS + lp] = (uint16_t)(vr[t] >> 16);
    }
  }
#pragma unroll
  for (int j = 0; j < 2 && !BIG; j++) {
    const int b = wave + 8 * j, pos = start + b, pp = pos - p_lo;
    if (b < m && pos >= p_lo && pos < p_hi) {
      float e0, e1;
      head_prep_pre(nk0[j], nk1[j], nkb0[j], nkb1[j], a.k_bias != nullptr, a.k_norm != nullptr, kn0, kn1, true, nkc[j], nks[j], HD, a.eps,
                    e0, e1);
      if (act) {
        const __half k0 = __float2half_rn(e0), k1 = __float2half_rn(e1);
        ks[pp * KS + da] = (_Float16)__half2float(k0);
        ks[pp * KS + db] = (_Float16)__half2float(k1);
        if (zb == 0) { __half *kd = a.kc + cache0 + (int64_t)pos * a.kv_dim; kd[da] = k0; kd[db] = k1; }
      }
      head_prep_pre(nv0[j], nv1[j], nvb0[j], nvb1[j], a.v_bias != nullptr, false, 0.0f, 0.0f, false, 1.0f, 0.0f, HD, a.eps, e0, e1);
      if (act) {
        const __half v0 = __float2half_rn(e0), v1 = __float2half_rn(e1);
        vt[da * VS + pp] = (_Float16)__half2float(v0);
        vt[db * VS + pp] = (_Float16)__half2float(v1);
        if (zb == 0) { __half *vd = a.vc + cache0 + (int64_t)pos * a.kv_dim; vd[da] = v0; vd[db] = v1; }
      }
    }
  }
  if constexpr (BIG) {
    // rows b in [b_lo, b_hi): wavefront w takes b_lo + w + 8 j, in batches of NB rows whose
    // loads (row values, rotation) are all issued before the first row's arithmetic; then
    // head_prep_pre, head_prep's operations on the loaded values (inactive lanes hold zeros)
    constexpr int NB = 8;
    const int b_lo = max(0, p_lo - start), b_hi = min(m, p_hi - start);
    const int dA = act ? da : 0, dB = act ? db : 0, ln = act ? lane : 0;
    float kb0 = 0.0f, kb1 = 0.0f, vb0 = 0.0f, vb1 = 0.0f;
    if (a.k_bias) { kb0 = a.k_bias[h * HD + dA]; kb1 = a.k_bias[h * HD + dB]; }
    if (a.v_bias) { vb0 = a.v_bias[h * HD + dA]; vb1 = a.v_bias[h * HD + dB]; }
    for (int b0 = b_lo + wave; b0 < b_hi; b0 += 8 * NB) {
      float rk0[NB], rk1[NB], rv0[NB], rv1[NB];
      float2 rcs[NB];
#pragma unroll
      for (int j = 0; j < NB; j++) {  // clamped rows: every load valid
        const int b = min(b0 + 8 * j, b_hi - 1);
        const float *kp = a.k + (int64_t)b * a.kv_dim + h * HD, *vp = a.v + (int64_t)b * a.kv_dim + h * HD;
        rk0[j] = kp[dA]; rk1[j] = kp[dB];
        rv0[j] = vp[dA]; rv1[j] = vp[dB];
        rcs[j] = a.rope[(int64_t)(start + b) * half + ln];
      }
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const int b = b0 + 8 * j, pos = start + b, pp = pos - p_lo;
        if (b >= b_hi) break;  // (uniform across the wavefront)
        float e0, e1;
        head_prep_pre(act ? rk0[j] : 0.0f, act ? rk1[j] : 0.0f, kb0, kb1, a.k_bias != nullptr, a.k_norm != nullptr, kn0, kn1, true, rcs[j].x,
                      rcs[j].y, HD, a.eps, e0, e1);
        if (act) {
          const __half k0 = __float2half_rn(e0), k1 = __float2half_rn(e1);
          ks[pp * KS + da] = (_Float16)__half2float(k0);
          ks[pp * KS + db] = (_Float16)__half2float(k1);
          if (zb == 0) { __half *kd = a.kc + cache0 + (int64_t)pos * a.kv_dim; kd[da] = k0; kd[db] = k1; }
        }
        head_prep_pre(act ? rv0[j] : 0.0f, act ? rv1[j] : 0.0f, vb0, vb1, a.v_bias != nullptr, false, 0.0f, 0.0f, false, 1.0f, 0.0f, HD, a.eps,
                      e0, e1);
        if (act) {
          const __half v0 = __float2half_rn(e0), v1 = __float2half_rn(e1);
          vt[da * VS + pp] = (_Float16)__half2float(v0);
          vt[db * VS + pp] = (_Float16)__half2float(v1);
          if (zb == 0) { __half *vd = a.vc + cache0 + (int64_t)pos * a.kv_dim; vd[da] = v0; vd[db] = v1; }
        }
      }
    }
  }

  __syncthreads();
  if (qa >= NQ) return;  // no tile (no barrier follows)

  // (6) scores S^T = K Q^T: sacc[pb] holds S[query ar][position 16 pb + kg + r]
  f4v sacc[4];
#pragma unroll
  for (int pb = 0; pb < 4; pb++) {
    sacc[pb] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kt = 0; kt < DT; kt++) {
      const h4v bk = *reinterpret_cast<const h4v *>(ks + (pb * 16 + ar) * KS + kt * 16 + kg);
      sacc[pb] = mfma16(bk, qhi[kt], sacc[pb]);
      sacc[pb] = mfma16(bk, qlo[kt], sacc[pb]);
    }
  }
  // (7) softmax of the chunk (the item's only sub-chunk: running max -inf, sum 0 before it)
  const int lim = qact ? min(p_hi, start + qi / g + 1) : p_lo;  // positions < lim are visible
  float sv[4][4], mx = -INFINITY;
#pragma unroll
  for (int pb = 0; pb < 4; pb++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int pos = p_lo + pb * 16 + kg + r;
      sv[pb][r] = pos < lim ? sacc[pb][r] * a.scale : -INFINITY;
      mx = fmaxf(mx, sv[pb][r]);
    }
  mx = max16(mx);
  mx = max32(mx);
  const float mn = fmaxf(-INFINITY, mx);
  float pv[4][4], ls4[4];
#pragma unroll
  for (int pb = 0; pb < 4; pb++) {
#pragma unroll
    for (int r = 0; r < 4; r++) pv[pb][r] = (sv[pb][r] == -INFINITY || mn == -INFINITY) ? 0.0f : expf(sv[pb][r] - mn);
    // wave_sum over positions (lane = position): bits 0, 1 in-lane, 2 lane ^ 16, 3 lane ^ 32
    ls4[pb] = (pv[pb][0] + pv[pb][1]) + (pv[pb][2] + pv[pb][3]);
    ls4[pb] = add16(ls4[pb]);
    ls4[pb] = add32(ls4[pb]);
  }
  const float ls = (ls4[0] + ls4[1]) + (ls4[2] + ls4[3]);  // position bits 4, 5
  const float al = mn == -INFINITY ? 1.0f : 0.0f;
  const float rl = 0.0f * al + ls;
  // (8) O = P V for every 16-dim tile (O starts at zero: attn_item's O * alpha is 0 here)
  h4v phv[4], plv[4];
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      _Float16 hh, ll;
      split_f16(pv[kt][r], hh, ll);
      phv[kt][r] = hh;
      plv[kt][r] = ll;
    }
  // partials written through the L2 (sc1): ~10 MB of them at M = 9 would otherwise sit dirty in
  // the eight L2s and be written back at the end of the launch, on the merge's critical path
  const rsrc_t r_ml = rsrc_of(a.part_ml + ((int64_t)h * a.nslot) * ATT_QMAX * 2);
  const rsrc_t r_o = rsrc_of(a.part_o + ((int64_t)h * a.nslot) * ATT_QMAX * HD);
#pragma unroll
  for (int dt = 0; dt < DT; dt++) {
    f4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
      const h4v bv = *reinterpret_cast<const h4v *>(vt + (dt * 16 + ar) * VS + kt * 16 + kg);
      acc = mfma16(phv[kt], bv, acc);
      acc = mfma16(plv[kt], bv, acc);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int q = qa + kg + r;
      if (q < NQ) st_coh1(r_o, ((c * ATT_QMAX + q) * HD + dt * 16 + ar) * 4, acc[r]);
    }
  }
  if (kq == 0 && qact) st_coh2(r_ml, (c * ATT_QMAX + qi) * 8, f2v{mn, rl});
}

// The merge of k_attn_mt's partials: one workgroup per (256 values of an att row, row); eight
// slices of 128 threads (two adjacent values each) merge chunk groups gs, gs + 8, .. (kd_merge's
// and attn_merge_q's operations per value: M = max, w = exp(m - M), L and O as fma chains in
// chunk order), then slice 0 merges the groups in group order, writes the att row and, when
// a.aq is set, the 256 values' Q8_K block (attn_tile_out's quantization).
template <int HD>
__global__ __launch_bounds__(1024) void k_attn_mrg(const AttnArgs a, const StepRec *st) {
  constexpr int NGS = 8, QPB = 256 / HD;
  __shared__ float sO[ATT_GMAX][256];
  __shared__ float sM[ATT_GMAX][QPB], sL[ATT_GMAX][QPB];
  __shared__ __align__(16) float sout[256];
  const int t = threadIdx.x, v = 2 * (t & 127), gs = t >> 7, b = blockIdx.y;
  const int qd = a.n_heads * HD, e = min(blockIdx.x * 256 + v, qd - 2);
  const int head = e / HD, d = e % HD, g = a.n_heads / a.n_kv, h = head / g, qi = b * g + head % g;
  const float2 *pml = reinterpret_cast<const float2 *>(a.part_ml) + (int64_t)h * a.nslot * ATT_QMAX + qi;
  const float2 *po = reinterpret_cast<const float2 *>(a.part_o + ((int64_t)h * a.nslot * ATT_QMAX + qi) * HD + d);
  // group gs's slots are requested before the step record arrives (slots past the pass's
  // chunks hold earlier values, never used)
  float2 ml0[ATT_GRP], ov0[ATT_GRP];
#pragma unroll
  for (int k = 0; k < ATT_GRP; k++) {
    const int c = min(gs * ATT_GRP + k, a.nslot - 1);
    ml0[k] = pml[(int64_t)c * ATT_QMAX];
    ov0[k] = po[(int64_t)c * ATT_QMAX * HD / 2];
  }
  const int total = st->start + st->m, nch = (total + 63) >> 6, ngrp = (nch + ATT_GRP - 1) / ATT_GRP;
  for (int gi = gs; gi < ngrp; gi += NGS) {
    const int s0 = gi * ATT_GRP, n = min(ATT_GRP, nch - s0);
    float2 ml[ATT_GRP], ov[ATT_GRP];
#pragma unroll
    for (int k = 0; k < ATT_GRP; k++) {
      if (gi == gs) {
        ml[k] = k < n ? ml0[k] : make_float2(-INFINITY, 0.0f);
        ov[k] = ov0[k];
      } else {
        const int c = s0 + min(k, n - 1);
        ml[k] = k < n ? pml[(int64_t)c * ATT_QMAX] : make_float2(-INFINITY, 0.0f);
        ov[k] = po[(int64_t)c * ATT_QMAX * HD / 2];
      }
    }
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < ATT_GRP; k++) M = fmaxf(M, ml[k].x);
    float L = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
    for (int k = 0; k < ATT_GRP; k++) {
      if (k < n) {
        const float w = ml[k].x == -INFINITY ? 0.0f : expf(ml[k].x - M);
        L = fmaf(ml[k].y, w, L);
        acc0 = fmaf(ov[k].x, w, acc0);
        acc1 = fmaf(ov[k].y, w, acc1);
      }
    }
    sO[gi][v] = acc0;
    sO[gi][v + 1] = acc1;
    if (d == 0) { sM[gi][v / HD] = M; sL[gi][v / HD] = L; }
  }
  __syncthreads();
  if (gs == 0) {
    const int hq = v / HD;
    float out[2];
    if (ngrp == 1) {
      const float il = __fdiv_rn(1.0f, fmaxf(sL[0][hq], 1e-30f));
      out[0] = sO[0][v] * il;
      out[1] = sO[0][v + 1] * il;
    } else {
      float M = -INFINITY;
      for (int k = 0; k < ngrp; k++) M = fmaxf(M, sM[k][hq]);
      float L = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
      for (int k = 0; k < ngrp; k++) {
        const float w = sM[k][hq] == -INFINITY ? 0.0f : expf(sM[k][hq] - M);
        L = fmaf(sL[k][hq], w, L);
        acc0 = fmaf(sO[k][v], w, acc0);
        acc1 = fmaf(sO[k][v + 1], w, acc1);
      }
      const float il = __fdiv_rn(1.0f, fmaxf(L, 1e-30f));
      out[0] = acc0 * il;
      out[1] = acc1 * il;
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
      if (blockIdx.x * 256 + v + u < qd) a.att[(int64_t)b * qd + blockIdx.x * 256 + v + u] = out[u];
      sout[v + u] = out[u];
    }
  }
  if (!a.aq.q) return;
  __syncthreads();
  if (t < 64) {  // the block's Q8_K (a.aq is set only when the att row is whole 256-blocks)
    const float4 xv = reinterpret_cast<const float4 *>(sout)[t];
    const float am = q8k_amax(xv);
    const int64_t vb = (int64_t)b * (qd / 256) + blockIdx.x;
    q8k_block_store(xv, am, a.aq.q + vb * 64, a.aq.d + vb, reinterpret_cast<int *>(a.aq.bs + vb * 8));
  }
}

// Row preparation of a prefill pass: one wavefront per (row b, head j); heads 0 .. n_heads-1
// are the queries (head_prep -> qp), then the n_kv keys (head_prep -> f16 RNE -> K cache) and
// the n_kv values (bias -> f16 -> V cache), the same operations as attn_item makes on them.
__global__ __launch_bounds__(64) void k_rows_prep(const AttnArgs a, float *qp, const StepRec *st) {
  const int b = blockIdx.x, j = blockIdx.y + (qp ? 0 : a.n_heads), lane = threadIdx.x & 63, hd = a.hd, half = hd >> 1;
  if (b >= st->m) return;
  const int pos = st->start + b;
  const int da = a.neox ? lane : 2 * lane, db = a.neox ? lane + half : 2 * lane + 1;
  const float2 *rope = a.rope + (int64_t)pos * half;
  float e0, e1;
  if (j < a.n_heads) {
    head_prep(a.q + ((int64_t)b * a.n_heads + j) * hd, a.q_bias ? a.q_bias + j * hd : nullptr, a.q_norm, rope, hd, a.neox, a.eps, e0, e1);
    if (lane < half) {
      float *o = qp + ((int64_t)b * a.n_heads + j) * hd;
      o[da] = e0;
      o[db] = e1;
    }
    return;
  }
  const int jj = j - a.n_heads, h = jj % a.n_kv;
  const bool is_k = jj < a.n_kv;
  if (is_k)
    head_prep(a.k + (int64_t)b * a.kv_dim + h * hd, a.k_bias ? a.k_bias + h * hd : nullptr, a.k_norm, rope, hd, a.neox, a.eps, e0, e1);
  else
    head_prep(a.v + (int64_t)b * a.kv_dim + h * hd, a.v_bias ? a.v_bias + h * hd : nullptr, nullptr, nullptr, hd, a.neox, a.eps, e0, e1);
  if (lane < half) {
    __half *d = (is_k ? a.kc : a.vc) + ((int64_t)a.layer * a.max_seq + pos) * a.kv_dim + h * hd;
    d[da] = __float2half_rn(e0);
    d[db] = __float2half_rn(e1);
  }
}

// ------------------------------------------------------------------ MoE router + routing
// F32 router rows (one per workgroup; wavefront w, lane j hold float4s w*64 + j + 256k of the
// row in registers; each vector's dot is the lane's fma chain, the wave tree, then the four
// wavefronts in order: a fixed order for every batch size, like matvec_multi's per-vector F32
// path :455-464), then the last workgroup routes, a wavefront per row: softmax (max, exp, sum, divide), top-n_used by
// probability (ties to the lower expert index), pruning (moe_prune >= 1: keep
// clamp(x, max(2, n/2), n); < 1: mass rule), weights p / sum(kept) when normalised
// (:1199-1239, :959-997), and the grouped job lists over the union of chosen experts in
// expert order, users in (row, slot) order (:982-986).
template <int MT>
__global__ __launch_bounds__(256) void k_router(const RouterArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];  // one-row passes with pro.nw: the normalised row
  __shared__ float part[4][MAX_M];
  const int m = st->m, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int dim = a.dim, n4 = dim >> 2, row = blockIdx.x;
  constexpr int NK = NORM_NT / 4;  // float4s per lane: wave w, lane j take float4s w*64 + j + 256k
  const float4 *wr = reinterpret_cast<const float4 *>(a.w.pl.p0 + (int64_t)row * dim * 4);
  const float4 *x4 = reinterpret_cast<const float4 *>(a.x);
  float4 wv[NK];
  NormRow<4> nr;
  if (MT == 1 && a.pro.nw) nr.load(a.pro);  // one-row passes: the input row normalised here
#pragma unroll
  for (int k = 0; k < NK; k++) {
    const int f = wave * 64 + lane + 256 * k;
    wv[k] = f < n4 ? wr[f] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (MT == 1 && a.pro.nw) {
    nr.finish(a.pro, reinterpret_cast<float *>(smem), nullptr);
    x4 = reinterpret_cast<const float4 *>(smem);
  }
  for (int v0 = 0; v0 < m; v0 += MT) {
    float pv[MT];
#pragma unroll
    for (int v = 0; v < MT; v++) {
      pv[v] = 0.0f;
      if (v0 + v < m) {
#pragma unroll
        for (int k = 0; k < NK; k++) {
          const int f = wave * 64 + lane + 256 * k;
          if (f < n4) {
            const float4 x = x4[(int64_t)(v0 + v) * n4 + f];
            pv[v] = fmaf(wv[k].x, x.x, pv[v]);
            pv[v] = fmaf(wv[k].y, x.y, pv[v]);
            pv[v] = fmaf(wv[k].z, x.z, pv[v]);
            pv[v] = fmaf(wv[k].w, x.w, pv[v]);
          }
        }
      }
    }
#pragma unroll
    for (int v = 0; v < MT; v++) {
      const float t = wave_sum(pv[v]);
      if (lane == 0 && v0 + v < m) part[wave][v0 + v] = t;
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < m) {
    const int v = threadIdx.x;
    st_dev(a.logits + (int64_t)v * a.n_expert + row, ((part[0][v] + part[1][v]) + part[2][v]) + part[3][v]);
  }
  if (a.logits_only) return;
  if (!arrive_last(a.counter, gridDim.x)) return;
  // routing: wave w takes rows w, w+4, ...; lane i < n_used ends up holding the row's i-th
  // choice (expert, probability)
  __shared__ signed char slot_of[MAX_M][256];  // slot of expert e among row b's kept choices, -1: none
  __shared__ int wcount[4];
  const int ne = a.n_expert, nu = a.n_used;
  for (int i = threadIdx.x; i < MAX_M * 256; i += 256) (&slot_of[0][0])[i] = -1;
  float lall[MAX_M / 4][4];  // logits of this wavefront's rows, all loaded in one round
#pragma unroll
  for (int rr = 0; rr < MAX_M / 4; rr++)
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int b = wave + 4 * rr, e = lane + 64 * k;
      lall[rr][k] = b < m && e < ne ? ld_dev(a.logits + (int64_t)b * ne + e) : -INFINITY;
    }
  __syncthreads();
#pragma unroll
  for (int rr = 0; rr < MAX_M / 4; rr++) {
    const int b = wave + 4 * rr;
    if (b >= m) break;
    float lv[4], mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; k++) { lv[k] = lall[rr][k]; mx = fmaxf(mx, lv[k]); }
    mx = wave_max(mx);
    float pv[4], sum = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) { const int e = lane + 64 * k; pv[k] = e < ne ? expf(lv[k] - mx) : 0.0f; sum += pv[k]; }
    sum = wave_sum(sum);
    // top-n_used by probability, ties to the lower expert index: repeated wave argmax over
    // keys (probability bits, ~index); a probability is >= 0, so its bits order as unsigned
    unsigned long long key[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int e = lane + 64 * k;
      if (e < ne) pv[k] = pv[k] / sum;
      key[k] = e < ne ? ((unsigned long long)__float_as_uint(pv[k]) << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)e) : 0ull;
    }
    int my_e = 0;
    float my_p = 0.0f;
    for (int i = 0; i < nu; i++) {
      unsigned long long bk = key[0];
#pragma unroll
      for (int k = 1; k < 4; k++) bk = key[k] > bk ? key[k] : bk;
      bk = wave_max_u64(bk);
      const int e = (int)(0xFFFFFFFFu - (unsigned)(bk & 0xFFFFFFFFull));
      if (lane == i) { my_e = e; my_p = __uint_as_float((uint32_t)(bk >> 32)); }
      if ((e & 63) == lane) key[e >> 6] = 0ull;
    }
    // pruning and the normalising sum, in choice order (the reference's sequential sums)
    int keep = nu;
    if (a.moe_prune > 0.0f && nu > 2) {
      const int min_keep = max(2, nu / 2);
      if (a.moe_prune >= 1.0f) keep = min(max((int)a.moe_prune, min_keep), nu);
      else {
        float top = 0.0f;
        for (int i = 0; i < nu; i++) top += __shfl(my_p, i);
        const float target = top * (1.0f - a.moe_prune);
        float cum = 0.0f;
        int k = 0;
        while (k < nu && (k < min_keep || cum < target)) { cum += __shfl(my_p, k); k++; }
        keep = k;
      }
    }
    float wsum = 0.0f;
    for (int i = 0; i < keep; i++) wsum += __shfl(my_p, i);
    if (lane < keep) {
      a.chosen[b * 32 + lane] = my_e;
      a.weights[b * 32 + lane] = a.norm ? my_p / wsum : my_p;
      slot_of[b][my_e] = (signed char)lane;
    }
    if (lane == 0) a.nkeep[b] = keep;
  }
  __syncthreads();
  // jobs: experts with at least one user, in expert order (thread e = expert e); users in
  // row order (a row chooses an expert at most once). Down jobs (jobs[256 + j]) hold all of
  // an expert's users; gate/up jobs (jobs[0 ..]) at most GU_USERS each, an expert's users in
  // consecutive jobs.
  __shared__ int ssub[4];
  const int e = threadIdx.x;
  int cnt = 0;
  if (e < ne)
    for (int b = 0; b < m; b++) cnt += slot_of[b][e] >= 0;
  const int nsj = (cnt + GU_USERS - 1) / GU_USERS;
  int incl = nsj;  // inclusive scan of the gate/up job counts over the wavefront
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(incl, d);
    if (lane >= d) incl += t;
  }
  const unsigned long long bal = __ballot(cnt > 0);
  if (lane == 0) wcount[wave] = __popcll(bal);
  if (lane == 63) ssub[wave] = incl;
  __syncthreads();
  int base = 0, sbase = 0;
  for (int w = 0; w < wave; w++) { base += wcount[w]; sbase += ssub[w]; }
  if (cnt > 0) {
    const int j = base + __popcll(bal & ((1ull << lane) - 1ull));
    Job &Jd = a.jobs[256 + j];
    int k = 0, sj = sbase + incl - nsj, ks = 0;
    for (int b = 0; b < m; b++) {
      const int s = slot_of[b][e];
      if (s >= 0) {
        Jd.vec[k] = b * nu + s;
        Jd.out[k] = b * nu + s;
        k++;
        Job &J = a.jobs[sj];
        J.vec[ks] = b;
        J.out[ks] = b * nu + s;
        if (++ks == GU_USERS) { J.expert = e; J.nvec = ks; sj++; ks = 0; }
      }
    }
    if (ks > 0) { a.jobs[sj].expert = e; a.jobs[sj].nvec = ks; }
    Jd.expert = e;
    Jd.nvec = k;
    if (a.expert_count) a.expert_count[e] += 1;
  }
  if (threadIdx.x == 0) {
    a.njobs[0] = wcount[0] + wcount[1] + wcount[2] + wcount[3];
    a.njobs[1] = ssub[0] + ssub[1] + ssub[2] + ssub[3];
  }
}

// ------------------------------------------------------------------ gate / up + SwiGLU
// h = silu(g) * u (silu :586-588, ffns_fused :407-417) for the rows of one job. With hq, the
// last of the workgroups that cover a 256-row block of h quantizes it (Q8_K for an integer
// down projection, :420-424). rpw = rows of h per workgroup. The arrivals of a block's
// workgroups are counted in two levels (GU_SUB sub-counters, then one top counter, each on
// its own 128-byte line) so that no counter takes more than a few atomics; the counters are
// left at zero for the next pass.
__device__ __forceinline__ void gateup_quant_tail(const GUArgs &a, int nvec, const int *jo, int rpw) {
  __shared__ int quant_u[MAX_M];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n_ff = a.n_ff, nbh = n_ff / 256, per = 256 / rpw, blk = blockIdx.x / per, sub = (blockIdx.x % per) % GU_SUB;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if ((int)threadIdx.x < nvec) {
    const int vo = jo ? jo[threadIdx.x] : threadIdx.x;
    int *base = a.counter + (int64_t)(vo * nbh + blk) * (1 + GU_SUB) * CNT_STRIDE;
    int *sc = base + (1 + sub) * CNT_STRIDE;
    int last = 0;
    if (atomicAdd(sc, 1) == per / GU_SUB - 1) {
      *sc = 0;
      last = atomicAdd(base, 1) == GU_SUB - 1;
      if (last) *base = 0;
    }
    quant_u[threadIdx.x] = last;
  }
  __syncthreads();
  for (int u = wave; u < nvec; u += (int)(blockDim.x >> 6)) {
    if (!quant_u[u]) continue;
    const int vo = jo ? jo[u] : u;
    const float *hp = a.h + (int64_t)vo * n_ff + blk * 256 + 4 * lane;
    const float4 xv = make_float4(ld_dev(hp), ld_dev(hp + 1), ld_dev(hp + 2), ld_dev(hp + 3));
    const float am = q8k_amax(xv);
    const int64_t vb = (int64_t)vo * nbh + blk;
    q8k_block_store(xv, am, a.hq.q + vb * 64, a.hq.d + vb, reinterpret_cast<int *>(a.hq.bs + vb * 8));
  }
}

struct GUJob {
  int expert, nvec;
  const int *jv, *jo;
};
__device__ __forceinline__ bool gu_job(const GUArgs &a, int m, GUJob &j) {
  j.expert = 0; j.nvec = m; j.jv = nullptr; j.jo = nullptr;
  if (!a.jobs) return true;
  const Job &J = a.jobs[blockIdx.y];  // always addressable: loaded together with the job count
  j.expert = J.expert; j.nvec = J.nvec; j.jv = J.vec; j.jo = J.out;
  return (int)blockIdx.y < *a.njobs;
}

// The job of a gate / up workgroup: from the router's job list (gu_job), or, for one-row float
// passes with a.rt.logits, routed here (route_row in wavefront 0; the workgroup takes the job of
// rank blockIdx.y among the kept choices in expert order; workgroup (0, 0) publishes the
// choices, weights, keep count, down jobs and selection counts). s_route: two LDS ints.
// False: the workgroup has no job (every thread returns).
__device__ __forceinline__ bool gu_job_one(const GUArgs &a, int m, bool one_row, GUJob &J, int *s_route) {
  if (!(one_row && a.rt.logits)) return gu_job(a, m, J);
  const F1Route &rt = a.rt;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    float lv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) lv[k] = lane + 64 * k < rt.n_expert ? rt.logits[lane + 64 * k] : -INFINITY;
    int my_e, keep;
    float my_p, wsum;
    route_row(lv, rt.n_expert, rt.n_used, rt.moe_prune, my_e, my_p, keep, wsum);
    int rank = 0;  // among the kept choices by expert index: the job order
    for (int i = 0; i < keep; i++) rank += __shfl(my_e, i) < my_e ? 1 : 0;
    if (lane == 0) s_route[0] = -1;
    __builtin_amdgcn_wave_barrier();
    if (lane < keep && rank == (int)blockIdx.y) { s_route[0] = my_e; s_route[1] = lane; }
    if (blockIdx.x == 0 && blockIdx.y == 0) {
      if (lane < keep) {
        rt.chosen[lane] = my_e;
        rt.weights[lane] = rt.norm ? my_p / wsum : my_p;
        Job &Jd = rt.jobs[rank];
        Jd.expert = my_e;
        Jd.nvec = 1;
        Jd.vec[0] = lane;
        Jd.out[0] = lane;
        if (rt.expert_count) rt.expert_count[my_e] += 1;
      }
      if (lane == 0) { rt.nkeep[0] = keep; rt.njobs[0] = keep; rt.njobs[1] = keep; }
    }
  }
  __syncthreads();
  if (s_route[0] < 0) return false;
  J.expert = s_route[0];
  J.nvec = 1;
  J.jv = nullptr;
  J.jo = s_route + 1;
  return true;
}

// Integer, eight rows per wavefront: 16 rows of h per workgroup; in each wavefront slots 0-3
// are gate rows r..r+3 and slots 4-7 the same rows of up.
template <int T, int MT>
__global__ __launch_bounds__(256) void k_gateup_kq(const GUArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];
  GUJob J;
  if (!gu_job(a, st->m, J)) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, slot = lane >> 3, l = lane & 7;
  const int nb = (int)a.gate.nb, n_ff = a.n_ff, dim = (int)a.gate.cols;
  const int rb = blockIdx.x * 16 + wave * 4;
  const int64_t eb = (int64_t)J.expert * a.gate.rows;
  constexpr bool ST = MT <= 2;  // activations staged in LDS (small m); else read through the caches
  const Q8KP ly = ST ? ldsq_of(smem, MT, dim) : a.y;
  uint8_t *tile = smem + (ST ? ldsq_bytes(MT, dim) : 0) + (size_t)wave * 8 * nb * tile_bpb();
  tile_fetch<T>(tile, a.gate.pl, 8, nb, [&](int sl) -> int64_t { return sl < 4 && rb + sl < n_ff ? eb + rb + sl : -1; });
  tile_fetch<T>(tile, a.up.pl, 8, nb, [&](int sl) -> int64_t { return sl >= 4 && rb + sl - 4 < n_ff ? eb + rb + sl - 4 : -1; });
  if (ST) stage_q8kp(ly, a.y, dim, J.nvec, 4, [&](int u) { return J.jv ? J.jv[u] : u; });
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int r = rb + (slot & 3);
  const bool valid = r < n_ff;
  int vidx[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) vidx[v] = ST ? v : (J.jv && v < J.nvec ? J.jv[v] : v);
  float res[MT];
  kq_walk_tile<T, MT>(tile, 8, nb, slot, eb + (valid ? r : n_ff - 1), ly, vidx, J.nvec, l, res);
#pragma unroll
  for (int v = 0; v < MT; v++) {
    const float u = __shfl_down(res[v], 32);
    if (slot < 4 && l == 0 && valid && v < J.nvec) {
      const float x = res[v];
      st_dev(a.h + (int64_t)(J.jo ? J.jo[v] : v) * n_ff + r, x / (1.0f + expf(-x)) * u);
    }
  }
  if (a.hq.q) gateup_quant_tail(a, J.nvec, J.jo, 16);
}

// Integer, row-parallel: one row of h per wavefront, four per workgroup; slot 0 is the gate
// row, slot 1 the up row, four lane groups each. m <= 2 stages the job's vectors in LDS.
template <int T, int MT>
__global__ __launch_bounds__(256) void k_gateup_rp(const GUArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr bool ST = MT <= 2;
  GUJob J;
  if (!gu_job(a, st->m, J)) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nb = (int)a.gate.nb, n_ff = a.n_ff, dim = (int)a.gate.cols;
  const int r = blockIdx.x * 4 + wave;
  const bool valid = r < n_ff;
  const int64_t grow = (int64_t)J.expert * a.gate.rows + (valid ? r : n_ff - 1);
  const Q8KP ly = ST ? ldsq_of(smem, MT, dim) : a.y;
  uint8_t *tile = smem + rp_act_bytes(MT, dim) + (size_t)wave * rp_wave_bytes(2, nb, MT);
  float *cb = reinterpret_cast<float *>(tile + (size_t)2 * nb * tile_bpb());
  float *ov = cb + (size_t)2 * nb * MT * 10;
  tile_fetch<T>(tile, a.gate.pl, 2, nb, [&](int sl) -> int64_t { return sl == 0 ? grow : -1; });
  tile_fetch<T>(tile, a.up.pl, 2, nb, [&](int sl) -> int64_t { return sl == 1 ? grow : -1; });
  if (ST) stage_q8kp(ly, a.y, dim, J.nvec, 4, [&](int u) { return J.jv ? J.jv[u] : u; });
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int nv = J.nvec;
  const int *jv = J.jv;
  auto vid = [&](int, int v) { return ST || !jv ? v : jv[v]; };
  kq_rows_par<T, MT>(tile, 2, nb, 4, 2, [&](int) { return grow; }, vid, [&](int) { return nv; }, ly, cb, ov);
  if (lane < nv && valid) {
    const float x = ov[lane], u = ov[MT + lane];
    st_dev(a.h + (int64_t)(J.jo ? J.jo[lane] : lane) * n_ff + r, x / (1.0f + expf(-x)) * u);
  }
  if (a.hq.q) gateup_quant_tail(a, nv, J.jo, 4);
}

// Float weights (Q8_0 / Q5_0) x fp32 activations: 16 rows of h per workgroup.
template <int T, int MT>
__global__ __launch_bounds__(256) void k_gateup_f(const GUArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];  // one-row passes with pro.nw: the normalised row
  GUJob J;
  __shared__ int s_route[2];  // this workgroup's job: expert (-1: none), slot
  NormRow<4> nr;
  if (MT == 1 && a.pro.nw) nr.load(a.pro);  // (in flight during the routing)
  if (!gu_job_one(a, st->m, MT == 1, J, s_route)) return;
  constexpr int D = f_depth<MT>();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, slot = lane >> 3, l = lane & 7;
  const TensorView &w = slot < 4 ? a.gate : a.up;
  const int nb = (int)w.nb, n_ff = a.n_ff;
  const int r = blockIdx.x * 16 + wave * 4 + (slot & 3);
  const bool valid = r < n_ff;
  const int64_t grow = (int64_t)J.expert * w.rows + (valid ? r : n_ff - 1);
  const Planes pl = slot < 4 ? a.gate.pl : a.up.pl;
  int vidx[MT];
#pragma unroll
  for (int v = 0; v < MT; v++) vidx[v] = J.jv && v < J.nvec ? J.jv[v] : v;
  float res[MT];
  if (MT == 1 && a.pro.nw) {  // the input row normalised here, once the first weights are requested
    float *lx = reinterpret_cast<float *>(smem);
    f_walk<T, MT, D>(pl, grow, nb, lx, w.cols, vidx, J.nvec, l, res, [&]() { nr.finish(a.pro, lx, nullptr); });
  } else {
    f_walk<T, MT, D>(pl, grow, nb, a.x, w.cols, vidx, J.nvec, l, res);
  }
#pragma unroll
  for (int v = 0; v < MT; v++) {
    const float u = __shfl_down(res[v], 32);
    if (slot < 4 && l == 0 && valid && v < J.nvec) {
      const float x = res[v];
      st_dev(a.h + (int64_t)(J.jo ? J.jo[v] : v) * n_ff + r, x / (1.0f + expf(-x)) * u);
    }
  }
  if (a.hq.q) gateup_quant_tail(a, J.nvec, J.jo, 16);
}

// Gate / up + SwiGLU of one row over Q8_0 weights with k_mv_f1's arithmetic spread over the
// wavefront (the bits of k_gateup_f's f_walk): a workgroup takes H = 16 / S h rows of one job
// (S = 8 / RW workgroups a 16-row block), wavefronts 0-1 their gate rows, 2-3 the same up rows,
// RW rows a wavefront, each wavefront's (row, block) items spread over its lanes with (d, dot)
// parked in LDS, then each row's eight block chains and the 8-lane tree; the 2H results meet in
// LDS and H lanes write silu(g) u. The job and the input row as in k_gateup_f.
template <int NI, int RW>
__global__ __launch_bounds__(MVF1_NW * 64) void k_gateup_f1(const GUArgs a, const StepRec *st) {
  constexpr int S = 8 / RW, H = 2 * RW;
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int s_route[2];
  __shared__ float sgu[2][H];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nb = (int)a.gate.nb, cols = 32 * nb, ni = RW * nb, n_ff = a.n_ff;
  float *lx = reinterpret_cast<float *>(smem);
  float2 *ldd = reinterpret_cast<float2 *>(smem + (size_t)cols * 4) + (size_t)wave * ni;  // (d, dot) [row][block]
  NormRow<MVF1_NW> nr;
  if (a.pro.nw) nr.load(a.pro);  // (in flight during the routing)
  GUJob J;
  if (!gu_job_one(a, st->m, true, J, s_route)) return;
  const int half = wave >> 1, sub = (int)blockIdx.x % S, blk = (int)blockIdx.x / S;
  const int64_t hr0 = (int64_t)blk * 16 + sub * H + (wave & 1) * RW;  // this wavefront's first h row
  const TensorView &w = half ? a.up : a.gate;
  const int64_t ebase = (int64_t)J.expert * w.rows;
  uint4 c0[NI], c1[NI];
  uint32_t dh[NI];
#pragma unroll
  for (int k = 0; k < NI; k++) {
    const int i = min(lane + 64 * k, ni - 1), r = i / nb, b = i - r * nb;
    const int64_t g = (ebase + min(hr0 + r, (int64_t)n_ff - 1)) * nb + b;
    c0[k] = ld16(w.pl.p0 + g * 32);
    c1[k] = ld16(w.pl.p0 + g * 32 + 16);
    dh[k] = *reinterpret_cast<const uint16_t *>(w.pl.p3 + g * 2);
  }
  if (a.pro.nw) {
    nr.finish(a.pro, lx, nullptr);
  } else {
    for (int i = threadIdx.x; i < cols / 4; i += MVF1_NW * 64) reinterpret_cast<float4 *>(lx)[i] = reinterpret_cast<const float4 *>(a.x)[i];
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < NI; k++) {
    const int i = lane + 64 * k;
    if (i < ni) {
      const int b = i % nb;
      const float4 *xv = reinterpret_cast<const float4 *>(lx + 32 * b);
      const uint32_t cw[8] = {c0[k].x, c0[k].y, c0[k].z, c0[k].w, c1[k].x, c1[k].y, c1[k].z, c1[k].w};
      float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
      for (int kk = 0; kk < 8; kk++) {
        const float4 xx = xv[kk];
        s0 = fmaf((float)(int8_t)(cw[kk]), xx.x, s0);
        s1 = fmaf((float)(int8_t)(cw[kk] >> 8), xx.y, s1);
        s2 = fmaf((float)(int8_t)(cw[kk] >> 16), xx.z, s2);
        s3 = fmaf((float)(int8_t)(cw[kk] >> 24), xx.w, s3);
      }
      ldd[i] = make_float2(h2f(dh[k]), (s0 + s1) + (s2 + s3));
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the items are parked
  __builtin_amdgcn_wave_barrier();
  const int r = lane >> 3, l = lane & 7;
  float acc = 0.0f;
  if (r < RW)
    for (int b = l; b < nb; b += 8) {
      const float2 e = ldd[r * nb + b];
      acc = fmaf(e.x, e.y, acc);
    }
  const float res = hsum_rows8(acc);
  if (r < RW && l == 0) sgu[half][(wave & 1) * RW + r] = res;
  __syncthreads();
  if ((int)threadIdx.x < H) {
    const int64_t row = (int64_t)blk * 16 + sub * H + threadIdx.x;
    const float x = sgu[0][threadIdx.x], u = sgu[1][threadIdx.x];
    if (row < n_ff) st_dev(a.h + (int64_t)(J.jo ? J.jo[0] : 0) * n_ff + row, x / (1.0f + expf(-x)) * u);
  }
}

// Gate / up + SwiGLU of 2..16 rows on the fp32 matrix cores (Q8_0), dense or one routed expert's
// users a job (vdiv: the down jobs, whose entries are h indices): 16 rows of h per workgroup of
// sixteen wavefronts: wavefront w takes part w >> 1 (fq_part) of the gate tile
// (w even) or the up tile (w odd); the parts meet in LDS (summed in part order) and
// h = silu(g) * u as k_gateup_f writes it.
__global__ __launch_bounds__(1024) void k_gateup_fq(const GUArgs a, const StepRec *st) {
  GUJob J;
  if (!gu_job(a, st->m, J)) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 15, kq = lane >> 4, mat = wave & 1, kp = wave >> 1;
  __shared__ float part[FQ_KP][2][4][64];
  const TensorView &w = mat ? a.up : a.gate;
  const int nb = (int)w.nb, n_ff = a.n_ff;
  const int64_t r0 = (int64_t)blockIdx.x * 16, grow = (int64_t)J.expert * w.rows + min(r0 + j, (int64_t)n_ff - 1);
  const bool vin = j < J.nvec;
  const int xv = vin ? (J.jv ? (a.vdiv > 1 ? J.jv[j] / a.vdiv : J.jv[j]) : j) : 0;
  float r[4];
  fq_part(w.pl.p0 + grow * nb * 32 + 8 * kq, reinterpret_cast<const uint16_t *>(w.pl.p3) + grow * nb, a.x + (int64_t)xv * w.cols + 8 * kq,
          vin, nb, kp, r);
#pragma unroll
  for (int q = 0; q < 4; q++) part[kp][mat][q][lane] = r[q];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int v = 4 * kq + q;
      const int64_t row = r0 + j;
      if (v < J.nvec && row < n_ff) {
        float g = part[0][0][q][lane], u = part[0][1][q][lane];
#pragma unroll
        for (int p2 = 1; p2 < FQ_KP; p2++) { g = g + part[p2][0][q][lane]; u = u + part[p2][1][q][lane]; }
        st_dev(a.h + (int64_t)(J.jo ? J.jo[v] : v) * n_ff + row, g / (1.0f + expf(-g)) * u);
      }
    }
  }
  if (a.hq.q) gateup_quant_tail(a, J.nvec, J.jo, 16);
}

// ------------------------------------------------------------------ down + combine
// One output row per wavefront; row slots take jobs eight at a time; each job's users get
// y_e[r] in LDS, then out[b][r] = sum over b's chosen slots, in chosen order, of w * y
// (non-fused multiply and add, ffns_fused :432-437, moe_forward_batch :1133-1140). With a
// tail, the outputs are stored coherently and the last workgroup runs it.
__device__ __forceinline__ void down_combine(const DownArgs &a, int m, float (*yb)[MAX_M * 32], int64_t r, int dim, bool coh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (r < dim && lane < m) {
    const int b = lane, nk = a.nkeep[b];
    float acc = 0.0f;
    for (int i = 0; i < nk; i++) acc = acc + a.weights[b * 32 + i] * yb[wave][b * a.n_used + i];
    out_store(a.out + (int64_t)b * dim + r, acc, coh);
    if (a.res_out) a.res_out[(int64_t)b * dim + r] = a.res_in[(int64_t)b * dim + r] + a.rscale * acc;
  }
}

template <int T, int MT, bool STAGE>
__global__ __launch_bounds__(256) void k_down_kq(const DownArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float yb[4][MAX_M * 32];
  const int m = st->m, nj = *a.njobs;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, slot = lane >> 3, l = lane & 7;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave;
  const int dim = (int)a.w.rows, nb = (int)a.w.nb, n_ff = (int)a.w.cols;
  const bool valid = r < dim;
  const bool coh = a.tail.nw != nullptr;
  const int npairs = m * a.n_used;
  const Q8KP ly = ldsq_of(smem, STAGE ? MT * a.n_used : 0, n_ff);
  uint8_t *tile = smem + (STAGE ? ldsq_bytes(MT * a.n_used, n_ff) : 0) + (size_t)wave * 8 * nb * tile_bpb();
  for (int j0 = 0; j0 < nj; j0 += 8) {
    const int j = j0 + slot;
    const bool has = j < nj;
    const Job &J = a.jobs[has ? j : 0];
    // lane s < 8 holds slot s's expert (the job array is always addressable, so this load
    // need not wait for the job count)
    const int ex = a.jobs[j0 + (lane & 7)].expert;
    tile_fetch<T>(tile, a.w.pl, 8, nb, [&](int sl) -> int64_t {
      const int e = __shfl(ex, sl);
      return j0 + sl < nj && valid ? (int64_t)e * dim + r : -1;
    });
    if (STAGE && j0 == 0) stage_q8kp(ly, a.y, n_ff, npairs, 4, [](int u) { return u; });
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int nvec = has ? J.nvec : 0;
    int vidx[MT];
#pragma unroll
    for (int v = 0; v < MT; v++) vidx[v] = v < nvec ? J.vec[v] : 0;
    float res[MT];
    kq_walk_tile<T, MT>(tile, 8, nb, slot, (int64_t)J.expert * dim + (valid ? r : 0), STAGE ? ly : a.y, vidx, nvec, l, res);
    if (l == 0) {
#pragma unroll
      for (int v = 0; v < MT; v++)
        if (v < nvec) yb[wave][J.out[v]] = res[v];
    }
    __syncthreads();
  }
  down_combine(a, m, yb, r, dim, coh);
  if (coh && arrive_last(a.tail.counter, gridDim.x)) norm_rows<4>(a.tail, 0, m);
}

// Verify / prefill passes: one output row per workgroup; its four wavefronts take the jobs in
// rounds of eight (slot = job), then the row's combine as above.
template <int T, int MT>
__global__ __launch_bounds__(256) void k_down_rj(const DownArgs a, const StepRec *st) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float yb[MAX_M * 32];
  const int m = st->m, nj = *a.njobs;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, slot = lane >> 3, l = lane & 7;
  const int64_t r = blockIdx.x;
  const int dim = (int)a.w.rows, nb = (int)a.w.nb;
  const bool coh = a.tail.nw != nullptr;
  uint8_t *tile = smem + (size_t)wave * 8 * nb * tile_bpb();
  for (int j0 = wave * 8; j0 < nj; j0 += 32) {
    const int j = j0 + slot;
    const bool has = j < nj;
    const Job &J = a.jobs[has ? j : 0];
    const int ex = a.jobs[min(j0 + (lane & 7), 255)].expert;
    tile_fetch<T>(tile, a.w.pl, 8, nb, [&](int sl) -> int64_t {
      const int e = __shfl(ex, sl);
      return j0 + sl < nj ? (int64_t)e * dim + r : -1;
    });
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    const int nvec = has ? J.nvec : 0;
    int vidx[MT];
#pragma unroll
    for (int v = 0; v < MT; v++) vidx[v] = v < nvec ? J.vec[v] : 0;
    float res[MT];
    kq_walk_tile<T, MT>(tile, 8, nb, slot, (int64_t)J.expert * dim + r, a.y, vidx, nvec, l, res);
    if (l == 0) {
#pragma unroll
      for (int v = 0; v < MT; v++)
        if (v < nvec) yb[J.out[v]] = res[v];
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();  // the tile is refilled next round
  }
  __syncthreads();
  if ((int)threadIdx.x < m) {
    const int b = threadIdx.x, nk = a.nkeep[b];
    float acc = 0.0f;
    for (int i = 0; i < nk; i++) acc = acc + a.weights[b * 32 + i] * yb[b * a.n_used + i];
    out_store(a.out + (int64_t)b * dim + r, acc, coh);
  }
  if (coh && arrive_last(a.tail.counter, gridDim.x)) norm_rows<4>(a.tail, 0, m);
}

template <int T, int MT>
__global__ __launch_bounds__(256) void k_down_f(const DownArgs a, const StepRec *st) {
  __shared__ float yb[4][MAX_M * 32];
  const int m = st->m, nj = *a.njobs;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, slot = lane >> 3, l = lane & 7;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave;
  const int dim = (int)a.w.rows, nb = (int)a.w.nb;
  const bool valid = r < dim;
  const bool coh = a.tail.nw != nullptr;
  constexpr int D = f_depth<MT>();
  for (int j0 = 0; j0 < nj; j0 += 8) {
    const int j = j0 + slot;
    const bool has = j < nj;
    const Job &J = a.jobs[has ? j : 0];
    const int nvec = has ? J.nvec : 0;
    const int64_t grow = (int64_t)J.expert * dim + (valid ? r : 0);
    int vidx[MT];
#pragma unroll
    for (int v = 0; v < MT; v++) vidx[v] = v < nvec ? J.vec[v] : 0;
    float res[MT];
    f_walk<T, MT, D>(a.w.pl, grow, nb, a.x, a.w.cols, vidx, nvec, l, res);
    if (l == 0) {
#pragma unroll
      for (int v = 0; v < MT; v++)
        if (v < nvec) yb[wave][J.out[v]] = res[v];
    }
  }
  __syncthreads();
  down_combine(a, m, yb, r, dim, coh);
  if (coh && arrive_last(a.tail.counter, gridDim.x)) norm_rows<4>(a.tail, 0, m);
}

// Routed experts' down projection of 2..16 rows on the fp32 matrix cores (Q8_0): workgroup
// (32 output rows, down job) of sixteen wavefronts as k_mv_fq's (tile w & 1, part w >> 1, the
// parts summed in part order), the job's users' h rows as the vectors; y of (user, row) goes to
// yd through the L2. The last of a row block's job workgroups combines its 32 rows for every
// pass row in choice order (down_combine's arithmetic), and the last row block runs the norm
// tail.
__global__ __launch_bounds__(1024) void k_down_fq(const DownArgs a, const StepRec *st) {
  const int m = st->m, nj = *a.njobs;
  if ((int)blockIdx.y >= nj) return;
  const Job &J = a.jobs[blockIdx.y];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, j = lane & 15, kq = lane >> 4;
  const int tile = wave & 1, kp = wave >> 1;
  __shared__ float part[FQ_KP][2][4][64];
  const int dim = (int)a.w.rows, nb = (int)a.w.nb, n_ff = (int)a.w.cols;
  const bool coh = a.tail.nw != nullptr;
  const int nvec = J.nvec;
  const bool vin = j < nvec;
  const int xv = vin ? J.vec[j] : 0;
  const int64_t r0 = (int64_t)blockIdx.x * 32 + tile * 16;
  float r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (r0 < dim) {
    const int64_t grow = (int64_t)J.expert * dim + min(r0 + j, (int64_t)dim - 1);
    fq_part(a.w.pl.p0 + grow * nb * 32 + 8 * kq, reinterpret_cast<const uint16_t *>(a.w.pl.p3) + grow * nb, a.x + (int64_t)xv * n_ff + 8 * kq,
            vin, nb, kp, r);
  }
#pragma unroll
  for (int q = 0; q < 4; q++) part[kp][tile][q][lane] = r[q];
  __syncthreads();
  const rsrc_t ry = rsrc_of(a.yd);
  if (kp == 0 && r0 < dim) {
    const int64_t row = r0 + j;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int v = 4 * kq + q;
      float res = part[0][tile][q][lane];
#pragma unroll
      for (int p2 = 1; p2 < FQ_KP; p2++) res = res + part[p2][tile][q][lane];
      if (v < nvec && row < dim) st_coh1(ry, (int)(((int64_t)J.out[v] * dim + row) * 4), res);
    }
  }
  int *tc = a.counter + (int64_t)(1 + blockIdx.x) * CNT_STRIDE;
  if (arrive(tc) != nj - 1) return;
  if (threadIdx.x == 0) *tc = 0;
  for (int i = threadIdx.x; i < m * 32; i += 1024) {
    const int b = i >> 5, row = blockIdx.x * 32 + (i & 31);
    if (row < dim) {
      const int nk = a.nkeep[b];
      float acc = 0.0f;
      for (int s2 = 0; s2 < nk; s2++) acc = acc + a.weights[b * 32 + s2] * ld_coh1(ry, (int)(((int64_t)(b * a.n_used + s2) * dim + row) * 4));
      out_store(a.out + (int64_t)b * dim + row, acc, coh);
    }
  }
  if (!coh) return;
  if (arrive(a.counter) != (int)gridDim.x - 1) return;
  if (threadIdx.x == 0) *a.counter = 0;
  norm_rows<16>(a.tail, 0, m);
}

// ------------------------------------------------------------------ final greedy pick
// With hist (one-row decode passes replayed back to back): the pick also becomes the next
// pass's token at the next position, and is appended to hist.
__global__ __launch_bounds__(256) void k_argmax_final(const unsigned long long *best, int nbest, int *out, StepRec *st, int *hist) {
  const int b = blockIdx.x;
  if (st && b >= st->m) return;
  unsigned long long v = 0;
  for (int i = threadIdx.x; i < nbest; i += 256) { const unsigned long long w = best[(int64_t)b * nbest + i]; v = w > v ? w : v; }
  v = wave_max_u64(v);
  __shared__ unsigned long long sb[4];
  if ((threadIdx.x & 63) == 0) sb[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long r = sb[0];
    for (int w = 1; w < 4; w++) r = sb[w] > r ? sb[w] : r;
    const int tok = (int)(uint32_t)(r & 0xffffffffull);
    out[b] = tok;
    if (hist) {
      hist[st->step] = tok;
      st->step += 1;
      st->ids[0] = tok;
      st->start += 1;
    }
  }
}

// ------------------------------------------------------------------ launchers
static inline int bucket(int m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : 16; }
static inline bool kq_type(int dt) { return dt == T_Q4K || dt == T_Q6K; }

// Rows per workgroup: float 32 (4 waves x 8), tiles 8 (1 wave), row-parallel 4R.
int mv_wgs(int64_t rows, int mt, int mode, int dtype, int R) {
  (void)mt;
  const int64_t per = !kq_type(dtype) ? 32 : mode == 1 ? 4 * R : 8;
  return (int)((rows + per - 1) / per);
}

static int mv_total(const MVArgs &a) {
  int t = 0;
  for (int i = 0; i < a.nseg; i++) t += a.seg[i].wgs;
  return t;
}

#define SPX_LDS(kern, sm) \
  if ((sm) > 65536) (void)hipFuncSetAttribute((const void *)(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)(sm))

static int cu_count_f() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
  }
  return n;
}

hipError_t launch_mv(const MVArgs &a, int mt, int mode, const StepRec *st, int grid, hipStream_t s) {
  mt = bucket(mt);
  const int dt = a.seg[0].w.dtype, cols = (int)a.seg[0].w.cols, nb = cols / 256;
  if (grid < 1) return hipErrorInvalidValue;
  const bool f1_only = a.pro.nw || a.res_out;  // prologue norm / residual epilogue: k_mv_f1 only
  if (f1_only && (kq_type(dt) || mt != 1 || (a.res_out && a.nseg != 1))) return hipErrorInvalidValue;
  if (!kq_type(dt)) {
    bool fq = a.fq && a.m >= FQ_MIN_ROWS;
    for (int i = 0; i < a.nseg; i++) fq = fq && a.seg[i].w.dtype == T_Q8_0;
    if (fq) {
      // one tile a workgroup (two tiles: Qwen3-0.6B M = 9 2.82 vs 2.26 ms a pass): twice the
      // workgroups when the grid covers the tasks, else the same grid (greedy-key slots follow it)
      hipLaunchKernelGGL(k_mv_fq<1>, dim3(!a.best && grid == mv_total(a) ? 2 * grid : grid), dim3(512), 0, s, a, st);
      return hipGetLastError();
    }
    if (mt == 1) {  // one row over Q8_0 segments: k_mv_f1 (the only kernel that takes pro / res_out)
      bool q8 = true;
      for (int i = 0; i < a.nseg; i++) q8 = q8 && a.seg[i].w.dtype == T_Q8_0 && a.seg[i].w.cols == a.seg[0].w.cols;
      // rows a wavefront: 8 with greedy keys (a slot per task) or tasks for the whole GPU, else
      // fewer, so that the launch has about 2 x CUs workgroups
      int rw = 8;
      while (!a.best && rw > 1 && grid * (8 / rw) < 2 * cu_count_f()) rw >>= 1;
      const int nb = (int)a.seg[0].w.nb, ni = (rw * nb + 63) / 64;
      const size_t sm = (size_t)32 * nb * 4 + (size_t)MVF1_NW * rw * nb * 8;
      if (q8 && ni <= 16 && sm <= 64 * 1024) {
        const dim3 g((unsigned)(grid * (8 / rw))), b(MVF1_NW * 64);
        auto go = [&](auto kern) {
          hipLaunchKernelGGL(kern, g, b, sm, s, a, st);
          return hipGetLastError();
        };
        auto by_ni = [&](auto RWc) {
          constexpr int RW = decltype(RWc)::value;
          return ni <= 2 ? go(k_mv_f1<2, RW>) : ni <= 4 ? go(k_mv_f1<4, RW>) : ni <= 8 ? go(k_mv_f1<8, RW>) : ni <= 12 ? go(k_mv_f1<12, RW>) : go(k_mv_f1<16, RW>);
        };
        if (rw == 8) return by_ni(std::integral_constant<int, 8>{});
        if (rw == 4) return by_ni(std::integral_constant<int, 4>{});
        if (rw == 2) return by_ni(std::integral_constant<int, 2>{});
        return by_ni(std::integral_constant<int, 1>{});
      }
    }
    if (f1_only) return hipErrorInvalidValue;
#define SPX_MVF(MTV) hipLaunchKernelGGL(k_mv_f<MTV>, dim3(grid), dim3(256), 0, s, a, st)
    switch (mt) {
    case 1: SPX_MVF(1); break;
    case 2: SPX_MVF(2); break;
    case 4: SPX_MVF(4); break;
    case 8: SPX_MVF(8); break;
    default: SPX_MVF(16); break;
    }
#undef SPX_MVF
    return hipGetLastError();
  }
  if (mode == 1) {
    if (a.G < 1 || a.R < 1 || a.G * a.R > 8 || (a.G & (a.G - 1))) return hipErrorInvalidValue;
    const size_t sm = rp_act_bytes(mt, cols) + 4 * rp_wave_bytes(a.R, nb, mt);
#define SPX_MVR(MTV) do { SPX_LDS(k_mvr<MTV>, sm); hipLaunchKernelGGL(k_mvr<MTV>, dim3(grid), dim3(256), sm, s, a, st); } while (0)
    switch (mt) {
    case 1: SPX_MVR(1); break;
    case 2: SPX_MVR(2); break;
    case 4: SPX_MVR(4); break;
    case 8: SPX_MVR(8); break;
    default: SPX_MVR(16); break;
    }
#undef SPX_MVR
    return hipGetLastError();
  }
  if (a.tail.nw) return hipErrorInvalidValue;  // tiles take no norm tail
  const size_t sm = (mt <= 2 ? ldsq_bytes(mt, cols) : 0) + (size_t)8 * nb * tile_bpb();
#define SPX_MVT(MTV) do { SPX_LDS(k_mvt<MTV>, sm); hipLaunchKernelGGL(k_mvt<MTV>, dim3(grid), dim3(64), sm, s, a, st); } while (0)
  switch (mt) {
  case 1: SPX_MVT(1); break;
  case 2: SPX_MVT(2); break;
  case 4: SPX_MVT(4); break;
  case 8: SPX_MVT(8); break;
  default: SPX_MVT(16); break;
  }
#undef SPX_MVT
  return hipGetLastError();
}

template <int HD>
static void launch_attn_t(const AttnArgs &a, int nqt, const StepRec *st, hipStream_t s) {
  const size_t sm = AttnLds<HD>::BYTES;
  SPX_LDS((k_attn<HD, true>), sm);
  hipLaunchKernelGGL((k_attn<HD, true>), dim3(a.nch, a.n_kv, nqt), dim3(256), sm, s, a, st);
}

hipError_t launch_attention_partials(const AttnArgs &a, const StepRec *st, hipStream_t s) {
  if (a.n_heads / a.n_kv > 8) return hipErrorInvalidValue;  // one 16-row query tile: rows 0-7 hold the queries
  if (a.hd == 128) {
    SPX_LDS((k_attn<128, false>), AttnLds<128>::BYTES);
    hipLaunchKernelGGL((k_attn<128, false>), dim3(a.nch, a.n_kv, 1), dim3(256), AttnLds<128>::BYTES, s, a, st);
  } else if (a.hd == 64) {
    SPX_LDS((k_attn<64, false>), AttnLds<64>::BYTES);
    hipLaunchKernelGGL((k_attn<64, false>), dim3(a.nch, a.n_kv, 1), dim3(256), AttnLds<64>::BYTES, s, a, st);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, int m, const StepRec *st, hipStream_t s) {
  const int nqt = (m * (a.n_heads / a.n_kv) + 15) / 16;
  if (nqt > ATT_QT || (m > MAX_M && !a.prepped)) return hipErrorInvalidValue;
  if (a.hd == 128) launch_attn_t<128>(a, nqt, st, s);
  else if (a.hd == 64) launch_attn_t<64>(a, nqt, st, s);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int HD>
static void launch_attn_pf_t(const AttnArgs &a, int m, const StepRec *st, hipStream_t s) {
  using LY = AttnLds<HD>;
  const size_t sm = (size_t)64 * LY::KS * 2 + (size_t)HD * LY::VS * 2 + 4 * ((size_t)16 * LY::SS * 4 + (size_t)2 * 16 * LY::PS * 2 + 16 * 4);
  const int nq = m * (a.n_heads / a.n_kv);
  SPX_LDS((k_attn_pf<HD>), sm);
  hipLaunchKernelGGL((k_attn_pf<HD>), dim3(a.nch, a.n_kv, (nq + 63) / 64), dim3(256), sm, s, a, st);
  hipLaunchKernelGGL((k_attn_pf_merge<HD>), dim3(a.n_kv, (nq + 15) / 16, (a.nch + ATT_GRP - 1) / ATT_GRP), dim3(256), (size_t)16 * HD * 4, s, a, st);
}

template <int HD>
static void launch_attn_fl_t(const AttnArgs &a, int m, const StepRec *st, hipStream_t s) {
  const int nq = m * (a.n_heads / a.n_kv), nqb = (nq + 63) / 64, per = (a.n_kv * FL_SPLITS + 7) / 8;
  // two halves' K / V tiles; after the walk, half 1's states (O [4][DT][4][64] + (M, L) [4][16])
  const size_t sm = std::max((size_t)2 * ((size_t)64 * (HD + 8) + (size_t)HD * (64 + 8)) * 2, (size_t)(4 * (HD / 16) * 4 * 64 + 4 * 16 * 2) * 4);
  SPX_LDS((k_attn_fl<HD>), sm);
  hipLaunchKernelGGL((k_attn_fl<HD>), dim3((unsigned)(8 * nqb * per)), dim3(512), sm, s, a, st);
  hipLaunchKernelGGL((k_attn_fl_merge<HD>), dim3(a.n_kv, (nq + 15) / 16), dim3(256), (size_t)16 * HD * 4, s, a, st);
}

hipError_t launch_attention_fl(const AttnArgs &a, int m, const StepRec *st, hipStream_t s) {
  // prepared rows only; the splits' partial slots must exist (nslot), queries fit ATT_QMAX
  if (!a.prepped || m < 1 || m > PMAX || a.n_heads % a.n_kv || m * (a.n_heads / a.n_kv) > ATT_QMAX || a.nslot < FL_SPLITS ||
      (a.aq.q && (a.n_heads * a.hd) % 256))
    return hipErrorInvalidValue;
  if (a.hd == 128) launch_attn_fl_t<128>(a, m, st, s);
  else if (a.hd == 64) launch_attn_fl_t<64>(a, m, st, s);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int HD>
static void launch_attn_fs_t(const AttnArgs &a, int m, const StepRec *st, hipStream_t s) {
  const int nqb = (m * (a.n_heads / a.n_kv) + 15) / 16, per = (a.n_kv * nqb + 7) / 8;
  // the eight states (O [8][DT][4][64] + (M, L) [8][16]) and the merged outputs [16][HD]
  const size_t sm = (size_t)(8 * (HD / 16) * 4 * 64 + 8 * 16 * 2 + 16 * HD) * 4;
  SPX_LDS((k_attn_fs<HD>), sm);
  hipLaunchKernelGGL((k_attn_fs<HD>), dim3((unsigned)(8 * per)), dim3(512), sm, s, a, st);
}

hipError_t launch_attention_fs(const AttnArgs &a, int m, const StepRec *st, hipStream_t s) {
  // the pass's K / V rows in the cache (prepped 1: prepared queries, 2: raw); a 256-value block of
  // the att rows' Q8_K holds 256 / hd queries of one row
  if (a.prepped < 1 || a.prepped > 2 || m < 1 || m > PMAX || a.n_heads % a.n_kv ||
      (a.aq.q && ((a.n_heads * a.hd) % 256 || (a.n_heads / a.n_kv) % (256 / a.hd))))
    return hipErrorInvalidValue;
  if (a.hd == 128) launch_attn_fs_t<128>(a, m, st, s);
  else if (a.hd == 64) launch_attn_fs_t<64>(a, m, st, s);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int HD>
static void launch_attn_mt_t(const AttnArgs &a, int m, const StepRec *st, hipStream_t s) {
  const int g = a.n_heads / a.n_kv, nqt = (m * g + 15) / 16;
  const size_t sm = MtLds<HD>::bytes(g, a.q_bias != nullptr, m);
  if (m > MAX_M) {  // merged per (query tile, chunk group): k_attn_pf_merge (41 vs 24 us a layer at 128 rows)
    SPX_LDS((k_attn_mt<HD, true>), sm);
    hipLaunchKernelGGL((k_attn_mt<HD, true>), dim3(a.nch, a.n_kv, (nqt + 7) / 8), dim3(512), sm, s, a, st);
    hipLaunchKernelGGL((k_attn_pf_merge<HD>), dim3(a.n_kv, nqt, (a.nch + ATT_GRP - 1) / ATT_GRP), dim3(256), (size_t)16 * HD * 4, s, a, st);
  } else {
    SPX_LDS((k_attn_mt<HD, false>), sm);
    hipLaunchKernelGGL((k_attn_mt<HD, false>), dim3(a.nch, a.n_kv, (nqt + 7) / 8), dim3(512), sm, s, a, st);
    hipLaunchKernelGGL((k_attn_mrg<HD>), dim3((a.n_heads * HD + 255) / 256, m), dim3(1024), 0, s, a, st);
  }
}

hipError_t launch_attention_mt(const AttnArgs &a, int m, const StepRec *st, hipStream_t s) {
  // (prefill passes: at least two queries a pass row, so a workgroup's rotations fit RPT = 5)
  // (the kv group's query biases are staged a float4 a thread: at most 512 of them)
  if (a.prepped || m < 1 || m > PMAX || a.n_heads % a.n_kv || (m > MAX_M && a.n_heads / a.n_kv < 2) ||
      (m * (a.n_heads / a.n_kv) + 15) / 16 > ATT_QT || (a.aq.q && (a.n_heads * a.hd) % 256) ||
      (a.q_bias && (a.n_heads / a.n_kv) * a.hd > 2048))
    return hipErrorInvalidValue;
  if (a.hd == 128) launch_attn_mt_t<128>(a, m, st, s);
  else if (a.hd == 64) launch_attn_mt_t<64>(a, m, st, s);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_attention_pf(const AttnArgs &a, int m, const StepRec *st, hipStream_t s) {
  if (!a.prepped || m < 1 || m > PMAX || (m * (a.n_heads / a.n_kv) + 15) / 16 > ATT_QT) return hipErrorInvalidValue;
  if (a.hd == 128) launch_attn_pf_t<128>(a, m, st, s);
  else if (a.hd == 64) launch_attn_pf_t<64>(a, m, st, s);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_rows_prep(const AttnArgs &a, float *qp, int m, const StepRec *st, hipStream_t s) {
  if (m < 1 || m > PMAX || (a.hd != 64 && a.hd != 128)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rows_prep, dim3(m, (qp ? a.n_heads : 0) + 2 * a.n_kv), dim3(64), 0, s, a, qp, st);
  return hipGetLastError();
}

hipError_t launch_router(const RouterArgs &a, int mt, const StepRec *st, hipStream_t s) {
  mt = bucket(mt);
  const int grid = a.n_expert;
  switch (mt) {
  case 1: hipLaunchKernelGGL(k_router<1>, dim3(grid), dim3(256), a.pro.nw ? (size_t)a.dim * 4 : 0, s, a, st); break;
  case 2: hipLaunchKernelGGL(k_router<2>, dim3(grid), dim3(256), 0, s, a, st); break;
  case 4: hipLaunchKernelGGL(k_router<4>, dim3(grid), dim3(256), 0, s, a, st); break;
  default: hipLaunchKernelGGL(k_router<8>, dim3(grid), dim3(256), 0, s, a, st); break;
  }
  return hipGetLastError();
}

// one-row Q8_0 gate / up on k_gateup_f1 (SPX_GU_F1=0: k_gateup_f, the same bits)
static bool gu_f1_on() {
  static const bool on = [] {
    const char *v = std::getenv("SPX_GU_F1");
    return !v || atoi(v) != 0;
  }();
  return on;
}

template <int T, int MT>
static hipError_t launch_gu_t(const GUArgs &a, int mode, const StepRec *st, int max_jobs, hipStream_t s) {
  const unsigned jobs = (unsigned)std::max(1, max_jobs);
  if constexpr (T == T_Q4K || T == T_Q6K) {
    const int dim = (int)a.gate.cols, nb = (int)a.gate.nb;
    if (mode == 1) {
      const size_t sm = rp_act_bytes(MT, dim) + 4 * rp_wave_bytes(2, nb, MT);
      SPX_LDS((k_gateup_rp<T, MT>), sm);
      hipLaunchKernelGGL((k_gateup_rp<T, MT>), dim3((unsigned)((a.n_ff + 3) / 4), jobs), dim3(256), sm, s, a, st);
      return hipGetLastError();
    }
    const size_t sm = (MT <= 2 ? ldsq_bytes(MT, dim) : 0) + (size_t)4 * 8 * nb * tile_bpb();
    SPX_LDS((k_gateup_kq<T, MT>), sm);
    hipLaunchKernelGGL((k_gateup_kq<T, MT>), dim3((unsigned)((a.n_ff + 15) / 16), jobs), dim3(256), sm, s, a, st);
  } else if (T == T_Q8_0 && MT >= 4 && a.fq) {
    hipLaunchKernelGGL(k_gateup_fq, dim3((unsigned)((a.n_ff + 15) / 16), jobs), dim3(1024), 0, s, a, st);
  } else if (T == T_Q8_0 && MT == 1 && !a.hq.q && a.gate.nb <= 128 && gu_f1_on()) {
    // one row: k_gateup_f1, RW rows a wavefront (fewer for more workgroups, up to 2 a CU)
    const int blocks = (a.n_ff + 15) / 16, nb = (int)a.gate.nb;
    int rw = 8;
    while (rw > 1 && (int64_t)blocks * jobs * (8 / rw) < 2 * cu_count_f()) rw >>= 1;
    const int ni = (rw * nb + 63) / 64;
    const size_t sm = (size_t)32 * nb * 4 + (size_t)MVF1_NW * rw * nb * 8;
    const dim3 g((unsigned)(blocks * (8 / rw)), jobs), b(MVF1_NW * 64);
    auto go = [&](auto kern) {
      SPX_LDS(kern, sm);
      hipLaunchKernelGGL(kern, g, b, sm, s, a, st);
      return hipGetLastError();
    };
    auto by_ni = [&](auto RWc) {
      constexpr int RW = decltype(RWc)::value;
      return ni <= 2 ? go(k_gateup_f1<2, RW>) : ni <= 4 ? go(k_gateup_f1<4, RW>) : ni <= 8 ? go(k_gateup_f1<8, RW>) : go(k_gateup_f1<16, RW>);
    };
    if (rw == 8) return by_ni(std::integral_constant<int, 8>{});
    if (rw == 4) return by_ni(std::integral_constant<int, 4>{});
    if (rw == 2) return by_ni(std::integral_constant<int, 2>{});
    return by_ni(std::integral_constant<int, 1>{});
  } else {
    hipLaunchKernelGGL((k_gateup_f<T, MT>), dim3((unsigned)((a.n_ff + 15) / 16), jobs), dim3(256),
                       MT == 1 && a.pro.nw ? (size_t)a.gate.cols * 4 : 0, s, a, st);
  }
  return hipGetLastError();
}

template <int T>
static hipError_t launch_gu_dt(const GUArgs &a, int mt, int mode, const StepRec *st, int max_jobs, hipStream_t s) {
  switch (mt) {
  case 1: return launch_gu_t<T, 1>(a, mode, st, max_jobs, s);
  case 2: return launch_gu_t<T, 2>(a, mode, st, max_jobs, s);
  case 4: return launch_gu_t<T, 4>(a, mode, st, max_jobs, s);
  case 8: return launch_gu_t<T, 8>(a, mode, st, max_jobs, s);
  default: return launch_gu_t<T, 16>(a, mode, st, max_jobs, s);
  }
}

hipError_t launch_gateup(const GUArgs &a, int mt, int mode, const StepRec *st, int max_jobs, hipStream_t s) {
  mt = bucket(mt);
  switch (a.gate.dtype) {
  case T_Q4K: return launch_gu_dt<T_Q4K>(a, mt, mode, st, max_jobs, s);
  case T_Q6K: return launch_gu_dt<T_Q6K>(a, mt, mode, st, max_jobs, s);
  case T_Q8_0: return launch_gu_dt<T_Q8_0>(a, mt, mode, st, max_jobs, s);
  case T_Q5_0: return launch_gu_dt<T_Q5_0>(a, mt, mode, st, max_jobs, s);
  case T_Q5K: return launch_gu_dt<T_Q5K>(a, mt, mode, st, max_jobs, s);
  default: return hipErrorInvalidValue;
  }
}

template <int T, int MT>
static hipError_t launch_down_t(const DownArgs &a, int mode, const StepRec *st, hipStream_t s) {
  const dim3 grid((unsigned)((a.w.rows + 3) / 4));
  if constexpr (T == T_Q4K || T == T_Q6K) {
    const int n_ff = (int)a.w.cols, nb = (int)a.w.nb;
    const size_t tiles = (size_t)4 * 8 * nb * tile_bpb();
    if (mode == 1) {
      SPX_LDS((k_down_rj<T, MT>), tiles);
      hipLaunchKernelGGL((k_down_rj<T, MT>), dim3((unsigned)a.w.rows), dim3(256), tiles, s, a, st);
      return hipGetLastError();
    }
    const size_t staged = ldsq_bytes(MT * a.n_used, n_ff) + tiles;
    if (MT <= 2 && staged <= 65536) {
      hipLaunchKernelGGL((k_down_kq<T, MT, true>), grid, dim3(256), staged, s, a, st);
    } else {
      SPX_LDS((k_down_kq<T, MT, false>), tiles);
      hipLaunchKernelGGL((k_down_kq<T, MT, false>), grid, dim3(256), tiles, s, a, st);
    }
  } else {
    hipLaunchKernelGGL((k_down_f<T, MT>), grid, dim3(256), 0, s, a, st);
  }
  return hipGetLastError();
}

template <int T>
static hipError_t launch_down_dt(const DownArgs &a, int mt, int mode, const StepRec *st, hipStream_t s) {
  switch (mt) {
  case 1: return launch_down_t<T, 1>(a, mode, st, s);
  case 2: return launch_down_t<T, 2>(a, mode, st, s);
  case 4: return launch_down_t<T, 4>(a, mode, st, s);
  case 8: return launch_down_t<T, 8>(a, mode, st, s);
  default: return launch_down_t<T, 16>(a, mode, st, s);
  }
}

// mode 0: four output rows per workgroup, a wavefront per row over the jobs; 1 (integer):
// one row per workgroup, the wavefronts split the jobs
hipError_t launch_down(const DownArgs &a, int mt, int mode, const StepRec *st, hipStream_t s) {
  mt = bucket(mt);
  switch (a.w.dtype) {
  case T_Q4K: return launch_down_dt<T_Q4K>(a, mt, mode, st, s);
  case T_Q6K: return launch_down_dt<T_Q6K>(a, mt, mode, st, s);
  case T_Q8_0: return launch_down_dt<T_Q8_0>(a, mt, mode, st, s);
  case T_Q5_0: return launch_down_dt<T_Q5_0>(a, mt, mode, st, s);
  case T_Q5K: return launch_down_dt<T_Q5K>(a, mt, mode, st, s);
  default: return hipErrorInvalidValue;
  }
}

hipError_t launch_down_fq(const DownArgs &a, int max_jobs, const StepRec *st, hipStream_t s) {
  if (a.w.dtype != T_Q8_0 || !a.yd || !a.counter || max_jobs < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_down_fq, dim3((unsigned)((a.w.rows + 31) / 32), (unsigned)max_jobs), dim3(1024), 0, s, a, st);
  return hipGetLastError();
}

hipError_t launch_embed(const TensorView &e, const StepRec *st, float escale, const NormTail &t, int m, hipStream_t s) {
  hipLaunchKernelGGL(k_embed, dim3(m), dim3(256), 0, s, e, st, escale, t);
  return hipGetLastError();
}

hipError_t launch_norm(const NormTail &t, const StepRec *st, int m, hipStream_t s) {
  hipLaunchKernelGGL(k_norm, dim3(m), dim3(256), 0, s, t, st);
  return hipGetLastError();
}

hipError_t launch_argmax_final(const unsigned long long *best, int nbest, int *out, StepRec *st, int *hist, int m, hipStream_t s) {
  if (hist && m != 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_argmax_final, dim3(m), dim3(256), 0, s, best, nbest, out, st, hist);
  return hipGetLastError();
}

hipError_t launch_q8kp_quantize(const float *x, int64_t n, int64_t ld_x, int m, Q8KP out, hipStream_t s) {
  const int64_t blocks = (n / 256) * m;
  hipLaunchKernelGGL(k_q8kp_quantize, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, s, x, n, ld_x, m, out);
  return hipGetLastError();
}

hipError_t launch_q8kp_from_ref(const float *d, const int8_t *qs, const int16_t *bs, int64_t n, int m, Q8KP out, hipStream_t s) {
  hipLaunchKernelGGL(k_q8kp_from_ref, dim3((unsigned)((n / 256) * m)), dim3(64), 0, s, d, qs, bs, n, out);
  return hipGetLastError();
}

hipError_t launch_kq_block_sums(const TensorView &w, int expert, int64_t row, Q8KP y, int32_t *sums, hipStream_t s) {
  dim3 grid((unsigned)((w.nb + 7) / 8));
  if (w.dtype == T_Q4K) hipLaunchKernelGGL(k_kq_block_sums<T_Q4K>, grid, dim3(64), 0, s, w, expert, row, y, sums);
  else hipLaunchKernelGGL(k_kq_block_sums<T_Q6K>, grid, dim3(64), 0, s, w, expert, row, y, sums);
  return hipGetLastError();
}

}  // namespace spx
