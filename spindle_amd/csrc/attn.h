// Attention over the f16 KV cache as device functions (used by the pass kernels of fused.hip,
// the one-row decode pipeline and the persistent decode pass): per-head q / k preparation
// (bias, RMSNorm, RoPE), the chunk item on the f16 matrix cores (QK^T and PV with queries and
// probabilities split into hi + lo f16 parts, online softmax over 64 positions), and the
// chunk merges. Also the arrival counters the in-kernel merges use.
#pragma once
#include "dev.h"
#include "fused.h"

namespace spx {

// Single counter: returns the counter's previous value to every thread.
__device__ __forceinline__ int arrive(int *counter) {
  __shared__ int prev;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) prev = atomicAdd(counter, 1);
  __syncthreads();
  return prev;
}
// Two-level count for launches with many workgroups (no hot counter): workgroup w counts
// into sub-counter w % CNT_SUB; the last of each sub-counter counts into the top counter.
// True in every thread of the last of the n workgroups. Counters are left at zero.
__device__ __forceinline__ bool arrive_last(int *cnt, int n) {
  __shared__ int last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int wg = blockIdx.x + blockIdx.y * gridDim.x, sub = wg % CNT_SUB;
    const int expect = (n - sub + CNT_SUB - 1) / CNT_SUB, nsub = n < CNT_SUB ? n : CNT_SUB;
    int l = 0;
    int *sc = cnt + (1 + sub) * CNT_STRIDE;
    if (atomicAdd(sc, 1) == expect - 1) {
      *sc = 0;
      l = atomicAdd(cnt, 1) == nsub - 1;
      if (l) *cnt = 0;
    }
    last = l;
  }
  __syncthreads();
  return last;
}

// ------------------------------------------------------------------ attention
// One workgroup per (position chunk, kv head, tile of 16 query rows): the tile's query heads
// (rows b of the pass x the kv group's heads, after bias, per-head RMSNorm and RoPE,
// :3226-3248 / :3432-3448) against the chunk's K/V (f16 cache), causal per row (row b sees
// positions <= start + b), online softmax over the chunk's 64-position sub-chunks. The new
// K/V rows (positions start..start+m-1) are normed / rotated by every workgroup that needs
// them (straight into its LDS tile) and written to the cache by the first query tile's.
// Scores and P.V run on the matrix cores (v_mfma_f32_16x16x16_f16): K and V are f16 already;
// queries and probabilities are split into two f16 parts (x = hi + lo, ~22 significant bits)
// whose products accumulate in fp32. Each workgroup leaves (max, sum, unnormalised output) per
// query; chunks are merged in two levels (flash-decoding, chunk order), the last merger of a
// query tile writes its output, optionally as Q8_K.
__device__ __forceinline__ void head_prep(const float *src, const float *bias, const float *nw, const float2 *rope_row, int hd, int neox,
                                          float eps, float &e0, float &e1) {
  const int lane = threadIdx.x & 63, half = hd >> 1;
  const bool act = lane < half;
  const int da = neox ? lane : 2 * lane, db = neox ? lane + half : 2 * lane + 1;
  float x0 = act ? src[da] : 0.0f, x1 = act ? src[db] : 0.0f;
  if (bias && act) { x0 += bias[da]; x1 += bias[db]; }
  if (nw) {
    const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
    const float inv = inv_rms(ss, (float)hd, eps);
    if (act) { x0 = x0 * inv * nw[da]; x1 = x1 * inv * nw[db]; }
  }
  if (rope_row && act) {  // Rope::rotate (:1404-1419)
    const float c = rope_row[lane].x, s = rope_row[lane].y;
    const float r0 = x0 * c - x1 * s, r1 = x0 * s + x1 * c;
    x0 = r0;
    x1 = r1;
  }
  e0 = x0;
  e1 = x1;
}

typedef _Float16 h4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4v mfma16(h4v a, h4v b, f4v c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

// x = hi + lo in f16 (hi = x rounded, lo = the rounded remainder)
__device__ __forceinline__ void split_f16(float x, _Float16 &hi, _Float16 &lo) {
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

// Merges n <= 16 partials (running max m, sum l, unnormalised output o) in slots s0 .. s0+n-1
// for the QPT queries qa .. qa+QPT-1 (< NQ): M = max m_c, w_c = exp(m_c - M),
// L = sum l_c w_c, O = sum w_c o_c in slot order. Thread: query qa + tid / (256 / QPT), a
// slice of its dims. Writes the normalised O / L to LDS (ol, rows from qa) or the merged
// partial to slot dst.
template <int HD, int QPT>
__device__ __forceinline__ void attn_merge_q(rsrc_t r_ml, rsrc_t r_o, int s0, int n, int qa, int NQ, float *ol, const rsrc_t *d_ml,
                                             const rsrc_t *d_o, int dst) {
  constexpr int TPQ = 256 / QPT, DW = HD / TPQ, NV = DW / 4;  // threads per query, dims per thread
  const int tid = threadIdx.x, qi = qa + tid / TPQ, d0 = (tid % TPQ) * DW;
  if (qi >= NQ) return;
  f2v ml[16];
#pragma unroll
  for (int k = 0; k < 16; k++) ml[k] = k < n ? ld_coh2(r_ml, ((s0 + k) * ATT_QMAX + qi) * 8) : f2v{-INFINITY, 0.0f};
  float M = -INFINITY;
#pragma unroll
  for (int k = 0; k < 16; k++) M = fmaxf(M, ml[k].x);
  float w[16], L = 0.0f;
#pragma unroll
  for (int k = 0; k < 16; k++) {
    w[k] = ml[k].x == -INFINITY ? 0.0f : expf(ml[k].x - M);
    if (k < n) L = fmaf(ml[k].y, w[k], L);
  }
  float acc[DW];
#pragma unroll
  for (int j = 0; j < DW; j++) acc[j] = 0.0f;
#pragma unroll
  for (int k0 = 0; k0 < 16; k0 += 8) {
    if (k0 < n) {
      f4v ov[8][NV];
#pragma unroll
      for (int k = 0; k < 8; k++)
#pragma unroll
        for (int v = 0; v < NV; v++)
          ov[k][v] = ld_coh4(r_o, (((s0 + min(k0 + k, n - 1)) * ATT_QMAX + qi) * HD + d0 + 4 * v) * 4);
#pragma unroll
      for (int k = 0; k < 8; k++) {
        if (k0 + k < n) {
#pragma unroll
          for (int v = 0; v < NV; v++) {
            acc[4 * v] = fmaf(ov[k][v].x, w[k0 + k], acc[4 * v]);
            acc[4 * v + 1] = fmaf(ov[k][v].y, w[k0 + k], acc[4 * v + 1]);
            acc[4 * v + 2] = fmaf(ov[k][v].z, w[k0 + k], acc[4 * v + 2]);
            acc[4 * v + 3] = fmaf(ov[k][v].w, w[k0 + k], acc[4 * v + 3]);
          }
        }
      }
    }
  }
  if (ol) {
    const float il = __fdiv_rn(1.0f, fmaxf(L, 1e-30f));
#pragma unroll
    for (int j = 0; j < DW; j++) ol[(qi - qa) * HD + d0 + j] = acc[j] * il;
  } else {
#pragma unroll
    for (int v = 0; v < NV; v++)
      st_coh4(*d_o, ((dst * ATT_QMAX + qi) * HD + d0 + 4 * v) * 4, f4v{acc[4 * v], acc[4 * v + 1], acc[4 * v + 2], acc[4 * v + 3]});
    if (tid % TPQ == 0) st_coh2(*d_ml, (dst * ATT_QMAX + qi) * 8, f2v{M, L});
  }
}

// The tile's merge with all 256 threads: 8 queries (32 threads each) when the tile has at
// most 8, else 16 (16 threads each).
template <int HD>
__device__ __forceinline__ void attn_merge16(rsrc_t r_ml, rsrc_t r_o, int s0, int n, int qa, int NQ, float *ol, const rsrc_t *d_ml,
                                             const rsrc_t *d_o, int dst) {
  if (NQ - qa <= 8 && HD / 32 >= 4) attn_merge_q<HD, 8>(r_ml, r_o, s0, n, qa, NQ, ol, d_ml, d_o, dst);
  else attn_merge_q<HD, 16>(r_ml, r_o, s0, n, qa, NQ, ol, d_ml, d_o, dst);
}

template <int NU>
__device__ __forceinline__ void attn_kv_load(const AttnArgs &a, int64_t off, uint32_t (&kr)[4 * NU], uint32_t (&vr)[4 * NU]) {
  const uint4 *kp = reinterpret_cast<const uint4 *>(a.kc + off), *vp = reinterpret_cast<const uint4 *>(a.vc + off);
#pragma unroll
  for (int u = 0; u < NU; u++) {
    const uint4 k = kp[u], v = vp[u];
    kr[4 * u] = k.x; kr[4 * u + 1] = k.y; kr[4 * u + 2] = k.z; kr[4 * u + 3] = k.w;
    vr[4 * u] = v.x; vr[4 * u + 1] = v.y; vr[4 * u + 2] = v.z; vr[4 * u + 3] = v.w;
  }
}

// LDS of k_attn (strides in halves / floats, padded against bank conflicts)
template <int HD> struct AttnLds {
  // row strides (f16 elements) of the MFMA operands: rows 4 dwords apart modulo 64 banks, so
  // the sixteen rows an 8-byte operand load touches fall on distinct banks (and K rows stay
  // 16-byte aligned for the row stores)
  static constexpr int QS = HD + 8, KS = HD + 8, VS = 64 + 8, PS = 64 + 8, SS = 64 + 4;
  static constexpr size_t QB = (size_t)2 * 16 * QS * 2;  // qh, ql; later the merged output [16][HD] f32
  static constexpr size_t BYTES = QB + (size_t)64 * KS * 2 + (size_t)HD * VS * 2 + (size_t)16 * SS * 4 + (size_t)2 * 16 * PS * 2 + 3 * 16 * 4;
  static_assert(QB >= (size_t)16 * HD * 4, "merged output fits over the queries");
};

// Chunks are 64 positions for every pass size and query tile, merged in chunk order in the
// same two levels (groups of ATT_GRP chunks, then the groups) as a one-row pass's kd_merge:
// a query's partials, and so its output bits, do not depend on how many rows the pass has.

// The K/V rows of chunk c of kv head h as thread tid of the item loads them (position p_lo +
// tid / 4, dims (tid % 4) * HD / 4 ..): a one-row pass clamps to the cache, so the loads do not
// depend on the step record and can be issued before it (or before a grid barrier) arrives.
template <int HD, bool MERGE>
__device__ __forceinline__ void attn_kv_first(const AttnArgs &a, int total, int c, int h, uint32_t (&kr)[HD / 8], uint32_t (&vr)[HD / 8]) {
  constexpr int DQ = HD / 4, NU = DQ / 8;
  const int tid = threadIdx.x & 255, lp = tid >> 2, lq = tid & 3;
  const int p_lo = c * 64, p_hi = min(p_lo + 64, total);
  const int64_t cache0 = (int64_t)a.layer * a.max_seq * a.kv_dim + (int64_t)h * HD;
  attn_kv_load<NU>(a, cache0 + (int64_t)min(p_lo + lp, MERGE ? p_hi - 1 : a.max_seq - 1) * a.kv_dim + lq * DQ, kr, vr);
}

// The merged outputs of query tile qa .. qa + 15 of kv head h (ol: [16][HD] in LDS, 256 threads)
// to the att rows, and their Q8_K when a.aq is set.
template <int HD>
__device__ __forceinline__ void attn_tile_out(const AttnArgs &a, int h, int qa, int NQ, const float *ol) {
  const int tid = threadIdx.x & 255, wave = tid >> 6, lane = tid & 63, g = a.n_heads / a.n_kv;
  const int nrow = min(16, NQ - qa);
  for (int i = tid; i < nrow * HD; i += 256) {
    const int qi = qa + i / HD, d = i % HD, b = qi / g, head = h * g + qi % g;
    a.att[(int64_t)b * a.n_heads * HD + head * HD + d] = ol[i];
  }
  if (a.aq.q) {  // 256-value blocks of att rows: (256 / HD) consecutive queries of the tile
    const int qpb = 256 / HD, nbr = a.n_heads * HD / 256;
    for (int j = wave; j < nrow / qpb; j += 4) {
      const int q0 = qa + j * qpb, b = q0 / g, head = h * g + q0 % g;
      const float4 xv = reinterpret_cast<const float4 *>(ol + j * 256)[lane];
      const float am = q8k_amax(xv);
      const int64_t vb = (int64_t)b * nbr + head * HD / 256;
      q8k_block_store(xv, am, a.aq.q + vb * 64, a.aq.d + vb, reinterpret_cast<int *>(a.aq.bs + vb * 8));
    }
  }
}

// Raw inputs of a multi-row item's head_prep rows (wavefront w: query rows w + 4j of the tile,
// new pass rows b = w + 4j when their position falls in the item's chunk), loaded before the
// chunk's K/V rows: memory returns in issue order, so a row loaded after the K/V would wait
// for all of it, and each row's norm reduction would wait for the next row's load.
struct AttnPre {
  float q0[4], q1[4], qb0[4], qb1[4], qc[4], qs[4];
  float k0[4], k1[4], kb0[4], kb1[4], v0[4], v1[4], vb0[4], vb1[4], kc[4], ks[4];
  float qn0, qn1, kn0, kn1;
};

template <int HD>
__device__ __forceinline__ void attn_pre_load(const AttnArgs &a, int m, int start, int c, int h, int qt, AttnPre &p) {
  const int tid = threadIdx.x & 255, wave = tid >> 6, lane = tid & 63, half = HD / 2;
  const bool act = lane < half;
  const int da = a.neox ? lane : 2 * lane, db = a.neox ? lane + half : 2 * lane + 1;
  const int g = a.n_heads / a.n_kv, NQ = m * g, qa = qt * 16, total = start + m;
  const int p_lo = c * 64, p_hi = min(p_lo + 64, total);
  p.qn0 = p.qn1 = p.kn0 = p.kn1 = 0.0f;
  if (a.q_norm && act) { p.qn0 = a.q_norm[da]; p.qn1 = a.q_norm[db]; }
  if (a.k_norm && act) { p.kn0 = a.k_norm[da]; p.kn1 = a.k_norm[db]; }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int qi = qa + wave + 4 * j;
    p.q0[j] = p.q1[j] = p.qb0[j] = p.qb1[j] = 0.0f;
    p.qc[j] = 1.0f;
    p.qs[j] = 0.0f;
    if (qi < NQ && act) {
      const int b = qi / g, head = h * g + qi % g;
      const float *src = a.q + (int64_t)b * a.n_heads * HD + head * HD;
      p.q0[j] = src[da];
      p.q1[j] = src[db];
      if (!a.prepped) {
        if (a.q_bias) { p.qb0[j] = a.q_bias[head * HD + da]; p.qb1[j] = a.q_bias[head * HD + db]; }
        const float2 cs = a.rope[(int64_t)(start + b) * half + lane];
        p.qc[j] = cs.x;
        p.qs[j] = cs.y;
      }
    }
    const int b = wave + 4 * j, pos = start + b;
    p.k0[j] = p.k1[j] = p.kb0[j] = p.kb1[j] = p.v0[j] = p.v1[j] = p.vb0[j] = p.vb1[j] = 0.0f;
    p.kc[j] = 1.0f;
    p.ks[j] = 0.0f;
    if (!a.prepped && b < m && pos >= p_lo && pos < p_hi && act) {
      const float *ks = a.k + (int64_t)b * a.kv_dim + h * HD, *vs = a.v + (int64_t)b * a.kv_dim + h * HD;
      p.k0[j] = ks[da];
      p.k1[j] = ks[db];
      p.v0[j] = vs[da];
      p.v1[j] = vs[db];
      if (a.k_bias) { p.kb0[j] = a.k_bias[h * HD + da]; p.kb1[j] = a.k_bias[h * HD + db]; }
      if (a.v_bias) { p.vb0[j] = a.v_bias[h * HD + da]; p.vb1[j] = a.v_bias[h * HD + db]; }
      const float2 cs = a.rope[(int64_t)pos * half + lane];
      p.kc[j] = cs.x;
      p.ks[j] = cs.y;
    }
  }
}

// head_prep's arithmetic on preloaded values (x: the row, xb: its bias, nw0 / nw1: the norm
// weights, c / s: the rotation), operation for operation
__device__ __forceinline__ void head_prep_pre(float x0, float x1, float xb0, float xb1, bool bias, bool norm, float nw0, float nw1,
                                              bool rope, float c, float s, int hd, float eps, float &e0, float &e1) {
  const bool act = (int)(threadIdx.x & 63) < (hd >> 1);
  if (bias && act) { x0 += xb0; x1 += xb1; }
  if (norm) {
    const float ss = wave_sum(fmaf(x0, x0, x1 * x1));
    const float inv = inv_rms(ss, (float)hd, eps);
    if (act) { x0 = x0 * inv * nw0; x1 = x1 * inv * nw1; }
  }
  if (rope && act) {
    const float r0 = x0 * c - x1 * s, r1 = x0 * s + x1 * c;
    x0 = r0;
    x1 = r1;
  }
  e0 = x0;
  e1 = x1;
}

// One attention item: chunk c (64 positions) of kv head h for query tile qt of a pass of m rows
// at start, with 256 threads, LDS at smem (AttnLds<HD>::BYTES) and the chunk's first K/V rows
// already in kr / vr (attn_kv_first). COH: the q / k / v rows and the partials are handed
// between workgroups of one launch (the persistent pass): read and written coherently. MERGE
// items take their query and new rows from pre (attn_pre_load, issued before attn_kv_first).
template <int HD, bool MERGE, bool COH>
__device__ __forceinline__ void attn_item(const AttnArgs &a, const int m, const int start, const int c, const int h, const int qt,
                                          uint8_t *smem, uint32_t (&kr)[HD / 8], uint32_t (&vr)[HD / 8], const AttnPre *pre = nullptr) {
  using LY = AttnLds<HD>;
  constexpr int QS = LY::QS, KS = LY::KS, VS = LY::VS, PS = LY::PS, SS = LY::SS;
  constexpr int DT = HD / 16, TPW = DT / 4;  // 16-dim output tiles, per wavefront
  constexpr int DQ = HD / 4, NU = DQ / 8;    // K/V loader: dims per thread, 16-byte pieces
  const int total = start + m;
  const int g = a.n_heads / a.n_kv, NQ = m * g, qa = qt * 16;
  constexpr int CS = 64;
  const int nch = (total + CS - 1) / CS;
  const int p_lo = c * CS, p_hi = min(p_lo + CS, total);
  const int tid = threadIdx.x & 255, wave = tid >> 6, lane = tid & 63;
  _Float16 *qh = reinterpret_cast<_Float16 *>(smem);            // [16][QS]
  _Float16 *ql = qh + 16 * QS;                                   // [16][QS]
  _Float16 *ks = reinterpret_cast<_Float16 *>(smem + LY::QB);    // [64][KS]
  _Float16 *vt = ks + 64 * KS;                                   // [HD][VS] (V transposed)
  float *ss = reinterpret_cast<float *>(vt + HD * VS);           // [16][SS] scores
  _Float16 *ph = reinterpret_cast<_Float16 *>(ss + 16 * SS);     // [16][PS]
  _Float16 *pl = ph + 16 * PS;                                   // [16][PS]
  float *rm = reinterpret_cast<float *>(pl + 16 * PS), *rl = rm + 16, *sa = rl + 16;  // running max, sum; rescale
  const int64_t cache0 = (int64_t)a.layer * a.max_seq * a.kv_dim + (int64_t)h * HD;
  const int half = HD / 2;
  const int da = a.neox ? lane : 2 * lane, db = a.neox ? lane + half : 2 * lane + 1;
  const int ar = lane & 15, kg = (lane >> 4) * 4;  // MFMA operand row / column, k offset

  const int lp = tid >> 2, lq = tid & 3;
  // queries of this tile -> LDS as hi / lo f16 (rows past NQ are zero)
  float nk_x[2] = {0.0f, 0.0f}, nv_x[2] = {0.0f, 0.0f}, nk_w[2] = {0.0f, 0.0f}, rc = 1.0f, rs = 0.0f;
  if constexpr (!MERGE) {
    // one-row pass: NQ = g <= 8 query rows, wavefront w takes rows w and w + 4; every load is
    // issued before the first reduction (head_prep's arithmetic, operation for operation)
    float x0[2], x1[2], n0 = 0.0f, n1 = 0.0f, c0[2], s0[2];
    const bool act = lane < half;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int qi = min(wave + 4 * j, NQ - 1), head = h * g + qi;
      const float *src = a.q + head * HD;
      if (COH) {
        const rsrc_t rq = rsrc_of(a.q);
        x0[j] = act ? ld_coh1(rq, (head * HD + da) * 4) : 0.0f;
        x1[j] = act ? ld_coh1(rq, (head * HD + db) * 4) : 0.0f;
      } else {
        x0[j] = act ? src[da] : 0.0f;
        x1[j] = act ? src[db] : 0.0f;
      }
      if (a.q_bias && act) { x0[j] += a.q_bias[head * HD + da]; x1[j] += a.q_bias[head * HD + db]; }
    }
    if (a.q_norm && act) { n0 = a.q_norm[da]; n1 = a.q_norm[db]; }
    // the pass row's new K / V values (wavefront 0 normalises them if its chunk holds them)
    if (wave == 0 && act) {
      if (COH) {
        const rsrc_t rk = rsrc_of(a.k), rv = rsrc_of(a.v);
        nk_x[0] = ld_coh1(rk, (h * HD + da) * 4); nk_x[1] = ld_coh1(rk, (h * HD + db) * 4);
        nv_x[0] = ld_coh1(rv, (h * HD + da) * 4); nv_x[1] = ld_coh1(rv, (h * HD + db) * 4);
      } else {
        nk_x[0] = a.k[h * HD + da]; nk_x[1] = a.k[h * HD + db];
        nv_x[0] = a.v[h * HD + da]; nv_x[1] = a.v[h * HD + db];
      }
      if (a.k_bias) { nk_x[0] += a.k_bias[h * HD + da]; nk_x[1] += a.k_bias[h * HD + db]; }
      if (a.v_bias) { nv_x[0] += a.v_bias[h * HD + da]; nv_x[1] += a.v_bias[h * HD + db]; }
      if (a.k_norm) { nk_w[0] = a.k_norm[da]; nk_w[1] = a.k_norm[db]; }
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      c0[j] = 1.0f; s0[j] = 0.0f;
      if (act) { const float2 cs = a.rope[(int64_t)start * half + lane]; c0[j] = cs.x; s0[j] = cs.y; }
    }
    rc = c0[0];
    rs = s0[0];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int r = wave + 4 * j;
      float e0 = x0[j], e1 = x1[j];
      if (a.q_norm) {
        const float ssq = wave_sum(fmaf(e0, e0, e1 * e1));
        const float inv = inv_rms(ssq, (float)HD, a.eps);
        if (act) { e0 = e0 * inv * n0; e1 = e1 * inv * n1; }
      }
      if (act) {
        const float r0 = e0 * c0[j] - e1 * s0[j], r1 = e0 * s0[j] + e1 * c0[j];
        e0 = r0;
        e1 = r1;
      }
      if (r >= NQ) { e0 = 0.0f; e1 = 0.0f; }
      if (act) {
        split_f16(e0, qh[r * QS + da], ql[r * QS + da]);
        split_f16(e1, qh[r * QS + db], ql[r * QS + db]);
        split_f16(0.0f, qh[(r + 8) * QS + da], ql[(r + 8) * QS + da]);
        split_f16(0.0f, qh[(r + 8) * QS + db], ql[(r + 8) * QS + db]);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int r = wave + 4 * j, qi = qa + r;
      float e0 = 0.0f, e1 = 0.0f;
      if (qi < NQ)  // prepared queries (a.prepped) are taken as they are
        head_prep_pre(pre->q0[j], pre->q1[j], pre->qb0[j], pre->qb1[j], a.q_bias && !a.prepped, a.q_norm && !a.prepped, pre->qn0,
                      pre->qn1, !a.prepped, pre->qc[j], pre->qs[j], HD, a.eps, e0, e1);
      if (lane < half) {
        split_f16(e0, qh[r * QS + da], ql[r * QS + da]);
        split_f16(e1, qh[r * QS + db], ql[r * QS + db]);
      }
    }
  }
  if (tid < 16) { rm[tid] = -INFINITY; rl[tid] = 0.0f; }
  f4v acc[TPW];
#pragma unroll
  for (int j = 0; j < TPW; j++) acc[j] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

  // first position whose K / V row this item makes itself (prepared passes: none)
  const int new0 = MERGE && a.prepped ? total : start;
  for (int s0 = p_lo; s0 < p_hi; s0 += 64) {
    __syncthreads();  // the previous sub-chunk is done with ks / vt / ph / pl
    // cached rows -> LDS (K row-major, V transposed); rows of this pass come from below; rows
    // past the pass are zero (their probabilities are zero, and 0 * V must stay 0)
    if (s0 + lp >= total) {
#pragma unroll
      for (int t = 0; t < 4 * NU; t++) { kr[t] = 0u; vr[t] = 0u; }
    }
    if (s0 + lp < new0 || s0 + lp >= total) {
      uint16_t *vt16 = reinterpret_cast<uint16_t *>(vt);
#pragma unroll
      for (int u = 0; u < NU; u++) reinterpret_cast<uint4 *>(ks + lp * KS + lq * DQ)[u] = make_uint4(kr[4 * u], kr[4 * u + 1], kr[4 * u + 2], kr[4 * u + 3]);
#pragma unroll
      for (int t = 0; t < 4 * NU; t++) {
        vt16[(lq * DQ + 2 * t) * VS + lp] = (uint16_t)(vr[t] & 0xffffu);
        vt16[(lq * DQ + 2 * t + 1) * VS + lp] = (uint16_t)(vr[t] >> 16);
      }
    }
    if (s0 + 64 < p_hi) attn_kv_load<NU>(a, cache0 + (int64_t)min(s0 + 64 + lp, p_hi - 1) * a.kv_dim + lq * DQ, kr, vr);
    // this pass's K/V rows in the sub-chunk: normed / rotated here, to the cache by tile 0
    if (!MERGE && wave == 0 && start >= s0 && start < s0 + 64 && start < p_hi) {
      // one-row pass, values loaded at entry: head_prep's arithmetic (k: norm, RoPE; v: as is)
      const int pos = start, pp = pos - s0;
      const bool act = lane < half;
      float e0 = nk_x[0], e1 = nk_x[1];
      if (a.k_norm) {
        const float ssq = wave_sum(fmaf(e0, e0, e1 * e1));
        const float inv = inv_rms(ssq, (float)HD, a.eps);
        if (act) { e0 = e0 * inv * nk_w[0]; e1 = e1 * inv * nk_w[1]; }
      }
      if (act) {
        const float r0 = e0 * rc - e1 * rs, r1 = e0 * rs + e1 * rc;
        const __half k0 = __float2half_rn(r0), k1 = __float2half_rn(r1);
        ks[pp * KS + da] = (_Float16)__half2float(k0);
        ks[pp * KS + db] = (_Float16)__half2float(k1);
        __half *kd = a.kc + cache0 + (int64_t)pos * a.kv_dim;
        kd[da] = k0;
        kd[db] = k1;
        const __half v0 = __float2half_rn(nv_x[0]), v1 = __float2half_rn(nv_x[1]);
        vt[da * VS + pp] = (_Float16)__half2float(v0);
        vt[db * VS + pp] = (_Float16)__half2float(v1);
        __half *vd = a.vc + cache0 + (int64_t)pos * a.kv_dim;
        vd[da] = v0;
        vd[db] = v1;
      }
    }
#pragma unroll
    for (int j = 0; MERGE && !a.prepped && j < 4; j++) {  // rows b = wave + 4j, preloaded
      const int b = wave + 4 * j, pos = start + b, pp = pos - s0;
      if (b >= m || pp < 0 || pp >= 64 || pos >= p_hi) continue;
      float e0, e1;
      head_prep_pre(pre->k0[j], pre->k1[j], pre->kb0[j], pre->kb1[j], a.k_bias != nullptr, a.k_norm != nullptr, pre->kn0, pre->kn1,
                    true, pre->kc[j], pre->ks[j], HD, a.eps, e0, e1);
      if (lane < half) {
        const __half k0 = __float2half_rn(e0), k1 = __float2half_rn(e1);
        ks[pp * KS + da] = (_Float16)__half2float(k0);
        ks[pp * KS + db] = (_Float16)__half2float(k1);
        if (qt == 0) { __half *kd = a.kc + cache0 + (int64_t)pos * a.kv_dim; kd[da] = k0; kd[db] = k1; }
      }
      head_prep_pre(pre->v0[j], pre->v1[j], pre->vb0[j], pre->vb1[j], a.v_bias != nullptr, false, 0.0f, 0.0f, false, 1.0f, 0.0f, HD,
                    a.eps, e0, e1);
      if (lane < half) {
        const __half v0 = __float2half_rn(e0), v1 = __float2half_rn(e1);
        vt[da * VS + pp] = (_Float16)__half2float(v0);
        vt[db * VS + pp] = (_Float16)__half2float(v1);
        if (qt == 0) { __half *vd = a.vc + cache0 + (int64_t)pos * a.kv_dim; vd[da] = v0; vd[db] = v1; }
      }
    }
    for (int b = wave + 16; MERGE && !a.prepped && b < m; b += 4) {  // rows past the preloaded ones
      const int pos = start + b, pp = pos - s0;
      if (pp < 0 || pp >= 64 || pos >= p_hi) continue;
      float e0, e1;
      head_prep(a.k + (int64_t)b * a.kv_dim + h * HD, a.k_bias ? a.k_bias + h * HD : nullptr, a.k_norm,
                a.rope + (int64_t)pos * half, HD, a.neox, a.eps, e0, e1);
      if (lane < half) {
        const __half k0 = __float2half_rn(e0), k1 = __float2half_rn(e1);
        ks[pp * KS + da] = (_Float16)__half2float(k0);
        ks[pp * KS + db] = (_Float16)__half2float(k1);
        if (qt == 0) { __half *kd = a.kc + cache0 + (int64_t)pos * a.kv_dim; kd[da] = k0; kd[db] = k1; }
      }
      head_prep(a.v + (int64_t)b * a.kv_dim + h * HD, a.v_bias ? a.v_bias + h * HD : nullptr, nullptr, nullptr, HD, a.neox, a.eps, e0, e1);
      if (lane < half) {
        const __half v0 = __float2half_rn(e0), v1 = __float2half_rn(e1);
        vt[da * VS + pp] = (_Float16)__half2float(v0);
        vt[db * VS + pp] = (_Float16)__half2float(v1);
        if (qt == 0) { __half *vd = a.vc + cache0 + (int64_t)pos * a.kv_dim; vd[da] = v0; vd[db] = v1; }
      }
    }
    __syncthreads();
    // scores S = Q K^T, wavefront w: positions 16w .. 16w+15
    {
      f4v sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kt = 0; kt < DT; kt++) {
        const h4v bk = *reinterpret_cast<const h4v *>(ks + (wave * 16 + ar) * KS + kt * 16 + kg);
        const h4v ahi = *reinterpret_cast<const h4v *>(qh + ar * QS + kt * 16 + kg);
        const h4v alo = *reinterpret_cast<const h4v *>(ql + ar * QS + kt * 16 + kg);
        sacc = mfma16(ahi, bk, sacc);
        sacc = mfma16(alo, bk, sacc);
      }
#pragma unroll
      for (int r = 0; r < 4; r++) ss[(kg + r) * SS + wave * 16 + ar] = sacc[r];
    }
    __syncthreads();
    // online softmax, wavefront w: query rows w, w+4, w+8, w+12 (rows past the pass: their
    // probabilities are zero), lane = position; the rows' reductions are interleaved
    if (!MERGE) {  // rows 8-15 hold no query in a one-row pass: their values as computed below
      const int row = wave + 8 + 4 * (lane >> 5);
      ph[row * PS + (lane & 31)] = (_Float16)0.0f; ph[row * PS + 32 + (lane & 31)] = (_Float16)0.0f;
      pl[row * PS + (lane & 31)] = (_Float16)0.0f; pl[row * PS + 32 + (lane & 31)] = (_Float16)0.0f;
      if ((lane & 31) == 0) { rm[row] = -INFINITY; rl[row] = rl[row] * 1.0f + 0.0f; sa[row] = 1.0f; }
    }
    {
      constexpr int NR4 = MERGE ? 4 : 2;
      float sv[4], mx[4];
#pragma unroll
      for (int r4 = 0; r4 < NR4; r4++) {
        const int row = wave + 4 * r4, qi = qa + row, pos = s0 + lane;
        sv[r4] = qi < NQ && pos < p_hi && pos <= start + qi / g ? ss[row * SS + lane] * a.scale : -INFINITY;
        mx[r4] = sv[r4];
      }
#pragma unroll
      for (int r4 = 0; r4 < NR4; r4++) mx[r4] = wave_max(mx[r4]);
      float pv[4], ls[4], mn[4], al[4];
#pragma unroll
      for (int r4 = 0; r4 < NR4; r4++) {
        const int row = wave + 4 * r4;
        const float m_old = rm[row];
        mn[r4] = fmaxf(m_old, mx[r4]);
        pv[r4] = (sv[r4] == -INFINITY || mn[r4] == -INFINITY) ? 0.0f : expf(sv[r4] - mn[r4]);
        al[r4] = mn[r4] == -INFINITY ? 1.0f : (m_old == -INFINITY ? 0.0f : expf(m_old - mn[r4]));
        ls[r4] = pv[r4];
      }
#pragma unroll
      for (int r4 = 0; r4 < NR4; r4++) ls[r4] = wave_sum(ls[r4]);
#pragma unroll
      for (int r4 = 0; r4 < NR4; r4++) {
        const int row = wave + 4 * r4;
        split_f16(pv[r4], ph[row * PS + lane], pl[row * PS + lane]);
        if (lane == 0) { rm[row] = mn[r4]; rl[row] = rl[row] * al[r4] + ls[r4]; sa[row] = al[r4]; }
      }
    }
    __syncthreads();
    // O = O * alpha + P V, wavefront w: dim tiles w*TPW .. w*TPW + TPW-1
#pragma unroll
    for (int j = 0; j < TPW; j++) {
      const int dt = wave * TPW + j;
#pragma unroll
      for (int r = 0; r < 4; r++) acc[j][r] *= sa[kg + r];
#pragma unroll
      for (int kt = 0; kt < 4; kt++) {
        const h4v bv = *reinterpret_cast<const h4v *>(vt + (dt * 16 + ar) * VS + kt * 16 + kg);
        const h4v ahi = *reinterpret_cast<const h4v *>(ph + ar * PS + kt * 16 + kg);
        const h4v alo = *reinterpret_cast<const h4v *>(pl + ar * PS + kt * 16 + kg);
        acc[j] = mfma16(ahi, bv, acc[j]);
        acc[j] = mfma16(alo, bv, acc[j]);
      }
    }
  }
  __syncthreads();

  // partials, written through the L2 (sc1: the merge reads them in this launch or the next,
  // and they need no write-back at the launch's end): O from the accumulators, (max, sum) per
  // query
  const rsrc_t r_ml = rsrc_of(a.part_ml + ((int64_t)h * a.nslot) * ATT_QMAX * 2);
  const rsrc_t r_o = rsrc_of(a.part_o + ((int64_t)h * a.nslot) * ATT_QMAX * HD);
#pragma unroll
  for (int j = 0; j < TPW; j++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int qi = qa + kg + r;
      if (qi < NQ) __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(acc[j][r]), r_o, ((c * ATT_QMAX + qi) * HD + (wave * TPW + j) * 16 + ar) * 4, 0, 16);
    }
  if (tid < 16 && qa + tid < NQ) st_coh2(r_ml, (c * ATT_QMAX + qa + tid) * 8, f2v{rm[tid], rl[tid]});
  if (!MERGE) return;  // merged by a kernel of its own (one-row decode passes)

  // merges of this query tile: the last chunk of each group of ATT_GRP chunks merges the
  // group, the last group merger merges the groups (chunk / group order)
  const int grp = c / ATT_GRP, ngrp = (nch + ATT_GRP - 1) / ATT_GRP, gcnt = min(ATT_GRP, nch - grp * ATT_GRP);
  int *hcnt = a.counter + ((int64_t)h * ATT_QT + qt) * (1 + ATT_GMAX) * CNT_STRIDE;
  if (arrive(hcnt + (1 + grp) * CNT_STRIDE) != gcnt - 1) return;
  if (tid == 0) hcnt[(1 + grp) * CNT_STRIDE] = 0;
  float *ol = reinterpret_cast<float *>(smem);  // merged output [16][HD] of the tile's queries
  if (ngrp == 1) {
    attn_merge16<HD>(r_ml, r_o, 0, gcnt, qa, NQ, ol, nullptr, nullptr, 0);
  } else {
    attn_merge16<HD>(r_ml, r_o, grp * ATT_GRP, gcnt, qa, NQ, nullptr, &r_ml, &r_o, a.nch + grp);  // -> slot a.nch + grp
    if (arrive(hcnt) != ngrp - 1) return;
    if (tid == 0) hcnt[0] = 0;
    attn_merge16<HD>(r_ml, r_o, a.nch, ngrp, qa, NQ, ol, nullptr, nullptr, 0);
  }
  __syncthreads();
  attn_tile_out<HD>(a, h, qa, NQ, ol);
}

}  // namespace spx
