// Device building blocks shared by the one-row decode pipeline (decode.hip) and the persistent
// decode pass (persist.hip): typed global / LDS accesses, a K-quant block as one lane of its row
// group loads it, the input-row prologue (RMSNorm + Q8_K into LDS), the row-parallel block dots
// and per-lane chain, and the routing of one row. Every function computes the same values,
// operation for operation, wherever it is called from.
#pragma once
#include "decode.h"
#include "dev.h"

namespace spx {

// Address spaces are spelled out: pointers picked with selects (segments, gate / up) would
// otherwise become flat accesses, which also count against the LDS / scalar wait counter.
#define SPX_G __attribute__((address_space(1)))
#define SPX_L __attribute__((address_space(3)))
typedef int spx_i4 __attribute__((ext_vector_type(4)));
typedef int spx_i2 __attribute__((ext_vector_type(2)));
template <int N> struct GWord;
template <> struct GWord<16> { typedef spx_i4 type; };
template <> struct GWord<8> { typedef spx_i2 type; };
template <> struct GWord<4> { typedef int type; };
template <> struct GWord<2> { typedef unsigned short type; };
template <class T>
__device__ __forceinline__ T gld(const void *p) {
  typedef typename GWord<sizeof(T)>::type W;
  return __builtin_bit_cast(T, *(const SPX_G W *)p);
}
template <class T>
__device__ __forceinline__ T lld(const SPX_L void *p) {
  typedef typename GWord<sizeof(T)>::type W;
  return __builtin_bit_cast(T, *(const SPX_L W *)p);
}
template <class T>
__device__ __forceinline__ void lst(SPX_L void *p, T v) {
  typedef typename GWord<sizeof(T)>::type W;
  *(SPX_L W *)p = __builtin_bit_cast(W, v);
}
template <class T>
__device__ __forceinline__ void gst(void *p, T v) {
  typedef typename GWord<sizeof(T)>::type W;
  *(SPX_G W *)p = __builtin_bit_cast(W, v);
}

// ------------------------------------------------------------------ weight blocks in registers
// Raw bytes of one K-quant block as lane l of its row group loads them (the planar layout of
// kq.h): Q4_K a = codes, b = header; Q6_K a = ql, b = scales, c = qh, d = d.
struct DRaw {
  uint4 a, b;
  uint2 c;
  uint32_t d;
};

template <int T>
__device__ __forceinline__ void draw_load(DRaw &r, const Planes &pl, int64_t g, int l) {
  if constexpr (T == T_Q4K) {
    r.a = gld<uint4>(pl.p0 + g * 128 + 16 * l);
    r.b = gld<uint4>(pl.p1 + g * 16);
  } else {
    r.a = gld<uint4>(pl.p0 + g * 128 + 16 * l);
    r.c = gld<uint2>(pl.p1 + g * 64 + 8 * l);
    r.b = gld<uint4>(pl.p2 + g * 16);
    r.d = gld<uint16_t>(pl.p3 + g * 2);
  }
}

// All NB blocks of global row grow (blocks past nb re-load the last one: every lane issues
// the same number of loads, so the input row's wait never waits for the weights).
template <int T, int NB>
__device__ __forceinline__ void draw_row(DRaw (&raw)[NB], const Planes &pl, int64_t grow, int nb, int l) {
#pragma unroll
  for (int i = 0; i < NB; i++) draw_load<T>(raw[i], pl, grow * nb + min(i, nb - 1), l);
}

template <int T>
__device__ __forceinline__ KQRaw<T> draw_kq(const DRaw &r) {
  KQRaw<T> k;
  if constexpr (T == T_Q4K) {
    k.c = r.a;
    k.h = r.b;
  } else {
    k.ql = r.a;
    k.qh = r.c;
    k.sc = r.b;
    k.d = r.d;
  }
  return k;
}

// One row against the Q8_K row in LDS (blocks 0..nb-1): the reference's chain of rows<B,T>
// (quant_q8k.rs:198-243) exactly as kq_walk_tile runs it: per block the lane's scaled integer
// dot P and the group's correction integer, acc = fma(d * xd, float(P), acc), corr += term;
// the row is hsum(acc) - corr, valid in lane 0 of the row group.
template <int T, int NB>
__device__ __forceinline__ float dot_row(const DRaw (&raw)[NB], int nb, int l, const SPX_L uint32_t *lq, const SPX_L float *ld,
                                        const SPX_L int2 *lbs) {
  float acc = 0.0f, corr = 0.0f;
#pragma unroll
  for (int i = 0; i < NB; i++) {
    if (i < nb) {
      KQDec<T> dec;
      dec.decode(draw_kq<T>(raw[i]), l);
      const uint4 y0 = lld<uint4>(lq + i * 64 + 8 * l), y1 = lld<uint4>(lq + i * 64 + 8 * l + 4);
      int P, s;
      dec.dot(y0, y1, lld<int2>(lbs + i * 8 + l), P, s);
      s = sum8(s);
      const float xd = ld[i];
      corr = corr + dec.corr_term(xd, s);
      acc = fmaf(dec.d * xd, (float)P, acc);
    }
  }
  return hsum_rows8(acc) - corr;
}

// ------------------------------------------------------------------ input row prologue
// Wave w, lane j hold float4 j of the 256-value blocks w, w + NW, ... (KB of them).
template <int KB>
struct InRow {
  float4 v[KB], w[KB];
};

template <int NW, int KB>
__device__ __forceinline__ void in_load(const DecIn &in, InRow<KB> &r) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nbq = in.cols >> 8;
#pragma unroll
  for (int k = 0; k < KB; k++) {
    const int tb = wave + NW * k;
    r.v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    r.w[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tb < nbq) {
      r.v[k] = gld<float4>(in.x + 4 * (tb * 64 + lane));
      if (in.nw) r.w[k] = gld<float4>(in.nw + 4 * (tb * 64 + lane));
    }
  }
}

// rmsnorm (:569-575) as the norm tails compute it (per 256 block a wavefront tree, then the
// blocks in order; inv = 1 / sqrt(S / cols + eps) correctly rounded; x * inv * w), then
// quantize_avx2 of each block into the LDS image (lq, ld, lbs). xn_out: the normalised row.
template <int NW, int KB, class QP, class DP, class BP>
__device__ __forceinline__ void in_quant(const DecIn &in, InRow<KB> &r, QP lq, DP ld, BP lbs, SPX_L float *bsum, float *xn_out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nbq = in.cols >> 8;
  if (in.nw) {
#pragma unroll
    for (int k = 0; k < KB; k++) {
      const int tb = wave + NW * k;
      if (tb < nbq) {
        float p = r.v[k].x * r.v[k].x;
        p = fmaf(r.v[k].y, r.v[k].y, p);
        p = fmaf(r.v[k].z, r.v[k].z, p);
        p = fmaf(r.v[k].w, r.v[k].w, p);
        p = wave_sum(p);
        if (lane == 0) bsum[tb] = p;
      }
    }
    __syncthreads();
    float S = 0.0f;
    for (int k = 0; k < nbq; k++) S = S + bsum[k];
    const float inv = inv_rms(S, (float)in.cols, in.eps);
#pragma unroll
    for (int k = 0; k < KB; k++) {
      const int tb = wave + NW * k;
      if (tb < nbq) {
        float4 v = r.v[k];
        const float4 w = r.w[k];
        v.x = v.x * inv * w.x; v.y = v.y * inv * w.y; v.z = v.z * inv * w.z; v.w = v.w * inv * w.w;
        r.v[k] = v;
        if (xn_out) gst<float4>(xn_out + 4 * (tb * 64 + lane), v);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < KB; k++) {
    const int tb = wave + NW * k;
    if (tb < nbq) {
      const float am = q8k_amax(r.v[k]);
      q8k_block_store(r.v[k], am, lq + tb * 64, ld + tb, lbs + tb * 16);  // lbs: the bsum pairs as ints
    }
  }
}

// ------------------------------------------------------------------ row-parallel block dots
// A row's nb blocks are spread over the G row groups of its wavefront: group gi takes blocks
// gi, gi + G, ... (BPG of them, raw bytes in registers) and leaves per block, in the chain
// buffer cb (LDS), the 8 lane dots as floats, d * xd and the correction term. Then group 0
// runs the reference's per-lane chain over the blocks in order (acc_l = fma(d * xd,
// float(P_l), acc_l), corr += term) exactly as kq_walk_tile does: the same fp32 values.
template <int T, int BPG>
__device__ __forceinline__ void rp_dots(const DRaw (&raw)[BPG], int nb, int G, int gi, int l, const SPX_L uint32_t *lq, const SPX_L float *ld,
                                        const SPX_L int2 *lbs, SPX_L float *cbr) {
#pragma unroll
  for (int j = 0; j < BPG; j++) {
    const int i = gi + G * j;
    if (i < nb) {
      KQDec<T> dec;
      dec.decode(draw_kq<T>(raw[j]), l);
      const uint4 y0 = lld<uint4>(lq + i * 64 + 8 * l), y1 = lld<uint4>(lq + i * 64 + 8 * l + 4);
      int P, s;
      dec.dot(y0, y1, lld<int2>(lbs + i * 8 + l), P, s);
      s = sum8(s);
      const float xd = ld[i];
      SPX_L float *e = cbr + i * 10;
      e[l] = (float)P;
      if (l == 0) { e[8] = dec.d * xd; e[9] = dec.corr_term(xd, s); }
    }
  }
}
// rp_dots for NV input rows against the same weights: each block decoded once, its dot with
// every row as rp_dots forms it (the same values), each row's results to its chain buffer.
template <int T, int BPG, int NV>
__device__ __forceinline__ void rp_dots_nv(const DRaw (&raw)[BPG], int nb, int G, int gi, int l, const SPX_L uint32_t *const (&lq)[NV],
                                           const SPX_L float *const (&ld)[NV], const SPX_L int2 *const (&lbs)[NV], SPX_L float *const (&cbr)[NV]) {
#pragma unroll
  for (int j = 0; j < BPG; j++) {
    const int i = gi + G * j;
    if (i < nb) {
      KQDec<T> dec;
      dec.decode(draw_kq<T>(raw[j]), l);
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const uint4 y0 = lld<uint4>(lq[v] + i * 64 + 8 * l), y1 = lld<uint4>(lq[v] + i * 64 + 8 * l + 4);
        int P, s;
        dec.dot(y0, y1, lld<int2>(lbs[v] + i * 8 + l), P, s);
        s = sum8(s);
        const float xd = ld[v][i];
        SPX_L float *e = cbr[v] + i * 10;
        e[l] = (float)P;
        if (l == 0) { e[8] = dec.d * xd; e[9] = dec.corr_term(xd, s); }
      }
    }
  }
}
// The chain over the row's blocks (group 0); the row result in lane 0 of the group.
__device__ __forceinline__ float rp_chain(const SPX_L float *cbr, int nb, int l) {
  float acc = 0.0f, cr = 0.0f;
  for (int i = 0; i < nb; i++) {
    const SPX_L float *e = cbr + i * 10;
    acc = fmaf(e[8], e[l], acc);
    cr = cr + e[9];
  }
  return hsum_rows8(acc) - cr;
}

template <int T, int BPG>
__device__ __forceinline__ void rp_load(DRaw (&raw)[BPG], const Planes &pl, int64_t grow, int nb, int G, int gi, int l) {
#pragma unroll
  for (int j = 0; j < BPG; j++) draw_load<T>(raw[j], pl, grow * nb + min(gi + G * j, nb - 1), l);
}

// ------------------------------------------------------------------ routing of one row
// moe_forward's routing (:1199-1239) as k_router computes it for a row: softmax (max, exp,
// sum, divide), top-n_used by probability (ties to the lower expert index), pruning
// (moe_prune >= 1: keep clamp(x, max(2, n/2), n); < 1: the mass rule), the weights' sum over
// the kept choices in choice order. lv[k] = logit of expert lane + 64k. Lane i < n_used ends
// with choice i (my_e, my_p); keep and wsum in every lane.
__device__ __forceinline__ void route_row(const float (&lv)[4], int ne, int nu, float moe_prune, int &my_e, float &my_p, int &keep,
                                          float &wsum) {
  const int lane = threadIdx.x & 63;
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < 4; k++) mx = fmaxf(mx, lv[k]);
  mx = wave_max(mx);
  float pv[4], sum = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) { const int e = lane + 64 * k; pv[k] = e < ne ? expf(lv[k] - mx) : 0.0f; sum += pv[k]; }
  sum = wave_sum(sum);
  // key = probability bits + 1 (non-negative floats order as their bits); 0: no expert or
  // taken. Each round: the wave's largest key, then the lowest expert index holding it
  // (experts lane + 64k, k ascending, by ballots).
  uint32_t key[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int e = lane + 64 * k;
    if (e < ne) pv[k] = pv[k] / sum;
    key[k] = e < ne ? __float_as_uint(pv[k]) + 1u : 0u;
  }
  my_e = 0;
  my_p = 0.0f;
  for (int i = 0; i < nu; i++) {
    const uint32_t bk = wave_max_u32(max(max(key[0], key[1]), max(key[2], key[3])));
    int e = 0;
#pragma unroll
    for (int k = 3; k >= 0; k--) {
      const unsigned long long bal = __ballot(key[k] == bk);
      if (bal) e = 64 * k + (int)__builtin_ctzll(bal);
    }
    if (lane == i) { my_e = e; my_p = __uint_as_float(bk - 1u); }
    if ((e & 63) == lane) {
      const int k = e >> 6;
      if (k == 0) key[0] = 0u; else if (k == 1) key[1] = 0u; else if (k == 2) key[2] = 0u; else key[3] = 0u;
    }
  }
  keep = nu;
  if (moe_prune > 0.0f && nu > 2) {
    const int min_keep = max(2, nu / 2);
    if (moe_prune >= 1.0f) keep = min(max((int)moe_prune, min_keep), nu);
    else {
      float top = 0.0f;
      for (int i = 0; i < nu; i++) top += lane_f(my_p, i);
      const float target = top * (1.0f - moe_prune);
      float cum = 0.0f;
      int k = 0;
      while (k < nu && (k < min_keep || cum < target)) { cum += lane_f(my_p, k); k++; }
      keep = k;
    }
  }
  wsum = 0.0f;
  for (int i = 0; i < keep; i++) wsum += lane_f(my_p, i);
}

}  // namespace spx
