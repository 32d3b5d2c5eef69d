// One-row decode pipeline for gfx950 (wave64): forward_slice (smollm_chat.rs:3364-3552) of a
// single token as a chain of kernels that meet only at kernel boundaries. Per layer:
//   kd_mv (q|k|v)     attn_norm + Q8_K of the residual row in every workgroup's LDS, then
//                     the three integer projections (eight rows per wavefront)
//   attention         split-K partials (k_attn without its merge, fused.hip), then kd_merge
//   kd_mv (wo)        Q8_K of the attention row, attn_output, + the residual add
//   kd_router         ffn_norm in every workgroup, one F32 router row per workgroup
//   kd_gateup         every wavefront routes the row (softmax, top-k, pruning, weights), then
//                     gate/up + SwiGLU of the chosen experts (or the dense FFN)
//   kd_down           Q8_K of h in every workgroup's LDS, the chosen experts' down rows, the
//                     weighted combine and the residual add (a dense down is kd_mv)
// and at the end kd_mv over the LM head (output_norm in every workgroup) with greedy keys.
// A workgroup first issues the loads of its input row, then its weight loads, then computes
// the norm / Q8_K while the weights are in flight. Every result is the same fp32 value, bit
// for bit, as the fused pipeline's (same operations in the same order: the norm's fixed-order
// sum, quantize_avx2, the reference's per-lane integer-dot chain, the router's lane chains
// and wave tree, the combine's chosen-order sum); only where the work is done changes.
#include <type_traits>
#include "decode.h"
#include "decode_dev.h"
#include "dev.h"

namespace spx {

// Lambdas of the matrix-core walks are inlined: a lambda left out of line would take its
// array arguments (the block ring, a tile's results) through scratch memory.
#define SPX_AI __attribute__((always_inline))

// ------------------------------------------------------------------ integer matvec, one row
// DEC_MV_NW wavefronts per workgroup; a wavefront takes R rows with G row groups each
// (G * R = 8, G = the power of two >= nb, at most 8), so tiles of DEC_MV_NW * R rows stride
// over the grid (the LM head runs on fewer workgroups than tiles). TT = the segments' format,
// or 0 when they differ (then per segment).
template <int TT, int BPG, int PD>
__global__ __launch_bounds__(DEC_MV_NW * 64) __attribute__((amdgpu_waves_per_eu(PD == 1 ? 8 : 4))) void kd_mv(const DecMVArgs a) {
  constexpr int NW = DEC_MV_NW, KB = (DEC_MAXNB + NW - 1) / NW;
  __shared__ __align__(16) uint32_t lq_[DEC_MAXNB * 64];
  __shared__ float ld_[DEC_MAXNB];
  __shared__ __align__(16) int2 lbs_[DEC_MAXNB * 8];
  __shared__ float bsum_[DEC_MAXNB];
  __shared__ float cb_[NW][8 * 10 * 2];  // per wavefront R * nb <= 16 blocks x 10 floats
  __shared__ unsigned long long sbest[NW];
  SPX_L uint32_t *lq = (SPX_L uint32_t *)lq_;
  SPX_L float *ld = (SPX_L float *)ld_, *bsum = (SPX_L float *)bsum_;
  SPX_L int2 *lbs = (SPX_L int2 *)lbs_;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane >> 3, l = lane & 7;
  const int nb = a.in.cols >> 8, G = a.G, R = 8 / G, r = grp / G, gi = grp - r * G;
  SPX_L float *cbr = (SPX_L float *)cb_[wave] + r * nb * 10;
  const int t0 = a.tiles[0], t1 = a.nseg > 1 ? a.tiles[1] : 0, t2 = a.nseg > 2 ? a.tiles[2] : 0;
  const int total = t0 + t1 + t2;
  // segment and row of tile t; the segments' fields are all read from the kernel arguments
  // up front and picked with wave-uniform selects (an indexed argument access would chain
  // dependent scalar loads ahead of the weight loads)
  const Planes pl0 = a.w[0].pl, pl1 = a.w[1].pl, pl2 = a.w[2].pl;
  const int64_t rw0 = a.w[0].rows, rw1 = a.w[1].rows, rw2 = a.w[2].rows;
  const int dt0 = a.w[0].dtype, dt1 = a.w[1].dtype, dt2 = a.w[2].dtype;
  float *const o0 = a.out[0], *const o1 = a.out[1], *const o2 = a.out[2];
  InRow<KB> in;
  in_load<NW, KB>(a.in, in);  // the input row's loads go first
  unsigned long long bestk = 0;
  if constexpr (PD == 1) {
    DRaw raw[BPG];
    const int t = min((int)blockIdx.x, total - 1);
    const int si = __builtin_amdgcn_readfirstlane(t >= t0 ? (t >= t0 + t1 ? 2 : 1) : 0);
    const int tt = t - (si > 0 ? t0 : 0) - (si > 1 ? t1 : 0);
    const int64_t row = ((int64_t)tt * NW + wave) * R + r;
    const int64_t rows = si == 0 ? rw0 : si == 1 ? rw1 : rw2;
    const int dt = si == 0 ? dt0 : si == 1 ? dt1 : dt2;
    float *const out = si == 0 ? o0 : si == 1 ? o1 : o2;
    Planes pl;
    pl.p0 = si == 0 ? pl0.p0 : si == 1 ? pl1.p0 : pl2.p0;
    pl.p1 = si == 0 ? pl0.p1 : si == 1 ? pl1.p1 : pl2.p1;
    pl.p2 = si == 0 ? pl0.p2 : si == 1 ? pl1.p2 : pl2.p2;
    pl.p3 = si == 0 ? pl0.p3 : si == 1 ? pl1.p3 : pl2.p3;
    const int64_t grow = row < rows ? row : rows - 1;
    if (TT == T_Q4K || (TT == 0 && dt == T_Q4K)) rp_load<T_Q4K, BPG>(raw, pl, grow, nb, G, gi, l);
    else rp_load<T_Q6K, BPG>(raw, pl, grow, nb, G, gi, l);
    in_quant<NW, KB>(a.in, in, lq, ld, (SPX_L int *)lbs, bsum, blockIdx.x == 0 ? a.xn_out : nullptr);
    __syncthreads();
    if ((int)blockIdx.x < total) {
      if (TT == T_Q4K || (TT == 0 && dt == T_Q4K)) rp_dots<T_Q4K, BPG>(raw, nb, G, gi, l, lq, ld, lbs, cbr);
      else rp_dots<T_Q6K, BPG>(raw, nb, G, gi, l, lq, ld, lbs, cbr);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the chain buffer is written
      __builtin_amdgcn_wave_barrier();
      if (gi == 0) {
        const float res = rp_chain(cbr, nb, l);
        if (l == 0 && row < rows) {
          if (out) gst<float>(out + row, res);
          if (a.res_out) gst<float>(a.res_out + row, gld<float>(a.res_in + row) + a.rscale * res);
          if (a.best) bestk = pick_key(res, a.lscale, row);
        }
      }
    }
  } else {
    // one segment (TT fixed), tiles blockIdx.x + k * gridDim.x; PD tiles' weights in flight
    static_assert(TT == T_Q4K || TT == T_Q6K, "prefetched launches take one format");
    DRaw raw[PD][BPG];
    const int64_t rows = rw0;
    const int g = gridDim.x;
    auto row_of = [&](int t) { return ((int64_t)t * NW + wave) * R + r; };
#pragma unroll
    for (int k = 0; k < PD; k++) {
      const int64_t row = row_of(min((int)blockIdx.x + k * g, total - 1));
      rp_load<TT, BPG>(raw[k], pl0, row < rows ? row : rows - 1, nb, G, gi, l);
    }
    in_quant<NW, KB>(a.in, in, lq, ld, (SPX_L int *)lbs, bsum, blockIdx.x == 0 ? a.xn_out : nullptr);
    __syncthreads();
    for (int t = blockIdx.x; t < total;) {
#pragma unroll
      for (int k = 0; k < PD; k++) {
        if (t < total) {
          rp_dots<TT, BPG>(raw[k], nb, G, gi, l, lq, ld, lbs, cbr);
          const int64_t nrow = row_of(min(t + PD * g, total - 1));
          rp_load<TT, BPG>(raw[k], pl0, nrow < rows ? nrow : rows - 1, nb, G, gi, l);  // tile t + PD * g
          __builtin_amdgcn_s_waitcnt(0xc07f);
          __builtin_amdgcn_wave_barrier();
          const int64_t row = row_of(t);
          if (gi == 0) {
            const float res = rp_chain(cbr, nb, l);
            if (l == 0 && row < rows) {
              if (o0) gst<float>(o0 + row, res);
              if (a.res_out) gst<float>(a.res_out + row, gld<float>(a.res_in + row) + a.rscale * res);
              if (a.best) {
                const unsigned long long key = pick_key(res, a.lscale, row);
                bestk = key > bestk ? key : bestk;
              }
            }
          }
          __builtin_amdgcn_s_waitcnt(0xc07f);
          __builtin_amdgcn_wave_barrier();  // the chain buffer is refilled by the next tile
        }
        t += g;
      }
    }
  }
  if (a.best) {
    const unsigned long long b = wave_max_u64(bestk);
    if (lane == 0) sbest[wave] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned long long rb = sbest[0];
      for (int w = 1; w < NW; w++) rb = sbest[w] > rb ? sbest[w] : rb;
      gst<unsigned long long>(a.best + blockIdx.x, rb);
    }
  }
}

// ------------------------------------------------------------------ integer matvec, two rows
// kd_mv for the NV rows of a two-row pass (input rows x + v cols, outputs out + v rows,
// greedy keys best + v gridDim.x): each row with its own prologue, chains and epilogue, the
// weights loaded once, so each row gets its one-row pass's bits.
template <int TT, int BPG, int PD, int NV>
__global__ __launch_bounds__(DEC_MV_NW * 64) __attribute__((amdgpu_waves_per_eu(PD == 1 ? 4 : 2))) void kd_mv2(const DecMVArgs a) {
  constexpr int NW = DEC_MV_NW, KB = (DEC_MAXNB + NW - 1) / NW;
  __shared__ __align__(16) uint32_t lq_[NV][DEC_MAXNB * 64];
  __shared__ float ld_[NV][DEC_MAXNB];
  __shared__ __align__(16) int2 lbs_[NV][DEC_MAXNB * 8];
  __shared__ float bsum_[NV][DEC_MAXNB];
  __shared__ float cb_[NV][NW][8 * 10 * 2];  // per wavefront R * nb <= 16 blocks x 10 floats
  __shared__ unsigned long long sbest[NV][NW];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane >> 3, l = lane & 7;
  const int nb = a.in.cols >> 8, G = a.G, R = 8 / G, r = grp / G, gi = grp - r * G;
  const int t0 = a.tiles[0], t1 = a.nseg > 1 ? a.tiles[1] : 0, t2 = a.nseg > 2 ? a.tiles[2] : 0;
  const int total = t0 + t1 + t2;
  // segment and row of tile t; the segments' fields are all read from the kernel arguments
  // up front and picked with wave-uniform selects (an indexed argument access would chain
  // dependent scalar loads ahead of the weight loads)
  const Planes pl0 = a.w[0].pl, pl1 = a.w[1].pl, pl2 = a.w[2].pl;
  const int64_t rw0 = a.w[0].rows, rw1 = a.w[1].rows, rw2 = a.w[2].rows;
  const int dt0 = a.w[0].dtype, dt1 = a.w[1].dtype, dt2 = a.w[2].dtype;
  float *const o0 = a.out[0], *const o1 = a.out[1], *const o2 = a.out[2];
  auto in_of = [&](int v) SPX_AI { return DecIn{a.in.x + (int64_t)v * a.in.cols, a.in.nw, a.in.eps, a.in.cols}; };
  auto xn_of = [&](int v) SPX_AI { return blockIdx.x == 0 && a.xn_out ? a.xn_out + (int64_t)v * a.in.cols : nullptr; };
  InRow<KB> in[NV];
#pragma unroll
  for (int v = 0; v < NV; v++) in_load<NW, KB>(in_of(v), in[v]);  // the input rows' loads go first
  const SPX_L uint32_t *lqv[NV];
  const SPX_L float *ldv[NV];
  const SPX_L int2 *lbsv[NV];
  SPX_L float *cbrv[NV];
#pragma unroll
  for (int v = 0; v < NV; v++) {
    lqv[v] = (SPX_L uint32_t *)lq_[v];
    ldv[v] = (SPX_L float *)ld_[v];
    lbsv[v] = (SPX_L int2 *)lbs_[v];
    cbrv[v] = (SPX_L float *)cb_[v][wave] + r * nb * 10;
  }
  unsigned long long bestk[NV];
#pragma unroll
  for (int v = 0; v < NV; v++) bestk[v] = 0;
  if constexpr (PD == 1) {
    DRaw raw[BPG];
    const int t = min((int)blockIdx.x, total - 1);
    const int si = __builtin_amdgcn_readfirstlane(t >= t0 ? (t >= t0 + t1 ? 2 : 1) : 0);
    const int tt = t - (si > 0 ? t0 : 0) - (si > 1 ? t1 : 0);
    const int64_t row = ((int64_t)tt * NW + wave) * R + r;
    const int64_t rows = si == 0 ? rw0 : si == 1 ? rw1 : rw2;
    const int dt = si == 0 ? dt0 : si == 1 ? dt1 : dt2;
    float *const out = si == 0 ? o0 : si == 1 ? o1 : o2;
    Planes pl;
    pl.p0 = si == 0 ? pl0.p0 : si == 1 ? pl1.p0 : pl2.p0;
    pl.p1 = si == 0 ? pl0.p1 : si == 1 ? pl1.p1 : pl2.p1;
    pl.p2 = si == 0 ? pl0.p2 : si == 1 ? pl1.p2 : pl2.p2;
    pl.p3 = si == 0 ? pl0.p3 : si == 1 ? pl1.p3 : pl2.p3;
    const int64_t grow = row < rows ? row : rows - 1;
    if (TT == T_Q4K || (TT == 0 && dt == T_Q4K)) rp_load<T_Q4K, BPG>(raw, pl, grow, nb, G, gi, l);
    else rp_load<T_Q6K, BPG>(raw, pl, grow, nb, G, gi, l);
#pragma unroll
    for (int v = 0; v < NV; v++)
      in_quant<NW, KB>(in_of(v), in[v], (SPX_L uint32_t *)lq_[v], (SPX_L float *)ld_[v], (SPX_L int *)lbs_[v], (SPX_L float *)bsum_[v], xn_of(v));
    __syncthreads();
    if ((int)blockIdx.x < total) {
      if (TT == T_Q4K || (TT == 0 && dt == T_Q4K)) rp_dots_nv<T_Q4K, BPG, NV>(raw, nb, G, gi, l, lqv, ldv, lbsv, cbrv);
      else rp_dots_nv<T_Q6K, BPG, NV>(raw, nb, G, gi, l, lqv, ldv, lbsv, cbrv);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the chain buffer is written
      __builtin_amdgcn_wave_barrier();
      if (gi == 0) {
#pragma unroll
        for (int v = 0; v < NV; v++) {
          const float res = rp_chain((SPX_L float *)cb_[v][wave] + r * nb * 10, nb, l);
          if (l == 0 && row < rows) {
            const int64_t ro = (int64_t)v * rows + row;
            if (out) gst<float>(out + ro, res);
            if (a.res_out) gst<float>(a.res_out + ro, gld<float>(a.res_in + ro) + a.rscale * res);
            if (a.best) bestk[v] = pick_key(res, a.lscale, row);
          }
        }
      }
    }
  } else {
    // one segment (TT fixed), tiles blockIdx.x + k * gridDim.x; PD tiles' weights in flight
    static_assert(TT == T_Q4K || TT == T_Q6K, "prefetched launches take one format");
    DRaw raw[PD][BPG];
    const int64_t rows = rw0;
    const int g = gridDim.x;
    auto row_of = [&](int t) { return ((int64_t)t * NW + wave) * R + r; };
#pragma unroll
    for (int k = 0; k < PD; k++) {
      const int64_t row = row_of(min((int)blockIdx.x + k * g, total - 1));
      rp_load<TT, BPG>(raw[k], pl0, row < rows ? row : rows - 1, nb, G, gi, l);
    }
#pragma unroll
    for (int v = 0; v < NV; v++)
      in_quant<NW, KB>(in_of(v), in[v], (SPX_L uint32_t *)lq_[v], (SPX_L float *)ld_[v], (SPX_L int *)lbs_[v], (SPX_L float *)bsum_[v], xn_of(v));
    __syncthreads();
    for (int t = blockIdx.x; t < total;) {
#pragma unroll
      for (int k = 0; k < PD; k++) {
        if (t < total) {
          rp_dots_nv<TT, BPG, NV>(raw[k], nb, G, gi, l, lqv, ldv, lbsv, cbrv);
          const int64_t nrow = row_of(min(t + PD * g, total - 1));
          rp_load<TT, BPG>(raw[k], pl0, nrow < rows ? nrow : rows - 1, nb, G, gi, l);  // tile t + PD * g
          __builtin_amdgcn_s_waitcnt(0xc07f);
          __builtin_amdgcn_wave_barrier();
          const int64_t row = row_of(t);
          if (gi == 0) {
#pragma unroll
            for (int v = 0; v < NV; v++) {
              const float res = rp_chain((SPX_L float *)cb_[v][wave] + r * nb * 10, nb, l);
              if (l == 0 && row < rows) {
                const int64_t ro = (int64_t)v * rows + row;
                if (o0) gst<float>(o0 + ro, res);
                if (a.res_out) gst<float>(a.res_out + ro, gld<float>(a.res_in + ro) + a.rscale * res);
                if (a.best) {
                  const unsigned long long key = pick_key(res, a.lscale, row);
                  bestk[v] = key > bestk[v] ? key : bestk[v];
                }
              }
            }
          }
          __builtin_amdgcn_s_waitcnt(0xc07f);
          __builtin_amdgcn_wave_barrier();  // the chain buffer is refilled by the next tile
        }
        t += g;
      }
    }
  }
  if (a.best) {
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const unsigned long long b = wave_max_u64(bestk[v]);
      if (lane == 0) sbest[v][wave] = b;
    }
    __syncthreads();
    if (threadIdx.x < NV) {
      const int v = threadIdx.x;
      unsigned long long rb = sbest[v][0];
      for (int w = 1; w < NW; w++) rb = sbest[v][w] > rb ? sbest[v][w] : rb;
      gst<unsigned long long>(a.best + (int64_t)v * gridDim.x + blockIdx.x, rb);
    }
  }
}

// ------------------------------------------------------------------ attention merge
// One workgroup per query head of the row, 1024 threads. Thread (d, gs): output value d of
// the head, chunk groups gs, gs + 1024 / HD, ...: each group of ATT_GRP chunks is merged as
// the fused kernel's first level does (M = max m_c, w_c = exp(m_c - M), L = sum l_c w_c,
// O = sum w_c o_c in chunk order), then the groups in group order; O / L is the output.
template <int HD>
__global__ __launch_bounds__(1024) void kd_merge(const DecMergeArgs a, const StepRec *st) {
  constexpr int NGS = 1024 / HD;
  __shared__ float sO[ATT_GMAX][HD];
  __shared__ float sM[ATT_GMAX], sL[ATT_GMAX];
  const int t = threadIdx.x, d = t % HD, gs = t / HD, head = blockIdx.x;
  const int g = a.n_heads / a.n_kv, h = head / g, qi = head % g;
  const float2 *pml = reinterpret_cast<const float2 *>(a.part_ml) + ((int64_t)h * a.nslot) * ATT_QMAX + qi;
  const float *po = a.part_o + ((int64_t)h * a.nslot * ATT_QMAX + qi) * HD + d;
  // group gs's slots are requested before the step record arrives (slots past the pass's
  // chunks hold earlier values, never used)
  float2 ml0[ATT_GRP];
  float ov0[ATT_GRP];
#pragma unroll
  for (int k = 0; k < ATT_GRP; k++) {
    const int c = min(gs * ATT_GRP + k, a.nslot - 1);
    ml0[k] = pml[(int64_t)c * ATT_QMAX];
    ov0[k] = po[(int64_t)c * ATT_QMAX * HD];
  }
  const int total = st->start + 1, nch = (total + 63) >> 6, ngrp = (nch + ATT_GRP - 1) / ATT_GRP;
  for (int gi = gs; gi < ngrp; gi += NGS) {
    const int s0 = gi * ATT_GRP, n = min(ATT_GRP, nch - s0);
    float2 ml[ATT_GRP];
    float ov[ATT_GRP];
#pragma unroll
    for (int k = 0; k < ATT_GRP; k++) {
      if (gi == gs) {
        ml[k] = k < n ? ml0[k] : make_float2(-INFINITY, 0.0f);
        ov[k] = ov0[k];
      } else {
        const int c = s0 + min(k, n - 1);
        ml[k] = k < n ? pml[(int64_t)c * ATT_QMAX] : make_float2(-INFINITY, 0.0f);
        ov[k] = po[(int64_t)c * ATT_QMAX * HD];
      }
    }
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < ATT_GRP; k++) M = fmaxf(M, ml[k].x);
    float L = 0.0f, acc = 0.0f;
#pragma unroll
    for (int k = 0; k < ATT_GRP; k++) {
      if (k < n) {  // chunks past n (padding: weight 0) are skipped
        const float w = ml[k].x == -INFINITY ? 0.0f : expf(ml[k].x - M);
        L = fmaf(ml[k].y, w, L);
        acc = fmaf(ov[k], w, acc);
      }
    }
    sO[gi][d] = acc;
    if (d == 0) { sM[gi] = M; sL[gi] = L; }
  }
  __syncthreads();
  if (gs != 0) return;
  float out;
  if (ngrp == 1) {
    out = sO[0][d] * __fdiv_rn(1.0f, fmaxf(sL[0], 1e-30f));
  } else {
    float M = -INFINITY;
    for (int k = 0; k < ngrp; k++) M = fmaxf(M, sM[k]);
    float L = 0.0f, acc = 0.0f;
    for (int k = 0; k < ngrp; k++) {
      const float w = sM[k] == -INFINITY ? 0.0f : expf(sM[k] - M);
      L = fmaf(sL[k], w, L);
      acc = fmaf(sO[k][d], w, acc);
    }
    out = acc * __fdiv_rn(1.0f, fmaxf(L, 1e-30f));
  }
  a.att[(int64_t)head * HD + d] = out;
}

// ------------------------------------------------------------------ router
// One F32 router row per workgroup (k_router's arithmetic: wavefront w, lane j hold float4s
// w*64 + j + 256k; the lane's fma chain, the wave tree, the four wavefronts in order) against
// the ffn_norm'd row, which every workgroup computes for itself. NV = 2: both rows of a
// two-row pass against the row's weights, logits [v][n_expert].
template <int NV = 1>
__global__ __launch_bounds__(256) void kd_router(const DecRouterArgs a) {
  constexpr int NK = DEC_MAXNB / 4;
  __shared__ float bsum[NV][DEC_MAXNB];
  __shared__ float part[NV][4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, row = blockIdx.x;
  const int dim = a.in.cols, n4 = dim >> 2;
  InRow<NK> in[NV];
#pragma unroll
  for (int v = 0; v < NV; v++) in_load<4, NK>(DecIn{a.in.x + (int64_t)v * dim, a.in.nw, a.in.eps, dim}, in[v]);
  const float4 *wr = reinterpret_cast<const float4 *>(a.w.pl.p0 + (int64_t)row * dim * 4);
  float4 wv[NK];
#pragma unroll
  for (int k = 0; k < NK; k++) {
    const int f = wave * 64 + lane + 256 * k;
    wv[k] = f < n4 ? wr[f] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // normalise in registers (block tb = wave + 4k holds float4 f = tb * 64 + lane)
  const int nbq = dim >> 8;
#pragma unroll
  for (int v = 0; v < NV; v++)
#pragma unroll
    for (int k = 0; k < NK; k++) {
      const int tb = wave + 4 * k;
      if (tb < nbq) {
        float p = in[v].v[k].x * in[v].v[k].x;
        p = fmaf(in[v].v[k].y, in[v].v[k].y, p);
        p = fmaf(in[v].v[k].z, in[v].v[k].z, p);
        p = fmaf(in[v].v[k].w, in[v].v[k].w, p);
        p = wave_sum(p);
        if (lane == 0) bsum[v][tb] = p;
      }
    }
  __syncthreads();
#pragma unroll
  for (int v = 0; v < NV; v++) {
    float S = 0.0f;
    for (int k = 0; k < nbq; k++) S = S + bsum[v][k];
    const float inv = inv_rms(S, (float)dim, a.in.eps);
    float pv = 0.0f;
#pragma unroll
    for (int k = 0; k < NK; k++) {
      const int f = wave * 64 + lane + 256 * k;
      if (f < n4) {
        float4 x = in[v].v[k];
        const float4 w = in[v].w[k];
        x.x = x.x * inv * w.x; x.y = x.y * inv * w.y; x.z = x.z * inv * w.z; x.w = x.w * inv * w.w;
        pv = fmaf(wv[k].x, x.x, pv);
        pv = fmaf(wv[k].y, x.y, pv);
        pv = fmaf(wv[k].z, x.z, pv);
        pv = fmaf(wv[k].w, x.w, pv);
      }
    }
    const float tsum = wave_sum(pv);
    if (lane == 0) part[v][wave] = tsum;
  }
  __syncthreads();
  if (threadIdx.x < NV) {
    const int v = threadIdx.x;
    a.logits[(int64_t)v * a.n_expert + row] = ((part[v][0] + part[v][1]) + part[v][2]) + part[v][3];
  }
}

// ------------------------------------------------------------------ gate / up + SwiGLU
// Grid (n_ff / DEC_MV_NW, n_used): workgroup (x, s) computes rows DEC_MV_NW * x .. of h for
// chosen slot s, one row per wavefront: lanes 0-31 take the gate row, 32-63 the up row, four
// row groups each (blocks gi, gi + 4, ...), chains as rp_chain. h[s][r] = silu(g) * u (silu
// :586-588). Wavefront 0 routes the row; workgroup (0, 0) publishes the routing for kd_down
// (chosen experts, weights, kept count). NV = 2: the two rows of a two-row pass, wavefront v
// routing row v; workgroup (x, s) takes slot s of both rows (each its own expert's gate / up
// rows and its own Q8_K input), h[v n_used + s], chosen / weights [v][n_used], nkeep [v].
template <int T, int BPG, int NV = 1>
__device__ __forceinline__ void gateup_body(const DecGateUpArgs &a) {
  constexpr int NW = DEC_MV_NW, KB = (DEC_MAXNB + NW - 1) / NW;
  __shared__ __align__(16) uint32_t lq_[NV][DEC_MAXNB * 64];
  __shared__ float ld_[NV][DEC_MAXNB];
  __shared__ __align__(16) int2 lbs_[NV][DEC_MAXNB * 8];
  __shared__ float bsum_[NV][DEC_MAXNB];
  __shared__ float cb_[NV][NW][2 * DEC_MAXNB * 10];
  __shared__ int s_route[NV][2];
  __shared__ int s_ch[NV > 1 ? NV : 1][32];  // NV = 2: each row's kept experts (the pass's union)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane >> 3, l = lane & 7;
  const int half = grp >> 2, gi = grp & 3;  // half 0: gate row, 1: up row
  const int n_ff = a.n_ff, nb = a.in.cols >> 8;
  const int r = blockIdx.x * NW + wave;
  const bool valid = r < n_ff;
  float lv[4];
  if (a.logits && wave < NV) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int e = lane + 64 * k;
      lv[k] = e < a.n_expert ? gld<float>(a.logits + (int64_t)wave * a.n_expert + e) : -INFINITY;
    }
  }
  auto in_of = [&](int v) SPX_AI { return DecIn{a.in.x + (int64_t)v * a.in.cols, a.in.nw, a.in.eps, a.in.cols}; };
  InRow<KB> in[NV];
#pragma unroll
  for (int v = 0; v < NV; v++) in_load<NW, KB>(in_of(v), in[v]);
  int expert[NV];
  bool live[NV];
#pragma unroll
  for (int v = 0; v < NV; v++) { expert[v] = 0; live[v] = true; }
  if (a.logits) {
    if (wave < NV) {
      const int v = wave;
      int my_e, keep;
      float my_p, wsum;
      route_row(lv, a.n_expert, a.n_used, a.moe_prune, my_e, my_p, keep, wsum);
      if (blockIdx.x == 0 && blockIdx.y == 0) {
        if (lane < keep) {
          gst<int>(a.chosen + v * a.n_used + lane, my_e);
          gst<float>(a.weights + v * a.n_used + lane, a.norm ? my_p / wsum : my_p);
          if constexpr (NV == 1) {
            if (a.expert_count) gst<int>(a.expert_count + my_e, gld<int>(a.expert_count + my_e) + 1);
          } else {
            s_ch[v][lane] = my_e;
          }
        }
        if (lane == 0) {
          gst<int>(a.nkeep + v, keep);
          if constexpr (NV == 1) gst<int>(a.njobs, keep);
        }
      }
      if (lane == 0) { s_route[v][0] = lane_i(my_e, blockIdx.y); s_route[v][1] = keep; }
    }
    __syncthreads();
    bool any = false;
#pragma unroll
    for (int v = 0; v < NV; v++) {
      live[v] = (int)blockIdx.y < s_route[v][1];
      any = any || live[v];
      expert[v] = s_route[v][0];
    }
    if constexpr (NV > 1) {
      // the pass's distinct experts (row 0's kept choices, then row 1's not among them): the
      // job count and one selection count each, as the multi-row passes count them
      if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0) {
        const int k0 = s_route[0][1], k1 = s_route[1][1];
        bool fresh = false;
        int e1 = 0;
        if (lane < k1) {
          e1 = s_ch[1][lane];
          fresh = true;
          for (int j = 0; j < k0; j++) fresh = fresh && s_ch[0][j] != e1;
        }
        if (a.expert_count) {
          if (lane < k0) gst<int>(a.expert_count + s_ch[0][lane], gld<int>(a.expert_count + s_ch[0][lane]) + 1);
          if (fresh) gst<int>(a.expert_count + e1, gld<int>(a.expert_count + e1) + 1);
        }
        const int nfresh = __popcll(__ballot(fresh));
        if (lane == 0) gst<int>(a.njobs, k0 + nfresh);
      }
    }
    if (!any) return;  // a pruned slot of every row (the whole workgroup)
  }
  DRaw raw[NV][BPG];
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int64_t grow = (int64_t)expert[v] * a.gate.rows + (valid ? r : n_ff - 1);
    rp_load<T, BPG>(raw[v], half ? a.up.pl : a.gate.pl, grow, nb, 4, gi, l);
  }
#pragma unroll
  for (int v = 0; v < NV; v++)
    in_quant<NW, KB>(in_of(v), in[v], (SPX_L uint32_t *)lq_[v], (SPX_L float *)ld_[v], (SPX_L int *)lbs_[v], (SPX_L float *)bsum_[v], nullptr);
  __syncthreads();
#pragma unroll
  for (int v = 0; v < NV; v++)
    rp_dots<T, BPG>(raw[v], nb, 4, gi, l, (SPX_L uint32_t *)lq_[v], (SPX_L float *)ld_[v], (SPX_L int2 *)lbs_[v],
                    (SPX_L float *)cb_[v][wave] + half * nb * 10);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the chain buffer is written
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const float res = gi == 0 ? rp_chain((SPX_L float *)cb_[v][wave] + half * nb * 10, nb, l) : 0.0f;
    uint32_t r_lo, r_hi;  // lanes 0-31 get the up row's result from lanes 32-63
    xchg32(__float_as_uint(res), r_lo, r_hi);
    const float u = __uint_as_float(r_hi);
    if (lane == 0 && valid && live[v]) {
      const float x = res;
      gst<float>(a.h + ((int64_t)v * gridDim.y + blockIdx.y) * n_ff + r, x / (1.0f + expf(-x)) * u);
    }
  }
}

template <int T, int BPG>
__global__ __launch_bounds__(DEC_MV_NW * 64) void kd_gateup(const DecGateUpArgs a) { gateup_body<T, BPG, 1>(a); }
// two rows: two workgroups a CU (the grid's 384 workgroups of Qwen3-30B-A3B in one round)
template <int T, int BPG>
__global__ __launch_bounds__(DEC_MV_NW * 64) __attribute__((amdgpu_waves_per_eu(8))) void kd_gateup2(const DecGateUpArgs a) {
  gateup_body<T, BPG, 2>(a);
}

// ------------------------------------------------------------------ down + combine
// Eight wavefronts per workgroup, one output row each; row group s of a wavefront takes the
// row of chosen expert s (rounds of eight for more). Every workgroup quantizes the kept
// slots' h rows into LDS (Q8_K, :420-424). out = sum over the kept choices, in choice order,
// of w * y (non-fused multiply and add, ffns_fused :432-437); res_out = res_in + rscale * out.
// NV = 2: the slots of both rows of a two-row pass (slot v n_used + i: row v's choice i, h and
// chosen / weights as kd_gateup leaves them), each row's combine and residual add on its own.
template <int T, int NB, int NV = 1>
__global__ __launch_bounds__(512) void kd_down(const DecDownArgs a) {
  constexpr int NWD = 8, QB = DEC_DOWN_Q / 256, HB = QB / NWD;
  __shared__ __align__(16) uint32_t lq_[DEC_DOWN_Q / 4];
  __shared__ float ld_[QB];
  __shared__ __align__(16) int2 lbs_[QB * 8];
  __shared__ float ys[NWD][32];
  SPX_L uint32_t *lq = (SPX_L uint32_t *)lq_;
  SPX_L float *ld = (SPX_L float *)ld_;
  SPX_L int2 *lbs = (SPX_L int2 *)lbs_;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, slot = lane >> 3, l = lane & 7;
  const int dim = (int)a.w.rows, n_ff = (int)a.w.cols, nbh = n_ff >> 8, nu = a.n_used, ns = NV * nu;
  const int64_t r = (int64_t)blockIdx.x * NWD + wave;
  const int64_t rr = r < dim ? r : dim - 1;
  // h blocks of every slot (wave w: blocks w, w + 8, ...) and the chosen experts' rows are
  // requested before the kept count arrives (slots past it hold earlier, valid expert ids)
  const int nqa = ns * nbh;
  float4 hv[HB];
#pragma unroll
  for (int k = 0; k < HB; k++) {
    const int vb = wave + NWD * k;
    hv[k] = vb < nqa ? gld<float4>(a.h + (int64_t)(vb / nbh) * n_ff + (vb % nbh) * 256 + 4 * lane) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  auto expert_of = [&](int sv) SPX_AI {  // (clamped: a slot never written holds a zero)
    return min(max(gld<int>(a.chosen + sv), 0), a.w.n_expert - 1);
  };
  DRaw raw[NB];
  draw_row<T, NB>(raw, a.w.pl, (int64_t)expert_of(min(slot, ns - 1)) * dim + rr, nbh, l);
  int nk[NV];
#pragma unroll
  for (int v = 0; v < NV; v++) nk[v] = gld<int>(a.nkeep + v);
  // a slot sv = v nu + i is kept when i < nk[v]; rows past the kept slots are quantized too
  // only for NV = 1 (its kept slots are a prefix)
  auto kept = [&](int sv) SPX_AI { return NV == 1 ? sv < nk[0] : (sv % nu) < nk[min(sv / nu, NV - 1)]; };
  const int nqb = NV == 1 ? nk[0] * nbh : nqa, s0max = NV == 1 ? (nk[0] + 7) / 8 : (ns + 7) / 8;
#pragma unroll
  for (int k = 0; k < HB; k++) {
    const int vb = wave + NWD * k;
    if (vb < nqb && kept(vb / nbh)) {
      const float am = q8k_amax(hv[k]);
      q8k_block_store(hv[k], am, lq + vb * 64, ld + vb, (SPX_L int *)(lbs + vb * 8));
    }
  }
  __syncthreads();
  for (int round = 0; round < s0max; round++) {
    const int s = round * 8 + slot;
    if constexpr (NV == 1) {
      if (round > 0) draw_row<T, NB>(raw, a.w.pl, (int64_t)gld<int>(a.chosen + min(s, nk[0] - 1)) * dim + rr, nbh, l);
      const int sv = min(s, nk[0] - 1);
      const float y = dot_row<T, NB>(raw, nbh, l, lq + sv * nbh * 64, ld + sv * nbh, lbs + sv * nbh * 8);
      if (l == 0 && s < nk[0]) ys[wave][s] = y;
    } else {
      if (round > 0) draw_row<T, NB>(raw, a.w.pl, (int64_t)expert_of(min(s, ns - 1)) * dim + rr, nbh, l);
      const int sv = min(s, ns - 1);  // (a slot not kept reads an image nobody wrote; its y is dropped)
      const float y = dot_row<T, NB>(raw, nbh, l, lq + sv * nbh * 64, ld + sv * nbh, lbs + sv * nbh * 8);
      if (l == 0 && s < ns && kept(s)) ys[wave][s] = y;
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  if (lane == 0 && r < dim) {
#pragma unroll
    for (int v = 0; v < NV; v++) {
      float acc = 0.0f;
      for (int i = 0; i < nk[v]; i++) acc = acc + gld<float>(a.weights + v * nu + i) * ys[wave][v * nu + i];
      gst<float>(a.res_out + (int64_t)v * dim + r, gld<float>(a.res_in + (int64_t)v * dim + r) + a.rscale * acc);
    }
  }
}

// ================================================================== passes of 2..16 rows
// ------------------------------------------------------------------ norm of m rows
// One workgroup per row: residual row -> rmsnorm (the norm tails' fixed-order sum) -> fp32
// normalised row and / or its Q8_K, in global memory.
__global__ __launch_bounds__(256) void kd_norm(const DecNormArgs a) {
  constexpr int NW = 4, KB = DEC_MAXNB / NW;
  __shared__ float bsum_[DEC_MAXNB];
  const int b = blockIdx.x, nbq = a.dim >> 8;
  const DecIn in{(a.yd ? a.res_in : a.x) + (int64_t)b * a.dim, a.nw, a.eps, a.dim};
  InRow<KB> r;
  in_load<NW, KB>(in, r);
  if (a.yd) {  // the MoE combine of row b: kept choices in choice order, then the residual add
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nk = gld<int>(a.nkeep + b);
    const float *yr = a.yd + (int64_t)b * a.n_used * a.dim;
    float4 acc[KB];
#pragma unroll
    for (int k = 0; k < KB; k++) acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int i0 = 0; i0 < nk; i0 += 4) {  // four choices' loads in flight, then their sums in order
      float wv[4];
      float4 yv[4][KB];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int i = min(i0 + t, nk - 1);
        wv[t] = gld<float>(a.cw + b * 32 + i);
#pragma unroll
        for (int k = 0; k < KB; k++) {
          const int tb = wave + NW * k;
          yv[t][k] = tb < nbq ? gld<float4>(yr + (int64_t)i * a.dim + 4 * (tb * 64 + lane)) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int t = 0; t < 4; t++)
        if (i0 + t < nk)
#pragma unroll
          for (int k = 0; k < KB; k++) {
            acc[k].x = acc[k].x + wv[t] * yv[t][k].x; acc[k].y = acc[k].y + wv[t] * yv[t][k].y;
            acc[k].z = acc[k].z + wv[t] * yv[t][k].z; acc[k].w = acc[k].w + wv[t] * yv[t][k].w;
          }
    }
#pragma unroll
    for (int k = 0; k < KB; k++) {
      const int tb = wave + NW * k;
      if (tb < nbq) {
        float4 x = r.v[k];
        x.x = x.x + a.rscale * acc[k].x; x.y = x.y + a.rscale * acc[k].y; x.z = x.z + a.rscale * acc[k].z; x.w = x.w + a.rscale * acc[k].w;
        r.v[k] = x;
        gst<float4>(a.x_out + (int64_t)b * a.dim + 4 * (tb * 64 + lane), x);
      }
    }
  }
  float *xn = a.xn_out ? a.xn_out + (int64_t)b * a.dim : nullptr;
  if (a.q_out.q) {
    in_quant<NW, KB>(in, r, (SPX_G uint32_t *)(a.q_out.q + (int64_t)b * a.dim / 4), (SPX_G float *)(a.q_out.d + (int64_t)b * nbq),
                     (SPX_G int *)(a.q_out.bs + (int64_t)b * nbq * 8), (SPX_L float *)bsum_, xn);
  } else {  // fp32 only: quantize into a scratch image nobody reads
    __shared__ uint32_t sq[DEC_MAXNB * 64];
    __shared__ float sd[DEC_MAXNB];
    __shared__ int sb[DEC_MAXNB * 16];
    in_quant<NW, KB>(in, r, (SPX_L uint32_t *)sq, (SPX_L float *)sd, (SPX_L int *)sb, (SPX_L float *)bsum_, xn);
  }
}

// ------------------------------------------------------------------ multi-vector matvec
// DEC_MM_NW wavefronts per workgroup, R rows x G row groups per wavefront (rp_shape); the m
// vectors' Q8_K rows are staged in LDS. Blocks are taken in rounds: in round j group gi
// computes block gi + G * j for every vector into the chain buffer; then the group that owns
// vector v (v mod G) advances v's chain over the round's blocks in order. The chain per
// vector is the reference's, block by block (the same fp32 values as one vector alone).
__host__ __device__ inline size_t mm_lds_bytes(int m, int cols) { return mm_act_bytes(m, cols) + (size_t)DEC_MM_NW * 80 * m * 4; }

// Copies m permuted Q8_K vectors (global y, cols columns; vector v from y's vector vsrc[v],
// or v) into LDS (lq, ld, lbs), all threads; each thread's loads go out before its stores.
// vs4: 16-byte words a vector row of lq (0: cols / 16, rows back to back).
template <int NT, class VP = const int *>
__device__ __forceinline__ void stage_q8(const Q8KP &y, VP vsrc, int m, int cols, SPX_L uint32_t *lq, SPX_L float *ld, SPX_L int2 *lbs,
                                         int vs4 = 0) {
  const int nbq = cols >> 8, n16 = cols / 16, nb16 = nbq * 4, nq = m * n16, nb4 = m * nb16;
  const int tid = threadIdx.x;
  for (int i0 = tid; i0 < nq; i0 += 4 * NT) {  // loads of four rounds go out before their stores
    uint4 t[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int i = i0 + k * NT;
      if (i < nq) {
        const int v = i / n16, kk = i - v * n16, sv = vsrc ? vsrc[v] : v;
        t[k] = gld<uint4>(reinterpret_cast<const uint8_t *>(y.q) + (int64_t)sv * cols + 16 * kk);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int i = i0 + k * NT;
      if (i < nq) {
        const int v = i / n16;
        lst<uint4>((SPX_L uint4 *)lq + (vs4 ? v * vs4 + (i - v * n16) : i), t[k]);
      }
    }
  }
  for (int i0 = tid; i0 < nb4; i0 += 2 * NT) {
    uint4 t[2];
    float dv[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int i = i0 + k * NT;
      if (i < nb4) {
        const int v = i / nb16, kk = i - v * nb16, sv = vsrc ? vsrc[v] : v;
        t[k] = gld<uint4>(reinterpret_cast<const uint8_t *>(y.bs) + ((int64_t)sv * nbq * 8) * 8 + 16 * kk);
      }
      if (i < m * nbq) {
        const int v = i / nbq, kk = i - v * nbq, sv = vsrc ? vsrc[v] : v;
        dv[k] = gld<float>(y.d + (int64_t)sv * nbq + kk);
      }
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int i = i0 + k * NT;
      if (i < nb4) lst<uint4>((SPX_L uint4 *)lbs + i, t[k]);
      if (i < m * nbq) ld[i] = dv[k];
    }
  }
}

// Round j of a row's blocks for vectors 0..m-1: group gi's block (raw[j]) against every
// vector into cb [G][m][10].
template <int T, int BPG>
__device__ __forceinline__ void mm_round_dots(const DRaw (&raw)[BPG], int j, int nb, int G, int gi, int l, int m, int nbq,
                                              const SPX_L uint32_t *lq, const SPX_L float *ld, const SPX_L int2 *lbs, SPX_L float *cbr) {
  const int i = gi + G * j;
  if (i >= nb) return;
  KQDec<T> dec;
  dec.decode(draw_kq<T>(raw[j]), l);
#pragma unroll 2
  for (int v = 0; v < m; v++) {
    const int vb = v * nbq + i;
    const uint4 y0 = lld<uint4>(lq + vb * 64 + 8 * l), y1 = lld<uint4>(lq + vb * 64 + 8 * l + 4);
    int P, s;
    dec.dot(y0, y1, lld<int2>(lbs + vb * 8 + l), P, s);
    s = sum8(s);
    const float xd = ld[vb];
    SPX_L float *e = cbr + (gi * m + v) * 10;
    e[l] = (float)P;
    if (l == 0) { e[8] = dec.d * xd; e[9] = dec.corr_term(xd, s); }
  }
}

// The chain owner's update over round j (blocks G*j .. G*j+G-1 in order) for its vectors
// v = gi, gi + G, ... (slot q = v / G).
template <int QN>
__device__ __forceinline__ void mm_round_chain(int j, int nb, int G, int gi, int l, int m, const SPX_L float *cbr, float (&acc)[QN],
                                               float (&cr)[QN]) {
#pragma unroll
  for (int q = 0; q < QN; q++) {
    const int v = gi + G * q;
    if (v < m) {
      for (int k = 0; k < G && G * j + k < nb; k++) {
        const SPX_L float *e = cbr + (k * m + v) * 10;
        acc[q] = fmaf(e[8], e[l], acc[q]);
        cr[q] = cr[q] + e[9];
      }
    }
  }
}

template <int TT, int BPG, int QN>  // QN = MAX_M / G: vectors whose chains one row group owns
__global__ __launch_bounds__(DEC_MM_NW * 64) __attribute__((amdgpu_waves_per_eu(4))) void kd_mm(const DecMMArgs a) {
  constexpr int NW = DEC_MM_NW;
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ unsigned long long sbest[MAX_M];
  const int m = a.m, cols = a.cols, nbq = cols >> 8, nb = nbq;
  SPX_L uint32_t *lq = (SPX_L uint32_t *)smem;
  SPX_L float *ld = (SPX_L float *)(smem + (((size_t)m * cols + 15) & ~(size_t)15));
  SPX_L int2 *lbs = (SPX_L int2 *)(smem + (((size_t)m * cols + 15) & ~(size_t)15) + (((size_t)m * nbq * 4 + 15) & ~(size_t)15));
  SPX_L float *cbw = (SPX_L float *)(smem + mm_act_bytes(m, cols));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane >> 3, l = lane & 7;
  const int G = a.G, R = 8 / G, r = grp / G, gi = grp - r * G;
  SPX_L float *cbr = cbw + (size_t)(wave * R + r) * G * m * 10;
  const int t0 = a.tiles[0], t1 = a.nseg > 1 ? a.tiles[1] : 0, t2 = a.nseg > 2 ? a.tiles[2] : 0;
  const int total = t0 + t1 + t2;
  const Planes pl0 = a.w[0].pl, pl1 = a.w[1].pl, pl2 = a.w[2].pl;
  const int64_t rw0 = a.w[0].rows, rw1 = a.w[1].rows, rw2 = a.w[2].rows;
  const int dt0 = a.w[0].dtype, dt1 = a.w[1].dtype, dt2 = a.w[2].dtype;
  if (threadIdx.x < MAX_M) sbest[threadIdx.x] = 0;
  DRaw raw[BPG];
  int t = blockIdx.x, si = 0, dt = dt0;
  int64_t row = 0, rows = rw0;
  Planes pl = pl0;
#define SPX_MM_LOCATE()                                                                          \
  do {                                                                                           \
    si = __builtin_amdgcn_readfirstlane(t >= t0 ? (t >= t0 + t1 ? 2 : 1) : 0);                   \
    const int tt = t - (si > 0 ? t0 : 0) - (si > 1 ? t1 : 0);                                    \
    row = ((int64_t)tt * NW + wave) * R + r;                                                     \
    rows = si == 0 ? rw0 : si == 1 ? rw1 : rw2;                                                  \
    dt = si == 0 ? dt0 : si == 1 ? dt1 : dt2;                                                    \
    pl.p0 = si == 0 ? pl0.p0 : si == 1 ? pl1.p0 : pl2.p0;                                        \
    pl.p1 = si == 0 ? pl0.p1 : si == 1 ? pl1.p1 : pl2.p1;                                        \
    pl.p2 = si == 0 ? pl0.p2 : si == 1 ? pl1.p2 : pl2.p2;                                        \
    pl.p3 = si == 0 ? pl0.p3 : si == 1 ? pl1.p3 : pl2.p3;                                        \
    const int64_t grow = row < rows ? row : rows - 1;                                            \
    if (TT == T_Q4K || (TT == 0 && dt == T_Q4K)) rp_load<T_Q4K, BPG>(raw, pl, grow, nb, G, gi, l); \
    else rp_load<T_Q6K, BPG>(raw, pl, grow, nb, G, gi, l);                                       \
  } while (0)
  if (t < total) SPX_MM_LOCATE();
  stage_q8<DEC_MM_NW * 64>(a.y, (const int *)nullptr, m, cols, lq, ld, lbs);
  __syncthreads();
  for (; t < total;) {
    float acc[QN], cr[QN];
#pragma unroll
    for (int q = 0; q < QN; q++) { acc[q] = 0.0f; cr[q] = 0.0f; }
#pragma unroll
    for (int j = 0; j < BPG; j++) {
      if (TT == T_Q4K || (TT == 0 && dt == T_Q4K)) mm_round_dots<T_Q4K, BPG>(raw, j, nb, G, gi, l, m, nbq, lq, ld, lbs, cbr);
      else mm_round_dots<T_Q6K, BPG>(raw, j, nb, G, gi, l, m, nbq, lq, ld, lbs, cbr);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
      mm_round_chain<QN>(j, nb, G, gi, l, m, cbr, acc, cr);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
    }
    const int64_t row_c = row, rows_c = rows;
    float *const out = si == 0 ? a.out[0] : si == 1 ? a.out[1] : a.out[2];
    const int64_t ldo = si == 0 ? a.ld_out[0] : si == 1 ? a.ld_out[1] : a.ld_out[2];
    t += gridDim.x;
    if (t < total) SPX_MM_LOCATE();  // the next tile's weights go out before the results
#pragma unroll
    for (int q = 0; q < QN; q++) {
      const int v = gi + G * q;
      if (v < m) {
        const float res = hsum_rows8(acc[q]) - cr[q];
        if (l == 0 && row_c < rows_c) {
          if (out) gst<float>(out + (int64_t)v * ldo + row_c, res);
          if (a.res_out) {
            const int64_t o = (int64_t)v * rows_c + row_c;
            gst<float>(a.res_out + o, gld<float>(a.res_in + o) + a.rscale * res);
          }
          if (a.best) atomicMax(&sbest[v], pick_key(res, a.lscale, row_c));
        }
      }
    }
  }
#undef SPX_MM_LOCATE
  if (a.best) {
    __syncthreads();
    if ((int)threadIdx.x < m) gst<unsigned long long>(a.best + (int64_t)threadIdx.x * a.nbest + blockIdx.x, sbest[threadIdx.x]);
  }
}

// ------------------------------------------------------------------ router, m rows
// k_router's arithmetic for each row: wavefront w, lane j hold float4s w*64 + j + 256k of the
// router row; the lane's fma chain against the normalised row, the wave tree, the four
// wavefronts in order. Workgroup (e, g): router row e against rows 16g .. 16g + 15.
__global__ __launch_bounds__(256) void kd_router_m(const DecRouterMArgs a) {
  constexpr int NK = DEC_MAXNB / 4;
  __shared__ float part[4][MAX_M];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, row = blockIdx.x;
  const int dim = a.dim, n4 = dim >> 2, vb = blockIdx.y * MAX_M, mg = min(MAX_M, a.m - vb);
  const float *xg = a.x + (int64_t)vb * dim;
  float *lg = a.logits + (int64_t)vb * a.n_expert;
  float4 wv[NK];
#pragma unroll
  for (int k = 0; k < NK; k++) {
    const int f = wave * 64 + lane + 256 * k;
    wv[k] = f < n4 ? gld<float4>(a.w.pl.p0 + ((int64_t)row * dim + 4 * f) * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int v0 = 0; v0 < MAX_M; v0 += 4) {
    if (v0 < mg) {
      float4 x[4][NK];
#pragma unroll
      for (int vv = 0; vv < 4; vv++)
#pragma unroll
        for (int k = 0; k < NK; k++) {
          const int f = wave * 64 + lane + 256 * k, v = min(v0 + vv, mg - 1);
          x[vv][k] = f < n4 ? gld<float4>(xg + (int64_t)v * dim + 4 * f) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
      for (int vv = 0; vv < 4; vv++) {
        float pv = 0.0f;
#pragma unroll
        for (int k = 0; k < NK; k++) {
          const int f = wave * 64 + lane + 256 * k;
          if (f < n4) {
            pv = fmaf(wv[k].x, x[vv][k].x, pv);
            pv = fmaf(wv[k].y, x[vv][k].y, pv);
            pv = fmaf(wv[k].z, x[vv][k].z, pv);
            pv = fmaf(wv[k].w, x[vv][k].w, pv);
          }
        }
        const float tsum = wave_sum(pv);
        if (lane == 0 && v0 + vv < mg) part[wave][v0 + vv] = tsum;
      }
    }
  }
  __syncthreads();
  if ((int)threadIdx.x < mg) {
    const int v = threadIdx.x;
    gst<float>(lg + (int64_t)v * a.n_expert + row, ((part[0][v] + part[1][v]) + part[2][v]) + part[3][v]);
  }
}

// ------------------------------------------------------------------ routing + jobs, m rows
// Every workgroup of kd_gateup_m (NW wavefronts, NW * 64 >= n_expert threads): wavefront w
// routes rows w and w + NW (route_row; route_load brings their logits), then thread e builds
// expert e's job if it has users:
// jobs in expert order, users in row order (a row chooses an expert at most once), into the
// LDS table sj (JR ints a job: expert, nvec, vec[MAX_M], out[MAX_M]), the job list of
// k_router's tail. publish: the routing results, the job list and the selection counts also go
// to global memory. Returns the job count.
template <int NW>
__device__ __forceinline__ void route_load(const DecRouteArgs &a, float (&lv)[2][4]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const int b = wave + NW * r;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int e = lane + 64 * k;
      lv[r][k] = b < a.m && e < a.n_expert ? gld<float>(a.logits + (int64_t)b * a.n_expert + e) : -INFINITY;
    }
  }
}

template <int NW>
__device__ int route_jobs(const DecRouteArgs &a, const float (&lv)[2][4], SPX_L int *sj, SPX_L signed char *slot_of, SPX_L int *wcount,
                          bool publish) {
  constexpr int JR = 2 + 2 * MAX_M;
  static_assert(2 * NW >= MAX_M, "two rows a wavefront");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ne = a.n_expert, nu = a.n_used, m = a.m;
  for (int i = threadIdx.x; i < MAX_M * 256; i += NW * 64) slot_of[i] = -1;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const int b = wave + NW * r;
    if (b < m) {
      int my_e, keep;
      float my_p, wsum;
      route_row(lv[r], ne, nu, a.moe_prune, my_e, my_p, keep, wsum);
      if (lane < keep) {
        slot_of[b * 256 + my_e] = (signed char)lane;
        if (publish) {
          gst<int>(a.chosen + b * 32 + lane, my_e);
          gst<float>(a.weights + b * 32 + lane, a.norm ? my_p / wsum : my_p);
        }
      }
      if (publish && lane == 0) gst<int>(a.nkeep + b, keep);
    }
  }
  __syncthreads();
  const int e = threadIdx.x;
  int cnt = 0;
  if (e < ne)
    for (int b = 0; b < m; b++) cnt += slot_of[b * 256 + e] >= 0;
  const unsigned long long bal = __ballot(cnt > 0);
  if (lane == 0) wcount[wave] = __popcll(bal);
  __syncthreads();
  int nj = 0, base = 0;
  for (int w = 0; w < NW; w++) {
    base += w < wave ? wcount[w] : 0;
    nj += wcount[w];
  }
  if (cnt > 0) {
    const int j = base + __popcll(bal & ((1ull << lane) - 1ull));
    SPX_L int *J = sj + j * JR;
    int k = 0;
    for (int b = 0; b < m; b++) {
      const int sl = slot_of[b * 256 + e];
      if (sl >= 0) { J[2 + k] = b; J[2 + MAX_M + k] = b * nu + sl; k++; }
    }
    for (int q = k; q < MAX_M; q++) { J[2 + q] = 0; J[2 + MAX_M + q] = 0; }
    J[0] = e;
    J[1] = k;
    if (publish) {
      int *G = reinterpret_cast<int *>(a.jobs + j);
      for (int f = 0; f < JR; f++) gst<int>(G + f, J[f]);
      if (a.expert_count) atomicAdd(a.expert_count + e, 1);
    }
  }
  if (publish && threadIdx.x == 0) gst<int>(a.njobs, nj);
  __syncthreads();
  return nj;
}

// ------------------------------------------------------------------ gate / up, m rows
// Items (job j, tile x) with TX = ceil(n_ff / DEC_MM_NW) tiles per job; workgroup b of the
// grid (at most two per CU) takes items [b n / G, (b + 1) n / G), consecutive tiles of one or
// two jobs, so a job's users are staged once and no workgroup is launched past the job count.
// Tile x: rows DEC_MM_NW * x .. of h, one row per wavefront: lanes 0-31 the gate row, 32-63 the
// up row, four groups each; rounds of four blocks as kd_mm. h[out][r] = silu(g) * u. The m
// rows' Q8_K image is staged once (its loads overlap the routing); the next item's weights are
// requested before the current item's dots.
template <int T, int BPG>
__device__ __forceinline__ void gum_load(DRaw (&raw)[BPG], const DecGateUpMArgs &a, const SPX_L int *sj, int j, int x, int half, int gi,
                                         int l, int nb) {
  constexpr int JR = 2 + 2 * MAX_M;
  const int r = x * DEC_MM_NW + (int)(threadIdx.x >> 6);
  const int e = min(max(sj[j * JR], 0), a.gate.n_expert - 1);
  const int64_t grow = (int64_t)e * a.gate.rows + (r < a.n_ff ? r : a.n_ff - 1);
  rp_load<T, BPG>(raw, half ? a.up.pl : a.gate.pl, grow, nb, 4, gi, l);
}

// The m rows' Q8_K image (global y -> LDS, row b at slot b) in two steps: the loads go out
// (get), other work runs, then the LDS stores (put). NT threads; at most MAX_M rows of
// DEC_MAXNB blocks.
template <int NT>
struct StageQ8 {
  static constexpr int NQ = (MAX_M * DEC_MAXNB * 16 + NT - 1) / NT, NS = (MAX_M * DEC_MAXNB * 4 + NT - 1) / NT,
                       ND = (MAX_M * DEC_MAXNB + NT - 1) / NT;
  uint4 q[NQ], bs[NS];
  float d[ND];
  __device__ __forceinline__ void get(const Q8KP &y, int m, int cols) {
    const int nbq = cols >> 8, nq = m * (cols / 16), nb4 = m * nbq * 4, nd = m * nbq, t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < NQ; k++)
      if (t + k * NT < nq) q[k] = gld<uint4>(reinterpret_cast<const uint8_t *>(y.q) + 16 * (int64_t)(t + k * NT));
#pragma unroll
    for (int k = 0; k < NS; k++)
      if (t + k * NT < nb4) bs[k] = gld<uint4>(reinterpret_cast<const uint8_t *>(y.bs) + 16 * (int64_t)(t + k * NT));
#pragma unroll
    for (int k = 0; k < ND; k++)
      if (t + k * NT < nd) d[k] = gld<float>(y.d + t + k * NT);
  }
  // vs4: 16-byte words a vector row of lq (0: cols / 16, rows back to back)
  __device__ __forceinline__ void put(int m, int cols, SPX_L uint32_t *lq, SPX_L float *ld, SPX_L int2 *lbs, int vs4 = 0) const {
    const int nbq = cols >> 8, n16 = cols / 16, nq = m * n16, nb4 = m * nbq * 4, nd = m * nbq, t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < NQ; k++) {
      const int i = t + k * NT, v = i / n16;
      if (i < nq) lst<uint4>((SPX_L uint4 *)lq + (vs4 ? v * vs4 + (i - v * n16) : i), q[k]);
    }
#pragma unroll
    for (int k = 0; k < NS; k++)
      if (t + k * NT < nb4) lst<uint4>((SPX_L uint4 *)lbs + t + k * NT, bs[k]);
#pragma unroll
    for (int k = 0; k < ND; k++)
      if (t + k * NT < nd) ld[t + k * NT] = d[k];
  }
};

// Round k of a row's blocks for the users of a job (user v = row rows[v] of the image): group
// gi's block against every user into cb [G][nv][10], as mm_round_dots.
template <int T, int BPG>
__device__ __forceinline__ void gum_round_dots(const DRaw (&raw)[BPG], int k, int nb, int gi, int l, int nv, int nbq,
                                               const SPX_L int *rows, const SPX_L uint32_t *lq, const SPX_L float *ld, const SPX_L int2 *lbs,
                                               SPX_L float *cbr) {
  const int i = gi + 4 * k;
  if (i >= nb) return;
  KQDec<T> dec;
  dec.decode(draw_kq<T>(raw[k]), l);
#pragma unroll 2
  for (int v = 0; v < nv; v++) {
    const int vb = rows[v] * nbq + i;
    const uint4 y0 = lld<uint4>(lq + vb * 64 + 8 * l), y1 = lld<uint4>(lq + vb * 64 + 8 * l + 4);
    int P, s;
    dec.dot(y0, y1, lld<int2>(lbs + vb * 8 + l), P, s);
    s = sum8(s);
    const float xd = ld[vb];
    SPX_L float *e = cbr + (gi * nv + v) * 10;  // the layout mm_round_chain reads (m = nv)
    e[l] = (float)P;
    if (l == 0) { e[8] = dec.d * xd; e[9] = dec.corr_term(xd, s); }
  }
}

template <int T, int BPG>
__global__ __launch_bounds__(DEC_MM_NW * 64) __attribute__((amdgpu_waves_per_eu(BPG > 2 ? 2 : 4))) void kd_gateup_m(const DecGateUpMArgs a) {
  constexpr int NW = DEC_MM_NW, JR = 2 + 2 * MAX_M;  // a Job record in ints: expert, nvec, vec[], out[]
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ signed char slot_of[MAX_M * 256];
  __shared__ int wcount[NW];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane >> 3, l = lane & 7;
  const int half = grp >> 2, gi = grp & 3;
  const int n_ff = a.n_ff, cols = (int)a.gate.cols, nbq = cols >> 8, nb = nbq, m = a.m;
  const int TX = (n_ff + NW - 1) / NW;
  const size_t act = mm_act_bytes(m, cols);
  SPX_L uint32_t *lq = (SPX_L uint32_t *)smem;
  SPX_L float *ld = (SPX_L float *)(smem + (((size_t)m * cols + 15) & ~(size_t)15));
  SPX_L int2 *lbs = (SPX_L int2 *)(smem + (((size_t)m * cols + 15) & ~(size_t)15) + (((size_t)m * nbq * 4 + 15) & ~(size_t)15));
  SPX_L float *cbr = (SPX_L float *)(smem + act) + (size_t)(wave * 2 + half) * 4 * m * 10;
  SPX_L int *sj = (SPX_L int *)(smem + act + (size_t)NW * 2 * 4 * m * 10 * 4);  // [max jobs][JR]
  int nj = 1;
  {
    StageQ8<NW * 64> st;
    if (a.rt.logits) {
      float lv[2][4];
      route_load<NW>(a.rt, lv);
      st.get(a.y, m, cols);  // the image's loads overlap the routing
      nj = route_jobs<NW>(a.rt, lv, sj, (SPX_L signed char *)slot_of, (SPX_L int *)wcount, blockIdx.x == 0);
    } else {  // dense: one job, expert 0, users = rows 0..m-1
      st.get(a.y, m, cols);
      for (int i = threadIdx.x; i < JR; i += blockDim.x) sj[i] = i == 0 ? 0 : i == 1 ? m : i < 2 + MAX_M ? i - 2 : i - 2 - MAX_M;
      __syncthreads();  // the job record (gum_load reads it)
    }
    st.put(m, cols, lq, ld, lbs);
  }
  const int n = TX * nj, G = gridDim.x;
  const int i0 = (int)((int64_t)blockIdx.x * n / G), i1 = (int)((int64_t)(blockIdx.x + 1) * n / G);
  if (i0 >= i1) return;  // the whole workgroup
  int i = i0, j = i0 / TX, x = i0 - (i0 / TX) * TX;
  DRaw raw[BPG];
  gum_load<T, BPG>(raw, a, sj, j, x, half, gi, l, nb);
  __syncthreads();  // the image and the job table
  for (;;) {
    const int nv = sj[j * JR + 1];
    int jn = j, xn = x + 1;
    if (xn == TX) { jn++; xn = 0; }
    DRaw nraw[BPG];
    if (i + 1 < i1) gum_load<T, BPG>(nraw, a, sj, jn, xn, half, gi, l, nb);
    float acc[MAX_M / 4], cr[MAX_M / 4];
#pragma unroll
    for (int q = 0; q < MAX_M / 4; q++) { acc[q] = 0.0f; cr[q] = 0.0f; }
#pragma unroll
    for (int k = 0; k < BPG; k++) {
      gum_round_dots<T, BPG>(raw, k, nb, gi, l, nv, nbq, sj + j * JR + 2, lq, ld, lbs, cbr);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
      mm_round_chain<MAX_M / 4>(k, nb, 4, gi, l, nv, cbr, acc, cr);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
    }
    const int r = x * NW + wave;
#pragma unroll
    for (int q = 0; q < MAX_M / 4; q++) {
      const int v = gi + 4 * q;
      if (v < nv) {  // wave-uniform per group pair: gate lanes and up lanes own the same v
        const float res = hsum_rows8(acc[q]) - cr[q];
        uint32_t r_lo, r_hi;
        xchg32(__float_as_uint(res), r_lo, r_hi);
        const float u = __uint_as_float(r_hi);
        if (half == 0 && l == 0 && r < n_ff) {
          const float xg = res;
          gst<float>(a.h + (int64_t)sj[j * JR + 2 + MAX_M + v] * n_ff + r, xg / (1.0f + expf(-xg)) * u);
        }
      }
    }
    if (++i >= i1) break;
#pragma unroll
    for (int k = 0; k < BPG; k++) raw[k] = nraw[k];
    j = jn;
    x = xn;
  }
}

// ------------------------------------------------------------------ down, m rows
// Items (job j, tile x of 64 rows of the expert's down matrix): a workgroup of eight
// wavefronts; row group g of wavefront w takes row 64x + 8w + g, all its blocks in order (the
// reference's chain in registers, as kq_walk_tile), against each of the job's users' h, which
// the workgroup quantizes into LDS from the fp32 h rows (quantize_avx2 per 256 block).
// y[out][r] for every (user, row); the weighted combine and the residual add are kd_norm's.
template <int T, int NB>
__global__ __launch_bounds__(DEC_MM_NW * 64) __attribute__((amdgpu_waves_per_eu(4))) void kd_down_m(const DecDownMArgs a) {
  constexpr int NW = DEC_MM_NW, RW = NW * 8, JF = 2 + MAX_M;  // rows per item; job fields: expert, nvec, out[]
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int s_job[JF];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 3, l = lane & 7;
  const int dim = (int)a.w.rows, n_ff = (int)a.w.cols, nbh = n_ff >> 8, TX = (dim + RW - 1) / RW;
  SPX_L uint32_t *lq = (SPX_L uint32_t *)smem;
  SPX_L float *ld = (SPX_L float *)(smem + (((size_t)MAX_M * n_ff + 15) & ~(size_t)15));
  SPX_L int *lbs = (SPX_L int *)(smem + (((size_t)MAX_M * n_ff + 15) & ~(size_t)15) + (((size_t)MAX_M * nbh * 4 + 15) & ~(size_t)15));
  const int n = TX * gld<int>(a.njobs);
  for (int it = blockIdx.x; it < n; it += gridDim.x) {
    const int j = it / TX, x = it - j * TX;
    if ((int)threadIdx.x < JF) {
      const int f = threadIdx.x;
      s_job[f] = gld<int>(reinterpret_cast<const int *>(a.jobs + j) + (f < 2 ? f : 2 + MAX_M + (f - 2)));
    }
    __syncthreads();
    const int e = min(max(s_job[0], 0), a.w.n_expert - 1), nv = min(max(s_job[1], 0), MAX_M);
    const int64_t r = (int64_t)x * RW + wave * 8 + g;
    const int64_t rr = r < dim ? r : dim - 1;
    DRaw raw[NB];
    draw_row<T, NB>(raw, a.w.pl, (int64_t)e * dim + rr, nbh, l);
    // users' h blocks q = k * nbh + i (user k, block i); wavefront w takes q = w, w + NW, ...
    const int nq = nv * nbh;
    for (int q0 = wave; q0 < nq; q0 += 4 * NW) {
      float4 hv[4];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int q = q0 + NW * t;
        if (q < nq) {
          const int k = q / nbh, i = q - k * nbh;
          hv[t] = gld<float4>(a.h + (int64_t)s_job[2 + k] * n_ff + i * 256 + 4 * lane);
        }
      }
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int q = q0 + NW * t;
        if (q < nq) {
          const float am = q8k_amax(hv[t]);
          q8k_block_store(hv[t], am, lq + q * 64, ld + q, lbs + q * 16);
        }
      }
    }
    __syncthreads();
    // blocks in order, each decoded once; every user's chain advances block by block
    float acc[MAX_M], corr[MAX_M];
#pragma unroll
    for (int k = 0; k < MAX_M; k++) { acc[k] = 0.0f; corr[k] = 0.0f; }
#pragma unroll
    for (int i = 0; i < NB; i++) {
      if (i < nbh) {
        KQDec<T> dec;
        dec.decode(draw_kq<T>(raw[i]), l);
#pragma unroll
        for (int k = 0; k < MAX_M; k++) {
          if (k < nv) {
            const int vb = k * nbh + i;
            const uint4 y0 = lld<uint4>(lq + vb * 64 + 8 * l), y1 = lld<uint4>(lq + vb * 64 + 8 * l + 4);
            int P, sm;
            dec.dot(y0, y1, lld<int2>(lbs + vb * 16 + 2 * l), P, sm);
            sm = sum8(sm);
            const float xd = ld[vb];
            corr[k] = corr[k] + dec.corr_term(xd, sm);
            acc[k] = fmaf(dec.d * xd, (float)P, acc[k]);
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < MAX_M; k++) {
      if (k < nv) {
        const float y = hsum_rows8(acc[k]) - corr[k];
        if (l == 0 && r < dim) gst<float>(a.yd + (int64_t)s_job[2 + k] * dim + r, y);
      }
    }
    __syncthreads();  // s_job and the LDS image are refilled by the next item
  }
}

// ================================================================== int8 MFMA, 2..16 rows
// The multi-row kernels on the int8 matrix cores (v_mfma_i32_16x16x32_i8; the verify pass of the
// speculative loop, prefill passes), bit for bit the per-lane dot chains. Operand layouts of
// 16x16x32 i8: A[i][k] in lane i + 16 (k / 8), byte k % 8; B[k][j] in lane j + 16 (k / 8); D[i][j]
// in lane j + 16 (i / 4), element i % 4. A holds the activations (i = vector), B the weights
// (j = matrix row), so lane c16 + 16 k4 owns matrix row c16 for vectors 4 k4 + t.
typedef int mq_v4i __attribute__((ext_vector_type(4)));
__device__ __forceinline__ mq_v4i mq_mfma(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1) {
  const long a = (long)(((unsigned long long)a1 << 32) | a0), b = (long)(((unsigned long long)b1 << 32) | b0);
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, mq_v4i{0, 0, 0, 0}, 0, 0, 0);
}
__device__ __forceinline__ mq_v4i mq_mfma_c(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, mq_v4i c) {
  const long a = (long)(((unsigned long long)a1 << 32) | a0), b = (long)(((unsigned long long)b1 << 32) | b0);
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ int mq_byte(uint4 v, int i) {  // byte i (0..15, constant after unrolling)
  const uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
  return (int)((w >> (8 * (i & 3))) & 0xffu);
}
__device__ __forceinline__ int mq_sbyte(uint4 v, int i) { return (int)(int8_t)mq_byte(v, i); }

struct MqIdentity {
  __device__ __forceinline__ int operator()(int v) const { return v; }
};
struct MqRows {
  const SPX_L int *r;
  __device__ __forceinline__ int operator()(int v) const { return r[v]; }
};

// The correction operands of the MFMA path, per (vector, 256-block) 12 words next to the Q8_K
// image: the sixteen 16-element bsums split as bs = 64 hi + lo (lo = bs & 63, hi = bs >> 6:
// |bs| <= 2032 keeps hi in int8), lo[16] then hi[16] (words 0-7, Q6_K groups), then the eight
// 32-element sums (|.| <= 4064) split the same way, lo[8] then hi[8] (words 8-11, Q4_K
// sub-blocks). The correction C = sum sc bs is then two MFMAs: D1 over lo and hi, D2 over hi
// alone, C = D1 + 63 D2 (exact).
constexpr int MQ_CW = 12;  // words a (vector, block)
__device__ __forceinline__ uint32_t mq_pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 255) | ((uint32_t)(b & 255) << 8) | ((uint32_t)(c & 255) << 16) | ((uint32_t)(d & 255) << 24);
}
// The tile's vectors: the A operand's vector (lane & 15) and the D elements' vectors
// 4 (lane >> 4) + t, as rows of the LDS Q8_K image (row 0 stands in past the last vector).
struct MqVec {
  bool ain;
  int a, d[4];
};
template <class VR>
__device__ __forceinline__ MqVec mq_vecs(int nv, VR vrow) {
  const int lane = threadIdx.x & 63, c16 = lane & 15, k4 = lane >> 4;
  MqVec v;
  v.ain = c16 < nv;
  v.a = v.ain ? vrow(c16) : 0;
#pragma unroll
  for (int t = 0; t < 4; t++) v.d[t] = 4 * k4 + t < nv ? vrow(4 * k4 + t) : 0;
  return v;
}
// ---- the reference's lane classes on the matrix cores
// The reference's result bits are fixed by eight int32 partials per (row, vector, block),
// P_l = sum_s sc_s sum_{j<4} q[32s + 4l + j] y[32s + 4l + j] (rows<B,T>, quant_q8k.rs:229-243:
// maddubs pairs, madd with the sub-block scale), each converted to fp32 and chained per lane
// class l over the blocks in order (acc_l = fma(d xd, float(P_l), acc_l)) before the 8 -> 1 hsum.
// Here one wavefront owns a tile of 16 matrix rows x 16 vectors and all eight classes: per block
// and class one contraction over the class's 32 codes, K = 4 s + j (lane c16 + 16 k4 holds
// K = 8 k4 .. 8 k4 + 7: sub-blocks 2 k4 and 2 k4 + 1), with the sub-block scales folded into
// the weight operand so that D is P_l itself, exactly:
//   Q4_K: sc (0..63) = 8 sh + sl (3 bits each); operands q sl and q sh (<= 105);
//         P_l = D(q sl) + 8 D(q sh)
//   Q6_K: q (0..63) = 8 qh + ql, sc (int8) = 16 sh + sl (sl = sc & 15, sh = sc >> 4 in -8..7);
//         operands ql sl, qh sl (<= 105) and ql sh, qh sh (-56..49);
//         P_l = D(ql sl) + 8 D(qh sl) + 16 D(ql sh) + 128 D(qh sh)
// (|P_l| < 2^25: exact in int32). A 64-code contraction (the x64 MFMA) would add two classes' or
// two scale digits' sums that the reference keeps apart, so each class takes x32 contractions.
// The eight chains stay in the lane's registers (acc[l][t]: matrix row lane & 15, vector
// 4 (lane >> 4) + t), the block's correction integer C (mins / -32 term, the reference's per
// block) is chained beside them, and out = ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)) - corr
// needs no other wavefront.
typedef unsigned short mx_u16x2 __attribute__((ext_vector_type(2)));
// Per byte of v (each <= 15) times s (<= 15) with both products of a 16-bit half <= 105: no
// carry leaves a byte (v_pk_mul_lo_u16).
__device__ __forceinline__ uint32_t mx_pmul(uint32_t v, uint32_t s) {
  const mx_u16x2 a = __builtin_bit_cast(mx_u16x2, v), b = {(unsigned short)s, (unsigned short)s};
  return __builtin_bit_cast(uint32_t, a * b);
}
typedef short mx_i16x2 __attribute__((ext_vector_type(2)));
// Per byte c (0..63) of q times the int8 scale s16 (sign-extended to a 16-bit lane): W = c s =
// 128 hi + lo with lo = W & 127 (0..127) and hi = W >> 7 (-63..62), each packed back into the
// byte's place (bytes 0, 2 and 1, 3 multiplied as 16-bit lanes, exact modulo 2^16).
__device__ __forceinline__ void q6_wsplit(uint32_t q, uint32_t s16, uint32_t &hi, uint32_t &lo) {
  const mx_u16x2 sv = {(unsigned short)s16, (unsigned short)s16};
  const mx_u16x2 we = __builtin_bit_cast(mx_u16x2, __builtin_amdgcn_perm(0u, q, 0x0C020C00u)) * sv;
  const mx_u16x2 wo = __builtin_bit_cast(mx_u16x2, __builtin_amdgcn_perm(0u, q, 0x0C030C01u)) * sv;
  lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, wo), __builtin_bit_cast(uint32_t, we), 0x06020400u) & 0x7F7F7F7Fu;
  const mx_i16x2 he = __builtin_bit_cast(mx_i16x2, we) >> (short)7, ho = __builtin_bit_cast(mx_i16x2, wo) >> (short)7;
  hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, ho), __builtin_bit_cast(uint32_t, he), 0x06020400u);
}

// 4 x 4 transpose over the wavefront's four 16-lane rows: row g of r[c] holds M[g][c] on entry
// and M[c][g] on return (v_permlane32_swap: rows 2, 3 of the first operand <-> rows 0, 1 of the
// second; v_permlane16_swap: rows 1, 3 of the first <-> rows 0, 2 of the second).
__device__ __forceinline__ void mw_t4(uint32_t (&r)[4]) {
  const auto p = __builtin_amdgcn_permlane32_swap(r[0], r[2], false, false);
  const auto q = __builtin_amdgcn_permlane32_swap(r[1], r[3], false, false);
  const auto u = __builtin_amdgcn_permlane16_swap(p[0], q[0], false, false);
  const auto v = __builtin_amdgcn_permlane16_swap(p[1], q[1], false, false);
  r[0] = u[0];
  r[1] = u[1];
  r[2] = v[0];
  r[3] = v[1];
}
// The same for rows (a, a, b, b): three swaps.
__device__ __forceinline__ void mw_t4d(uint32_t a, uint32_t b, uint32_t (&r)[4]) {
  const auto p = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  const auto u = __builtin_amdgcn_permlane16_swap(p[0], p[0], false, false);
  const auto v = __builtin_amdgcn_permlane16_swap(p[1], p[1], false, false);
  r[0] = u[0];
  r[1] = u[1];
  r[2] = v[0];
  r[3] = v[1];
}

// The LDS image of a tile's vectors (at most 16): codes lq (vector v's block b at dword
// v mw_vs + 64 b; eight pad dwords a vector put the sixteen vectors' reads of one class word in
// different banks), block scales ld [v nb + b], the correction words lc (vector v's block b at
// v mw_cs + MQ_CW b, padded likewise), and last the bsum pairs lbs [v nb + b][8], needed only to
// build lc (mw_tail_off: where lbs starts; a kernel may reuse the space from there on).
__host__ __device__ inline int mw_vs(int nb) { return nb * 64 + 8; }
__host__ __device__ inline int mw_cs(int nb) { return nb * MQ_CW + ((8 - nb * MQ_CW) % 64 + 64) % 64; }
__host__ __device__ inline size_t mw_tail_off(int m, int nb) {
  return (size_t)m * mw_vs(nb) * 4 + (((size_t)m * nb * 4 + 15) & ~(size_t)15) + (size_t)m * mw_cs(nb) * 4;
}
__host__ __device__ inline size_t mw_act_bytes(int m, int nb) { return mw_tail_off(m, nb) + (size_t)m * nb * 64; }
struct MwLds {
  SPX_L uint32_t *lq;
  SPX_L float *ld;
  SPX_L int2 *lbs;
  SPX_L uint32_t *lc;
};
__device__ __forceinline__ MwLds mw_lds(uint8_t *base, int m, int nb) {
  MwLds L;
  size_t o = (size_t)m * mw_vs(nb) * 4;
  L.lq = (SPX_L uint32_t *)base;
  L.ld = (SPX_L float *)(base + o);
  o += ((size_t)m * nb * 4 + 15) & ~(size_t)15;
  L.lc = (SPX_L uint32_t *)(base + o);
  L.lbs = (SPX_L int2 *)(base + mw_tail_off(m, nb));
  return L;
}
// The correction words of the image's m vectors (from the staged bsum pairs).
__device__ __forceinline__ void mq_corr_stage(int m, int nb, const SPX_L int2 *lbs, SPX_L uint32_t *lc) {
  const int cs = mw_cs(nb);
  for (int q = threadIdx.x; q < m * nb; q += blockDim.x) {
    int bs[16];
#pragma unroll
    for (int i = 0; i < 8; i++) { const int2 v = lld<int2>(lbs + q * 8 + i); bs[2 * i] = v.x; bs[2 * i + 1] = v.y; }
    uint32_t w[MQ_CW];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      w[i] = mq_pack4(bs[4 * i] & 63, bs[4 * i + 1] & 63, bs[4 * i + 2] & 63, bs[4 * i + 3] & 63);
      w[4 + i] = mq_pack4(bs[4 * i] >> 6, bs[4 * i + 1] >> 6, bs[4 * i + 2] >> 6, bs[4 * i + 3] >> 6);
    }
    int s32[8];
#pragma unroll
    for (int i = 0; i < 8; i++) s32[i] = bs[2 * i] + bs[2 * i + 1];
#pragma unroll
    for (int i = 0; i < 2; i++) {
      w[8 + i] = mq_pack4(s32[4 * i] & 63, s32[4 * i + 1] & 63, s32[4 * i + 2] & 63, s32[4 * i + 3] & 63);
      w[10 + i] = mq_pack4(s32[4 * i] >> 6, s32[4 * i + 1] >> 6, s32[4 * i + 2] >> 6, s32[4 * i + 3] >> 6);
    }
    const int v = q / nb, b = q - v * nb;
    SPX_L uint32_t *o = lc + v * cs + b * MQ_CW;
#pragma unroll
    for (int i = 0; i < MQ_CW; i += 4) lst<uint4>((SPX_L uint4 *)(o + i), make_uint4(w[i], w[i + 1], w[i + 2], w[i + 3]));
  }
}

// One block of a tile as lane c16 + 16 k4 loads it, from matrix row c16's bytes in 16-byte
// pieces (the row's four lanes read its 128 code bytes as two 64-byte halves): Q4_K c[e] = code
// dwords 16 e + 4 k4 .. + 3; Q6_K c[e] = ql dwords 16 e + 4 k4 .. + 3 and h[e] = qh dwords
// 8 e + 2 k4, + 1; s = the row's scale line (Q4_K: 8 scales, 8 mins; Q6_K: 16 int8 scales);
// d = Q4_K d | dmin << 16, Q6_K d.
struct MwRaw {
  uint4 c[2], s;
  uint2 h[2];
  uint32_t d;
};
// A tile's planes at its first row (wave-uniform: scalar registers) and this lane's row as a
// block offset from there, so the loads take a scalar base and a 32-bit lane offset.
struct MwSrc {
  const uint8_t *p0, *p1, *p2, *p3;
  int rb;  // (row c16, clamped to the tile) x nb
  int dt;
};
__device__ __forceinline__ int64_t mw_uni64(int64_t v) {
  const uint64_t u = (uint64_t)v;
  return (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(u >> 32)) << 32) | (uint32_t)__builtin_amdgcn_readfirstlane((int)u));
}
__device__ __forceinline__ MwSrc mw_src(const Planes &pl, int dt, int64_t row0, int nrows, int nb) {
  const int64_t r0 = mw_uni64(row0) * nb;
  MwSrc s;
  s.dt = __builtin_amdgcn_readfirstlane(dt);
  s.p0 = pl.p0 + r0 * 128;
  s.p2 = pl.p2 + r0 * 16;
  if (s.dt == T_Q4K) {
    s.p1 = pl.p1 + r0 * 16;
    s.p3 = s.p1;
  } else {
    s.p1 = pl.p1 + r0 * 64;
    s.p3 = pl.p3 + r0 * 2;
  }
  s.rb = min((int)(threadIdx.x & 15), __builtin_amdgcn_readfirstlane(nrows) - 1) * nb;
  return s;
}
template <int TT>  // TT: the tile's format when fixed for the launch, 0: s.dt at run time
__device__ __forceinline__ void mw_fetch(MwRaw &r, const MwSrc &s, int b) {
  const uint32_t k4 = (threadIdx.x & 63) >> 4, ob = (uint32_t)(s.rb + b);
  r.c[0] = gld<uint4>(s.p0 + (ob * 128u + 16u * k4));
  r.c[1] = gld<uint4>(s.p0 + (ob * 128u + 16u * k4 + 64u));
  r.s = gld<uint4>(s.p2 + ob * 16u);
  if (TT == T_Q4K || (TT == 0 && s.dt == T_Q4K)) {
    r.d = gld<uint32_t>(s.p1 + ob * 16u);
  } else {
    r.h[0] = gld<uint2>(s.p1 + (ob * 64u + 8u * k4));
    r.h[1] = gld<uint2>(s.p1 + (ob * 64u + 8u * k4 + 32u));
    r.d = gld<uint16_t>(s.p3 + ob * 2u);
  }
}
// The tile's LDS operands for this lane: A (vector lane & 15's class words, dword 2 k4 of each),
// its correction words, the block scales of vectors 4 (lane >> 4) + t. Rows of A past the
// vectors read vector 0's: a row of A reaches only the same row of D, never stored.
struct MwDst {
  const SPX_L uint32_t *py, *pw;
  const SPX_L float *px[4];
  int dt;
};
__device__ __forceinline__ MwDst mw_dst(const MwLds &L, const MqVec &vv, int nb, int dt) {
  const int k4 = (threadIdx.x & 63) >> 4;
  MwDst d;
  d.dt = dt;
  d.py = L.lq + vv.a * mw_vs(nb) + 2 * k4;
  d.pw = L.lc + vv.a * mw_cs(nb);
#pragma unroll
  for (int t = 0; t < 4; t++) d.px[t] = L.ld + vv.d[t] * nb;
  return d;
}

// The lane classes a wavefront takes: part C of WPT (WPT 1: all eight; 2: C, C + 2, C + 4, C + 6;
// 4: p and p + 4 with p = 0, 2, 1, 3 for C = 0 .. 3); slot j of its chains holds class
// mw_cls<WPT, C>(j). The parts' partial sums then meet in the reference's hsum order
// ((a0 + a4) + (a2 + a6)) + ((a1 + a5) + (a3 + a7)): WPT 2: A0 + A1 with
// A_C = (a_C + a_C+4) + (a_C+2 + a_C+6); WPT 4: (P0 + P1) + (P2 + P3) with P_C = a_p + a_p+4.
// Part 0 also chains the correction.
template <int WPT, int C>
__host__ __device__ constexpr int mw_cls(int j) {
  return WPT == 1 ? j : WPT == 2 ? C + 2 * j : (C == 0 ? 0 : C == 1 ? 2 : C == 2 ? 1 : 3) + 4 * j;
}
template <int WPT, int C>
__host__ __device__ constexpr int mw_slot(int l) {  // the slot of class l, -1: another part's
  for (int j = 0; j < 8 / WPT; j++)
    if (mw_cls<WPT, C>(j) == l) return j;
  return -1;
}

// One block's integers and scale factors for part C: P[j] = P_l of class slot j (D rows: vectors
// 4 (lane >> 4) + t, columns: matrix rows), Cc the correction integer (part 0; Q6_K 32 C), dx[t] =
// d xd and cf[t] = dmin xd (Q6_K d xd). The arithmetic of several blocks is issued before their
// fp32 chains advance (mw_chain), so the matrix-core latencies overlap.
template <int WPT>
struct MwProd {
  mq_v4i P[8 / WPT], Cc;
  float dx[4], cf[4];
};

// Q6_K classes 4 E .. 4 E + 3 of a block (those of part C) from its ql words c (dwords
// 16 E + 4 k4 ..) and qh words h (dwords 8 E + 2 k4, + 1); sw = the lane's four int8 scales
// (groups 4 k4 .. 4 k4 + 3). Each 6-bit code c times its group's scale sc, W = c sc = 128 hi +
// lo (q6_wsplit: lo 0..127, hi -63..62, both int8): P = 128 D(hi) + D(lo), accumulated on the
// matrix core (exact in int32, the same integer as the digit products of c and sc).
template <int E, int WPT, int C>
__device__ __forceinline__ void mw_q6_half(const uint4 &c, const uint2 &h, uint32_t sw, const SPX_L uint32_t *py, mq_v4i (&P)[8 / WPT]) {
  const int sh = 4 * ((threadIdx.x >> 4) & 1);
  uint32_t q0[4], q1[4], qh[4];
  mw_t4d(c.x, c.z, q0);
  mw_t4d(c.y, c.w, q1);
  mw_t4d(h.x, h.y, qh);
  const uint32_t s0 = (uint32_t)(uint16_t)(int16_t)(int8_t)(sw >> (8 * E)), s1 = (uint32_t)(uint16_t)(int16_t)(int8_t)(sw >> (16 + 8 * E));
  uint32_t wh0[4], wl0[4], wh1[4], wl1[4];
  uint2 y[4];
#pragma unroll
  for (int a = 0; a < 4; a++) {
    if (mw_slot<WPT, C>(4 * E + a) < 0) continue;
    const uint32_t c0 = ((q0[a] >> sh) & 0x0F0F0F0Fu) | (((qh[a] >> sh) & 0x03030303u) << 4);
    const uint32_t c1 = ((q1[a] >> sh) & 0x0F0F0F0Fu) | (((qh[a] >> (sh + 2)) & 0x03030303u) << 4);
    q6_wsplit(c0, s0, wh0[a], wl0[a]);
    q6_wsplit(c1, s1, wh1[a], wl1[a]);
    y[a] = lld<uint2>(py + 8 * (4 * E + a));
  }
  // the classes' contractions interleaved, one dependent step at a time
#pragma unroll
  for (int a = 0; a < 4; a++) {
    const int j = mw_slot<WPT, C>(4 * E + a);
    if (j >= 0) P[j] = mq_mfma(y[a].x, y[a].y, wh0[a], wh1[a]) * 128;
  }
#pragma unroll
  for (int a = 0; a < 4; a++) {
    const int j = mw_slot<WPT, C>(4 * E + a);
    if (j >= 0) P[j] = mq_mfma_c(y[a].x, y[a].y, wl0[a], wl1[a], P[j]);
  }
}

// Block b of a tile, part C: its integers (mw_prod). The class words are regrouped across the
// four 16-lane rows (mw_t4): lane row k4 then holds, for class l, the code word of sub-blocks
// 2 k4, 2 k4 + 1 (Q4_K dword 4 l + k4; Q6_K ql dwords 4 l + 2 (k4 >> 1) + 0, 1 and qh dword
// 2 l + (k4 >> 1)).
template <int T, int WPT, int C>
__device__ __forceinline__ void mw_prod(const MwRaw &r, const MwDst &d, int b, MwProd<WPT> &o) {
  const int k4 = (threadIdx.x & 63) >> 4;
  const SPX_L uint32_t *py = d.py + b * 64, *pw = d.pw + b * MQ_CW;
  float xd[4];
  const float dd = h2f(r.d);
#pragma unroll
  for (int t = 0; t < 4; t++) {
    xd[t] = d.px[t][b];
    o.dx[t] = dd * xd[t];
  }
  if constexpr (T == T_Q4K) {
    uint32_t w[2][4] = {{r.c[0].x, r.c[0].y, r.c[0].z, r.c[0].w}, {r.c[1].x, r.c[1].y, r.c[1].z, r.c[1].w}};
    mw_t4(w[0]);
    mw_t4(w[1]);
    const uint32_t sw = k4 < 2 ? r.s.x : r.s.y, sp = (k4 & 1) ? sw >> 16 : sw;
    const uint32_t s0 = sp & 0xFFu, s1 = (sp >> 8) & 0xFFu;
    const uint32_t lo0 = s0 & 7u, hi0 = s0 >> 3, lo1 = s1 & 7u, hi1 = s1 >> 3;
    // P = D(q sl) + 8 D(q sh), the digits accumulated on the matrix core (exact in int32); the
    // classes interleaved four at a time
    constexpr int CG = 8 / WPT < 4 ? 8 / WPT : 4;
#pragma unroll
    for (int j0 = 0; j0 < 8 / WPT; j0 += CG) {
      uint32_t c0[CG], c1[CG];
      uint2 y[CG];
#pragma unroll
      for (int q = 0; q < CG; q++) {
        const int l = mw_cls<WPT, C>(j0 + q);
        const uint32_t wl = w[l >> 2][l & 3];
        c0[q] = wl & 0x0F0F0F0Fu;
        c1[q] = (wl >> 4) & 0x0F0F0F0Fu;
        y[q] = lld<uint2>(py + 8 * l);
      }
#pragma unroll
      for (int q = 0; q < CG; q++) o.P[j0 + q] = mq_mfma(y[q].x, y[q].y, mx_pmul(c0[q], hi0), mx_pmul(c1[q], hi1)) * 8;
#pragma unroll
      for (int q = 0; q < CG; q++) o.P[j0 + q] = mq_mfma_c(y[q].x, y[q].y, mx_pmul(c0[q], lo0), mx_pmul(c1[q], lo1), o.P[j0 + q]);
    }
    if (C == 0) {
      // C = sum_s mn_s (bsum_2s + bsum_2s+1): K 0-7 the sums' lo, 8-15 their hi, against the mins
      const uint2 cw = lld<uint2>(pw + 8 + 2 * (k4 & 1));
      const uint32_t a0 = k4 < 2 ? cw.x : 0u, a1 = k4 < 2 ? cw.y : 0u;
      o.Cc = mq_mfma_c(a0, a1, r.s.z, r.s.w, mq_mfma(k4 == 1 ? a0 : 0u, k4 == 1 ? a1 : 0u, r.s.z, r.s.w) * 63);
      const float dm = h2f(r.d >> 16);
#pragma unroll
      for (int t = 0; t < 4; t++) o.cf[t] = dm * xd[t];
    }
  } else {
    // the lane's scale dword k4, by shifts of the line (a select among the raw fields would have
    // the compiler index the block buffer in scratch memory)
    const uint64_t s01 = ((uint64_t)r.s.y << 32) | r.s.x, s23 = ((uint64_t)r.s.w << 32) | r.s.z;
    const uint32_t sw = (uint32_t)(((k4 & 2) ? s23 : s01) >> (32 * (k4 & 1)));
    mw_q6_half<0, WPT, C>(r.c[0], r.h[0], sw, py, o.P);
    mw_q6_half<1, WPT, C>(r.c[1], r.h[1], sw, py, o.P);
    if (C == 0) {
      // C = sum_g sc_g bsum_g: K 0-15 the bsums' lo, 16-31 their hi, against the scales
      const uint2 cw = lld<uint2>(pw + 2 * k4);
      const uint32_t b0 = (k4 & 1) ? r.s.z : r.s.x, b1 = (k4 & 1) ? r.s.w : r.s.y;
      const bool lo = k4 < 2;
      o.Cc = mq_mfma_c(cw.x, cw.y, b0, b1, mq_mfma(lo ? 0u : cw.x, lo ? 0u : cw.y, b0, b1) * 63) * 32;
#pragma unroll
      for (int t = 0; t < 4; t++) o.cf[t] = dd * xd[t];
    }
  }
}
// The chains advance by one block: acc_l = fma(d xd, float(P_l), acc_l) and, part 0,
// corr = corr + (dmin xd) float(C) (Q6_K (d xd) float(32 C)).
template <int WPT, int C>
__device__ __forceinline__ void mw_chain(const MwProd<WPT> &o, float (&acc)[8 / WPT][4], float (&cr)[4]) {
#pragma unroll
  for (int j = 0; j < 8 / WPT; j++)
#pragma unroll
    for (int t = 0; t < 4; t++) acc[j][t] = fmaf(o.dx[t], (float)o.P[j][t], acc[j][t]);
  if (C == 0)
#pragma unroll
    for (int t = 0; t < 4; t++) cr[t] = cr[t] + o.cf[t] * (float)o.Cc[t];
}

// The walk of one wavefront (part C of WPT) over its tiles 0 .. ntiles - 1: tile i's bytes from
// src(i), its LDS operands from dst(i). A tile's blocks are taken in stages of PD (mw_pd: NB up
// to three blocks a row, two at four, else four); each block's bytes are requested one stage
// ahead of its arithmetic into a ring of PD buffers (the next tile's first stage during the last
// one, the last tile's first stage again at the end), the same loads on every path, so the
// compiler's wait for a block leaves the PD later blocks in flight. done(i, part, cr) takes
// tile i's partial sums part[t] (WPT 1: the whole hsum less the correction; matrix row lane & 15,
// vector 4 (lane >> 4) + t) and, part 0, the correction chain cr; a done() with barriers is met
// by every wavefront of the workgroup as long as they walk the same number of tiles.
template <int NB>
constexpr int mw_pd() { return NB <= 3 ? NB : NB == 4 ? 2 : 4; }
template <int NB, int TT, int WPT, int C, int PD = mw_pd<NB>(), class Src, class Dst, class Done>
__device__ __forceinline__ void mw_walk(int ntiles, Src src, Dst dst, Done done) {
  constexpr int NS = NB / PD, CPW = 8 / WPT;
  constexpr int BB = WPT == 4 ? PD : WPT == 2 && PD % 2 == 0 ? 2 : 1;  // blocks whose integers are issued together
  static_assert(NB % PD == 0, "whole stages");
  if (ntiles <= 0) return;
  MwRaw r[PD];
  MwSrc sc = src(0);
#pragma unroll
  for (int p = 0; p < PD; p++) mw_fetch<TT>(r[p], sc, p);
  for (int i = 0; i < ntiles; i++) {
    const MwDst dc = dst(i);
    const MwSrc sn = i + 1 < ntiles ? src(i + 1) : sc;
    float acc[CPW][4], cr[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      cr[t] = 0.0f;
#pragma unroll
      for (int j = 0; j < CPW; j++) acc[j][t] = 0.0f;
    }
    for (int st = 0; st < NS; st++) {
      const bool last = st == NS - 1;
      // the stage's integers in groups of BB blocks, then their chains in block order
#pragma unroll
      for (int p0 = 0; p0 < PD; p0 += BB) {
        MwProd<WPT> pr[BB];
#pragma unroll
        for (int q = 0; q < BB; q++) {
          if (TT == T_Q4K || (TT == 0 && dc.dt == T_Q4K)) mw_prod<T_Q4K, WPT, C>(r[p0 + q], dc, st * PD + p0 + q, pr[q]);
          else mw_prod<T_Q6K, WPT, C>(r[p0 + q], dc, st * PD + p0 + q, pr[q]);
        }
#pragma unroll
        for (int q = 0; q < BB; q++) mw_chain<WPT, C>(pr[q], acc, cr);
      }
#pragma unroll
      for (int p = 0; p < PD; p++) {
        const int b = st * PD + p;
        MwSrc fs;
        fs.p0 = last ? sn.p0 : sc.p0;
        fs.p1 = last ? sn.p1 : sc.p1;
        fs.p2 = last ? sn.p2 : sc.p2;
        fs.p3 = last ? sn.p3 : sc.p3;
        fs.rb = last ? sn.rb : sc.rb;
        fs.dt = last ? sn.dt : sc.dt;
        mw_fetch<TT>(r[p], fs, last ? p : b + PD);
      }
    }
    float part[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      if constexpr (WPT == 1)
        part[t] = (((acc[0][t] + acc[4][t]) + (acc[2][t] + acc[6][t])) + ((acc[1][t] + acc[5][t]) + (acc[3][t] + acc[7][t]))) - cr[t];
      else if constexpr (WPT == 2)
        part[t] = (acc[0][t] + acc[2][t]) + (acc[1][t] + acc[3][t]);
      else
        part[t] = acc[0][t] + acc[1][t];
    }
    done(i, part, cr);
    sc = sn;
  }
}
// The walk of part c (wave-uniform) of WPT: one instance per part.
template <int NB, int TT, int WPT, class Src, class Dst, class Done>
__device__ __forceinline__ void mw_walk_part(int c, int ntiles, Src src, Dst dst, Done done) {
  if constexpr (WPT == 1) {
    mw_walk<NB, TT, 1, 0>(ntiles, src, dst, done);
  } else if constexpr (WPT == 2) {
    if (c == 0) mw_walk<NB, TT, 2, 0>(ntiles, src, dst, done);
    else mw_walk<NB, TT, 2, 1>(ntiles, src, dst, done);
  } else {
    switch (c) {
    case 0: mw_walk<NB, TT, 4, 0>(ntiles, src, dst, done); break;
    case 1: mw_walk<NB, TT, 4, 1>(ntiles, src, dst, done); break;
    case 2: mw_walk<NB, TT, 4, 2>(ntiles, src, dst, done); break;
    default: mw_walk<NB, TT, 4, 3>(ntiles, src, dst, done); break;
    }
  }
}
// The parts' partial sums of a tile meet in LDS (xch: [WPT][4][64] floats of the tile's parts, one
// barrier; the caller alternates two such areas between tiles): part 0 returns the tile's
// results (hsum order as at mw_cls, less the correction), other parts return zeros.
template <int WPT>
__device__ __forceinline__ void mw_meet(SPX_L float *xch, int c, const float (&part)[4], const float (&cr)[4], float (&out)[4]) {
  const int lane = threadIdx.x & 63;
  if constexpr (WPT == 1) {
#pragma unroll
    for (int t = 0; t < 4; t++) out[t] = part[t];
  } else {
#pragma unroll
    for (int t = 0; t < 4; t++) xch[(c * 4 + t) * 64 + lane] = part[t];
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 4; t++) {
      auto P = [&](int q) { return xch[(q * 4 + t) * 64 + lane]; };
      if constexpr (WPT == 2) out[t] = c == 0 ? (part[t] + P(1)) - cr[t] : 0.0f;
      else out[t] = c == 0 ? ((part[t] + P(1)) + (P(2) + P(3))) - cr[t] : 0.0f;
    }
  }
}

// ---- staged tiles: a workgroup brings a tile's bytes into LDS once (16-byte coalesced loads)
// and its wavefronts read their classes' words from there (no lane swaps, one memory round a
// tile). Layout of one tile (16 rows, NB blocks a row, row r's block b):
//   codes  r MS_CR + 128 b   (MS_CR = 128 NB + 16: the 16 rows' words of one class in different banks)
//   qh     r MS_HR + 64 b    (Q6_K; MS_HR = 64 NB + 16)
//   scales r MS_SR + 16 b    (MS_SR = 16 NB + 8)
//   d      (r NB + b) 4      (Q4_K d | dmin << 16; Q6_K d in the low half)
template <int NB, bool Q6 = true>  // Q6: room for Q6_K tiles (qh)
struct MsGeo {
  static constexpr int CR = 128 * NB + 16, HR = 64 * NB + 16, SR = 16 * NB + 8;
  static constexpr int OC = 0, OH = OC + 16 * CR, OS = OH + (Q6 ? 16 * HR : 0), OD = OS + 16 * SR, BYTES = OD + 16 * NB * 4;
  // 16-byte chunks of a tile: codes, qh (Q6_K), scale lines
  static constexpr int NCC = 128 * NB, NCH = Q6 ? 64 * NB : 0, NCS = 16 * NB, NC = NCC + NCH + NCS, ND = 16 * NB;
};
// TP (1 or 2) tiles' bytes in registers on their way to LDS: NT threads, chunk i = tid + NT k
// over the tiles' chunks in turn; tile u's image at tl + u MsGeo::BYTES.
struct MsSrc {
  Planes pl;
  int64_t row0;
  int nrows;  // rows past nrows repeat the last
};
template <int NB, int NT, bool Q6, int TP = 1>
struct MsLoad {
  static_assert(TP == 1 || TP == 2, "one or two tiles");
  using G = MsGeo<NB, Q6>;
  static constexpr int KC = (TP * G::NC + NT - 1) / NT, KD = (TP * G::ND + NT - 1) / NT;
  uint4 v[KC];
  uint32_t d[KD];
  __device__ __forceinline__ void get(int dt, const MsSrc &s0, const MsSrc &s1) {
    const int t = threadIdx.x;
    const bool q6 = dt == T_Q6K;
#pragma unroll
    for (int k = 0; k < KC; k++) {
      const int i0 = t + NT * k, u = i0 >= G::NC ? 1 : 0, i = i0 - u * G::NC;
      if (i0 >= TP * G::NC) continue;  // (past the last tile's chunks)
      const MsSrc &sr = u ? s1 : s0;
      const uint8_t *src;
      if (i < G::NCC) {
        const int r = i / (8 * NB), o = i - r * 8 * NB;
        src = sr.pl.p0 + ((sr.row0 + min(r, sr.nrows - 1)) * NB) * 128 + 16 * o;
      } else if (i < G::NCC + G::NCH) {
        const int j = i - G::NCC, r = j / (4 * NB), o = j - r * 4 * NB;
        if (!q6) continue;
        src = sr.pl.p1 + ((sr.row0 + min(r, sr.nrows - 1)) * NB) * 64 + 16 * o;
      } else {
        const int r = (i - G::NCC - G::NCH) / NB, b = (i - G::NCC - G::NCH) - r * NB;
        src = sr.pl.p2 + ((sr.row0 + min(r, sr.nrows - 1)) * NB + b) * 16;
      }
      v[k] = gld<uint4>(src);
    }
#pragma unroll
    for (int k = 0; k < KD; k++) {
      const int i0 = t + NT * k, u = i0 >= G::ND ? 1 : 0, i = i0 - u * G::ND;
      if (i0 >= TP * G::ND) continue;
      const MsSrc &sr = u ? s1 : s0;
      const int r = i / NB, b = i - r * NB;
      const int64_t ra = (sr.row0 + min(r, sr.nrows - 1)) * NB + b;
      d[k] = q6 ? (uint32_t)gld<uint16_t>(sr.pl.p3 + ra * 2) : gld<uint32_t>(sr.pl.p1 + ra * 16);
    }
  }
  __device__ __forceinline__ void get(int dt, const MsSrc &s0) { get(dt, s0, s0); }
  __device__ __forceinline__ void put(SPX_L uint8_t *tl, int dt) const {
    const int t = threadIdx.x;
    const bool q6 = dt == T_Q6K;
#pragma unroll
    for (int k = 0; k < KC; k++) {
      const int i0 = t + NT * k, u = i0 >= G::NC ? 1 : 0, i = i0 - u * G::NC;
      if (i0 >= TP * G::NC) continue;  // (past the last tile's chunks)
      SPX_L uint8_t *tu = tl + u * G::BYTES;
      int o;
      if (i < G::NCC) {
        const int r = i / (8 * NB);
        o = G::OC + r * G::CR + 16 * (i - r * 8 * NB);
      } else if (i < G::NCC + G::NCH) {
        if (!q6) continue;
        const int j = i - G::NCC, r = j / (4 * NB);
        o = G::OH + r * G::HR + 16 * (j - r * 4 * NB);
      } else {
        const int j = i - G::NCC - G::NCH, r = j / NB;
        o = G::OS + r * G::SR + 16 * (j - r * NB);
      }
      // scale lines sit 8-byte aligned: two 8-byte stores
      if (i >= G::NCC + G::NCH) {
        lst<uint2>((SPX_L uint2 *)(tu + o), make_uint2(v[k].x, v[k].y));
        lst<uint2>((SPX_L uint2 *)(tu + o + 8), make_uint2(v[k].z, v[k].w));
      } else {
        lst<uint4>((SPX_L uint4 *)(tu + o), v[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < KD; k++) {
      const int i0 = t + NT * k, u = i0 >= G::ND ? 1 : 0, i = i0 - u * G::ND;
      if (i0 < TP * G::ND) lst<uint32_t>((SPX_L uint32_t *)(tl + u * G::BYTES + G::OD + 4 * i), d[k]);
    }
  }
};
// Block b of a staged tile, part C: its integers (MwProd), as mw_prod from the LDS image.
template <int T, int NB, bool Q6, int WPT, int C>
__device__ __forceinline__ void ms_prod(const SPX_L uint8_t *tl, const MwDst &d, int b, MwProd<WPT> &o) {
  using G = MsGeo<NB, Q6>;
  const int lane = threadIdx.x & 63, k4 = lane >> 4, c16 = lane & 15;
  const SPX_L uint32_t *py = d.py + b * 64, *pw = d.pw + b * MQ_CW;
  const SPX_L uint8_t *rc = tl + G::OC + c16 * G::CR + 128 * b, *rs = tl + G::OS + c16 * G::SR + 16 * b;
  const uint32_t dw = lld<uint32_t>((const SPX_L uint32_t *)(tl + G::OD + 4 * (c16 * NB + b)));
  float xd[4];
  const float dd = h2f(dw);
#pragma unroll
  for (int t = 0; t < 4; t++) {
    xd[t] = d.px[t][b];
    o.dx[t] = dd * xd[t];
  }
  if constexpr (T == T_Q4K) {
    const uint32_t sp = lld<uint16_t>((const SPX_L uint16_t *)(rs + 2 * k4));
    const uint32_t s0 = sp & 0xFFu, s1 = (sp >> 8) & 0xFFu;
    const uint32_t lo0 = s0 & 7u, hi0 = s0 >> 3, lo1 = s1 & 7u, hi1 = s1 >> 3;
    constexpr int CG = 8 / WPT < 4 ? 8 / WPT : 4;
#pragma unroll
    for (int j0 = 0; j0 < 8 / WPT; j0 += CG) {
      uint32_t c0[CG], c1[CG];
      uint2 y[CG];
#pragma unroll
      for (int q = 0; q < CG; q++) {
        const int l = mw_cls<WPT, C>(j0 + q);
        const uint32_t wl = lld<uint32_t>((const SPX_L uint32_t *)(rc + 16 * l + 4 * k4));
        c0[q] = wl & 0x0F0F0F0Fu;
        c1[q] = (wl >> 4) & 0x0F0F0F0Fu;
        y[q] = lld<uint2>(py + 8 * l);
      }
      // P = D(q sl) + 8 D(q sh), the digits accumulated on the matrix core (exact in int32)
#pragma unroll
      for (int q = 0; q < CG; q++) o.P[j0 + q] = mq_mfma(y[q].x, y[q].y, mx_pmul(c0[q], hi0), mx_pmul(c1[q], hi1)) * 8;
#pragma unroll
      for (int q = 0; q < CG; q++) o.P[j0 + q] = mq_mfma_c(y[q].x, y[q].y, mx_pmul(c0[q], lo0), mx_pmul(c1[q], lo1), o.P[j0 + q]);
    }
    if (C == 0) {
      // C = sum_s mn_s (bsum_2s + bsum_2s+1): K 0-7 the sums' lo, 8-15 their hi, against the mins
      const uint2 mn = lld<uint2>((const SPX_L uint2 *)(rs + 8));
      const uint2 cw = lld<uint2>(pw + 8 + 2 * (k4 & 1));
      const uint32_t a0 = k4 < 2 ? cw.x : 0u, a1 = k4 < 2 ? cw.y : 0u;
      o.Cc = mq_mfma_c(a0, a1, mn.x, mn.y, mq_mfma(k4 == 1 ? a0 : 0u, k4 == 1 ? a1 : 0u, mn.x, mn.y) * 63);
      const float dm = h2f(dw >> 16);
#pragma unroll
      for (int t = 0; t < 4; t++) o.cf[t] = dm * xd[t];
    }
  } else {
    const SPX_L uint8_t *rh = tl + G::OH + c16 * G::HR + 64 * b;
    const int h = k4 >> 1, sh = 4 * (k4 & 1);
    const uint32_t sw = lld<uint32_t>((const SPX_L uint32_t *)(rs + 4 * k4));
    uint32_t wh0[8 / WPT], wl0[8 / WPT], wh1[8 / WPT], wl1[8 / WPT];
    uint2 y[8 / WPT];
    // W = c sc = 128 hi + lo per code (q6_wsplit), P = 128 D(hi) + D(lo) on the matrix core; a
    // class's scales: groups 2 s + (l >= 4) of its sub-blocks s = 2 k4, 2 k4 + 1
#pragma unroll
    for (int j = 0; j < 8 / WPT; j++) {
      const int l = mw_cls<WPT, C>(j), hb = l >= 4 ? 8 : 0;
      const uint2 ql = lld<uint2>((const SPX_L uint2 *)(rc + 16 * l + 8 * h));
      const uint32_t qh = lld<uint32_t>((const SPX_L uint32_t *)(rh + 8 * l + 4 * h));
      const uint32_t c0 = ((ql.x >> sh) & 0x0F0F0F0Fu) | (((qh >> sh) & 0x03030303u) << 4);
      const uint32_t c1 = ((ql.y >> sh) & 0x0F0F0F0Fu) | (((qh >> (sh + 2)) & 0x03030303u) << 4);
      q6_wsplit(c0, (uint32_t)(uint16_t)(int16_t)(int8_t)(sw >> hb), wh0[j], wl0[j]);
      q6_wsplit(c1, (uint32_t)(uint16_t)(int16_t)(int8_t)(sw >> (16 + hb)), wh1[j], wl1[j]);
      y[j] = lld<uint2>(py + 8 * l);
    }
#pragma unroll
    for (int j = 0; j < 8 / WPT; j++) o.P[j] = mq_mfma(y[j].x, y[j].y, wh0[j], wh1[j]) * 128;
#pragma unroll
    for (int j = 0; j < 8 / WPT; j++) o.P[j] = mq_mfma_c(y[j].x, y[j].y, wl0[j], wl1[j], o.P[j]);
    if (C == 0) {
      // C = sum_g sc_g bsum_g: K 0-15 the bsums' lo, 16-31 their hi, against the scales
      const uint2 bb = lld<uint2>((const SPX_L uint2 *)(rs + 8 * (k4 & 1)));
      const uint2 cw = lld<uint2>(pw + 2 * k4);
      const bool lo = k4 < 2;
      o.Cc = mq_mfma_c(cw.x, cw.y, bb.x, bb.y, mq_mfma(lo ? 0u : cw.x, lo ? 0u : cw.y, bb.x, bb.y) * 63) * 32;
#pragma unroll
      for (int t = 0; t < 4; t++) o.cf[t] = dd * xd[t];
    }
  }
}
// Part C's chains over a staged tile's NB blocks (integers of BB blocks issued together).
template <int NB, int TT, int WPT, int C>
__device__ __forceinline__ void ms_tile(const SPX_L uint8_t *tl, int dt, const MwDst &d, float (&part)[4], float (&cr)[4]) {
  constexpr int BB = NB % 4 == 0 ? 4 : NB % 2 == 0 ? 2 : 1;
  float acc[8 / WPT][4];
#pragma unroll
  for (int t = 0; t < 4; t++) {
    cr[t] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8 / WPT; j++) acc[j][t] = 0.0f;
  }
  for (int b0 = 0; b0 < NB; b0 += BB) {
    MwProd<WPT> pr[BB];
#pragma unroll
    for (int q = 0; q < BB; q++) {
      if (TT == T_Q4K || (TT == 0 && dt == T_Q4K)) ms_prod<T_Q4K, NB, TT != T_Q4K, WPT, C>(tl, d, b0 + q, pr[q]);
      else ms_prod<T_Q6K, NB, true, WPT, C>(tl, d, b0 + q, pr[q]);
    }
#pragma unroll
    for (int q = 0; q < BB; q++) mw_chain<WPT, C>(pr[q], acc, cr);
  }
#pragma unroll
  for (int t = 0; t < 4; t++) {
    if constexpr (WPT == 1)
      part[t] = (((acc[0][t] + acc[4][t]) + (acc[2][t] + acc[6][t])) + ((acc[1][t] + acc[5][t]) + (acc[3][t] + acc[7][t]))) - cr[t];
    else if constexpr (WPT == 2)
      part[t] = (acc[0][t] + acc[2][t]) + (acc[1][t] + acc[3][t]);
    else
      part[t] = acc[0][t] + acc[1][t];
  }
}
template <int NB, int TT, int WPT>
__device__ __forceinline__ void ms_tile_part(int c, const SPX_L uint8_t *tl, int dt, const MwDst &d, float (&part)[4], float (&cr)[4]) {
  if constexpr (WPT == 2) {
    if (c == 0) ms_tile<NB, TT, 2, 0>(tl, dt, d, part, cr);
    else ms_tile<NB, TT, 2, 1>(tl, dt, d, part, cr);
  } else {
    switch (c) {
    case 0: ms_tile<NB, TT, 4, 0>(tl, dt, d, part, cr); break;
    case 1: ms_tile<NB, TT, 4, 1>(tl, dt, d, part, cr); break;
    case 2: ms_tile<NB, TT, 4, 2>(tl, dt, d, part, cr); break;
    default: ms_tile<NB, TT, 4, 3>(tl, dt, d, part, cr); break;
    }
  }
}

// A unit of kd_mq: tile t (segment si, rows row0 .. row0 + nrows - 1). The bookkeeping is
// wave-uniform and kept scalar (readfirstlane), so the segment's fields are read from the
// arguments with scalar loads.
struct MqPos {
  int t, si, nrows;
  int64_t row0;
};
__device__ __forceinline__ void mq_locate(const DecMMArgs &a, int total, MqPos &p) {
  const int t0 = a.tiles[0], t1 = a.nseg > 1 ? a.tiles[1] : 0, tt = min(p.t, total - 1);
  p.si = __builtin_amdgcn_readfirstlane(tt >= t0 ? (tt >= t0 + t1 ? 2 : 1) : 0);
  p.row0 = (int64_t)(tt - (p.si > 0 ? t0 : 0) - (p.si > 1 ? t1 : 0)) * 16;
  p.nrows = (int)min((int64_t)16, a.w[p.si].rows - p.row0);
}
// Multi-vector matvec on the matrix cores: tiles of 16 rows over up to three segments (the
// formats may differ by segment), the m vectors' Q8_K staged in LDS with their correction
// words. A tile is walked by WPT wavefronts (mw_walk, each a part of the lane classes; their
// partial sums meet in LDS), so a workgroup of MW_NW walks TP = MW_NW / WPT tiles at a time:
// round i of workgroup r takes tiles (r + R i) TP .. + TP - 1. Part 0 runs the epilogue
// (residual, greedy keys). Few tiles (q|k|v, the attention output) take WPT 4: a quarter of the
// classes' arithmetic on each wavefront's path; many (the LM head) WPT 1 (mq_wpt).
//
// Passes of more than 16 rows (prefill) take the vectors in groups of 16: the launch holds
// R x groups workgroups; workgroup i = 8k + x (x: its XCD) takes group k mod groups and tile
// range r = 8 (k / groups) + x, so the groups' workgroups of one tile range share an XCD and its
// L2: the weights come from HBM about once.
constexpr int MW_NW = 4;  // wavefronts a workgroup of kd_mq
template <int NB, int TT, int WPT>  // TT: the segments' one format, or 0 when they differ
__global__ __launch_bounds__(MW_NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void kd_mq(const DecMMArgs a) {
  constexpr int TP = MW_NW / WPT;
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ unsigned long long sbest[MAX_M];
  __shared__ float xch[WPT > 1 ? 2 : 1][MW_NW][4][64];
  const int nvg = (a.m + 15) >> 4;
  int vg = 0, r0 = blockIdx.x, R = gridDim.x;
  if (nvg > 1) {
    const int k = blockIdx.x >> 3;
    vg = k % nvg;
    r0 = (k / nvg) * 8 + (blockIdx.x & 7);
    R = gridDim.x / nvg;
  }
  const int v0 = vg * 16, m = min(16, a.m - v0), cols = a.cols, nb = cols >> 8;
  Q8KP y = a.y;
  y.q += (int64_t)v0 * (cols >> 2);
  y.d += (int64_t)v0 * nb;
  y.bs += (int64_t)v0 * nb * 8;
  const MwLds L = mw_lds(smem, m, nb);
  const int total = a.tiles[0] + (a.nseg > 1 ? a.tiles[1] : 0) + (a.nseg > 2 ? a.tiles[2] : 0);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, c16 = lane & 15;
  const int g = wave / WPT, c = wave - g * WPT;
  if (threadIdx.x < MAX_M) sbest[threadIdx.x] = 0;
  stage_q8<MW_NW * 64>(y, (const int *)nullptr, m, cols, L.lq, L.ld, L.lbs, mw_vs(nb) / 4);
  __syncthreads();
  mq_corr_stage(m, nb, L.lbs, L.lc);
  __syncthreads();
  const MqVec vv = mq_vecs(m, MqIdentity{});
  const int base = r0 * TP, S = R * TP, nr = base < total ? (total - base + S - 1) / S : 0;
  auto pos_of = [&](int i) SPX_AI {
    MqPos p;
    p.t = base + i * S + g;  // (past the last tile: mq_locate's clamp, results not stored)
    mq_locate(a, total, p);
    return p;
  };
  auto src = [&](int i) SPX_AI {
    const MqPos p = pos_of(i);
    const TensorView &w = a.w[p.si];
    return mw_src(w.pl, w.dtype, p.row0, p.nrows, NB);
  };
  auto dst = [&](int i) SPX_AI { return mw_dst(L, vv, NB, a.w[pos_of(i).si].dtype); };
  auto done = [&](int i, const float(&part)[4], const float(&cr)[4]) SPX_AI {
    float out[4];
    mw_meet<WPT>((SPX_L float *)&xch[WPT > 1 ? (i & 1) : 0][g * WPT][0][0], c, part, cr, out);
    if (c != 0 || base + i * S + g >= total) return;
    const MqPos p = pos_of(i);
    float *const o = a.out[p.si];
    const int64_t wrows = a.w[p.si].rows, ldo = a.ld_out[p.si];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const int v = 4 * (lane >> 4) + t;
      if (v < m && c16 < p.nrows) {
        const int64_t row = p.row0 + c16, gv = v0 + v;
        if (o) gst<float>(o + gv * ldo + row, out[t]);
        if (a.res_out) {
          const int64_t q = gv * wrows + row;
          gst<float>(a.res_out + q, gld<float>(a.res_in + q) + a.rscale * out[t]);
        }
        if (a.best) atomicMax(&sbest[v], pick_key(out[t], a.lscale, row));
      }
    }
  };
  mw_walk_part<NB, TT, WPT>(c, nr, src, dst, done);
  if (a.best) {  // per vector, the best key of each tile range
    __syncthreads();
    if ((int)threadIdx.x < m) gst<unsigned long long>(a.best + (int64_t)(v0 + threadIdx.x) * a.nbest + r0, sbest[threadIdx.x]);
  }
}

// kd_mq for up to 16 vectors on staged tiles (few tiles: q|k|v, the attention output): workgroup
// r takes tiles r, r + R, ...; the tile's bytes come into LDS in one round (MsLoad: the next
// tile's loads fly while this one is multiplied), its four wavefronts each take a quarter of the
// lane classes (mw_cls, WPT 4) and their partial sums meet in LDS; part 0 runs the epilogue.
template <int NB, int TT>
__global__ __launch_bounds__(MW_NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void kd_mqs(const DecMMArgs a) {
  static_assert(MW_NW == 4, "a wavefront per part of four");
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ unsigned long long sbest[MAX_M];
  __shared__ float xch[2][MW_NW][4][64];
  const int m = a.m, cols = a.cols;
  const MwLds L = mw_lds(smem, m, NB);
  SPX_L uint8_t *tl = (SPX_L uint8_t *)(smem + mw_tail_off(m, NB));  // (over lbs, once lc is built)
  const int total = a.tiles[0] + (a.nseg > 1 ? a.tiles[1] : 0) + (a.nseg > 2 ? a.tiles[2] : 0);
  const int c = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, c16 = lane & 15;
  const int R = gridDim.x, nr = (int)blockIdx.x < total ? (total - (int)blockIdx.x + R - 1) / R : 0;
  auto pos_of = [&](int i) SPX_AI {
    MqPos p;
    p.t = blockIdx.x + i * R;
    mq_locate(a, total, p);
    return p;
  };
  MsLoad<NB, MW_NW * 64, TT != T_Q4K> ld;
  auto msrc = [&](const MqPos &p) SPX_AI { return MsSrc{a.w[p.si].pl, p.row0, p.nrows}; };
  if (nr > 0) {
    const MqPos p = pos_of(0);
    ld.get(a.w[p.si].dtype, msrc(p));
  }
  if (threadIdx.x < MAX_M) sbest[threadIdx.x] = 0;
  stage_q8<MW_NW * 64>(a.y, (const int *)nullptr, m, cols, L.lq, L.ld, L.lbs, mw_vs(NB) / 4);
  __syncthreads();
  mq_corr_stage(m, NB, L.lbs, L.lc);
  __syncthreads();  // lbs read: the tile may take its place
  const MqVec vv = mq_vecs(m, MqIdentity{});
  for (int i = 0; i < nr; i++) {
    const MqPos p = pos_of(i);
    const int dt = __builtin_amdgcn_readfirstlane(a.w[p.si].dtype);
    ld.put(tl, dt);
    __syncthreads();
    if (i + 1 < nr) {  // the next tile's bytes requested before this one's arithmetic
      const MqPos q = pos_of(i + 1);
      ld.get(a.w[q.si].dtype, msrc(q));
    }
    float part[4], cr[4], out[4];
    ms_tile_part<NB, TT, 4>(c, tl, dt, mw_dst(L, vv, NB, dt), part, cr);
    mw_meet<4>((SPX_L float *)&xch[i & 1][0][0][0], c, part, cr, out);  // (its barrier: the tile is read)
    if (c != 0) continue;
    float *const o = a.out[p.si];
    const int64_t wrows = a.w[p.si].rows, ldo = a.ld_out[p.si];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const int v = 4 * (lane >> 4) + t;
      if (v < m && c16 < p.nrows) {
        const int64_t row = p.row0 + c16;
        if (o) gst<float>(o + v * ldo + row, out[t]);
        if (a.res_out) {
          const int64_t q = v * wrows + row;
          gst<float>(a.res_out + q, gld<float>(a.res_in + q) + a.rscale * out[t]);
        }
        if (a.best) atomicMax(&sbest[v], pick_key(out[t], a.lscale, row));
      }
    }
  }
  if (a.best) {
    __syncthreads();
    if ((int)threadIdx.x < m) gst<unsigned long long>(a.best + (int64_t)threadIdx.x * a.nbest + blockIdx.x, sbest[threadIdx.x]);
  }
}

// Routing + gate/up + SwiGLU over the jobs on the matrix cores (kd_gateup_m's prologue and job
// list): items (job, 16 h rows), TP = NW / WPT of them a round: round i of workgroup b takes
// items (b + G i) TP .. + TP - 1, each walked (gate tile, then up tile) by WPT wavefronts whose
// partial sums meet in LDS; part 0 applies SwiGLU.
template <int T, int NB, int WPT>
__global__ __launch_bounds__(DEC_MM_NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void kd_gateup_mq(const DecGateUpMArgs a) {
  constexpr int NW = DEC_MM_NW, JR = 2 + 2 * MAX_M, TP = NW / WPT;
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ signed char slot_of[MAX_M * 256];
  __shared__ int wcount[NW];
  __shared__ float xch[WPT > 1 ? 2 : 1][NW][4][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int g = wave / WPT, c = wave - g * WPT;
  const int n_ff = a.n_ff, cols = (int)a.gate.cols, nb = cols >> 8, m = a.m;
  const int TX = (n_ff + 15) / 16;
  const MwLds L = mw_lds(smem, m, nb);
  SPX_L int *sj = (SPX_L int *)(smem + mw_act_bytes(m, nb));  // [max jobs][JR]
  int nj = 1;
  {
    StageQ8<NW * 64> st;
    if (a.rt.logits) {
      float lv[2][4];
      route_load<NW>(a.rt, lv);
      st.get(a.y, m, cols);
      nj = route_jobs<NW>(a.rt, lv, sj, (SPX_L signed char *)slot_of, (SPX_L int *)wcount, blockIdx.x == 0);
    } else {
      st.get(a.y, m, cols);
      for (int i = threadIdx.x; i < JR; i += blockDim.x) sj[i] = i == 0 ? 0 : i == 1 ? m : i < 2 + MAX_M ? i - 2 : i - 2 - MAX_M;
    }
    st.put(m, cols, L.lq, L.ld, L.lbs, mw_vs(nb) / 4);
  }
  __syncthreads();
  mq_corr_stage(m, nb, L.lbs, L.lc);
  __syncthreads();
  const int n = TX * nj, base = blockIdx.x * TP, S = gridDim.x * TP, nr = base < n ? (n - base + S - 1) / S : 0;
  auto item = [&](int k) SPX_AI { return min(base + S * (k >> 1) + g, n - 1); };  // tile k: gate (k even) or up
  float gv[4];
  auto src = [&](int k) SPX_AI {
    const int i = item(k), j = i / TX, x = i - j * TX;
    const int e = min(max(sj[j * JR], 0), a.gate.n_expert - 1);
    return mw_src((k & 1) ? a.up.pl : a.gate.pl, T, (int64_t)e * a.gate.rows + (int64_t)x * 16, min(16, n_ff - x * 16), NB);
  };
  auto dst = [&](int k) SPX_AI {
    const int j = item(k) / TX;
    return mw_dst(L, mq_vecs(sj[j * JR + 1], MqRows{sj + j * JR + 2}), NB, T);
  };
  auto done = [&](int k, const float(&part)[4], const float(&cr)[4]) SPX_AI {
    float out[4];
    mw_meet<WPT>((SPX_L float *)&xch[WPT > 1 ? (k & 1) : 0][g * WPT][0][0], c, part, cr, out);
    if (c != 0) return;
    if (!(k & 1)) {
#pragma unroll
      for (int t = 0; t < 4; t++) gv[t] = out[t];
      return;
    }
    if (base + S * (k >> 1) + g >= n) return;
    const int i = item(k), j = i / TX, x = i - j * TX, nv = sj[j * JR + 1], r = lane & 15;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const int v = 4 * (lane >> 4) + t;
      if (v < nv && x * 16 + r < n_ff)
        gst<float>(a.h + (int64_t)sj[j * JR + 2 + MAX_M + v] * n_ff + x * 16 + r, gv[t] / (1.0f + expf(-gv[t])) * out[t]);
    }
  };
  mw_walk_part<NB, T, WPT>(c, 2 * nr, src, dst, done);
}

// kd_gateup_mq on staged tiles: rounds of two items' gate tiles, then their up tiles (MsLoad: a
// round's bytes come into LDS at once, the next round's loads fly during this one); wavefronts
// 0-3 take the first item's tile, 4-7 the second's, a quarter of the lane classes each, their
// partial sums meeting in LDS; part 0 applies SwiGLU. Workgroup b takes item pairs b, b + G, ...
template <int T, int NB>
__global__ __launch_bounds__(DEC_MM_NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void kd_gateup_mqs(const DecGateUpMArgs a) {
  constexpr int NW = DEC_MM_NW, JR = 2 + 2 * MAX_M;
  static_assert(NW == 8, "two items of four wavefronts");
  using G = MsGeo<NB, T == T_Q6K>;
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ signed char slot_of[MAX_M * 256];
  __shared__ int wcount[NW];
  __shared__ float xch[2][NW][4][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int g = wave >> 2, c = wave & 3;
  const int n_ff = a.n_ff, cols = (int)a.gate.cols, m = a.m;
  const int TX = (n_ff + 15) / 16;
  const MwLds L = mw_lds(smem, m, NB);
  SPX_L uint8_t *tl = (SPX_L uint8_t *)(smem + mw_tail_off(m, NB));  // (over lbs, once lc is built)
  SPX_L int *sj = (SPX_L int *)(smem + mw_tail_off(m, NB) + (((size_t)std::max(m * NB * 64, 2 * G::BYTES) + 15) & ~(size_t)15));
  int nj = 1;
  StageQ8<NW * 64> st;
  if (a.rt.logits) {
    float lv[2][4];
    route_load<NW>(a.rt, lv);
    st.get(a.y, m, cols);
    nj = route_jobs<NW>(a.rt, lv, sj, (SPX_L signed char *)slot_of, (SPX_L int *)wcount, blockIdx.x == 0);
  } else {
    st.get(a.y, m, cols);
    for (int i = threadIdx.x; i < JR; i += blockDim.x) sj[i] = i == 0 ? 0 : i == 1 ? m : i < 2 + MAX_M ? i - 2 : i - 2 - MAX_M;
    __syncthreads();
  }
  const int n = TX * nj, R = gridDim.x, np = (n + 1) / 2, nr = (int)blockIdx.x < np ? (np - (int)blockIdx.x + R - 1) / R : 0;
  // round k: item pair blockIdx.x + R (k / 2), gate (k even) or up tiles
  auto item = [&](int k, int u) SPX_AI { return min(2 * ((int)blockIdx.x + R * (k >> 1)) + u, n - 1); };
  auto msrc = [&](int k, int u) SPX_AI {
    const int i = item(k, u), j = i / TX, x = i - j * TX;
    const int e = __builtin_amdgcn_readfirstlane(min(max(sj[j * JR], 0), a.gate.n_expert - 1));
    return MsSrc{(k & 1) ? a.up.pl : a.gate.pl, (int64_t)e * a.gate.rows + (int64_t)x * 16, min(16, n_ff - x * 16)};
  };
  MsLoad<NB, NW * 64, T == T_Q6K, 2> ld;
  if (nr > 0) ld.get(T, msrc(0, 0), msrc(0, 1));
  st.put(m, cols, L.lq, L.ld, L.lbs, mw_vs(NB) / 4);
  __syncthreads();
  mq_corr_stage(m, NB, L.lbs, L.lc);
  __syncthreads();  // lbs read: the tiles may take its place
  float gv[4];
  for (int k = 0; k < 2 * nr; k++) {
    ld.put(tl, T);
    __syncthreads();
    if (k + 1 < 2 * nr) ld.get(T, msrc(k + 1, 0), msrc(k + 1, 1));
    const int i = item(k, g), j = i / TX, x = i - j * TX;
    float part[4], cr[4], out[4];
    ms_tile_part<NB, T, 4>(c, tl + g * G::BYTES, T, mw_dst(L, mq_vecs(sj[j * JR + 1], MqRows{sj + j * JR + 2}), NB, T), part, cr);
    mw_meet<4>((SPX_L float *)&xch[k & 1][4 * g][0][0], c, part, cr, out);  // (its barrier: the tiles are read)
    if (c != 0) continue;
    if (!(k & 1)) {
#pragma unroll
      for (int t = 0; t < 4; t++) gv[t] = out[t];
      continue;
    }
    if (2 * ((int)blockIdx.x + R * (k >> 1)) + g >= n) continue;
    const int nv = sj[j * JR + 1], r = lane & 15;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const int v = 4 * (lane >> 4) + t;
      if (v < nv && x * 16 + r < n_ff)
        gst<float>(a.h + (int64_t)sj[j * JR + 2 + MAX_M + v] * n_ff + x * 16 + r, gv[t] / (1.0f + expf(-gv[t])) * out[t]);
    }
  }
}

// Down projection of the jobs' users on the matrix cores: items (job, DOWN_MQ_ROWS = 8 tiles),
// workgroup b the items b, b + G, ...; at each item the job's users' h rows are quantized into
// LDS (quantize_avx2 per 256 block) as kd_down_m does, and the item's tiles are walked TP =
// NW / WPT at a time (WPT wavefronts a tile, their partial sums meeting in LDS; mw_walk: the
// next item's bytes are requested before its staging); y per (row, choice) to yd.
constexpr int DOWN_MQ_ROWS = 16 * DEC_MM_NW, DOWN_MQ_ITEMS = 64;
template <int T, int NB, int WPT>
__global__ __launch_bounds__(DEC_MM_NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void kd_down_mq(const DecDownMArgs a) {
  constexpr int NW = DEC_MM_NW, JF = 2 + MAX_M, TP = NW / WPT, RI = NW / TP;  // RI: rounds an item
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int s_job[JF];
  __shared__ int ihead[DOWN_MQ_ITEMS][2];  // expert, users of the workgroup's items
  __shared__ float xch[WPT > 1 ? 2 : 1][NW][4][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int g = wave / WPT, c = wave - g * WPT;
  const int dim = (int)a.w.rows, n_ff = (int)a.w.cols, TX = (dim + DOWN_MQ_ROWS - 1) / DOWN_MQ_ROWS, G = gridDim.x;
  const MwLds L = mw_lds(smem, MAX_M, NB);
  const int n = TX * gld<int>(a.njobs), nit = (int)blockIdx.x < n ? (n - (int)blockIdx.x + G - 1) / G : 0;
  for (int k = threadIdx.x; k < min(nit, DOWN_MQ_ITEMS); k += blockDim.x) {
    const int j = ((int)blockIdx.x + G * k) / TX;
    ihead[k][0] = min(max(gld<int>(reinterpret_cast<const int *>(a.jobs + j)), 0), a.w.n_expert - 1);
    ihead[k][1] = min(max(gld<int>(reinterpret_cast<const int *>(a.jobs + j) + 1), 0), MAX_M);
  }
  auto stage = [&](int k) SPX_AI {  // item k's users' h rows, quantized
    __syncthreads();
    const int j = ((int)blockIdx.x + G * k) / TX;
    if ((int)threadIdx.x < JF) {
      const int f = threadIdx.x;
      s_job[f] = gld<int>(reinterpret_cast<const int *>(a.jobs + j) + (f < 2 ? f : 2 + MAX_M + (f - 2)));
    }
    __syncthreads();
    const int nv = min(max(s_job[1], 0), MAX_M), nq = nv * NB;
    for (int q0 = wave; q0 < nq; q0 += 4 * NW) {
      float4 hv[4];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int q = q0 + NW * t;
        if (q < nq) {
          const int u = q / NB, i = q - u * NB;
          hv[t] = gld<float4>(a.h + (int64_t)s_job[2 + u] * n_ff + i * 256 + 4 * lane);
        }
      }
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int q = q0 + NW * t;
        if (q < nq) {
          const int u = q / NB, i = q - u * NB;
          const float am = q8k_amax(hv[t]);
          q8k_block_store(hv[t], am, L.lq + u * mw_vs(NB) + i * 64, L.ld + q, (SPX_L int *)L.lbs + q * 16);
        }
      }
    }
    __syncthreads();
    mq_corr_stage(nv, NB, L.lbs, L.lc);
    __syncthreads();
  };
  auto row0 = [&](int k) SPX_AI {  // tile k: item k / RI, its tile (k % RI) TP + g
    const int it = (int)blockIdx.x + G * (k / RI);
    return (it - (it / TX) * TX) * DOWN_MQ_ROWS + 16 * ((k % RI) * TP + g);
  };
  auto src = [&](int k) SPX_AI {
    const int r0 = row0(k);
    return mw_src(a.w.pl, T, (int64_t)ihead[k / RI][0] * dim + min(r0, dim - 1), max(1, min(16, dim - r0)), NB);
  };
  auto dst = [&](int k) SPX_AI { return mw_dst(L, mq_vecs(ihead[k / RI][1], MqIdentity{}), NB, T); };
  auto done = [&](int k, const float(&part)[4], const float(&cr)[4]) SPX_AI {
    float out[4];
    mw_meet<WPT>((SPX_L float *)&xch[WPT > 1 ? (k & 1) : 0][g * WPT][0][0], c, part, cr, out);
    if (c == 0) {
      const int r0 = row0(k), nv = ihead[k / RI][1], r = lane & 15;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int v = 4 * (lane >> 4) + t;
        if (v < nv && r0 + r < dim) gst<float>(a.yd + (int64_t)s_job[2 + v] * dim + r0 + r, out[t]);
      }
    }
    if (k % RI == RI - 1 && k / RI + 1 < nit) stage(k / RI + 1);  // (its first barrier: every reader of s_job is done)
  };
  if (nit > 0) stage(0);
  mw_walk_part<NB, T, WPT>(c, nit * RI, src, dst, done);
}

// kd_down_mq for passes of up to 16 rows on staged tiles: an item's eight tiles in four rounds
// of two (MsLoad; the next round's loads, the next item's included, fly during this one),
// wavefronts 0-3 on the first tile, 4-7 on the second, a quarter of the lane classes each.
template <int T, int NB>
__global__ __launch_bounds__(DEC_MM_NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void kd_down_mqs(const DecDownMArgs a) {
  constexpr int NW = DEC_MM_NW, JF = 2 + MAX_M, RI = 4;  // RI: rounds an item
  static_assert(DOWN_MQ_ROWS == 16 * 2 * RI, "eight tiles an item");
  using G = MsGeo<NB, T == T_Q6K>;
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int s_job[JF];
  __shared__ int ihead[DOWN_MQ_ITEMS][2];  // expert, users of the workgroup's items
  __shared__ float xch[2][NW][4][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int g = wave >> 2, c = wave & 3;
  const int dim = (int)a.w.rows, n_ff = (int)a.w.cols, TX = (dim + DOWN_MQ_ROWS - 1) / DOWN_MQ_ROWS, R = gridDim.x;
  const MwLds L = mw_lds(smem, MAX_M, NB);
  SPX_L uint8_t *tl = (SPX_L uint8_t *)(smem + mw_tail_off(MAX_M, NB));  // (over lbs between the items' stagings)
  const int n = TX * gld<int>(a.njobs), nit = (int)blockIdx.x < n ? (n - (int)blockIdx.x + R - 1) / R : 0;
  for (int k = threadIdx.x; k < min(nit, DOWN_MQ_ITEMS); k += blockDim.x) {
    const int j = ((int)blockIdx.x + R * k) / TX;
    ihead[k][0] = min(max(gld<int>(reinterpret_cast<const int *>(a.jobs + j)), 0), a.w.n_expert - 1);
    ihead[k][1] = min(max(gld<int>(reinterpret_cast<const int *>(a.jobs + j) + 1), 0), MAX_M);
  }
  __syncthreads();
  // round k: item k / RI, its tiles 2 (k % RI) + u
  auto row0 = [&](int k, int u) SPX_AI {
    const int it = (int)blockIdx.x + R * (k / RI);
    return (it - (it / TX) * TX) * DOWN_MQ_ROWS + 16 * (2 * (k % RI) + u);
  };
  auto msrc = [&](int k, int u) SPX_AI {
    const int r0 = row0(k, u);
    return MsSrc{a.w.pl, (int64_t)ihead[k / RI][0] * dim + min(r0, dim - 1), max(1, min(16, dim - r0))};
  };
  MsLoad<NB, NW * 64, T == T_Q6K, 2> ld;
  if (nit > 0) ld.get(T, msrc(0, 0), msrc(0, 1));
  for (int k = 0; k < nit * RI; k++) {
    if (k % RI == 0) {  // item k / RI: its users' h rows, quantized (quantize_avx2 per 256 block)
      const int j = ((int)blockIdx.x + R * (k / RI)) / TX;
      if ((int)threadIdx.x < JF) {
        const int f = threadIdx.x;
        s_job[f] = gld<int>(reinterpret_cast<const int *>(a.jobs + j) + (f < 2 ? f : 2 + MAX_M + (f - 2)));
      }
      __syncthreads();
      const int nv = min(max(s_job[1], 0), MAX_M), nq = nv * NB;
      for (int q0 = wave; q0 < nq; q0 += 4 * NW) {
        float4 hv[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int q = q0 + NW * t;
          if (q < nq) {
            const int u = q / NB, i = q - u * NB;
            hv[t] = gld<float4>(a.h + (int64_t)s_job[2 + u] * n_ff + i * 256 + 4 * lane);
          }
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const int q = q0 + NW * t;
          if (q < nq) {
            const int u = q / NB, i = q - u * NB;
            const float am = q8k_amax(hv[t]);
            q8k_block_store(hv[t], am, L.lq + u * mw_vs(NB) + i * 64, L.ld + q, (SPX_L int *)L.lbs + q * 16);
          }
        }
      }
      __syncthreads();
      mq_corr_stage(nv, NB, L.lbs, L.lc);
      __syncthreads();  // lbs read: the tiles may take its place
    }
    ld.put(tl, T);
    __syncthreads();
    if (k + 1 < nit * RI) ld.get(T, msrc(k + 1, 0), msrc(k + 1, 1));
    float part[4], cr[4], out[4];
    ms_tile_part<NB, T, 4>(c, tl + g * G::BYTES, T, mw_dst(L, mq_vecs(ihead[k / RI][1], MqIdentity{}), NB, T), part, cr);
    mw_meet<4>((SPX_L float *)&xch[k & 1][4 * g][0][0], c, part, cr, out);  // (its barrier: the tiles are read)
    if (c == 0) {
      const int r0 = row0(k, g), nv = ihead[k / RI][1], r = lane & 15;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int v = 4 * (lane >> 4) + t;
        if (v < nv && r0 + r < dim) gst<float>(a.yd + (int64_t)s_job[2 + v] * dim + r0 + r, out[t]);
      }
    }
    if (k % RI == RI - 1) __syncthreads();  // every reader of s_job and the staged h is done
  }
}

// ------------------------------------------------------------------ prefill passes (17..128 rows)
// Routing of m <= PMAX rows, a wavefront per row (route_row; the rows' results to chosen /
// weights / nkeep), four rows a workgroup.
__global__ __launch_bounds__(256) void kp_route_rows(const DecRouteArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, ne = a.n_expert, b = blockIdx.x * 4 + wave;
  if (b >= a.m) return;
  float lv[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int e = lane + 64 * k;
    lv[k] = e < ne ? gld<float>(a.logits + (int64_t)b * ne + e) : -INFINITY;
  }
  int my_e, keep;
  float my_p, wsum;
  route_row(lv, ne, a.n_used, a.moe_prune, my_e, my_p, keep, wsum);
  if (lane < keep) {
    gst<int>(a.chosen + b * 32 + lane, my_e);
    gst<float>(a.weights + b * 32 + lane, a.norm ? my_p / wsum : my_p);
  }
  if (lane == 0) gst<int>(a.nkeep + b, keep);
}

// The job list of the routed rows in global memory: expert e's users in row order, sixteen a
// job, jobs in expert order (user (b, slot): vec = b, out = b * n_used + slot). A bit mask of
// the rows per expert gives each user its rank, so every user is placed by its own thread.
// njobs[0] = the job count, njobs[2] = the experts with users; expert_count counts each once.
// Every workgroup of the grid (kp_jobs_grid) builds the masks and the job offsets; workgroup g
// places the users of slots 256 (g + G k) + thread and writes the jobs of experts e = g mod G.
__global__ __launch_bounds__(256) void kp_jobs(const DecRouteArgs a) {
  __shared__ unsigned long long mask[256][PMAX / 64];
  __shared__ int jbase[257];
  __shared__ int sch[PMAX * 32], snk[PMAX];  // the rows' choices (-1: none)
  const int tid = threadIdx.x, m = a.m, nu = a.n_used;
  for (int i = tid; i < 256 * (PMAX / 64); i += 256) (&mask[0][0])[i] = 0ull;
  if (tid < m) snk[tid] = gld<int>(a.nkeep + tid);
  {
    constexpr int NL = PMAX * 32 / 256;  // every load in flight at once
    int v[NL];
#pragma unroll
    for (int k = 0; k < NL; k++) v[k] = tid + 256 * k < m * 32 ? gld<int>(a.chosen + tid + 256 * k) : 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NL; k++) {
      const int i = tid + 256 * k;
      if (i < m * 32) sch[i] = (i & 31) < snk[i >> 5] ? v[k] : -1;
    }
  }
  __syncthreads();
  for (int i = tid; i < m * 32; i += 256)
    if (sch[i] >= 0) atomicOr(&mask[sch[i]][i >> 11], 1ull << ((i >> 5) & 63));  // row i >> 5
  __syncthreads();
  int cnt = 0;
#pragma unroll
  for (int w = 0; w < PMAX / 64; w++) cnt += __popcll(mask[tid][w]);
  const int nje = (cnt + MAX_M - 1) / MAX_M;
  // exclusive scan of the experts' job counts (four wavefronts, then their totals)
  const int wave = tid >> 6, lane = tid & 63;
  int incl = nje;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(incl, d, 64);
    if (lane >= d) incl += t;
  }
  __shared__ int wsum[4], wnx[4];
  const unsigned long long used = __ballot(cnt > 0);
  if (lane == 63) wsum[wave] = incl;
  if (lane == 0) wnx[wave] = __popcll(used);
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wave; w++) off += wsum[w];
  jbase[tid] = off + incl - nje;
  const int G = gridDim.x, g = blockIdx.x;
  if (tid == 255 && g == 0) {
    gst<int>(a.njobs, off + incl);
    gst<int>(a.njobs + 2, wnx[0] + wnx[1] + wnx[2] + wnx[3]);
  }
  __syncthreads();
  for (int i = tid + 256 * g; i < m * 32; i += 256 * G) {  // each user at its rank
    const int b = i >> 5, sl = i & 31, e = sch[i];
    if (e < 0) continue;
    int rank = 0;
#pragma unroll
    for (int w = 0; w < PMAX / 64; w++) {
      const unsigned long long mw = mask[e][w];
      rank += w < (b >> 6) ? __popcll(mw) : w == (b >> 6) ? __popcll(mw & ((1ull << (b & 63)) - 1ull)) : 0;
    }
    int *J = reinterpret_cast<int *>(a.jobs + jbase[e] + rank / MAX_M);
    gst<int>(J + 2 + rank % MAX_M, b);
    gst<int>(J + 2 + MAX_M + rank % MAX_M, b * nu + sl);
  }
  if (tid < a.n_expert && cnt > 0 && tid % G == g) {  // each job's expert, user count and unused entries
    for (int j = 0; j < nje; j++) {
      int *J = reinterpret_cast<int *>(a.jobs + jbase[tid] + j);
      const int k = min(MAX_M, cnt - j * MAX_M);
      gst<int>(J, tid);
      gst<int>(J + 1, k);
      for (int q = k; q < MAX_M; q++) { gst<int>(J + 2 + q, 0); gst<int>(J + 2 + MAX_M + q, 0); }
    }
    if (a.expert_count) atomicAdd(a.expert_count + tid, 1);
  }
}

// spx_moe_dev's routing in device memory: row b's k choices (chosen / weights [m][k]) into the
// pipeline's layout (ch32 / w32 [m][32], nkeep [m] = k), a row with an expert id out of range
// or chosen twice kept with no choices (nkeep 0: its output is NaN); one thread a row.
__global__ __launch_bounds__(256) void kp_moe_in(const int *chosen, const float *weights, int m, int k, int ne, int *ch32, float *w32,
                                                 int *nkeep) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= m) return;
  bool ok = true;
  for (int j = 0; j < k; j++) {
    const int e = gld<int>(chosen + (int64_t)b * k + j);
    ok = ok && e >= 0 && e < ne;
    for (int i = 0; i < j; i++) ok = ok && gld<int>(chosen + (int64_t)b * k + i) != e;
    gst<int>(ch32 + b * 32 + j, ok ? e : 0);
    gst<float>(w32 + b * 32 + j, gld<float>(weights + (int64_t)b * k + j));
  }
  gst<int>(nkeep + b, ok ? k : 0);
}
// y[b] = sum over j < nkeep[b], in j order, of w32[b][j] * yd[b k + j] (each product and sum
// rounded, from 0: the combine of moe_forward_batch :1133-1140); NaN for a row kept with no
// choices. A thread per output value.
__global__ __launch_bounds__(256) void kp_moe_combine(const float *yd, const float *w32, const int *nkeep, int k, int dim, float *y,
                                                      int64_t ld_y) {
  const int b = blockIdx.y, i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= dim) return;
  const int nk = gld<int>(nkeep + b);
  float acc = 0.0f;
  for (int j = 0; j < nk; j++) acc = acc + gld<float>(w32 + b * 32 + j) * gld<float>(yd + ((int64_t)b * k + j) * dim + i);
  gst<float>(y + (int64_t)b * ld_y + i, nk > 0 ? acc : __int_as_float(0x7fc00000));
}

// Gate / up + SwiGLU of a prefill pass on the matrix cores over a job list of at most sixteen
// users a job (MoE: kp_route's, in global memory; dense, jobs null: rows 16j .. 16j + 15 as
// job j): items (job, 16 h rows) as kd_gateup_mq takes them, workgroup b the items
// [b n / G, (b + 1) n / G), job by job: the job's users' Q8_K rows are staged in LDS (slot =
// the user's place in the job), then wavefront w walks the job's items w, w + NW, ... of the
// range. An item's arithmetic, and so each h value, is kd_gateup_mq's.
template <int NB>
constexpr int KP_PD() { return NB >= 8 ? 2 : mw_pd<NB>(); }
template <int T, int NB>
__global__ __launch_bounds__(DEC_MM_NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void kp_gateup_mq(const DecGateUpMArgs a,
                                                                                                     const Job *jobs,
                                                                                                     const int *njobs) {
  constexpr int NW = DEC_MM_NW, JR = 2 + 2 * MAX_M;
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int sj[JR];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n_ff = a.n_ff, cols = (int)a.gate.cols, nb = cols >> 8, m = a.m;
  const int TX = (n_ff + 15) / 16;
  const MwLds L = mw_lds(smem, MAX_M, nb);
  const int nj = jobs ? gld<int>(njobs) : (m + MAX_M - 1) / MAX_M;
  const int n = TX * nj, G = gridDim.x;
  const int i0 = (int)((int64_t)blockIdx.x * n / G), i1 = (int)((int64_t)(blockIdx.x + 1) * n / G);
  for (int s0 = i0; s0 < i1;) {
    const int j = s0 / TX, s1 = min(i1, (j + 1) * TX);
    __syncthreads();  // the previous job's users are done with
    if ((int)threadIdx.x < JR) {
      const int f = threadIdx.x;
      sj[f] = jobs ? gld<int>(reinterpret_cast<const int *>(jobs + j) + f)
                   : f == 0 ? 0 : f == 1 ? min(MAX_M, m - MAX_M * j) : MAX_M * j + (f - 2) % MAX_M;
    }
    __syncthreads();
    const int nv = __builtin_amdgcn_readfirstlane(min(max(sj[1], 0), MAX_M));
    const int e = __builtin_amdgcn_readfirstlane(min(max(sj[0], 0), a.gate.n_expert - 1));
    stage_q8<NW * 64>(a.y, (const SPX_L int *)(sj + 2), nv, cols, L.lq, L.ld, L.lbs, mw_vs(nb) / 4);
    __syncthreads();
    mq_corr_stage(nv, nb, L.lbs, L.lc);
    __syncthreads();
    const int cnt = s1 - s0, nit = wave < cnt ? (cnt - wave + NW - 1) / NW : 0;
    const MqVec vv = mq_vecs(nv, MqIdentity{});
    float g[4];
    auto src = [&](int k) SPX_AI {  // tile k: item s0 + wave + NW (k / 2), gate (k even) or up
      const int x = s0 + wave + NW * (k >> 1) - j * TX;
      return mw_src((k & 1) ? a.up.pl : a.gate.pl, T, (int64_t)e * a.gate.rows + (int64_t)x * 16, min(16, n_ff - x * 16), NB);
    };
    auto dst = [&](int) SPX_AI { return mw_dst(L, vv, NB, T); };
    auto done = [&](int k, const float (&out)[4], const float (&)[4]) SPX_AI {
#pragma unroll
      for (int t = 0; t < 4; t++)
        if (!(k & 1)) g[t] = out[t];
      if (!(k & 1)) return;
      const int x = s0 + wave + NW * (k >> 1) - j * TX, r = lane & 15;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int v = 4 * (lane >> 4) + t;
        if (v < nv && x * 16 + r < n_ff) gst<float>(a.h + (int64_t)sj[2 + MAX_M + v] * n_ff + x * 16 + r, g[t] / (1.0f + expf(-g[t])) * out[t]);
      }
    };
    mw_walk<NB, T, 1, 0, KP_PD<NB>()>(2 * nit, src, dst, done);
    s0 = s1;
  }
}

// Down projection of a prefill pass over its job list: tiles (job, 16 rows of the expert's down
// matrix), workgroup b the tiles [b n / G, (b + 1) n / G), job by job as kp_gateup_mq takes its
// items: the job's users' h rows are quantized into LDS once (kd_down_mq's staging, quantize_avx2
// per 256 block), then wavefront w walks the job's tiles w, w + NW, ... of the range with no
// barrier between tiles. A tile's arithmetic is kd_down_mq's one-wavefront tile, so each y value
// has its bits; y per (row, choice) to yd.
template <int T, int NB>
__global__ __launch_bounds__(DEC_MM_NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void kp_down_mq(const DecDownMArgs a) {
  constexpr int NW = DEC_MM_NW, JF = 2 + MAX_M;  // job fields: expert, nvec, out[]
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int s_job[JF];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int dim = (int)a.w.rows, n_ff = (int)a.w.cols, TX = (dim + 15) / 16, G = gridDim.x;
  const MwLds L = mw_lds(smem, MAX_M, NB);
  const int n = TX * gld<int>(a.njobs);
  const int i0 = (int)((int64_t)blockIdx.x * n / G), i1 = (int)((int64_t)(blockIdx.x + 1) * n / G);
  for (int s0 = i0; s0 < i1;) {
    const int j = s0 / TX, s1 = min(i1, (j + 1) * TX);
    __syncthreads();  // the previous job's users are done with
    if ((int)threadIdx.x < JF) {
      const int f = threadIdx.x;
      s_job[f] = gld<int>(reinterpret_cast<const int *>(a.jobs + j) + (f < 2 ? f : 2 + MAX_M + (f - 2)));
    }
    __syncthreads();
    const int nv = __builtin_amdgcn_readfirstlane(min(max(s_job[1], 0), MAX_M));
    const int e = __builtin_amdgcn_readfirstlane(min(max(s_job[0], 0), a.w.n_expert - 1)), nq = nv * NB;
    for (int q0 = wave; q0 < nq; q0 += 4 * NW) {
      float4 hv[4];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int q = q0 + NW * t;
        if (q < nq) {
          const int u = q / NB, i = q - u * NB;
          hv[t] = gld<float4>(a.h + (int64_t)s_job[2 + u] * n_ff + i * 256 + 4 * lane);
        }
      }
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int q = q0 + NW * t;
        if (q < nq) {
          const int u = q / NB, i = q - u * NB;
          const float am = q8k_amax(hv[t]);
          q8k_block_store(hv[t], am, L.lq + u * mw_vs(NB) + i * 64, L.ld + q, (SPX_L int *)L.lbs + q * 16);
        }
      }
    }
    __syncthreads();
    mq_corr_stage(nv, NB, L.lbs, L.lc);
    __syncthreads();
    const int cnt = s1 - s0, nit = wave < cnt ? (cnt - wave + NW - 1) / NW : 0;
    const MqVec vv = mq_vecs(nv, MqIdentity{});
    auto row0 = [&](int k) SPX_AI { return (s0 + wave + NW * k - j * TX) * 16; };
    auto src = [&](int k) SPX_AI {
      const int r0 = row0(k);
      return mw_src(a.w.pl, T, (int64_t)e * dim + r0, min(16, dim - r0), NB);
    };
    auto dst = [&](int) SPX_AI { return mw_dst(L, vv, NB, T); };
    auto done = [&](int k, const float (&out)[4], const float (&)[4]) SPX_AI {
      const int r0 = row0(k), r = lane & 15;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int v = 4 * (lane >> 4) + t;
        if (v < nv && r0 + r < dim) gst<float>(a.yd + (int64_t)s_job[2 + v] * dim + r0 + r, out[t]);
      }
    };
    mw_walk<NB, T, 1, 0, 1>(nit, src, dst, done);
    s0 = s1;
  }
}

// ------------------------------------------------------------------ launchers
static int cu_count() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
  }
  return n;
}

static int nb_bucket(int nb) { return nb <= 1 ? 1 : nb <= 2 ? 2 : nb <= 3 ? 3 : nb <= 4 ? 4 : nb <= 8 ? 8 : 16; }

// kd_mv for one row, kd_mv2 for the two rows of a two-row pass
template <int TT, int BPG, int PD, int NV>
constexpr auto kd_mvn() {
  if constexpr (NV == 1) return kd_mv<TT, BPG, PD>;
  else return kd_mv2<TT, BPG, PD, NV>;
}

template <int TT, int NV>
static hipError_t dec_mv_tt(const DecMVArgs &a, int grid, hipStream_t s) {
  const int nb = a.in.cols >> 8, bpg = (nb + a.G - 1) / a.G;
  const int total = a.tiles[0] + (a.nseg > 1 ? a.tiles[1] : 0) + (a.nseg > 2 ? a.tiles[2] : 0);
  const dim3 b(DEC_MV_NW * 64);
  if constexpr (TT != 0) {
    if (grid < total) {  // tiles stride over the grid: four (two) tiles' weights in flight
      if (a.nseg != 1) return hipErrorInvalidValue;
      if (bpg == 1) hipLaunchKernelGGL((kd_mvn<TT, 1, 4, NV>()), dim3(grid), b, 0, s, a);
      else hipLaunchKernelGGL((kd_mvn<TT, 2, 2, NV>()), dim3(grid), b, 0, s, a);
      return hipGetLastError();
    }
  }
  if (grid != total) return hipErrorInvalidValue;
  if (bpg == 1) hipLaunchKernelGGL((kd_mvn<TT, 1, 1, NV>()), dim3(grid), b, 0, s, a);
  else hipLaunchKernelGGL((kd_mvn<TT, 2, 1, NV>()), dim3(grid), b, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_dec_mv(const DecMVArgs &a, int grid, hipStream_t s) {
  const int nb = a.in.cols >> 8;
  if (a.nseg < 1 || a.nseg > 3 || grid < 1 || nb < 1 || nb > DEC_MAXNB || a.in.cols % 256) return hipErrorInvalidValue;
  int G, R;
  rp_shape(nb, G, R);
  // row groups: rp_shape's, or half as many (two blocks a group, twice the rows a workgroup)
  if (a.G != G && !(a.G == G / 2 && (nb + a.G - 1) / a.G <= 2)) return hipErrorInvalidValue;
  bool all4 = true, all6 = true;
  for (int i = 0; i < a.nseg; i++) {
    if (a.w[i].dtype != T_Q4K && a.w[i].dtype != T_Q6K) return hipErrorInvalidValue;
    if (a.w[i].nb != nb) return hipErrorInvalidValue;
    all4 = all4 && a.w[i].dtype == T_Q4K;
    all6 = all6 && a.w[i].dtype == T_Q6K;
  }
  if (a.nv < 0 || a.nv > 2) return hipErrorInvalidValue;
  if (a.nv == 2) {
    if (all4) return dec_mv_tt<T_Q4K, 2>(a, grid, s);
    if (all6) return dec_mv_tt<T_Q6K, 2>(a, grid, s);
    return dec_mv_tt<0, 2>(a, grid, s);
  }
  if (all4) return dec_mv_tt<T_Q4K, 1>(a, grid, s);
  if (all6) return dec_mv_tt<T_Q6K, 1>(a, grid, s);
  return dec_mv_tt<0, 1>(a, grid, s);
}

hipError_t launch_dec_merge(const DecMergeArgs &a, const StepRec *st, hipStream_t s) {
  if (a.hd == 128) hipLaunchKernelGGL(kd_merge<128>, dim3(a.n_heads), dim3(1024), 0, s, a, st);
  else if (a.hd == 64) hipLaunchKernelGGL(kd_merge<64>, dim3(a.n_heads), dim3(1024), 0, s, a, st);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_dec_router(const DecRouterArgs &a, hipStream_t s) {
  if (a.in.cols % 256 || a.in.cols > 256 * DEC_MAXNB || !a.in.nw || a.nv < 0 || a.nv > 2) return hipErrorInvalidValue;
  if (a.nv == 2) hipLaunchKernelGGL(kd_router<2>, dim3(a.n_expert), dim3(256), 0, s, a);
  else hipLaunchKernelGGL(kd_router<1>, dim3(a.n_expert), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int T, int NV>
static hipError_t dec_gu_t(const DecGateUpArgs &a, dim3 grid, hipStream_t s) {
  const int bpg = ((a.in.cols >> 8) + 3) / 4;
  if constexpr (NV == 2) {
    if (bpg == 1) hipLaunchKernelGGL((kd_gateup2<T, 1>), grid, dim3(DEC_MV_NW * 64), 0, s, a);
    else if (bpg == 2) hipLaunchKernelGGL((kd_gateup2<T, 2>), grid, dim3(DEC_MV_NW * 64), 0, s, a);
    else hipLaunchKernelGGL((kd_gateup2<T, 4>), grid, dim3(DEC_MV_NW * 64), 0, s, a);
  } else {
    if (bpg == 1) hipLaunchKernelGGL((kd_gateup<T, 1>), grid, dim3(DEC_MV_NW * 64), 0, s, a);
    else if (bpg == 2) hipLaunchKernelGGL((kd_gateup<T, 2>), grid, dim3(DEC_MV_NW * 64), 0, s, a);
    else hipLaunchKernelGGL((kd_gateup<T, 4>), grid, dim3(DEC_MV_NW * 64), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_dec_gateup(const DecGateUpArgs &a, hipStream_t s) {
  const int nb = a.in.cols >> 8;
  if (a.in.cols % 256 || nb > DEC_MAXNB || a.gate.nb != nb || a.up.nb != nb || a.gate.dtype != a.up.dtype || !a.in.nw) return hipErrorInvalidValue;
  if (a.logits && (a.n_expert < 1 || a.n_expert > 256 || a.n_used < 1 || a.n_used > 32 || a.n_used > a.n_expert)) return hipErrorInvalidValue;
  if (a.nv < 0 || a.nv > 2) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((a.n_ff + DEC_MV_NW - 1) / DEC_MV_NW), a.logits ? (unsigned)a.n_used : 1u);
  if (a.nv == 2) {
    if (a.gate.dtype == T_Q4K) return dec_gu_t<T_Q4K, 2>(a, grid, s);
    if (a.gate.dtype == T_Q6K) return dec_gu_t<T_Q6K, 2>(a, grid, s);
    return hipErrorInvalidValue;
  }
  if (a.gate.dtype == T_Q4K) return dec_gu_t<T_Q4K, 1>(a, grid, s);
  if (a.gate.dtype == T_Q6K) return dec_gu_t<T_Q6K, 1>(a, grid, s);
  return hipErrorInvalidValue;
}

template <int T, int NV>
static hipError_t dec_down_t(const DecDownArgs &a, hipStream_t s) {
  const dim3 grid((unsigned)((a.w.rows + 7) / 8));
  switch (nb_bucket((int)a.w.nb)) {
  case 1: hipLaunchKernelGGL((kd_down<T, 1, NV>), grid, dim3(512), 0, s, a); break;
  case 2: hipLaunchKernelGGL((kd_down<T, 2, NV>), grid, dim3(512), 0, s, a); break;
  case 3: hipLaunchKernelGGL((kd_down<T, 3, NV>), grid, dim3(512), 0, s, a); break;
  case 4: hipLaunchKernelGGL((kd_down<T, 4, NV>), grid, dim3(512), 0, s, a); break;
  case 8: hipLaunchKernelGGL((kd_down<T, 8, NV>), grid, dim3(512), 0, s, a); break;
  default: hipLaunchKernelGGL((kd_down<T, 16, NV>), grid, dim3(512), 0, s, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_dec_down(const DecDownArgs &a, hipStream_t s) {
  const int nv = a.nv == 2 ? 2 : 1;
  if (a.w.cols % 256 || a.w.nb > DEC_MAXNB || a.n_used < 1 || a.nv < 0 || a.nv > 2 || nv * a.n_used > 32 ||
      (int64_t)nv * a.n_used * a.w.cols > DEC_DOWN_Q)
    return hipErrorInvalidValue;
  if (nv == 2) {
    if (a.w.dtype == T_Q4K) return dec_down_t<T_Q4K, 2>(a, s);
    if (a.w.dtype == T_Q6K) return dec_down_t<T_Q6K, 2>(a, s);
    return hipErrorInvalidValue;
  }
  if (a.w.dtype == T_Q4K) return dec_down_t<T_Q4K, 1>(a, s);
  if (a.w.dtype == T_Q6K) return dec_down_t<T_Q6K, 1>(a, s);
  return hipErrorInvalidValue;
}

// ------------------------------------------------------------------ launchers, m rows
hipError_t launch_dec_norm(const DecNormArgs &a, int m, hipStream_t s) {
  if (a.dim % 256 || a.dim > 256 * DEC_MAXNB || !a.nw || m < 1 || m > PMAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kd_norm, dim3(m), dim3(256), 0, s, a);
  return hipGetLastError();
}

#define SPX_DLDS(kern, sm) \
  if ((sm) > 65536) (void)hipFuncSetAttribute((const void *)(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)(sm))

template <int TT, int QN>
static hipError_t dec_mm_q(const DecMMArgs &a, int grid, int bpg, size_t sm, hipStream_t s) {
  const dim3 b(DEC_MM_NW * 64);
  if (bpg == 1) { SPX_DLDS((kd_mm<TT, 1, QN>), sm); hipLaunchKernelGGL((kd_mm<TT, 1, QN>), dim3(grid), b, sm, s, a); }
  else { SPX_DLDS((kd_mm<TT, 2, QN>), sm); hipLaunchKernelGGL((kd_mm<TT, 2, QN>), dim3(grid), b, sm, s, a); }
  return hipGetLastError();
}

template <int TT>
static hipError_t dec_mm_tt(const DecMMArgs &a, int grid, hipStream_t s) {
  const int nb = a.cols >> 8, bpg = (nb + a.G - 1) / a.G;
  const size_t sm = mm_lds_bytes(a.m, a.cols);
  switch (a.G) {
  case 8: return dec_mm_q<TT, MAX_M / 8>(a, grid, bpg, sm, s);
  case 4: return dec_mm_q<TT, MAX_M / 4>(a, grid, bpg, sm, s);
  case 2: return dec_mm_q<TT, MAX_M / 2>(a, grid, bpg, sm, s);
  default: return dec_mm_q<TT, MAX_M>(a, grid, bpg, sm, s);
  }
}

hipError_t launch_dec_mm(const DecMMArgs &a, int grid, hipStream_t s) {
  const int nb = a.cols >> 8;
  if (a.nseg < 1 || a.nseg > 3 || grid < 1 || nb < 1 || nb > DEC_MAXNB || a.cols % 256 || a.m < 1 || a.m > MAX_M) return hipErrorInvalidValue;
  int G, R;
  rp_shape(nb, G, R);
  if (a.G != G || mm_lds_bytes(a.m, a.cols) > 160 * 1024) return hipErrorInvalidValue;
  bool all4 = true, all6 = true;
  for (int i = 0; i < a.nseg; i++) {
    if ((a.w[i].dtype != T_Q4K && a.w[i].dtype != T_Q6K) || a.w[i].nb != nb) return hipErrorInvalidValue;
    all4 = all4 && a.w[i].dtype == T_Q4K;
    all6 = all6 && a.w[i].dtype == T_Q6K;
  }
  if (a.res_out && a.nseg != 1) return hipErrorInvalidValue;
  if (all4) return dec_mm_tt<T_Q4K>(a, grid, s);
  if (all6) return dec_mm_tt<T_Q6K>(a, grid, s);
  return dec_mm_tt<0>(a, grid, s);
}

// Calls f(std::integral_constant<int, NB>) with the compile-time block count of nb, for the counts
// the matrix-core kernels take (mq_nb_ok: 1, 2, 3, 4, 8, 16); other counts are refused.
template <class F>
static hipError_t with_nb(int nb, F &&f) {
  switch (nb) {
  case 1: return f(std::integral_constant<int, 1>{});
  case 2: return f(std::integral_constant<int, 2>{});
  case 3: return f(std::integral_constant<int, 3>{});
  case 4: return f(std::integral_constant<int, 4>{});
  case 8: return f(std::integral_constant<int, 8>{});
  case 16: return f(std::integral_constant<int, 16>{});
  default: return hipErrorInvalidValue;
  }
}

static size_t ms_tile_bytes(int nb, bool q6) {
  switch (nb) {
  case 1: return q6 ? MsGeo<1, true>::BYTES : MsGeo<1, false>::BYTES;
  case 2: return q6 ? MsGeo<2, true>::BYTES : MsGeo<2, false>::BYTES;
  case 3: return q6 ? MsGeo<3, true>::BYTES : MsGeo<3, false>::BYTES;
  case 4: return q6 ? MsGeo<4, true>::BYTES : MsGeo<4, false>::BYTES;
  case 8: return q6 ? MsGeo<8, true>::BYTES : MsGeo<8, false>::BYTES;
  default: return q6 ? MsGeo<16, true>::BYTES : MsGeo<16, false>::BYTES;
  }
}
// kd_mq's form: up to 16 vectors and up to four tiles a CU, the staged tiles (kd_mqs: four
// wavefronts a tile); taller matrices (the LM head), one wavefront a tile (kd_mq's walk, WPT 1);
// prefill, two (WPT 2: the walk's eight chains and block ring exceed the registers of one
// wavefront when the formats are mixed).
static int mq_wpt(int tiles, int m) { return m > MAX_M ? 2 : tiles > 4 * cu_count() ? 1 : 4; }

hipError_t launch_dec_mq(const DecMMArgs &a, int grid, hipStream_t s) {
  const int nb = a.cols >> 8, nvg = (a.m + 15) / 16;
  if (a.nseg < 1 || a.nseg > 3 || grid < 1 || nb < 1 || nb > DEC_MAXNB || a.cols % 256 || a.m < 1 || a.m > PMAX) return hipErrorInvalidValue;
  if (nvg > 1 && grid % 8) return hipErrorInvalidValue;  // tile ranges come in eights (one per XCD)
  for (int i = 0; i < a.nseg; i++)
    if ((a.w[i].dtype != T_Q4K && a.w[i].dtype != T_Q6K) || a.w[i].nb != nb) return hipErrorInvalidValue;
  if (a.res_out && a.nseg != 1) return hipErrorInvalidValue;
  if (a.best && a.nbest != grid) return hipErrorInvalidValue;
  const size_t sm = mw_act_bytes(std::min(a.m, MAX_M), nb);
  const int total = a.tiles[0] + (a.nseg > 1 ? a.tiles[1] : 0) + (a.nseg > 2 ? a.tiles[2] : 0), wpt = mq_wpt(total, a.m);
  int tt = a.w[0].dtype;
  for (int i = 1; i < a.nseg; i++)
    if (a.w[i].dtype != tt) tt = 0;
  const dim3 g(grid * nvg), b(MW_NW * 64);
  auto go = [&](auto kern) {
    SPX_DLDS(kern, sm);
    hipLaunchKernelGGL(kern, g, b, sm, s, a);
    return hipGetLastError();
  };
  const int mv = std::min(a.m, MAX_M);
  const size_t sms = mw_tail_off(mv, nb) + std::max((size_t)mv * nb * 64, ms_tile_bytes(nb, tt != T_Q4K));
  auto gos = [&](auto kern) {
    SPX_DLDS(kern, sms);
    hipLaunchKernelGGL(kern, g, b, sms, s, a);
    return hipGetLastError();
  };
  return with_nb(nb, [&](auto NBc) {
    constexpr int NB = decltype(NBc)::value;
    auto by_wpt = [&](auto TTc) {
      constexpr int TT = decltype(TTc)::value;
      return wpt == 4 ? gos(kd_mqs<NB, TT>) : wpt == 2 ? go(kd_mq<NB, TT, 2>) : go(kd_mq<NB, TT, 1>);
    };
    if (tt == T_Q4K) return by_wpt(std::integral_constant<int, T_Q4K>{});
    if (tt == T_Q6K) return by_wpt(std::integral_constant<int, T_Q6K>{});
    return by_wpt(std::integral_constant<int, 0>{});
  });
}

bool dec_mq_nb_ok(int nb) { return nb == 1 || nb == 2 || nb == 3 || nb == 4 || nb == 8 || nb == 16; }

// kd_mq's workgroups: MW_NW wavefronts, MW_NW / mq_wpt tiles at a time, two workgroups a CU.
int dec_mq_grid(int tiles, int m) {
  const int slots = 2 * cu_count(), tp = MW_NW / mq_wpt(tiles, m), need = (tiles + tp - 1) / tp;
  if (m <= MAX_M) return std::max(1, std::min(need, slots));
  const int nvg = (m + 15) / 16, per = (slots / nvg + 7) / 8 * 8;
  return std::max(8, std::min((need + 7) / 8 * 8, per));
}

hipError_t launch_dec_gateup_mq(const DecGateUpMArgs &args, int max_jobs, hipStream_t s) {
  DecGateUpMArgs a = args;
  a.max_jobs = max_jobs;
  const int nb = (int)(a.gate.cols >> 8);
  if (a.gate.cols % 256 || nb > DEC_MAXNB || a.gate.nb != nb || a.up.nb != nb || a.gate.dtype != a.up.dtype || a.m < 1 || a.m > MAX_M || max_jobs < 1 ||
      max_jobs > 512 || (a.rt.logits && (max_jobs > a.gate.n_expert || a.rt.m != a.m || a.rt.n_expert < 1 || a.rt.n_expert > 256 || a.rt.n_used < 1 ||
                                         a.rt.n_used > 32 || a.rt.n_used > a.rt.n_expert)))
    return hipErrorInvalidValue;
  if (a.gate.dtype != T_Q4K && a.gate.dtype != T_Q6K) return hipErrorInvalidValue;
  // staged tiles: two items a round, one workgroup a CU; every workgroup routes the pass (the
  // items beyond the job count end at once)
  const size_t jb = (size_t)(a.rt.logits ? max_jobs : 1) * (2 + 2 * MAX_M) * 4;
  const size_t sm = mw_tail_off(a.m, nb) + ((std::max((size_t)a.m * nb * 64, 2 * ms_tile_bytes(nb, a.gate.dtype == T_Q6K)) + 15) & ~(size_t)15) + jb;
  if (sm > 136 * 1024) return hipErrorInvalidValue;
  const int items = ((a.n_ff + 15) / 16) * (a.rt.logits ? max_jobs : 1);
  const dim3 grid((unsigned)std::max(1, std::min((items + 1) / 2, cu_count()))), b(DEC_MM_NW * 64);
  auto go = [&](auto kern) {
    SPX_DLDS(kern, sm);
    hipLaunchKernelGGL(kern, grid, b, sm, s, a);
    return hipGetLastError();
  };
  return with_nb(nb, [&](auto NBc) {
    constexpr int NB = decltype(NBc)::value;
    return a.gate.dtype == T_Q4K ? go(kd_gateup_mqs<T_Q4K, NB>) : go(kd_gateup_mqs<T_Q6K, NB>);
  });
}

static unsigned kp_jobs_grid(int m) { return (unsigned)std::min(16, (m * 32 + 255) / 256); }  // a slot a thread

hipError_t launch_kp_route(const DecRouteArgs &a, hipStream_t s) {
  if (a.m < 1 || a.m > PMAX || a.n_expert < 1 || a.n_expert > 256 || a.n_used < 1 || a.n_used > 32 || a.n_used > a.n_expert || !a.jobs ||
      !a.njobs)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(kp_route_rows, dim3((a.m + 3) / 4), dim3(256), 0, s, a);
  hipLaunchKernelGGL(kp_jobs, dim3(kp_jobs_grid(a.m)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_kp_moe_in(const int *chosen, const float *weights, int m, int k, int ne, int *ch32, float *w32, int *nkeep, hipStream_t s) {
  if (m < 1 || m > PMAX || k < 1 || k > 32 || ne < 1 || ne > 256) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kp_moe_in, dim3((m + 255) / 256), dim3(256), 0, s, chosen, weights, m, k, ne, ch32, w32, nkeep);
  return hipGetLastError();
}

hipError_t launch_kp_jobs(const DecRouteArgs &a, hipStream_t s) {
  if (a.m < 1 || a.m > PMAX || a.n_expert < 1 || a.n_expert > 256 || a.n_used < 1 || a.n_used > 32 || !a.jobs || !a.njobs || !a.chosen ||
      !a.nkeep)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(kp_jobs, dim3(kp_jobs_grid(a.m)), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_kp_moe_combine(const float *yd, const float *w32, const int *nkeep, int m, int k, int dim, float *y, int64_t ld_y, hipStream_t s) {
  if (m < 1 || m > PMAX || k < 1 || k > 32 || dim < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kp_moe_combine, dim3((dim + 255) / 256, m), dim3(256), 0, s, yd, w32, nkeep, k, dim, y, ld_y);
  return hipGetLastError();
}

hipError_t launch_kp_gateup_mq(const DecGateUpMArgs &a, const Job *jobs, const int *njobs, int max_jobs, hipStream_t s) {
  const int nb = (int)(a.gate.cols >> 8);
  if (a.gate.cols % 256 || nb > DEC_MAXNB || a.gate.nb != nb || a.up.nb != nb || a.gate.dtype != a.up.dtype || a.m < 1 || a.m > PMAX ||
      max_jobs < 1 || max_jobs > 512 || (jobs && !njobs))
    return hipErrorInvalidValue;
  const size_t sm = mw_act_bytes(MAX_M, nb);
  const int njob = jobs ? max_jobs : (a.m + MAX_M - 1) / MAX_M, items = ((a.n_ff + 15) / 16) * njob;
  const dim3 grid((unsigned)std::max(1, std::min((items + DEC_MM_NW - 1) / DEC_MM_NW, cu_count()))), b(DEC_MM_NW * 64);
  if (a.gate.dtype != T_Q4K && a.gate.dtype != T_Q6K) return hipErrorInvalidValue;
  return with_nb(nb, [&](auto NBc) {
    constexpr int NB = decltype(NBc)::value;
    if (a.gate.dtype == T_Q4K) { SPX_DLDS((kp_gateup_mq<T_Q4K, NB>), sm); hipLaunchKernelGGL((kp_gateup_mq<T_Q4K, NB>), grid, b, sm, s, a, jobs, njobs); }
    else { SPX_DLDS((kp_gateup_mq<T_Q6K, NB>), sm); hipLaunchKernelGGL((kp_gateup_mq<T_Q6K, NB>), grid, b, sm, s, a, jobs, njobs); }
    return hipGetLastError();
  });
}

hipError_t launch_kp_down_mq(const DecDownMArgs &a, hipStream_t s) {
  if (a.w.cols % 256 || a.w.nb > 4 || a.max_jobs < 1 || a.max_jobs > 512 || !a.h || !a.yd) return hipErrorInvalidValue;
  if (a.w.dtype != T_Q4K && a.w.dtype != T_Q6K) return hipErrorInvalidValue;
  const int items = (int)((a.w.rows + 15) / 16) * a.max_jobs;
  const dim3 grid((unsigned)std::max(1, std::min((items + DEC_MM_NW - 1) / DEC_MM_NW, cu_count()))), b(DEC_MM_NW * 64);
  const size_t sm = mw_act_bytes(MAX_M, (int)a.w.nb);
  return with_nb((int)a.w.nb, [&](auto NBc) {
    constexpr int NB = decltype(NBc)::value;
    auto kern = a.w.dtype == T_Q4K ? kp_down_mq<T_Q4K, NB> : kp_down_mq<T_Q6K, NB>;
    SPX_DLDS(kern, sm);
    hipLaunchKernelGGL(kern, grid, b, sm, s, a);
    return hipGetLastError();
  });
}

// passes of more than 128 jobs on kp_down_mq (SPX_PF_DOWN=0: kd_down_mq, the same bits)
static bool pf_down_on() {
  static const bool on = [] {
    const char *v = std::getenv("SPX_PF_DOWN");
    return !v || atoi(v) != 0;
  }();
  return on;
}

hipError_t launch_dec_down_mq(const DecDownMArgs &a, hipStream_t s) {
  if (a.w.cols % 256 || a.w.nb > 4 || a.max_jobs < 1 || a.max_jobs > 512 || !a.h || !a.yd) return hipErrorInvalidValue;
  const int tx = (int)((a.w.rows + DOWN_MQ_ROWS - 1) / DOWN_MQ_ROWS), G = std::min(tx * a.max_jobs, cu_count());
  if ((tx * a.max_jobs + G - 1) / G > DOWN_MQ_ITEMS) return hipErrorInvalidValue;  // items a workgroup, cached in LDS
  const dim3 grid((unsigned)G), b(DEC_MM_NW * 64);
  const size_t sm = mw_act_bytes(MAX_M, (int)a.w.nb);
  if (a.w.dtype != T_Q4K && a.w.dtype != T_Q6K) return hipErrorInvalidValue;
  auto go = [&](auto kern) {
    SPX_DLDS(kern, sm);
    hipLaunchKernelGGL(kern, grid, b, sm, s, a);
    return hipGetLastError();
  };
  // a pass of up to 16 rows (at most 128 jobs): staged tiles, four wavefronts a tile; prefill:
  // one wavefront a tile
  const size_t sms = mw_tail_off(MAX_M, (int)a.w.nb) + std::max((size_t)MAX_M * a.w.nb * 64, 2 * ms_tile_bytes((int)a.w.nb, a.w.dtype == T_Q6K));
  auto gos = [&](auto kern) {
    SPX_DLDS(kern, sms);
    hipLaunchKernelGGL(kern, grid, b, sms, s, a);
    return hipGetLastError();
  };
  const bool staged = a.max_jobs <= 128;
  if (!staged && pf_down_on()) return launch_kp_down_mq(a, s);  // prefill: contiguous tile ranges, job by job
  return with_nb((int)a.w.nb, [&](auto NBc) {
    constexpr int NB = decltype(NBc)::value;
    if (a.w.dtype == T_Q4K) return staged ? gos(kd_down_mqs<T_Q4K, NB>) : go(kd_down_mq<T_Q4K, NB, 1>);
    return staged ? gos(kd_down_mqs<T_Q6K, NB>) : go(kd_down_mq<T_Q6K, NB, 1>);
  });
}

hipError_t launch_dec_router_m(const DecRouterMArgs &a, hipStream_t s) {
  if (a.dim % 256 || a.dim > 256 * DEC_MAXNB || a.m < 1 || a.m > PMAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kd_router_m, dim3(a.n_expert, (a.m + MAX_M - 1) / MAX_M), dim3(256), 0, s, a);
  return hipGetLastError();
}

int dec_mm_grid(int tiles) {
  const int slots = 2 * cu_count(), per = (tiles + slots - 1) / slots;
  return (tiles + per - 1) / per;
}

template <int T>
static hipError_t dec_gum_t(const DecGateUpMArgs &a, hipStream_t s) {
  const int cols = (int)a.gate.cols, bpg = ((cols >> 8) + 3) / 4;
  const size_t sm = gum_lds_bytes(a.m, cols, a.rt.logits ? a.max_jobs : 1);
  if (sm > 160 * 1024) return hipErrorInvalidValue;
  const int tx = (a.n_ff + DEC_MM_NW - 1) / DEC_MM_NW, items = tx * (a.rt.logits ? a.max_jobs : 1);
  const dim3 grid((unsigned)std::min(items, 2 * cu_count())), b(DEC_MM_NW * 64);
  if (bpg == 1) { SPX_DLDS((kd_gateup_m<T, 1>), sm); hipLaunchKernelGGL((kd_gateup_m<T, 1>), grid, b, sm, s, a); }
  else if (bpg == 2) { SPX_DLDS((kd_gateup_m<T, 2>), sm); hipLaunchKernelGGL((kd_gateup_m<T, 2>), grid, b, sm, s, a); }
  else { SPX_DLDS((kd_gateup_m<T, 4>), sm); hipLaunchKernelGGL((kd_gateup_m<T, 4>), grid, b, sm, s, a); }
  return hipGetLastError();
}

hipError_t launch_dec_gateup_m(const DecGateUpMArgs &args, int max_jobs, hipStream_t s) {
  DecGateUpMArgs a = args;
  a.max_jobs = max_jobs;
  const int nb = (int)(a.gate.cols >> 8);
  if (a.gate.cols % 256 || nb > DEC_MAXNB || a.gate.nb != nb || a.up.nb != nb || a.gate.dtype != a.up.dtype || a.m < 1 || a.m > MAX_M || max_jobs < 1 ||
      max_jobs > 512 || (a.rt.logits && (max_jobs > a.gate.n_expert || a.rt.m != a.m || a.rt.n_expert < 1 || a.rt.n_expert > DEC_MM_NW * 64 ||
                                         a.rt.n_expert > 256 || a.rt.n_used < 1 || a.rt.n_used > 32 || a.rt.n_used > a.rt.n_expert)))
    return hipErrorInvalidValue;
  if (a.gate.dtype == T_Q4K) return dec_gum_t<T_Q4K>(a, s);
  if (a.gate.dtype == T_Q6K) return dec_gum_t<T_Q6K>(a, s);
  return hipErrorInvalidValue;
}

template <int T>
static hipError_t dec_downm_t(const DecDownMArgs &a, hipStream_t s) {
  const int tx = (int)((a.w.rows + DEC_MM_NW * 8 - 1) / (DEC_MM_NW * 8));
  const dim3 grid((unsigned)std::min(tx * a.max_jobs, 2 * cu_count())), b(DEC_MM_NW * 64);
  const size_t sm = downm_lds_bytes((int)a.w.cols);
  switch (nb_bucket((int)a.w.nb)) {
  case 1: hipLaunchKernelGGL((kd_down_m<T, 1>), grid, b, sm, s, a); break;
  case 2: hipLaunchKernelGGL((kd_down_m<T, 2>), grid, b, sm, s, a); break;
  case 3: hipLaunchKernelGGL((kd_down_m<T, 3>), grid, b, sm, s, a); break;
  case 4: hipLaunchKernelGGL((kd_down_m<T, 4>), grid, b, sm, s, a); break;
  default: return hipErrorInvalidValue;  // n_ff > 1024: the expert rows take the fused kernels
  }
  return hipGetLastError();
}

hipError_t launch_dec_down_m(const DecDownMArgs &a, hipStream_t s) {
  if (a.w.cols % 256 || a.w.nb > 4 || a.max_jobs < 1 || a.max_jobs > 512 || a.max_jobs > a.w.n_expert || !a.h || !a.yd) return hipErrorInvalidValue;
  if (a.w.dtype == T_Q4K) return dec_downm_t<T_Q4K>(a, s);
  if (a.w.dtype == T_Q6K) return dec_downm_t<T_Q6K>(a, s);
  return hipErrorInvalidValue;
}

}  // namespace spx
