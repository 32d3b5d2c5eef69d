// The layers of a one-row decode pass as cooperative launches, one a layer (see persist.h).
//
// Grid: two workgroups of 256 threads a CU, all resident at once (hipLaunchCooperativeKernel
// refuses a grid that is not). A MoE layer's seven phases meet at six device-wide barriers:
//   qkv      attn_norm + Q8_K of the residual row (every workgroup), q | k | v rows
//   attn     one (64-position chunk, kv head) item per workgroup: partials (attn.h)
//   merge    one (query head, 32 output values) item per workgroup: the chunks merged in the
//            decode pipeline's order (kd_merge)
//   wo       Q8_K of the attention row, attn_output rows, + residual
//   router   ffn_norm of the row, one F32 router row per workgroup
//   gateup   every workgroup routes the row (route_row), gate / up + SwiGLU of its items
//   down     the chosen experts' down rows, the weighted combine in choice order, + residual
// (a dense layer: gate / up of expert 0, then the down projection as a matvec phase); the launch
// boundary ends the layer. At the start of each phase a workgroup pulls the next phase's weight
// lines into its L2, so their HBM latency overlaps the barrier instead of following it. (The
// layer loop stays on the host: inside one kernel, invariants hoisted out of a 48-layer loop
// would be live across all seven phases and spill.)
//
// Values one workgroup hands to another inside the launch (the residual row, q / k / v,
// attention partials and output, router logits, h, greedy keys) are stored and loaded with
// the sc1 (device-coherent) bit: the L2s of the eight XCDs are not coherent with each other.
// A barrier: every workgroup waits for its own stores (s_waitcnt 0), counts itself in one of 32
// sub-counters, the last of a sub-counter counts into the top counter, and all poll the top
// counter; counters only grow within a pass (epochs continue across the layers' launches) and
// are zeroed before it. A barrier that waits
// longer than BAR_LIMIT sets the error word and every workgroup leaves: the launch always ends.
#include "attn.h"
#include "decode_dev.h"
#include "persist.h"

namespace spx {
namespace {

constexpr int NW = 4;                   // wavefronts per workgroup
constexpr int KB = DEC_MAXNB / NW;      // input-row 256-blocks per wavefront (cols <= 4096)
constexpr int QKV_NT = 3, QKV_BPG = 1;  // q|k|v: row tiles per workgroup, blocks per lane group
constexpr int WO_NT = 1, WO_BPG = 2;    // attn_output and a dense down projection
constexpr int GU_NI = 3, GU_BPG = 2;    // gate/up: (slot, 4-row) items per workgroup, blocks per group
constexpr int DN_NB = 4;                // down: blocks per expert row (n_ff <= 1024)
constexpr int DN_HB = (8 * DN_NB + NW - 1) / NW;  // h blocks per wavefront (8 slots)
constexpr uint64_t BAR_LIMIT = 10000000ull;       // 100 ms of the 100 MHz real-time counter

__device__ __forceinline__ uint32_t ld_coh_u32(rsrc_t r, int off) { return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 16); }

__device__ __forceinline__ bool grid_sync(const PersistArgs &a, unsigned &epoch) {
  __shared__ int s_ok;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (a.tstamp && blockIdx.x == 0 && threadIdx.x == 0) a.tstamp[epoch * 2] = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    const unsigned nwg = gridDim.x, S = nwg < 32u ? nwg : 32u, sub = blockIdx.x % S, per = (nwg - sub + S - 1) / S;
    const unsigned e1 = epoch + 1;
    unsigned *sc = a.bar + 32 * (1 + sub), *top = a.bar;
    int ok = 1;
    bool last = false;
    if (__hip_atomic_fetch_add(sc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == per * e1 - 1)
      last = __hip_atomic_fetch_add(top, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S * e1 - 1;
    if (!last) {
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      while (__hip_atomic_load(top, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < S * e1) {
        if (__hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0 ||
            __builtin_amdgcn_s_memrealtime() - t0 > BAR_LIMIT) {
          __hip_atomic_store(a.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = 0;
          break;
        }
      }
    }
    s_ok = ok;
    if (a.tstamp && blockIdx.x == 0) a.tstamp[epoch * 2 + 1] = __builtin_amdgcn_s_memrealtime();
  }
  epoch++;
  __syncthreads();
  return s_ok != 0;
}

// The input row x (handed over in this launch: coherent loads) and its norm weights, as in_load.
__device__ __forceinline__ void in_load_coh(const DecIn &in, InRow<KB> &r) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nbq = in.cols >> 8;
  const rsrc_t rx = rsrc_of(in.x);
#pragma unroll
  for (int k = 0; k < KB; k++) {
    const int tb = wave + NW * k;
    r.v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    r.w[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tb < nbq) {
      const f4v v = ld_coh4(rx, 16 * (tb * 64 + lane));
      r.v[k] = make_float4(v[0], v[1], v[2], v[3]);
      if (in.nw) r.w[k] = gld<float4>(in.nw + 4 * (tb * 64 + lane));
    }
  }
}

// LDS of the row prologues and chains (the attention item and the down / merge phases use
// `big`, below).
struct InLds {
  uint32_t lq[DEC_MAXNB * 64];
  float ld[DEC_MAXNB];
  int2 lbs[DEC_MAXNB * 8];
  float bsum[DEC_MAXNB];
  float cb[NW][2 * DEC_MAXNB * 10];
};

// ------------------------------------------------------------------ L2 prefetch
// Pulls the 128-byte lines of [p, p + bytes) into this workgroup's L2 ahead of the phase that
// reads them: one direct global->LDS dword per line, into a per-wavefront scratch area that is
// never read (no registers are held across the barrier in between).
typedef __attribute__((address_space(3))) void *lds_ptr;
__device__ __forceinline__ void l2_pull(const void *p, int64_t bytes, uint32_t *scratch) {
  const int wave = threadIdx.x >> 6;
  const int64_t nl = (bytes + 127) >> 7;
  for (int64_t i = threadIdx.x; i < nl; i += PERSIST_NT)
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t *>(p) + 128 * i, (lds_ptr)(scratch + 64 * wave), 4, 0, 0);
}
// rows [r0, r0 + n) (n contiguous rows of nb blocks each) of every plane of a K-quant / F32 tensor
__device__ __forceinline__ void l2_pull_rows(const TensorView &w, int64_t r0, int64_t n, uint32_t *scratch) {
  if (w.dtype == T_Q4K) {
    l2_pull(w.pl.p0 + r0 * w.nb * 128, n * w.nb * 128, scratch);
    l2_pull(w.pl.p1 + r0 * w.nb * 16, n * w.nb * 16, scratch);
  } else if (w.dtype == T_Q6K) {
    l2_pull(w.pl.p0 + r0 * w.nb * 128, n * w.nb * 128, scratch);
    l2_pull(w.pl.p1 + r0 * w.nb * 64, n * w.nb * 64, scratch);
    l2_pull(w.pl.p2 + r0 * w.nb * 16, n * w.nb * 16, scratch);
    l2_pull(w.pl.p3 + r0 * w.nb * 2, n * w.nb * 2, scratch);
  } else if (w.dtype == T_F32) {
    l2_pull(w.pl.p0 + r0 * w.cols * 4, n * w.cols * 4, scratch);
  }
}

// ------------------------------------------------------------------ row-parallel matvec phase
// Tiles of NW * R rows over up to three segments (q | k | v), as kd_mv takes them; workgroup w
// owns tiles w, w + grid, ... (at most NT), their weights held in registers from load() on.
struct MvSeg3 {
  Planes pl[3];
  int dt[3];
  int rows[3];
  int tiles[3];
  int nseg, total, nb, G;
};

__device__ __forceinline__ MvSeg3 mv_segs(const TensorView *w, int nseg) {
  MvSeg3 s{};
  int G, R;
  rp_shape(w[0].nb, G, R);
  s.nseg = nseg;
  s.nb = (int)w[0].nb;
  s.G = G;
  s.total = 0;
  for (int i = 0; i < 3; i++) {
    const bool on = i < nseg;
    s.pl[i] = w[on ? i : 0].pl;
    s.dt[i] = w[on ? i : 0].dtype;
    s.rows[i] = on ? (int)w[i].rows : 0;
    s.tiles[i] = on ? (s.rows[i] + NW * R - 1) / (NW * R) : 0;
    s.total += s.tiles[i];
  }
  return s;
}

struct TileAt {
  int si, row;
};
__device__ __forceinline__ TileAt mv_tile(const MvSeg3 &s, int t) {
  const int wave = threadIdx.x >> 6, grp = (threadIdx.x & 63) >> 3, R = 8 / s.G, r = grp / s.G;
  const int si = t >= s.tiles[0] ? (t >= s.tiles[0] + s.tiles[1] ? 2 : 1) : 0;
  const int tt = t - (si > 0 ? s.tiles[0] : 0) - (si > 1 ? s.tiles[1] : 0);
  return TileAt{si, (tt * NW + wave) * R + r};
}

template <int NT, int BPG, int TT>  // TT: the tensors' format, or 0 when the segments differ
struct MvPhase {
  DRaw raw[NT][BPG];

  __device__ __forceinline__ void load(const MvSeg3 &s) {
    const int grp = (threadIdx.x & 63) >> 3, l = threadIdx.x & 7, gi = grp % s.G;
#pragma unroll
    for (int i = 0; i < NT; i++) {
      const int t = blockIdx.x + gridDim.x * i;
      if (t < s.total) {
        const TileAt ta = mv_tile(s, t);
        const int si = ta.si;
        const Planes pl = si == 0 ? s.pl[0] : si == 1 ? s.pl[1] : s.pl[2];
        const int rows = si == 0 ? s.rows[0] : si == 1 ? s.rows[1] : s.rows[2];
        const int dt = si == 0 ? s.dt[0] : si == 1 ? s.dt[1] : s.dt[2];
        const int64_t grow = ta.row < rows ? ta.row : rows - 1;
        if (TT == T_Q4K || (TT == 0 && dt == T_Q4K)) rp_load<T_Q4K, BPG>(raw[i], pl, grow, s.nb, s.G, gi, l);
        else rp_load<T_Q6K, BPG>(raw[i], pl, grow, s.nb, s.G, gi, l);
      }
    }
  }

  // the weight lines of this workgroup's tiles toward L2 (each tile's rows are contiguous)
  __device__ __forceinline__ static void pull(const MvSeg3 &s, const TensorView *w, uint32_t *scratch) {
    const int R = 8 / s.G;
    for (int i = 0; i < NT; i++) {
      const int t = blockIdx.x + gridDim.x * i;
      if (t >= s.total) break;
      const int si = t >= s.tiles[0] ? (t >= s.tiles[0] + s.tiles[1] ? 2 : 1) : 0;
      const int tt = t - (si > 0 ? s.tiles[0] : 0) - (si > 1 ? s.tiles[1] : 0);
      const int64_t r0 = (int64_t)tt * NW * R, n = min((int64_t)NW * R, (int64_t)s.rows[si] - r0);
      l2_pull_rows(w[si], r0, n, scratch);
    }
  }

  // in: the input row (coherent) and its norm; out[si] (coherent) and / or the residual
  // res_out = res_in + rscale * y (coherent; one segment).
  __device__ __forceinline__ void run(const MvSeg3 &s, const DecIn &in, float *const *out, const float *res_in, float *res_out,
                                      float rscale, InLds &L) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane >> 3, l = lane & 7;
    const int G = s.G, R = 8 / G, r = grp / G, gi = grp - r * G, nb = s.nb;
    SPX_L uint32_t *lq = (SPX_L uint32_t *)L.lq;
    SPX_L float *ld = (SPX_L float *)L.ld, *bsum = (SPX_L float *)L.bsum;
    SPX_L int2 *lbs = (SPX_L int2 *)L.lbs;
    SPX_L float *cbr = (SPX_L float *)L.cb[wave] + r * nb * 10;
    InRow<KB> x;
    in_load_coh(in, x);
    in_quant<NW, KB>(in, x, lq, ld, (SPX_L int *)lbs, bsum, nullptr);
    __syncthreads();
    const rsrc_t rres = rsrc_of(res_in ? res_in : res_out), rout = rsrc_of(res_out ? res_out : out[0]);
#pragma unroll
    for (int i = 0; i < NT; i++) {
      const int t = blockIdx.x + gridDim.x * i;
      if (t < s.total) {
        const TileAt ta = mv_tile(s, t);
        const int si = ta.si;
        const int rows = si == 0 ? s.rows[0] : si == 1 ? s.rows[1] : s.rows[2];
        const int dt = si == 0 ? s.dt[0] : si == 1 ? s.dt[1] : s.dt[2];
        if (TT == T_Q4K || (TT == 0 && dt == T_Q4K)) rp_dots<T_Q4K, BPG>(raw[i], nb, G, gi, l, lq, ld, lbs, cbr);
        else rp_dots<T_Q6K, BPG>(raw[i], nb, G, gi, l, lq, ld, lbs, cbr);
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the chain buffer is written
        __builtin_amdgcn_wave_barrier();
        if (gi == 0) {
          const float res = rp_chain(cbr, nb, l);
          if (l == 0 && ta.row < rows) {
            float *o = si == 0 ? out[0] : si == 1 ? out[1] : out[2];
            if (o) st_coh1(rsrc_of(o), ta.row * 4, res);
            if (res_out) st_coh1(rout, ta.row * 4, ld_coh1(rres, ta.row * 4) + rscale * res);
          }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();  // the chain buffer is refilled by the next tile
      }
    }
  }
};

constexpr int TGU = T_Q4K, TDN = T_Q6K, TWO = T_Q4K;  // the Q4_K_M formats (persist_fits)

// ------------------------------------------------------------------ attention partials
template <int HD>
__device__ __forceinline__ AttnArgs attn_args(const PersistArgs &a, const PLayer &ly, int layer) {
  AttnArgs aa{};
  aa.q = a.q; aa.k = a.k; aa.v = a.v;
  aa.q_bias = ly.q_bias; aa.k_bias = ly.k_bias; aa.v_bias = ly.v_bias; aa.q_norm = ly.q_norm; aa.k_norm = ly.k_norm;
  aa.rope = a.rope; aa.kc = a.kc; aa.vc = a.vc; aa.part_ml = a.part_ml; aa.part_o = a.part_o;
  aa.layer = layer; aa.max_seq = a.max_seq; aa.kv_dim = a.kv_dim; aa.hd = HD; aa.n_heads = a.n_heads; aa.n_kv = a.n_kv;
  aa.neox = a.neox; aa.nch = a.nch; aa.nslot = a.nslot; aa.eps = a.eps; aa.scale = a.attn_scale;
  return aa;
}

// ------------------------------------------------------------------ the pass
template <int HD>
__global__ __launch_bounds__(PERSIST_NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void kp_layer(const PersistArgs a, const PLayer ly,
                                                                                                   const int li, unsigned epoch) {
  __shared__ __align__(16) uint8_t big[AttnLds<HD>::BYTES];
  __shared__ __align__(16) InLds L;
  __shared__ __align__(16) uint32_t pf[NW * 64];  // L2-pull scratch (written, never read)
  __shared__ int s_e[32];
  __shared__ float s_w[32];
  __shared__ int s_keep;
  __shared__ float ys[NW][8];
  __shared__ unsigned long long sbest[NW];
  __shared__ float part[NW];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, grp = lane >> 3, l = lane & 7;
  const int W = gridDim.x, w0 = blockIdx.x;
  const int start = a.st->start, total = start + 1;
  const int nch_act = (total + 63) >> 6, nitems = nch_act * a.n_kv;
  const int dim = a.dim, n_ff = a.n_ff;
  if (a.tstamp && w0 == 0 && threadIdx.x == 0) a.tstamp[1024 + 2 * li] = __builtin_amdgcn_s_memrealtime();

  auto qkv_w = [&](const PLayer &ly, TensorView *w3) { w3[0] = ly.wq; w3[1] = ly.wk; w3[2] = ly.wv; };
  // K and V rows of this workgroup's first attention item toward L2
  auto pull_kv = [&](int layer) {
    if (w0 >= nitems) return;
    const int c = w0 / a.n_kv, h = w0 % a.n_kv;
    const int64_t row0 = (int64_t)layer * a.max_seq + (int64_t)c * 64, n = min(64, total - c * 64);
    for (int p = threadIdx.x; p < 2 * n * HD * 2 / 128; p += PERSIST_NT) {  // (position, 128-byte piece), K then V
      const int kv = p / (n * HD * 2 / 128), q = p % (n * HD * 2 / 128), pos = q / (HD * 2 / 128), piece = q % (HD * 2 / 128);
      const __half *base = (kv ? a.vc : a.kc) + (row0 + pos) * a.kv_dim + (int64_t)h * HD;
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t *>(base) + 128 * piece, (lds_ptr)(pf + 64 * wave), 4, 0, 0);
    }
  };
  {
    // ---------------- q | k | v
    {
      TensorView w3[3];
      qkv_w(ly, w3);
      const MvSeg3 sg = mv_segs(w3, 3);
      MvPhase<QKV_NT, QKV_BPG, 0> qkv;
      qkv.load(sg);
      pull_kv(li);
      float *o3[3] = {a.q, a.k, a.v};
      qkv.run(sg, DecIn{a.xa, ly.attn_norm, a.eps, dim}, o3, nullptr, nullptr, 0.0f, L);
    }
    if (!grid_sync(a, epoch)) return;
    // ---------------- attention partials
    {
      const TensorView w1[1] = {ly.wo};
      MvPhase<WO_NT, WO_BPG, TWO>::pull(mv_segs(w1, 1), w1, pf);
    }
    for (int i = w0; i < nitems; i += W) {
      const AttnArgs aa = attn_args<HD>(a, ly, li);
      uint32_t kr[HD / 8], vr[HD / 8];
      attn_kv_first<HD, false>(aa, total, i / a.n_kv, i % a.n_kv, kr, vr);
      attn_item<HD, false, true>(aa, 1, start, i / a.n_kv, i % a.n_kv, 0, big, kr, vr);
      __syncthreads();
    }
    if (!grid_sync(a, epoch)) return;
    // ---------------- merge (kd_merge's order: groups of ATT_GRP chunks, then the groups)
    if (ly.moe && w0 < a.n_expert) l2_pull_rows(ly.router, w0, 1, pf);
    {
      float(*sO)[32] = reinterpret_cast<float(*)[32]>(big);
      float *sM = reinterpret_cast<float *>(big + ATT_GMAX * 32 * 4), *sL = sM + ATT_GMAX;
      const int g = a.n_heads / a.n_kv, nq = HD / 32, nmi = a.n_heads * nq;
      const int dl = threadIdx.x & 31, gs = threadIdx.x >> 5;  // 8 group lanes
      const int ngrp = (nch_act + ATT_GRP - 1) / ATT_GRP;
      const rsrc_t rml = rsrc_of(a.part_ml), ro = rsrc_of(a.part_o);
      for (int it = w0; it < nmi; it += W) {
        const int head = it / nq, d = (it % nq) * 32 + dl, h = head / g, qi = head % g;
        for (int gi = gs; gi < ngrp; gi += 8) {
          const int s0 = gi * ATT_GRP, n = min(ATT_GRP, nch_act - s0);
          float2 ml[ATT_GRP];
          float ov[ATT_GRP];
#pragma unroll
          for (int k = 0; k < ATT_GRP; k++) {
            const int c = s0 + min(k, n - 1);
            const f2v mv = ld_coh2(rml, (((h * a.nslot) + c) * ATT_QMAX + qi) * 8);
            ml[k] = k < n ? make_float2(mv[0], mv[1]) : make_float2(-INFINITY, 0.0f);
            ov[k] = ld_coh1(ro, ((((h * a.nslot) + c) * ATT_QMAX + qi) * HD + d) * 4);
          }
          float M = -INFINITY;
#pragma unroll
          for (int k = 0; k < ATT_GRP; k++) M = fmaxf(M, ml[k].x);
          float Ls = 0.0f, acc = 0.0f;
#pragma unroll
          for (int k = 0; k < ATT_GRP; k++) {
            if (k < n) {
              const float wgt = ml[k].x == -INFINITY ? 0.0f : expf(ml[k].x - M);
              Ls = fmaf(ml[k].y, wgt, Ls);
              acc = fmaf(ov[k], wgt, acc);
            }
          }
          sO[gi][dl] = acc;
          if (dl == 0) { sM[gi] = M; sL[gi] = Ls; }
        }
        __syncthreads();
        if (gs == 0) {
          float out;
          if (ngrp == 1) {
            out = sO[0][dl] * __fdiv_rn(1.0f, fmaxf(sL[0], 1e-30f));
          } else {
            float M = -INFINITY;
            for (int k = 0; k < ngrp; k++) M = fmaxf(M, sM[k]);
            float Ls = 0.0f, acc = 0.0f;
            for (int k = 0; k < ngrp; k++) {
              const float wgt = sM[k] == -INFINITY ? 0.0f : expf(sM[k] - M);
              Ls = fmaf(sL[k], wgt, Ls);
              acc = fmaf(sO[k][dl], wgt, acc);
            }
            out = acc * __fdiv_rn(1.0f, fmaxf(Ls, 1e-30f));
          }
          st_coh1(rsrc_of(a.att), (head * HD + d) * 4, out);
        }
        __syncthreads();
      }
    }
    if (!grid_sync(a, epoch)) return;
    // ---------------- attn_output + residual (xa -> xb)
    {
      const TensorView w1[1] = {ly.wo};
      const MvSeg3 sg = mv_segs(w1, 1);
      MvPhase<WO_NT, WO_BPG, TWO> wo;
      wo.load(sg);
      float *o1[3] = {nullptr, nullptr, nullptr};
      wo.run(sg, DecIn{a.att, nullptr, 0.0f, a.q_dim}, o1, a.xa, a.xb, a.rscale, L);
    }
    if (!grid_sync(a, epoch)) return;
    // ---------------- router (one F32 row per workgroup; kd_router's arithmetic)
    if (ly.moe) {
      const int e = w0;
      if (e < a.n_expert) {
        const DecIn in{a.xb, ly.ffn_norm, a.eps, dim};
        InRow<KB> x;
        in_load_coh(in, x);
        float4 rw[KB];
        const float4 *wr = reinterpret_cast<const float4 *>(ly.router.pl.p0 + (int64_t)e * dim * 4);
#pragma unroll
        for (int k = 0; k < KB; k++) {
          const int f = wave * 64 + lane + 256 * k;
          rw[k] = f < dim / 4 ? wr[f] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        const int nbq = dim >> 8;
#pragma unroll
        for (int k = 0; k < KB; k++) {
          const int tb = wave + NW * k;
          if (tb < nbq) {
            float p = x.v[k].x * x.v[k].x;
            p = fmaf(x.v[k].y, x.v[k].y, p);
            p = fmaf(x.v[k].z, x.v[k].z, p);
            p = fmaf(x.v[k].w, x.v[k].w, p);
            p = wave_sum(p);
            if (lane == 0) L.bsum[tb] = p;
          }
        }
        __syncthreads();
        float S = 0.0f;
        for (int k = 0; k < nbq; k++) S = S + L.bsum[k];
        const float inv = inv_rms(S, (float)dim, a.eps);
        float pv = 0.0f;
#pragma unroll
        for (int k = 0; k < KB; k++) {
          const int f = wave * 64 + lane + 256 * k;
          if (f < dim / 4) {
            float4 xv = x.v[k];
            const float4 wn = x.w[k];
            xv.x = xv.x * inv * wn.x; xv.y = xv.y * inv * wn.y; xv.z = xv.z * inv * wn.z; xv.w = xv.w * inv * wn.w;
            pv = fmaf(rw[k].x, xv.x, pv);
            pv = fmaf(rw[k].y, xv.y, pv);
            pv = fmaf(rw[k].z, xv.z, pv);
            pv = fmaf(rw[k].w, xv.w, pv);
          }
        }
        const float tsum = wave_sum(pv);
        if (lane == 0) part[wave] = tsum;
        __syncthreads();
        if (threadIdx.x == 0) st_coh1(rsrc_of(a.rlog), e * 4, ((part[0] + part[1]) + part[2]) + part[3]);
      }
      if (!grid_sync(a, epoch)) return;
    }
    // ---------------- routing + gate / up + SwiGLU (kd_gateup's arithmetic)
    {
      const int nb = dim >> 8, half = grp >> 2, gi = grp & 3;
      float lv[4];
      if (ly.moe && wave == 0) {
        const rsrc_t rl = rsrc_of(a.rlog);
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int e = lane + 64 * k;
          lv[k] = e < a.n_expert ? ld_coh1(rl, e * 4) : -INFINITY;
        }
      }
      const DecIn in{a.xb, ly.ffn_norm, a.eps, dim};
      InRow<KB> x;
      in_load_coh(in, x);
      if (ly.moe) {
        if (wave == 0) {
          int my_e, keep;
          float my_p, wsum;
          route_row(lv, a.n_expert, a.n_used, a.moe_prune, my_e, my_p, keep, wsum);
          const float wt = a.expert_norm ? my_p / wsum : my_p;
          if (lane < a.n_used) { s_e[lane] = my_e; s_w[lane] = wt; }
          if (lane == 0) s_keep = keep;
          if (w0 == 0) {
            if (lane < keep) {
              gst<int>(a.chosen + lane, my_e);
              gst<float>(a.weights + lane, wt);
              if (ly.expert_count) gst<int>(ly.expert_count + my_e, gld<int>(ly.expert_count + my_e) + 1);
            }
            if (lane == 0) { gst<int>(a.nkeep, keep); gst<int>(ly.njobs, keep); }
          }
        }
      } else if (threadIdx.x == 0) {
        s_e[0] = 0;
        s_w[0] = 1.0f;
        s_keep = 1;
      }
      __syncthreads();
      const int keep = s_keep, nrb = (n_ff + NW - 1) / NW, nitem = keep * nrb;
      DRaw raw[GU_NI][GU_BPG];
#pragma unroll
      for (int j = 0; j < GU_NI; j++) {
        const int it = w0 + W * j;
        if (it < nitem) {
          const int s = it / nrb, r = (it % nrb) * NW + wave;
          const int64_t grow = (int64_t)s_e[s] * ly.gate.rows + (r < n_ff ? r : n_ff - 1);
          rp_load<TGU, GU_BPG>(raw[j], half ? ly.up.pl : ly.gate.pl, grow, nb, 4, gi, l);
        }
      }
      // the down rows of the chosen experts toward L2 (this workgroup's NW output rows)
      if (ly.moe && w0 * NW < dim)
        for (int s = 0; s < keep; s++) l2_pull_rows(ly.down, (int64_t)s_e[s] * dim + w0 * NW, min(NW, dim - w0 * NW), pf);
      SPX_L uint32_t *lq = (SPX_L uint32_t *)L.lq;
      SPX_L float *ld = (SPX_L float *)L.ld, *bsum = (SPX_L float *)L.bsum;
      SPX_L int2 *lbs = (SPX_L int2 *)L.lbs;
      SPX_L float *cbr = (SPX_L float *)L.cb[wave] + half * nb * 10;
      in_quant<NW, KB>(in, x, lq, ld, (SPX_L int *)lbs, bsum, nullptr);
      __syncthreads();
      const rsrc_t rh = rsrc_of(a.h);
#pragma unroll
      for (int j = 0; j < GU_NI; j++) {
        const int it = w0 + W * j;
        if (it < nitem) {
          const int s = it / nrb, r = (it % nrb) * NW + wave;
          rp_dots<TGU, GU_BPG>(raw[j], nb, 4, gi, l, lq, ld, lbs, cbr);
          __builtin_amdgcn_s_waitcnt(0xc07f);
          __builtin_amdgcn_wave_barrier();
          const float res = gi == 0 ? rp_chain(cbr, nb, l) : 0.0f;
          uint32_t r_lo, r_hi;  // lanes 0-31 get the up row's result from lanes 32-63
          xchg32(__float_as_uint(res), r_lo, r_hi);
          const float u = __uint_as_float(r_hi);
          if (lane == 0 && r < n_ff) {
            const float xg = res;
            st_coh1(rh, (s * n_ff + r) * 4, xg / (1.0f + expf(-xg)) * u);
          }
          __builtin_amdgcn_s_waitcnt(0xc07f);
          __builtin_amdgcn_wave_barrier();
        }
      }
    }
    if (!grid_sync(a, epoch)) return;
    // ---------------- down + weighted combine + residual (xb -> xa)
    if (ly.moe) {  // kd_down's arithmetic with one wavefront per output row
      const int nbh = n_ff >> 8, nk = s_keep, nqa = a.n_used * nbh, nqb = nk * nbh;
      const int r = w0 * NW + wave, rr = r < dim ? r : dim - 1;
      const int s = grp, sv = s < nk ? s : nk - 1;
      DRaw dnr[DN_NB];
      draw_row<TDN, DN_NB>(dnr, ly.down.pl, (int64_t)s_e[sv] * dim + rr, nbh, l);
      SPX_L uint32_t *lqh = (SPX_L uint32_t *)big;
      SPX_L float *ldh = (SPX_L float *)(big + 8 * DN_NB * 256);
      SPX_L int2 *lbsh = (SPX_L int2 *)(big + 8 * DN_NB * 256 + 8 * DN_NB * 4);
      const rsrc_t rh = rsrc_of(a.h);
      float4 hv[DN_HB];
#pragma unroll
      for (int k = 0; k < DN_HB; k++) {
        const int vb = wave + NW * k;
        hv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (vb < nqa) {
          const f4v t = ld_coh4(rh, (((vb / nbh) * n_ff) + (vb % nbh) * 256 + 4 * lane) * 4);
          hv[k] = make_float4(t[0], t[1], t[2], t[3]);
        }
      }
#pragma unroll
      for (int k = 0; k < DN_HB; k++) {
        const int vb = wave + NW * k;
        if (vb < nqb) {
          const float am = q8k_amax(hv[k]);
          q8k_block_store(hv[k], am, lqh + vb * 64, ldh + vb, (SPX_L int *)(lbsh + vb * 8));
        }
      }
      __syncthreads();
      float y;
      y = dot_row<TDN, DN_NB>(dnr, nbh, l, lqh + sv * nbh * 64, ldh + sv * nbh, lbsh + sv * nbh * 8);
      if (l == 0 && s < nk) ys[wave][s] = y;
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
      if (lane == 0 && r < dim) {
        float acc = 0.0f;
        for (int i = 0; i < nk; i++) acc = acc + s_w[i] * ys[wave][i];
        const rsrc_t rb = rsrc_of(a.xb);
        st_coh1(rsrc_of(a.xa), r * 4, ld_coh1(rb, r * 4) + a.rscale * acc);
      }
    } else {  // dense down: a matvec phase over the h row
      const TensorView w1[1] = {ly.down};
      const MvSeg3 sd = mv_segs(w1, 1);
      MvPhase<WO_NT, WO_BPG, TDN> dn;
      dn.load(sd);
      float *o1[3] = {nullptr, nullptr, nullptr};
      dn.run(sd, DecIn{a.h, nullptr, 0.0f, n_ff}, o1, a.xb, a.xa, a.rscale, L);
    }
  }
}

}  // namespace

int persist_grid(int hd, int n_cu) {
  int occ = 0;
  hipError_t e = hd == 128 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kp_layer<128>, PERSIST_NT, 0)
                           : hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kp_layer<64>, PERSIST_NT, 0);
  if (e != hipSuccess || occ < 1) return 0;
  return std::min(occ, 2) * n_cu;
}

bool persist_fits(const PersistArgs &a, int grid) {
  auto tiles = [](int64_t rows, int64_t nb) { int G, R; rp_shape(nb, G, R); return (rows + NW * R - 1) / (NW * R); };
  auto bpg = [](int64_t nb) { int G, R; rp_shape(nb, G, R); return (nb + G - 1) / G; };
  if (grid < 1 || (a.hd != 64 && a.hd != 128) || a.dim % 256 || a.q_dim % 256 || a.n_ff % 256) return false;
  if (a.n_heads % a.n_kv || a.n_heads / a.n_kv > 8 || a.n_used > 8) return false;
  const int64_t nb = a.dim / 256, nbo = a.q_dim / 256, nbf = a.n_ff / 256;
  if (bpg(nb) > QKV_BPG || tiles(a.q_dim, nb) + 2 * tiles(a.kv_dim, nb) > (int64_t)QKV_NT * grid) return false;
  if (bpg(nbo) > WO_BPG || tiles(a.dim, nbo) > (int64_t)WO_NT * grid) return false;
  if ((nb + 3) / 4 > GU_BPG) return false;
  if ((int64_t)std::max(a.n_used, 1) * ((a.n_ff + NW - 1) / NW) > (int64_t)GU_NI * grid) return false;
  if (a.n_expert > 0 && (a.n_expert > grid || a.n_expert > 256 || nbf > DN_NB || a.dim > NW * grid)) return false;
  if (bpg(nbf) > WO_BPG || tiles(a.dim, nbf) > (int64_t)WO_NT * grid) return false;  // a dense down projection
  return true;
}

hipError_t launch_persist_layer(const PersistArgs &a, const PLayer &ly, int layer, unsigned epoch0, int grid, hipStream_t s) {
  int li = layer;
  unsigned e0 = epoch0;
  void *args[] = {const_cast<PersistArgs *>(&a), const_cast<PLayer *>(&ly), &li, &e0};
  if (a.hd == 128) return hipLaunchCooperativeKernel((const void *)kp_layer<128>, dim3(grid), dim3(PERSIST_NT), args, 0, s);
  if (a.hd == 64) return hipLaunchCooperativeKernel((const void *)kp_layer<64>, dim3(grid), dim3(PERSIST_NT), args, 0, s);
  return hipErrorInvalidValue;
}

}  // namespace spx
