// Per-layer kernels of the decode / verify forward pass on gfx950 (smollm_chat.rs:3142-3558).
// Every kernel takes m <= 16 token rows; positions come from the device-side step record so
// a captured HIP graph replays at any position.
#include "common.h"
#include "layer_kernels.h"

namespace spx {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Block-wide sum of one value per thread (256 threads), identical result in every thread.
__device__ float block_sum256(float v, float *red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// Quantizes n (multiple of 256) values held in LDS to Q8_K (quantize_avx2,
// quant_q8k.rs:84-121); 256 threads, one wave per 256-block.
__device__ void q8k_from_lds(const float *xs, int n, float *d, int8_t *qs, int16_t *bs) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int b = wv; b < n / 256; b += 4) {
    const float4 xv = reinterpret_cast<const float4 *>(xs + b * 256)[lane];
    float am = fmaxf(fmaxf(fabsf(xv.x), fabsf(xv.y)), fmaxf(fabsf(xv.z), fabsf(xv.w)));
    am = wave_max(am);
    float dv = 0.0f;
    int q[4] = {0, 0, 0, 0};
    if (am > 0.0f && !isinf(am)) {
      const float iscale = __fdiv_rn(127.0f, am);
      dv = __fdiv_rn(am, 127.0f);
      const float xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int j = 0; j < 4; j++) q[j] = (int)fminf(fmaxf(rintf(__fmul_rn(xx[j], iscale)), -128.0f), 127.0f);
    }
    reinterpret_cast<uint32_t *>(qs + b * 256)[lane] = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                                                       ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    const int s = quad_sum(q[0] + q[1] + q[2] + q[3]);
    if ((lane & 3) == 0) bs[b * 16 + (lane >> 2)] = (int16_t)s;
    if (lane == 0) d[b] = dv;
  }
}

// ------------------------------------------------------------------ embedding
// dequant_row (quant.rs:1548-1660) of token rows, times embedding_scale (:3381-3388).
__global__ __launch_bounds__(256) void k_embed(TensorView e, const StepRec *st, float *x, int64_t ld_x, float escale) {
  const int b = blockIdx.x;
  if (b >= st->m) return;
  const int64_t tok = st->ids[b];
  const int64_t cols = e.cols;
  float *out = x + b * ld_x;
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
    } else if (e.dtype == T_Q4K) {
      const int64_t g = tok * e.nb + j / 256;
      const int k = (int)(j % 256), c = k / 64, l = k % 32, hi = (k % 64) >= 32;
      const uint8_t *hd = e.pl.p1 + g * 16;
      const float dd = h2f(hd[0] | (hd[1] << 8)), dm = h2f(hd[2] | (hd[3] << 8));
      const uint8_t *s = hd + 4;
      const int jj = 2 * c + hi;
      int sc, mn;
      if (jj < 4) { sc = s[jj] & 63; mn = s[jj + 4] & 63; }
      else { sc = (s[jj + 4] & 0xF) | ((s[jj - 4] >> 6) << 4); mn = (s[jj + 4] >> 4) | ((s[jj] >> 6) << 4); }
      const int byte = e.pl.p0[g * 128 + c * 32 + l];
      const int q = hi ? (byte >> 4) : (byte & 0xF);
      v = dd * (float)sc * (float)q - dm * (float)mn;
    } else if (e.dtype == T_Q6K) {
      const int64_t g = tok * e.nb + j / 256;
      const int k = (int)(j % 256), h = k / 128, r = k % 128, mq = r / 32, l = r % 32;
      const uint8_t *ql = e.pl.p0 + g * 128 + h * 64, *qh = e.pl.p1 + g * 64 + h * 32;
      const int8_t *sc = reinterpret_cast<const int8_t *>(e.pl.p2 + g * 16);
      const float dd = h2f(*reinterpret_cast<const uint16_t *>(e.pl.p3 + g * 2));
      int q;
      if (mq == 0) q = (ql[l] & 0xF) | ((qh[l] & 3) << 4);
      else if (mq == 1) q = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4);
      else if (mq == 2) q = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
      else q = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
      v = dd * (float)sc[h * 8 + l / 16 + 2 * mq] * (float)(q - 32);
    }
    if (escale != 1.0f) v *= escale;
    out[j] = v;
  }
}

// ------------------------------------------------------------------ residual + RMSNorm + Q8_K
// x += rscale * add (when add != null; :3518-3520, :3538-3540), then out = x * inv * w with
// inv = 1/sqrt(sum(x^2)/n + eps) (rmsnorm :569-575), optionally quantized to Q8_K.
__global__ __launch_bounds__(256) void k_res_norm(float *x, int64_t ld_x, const float *add, int64_t ld_add, float rscale,
                                                  const float *w, int n, float eps, float *out, int64_t ld_out,
                                                  float *qd, int8_t *qq, int16_t *qb, const StepRec *st) {
  __shared__ __align__(16) float xs[4096];
  __shared__ float red[4];
  const int b = blockIdx.x;
  if (b >= st->m) return;
  float *xr = x + b * ld_x;
  float ss = 0.0f;
  for (int j = threadIdx.x; j < n; j += 256) {
    float v = xr[j];
    if (add) { v = v + rscale * add[b * ld_add + j]; xr[j] = v; }
    xs[j] = v;
    ss = fmaf(v, v, ss);
  }
  ss = block_sum256(ss, red);
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)n) + eps));
  for (int j = threadIdx.x; j < n; j += 256) {
    const float v = xs[j] * inv * w[j];
    xs[j] = v;
    if (out) out[b * ld_out + j] = v;
  }
  if (qq) {
    __syncthreads();
    const int nb = n / 256;
    q8k_from_lds(xs, n, qd + b * nb, qq + (int64_t)b * n, qb + b * nb * 16);
  }
}

// ------------------------------------------------------------------ q/k post-processing
// bias, per-head q/k RMSNorm (Qwen3), RoPE from the (cos, sin) table, K/V -> f16 cache
// (:3226-3248, :3432-3448). One wavefront per head; grid (heads_total, m).
__global__ __launch_bounds__(64) void k_qk_rope_kv(const QKArgs a, const StepRec *st) {
  const int b = blockIdx.y;
  if (b >= st->m) return;
  const int pos = st->start + b;
  const int hidx = blockIdx.x, lane = threadIdx.x;
  const int hd = a.head_dim, half = hd / 2;
  const bool is_q = hidx < a.n_heads;
  const bool is_k = !is_q && hidx < a.n_heads + a.n_kv;
  float *v;
  const float *bias, *nw;
  if (is_q) { v = a.q + b * a.ld_q + hidx * hd; bias = a.q_bias ? a.q_bias + hidx * hd : nullptr; nw = a.q_norm; }
  else if (is_k) { const int kh = hidx - a.n_heads; v = a.k + b * a.ld_kv + kh * hd; bias = a.k_bias ? a.k_bias + kh * hd : nullptr; nw = a.k_norm; }
  else { const int kh = hidx - a.n_heads - a.n_kv; v = a.v + b * a.ld_kv + kh * hd; bias = a.v_bias ? a.v_bias + kh * hd : nullptr; nw = nullptr; }
  // each lane holds elements lane, lane+64 (head_dim <= 128)
  float e0 = lane < hd ? v[lane] : 0.0f, e1 = lane + 64 < hd ? v[lane + 64] : 0.0f;
  if (bias) { if (lane < hd) e0 += bias[lane]; if (lane + 64 < hd) e1 += bias[lane + 64]; }
  if (nw) {
    const float ss = wave_sum(fmaf(e0, e0, e1 * e1));
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(ss, (float)hd) + a.eps));
    if (lane < hd) e0 = e0 * inv * nw[lane];
    if (lane + 64 < hd) e1 = e1 * inv * nw[lane + 64];
  }
  __shared__ float sh[128];
  if (lane < hd) sh[lane] = e0;
  if (lane + 64 < hd) sh[lane + 64] = e1;
  __syncthreads();
  if (is_q || is_k) {  // Rope::rotate (:1404-1419); head_dim <= 128, so one pair per lane
    const float2 *cs = a.rope + (int64_t)pos * half;
    const bool act = lane < half;
    const int ia = a.neox ? lane : 2 * lane, ib = a.neox ? lane + half : 2 * lane + 1;
    float r0 = 0.0f, r1 = 0.0f;
    if (act) {
      const float x0 = sh[ia], x1 = sh[ib], c = cs[lane].x, s = cs[lane].y;
      r0 = x0 * c - x1 * s;
      r1 = x0 * s + x1 * c;
    }
    __syncthreads();
    if (act) { sh[ia] = r0; sh[ib] = r1; }
    __syncthreads();
  }
  if (is_q) {
    for (int i = lane; i < hd; i += 64) v[i] = sh[i];
  } else {
    const int kh = is_k ? hidx - a.n_heads : hidx - a.n_heads - a.n_kv;
    __half *cache = (is_k ? a.k_cache : a.v_cache) + ((int64_t)a.layer * a.max_seq + pos) * a.kv_dim + kh * hd;
    for (int i = lane; i < hd; i += 64) cache[i] = __float2half_rn(sh[i]);
  }
}

// ------------------------------------------------------------------ attention
// Causal GQA attention over the f16 KV cache (:3250-3319, :3456-3495), split over position
// chunks (flash-decoding): each workgroup takes one kv head and ATT_CHUNK positions for all
// m rows and the kv head's query heads, writes (max, sum, unnormalised out) per query, and
// k_attn_merge combines the chunks. Row b attends to positions <= start + b.
__global__ __launch_bounds__(256) void k_attn_chunk(const AttnArgs a, const StepRec *st) {
  const int kvh = blockIdx.y, chunk = blockIdx.x;
  const int m = st->m, start = st->start;
  const int t0 = chunk * ATT_CHUNK;
  const int last = start + m - 1;  // highest position any row sees
  if (t0 > last) return;
  const int hd = a.head_dim, g = a.n_heads / a.n_kv, nq = m * g;
  const int tn = min(ATT_CHUNK, last + 1 - t0);
  const int kst = hd + 2;                       // padded K row (halves): 65-dword stride, conflict-free
  __shared__ __align__(16) __half ks[ATT_CHUNK * (128 + 2)];
  __shared__ __align__(16) __half vs[ATT_CHUNK * 128];
  __shared__ __align__(16) float qs[ATT_QG * 128];
  __shared__ float ps[ATT_QG * ATT_CHUNK];
  const int64_t base = (int64_t)a.layer * a.max_seq * a.kv_dim + kvh * hd;
  const int n8 = hd / 8;                        // 16-byte pieces per K/V row
#pragma unroll 4
  for (int i = threadIdx.x; i < ATT_CHUNK * n8; i += 256) {
    const int t = i / n8, j = i % n8;
    uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
    if (t < tn) {
      const int64_t off = base + (int64_t)(t0 + t) * a.kv_dim + 8 * j;
      kv = *reinterpret_cast<const uint4 *>(a.k_cache + off);
      vv = *reinterpret_cast<const uint4 *>(a.v_cache + off);
    }
    uint32_t *kd = reinterpret_cast<uint32_t *>(ks + t * kst + 8 * j);
    kd[0] = kv.x; kd[1] = kv.y; kd[2] = kv.z; kd[3] = kv.w;
    *reinterpret_cast<uint4 *>(vs + t * hd + 8 * j) = vv;
  }
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int q0 = 0; q0 < nq; q0 += ATT_QG) {
    const int nqg = min(ATT_QG, nq - q0);
    __syncthreads();
    for (int i = threadIdx.x; i < nqg * hd; i += 256) {
      const int qi = q0 + i / hd, dd = i % hd, b = qi / g, h = kvh * g + qi % g;
      qs[i] = a.q[b * a.ld_q + h * hd + dd];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < ATT_QG * ATT_CHUNK; i += 256) {  // scores = (q . k) * scale
      const int ql = i / ATT_CHUNK, t = i % ATT_CHUNK, b = (q0 + ql) / g;
      float s = -INFINITY;
      if (ql < nqg && t < tn && t0 + t <= start + b) {
        const __half *kr = ks + t * kst;
        const float *qr = qs + ql * hd;
        float acc = 0.0f;
        for (int dd = 0; dd < hd; dd += 2) {
          const float2 kf = __half22float2(*reinterpret_cast<const __half2 *>(kr + dd));
          acc = fmaf(kf.x, qr[dd], acc);
          acc = fmaf(kf.y, qr[dd + 1], acc);
        }
        s = acc * a.scale;
      }
      ps[i] = s;
    }
    __syncthreads();
    for (int ql = wv; ql < nqg; ql += 4) {  // chunk max, exp, sum
      const float s = ps[ql * ATT_CHUNK + lane];
      const float mx = wave_max(s);
      const float p = s == -INFINITY ? 0.0f : expf(s - mx);
      ps[ql * ATT_CHUNK + lane] = p;
      const float l = wave_sum(p);
      if (lane == 0) {
        const int64_t o = ((int64_t)(kvh * (16 * g)) + q0 + ql) * a.max_chunks + chunk;
        a.part_m[o] = mx;
        a.part_l[o] = l;
      }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nqg * hd; i += 256) {  // unnormalised p . V
      const int ql = i / hd, dd = i % hd;
      float acc = 0.0f;
      for (int t = 0; t < tn; t++) acc = fmaf(ps[ql * ATT_CHUNK + t], __half2float(vs[t * hd + dd]), acc);
      a.part_o[(((int64_t)(kvh * (16 * g)) + q0 + ql) * a.max_chunks + chunk) * hd + dd] = acc;
    }
  }
}

__global__ __launch_bounds__(128) void k_attn_merge(const AttnArgs a, const StepRec *st) {
  const int qi = blockIdx.x, kvh = blockIdx.y;
  const int g = a.n_heads / a.n_kv, m = st->m;
  if (qi >= m * g) return;
  const int b = qi / g, h = kvh * g + qi % g, hd = a.head_dim;
  const int nch = (st->start + b) / ATT_CHUNK + 1;  // chunks row b sees
  const int64_t row = (int64_t)(kvh * (16 * g)) + qi;
  __shared__ float wsm[MAX_CHUNKS];
  __shared__ float red[2];
  // chunk weights exp(m_c - max) and the normaliser, computed once
  float mx = -INFINITY;
  for (int c = threadIdx.x; c < nch; c += 128) mx = fmaxf(mx, a.part_m[row * a.max_chunks + c]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(red[0], red[1]);
  for (int c = threadIdx.x; c < nch; c += 128) {
    const float mc = a.part_m[row * a.max_chunks + c];
    wsm[c] = mc == -INFINITY ? 0.0f : expf(mc - mx);
  }
  __syncthreads();
  float l = 0.0f;
  for (int c = 0; c < nch; c++) l = fmaf(a.part_l[row * a.max_chunks + c], wsm[c], l);
  const float invl = __fdiv_rn(1.0f, fmaxf(l, 1e-9f));
  for (int dd = threadIdx.x; dd < hd; dd += 128) {
    float acc = 0.0f;
    for (int c = 0; c < nch; c++) acc = fmaf(a.part_o[(row * a.max_chunks + c) * hd + dd], wsm[c], acc);
    a.out[b * a.ld_out + h * hd + dd] = acc * invl;
  }
}

// ------------------------------------------------------------------ MoE routing
// Router softmax, top-n_used by probability (ties: lower expert index), pruning and weight
// normalisation (:1199-1239, :959-997), then the grouped job lists over the union of chosen
// experts (:982-986, :648-700). One workgroup.
__global__ __launch_bounds__(256) void k_moe_route(const RouteArgs a, const StepRec *st) {
  __shared__ float probs[16][256];
  __shared__ int chosen[16][32];
  __shared__ int nkeep[16];
  __shared__ int jcount[256], jbase[4];
  const int m = st->m, ne = a.n_expert, nu = a.n_used;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int b = wv; b < m; b += 4) {
    const float *lg = a.logits + b * a.ld_logits;
    float mx = -INFINITY;
    for (int e = lane; e < ne; e += 64) mx = fmaxf(mx, lg[e]);
    mx = wave_max(mx);
    float sum = 0.0f;
    for (int e = lane; e < ne; e += 64) { const float p = expf(lg[e] - mx); probs[b][e] = p; sum += p; }
    sum = wave_sum(sum);
    for (int e = lane; e < ne; e += 64) probs[b][e] = probs[b][e] / sum;
    // top-n_used by probability, ties to the lower expert index
    unsigned long long taken[4] = {0, 0, 0, 0};
    for (int i = 0; i < nu; i++) {
      float bp = -1.0f;
      int be = 1 << 30;
      for (int e = lane; e < ne; e += 64) {
        if ((taken[e >> 6] >> (e & 63)) & 1ull) continue;
        const float p = probs[b][e];
        if (p > bp || (p == bp && e < be)) { bp = p; be = e; }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const float p2 = __shfl_xor(bp, o);
        const int e2 = __shfl_xor(be, o);
        if (p2 > bp || (p2 == bp && e2 < be)) { bp = p2; be = e2; }
      }
      taken[be >> 6] |= 1ull << (be & 63);
      if (lane == 0) chosen[b][i] = be;
    }
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {  // pruning and weights, in chosen order
      int keep = nu;
      if (a.moe_prune > 0.0f && nu > 2) {
        const int min_keep = max(2, nu / 2);
        if (a.moe_prune >= 1.0f) keep = min(max((int)a.moe_prune, min_keep), nu);
        else {
          float top = 0.0f;
          for (int i = 0; i < nu; i++) top += probs[b][chosen[b][i]];
          const float target = top * (1.0f - a.moe_prune);
          float cum = 0.0f;
          int k = 0;
          while (k < nu && (k < min_keep || cum < target)) { cum += probs[b][chosen[b][k]]; k++; }
          keep = k;
        }
      }
      float wsum = 0.0f;
      for (int i = 0; i < keep; i++) wsum += probs[b][chosen[b][i]];
      for (int i = 0; i < keep; i++) {
        a.chosen[b * 32 + i] = chosen[b][i];
        a.weights[b * 32 + i] = a.norm ? probs[b][chosen[b][i]] / wsum : probs[b][chosen[b][i]];
      }
      nkeep[b] = keep;
      a.nkeep[b] = keep;
    }
  }
  __syncthreads();
  // one job per selected expert, in expert order; users in (row, slot) order
  const int e = threadIdx.x;
  int cnt = 0;
  if (e < ne)
    for (int b = 0; b < m; b++)
      for (int i = 0; i < nkeep[b]; i++) cnt += chosen[b][i] == e;
  const unsigned long long bal = __ballot(cnt > 0);
  const int before = __popcll(bal & ((1ull << lane) - 1ull));
  if (lane == 0) jbase[wv] = __popcll(bal);
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wv; w++) off += jbase[w];
  if (cnt > 0) {
    const int j = off + before;
    int k = 0;
    for (int b = 0; b < m; b++)
      for (int i = 0; i < nkeep[b]; i++)
        if (chosen[b][i] == e) {
          a.jobs_gu[j].vec[k] = b;
          a.jobs_gu[j].out[k] = b * nu + i;
          a.jobs_dn[j].vec[k] = b * nu + i;
          a.jobs_dn[j].out[k] = b * nu + i;
          k++;
        }
    a.jobs_gu[j].expert = e;
    a.jobs_dn[j].expert = e;
    a.jobs_gu[j].nvec = k;
    a.jobs_dn[j].nvec = k;
    if (a.expert_count) a.expert_count[e] += 1;
  }
  if (threadIdx.x == 0) *a.njobs = jbase[0] + jbase[1] + jbase[2] + jbase[3];
  (void)jcount;
}

// ------------------------------------------------------------------ SwiGLU
// h = silu(g) * u (silu :586-588), for rows listed in the job table (or the first m rows), then
// optionally Q8_K-quantized for an integer down projection. One workgroup per vector.
__global__ __launch_bounds__(256) void k_swiglu(const SwigluArgs a, const StepRec *st) {
  __shared__ __align__(16) float hs[4096];
  int vrow;
  if (a.jobs) {
    // vector index = blockIdx.x among all (job, user) pairs
    int idx = blockIdx.x, j = 0;
    const int nj = *a.njobs;
    while (j < nj && idx >= a.jobs[j].nvec) { idx -= a.jobs[j].nvec; j++; }
    if (j >= nj) return;
    vrow = a.jobs[j].out[idx];
  } else {
    vrow = blockIdx.x;
    if (vrow >= st->m) return;
  }
  const int n = a.n;
  float *g = a.g + vrow * a.ld;
  const float *u = a.u + vrow * a.ld;
  for (int j = threadIdx.x; j < n; j += 256) {
    const float x = g[j];
    const float h = x / (1.0f + expf(-x)) * u[j];
    hs[j] = h;
    g[j] = h;
  }
  if (a.qq) {
    __syncthreads();
    const int nb = n / 256;
    q8k_from_lds(hs, n, a.qd + vrow * nb, a.qq + (int64_t)vrow * n, a.qb + vrow * nb * 16);
  }
}

// ------------------------------------------------------------------ MoE combine
// out[b] = sum over chosen slots, in chosen order, of w * y (ffns_fused :432-437,
// moe_forward_batch :1133-1140), then x[b] += rscale * out[b].
__global__ __launch_bounds__(256) void k_moe_combine(const CombineArgs a, const StepRec *st) {
  const int b = blockIdx.y;
  if (b >= st->m) return;
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= a.dim) return;
  const int nk = a.nkeep[b];
  float acc = 0.0f;
  for (int i = 0; i < nk; i++) acc = acc + a.weights[b * 32 + i] * a.y[(int64_t)(b * a.n_used + i) * a.ld_y + r];
  if (a.out) a.out[b * a.ld_out + r] = acc;
}

// ------------------------------------------------------------------ greedy argmax
// logits / logit_scale, then the last maximum under f32 total order (max_by(total_cmp),
// :3661-3671). Ties go to the higher index, as Iterator::max_by returns the last maximum.
__device__ __forceinline__ int total_key(float f) {
  const int i = __float_as_int(f);
  return i ^ (int)(((unsigned)(i >> 31)) >> 1);
}
__global__ __launch_bounds__(1024) void k_argmax(const float *logits, int64_t ld, int n, float lscale, int *out, const StepRec *st) {
  const int b = blockIdx.x;
  if (b >= st->m) return;
  const float *lg = logits + b * ld;
  int bk = INT_MIN, bi = -1;
  for (int i = threadIdx.x; i < n; i += 1024) {
    const float v = lscale != 1.0f ? lg[i] / lscale : lg[i];
    const int k = total_key(v);
    if (bi < 0 || k > bk || (k == bk && i > bi)) { bk = k; bi = i; }
  }
  __shared__ int sk[1024], si[1024];
  sk[threadIdx.x] = bk;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int s = 512; s >= 1; s >>= 1) {
    if ((int)threadIdx.x < s) {
      const int k2 = sk[threadIdx.x + s], i2 = si[threadIdx.x + s];
      const int k1 = sk[threadIdx.x], i1 = si[threadIdx.x];
      if (i2 >= 0 && (i1 < 0 || k2 > k1 || (k2 == k1 && i2 > i1))) { sk[threadIdx.x] = k2; si[threadIdx.x] = i2; }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[b] = si[0];
}

// ------------------------------------------------------------------ launchers
#define LAUNCH(...) do { hipLaunchKernelGGL(__VA_ARGS__); return hipGetLastError(); } while (0)

hipError_t launch_embed(const TensorView &e, const StepRec *st, float *x, int64_t ld_x, float escale, int m, hipStream_t s) {
  LAUNCH(k_embed, dim3(m), dim3(256), 0, s, e, st, x, ld_x, escale);
}
hipError_t launch_res_norm(float *x, int64_t ld_x, const float *add, int64_t ld_add, float rscale, const float *w, int n, float eps,
                           float *out, int64_t ld_out, float *qd, int8_t *qq, int16_t *qb, const StepRec *st, int m, hipStream_t s) {
  LAUNCH(k_res_norm, dim3(m), dim3(256), 0, s, x, ld_x, add, ld_add, rscale, w, n, eps, out, ld_out, qd, qq, qb, st);
}
hipError_t launch_qk_rope_kv(const QKArgs &a, const StepRec *st, int m, hipStream_t s) {
  LAUNCH(k_qk_rope_kv, dim3(a.n_heads + 2 * a.n_kv, m), dim3(64), 0, s, a, st);
}
hipError_t launch_attention(const AttnArgs &a, const StepRec *st, int m, hipStream_t s) {
  const int g = a.n_heads / a.n_kv, nq = m * g;
  hipLaunchKernelGGL(k_attn_chunk, dim3(a.max_chunks, a.n_kv), dim3(256), 0, s, a, st);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  LAUNCH(k_attn_merge, dim3(nq, a.n_kv), dim3(128), 0, s, a, st);
}
hipError_t launch_moe_route(const RouteArgs &a, const StepRec *st, hipStream_t s) {
  LAUNCH(k_moe_route, dim3(1), dim3(256), 0, s, a, st);
}
hipError_t launch_swiglu(const SwigluArgs &a, const StepRec *st, int nvec, hipStream_t s) {
  LAUNCH(k_swiglu, dim3(nvec), dim3(256), 0, s, a, st);
}
hipError_t launch_moe_combine(const CombineArgs &a, const StepRec *st, int m, hipStream_t s) {
  LAUNCH(k_moe_combine, dim3((a.dim + 255) / 256, m), dim3(256), 0, s, a, st);
}
hipError_t launch_argmax(const float *logits, int64_t ld, int n, float lscale, int *out, const StepRec *st, int m, hipStream_t s) {
  LAUNCH(k_argmax, dim3(m), dim3(1024), 0, s, logits, ld, n, lscale, out, st);
}

}  // namespace spx
