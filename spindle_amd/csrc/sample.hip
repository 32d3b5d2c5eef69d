// Token sampling over device logits (sample_from_logits, smollm_chat.rs:3624-3726).
//
// k_sample, one workgroup of 1024 threads per logits row:
//   1. the row's penalty window and masked ids as LDS bitmaps (one bit per token)
//   2. one pass over the logits: v / logit_scale, the repeat penalty on window tokens
//      (v > 0 ? v / p : v * p, each token once however often it recurs), -inf on masked ids;
//      the result goes to a scratch row; the greedy key (total order, last index on ties), the
//      count of finite values and the histogram of the top key byte come out of the same pass
//   3. with 0 < top_k <= SAMPLE_KMAX and temperature > 0: a most-significant-digit radix
//      select of the top_k finite values on the 64-bit key (total-order bits of the logit,
//      then the complemented token id, so equal logits rank by ascending id), 8 bits a pass
//      over the scratch row, stopping at the first digit whose bin holds exactly the rest
//   4. the selected keys gathered into LDS and bitonic-sorted, largest first: candidate ids
//      and logits in the reference's order
// The host tail (Sampler::pick) then does the softmax over those k logits with the C
// library's expf, min-p, top-p and the SplitMix64 draw, as the reference does on its CPU.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <new>

#include "dev.h"
#include "internal.h"
#include "sample.h"

namespace spx {

// f32::total_cmp as an unsigned key: -NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN
__device__ __host__ __forceinline__ uint32_t total_u32(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct SampleArgs {
  const float *x;
  int64_t ld;
  int V;
  float lscale, penalty;
  const int32_t *win;   // penalty window of row r: win[0 .. n_win + r)
  int n_win;
  const int32_t *stop;  // stop ids, masked on rows whose bit is set in fstop
  int n_stop;
  uint32_t fstop;
  int think;            // masked on every row when fthink (-1: none)
  int fthink;
  int sel_k;            // device selection of this many (0: none)
  float *scratch;       // [m][V]
  int32_t *cidx;        // [m][SAMPLE_KMAX]
  float *cval;
  int32_t *meta;        // [m][4]: finite count, greedy id, selected count
};

__global__ __launch_bounds__(1024) void k_sample(const SampleArgs a) {
  extern __shared__ uint32_t bm[];  // [2][nw] penalty and mask bitmaps
  __shared__ uint32_t hist[256];
  __shared__ unsigned long long skey[SAMPLE_KMAX];
  __shared__ unsigned long long s_g[16];
  __shared__ int s_n[16];
  __shared__ unsigned long long s_prefix;
  __shared__ int s_need, s_done, s_cnt;
  const int r = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int V = a.V, nw = (V + 31) >> 5;
  uint32_t *pen = bm, *msk = bm + nw;
  for (int i = t; i < 2 * nw; i += 1024) bm[i] = 0;
  if (t < 256) hist[t] = 0;
  __syncthreads();
  if (a.penalty != 1.0f)
    for (int i = t; i < a.n_win + r; i += 1024) {
      const int id = a.win[i];
      if (id >= 0 && id < V) atomicOr(&pen[id >> 5], 1u << (id & 31));
    }
  if ((a.fstop >> r) & 1u)
    for (int i = t; i < a.n_stop; i += 1024) {
      const int id = a.stop[i];
      if (id >= 0 && id < V) atomicOr(&msk[id >> 5], 1u << (id & 31));
    }
  if (a.fthink && t == 0 && a.think >= 0 && a.think < V) atomicOr(&msk[a.think >> 5], 1u << (a.think & 31));
  __syncthreads();

  const float *x = a.x + (int64_t)r * a.ld;
  float *sc = a.scratch + (int64_t)r * V;
  unsigned long long g = 0;
  int nf = 0;
  for (int i = t; i < V; i += 1024) {
    float v = x[i];
    if (a.lscale != 1.0f) v = v / a.lscale;
    const uint32_t bit = 1u << (i & 31);
    if (pen[i >> 5] & bit) v = v > 0.0f ? v / a.penalty : v * a.penalty;
    if (msk[i >> 5] & bit) v = -INFINITY;
    sc[i] = v;
    const uint32_t k = total_u32(v);
    const unsigned long long c = ((unsigned long long)k << 32) | (uint32_t)i;
    g = c > g ? c : g;
    if (isfinite(v)) {
      nf++;
      if (a.sel_k) atomicAdd(&hist[k >> 24], 1u);
    }
  }
  g = wave_max_u64(g);
  for (int o = 32; o >= 1; o >>= 1) nf += __shfl_xor(nf, o);
  if (lane == 0) { s_g[wave] = g; s_n[wave] = nf; }
  __syncthreads();
  g = s_g[0];
  nf = s_n[0];
  for (int w = 1; w < 16; w++) { g = s_g[w] > g ? s_g[w] : g; nf += s_n[w]; }
  if (t == 0) {
    a.meta[r * 4 + 0] = nf;
    a.meta[r * 4 + 1] = (int)(uint32_t)g;
    a.meta[r * 4 + 2] = 0;
  }
  const int k = min(a.sel_k, nf);
  if (k == 0) return;

  // radix select on key = total << 32 | ~id, most significant byte first
  int need = k, shift = 56;
  unsigned long long prefix = 0;
  for (;;) {
    __syncthreads();  // the digit's histogram is complete
    if (wave == 0) {
      // lane l owns bins 255 - 4l .. 252 - 4l (descending); exclusive scan of the lane sums
      uint32_t hv[4], s = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) { hv[j] = hist[255 - 4 * lane - j]; s += hv[j]; }
      uint32_t inc = s;
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = __shfl_up(inc, o);
        if (lane >= o) inc += u;
      }
      uint32_t acc = inc - s;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if (acc < (uint32_t)need && acc + hv[j] >= (uint32_t)need) {
          const int b = 255 - 4 * lane - j;
          s_need = need - (int)acc;
          s_prefix = prefix | ((unsigned long long)b << shift);
          s_done = hv[j] == (uint32_t)(need - (int)acc);
        }
        acc += hv[j];
      }
    }
    __syncthreads();
    need = s_need;
    prefix = s_prefix;
    if (s_done || shift == 0) break;
    if (t < 256) hist[t] = 0;
    __syncthreads();
    const unsigned long long fixed = ~0ull << shift;
    shift -= 8;
    for (int i = t; i < V; i += 1024) {
      const float v = sc[i];
      if (!isfinite(v)) continue;
      const unsigned long long c = ((unsigned long long)total_u32(v) << 32) | (uint32_t)~(uint32_t)i;
      if ((c & fixed) == prefix) atomicAdd(&hist[(c >> shift) & 255], 1u);
    }
  }
  // the selected keys are exactly those >= prefix (its bits below the last digit are zero)
  if (t == 0) s_cnt = 0;
  __syncthreads();
  for (int i = t; i < V; i += 1024) {
    const float v = sc[i];
    if (!isfinite(v)) continue;
    const unsigned long long c = ((unsigned long long)total_u32(v) << 32) | (uint32_t)~(uint32_t)i;
    if (c >= prefix) {
      const int slot = atomicAdd(&s_cnt, 1);
      if (slot < SAMPLE_KMAX) skey[slot] = c;
    }
  }
  __syncthreads();
  const int cnt = min(s_cnt, SAMPLE_KMAX);
  int P = 1;
  while (P < cnt) P <<= 1;
  if (t >= cnt && t < P) skey[t] = 0;  // below every finite key
  __syncthreads();
  for (int size = 2; size <= P; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (t < P) {
        const int j = t ^ stride;
        if (j > t) {
          const unsigned long long u = skey[t], w = skey[j];
          const bool desc = (t & size) == 0;
          if (desc ? u < w : u > w) { skey[t] = w; skey[j] = u; }
        }
      }
      __syncthreads();
    }
  if (t < cnt) {
    const int id = (int)~(uint32_t)skey[t];
    a.cidx[r * SAMPLE_KMAX + t] = id;
    a.cval[r * SAMPLE_KMAX + t] = sc[id];
  }
  if (t == 0) a.meta[r * 4 + 2] = cnt;
}

// ------------------------------------------------------------------ host side
Sampler::~Sampler() {
  if (d_scratch) {
    (void)hipSetDevice(device);
    (void)hipStreamSynchronize(stream);
  }
  (void)hipFree(d_scratch);
  (void)hipFree(d_cidx);
  (void)hipFree(d_cval);
  (void)hipFree(d_meta);
  (void)hipFree(d_ids);
  (void)hipHostFree(h_cidx);
  (void)hipHostFree(h_cval);
  (void)hipHostFree(h_meta);
  (void)hipHostFree(h_ids);
  (void)hipHostFree(h_row);
}

int Sampler::init(const spx_sampler_params *pp, int V, int dev, hipStream_t s) {
  if (!pp) return fail("sampler: null parameters");
  if (V < 1 || V > SAMPLE_VMAX) return fail("sampler: vocabulary must be in 1..524288");
  if (pp->n_stop < 0 || (pp->n_stop > 0 && !pp->stop_ids)) return fail("sampler: bad stop id list");
  if (!(pp->top_p == pp->top_p) || !(pp->min_p == pp->min_p) || !(pp->temperature == pp->temperature))
    return fail("sampler: NaN parameter");
  if (pp->top_k < 0) return fail("sampler: top_k must be >= 0");
  p = *pp;
  stop.assign(pp->stop_ids, pp->stop_ids + pp->n_stop);
  p.stop_ids = nullptr;
  rng = pp->seed;
  vocab = V;
  device = dev;
  stream = s;
  SPX_HIP(hipSetDevice(dev));
  SPX_HIP(hipMalloc(&d_scratch, sizeof(float) * (size_t)SAMPLE_MMAX * V));
  SPX_HIP(hipMalloc(&d_cidx, sizeof(int32_t) * SAMPLE_MMAX * SAMPLE_KMAX));
  SPX_HIP(hipMalloc(&d_cval, sizeof(float) * SAMPLE_MMAX * SAMPLE_KMAX));
  SPX_HIP(hipMalloc(&d_meta, sizeof(int32_t) * SAMPLE_MMAX * 4));
  SPX_HIP(hipHostMalloc(&h_cidx, sizeof(int32_t) * SAMPLE_MMAX * SAMPLE_KMAX, hipHostMallocDefault));
  SPX_HIP(hipHostMalloc(&h_cval, sizeof(float) * SAMPLE_MMAX * SAMPLE_KMAX, hipHostMallocDefault));
  SPX_HIP(hipHostMalloc(&h_meta, sizeof(int32_t) * SAMPLE_MMAX * 4, hipHostMallocDefault));
  return 0;
}

bool Sampler::greedy_plain() const { return p.temperature <= 0.0f && p.repeat_penalty == 1.0f && stop.empty() && p.think_open < 0; }

uint64_t Sampler::next_u64() {  // SplitMix64::next_u64 (:1560-1566)
  uint64_t z = (rng += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

float Sampler::next_f32() { return (float)(next_u64() >> 40) / (float)(1u << 24); }  // :1569-1571

static bool device_select(const spx_sampler_params &p) { return p.temperature > 0.0f && p.top_k > 0 && p.top_k <= SAMPLE_KMAX; }

int Sampler::prepare(const float *logits, int64_t ld, int m, float lscale, const int32_t *window, int n_window,
                     uint32_t fstop, bool fthink) {
  if (!logits || m < 1 || m > SAMPLE_MMAX || ld < vocab) return fail("sampler: bad logits rows");
  if (n_window < 0 || (n_window + m - 1 > 0 && !window)) return fail("sampler: bad penalty window");
  const int n_ids = n_window + m - 1 + (int)stop.size();
  SPX_HIP(hipSetDevice(device));
  if (n_ids > ids_cap) {
    const int cap = std::max(n_ids, 4096);
    SPX_HIP(hipStreamSynchronize(stream));
    (void)hipFree(d_ids);
    (void)hipHostFree(h_ids);
    d_ids = nullptr;
    h_ids = nullptr;
    SPX_HIP(hipMalloc(&d_ids, sizeof(int32_t) * cap));
    SPX_HIP(hipHostMalloc(&h_ids, sizeof(int32_t) * cap, hipHostMallocDefault));
    ids_cap = cap;
  }
  const int nw_ = n_window + m - 1;
  if (nw_ > 0) memcpy(h_ids, window, sizeof(int32_t) * nw_);
  if (!stop.empty()) memcpy(h_ids + nw_, stop.data(), sizeof(int32_t) * stop.size());
  if (n_ids > 0) SPX_HIP(hipMemcpyAsync(d_ids, h_ids, sizeof(int32_t) * n_ids, hipMemcpyHostToDevice, stream));
  SampleArgs a{};
  a.x = logits;
  a.ld = ld;
  a.V = vocab;
  a.lscale = lscale;
  a.penalty = p.repeat_penalty;
  a.win = d_ids;
  a.n_win = n_window;
  a.stop = d_ids + nw_;
  a.n_stop = (int)stop.size();
  a.fstop = fstop;
  a.think = p.think_open;
  a.fthink = fthink ? 1 : 0;
  a.sel_k = device_select(p) ? p.top_k : 0;
  a.scratch = d_scratch;
  a.cidx = d_cidx;
  a.cval = d_cval;
  a.meta = d_meta;
  const size_t lds = sizeof(uint32_t) * 2 * ((vocab + 31) / 32);
  if (lds > 65536) SPX_HIP(hipFuncSetAttribute((const void *)k_sample, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  hipLaunchKernelGGL(k_sample, dim3(m), dim3(1024), lds, stream, a);
  SPX_HIP(hipGetLastError());
  SPX_HIP(hipMemcpyAsync(h_meta, d_meta, sizeof(int32_t) * 4 * m, hipMemcpyDeviceToHost, stream));
  if (a.sel_k) {
    SPX_HIP(hipMemcpyAsync(h_cidx, d_cidx, sizeof(int32_t) * SAMPLE_KMAX * m, hipMemcpyDeviceToHost, stream));
    SPX_HIP(hipMemcpyAsync(h_cval, d_cval, sizeof(float) * SAMPLE_KMAX * m, hipMemcpyDeviceToHost, stream));
  } else if (p.temperature > 0.0f) {  // top_k 0 or above SAMPLE_KMAX: the whole processed rows
    if (!h_row) SPX_HIP(hipHostMalloc(&h_row, sizeof(float) * (size_t)SAMPLE_MMAX * vocab, hipHostMallocDefault));
    SPX_HIP(hipMemcpyAsync(h_row, d_scratch, sizeof(float) * (size_t)vocab * m, hipMemcpyDeviceToHost, stream));
  }
  SPX_HIP(hipStreamSynchronize(stream));
  return 0;
}

int Sampler::pick(int r) {
  const int nf = h_meta[r * 4 + 0], greedy = h_meta[r * 4 + 1];
  if (p.temperature <= 0.0f) return greedy;  // argmax (:3662-3673)
  const int k = p.top_k == 0 ? nf : std::min(p.top_k, nf);
  if (k == 0) return greedy;  // nothing finite
  const int32_t *ci;
  const float *cv;
  std::vector<float> vals;
  if (device_select(p)) {
    ci = h_cidx + r * SAMPLE_KMAX;
    cv = h_cval + r * SAMPLE_KMAX;
  } else {
    const float *row = h_row + (size_t)r * vocab;
    order.clear();
    for (int i = 0; i < vocab; i++)
      if (std::isfinite(row[i])) order.push_back(i);
    std::sort(order.begin(), order.end(), [row](int a, int b) {
      const uint32_t ka = total_u32(row[a]), kb = total_u32(row[b]);
      return ka != kb ? ka > kb : a < b;
    });
    vals.resize(k);
    for (int i = 0; i < k; i++) vals[i] = row[order[i]];
    ci = order.data();
    cv = vals.data();
  }
  // softmax with temperature over the candidates in order (:3684-3700)
  probs.resize(k);
  const float mx = cv[0], temp = p.temperature;
  for (int i = 0; i < k; i++) probs[i] = expf((cv[i] - mx) / temp);
  float sum = 0.0f;
  for (int i = 0; i < k; i++) sum += probs[i];
  for (int i = 0; i < k; i++) probs[i] /= sum;
  // min-p, then top-p; both keep the best (:3702-3711)
  const float floor_ = p.min_p * probs[0];
  int keep = 0;
  while (keep < k && probs[keep] >= floor_) keep++;
  keep = std::max(keep, 1);
  float cum = 0.0f;
  for (int i = 0; i < keep; i++) {
    cum += probs[i];
    if (cum >= p.top_p) { keep = i + 1; break; }
  }
  // the draw over the survivors (:3714-3725)
  float total = 0.0f;
  for (int i = 0; i < keep; i++) total += probs[i];
  float rr = next_f32() * total;
  for (int i = 0; i < keep; i++) {
    rr -= probs[i];
    if (rr <= 0.0f) return ci[i];
  }
  return ci[keep - 1];
}

}  // namespace spx

// ------------------------------------------------------------------ C ABI
struct spx_sampler {
  spx::Sampler s;
};

extern "C" {

int spx_sampler_create(spx_ctx *ctx, const spx_sampler_params *p, int vocab, spx_sampler **out) {
  if (!ctx || !p || !out) return spx::fail("spx_sampler_create: null argument");
  *out = nullptr;
  spx_sampler *s = new (std::nothrow) spx_sampler();
  if (!s) return spx::fail("spx_sampler_create: out of memory");
  if (int r = s->s.init(p, vocab, ctx->device, ctx->stream)) {
    delete s;
    return r;
  }
  *out = s;
  return 0;
}

int spx_sampler_destroy(spx_sampler *s) {
  delete s;
  return 0;
}

int spx_sampler_reseed(spx_sampler *s, uint64_t seed) {
  if (!s) return spx::fail("spx_sampler_reseed: null sampler");
  s->s.rng = seed;
  return 0;
}

int spx_sample(spx_sampler *s, const float *logits, float logit_scale, const int32_t *recent, int n_recent, int forbid_stop,
               int forbid_think, int32_t *token) {
  if (!s || !logits || !token) return spx::fail("spx_sample: null argument");
  if (int r = s->s.prepare(logits, s->s.vocab, 1, logit_scale, recent, n_recent, forbid_stop ? 1u : 0u, forbid_think != 0)) return r;
  *token = s->s.pick(0);
  return 0;
}

int spx_sample_verify(spx_sampler *s, const float *logits, int64_t ld, int n_draft, float logit_scale, const int32_t *recent,
                      int n_recent, const int32_t *draft, int generated, int max_accept, int forbid_think, int32_t *tokens,
                      int *n_out) {
  if (!s || !logits || !tokens || !n_out || (n_draft > 0 && !draft)) return spx::fail("spx_sample_verify: null argument");
  if (n_draft < 0 || n_draft + 1 > spx::SAMPLE_MMAX) return spx::fail("spx_sample_verify: n_draft must be in 0..15");
  if (n_recent < 0 || (n_recent > 0 && !recent) || generated < 0) return spx::fail("spx_sample_verify: bad window");
  std::vector<int32_t> win(recent, recent + n_recent);
  win.insert(win.end(), draft, draft + n_draft);
  uint32_t fstop = 0;
  for (int i = 0; i <= n_draft; i++)
    if (generated + i < 2) fstop |= 1u << i;
  if (int r = s->s.prepare(logits, ld, n_draft + 1, logit_scale, win.data(), n_recent, fstop, forbid_think != 0)) return r;
  int n = 0;
  for (int i = 0; i <= n_draft; i++) {
    const int tok = s->s.pick(i);
    tokens[n++] = tok;
    if (i == n_draft || tok != draft[i]) break;  // the correction, or the bonus token
    if (n >= max_accept) break;                  // the reply is full: no further draw
  }
  *n_out = n;
  return 0;
}

}  // extern "C"
