/*
 * oracle.c -- CPU restatement of WiseHax/spindle's decode/verify arithmetic.
 * TEST INFRASTRUCTURE ONLY (see oracle.h for the pinning table). Build: oracle/Makefile
 * (gcc -O3 -mavx2 -mfma -ffp-contract=off). The 8-element arrays below stand for one
 * YMM register each; fmaf() stands for _mm256_fmadd_ps lane by lane.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------ threads
 * Row split of worker_pool.rs:78-105 / par_rows smollm_chat.rs:332-337: thread t of n
 * takes rows [rows*t/n, rows*(t+1)/n). Rows are independent, so the split never changes a
 * result bit; it only sets how fast the CPU baseline runs. */
typedef void (*or_job_fn)(void *ctx, int t, int n);
static int g_threads = 1;
static pthread_t g_workers[128];
static atomic_int g_gen, g_remaining, g_started;
static or_job_fn g_job;
static void *g_ctx;

static void *worker_main(void *arg) {
  int t = (int)(intptr_t)arg;
  int seen = 0;
  for (;;) {
    int spins = 0;
    while (atomic_load_explicit(&g_gen, memory_order_acquire) == seen) {
      if (++spins > 2000) sched_yield();
    }
    seen = atomic_load_explicit(&g_gen, memory_order_acquire);
    if (t >= g_threads) continue; /* started by an earlier, larger or_set_threads: idle */
    g_job(g_ctx, t, g_threads);
    atomic_fetch_sub_explicit(&g_remaining, 1, memory_order_acq_rel);
  }
  return NULL;
}

void or_set_threads(int n) {
  if (n < 1) n = 1;
  if (n > 128) n = 128;
  int have = atomic_load(&g_started);
  for (int t = have; t < n; t++) {
    if (t == 0) continue;
    pthread_create(&g_workers[t], NULL, worker_main, (void *)(intptr_t)t);
  }
  if (n > have) atomic_store(&g_started, n);
  g_threads = n;
}
int or_get_threads(void) { return g_threads; }

static void run_pool(or_job_fn f, void *ctx) {
  if (g_threads <= 1) { f(ctx, 0, 1); return; }
  g_job = f; g_ctx = ctx;
  atomic_store_explicit(&g_remaining, g_threads - 1, memory_order_release);
  atomic_fetch_add_explicit(&g_gen, 1, memory_order_acq_rel);
  f(ctx, 0, g_threads);
  while (atomic_load_explicit(&g_remaining, memory_order_acquire) > 0) { }
}

#define PAR_MIN_WEIGHTS (16 * 1024) /* smollm_chat.rs:306 */

/* ------------------------------------------------------------------ formats */
size_t or_row_bytes(int dtype, size_t cols) { /* quant.rs:1527-1542 */
  size_t block, bytes;
  switch (dtype) {
  case OR_F32: block = 1; bytes = 4; break;
  case OR_F16: case OR_BF16: block = 1; bytes = 2; break;
  case OR_Q4_0: block = 32; bytes = 18; break;
  case OR_Q4_1: block = 32; bytes = 20; break;
  case OR_Q5_0: block = 32; bytes = 22; break;
  case OR_Q5_1: block = 32; bytes = 24; break;
  case OR_Q8_0: block = 32; bytes = 34; break;
  case OR_Q4K: block = 256; bytes = 144; break;
  case OR_Q5K: block = 256; bytes = 176; break;
  case OR_Q6K: block = 256; bytes = 210; break;
  default: return 0;
  }
  if (cols % block) return 0;
  return cols / block * bytes;
}

float or_f16_to_f32(uint16_t h) { /* f16_to_f32_exact quant.rs:876-899 */
  uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  uint32_t exp = (h >> 10) & 0x1f, mant = h & 0x3ff, bits;
  if (exp == 0) {
    if (mant == 0) bits = sign;
    else {
      uint32_t m = mant; int e = 127 - 14;
      while ((m & 0x400) == 0) { m <<= 1; e -= 1; }
      bits = sign | ((uint32_t)e << 23) | ((m & 0x3ff) << 13);
    }
  } else if (exp == 31) bits = sign | 0x7f800000u | (mant << 13);
  else bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
  float f; memcpy(&f, &bits, 4); return f;
}

uint16_t or_f32_to_f16(float f) { /* IEEE binary16, round to nearest even */
  uint32_t x; memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000;
  uint32_t ax = x & 0x7fffffff;
  if (ax >= 0x7f800000u) { /* inf / nan */
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00 | ((ax >> 13) & 0x3ff));
    return (uint16_t)(sign | 0x7c00);
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00); /* rounds to >= 65520 -> inf */
  if (ax < 0x38800000u) { /* below smallest normal half: subnormal or zero */
    if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
    int e = (int)(ax >> 23);
    uint32_t m = (ax & 0x7fffff) | 0x800000;
    int s = 126 - e; /* value = m * 2^(e-150); half subnormal unit = 2^-24 */
    uint32_t q = m >> s;
    uint32_t rem = m & ((1u << s) - 1), half = 1u << (s - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t e = ((ax >> 23) - 127 + 15), m = ax & 0x7fffff;
  uint32_t q = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) q++;
  return (uint16_t)(sign | q);
}

static inline float rd16(const uint8_t *p) { return or_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

void or_unpack_q4k_scales(const uint8_t sc[12], uint8_t s[8], uint8_t m[8]) { /* q4k_gemv.rs:70-85 */
  for (int j = 0; j < 4; j++) {
    s[j] = sc[j] & 63;
    m[j] = sc[j + 4] & 63;
    s[j + 4] = (uint8_t)((sc[j + 8] & 0x0F) | ((sc[j] >> 6) << 4));
    m[j + 4] = (uint8_t)((sc[j + 8] >> 4) | ((sc[j + 4] >> 6) << 4));
  }
}

int or_dequant_row(int dtype, const uint8_t *row, size_t n, float *y) { /* quant.rs:1548-1660 */
  switch (dtype) {
  case OR_F32: memcpy(y, row, n * 4); return 0;
  case OR_F16: for (size_t i = 0; i < n; i++) y[i] = rd16(row + 2 * i); return 0;
  case OR_BF16:
    for (size_t i = 0; i < n; i++) { uint32_t b = (uint32_t)(row[2 * i] | (row[2 * i + 1] << 8)) << 16; memcpy(&y[i], &b, 4); }
    return 0;
  case OR_Q8_0:
    for (size_t b = 0; b < n / 32; b++) {
      const uint8_t *blk = row + b * 34; float d = rd16(blk);
      for (int j = 0; j < 32; j++) y[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
    }
    return 0;
  case OR_Q4_0: case OR_Q4_1: case OR_Q5_0: case OR_Q5_1: {
    int size = dtype == OR_Q4_0 ? 18 : dtype == OR_Q4_1 ? 20 : dtype == OR_Q5_0 ? 22 : 24;
    int has_m = dtype == OR_Q4_1 || dtype == OR_Q5_1, has_h = dtype == OR_Q5_0 || dtype == OR_Q5_1;
    for (size_t b = 0; b < n / 32; b++) {
      const uint8_t *blk = row + b * size; float d = rd16(blk), m = has_m ? rd16(blk + 2) : 0.0f;
      int p = has_m ? 4 : 2; uint32_t qh = 0;
      if (has_h) { qh = (uint32_t)blk[p] | ((uint32_t)blk[p + 1] << 8) | ((uint32_t)blk[p + 2] << 16) | ((uint32_t)blk[p + 3] << 24); p += 4; }
      const uint8_t *qs = blk + p;
      int center = has_m ? 0 : has_h ? 16 : 8;
      for (int j = 0; j < 16; j++) {
        int lo = qs[j] & 0x0F, hi = qs[j] >> 4;
        if (has_h) { lo |= (int)(((qh >> j) & 1) << 4); hi |= (int)(((qh >> (j + 16)) & 1) << 4); }
        y[b * 32 + j] = (float)(lo - center) * d + m;
        y[b * 32 + j + 16] = (float)(hi - center) * d + m;
      }
    }
    return 0;
  }
  case OR_Q4K: case OR_Q5K: {
    int size = dtype == OR_Q4K ? 144 : 176;
    for (size_t b = 0; b < n / 256; b++) {
      const uint8_t *blk = row + b * size; float d = rd16(blk), dmin = rd16(blk + 2);
      uint8_t sc[8], mn[8]; or_unpack_q4k_scales(blk + 4, sc, mn);
      const uint8_t *qh = blk + 16, *qs = size == 176 ? blk + 48 : blk + 16;
      float *out = y + b * 256;
      for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) {
          uint8_t q = qs[c * 32 + l]; uint32_t lo = q & 0x0F, hi = q >> 4;
          if (size == 176) { lo |= ((uint32_t)(qh[l] >> (2 * c)) & 1) << 4; hi |= ((uint32_t)(qh[l] >> (2 * c + 1)) & 1) << 4; }
          out[c * 64 + l] = d * (float)sc[2 * c] * (float)lo - dmin * (float)mn[2 * c];
          out[c * 64 + 32 + l] = d * (float)sc[2 * c + 1] * (float)hi - dmin * (float)mn[2 * c + 1];
        }
    }
    return 0;
  }
  case OR_Q6K:
    for (size_t b = 0; b < n / 256; b++) {
      const uint8_t *blk = row + b * 210, *ql0 = blk, *qh0 = blk + 128;
      float d = rd16(blk + 208);
      for (int half = 0; half < 2; half++) {
        const uint8_t *ql = ql0 + half * 64, *qh = qh0 + half * 32;
        float *o = y + b * 256 + half * 128; int s = half * 8;
        for (int l = 0; l < 32; l++) {
          int is = l / 16;
          int q1 = ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
          int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
          int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
          int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
          o[l] = d * (float)(int8_t)blk[192 + s + is] * (float)q1;
          o[l + 32] = d * (float)(int8_t)blk[192 + s + is + 2] * (float)q2;
          o[l + 64] = d * (float)(int8_t)blk[192 + s + is + 4] * (float)q3;
          o[l + 96] = d * (float)(int8_t)blk[192 + s + is + 6] * (float)q4;
        }
      }
    }
    return 0;
  default: return -1;
  }
}

/* ------------------------------------------------------------------ horizontal sums */
/* quant_q8k.rs:151-158 and quant_multi.rs:34-40: (a0+a4)+(a2+a6) + ((a1+a5)+(a3+a7)) */
static inline float hsum_int(const float a[8]) {
  float x0 = a[0] + a[4], x1 = a[1] + a[5], x2 = a[2] + a[6], x3 = a[3] + a[7];
  return (x0 + x2) + (x1 + x3);
}
/* quant.rs:901-908 (two hadds): ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)) */
static inline float hsum_hadd(const float a[8]) {
  float x0 = a[0] + a[4], x1 = a[1] + a[5], x2 = a[2] + a[6], x3 = a[3] + a[7];
  return (x0 + x1) + (x2 + x3);
}

/* ------------------------------------------------------------------ Q8_K */
static inline float max_ps(float a, float b) { return a > b ? a : b; } /* maxps: 2nd if unordered */

void or_q8k_quantize(const float *x, size_t n, float *d, int8_t *qs, int16_t *bsums) {
  /* quantize_avx2 quant_q8k.rs:84-121 */
  for (size_t b = 0; b < n / 256; b++) {
    const float *xb = x + b * 256;
    float am[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < 256; j += 8)
      for (int l = 0; l < 8; l++) am[l] = max_ps(am[l], fabsf(xb[j + l]));
    float v[4];
    for (int t = 0; t < 4; t++) v[t] = max_ps(am[t], am[t + 4]);
    float v0 = max_ps(v[0], v[2]), v1 = max_ps(v[1], v[3]);
    float m = max_ps(v0, v1);
    int8_t *out = qs + b * 256;
    if (!(m > 0.0f) || !isfinite(m)) {
      d[b] = 0.0f; memset(out, 0, 256);
      memset(bsums + b * 16, 0, 16 * sizeof(int16_t));
      continue;
    }
    float iscale = 127.0f / m;
    d[b] = m / 127.0f;
    for (int j = 0; j < 256; j++) {
      float p = xb[j] * iscale;
      /* cvtps_epi32 (round to nearest even; out of range -> INT_MIN) then packs (saturate) */
      int32_t q;
      float r = nearbyintf(p);
      if (!(r >= -2147483648.0f && r < 2147483648.0f)) q = INT32_MIN; else q = (int32_t)r;
      if (q > 127) q = 127;
      if (q < -128) q = -128;
      out[j] = (int8_t)q;
    }
    for (int g = 0; g < 16; g++) {
      int s = 0;
      for (int j = 0; j < 16; j++) s += out[g * 16 + j];
      bsums[b * 16 + g] = (int16_t)s;
    }
  }
}

/* ------------------------------------------------------------------ integer kernel
 * rows<B,T> quant_q8k.rs:163-250. Lane l of `sumi` holds elements 32k+4l..32k+4l+3 of the
 * eight 32-weight chunks k, each multiplied by its scale (maddubs -> madd). */
static void q8k_block_lanes(const uint8_t *blk, int dtype, const int8_t *y, const int16_t *bs,
                            int32_t lanes[8], int32_t *corr_int, float *d_out, float *dmin_out) {
  uint8_t w[256];
  int16_t scv[256]; /* scale of element e */
  if (dtype == OR_Q4K) {
    uint8_t sc[8], mn[8]; or_unpack_q4k_scales(blk + 4, sc, mn);
    const uint8_t *q = blk + 16;
    for (int c = 0; c < 4; c++)
      for (int b = 0; b < 32; b++) {
        w[64 * c + b] = q[32 * c + b] & 0x0F; scv[64 * c + b] = sc[2 * c];
        w[64 * c + 32 + b] = q[32 * c + b] >> 4; scv[64 * c + 32 + b] = sc[2 * c + 1];
      }
    int s = 0;
    for (int j = 0; j < 8; j++) s += mn[j] * ((int)bs[2 * j] + (int)bs[2 * j + 1]);
    *corr_int = s;
    *d_out = rd16(blk); *dmin_out = rd16(blk + 2);
  } else {
    const int8_t *sc = (const int8_t *)(blk + 192);
    for (int h = 0; h < 2; h++) {
      const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
      for (int b = 0; b < 32; b++) {
        w[128 * h + b] = (uint8_t)((ql[b] & 0xF) | ((qh[b] & 3) << 4));
        w[128 * h + 32 + b] = (uint8_t)((ql[32 + b] & 0xF) | (((qh[b] >> 2) & 3) << 4));
        w[128 * h + 64 + b] = (uint8_t)((ql[b] >> 4) | (((qh[b] >> 4) & 3) << 4));
        w[128 * h + 96 + b] = (uint8_t)((ql[32 + b] >> 4) | ((qh[b] >> 6) << 4));
      }
    }
    for (int e = 0; e < 256; e++) scv[e] = sc[e / 16];
    int s = 0;
    for (int g = 0; g < 16; g++) s += (int)sc[g] * (int)bs[g];
    *corr_int = 32 * s;
    *d_out = rd16(blk + 208); *dmin_out = 0.0f;
  }
  for (int l = 0; l < 8; l++) {
    int32_t acc = 0;
    for (int k = 0; k < 8; k++) {
      int e0 = 32 * k + 4 * l;
      /* maddubs: two u8*i8 pairs -> i16 (no saturation is reachable: |pair| <= 2*63*127) */
      int32_t p0 = (int32_t)w[e0] * y[e0] + (int32_t)w[e0 + 1] * y[e0 + 1];
      int32_t p1 = (int32_t)w[e0 + 2] * y[e0 + 2] + (int32_t)w[e0 + 3] * y[e0 + 3];
      if (p0 > 32767) p0 = 32767; if (p0 < -32768) p0 = -32768;
      if (p1 > 32767) p1 = 32767; if (p1 < -32768) p1 = -32768;
      /* madd with the broadcast i16 scale (per 16 for Q6_K: e0 and e0+3 share it) */
      acc += p0 * scv[e0] + p1 * scv[e0 + 2];
    }
    lanes[l] = acc;
  }
}

void or_q8k_block_sums(const uint8_t *row, int dtype, size_t cols, const int8_t *xs,
                       const int16_t *xb, int32_t *sumi, int32_t *corr, int32_t *lanes) {
  size_t nb = cols / 256, bb = dtype == OR_Q4K ? 144 : 210;
  for (size_t i = 0; i < nb; i++) {
    int32_t l8[8], ci; float d, dm;
    q8k_block_lanes(row + i * bb, dtype, xs + i * 256, xb + i * 16, l8, &ci, &d, &dm);
    int32_t s = 0;
    for (int l = 0; l < 8; l++) s += l8[l];
    sumi[i] = s; corr[i] = ci;
    if (lanes) memcpy(lanes + 8 * i, l8, sizeof l8);
  }
}

static float q8k_row_dot(const uint8_t *row, int dtype, size_t nb, const float *xd, const int8_t *xs, const int16_t *xb) {
  size_t bb = dtype == OR_Q4K ? 144 : 210;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float corr = 0.0f;
  for (size_t i = 0; i < nb; i++) {
    int32_t l8[8], ci; float d, dmin;
    q8k_block_lanes(row + i * bb, dtype, xs + i * 256, xb + i * 16, l8, &ci, &d, &dmin);
    if (dtype == OR_Q4K) corr += dmin * xd[i] * (float)ci;   /* :204 */
    else corr += d * xd[i] * (float)ci;                      /* :232, ci = 32*s */
    float dd = d * xd[i];                                    /* set1_ps(d * xd) :243 */
    for (int l = 0; l < 8; l++) acc[l] = fmaf(dd, (float)l8[l], acc[l]);
  }
  return hsum_int(acc) - corr;                               /* :247 */
}

/* The same kernel with the reference's AVX2 instructions (rows<B,T> quant_q8k.rs:163-245):
 * each block's codes unpacked once into eight 32-byte chunks (chunk k = elements 32k..32k+31)
 * and applied to every vector: maddubs (u8 x i8 pairs -> i16), madd with the chunk's i16
 * scales (Q6_K: one per 16 elements), eight int32 lanes; the fp32 chain per lane. Lane l's
 * integer and every rounding are those of q8k_block_lanes / q8k_row_dot (checked bit for bit). */
static int g_simd = 1;
void or_set_simd(int on) { g_simd = on; }

static inline void q8k_block_decode_avx2(const uint8_t *blk, int dtype, __m256i w[8], __m256i scv[8], int8_t sc6[16],
                                         uint8_t mn4[8], float *d, float *dmin) {
  const __m256i m4 = _mm256_set1_epi8(0x0F), m3 = _mm256_set1_epi8(3);
  if (dtype == OR_Q4K) {
    uint8_t sc[8];
    or_unpack_q4k_scales(blk + 4, sc, mn4);
    for (int c = 0; c < 4; c++) {
      __m256i q = _mm256_loadu_si256((const __m256i *)(blk + 16 + 32 * c));
      w[2 * c] = _mm256_and_si256(q, m4);
      w[2 * c + 1] = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
      scv[2 * c] = _mm256_set1_epi16(sc[2 * c]);
      scv[2 * c + 1] = _mm256_set1_epi16(sc[2 * c + 1]);
    }
    *d = rd16(blk); *dmin = rd16(blk + 2);
  } else {
    const int8_t *sc = (const int8_t *)(blk + 192);
    for (int h = 0; h < 2; h++) {
      __m256i l0 = _mm256_loadu_si256((const __m256i *)(blk + 64 * h)), l1 = _mm256_loadu_si256((const __m256i *)(blk + 64 * h + 32));
      __m256i qh = _mm256_loadu_si256((const __m256i *)(blk + 128 + 32 * h));
      w[4 * h + 0] = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(qh, m3), 4));
      w[4 * h + 1] = _mm256_or_si256(_mm256_and_si256(l1, m4), _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 2), m3), 4));
      w[4 * h + 2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4), _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 4), m3), 4));
      w[4 * h + 3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4), _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 6), m3), 4));
    }
    for (int k = 0; k < 8; k++) {
      __m128i lo = _mm_set1_epi16(sc[2 * k]), hi = _mm_set1_epi16(sc[2 * k + 1]);
      scv[k] = _mm256_set_m128i(hi, lo);
    }
    memcpy(sc6, sc, 16);
    *d = rd16(blk + 208); *dmin = 0.0f;
  }
}

static void q8k_rows_avx2(const uint8_t *tensor, int dtype, size_t cols, int nvec, const float *const *xd, const int8_t *const *xs,
                          const int16_t *const *xb, float *const *outs, size_t r0, size_t r1) {
  size_t nb = cols / 256, rb = or_row_bytes(dtype, cols);
  __m256 acc[16];
  float corr[16];
  for (size_t r = r0; r < r1; r++) {
    const uint8_t *row = tensor + r * rb;
    for (int v0 = 0; v0 < nvec; v0 += 16) {
      int nv = nvec - v0 < 16 ? nvec - v0 : 16;
      for (int v = 0; v < nv; v++) { acc[v] = _mm256_setzero_ps(); corr[v] = 0.0f; }
      for (size_t i = 0; i < nb; i++) {
        __m256i w[8], scv[8];
        int8_t sc6[16];
        uint8_t mn[8];
        float d, dmin;
        q8k_block_decode_avx2(row + i * (dtype == OR_Q4K ? 144 : 210), dtype, w, scv, sc6, mn, &d, &dmin);
        for (int v = 0; v < nv; v++) {
          const int8_t *y = xs[v0 + v] + i * 256;
          const int16_t *bs = xb[v0 + v] + i * 16;
          __m256i l8 = _mm256_setzero_si256();
          for (int k = 0; k < 8; k++) {
            __m256i p = _mm256_maddubs_epi16(w[k], _mm256_loadu_si256((const __m256i *)(y + 32 * k)));
            l8 = _mm256_add_epi32(l8, _mm256_madd_epi16(p, scv[k]));
          }
          int ci = 0;
          if (dtype == OR_Q4K) {
            for (int j = 0; j < 8; j++) ci += mn[j] * ((int)bs[2 * j] + (int)bs[2 * j + 1]);
            corr[v] += dmin * xd[v0 + v][i] * (float)ci;
          } else {
            for (int g = 0; g < 16; g++) ci += (int)sc6[g] * (int)bs[g];
            corr[v] += d * xd[v0 + v][i] * (float)(32 * ci);
          }
          acc[v] = _mm256_fmadd_ps(_mm256_set1_ps(d * xd[v0 + v][i]), _mm256_cvtepi32_ps(l8), acc[v]);
        }
      }
      for (int v = 0; v < nv; v++) {
        float a[8];
        _mm256_storeu_ps(a, acc[v]);
        outs[v0 + v][r] = hsum_int(a) - corr[v];
      }
    }
  }
}

typedef struct {
  const uint8_t *tensor; int dtype; size_t cols; int nvec;
  const float *const *xd; const int8_t *const *xs; const int16_t *const *xb; float *const *outs;
  size_t r0, r1;
} q8k_job;

static void q8k_job_run(void *p, int t, int n) {
  q8k_job *j = (q8k_job *)p;
  size_t rows = j->r1 - j->r0, a = j->r0 + rows * t / n, b = j->r0 + rows * (t + 1) / n;
  if (g_simd) { q8k_rows_avx2(j->tensor, j->dtype, j->cols, j->nvec, j->xd, j->xs, j->xb, j->outs, a, b); return; }
  size_t nb = j->cols / 256, rb = or_row_bytes(j->dtype, j->cols);
  for (size_t r = a; r < b; r++)
    for (int v = 0; v < j->nvec; v++)
      j->outs[v][r] = q8k_row_dot(j->tensor + r * rb, j->dtype, nb, j->xd[v], j->xs[v], j->xb[v]);
}

void or_q8k_matmul_rows(const uint8_t *tensor, int dtype, size_t cols, int nvec,
                        const float *const *xd, const int8_t *const *xs,
                        const int16_t *const *xb, float *const *outs, size_t r0, size_t r1) {
  if (r1 <= r0 || nvec <= 0) return;
  q8k_job j = {tensor, dtype, cols, nvec, xd, xs, xb, outs, r0, r1};
  if ((r1 - r0) * cols >= PAR_MIN_WEIGHTS) run_pool(q8k_job_run, &j);
  else q8k_job_run(&j, 0, 1);
}

/* ------------------------------------------------------------------ float kernels */
/* Q8_0 / Q5_0 block: s_l = fma chain over sub 0,8,16,24 (quant.rs:62-66, 149-152) */
static inline void block32_lanes(const float q[32], const float *x, float s[8]) {
  for (int l = 0; l < 8; l++) {
    float a = 0.0f;
    for (int sub = 0; sub < 32; sub += 8) a = fmaf(q[sub + l], x[sub + l], a);
    s[l] = a;
  }
}

static void q8_0_codes(const uint8_t *blk, float q[32]) { for (int j = 0; j < 32; j++) q[j] = (float)(int8_t)blk[2 + j]; }
static void q5_0_codes(const uint8_t *blk, float q[32]) {
  uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
  const uint8_t *qs = blk + 6;
  for (int j = 0; j < 16; j++) {
    int lo = (qs[j] & 0x0F) | (int)(((qh >> j) & 1) << 4);
    int hi = (qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1) << 4);
    q[j] = (float)(lo - 16); q[j + 16] = (float)(hi - 16);
  }
}

/* Q5_K (quant.rs:1266-1313, dot_q5_k_row_avx2_presum with compute_subblock_sums_32 :167-178):
 * per 32-value sub-block the activation sum act = hsum((x_l + x_{8+l}) + (x_{16+l} + x_{24+l}));
 * per block min_term = sum_k mn_k * act_k (in k order), total_min += min_term * dmin; per
 * sub-block j = 2c + h lane l: sqx_l = fma chain over elements l, 8+l, 16+l, 24+l (fma_u8x16
 * :1163-1172), acc_l = fma(d * sc_j, sqx_l, acc_l); the row is hsum(acc) - total_min. */
static float act_sum32(const float *p) {
  float s[8];
  for (int l = 0; l < 8; l++) s[l] = (p[l] + p[8 + l]) + (p[16 + l] + p[24 + l]);
  return hsum_hadd(s);
}
static float dot_q5k_row(const uint8_t *row, size_t n, const float *x) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, total_min = 0.0f;
  for (size_t b = 0; b < n / 256; b++) {
    const uint8_t *blk = row + b * 176;
    const float d = rd16(blk), dmin = rd16(blk + 2);
    uint8_t sc[8], mn[8];
    or_unpack_q4k_scales(blk + 4, sc, mn);
    const uint8_t *qh = blk + 16, *qs = blk + 48;
    const float *xb = x + b * 256;
    float min_term = 0.0f;
    for (int k = 0; k < 8; k++) min_term += (float)mn[k] * act_sum32(xb + 32 * k);
    total_min += min_term * dmin;
    for (int c = 0; c < 4; c++)
      for (int h = 0; h < 2; h++) {
        float q[32];
        for (int t = 0; t < 32; t++) {
          const uint32_t byte = qs[32 * c + t], nib = h ? byte >> 4 : byte & 0x0F;
          q[t] = (float)(nib | (((uint32_t)(qh[t] >> (2 * c + h)) & 1u) << 4));
        }
        const float *xs = xb + 64 * c + 32 * h, dsc = d * (float)sc[2 * c + h];
        for (int l = 0; l < 8; l++) {
          float sq = 0.0f;
          for (int k = 0; k < 4; k++) sq = fmaf(q[8 * k + l], xs[8 * k + l], sq);
          acc[l] = fmaf(dsc, sq, acc[l]);
        }
      }
  }
  return hsum_hadd(acc) - total_min;
}

static float dot_float_row(const uint8_t *row, int dtype, size_t n, const float *x) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (dtype == OR_Q5K) return dot_q5k_row(row, n, x);
  if (dtype == OR_Q8_0 || dtype == OR_Q5_0) { /* quant.rs:48-161 */
    size_t bb = dtype == OR_Q8_0 ? 34 : 22;
    for (size_t b = 0; b < n / 32; b++) {
      const uint8_t *blk = row + b * bb; float q[32], s[8];
      if (dtype == OR_Q8_0) q8_0_codes(blk, q); else q5_0_codes(blk, q);
      block32_lanes(q, x + b * 32, s);
      float d = rd16(blk);
      for (int l = 0; l < 8; l++) acc[l] = fmaf(d, s[l], acc[l]);
    }
    return hsum_hadd(acc);
  }
  /* F32 / F16: dot_f32_avx2 quant.rs:860-874, dot_f16_row_avx2 :1409-1425 */
  size_t main = n & ~(size_t)7; float tail = 0.0f;
  for (size_t i = 0; i < main; i += 8)
    for (int l = 0; l < 8; l++) {
      float w = dtype == OR_F32 ? ((const float *)row)[i + l] : rd16(row + 2 * (i + l));
      acc[l] = fmaf(w, x[i + l], acc[l]);
    }
  for (size_t i = main; i < n; i++) {
    float w = dtype == OR_F32 ? ((const float *)row)[i] : rd16(row + 2 * i);
    tail += w * x[i];
  }
  return hsum_hadd(acc) + tail;
}

typedef struct { const uint8_t *tensor; int dtype; size_t cols; const float *x; float *out; size_t r0, n; } fjob;
static void fjob_run(void *p, int t, int nt) {
  fjob *j = (fjob *)p; size_t rb = or_row_bytes(j->dtype, j->cols);
  size_t a = j->n * t / nt, b = j->n * (t + 1) / nt;
  for (size_t i = a; i < b; i++) j->out[i] = dot_float_row(j->tensor + (j->r0 + i) * rb, j->dtype, j->cols, j->x);
}

int or_matvec_rows(const uint8_t *tensor, int dtype, size_t cols, const float *x, float *out, size_t r0, size_t nrows) {
  if (!(dtype == OR_F32 || dtype == OR_F16 || dtype == OR_Q8_0 || dtype == OR_Q5_0 || dtype == OR_Q5K)) return -1;
  if (!or_row_bytes(dtype, cols)) return -1;
  fjob j = {tensor, dtype, cols, x, out, r0, nrows};
  if (nrows * cols >= PAR_MIN_WEIGHTS) run_pool(fjob_run, &j); else fjob_run(&j, 0, 1);
  return 0;
}

/* quant_multi rows_multi (quant_multi.rs:124-217): Q8_0 alternates acc0/acc1 by block
 * parity, F32 by 8-chunk parity; result hsum(acc0 + acc1) with the integer-path tree. */
static float dot_multi_row(const uint8_t *row, int dtype, size_t n, const float *x) {
  float a0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, a1[8] = {0, 0, 0, 0, 0, 0, 0, 0}, v[8];
  if (dtype == OR_F32) {
    const float *w = (const float *)row; size_t j = 0;
    for (; j + 16 <= n; j += 16)
      for (int l = 0; l < 8; l++) { a0[l] = fmaf(w[j + l], x[j + l], a0[l]); a1[l] = fmaf(w[j + 8 + l], x[j + 8 + l], a1[l]); }
    for (; j < n; j += 8)
      for (int l = 0; l < 8; l++) a0[l] = fmaf(w[j + l], x[j + l], a0[l]);
  } else { /* Q8_0 */
    for (size_t b = 0; b < n / 32; b++) {
      const uint8_t *blk = row + b * 34; float q[32], s[8];
      q8_0_codes(blk, q);
      block32_lanes(q, x + b * 32, s);
      float d = rd16(blk); float *acc = (b & 1) ? a1 : a0;
      for (int l = 0; l < 8; l++) acc[l] = fmaf(d, s[l], acc[l]);
    }
  }
  for (int l = 0; l < 8; l++) v[l] = a0[l] + a1[l];
  return hsum_int(v);
}

typedef struct { const uint8_t *tensor; int dtype; size_t cols; int nvec; const float *const *xs; float *const *outs; size_t r0, r1; } mjob;
static void mjob_run(void *p, int t, int nt) {
  mjob *j = (mjob *)p; size_t rb = or_row_bytes(j->dtype, j->cols), rows = j->r1 - j->r0;
  size_t a = j->r0 + rows * t / nt, b = j->r0 + rows * (t + 1) / nt;
  for (size_t r = a; r < b; r++)
    for (int v = 0; v < j->nvec; v++) j->outs[v][r] = dot_multi_row(j->tensor + r * rb, j->dtype, j->cols, j->xs[v]);
}

int or_matmul_rows_multi(const uint8_t *tensor, int dtype, size_t cols, int nvec,
                         const float *const *xs, float *const *outs, size_t r0, size_t r1) {
  if (r1 <= r0 || nvec <= 0) return 0;
  int has_multi = (dtype == OR_Q8_0 && cols % 32 == 0) || (dtype == OR_F32 && cols % 8 == 0);
  if (!has_multi || nvec == 1) { /* quant_multi.rs:240-247 */
    for (int v = 0; v < nvec; v++)
      if (or_matvec_rows(tensor, dtype, cols, xs[v], outs[v] + r0, r0, r1 - r0)) return -1;
    return 0;
  }
  mjob j = {tensor, dtype, cols, nvec, xs, outs, r0, r1};
  if ((r1 - r0) * cols >= PAR_MIN_WEIGHTS) run_pool(mjob_run, &j); else mjob_run(&j, 0, 1);
  return 0;
}

/* ------------------------------------------------------------------ operators */
static int q8k_supports(const or_mat *m) { return (m->dtype == OR_Q4K || m->dtype == OR_Q6K) && m->cols % 256 == 0 && m->cols > 0; }

or_mat or_expert(or_mat m, int e) { m.data += (size_t)e * m.rows * or_row_bytes(m.dtype, m.cols); return m; }

typedef struct { float *d; int8_t *qs; int16_t *bs; } q8k_buf;
static q8k_buf q8k_alloc(size_t n) {
  q8k_buf b; b.d = (float *)malloc(sizeof(float) * (n / 256 + 1)); b.qs = (int8_t *)malloc(n + 1); b.bs = (int16_t *)malloc(sizeof(int16_t) * (n / 16 + 1)); return b;
}
static void q8k_free(q8k_buf b) { free(b.d); free(b.qs); free(b.bs); }

static void rows_into_q8k(const or_mat *m, const q8k_buf *q, float *out, size_t r0, size_t r1) {
  const float *xd = q->d; const int8_t *xs = q->qs; const int16_t *xb = q->bs;
  or_q8k_matmul_rows(m->data, m->dtype, m->cols, 1, &xd, &xs, &xb, &out, r0, r1);
}

int or_matvec(const or_mat *m, const float *x, float *out) { /* smollm_chat.rs:309-349 */
  if (q8k_supports(m)) {
    q8k_buf q = q8k_alloc(m->cols);
    or_q8k_quantize(x, m->cols, q.d, q.qs, q.bs);
    rows_into_q8k(m, &q, out, 0, m->rows);
    q8k_free(q);
    return 0;
  }
  return or_matvec_rows(m->data, m->dtype, m->cols, x, out, 0, m->rows);
}

int or_matvec_multi(const or_mat *m, int nvec, const float *const *xs, float *const *outs) { /* :447-512 */
  if (nvec <= 0) return 0;
  if (nvec == 1) return or_matvec(m, xs[0], outs[0]);
  if (m->dtype == OR_F32) {
    for (int v = 0; v < nvec; v++) if (or_matvec(m, xs[v], outs[v])) return -1;
    return 0;
  }
  if (q8k_supports(m)) {
    const float **xd = malloc(sizeof(void *) * nvec); const int8_t **xq = malloc(sizeof(void *) * nvec);
    const int16_t **xb = malloc(sizeof(void *) * nvec); q8k_buf *bufs = malloc(sizeof(q8k_buf) * nvec);
    for (int v = 0; v < nvec; v++) {
      bufs[v] = q8k_alloc(m->cols); or_q8k_quantize(xs[v], m->cols, bufs[v].d, bufs[v].qs, bufs[v].bs);
      xd[v] = bufs[v].d; xq[v] = bufs[v].qs; xb[v] = bufs[v].bs;
    }
    or_q8k_matmul_rows(m->data, m->dtype, m->cols, nvec, xd, xq, xb, outs, 0, m->rows);
    for (int v = 0; v < nvec; v++) q8k_free(bufs[v]);
    free(xd); free(xq); free(xb); free(bufs);
    return 0;
  }
  return or_matmul_rows_multi(m->data, m->dtype, m->cols, nvec, xs, outs, 0, m->rows);
}

/* ------------------------------------------------------------------ small ops */
/* Test knob (never on by default): g_norm_order = 1 sums the RMSNorm squares in the order the
 * GPU kernels use instead of the reference's sequential order, to measure how far a last-bit
 * difference in one norm carries through a whole model (tests/test_gpu_configs.py). Per
 * 256-value block, value group j = x[4j..4j+3] gives fma(x3,x3,fma(x2,x2,fma(x1,x1,x0*x0))),
 * the 64 groups are added in a pairwise tree in index order, the blocks in order; a head of
 * hd <= 128 values gives fma(a,a,b*b) per pair (a, b) = the RoPE pair, then the same tree. */
static int g_norm_order = 0;
void or_set_norm_order(int gpu_order) { g_norm_order = gpu_order; }
/* Test capture (never set by default): or_ffns_fused copies its k x n_ff SwiGLU rows here. */
static float *g_dbg_h = NULL;
void or_set_dbg_h(float *h) { g_dbg_h = h; }
static float tree64(float p[64]) {
  for (int w = 1; w < 64; w *= 2)
    for (int i = 0; i < 64; i += 2 * w) p[i] = p[i] + p[i + w];
  return p[0];
}
static float sumsq_blocks(const float *x, size_t n) {
  float S = 0.0f;
  for (size_t b = 0; b < n / 256; b++) {
    float p[64];
    for (int j = 0; j < 64; j++) {
      const float *v = x + 256 * b + 4 * j;
      float t = v[0] * v[0];
      t = fmaf(v[1], v[1], t);
      t = fmaf(v[2], v[2], t);
      t = fmaf(v[3], v[3], t);
      p[j] = t;
    }
    S = S + tree64(p);
  }
  return S;
}
static float sumsq_head(const float *x, size_t hd, int neox) {
  float p[64];
  size_t half = hd / 2;
  for (int j = 0; j < 64; j++) {
    if ((size_t)j < half) {
      float a = x[neox ? (size_t)j : 2 * (size_t)j], b = x[neox ? j + half : 2 * (size_t)j + 1];
      p[j] = fmaf(a, a, b * b);
    } else p[j] = 0.0f;
  }
  return tree64(p);
}
void or_rmsnorm(const float *x, const float *w, float *out, size_t n, float eps) { /* :569-575 */
  float ss = 0.0f;
  if (g_norm_order && n % 256 == 0) ss = sumsq_blocks(x, n);
  else for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
  float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (size_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}
static void rmsnorm_heads_neox(float *v, const float *w, size_t len, size_t hd, float eps, int neox) {
  float *tmp = malloc(sizeof(float) * hd);
  for (size_t h = 0; h + hd <= len; h += hd) {
    if (g_norm_order && hd <= 128) {
      float inv = 1.0f / sqrtf(sumsq_head(v + h, hd, neox) / (float)hd + eps);
      for (size_t i = 0; i < hd; i++) tmp[i] = v[h + i] * inv * w[i];
    } else or_rmsnorm(v + h, w, tmp, hd, eps);
    memcpy(v + h, tmp, hd * 4);
  }
  free(tmp);
}
void or_rmsnorm_heads(float *v, const float *w, size_t len, size_t hd, float eps) { /* :577-584 */
  rmsnorm_heads_neox(v, w, len, hd, eps, 1);
}
float or_silu(float x) { return x / (1.0f + expf(-x)); } /* :586-588 */

void or_rope_inv_freq(size_t hd, float theta, float *f) { /* Rope::new :1399-1402 */
  for (size_t i = 0; i < hd / 2; i++) f[i] = 1.0f / powf(theta, 2.0f * (float)i / (float)hd);
}
void or_rope_rotate(const float *f, int neox, float *v, size_t len, size_t hd, float pos) { /* :1404-1419 */
  size_t half = hd / 2;
  for (size_t h = 0; h + hd <= len; h += hd)
    for (size_t i = 0; i < half; i++) {
      float ang = pos * f[i], s = sinf(ang), c = cosf(ang);
      size_t a = neox ? i : 2 * i, b = neox ? i + half : 2 * i + 1;
      float x0 = v[h + a], x1 = v[h + b];
      v[h + a] = x0 * c - x1 * s;
      v[h + b] = x0 * s + x1 * c;
    }
}

/* ------------------------------------------------------------------ FFN / MoE */
static void swiglu_rows(const or_mat *g, const or_mat *u, const float *x, const q8k_buf *xq, float *h, float *t) {
  /* gate_up_rows :351-360 */
  if (xq && q8k_supports(g)) rows_into_q8k(g, xq, h, 0, g->rows); else or_matvec_rows(g->data, g->dtype, g->cols, x, h, 0, g->rows);
  if (xq && q8k_supports(u)) rows_into_q8k(u, xq, t, 0, u->rows); else or_matvec_rows(u->data, u->dtype, u->cols, x, t, 0, u->rows);
  for (size_t r = 0; r < g->rows; r++) h[r] = or_silu(h[r]) * t[r];
}

/* ffns_fused's second pass and combine (:410-437): y_e = down_e(h_e) (h_e re-quantized to Q8_K
 * for an integer down), then out[r] += w_e y_e[r] in chosen order, each product and sum rounded
 * separately. h: k rows of down->cols. */
int or_down_combine(const or_mat *down, int k, const int *experts, const float *weights, const float *h, float *out) {
  if (k <= 0) return 0;
  size_t nff = down->cols, dim = down->rows;
  int int_down = q8k_supports(down);
  float *y = malloc(sizeof(float) * k * dim);
  for (int e = 0; e < k; e++) {
    or_mat d = or_expert(*down, experts[e]);
    if (int_down) {
      q8k_buf hq = q8k_alloc(nff);
      or_q8k_quantize(h + e * nff, nff, hq.d, hq.qs, hq.bs);
      rows_into_q8k(&d, &hq, y + e * dim, 0, dim);
      q8k_free(hq);
    } else or_matvec_rows(d.data, d.dtype, d.cols, h + e * nff, y + e * dim, 0, dim);
  }
  for (size_t r = 0; r < dim; r++) { /* :432-437, non-fused adds in chosen order */
    float acc = out[r];
    for (int e = 0; e < k; e++) acc += weights[e] * y[e * dim + r];
    out[r] = acc;
  }
  free(y);
  return 0;
}

int or_ffns_fused(const or_mat *gate, const or_mat *up, const or_mat *down, int k,
                  const int *experts, const float *weights, const float *x, float *out) {
  if (k <= 0) return 0;
  size_t nff = gate->rows;
  int use_int = q8k_supports(gate) || q8k_supports(up);
  float *h = malloc(sizeof(float) * k * nff), *t = malloc(sizeof(float) * nff);
  q8k_buf xq = q8k_alloc(gate->cols);
  if (use_int) or_q8k_quantize(x, gate->cols, xq.d, xq.qs, xq.bs);
  for (int e = 0; e < k; e++) {
    or_mat g = or_expert(*gate, experts[e]), u = or_expert(*up, experts[e]);
    swiglu_rows(&g, &u, x, use_int ? &xq : NULL, h + e * nff, t);
  }
  if (g_dbg_h) memcpy(g_dbg_h, h, sizeof(float) * k * nff);
  or_down_combine(down, k, experts, weights, h, out);
  q8k_free(xq); free(h); free(t);
  return 0;
}

/* router softmax + top-k + prune (:1199-1239, :959-997). Ties in probability go to the lower
 * expert index (the reference's select_nth_unstable_by leaves tie order unspecified). */
static int route(const or_config *c, const float *logits, float *probs, int *chosen, float *wts) {
  int ne = c->n_expert, nu = c->n_expert_used;
  float mx = -INFINITY;
  for (int e = 0; e < ne; e++) mx = fmaxf(mx, logits[e]);
  for (int e = 0; e < ne; e++) probs[e] = expf(logits[e] - mx);
  float sum = 0.0f;
  for (int e = 0; e < ne; e++) sum += probs[e];
  for (int e = 0; e < ne; e++) probs[e] /= sum;
  int idx[512];
  for (int e = 0; e < ne; e++) idx[e] = e;
  for (int i = 0; i < nu; i++) { /* partial selection sort: stable, descending */
    int best = i;
    for (int j = i + 1; j < ne; j++)
      if (probs[idx[j]] > probs[idx[best]] || (probs[idx[j]] == probs[idx[best]] && idx[j] < idx[best])) best = j;
    int tmp = idx[i]; idx[i] = idx[best]; idx[best] = tmp;
  }
  int keep = nu;
  if (c->moe_prune > 0.0f && nu > 2) {
    int min_keep = nu / 2 > 2 ? nu / 2 : 2;
    if (c->moe_prune >= 1.0f) {
      keep = (int)c->moe_prune;
      if (keep < min_keep) keep = min_keep;
      if (keep > nu) keep = nu;
    } else {
      float top = 0.0f;
      for (int i = 0; i < nu; i++) top += probs[idx[i]];
      float target = top * (1.0f - c->moe_prune), cum = 0.0f;
      int k = 0;
      while (k < nu && (k < min_keep || cum < target)) { cum += probs[idx[k]]; k++; }
      keep = k;
    }
  }
  float wsum = 0.0f;
  for (int i = 0; i < keep; i++) wsum += probs[idx[i]];
  for (int i = 0; i < keep; i++) { chosen[i] = idx[i]; wts[i] = c->expert_norm ? probs[idx[i]] / wsum : probs[idx[i]]; }
  return keep;
}

int or_moe_forward(const or_config *c, const or_layer *ly, int n, const float *const *xs,
                   float *const *outs, int *chosen_out, int *nkeep_out) {
  int ne = c->n_expert; size_t dim = ly->down.rows, nff = ly->gate.rows;
  float *logits = malloc(sizeof(float) * ne * n), *probs = malloc(sizeof(float) * ne);
  int chosen[16][32]; float wts[16][32]; int nk[16];
  if (n > 16 || c->n_expert_used > 32) return -1;
  for (int b = 0; b < n; b++) { /* router: F32 -> one vector at a time (:455-464) */
    if (or_matvec(&ly->router, xs[b], logits + b * ne)) return -1;
    nk[b] = route(c, logits + b * ne, probs, chosen[b], wts[b]);
    if (chosen_out) for (int i = 0; i < nk[b]; i++) chosen_out[b * 32 + i] = chosen[b][i];
    if (nkeep_out) nkeep_out[b] = nk[b];
  }
  if (n == 1) { /* moe_forward fused path: out.fill(0); ffns_fused */
    memset(outs[0], 0, dim * 4);
    int r = or_ffns_fused(&ly->gate, &ly->up, &ly->down, nk[0], chosen[0], wts[0], xs[0], outs[0]);
    free(logits); free(probs); return r;
  }
  /* moe_batch_fused (:648-766): users of each expert; a float expert with one user takes
   * the single-vector kernel (quant_multi.rs:240). Integer kernels are per-vector exact. */
  int users[512];
  memset(users, 0, sizeof users);
  for (int b = 0; b < n; b++) for (int i = 0; i < nk[b]; i++) users[chosen[b][i]]++;
  int int_gu = q8k_supports(&ly->gate) || q8k_supports(&ly->up), int_down = q8k_supports(&ly->down);
  float *h = malloc(sizeof(float) * nff), *t = malloc(sizeof(float) * nff), *y = malloc(sizeof(float) * dim);
  for (int b = 0; b < n; b++) {
    memset(outs[b], 0, dim * 4);
    q8k_buf xq = q8k_alloc(ly->gate.cols);
    if (int_gu) or_q8k_quantize(xs[b], ly->gate.cols, xq.d, xq.qs, xq.bs);
    for (int i = 0; i < nk[b]; i++) {
      int e = chosen[b][i];
      or_mat g = or_expert(ly->gate, e), u = or_expert(ly->up, e), d = or_expert(ly->down, e);
      int multi = users[e] > 1;
      if (q8k_supports(&g)) rows_into_q8k(&g, &xq, h, 0, nff);
      else if (multi) { const float *xv = xs[b]; or_matmul_rows_multi(g.data, g.dtype, g.cols, 2, (const float *const[]){xv, xv}, (float *const[]){h, t}, 0, nff); }
      else or_matvec_rows(g.data, g.dtype, g.cols, xs[b], h, 0, nff);
      if (q8k_supports(&u)) rows_into_q8k(&u, &xq, t, 0, nff);
      else if (multi) { const float *xv = xs[b]; float *tmp2 = malloc(sizeof(float) * nff); or_matmul_rows_multi(u.data, u.dtype, u.cols, 2, (const float *const[]){xv, xv}, (float *const[]){t, tmp2}, 0, nff); free(tmp2); }
      else or_matvec_rows(u.data, u.dtype, u.cols, xs[b], t, 0, nff);
      for (size_t r = 0; r < nff; r++) h[r] = or_silu(h[r]) * t[r];
      if (int_down) {
        q8k_buf hq = q8k_alloc(nff); or_q8k_quantize(h, nff, hq.d, hq.qs, hq.bs);
        rows_into_q8k(&d, &hq, y, 0, dim); q8k_free(hq);
      } else if (multi) { const float *hv = h; float *tmp2 = malloc(sizeof(float) * dim); or_matmul_rows_multi(d.data, d.dtype, d.cols, 2, (const float *const[]){hv, hv}, (float *const[]){y, tmp2}, 0, dim); free(tmp2); }
      else or_matvec_rows(d.data, d.dtype, d.cols, h, y, 0, dim);
      for (size_t r = 0; r < dim; r++) outs[b][r] += wts[b][i] * y[r]; /* :1133-1140 */
    }
    q8k_free(xq);
  }
  (void)int_gu;
  free(h); free(t); free(y); free(logits); free(probs);
  return 0;
}

/* ------------------------------------------------------------------ attention */
typedef struct {
  const or_model *m; int layer, pos; const float *q; float *out; float scale;
} attn_job;

static void attn_head(const attn_job *j, int h) { /* :3456-3495 */
  const or_config *c = &j->m->c;
  int hd = c->head_dim, kv_dim = c->n_kv_heads * hd, hpk = c->n_heads / c->n_kv_heads, kvh = h / hpk;
  const float *qh = j->q + (size_t)h * hd;
  float *oh = j->out + (size_t)h * hd;
  float mprev = -INFINITY, lprev = 0.0f, acc[256];
  for (int d = 0; d < hd; d++) acc[d] = 0.0f;
  for (int t = 0; t <= j->pos; t++) {
    size_t off = ((size_t)j->layer * c->max_seq + t) * kv_dim + (size_t)kvh * hd;
    const uint16_t *kh = j->m->k_cache + off, *vh = j->m->v_cache + off;
    float a8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (g_simd) { /* dot_f16_row_avx2: cvtph, fmadd over 8 lanes */
      __m256 av = _mm256_setzero_ps();
      for (int i = 0; i < hd; i += 8)
        av = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(kh + i))), _mm256_loadu_ps(qh + i), av);
      _mm256_storeu_ps(a8, av);
    } else {
      for (int i = 0; i < hd; i += 8)
        for (int l = 0; l < 8; l++) a8[l] = fmaf(or_f16_to_f32(kh[i + l]), qh[i + l], a8[l]);
    }
    float score = (hsum_hadd(a8) + 0.0f) * j->scale;
    float mnew = fmaxf(mprev, score);
    float alpha = expf(mprev - mnew), p = expf(score - mnew);
    lprev = lprev * alpha + p;
    mprev = mnew;
    if (g_simd) { /* acc = fmadd(p, v, acc * alpha) per 8 dims */
      __m256 va = _mm256_set1_ps(alpha), vp = _mm256_set1_ps(p);
      for (int d = 0; d < hd; d += 8)
        _mm256_storeu_ps(acc + d, _mm256_fmadd_ps(vp, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(vh + d))), _mm256_mul_ps(_mm256_loadu_ps(acc + d), va)));
    } else {
      for (int d = 0; d < hd; d++) acc[d] = fmaf(p, or_f16_to_f32(vh[d]), acc[d] * alpha);
    }
  }
  float invl = 1.0f / fmaxf(lprev, 1e-9f);
  for (int d = 0; d < hd; d++) oh[d] = acc[d] * invl;
}

static void attn_job_run(void *p, int t, int n) {
  attn_job *j = (attn_job *)p; int nh = j->m->c.n_heads;
  for (int h = nh * t / n; h < nh * (t + 1) / n; h++) attn_head(j, h);
}

static void attention(const or_model *m, int layer, int pos, const float *q, float *out) {
  const or_config *c = &m->c;
  attn_job j = {m, layer, pos, q, out, c->attn_scale > 0.0f ? c->attn_scale : 1.0f / sqrtf((float)c->head_dim)};
  if (g_threads > 1 && c->n_heads >= g_threads) run_pool(attn_job_run, &j); else attn_job_run(&j, 0, 1);
}

/* ------------------------------------------------------------------ model */
void or_model_init(or_model *m) {
  if (!m->inv_freq) m->inv_freq = malloc(sizeof(float) * (m->c.head_dim / 2 + 1));
  or_rope_inv_freq(m->c.head_dim, m->c.rope_theta, m->inv_freq);
}

static void embed_row(const or_model *m, int tok, float *x) {
  size_t rb = or_row_bytes(m->embed.dtype, m->c.dim);
  or_dequant_row(m->embed.dtype, m->embed.data + (size_t)tok * rb, m->c.dim, x);
  if (m->c.embedding_scale != 1.0f) for (int i = 0; i < m->c.dim; i++) x[i] *= m->c.embedding_scale;
}

static void add_bias(float *v, const float *b, size_t n) { if (b) for (size_t i = 0; i < n; i++) v[i] += b[i]; }

static void qkv_post(or_model *m, const or_layer *ly, int layer, int pos, float *q, float *k, float *v) {
  const or_config *c = &m->c;
  int q_dim = c->n_heads * c->head_dim, kv_dim = c->n_kv_heads * c->head_dim;
  add_bias(q, ly->q_bias, q_dim); add_bias(k, ly->k_bias, kv_dim); add_bias(v, ly->v_bias, kv_dim);
  if (ly->q_norm) { int nn = ly->qk_norm_full ? q_dim : c->head_dim; rmsnorm_heads_neox(q, ly->q_norm, q_dim, nn, c->rms_eps, c->rope_neox); }
  if (ly->k_norm) { int nn = ly->qk_norm_full ? kv_dim : c->head_dim; rmsnorm_heads_neox(k, ly->k_norm, kv_dim, nn, c->rms_eps, c->rope_neox); }
  or_rope_rotate(m->inv_freq, c->rope_neox, q, q_dim, c->head_dim, (float)pos);
  or_rope_rotate(m->inv_freq, c->rope_neox, k, kv_dim, c->head_dim, (float)pos);
  size_t off = ((size_t)layer * c->max_seq + pos) * kv_dim;
  for (int i = 0; i < kv_dim; i++) { m->k_cache[off + i] = or_f32_to_f16(k[i]); m->v_cache[off + i] = or_f32_to_f16(v[i]); }
}

int or_shift_kv(uint16_t *kc, uint16_t *vc, int n_layers, int max_seq, int kv_dim, int hd, int neox, const float *inv_freq,
                int n_keep, int n_discard, int cur_pos) {
  int n_ctx = cur_pos > n_keep ? cur_pos - n_keep : 0; /* :2944-2971 */
  if (n_discard > n_ctx) n_discard = n_ctx;
  if (n_discard <= 0) return cur_pos;
  int n_move = n_ctx - n_discard;
  float *tmp = malloc(sizeof(float) * kv_dim);
  for (int l = 0; l < n_layers; l++)
    for (int i = 0; i < n_move; i++) {
      size_t src = ((size_t)l * max_seq + n_keep + n_discard + i) * kv_dim, dst = ((size_t)l * max_seq + n_keep + i) * kv_dim;
      for (int j = 0; j < kv_dim; j++) tmp[j] = or_f16_to_f32(kc[src + j]);
      or_rope_rotate(inv_freq, neox, tmp, kv_dim, hd, -(float)n_discard);
      for (int j = 0; j < kv_dim; j++) kc[dst + j] = or_f32_to_f16(tmp[j]);
      memmove(vc + dst, vc + src, sizeof(uint16_t) * kv_dim);
    }
  free(tmp);
  return cur_pos - n_discard;
}

int or_ensure_kv_room(or_model *m, int n_keep, int cur_pos, int needed) {
  const or_config *c = &m->c;
  if (cur_pos + needed <= c->max_seq) return cur_pos; /* :2924-2940 */
  int n_ctx = cur_pos - n_keep, want = cur_pos + needed - c->max_seq;
  if (want < n_ctx / 2) want = n_ctx / 2;
  int n_discard = want < n_ctx ? want : n_ctx;
  if (!m->inv_freq) { m->inv_freq = malloc(sizeof(float) * (c->head_dim / 2 + 1)); or_rope_inv_freq(c->head_dim, c->rope_theta, m->inv_freq); }
  return or_shift_kv(m->k_cache, m->v_cache, c->n_layers, c->max_seq, c->n_kv_heads * c->head_dim, c->head_dim, c->rope_neox,
                     m->inv_freq, n_keep, n_discard, cur_pos);
}

/* qkv_post + attention for n rows at positions start..start+n-1 (forward_slice :3401-3495,
 * forward_batch_slice :3235-3319): bias, q/k norms and RoPE applied to q, k, v in place, the n
 * K/V rows written first, then row b attends over positions 0..start+b. */
int or_attn_rows(or_model *m, int layer, int n, int start, float *q, float *k, float *v, float *att) {
  const or_config *c = &m->c;
  const or_layer *ly = &m->layers[layer];
  int q_dim = c->n_heads * c->head_dim, kv_dim = c->n_kv_heads * c->head_dim;
  if (layer < 0 || layer >= c->n_layers || n < 1 || start < 0 || start + n > c->max_seq) return -1;
  for (int b = 0; b < n; b++) qkv_post(m, ly, layer, start + b, q + (size_t)b * q_dim, k + (size_t)b * kv_dim, v + (size_t)b * kv_dim);
  for (int b = 0; b < n; b++) attention(m, layer, start + b, q + (size_t)b * q_dim, att + (size_t)b * q_dim);
  return 0;
}

/* One layer on x [n][dim] in place: forward_slice's layer body for n == 1 (:3389-3548: matvec,
 * moe_forward / the fused dense FFN), forward_batch_slice's for n > 1 (:3190-3356:
 * matvec_multi, moe_forward_batch / ffn_forward_multi). */
int or_layer_forward(or_model *m, int l, int n, int start, float *x) {
  const or_config *c = &m->c;
  int dim = c->dim, q_dim = c->n_heads * c->head_dim, kv_dim = c->n_kv_heads * c->head_dim;
  if (l < 0 || l >= c->n_layers || n < 1 || n > 128 || start < 0 || start + n > c->max_seq) return -1;
  const or_layer *ly = &m->layers[l];
  float *xn = malloc(4 * (size_t)dim * n), *q = malloc(4 * (size_t)q_dim * n), *k = malloc(4 * (size_t)kv_dim * n),
        *v = malloc(4 * (size_t)kv_dim * n), *ao = malloc(4 * (size_t)q_dim * n), *proj = malloc(4 * (size_t)dim * n);
  const float *xr[128]; float *qr[128], *kr[128], *vr[128], *pr[128]; const float *ar[128];
  for (int b = 0; b < n; b++) {
    xr[b] = xn + (size_t)b * dim; qr[b] = q + (size_t)b * q_dim; kr[b] = k + (size_t)b * kv_dim;
    vr[b] = v + (size_t)b * kv_dim; pr[b] = proj + (size_t)b * dim; ar[b] = ao + (size_t)b * q_dim;
  }
  int rc = 0;
  for (int b = 0; b < n; b++) or_rmsnorm(x + (size_t)b * dim, ly->attn_norm, xn + (size_t)b * dim, dim, c->rms_eps);
  if (n == 1) { or_matvec(&ly->wq, xn, q); or_matvec(&ly->wk, xn, k); or_matvec(&ly->wv, xn, v); }
  else { or_matvec_multi(&ly->wq, n, xr, qr); or_matvec_multi(&ly->wk, n, xr, kr); or_matvec_multi(&ly->wv, n, xr, vr); }
  or_attn_rows(m, l, n, start, q, k, v, ao);
  if (n == 1) or_matvec(&ly->wo, ao, proj); else or_matvec_multi(&ly->wo, n, ar, pr);
  if (m->dbg_q) { memcpy(m->dbg_q, q, 4 * q_dim); memcpy(m->dbg_att, ao, 4 * q_dim); memcpy(m->dbg_proj, proj, 4 * dim); }
  for (int b = 0; b < n; b++) {
    float *xb = x + (size_t)b * dim;
    for (int i = 0; i < dim; i++) xb[i] += c->residual_scale * pr[b][i];
    or_rmsnorm(xb, ly->ffn_norm, xn + (size_t)b * dim, dim, c->rms_eps);
  }
  if (ly->is_moe) {
    if (n == 1) {
      const float *xs[1] = {xn}; float *os[1] = {proj};
      rc = or_moe_forward(c, ly, 1, xs, os, m->last_chosen, NULL);
    } else if (n > 16) { /* MoE batches above 16 rows: split (per-row results do not depend on it) */
      for (int s0 = 0; s0 < n && !rc; s0 += 16) { int cnt = n - s0 < 16 ? n - s0 : 16; rc = or_moe_forward(c, ly, cnt, xr + s0, pr + s0, NULL, NULL); }
    } else rc = or_moe_forward(c, ly, n, xr, pr, m->last_chosen, NULL);
  } else if (n == 1) { /* ffn_forward :590-614: the fused job with k = 1, w = 1 */
    int e0 = 0; float w1 = 1.0f;
    memset(proj, 0, 4 * dim);
    or_ffns_fused(&ly->gate, &ly->up, &ly->down, 1, &e0, &w1, xn, proj);
  } else { /* ffn_forward_multi :616-646 */
    int nff = (int)ly->gate.rows;
    float *g = malloc(4 * (size_t)nff * n), *u = malloc(4 * (size_t)nff * n);
    float *gr[128], *ur[128]; const float *gc[128];
    for (int b = 0; b < n; b++) { gr[b] = g + (size_t)b * nff; ur[b] = u + (size_t)b * nff; gc[b] = gr[b]; }
    or_matvec_multi(&ly->gate, n, xr, gr); or_matvec_multi(&ly->up, n, xr, ur);
    for (size_t i = 0; i < (size_t)nff * n; i++) g[i] = or_silu(g[i]) * u[i];
    or_matvec_multi(&ly->down, n, gc, pr);
    free(g); free(u);
  }
  if (m->dbg_ffn) memcpy(m->dbg_ffn, proj, 4 * dim);
  for (int b = 0; b < n; b++) {
    float *xb = x + (size_t)b * dim;
    for (int i = 0; i < dim; i++) xb[i] += c->residual_scale * pr[b][i];
  }
  free(xn); free(q); free(k); free(v); free(ao); free(proj);
  return rc;
}

int or_forward_slice(or_model *m, int token, int pos, float *hidden) {
  const or_config *c = &m->c;
  if (pos < 0 || pos >= c->max_seq || token < 0 || token >= c->vocab) return -1;
  float *x = malloc(4 * (size_t)c->dim);
  embed_row(m, token, x);
  int rc = 0;
  for (int l = 0; l < c->n_layers && !rc; l++) rc = or_layer_forward(m, l, 1, pos, x);
  if (!rc) or_rmsnorm(x, m->output_norm, hidden, c->dim, c->rms_eps);
  free(x);
  return rc;
}

int or_forward_batch(or_model *m, const int *ids, int n, int start, float *hidden) {
  if (n == 1) return or_forward_slice(m, ids[0], start, hidden);
  const or_config *c = &m->c;
  int dim = c->dim;
  if (n < 1 || n > 128 || start < 0 || start + n > c->max_seq) return -1;
  for (int b = 0; b < n; b++)
    if (ids[b] < 0 || ids[b] >= c->vocab) return -1;
  float *x = malloc(4 * (size_t)dim * n);
  for (int b = 0; b < n; b++) embed_row(m, ids[b], x + (size_t)b * dim);
  int rc = 0;
  for (int l = 0; l < c->n_layers && !rc; l++) rc = or_layer_forward(m, l, n, start, x);
  if (!rc)
    for (int b = 0; b < n; b++) or_rmsnorm(x + (size_t)b * dim, m->output_norm, hidden + (size_t)b * dim, dim, c->rms_eps);
  free(x);
  return rc;
}

int or_logits(or_model *m, const float *hidden, int n, float *logits) {
  const float *xs[128]; float *os[128];
  if (n > 128) return -1;
  for (int b = 0; b < n; b++) { xs[b] = hidden + (size_t)b * m->c.dim; os[b] = logits + (size_t)b * m->c.vocab; }
  return or_matvec_multi(&m->lm_head, n, xs, os);
}

static inline int32_t total_key(float f) { /* f32::total_cmp ordering key */
  int32_t i; memcpy(&i, &f, 4); return i ^ (int32_t)(((uint32_t)(i >> 31)) >> 1);
}

int or_argmax(const float *logits, int n, float logit_scale) {
  int best = 0; int32_t bk = 0;
  for (int i = 0; i < n; i++) {
    float v = logit_scale != 1.0f ? logits[i] / logit_scale : logits[i];
    int32_t k = total_key(v);
    if (i == 0 || k >= bk) { bk = k; best = i; } /* max_by keeps the last maximum */
  }
  return best;
}

/* ------------------------------------------------------------------ sampling */
uint64_t or_splitmix_next(uint64_t *x) { /* SplitMix64::next_u64 :1560-1566 */
  uint64_t z = (*x += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

float or_splitmix_f32(uint64_t *x) { /* next_f32 :1569-1571: top 24 bits / 2^24 */
  return (float)(or_splitmix_next(x) >> 40) / (float)(1u << 24);
}

void or_sampler_init(or_sampler *s, const or_sampler_params *p) { s->p = *p; s->rng = p->seed; }

static int argmax_total(const float *l, int n) { /* max_by(total_cmp): the last maximum */
  int best = 0; int32_t bk = 0;
  for (int i = 0; i < n; i++) { int32_t k = total_key(l[i]); if (i == 0 || k >= bk) { bk = k; best = i; } }
  return best;
}

static const float *g_sort_l;
static int cand_cmp(const void *a, const void *b) { /* total_cmp descending, then index ascending */
  int i = *(const int *)a, j = *(const int *)b;
  int32_t ki = total_key(g_sort_l[i]), kj = total_key(g_sort_l[j]);
  if (ki != kj) return ki > kj ? -1 : 1;
  return i < j ? -1 : i > j;
}

int or_sample(or_sampler *S, const float *in, int V, float lscale, const int *recent, int nr, int forbid_stop, int forbid_think) {
  const or_sampler_params *sc = &S->p;
  float *l = malloc(sizeof(float) * V);
  for (int i = 0; i < V; i++) l[i] = lscale != 1.0f ? in[i] / lscale : in[i];  /* :3626-3628 */
  if (sc->repeat_penalty != 1.0f) {  /* :3631-3646, each distinct recent token once */
    unsigned char *seen = calloc(V, 1);
    for (int i = 0; i < nr; i++) {
      int t = recent[i];
      if (t < 0 || t >= V || seen[t]) continue;
      seen[t] = 1;
      l[t] = l[t] > 0.0f ? l[t] / sc->repeat_penalty : l[t] * sc->repeat_penalty;
    }
    free(seen);
  }
  if (forbid_stop)
    for (int i = 0; i < sc->n_stop; i++)
      if (sc->stop_ids[i] >= 0 && sc->stop_ids[i] < V) l[sc->stop_ids[i]] = -INFINITY;
  if (forbid_think && sc->think_open >= 0 && sc->think_open < V) l[sc->think_open] = -INFINITY;
  int tok;
  if (sc->temperature <= 0.0f) { tok = argmax_total(l, V); free(l); return tok; }
  int *cand = malloc(sizeof(int) * V), n = 0;  /* finite candidates :3671 */
  for (int i = 0; i < V; i++) if (isfinite(l[i])) cand[n++] = i;
  int k = sc->top_k == 0 ? n : (sc->top_k < n ? sc->top_k : n);
  if (k == 0) { tok = argmax_total(l, V); free(cand); free(l); return tok; }
  g_sort_l = l;
  qsort(cand, n, sizeof(int), cand_cmp);  /* select_nth_unstable + sort_unstable :3677-3681 */
  float *pr = malloc(sizeof(float) * k), mx = l[cand[0]], sum = 0.0f;
  for (int i = 0; i < k; i++) pr[i] = expf((l[cand[i]] - mx) / sc->temperature);  /* :3684-3699 */
  for (int i = 0; i < k; i++) sum += pr[i];
  for (int i = 0; i < k; i++) pr[i] /= sum;
  float floor_ = sc->min_p * pr[0];  /* min-p, then top-p :3702-3711 */
  int keep = 0;
  while (keep < k && pr[keep] >= floor_) keep++;
  if (keep < 1) keep = 1;
  float cum = 0.0f;
  for (int i = 0; i < keep; i++) { cum += pr[i]; if (cum >= sc->top_p) { keep = i + 1; break; } }
  float total = 0.0f;  /* :3714-3725 */
  for (int i = 0; i < keep; i++) total += pr[i];
  float r = or_splitmix_f32(&S->rng) * total;
  tok = cand[keep - 1];
  for (int i = 0; i < keep; i++) { r -= pr[i]; if (r <= 0.0f) { tok = cand[i]; break; } }
  free(pr); free(cand); free(l);
  return tok;
}

/* ------------------------------------------------------------------ speculation */
int or_lookup_draft(const int *c, int n, int k, const int *stop, int n_stop, int min_ng, int max_ng, int *draft, int *ngram) {
  /* lookup_draft smollm_chat.rs:2982-3015 */
  *ngram = 0;
  if (k == 0) return 0;
  for (int ng = max_ng; ng >= min_ng; ng--) {
    if (n <= ng) continue;
    const int *pat = c + n - ng;
    int i = n - ng;
    while (i > 0) {
      i--;
      if (c[i + ng - 1] == pat[ng - 1] && memcmp(c + i, pat, sizeof(int) * ng) == 0) {
        int s = i + ng, kk = ng == 2 ? (k < 2 ? k : 2) : k; /* LOOKUP_MIN_NGRAM = 2 */
        int e = s + kk < n ? s + kk : n, len = 0;
        for (int j = s; j < e; j++) {
          int is_stop = 0;
          for (int q = 0; q < n_stop; q++) if (stop[q] == c[j]) is_stop = 1;
          if (is_stop) break;
          draft[len++] = c[j];
        }
        if (len > 0) { *ngram = ng; return len; }
      }
    }
  }
  return 0;
}

void or_spec_init(or_spec_model *s, int fixed) { /* SpecModel::default :1700-1713 */
  for (int i = 0; i < 4; i++) { s->acc[i] = 1.0; s->fail[i] = 1.0; }
  s->t1_us = 100000.0; s->extra_us = 30000.0; s->have_t1 = 0; s->have_extra = 0; s->since_try = 0; s->fixed = fixed;
}
int or_spec_class(int ng) { return ng == 0 ? 3 : ng <= 2 ? 0 : ng == 3 ? 1 : 2; }
double or_spec_accept_rate(const or_spec_model *s, int c) { return s->acc[c] / (s->acc[c] + s->fail[c]); }
static double spec_cost(const or_spec_model *s, int b) { return s->t1_us + s->extra_us * (double)(b > 1 ? b - 1 : 0); }
int or_spec_best_len(or_spec_model *s, int c, int avail) { /* :1728-1753 */
  if (s->fixed || avail == 0) return avail;
  double p = or_spec_accept_rate(s, c), best_rate = 1.0 / spec_cost(s, 1), gain = 1.0, pk = 1.0;
  int best = 0;
  for (int k = 1; k <= avail; k++) {
    pk *= p; gain += pk;
    double rate = gain / spec_cost(s, k + 1);
    if (rate > best_rate) { best_rate = rate; best = k; }
  }
  if (best == 0) {
    s->since_try++;
    if (s->since_try >= 24) { s->since_try = 0; return avail < 2 ? avail : 2; }
  }
  return best;
}
void or_spec_reset_rates(or_spec_model *s) { /* :1756-1760 */
  for (int i = 0; i < 4; i++) { s->acc[i] = 1.0; s->fail[i] = 1.0; }
  s->since_try = 0;
}
void or_spec_record_draft(or_spec_model *s, int c, int drafted, int accepted) { /* :1763-1775 */
  for (int i = 0; i < 4; i++) { s->acc[i] = fmax(s->acc[i] * 0.97, 0.5); s->fail[i] = fmax(s->fail[i] * 0.97, 0.5); }
  s->acc[c] += accepted;
  if (accepted < drafted) s->fail[c] += 1.0;
}
void or_spec_record_step(or_spec_model *s, uint64_t us) { /* :1778-1786 */
  double u = (double)us;
  s->t1_us = s->have_t1 ? 0.9 * s->t1_us + 0.1 * u : u;
  if (!s->have_extra) s->extra_us = 0.3 * s->t1_us;
  s->have_t1 = 1;
}
void or_spec_record_verify(or_spec_model *s, int b, uint64_t us) { /* :1789-1799 */
  if (b < 2 || !s->have_t1) return;
  double m = ((double)us - s->t1_us) / (double)(b - 1);
  if (m < 0.0) m = 0.0;
  if (m > 1.5 * s->t1_us) m = 1.5 * s->t1_us;
  s->extra_us = s->have_extra ? 0.85 * s->extra_us + 0.15 * m : m;
  s->have_extra = 1;
}

static uint64_t now_us(void) { struct timespec ts; clock_gettime(CLOCK_MONOTONIC, &ts); return (uint64_t)ts.tv_sec * 1000000u + ts.tv_nsec / 1000; }

#define CORPUS_MAX (16 * 1024) /* LOOKUP_CORPUS_MAX :28 */
static void remember(int *corpus, int *n, const int *ids, int cnt) { /* :2973-2980 */
  for (int i = 0; i < cnt; i++) corpus[(*n)++] = ids[i];
  if (*n > CORPUS_MAX) { int drop = *n - CORPUS_MAX / 2; memmove(corpus, corpus + drop, sizeof(int) * (*n - drop)); *n -= drop; }
}

/* One token for row `row` of the pass's logits: the sampler's, or greedy (argmax after
 * logit_scale) without one. */
static int gen_pick(or_model *m, or_sampler *sp, const float *logits, const int *out, int gen) {
  if (!sp) return or_argmax(logits, m->c.vocab, m->c.logit_scale);
  return or_sample(sp, logits, m->c.vocab, m->c.logit_scale, out, gen, gen < 2, 0);  /* :4220, 4292, 4311 */
}

static int is_stop(const or_sampler *sp, int t) {
  if (!sp) return 0;
  for (int i = 0; i < sp->p.n_stop; i++) if (sp->p.stop_ids[i] == t) return 1;
  return 0;
}

int or_generate(or_model *m, const int *prompt, int n_prompt, int max_new, const or_gen_params *p, int *out, or_gen_stats *st) {
  return or_generate_sampled(m, prompt, n_prompt, max_new, p, NULL, out, st);
}

int or_generate_sampled(or_model *m, const int *prompt, int n_prompt, int max_new, const or_gen_params *p,
                        or_sampler *sp, int *out, or_gen_stats *st) {
  return or_generate_full(m, NULL, prompt, n_prompt, max_new, p, sp, out, st);
}

int or_generate_full(or_model *m, or_model *dm, const int *prompt, int n_prompt, int max_new, const or_gen_params *p,
                     or_sampler *sp, int *out, or_gen_stats *st) {
  const or_config *c = &m->c;
  int dim = c->dim, vocab = c->vocab, chunk = p->prefill_chunk > 0 ? p->prefill_chunk : 128;
  const int *stop = sp ? sp->p.stop_ids : NULL, n_stop = sp ? sp->p.n_stop : 0;
  memset(st, 0, sizeof *st);
  if (p->n_cached < 0 || p->n_cached >= n_prompt || p->kv_keep < 0 || p->kv_keep + chunk + 16 > c->max_seq) return -1;
  int *corpus = malloc(sizeof(int) * (CORPUS_MAX + n_prompt + 64)), nc = 0;
  float *hid = malloc(sizeof(float) * dim * 17), *logits = malloc(sizeof(float) * (size_t)vocab * 17);
  remember(corpus, &nc, prompt, n_prompt);
  int pos = p->n_cached;
  /* feed :3041-3104 (chunks; a chunk of one token goes through forward_slice) */
  float *hbuf = malloc(sizeof(float) * (size_t)dim * chunk);
  for (int s = p->n_cached; s < n_prompt; s += chunk) {
    int cnt = n_prompt - s < chunk ? n_prompt - s : chunk;
    pos = or_ensure_kv_room(m, p->kv_keep, pos, cnt); /* feed :3089-3090 */
    if (or_forward_batch(m, prompt + s, cnt, pos, hbuf)) return -1;
    memcpy(hid, hbuf + (size_t)(cnt - 1) * dim, 4 * dim);
    pos += cnt;
  }
  /* the draft model is fed the same turn (:4141-4143) */
  int d_pos = p->n_cached, shifted = 0;
  float *dhid = dm ? malloc(sizeof(float) * dm->c.dim * 17) : NULL, *dlog = dm ? malloc(sizeof(float) * (size_t)dm->c.vocab) : NULL;
  if (dm) {
    for (int s = p->n_cached; s < n_prompt; s += chunk) {
      int cnt = n_prompt - s < chunk ? n_prompt - s : chunk;
      d_pos = or_ensure_kv_room(dm, p->kv_keep, d_pos, cnt);
      if (or_forward_batch(dm, prompt + s, cnt, d_pos, hbuf)) return -1;
      d_pos += cnt;
    }
  }
  free(hbuf);
  int reply_start = pos;
  or_logits(m, hid, 1, logits);
  int gen = 0, tok = gen_pick(m, sp, logits, out, gen);
  or_spec_model sm; or_spec_init(&sm, p->fixed);
  int backoff = 0, skip = 0, k_dyn = p->draft_len;
  for (;;) {
    if (is_stop(sp, tok)) break;                                  /* :4226 */
    out[gen++] = tok; remember(corpus, &nc, &tok, 1);           /* emit! */
    if (gen >= max_new) break;
    int budget = max_new - gen, k = k_dyn < budget - 1 ? k_dyn : budget - 1;
    int draft[64], nd = 0, cls = 3, use_lookup = p->speculate && !dm;
    if (k > 0 && (skip == 0 || use_lookup)) {
      if (dm) { /* draft_engine :4244-4269, greedy draft picks */
        if (!shifted && d_pos >= reply_start) {
          int have = 0, dshift = 0, from = d_pos - reply_start < gen ? d_pos - reply_start : gen;
          for (int i = from; i < gen; i++) {
            int np = or_ensure_kv_room(dm, p->kv_keep, d_pos, 1);
            if (np < d_pos) dshift = 1;
            d_pos = np;
            if (or_forward_slice(dm, out[i], d_pos, dhid)) return -1;
            d_pos++; have = 1;
          }
          for (int j = 0; have && !dshift && j < k; j++) {
            or_logits(dm, dhid, 1, dlog);
            int x = or_argmax(dlog, dm->c.vocab, dm->c.logit_scale);
            draft[nd++] = x;
            if (j + 1 < k) {
              int np = or_ensure_kv_room(dm, p->kv_keep, d_pos, 1);
              if (np < d_pos) dshift = 1;
              d_pos = np;
              if (or_forward_slice(dm, x, d_pos, dhid)) return -1;
              d_pos++;
            }
          }
          if (dshift) { nd = 0; shifted = 1; }
        }
      } else if (use_lookup) {
        int d[64], ng = 0, len = or_lookup_draft(corpus, nc, k, stop, n_stop, p->min_ngram, p->max_ngram, d, &ng);
        if (skip == 0 || ng > 2) /* weak = 2-gram (:4274) */ { memcpy(draft, d, sizeof(int) * len); nd = len; cls = or_spec_class(ng); }
      }
    }
    nd = or_spec_best_len(&sm, cls, nd);
    if (skip > 0) skip--;
    if (nd == 0) {
      { int np = or_ensure_kv_room(m, p->kv_keep, pos, 1); if (np < pos) shifted = 1; pos = np; } /* :4283 */
      uint64_t t0 = now_us();
      if (or_forward_slice(m, tok, pos, hid)) return -1;
      pos++;
      or_logits(m, hid, 1, logits);
      tok = gen_pick(m, sp, logits, out, gen);
      or_spec_record_step(&sm, now_us() - t0);
      st->steps++;
      continue;
    }
    int batch[65]; batch[0] = tok; memcpy(batch + 1, draft, sizeof(int) * nd);
    { int np = or_ensure_kv_room(m, p->kv_keep, pos, nd + 1); if (np < pos) shifted = 1; pos = np; } /* :4298 */
    int start = pos; uint64_t t0 = now_us();
    if (or_forward_batch(m, batch, nd + 1, start, hid)) return -1;
    or_logits(m, hid, nd + 1, logits);
    or_spec_record_verify(&sm, nd + 1, now_us() - t0);
    st->drafted += nd; st->verifies++;
    int accepted = 0, correction = -1, done = 0;
    for (int i = 0; i < nd; i++) {
      int s = gen_pick(m, sp, logits + (size_t)i * vocab, out, gen);
      if (s != draft[i]) { correction = s; break; }
      accepted++;
      out[gen++] = s; remember(corpus, &nc, &s, 1);
      if (gen >= max_new) { done = 1; break; }
    }
    st->accepted += accepted;
    or_spec_record_draft(&sm, cls, nd, accepted);
    pos = start + 1 + accepted;
    if (dm && d_pos > reply_start + gen) d_pos = reply_start + gen; /* :4334-4336 */
    if (done) break;
    if (accepted == 0) { backoff = backoff * 2; if (backoff < 1) backoff = 1; if (backoff > 16) backoff = 16; skip = backoff; }
    else backoff = 0;
    if (p->adaptive_k) {
      if (accepted == nd) { int kk = k_dyn + 2 < 7 ? k_dyn + 2 : 7; k_dyn = kk > p->draft_len ? kk : p->draft_len; }
      else k_dyn = p->draft_len;
    }
    tok = correction >= 0 ? correction : gen_pick(m, sp, logits + (size_t)nd * vocab, out, gen);
  }
  free(corpus); free(hid); free(logits); free(dhid); free(dlog);
  return gen;
}
