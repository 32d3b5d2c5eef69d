// C ABI: context, weight tensors (planar re-layout), Q8_K quantization and matvec entry points.
#include <string.h>

#include <algorithm>
#include <cstdlib>
#include <functional>
#include <mutex>
#include <thread>

#include "../../include/spx.h"
#include "decode.h"
#include "fused.h"
#include "internal.h"

namespace spx {

static thread_local std::string g_err;

void set_error(const std::string &msg) { g_err = msg; }
int fail(const std::string &msg) { g_err = msg; return -1; }
int hip_fail(hipError_t e, const char *what) {
  g_err = std::string(what) + ": " + hipGetErrorString(e);
  return -2;
}

int64_t block_elems(int dtype) {
  switch (dtype) {
  case T_F32: case T_F16: return 1;
  case T_Q5_0: case T_Q8_0: return 32;
  case T_Q4K: case T_Q5K: case T_Q6K: return 256;
  default: return 0;
  }
}

int64_t row_bytes(int dtype, int64_t cols) {
  int64_t be = block_elems(dtype), bb;
  switch (dtype) {
  case T_F32: bb = 4; break;
  case T_F16: bb = 2; break;
  case T_Q5_0: bb = 22; break;
  case T_Q8_0: bb = 34; break;
  case T_Q4K: bb = 144; break;
  case T_Q5K: bb = 176; break;
  case T_Q6K: bb = 210; break;
  default: return 0;
  }
  if (cols <= 0 || cols % be) return 0;
  return cols / be * bb;
}

void *ws_get(spx_ctx *ctx, size_t bytes) {
  if (bytes <= ctx->ws_bytes) return ctx->ws;
  if (ctx->ws) { (void)hipStreamSynchronize(ctx->stream); (void)hipFree(ctx->ws); }
  ctx->ws = nullptr;
  ctx->ws_bytes = 0;
  size_t want = std::max(bytes, (size_t)1 << 20);
  if (hipMalloc(&ctx->ws, want) != hipSuccess) return nullptr;
  ctx->ws_bytes = want;
  return ctx->ws;
}

// Fixed scratch for spx_matvec_noalloc: the permuted Q8_K image of its activations. Each device
// the library runs on holds one copy until the process ends; every call on that device shares
// it (calls that overlap on one device race).
static __device__ __align__(256) uint8_t g_noalloc_scratch[SPX_NOALLOC_SCRATCH_BYTES];
// Per device, the event recorded after the last call's kernels: the next call, from any context
// (each has its own stream), waits for it before it writes the array, so calls from different
// streams take turns instead of overwriting each other's staging. Created once per device (an
// event holds no device memory) and kept until the process ends.
constexpr int NOALLOC_MAX_DEV = 64;
static std::mutex g_noalloc_mu;
static hipEvent_t g_noalloc_ev[NOALLOC_MAX_DEV];
static bool g_noalloc_used[NOALLOC_MAX_DEV];

// Layout of m permuted Q8_K vectors of n columns in one buffer (codes, d, bsum pairs; each
// region 256-byte aligned); total bytes in *bytes.
static Q8KP q8kp_layout(uint8_t *base, int m, int64_t n, size_t *bytes) {
  const int64_t nb = n / 256;
  const size_t qb = ((size_t)m * n + 255) & ~(size_t)255, db = ((size_t)m * nb * 4 + 255) & ~(size_t)255;
  *bytes = qb + db + (size_t)m * nb * 64;
  Q8KP r{};
  r.q = reinterpret_cast<uint32_t *>(base);
  r.d = reinterpret_cast<float *>(base + qb);
  r.bs = reinterpret_cast<int2 *>(base + qb + db);
  return r;
}

// Field records of one GGUF block: (offset in block, length, plane).
struct Field { int off, len, plane; };
static int fields_of(int dtype, Field *f) {
  switch (dtype) {
  case T_Q4K: f[0] = {16, 128, 0}; f[1] = {0, 16, 1}; return 2;
  case T_Q6K: f[0] = {0, 128, 0}; f[1] = {128, 64, 1}; f[2] = {192, 16, 2}; f[3] = {208, 2, 3}; return 4;
  case T_Q8_0: f[0] = {2, 32, 0}; f[1] = {0, 2, 3}; return 2;
  case T_Q5_0: f[0] = {6, 16, 0}; f[1] = {2, 4, 1}; f[2] = {0, 2, 3}; return 3;
  case T_Q5K: f[0] = {48, 128, 0}; f[1] = {16, 32, 1}; f[2] = {0, 16, 2}; return 3;
  default: return 0;
  }
}
static int block_bytes(int dtype) {
  switch (dtype) { case T_Q4K: return 144; case T_Q5K: return 176; case T_Q6K: return 210; case T_Q8_0: return 34; case T_Q5_0: return 22; default: return 0; }
}

// Byte order inside one plane record: device position of GGUF byte b of the field, so that
// the eight lanes of a row group each load one contiguous piece (16 B of codes):
//   Q4_K codes  qs[32c + 4l + j]        -> 16l + 4c + j      (lane l: dword c, c = 0..3)
//   Q6_K ql     ql[64h + 32mm + 4l + j] -> 16l + 8h + 4mm + j
//   Q6_K qh     qh[32h + 4l + j]        -> 8l + 4h + j
//   Q5_K codes  qs[32c + 8k + l]        -> 16l + 4c + k      (lane l: elements 8k + l of each 32)
//   Q5_K qh     qh[8k + l]              -> 4l + k
// Every other field keeps the GGUF order.
static int perm_of(int dtype, int plane, int b) {
  if (dtype == T_Q4K && plane == 0) { const int c = b >> 5, l = (b >> 2) & 7, j = b & 3; return 16 * l + 4 * c + j; }
  if (dtype == T_Q6K && plane == 0) { const int h = b >> 6, mm = (b >> 5) & 1, l = (b >> 2) & 7, j = b & 3; return 16 * l + 8 * h + 4 * mm + j; }
  if (dtype == T_Q6K && plane == 1) { const int h = b >> 5, l = (b >> 2) & 7, j = b & 3; return 8 * l + 4 * h + j; }
  if (dtype == T_Q5K && plane == 0) { const int c = b >> 5, k = (b >> 3) & 3, l = b & 7; return 16 * l + 4 * c + k; }
  if (dtype == T_Q5K && plane == 1) { const int k = b >> 3, l = b & 7; return 4 * l + k; }
  return b;
}

// GGUF <-> planar, over block range [g0, g1).
static void relayout(int dtype, const uint8_t *ggml, uint8_t *planar, const size_t *poff, int64_t g0, int64_t g1, bool to_planar) {
  Field f[4];
  const int nf = fields_of(dtype, f), bb = block_bytes(dtype);
  int perm[4][128];
  bool permuted[4] = {false, false, false, false};
  for (int k = 0; k < nf; k++)
    for (int b = 0; b < f[k].len && b < 128; b++) {
      perm[k][b] = perm_of(dtype, f[k].plane, b);
      permuted[k] |= perm[k][b] != b;
    }
  for (int64_t g = g0; g < g1; g++)
    for (int k = 0; k < nf; k++) {
      uint8_t *p = planar + poff[f[k].plane] + (size_t)g * f[k].len;
      uint8_t *q = const_cast<uint8_t *>(ggml) + (size_t)g * bb + f[k].off;
      if (!permuted[k]) {
        if (to_planar) memcpy(p, q, f[k].len); else memcpy(q, p, f[k].len);
      } else if (to_planar) {
        for (int b = 0; b < f[k].len; b++) p[perm[k][b]] = q[b];
      } else {
        for (int b = 0; b < f[k].len; b++) q[b] = p[perm[k][b]];
      }
    }
}

static void parallel_blocks(int64_t nblk, const std::function<void(int64_t, int64_t)> &fn) {
  const int64_t min_per = 1 << 16;
  int nt = (int)std::min<int64_t>(std::max(1u, std::thread::hardware_concurrency()), std::max<int64_t>(1, nblk / min_per));
  nt = std::min(nt, 16);
  if (nt <= 1) { fn(0, nblk); return; }
  std::vector<std::thread> th;
  for (int t = 0; t < nt; t++) th.emplace_back([&, t] { fn(nblk * t / nt, nblk * (t + 1) / nt); });
  for (auto &x : th) x.join();
}

}  // namespace spx

using namespace spx;

extern "C" {

const char *spx_last_error(void) { return g_err.c_str(); }

int spx_create(int device, spx_ctx **out) {
  if (!out) return fail("spx_create: out is null");
  int n = 0;
  SPX_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail("spx_create: no such device");
  SPX_HIP(hipSetDevice(device));
  spx_ctx *c = new spx_ctx();
  c->device = device;
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) { delete c; return hip_fail(e, "hipStreamCreate"); }
  // this device's address of the fixed scratch array (the host-side name is not a device address)
  e = hipGetSymbolAddress(reinterpret_cast<void **>(&c->scratch), HIP_SYMBOL(g_noalloc_scratch));
  if (e != hipSuccess) {
    (void)hipStreamDestroy(c->stream);
    delete c;
    return hip_fail(e, "hipGetSymbolAddress(scratch)");
  }
  if (device < NOALLOC_MAX_DEV) {
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ev[device]) {
      e = hipEventCreateWithFlags(&g_noalloc_ev[device], hipEventDisableTiming);
      if (e != hipSuccess) {
        g_noalloc_ev[device] = nullptr;
        (void)hipStreamDestroy(c->stream);
        delete c;
        return hip_fail(e, "hipEventCreate(scratch turn)");
      }
    }
  }
  *out = c;
  return 0;
}

int spx_destroy(spx_ctx *ctx) {
  if (!ctx) return 0;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->ws) (void)hipFree(ctx->ws);
  if (ctx->moe_pin) (void)hipHostFree(ctx->moe_pin);
  if (ctx->moe_ev) (void)hipEventDestroy(ctx->moe_ev);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return 0;
}

int spx_sync(spx_ctx *ctx) {
  if (!ctx) return fail("spx_sync: null context");
  SPX_HIP(hipStreamSynchronize(ctx->stream));
  return 0;
}

void *spx_get_stream(spx_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int64_t spx_row_bytes(int dtype, int64_t cols) { return row_bytes(dtype, cols); }

int spx_tensor_upload(spx_ctx *ctx, int dtype, int64_t cols, int64_t rows, int n_expert, const void *ggml, spx_tensor **out) {
  if (!ctx || !out || !ggml) return fail("spx_tensor_upload: null argument");
  const int64_t rb = row_bytes(dtype, cols);
  if (!rb || rows <= 0 || n_expert <= 0) return fail("spx_tensor_upload: unsupported dtype or shape (dtype " + std::to_string(dtype) + ", cols " + std::to_string(cols) + ")");
  SPX_HIP(hipSetDevice(ctx->device));
  spx_tensor *t = new spx_tensor();
  t->v.dtype = dtype;
  t->v.cols = cols;
  t->v.rows = rows;
  t->v.n_expert = n_expert;
  t->v.nb = cols / block_elems(dtype);
  const int64_t total_rows = rows * n_expert, nblk = total_rows * t->v.nb;
  std::vector<uint8_t> img;
  size_t bytes = 0;
  if (dtype == T_F32 || dtype == T_F16) {
    bytes = (size_t)rb * total_rows;
    t->plane_off[0] = 0;
  } else {
    Field f[4];
    const int nf = fields_of(dtype, f);
    for (int k = 0; k < nf; k++) {
      t->plane_off[f[k].plane] = bytes;
      bytes += (((size_t)nblk * f[k].len + 255) & ~(size_t)255) + 256;  // slack: 16-byte loads may run past a plane's end
    }
    if (dtype == T_Q4K) {  // derived plane 2: scales and mins unpacked to bytes (below)
      t->plane_off[2] = bytes;
      bytes += (((size_t)nblk * 16 + 255) & ~(size_t)255) + 256;
    }
  }
  hipError_t e = hipMalloc(&t->dev, std::max<size_t>(bytes, 256));
  if (e != hipSuccess) { delete t; return hip_fail(e, "hipMalloc(tensor)"); }
  t->bytes = bytes;
  const uint8_t *src = static_cast<const uint8_t *>(ggml);
  if (dtype == T_F32 || dtype == T_F16) {
    e = hipMemcpy(t->dev, src, bytes, hipMemcpyHostToDevice);
  } else {
    img.resize(bytes);
    parallel_blocks(nblk, [&](int64_t a, int64_t b) { relayout(dtype, src, img.data(), t->plane_off, a, b, true); });
    if (dtype == T_Q4K) {
      // sc[0..7], mn[0..7] of each block as bytes (unpack_q4k_scales, q4k_gemv.rs:70-85), read
      // by the multi-row MFMA kernels; a copy of the header's information, so download ignores it
      parallel_blocks(nblk, [&](int64_t a0, int64_t a1) {
        for (int64_t g = a0; g < a1; g++) {
          const uint8_t *sc = src + (size_t)g * 144 + 4;
          uint8_t *o = img.data() + t->plane_off[2] + (size_t)g * 16;
          for (int k = 0; k < 4; k++) {
            o[k] = sc[k] & 63;
            o[4 + k] = (uint8_t)((sc[8 + k] & 15) | ((sc[k] >> 6) << 4));
            o[8 + k] = sc[4 + k] & 63;
            o[12 + k] = (uint8_t)((sc[8 + k] >> 4) | ((sc[4 + k] >> 6) << 4));
          }
        }
      });
    }
    e = hipMemcpy(t->dev, img.data(), bytes, hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) { (void)hipFree(t->dev); delete t; return hip_fail(e, "hipMemcpy(tensor)"); }
  uint8_t *base = static_cast<uint8_t *>(t->dev);
  t->v.pl.p0 = base + t->plane_off[0];
  t->v.pl.p1 = base + t->plane_off[1];
  t->v.pl.p2 = base + t->plane_off[2];
  t->v.pl.p3 = base + t->plane_off[3];
  *out = t;
  return 0;
}

int spx_tensor_download(spx_ctx *ctx, const spx_tensor *t, void *ggml) {
  if (!ctx || !t || !ggml) return fail("spx_tensor_download: null argument");
  SPX_HIP(hipSetDevice(ctx->device));
  SPX_HIP(hipStreamSynchronize(ctx->stream));
  const int dtype = t->v.dtype;
  const int64_t nblk = t->v.rows * t->v.n_expert * t->v.nb;
  if (dtype == T_F32 || dtype == T_F16) {
    SPX_HIP(hipMemcpy(ggml, t->dev, t->bytes, hipMemcpyDeviceToHost));
    return 0;
  }
  std::vector<uint8_t> img(t->bytes);
  SPX_HIP(hipMemcpy(img.data(), t->dev, t->bytes, hipMemcpyDeviceToHost));
  parallel_blocks(nblk, [&](int64_t a, int64_t b) { relayout(dtype, static_cast<uint8_t *>(ggml), img.data(), t->plane_off, a, b, false); });
  return 0;
}

int spx_tensor_free(spx_ctx *ctx, spx_tensor *t) {
  if (!t) return 0;
  if (ctx) { (void)hipSetDevice(ctx->device); (void)hipStreamSynchronize(ctx->stream); }
  if (t->dev) (void)hipFree(t->dev);
  delete t;
  return 0;
}

int spx_q8k_quantize(spx_ctx *ctx, const float *x, int64_t n, int64_t ld_x, int m, float *d, int8_t *qs, int16_t *bsums) {
  if (!ctx || !x || !d || !qs || !bsums) return fail("spx_q8k_quantize: null argument");
  if (n <= 0 || n % 256 || m <= 0 || ld_x < n || ld_x % 4) return fail("spx_q8k_quantize: n must be a positive multiple of 256, ld_x >= n and a multiple of 4");
  SPX_HIP(launch_q8k_quantize(x, n, ld_x, m, d, qs, bsums, ctx->stream));
  return 0;
}

static int check_kq(const spx_tensor *w, int expert, int m) {
  if (!w) return fail("null tensor");
  if (w->v.dtype != T_Q4K && w->v.dtype != T_Q6K) return fail("integer kernel needs a Q4_K or Q6_K tensor");
  if (expert < 0 || expert >= w->v.n_expert) return fail("expert index out of range");
  if (m < 1 || m > 16) return fail("m must be in 1..16");
  return 0;
}

// Workspace image of m permuted Q8_K vectors of n columns.
static Q8KP ws_q8kp(spx_ctx *ctx, int m, int64_t n, bool *ok) {
  size_t bytes = 0;
  (void)q8kp_layout(nullptr, m, n, &bytes);
  uint8_t *w = static_cast<uint8_t *>(ws_get(ctx, bytes));
  *ok = w != nullptr;
  if (!w) return Q8KP{};
  return q8kp_layout(w, m, n, &bytes);
}

// Expert e's rows r0.. of a K-quant tensor as a view of its own (n_expert 1): each plane's
// bytes per 256-value block are fixed (codes 128, scales 16, Q4_K header 16 / Q6_K high bits
// 64, Q6_K d 2), so the planes start (e rows + r0) nb blocks further on.
static TensorView kq_rows_view(const TensorView &v, int expert, int64_t r0, int64_t r1) {
  TensorView o = v;
  const int64_t blk = ((int64_t)expert * v.rows + r0) * v.nb;
  o.pl.p0 = v.pl.p0 + blk * 128;
  o.pl.p2 = v.pl.p2 + blk * 16;
  if (v.dtype == T_Q4K) {
    o.pl.p1 = v.pl.p1 + blk * 16;
  } else {
    o.pl.p1 = v.pl.p1 + blk * 64;
    o.pl.p3 = v.pl.p3 + blk * 2;
  }
  o.rows = r1 - r0;
  o.n_expert = 1;
  return o;
}

// Launch choice. Integer weights: one row, row-parallel lanes; two or more, the int8 matrix
// cores (kd_mq: 16-row tiles, the reference's lane classes and fp32 chains) where the row width
// is one they take, else the eight-row lane tiles. Every choice gives the reference's bits;
// SPX_MV_MODE forces one (0: lane tiles, 1: row-parallel, 2: matrix cores where they apply).
// Float formats: eight rows a wavefront (the reference's M = 1 order); Q8_0 with two or more
// rows on the fp32 matrix cores (k_mv_fq, the multi-row order of quant_multi.rs's kernel,
// within 1e-4 of it; a row's bits do not depend on the other rows of the batch).
static int mv_launch(spx_ctx *ctx, const spx_tensor *w, int expert, int m, const float *x, int64_t ld_x, Q8KP y, float *out,
                     int64_t ld_out, int64_t r0, int64_t r1) {
  const bool kq = w->v.dtype == T_Q4K || w->v.dtype == T_Q6K;
  int mode = kq ? (m >= 2 ? 2 : 1) : 0;
  if (const char *v = std::getenv("SPX_MV_MODE")) mode = kq ? std::min(std::max(atoi(v), 0), 2) : 0;
  if (mode == 2 && !dec_mq_nb_ok((int)w->v.nb)) mode = m >= 2 ? 0 : 1;
  if (mode == 2) {
    DecMMArgs a{};
    a.w[0] = kq_rows_view(w->v, expert, r0, r1);
    a.out[0] = out + r0;
    a.ld_out[0] = ld_out;
    a.tiles[0] = (int)((r1 - r0 + 15) / 16);
    a.nseg = 1;
    a.y = y;
    a.cols = (int)w->v.cols;
    a.m = m;
    SPX_HIP(launch_dec_mq(a, dec_mq_grid(a.tiles[0], m), ctx->stream));
    return 0;
  }
  int G = 8, R = 1;
  rp_shape(w->v.nb, G, R);
  MVArgs a{};
  a.seg[0].w = w->v;
  a.seg[0].out = out;
  a.seg[0].ld_out = ld_out;
  a.seg[0].r0 = r0;
  a.seg[0].r1 = r1;
  a.seg[0].expert = expert;
  a.seg[0].wgs = mv_wgs(r1 - r0, m, mode, w->v.dtype, R);
  a.nseg = 1;
  a.x = x;
  a.ld_x = ld_x;
  a.y = y;
  a.m = m;
  a.G = G;
  a.R = R;
  a.fq = !kq && m >= FQ_MIN_ROWS ? 1 : 0;
  SPX_HIP(launch_mv(a, m, mode, nullptr, a.seg[0].wgs, ctx->stream));
  return 0;
}

// One vector against a K-quant matrix on the one-row decode kernel (kd_mv: the row's Q8_K made
// in each workgroup's prologue, row-parallel lanes, the reference's bits; no workspace): a
// workgroup a tile up to 512 tiles, else one a CU striding over them (as for an LM head).
static int mv_one_row(spx_ctx *ctx, const spx_tensor *w, int expert, const float *x, float *out) {
  int G = 8, R = 1;
  rp_shape(w->v.nb, G, R);
  DecMVArgs a{};
  a.w[0] = kq_rows_view(w->v, expert, 0, w->v.rows);
  a.out[0] = out;
  a.tiles[0] = (int)((w->v.rows + DEC_MV_NW * R - 1) / (DEC_MV_NW * R));
  a.nseg = 1;
  a.G = G;
  a.in = DecIn{x, nullptr, 0.0f, (int)w->v.cols};
  int cus = 0;
  SPX_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device));
  SPX_HIP(launch_dec_mv(a, a.tiles[0] <= 512 ? a.tiles[0] : std::max(cus, 1), ctx->stream));
  return 0;
}

int spx_matmul_rows_q8k(spx_ctx *ctx, const spx_tensor *w, int expert, const float *xd, const int8_t *xs, const int16_t *xb, int m, float *out, int64_t ld_out, int64_t r0, int64_t r1) {
  if (!ctx || !xd || !xs || !xb || !out) return fail("spx_matmul_rows_q8k: null argument");
  if (int r = check_kq(w, expert, m)) return r;
  if (r0 < 0 || r1 > w->v.rows || r0 > r1) return fail("spx_matmul_rows_q8k: bad row range");
  if (m > 1 && ld_out < r1) return fail("spx_matmul_rows_q8k: ld_out smaller than the row range");
  if (r1 == r0) return 0;
  bool ok = false;
  Q8KP y = ws_q8kp(ctx, m, w->v.cols, &ok);
  if (!ok) return fail("spx_matmul_rows_q8k: workspace allocation failed");
  SPX_HIP(launch_q8kp_from_ref(xd, xs, xb, w->v.cols, m, y, ctx->stream));
  return mv_launch(ctx, w, expert, m, nullptr, 0, y, out, ld_out, r0, r1);
}

int spx_block_sums_q8k(spx_ctx *ctx, const spx_tensor *w, int expert, int64_t row, const int8_t *xs, const int16_t *xb, int32_t *sums) {
  if (!ctx || !xs || !xb || !sums) return fail("spx_block_sums_q8k: null argument");
  if (int r = check_kq(w, expert, 1)) return r;
  if (row < 0 || row >= w->v.rows) return fail("spx_block_sums_q8k: row out of range");
  bool ok = false;
  Q8KP y = ws_q8kp(ctx, 1, w->v.cols, &ok);
  if (!ok) return fail("spx_block_sums_q8k: workspace allocation failed");
  SPX_HIP(launch_q8kp_from_ref(nullptr, xs, xb, w->v.cols, 1, y, ctx->stream));
  SPX_HIP(launch_kq_block_sums(w->v, expert, row, y, sums, ctx->stream));
  return 0;
}

int spx_matvec(spx_ctx *ctx, const spx_tensor *w, int expert, const float *x, int64_t ld_x, int m, float *out, int64_t ld_out) {
  if (!ctx || !w || !x || !out) return fail("spx_matvec: null argument");
  if (m < 1 || m > 16) return fail("spx_matvec: m must be in 1..16");
  if (expert < 0 || expert >= w->v.n_expert) return fail("spx_matvec: expert index out of range");
  const int64_t cols = w->v.cols, rows = w->v.rows;
  if (ld_x < cols || (m > 1 && ld_out < rows)) return fail("spx_matvec: leading dimension too small");
  if (ld_x % 4) return fail("spx_matvec: ld_x must be a multiple of 4 (16-byte rows)");
  if (w->v.dtype == T_Q4K || w->v.dtype == T_Q6K) {
    if (m == 1 && w->v.nb <= DEC_MAXNB && !std::getenv("SPX_MV_MODE")) return mv_one_row(ctx, w, expert, x, out);
    bool ok = false;
    Q8KP y = ws_q8kp(ctx, m, cols, &ok);
    if (!ok) return fail("spx_matvec: workspace allocation failed");
    SPX_HIP(launch_q8kp_quantize(x, cols, ld_x, m, y, ctx->stream));
    return mv_launch(ctx, w, expert, m, nullptr, 0, y, out, ld_out, 0, rows);
  }
  if (w->v.dtype == T_F32 && cols % 16) return fail("spx_matvec: F32 needs cols % 16 == 0");
  if (w->v.dtype != T_Q8_0 && w->v.dtype != T_Q5_0 && w->v.dtype != T_Q5K && w->v.dtype != T_F32)
    return fail("spx_matvec: unsupported dtype " + std::to_string(w->v.dtype));
  return mv_launch(ctx, w, expert, m, x, ld_x, Q8KP{}, out, ld_out, 0, rows);
}

int spx_matvec_noalloc(spx_ctx *ctx, const spx_tensor *w, int expert, const float *x, int64_t ld_x, int m, float *out, int64_t ld_out) {
  if (!ctx || !w || !x || !out) return fail("spx_matvec_noalloc: null argument");
  if (m < 1 || m > 16) return fail("spx_matvec_noalloc: m must be in 1..16");
  if (expert < 0 || expert >= w->v.n_expert) return fail("spx_matvec_noalloc: expert index out of range");
  const int64_t cols = w->v.cols, rows = w->v.rows;
  if (ld_x < cols || (m > 1 && ld_out < rows)) return fail("spx_matvec_noalloc: leading dimension too small");
  if (ld_x % 4) return fail("spx_matvec_noalloc: ld_x must be a multiple of 4 (16-byte rows)");
  if (w->v.dtype == T_Q4K || w->v.dtype == T_Q6K) {
    if (!ctx->scratch) return fail("spx_matvec_noalloc: the scratch array has no device address in this context");
    size_t bytes = 0;
    const Q8KP y = q8kp_layout(ctx->scratch, m, cols, &bytes);
    if (bytes > SPX_NOALLOC_SCRATCH_BYTES)
      return fail("spx_matvec_noalloc: m x cols needs " + std::to_string(bytes) + " bytes of Q8_K staging, above the fixed scratch of " +
                  std::to_string(SPX_NOALLOC_SCRATCH_BYTES) + " (use spx_matvec)");
    if (ctx->device >= NOALLOC_MAX_DEV) return fail("spx_matvec_noalloc: device index above 63");
    // take this device's turn on the array: wait for the previous call's kernels (any stream),
    // then mark this call's end. A stream under graph capture skips both: the replay order of
    // the captured graph is the caller's to arrange.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    SPX_HIP(hipStreamIsCapturing(ctx->stream, &cap));
    const bool turn = cap == hipStreamCaptureStatusNone;
    std::unique_lock<std::mutex> lk(g_noalloc_mu, std::defer_lock);
    if (turn) {
      lk.lock();
      if (g_noalloc_used[ctx->device]) SPX_HIP(hipStreamWaitEvent(ctx->stream, g_noalloc_ev[ctx->device], 0));
    }
    SPX_HIP(launch_q8kp_quantize(x, cols, ld_x, m, y, ctx->stream));
    if (int r = mv_launch(ctx, w, expert, m, nullptr, 0, y, out, ld_out, 0, rows)) return r;
    if (turn) {
      SPX_HIP(hipEventRecord(g_noalloc_ev[ctx->device], ctx->stream));
      g_noalloc_used[ctx->device] = true;
    }
    return 0;
  }
  if (w->v.dtype == T_F32 && cols % 16) return fail("spx_matvec_noalloc: F32 needs cols % 16 == 0");
  if (w->v.dtype != T_Q8_0 && w->v.dtype != T_Q5_0 && w->v.dtype != T_Q5K && w->v.dtype != T_F32)
    return fail("spx_matvec_noalloc: unsupported dtype " + std::to_string(w->v.dtype));
  return mv_launch(ctx, w, expert, m, x, ld_x, Q8KP{}, out, ld_out, 0, rows);
}

}  // extern "C"

// ------------------------------------------------------------------ routed experts
// ffns_fused (smollm_chat.rs:379-442) for one row and moe_batch_fused (:650-760) plus
// moe_forward_batch's combine (:1133-1140) for 2..16 rows, with the routing given: the pass
// kernels' gate/up + SwiGLU (+ Q8_K of h) and down + combine over jobs built here the way the
// router kernel builds them (experts in index order, users in row order, gate/up jobs of at
// most GU_USERS users).
namespace {
struct MoeHost {  // copied to the device in one piece
  Job jobs[512];
  int njobs[2];
  int nkeep[MAX_M];
  float weights[MAX_M * 32];
  StepRec st;
};
size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }
}  // namespace

extern "C" int spx_moe(spx_ctx *ctx, const spx_tensor *gate, const spx_tensor *up, const spx_tensor *down, const float *x,
                       int64_t ld_x, int m, int k, const int32_t *chosen, const float *weights, float *y, int64_t ld_y) {
  if (!ctx || !gate || !up || !down || !x || !chosen || !weights || !y) return fail("spx_moe: null argument");
  if (m < 1 || m > MAX_M || k < 1 || k > 32 || m * k > 256) return fail("spx_moe: m must be in 1..16, k in 1..32, m * k <= 256");
  const int64_t dim = gate->v.cols, n_ff = gate->v.rows;
  const int ne = gate->v.n_expert;
  if (up->v.cols != dim || up->v.rows != n_ff || up->v.n_expert != ne || down->v.cols != n_ff || down->v.rows != dim ||
      down->v.n_expert != ne)
    return fail("spx_moe: gate/up must be [n_expert][n_ff][dim] and down [n_expert][dim][n_ff]");
  if (gate->v.dtype != up->v.dtype) return fail("spx_moe: gate and up must share a format");
  const bool g_int = gate->v.dtype == T_Q4K || gate->v.dtype == T_Q6K, d_int = down->v.dtype == T_Q4K || down->v.dtype == T_Q6K;
  if (n_ff % 16 || (d_int && n_ff % 256) || (g_int && dim % 256) || dim % 4) return fail("spx_moe: unsupported widths");
  if (ld_x < dim || ld_y < dim || ld_x % 4) return fail("spx_moe: leading dimension too small (or ld_x not a multiple of 4)");
  // the job list is built in the context's pinned staging block and copied with the other
  // launches (no wait on the stream: only a previous call's copy out of the block, if still
  // pending, is waited for before the block is rewritten)
  if (!ctx->moe_pin) {
    SPX_HIP(hipHostMalloc(&ctx->moe_pin, sizeof(MoeHost), hipHostMallocDefault));
    SPX_HIP(hipEventCreateWithFlags(&ctx->moe_ev, hipEventDisableTiming));
  } else {
    SPX_HIP(hipEventSynchronize(ctx->moe_ev));
  }
  MoeHost &hb = *static_cast<MoeHost *>(ctx->moe_pin);
  memset(&hb, 0, sizeof hb);
  std::vector<std::vector<int>> slot_of(m, std::vector<int>(ne, -1));
  for (int b = 0; b < m; b++)
    for (int s = 0; s < k; s++) {
      const int e = chosen[b * k + s];
      if (e < 0 || e >= ne) return fail("spx_moe: expert id out of range");
      if (slot_of[b][e] >= 0) return fail("spx_moe: a row chooses an expert twice");
      slot_of[b][e] = s;
      hb.weights[b * 32 + s] = weights[b * k + s];
    }
  int nd = 0, ng = 0;
  for (int e = 0; e < ne; e++) {
    Job &Jd = hb.jobs[256 + nd];
    int kk = 0, ks = 0;
    for (int b = 0; b < m; b++) {
      const int s = slot_of[b][e];
      if (s < 0) continue;
      Jd.vec[kk] = Jd.out[kk] = b * k + s;
      kk++;
      Job &J = hb.jobs[ng];
      J.vec[ks] = b;
      J.out[ks] = b * k + s;
      if (++ks == GU_USERS) { J.expert = e; J.nvec = ks; ng++; ks = 0; }
    }
    if (ks > 0) { hb.jobs[ng].expert = e; hb.jobs[ng].nvec = ks; ng++; }
    if (kk > 0) { Jd.expert = e; Jd.nvec = kk; nd++; }
  }
  hb.njobs[0] = nd;
  hb.njobs[1] = ng;
  for (int b = 0; b < m; b++) hb.nkeep[b] = k;
  hb.st.m = m;
  // workspace: host block, x (packed), y (Q8_K), h, hq, gate/up counters, output rows
  const int nv = m * k, nbh = (int)(n_ff / 256);
  size_t yq_b = 0, hq_b = 0;
  (void)q8kp_layout(nullptr, m, dim, &yq_b);
  (void)q8kp_layout(nullptr, nv, n_ff, &hq_b);
  const size_t cnt_b = sizeof(int) * (size_t)nv * std::max(nbh, 1) * (1 + GU_SUB) * CNT_STRIDE;
  const size_t sz[7] = {al256(sizeof hb), al256(sizeof(float) * m * dim), al256(g_int ? yq_b : 0), al256(sizeof(float) * nv * n_ff),
                        al256(d_int ? hq_b : 0), al256(cnt_b), al256(sizeof(float) * m * dim)};
  size_t tot = 0;
  for (size_t v : sz) tot += v;
  uint8_t *w = static_cast<uint8_t *>(ws_get(ctx, tot));
  if (!w) return fail("spx_moe: workspace allocation failed");
  uint8_t *p[7];
  for (int i = 0, o = 0; i < 7; o += (int)sz[i], i++) p[i] = w + o;
  hipStream_t s = ctx->stream;
  SPX_HIP(hipMemcpyAsync(p[0], &hb, sizeof hb, hipMemcpyHostToDevice, s));
  SPX_HIP(hipEventRecord(ctx->moe_ev, s));
  const MoeHost *dh = reinterpret_cast<const MoeHost *>(p[0]);
  float *xp = reinterpret_cast<float *>(p[1]), *h = reinterpret_cast<float *>(p[3]), *out = reinterpret_cast<float *>(p[6]);
  int *cnt = reinterpret_cast<int *>(p[5]);
  SPX_HIP(hipMemcpy2DAsync(xp, sizeof(float) * dim, x, sizeof(float) * ld_x, sizeof(float) * dim, m, hipMemcpyDeviceToDevice, s));
  SPX_HIP(hipMemsetAsync(cnt, 0, cnt_b, s));
  Q8KP yq{}, hq{};
  if (g_int) {
    yq = q8kp_layout(p[2], m, dim, &yq_b);
    SPX_HIP(launch_q8kp_quantize(xp, dim, dim, m, yq, s));
  }
  if (d_int) hq = q8kp_layout(p[4], nv, n_ff, &hq_b);
  GUArgs ga{};
  ga.gate = gate->v; ga.up = up->v; ga.y = yq; ga.x = xp; ga.jobs = dh->jobs; ga.njobs = dh->njobs + 1; ga.h = h;
  ga.counter = cnt; ga.n_ff = (int)n_ff;
  if (d_int) ga.hq = hq;
  SPX_HIP(launch_gateup(ga, std::min(m, GU_USERS), g_int ? 1 : 0, &dh->st, std::min(256, nv), s));
  DownArgs da{};
  da.w = down->v; da.y = hq; da.x = h; da.jobs = dh->jobs + 256; da.njobs = dh->njobs; da.weights = dh->weights;
  da.nkeep = dh->nkeep; da.n_used = k; da.out = out;
  SPX_HIP(launch_down(da, m, 0, &dh->st, s));
  SPX_HIP(hipMemcpy2DAsync(y, sizeof(float) * ld_y, out, sizeof(float) * dim, sizeof(float) * dim, m, hipMemcpyDeviceToDevice, s));
  return 0;
}

// The routed experts with the routing in device memory: nothing waits on the host. The routing
// goes into the pipeline's layout (kp_moe_in), the job list is built on the device (kp_jobs: at
// most 16 users a job), x is quantized to Q8_K, and the prefill pass's grouped kernels run on
// the int8 matrix cores (kp_gateup_mq, kd_down_mq: the reference's per-lane integer dots and fp32
// chains); kp_moe_combine sums each row's choices in order.
extern "C" int spx_moe_dev(spx_ctx *ctx, const spx_tensor *gate, const spx_tensor *up, const spx_tensor *down, const float *x,
                           int64_t ld_x, int m, int k, const int32_t *chosen, const float *weights, float *y, int64_t ld_y) {
  if (!ctx || !gate || !up || !down || !x || !chosen || !weights || !y) return fail("spx_moe_dev: null argument");
  if (m < 1 || m > PMAX || k < 1 || k > 32) return fail("spx_moe_dev: m must be in 1..128, k in 1..32");
  const int64_t dim = gate->v.cols, n_ff = gate->v.rows;
  const int ne = gate->v.n_expert;
  if (up->v.cols != dim || up->v.rows != n_ff || up->v.n_expert != ne || down->v.cols != n_ff || down->v.rows != dim ||
      down->v.n_expert != ne)
    return fail("spx_moe_dev: gate/up must be [n_expert][n_ff][dim] and down [n_expert][dim][n_ff]");
  auto kq = [](const spx_tensor *t) { return t->v.dtype == T_Q4K || t->v.dtype == T_Q6K; };
  if (!kq(gate) || !kq(down) || gate->v.dtype != up->v.dtype) return fail("spx_moe_dev: gate / up (one format) and down must be Q4_K or Q6_K");
  if (ne > 256 || dim % 256 || n_ff % 256 || n_ff > 1024 || !dec_mq_nb_ok((int)(dim / 256)) || !dec_mq_nb_ok((int)(n_ff / 256)))
    return fail("spx_moe_dev: unsupported widths (dim and n_ff multiples of 256, n_ff <= 1024, blocks a row 1, 2, 3, 4, 8 or 16; n_expert <= 256)");
  if (ld_x < dim || ld_y < dim) return fail("spx_moe_dev: leading dimension too small");
  const int nv = m * k, max_jobs = std::min(512, std::min(ne, nv) + nv / MAX_M);
  size_t yq_b = 0;
  (void)q8kp_layout(nullptr, m, dim, &yq_b);
  const size_t sz[8] = {al256(sizeof(int) * m * 32), al256(sizeof(float) * m * 32), al256(sizeof(int) * m), al256(sizeof(Job) * max_jobs),
                        al256(sizeof(int) * 4), al256(yq_b), al256(sizeof(float) * nv * n_ff), al256(sizeof(float) * nv * dim)};
  size_t tot = 0;
  for (size_t v : sz) tot += v;
  uint8_t *w = static_cast<uint8_t *>(ws_get(ctx, tot));
  if (!w) return fail("spx_moe_dev: workspace allocation failed");
  uint8_t *p[8];
  for (int i = 0, o = 0; i < 8; o += (int)sz[i], i++) p[i] = w + o;
  int *ch32 = reinterpret_cast<int *>(p[0]), *nkeep = reinterpret_cast<int *>(p[2]), *njobs = reinterpret_cast<int *>(p[4]);
  float *w32 = reinterpret_cast<float *>(p[1]), *h = reinterpret_cast<float *>(p[6]), *yd = reinterpret_cast<float *>(p[7]);
  Job *jobs = reinterpret_cast<Job *>(p[3]);
  hipStream_t s = ctx->stream;
  SPX_HIP(launch_kp_moe_in(chosen, weights, m, k, ne, ch32, w32, nkeep, s));
  DecRouteArgs rt{};
  rt.n_expert = ne; rt.n_used = k; rt.m = m; rt.chosen = ch32; rt.weights = w32; rt.nkeep = nkeep; rt.jobs = jobs; rt.njobs = njobs;
  SPX_HIP(launch_kp_jobs(rt, s));
  const Q8KP yq = q8kp_layout(p[5], m, dim, &yq_b);
  SPX_HIP(launch_q8kp_quantize(x, dim, ld_x, m, yq, s));
  DecGateUpMArgs ga{};
  ga.gate = gate->v; ga.up = up->v; ga.y = yq; ga.h = h; ga.n_ff = (int)n_ff; ga.m = m;
  SPX_HIP(launch_kp_gateup_mq(ga, jobs, njobs, max_jobs, s));
  DecDownMArgs da{down->v, h, jobs, njobs, yd, max_jobs};
  SPX_HIP(launch_dec_down_mq(da, s));
  SPX_HIP(launch_kp_moe_combine(yd, w32, nkeep, m, k, (int)dim, y, ld_y, s));
  return 0;
}
