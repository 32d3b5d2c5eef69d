/*
 * spx.h -- C ABI of the MI355X (gfx950) decode/verify engine.
 *
 * Plain C types only (pointers, sizes, ints); every call returns an int status (0 = ok,
 * negative = error, message from spx_last_error() on the calling thread). Device pointers
 * are HIP device addresses the caller owns; host pointers are borrowed for the duration of
 * the call. A context is used from one host thread and runs on one HIP stream; calls are
 * asynchronous on that stream unless they return host data, and spx_sync() waits for it.
 *
 * Each entry point names the reference interface it replaces (file:line in WiseHax/spindle).
 */
#ifndef SPX_H
#define SPX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (gguf_loader.rs:24-42) */
enum { SPX_F32 = 0, SPX_F16 = 1, SPX_Q5_0 = 6, SPX_Q8_0 = 8, SPX_Q4_K = 12, SPX_Q6_K = 14 };

typedef struct spx_ctx spx_ctx;
typedef struct spx_tensor spx_tensor;

/* Error text of the last failed call on this thread. */
const char *spx_last_error(void);

/* Context = device + stream + scratch (replaces the WorkerPool the operators run on,
 * worker_pool.rs:43-105, and the thread-local scratch of quant_q8k.rs:123-142). */
int spx_create(int device, spx_ctx **out);
int spx_destroy(spx_ctx *ctx);
int spx_sync(spx_ctx *ctx);
void *spx_get_stream(spx_ctx *ctx); /* the hipStream_t calls are queued on */

/* Bytes per GGUF row (row_bytes, quant.rs:1527-1542); 0 when unsupported / bad width. */
int64_t spx_row_bytes(int dtype, int64_t cols);

/* Uploads one weight tensor: n_expert slabs of rows x cols in GGUF block layout, exactly the
 * bytes Mat::of / Mat::expert address in the mapped file (quant.rs:910-935). The device copy
 * is re-laid out per block field (planar) for aligned, coalesced loads. */
int spx_tensor_upload(spx_ctx *ctx, int dtype, int64_t cols, int64_t rows, int n_expert,
                      const void *ggml_bytes, spx_tensor **out);
/* Copies the tensor back in GGUF block layout (the inverse of the upload's re-layout). */
int spx_tensor_download(spx_ctx *ctx, const spx_tensor *t, void *ggml_bytes);
int spx_tensor_free(spx_ctx *ctx, spx_tensor *t);

/* Q8_K quantization of m vectors of n floats (n % 256 == 0), vector v at x + v*ld_x
 * (Q8K::quantize, quant_q8k.rs:73-121). Outputs: d[m][n/256], qs[m][n], bsums[m][n/16]. */
int spx_q8k_quantize(spx_ctx *ctx, const float *x, int64_t n, int64_t ld_x, int m, float *d,
                     int8_t *qs, int16_t *bsums);

/* Rows [r0, r1) of expert `expert` times m <= 16 Q8_K vectors (quant_q8k::matmul_rows,
 * quant_q8k.rs:252-295). Vector v's Q8_K is (xd + v*nb, xs + v*cols, xb + v*nb*16); row r of
 * vector v goes to out[v*ld_out + r]. Q4_K / Q6_K only. */
int spx_matmul_rows_q8k(spx_ctx *ctx, const spx_tensor *w, int expert, const float *xd,
                        const int8_t *xs, const int16_t *xb, int m, float *out, int64_t ld_out,
                        int64_t r0, int64_t r1);

/* The exact per-block integers of one row against one Q8_K vector (the quantities summed and
 * scaled inside rows<B,T>, quant_q8k.rs:198-243): sums[2i] = sum_lanes sumi, sums[2i+1] = the
 * integer of the min/offset correction (Q6_K: 32*s). Device pointers; nb = cols/256 pairs. */
int spx_block_sums_q8k(spx_ctx *ctx, const spx_tensor *w, int expert, int64_t row,
                       const int8_t *xs, const int16_t *xb, int32_t *sums);

/* out = W x for m <= 16 fp32 vectors (matvec smollm_chat.rs:309-317 for m == 1,
 * matvec_multi :447-512 for m > 1). Q4_K / Q6_K quantize x to Q8_K first and take the
 * integer kernel; Q8_0 / Q5_0 / F32 keep fp32 activations. Vector v: x + v*ld_x,
 * out + v*ld_out. */
int spx_matvec(spx_ctx *ctx, const spx_tensor *w, int expert, const float *x, int64_t ld_x, int m,
               float *out, int64_t ld_out);

#ifdef __cplusplus
}
#endif
#endif
