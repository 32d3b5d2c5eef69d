// Argument records and launchers of the one-row decode pipeline (decode.hip).
//
// A decode pass (M = 1, forward_slice smollm_chat.rs:3364-3552) is a chain of kernels that
// hand their results to each other only through kernel boundaries: no arrival counters and
// no last-workgroup tails. A producer writes the residual add itself (x + rscale * y, row by
// row), and every workgroup of a consumer recomputes the RMSNorm and Q8_K of the row it
// needs (a few KB, read while its weights are already in flight). The arithmetic is the same
// as the fused kernels' (fused.hip) operation for operation, so both pipelines give the same
// bits.
#pragma once
#include "fused.h"

namespace spx {

// Activation prologue: the fp32 row x (cols values) read by every workgroup, RMS-normalised
// with nw unless nw is null, and quantized to permuted Q8_K in LDS.
struct DecIn {
  const float *x;
  const float *nw;
  float eps;
  int cols;
};

// Integer matvec of one row over up to three tensors (segments) sharing the input. Rows are
// taken in tiles of DEC_MV_NW * R rows (G, R: rp_shape of the blocks per row).
struct DecMVArgs {
  TensorView w[3];
  float *out[3];      // segment outputs (null: not written)
  int tiles[3];       // row tiles (DEC_MV_NW * R rows) of each segment
  int nseg;
  int G;              // row groups per row (rp_shape of the blocks per row)
  DecIn in;
  // residual epilogue (one segment): res_out[r] = res_in[r] + rscale * y[r]
  const float *res_in;
  float *res_out;
  float rscale;
  // greedy pick (LM head): best key of each workgroup -> best[blockIdx.x]
  unsigned long long *best;
  float lscale;
  float *xn_out;      // the normalised input row, written by workgroup 0 (null: not written)
  int nv;             // rows of the pass: 0 or 1, or 2 (a two-row pass: rows v of in.x / out / res / xn_out, best [v][grid])
};

// Merge of the attention partials of one pass row: one workgroup per query head, written as
// fp32.
struct DecMergeArgs {
  const float *part_ml, *part_o;  // as AttnArgs
  float *att;
  int nslot, hd, n_heads, n_kv;
};

// F32 router rows (one per workgroup) of the ffn_norm'd row.
struct DecRouterArgs {
  TensorView w;
  DecIn in;
  float *logits;      // [nv][n_expert]
  int n_expert;
  int nv;             // rows: 0 or 1, or 2 (rows v of in.x)
};

// Routing (MoE) and gate/up + SwiGLU of the chosen experts; a dense FFN is expert 0 with no
// routing (logits null).
struct DecGateUpArgs {
  TensorView gate, up;
  DecIn in;
  const float *logits;  // null: dense
  int n_expert, n_used, norm;
  float moe_prune;
  float *h;             // [n_used][n_ff]
  int *chosen;          // [n_used] kept experts in choice order
  float *weights;       // [n_used]
  int *nkeep;           // [1]
  int *njobs;           // [1]: distinct experts of the pass (kept choices)
  int *expert_count;    // [n_expert] selection counter (null: none)
  int n_ff;
  int nv;               // rows: 0 or 1, or 2 (h [v n_used + s], chosen / weights [v][n_used], nkeep [v])
};

// Down projection of the chosen experts + weighted combine + residual add.
struct DecDownArgs {
  TensorView w;
  const float *h;
  const int *chosen;
  const float *weights;
  const int *nkeep;
  int n_used;
  const float *res_in;
  float *res_out;
  float rscale;
  int nv;               // rows: 0 or 1, or 2 (slots v n_used + i; res rows v)
};

constexpr int DEC_MV_NW = 16;   // wavefronts per matvec workgroup
constexpr int DEC_MM_NW = 8;    // wavefronts per workgroup of the multi-row kernels
constexpr int DEC_MAXNB = 16;   // blocks per row (cols <= 4096) of the decode kernels
constexpr int DEC_DOWN_Q = 16384;  // n_used * n_ff values of h quantized in LDS by the down kernel

hipError_t launch_dec_mv(const DecMVArgs &a, int grid, hipStream_t s);

// ---- passes of 2..16 rows (verify / prefill): the same arithmetic per row as the one-row
// kernels; the activations are normalised once per layer (kd_norm) and read as Q8_K.

// RMSNorm (+ the fp32 normalised rows and / or their Q8_K) of m rows, one workgroup per row.
struct DecNormArgs {
  const float *x;     // [m][dim]
  const float *nw;
  float eps;
  int dim;
  float *xn_out;      // [m][dim] (null: not written)
  Q8KP q_out;         // [m] (q null: not written)
  // MoE combine ahead of the norm (yd null: none): row b is
  // res_in[b] + rscale * sum_i cw[b][i] * yd[b * n_used + i] over its kept choices in choice
  // order (unfused multiply and add, ffns_fused :432-437), written to x_out, then normalised
  const float *yd;    // [m * n_used][dim]
  const float *cw;    // [m][32] choice weights
  const int *nkeep;   // [m]
  const float *res_in;
  float *x_out;
  int n_used;
  float rscale;
};

// Integer matvec of m vectors (Q8_K, global) over up to three segments.
struct DecMMArgs {
  TensorView w[3];
  float *out[3];      // row r of vector v -> out[v * ld_out + r]
  int64_t ld_out[3];
  int tiles[3];       // row tiles (DEC_MM_NW * R rows)
  int nseg;
  int G;
  Q8KP y;
  int cols, m;
  const float *res_in;  // residual epilogue (one segment): res_out[v][r] = res_in[v][r] + rscale * y
  float *res_out;
  float rscale;
  unsigned long long *best;  // greedy keys: best[v * nbest + blockIdx.x]
  int nbest;
  float lscale;
};

// F32 router rows (one per workgroup) of m fp32 normalised rows.
struct DecRouterMArgs {
  TensorView w;
  const float *x;     // [m][dim]
  float *logits;      // [m][n_expert]
  int n_expert, dim, m;
};

// Routing of m rows and the grouped job list: experts with at least one user, in expert order,
// users in (row, slot) order; job j: vec[k] = the user's row, out[k] = row * n_used + slot.
struct DecRouteArgs {
  const float *logits;
  int n_expert, n_used, norm, m;
  float moe_prune;
  int *chosen;        // [m][32]
  float *weights;     // [m][32]
  int *nkeep;         // [m]
  Job *jobs;          // [<= 512]
  int *njobs;         // [0]: jobs; [2]: experts with users (kp_route)
  int *expert_count;  // [n_expert] (null: none)
};

// Routing of the m rows, then gate/up + SwiGLU over the jobs (rt.logits null: dense, one job
// of users 0..m-1). Every workgroup routes the rows and builds the job list itself; workgroup 0
// publishes the routing results, the job list and the selection counts (rt's outputs).
struct DecGateUpMArgs {
  TensorView gate, up;
  Q8KP y;             // normalised rows [m]
  DecRouteArgs rt;
  float *h;           // [m * n_used][n_ff] (dense: [m][n_ff])
  int n_ff, m;
  int max_jobs;       // bound of the job count (set by the launcher)
};

// Down projection of the jobs' users (y per (user, row), combined by the next kd_norm).
struct DecDownMArgs {
  TensorView w;
  const float *h;     // [m * n_used][n_ff] fp32 (quantized to Q8_K by the kernel)
  const Job *jobs;
  const int *njobs;
  float *yd;          // [m * n_used][dim]: y of each (row, choice), combined by the next kd_norm
  int max_jobs;       // bound of the job count
};

// LDS image of m Q8_K vectors of cols columns (codes, scales, bsum pairs), as kd_mm and the
// grouped expert kernels stage them.
__host__ __device__ inline size_t mm_act_bytes(int m, int cols) {
  const int nbq = cols >> 8;
  return (((size_t)m * cols + 15) & ~(size_t)15) + (((size_t)m * nbq * 4 + 15) & ~(size_t)15) + (size_t)m * nbq * 64;
}
// kd_down_m's LDS: one job's users' Q8_K h
__host__ __device__ inline size_t downm_lds_bytes(int n_ff) { return mm_act_bytes(MAX_M, n_ff); }

// kd_gateup_m's LDS: one job's users' Q8_K rows, the chain buffers, the job table
__host__ __device__ inline size_t gum_lds_bytes(int m, int cols, int max_jobs) {
  return mm_act_bytes(m, cols) + (size_t)DEC_MM_NW * 2 * 4 * m * 10 * 4 + (size_t)max_jobs * (2 + 2 * MAX_M) * 4;
}

hipError_t launch_dec_norm(const DecNormArgs &a, int m, hipStream_t s);
hipError_t launch_dec_mm(const DecMMArgs &a, int grid, hipStream_t s);
// The same matvec on the int8 matrix cores (16-row tiles, a wavefront per tile; the reference's
// per-lane-class int32 partials and fp32 chains, so the results are kd_mm's bit for bit):
// tiles[i] counts 16-row tiles; tiles stride over the grid's wavefronts.
hipError_t launch_dec_mq(const DecMMArgs &a, int grid, hipStream_t s);
// The blocks-per-row counts (cols / 256) the matrix-core kernels take: 1, 2, 3, 4, 8, 16.
bool dec_mq_nb_ok(int nb);
// kd_mq's grid argument for a number of tiles and m vectors: up to 16 vectors, workgroups (at
// most two a CU); more (prefill), tile ranges, a multiple of eight (the launch holds
// ceil(m / 16) workgroups per range). With greedy keys, nbest = this value.
int dec_mq_grid(int tiles, int m);
// kd_mm grid for a number of tiles: at most two workgroups a CU, the same number of tiles each
// (tiles stride over the grid; the next tile's weights are requested before the results)
int dec_mm_grid(int tiles);
hipError_t launch_dec_router_m(const DecRouterMArgs &a, hipStream_t s);
hipError_t launch_dec_gateup_m(const DecGateUpMArgs &a, int max_jobs, hipStream_t s);
hipError_t launch_dec_down_m(const DecDownMArgs &a, hipStream_t s);
// The grouped expert kernels on the int8 matrix cores (16-row tiles)
hipError_t launch_dec_gateup_mq(const DecGateUpMArgs &a, int max_jobs, hipStream_t s);
hipError_t launch_dec_down_mq(const DecDownMArgs &a, hipStream_t s);
hipError_t launch_kp_down_mq(const DecDownMArgs &a, hipStream_t s);
// Prefill passes (17..PMAX rows): routing + the job list (at most 16 users a job) in global
// memory; gate/up over such a list (jobs null: dense, rows in sixteens), max_jobs bounds it
hipError_t launch_kp_route(const DecRouteArgs &a, hipStream_t s);
hipError_t launch_kp_gateup_mq(const DecGateUpMArgs &a, const Job *jobs, const int *njobs, int max_jobs, hipStream_t s);
// Routing given in device memory (spx_moe_dev): chosen / weights [m][k] into the [m][32] layout
// with nkeep (rows with bad ids: nkeep 0); the job list from it (kp_jobs); the weighted combine
// of the expert rows yd [m k][dim] into y (NaN rows for nkeep 0).
hipError_t launch_kp_moe_in(const int *chosen, const float *weights, int m, int k, int ne, int *ch32, float *w32, int *nkeep, hipStream_t s);
hipError_t launch_kp_jobs(const DecRouteArgs &a, hipStream_t s);
hipError_t launch_kp_moe_combine(const float *yd, const float *w32, const int *nkeep, int m, int k, int dim, float *y, int64_t ld_y, hipStream_t s);
hipError_t launch_dec_merge(const DecMergeArgs &a, const StepRec *st, hipStream_t s);
hipError_t launch_dec_router(const DecRouterArgs &a, hipStream_t s);
hipError_t launch_dec_gateup(const DecGateUpArgs &a, hipStream_t s);
hipError_t launch_dec_down(const DecDownArgs &a, hipStream_t s);
// partials only (no merge): one-row decode passes, merged by launch_dec_merge
hipError_t launch_attention_partials(const AttnArgs &a, const StepRec *st, hipStream_t s);

}  // namespace spx
