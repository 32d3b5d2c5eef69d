// Argument records and launchers of the fused decode / verify kernels (fused.hip).
#pragma once
#include "common.h"
#include "kq.h"

namespace spx {

constexpr int MAX_M = 16;       // rows per verify pass (and per pass of the fused kernels)
constexpr int PMAX = 128;       // rows per prefill pass (forward_batch_slice's prompt chunks)
constexpr int ATT_QMAX = PMAX * 8;  // query heads x rows per kv head in one pass (128 rows x 8)
constexpr int ATT_QT = ATT_QMAX / 16;  // attention: 16-query tiles per kv head
constexpr int ATT_GRP = 16;     // attention: chunks merged per group
constexpr int ATT_GMAX = 16;    // attention: groups per kv head (max_seq <= 64 * 16 * 16)
constexpr int NORM_NT = 16;     // norm tails handle dim <= 256 * NORM_NT
constexpr int CNT_SUB = 64;     // first-level arrival counters of a two-level count
constexpr int CNT_STRIDE = 32;  // ints between counters (own 128-byte line each)
constexpr int GU_SUB = 8;       // first-level counters per 256-row block of h (gate/up Q8_K tail)
constexpr int GU_USERS = 2;     // users per gate/up job (an expert's users split over jobs)

// Device-side step record: the token rows of this pass and where they go in the KV cache.
struct StepRec {
  int m;
  int start;
  int ids[PMAX];
  int step;           // back-to-back decode: passes done (index into the token history)
};

// Residual add + RMSNorm (+ Q8_K) of the pass's rows, run once by the last workgroup of the
// kernel that produced `add` (rmsnorm smollm_chat.rs:569-575 after the residual add
// :3518-3520 / :3538-3540): x_out = x + rscale * add, then xn = x_out * inv * nw with
// inv = 1/sqrt(sum(x_out^2)/dim + eps), written as fp32 (xn_out) and / or permuted Q8_K
// (q_out). The sum is taken in a fixed order: per 256-value block a wavefront tree, then the
// blocks in order, so a row's result does not depend on how many rows the pass has.
// nw == null: no tail.
struct NormTail {
  const float *x;     // residual input [m][dim]
  const float *add;   // this kernel's output [m][dim] (null: none), read coherently
  float rscale;
  const float *nw;
  float eps;
  float *x_out;       // [m][dim] (null: not written)
  float *xn_out;      // [m][dim] (null: not written)
  Q8KP q_out;         // q null: not written (needs dim % 256 == 0)
  int dim;
  int *counter;       // (1 + CNT_SUB) * CNT_STRIDE ints, zero between passes
};

// One weight tensor's rows as a matvec segment.
struct Seg {
  TensorView w;
  float *out;         // row r of vector v -> out[v * ld_out + r]
  int64_t ld_out;
  int64_t r0, r1;     // rows [r0, r1) of the expert
  int expert;
  int wgs;            // workgroups of this segment
};

struct MVArgs {
  Seg seg[3];
  int nseg;
  Q8KP y;             // integer path: activations (permuted Q8_K, cols of the segments)
  const float *x;     // float path: fp32 activations [m][ld_x]
  int64_t ld_x;
  int m;              // rows of activations when no step record is given
  int G, R;           // row-parallel launches: lane groups per row, rows per wavefront
  // optional greedy-pick partials (LM head): per vector, the best packed (key, index) of
  // each workgroup -> best[v * nbest + blockIdx.x]
  unsigned long long *best;
  int nbest;
  float lscale;
  NormTail tail;
  // float path, passes of FQ_MIN_ROWS..16 rows: Q8_0 segments on the fp32 matrix cores
  // (k_mv_fq) instead of the per-lane walk (the same products, summed in another order)
  int fq;
  // one-row Q8_0 passes (k_mv_f1 only): pro.nw set: the input row is pro.x, normalised by every
  // workgroup as norm_rows would (workgroup 0 also writes pro.xn_out); res_out set: residual
  // epilogue res_out[r] = res_in[r] + rscale * y[r] (one segment)
  NormTail pro;
  const float *res_in;
  float *res_out;
  float rscale;
};
constexpr int FQ_MIN_ROWS = 2;  // one-row passes keep the per-lane walk (a 16-vector tile would idle 15 columns)

struct AttnArgs {
  const float *q, *k, *v;             // raw projections [m][q_dim], [m][kv_dim]
  const float *q_bias, *k_bias, *v_bias, *q_norm, *k_norm;
  const float2 *rope;                 // [max_seq][head_dim/2] (cos, sin)
  __half *kc, *vc;                    // [n_layers][max_seq][kv_dim]
  float *part_ml;                     // [n_kv][nslot][ATT_QMAX][2] (running max, sum)
  float *part_o;                      // [n_kv][nslot][ATT_QMAX][hd] (unnormalised output)
  int *counter;                       // [n_kv][ATT_QT][1 + ATT_GMAX][CNT_STRIDE], zero between passes
  float *att;                         // [m][q_dim]
  Q8KP aq;                            // permuted Q8_K of att (q null: not produced)
  int layer, max_seq, kv_dim, hd, n_heads, n_kv, neox;
  int nch;                            // chunks launched per kv head (>= max_seq / 64)
  int nslot;                          // partial slots per kv head: nch chunks, then group partials
  // 1: q holds the prepared queries (bias, norm, RoPE applied) and the pass's K / V rows are in
  // the cache already (launch_rows_prep); 2: the K / V rows are in the cache, q holds the raw
  // projections (launch_attention_fs only); multi-row passes only
  int prepped;
  float eps, scale;
};

// Grouped MoE job: an expert and its users (vector index in, vector index out).
struct Job {
  int expert;
  int nvec;
  int vec[MAX_M];
  int out[MAX_M];
};

struct RouterArgs {
  TensorView w;                       // F32 [n_expert][dim]
  const float *x;                     // normalised rows [m][dim]
  float *logits;                      // [m][n_expert]
  int n_expert, n_used, norm, dim;
  float moe_prune;
  int *counter;                       // (1 + CNT_SUB) * CNT_STRIDE ints, zero between passes
  int *chosen;                        // [16][32]
  float *weights;                     // [16][32]
  int *nkeep;                         // [16]
  Job *jobs;                          // gate/up jobs [256] (<= GU_USERS users), then down jobs [256]
  int *njobs;                         // [2]: down jobs (= distinct experts), gate/up jobs
  int *expert_count;                  // optional [n_expert] selection counter
  NormTail pro;                       // one-row passes: pro.nw set: x is pro.x, normalised in every workgroup
  int logits_only;                    // the logits only (the routing runs in the gate/up prologue)
};

// One-row passes of a float MoE: the routing in every gate/up workgroup from the router's
// logits (route_row), workgroup b.y taking the job of rank b.y among the kept choices in expert
// order; workgroup (0, 0) writes the choices, weights, keep count, the down jobs (one user each),
// the job counts and the selection counts, as the router's last workgroup would.
struct F1Route {
  const float *logits;                // [n_expert]; null: jobs come from the router
  int n_expert, n_used, norm;
  float moe_prune;
  int *chosen;                        // [32]
  float *weights;                     // [32]
  int *nkeep;                         // [1]
  Job *jobs;                          // down jobs
  int *njobs;                         // [2]: down jobs, gate/up jobs
  int *expert_count;                  // optional [n_expert]
};

// Gate/up + SwiGLU (+ Q8_K of h by the last workgroup covering each 256-row block) over
// jobs; a dense FFN is one job whose users are the pass's rows.
struct GUArgs {
  TensorView gate, up;
  Q8KP y;                             // integer path input
  const float *x;                     // float path input, ld = dim
  const Job *jobs;                    // null: dense, users = rows 0..m-1
  const int *njobs;
  float *h;                           // [vec][n_ff]
  Q8KP hq;                            // q null: no quantization
  int *counter;                       // [vectors][n_ff/256][1 + GU_SUB][CNT_STRIDE], zero between passes
  int n_ff;
  int G;                              // row-parallel launch: lane groups per row
  int fq;                             // Q8_0, 2..16 rows: on the fp32 matrix cores (k_gateup_fq)
  int vdiv;                           // > 1: a job's vec entries are h indices (row * vdiv + slot), the input row their quotient
  NormTail pro;                       // one-row float passes (k_gateup_f): pro.nw set: x is pro.x, normalised in every workgroup
  F1Route rt;                         // one-row float passes (k_gateup_f): routing in the prologue
};

struct DownArgs {
  TensorView w;                       // [n_expert] x [dim][n_ff]
  Q8KP y;                             // hq (integer path)
  const float *x;                     // h (float path)
  const Job *jobs;
  const int *njobs;
  const float *weights;
  const int *nkeep;
  int n_used;
  float *out;                         // [m][dim]
  int G;                              // row-parallel launch: lane groups per row
  NormTail tail;
  float *yd;                          // launch_down_fq: y per (row, slot) [m * n_used][dim]
  int *counter;                       // launch_down_fq: arrivals per 32 output rows [dim / 32][CNT_STRIDE] (+ one), zero between passes
  const float *res_in;                // k_down_f: residual epilogue res_out = res_in + rscale * out (instead of a tail)
  float *res_out;
  float rscale;
};

hipError_t launch_embed(const TensorView &e, const StepRec *st, float escale, const NormTail &t, int m, hipStream_t s);
// mode 0: eight rows per wavefront (tiles); 1: row-parallel (integer only)
hipError_t launch_mv(const MVArgs &a, int mt, int mode, const StepRec *st, int grid, hipStream_t s);
hipError_t launch_attention(const AttnArgs &a, int m, const StepRec *st, hipStream_t s);
// The attention block's row preparation of the step record's pass of m rows (bias, per-head RMSNorm and RoPE of
// q and k, as the attention kernel does it): prepared queries to qp [m][q_dim] (qp null: none),
// K / V rows to the cache (f16 RNE); then launch_attention with a.prepped = 1 reads them from there
hipError_t launch_rows_prep(const AttnArgs &a, float *qp, int m, const StepRec *st, hipStream_t s);
// Prefill attention with bits of its own (rows prepared by launch_rows_prep, a.prepped = 1): a
// chunk loop per (kv head, 64 queries, one of four splits of the chunks) with an online softmax,
// then the splits merged in order into the att rows (and their Q8_K when a.aq is set).
hipError_t launch_attention_fl(const AttnArgs &a, int m, const StepRec *st, hipStream_t s);
// Prefill attention with bits of its own and no partials in memory (the pass's K / V rows put in
// the cache by launch_rows_prep; a.prepped 1: prepared queries in q, 2: raw projections, prepared
// here): a workgroup per (kv head, 16 queries), each wavefront an online softmax over every
// eighth 32-position slice of the positions they see, the eight states merged in LDS into the
// att rows (and their Q8_K when a.aq is set).
hipError_t launch_attention_fs(const AttnArgs &a, int m, const StepRec *st, hipStream_t s);
// The same attention for prepared rows as partials (a workgroup per chunk, kv head and four
// query tiles, a wavefront per tile) and a merge launch: each output has launch_attention's bits
hipError_t launch_attention_pf(const AttnArgs &a, int m, const StepRec *st, hipStream_t s);
// Passes of up to 16 rows, unprepared: the same outputs (att rows, Q8_K, the pass's K / V rows in
// the cache) as launch_attention, bit for bit, from a workgroup per (chunk, kv head) whose
// wavefronts take a query tile each, then a merge launch a workgroup per 256 att values and row
hipError_t launch_attention_mt(const AttnArgs &a, int m, const StepRec *st, hipStream_t s);
hipError_t launch_router(const RouterArgs &a, int mt, const StepRec *st, hipStream_t s);
hipError_t launch_gateup(const GUArgs &a, int mt, int mode, const StepRec *st, int max_jobs, hipStream_t s);
hipError_t launch_down(const DownArgs &a, int mt, int mode, const StepRec *st, hipStream_t s);
// Routed experts' down projection of 2..16 rows, Q8_0 weights, on the fp32 matrix cores: a
// workgroup per (32 output rows, down job), then per 32 rows the combine in choice order, then
// the norm tail (a.tail.nw set) in the last of them
hipError_t launch_down_fq(const DownArgs &a, int max_jobs, const StepRec *st, hipStream_t s);
hipError_t launch_norm(const NormTail &t, const StepRec *st, int m, hipStream_t s);
// hist non-null (m == 1): the pick advances the step record (next token and position) and is
// appended to hist[step]
hipError_t launch_argmax_final(const unsigned long long *best, int nbest, int *out, StepRec *st, int *hist, int m, hipStream_t s);
hipError_t launch_q8kp_quantize(const float *x, int64_t n, int64_t ld_x, int m, Q8KP out, hipStream_t s);
hipError_t launch_q8kp_from_ref(const float *d, const int8_t *qs, const int16_t *bs, int64_t n, int m, Q8KP out, hipStream_t s);
hipError_t launch_kq_block_sums(const TensorView &w, int expert, int64_t row, Q8KP y, int32_t *sums, hipStream_t s);
// workgroups a matvec segment needs for the launch mode (rows per workgroup as launched)
int mv_wgs(int64_t rows, int mt, int mode, int dtype, int R);

// Row-parallel shape for rows of nb blocks: G lane groups per row (the smallest power of two
// >= nb, at most 8), R = 8 / G rows per wavefront.
__host__ __device__ inline void rp_shape(int64_t nb, int &G, int &R) {
  G = 1;
  while (G < nb && G < 8) G *= 2;
  R = 8 / G;
}

}  // namespace spx
