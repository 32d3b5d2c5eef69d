// Argument records and launchers of the fused decode / verify kernels (fused.hip).
#pragma once
#include "common.h"
#include "kq.h"

namespace spx {

constexpr int MAX_M = 16;       // rows per verify / prefill pass
constexpr int ATT_QMAX = 128;   // query heads x rows per kv head in one pass (16 rows x 8)
constexpr int PRO_NT = 8;       // fused prologues handle dim <= 256 * PRO_NT

// Device-side step record: the token rows of this pass and where they go in the KV cache.
struct StepRec {
  int m;
  int start;
  int ids[MAX_M];
};

// Residual + RMSNorm prologue of a kernel (rmsnorm smollm_chat.rs:569-575 after the residual
// add :3518-3520 / :3538-3540): row b's input is xa[b] + rscale * pa[b] (pa may be null),
// normalised with weight nw. The normalised row stays in the workgroup (LDS), as fp32 or as
// permuted Q8_K; workgroup 0 also writes the un-normalised sum to xb and, optionally, the
// normalised row (xn_out, fp32) and its Q8_K (q_out) for later kernels.
struct Pro {
  const float *xa, *pa;
  float rscale;
  const float *nw;
  float eps;
  float *xb;
  float *xn_out;
  Q8KP q_out;
  int dim;
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
  Q8KP y;             // integer path without prologue: activations (cols of the segments)
  const float *x;     // float path without prologue: fp32 activations [m][ld_x]
  int64_t ld_x;
  Pro pro;
  int m;              // rows of activations when no step record is given
  // optional greedy-pick partials (LM head): per vector, the best packed (key, index) of
  // each workgroup -> best[v * nbest + blockIdx.x]
  unsigned long long *best;
  int nbest;
  float lscale;
};

struct AttnArgs {
  const float *q, *k, *v;             // raw projections [m][q_dim], [m][kv_dim]
  const float *q_bias, *k_bias, *v_bias, *q_norm, *k_norm;
  const float2 *rope;                 // [max_seq][head_dim/2] (cos, sin)
  __half *kc, *vc;                    // [n_layers][max_seq][kv_dim]
  float *part_ml;                     // [n_kv][nch][ATT_QMAX][2] (running max, sum)
  float *part_o;                      // [n_kv][nch][ATT_QMAX][hd] (unnormalised output)
  int *counter;                       // [n_kv], zero between passes
  float *att;                         // [m][q_dim]
  Q8KP aq;                            // permuted Q8_K of att (q null: not produced)
  int layer, max_seq, kv_dim, hd, n_heads, n_kv, neox, nch;
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
  float *logits;                      // [m][n_expert]
  Pro pro;
  int n_expert, n_used, norm;
  float moe_prune;
  int *counter;                       // zero between passes
  int *chosen;                        // [16][32]
  float *weights;                     // [16][32]
  int *nkeep;                         // [16]
  Job *jobs;                          // union of chosen experts, expert order
  int *njobs;
  int *expert_count;                  // optional [n_expert] selection counter
  int rows_per_wg;
};

// Gate/up (+ SwiGLU, + Q8_K of the result) over jobs; a dense FFN is one job whose users are
// the pass's rows (with the residual + RMSNorm prologue).
struct GUArgs {
  TensorView gate, up;
  Q8KP y;                             // integer path input (no prologue)
  const float *x;                     // float path input (no prologue), ld = dim
  Pro pro;
  bool use_pro;
  const Job *jobs;                    // null: dense, users = rows 0..m-1
  const int *njobs;
  float *h;                           // [vec][n_ff]
  Q8KP hq;                            // q null: no quantization
  int *counter;                       // [16*32][n_ff/256], zero between passes
  int n_ff;
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
};

hipError_t launch_embed(const TensorView &e, const StepRec *st, float *x, int64_t ld_x, float escale, int m, hipStream_t s);
hipError_t launch_mv(const MVArgs &a, int mt, bool pro, const StepRec *st, int total_wgs, hipStream_t s);
hipError_t launch_attention(const AttnArgs &a, int m, const StepRec *st, hipStream_t s);
hipError_t launch_router(const RouterArgs &a, int mt, const StepRec *st, hipStream_t s);
hipError_t launch_gateup(const GUArgs &a, int mt, const StepRec *st, int max_jobs, hipStream_t s);
hipError_t launch_down(const DownArgs &a, int mt, const StepRec *st, int njob_max, hipStream_t s);
hipError_t launch_norm(const Pro &p, const StepRec *st, int m, hipStream_t s);
hipError_t launch_argmax_final(const unsigned long long *best, int nbest, int *out, const StepRec *st, int m, hipStream_t s);
hipError_t launch_q8kp_quantize(const float *x, int64_t n, int64_t ld_x, int m, Q8KP out, hipStream_t s);
hipError_t launch_q8kp_from_ref(const float *d, const int8_t *qs, const int16_t *bs, int64_t n, int m, Q8KP out, hipStream_t s);
hipError_t launch_kq_block_sums(const TensorView &w, int expert, int64_t row, Q8KP y, int32_t *sums, hipStream_t s);
// workgroups a matvec segment needs (8 rows per wavefront, waves per workgroup as launched)
int mv_wgs(int64_t rows, int mt, bool pro, int dtype);
size_t mv_smem(const MVArgs &a, int mt, bool pro, int dtype);

}  // namespace spx
