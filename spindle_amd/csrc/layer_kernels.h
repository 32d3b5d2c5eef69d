// Argument records and launchers of the per-layer kernels (layer_kernels.hip).
#pragma once
#include "common.h"

namespace spx {

constexpr int ATT_CHUNK = 64;  // positions per attention workgroup (one per lane)
constexpr int ATT_QG = 16;     // query vectors per pass inside an attention workgroup
constexpr int MAX_M = 16;      // rows per verify / prefill pass
constexpr int MAX_CHUNKS = 512; // attention chunks: max_seq <= MAX_CHUNKS * ATT_CHUNK

// Device-side step record: the token rows of this pass and where they go in the KV cache.
struct StepRec {
  int m;
  int start;
  int ids[MAX_M];
};

struct QKArgs {
  float *q, *k, *v;
  int64_t ld_q, ld_kv;
  const float *q_bias, *k_bias, *v_bias, *q_norm, *k_norm;
  const float2 *rope;       // [max_seq][head_dim/2] (cos, sin)
  __half *k_cache, *v_cache;
  int layer, max_seq, kv_dim, head_dim, n_heads, n_kv, neox;
  float eps;
};

struct AttnArgs {
  const float *q;
  int64_t ld_q;
  const __half *k_cache, *v_cache;
  float *part_m, *part_l, *part_o;   // [n_kv][16*g][max_chunks] (+ [head_dim])
  float *out;
  int64_t ld_out;
  int layer, max_seq, kv_dim, head_dim, n_heads, n_kv, max_chunks;
  float scale;
};

struct RouteArgs {
  const float *logits;
  int64_t ld_logits;
  int n_expert, n_used, norm;
  float moe_prune;
  int *chosen;       // [16][32]
  float *weights;    // [16][32]
  int *nkeep;        // [16]
  Job *jobs_gu, *jobs_dn;
  int *njobs;
  int *expert_count; // optional [n_expert] selection counter
};

struct SwigluArgs {
  float *g;
  const float *u;
  int64_t ld;
  int n;
  const Job *jobs;   // grouped: vectors = jobs' out indices; else rows 0..m-1
  const int *njobs;
  float *qd;
  int8_t *qq;
  int16_t *qb;
};

struct CombineArgs {
  const float *y;
  int64_t ld_y;
  const float *weights;
  const int *nkeep;
  int n_used, dim;
  float *out;
  int64_t ld_out;
};

hipError_t launch_embed(const TensorView &e, const StepRec *st, float *x, int64_t ld_x, float escale, int m, hipStream_t s);
hipError_t launch_res_norm(float *x, int64_t ld_x, const float *add, int64_t ld_add, float rscale, const float *w, int n, float eps,
                           float *out, int64_t ld_out, float *qd, int8_t *qq, int16_t *qb, const StepRec *st, int m, hipStream_t s);
hipError_t launch_qk_rope_kv(const QKArgs &a, const StepRec *st, int m, hipStream_t s);
hipError_t launch_attention(const AttnArgs &a, const StepRec *st, int m, hipStream_t s);
hipError_t launch_moe_route(const RouteArgs &a, const StepRec *st, hipStream_t s);
hipError_t launch_swiglu(const SwigluArgs &a, const StepRec *st, int nvec, hipStream_t s);
hipError_t launch_moe_combine(const CombineArgs &a, const StepRec *st, int m, hipStream_t s);
hipError_t launch_argmax(const float *logits, int64_t ld, int n, float lscale, int *out, const StepRec *st, int m, hipStream_t s);

}  // namespace spx
