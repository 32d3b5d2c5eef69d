/*
 * oracle.h -- CPU restatement of WiseHax/spindle's decode/verify arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (spindle_amd/, include/) may link,
 * import or call this code. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / the timed CPU baseline.
 *
 * Every function restates the reference's operation order (8-lane AVX2 accumulators,
 * the two horizontal-sum trees, non-contracted scalar arithmetic) so that its fp32 bit
 * patterns are the reference's, not merely close to them. Build with -ffp-contract=off
 * and without -ffast-math; fused multiply-adds appear only where the reference issues
 * _mm256_fmadd_ps and are written as fmaf().
 *
 * Pinning (what checks each function; see tests/test_oracle_*.py):
 *   or_f16_to_f32 / or_f32_to_f16 ...... exhaustive over all 65536 halfs (round trip),
 *                                         numpy float16 as the independent RNE reference
 *   or_unpack_q4k_scales / or_dequant_row  known-answer block from the reference's
 *                                         transformer.rs:311-316 (hand-derived expectation),
 *                                         numpy restatement from the ggml format text
 *   or_q8k_quantize .................... reference property test quant_q8k.rs:342-362
 *                                         (round trip <= amax/254, bsums = sums of qs)
 *   or_q8k_block_sums .................. brute-force integer identity on tiny inputs
 *   or_q8k_matmul_rows ................. reference test quant_q8k.rs:364-411 (f64 dot of
 *                                         dequantized weights and dequantized Q8_K, 1e-4) and
 *                                         :413-442 (batch bitwise); lane split checked by
 *                                         recomputing sum from per-lane int partials
 *   or_matvec_rows / or_matmul_rows_multi  reference test quant.rs:1727-1771 and
 *                                         quant_multi.rs:369-417 (f64 dot, 1e-4)
 *   or_rope_* .......................... textbook rope smollm_chat.rs:4852-4886 + composition
 *   or_moe_* ........................... loop reference smollm_chat.rs:4936-4973 (1e-4)
 *   or_lookup_draft / or_spec_* ........ hand-built corpora / the reference test
 *                                         smollm_chat.rs:4667-4694
 *   or_forward_* ....................... a float64 numpy forward restated from the formulas
 *                                         (tests/test_oracle_forward.py: GQA hpk 1/3/8, hd 64/128,
 *                                         both RoPE layouts, QK-norm, Granite scales, pruning;
 *                                         a planted head-mapping mistake must fail), and batched
 *                                         == sequential on all-K-quant models (bitwise)
 *   MoE routing / pruning .............. hand-derived choice lists for both pruning rules and
 *                                         for exact ties (tests/test_oracle_ops.py)
 *   or_argmax .......................... last maximum under total order, -0/+0, NaN, scale
 * Parity unpinned at the bit level (no reference build exists here: no Rust toolchain):
 *   the exact fp32 bits of expf/sinf/cosf/powf (Rust's libm vs glibc), and the order of
 *   exactly tied router probabilities (select_nth_unstable_by is implementation-defined).
 */
#ifndef SPX_ORACLE_H
#define SPX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (gguf_loader.rs:24-42). */
enum {
  OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q4_1 = 3, OR_Q5_0 = 6, OR_Q5_1 = 7,
  OR_Q8_0 = 8, OR_Q4K = 12, OR_Q5K = 13, OR_Q6K = 14, OR_BF16 = 30
};

/* ---- formats (quant.rs:876-899, 1504-1660; q4k_gemv.rs:70-85) ---- */
size_t or_row_bytes(int dtype, size_t cols); /* 0 = unsupported / bad width */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f); /* round to nearest even, like _mm256_cvtps_ph */
void or_unpack_q4k_scales(const uint8_t sc[12], uint8_t s[8], uint8_t m[8]);
int or_dequant_row(int dtype, const uint8_t *row, size_t cols, float *out);

/* ---- Q8_K activations (quant_q8k.rs:59-121) ---- */
void or_q8k_quantize(const float *x, size_t n, float *d, int8_t *qs, int16_t *bsums);

/* ---- integer K-quant kernel (quant_q8k.rs:163-295) ----
 * outs[b][r] for r in [r0,r1). xd/xs/xb: per vector Q8_K (d, qs, bsums). */
void or_q8k_matmul_rows(const uint8_t *tensor, int dtype, size_t cols, int nvec,
                        const float *const *xd, const int8_t *const *xs,
                        const int16_t *const *xb, float *const *outs, size_t r0, size_t r1);
/* Per-block integer quantities of one row against one Q8_K vector: sumi[i] = sum over the
 * eight 32-bit lanes of the block's scaled dot (quant_q8k.rs:235-242), corr[i] = the
 * integer inside the min/offset correction (Q4_K :198-204, Q6_K :226-232; for Q6_K this is
 * 32*s, the value converted to f32 there). lanes (optional, 8 per block) = the per-lane
 * int32 partials. */
void or_q8k_block_sums(const uint8_t *row, int dtype, size_t cols, const int8_t *xs,
                       const int16_t *xb, int32_t *sumi, int32_t *corr, int32_t *lanes);

/* ---- float kernels ----
 * M=1 (quant.rs:937-1094): out[i] = row r0+i. Supported: F32, F16, Q8_0, Q5_0, Q5_K. */
int or_matvec_rows(const uint8_t *tensor, int dtype, size_t cols, const float *x, float *out,
                   size_t r0, size_t nrows);
/* M>1 shared-decode (quant_multi.rs:124-273): Q8_0, F32; others fall back per vector. */
int or_matmul_rows_multi(const uint8_t *tensor, int dtype, size_t cols, int nvec,
                         const float *const *xs, float *const *outs, size_t r0, size_t r1);

/* ---- operator boundary (smollm_chat.rs:304-512) ---- */
typedef struct { int dtype; size_t cols, rows; const uint8_t *data; } or_mat;
int or_matvec(const or_mat *m, const float *x, float *out);
int or_matvec_multi(const or_mat *m, int nvec, const float *const *xs, float *const *outs);
or_mat or_expert(or_mat m, int e);

/* ---- small ops (smollm_chat.rs:528-588, 1394-1420) ---- */
void or_rmsnorm(const float *x, const float *w, float *out, size_t n, float eps);
void or_rmsnorm_heads(float *v, const float *w, size_t len, size_t head_dim, float eps);
float or_silu(float x);
void or_rope_inv_freq(size_t head_dim, float theta, float *inv_freq);
void or_rope_rotate(const float *inv_freq, int neox, float *v, size_t len, size_t head_dim, float pos);

/* ---- model (smollm_chat.rs:38-284, 1574-1668) ---- */
typedef struct {
  int dim, n_heads, n_kv_heads, head_dim, n_layers, vocab, max_seq;
  float rope_theta, rms_eps;
  int rope_neox;
  int n_expert, n_expert_used, expert_norm;
  float moe_prune;
  float embedding_scale, residual_scale, logit_scale, attn_scale; /* attn_scale<=0: 1/sqrt(hd) */
} or_config;

typedef struct {
  const float *attn_norm, *ffn_norm;
  or_mat wq, wk, wv, wo;
  const float *q_bias, *k_bias, *v_bias, *q_norm, *k_norm;
  int qk_norm_full;
  int is_moe;
  or_mat gate, up, down, router; /* dense: gate/up/down; MoE: expert tensors + router */
} or_layer;

typedef struct {
  or_config c;
  or_layer *layers;
  or_mat embed, lm_head;
  const float *output_norm;
  uint16_t *k_cache, *v_cache; /* [n_layers][max_seq][kv_dim] f16 */
  float *inv_freq;             /* head_dim/2, filled by or_model_init */
  /* statistics of the last MoE layer evaluation (tests) */
  int last_chosen[16 * 32];
  /* optional debug capture (tests): forward_slice copies the last layer's q (after RoPE),
   * attention output, attention projection and FFN output here when non-null */
  float *dbg_q, *dbg_att, *dbg_proj, *dbg_ffn;
} or_model;

void or_model_init(or_model *m);
/* forward_slice: one token at pos -> output-normed hidden (smollm_chat.rs:3364-3552) */
int or_forward_slice(or_model *m, int token, int pos, float *hidden);
/* shift_kv (smollm_chat.rs:2944-2971) on f16 caches [n_layers][max_seq][kv_dim]: drops n_discard
 * positions after the n_keep pinned ones (clamped to cur_pos - n_keep), moves the rest down and
 * re-rotates each moved K by -n_discard (f16 -> f32, Rope::rotate, f32 -> f16 RNE); V moves as
 * is. Returns the new cur_pos. */
int or_shift_kv(uint16_t *k_cache, uint16_t *v_cache, int n_layers, int max_seq, int kv_dim, int head_dim, int neox,
                const float *inv_freq, int n_keep, int n_discard, int cur_pos);
/* ensure_kv_room (:2924-2940): when cur_pos + needed > max_seq, discards max(overflow, half of
 * the unpinned context), at most all of it; returns the new cur_pos. */
int or_ensure_kv_room(or_model *m, int n_keep, int cur_pos, int needed);
/* qkv_post + attention for n rows at start..start+n-1: q [n][q_dim], k, v [n][kv_dim] are the raw
 * projections (bias, q/k norms, RoPE applied in place), their K/V rows written to the cache
 * first; att [n][q_dim] (forward_slice :3401-3495, forward_batch_slice :3235-3319). */
int or_attn_rows(or_model *m, int layer, int n, int start, float *q, float *k, float *v, float *att);
/* One layer on x [n][dim] in place (forward_slice's layer for n == 1, forward_batch_slice's for
 * n > 1); the rows' K/V written at start..start+n-1. */
int or_layer_forward(or_model *m, int layer, int n, int start, float *x);
/* forward_batch_slice: m tokens at start_pos (m==1 delegates to forward_slice) */
int or_forward_batch(or_model *m, const int *ids, int n, int start_pos, float *hidden);
/* LM head: matvec (n==1) or matvec_multi (smollm_chat.rs:3560-3602) */
int or_logits(or_model *m, const float *hidden, int n, float *logits);
/* greedy: logit_scale, then argmax with the last maximum on ties (:3624-3671) */
int or_argmax(const float *logits, int n, float logit_scale);

/* MoE layer on its own (moe_forward / moe_forward_batch, :925-1392) */
int or_moe_forward(const or_config *c, const or_layer *ly, int n, const float *const *xs,
                   float *const *outs, int *chosen_out, int *nkeep_out);
/* ffns_fused's down pass and combine (:410-437): out += sum_e w_e down_e(h_e), h: k rows of
 * down->cols (Q8_K-quantized for an integer down), adds in chosen order */
int or_down_combine(const or_mat *down, int k, const int *experts, const float *weights, const float *h, float *out);
/* fused SwiGLU job, M=1 (ffns_fused :379-442): out += sum_e w_e FFN_e(x) */
int or_ffns_fused(const or_mat *gate, const or_mat *up, const or_mat *down, int k,
                  const int *experts, const float *weights, const float *x, float *out);

/* ---- speculation (smollm_chat.rs:1670-1809, 2973-3015, 4205-4348) ---- */
int or_lookup_draft(const int *corpus, int n, int k, const int *stop_ids, int n_stop,
                    int min_ngram, int max_ngram, int *draft, int *ngram);

typedef struct {
  double acc[4], fail[4], t1_us, extra_us;
  int have_t1, have_extra, since_try, fixed;
} or_spec_model;
void or_spec_init(or_spec_model *s, int fixed);
int or_spec_class(int ngram);
double or_spec_accept_rate(const or_spec_model *s, int c);
int or_spec_best_len(or_spec_model *s, int c, int avail);
void or_spec_reset_rates(or_spec_model *s);
void or_spec_record_draft(or_spec_model *s, int c, int drafted, int accepted);
void or_spec_record_step(or_spec_model *s, uint64_t us);
void or_spec_record_verify(or_spec_model *s, int b, uint64_t us);

typedef struct {
  int draft_len;   /* k */
  int min_ngram, max_ngram;
  int fixed;       /* SPINDLE_SPEC_FIXED */
  int speculate;   /* 0: plain decode */
  int adaptive_k;  /* k_dyn growth after full accepts (:4343) */
  int prefill_chunk;
  int n_cached;    /* prompt tokens already in the KV cache (positions 0..n_cached-1) */
  int kv_keep;     /* n_keep: positions the sliding window never evicts */
} or_gen_params;

typedef struct { int accepted, drafted, verifies, steps; } or_gen_stats;

/* ---- sampling (SamplerConfig :1523-1555, SplitMix64 :1557-1572, sample_from_logits :3624-3726) */
typedef struct {
  float temperature;   /* <= 0: greedy */
  int top_k;           /* 0: every finite logit */
  float top_p, min_p, repeat_penalty;
  uint64_t seed;
  const int *stop_ids; /* -inf while forbid_stop; generation ends on one */
  int n_stop;
  int think_open;      /* -1: none; -inf while forbid_think */
} or_sampler_params;
typedef struct { or_sampler_params p; uint64_t rng; } or_sampler;
void or_sampler_init(or_sampler *s, const or_sampler_params *p);
uint64_t or_splitmix_next(uint64_t *state);
float or_splitmix_f32(uint64_t *state);
/* One token from one row of logits; recent = the penalty window (ids outside 0..vocab-1 are
 * skipped, repeats count once). Candidates equal under total order are ordered by index. */
int or_sample(or_sampler *s, const float *logits, int vocab, float logit_scale, const int *recent, int n_recent,
              int forbid_stop, int forbid_think);

/* Generation with prompt-lookup speculation (generate_reply minus chat framing). Writes up to
 * max_new tokens; returns the count. Greedy, no penalty, no stop ids: */
int or_generate(or_model *m, const int *prompt, int n_prompt, int max_new,
                const or_gen_params *p, int *out, or_gen_stats *st);
/* ... and with a sampler: every token drawn by or_sample over the reply's tokens so far, stop
 * ids forbidden while fewer than 2 are out, generation ending before a stop id. */
int or_generate_sampled(or_model *m, const int *prompt, int n_prompt, int max_new, const or_gen_params *p,
                        or_sampler *s, int *out, or_gen_stats *st);
/* ... and with a draft model (draft_engine :4244-4269, greedy draft picks) instead of prompt
 * lookup when draft is not NULL. */
int or_generate_full(or_model *m, or_model *draft, const int *prompt, int n_prompt, int max_new, const or_gen_params *p,
                     or_sampler *s, int *out, or_gen_stats *st);

void or_set_threads(int n);
/* 1 (default): the integer rows kernel and attention with the reference's AVX2 instructions;
 * 0: the scalar restatement (the same bits; the tests compare the two). */
void or_set_simd(int on);
/* Test knob, off by default: 1 = RMSNorm sums in the GPU kernels' order (sensitivity tests). */
void or_set_norm_order(int gpu_order);
/* Test capture, off by default: or_ffns_fused copies its k x n_ff SwiGLU rows to h (NULL: off). */
void or_set_dbg_h(float *h);
int or_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
