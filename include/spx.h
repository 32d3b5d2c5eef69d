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

/* spx_matvec without any allocation: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in
 * the reference. The Q8_K staging of K-quant activations lives in a fixed device array of
 * SPX_NOALLOC_SCRATCH_BYTES per device (m * cols up to 786432 codes, e.g. 16 vectors of 49152
 * columns); larger requests are rejected with an error. Float formats need no staging. The array
 * is shared by every call on a device and fully rewritten by each call before use; calls from
 * different contexts (streams) take turns on it through a per-device event (each call's stream
 * waits for the previous call's kernels). Under graph capture that wait is skipped: captured
 * calls whose replays overlap on one device race. Same results, bit for bit, as spx_matvec. */
#define SPX_NOALLOC_SCRATCH_BYTES (1u << 20)
int spx_matvec_noalloc(spx_ctx *ctx, const spx_tensor *w, int expert, const float *x, int64_t ld_x,
                       int m, float *out, int64_t ld_out);

/* The routed experts of a MoE layer with the routing given (ffns_fused smollm_chat.rs:379-442
 * for m == 1; moe_batch_fused :650-760 with moe_forward_batch's combine :1133-1140 for m <= 16):
 * y[b] = sum over j < k, in j order, of weights[b*k + j] * FFN_e(x_b), e = chosen[b*k + j]
 * (each row's experts distinct), FFN_e = down_e(silu(gate_e x) * up_e x), each product and sum
 * rounded separately from 0. gate / up: [n_expert][n_ff][dim] (one format), down:
 * [n_expert][dim][n_ff]; K-quant matrices take Q8_K activations (x, then h), the others fp32.
 * x, y: device rows at x + b*ld_x, y + b*ld_y; chosen / weights: host arrays, read before the
 * call returns (the job list goes to the device with the launches; the call does not wait for
 * them). m * k <= 256, k <= 32. Each row's result does not depend on the others. */
int spx_moe(spx_ctx *ctx, const spx_tensor *gate, const spx_tensor *up, const spx_tensor *down, const float *x,
            int64_t ld_x, int m, int k, const int32_t *chosen, const float *weights, float *y, int64_t ld_y);

/* spx_moe with the routing in device memory (chosen / weights: device arrays [m][k], as a router
 * on the GPU leaves them; moe_batch_fused :650-760 with the combine :1133-1140): nothing waits
 * on the host, so the call can follow a device-side router in one stream or a captured graph.
 * K-quant experts only (gate / up Q4_K or Q6_K in one format, down Q4_K or Q6_K; dim and n_ff
 * multiples of 256 with 1, 2, 3, 4, 8 or 16 blocks a row, n_ff <= 1024, n_expert <= 256), on the
 * int8 matrix cores; m <= 128, k <= 32. A row whose ids are out of range or repeated gets NaN.
 * The same bits as spx_moe for the same routing. */
int spx_moe_dev(spx_ctx *ctx, const spx_tensor *gate, const spx_tensor *up, const spx_tensor *down, const float *x,
                int64_t ld_x, int m, int k, const int32_t *chosen, const float *weights, float *y, int64_t ld_y);

/* ------------------------------------------------------------------ synthetic weights */
/* Seeded synthetic tensor in GGUF block layout (n_expert slabs of rows x cols). kind 0:
 * quantized weights (Q4_K/Q6_K/Q8_0/Q5_0) whose dequantised values have std sigma; kind 1:
 * F32 uniform with std sigma; kind 2: F32 1 + sigma*U(-1,1) (norm weights). Host memory;
 * needs no GPU. No reference counterpart: the reference loads GGUF files only. */
int spx_synth_tensor(int dtype, int64_t cols, int64_t rows, int n_expert, uint64_t seed, float sigma,
                     int kind, void *out);

/* ------------------------------------------------------------------ engine */
/* Model hyperparameters (ModelConfig, smollm_chat.rs:38-120). attn_scale <= 0 means
 * 1/sqrt(head_dim); embedding/residual/logit scales of 0 mean 1 (the non-Granite default). */
typedef struct {
  int dim, n_heads, n_kv_heads, head_dim, n_layers, vocab, max_seq;
  float rope_theta, rms_eps;
  int rope_neox;
  int n_expert, n_expert_used, expert_norm;
  float moe_prune;
  float embedding_scale, residual_scale, logit_scale, attn_scale;
} spx_model_config;

typedef struct spx_engine spx_engine;

/* SmolLm2Engine::load_with_index (smollm_chat.rs:1905-2154), split in three: create with the
 * config, set every tensor by its GGUF name (resolve_layers :214-284: token_embd.weight,
 * output.weight (optional, tied otherwise), output_norm.weight, blk.N.{attn_norm, attn_q,
 * attn_k, attn_v, attn_output, attn_q_norm, attn_k_norm, ffn_norm, ffn_gate, ffn_up, ffn_down,
 * ffn_gate_inp, ffn_gate_exps, ffn_up_exps, ffn_down_exps}.weight, attn_{q,k,v}.bias), then
 * prepare (validates shapes, allocates the f16 KV cache [n_layers][max_seq][kv_dim]). */
int spx_engine_create(spx_ctx *ctx, const spx_model_config *cfg, spx_engine **out);
int spx_engine_set_tensor(spx_engine *e, const char *name, int dtype, int64_t cols, int64_t rows,
                          int n_expert, const void *ggml_bytes);
int spx_engine_prepare(spx_engine *e);
/* 1 (default): each pass length m is captured once into a HIP graph and replayed. */
int spx_engine_set_graphs(spx_engine *e, int on);
/* 1 (default): passes (forward_slice :3364-3552 for one token, forward_batch_slice :3142-3362
 * for 2..16 rows, as in the decode and verify steps of generate_reply :4205-4348) run on the
 * decode pipeline, launch chains whose kernels meet only at kernel boundaries; 0: on the fused
 * pass kernels. Both give the same values, bit for bit. The pipeline takes models whose
 * matrices are all Q4_K / Q6_K (others always use the fused kernels);
 * spx_engine_decode_pipeline reports whether passes use it. No counterpart in the reference
 * (a choice between two implementations of its passes). */
int spx_engine_set_decode(spx_engine *e, int on);
int spx_engine_decode_pipeline(spx_engine *e, int *active);  /* *active = 1: the pipeline runs */
/* 1 (default): the pipeline's passes of 2..16 rows (the verify step of generate_reply
 * :4251-4348, and prefill) take their integer matvecs on the int8 matrix cores: per block the
 * exact integer totals of the reference's kernel (rows<B,T>, quant_q8k.rs:163-245), their fp32
 * sums to rounding (a matvec within ~1e-6 relative of the lane-exact result; a whole pass can
 * differ more where that moves a downstream Q8_K code or a near-tied expert choice, and greedy
 * picks only at near-ties). 0: the lane-exact dot chains, the same bits as one-row passes, so
 * speculation reproduces plain greedy decoding bit for bit. No counterpart in the reference (a
 * choice between two implementations of its batched kernel). */
int spx_engine_set_mfma(spx_engine *e, int on);
/* One-row passes (decode) with each layer as one cooperative launch of co-resident workgroups
 * whose phases meet at device-wide barriers (the persistent pass, for Q4_K_M-format models with
 * head_dim 64 or 128): the same bits as the decode pipeline's kernels. Off by default (slower
 * than the pipeline as measured); set_persist(1) selects it where the model fits.
 * persist_active reports whether one-row passes take it. No counterpart in the reference,
 * whose passes are CPU loops (forward_slice smollm_chat.rs:3364-3552). */
int spx_engine_set_persist(spx_engine *e, int on);
int spx_engine_persist_active(spx_engine *e, int *active);

/* One pass of m <= 128 tokens at positions start_pos.. (forward_slice :3364-3552 for m == 1,
 * forward_batch_slice :3142-3362 for m > 1 — verify passes of k+1 rows and feed's prompt
 * chunks of up to 128 rows :3090-3101 — then compute_logits_batch :3588-3602 and the greedy
 * pick of sample_from_logits :3624-3671). K/V of every row are written before any row
 * attends, row b sees positions <= start_pos + b. A pass of more than 16 rows runs on the
 * prefill kernels (K-quant models, matrix cores on), else as consecutive passes of at most
 * 16 rows; either way each row gets the bits it would get in a pass of 16. Optional host
 * outputs: hidden [m][dim] (after output_norm), logits [m][vocab], argmax [m]. Synchronous. */
int spx_engine_forward(spx_engine *e, const int32_t *ids, int m, int start_pos, float *hidden,
                       float *logits, int32_t *argmax);
/* feed (smollm_chat.rs:3044-3104): the prompt ids[0..n) at positions start_pos.. in passes of
 * up to 128 rows (spx_engine_forward's passes, the same K/V bits), keeping only what feed keeps:
 * the last row's hidden state (after output_norm) and, as the reference computes them from it
 * afterwards, its logits and greedy pick. No LM head runs for the other rows. Optional host
 * outputs: hidden_last [dim], logits_last [vocab], argmax_last [1]. Synchronous. */
int spx_engine_feed(spx_engine *e, const int32_t *ids, int n, int start_pos, float *hidden_last,
                    float *logits_last, int32_t *argmax_last);
/* Greedy decoding of n tokens, one pass each (step_token :3106-3132 + the greedy pick):
 * feeds `token` at start_pos, then each pass's argmax at the next position; out[i] is the
 * token chosen by pass i. */
int spx_engine_decode(spx_engine *e, int32_t token, int start_pos, int n, int32_t *out);
/* Kernel timing: while on, passes run eagerly with a HIP event pair on the engine's stream
 * around every launch; totals per kernel class accumulate until the next spx_engine_profile(e,1).
 * bytes = algorithmic bytes (weights of the experts actually selected; KV for attention).
 * No reference counterpart (the reference keeps StepTiming per phase, smollm_chat.rs:1811-1858). */
int spx_engine_profile(spx_engine *e, int on);
int spx_engine_profile_read(spx_engine *e, int cls, const char **name, int64_t *launches,
                            double *total_us, double *bytes);
/* Copies `bytes` of an internal buffer of the last pass (x, xn, q, k, v, att, proj, rlog,
 * chosen, weights, nkeep, h, y: the last layer's values) to host memory; for tests. */
int spx_engine_debug_read(spx_engine *e, const char *what, void *host, int64_t bytes);
/* Layer snapshots for the layer-by-layer parity tests (no reference counterpart; the oracle's
 * stages are fed the GPU's own inputs). While on, passes run eagerly on the decode pipelines
 * (K-quant models; refused otherwise) and each layer l copies, for each row b < m of the pass,
 * its values into a device record read back with spx_engine_debug_read(e, "layers", ...):
 * record (l * 16 + b) * R + off[f] holds field f, f = 0 x_in (the residual entering layer l;
 * l = n_layers: the final residual), 1 q, 2 k, 3 v (raw projections), 4 att (attention output),
 * 5 proj (attn_output projection), 6 x_mid (x_in + residual_scale * proj), 7 router logits,
 * 8 h (the SwiGLU rows of the chosen experts in chosen order, n_used x n_ff; dense: n_ff),
 * 9 chosen (int32, 32 slots), 10 weights (32), 11 nkeep (int32); off[12] = R (floats a row).
 * spx_engine_debug_layout fills off[0..12]. */
int spx_engine_debug_layers(spx_engine *e, int on);
int spx_engine_debug_layout(spx_engine *e, int64_t *off);
/* Number of distinct experts each MoE layer ran in the last pass (0 for dense layers). */
int spx_engine_last_experts(spx_engine *e, int32_t *njobs_per_layer);
/* Per layer and expert: passes that selected the expert since prepare ([n_layers][n_expert]). */
int spx_engine_expert_counts(spx_engine *e, int32_t *counts);
/* The attention block of a pass (forward_batch_slice :3226-3300; forward_slice :3432-3470) for
 * m <= 16 rows at positions start_pos.. of one layer, on the engine's KV cache: q [m][q_dim],
 * k / v [m][kv_dim] are the projections' outputs (device); biases, per-head Q/K RMSNorm and
 * RoPE are applied, the rows' K / V written to the cache (f16 RNE), then row b attends to
 * positions <= start_pos + b; att [m][q_dim] (device) gets the heads' outputs. The same
 * kernels and bits as inside spx_engine_forward. */
int spx_engine_attention(spx_engine *e, int layer, const float *q, const float *k, const float *v, int m,
                         int start_pos, float *att);
/* The KV window (shift_kv :2944-2971, ensure_kv_room :2924-2940): shift_kv drops n_discard
 * positions (at most cur_pos - n_keep) after the n_keep pinned ones, moves the rest down and
 * re-rotates their keys by -n_discard (f16 -> f32 -> RoPE -> f16 RNE; values move as they are);
 * ensure_kv_room slides by max(overflow, half the unpinned context) when cur_pos + needed >
 * max_seq, and fails when the pinned positions leave no room. *new_pos = the next position. */
int spx_engine_shift_kv(spx_engine *e, int n_keep, int n_discard, int cur_pos, int *new_pos);
int spx_engine_ensure_kv_room(spx_engine *e, int n_keep, int cur_pos, int needed, int *new_pos);
/* Copies the f16 K and V caches ([n_layers][max_seq][kv_dim] each) to host memory. */
int spx_engine_kv_download(spx_engine *e, void *k_host, void *v_host);
int spx_engine_destroy(spx_engine *e);

/* ------------------------------------------------------------------ GGUF files */
/* A GGUF v2/v3 file opened read-only and mapped (GgufModelIndex::parse_file,
 * gguf_loader.rs:142-247): the metadata table, the tensor table, general.alignment (U32/U64,
 * at least 32, default 32) and the data section at the header's end rounded up to it; tensor
 * offsets are absolute file offsets. Strings over 16 MiB, unknown value types and nested
 * arrays are errors, as there. Host only, no GPU needed. */
typedef struct spx_gguf spx_gguf;
int spx_gguf_open(const char *path, spx_gguf **out);
int spx_gguf_close(spx_gguf *g);
int spx_gguf_info(const spx_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset,
                  int64_t *n_tensors, int64_t *n_meta);
/* Tensor i: name (valid until close), ggml type, dims (GGUF order: dims[0] = columns; unused
 * dims are 1) and absolute file offset. */
int spx_gguf_tensor(const spx_gguf *g, int64_t i, const char **name, int *dtype, int *n_dims, uint64_t *dims,
                    uint64_t *abs_offset);
int64_t spx_gguf_find(const spx_gguf *g, const char *name); /* index, -1 when absent */
/* Metadata: the GGUF value type of key (-1 absent); a non-negative integer of any integer
 * type (GgufValue::as_usize :88-101); a number as f32 (as_f32 :104-110); bool; string (valid
 * until close); an array's element type and count. Each fails when the key has no such value. */
int spx_gguf_meta_type(const spx_gguf *g, const char *key);
int spx_gguf_meta_index(const spx_gguf *g, const char *key, uint64_t *out);
int spx_gguf_meta_f32(const spx_gguf *g, const char *key, float *out);
int spx_gguf_meta_bool(const spx_gguf *g, const char *key, int *out);
int spx_gguf_meta_str(const spx_gguf *g, const char *key, const char **out);
int spx_gguf_meta_array(const spx_gguf *g, const char *key, int *elem_type, uint64_t *count);
/* tokenizer.ggml.tokens: count (0 when absent) and token strings (NULL out of range). */
int64_t spx_gguf_vocab_size(const spx_gguf *g);
const char *spx_gguf_token(const spx_gguf *g, int64_t id);
/* ModelConfig::from_gguf (smollm_chat.rs:69-120): architecture llama / granite / granitemoe
 * (rope pairs) or qwen2 / qwen2moe / qwen3 / qwen3moe / olmoe (NeoX halves); softmax gating
 * only; required embedding_length, attention.head_count, block_count; head_count_kv,
 * key_length, context_length (-> max_seq, default 2048), rope.freq_base (10000),
 * layer_norm_rms_epsilon (1e-5), expert counts, expert_weights_norm (default: true except
 * qwen2moe / olmoe), Granite's embedding / residual / logit scales and attention.scale;
 * head_dim a multiple of 8 and n_heads a multiple of n_kv_heads. vocab = the tokenizer
 * table's length (without one: token_embd's rows). */
int spx_gguf_config(const spx_gguf *g, spx_model_config *cfg);
/* The stop ids of load_with_index_sharded (:1925-1936): eos_token_id, then <|endoftext|>,
 * <|im_end|>, <|end_of_text|> where the vocabulary has them, without repeats (*n = how many;
 * the first cap are written); <think> / </think> ids (:1937) or -1 / -1. */
int spx_gguf_stop_ids(const spx_gguf *g, int32_t *ids, int cap, int *n);
int spx_gguf_think_ids(const spx_gguf *g, int32_t *open_id, int32_t *close_id);
/* Fails when a tensor's rows end past the file's end (a cut-off download, :1944-1963). */
int spx_gguf_check(const spx_gguf *g);
/* SmolLm2Engine::load (:1887-2154) onto the GPU: the config from the file (max_seq > 0
 * overrides context_length; moe_prune as set_moe_prune :2401), resolve_layers' tensors
 * (:214-284) uploaded from the mapping, prepared. Refused like there: old per-expert Mixtral
 * tensors, MoE tensors without expert counts; and what this engine does not run: shared
 * experts, whole-projection Q/K norms (OLMoE). */
int spx_engine_load_gguf(spx_ctx *ctx, const spx_gguf *g, int max_seq, float moe_prune, spx_engine **out);

/* Prompt-lookup drafting (lookup_draft, smollm_chat.rs:2982-3015) with the n-gram range as a
 * parameter: the reference uses min_ngram 2, max_ngram 4. Returns the draft length. */
int spx_lookup_draft(const int32_t *corpus, int n, int k, const int32_t *stop_ids, int n_stop,
                     int min_ngram, int max_ngram, int32_t *draft, int *ngram);

/* The speculative loop's draft-length model (SpecModel, smollm_chat.rs:1670-1809), the object
 * spx_engine_generate drives: accept rates per draft class decayed by 0.97 (floor 0.5), the
 * one-token step cost and the per-extra-row verify cost, which choose how many drafted tokens
 * a verify takes. For a host that runs its own loop over spx_engine_forward. Classes: 0 =
 * 1-2-gram lookup, 1 = 3-gram, 2 = 4+-gram, 3 = draft model; times in whole microseconds.
 * Entry points returning int give -1 on a null model or an argument out of range. */
typedef struct spx_spec_model spx_spec_model;
spx_spec_model *spx_spec_create(int fixed);            /* SpecModel::default, fixed = SPINDLE_SPEC_FIXED (:1693-1706) */
spx_spec_model *spx_spec_clone(const spx_spec_model *m); /* Clone */
void spx_spec_destroy(spx_spec_model *m);
int spx_spec_class(int ngram);                                      /* SpecModel::class (:1710) */
double spx_spec_accept_rate(const spx_spec_model *m, int cls);      /* :1719 */
int spx_spec_best_len(spx_spec_model *m, int cls, int avail);       /* :1728 */
void spx_spec_reset_rates(spx_spec_model *m);                       /* :1756 */
int spx_spec_record_draft(spx_spec_model *m, int cls, int drafted, int accepted); /* :1763 */
void spx_spec_record_step(spx_spec_model *m, uint64_t us);          /* :1777 */
void spx_spec_record_verify(spx_spec_model *m, int rows, uint64_t us); /* :1788 */

typedef struct {
  int draft_len;     /* k: tokens proposed per verify (draft_len, :1952) */
  int min_ngram, max_ngram;
  int fixed;         /* SPINDLE_SPEC_FIXED: always verify the whole draft (:1703) */
  int speculate;     /* 0: plain one-token decoding */
  int adaptive_k;    /* grow k after a fully accepted draft (:4343) */
  int prefill_chunk; /* prompt rows per pass, <= 128; 0: 128 (feed's chunks :3090) */
  int n_cached;      /* prompt tokens already in the KV cache at positions 0..n_cached-1 (a
                        session's earlier turns, generate_reply's cur_pos): only the rest of the
                        prompt is fed; 0 <= n_cached < n_prompt */
  int kv_keep;       /* n_keep: positions the sliding window never evicts (the system prompt);
                        before each pass the window slides as ensure_kv_room does */
} spx_gen_params;

typedef struct {
  int accepted, drafted, verifies, steps; /* spec_stats (:1642-1643) plus one-token steps */
  double prefill_us, step_us, verify_us;  /* host wall time of the passes */
} spx_gen_stats;

/* Token sampling (SamplerConfig :1523-1555, sample_from_logits :3624-3726, SplitMix64
 * :1557-1572) over device logits: logits / logit_scale; the repeat penalty on each distinct
 * token of the window (positive / p, others * p); stop ids to -inf while forbid_stop, the
 * think-open id while forbid_think; then temperature <= 0: the last maximum under f32 total
 * order; else top-k (0: every finite logit) by logit, softmax with temperature (the C
 * library's expf, sequential sums), min-p, top-p, one SplitMix64 draw. Candidates with equal
 * logits rank by ascending id (the reference's unstable sorts leave that order unspecified).
 * The per-vocabulary work runs on the GPU (top_k up to 1024 selected there; top_k 0 or above
 * 1024 copies the processed rows to the host and sorts them there); the O(k) tail on the host. */
typedef struct {
  float temperature;       /* 0.6 in the reference's default */
  int top_k;               /* 40 */
  float top_p, min_p;      /* 0.9, 0.05 */
  float repeat_penalty;    /* 1.1 */
  uint64_t seed;           /* SplitMix64 state at creation */
  const int32_t *stop_ids; /* copied at creation */
  int n_stop;
  int think_open;          /* -1: none */
} spx_sampler_params;
typedef struct spx_sampler spx_sampler;
int spx_sampler_create(spx_ctx *ctx, const spx_sampler_params *p, int vocab, spx_sampler **out);
int spx_sampler_destroy(spx_sampler *s);
int spx_sampler_reseed(spx_sampler *s, uint64_t seed);  /* set_sampler's SplitMix64(seed) (:2238) */
/* sample_from_logits for one row of vocab device logits. */
int spx_sample(spx_sampler *s, const float *logits, float logit_scale, const int32_t *recent, int n_recent,
               int forbid_stop, int forbid_think, int32_t *token);
/* The verify loop's sampling (:4305-4331): rows 0..n_draft of a pass (row i at logits + i*ld)
 * sampled in order, row i over the window recent + draft[0..i) with stop ids forbidden while
 * generated + i < 2, until a sample differs from draft[i] (the correction) or row n_draft (the
 * bonus token). tokens gets the accepted drafts then that token (*n_out = accepted + 1); when
 * accepted reaches max_accept first (the reply is full), no further row is drawn and
 * *n_out = accepted. */
int spx_sample_verify(spx_sampler *s, const float *logits, int64_t ld, int n_draft, float logit_scale,
                      const int32_t *recent, int n_recent, const int32_t *draft, int generated, int max_accept,
                      int forbid_think, int32_t *tokens, int *n_out);
/* The engine's sampler for spx_engine_generate (a copy of p, its SplitMix64 state kept across
 * calls like the reference's engine); NULL: plain greedy, no penalty, no stop ids. */
int spx_engine_set_sampler(spx_engine *e, const spx_sampler_params *p);

/* A draft model for spx_engine_generate (draft_engine, generate_reply :4244-4269; NULL: prompt
 * lookup). The draft engine is fed the same prompt; before each verify it catches up on the
 * committed tokens it has not seen, one pass each, then proposes up to k tokens with its own
 * pick (greedy, or its sampler with no penalty window), stopping at its stop ids; after the
 * verify its position falls back to the committed tokens. Drafting stops for the rest of a
 * reply once either window slides. The engine must outlive its use here. */
int spx_engine_set_draft(spx_engine *e, spx_engine *draft);

/* Generation with prompt-lookup speculation (generate_reply's loop :4205-4348 minus chat
 * framing): feeds the prompt from position n_cached, writes up to max_new tokens to out and
 * returns how many. Tokens come from the engine's sampler (spx_engine_set_sampler) over the
 * tokens of this call so far, stop ids forbidden while fewer than 2 are out and ending the
 * reply before one is emitted; without a sampler, plain greedy picks. */
int spx_engine_generate(spx_engine *e, const int32_t *prompt, int n_prompt, int max_new,
                        const spx_gen_params *params, int32_t *out, spx_gen_stats *stats);

#ifdef __cplusplus
}
#endif
#endif
