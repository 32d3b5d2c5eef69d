// The layers of the one-row decode pass (forward_slice smollm_chat.rs:3364-3552) as cooperative
// launches of co-resident workgroups, one a layer, whose phases meet at device-wide barriers
// instead of kernel boundaries (persist.hip). Every phase computes what the decode pipeline's
// kernel for it computes (decode.hip, attention in attn.h), operation for operation, so a pass
// gives the same bits on both; what changes is that each phase's weights are pulled into L2 one
// phase ahead, while the previous phase and its barrier are still running. The embedding, LM
// head and greedy pick stay the pipeline's kernels.
#pragma once
#include "decode.h"

namespace spx {

// One layer's tensors.
struct PLayer {
  TensorView wq, wk, wv, wo, router, gate, up, down;
  const float *attn_norm, *ffn_norm, *q_norm, *k_norm, *q_bias, *k_bias, *v_bias;
  int moe;
  int *njobs;          // [1] kept experts of the pass (routing statistics)
  int *expert_count;   // [n_expert] selection counter (null: none)
};

struct PersistArgs {
  int n_layers;
  TensorView lm_head;
  const float *out_norm;
  int dim, q_dim, kv_dim, hd, n_heads, n_kv, n_ff, n_expert, n_used, expert_norm;
  float moe_prune, eps, rscale, lscale, attn_scale;
  int neox, max_seq, nch, nslot;
  float *xa, *xb;       // residual stream: the embedding in xa; a layer goes xa -> xb -> xa
  float *q, *k, *v, *att, *h, *rlog, *logits, *xn;
  float *part_ml, *part_o;
  __half *kc, *vc;
  const float2 *rope;
  unsigned long long *best;  // [grid] greedy keys of the LM head's workgroups
  int *chosen, *nkeep;
  float *weights;
  StepRec *st;
  int *hist, *amax;
  unsigned *bar;        // barrier counters, zero at launch (PERSIST_BAR_WORDS)
  int *err;             // set when a barrier waits longer than its limit (the pass is void)
  int advance;          // the pick becomes the next pass's token (back-to-back decoding)
  uint64_t *tstamp;     // optional [n_layers][16]: real-time counter at each phase end (workgroup 0)
};

constexpr int PERSIST_NT = 256;          // threads per workgroup
constexpr int PERSIST_BAR_WORDS = 32 * 34;  // top counter + 32 sub-counters, 128 bytes apart

// Workgroups of a launch: two a CU when the kernel fits that many (0: the device cannot hold
// the grid at once, and the persistent pass must not be used).
int persist_grid(int hd, int n_cu);
// Whether a model's shapes fit the kernel's register tiles (see persist.hip).
bool persist_fits(const PersistArgs &a, int grid);
// Barriers a layer's launch passes: 6 for a MoE layer (after q|k|v, attention, merge, wo,
// router, gate/up), 5 for a dense one. epoch0: the barriers of the pass's earlier layers.
inline int persist_layer_barriers(bool moe) { return moe ? 6 : 5; }
// ly: the layer's tensors, passed by value (kernel arguments are read with scalar loads, which
// never wait on the vector loads in flight)
hipError_t launch_persist_layer(const PersistArgs &a, const PLayer &ly, int layer, unsigned epoch0, int grid, hipStream_t s);

}  // namespace spx
