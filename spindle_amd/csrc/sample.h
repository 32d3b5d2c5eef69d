// Token sampling (sample_from_logits, smollm_chat.rs:3624-3726) over device logits: the O(vocab)
// part on the GPU (logit_scale, repeat penalty, stop / think masks, the greedy key and a radix
// top-k selection sorted by logit), the O(k) tail on the host (softmax with temperature, min-p,
// top-p and the SplitMix64 draw), where the C library's expf gives the reference's own
// probabilities bit for bit. Used by spx_sample*, and by the engine's generate loop.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "../../include/spx.h"

namespace spx {

constexpr int SAMPLE_KMAX = 1024;         // top_k selected on the device; larger (or 0) -> whole row
constexpr int SAMPLE_VMAX = 1 << 19;      // vocabulary bound of the LDS bitmaps
constexpr int SAMPLE_MMAX = 16;           // rows per call

struct Sampler {
  spx_sampler_params p{};
  std::vector<int32_t> stop;  // copy of p.stop_ids
  uint64_t rng = 0;           // SplitMix64 state
  int vocab = 0;
  hipStream_t stream = nullptr;
  int device = 0;
  // device: processed logits [MMAX][vocab], candidates, row summaries, the id lists
  float *d_scratch = nullptr;
  int32_t *d_cidx = nullptr, *d_meta = nullptr, *d_ids = nullptr;
  // pinned host copies
  int32_t *h_cidx = nullptr, *h_meta = nullptr, *h_ids = nullptr;
  float *h_cval = nullptr, *d_cval = nullptr, *h_row = nullptr;
  int ids_cap = 0;
  std::vector<float> probs;
  std::vector<int32_t> order;

  ~Sampler();
  int init(const spx_sampler_params *p, int vocab, int device, hipStream_t s);
  bool greedy_plain() const;  // temperature <= 0, penalty 1, nothing masked: the plain argmax
  // Device part for rows 0..m-1 of logits (row r at logits + r * ld): row r's penalty window is
  // window[0 .. n_window + r) (a verify's drafts appended after the reply's tokens), stop ids
  // masked on row r when bit r of forbid_stop_rows is set. Waits for the results.
  int prepare(const float *logits, int64_t ld, int m, float logit_scale, const int32_t *window, int n_window,
              uint32_t forbid_stop_rows, bool forbid_think);
  // Host tail of row r after prepare (consumes one draw when it samples).
  int pick(int r);
  uint64_t next_u64();
  float next_f32();
};

}  // namespace spx
