// The KV window's slide on the device (kv.hip).
#pragma once
#include "common.h"

namespace spx {

struct KVShiftArgs {
  __half *kc, *vc;
  __half *kt, *vt;       // staging [n_layers][n_move][kv_dim]
  const float2 *cs;      // [head_dim / 2]: cos, sin of -n_discard * inv_freq[i]
  int n_layers, max_seq, kv_dim, head_dim, neox, n_keep, n_discard, n_move;
};

hipError_t launch_kv_shift(const KVShiftArgs &a, hipStream_t s);

}  // namespace spx
