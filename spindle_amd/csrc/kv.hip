// The KV window's slide (shift_kv, smollm_chat.rs:2944-2971) on the f16 caches
// [n_layers][max_seq][kv_dim]: positions n_keep + n_discard .. cur_pos - 1 move down by n_discard,
// each moved key re-rotated by -n_discard (f16 -> f32, the RoPE pair rotation with the shift's
// cos / sin, f32 -> f16 round to nearest even), values copied as they are. Moves overlap, so a
// first launch reads every moved row into a staging buffer and a second writes them back.
#include "kv.h"

namespace spx {


// One thread per (layer, moved row, rotation pair): reads the pair of K and V, writes the
// rotated K pair and the V pair to the staging rows.
__global__ __launch_bounds__(256) void k_kv_stage(const KVShiftArgs a) {
  const int half = a.head_dim / 2, pairs = a.kv_dim / 2;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x, per_layer = (int64_t)a.n_move * pairs;
  if (t >= per_layer * a.n_layers) return;
  const int l = (int)(t / per_layer), r = (int)((t % per_layer) / pairs), q = (int)(t % pairs);
  const int h = q / half, i = q % half;  // head, pair within the head
  const int da = h * a.head_dim + (a.neox ? i : 2 * i), db = h * a.head_dim + (a.neox ? i + half : 2 * i + 1);
  const int64_t src = ((int64_t)l * a.max_seq + a.n_keep + a.n_discard + r) * a.kv_dim;
  const int64_t dst = ((int64_t)l * a.n_move + r) * a.kv_dim;
  const float x0 = __half2float(a.kc[src + da]), x1 = __half2float(a.kc[src + db]);
  const float c = a.cs[i].x, s = a.cs[i].y;
  a.kt[dst + da] = __float2half_rn(__fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s)));
  a.kt[dst + db] = __float2half_rn(__fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c)));
  a.vt[dst + da] = a.vc[src + da];
  a.vt[dst + db] = a.vc[src + db];
}

// Staging rows back to positions n_keep .. n_keep + n_move - 1, four halves a thread.
__global__ __launch_bounds__(256) void k_kv_commit(const KVShiftArgs a) {
  const int q4 = a.kv_dim / 4;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x, per_layer = (int64_t)a.n_move * q4;
  if (t >= per_layer * a.n_layers) return;
  const int l = (int)(t / per_layer), r = (int)((t % per_layer) / q4), j = (int)(t % q4);
  const int64_t src = ((int64_t)l * a.n_move + r) * a.kv_dim + 4 * j;
  const int64_t dst = ((int64_t)l * a.max_seq + a.n_keep + r) * a.kv_dim + 4 * j;
  *reinterpret_cast<uint2 *>(a.kc + dst) = *reinterpret_cast<const uint2 *>(a.kt + src);
  *reinterpret_cast<uint2 *>(a.vc + dst) = *reinterpret_cast<const uint2 *>(a.vt + src);
}

hipError_t launch_kv_shift(const KVShiftArgs &a, hipStream_t s) {
  if (a.kv_dim % 4 || a.head_dim % 2 || a.n_move < 0) return hipErrorInvalidValue;
  if (a.n_move == 0) return hipSuccess;
  const int64_t n1 = (int64_t)a.n_layers * a.n_move * (a.kv_dim / 2), n2 = (int64_t)a.n_layers * a.n_move * (a.kv_dim / 4);
  hipLaunchKernelGGL(k_kv_stage, dim3((unsigned)((n1 + 255) / 256)), dim3(256), 0, s, a);
  hipLaunchKernelGGL(k_kv_commit, dim3((unsigned)((n2 + 255) / 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace spx
