// Q8_K activation quantization on gfx950 (quantize_avx2, quant_q8k.rs:84-121).
// One wavefront per 256-value block: lane l holds x[4l..4l+3]; amax and the codes as
// q8k_amax / q8k_codes state (the reference's max order, NaN included), bsums = sums of 16
// codes, in the reference's plain layout.
#include "dev.h"

namespace spx {

__global__ __launch_bounds__(256) void k_q8k_quantize(const float *x, int64_t n, int64_t ld_x, int m,
                                                      float *d, int8_t *qs, int16_t *bsums) {
  const int lane = threadIdx.x & 63;
  const int64_t nblk = n / 256;
  const int64_t gb = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gb >= nblk * m) return;
  const int64_t v = gb / nblk, b = gb % nblk;
  const float4 xv = reinterpret_cast<const float4 *>(x + v * ld_x + b * 256)[lane];
  const float am = q8k_amax(xv);
  int q[4];
  const float dv = q8k_codes(xv, am, q);
  const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) | ((uint32_t)(q[2] & 0xff) << 16) |
                          ((uint32_t)(q[3] & 0xff) << 24);
  reinterpret_cast<uint32_t *>(qs + v * n + b * 256)[lane] = packed;
  const int sum = quad_sum(q[0] + q[1] + q[2] + q[3]);
  if ((lane & 3) == 0) bsums[(v * nblk + b) * 16 + (lane >> 2)] = (int16_t)sum;
  if (lane == 0) d[v * nblk + b] = dv;
}

hipError_t launch_q8k_quantize(const float *x, int64_t n, int64_t ld_x, int m, float *d, int8_t *qs,
                               int16_t *bsums, hipStream_t st) {
  const int64_t blocks = (n / 256) * m;
  hipLaunchKernelGGL(k_q8k_quantize, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0, st, x, n, ld_x, m, d, qs, bsums);
  return hipGetLastError();
}

}  // namespace spx
