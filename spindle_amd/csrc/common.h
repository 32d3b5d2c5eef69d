// Shared device/host definitions for the gfx950 kernels.
//
// Weights live in HBM in a planar layout built at upload time (tensor.cpp): every field of
// every super-block goes to its own plane, so each plane is a dense array of 16-byte-aligned
// records (Q4_K: 128-byte code plane + 16-byte header plane; Q6_K: 128 B low bits, 64 B high
// bits, 16 B scales, 2 B d; Q8_0: 32 B codes + 2 B d; Q5_0: 16 B + 4 B + 2 B). The byte count
// equals the GGUF row bytes, only the order changes, so a wavefront streams each plane with
// aligned dwordx4 loads instead of straddling 210- or 34-byte records.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace spx {

enum DType : int {
  T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8,
  T_Q4K = 12, T_Q5K = 13, T_Q6K = 14, T_BF16 = 30
};

// Device view of one uploaded tensor (all experts). Plane pointers by dtype:
//   Q4_K: p0 = codes (128 B/blk, lane-permuted, see kq.h), p1 = header (16 B/blk: d, dmin,
//         scales[12]), p2 = the scales and mins unpacked to bytes (16 B/blk: sc[0..7], mn[0..7])
//   Q6_K: p0 = ql (128, lane-permuted), p1 = qh (64, lane-permuted), p2 = scales (16), p3 = d (2)
//   Q8_0: p0 = codes (32), p3 = d (2)
//   Q5_0: p0 = low nibbles (16), p1 = high bits (4), p3 = d (2)
//   Q5_K: p0 = codes (128, lane-permuted), p1 = high bits (32, lane-permuted), p2 = header (16 B:
//         d, dmin, scales[12])
//   F32 / F16: p0 = row-major values
struct Planes {
  const uint8_t *p0, *p1, *p2, *p3;
};

struct TensorView {
  Planes pl;
  int dtype;
  int64_t cols, rows;   // rows per expert
  int n_expert;
  int64_t nb;           // blocks per row
};

__device__ __forceinline__ float h2f(uint32_t h) {
  return __half2float(__ushort_as_half((unsigned short)(h & 0xffffu)));
}

// Intra-quad reductions (lanes 4k..4k+3) through DPP quad permutes.
// RMSNorm's 1 / sqrt(S / n + eps) with the reference's IEEE rounding (f32::sqrt and the division
// both correctly rounded). HIP's __fsqrt_rn is the native v_sqrt_f32 (up to 1 ulp off) unless
// OCML_BASIC_ROUNDED_OPERATIONS is defined, while sqrtf lowers to v_sqrt_f32 plus the +-1 ulp
// fma correction (correctly rounded; the build also passes -fhip-fp32-correctly-rounded-divide-
// sqrt); the division is the full div_scale / div_fmas / div_fixup sequence.
__device__ __forceinline__ float inv_rms(float sumsq, float n, float eps) { return 1.0f / sqrtf(sumsq / n + eps); }

__device__ __forceinline__ int quad_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true); }
__device__ __forceinline__ int quad_xor2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true); }
__device__ __forceinline__ int quad_sum(int v) { v += quad_xor1(v); v += quad_xor2(v); return v; }
__device__ __forceinline__ float quad_xor1f(float v) { return __int_as_float(quad_xor1(__float_as_int(v))); }
__device__ __forceinline__ float quad_xor2f(float v) { return __int_as_float(quad_xor2(__float_as_int(v))); }

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

}  // namespace spx
