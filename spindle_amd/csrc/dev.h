// Device helpers shared by the fused kernels (fused.hip) and the one-row decode pipeline
// (decode.hip): wavefront reductions, agent-coherent loads / stores, the Q8_K block quantizer
// and the greedy-pick key.
#pragma once
#include "common.h"

namespace spx {

// ------------------------------------------------------------------ wave reductions
#define SPX_DPPF(v, ctrl) __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), (ctrl), 0xF, 0xF, true))

// Exchange across 16-lane rows / 32-lane halves with the gfx950 permlane swaps (VALU ops, no
// LDS crossbar): with both operands v, lane i ends up holding {v_i, v_(i^16)} (resp. i^32) as
// the pair (r0, r1), in one order or the other; combined with a commutative operation the
// result is the butterfly step v_i (op) v_(i^k), bit for bit.
__device__ __forceinline__ void xchg16(uint32_t v, uint32_t &a, uint32_t &b) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  a = r[0];
  b = r[1];
}
__device__ __forceinline__ void xchg32(uint32_t v, uint32_t &a, uint32_t &b) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  a = r[0];
  b = r[1];
}
__device__ __forceinline__ float add16(float v) { uint32_t a, b; xchg16(__float_as_uint(v), a, b); return __uint_as_float(a) + __uint_as_float(b); }
__device__ __forceinline__ float add32(float v) { uint32_t a, b; xchg32(__float_as_uint(v), a, b); return __uint_as_float(a) + __uint_as_float(b); }
__device__ __forceinline__ float max16(float v) { uint32_t a, b; xchg16(__float_as_uint(v), a, b); return fmaxf(__uint_as_float(a), __uint_as_float(b)); }
__device__ __forceinline__ float max32(float v) { uint32_t a, b; xchg32(__float_as_uint(v), a, b); return fmaxf(__uint_as_float(a), __uint_as_float(b)); }

// Butterfly sum / max over the 64 lanes; every lane gets the same bits (each step combines
// a value with its partner's, and fp add / max are commutative).
__device__ __forceinline__ float wave_sum(float v) {
  v = v + SPX_DPPF(v, 0xB1);
  v = v + SPX_DPPF(v, 0x4E);
  v = v + SPX_DPPF(v, 0x141);
  v = v + SPX_DPPF(v, 0x140);
  v = add16(v);
  return add32(v);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, SPX_DPPF(v, 0xB1));
  v = fmaxf(v, SPX_DPPF(v, 0x4E));
  v = fmaxf(v, SPX_DPPF(v, 0x141));
  v = fmaxf(v, SPX_DPPF(v, 0x140));
  v = max16(v);
  return max32(v);
}
#define SPX_DPP64(v, ctrl)                                                                                         \
  (((unsigned long long)(uint32_t)__builtin_amdgcn_mov_dpp((int)((v) >> 32), (ctrl), 0xF, 0xF, true) << 32) | \
   (unsigned long long)(uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v), (ctrl), 0xF, 0xF, true))
__device__ __forceinline__ unsigned long long max_u64_x(unsigned long long v, bool x32) {
  uint32_t la, lb, ha, hb;
  if (x32) { xchg32((uint32_t)v, la, lb); xchg32((uint32_t)(v >> 32), ha, hb); }
  else { xchg16((uint32_t)v, la, lb); xchg16((uint32_t)(v >> 32), ha, hb); }
  const unsigned long long a = ((unsigned long long)ha << 32) | la, b = ((unsigned long long)hb << 32) | lb;
  return a > b ? a : b;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, true));
  uint32_t a, b;
  xchg16(v, a, b);
  v = max(a, b);
  xchg32(v, a, b);
  return max(a, b);
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  unsigned long long w;
  w = SPX_DPP64(v, 0xB1); v = w > v ? w : v;
  w = SPX_DPP64(v, 0x4E); v = w > v ? w : v;
  w = SPX_DPP64(v, 0x141); v = w > v ? w : v;
  w = SPX_DPP64(v, 0x140); v = w > v ? w : v;
  v = max_u64_x(v, false);
  return max_u64_x(v, true);
}
// Lane i's value of lane src (src wave-uniform).
__device__ __forceinline__ float lane_f(float v, int src) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src)); }
__device__ __forceinline__ int lane_i(int v, int src) { return __builtin_amdgcn_readlane(v, src); }

// ------------------------------------------------------------------ cross-workgroup hand-off
// Values one workgroup leaves for the last workgroup of a launch go through agent-coherent
// (sc1) stores and loads: relaxed agent-scope atomics for scalars, raw buffer operations with
// the sc1 bit for vectors (these the compiler can batch). No workgroup writes back or
// invalidates a whole L2. Before a workgroup counts itself in, all its stores have completed
// (s_waitcnt 0) and its waves have met at a barrier.
typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f2v __attribute__((ext_vector_type(2)));
typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i2v __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t rsrc_of(const void *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ f4v ld_coh4(rsrc_t r, int off) { return __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16)); }
__device__ __forceinline__ float ld_coh1(rsrc_t r, int off) { return __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 16)); }
__device__ __forceinline__ void st_coh1(rsrc_t r, int off, float v) { __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(v), r, off, 0, 16); }
__device__ __forceinline__ f2v ld_coh2(rsrc_t r, int off) { return __builtin_bit_cast(f2v, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 16)); }
__device__ __forceinline__ void st_coh4(rsrc_t r, int off, f4v v) { __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i4v, v), r, off, 0, 16); }
__device__ __forceinline__ void st_coh2(rsrc_t r, int off, f2v v) { __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i2v, v), r, off, 0, 16); }
__device__ __forceinline__ void st_dev(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ float ld_dev(const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// ------------------------------------------------------------------ Q8_K of one block
// quantize_avx2 (quant_q8k.rs:84-121) of 256 values, lane j holding values 4j..4j+3.
__device__ __forceinline__ float amax4(float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); }

// maxps: the first operand when it compares greater, else the second (so the second when
// either is NaN).
__device__ __forceinline__ float max_ps(float a, float b) { return a > b ? a : b; }

// The reference's amax (:89-98): eight running maxima, lane l over the values 8i + l in
// order i = 0..31, then max_ps(l, l + 4), max_ps of (0, 2) and (1, 3), max_ps of the two.
// A NaN resets its lane's running maximum to the next value of that lane, so a running
// maximum is the plain maximum of the values after the lane's last NaN, or NaN when that
// NaN is in the last group (i = 31); the tree keeps a NaN only as a second operand.
// Value 8i + l sits in wave lane 2i + l / 4, component l % 4: running lane c < 4 is
// component c of the even wave lanes, running lane 4 + c that of the odd ones. Every lane
// returns the result.
__device__ __forceinline__ float q8k_amax_nan(float4 v) {
  const int lane = threadIdx.x & 63;
  const float xs[4] = {v.x, v.y, v.z, v.w};
  float a[8];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const unsigned long long nm = __builtin_amdgcn_ballot_w64(isnan(xs[c]));
    const unsigned long long ne = nm & 0x5555555555555555ull, no = nm & 0xAAAAAAAAAAAAAAAAull;
    const int he = ne ? 63 - __builtin_clzll(ne) : -1, ho = no ? 63 - __builtin_clzll(no) : -1;  // last NaN lanes
    float r = lane > ((lane & 1) ? ho : he) ? fabsf(xs[c]) : 0.0f;
    // maximum over the lanes of one parity: xor 2, rotations by 4 and 8 in rows of 16, xor 16, xor 32
    r = fmaxf(r, SPX_DPPF(r, 0x4E));
    r = fmaxf(r, SPX_DPPF(r, 0x124));
    r = fmaxf(r, SPX_DPPF(r, 0x128));
    r = max16(r);
    r = max32(r);
    a[c] = he == 62 ? __builtin_nanf("") : lane_f(r, 0);
    a[4 + c] = ho == 63 ? __builtin_nanf("") : lane_f(r, 1);
  }
  const float v0 = max_ps(max_ps(a[0], a[4]), max_ps(a[2], a[6]));
  const float v1 = max_ps(max_ps(a[1], a[5]), max_ps(a[3], a[7]));
  return max_ps(v0, v1);
}

// amax of the wave's block: without a NaN the reference's result is the exact maximum, which
// the butterfly gives in any order; a block with a NaN (rare) takes the literal order.
__device__ __forceinline__ float q8k_amax(float4 v) {
  const bool nan = isnan(v.x) || isnan(v.y) || isnan(v.z) || isnan(v.w);
  if (__builtin_expect(__builtin_amdgcn_ballot_w64(nan) != 0, 0)) return q8k_amax_nan(v);
  return wave_max(amax4(v));
}

// The code of x * iscale: cvtps_epi32 (round half to even; NaN or out of int32 range gives
// INT_MIN) then the int8 saturation of packs. A value outside [-amax, amax] (possible only
// when a NaN reset the maximum) saturates as there, +inf included (-128).
__device__ __forceinline__ int q8k_code(float x, float iscale) {
  const float r = rintf(__fmul_rn(x, iscale));
  return (r >= -2147483648.0f && r < 2147483648.0f) ? (int)fminf(fmaxf(r, -128.0f), 127.0f) : -128;
}

// The codes of lane j's four values and the block scale: iscale = 127/amax and d = amax/127
// correctly rounded; zero, NaN or infinite amax gives zero codes and d = 0.
__device__ __forceinline__ float q8k_codes(float4 x, float amax, int qv[4]) {
  qv[0] = qv[1] = qv[2] = qv[3] = 0;
  if (!(amax > 0.0f) || isinf(amax)) return 0.0f;
  const float iscale = __fdiv_rn(127.0f, amax);
  qv[0] = q8k_code(x.x, iscale);
  qv[1] = q8k_code(x.y, iscale);
  qv[2] = q8k_code(x.z, iscale);
  qv[3] = q8k_code(x.w, iscale);
  return __fdiv_rn(amax, 127.0f);
}

// The block quantized (amax from q8k_amax), bsums = sums of 16 codes, written in the permuted
// layout (lane j's dword goes to [l = j % 8][k = j / 8]).
template <class QP, class DP, class BP>  // pointers (global or LDS) to uint32_t, float, int
__device__ __forceinline__ void q8k_block_store(float4 x, float amax, QP q, DP d, BP bs) {
  const int lane = threadIdx.x & 63;
  int qv[4];
  const float dv = q8k_codes(x, amax, qv);
  q[(lane & 7) * 8 + (lane >> 3)] = (uint32_t)(qv[0] & 0xff) | ((uint32_t)(qv[1] & 0xff) << 8) |
                                    ((uint32_t)(qv[2] & 0xff) << 16) | ((uint32_t)(qv[3] & 0xff) << 24);
  const int s = quad_sum(qv[0] + qv[1] + qv[2] + qv[3]);
  if ((lane & 3) == 0) bs[lane >> 2] = s;
  if (lane == 0) *d = dv;
}

// ------------------------------------------------------------------ greedy-pick keys
// logits / logit_scale, then the last maximum under f32 total order (max_by(total_cmp),
// :3661-3671): key = total-order bits as unsigned, packed above the row index so that the
// larger packed value is the larger logit and, on ties, the higher index.
__device__ __forceinline__ unsigned long long pick_key(float v, float lscale, int64_t row) {
  const float x = lscale != 1.0f ? v / lscale : v;
  const int i = __float_as_int(x);
  const int k = i ^ (int)(((unsigned)(i >> 31)) >> 1);
  return ((unsigned long long)((unsigned)k ^ 0x80000000u) << 32) | (unsigned long long)(uint32_t)row;
}

}  // namespace spx
