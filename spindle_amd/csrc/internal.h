// Host-side internals shared by the C ABI, the engine and the launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>
#include <vector>

#include "common.h"

struct spx_tensor {
  spx::TensorView v;
  void *dev = nullptr;
  size_t bytes = 0;        // device allocation
  size_t plane_off[4] = {0, 0, 0, 0};
};

struct spx_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  void *ws = nullptr;      // grow-only workspace for internal Q8_K staging
  size_t ws_bytes = 0;
  uint8_t *scratch = nullptr;  // this device's copy of the fixed scratch array (spx_matvec_noalloc)
  void *moe_pin = nullptr;     // spx_moe's pinned staging block for its job list
  hipEvent_t moe_ev = nullptr; // recorded after the block's copy to the device
};

namespace spx {
void set_error(const std::string &msg);
int fail(const std::string &msg);
int hip_fail(hipError_t e, const char *what);
int64_t row_bytes(int dtype, int64_t cols);
int64_t block_elems(int dtype);
void *ws_get(spx_ctx *ctx, size_t bytes);

hipError_t launch_q8k_quantize(const float *x, int64_t n, int64_t ld_x, int m, float *d, int8_t *qs,
                               int16_t *bsums, hipStream_t st);
}  // namespace spx

#define SPX_HIP(call)                                  \
  do {                                                 \
    hipError_t e_ = (call);                            \
    if (e_ != hipSuccess) return spx::hip_fail(e_, #call); \
  } while (0)
