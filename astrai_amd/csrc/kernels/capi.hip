// Host-side plumbing of libastrai_moe.so: per-thread error messages, launch
// checking, ABI version and the row-tile policy.
#include <stdarg.h>
#include <stdio.h>

#include "moe_common.h"
#include "moe_gemm.h"

namespace astrai_moe {

namespace {
thread_local char g_last_error[512] = "";
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(ASTRAI_MOE_ELAUNCH, "%s: %s", what, hipGetErrorString(err));
  return ASTRAI_MOE_OK;
}

}  // namespace astrai_moe

using namespace astrai_moe;

extern "C" int astrai_moe_abi_version(void) { return ASTRAI_MOE_ABI_VERSION; }

extern "C" const char* astrai_moe_last_error(void) { return g_last_error; }

// Row-tile policy. The bf16 matrix-core kernels need K % 64 == 0 for both
// GEMMs, dim_ffn % 128 == 0 (gate/up column tiles) and dim % 256 == 0 (down
// column tiles); other shapes and fp32 use the general kernel with 64-row
// tiles. Among matrix-core tiles, 256-row tiles serve prefill-sized expert
// loads and 32-row tiles decode-sized loads, where streaming expert weights
// dominates and computing padded rows would cost more than the weights.
extern "C" int astrai_moe_select_block_m(int64_t n_tokens, int n_experts,
                                         int top_k, int64_t dim,
                                         int64_t dim_ffn, int dtype) {
  clear_error();
  if (n_tokens < 0 || n_experts < 1 || top_k < 1 || dim < 1 || dim_ffn < 1)
    return fail(ASTRAI_MOE_EINVAL, "select_block_m: bad sizes");
  if (dtype != ASTRAI_MOE_BF16 && dtype != ASTRAI_MOE_F32)
    return fail(ASTRAI_MOE_EINVAL, "select_block_m: unsupported dtype %d", dtype);
  const bool mfma_shapes = dtype == ASTRAI_MOE_BF16 && dim % 64 == 0 &&
                           dim_ffn % 128 == 0 && dim % 256 == 0 &&
                           dim <= (1ll << 22) && dim_ffn <= (1ll << 22);
  if (!mfma_shapes) return 64;
  const int64_t rows_per_expert = n_tokens * top_k / n_experts;
  return rows_per_expert >= 128 ? kMfmaBigBM : kMfmaSmallBM;
}
