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
// GEMMs (dim and dim_ffn multiples of 64); other shapes and fp32 use 64-row
// tiles (the fp32 matrix-core kernel's and the general kernel's). Among
// matrix-core tiles (measured on MI355X, both GEMMs, one process; the 32-,
// 64- and 128-row tiles sum in the same order and give equal bits):
// - routed experts, by average rows per expert: 32-row tiles below 24 rows
//   (decode: the work is streaming the experts' weights), 64-row tiles below
//   48, 128-row tiles below 128 (one tile per expert reads its weights once;
//   at 64 rows per expert 10 % faster than 64-row tiles, at 80 rows 17 %),
//   256-row tiles from 128 (crossing between 112 and 160 rows for E128/F1536,
//   E64/F1408 and E8/F14336);
// - one dense MLP over all tokens (n_experts = top_k = 1, the shared
//   experts): all row tiles read the same weights, so the tile height trades
//   launch occupancy against per-tile efficiency. With u = T * (dim_ffn / 128
//   + dim / 256) (256-row work units x 256): 64-row tiles below one work unit
//   per CU (u < 65536), 128-row tiles up to 2.25 per CU, 256-row tiles beyond
//   (D2048/F2816, D4096/F14336, D7168/F2048 at 64-4096 tokens).
extern "C" int astrai_moe_select_block_m(int64_t n_tokens, int n_experts,
                                         int top_k, int64_t dim,
                                         int64_t dim_ffn, int dtype) {
  clear_error();
  if (n_tokens < 0 || n_experts < 1 || top_k < 1 || dim < 1 || dim_ffn < 1)
    return fail(ASTRAI_MOE_EINVAL, "select_block_m: bad sizes");
  if (dtype != ASTRAI_MOE_BF16 && dtype != ASTRAI_MOE_F32)
    return fail(ASTRAI_MOE_EINVAL, "select_block_m: unsupported dtype %d", dtype);
  const bool mfma_shapes = dtype == ASTRAI_MOE_BF16 && dim % 64 == 0 && dim_ffn % 64 == 0 &&
                           dim <= (1ll << 22) && dim_ffn <= (1ll << 22);
  if (!mfma_shapes) return 64;
  if (n_experts == 1 && top_k == 1) {
    if (n_tokens < 96) return kMfmaSmallBM;
    // gate/up + down column tiles per row
    const int64_t units = n_tokens * (ceil_div(dim_ffn, 128) + ceil_div(dim, 256));
    if (units < 256 * 256) return kMfmaMidBM;
    return units * 4 < 9 * 256 * 256 ? kMfmaMid2BM : kMfmaBigBM;
  }
  const int64_t rows_per_expert = n_tokens * top_k / n_experts;
  if (rows_per_expert < 24) return kMfmaSmallBM;
  if (rows_per_expert < 48) return kMfmaMidBM;
  return rows_per_expert < 128 ? kMfmaMid2BM : kMfmaBigBM;
}
