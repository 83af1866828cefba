// Grouped expert GEMMs: entry points, tile scheduling and the general-shape
// kernel.
//
// Reference semantics (astrai/model/components/mlp.py:22-25, :96-97):
//   gated = up(x) * silu(gate(x))        (GEMM 1, rounded to x.dtype after
//                                          gate, up, silu and the product)
//   y     = down(gated) * w               (GEMM 2, rounded after down and
//                                          after the weight product)
// applied to every expert's rows of the permuted activations. nn.Linear
// weights are [out, in] (astrai/model/components/linear.py:12), so both GEMMs
// are C[rows, N] = A[rows, K] . W[N, K]^T with both operands K-contiguous.
//
// Work decomposition: one workgroup per (row tile, column tile). Row tiles
// come from the device-built tile list (astrai_moe_permute), so the grid is
// sized by the tile-list capacity and workgroups past the live tile count exit
// at once; skewed and empty experts cost nothing beyond their own tiles.
//
// Kernels:
//   * gemm_mfma_* (moe_gemm_mfma.hip): bf16 on CDNA4 matrix cores, used when
//     the shapes meet its tiling constraints.
//   * gemm_f32_mfma_kernel (moe_gemm_mfma_f32.hip): fp32 on CDNA4 matrix
//     cores (v_mfma_f32_16x16x4_f32), 64-row tiles, K a multiple of 32.
//   * gemm_generic_kernel (here): any shape, fp32 or bf16, fp32 FMA; 64x64
//     output tiles walked over the row tile in 64-row steps. Used for the
//     shapes neither matrix-core kernel tiles.
#include "moe_common.h"
#include "moe_gemm.h"

namespace astrai_moe {
namespace {

constexpr int kGenThreads = 256;
constexpr int kGenBM = 64;
constexpr int kGenBN = 64;
constexpr int kGenBK = 16;

// kSave (training forward): also store what the backward needs — for gate/up
// the rounded gate and up projections in S0 [rows, 2 N] in the blocked
// layout of gu_index, for down the rounded output before the routing weight
// in S0 [rows, N].
template <typename T, bool kGateUp, bool kSave = false>
__global__ __launch_bounds__(kGenThreads) void gemm_generic_kernel(
    const T* __restrict__ A, const int32_t* __restrict__ tiles,
    const void* const* __restrict__ W0, const void* const* __restrict__ W1,
    const T* __restrict__ row_w, int64_t K, int64_t N, T* __restrict__ C,
    T* __restrict__ S0 = nullptr) {
  const int tile = blockIdx.x;
  const int n_live = min(tiles[0], tiles[2]);
  if (tile >= n_live) return;
  const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)tile * ASTRAI_MOE_TILE_STRIDE;
  const int e = ti[0];
  const int64_t row0 = ti[1];
  const int64_t rows_total = min((int64_t)tiles[1], (int64_t)ti[2] - row0);
  const T* B0 = static_cast<const T*>(W0[e]);
  const T* B1 = kGateUp ? static_cast<const T*>(W1[e]) : nullptr;
  const int64_t n0 = (int64_t)blockIdx.y * kGenBN;

  __shared__ float As[kGenBK][kGenBM + 1];
  __shared__ float Bs0[kGenBK][kGenBN + 1];
  __shared__ float Bs1[kGateUp ? kGenBK : 1][kGateUp ? kGenBN + 1 : 1];

  const int tx = threadIdx.x % 16;
  const int ty = threadIdx.x / 16;
  for (int64_t rs = 0; rs < rows_total; rs += kGenBM) {
    float acc0[4][4], acc1[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc0[i][j] = acc1[i][j] = 0.0f;

    for (int64_t k0 = 0; k0 < K; k0 += kGenBK) {
#pragma unroll
      for (int j = 0; j < (kGenBM * kGenBK) / kGenThreads; ++j) {
        const int idx = threadIdx.x + j * kGenThreads;
        const int r = idx / kGenBK;
        const int kk = idx % kGenBK;
        const int64_t gk = k0 + kk;
        const bool kin = gk < K;
        As[kk][r] = (rs + r < rows_total && kin)
                        ? Elem<T>::to_f32(A[(row0 + rs + r) * K + gk]) : 0.0f;
        const int64_t n = n0 + r;
        Bs0[kk][r] = (n < N && kin) ? Elem<T>::to_f32(B0[n * K + gk]) : 0.0f;
        if (kGateUp)
          Bs1[kk][r] = (n < N && kin) ? Elem<T>::to_f32(B1[n * K + gk]) : 0.0f;
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < kGenBK; ++kk) {
        float a[4], b0[4], b1[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          b0[j] = Bs0[kk][tx * 4 + j];
          if (kGateUp) b1[j] = Bs1[kk][tx * 4 + j];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc0[i][j] = fmaf(a[i], b0[j], acc0[i][j]);
            if (kGateUp) acc1[i][j] = fmaf(a[i], b1[j], acc1[i][j]);
          }
      }
      __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r = rs + ty * 4 + i;
      if (r >= rows_total) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + tx * 4 + j;
        if (n >= N) continue;
        float v;
        if (kGateUp) {
          const float g = Elem<T>::round(acc0[i][j]);
          const float u = Elem<T>::round(acc1[i][j]);
          const float s = Elem<T>::round(silu_f32(g));
          v = u * s;
          if constexpr (kSave) {
            T* gu = S0 + (row0 + r) * 2 * N;
            gu[gu_index(n, N, false)] = Elem<T>::from_f32(g);
            gu[gu_index(n, N, true)] = Elem<T>::from_f32(u);
          }
        } else {
          if constexpr (kSave) S0[(row0 + r) * N + n] = Elem<T>::from_f32(acc0[i][j]);
          // no row weights (a dense expert): weight 1, an exact product
          v = Elem<T>::round(acc0[i][j]) * (row_w ? Elem<T>::to_f32(row_w[row0 + r]) : 1.0f);
        }
        C[(row0 + r) * N + n] = Elem<T>::from_f32(v);
      }
    }
  }
}

template <typename T, bool kGateUp, bool kSave = false>
int launch_generic(const void* A, const int32_t* tiles, int64_t capacity,
                   const void* const* W0, const void* const* W1,
                   const void* row_w, int64_t K, int64_t N, void* C,
                   hipStream_t s, void* S0 = nullptr) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  const dim3 grid((unsigned)capacity, (unsigned)ceil_div(N, kGenBN));
  hipLaunchKernelGGL((gemm_generic_kernel<T, kGateUp, kSave>), grid, dim3(kGenThreads), 0,
                     s, static_cast<const T*>(A), tiles, W0, W1,
                     static_cast<const T*>(row_w), K, N, static_cast<T*>(C),
                     static_cast<T*>(S0));
  return check_launch(kGateUp ? "gemm_generic_kernel<gate_up>"
                              : "gemm_generic_kernel<down>");
}

int check_common(const char* who, const void* A, const int32_t* tiles,
                 int64_t tiles_len, int dtype, int64_t n_rows, int n_experts,
                 int64_t K, int64_t N, int block_m, const void* C) {
  ASTRAI_REQUIRE(dtype == ASTRAI_MOE_BF16 || dtype == ASTRAI_MOE_F32,
                 "%s: unsupported dtype %d", who, dtype);
  ASTRAI_REQUIRE(n_rows >= 0 && n_rows < (1ll << 31),
                 "%s: n_rows must be in [0, 2^31) (got %lld)", who,
                 (long long)n_rows);
  ASTRAI_REQUIRE(n_experts >= 1 && n_experts <= ASTRAI_MOE_MAX_EXPERTS,
                 "%s: n_experts must be in [1, %d] (got %d)", who,
                 ASTRAI_MOE_MAX_EXPERTS, n_experts);
  ASTRAI_REQUIRE(K >= 1 && N >= 1, "%s: dims must be >= 1", who);
  ASTRAI_REQUIRE(block_m >= 1, "%s: block_m must be >= 1", who);
  ASTRAI_REQUIRE(tiles_len >= ASTRAI_MOE_TILE_HEADER,
                 "%s: tile list too short", who);
  if (n_rows > 0) ASTRAI_REQUIRE(A && tiles && C, "%s: null buffer", who);
  return ASTRAI_MOE_OK;
}

// The GEMM workspace: optional; when given, 16-byte aligned with a
// non-negative size (one smaller than astrai_moe_gemm_workspace_bytes()
// gives turns the run-time claims or the split tail off).
int check_workspace(const char* who, const void* workspace, int64_t workspace_bytes) {
  ASTRAI_REQUIRE(workspace_bytes >= 0, "%s: negative workspace size %lld", who, (long long)workspace_bytes);
  ASTRAI_REQUIRE(workspace == nullptr || reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
                 "%s: workspace must be 16-byte aligned", who);
  return ASTRAI_MOE_OK;
}

}  // namespace
}  // namespace astrai_moe

using namespace astrai_moe;

extern "C" int astrai_moe_gemm_gate_up(const void* x_perm, const int32_t* tiles,
                                       int64_t tiles_len,
                                       const void* const* w_gate,
                                       const void* const* w_up, int dtype,
                                       int64_t n_rows, int n_experts,
                                       int64_t dim, int64_t dim_ffn,
                                       int block_m, void* h, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_common("gemm_gate_up", x_perm, tiles, tiles_len, dtype, n_rows,
                        n_experts, dim, dim_ffn, block_m, h);
  if (rc) return rc;
  if ((rc = check_workspace("gemm_gate_up", workspace, workspace_bytes))) return rc;
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(w_gate && w_up, "gemm_gate_up: null weight table");
  const int64_t capacity = (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ASTRAI_MOE_BF16) {
    if (mfma_gate_up_supported(dim, dim_ffn, block_m, x_perm, h))
      return launch_mfma_gate_up(x_perm, tiles, capacity, w_gate, w_up, dim,
                                 dim_ffn, block_m, false, h, s,
                                 GemmWorkspace{workspace, workspace_bytes});
    return launch_generic<bf16_t, true>(x_perm, tiles, capacity, w_gate, w_up,
                                        nullptr, dim, dim_ffn, h, s);
  }
  if (mfma_f32_supported(dim, dim_ffn, true, block_m, x_perm, h, nullptr))
    return launch_mfma_f32_gate_up(x_perm, tiles, capacity, w_gate, w_up, n_rows, n_experts, dim, dim_ffn, h,
                                   nullptr, s);
  return launch_generic<float, true>(x_perm, tiles, capacity, w_gate, w_up,
                                     nullptr, dim, dim_ffn, h, s);
}

extern "C" int astrai_moe_gemm_gate_up_gather(const void* x, const int32_t* sorted_token, int64_t n_tokens,
                                              const int32_t* tiles, int64_t tiles_len, const void* const* w_gate,
                                              const void* const* w_up, int dtype, int64_t n_rows, int n_experts,
                                              int64_t dim, int64_t dim_ffn, int block_m, void* h, void* workspace,
                                              int64_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_common("gemm_gate_up_gather", x, tiles, tiles_len, dtype, n_rows, n_experts, dim, dim_ffn, block_m,
                        h);
  if (rc) return rc;
  if ((rc = check_workspace("gemm_gate_up_gather", workspace, workspace_bytes))) return rc;
  ASTRAI_REQUIRE(dtype == ASTRAI_MOE_BF16, "gemm_gate_up_gather: bf16 only (dtype %d)", dtype);
  ASTRAI_REQUIRE(n_tokens >= 0 && n_tokens * dim * 2 < (1ll << 32),
                 "gemm_gate_up_gather: x must be under 4 GiB (n_tokens %lld, dim %lld)", (long long)n_tokens,
                 (long long)dim);
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(mfma_gate_up_supported(dim, dim_ffn, block_m, x, h),
                 "gemm_gate_up_gather: unsupported shape (dim %lld, dim_ffn %lld, block_m %d) or alignment",
                 (long long)dim, (long long)dim_ffn, block_m);
  ASTRAI_REQUIRE(sorted_token && w_gate && w_up, "gemm_gate_up_gather: null row list or weight table");
  const int64_t capacity = (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  return launch_mfma_gate_up_gather(x, sorted_token, tiles, capacity, w_gate, w_up, dim, dim_ffn, block_m, h,
                                    static_cast<hipStream_t>(stream), GemmWorkspace{workspace, workspace_bytes});
}

extern "C" int astrai_moe_gemm_down(const void* h, const int32_t* tiles,
                                    int64_t tiles_len,
                                    const void* const* w_down,
                                    const void* sorted_w, int dtype,
                                    int64_t n_rows, int n_experts,
                                    int64_t dim_ffn, int64_t dim, int block_m,
                                    void* y, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_common("gemm_down", h, tiles, tiles_len, dtype, n_rows,
                        n_experts, dim_ffn, dim, block_m, y);
  if (rc) return rc;
  if ((rc = check_workspace("gemm_down", workspace, workspace_bytes))) return rc;
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(w_down, "gemm_down: null weight table");
  const int64_t capacity = (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ASTRAI_MOE_BF16) {
    if (mfma_down_supported(dim_ffn, dim, block_m, h, y))
      return launch_mfma_down(h, tiles, capacity, w_down, sorted_w, dim_ffn,
                              dim, block_m, false, y, s,
                              GemmWorkspace{workspace, workspace_bytes});
    return launch_generic<bf16_t, false>(h, tiles, capacity, w_down, nullptr,
                                         sorted_w, dim_ffn, dim, y, s);
  }
  if (mfma_f32_supported(dim_ffn, dim, false, block_m, h, y, nullptr))
    return launch_mfma_f32_down(h, tiles, capacity, w_down, sorted_w, n_rows, n_experts, dim_ffn, dim, y, nullptr,
                                s);
  return launch_generic<float, false>(h, tiles, capacity, w_down, nullptr,
                                      sorted_w, dim_ffn, dim, y, s);
}

extern "C" int64_t astrai_moe_gemm_workspace_bytes(int down) { return gemm_workspace_bytes(down != 0); }

static bool aligned16_ptr(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

extern "C" int astrai_moe_pack_gate_up(const void* w_gate, const void* w_up,
                                       int dtype, int64_t dim_ffn, int64_t dim,
                                       void* packed, void* stream) {
  clear_error();
  ASTRAI_REQUIRE(dtype == ASTRAI_MOE_BF16, "pack_gate_up: packed weights are bf16 only (dtype %d)", dtype);
  ASTRAI_REQUIRE(dim_ffn > 0 && dim > 0 && dim_ffn % 128 == 0 && dim % 64 == 0 && dim <= (1ll << 22),
                 "pack_gate_up: needs dim_ffn %% 128 == 0 and dim %% 64 == 0 (got %lld, %lld)",
                 (long long)dim_ffn, (long long)dim);
  ASTRAI_REQUIRE(w_gate && w_up && packed, "pack_gate_up: null buffer");
  ASTRAI_REQUIRE(aligned16_ptr(w_gate) && aligned16_ptr(w_up) && aligned16_ptr(packed),
                 "pack_gate_up: buffers must be 16-byte aligned");
  return launch_pack(w_gate, w_up, dim_ffn, dim, true, packed, static_cast<hipStream_t>(stream));
}

extern "C" int astrai_moe_pack_down(const void* w_down, int dtype, int64_t dim,
                                    int64_t dim_ffn, void* packed, void* stream) {
  clear_error();
  ASTRAI_REQUIRE(dtype == ASTRAI_MOE_BF16, "pack_down: packed weights are bf16 only (dtype %d)", dtype);
  ASTRAI_REQUIRE(dim > 0 && dim_ffn > 0 && dim % 256 == 0 && dim_ffn % 64 == 0 && dim_ffn <= (1ll << 22),
                 "pack_down: needs dim %% 256 == 0 and dim_ffn %% 64 == 0 (got %lld, %lld)", (long long)dim,
                 (long long)dim_ffn);
  ASTRAI_REQUIRE(w_down && packed, "pack_down: null buffer");
  ASTRAI_REQUIRE(aligned16_ptr(w_down) && aligned16_ptr(packed), "pack_down: buffers must be 16-byte aligned");
  return launch_pack(w_down, w_down, dim, dim_ffn, false, packed, static_cast<hipStream_t>(stream));
}

extern "C" int astrai_moe_gemm_gate_up_packed(const void* x_perm, const int32_t* tiles, int64_t tiles_len,
                                              const void* const* w_packed, int dtype, int64_t n_rows,
                                              int n_experts, int64_t dim, int64_t dim_ffn, int block_m, void* h,
                                              void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_common("gemm_gate_up_packed", x_perm, tiles, tiles_len, dtype, n_rows, n_experts, dim, dim_ffn,
                        block_m, h);
  if (rc) return rc;
  if ((rc = check_workspace("gemm_gate_up_packed", workspace, workspace_bytes))) return rc;
  ASTRAI_REQUIRE(dtype == ASTRAI_MOE_BF16, "gemm_gate_up_packed: packed weights are bf16 only");
  // packed weights come in whole 256-row tiles (128 gate + 128 up rows)
  ASTRAI_REQUIRE(n_rows == 0 || (dim_ffn % 128 == 0 && mfma_gate_up_supported(dim, dim_ffn, block_m, x_perm, h)),
                 "gemm_gate_up_packed: unsupported shape (dim %lld, dim_ffn %lld, block_m %d) or alignment",
                 (long long)dim, (long long)dim_ffn, block_m);
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(w_packed, "gemm_gate_up_packed: null weight table");
  const int64_t capacity = (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  return launch_mfma_gate_up(x_perm, tiles, capacity, w_packed, w_packed, dim, dim_ffn, block_m, true, h,
                             static_cast<hipStream_t>(stream), GemmWorkspace{workspace, workspace_bytes});
}

extern "C" int astrai_moe_gemm_down_packed(const void* h, const int32_t* tiles, int64_t tiles_len,
                                           const void* const* w_packed, const void* sorted_w, int dtype,
                                           int64_t n_rows, int n_experts, int64_t dim_ffn, int64_t dim,
                                           int block_m, void* y, void* workspace, int64_t workspace_bytes,
                                           void* stream) {
  clear_error();
  int rc = check_common("gemm_down_packed", h, tiles, tiles_len, dtype, n_rows, n_experts, dim_ffn, dim, block_m,
                        y);
  if (rc) return rc;
  if ((rc = check_workspace("gemm_down_packed", workspace, workspace_bytes))) return rc;
  ASTRAI_REQUIRE(dtype == ASTRAI_MOE_BF16, "gemm_down_packed: packed weights are bf16 only");
  ASTRAI_REQUIRE(n_rows == 0 || (dim % 256 == 0 && mfma_down_supported(dim_ffn, dim, block_m, h, y)),
                 "gemm_down_packed: unsupported shape (dim_ffn %lld, dim %lld, block_m %d) or alignment",
                 (long long)dim_ffn, (long long)dim, block_m);
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(w_packed, "gemm_down_packed: null weight table");
  const int64_t capacity = (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  return launch_mfma_down(h, tiles, capacity, w_packed, sorted_w, dim_ffn, dim, block_m, true, y,
                          static_cast<hipStream_t>(stream),
                          GemmWorkspace{workspace, workspace_bytes});
}

// ---------------------------------------------------------------------------
// Training forward and backward. bf16 with dim and dim_ffn multiples of 64
// runs the matrix-core kernels (256-row tile lists; partial last column tiles
// clamp and mask); every other shape and fp32 runs the general-shape kernels
// (any tile height).
// ---------------------------------------------------------------------------

static bool mfma_train_shape(int dtype, int64_t dim, int64_t dim_ffn) {
  return dtype == ASTRAI_MOE_BF16 && dim > 0 && dim_ffn > 0 && dim % 64 == 0 && dim_ffn % 64 == 0 &&
         dim <= (1ll << 22) && dim_ffn <= (1ll << 22);
}

static int check_train(const char* who, int dtype, int64_t dim, int64_t dim_ffn, int block_m) {
  ASTRAI_REQUIRE(dtype == ASTRAI_MOE_BF16 || dtype == ASTRAI_MOE_F32, "%s: unsupported dtype %d", who, dtype);
  ASTRAI_REQUIRE(dim > 0 && dim_ffn > 0, "%s: dims must be >= 1", who);
  if (mfma_train_shape(dtype, dim, dim_ffn))
    ASTRAI_REQUIRE(block_m == kMfmaBigBM, "%s: bf16 matrix-core shapes need the 256-row tile list (block_m %d)", who,
                   block_m);
  return ASTRAI_MOE_OK;
}

extern "C" int astrai_moe_gemm_gate_up_train(const void* x_perm, const int32_t* tiles, int64_t tiles_len,
                                             const void* const* w_gate, const void* const* w_up, int dtype,
                                             int64_t n_rows, int n_experts, int64_t dim, int64_t dim_ffn,
                                             int block_m, void* h, void* gu, void* workspace,
                                             int64_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_common("gemm_gate_up_train", x_perm, tiles, tiles_len, dtype, n_rows, n_experts, dim, dim_ffn,
                        block_m, h);
  if (rc) return rc;
  if ((rc = check_workspace("gemm_gate_up_train", workspace, workspace_bytes))) return rc;
  if ((rc = check_train("gemm_gate_up_train", dtype, dim, dim_ffn, block_m))) return rc;
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(w_gate && w_up && gu, "gemm_gate_up_train: null weight table or output");
  const int64_t capacity = (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mfma_train_shape(dtype, dim, dim_ffn)) {
    ASTRAI_REQUIRE(aligned16_ptr(x_perm) && aligned16_ptr(h) && aligned16_ptr(gu),
                   "gemm_gate_up_train: buffers must be 16-byte aligned");
    return launch_mfma_gate_up_save(x_perm, tiles, capacity, w_gate, w_up, dim, dim_ffn, h, gu, s,
                                    GemmWorkspace{workspace, workspace_bytes});
  }
  if (dtype == ASTRAI_MOE_BF16)
    return launch_generic<bf16_t, true, true>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s,
                                              gu);
  if (mfma_f32_supported(dim, dim_ffn, true, block_m, x_perm, h, gu))
    return launch_mfma_f32_gate_up(x_perm, tiles, capacity, w_gate, w_up, n_rows, n_experts, dim, dim_ffn, h, gu, s);
  return launch_generic<float, true, true>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s, gu);
}

extern "C" int astrai_moe_gemm_down_train(const void* h, const int32_t* tiles, int64_t tiles_len,
                                          const void* const* w_down, const void* sorted_w, int dtype,
                                          int64_t n_rows, int n_experts, int64_t dim_ffn, int64_t dim, int block_m,
                                          void* y, void* y_unweighted, void* workspace, int64_t workspace_bytes,
                                          void* stream) {
  clear_error();
  int rc = check_common("gemm_down_train", h, tiles, tiles_len, dtype, n_rows, n_experts, dim_ffn, dim, block_m, y);
  if (rc) return rc;
  if ((rc = check_workspace("gemm_down_train", workspace, workspace_bytes))) return rc;
  if ((rc = check_train("gemm_down_train", dtype, dim, dim_ffn, block_m))) return rc;
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(w_down && sorted_w && y_unweighted, "gemm_down_train: null weight table, row weights or output");
  const int64_t capacity = (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mfma_train_shape(dtype, dim, dim_ffn)) {
    ASTRAI_REQUIRE(aligned16_ptr(h) && aligned16_ptr(y) && aligned16_ptr(y_unweighted),
                   "gemm_down_train: buffers must be 16-byte aligned");
    return launch_mfma_down_save(h, tiles, capacity, w_down, sorted_w, dim_ffn, dim, y, y_unweighted, s,
                                 GemmWorkspace{workspace, workspace_bytes});
  }
  if (dtype == ASTRAI_MOE_BF16)
    return launch_generic<bf16_t, false, true>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s,
                                               y_unweighted);
  if (mfma_f32_supported(dim_ffn, dim, false, block_m, h, y, y_unweighted))
    return launch_mfma_f32_down(h, tiles, capacity, w_down, sorted_w, n_rows, n_experts, dim_ffn, dim, y,
                                y_unweighted, s);
  return launch_generic<float, false, true>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s,
                                            y_unweighted);
}

extern "C" int astrai_moe_row_grad(const void* dout, const int32_t* sorted_token, const void* sorted_w,
                                   const void* y_unweighted, int dtype, int64_t n_rows, int64_t dim, void* dy,
                                   void* dw_rows, void* stream) {
  clear_error();
  ASTRAI_REQUIRE(dtype == ASTRAI_MOE_BF16 || dtype == ASTRAI_MOE_F32, "row_grad: unsupported dtype %d", dtype);
  ASTRAI_REQUIRE(n_rows >= 0 && n_rows < (1ll << 31), "row_grad: n_rows must be in [0, 2^31)");
  ASTRAI_REQUIRE(dim > 0, "row_grad: dim must be >= 1 (got %lld)", (long long)dim);
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(dout && sorted_token && sorted_w && y_unweighted && dy && dw_rows, "row_grad: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ASTRAI_MOE_BF16 && dim % 8 == 0 && aligned16_ptr(dout) && aligned16_ptr(y_unweighted) &&
      aligned16_ptr(dy))
    return launch_row_grad(dout, sorted_token, sorted_w, y_unweighted, n_rows, dim, dy, dw_rows, s);
  return launch_generic_row_grad(dtype, dout, sorted_token, sorted_w, y_unweighted, n_rows, dim, dy, dw_rows, s);
}

extern "C" int astrai_moe_gemm_dgrad_down(const void* dy, const int32_t* tiles, int64_t tiles_len,
                                          const void* const* w_down, const void* gu, int dtype, int64_t n_rows,
                                          int n_experts, int64_t dim, int64_t dim_ffn, int block_m, void* dg,
                                          void* du, void* stream) {
  clear_error();
  int rc = check_common("gemm_dgrad_down", dy, tiles, tiles_len, dtype, n_rows, n_experts, dim, dim_ffn, block_m,
                        dg);
  if (rc) return rc;
  if ((rc = check_train("gemm_dgrad_down", dtype, dim, dim_ffn, block_m))) return rc;
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(w_down && gu && du, "gemm_dgrad_down: null weight table or buffer");
  const int64_t capacity = (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (mfma_train_shape(dtype, dim, dim_ffn)) {
    ASTRAI_REQUIRE(aligned16_ptr(dy) && aligned16_ptr(gu) && aligned16_ptr(dg) && aligned16_ptr(du),
                   "gemm_dgrad_down: buffers must be 16-byte aligned");
    return launch_dgrad_down(dy, tiles, capacity, w_down, gu, dim, dim_ffn, dg, du, s);
  }
  if (dtype == ASTRAI_MOE_F32 && mfma_f32_bwd_supported(dim, dim_ffn, block_m, dy, dg, du, gu))
    return launch_mfma_f32_dgrad_down(dy, tiles, capacity, w_down, gu, dim, dim_ffn, dg, du, s);
  return launch_generic_dgrad_down(dtype, dy, tiles, capacity, w_down, gu, dim, dim_ffn, dg, du, s);
}

extern "C" int astrai_moe_gemm_dgrad_gate_up(const void* dg, const void* du, const int32_t* tiles, int64_t tiles_len,
                                             const void* const* w_gate, const void* const* w_up, int dtype,
                                             int64_t n_rows, int n_experts, int64_t dim_ffn, int64_t dim,
                                             int block_m, void* dx_perm, void* workspace, int64_t workspace_bytes,
                                             void* stream) {
  clear_error();
  int rc = check_common("gemm_dgrad_gate_up", dg, tiles, tiles_len, dtype, n_rows, n_experts, dim_ffn, dim, block_m,
                        dx_perm);
  if (rc) return rc;
  if ((rc = check_workspace("gemm_dgrad_gate_up", workspace, workspace_bytes))) return rc;
  if ((rc = check_train("gemm_dgrad_gate_up", dtype, dim, dim_ffn, block_m))) return rc;
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(du && w_gate && w_up, "gemm_dgrad_gate_up: null weight table or buffer");
  const int64_t capacity = (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // dx_perm = round(dg . W_gate), then dx_perm = round(round(du . W_up) + dx_perm)
  if (mfma_train_shape(dtype, dim, dim_ffn)) {
    ASTRAI_REQUIRE(aligned16_ptr(dg) && aligned16_ptr(du) && aligned16_ptr(dx_perm),
                   "gemm_dgrad_gate_up: buffers must be 16-byte aligned");
    const GemmWorkspace ws{workspace, workspace_bytes};
    if ((rc = launch_dgrad_in(dg, tiles, capacity, w_gate, dim_ffn, dim, nullptr, dx_perm, s, ws))) return rc;
    return launch_dgrad_in(du, tiles, capacity, w_up, dim_ffn, dim, dx_perm, dx_perm, s, ws);
  }
  if (dtype == ASTRAI_MOE_F32 && mfma_f32_bwd_supported(dim_ffn, dim, block_m, dg, dx_perm, du, nullptr)) {
    if ((rc = launch_mfma_f32_dgrad_in(dg, tiles, capacity, w_gate, dim_ffn, dim, nullptr, dx_perm, s))) return rc;
    return launch_mfma_f32_dgrad_in(du, tiles, capacity, w_up, dim_ffn, dim, dx_perm, dx_perm, s);
  }
  if ((rc = launch_generic_dgrad_in(dtype, dg, tiles, capacity, w_gate, dim_ffn, dim, nullptr, dx_perm, s))) return rc;
  return launch_generic_dgrad_in(dtype, du, tiles, capacity, w_up, dim_ffn, dim, dx_perm, dx_perm, s);
}

extern "C" int astrai_moe_gemm_wgrad(const void* a, const void* b, const int32_t* expert_offsets, int dtype,
                                     int64_t n_rows, int n_experts, int64_t m, int64_t n, void* dw, void* stream) {
  clear_error();
  ASTRAI_REQUIRE(dtype == ASTRAI_MOE_BF16 || dtype == ASTRAI_MOE_F32, "gemm_wgrad: unsupported dtype %d", dtype);
  ASTRAI_REQUIRE(n_rows >= 0 && n_rows < (1ll << 31), "gemm_wgrad: n_rows must be in [0, 2^31)");
  ASTRAI_REQUIRE(n_experts >= 1 && n_experts <= ASTRAI_MOE_MAX_EXPERTS, "gemm_wgrad: n_experts must be in [1, %d]",
                 ASTRAI_MOE_MAX_EXPERTS);
  ASTRAI_REQUIRE(m > 0 && n > 0 && m <= (1ll << 22) && n <= (1ll << 22),
                 "gemm_wgrad: m and n must be in [1, 2^22] (got %lld, %lld)", (long long)m, (long long)n);
  if (n_rows == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(a && b && expert_offsets && dw, "gemm_wgrad: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ASTRAI_MOE_BF16 && m % 8 == 0 && n % 8 == 0 && aligned16_ptr(a) && aligned16_ptr(b) &&
      aligned16_ptr(dw))
    return launch_wgrad(a, b, expert_offsets, n_experts, m, n, dw, s);
  if (dtype == ASTRAI_MOE_F32 && mfma_f32_wgrad_supported(m, n, a, b, dw))
    return launch_mfma_f32_wgrad(a, b, expert_offsets, n_experts, m, n, dw, s);
  return launch_generic_wgrad(dtype, a, b, expert_offsets, n_experts, m, n, dw, s);
}
