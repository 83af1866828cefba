// Backward of the routed experts for any shape and for fp32: the grouped
// dgrad and wgrad GEMMs and the per-row gradient of the weighted combine,
// with fp32 FMA over 64 x 64 output tiles staged through LDS (the general
// forward kernel's scheme, moe_gemm.hip). The bf16 matrix-core shapes
// (dim % 256 == 0, dim_ffn % 128 == 0) run moe_gemm_bwd.hip instead.
//
// The reference layer is plain torch (astrai/model/components/mlp.py:22-25,
// 89-98) and autograd differentiates it op by op; per expert e with rows R_e:
//   dy   = dout[tok] * w,  dw = sum_d dout[tok] * y       (row_grad_generic_kernel)
//   dh   = dy . W_down                   [R_e, F]         (NN, W_down [D, F])
//   du   = dh * silu(g),  dg = silu'(g) * (dh * u)        (its epilogue)
//   dx   = (dg . W_gate) + (du . W_up)   [R_e, D]         (NN twice, the second
//          adding the first's rounded result in its epilogue)
//   dW_down = dy^T h,  dW_gate = dg^T x,  dW_up = du^T x  (TN per expert)
// rounding to the element type where autograd does (each op's output; for
// fp32 rounding is the identity). silu and sigmoid are evaluated as torch's
// float kernels do: x / (1 + exp(-x)) and 1 / (1 + exp(-x)).
#include "moe_common.h"
#include "moe_gemm.h"

namespace astrai_moe {
namespace {

constexpr int kThreads = 256;
constexpr int kBM = 64, kBN = 64, kBK = 16;

enum class Nn { kDgradDown, kDgradIn, kDgradInAdd };

__device__ inline float sigmoid_precise(float x) { return 1.0f / (1.0f + expf(-x)); }

// C[rows, N] = A[rows, K] . W_e[K, N] for every row tile of the tile list
// (e = the tile's expert), W_e row-major [K, N]. Grid: (tile-list capacity,
// column tiles); each block walks its row tile in 64-row steps. E0 and C0
// may be the same buffer (kDgradInAdd adds in place: each element is read
// and then written by the same thread), so neither is declared restrict.
template <typename T, Nn kMode>
__global__ __launch_bounds__(kThreads) void gemm_nn_generic_kernel(
    const T* __restrict__ A, const int32_t* __restrict__ tiles, const void* const* __restrict__ W,
    const T* E0, int64_t K, int64_t N, T* C0, T* C1) {
  const int tile = blockIdx.x;
  const int n_live = min(tiles[0], tiles[2]);
  if (tile >= n_live) return;
  const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)tile * ASTRAI_MOE_TILE_STRIDE;
  const int e = ti[0];
  const int64_t row0 = ti[1];
  const int64_t rows_total = min((int64_t)tiles[1], (int64_t)ti[2] - row0);
  const T* B = static_cast<const T*>(W[e]);
  const int64_t n0 = (int64_t)blockIdx.y * kBN;

  __shared__ float As[kBK][kBM + 1];
  __shared__ float Bs[kBK][kBN + 1];
  const int tx = threadIdx.x % 16;
  const int ty = threadIdx.x / 16;
  for (int64_t rs = 0; rs < rows_total; rs += kBM) {
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (int64_t k0 = 0; k0 < K; k0 += kBK) {
#pragma unroll
      for (int q = 0; q < (kBM * kBK) / kThreads; ++q) {
        const int idx = threadIdx.x + q * kThreads;
        // A tile: row idx / kBK, K offset idx % kBK (K-contiguous rows)
        const int r = idx / kBK, kk = idx % kBK;
        const int64_t gk = k0 + kk;
        As[kk][r] = (rs + r < rows_total && gk < K) ? Elem<T>::to_f32(A[(row0 + rs + r) * K + gk]) : 0.0f;
        // B tile: K row idx / kBN, column idx % kBN (N-contiguous rows)
        const int kb = idx / kBN, c = idx % kBN;
        const int64_t gkb = k0 + kb, n = n0 + c;
        Bs[kb][c] = (gkb < K && n < N) ? Elem<T>::to_f32(B[gkb * N + n]) : 0.0f;
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < kBK; ++kk) {
        float a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r = rs + ty * 4 + i;
      if (r >= rows_total) continue;
      const int64_t row = row0 + r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + tx * 4 + j;
        if (n >= N) continue;
        const float v = Elem<T>::round(acc[i][j]);
        if constexpr (kMode == Nn::kDgradDown) {
          // v = dh; E0 = gu [rows, 2 N] (blocked layout), C0 = dg, C1 = du
          const T* gu = E0 + row * 2 * N;
          const float g = Elem<T>::to_f32(gu[gu_index(n, N, false)]);
          const float u = Elem<T>::to_f32(gu[gu_index(n, N, true)]);
          const float sg = sigmoid_precise(g);
          const float act = Elem<T>::round(g * sg);        // silu(g) as the forward rounded it
          C1[row * N + n] = Elem<T>::from_f32(v * act);   // du = dh * silu(g)
          const float dact = Elem<T>::round(v * u);        // d silu(g) = dh * u
          C0[row * N + n] = Elem<T>::from_f32(dact * (sg * (1.0f + g * (1.0f - sg))));  // dg
        } else if constexpr (kMode == Nn::kDgradInAdd) {
          C0[row * N + n] = Elem<T>::from_f32(v + Elem<T>::to_f32(E0[row * N + n]));
        } else {
          C0[row * N + n] = Elem<T>::from_f32(v);
        }
      }
    }
  }
}

// dw[e] [M, N] = a[rows_e]^T . b[rows_e] for every expert with rows
// (a [rows, M], b [rows, N]); experts without rows are not written. Grid:
// (M tiles, N tiles, experts).
template <typename T>
__global__ __launch_bounds__(kThreads) void gemm_wgrad_generic_kernel(
    const T* __restrict__ a, const T* __restrict__ b, const int32_t* __restrict__ offsets, int64_t M, int64_t N,
    T* __restrict__ dw) {
  const int e = blockIdx.z;
  const int64_t r0 = offsets[e], r1 = offsets[e + 1];
  if (r0 >= r1) return;
  const int64_t m0 = (int64_t)blockIdx.x * kBM, n0 = (int64_t)blockIdx.y * kBN;
  __shared__ float As[kBK][kBM + 1];
  __shared__ float Bs[kBK][kBN + 1];
  const int tx = threadIdx.x % 16;
  const int ty = threadIdx.x / 16;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  for (int64_t k0 = r0; k0 < r1; k0 += kBK) {
#pragma unroll
    for (int q = 0; q < (kBM * kBK) / kThreads; ++q) {
      const int idx = threadIdx.x + q * kThreads;
      const int kk = idx / kBM, c = idx % kBM;  // both operands are contiguous along M / N
      const int64_t row = k0 + kk;
      As[kk][c] = (row < r1 && m0 + c < M) ? Elem<T>::to_f32(a[row * M + m0 + c]) : 0.0f;
      Bs[kk][c] = (row < r1 && n0 + c < N) ? Elem<T>::to_f32(b[row * N + n0 + c]) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n < N) dw[((int64_t)e * M + m) * N + n] = Elem<T>::from_f32(acc[i][j]);
    }
  }
}

// One wave per permuted row r: dy[r] = dout[token] * w (rounded per element),
// dw_rows[r] = sum_d round(dout[token, d] * y[r, d]) (autograd's mul, then
// sum with float accumulation and one rounding).
template <typename T>
__global__ __launch_bounds__(256) void row_grad_generic_kernel(
    const T* __restrict__ dout, const int32_t* __restrict__ sorted_token, const T* __restrict__ sorted_w,
    const T* __restrict__ y, int64_t n_rows, int64_t dim, T* __restrict__ dy, T* __restrict__ dw_rows) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= n_rows) return;
  const int64_t tok = sorted_token[r];
  const float w = Elem<T>::to_f32(sorted_w[r]);
  float acc = 0.0f;
  for (int64_t d = lane; d < dim; d += 64) {
    const float g = Elem<T>::to_f32(dout[tok * dim + d]);
    dy[r * dim + d] = Elem<T>::from_f32(g * w);
    acc += Elem<T>::round(g * Elem<T>::to_f32(y[r * dim + d]));
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) acc += __shfl_xor(acc, s, 64);
  if (lane == 0) dw_rows[r] = Elem<T>::from_f32(acc);
}

template <typename T, Nn kMode>
int launch_nn(const void* a, const int32_t* tiles, int64_t capacity, const void* const* w, const void* e0,
              int64_t k, int64_t n, void* c0, void* c1, hipStream_t s, const char* name) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  const dim3 grid((unsigned)capacity, (unsigned)ceil_div(n, kBN));
  hipLaunchKernelGGL((gemm_nn_generic_kernel<T, kMode>), grid, dim3(kThreads), 0, s, static_cast<const T*>(a),
                     tiles, w, static_cast<const T*>(e0), k, n, static_cast<T*>(c0), static_cast<T*>(c1));
  return check_launch(name);
}

template <typename T>
int dgrad_down(const void* dy, const int32_t* tiles, int64_t capacity, const void* const* w_down, const void* gu,
               int64_t dim, int64_t dim_ffn, void* dg, void* du, hipStream_t s) {
  return launch_nn<T, Nn::kDgradDown>(dy, tiles, capacity, w_down, gu, dim, dim_ffn, dg, du, s,
                                      "gemm_nn_generic_kernel<dgrad_down>");
}

template <typename T>
int dgrad_in(const void* d, const int32_t* tiles, int64_t capacity, const void* const* w, int64_t k, int64_t n,
             const void* add, void* dx, hipStream_t s) {
  if (add != nullptr)
    return launch_nn<T, Nn::kDgradInAdd>(d, tiles, capacity, w, add, k, n, dx, nullptr, s,
                                         "gemm_nn_generic_kernel<dgrad_in_add>");
  return launch_nn<T, Nn::kDgradIn>(d, tiles, capacity, w, nullptr, k, n, dx, nullptr, s,
                                    "gemm_nn_generic_kernel<dgrad_in>");
}

template <typename T>
int wgrad(const void* a, const void* b, const int32_t* offsets, int n_experts, int64_t m, int64_t n, void* dw,
          hipStream_t s) {
  const dim3 grid((unsigned)ceil_div(m, kBM), (unsigned)ceil_div(n, kBN), (unsigned)n_experts);
  hipLaunchKernelGGL(gemm_wgrad_generic_kernel<T>, grid, dim3(kThreads), 0, s, static_cast<const T*>(a),
                     static_cast<const T*>(b), offsets, m, n, static_cast<T*>(dw));
  return check_launch("gemm_wgrad_generic_kernel");
}

template <typename T>
int row_grad(const void* dout, const int32_t* sorted_token, const void* sorted_w, const void* y, int64_t n_rows,
             int64_t dim, void* dy, void* dw_rows, hipStream_t s) {
  if (n_rows == 0) return ASTRAI_MOE_OK;
  hipLaunchKernelGGL(row_grad_generic_kernel<T>, dim3((unsigned)ceil_div(n_rows, 4)), dim3(256), 0, s,
                     static_cast<const T*>(dout), sorted_token, static_cast<const T*>(sorted_w),
                     static_cast<const T*>(y), n_rows, dim, static_cast<T*>(dy), static_cast<T*>(dw_rows));
  return check_launch("row_grad_generic_kernel");
}

}  // namespace

int launch_generic_dgrad_down(int dtype, const void* dy, const int32_t* tiles, int64_t capacity,
                              const void* const* w_down, const void* gu, int64_t dim, int64_t dim_ffn, void* dg,
                              void* du, hipStream_t s) {
  return dtype == ASTRAI_MOE_BF16
             ? dgrad_down<bf16_t>(dy, tiles, capacity, w_down, gu, dim, dim_ffn, dg, du, s)
             : dgrad_down<float>(dy, tiles, capacity, w_down, gu, dim, dim_ffn, dg, du, s);
}

int launch_generic_dgrad_in(int dtype, const void* d, const int32_t* tiles, int64_t capacity,
                            const void* const* w, int64_t k, int64_t n, const void* add, void* dx, hipStream_t s) {
  return dtype == ASTRAI_MOE_BF16 ? dgrad_in<bf16_t>(d, tiles, capacity, w, k, n, add, dx, s)
                                  : dgrad_in<float>(d, tiles, capacity, w, k, n, add, dx, s);
}

int launch_generic_wgrad(int dtype, const void* a, const void* b, const int32_t* offsets, int n_experts, int64_t m,
                         int64_t n, void* dw, hipStream_t s) {
  return dtype == ASTRAI_MOE_BF16 ? wgrad<bf16_t>(a, b, offsets, n_experts, m, n, dw, s)
                                  : wgrad<float>(a, b, offsets, n_experts, m, n, dw, s);
}

int launch_generic_row_grad(int dtype, const void* dout, const int32_t* sorted_token, const void* sorted_w,
                            const void* y, int64_t n_rows, int64_t dim, void* dy, void* dw_rows, hipStream_t s) {
  return dtype == ASTRAI_MOE_BF16 ? row_grad<bf16_t>(dout, sorted_token, sorted_w, y, n_rows, dim, dy, dw_rows, s)
                                  : row_grad<float>(dout, sorted_token, sorted_w, y, n_rows, dim, dy, dw_rows, s);
}

}  // namespace astrai_moe
