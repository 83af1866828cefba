// Weighted un-permute and combine.
//
// Reference semantics (astrai/model/components/mlp.py):
//   :89  output = zeros(N, D)
//   :98  for e ascending: output.index_add_(0, token_idx, y_e * w)  — each add
//        rounds to x.dtype; a token meets each of its experts once
//   :77  shared_out = sum(e(x) for e in shared_experts) / n_shared — Python's
//        sum starts from 0 and rounds after every add; torch divides a tensor
//        by a Python number as a multiply by the float reciprocal
//        (1.0f / n_shared), rounded to x.dtype
//   :71  out = shared_out + routed_out (shared_out = zeros when there are no
//        shared experts, mlp.py:75-76)
// The rows y already carry the routing weight (fused into the down GEMM).
// Expert order equals ascending permuted-row order (rows are expert-major),
// so each token's top_k row indices are sorted and summed in that order,
// rounding after every add, then added to the shared output. Results are
// bit-identical to the reference's sequence of bf16/fp32 adds.
//
// One wave per (token, column segment); lanes stream the segment in 16-byte
// vectors, U vectors per lane per pass with every row's loads issued before
// the adds (more bytes in flight per wave: +15-30 % over one vector per pass;
// at top-2, U = 8 takes a 4096-wide bf16 row in one pass: 83 -> 74 us at the
// Mixtral shape, 5.4 TB/s, above a plain torch copy's 5.3 TB/s on the same
// part).
// Rows are split into segments only when there are too few tokens to keep the
// GPU busy (decode); otherwise a wave takes the whole row. KMAX bounds top_k
// at compile time so the row table stays in a few registers; at top-2 the
// rows are read and the output written with non-temporal hints (each byte is
// touched once), which measured faster there and slower at top-6.
#include "moe_common.h"

namespace astrai_moe {
namespace {

constexpr int kCombineThreads = 256;
constexpr int kWavesPerBlock = kCombineThreads / 64;
constexpr int64_t kTargetWaves = 4096;

template <int VW, typename T>
struct Vec {  // VW elements of T as one load / store unit
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  static constexpr bool kWide = VW * sizeof(T) == 16;
  T v[VW];
  template <bool NT>
  __device__ void load(const T* p) {
    if constexpr (kWide) {
      const u32x4* q = reinterpret_cast<const u32x4*>(p);
      *reinterpret_cast<u32x4*>(v) = NT ? __builtin_nontemporal_load(q) : *q;
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) v[j] = p[j];
    }
  }
  template <bool NT>
  __device__ void store(T* p) const {
    if constexpr (kWide) {
      u32x4* q = reinterpret_cast<u32x4*>(p);
      if (NT)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(v), q);
      else
        *q = *reinterpret_cast<const u32x4*>(v);
    } else {
#pragma unroll
      for (int j = 0; j < VW; ++j) p[j] = v[j];
    }
  }
};

template <typename T, int VW, int KMAX, int U, bool NT>
__global__ __launch_bounds__(kCombineThreads) void combine_kernel(
    const T* __restrict__ y, const int32_t* __restrict__ token_pos, const T* __restrict__ row_w,
    const T* __restrict__ shared, int n_shared, float inv_shared,
    int64_t n_tokens, int top_k, int64_t dim, int64_t seg_units, T* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t nvec = dim / VW;
  const int64_t nseg = (nvec + seg_units - 1) / seg_units;
  const int64_t gw = (int64_t)blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  const int64_t t = gw / nseg;
  const int64_t seg = gw - t * nseg;
  if (t >= n_tokens) return;

  // Lane k < top_k holds row k; rank rows by position (distinct values, an
  // invalid -1 sorts first and is skipped).
  const int my_pos = lane < top_k ? token_pos[t * top_k + lane] : 0x7fffffff;
  int rank = 0;
  for (int k = 0; k < top_k; ++k) {
    const int o = __shfl(my_pos, k, 64);
    rank += (o < my_pos) ? 1 : 0;
  }
  int rows[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    rows[r] = -1;
    if (r < top_k) {
      // m is wave-uniform; duplicate positions leave some rank unclaimed.
      const uint64_t m = __ballot(lane < top_k && rank == r);
      const int src = m ? (int)(__ffsll((unsigned long long)m) - 1) : 0;
      const int p = __shfl(my_pos, src, 64);
      rows[r] = (m && p < n_tokens * top_k) ? p : -1;
    }
  }
  // row_w: y holds unweighted rows; each is scaled by its routing weight and
  // rounded before the sum, as the down GEMM's epilogue does (mlp.py:97)
  float wr[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) wr[r] = (row_w != nullptr && rows[r] >= 0) ? Elem<T>::to_f32(row_w[rows[r]]) : 1.0f;

  const int64_t v_end = min(nvec, (seg + 1) * seg_units);
  for (int64_t v0 = seg * seg_units + lane; v0 < v_end; v0 += 64 * U) {
    Vec<VW, T> in[KMAX][U];
#pragma unroll
    for (int r = 0; r < KMAX; ++r)
      if (rows[r] >= 0)
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (v0 + u * 64 < v_end) in[r][u].template load<NT>(y + (int64_t)rows[r] * dim + (v0 + u * 64) * VW);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = v0 + u * 64;
      if (v >= v_end) break;
      float acc[VW];
#pragma unroll
      for (int j = 0; j < VW; ++j) acc[j] = 0.0f;
#pragma unroll
      for (int r = 0; r < KMAX; ++r)
        if (rows[r] >= 0)
#pragma unroll
          for (int j = 0; j < VW; ++j) {
            float val = Elem<T>::to_f32(in[r][u].v[j]);
            if (row_w != nullptr) val = Elem<T>::round(val * wr[r]);
            acc[j] = Elem<T>::round(acc[j] + val);
          }
      float sh[VW];
#pragma unroll
      for (int j = 0; j < VW; ++j) sh[j] = 0.0f;
      for (int si = 0; si < n_shared; ++si) {
        Vec<VW, T> s_in;
        s_in.template load<false>(shared + ((int64_t)si * n_tokens + t) * dim + v * VW);
#pragma unroll
        for (int j = 0; j < VW; ++j) sh[j] = Elem<T>::round(sh[j] + Elem<T>::to_f32(s_in.v[j]));
      }
      if (n_shared > 0)
#pragma unroll
        for (int j = 0; j < VW; ++j) sh[j] = Elem<T>::round(sh[j] * inv_shared);
      Vec<VW, T> res;
#pragma unroll
      for (int j = 0; j < VW; ++j) res.v[j] = Elem<T>::from_f32(sh[j] + acc[j]);
      res.template store<NT>(out + t * dim + v * VW);
    }
  }
}

template <typename T, int VW, int KMAX, int U, bool NT>
void launch_combine_cfg(const void* y, const int32_t* token_pos, const void* row_w, const void* shared, int n_shared,
                        float inv_shared, int64_t n_tokens, int top_k, int64_t dim, int64_t seg_units, int64_t grid,
                        void* out, hipStream_t s) {
  hipLaunchKernelGGL((combine_kernel<T, VW, KMAX, U, NT>), dim3((unsigned)grid), dim3(kCombineThreads), 0, s,
                     static_cast<const T*>(y), token_pos, static_cast<const T*>(row_w), static_cast<const T*>(shared),
                     n_shared, inv_shared,
                     n_tokens, top_k, dim, seg_units, static_cast<T*>(out));
}

template <typename T, int VW>
void dispatch_k(const void* y, const int32_t* token_pos, const void* row_w, const void* shared, int n_shared,
                float inv_shared, int64_t n_tokens, int top_k, int64_t dim, int64_t seg_units, int64_t grid, void* out,
                hipStream_t s) {
  if (top_k <= 2)
    launch_combine_cfg<T, VW, 2, 8, true>(y, token_pos, row_w, shared, n_shared, inv_shared, n_tokens, top_k, dim,
                                          seg_units, grid, out, s);
  else if (top_k <= 8)
    launch_combine_cfg<T, VW, 8, 2, false>(y, token_pos, row_w, shared, n_shared, inv_shared, n_tokens, top_k, dim,
                                           seg_units, grid, out, s);
  else
    launch_combine_cfg<T, VW, ASTRAI_MOE_MAX_TOPK, 1, false>(y, token_pos, row_w, shared, n_shared, inv_shared,
                                                            n_tokens, top_k, dim, seg_units, grid, out, s);
}

template <typename T>
int launch_combine(const void* y, const int32_t* token_pos, const void* row_w, const void* shared,
                   int n_shared, int64_t n_tokens, int top_k, int64_t dim,
                   void* out, hipStream_t s) {
  const float inv_shared = n_shared > 0 ? 1.0f / (float)n_shared : 0.0f;
  constexpr int kVW = 16 / sizeof(T);
  const bool vec = dim % kVW == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                   (!shared || reinterpret_cast<uintptr_t>(shared) % 16 == 0);
  const int64_t nvec = vec ? dim / kVW : dim;
  // segments of >= 128 units, as many as needed to reach kTargetWaves waves
  int64_t nseg = ceil_div(kTargetWaves, n_tokens);
  if (nseg > nvec / 128) nseg = nvec / 128;
  if (nseg < 1) nseg = 1;
  const int64_t seg_units = ceil_div(nvec, nseg);
  const int64_t waves = n_tokens * ceil_div(nvec, seg_units);
  const int64_t grid = ceil_div(waves, kWavesPerBlock);
  if (grid >= (1ll << 31)) return fail(ASTRAI_MOE_EINVAL, "combine: too many tokens");
  if (vec)
    dispatch_k<T, kVW>(y, token_pos, row_w, shared, n_shared, inv_shared, n_tokens, top_k, dim, seg_units, grid, out,
                       s);
  else
    dispatch_k<T, 1>(y, token_pos, row_w, shared, n_shared, inv_shared, n_tokens, top_k, dim, seg_units, grid, out,
                     s);
  return check_launch("combine_kernel");
}

}  // namespace
}  // namespace astrai_moe

using namespace astrai_moe;

extern "C" int astrai_moe_combine(const void* y, const int32_t* token_pos, const void* row_w,
                                  const void* shared, int n_shared, int dtype,
                                  int64_t n_tokens, int top_k, int64_t dim,
                                  void* out, void* stream) {
  clear_error();
  ASTRAI_REQUIRE(n_tokens >= 0, "combine: n_tokens must be >= 0");
  ASTRAI_REQUIRE(top_k >= 1 && top_k <= ASTRAI_MOE_MAX_TOPK,
                 "combine: top_k must be in [1, %d] (got %d)",
                 ASTRAI_MOE_MAX_TOPK, top_k);
  ASTRAI_REQUIRE(dim >= 1, "combine: dim must be >= 1");
  if (n_tokens == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(y && token_pos && out, "combine: null buffer");
  ASTRAI_REQUIRE(n_shared >= 0 && (n_shared == 0 || shared),
                 "combine: n_shared must be >= 0 with a buffer when > 0");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ASTRAI_MOE_BF16)
    return launch_combine<bf16_t>(y, token_pos, row_w, shared, n_shared, n_tokens, top_k, dim, out, s);
  if (dtype == ASTRAI_MOE_F32)
    return launch_combine<float>(y, token_pos, row_w, shared, n_shared, n_tokens, top_k, dim, out, s);
  return fail(ASTRAI_MOE_EINVAL, "combine: unsupported dtype %d", dtype);
}
