// Router softmax, top-k selection and renormalisation for the MoE layer.
//
// Reference semantics (astrai/model/components/mlp.py):
//   :84  probs = softmax(logits.float(), dim=-1).to(x.dtype)
//   :86  w, idx = topk(probs, K, dim=-1)          (largest, sorted)
//   :87  w = w / w.sum(dim=-1, keepdim=True)       (in x.dtype)
//
// Bit-exactness with torch on the same device comes from evaluating the same
// arithmetic in the same order:
//   * softmax: each row is spread over WS = min(next_pow2(E), 64) lanes, lane
//     l holding columns l, l+WS, ...; max and sum are reduced per lane in
//     column order, then across lanes with an xor butterfly (offsets WS/2..1);
//     p = exp(x - max) / sum in float. This is the evaluation order of torch's
//     persistent warp softmax (ATen/native/cuda/PersistentSoftmax.cuh:72-206).
//   * top-k: the selected set is every value above the k-th largest plus the
//     lowest-index entries equal to it; the kernel emits values in descending
//     order (ties: lower expert first), by repeated arg-max over keys that
//     pack the probability's bits above the inverted expert id.
//   * renorm sum: torch reduces a row of K contiguous values with
//     bw = last_pow2(K) lanes, lane j adding elements j and j+bw, then a
//     shfl_down tree with offsets 1, 2, 4, ... (ATen/native/cuda/Reduce.cuh:
//     100-107 and 660-670, ROCm branch); the sum is rounded to x.dtype and
//     every weight is float(w) / float(sum) rounded to x.dtype.
//
// Each block handles one chunk of ASTRAI_MOE_CHUNK_TOKENS tokens and also
// writes that chunk's per-expert routed-token histogram, which the permute
// step scans into per-expert offsets.
#include "moe_common.h"

namespace astrai_moe {
namespace {

constexpr int kRouteThreads = 1024;  // 16 waves: a 32-token chunk is 2 rounds of 16 tokens at E >= 64

// Packed (probability, column) keys for the top-k arg-max.
template <typename T>
struct KeyOf;
template <>
struct KeyOf<bf16_t> {  // bf16 bits above a 16-bit inverted column
  typedef uint32_t type;
  static constexpr int kIdxBits = 16;
  __device__ static inline uint32_t bits(float v) { return (uint32_t)(__float_as_uint(v) >> 16); }
  __device__ static inline float value(uint32_t b) { return __uint_as_float(b << 16); }
  __device__ static inline uint32_t shfl_xor(uint32_t v, int off, int w) { return __shfl_xor(v, off, w); }
};
template <>
struct KeyOf<float> {  // fp32 bits above a 32-bit inverted column
  typedef uint64_t type;
  static constexpr int kIdxBits = 32;
  __device__ static inline uint64_t bits(float v) { return (uint64_t)__float_as_uint(v); }
  __device__ static inline float value(uint64_t b) { return __uint_as_float((uint32_t)b); }
  __device__ static inline uint64_t shfl_xor(uint64_t v, int off, int w) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off, w), hi = __shfl_xor((uint32_t)(v >> 32), off, w);
    return ((uint64_t)hi << 32) | lo;
  }
};

template <typename T, int WS, int ITER>
__global__ __launch_bounds__(kRouteThreads) void route_kernel(
    const T* __restrict__ logits, int64_t n_tokens, int n_experts, int top_k,
    int32_t* __restrict__ topk_idx, T* __restrict__ topk_w,
    int32_t* __restrict__ chunk_hist) {
  __shared__ int hist[ASTRAI_MOE_MAX_EXPERTS];
  const int64_t chunk = blockIdx.x;
  for (int e = threadIdx.x; e < n_experts; e += kRouteThreads) hist[e] = 0;
  __syncthreads();

  constexpr int kGroups = kRouteThreads / WS;
  const int lane = threadIdx.x % WS;
  const int group = threadIdx.x / WS;
  const int64_t t_begin = chunk * ASTRAI_MOE_CHUNK_TOKENS;
  const int64_t t_end = min(t_begin + (int64_t)ASTRAI_MOE_CHUNK_TOKENS, n_tokens);
  // bw = last_pow2(K): lanes that torch's row reduction uses for K values.
  int bw = 1;
  while (bw * 2 <= top_k) bw *= 2;

  for (int64_t t = t_begin + group; t < t_end; t += kGroups) {
    const T* row = logits + t * n_experts;
    float el[ITER];
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      const int c = lane + it * WS;
      el[it] = c < n_experts ? Elem<T>::to_f32(row[c]) : -INFINITY;
    }
    // max: per lane over its columns, then butterfly.
    float mx = el[0];
#pragma unroll
    for (int it = 0; it < ITER; ++it) mx = mx > el[it] ? mx : el[it];
#pragma unroll
    for (int off = WS / 2; off > 0; off /= 2) {
      const float o = __shfl_xor(mx, off, WS);
      mx = mx < o ? o : mx;
    }
    // exp and sum: per lane in column order, then butterfly.
    float sum = 0.0f;
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      el[it] = expf(el[it] - mx);
      sum += el[it];
    }
#pragma unroll
    for (int off = WS / 2; off > 0; off /= 2) sum += __shfl_xor(sum, off, WS);
    // probabilities, rounded to the activation dtype (mlp.py:84 .to(dtype)).
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      const float p = sum == 0.0f ? NAN : el[it] / sum;
      el[it] = Elem<T>::round(p);
    }

    // top-k by repeated arg-max over packed keys: the probability's bit
    // pattern (non-negative floats order like their bits) above the inverted
    // column index, so one max picks the largest value and, among equal
    // values, the lowest column. Taken or padded columns hold key 0, below
    // every live key, so each round picks a distinct valid column.
    using Key = typename KeyOf<T>::type;
    constexpr int kIdxBits = KeyOf<T>::kIdxBits;
    constexpr Key kIdxMask = (Key(1) << kIdxBits) - 1;
    Key key[ITER];
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      const int c = lane + it * WS;
      key[it] = c < n_experts ? ((KeyOf<T>::bits(el[it]) << kIdxBits) | (kIdxMask - (Key)c)) : Key(0);
    }
    float my_v = 0.0f;
    int my_i = 0;
    for (int k = 0; k < top_k; ++k) {
      Key best = 0;
#pragma unroll
      for (int it = 0; it < ITER; ++it) best = key[it] > best ? key[it] : best;
#pragma unroll
      for (int off = WS / 2; off > 0; off /= 2) {
        const Key o = KeyOf<T>::shfl_xor(best, off, WS);
        best = o > best ? o : best;
      }
#pragma unroll
      for (int it = 0; it < ITER; ++it)
        if (key[it] == best) key[it] = 0;
      if (lane == k) {
        my_i = (int)(kIdxMask - (best & kIdxMask));
        my_v = KeyOf<T>::value(best >> kIdxBits);
      }
    }

    // renormalise: torch's reduction tree over the sorted values.
    const float v = lane < top_k ? my_v : 0.0f;
    const float v_hi = __shfl(v, (lane + bw) % WS, WS);
    float part = (lane + bw < top_k) ? v + v_hi : v;
    for (int off = 1; off < bw; off <<= 1) part = part + __shfl_down(part, off, WS);
    const float denom = Elem<T>::round(__shfl(part, 0, WS));
    if (lane < top_k) {
      const float w = v / denom;
      topk_idx[t * top_k + lane] = my_i;
      topk_w[t * top_k + lane] = Elem<T>::from_f32(w);
      atomicAdd(&hist[my_i], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < n_experts; e += kRouteThreads)
    chunk_hist[chunk * n_experts + e] = hist[e];
}

template <typename T, int WS, int ITER>
void launch_route(const void* logits, int64_t n_tokens, int n_experts,
                  int top_k, int32_t* topk_idx, void* topk_w,
                  int32_t* chunk_hist, hipStream_t stream) {
  const int64_t grid = n_chunks(n_tokens);
  hipLaunchKernelGGL((route_kernel<T, WS, ITER>), dim3((unsigned)grid),
                     dim3(kRouteThreads), 0, stream,
                     static_cast<const T*>(logits), n_tokens, n_experts, top_k,
                     topk_idx, static_cast<T*>(topk_w), chunk_hist);
}

template <typename T>
int dispatch_route(const void* logits, int64_t n_tokens, int n_experts,
                   int top_k, int32_t* topk_idx, void* topk_w,
                   int32_t* chunk_hist, hipStream_t s) {
  int p2 = 1;
  while (p2 < n_experts) p2 *= 2;
#define ROUTE_CASE(WS, IT)                                                   \
  launch_route<T, WS, IT>(logits, n_tokens, n_experts, top_k, topk_idx,     \
                          topk_w, chunk_hist, s);                           \
  break;
  switch (p2) {
    case 1: ROUTE_CASE(1, 1)
    case 2: ROUTE_CASE(2, 1)
    case 4: ROUTE_CASE(4, 1)
    case 8: ROUTE_CASE(8, 1)
    case 16: ROUTE_CASE(16, 1)
    case 32: ROUTE_CASE(32, 1)
    case 64: ROUTE_CASE(64, 1)
    case 128: ROUTE_CASE(64, 2)
    case 256: ROUTE_CASE(64, 4)
    case 512: ROUTE_CASE(64, 8)
    case 1024: ROUTE_CASE(64, 16)
    default:
      return fail(ASTRAI_MOE_EINVAL, "route: unsupported n_experts %d", n_experts);
  }
#undef ROUTE_CASE
  return check_launch("route_kernel");
}

}  // namespace
}  // namespace astrai_moe

using namespace astrai_moe;

extern "C" int astrai_moe_route(const void* logits, int dtype, int64_t n_tokens,
                                int n_experts, int top_k, int32_t* topk_idx,
                                void* topk_w, int32_t* chunk_hist,
                                void* stream) {
  clear_error();
  ASTRAI_REQUIRE(n_tokens >= 0, "route: n_tokens must be >= 0 (got %lld)",
                 (long long)n_tokens);
  ASTRAI_REQUIRE(n_experts >= 1 && n_experts <= ASTRAI_MOE_MAX_EXPERTS,
                 "route: n_experts must be in [1, %d] (got %d)",
                 ASTRAI_MOE_MAX_EXPERTS, n_experts);
  ASTRAI_REQUIRE(top_k >= 1 && top_k <= n_experts && top_k <= ASTRAI_MOE_MAX_TOPK,
                 "route: top_k must be in [1, min(n_experts, %d)] (got %d)",
                 ASTRAI_MOE_MAX_TOPK, top_k);
  if (n_tokens == 0) return ASTRAI_MOE_OK;
  ASTRAI_REQUIRE(logits && topk_idx && topk_w && chunk_hist,
                 "route: null buffer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ASTRAI_MOE_BF16)
    return dispatch_route<bf16_t>(logits, n_tokens, n_experts, top_k, topk_idx,
                                  topk_w, chunk_hist, s);
  if (dtype == ASTRAI_MOE_F32)
    return dispatch_route<float>(logits, n_tokens, n_experts, top_k, topk_idx,
                                 topk_w, chunk_hist, s);
  return fail(ASTRAI_MOE_EINVAL, "route: unsupported dtype %d", dtype);
}
