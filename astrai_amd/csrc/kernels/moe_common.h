// Shared device helpers and host error plumbing for libastrai_moe.so.
// Target: gfx950 (CDNA4), wave64.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "astrai_moe.h"

namespace astrai_moe {

typedef uint16_t bf16_t;  // bfloat16 bit pattern

// ---------------------------------------------------------------------------
// bfloat16 <-> float. Rounding is round-to-nearest-even with NaN mapped to the
// quiet NaN 0x7FC0, which is what torch's float -> bfloat16 cast produces, so
// every rounding point below lands on the same bits as the torch ops of
// astrai/model/components/mlp.py.
// ---------------------------------------------------------------------------
__host__ __device__ inline float bf16_bits_to_f32(bf16_t v) {
  union {
    uint32_t u;
    float f;
  } c;
  c.u = (uint32_t)v << 16;
  return c.f;
}

__host__ __device__ inline bf16_t f32_to_bf16_bits(float f) {
  union {
    uint32_t u;
    float f;
  } c;
  c.f = f;
  uint32_t u = c.u;
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}

// Element traits: storage type T, arithmetic in float. `round` maps a float
// to the nearest value representable in T (identity for float).
template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static constexpr int kDtype = ASTRAI_MOE_F32;
  __device__ static inline float to_f32(float v) { return v; }
  __device__ static inline float from_f32(float v) { return v; }
  __device__ static inline float round(float v) { return v; }
};

template <>
struct Elem<bf16_t> {
  static constexpr int kDtype = ASTRAI_MOE_BF16;
  __device__ static inline float to_f32(bf16_t v) { return bf16_bits_to_f32(v); }
  __device__ static inline bf16_t from_f32(float v) { return f32_to_bf16_bits(v); }
  __device__ static inline float round(float v) {
    return bf16_bits_to_f32(f32_to_bf16_bits(v));
  }
};

// SiLU as torch evaluates it for float and for bfloat16 (opmath float):
// x / (1 + exp(-x)).
__device__ inline float silu_f32(float x) { return x / (1.0f + expf(-x)); }

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) {
  return (a + b - 1) / b;
}

// Position of the gate (or up) projection of column c in a training
// forward's saved gu row of 2 n values: columns go in blocks of 4, each block
// as its gate values followed by the same columns' up values; the last block
// holds the n % 4 columns left (when n is not a multiple of 4). For n a
// multiple of 4: g[c .. c+3] at 2 c, u[c .. c+3] at 2 c + 4.
__host__ __device__ inline int64_t gu_index(int64_t c, int64_t n, bool up) {
  const int64_t b = c >> 2;
  const int64_t w = n - 4 * b < 4 ? n - 4 * b : 4;
  return 8 * b + (up ? w : 0) + (c & 3);
}

// ---------------------------------------------------------------------------
// Host side: per-thread error message and launch checking (capi.hip).
// ---------------------------------------------------------------------------
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
void clear_error();

inline int64_t n_chunks(int64_t n_tokens) {
  return ceil_div(n_tokens, ASTRAI_MOE_CHUNK_TOKENS);
}

// Row tiles per group of the GEMMs' tile walk (the 32 workgroups of one XCD
// take a group's row tiles for a run of column tiles).
constexpr int kTileGroup = 8;
// K steps (of 64) per tile below which the 256-row GEMM kernels let the
// matrix-core waves whose rows are all padding (an expert's last tile of at
// most 128 rows) skip their MFMAs and stores on every tile; with longer tiles
// only in the tail of the tile list (tiles[3] on).
constexpr int kIdleMaxSteps = 48;
// Rows of at least this many elements (gate/up tiles of kIdleMaxSteps K
// steps or more): the permutation writes each expert's whole groups of
// kTileGroup tiles first, so that a group of the walk holds one expert's
// tiles, and the rest as the list's tail. Narrower rows keep expert order
// (with short tiles the grouped order measured slower on a skewed router).
constexpr int64_t kGroupTilesMinDim = 64 * kIdleMaxSteps;

}  // namespace astrai_moe

#define ASTRAI_REQUIRE(cond, ...)                                  \
  do {                                                             \
    if (!(cond)) return ::astrai_moe::fail(ASTRAI_MOE_EINVAL, __VA_ARGS__); \
  } while (0)
