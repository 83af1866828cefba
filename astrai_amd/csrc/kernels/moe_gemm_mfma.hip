// bf16 grouped expert GEMMs on CDNA4 matrix cores (gfx950).
//
// C[rows, N] = A[rows, K] . W_e[N, K]^T for every row tile of the device-built
// tile list, e = the tile's expert. Both operands are K-contiguous (row-major
// activations, nn.Linear [out, in] weights), which is exactly the operand
// layout of v_mfma_f32_32x32x16_bf16: lane l supplies row (l % 32) and the
// eight consecutive K values starting at 8 * (l / 32) of both A and B, so no
// transposes are needed anywhere.
//
// Workgroup: 256 threads (4 waves), output tile BM x BN, K staged 64 at a
// time. The gate/up kernel's BN columns are BN/2 gate rows followed by the
// same BN/2 up rows of the expert, so each wave holds matching gate and up
// accumulators and applies SiLU * mul in registers (mlp.py:23); the down
// kernel multiplies by the row's routing weight in its epilogue (mlp.py:97).
//
// Global -> LDS: global_load_lds_dwordx4 (LDS DMA) moves 16 bytes per lane
// straight into LDS without passing through VGPRs; each wave instruction fills
// 1 KB = eight 128-byte rows. Rows are stored with the 16-byte chunk index
// XOR-swizzled by (row & 7); the swizzle is applied on the global side by the
// choice of source chunk for each lane, so that the ds_read_b128 fragment
// reads of eight consecutive rows hit eight distinct chunks (no bank
// conflicts). Stages are double-buffered: the DMA of K-step k+1 overlaps the
// matrix-core work of K-step k.
//
// Block scheduling: workgroup ids are remapped so each of the 8 XCDs (ids are
// dealt round-robin to XCDs) gets a contiguous range of the logical tile
// order, and the logical order walks GROUP_M row tiles for every column tile
// before moving on, so concurrently resident workgroups on one XCD share both
// activation rows and expert-weight rows in that XCD's L2.
#include "moe_gemm.h"

namespace astrai_moe {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBK = 64;             // K elements per stage
constexpr int kRowBytes = kBK * 2;  // 128 bytes per staged row
constexpr int kGroupM = 8;
constexpr int kXcds = 8;

template <int BM_, int BN_, int WGM_, int WGN_>
struct TileCfg {
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int WGM = WGM_;
  static constexpr int WGN = WGN_;
  static constexpr int WM = BM / WGM;  // rows per wave
  static constexpr int WN = BN / WGN;  // columns per wave
  static constexpr int MT = WM / 32;   // 32x32 MFMA tiles per wave along M
  static constexpr int NT = WN / 32;   // ... along N
  static constexpr int A_BYTES = BM * kRowBytes;
  static constexpr int B_BYTES = BN * kRowBytes;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int A_DMA = A_BYTES / 1024;  // wave-wide 1 KB DMA ops
  static constexpr int B_DMA = B_BYTES / 1024;
  static_assert(WGM * WGN == kThreads / 64, "4 waves");
  static_assert(A_DMA % 4 == 0 && B_DMA % 4 == 0, "DMA ops split over 4 waves");
  static_assert(WM % 32 == 0 && WN % 32 == 0, "32x32 MFMA tiles");
};

__device__ inline void lds_dma_16(const void* gsrc, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(
      (const __attribute__((address_space(1))) void*)gsrc,
      (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 0);
}

__device__ inline void wait_dma_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <typename Cfg, bool kGateUp>
__global__ __launch_bounds__(kThreads, 1) void gemm_mfma_kernel(
    const bf16_t* __restrict__ A, const int32_t* __restrict__ tiles,
    const void* const* __restrict__ W0, const void* const* __restrict__ W1,
    const bf16_t* __restrict__ row_w, int K, int N, int n_tiles_n,
    int capacity, bf16_t* __restrict__ C) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, MT = Cfg::MT, NT = Cfg::NT;
  __shared__ __attribute__((aligned(1024))) char smem[2 * Cfg::STAGE_BYTES];

  // ---- workgroup -> (row tile, column tile) ----
  const int bid = blockIdx.x;
  const int G = gridDim.x;
  const int per_xcd = G / kXcds, rem = G % kXcds;
  const int xcd = bid % kXcds;
  const int logical = xcd * per_xcd + min(xcd, rem) + bid / kXcds;
  const int group_size = kGroupM * n_tiles_n;
  const int first_m = (logical / group_size) * kGroupM;
  const int gm = min(kGroupM, capacity - first_m);
  const int in_group = logical % group_size;
  const int mt = first_m + in_group % gm;
  const int nt = in_group / gm;

  const int n_live = min(tiles[0], tiles[2]);
  if (mt >= n_live) return;
  const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)mt * ASTRAI_MOE_TILE_STRIDE;
  const int e = ti[0];
  const int row0 = ti[1];
  const int rows = min(BM, ti[2] - row0);

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wm = wave / Cfg::WGN;
  const int wn = wave % Cfg::WGN;

  // ---- LDS DMA source offsets (bytes, relative to the K-step base) ----
  // Lane -> (row in its 8-row group, physical chunk); it fetches the logical
  // chunk that the swizzle stores at that physical chunk.
  const int dma_row = lane >> 3;
  const int dma_chunk = (lane & 7) ^ (dma_row & 7);
  constexpr int A_PER_WAVE = Cfg::A_DMA / 4;
  constexpr int B_PER_WAVE = Cfg::B_DMA / 4;
  const char* a_src[A_PER_WAVE];
#pragma unroll
  for (int i = 0; i < A_PER_WAVE; ++i) {
    const int r = (wave * A_PER_WAVE + i) * 8 + dma_row;
    const int gr = row0 + min(r, rows - 1);  // pad rows re-read a valid row
    a_src[i] = reinterpret_cast<const char*>(A + (int64_t)gr * K) + dma_chunk * 16;
  }
  const char* b_src[B_PER_WAVE];
  const bf16_t* B0 = static_cast<const bf16_t*>(W0[e]);
  const bf16_t* B1 = kGateUp ? static_cast<const bf16_t*>(W1[e]) : nullptr;
#pragma unroll
  for (int i = 0; i < B_PER_WAVE; ++i) {
    const int r = (wave * B_PER_WAVE + i) * 8 + dma_row;
    const bf16_t* base;
    int n;
    if (kGateUp) {
      const bool up = r >= BN / 2;
      base = up ? B1 : B0;
      n = nt * (BN / 2) + (up ? r - BN / 2 : r);
    } else {
      base = B0;
      n = nt * BN + r;
    }
    b_src[i] = reinterpret_cast<const char*>(base + (int64_t)n * K) + dma_chunk * 16;
  }

  auto issue_stage = [&](int kstep, int buf) {
    char* sa = smem + buf * Cfg::STAGE_BYTES;
    char* sb = sa + Cfg::A_BYTES;
    const int koff = kstep * kRowBytes;
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i)
      lds_dma_16(a_src[i] + koff, sa + (wave * A_PER_WAVE + i) * 1024);
#pragma unroll
    for (int i = 0; i < B_PER_WAVE; ++i)
      lds_dma_16(b_src[i] + koff, sb + (wave * B_PER_WAVE + i) * 1024);
  };

  // ---- fragment read offsets ----
  const int frag_row = lane & 31;
  int a_off[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) a_off[i] = (wm * Cfg::WM + i * 32 + frag_row) * kRowBytes;
  int b_off[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    int r;
    if (kGateUp) {
      constexpr int half = NT / 2;
      r = (j < half) ? wn * (Cfg::WN / 2) + j * 32
                     : BN / 2 + wn * (Cfg::WN / 2) + (j - half) * 32;
    } else {
      r = wn * Cfg::WN + j * 32;
    }
    b_off[j] = (r + frag_row) * kRowBytes;
  }

  f32x16_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int KT = K / kBK;
  issue_stage(0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    wait_dma_all();
    __syncthreads();
    if (kt + 1 < KT) issue_stage(kt + 1, (kt + 1) & 1);
    const char* sa = smem + (kt & 1) * Cfg::STAGE_BYTES;
    const char* sb = sa + Cfg::A_BYTES;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int sw = (((ks * 2) + (lane >> 5)) ^ (lane & 7)) << 4;
      bf16x8_t a[MT], b[NT];
#pragma unroll
      for (int i = 0; i < MT; ++i)
        a[i] = *reinterpret_cast<const bf16x8_t*>(sa + a_off[i] + sw);
#pragma unroll
      for (int j = 0; j < NT; ++j)
        b[j] = *reinterpret_cast<const bf16x8_t*>(sb + b_off[j] + sw);
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // ---- epilogue ----
  // Accumulator element r of lane l sits at row 8*(r/4) + 4*(l/32) + r%4,
  // column l%32 of its 32x32 tile.
  const int col_lane = lane & 31;
  const int row_lane = 4 * (lane >> 5);
  if (kGateUp) {
    constexpr int half = NT / 2;
    const int n_base = nt * (BN / 2) + wn * (Cfg::WN / 2);
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = wm * Cfg::WM + i * 32 + 8 * (r / 4) + row_lane + (r % 4);
        if (m >= rows) continue;
        bf16_t* crow = C + (int64_t)(row0 + m) * N + n_base + col_lane;
#pragma unroll
        for (int j = 0; j < half; ++j) {
          const float g = Elem<bf16_t>::round(acc[i][j][r]);
          const float u = Elem<bf16_t>::round(acc[i][j + half][r]);
          const float s = Elem<bf16_t>::round(silu_f32(g));
          crow[j * 32] = f32_to_bf16_bits(u * s);
        }
      }
  } else {
    const int n_base = nt * BN + wn * Cfg::WN;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = wm * Cfg::WM + i * 32 + 8 * (r / 4) + row_lane + (r % 4);
        if (m >= rows) continue;
        const float w = bf16_bits_to_f32(row_w[row0 + m]);
        bf16_t* crow = C + (int64_t)(row0 + m) * N + n_base + col_lane;
#pragma unroll
        for (int j = 0; j < NT; ++j)
          crow[j * 32] = f32_to_bf16_bits(Elem<bf16_t>::round(acc[i][j][r]) * w);
      }
  }
}

using BigCfg = TileCfg<kMfmaBigBM, 256, 2, 2>;
using SmallCfg = TileCfg<kMfmaSmallBM, 256, 1, 4>;

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

template <typename Cfg, bool kGateUp>
int launch(const void* A, const int32_t* tiles, int64_t capacity,
           const void* const* W0, const void* const* W1, const void* row_w,
           int64_t K, int64_t N, void* C, hipStream_t s) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  const int64_t n_tiles_n = kGateUp ? N / (Cfg::BN / 2) : N / Cfg::BN;
  const int64_t grid = capacity * n_tiles_n;
  if (grid >= (1ll << 31))
    return fail(ASTRAI_MOE_EINVAL, "gemm: %lld workgroups exceed the grid limit",
                (long long)grid);
  hipLaunchKernelGGL((gemm_mfma_kernel<Cfg, kGateUp>), dim3((unsigned)grid),
                     dim3(kThreads), 0, s, static_cast<const bf16_t*>(A), tiles,
                     W0, W1, static_cast<const bf16_t*>(row_w), (int)K, (int)N,
                     (int)n_tiles_n, (int)capacity, static_cast<bf16_t*>(C));
  return check_launch(kGateUp ? "gemm_mfma_kernel<gate_up>" : "gemm_mfma_kernel<down>");
}

}  // namespace

bool mfma_gate_up_supported(int64_t dim, int64_t dim_ffn, int block_m,
                            const void* a, const void* c) {
  return (block_m == kMfmaBigBM || block_m == kMfmaSmallBM) && dim % kBK == 0 &&
         dim_ffn % 128 == 0 && dim < (1ll << 30) && dim_ffn < (1ll << 30) &&
         aligned16(a) && aligned16(c);
}

bool mfma_down_supported(int64_t dim_ffn, int64_t dim, int block_m,
                         const void* a, const void* c) {
  return (block_m == kMfmaBigBM || block_m == kMfmaSmallBM) &&
         dim_ffn % kBK == 0 && dim % 256 == 0 && dim < (1ll << 30) &&
         dim_ffn < (1ll << 30) && aligned16(a) && aligned16(c);
}

int launch_mfma_gate_up(const void* x_perm, const int32_t* tiles,
                        int64_t capacity, const void* const* w_gate,
                        const void* const* w_up, int64_t dim, int64_t dim_ffn,
                        int block_m, void* h, hipStream_t s) {
  if (block_m == kMfmaBigBM)
    return launch<BigCfg, true>(x_perm, tiles, capacity, w_gate, w_up, nullptr,
                                dim, dim_ffn, h, s);
  return launch<SmallCfg, true>(x_perm, tiles, capacity, w_gate, w_up, nullptr,
                                dim, dim_ffn, h, s);
}

int launch_mfma_down(const void* h, const int32_t* tiles, int64_t capacity,
                     const void* const* w_down, const void* sorted_w,
                     int64_t dim_ffn, int64_t dim, int block_m, void* y,
                     hipStream_t s) {
  if (block_m == kMfmaBigBM)
    return launch<BigCfg, false>(h, tiles, capacity, w_down, nullptr, sorted_w,
                                 dim_ffn, dim, y, s);
  return launch<SmallCfg, false>(h, tiles, capacity, w_down, nullptr, sorted_w,
                                 dim_ffn, dim, y, s);
}

}  // namespace astrai_moe
