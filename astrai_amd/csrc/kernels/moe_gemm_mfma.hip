// bf16 grouped expert GEMMs on CDNA4 matrix cores (gfx950).
//
// C[rows, N] = A[rows, K] . W_e[N, K]^T for every row tile of the device-built
// tile list, e = the tile's expert. Both operands are K-contiguous (row-major
// activations, nn.Linear [out, in] weights), which is exactly the operand
// layout of v_mfma_f32_32x32x16_bf16: lane l supplies row (l % 32) and the
// eight consecutive K values starting at 8 * (l / 32) of both A and B, so no
// transposes are needed anywhere.
//
// Workgroup: WGM x WGN waves over a BM x BN output tile, K staged BK = 64 at a
// time through STAGES LDS buffers. The gate/up kernel's BN columns are BN/2
// gate rows followed by the same BN/2 up rows of the expert, so each wave
// holds matching gate and up accumulators and applies SiLU * mul in registers
// (mlp.py:23); the down kernel multiplies by the row's routing weight in its
// epilogue (mlp.py:97).
//
// Global -> LDS: global_load_lds_dwordx4 (LDS DMA) moves 16 bytes per lane
// straight into LDS without passing through VGPRs; one wave instruction fills
// 1 KB = eight 128-byte rows. The 16-byte chunk c of row r is stored at chunk
// c ^ ((r >> 1) & 7): gfx950's LDS serves 16 lanes of a ds_read_b128 per
// cycle from 64 banks, and this swizzle puts the 16 rows x 1 chunk that such a
// lane group reads on 16 distinct 16-byte bank groups (measured: zero
// SQ_LDS_BANK_CONFLICT; the row-only swizzle (r & 7) measured a 2-way
// conflict on every read). The swizzle is applied on the global side by the
// choice of source chunk for each lane.
//
// Pipeline: the DMA of step k+STAGES-1 is in flight while step k computes.
// MFMA fragments are double-buffered in registers (fragments of substep s+1
// are read while substep s's MFMAs run, one ds_read per MFMA slot), and the
// barrier that publishes step k+1 sits before step k's last MFMA substep so
// its latency hides behind those MFMAs.
//
// Epilogue: accumulators are rounded to bf16 with the hardware converter
// (v_cvt_pk_bf16_f32, round-to-nearest-even), SiLU is g * rcp(1 + 2^(-g*log2e))
// on v_exp_f32 / v_rcp_f32 (within 2 ulp of the libm form before its bf16
// rounding), and each wave stages 32-row pieces of its output in LDS so the
// global stores are 16-byte row segments.
//
// Block scheduling: workgroup ids are remapped so each of the 8 XCDs (ids are
// dealt round-robin to XCDs) gets a contiguous range of the logical tile
// order, and the logical order walks GM row tiles for every column tile before
// moving on, so concurrently resident workgroups on one XCD share both
// activation rows and expert-weight rows in that XCD's L2.
#include "moe_gemm.h"

namespace astrai_moe {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;             // K elements per stage
constexpr int kRowBytes = kBK * 2;  // 128 bytes per staged row
constexpr int kXcds = 8;

template <int BM_, int BN_, int STAGES_, int WGM_, int WGN_, int GM_, int DMAW_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, STAGES = STAGES_, WGM = WGM_, WGN = WGN_, GM = GM_;
  static constexpr int DMAW = DMAW_;  // waves [0, DMAW) issue the LDS DMA
  static constexpr int WAVES = WGM * WGN;
  static constexpr int THREADS = WAVES * 64;
  static constexpr int WM = BM / WGM;  // rows per wave
  static constexpr int WN = BN / WGN;  // columns per wave
  static constexpr int MT = WM / 32;   // 32x32 MFMA tiles per wave along M
  static constexpr int NT = WN / 32;   // ... along N
  static constexpr int KSUB = kBK / 16;
  static constexpr int A_BYTES = BM * kRowBytes;
  static constexpr int B_BYTES = BN * kRowBytes;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int A_PER_WAVE = A_BYTES / 1024 / DMAW;  // 1 KB DMA ops per issuing wave
  static constexpr int B_PER_WAVE = B_BYTES / 1024 / DMAW;
  static constexpr int DMA_PER_WAVE = A_PER_WAVE + B_PER_WAVE;
  static_assert(DMAW >= 1 && DMAW <= WAVES, "DMA waves");
  static_assert(A_BYTES % (1024 * DMAW) == 0 && B_BYTES % (1024 * DMAW) == 0, "DMA ops split over waves");
  static_assert(WM % 32 == 0 && WN % 64 == 0, "32x32 MFMA tiles; gate/up halves");
  static_assert(STAGES >= 2 && STAGES * STAGE_BYTES <= 160 * 1024, "LDS");
  static_assert(DMA_PER_WAVE * (STAGES - 1) <= 63, "vmcnt range");
  static_assert(WAVES * 32 * WN * 2 <= STAGES * STAGE_BYTES, "epilogue staging");
  // physical 16-byte chunk of logical chunk c in row r
  __device__ static inline int swz(int r) { return (r >> 1) & 7; }
};

__device__ inline void lds_dma_16(const void* gsrc, void* lds_dst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)gsrc,
                                   (__attribute__((address_space(3))) void*)lds_dst, 16, 0, 0);
}

template <int N>
__device__ inline void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until at most min(pending, MAXP) groups of PER DMA ops are in flight.
template <int PER, int MAXP>
__device__ inline void wait_groups(int pending) {
  if constexpr (MAXP <= 0) {
    wait_vmcnt<0>();
  } else {
    if (pending >= MAXP)
      wait_vmcnt<MAXP * PER>();
    else
      wait_groups<PER, MAXP - 1>(pending);
  }
}

__device__ inline void wait_lds() { __builtin_amdgcn_s_waitcnt(0xc07f); }  // lgkmcnt(0)

template <typename Cfg, bool kGateUp>
__global__ __launch_bounds__(Cfg::THREADS, 1) void gemm_mfma_kernel(
    const bf16_t* __restrict__ A, const int32_t* __restrict__ tiles, const void* const* __restrict__ W0,
    const void* const* __restrict__ W1, const bf16_t* __restrict__ row_w, int K, int N, int n_tiles_n,
    int capacity, bf16_t* __restrict__ C) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, MT = Cfg::MT, NT = Cfg::NT, S = Cfg::STAGES;
  __shared__ __attribute__((aligned(1024))) char smem[S * Cfg::STAGE_BYTES];

  // ---- workgroup -> (row tile, column tile) ----
  const int bid = blockIdx.x;
  const int G = gridDim.x;
  const int per_xcd = G / kXcds, rem = G % kXcds;
  const int xcd = bid % kXcds;
  const int logical = xcd * per_xcd + min(xcd, rem) + bid / kXcds;
  const int group_size = Cfg::GM * n_tiles_n;
  const int first_m = (logical / group_size) * Cfg::GM;
  const int gm = min(Cfg::GM, capacity - first_m);
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

  // ---- LDS DMA sources ----
  // Waves [0, DMAW) issue all DMA ops (DMAW = 4 of 8 waves puts one issuing
  // wave on each SIMD: an LDS-DMA op holds its wave until the CU's vector
  // memory path accepts it, and meanwhile the SIMD's other wave keeps the
  // matrix core busy). Lane -> (row in its 8-row group, physical chunk); it
  // fetches the logical chunk stored at that physical chunk. Sources are
  // 32-bit byte offsets from uniform tile bases.
  const int dma_row = lane >> 3;
  const int dw = wave < Cfg::DMAW ? wave : 0;
  const char* a_base = reinterpret_cast<const char*>(A + (int64_t)row0 * K);
  const char* b_base0 = reinterpret_cast<const char*>(
      static_cast<const bf16_t*>(W0[e]) + (int64_t)nt * (kGateUp ? BN / 2 : BN) * K);
  const char* b_base1 =
      kGateUp ? reinterpret_cast<const char*>(static_cast<const bf16_t*>(W1[e]) + (int64_t)nt * (BN / 2) * K)
              : b_base0;
  uint32_t a_src[Cfg::A_PER_WAVE];
#pragma unroll
  for (int i = 0; i < Cfg::A_PER_WAVE; ++i) {
    const int r = (dw * Cfg::A_PER_WAVE + i) * 8 + dma_row;
    a_src[i] = (uint32_t)min(r, rows - 1) * (uint32_t)K * 2u + (uint32_t)(((lane & 7) ^ Cfg::swz(r)) << 4);
  }  // pad rows re-read a valid row
  uint32_t b_src[Cfg::B_PER_WAVE];
#pragma unroll
  for (int i = 0; i < Cfg::B_PER_WAVE; ++i) {
    const int r = (dw * Cfg::B_PER_WAVE + i) * 8 + dma_row;
    const int rr = (kGateUp && r >= BN / 2) ? r - BN / 2 : r;  // up rows follow the gate rows
    b_src[i] = (uint32_t)rr * (uint32_t)K * 2u + (uint32_t)(((lane & 7) ^ Cfg::swz(r)) << 4);
  }
  auto issue_stage = [&](int kstep, int buf) {
    if (wave >= Cfg::DMAW) return;
    char* sa = smem + buf * Cfg::STAGE_BYTES;
    char* sb = sa + Cfg::A_BYTES;
    const uint32_t koff = kstep * kRowBytes;
#pragma unroll
    for (int i = 0; i < Cfg::A_PER_WAVE; ++i)
      lds_dma_16(a_base + (a_src[i] + koff), sa + (wave * Cfg::A_PER_WAVE + i) * 1024);
#pragma unroll
    for (int i = 0; i < Cfg::B_PER_WAVE; ++i) {
      const int r0 = (wave * Cfg::B_PER_WAVE + i) * 8;  // uniform
      const char* bb = (kGateUp && r0 >= BN / 2) ? b_base1 : b_base0;
      lds_dma_16(bb + (b_src[i] + koff), sb + (wave * Cfg::B_PER_WAVE + i) * 1024);
    }
  };

  // ---- MFMA fragment reads ----
  const int frag_row = lane & 31;
  const int fsw = Cfg::swz(frag_row);  // row bases are multiples of 32
  int a_off[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) a_off[i] = (wm * Cfg::WM + i * 32 + frag_row) * kRowBytes;
  int b_off[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    int r;
    if (kGateUp) {
      constexpr int half = NT / 2;
      r = (j < half) ? wn * (Cfg::WN / 2) + j * 32 : BN / 2 + wn * (Cfg::WN / 2) + (j - half) * 32;
    } else {
      r = wn * Cfg::WN + j * 32;
    }
    b_off[j] = (r + frag_row) * kRowBytes;
  }
  bf16x8_t fa[2][MT], fb[2][NT];
  auto read_frags = [&](int buf, int ks, int slot) {
    const char* sa = smem + buf * Cfg::STAGE_BYTES;
    const char* sb = sa + Cfg::A_BYTES;
    const int sw = ((ks * 2 + (lane >> 5)) ^ fsw) << 4;
#pragma unroll
    for (int i = 0; i < MT; ++i) fa[slot][i] = *reinterpret_cast<const bf16x8_t*>(sa + a_off[i] + sw);
#pragma unroll
    for (int j = 0; j < NT; ++j) fb[slot][j] = *reinterpret_cast<const bf16x8_t*>(sb + b_off[j] + sw);
  };
  f32x16_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[slot][i], fb[slot][j], acc[i][j], 0, 0, 0);
  };
  // one fragment read per MFMA issue slot, then the remaining MFMAs
  auto interleave = [&]() {
#pragma unroll
    for (int q = 0; q < MT + NT; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    }
    if constexpr (MT * NT > MT + NT) __builtin_amdgcn_sched_group_barrier(0x008, MT * NT - (MT + NT), 0);
  };

  // ---- main loop ----
  const int KT = K / kBK;
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < KT) issue_stage(s, s);
  wait_groups<Cfg::DMA_PER_WAVE, S - 1>(min(S - 1, KT - 1));  // step 0 landed
  __syncthreads();
  read_frags(0, 0, 0);
  int buf = 0;
  for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
    for (int ks = 0; ks < Cfg::KSUB; ++ks) {
      const int slot = ks & 1;
      if (ks < Cfg::KSUB - 1) {
        read_frags(buf, ks + 1, slot ^ 1);
        interleave();
        mfmas(slot);
      } else {
        const int nbuf = (buf + 1 == S) ? 0 : buf + 1;
        if (kt + 1 < KT) {
          // step kt+1 landed (later stages may still be in flight); after the
          // barrier every wave is done reading step kt's buffer
          wait_groups<Cfg::DMA_PER_WAVE, S - 2>(min(S - 2, KT - 2 - kt));
          __builtin_amdgcn_sched_barrier(0);
          __syncthreads();
          __builtin_amdgcn_sched_barrier(0);
          if (kt + S < KT) issue_stage(kt + S, buf);
          read_frags(nbuf, 0, slot ^ 1);
          interleave();
        }
        mfmas(slot);
        buf = nbuf;
      }
    }
  }

  // ---- epilogue ----
  // Accumulator element r of lane l sits at row 8*(r/4) + 4*(l/32) + r%4,
  // column l%32 of its 32x32 tile.
  constexpr int OUTC = kGateUp ? Cfg::WN / 2 : Cfg::WN;  // output columns per wave
  constexpr int OROW = OUTC * 2;                          // staged row bytes
  constexpr int SEGS = OROW / 16;                         // 16-byte segments per row
  constexpr int ROWS_PER_PASS = 64 / SEGS;
  const int col_lane = lane & 31;
  const int row_lane = 4 * (lane >> 5);
  const int n_base = kGateUp ? nt * (BN / 2) + wn * (Cfg::WN / 2) : nt * BN + wn * Cfg::WN;
  __syncthreads();  // all waves are done with the stage buffers
  char* stage = smem + wave * (32 * OROW);
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 8 * (r / 4) + row_lane + (r % 4);
      if (kGateUp) {
        constexpr int half = NT / 2;
#pragma unroll
        for (int j = 0; j < half; ++j) {
          const float g = (float)(__bf16)acc[i][j][r];
          const float u = (float)(__bf16)acc[i][j + half][r];
          const float ex = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
          const float sv = (float)(__bf16)(g * __builtin_amdgcn_rcpf(1.0f + ex));
          *reinterpret_cast<__bf16*>(stage + m * OROW + (j * 32 + col_lane) * 2) = (__bf16)(u * sv);
        }
      } else {
        const int gmr = wm * Cfg::WM + i * 32 + m;
        const float w = bf16_bits_to_f32(row_w[row0 + min(gmr, rows - 1)]);
#pragma unroll
        for (int j = 0; j < NT; ++j)
          *reinterpret_cast<__bf16*>(stage + m * OROW + (j * 32 + col_lane) * 2) =
              (__bf16)((float)(__bf16)acc[i][j][r] * w);
      }
    }
    // the staging area is private to this wave
    wait_lds();
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int p = 0; p < 32 / ROWS_PER_PASS; ++p) {
      const int m = p * ROWS_PER_PASS + lane / SEGS;
      const int seg = lane % SEGS;
      const int gmr = wm * Cfg::WM + i * 32 + m;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + m * OROW + seg * 16);
      if (gmr < rows) *reinterpret_cast<uint4*>(C + (int64_t)(row0 + gmr) * N + n_base + seg * 8) = v;
    }
    wait_lds();
    __builtin_amdgcn_wave_barrier();
  }
}

// Prefill tiles: 256 x 256 outputs, 8 waves (2 per SIMD) of 128 x 64 each;
// waves 0-3 (one per SIMD) issue the DMA.
using BigCfg = TileCfg<kMfmaBigBM, 256, 2, 2, 4, 8, 4>;
// Decode tiles: 32 x 256 outputs, 4 waves of 32 x 64, four stages in flight
// to keep the expert-weight stream busy; every wave issues DMA.
using SmallCfg = TileCfg<kMfmaSmallBM, 256, 4, 1, 4, 8, 4>;

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

template <typename Cfg, bool kGateUp>
int launch(const void* A, const int32_t* tiles, int64_t capacity, const void* const* W0, const void* const* W1,
           const void* row_w, int64_t K, int64_t N, void* C, hipStream_t s) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  const int64_t n_tiles_n = kGateUp ? N / (Cfg::BN / 2) : N / Cfg::BN;
  const int64_t grid = capacity * n_tiles_n;
  if (grid >= (1ll << 31))
    return fail(ASTRAI_MOE_EINVAL, "gemm: %lld workgroups exceed the grid limit", (long long)grid);
  hipLaunchKernelGGL((gemm_mfma_kernel<Cfg, kGateUp>), dim3((unsigned)grid), dim3(Cfg::THREADS), 0, s,
                     static_cast<const bf16_t*>(A), tiles, W0, W1, static_cast<const bf16_t*>(row_w), (int)K, (int)N,
                     (int)n_tiles_n, (int)capacity, static_cast<bf16_t*>(C));
  return check_launch(kGateUp ? "gemm_mfma_kernel<gate_up>" : "gemm_mfma_kernel<down>");
}

}  // namespace

bool mfma_gate_up_supported(int64_t dim, int64_t dim_ffn, int block_m, const void* a, const void* c) {
  // 32-bit DMA offsets: a tile spans at most 256 rows of K * 2 bytes
  return (block_m == kMfmaBigBM || block_m == kMfmaSmallBM) && dim % kBK == 0 && dim_ffn % 128 == 0 &&
         dim <= (1ll << 22) && dim_ffn <= (1ll << 22) && aligned16(a) && aligned16(c);
}

bool mfma_down_supported(int64_t dim_ffn, int64_t dim, int block_m, const void* a, const void* c) {
  return (block_m == kMfmaBigBM || block_m == kMfmaSmallBM) && dim_ffn % kBK == 0 && dim % 256 == 0 &&
         dim <= (1ll << 22) && dim_ffn <= (1ll << 22) && aligned16(a) && aligned16(c);
}

int launch_mfma_gate_up(const void* x_perm, const int32_t* tiles, int64_t capacity, const void* const* w_gate,
                        const void* const* w_up, int64_t dim, int64_t dim_ffn, int block_m, void* h, hipStream_t s) {
  if (block_m == kMfmaBigBM)
    return launch<BigCfg, true>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s);
  return launch<SmallCfg, true>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s);
}

int launch_mfma_down(const void* h, const int32_t* tiles, int64_t capacity, const void* const* w_down,
                     const void* sorted_w, int64_t dim_ffn, int64_t dim, int block_m, void* y, hipStream_t s) {
  if (block_m == kMfmaBigBM)
    return launch<BigCfg, false>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s);
  return launch<SmallCfg, false>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s);
}

}  // namespace astrai_moe
