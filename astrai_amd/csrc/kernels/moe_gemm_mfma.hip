// bf16 grouped expert GEMMs on CDNA4 matrix cores (gfx950).
//
// C[rows, N] = A[rows, K] . W_e[N, K]^T for every row tile of the device-built
// tile list, e = the tile's expert. Both operands are K-contiguous (row-major
// activations, nn.Linear [out, in] weights), which is exactly the operand
// layout of v_mfma_f32_16x16x32_bf16: lane l supplies row (l % 16) and the
// eight consecutive K values starting at 8 * (l / 16) of both A and B, so no
// transposes are needed anywhere. (The 16x16x32 shape sustains more than the
// 32x32x16 one on gfx950: measured 2.0-2.1 vs 1.6-1.9 PFLOP/s in a
// register-only loop, and its results here are bit-identical.)
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
// MFMA fragments are double-buffered in registers (fragments of the second
// 32-K half of a step are read while the first half's MFMAs run), and the
// barrier that publishes step k+1 sits before step k's second half so its
// latency hides behind those MFMAs; after it a DMA wave reads its fragments
// before issuing its burst of DMA ops, which hold it until the CU's vector
// memory path accepts them.
//
// Epilogue: accumulators are rounded to bf16 with the hardware converter
// (v_cvt_pk_bf16_f32, round-to-nearest-even), SiLU is g * rcp(1 + 2^(-g*log2e))
// on v_exp_f32 / v_rcp_f32 (within 2 ulp of the libm form before its bf16
// rounding). The weight fragment is the MFMA's first operand, which leaves
// each lane 4 consecutive output columns of one row; each wave stages
// 16-row pieces in LDS with 8-byte writes and stores 16-byte row segments.
//
// Scheduling: one persistent workgroup per CU walks the tile list. Workgroup
// ids are dealt round-robin to the 8 XCDs, so each XCD's workgroups take a
// contiguous range of the logical tile order in every round, and the logical
// order walks GM row tiles for every column tile before moving on: the
// workgroups resident on one XCD share activation rows and expert-weight rows
// in that XCD's L2. The first stages of a workgroup's next tile are issued
// before the epilogue of the current one.
//
// Accumulator layout (16x16x32 with operands (W, A)): lane l, element r of
// tile (i, j) is output row 16 i + l % 16, column 16 j + 4 (l / 16) + r.
#include "moe_gemm.h"

#include <algorithm>
#include <atomic>

namespace astrai_moe {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

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
  static constexpr int A_BYTES = BM * kRowBytes;
  static constexpr int B_BYTES = BN * kRowBytes;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int A_PER_WAVE = A_BYTES / 1024 / DMAW;  // 1 KB DMA ops per issuing wave
  static constexpr int B_PER_WAVE = B_BYTES / 1024 / DMAW;
  static constexpr int DMA_PER_WAVE = A_PER_WAVE + B_PER_WAVE;
  static_assert(DMAW >= 1 && DMAW <= WAVES, "DMA waves");
  static_assert(A_BYTES % (1024 * DMAW) == 0 && B_BYTES % (1024 * DMAW) == 0, "DMA ops split over waves");
  static_assert(WM % 16 == 0 && WN % 32 == 0, "16x16 MFMA tiles; gate/up halves");
  static_assert(STAGES >= 2 && STAGES * STAGE_BYTES <= 160 * 1024, "LDS");
  static_assert(DMA_PER_WAVE * (STAGES - 1) <= 63, "vmcnt range");
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
  constexpr int BM = Cfg::BM, BN = Cfg::BN, S = Cfg::STAGES;
  constexpr int DPW = Cfg::DMA_PER_WAVE;
  constexpr int STAGE_AREA = S * Cfg::STAGE_BYTES;
  constexpr int OUTC = kGateUp ? Cfg::WN / 2 : Cfg::WN;  // output columns per wave
  constexpr int OROW = OUTC * 2 + 16;                     // staged row bytes (padded)
  static_assert(STAGE_AREA + Cfg::WAVES * 16 * OROW <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char smem[STAGE_AREA + Cfg::WAVES * 16 * OROW];

  // ---- this workgroup's tiles ----
  // Round r takes logical tile r * G + slot. Workgroup ids are dealt to the 8
  // XCDs round-robin, so slot gives the workgroups of one XCD a contiguous
  // range of logical tiles in every round; the logical order walks GM row
  // tiles for every column tile before moving on.
  const int G = gridDim.x;
  const int bid = blockIdx.x;
  const int slot = (G % kXcds == 0) ? (bid % kXcds) * (G / kXcds) + bid / kXcds : bid;
  const int total = capacity * n_tiles_n;
  const int n_live = min(tiles[0], tiles[2]);
  const int group_size = Cfg::GM * n_tiles_n;
  auto decode = [&](int logical, int& mt_o, int& nt_o) -> bool {
    const int first_m = (logical / group_size) * Cfg::GM;
    const int gm = min(Cfg::GM, capacity - first_m);
    const int in_group = logical - (first_m / Cfg::GM) * group_size;
    mt_o = first_m + in_group % gm;
    nt_o = in_group / gm;
    return mt_o < n_live;
  };
  int logical = slot, mt = 0, nt = 0;
  while (logical < total && !decode(logical, mt, nt)) logical += G;
  if (logical >= total) return;

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
  // per-tile state
  int row0 = 0, rows = 0;
  const char* a_base = nullptr;
  const char* b_base0 = nullptr;
  const char* b_base1 = nullptr;
  auto setup = [&](int mt_, int nt_) {
    const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)mt_ * ASTRAI_MOE_TILE_STRIDE;
    const int e = ti[0];
    row0 = ti[1];
    rows = min(BM, ti[2] - row0);
    a_base = reinterpret_cast<const char*>(A + (int64_t)row0 * K);
    b_base0 = reinterpret_cast<const char*>(static_cast<const bf16_t*>(W0[e]) +
                                            (int64_t)nt_ * (kGateUp ? BN / 2 : BN) * K);
    b_base1 = kGateUp ? reinterpret_cast<const char*>(static_cast<const bf16_t*>(W1[e]) + (int64_t)nt_ * (BN / 2) * K)
                      : b_base0;
  };
  // The source offsets are recomputed at every issue from an opaque copy of the
  // lane's row: hoisted out of the K loop they would hold 16 VGPRs for its
  // whole length, and the register file is full.
  auto issue_stage = [&](int kstep, int buf) {
    if constexpr (Cfg::DMAW < Cfg::WAVES) {
      if (wave >= Cfg::DMAW) return;
    }
    char* sa = smem + buf * Cfg::STAGE_BYTES;
    char* sb = sa + Cfg::A_BYTES;
    const uint32_t koff = kstep * kRowBytes;
    int dr = dma_row;
    asm volatile("" : "+v"(dr));
    const uint32_t k2 = (uint32_t)K * 2u;
    const uint32_t chk0 = (uint32_t)(((lane & 7) ^ ((dr >> 1) & 7)) << 4) + koff;
    const uint32_t chk1 = (uint32_t)(((lane & 7) ^ (((dr >> 1) + 4) & 7)) << 4) + koff;
#pragma unroll
    for (int i = 0; i < Cfg::A_PER_WAVE; ++i) {
      const int q = wave * Cfg::A_PER_WAVE + i;  // uniform 8-row group
      // pad rows past the tile's last row re-read that row
      const uint32_t row = (uint32_t)min(q * 8 + dr, rows - 1);
      lds_dma_16(a_base + (row * k2 + ((q & 1) ? chk1 : chk0)), sa + (wave * Cfg::A_PER_WAVE + i) * 1024);
    }
    const uint32_t b_row = (uint32_t)dr * k2;
#pragma unroll
    for (int i = 0; i < Cfg::B_PER_WAVE; ++i) {
      const int q = wave * Cfg::B_PER_WAVE + i;  // uniform 8-row group
      const int r0 = q * 8;
      const char* bb = (kGateUp && r0 >= BN / 2) ? b_base1 : b_base0;
      const int rq = (kGateUp && r0 >= BN / 2) ? r0 - BN / 2 : r0;  // up rows follow the gate rows
      lds_dma_16(bb + ((uint32_t)rq * k2 + b_row + ((q & 1) ? chk1 : chk0)), sb + (wave * Cfg::B_PER_WAVE + i) * 1024);
    }
  };

  // ---- MFMA fragment reads (16x16x32: lane l holds row l % 16, K 8*(l/16)..+7) ----
  constexpr int MT16 = Cfg::WM / 16, NT16 = Cfg::WN / 16;
  const int frag_row = lane & 15;
  const int fq = lane >> 4;
  const int fsw = Cfg::swz(frag_row);  // row bases are multiples of 16
  int a_off[MT16];
#pragma unroll
  for (int i = 0; i < MT16; ++i) a_off[i] = (wm * Cfg::WM + i * 16 + frag_row) * kRowBytes;
  int b_off[NT16];
#pragma unroll
  for (int j = 0; j < NT16; ++j) {
    int r;
    if (kGateUp) {
      constexpr int half = NT16 / 2;
      r = (j < half) ? wn * (Cfg::WN / 2) + j * 16 : BN / 2 + wn * (Cfg::WN / 2) + (j - half) * 16;
    } else {
      r = wn * Cfg::WN + j * 16;
    }
    b_off[j] = (r + frag_row) * kRowBytes;
  }
  bf16x8_t fa[2][MT16], fb[2][NT16];
  auto read_frags = [&](int buf, int kh, int slot_) {
    const char* sa = smem + buf * Cfg::STAGE_BYTES;
    const char* sb = sa + Cfg::A_BYTES;
    const int sw = ((kh * 4 + fq) ^ fsw) << 4;
#pragma unroll
    for (int i = 0; i < MT16; ++i) fa[slot_][i] = *reinterpret_cast<const bf16x8_t*>(sa + a_off[i] + sw);
#pragma unroll
    for (int j = 0; j < NT16; ++j) fb[slot_][j] = *reinterpret_cast<const bf16x8_t*>(sb + b_off[j] + sw);
  };
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  f32x4_t acc[MT16][NT16];
  auto mfmas = [&](int slot_) {
#pragma unroll
    for (int i = 0; i < MT16; ++i)
#pragma unroll
      for (int j = 0; j < NT16; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[slot_][j], fa[slot_][i], acc[i][j], 0, 0, 0);
  };
  auto interleave = [&]() {
#pragma unroll
    for (int q = 0; q < MT16 + NT16; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, MT16 * NT16 - (MT16 + NT16), 0);
  };

  // ---- epilogue of one tile ----
  // With the weight fragment as the MFMA's first operand, lane l holds output
  // row l % 16 of its 16x16 tile and the 4 consecutive columns 4 * (l / 16)..+3.
  // Each wave stages 16-row pieces in its own LDS slice with 8-byte writes
  // (rows padded by 16 bytes, which spreads the 16 rows of a write over
  // distinct banks) and stores them as 16-byte row segments.
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  auto epilogue = [&](int t_row0, int t_rows, int t_nt) {
    int el = lane;
    asm volatile("" : "+v"(el));
    const int row_l = el & 15;
    const int col_l = 4 * (el >> 4);
    const int n_base = kGateUp ? t_nt * (BN / 2) + wn * (Cfg::WN / 2) : t_nt * BN + wn * Cfg::WN;
    char* stage = smem + STAGE_AREA + wave * (16 * OROW);
#pragma unroll
    for (int i = 0; i < MT16; ++i) {
      const int gmr = wm * Cfg::WM + i * 16 + row_l;
      const int srow = t_row0 + min(gmr, t_rows - 1);
      constexpr int NJ = kGateUp ? NT16 / 2 : NT16;
      float w = 1.0f;
      if (!kGateUp) w = bf16_bits_to_f32(row_w[srow]);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        bf16x4_t o;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (kGateUp) {
            const float g = (float)(__bf16)acc[i][j][r];
            const float u = (float)(__bf16)acc[i][j + NJ][r];
            const float ex = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
            const float sv = (float)(__bf16)(g * __builtin_amdgcn_rcpf(1.0f + ex));
            o[r] = (__bf16)(u * sv);
          } else {
            o[r] = (__bf16)((float)(__bf16)acc[i][j][r] * w);
          }
        }
        *reinterpret_cast<bf16x4_t*>(stage + row_l * OROW + (j * 16 + col_l) * 2) = o;
      }
      // the staging slice is private to this wave: 16 rows back out as 16-byte row segments
      constexpr int SEGS = OUTC * 2 / 16;
      constexpr int RPP = 64 / SEGS;
      wait_lds();
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int p = 0; p < 16 / RPP; ++p) {
        const int m = p * RPP + el / SEGS;
        const int seg = el % SEGS;
        const int gm = wm * Cfg::WM + i * 16 + m;
        const uint4 v = *reinterpret_cast<const uint4*>(stage + m * OROW + seg * 16);
        if (gm < t_rows) *reinterpret_cast<uint4*>(C + (int64_t)(t_row0 + gm) * N + n_base + seg * 8) = v;
      }
      wait_lds();
      __builtin_amdgcn_wave_barrier();
    }
  };

  // Barriers are s_barrier after explicit waits: LDS-DMA completion is tracked
  // by vmcnt, so the waits are placed by hand rather than by a fence.
  auto barrier = [&]() {
    wait_lds();
    __builtin_amdgcn_s_barrier();
  };

  const int KT = K / kBK;
  setup(mt, nt);
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < KT) issue_stage(s, s);
  wait_groups<DPW, S - 1>(min(S - 1, KT - 1));  // step 0 landed
  barrier();
  while (true) {
    // ---- main loop over K ----
#pragma unroll
    for (int i = 0; i < MT16; ++i)
#pragma unroll
      for (int j = 0; j < NT16; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;
    read_frags(0, 0, 0);
    int buf = 0;
    for (int kt = 0; kt < KT; ++kt) {
      read_frags(buf, 1, 1);
      interleave();
      mfmas(0);
      const int nbuf = (buf + 1 == S) ? 0 : buf + 1;
      if (kt + 1 < KT) {
        wait_groups<DPW, S - 2>(min(S - 2, KT - 2 - kt));
        __builtin_amdgcn_sched_barrier(0);
        barrier();
        __builtin_amdgcn_sched_barrier(0);
        // this wave's fragments first, so they are in flight while the DMA ops
        // wait for the vector memory path
        read_frags(nbuf, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (kt + S < KT) issue_stage(kt + S, buf);
        __builtin_amdgcn_sched_barrier(0);
      }
      mfmas(1);
      buf = nbuf;
    }

    // ---- next tile's first stages, then this tile's epilogue ----
    int nlogical = logical + G, nmt = 0, nnt = 0;
    while (nlogical < total && !decode(nlogical, nmt, nnt)) nlogical += G;
    const bool has_next = nlogical < total;
    const int t_row0 = row0, t_rows = rows, t_nt = nt;
    __builtin_amdgcn_sched_barrier(0);
    barrier();  // every wave is done reading the stage buffers
    __builtin_amdgcn_sched_barrier(0);
    if (has_next) {
      setup(nmt, nnt);
#pragma unroll
      for (int s = 0; s < S; ++s)
        if (s < KT) issue_stage(s, s);
    }
    epilogue(t_row0, t_rows, t_nt);
    if (!has_next) break;
    logical = nlogical;
    mt = nmt;
    nt = nnt;
    wait_vmcnt<0>();  // the next tile's stages (and this wave's stores) are done
    barrier();
  }
}

// Prefill tiles: 256 x 256 outputs, 8 waves (2 per SIMD) of 128 x 64 each;
// waves 0-3 (one per SIMD) issue the DMA.
using BigCfg = TileCfg<kMfmaBigBM, 256, 2, 2, 4, 8, 4>;
// Decode tiles: 32 x 256 outputs, 4 waves of 32 x 64, four stages in flight
// to keep the expert-weight stream busy; every wave issues DMA.
using SmallCfg = TileCfg<kMfmaSmallBM, 256, 4, 1, 4, 8, 4>;

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Compute units of the current device (one persistent workgroup each).
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <typename Cfg, bool kGateUp>
int launch(const void* A, const int32_t* tiles, int64_t capacity, const void* const* W0, const void* const* W1,
           const void* row_w, int64_t K, int64_t N, void* C, hipStream_t s) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  const int64_t n_tiles_n = kGateUp ? N / (Cfg::BN / 2) : N / Cfg::BN;
  const int64_t total = capacity * n_tiles_n;
  if (total >= (1ll << 31))
    return fail(ASTRAI_MOE_EINVAL, "gemm: %lld tiles exceed the tile-index range", (long long)total);
  // one workgroup per compute unit (the LDS footprint allows no more), each
  // walking its share of the tile list
  const int64_t grid = std::min<int64_t>(total, cu_count());
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
