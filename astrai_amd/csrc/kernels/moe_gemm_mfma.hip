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
// The gate/up kernels' BN columns are BN/2 gate rows followed by the same BN/2
// up rows of the expert, so each wave holds matching gate and up accumulators
// and applies SiLU * mul in registers (mlp.py:23); the down kernels multiply
// by the row's routing weight in their epilogue (mlp.py:97).
//
// Global -> LDS: global_load_lds_dwordx4 (LDS DMA) moves 16 bytes per lane
// straight into LDS without passing through VGPRs; one wave instruction fills
// 1 KB = eight 128-byte rows (K = 64 per stage). The 16-byte chunk c of row r
// is stored at chunk c ^ ((r >> 1) & 7): gfx950's LDS serves 16 lanes of a
// ds_read_b128 per cycle from 64 banks, and this swizzle puts the 16 rows x 1
// chunk that such a lane group reads on 16 distinct 16-byte bank groups
// (measured: zero SQ_LDS_BANK_CONFLICT; the row-only swizzle (r & 7) measured
// a 2-way conflict on every read). The swizzle is applied on the global side
// by the choice of source chunk for each lane.
//
// Two kernels:
//
// * gemm_stream_kernel (256-row tiles, prefill): 12 waves. Waves 0-7 (two per
//   SIMD) only read fragments and issue MFMAs over a 256 x 256 output tile,
//   128 x 64 each; waves 8-11 (one per SIMD) only issue the LDS DMA. An LDS-DMA
//   op holds its wave until the CU's vector memory path accepts it (about 1 KB
//   per 15 cycles), so in the earlier design, where matrix-core waves issued
//   the DMA themselves, that wait came out of their MFMA schedule. Two 64 KB
//   stages; one s_barrier per 64-K step, placed where every matrix-core wave
//   has finished reading the step's buffer: after it the DMA waves refill that
//   buffer with step g + 2 (expert weights first: they come from HBM and land
//   last) and the matrix-core waves read step g + 1, whose data the DMA waves
//   waited for before the barrier. The matrix-core waves stream A fragments
//   through a ring of four registers two rows ahead and reload each B fragment
//   in place right after its last use, which keeps them at 166 VGPRs (the
//   register file holds three waves of 168 per SIMD) with no spills.
//
// * gemm_mfma_kernel (32-row tiles, decode): 4 waves of 32 x 64, every wave
//   issues DMA, four 32 KB stages in flight to keep the expert-weight stream
//   busy; MFMA fragments are double-buffered per 32-K half.
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
// in that XCD's L2. The next tile's first stages are in flight while the
// current tile's epilogue runs.
//
// Accumulator layout (16x16x32 with operands (W, A)): lane l, element r of
// tile (i, j) is output row 16 i + l % 16, column 16 j + 4 (l / 16) + r.
#include "moe_gemm.h"

#include <algorithm>
#include <atomic>
#include <utility>

namespace astrai_moe {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;             // K elements per stage
constexpr int kRowBytes = kBK * 2;  // 128 bytes per staged row
constexpr int kXcds = 8;

template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

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

// Barriers are s_barrier after explicit waits: LDS-DMA completion is tracked
// by vmcnt, so the waits are placed by hand rather than by a fence.
__device__ inline void lds_barrier() {
  wait_lds();
  __builtin_amdgcn_s_barrier();
}

// The persistent tile walk. Round r takes logical tile r * G + slot, where
// slot gives the workgroups of one XCD a contiguous range of logical tiles;
// logical tiles walk GM row tiles for every column tile. Dead row tiles (past
// the live count the tile list reports) are skipped.
template <int GM>
struct TileWalk {
  int G, total, n_live, group_size, capacity;
  __device__ TileWalk(const int32_t* tiles, int capacity_, int n_tiles_n)
      : G((int)gridDim.x), total(capacity_ * n_tiles_n), n_live(min(tiles[0], tiles[2])),
        group_size(GM * n_tiles_n), capacity(capacity_) {}
  __device__ int first_slot() const {
    const int bid = blockIdx.x;
    return (G % kXcds == 0) ? (bid % kXcds) * (G / kXcds) + bid / kXcds : bid;
  }
  __device__ bool decode(int logical, int& mt, int& nt) const {
    const int first_m = (logical / group_size) * GM;
    const int gm = min(GM, capacity - first_m);
    const int in_group = logical - (first_m / GM) * group_size;
    mt = first_m + in_group % gm;
    nt = in_group / gm;
    return mt < n_live;
  }
  // the first live logical tile at or after `logical` in this workgroup's sequence (>= total: none)
  __device__ int seek(int logical, int& mt, int& nt) const {
    while (logical < total && !decode(logical, mt, nt)) logical += G;
    return logical;
  }
};

// One 8-row DMA group of a stage: lane l loads row (l >> 3) of the group and
// physical chunk l & 7, which holds logical chunk (l & 7) ^ ((row >> 1) & 7).
// The source offsets are 32-bit byte offsets from uniform bases.
struct DmaLane {
  uint32_t chk0, chk1;  // byte offsets of the lane's chunk in even / odd 8-row groups
  int row;              // row within the 8-row group
  __device__ DmaLane(int lane, int kstep) {
    row = lane >> 3;
    const uint32_t koff = (uint32_t)kstep * kRowBytes;
    chk0 = (uint32_t)(((lane & 7) ^ ((row >> 1) & 7)) << 4) + koff;
    chk1 = (uint32_t)(((lane & 7) ^ (((row >> 1) + 4) & 7)) << 4) + koff;
  }
  // (arithmetic select: q's parity may be a runtime value)
  __device__ uint32_t chunk(int q) const {
    const uint32_t m = 0u - (uint32_t)(q & 1);
    return (chk0 & ~m) | (chk1 & m);
  }
};

// Per-tile global bases: activation rows and the expert's weight rows.
template <int BM, int BN, bool kGateUp>
struct TileSrc {
  const char* a_base = nullptr;
  const char* b_base0 = nullptr;
  const char* b_base1 = nullptr;
  int row0 = 0, rows = 0;
  __device__ void setup(const int32_t* tiles, const bf16_t* A, const void* const* W0, const void* const* W1, int K,
                        int mt, int nt) {
    const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)mt * ASTRAI_MOE_TILE_STRIDE;
    const int e = ti[0];
    row0 = ti[1];
    rows = min(BM, ti[2] - row0);
    a_base = reinterpret_cast<const char*>(A + (int64_t)row0 * K);
    b_base0 = reinterpret_cast<const char*>(static_cast<const bf16_t*>(W0[e]) +
                                            (int64_t)nt * (kGateUp ? BN / 2 : BN) * K);
    b_base1 = kGateUp ? reinterpret_cast<const char*>(static_cast<const bf16_t*>(W1[e]) + (int64_t)nt * (BN / 2) * K)
                      : b_base0;
  }
  // 8-row group q of the A tile (pad rows past the tile's last row re-read that row)
  __device__ void dma_a(const DmaLane& dl, int q, uint32_t k2, char* lds) const {
    const uint32_t row = (uint32_t)min(q * 8 + dl.row, rows - 1);
    lds_dma_16(a_base + (row * k2 + dl.chunk(q)), lds);
  }
  // 8-row group q of the B tile (up rows follow the gate rows)
  __device__ void dma_b(const DmaLane& dl, int q, uint32_t k2, char* lds) const {
    const int r0 = q * 8;
    const char* bb = (kGateUp && r0 >= BN / 2) ? b_base1 : b_base0;
    const int rq = (kGateUp && r0 >= BN / 2) ? r0 - BN / 2 : r0;
    lds_dma_16(bb + ((uint32_t)(rq + dl.row) * k2 + dl.chunk(q)), lds);
  }
};

// Epilogue of one wave's WM x WN accumulator block: bf16 rounding, SiLU * up
// (gate/up) or * routing weight (down), staged per 16 rows in the wave's own
// LDS slice (rows padded by 16 bytes, which spreads the 16 rows of an 8-byte
// write over distinct banks) and stored as 16-byte row segments.
template <bool kGateUp, int WM, int WN, int BN>
__device__ __forceinline__ void store_tile(f32x4_t (&acc)[WM / 16][WN / 16], char* stage, const bf16_t* row_w,
                                           bf16_t* C, int N, int wm, int wn, int t_row0, int t_rows, int t_nt) {
  constexpr int MT16 = WM / 16, NT16 = WN / 16;
  constexpr int OUTC = kGateUp ? WN / 2 : WN;  // output columns of the wave
  constexpr int OROW = OUTC * 2 + 16;
  // the lane id from mbcnt rather than a register held across the K loop
  const int el = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int row_l = el & 15;
  const int col_l = 4 * (el >> 4);
  const int n_base = kGateUp ? t_nt * (BN / 2) + wn * (WN / 2) : t_nt * BN + wn * WN;
#pragma unroll
  for (int i = 0; i < MT16; ++i) {
    const int gmr = wm * WM + i * 16 + row_l;
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
    constexpr int SEGS = OUTC * 2 / 16;
    constexpr int RPP = 64 / SEGS;
    wait_lds();
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int p = 0; p < 16 / RPP; ++p) {
      const int m = p * RPP + el / SEGS;
      const int seg = el % SEGS;
      const int gm = wm * WM + i * 16 + m;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + m * OROW + seg * 16);
      if (gm < t_rows) *reinterpret_cast<uint4*>(C + (int64_t)(t_row0 + gm) * N + n_base + seg * 8) = v;
    }
    wait_lds();
    __builtin_amdgcn_wave_barrier();
  }
}

template <bool kGateUp, int WN>
__host__ __device__ constexpr int staged_row_bytes() {
  return (kGateUp ? WN / 2 : WN) * 2 + 16;
}

// ===========================================================================
// Streaming kernel: 256 x 256 tiles, 8 matrix-core waves + 4 DMA waves.
// ===========================================================================
struct StreamCfg {
  static constexpr int BM = 256, BN = 256, GM = 8;
  static constexpr int WGM = 2, WGN = 4, MW = 8, DW = 4;  // matrix-core waves (WGM x WGN), DMA waves
  static constexpr int WAVES = MW + DW, THREADS = WAVES * 64;
  static constexpr int WM = BM / WGM, WN = BN / WGN;  // 128 x 64 per matrix-core wave
  static constexpr int A_BYTES = BM * kRowBytes, B_BYTES = BN * kRowBytes;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;  // 64 KB, two stages
  static constexpr int A_OPS = A_BYTES / 1024 / DW;      // 1 KB DMA ops per DMA wave per step
  static constexpr int B_OPS = B_BYTES / 1024 / DW;
  static constexpr int AR = 4;  // A-fragment ring slots
  static constexpr int PD = 2;  // A-fragment prefetch distance (rows of 16)
  static_assert(STAGE_BYTES == 65536, "stage buffers toggle by xor 65536");
  static_assert(16 % AR == 0 && PD >= 1 && PD < AR, "the prefetch slot is never the current row's");
  static_assert((A_OPS + B_OPS) * 2 <= 63, "vmcnt range");
};

template <bool kGateUp>
__global__ __launch_bounds__(StreamCfg::THREADS, 1) void gemm_stream_kernel(
    const bf16_t* __restrict__ A, const int32_t* __restrict__ tiles, const void* const* __restrict__ W0,
    const void* const* __restrict__ W1, const bf16_t* __restrict__ row_w, int K, int N, int n_tiles_n,
    int capacity, bf16_t* __restrict__ C) {
  using Cfg = StreamCfg;
  constexpr int STAGE_AREA = 2 * Cfg::STAGE_BYTES;
  constexpr int OROW = staged_row_bytes<kGateUp, Cfg::WN>();
  static_assert(STAGE_AREA + Cfg::MW * 16 * OROW <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char smem[STAGE_AREA + Cfg::MW * 16 * OROW];

  const TileWalk<Cfg::GM> walk(tiles, capacity, n_tiles_n);
  int mt = 0, nt = 0;
  int logical = walk.seek(walk.first_slot(), mt, nt);
  if (logical >= walk.total) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int KT = K / kBK;  // steps per tile

  // Global steps g = 0, 1, ... run over this workgroup's tiles back to back;
  // step g lives in buffer g % 2. Barrier X_g: every matrix-core wave has
  // read all of step g, and step g + 1 has landed. Every wave executes one
  // X_{-1} and then exactly one X_g per step.
  if (wave >= Cfg::MW) {
    // ---------------- DMA waves ----------------
    const int dw = wave - Cfg::MW;
    const uint32_t k2 = (uint32_t)K * 2u;
    TileSrc<Cfg::BM, Cfg::BN, kGateUp> src;
    // cursor: the next step to issue
    int c_logical = logical, c_mt = mt, c_nt = nt, c_kt = 0;
    bool c_live = true;
    src.setup(tiles, A, W0, W1, K, c_mt, c_nt);
    auto issue_next = [&](int buf) {
      char* sa = smem + buf * Cfg::STAGE_BYTES;
      char* sb = sa + Cfg::A_BYTES;
      const DmaLane dl(lane, c_kt);
      // expert weights first: they come from HBM and take longest to land
#pragma unroll
      for (int i = 0; i < Cfg::B_OPS; ++i) {
        const int q = dw * Cfg::B_OPS + i;
        src.dma_b(dl, q, k2, sb + q * 1024);
      }
#pragma unroll
      for (int i = 0; i < Cfg::A_OPS; ++i) {
        const int q = dw * Cfg::A_OPS + i;
        src.dma_a(dl, q, k2, sa + q * 1024);
      }
      if (++c_kt == KT) {
        c_kt = 0;
        c_logical = walk.seek(c_logical + walk.G, c_mt, c_nt);
        c_live = c_logical < walk.total;
        if (c_live) src.setup(tiles, A, W0, W1, K, c_mt, c_nt);
      }
    };
    int issued = 1;
    issue_next(0);
    if (c_live) {
      issue_next(1);
      ++issued;
      wait_vmcnt<Cfg::A_OPS + Cfg::B_OPS>();  // step 0 landed
    } else {
      wait_vmcnt<0>();
    }
    __builtin_amdgcn_s_barrier();  // X_{-1}
    for (int g = 0;; ++g) {
      wait_vmcnt<0>();               // step g + 1 landed (the only one in flight)
      __builtin_amdgcn_s_barrier();  // X_g
      if (c_live) {
        issue_next(g & 1);  // step g + 2 into step g's buffer
        ++issued;
      } else if (g + 1 >= issued) {
        break;  // X_g was the last step's barrier
      }
    }
    return;
  }

  // ---------------- matrix-core waves ----------------
  const int wm = wave / Cfg::WGN;
  const int wn = wave % Cfg::WGN;
  constexpr int MT16 = Cfg::WM / 16, NT16 = Cfg::WN / 16;
  constexpr int AR = Cfg::AR, PD = Cfg::PD;
  const int frag_row = lane & 15;
  const int fq = lane >> 4;
  // LDS byte addresses of the lane's fragments: the second 32-K half is the
  // first with chunk bit 2 flipped (xor 64), buffer 1 is buffer 0 xor 65536,
  // and row / column block offsets are immediates.
  const uint32_t v_lane = frag_row * kRowBytes + ((fq ^ ((frag_row >> 1) & 7)) << 4);
  const uint32_t b_row = kGateUp ? wn * (Cfg::WN / 2) : wn * Cfg::WN;
  uint32_t vA = (uint32_t)(wm * Cfg::WM) * kRowBytes + v_lane;
  uint32_t vB = (uint32_t)Cfg::A_BYTES + b_row * kRowBytes + v_lane;
  auto toggle = [&]() {
    vA ^= 65536u;
    vB ^= 65536u;
    asm volatile("" : "+v"(vA), "+v"(vB));
  };
  bf16x8_t fa[AR], fb[NT16];
  f32x4_t acc[MT16][NT16];
  auto lds128 = [&](uint32_t addr) -> bf16x8_t { return *reinterpret_cast<const bf16x8_t*>(smem + addr); };
  auto rdA = [&](bool other, int kh, int i) -> bf16x8_t {
    return lds128((vA ^ ((other ? 65536u : 0u) | (kh ? 64u : 0u))) + i * 16 * kRowBytes);
  };
  auto rdB = [&](bool other, int kh, int j) -> bf16x8_t {
    constexpr int half = NT16 / 2;
    const int r = kGateUp ? ((j < half) ? j * 16 : Cfg::BN / 2 + (j - half) * 16) : j * 16;
    return lds128((vB ^ ((other ? 65536u : 0u) | (kh ? 64u : 0u))) + r * kRowBytes);
  };
  // one 64-K step as 16 rows of 16 (two 32-K halves x 8 row blocks), 4 MFMAs
  // each; A rows are prefetched PD rows ahead into the ring; B fragments of
  // the next half are reloaded right after their last use; X_g sits before
  // the first read that targets the next step (from the other buffer, only if
  // kNext).
  auto step = [&](auto next_c) {
    constexpr bool kNext = decltype(next_c)::value;
    static_for<16>([&](auto rr) {
      constexpr int r = decltype(rr)::value;
      constexpr int i = r % 8;
      constexpr int rp = r + PD;
      if constexpr (rp == 16) {
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();  // X_g
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (rp < 16) {
        fa[rp % AR] = rdA(false, rp / 8, rp % 8);
      } else if constexpr (kNext) {
        fa[rp % AR] = rdA(true, 0, rp - 16);
      }
#pragma unroll
      for (int j = 0; j < NT16; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[r % AR], acc[i][j], 0, 0, 0);
        if constexpr (r == 7) fb[j] = rdB(false, 1, j);
        if constexpr (r == 15 && kNext) fb[j] = rdB(true, 0, j);
      }
      // a tile's last step keeps source order: scheduled freely, its reads
      // move up and the epilogue that follows runs out of registers
      if constexpr (!kNext) __builtin_amdgcn_sched_barrier(0);
    });
  };

  lds_barrier();  // X_{-1}
  char* stage = smem + STAGE_AREA + wave * (16 * OROW);
  while (true) {
    const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)mt * ASTRAI_MOE_TILE_STRIDE;
    const int t_row0 = ti[1];
    const int t_rows = min(Cfg::BM, ti[2] - t_row0);
#pragma unroll
    for (int i = 0; i < MT16; ++i)
#pragma unroll
      for (int j = 0; j < NT16; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;
    // the step's first fragments: B of the first half and A rows 0..PD-1
#pragma unroll
    for (int j = 0; j < NT16; ++j) fb[j] = rdB(false, 0, j);
#pragma unroll
    for (int r = 0; r < PD; ++r) fa[r % AR] = rdA(false, 0, r);
    for (int kt = 0; kt + 1 < KT; ++kt) {
      step(std::true_type{});
      toggle();
    }
    step(std::false_type{});
    toggle();
    __builtin_amdgcn_sched_barrier(0);
    store_tile<kGateUp, Cfg::WM, Cfg::WN, Cfg::BN>(acc, stage, row_w, C, N, wm, wn, t_row0, t_rows, nt);
    logical = walk.seek(logical + walk.G, mt, nt);
    if (logical >= walk.total) break;
  }
}

// ===========================================================================
// Decode kernel: 32-row tiles, every wave issues DMA, several stages in flight.
// ===========================================================================
template <int BM_, int BN_, int STAGES_, int WGM_, int WGN_, int GM_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, STAGES = STAGES_, WGM = WGM_, WGN = WGN_, GM = GM_;
  static constexpr int WAVES = WGM * WGN;
  static constexpr int THREADS = WAVES * 64;
  static constexpr int WM = BM / WGM;  // rows per wave
  static constexpr int WN = BN / WGN;  // columns per wave
  static constexpr int A_BYTES = BM * kRowBytes;
  static constexpr int B_BYTES = BN * kRowBytes;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int A_PER_WAVE = A_BYTES / 1024 / WAVES;  // 1 KB DMA ops per wave
  static constexpr int B_PER_WAVE = B_BYTES / 1024 / WAVES;
  static constexpr int DMA_PER_WAVE = A_PER_WAVE + B_PER_WAVE;
  static_assert(A_BYTES % (1024 * WAVES) == 0 && B_BYTES % (1024 * WAVES) == 0, "DMA ops split over waves");
  static_assert(WM % 16 == 0 && WN % 32 == 0, "16x16 MFMA tiles; gate/up halves");
  static_assert(STAGES >= 2 && STAGES * STAGE_BYTES <= 160 * 1024, "LDS");
  static_assert(DMA_PER_WAVE * (STAGES - 1) <= 63, "vmcnt range");
};

template <typename Cfg, bool kGateUp>
__global__ __launch_bounds__(Cfg::THREADS, 1) void gemm_mfma_kernel(
    const bf16_t* __restrict__ A, const int32_t* __restrict__ tiles, const void* const* __restrict__ W0,
    const void* const* __restrict__ W1, const bf16_t* __restrict__ row_w, int K, int N, int n_tiles_n,
    int capacity, bf16_t* __restrict__ C) {
  constexpr int S = Cfg::STAGES;
  constexpr int DPW = Cfg::DMA_PER_WAVE;
  constexpr int STAGE_AREA = S * Cfg::STAGE_BYTES;
  constexpr int OROW = staged_row_bytes<kGateUp, Cfg::WN>();
  static_assert(STAGE_AREA + Cfg::WAVES * 16 * OROW <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char smem[STAGE_AREA + Cfg::WAVES * 16 * OROW];

  const TileWalk<Cfg::GM> walk(tiles, capacity, n_tiles_n);
  int mt = 0, nt = 0;
  int logical = walk.seek(walk.first_slot(), mt, nt);
  if (logical >= walk.total) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wm = wave / Cfg::WGN;
  const int wn = wave % Cfg::WGN;
  const uint32_t k2 = (uint32_t)K * 2u;

  TileSrc<Cfg::BM, Cfg::BN, kGateUp> src;
  auto issue_stage = [&](int kstep, int buf) {
    char* sa = smem + buf * Cfg::STAGE_BYTES;
    char* sb = sa + Cfg::A_BYTES;
    const DmaLane dl(lane, kstep);
#pragma unroll
    for (int i = 0; i < Cfg::A_PER_WAVE; ++i) {
      const int q = wave * Cfg::A_PER_WAVE + i;
      src.dma_a(dl, q, k2, sa + q * 1024);
    }
#pragma unroll
    for (int i = 0; i < Cfg::B_PER_WAVE; ++i) {
      const int q = wave * Cfg::B_PER_WAVE + i;
      src.dma_b(dl, q, k2, sb + q * 1024);
    }
  };

  // ---- MFMA fragment reads (16x16x32: lane l holds row l % 16, K 8*(l/16)..+7) ----
  constexpr int MT16 = Cfg::WM / 16, NT16 = Cfg::WN / 16;
  const int frag_row = lane & 15;
  const int fq = lane >> 4;
  const int fsw = (frag_row >> 1) & 7;  // row bases are multiples of 16
  int a_off[MT16];
#pragma unroll
  for (int i = 0; i < MT16; ++i) a_off[i] = (wm * Cfg::WM + i * 16 + frag_row) * kRowBytes;
  int b_off[NT16];
#pragma unroll
  for (int j = 0; j < NT16; ++j) {
    int r;
    if (kGateUp) {
      constexpr int half = NT16 / 2;
      r = (j < half) ? wn * (Cfg::WN / 2) + j * 16 : Cfg::BN / 2 + wn * (Cfg::WN / 2) + (j - half) * 16;
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
  f32x4_t acc[MT16][NT16];
  auto mfmas = [&](int slot_) {
#pragma unroll
    for (int i = 0; i < MT16; ++i)
#pragma unroll
      for (int j = 0; j < NT16; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[slot_][j], fa[slot_][i], acc[i][j], 0, 0, 0);
  };
  // pair each fragment read of the next half with an MFMA of this one
  auto interleave = [&]() {
#pragma unroll
    for (int q = 0; q < MT16 + NT16; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, MT16 * NT16 - (MT16 + NT16), 0);
  };

  const int KT = K / kBK;
  src.setup(tiles, A, W0, W1, K, mt, nt);
#pragma unroll
  for (int s = 0; s < S; ++s)
    if (s < KT) issue_stage(s, s);
  wait_groups<DPW, S - 1>(min(S - 1, KT - 1));  // step 0 landed
  lds_barrier();
  char* stage = smem + STAGE_AREA + wave * (16 * OROW);
  while (true) {
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
        lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
        read_frags(nbuf, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (kt + S < KT) issue_stage(kt + S, buf);
        __builtin_amdgcn_sched_barrier(0);
      }
      mfmas(1);
      buf = nbuf;
    }

    // ---- next tile's first stages, then this tile's epilogue ----
    int nmt = 0, nnt = 0;
    const int nlogical = walk.seek(logical + walk.G, nmt, nnt);
    const bool has_next = nlogical < walk.total;
    const int t_row0 = src.row0, t_rows = src.rows, t_nt = nt;
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();  // every wave is done reading the stage buffers
    __builtin_amdgcn_sched_barrier(0);
    if (has_next) {
      src.setup(tiles, A, W0, W1, K, nmt, nnt);
#pragma unroll
      for (int s = 0; s < S; ++s)
        if (s < KT) issue_stage(s, s);
    }
    store_tile<kGateUp, Cfg::WM, Cfg::WN, Cfg::BN>(acc, stage, row_w, C, N, wm, wn, t_row0, t_rows, t_nt);
    if (!has_next) break;
    logical = nlogical;
    mt = nmt;
    nt = nnt;
    wait_vmcnt<0>();  // the next tile's stages (and this wave's stores) are done
    lds_barrier();
  }
}

// Decode tiles: 32 x 256 outputs, 4 waves of 32 x 64, four stages in flight
// to keep the expert-weight stream busy; every wave issues DMA.
using SmallCfg = TileCfg<kMfmaSmallBM, 256, 4, 1, 4, 8>;
static_assert(StreamCfg::BM == kMfmaBigBM, "prefill tile height");

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

// Grid of a persistent launch: one workgroup per compute unit (the LDS
// footprint allows no more), each walking its share of the tile list.
int persistent_grid(int64_t capacity, int64_t n_tiles_n, int64_t* grid) {
  const int64_t total = capacity * n_tiles_n;
  if (total >= (1ll << 31))
    return fail(ASTRAI_MOE_EINVAL, "gemm: %lld tiles exceed the tile-index range", (long long)total);
  *grid = std::min<int64_t>(total, cu_count());
  return ASTRAI_MOE_OK;
}

template <bool kGateUp>
int launch_stream(const void* A, const int32_t* tiles, int64_t capacity, const void* const* W0, const void* const* W1,
                  const void* row_w, int64_t K, int64_t N, void* C, hipStream_t s) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  const int64_t n_tiles_n = kGateUp ? N / (StreamCfg::BN / 2) : N / StreamCfg::BN;
  int64_t grid = 0;
  if (int rc = persistent_grid(capacity, n_tiles_n, &grid)) return rc;
  hipLaunchKernelGGL((gemm_stream_kernel<kGateUp>), dim3((unsigned)grid), dim3(StreamCfg::THREADS), 0, s,
                     static_cast<const bf16_t*>(A), tiles, W0, W1, static_cast<const bf16_t*>(row_w), (int)K, (int)N,
                     (int)n_tiles_n, (int)capacity, static_cast<bf16_t*>(C));
  return check_launch(kGateUp ? "gemm_stream_kernel<gate_up>" : "gemm_stream_kernel<down>");
}

template <typename Cfg, bool kGateUp>
int launch(const void* A, const int32_t* tiles, int64_t capacity, const void* const* W0, const void* const* W1,
           const void* row_w, int64_t K, int64_t N, void* C, hipStream_t s) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  const int64_t n_tiles_n = kGateUp ? N / (Cfg::BN / 2) : N / Cfg::BN;
  int64_t grid = 0;
  if (int rc = persistent_grid(capacity, n_tiles_n, &grid)) return rc;
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
    return launch_stream<true>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s);
  return launch<SmallCfg, true>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s);
}

int launch_mfma_down(const void* h, const int32_t* tiles, int64_t capacity, const void* const* w_down,
                     const void* sorted_w, int64_t dim_ffn, int64_t dim, int block_m, void* y, hipStream_t s) {
  if (block_m == kMfmaBigBM)
    return launch_stream<false>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s);
  return launch<SmallCfg, false>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s);
}

}  // namespace astrai_moe
