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
//   the DMA themselves, that wait came out of their MFMA schedule. LDS holds
//   two 32 KB activation stages and three 32 KB weight stages (160 KB); one
//   s_barrier per 64-K step, placed where every matrix-core wave has finished
//   reading the step's buffers: after it the DMA waves load the activations of
//   step g + 2 and the weights of step g + 3 (they come from HBM and get two
//   steps to land) and the matrix-core waves read step g + 1, whose data the
//   DMA waves waited for before the barrier. The matrix-core waves stream A
//   fragments through a ring of four registers two rows ahead and reload each
//   B fragment in place right after its last use, which keeps them within 168
//   VGPRs (the register file holds three waves of 168 per SIMD) with no
//   spills; every step, a tile's last included, prefetches the next step's
//   first fragments, so the K loop is one body with one register assignment.
//   The epilogue stores straight from the accumulators, after a lane-group
//   transpose (v_permlane32/16_swap) that gives each lane 16-byte row pieces.
//
// * gemm_mfma_kernel (32-row tiles, decode): 4 waves of 32 x 64, every wave
//   issues DMA, four 36 KB stages in flight to keep the expert-weight stream
//   busy; MFMA fragments are double-buffered per 32-K half; the epilogue
//   stages 16-row pieces per wave in LDS and stores 16-byte row segments.
//
// Variants (template flags): kPacked reads the weights from a packed copy
// (pack_kernel: one contiguous 32 KB block per 256-row tile and 64-K step);
// kSave (training forward) also stores what the backward needs; kGather
// (gate/up) reads the activation rows as x[sorted_token[r]] instead of from a
// copied x_perm.
//
// Epilogue: accumulators are rounded to bf16 with the hardware converter
// (v_cvt_pk_bf16_f32, round-to-nearest-even), SiLU is g * rcp(1 + 2^(-g*log2e))
// on v_exp_f32 / v_rcp_f32 (within 2 ulp of the libm form before its bf16
// rounding). The weight fragment is the MFMA's first operand, which leaves
// each lane 4 consecutive output columns of one row.
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
#include "mfma_tile.h"

#include <type_traits>


namespace astrai_moe {
namespace {

// Per-tile global bases: activation rows and the expert's weight rows. With
// kPacked the expert's weight comes as a packed copy (pack_kernel): the BN
// weight rows of column tile nt are K / 64 contiguous blocks of BN x 128
// bytes, each already in the staged (swizzled) LDS order, so a step's weight
// load is one contiguous block.
// With kGather the activation rows are token rows of x read through the
// permutation (GatherRows) rather than rows of a copied x_perm.
template <int BM, int BN, bool kGateUp, bool kPacked = false, bool kGather = false>
struct TileSrc {
  const char* a_base = nullptr;
  const char* b_base0 = nullptr;
  const char* b_base1 = nullptr;
  int row0 = 0, rows = 0;
  int b_rows = 0;  // weight rows of this column tile inside the matrix (per operand for gate/up)
  __device__ void setup(const int32_t* tiles, const bf16_t* A, const void* const* W0, const void* const* W1, int K,
                        int N, int mt, int nt) {
    const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)mt * ASTRAI_MOE_TILE_STRIDE;
    const int e = ti[0];
    row0 = ti[1];
    rows = min(BM, ti[2] - row0);
    constexpr int kTileRows = kGateUp ? BN / 2 : BN;
    b_rows = min(kTileRows, N - nt * kTileRows);
    a_base = reinterpret_cast<const char*>(kGather ? A : A + (int64_t)row0 * K);
    if constexpr (kPacked) {
      b_base0 = static_cast<const char*>(W0[e]) + (int64_t)nt * (K / kBK) * (BN * kRowBytes);
      b_base1 = b_base0;
    } else {
      b_base0 = reinterpret_cast<const char*>(static_cast<const bf16_t*>(W0[e]) +
                                              (int64_t)nt * (kGateUp ? BN / 2 : BN) * K);
      b_base1 = kGateUp ? reinterpret_cast<const char*>(static_cast<const bf16_t*>(W1[e]) + (int64_t)nt * (BN / 2) * K)
                        : b_base0;
    }
  }
  // 8-row group q of the A tile (pad rows past the tile's last row re-read that row)
  __device__ void dma_a(const DmaLane& dl, int q, uint32_t k2, char* lds) const {
    const uint32_t row = (uint32_t)min(q * 8 + dl.row, rows - 1);
    lds_dma_16(a_base + (row * k2 + dl.chunk(q)), lds);
  }
  // 8-row group q of the A tile, the lane's row at byte offset row_off of x (gather)
  __device__ void dma_a_rows(const DmaLane& dl, uint32_t row_off, int q, char* lds) const {
    lds_dma_16(a_base + (row_off + dl.chunk(q)), lds);
  }
  // 8-row group q of the B tile of K step kstep (up rows follow the gate rows;
  // in a partial last column tile, rows past the matrix re-read its last row,
  // and the epilogue stores none of their columns)
  __device__ void dma_b(const DmaLane& dl, int lane, int kstep, int q, uint32_t k2, char* lds) const {
    if constexpr (kPacked) {
      lds_dma_16(b_base0 + ((uint32_t)kstep * (BN * kRowBytes) + (uint32_t)q * 1024 + (uint32_t)lane * 16), lds);
    } else {
      (void)lane, (void)kstep;
      const int r0 = q * 8;
      const char* bb = (kGateUp && r0 >= BN / 2) ? b_base1 : b_base0;
      const int rq = (kGateUp && r0 >= BN / 2) ? r0 - BN / 2 : r0;
      lds_dma_16(bb + ((uint32_t)min(rq + dl.row, b_rows - 1) * k2 + dl.chunk(q)), lds);
    }
  }
};

// Byte offsets in x of the token rows one lane loads in its NQ activation DMA
// ops of a tile (ops qbase .. qbase + NQ - 1, row (q * 8 + lane / 8) of the
// tile, pad rows re-reading the tile's last row), read from the permutation's
// source-token list.
template <int NQ>
struct GatherRows {
  uint32_t off[NQ];
  __device__ void load(const int32_t* row_src, int row0, int rows, int qbase, int lane, uint32_t k2) {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int r = min((qbase + i) * 8 + (lane >> 3), rows - 1);
      off[i] = (uint32_t)row_src[row0 + r] * k2;
    }
  }
};

// Packs one expert's weight for kPacked kernels: for every column tile of BN
// = 256 weight rows (gate/up: 128 gate rows, then the same 128 up rows) and
// every 64-K step, the 256 x 128-byte block in staged order: row r's 16-byte
// chunk c at chunk c ^ ((r >> 1) & 7), as the DMA would have placed it. One
// thread per 16-byte unit.
template <bool kGateUp>
__global__ __launch_bounds__(256) void pack_kernel(const bf16_t* __restrict__ w0, const bf16_t* __restrict__ w1,
                                                   int64_t n_tiles, int K, uint4* __restrict__ out) {
  constexpr int BN = 256;
  const int KT = K / kBK;
  const int64_t units = n_tiles * KT * BN * 8;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x) {
    const int p = (int)(u & 7);
    const int r = (int)((u >> 3) & (BN - 1));
    const int64_t tk = u >> 11;  // (tile, step)
    const int kt = (int)(tk % KT);
    const int64_t nt = tk / KT;
    const int c = p ^ ((r >> 1) & 7);
    const bf16_t* row;
    if (kGateUp)
      row = (r < BN / 2) ? w0 + (nt * (BN / 2) + r) * (int64_t)K : w1 + (nt * (BN / 2) + r - BN / 2) * (int64_t)K;
    else
      row = w0 + (nt * BN + r) * (int64_t)K;
    out[u] = *reinterpret_cast<const uint4*>(row + kt * kBK + c * 8);
  }
}

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
    if (!kGateUp && row_w != nullptr) w = bf16_bits_to_f32(row_w[srow]);  // no row weights: 1
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
    // the 16 staged rows go out as 16 x SEGS pieces of 16 bytes, lane by lane
    // (one pass covers 64 pieces; narrow waves leave lanes idle)
    constexpr int SEGS = OUTC * 2 / 16;
    constexpr int PIECES = 16 * SEGS;
    wait_lds();
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int p = 0; p < (PIECES + 63) / 64; ++p) {
      const int idx = p * 64 + el;
      const int m = idx / SEGS;
      const int seg = idx % SEGS;
      const int gm = wm * WM + i * 16 + m;
      if (idx < PIECES) {
        const uint4 v = *reinterpret_cast<const uint4*>(stage + m * OROW + seg * 16);
        if (gm < t_rows && n_base + seg * 8 < N)
          *reinterpret_cast<uint4*>(C + (int64_t)(t_row0 + gm) * N + n_base + seg * 8) = v;
      }
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
template <bool kGateUp>
struct StreamCfg {
  // row tiles per group of the walk: gate/up walks 8 row tiles for every
  // column tile (each round's 8 activation strips are read by all 8 XCDs);
  // down walks paired halves of 8 (TileWalk, GM = 16). Measured in one
  // process, builds alternating, on two boxes: the paired walk took the down
  // GEMMs +0.1 / +0.5 % (Mixtral shape) and +1.1 / +4.8 % (fine-grained),
  // gate/up -2.7 % and -8.7 % (its activation strips then serve 4 XCDs).
  static constexpr int BM = 256, BN = 256, GM = kGateUp ? 8 : 16;
  static_assert(GM % kTileGroup == 0, "walk groups hold whole groups of the tile list");
  static constexpr int WGM = 2, WGN = 4, MW = 8, DW = 4;  // matrix-core waves (WGM x WGN), DMA waves
  static constexpr int WAVES = MW + DW, THREADS = WAVES * 64;
  static constexpr int WM = BM / WGM, WN = BN / WGN;  // 128 x 64 per matrix-core wave
  static constexpr int A_BYTES = BM * kRowBytes, B_BYTES = BN * kRowBytes;  // 32 KB per 64-K step each
  static constexpr int A_STAGES = 2, B_STAGES = 3;
  static constexpr int A_OFF = 0, B_OFF = A_STAGES * A_BYTES;
  static constexpr int LDS = B_OFF + B_STAGES * B_BYTES;  // 160 KB
  static constexpr int OPS = A_BYTES / 1024 / DW;         // 1 KB DMA ops per DMA wave per operand and step
  // Rows of 16 are taken in pairs, columns outer within a pair, so each B
  // fragment reloaded after its last use in a half has 6 MFMAs of lead; A
  // fragments stream through a ring of AR slots PD rows ahead.
  static constexpr int RG = 2, AR = 4, PD = 2;
  static_assert(A_BYTES == B_BYTES && A_BYTES % (1024 * DW) == 0, "one DMA group size");
  static_assert(A_BYTES == 32768 && A_STAGES == 2, "activation buffers toggle by xor 32768");
  static_assert(LDS <= 160 * 1024, "LDS");
  static_assert(16 % AR == 0 && 8 % RG == 0 && PD >= RG && PD + RG <= AR, "ring slots of a pair and its prefetch");
  static_assert(3 * OPS <= 63, "vmcnt range");
};

// Epilogue straight from the accumulators. Lane l holds 4 consecutive output
// columns of one row per 16x16 tile; a lane-group transpose (above) per pair
// of tiles first gathers each lane 8 consecutive columns, so a row block of 16
// rows goes out in 16-byte stores, each instruction covering 64 contiguous
// bytes of each of its 16 rows (half the store instructions and cache-line
// requests of 8-byte pieces; the stores share the load path with the next
// tile's DMA). kSave (training forward) also stores what the backward needs:
// for gate/up the bf16 gate and up projections interleaved in blocks of 4
// columns (S0 [rows, 2 N]: g[c..c+3] then u[c..c+3] at 2 c, one 16-byte store
// per lane, so each wave completes whole 128-byte lines), for down the
// unweighted bf16 expert output (S0, at C's positions).
template <bool kGateUp, int WM, int WN, int BN, bool kSave>
__device__ __forceinline__ void store_tile_direct(f32x4_t (&acc)[WM / 16][WN / 16], const bf16_t* row_w, bf16_t* C,
                                                  int N, int wm, int wn, int t_row0, int t_rows, int t_nt,
                                                  bf16_t* S0, bf16_t* S1) {
  constexpr int MT16 = WM / 16, NT16 = WN / 16;
  constexpr int NJ = kGateUp ? NT16 / 2 : NT16;  // output tiles of 16 columns
  static_assert(NJ % 2 == 0, "tiles are transposed in pairs");
  (void)S1;
  const int el = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int row_l = el & 15;
  const int q = el >> 4;
  const int n_base = kGateUp ? t_nt * (BN / 2) + wn * (WN / 2) : t_nt * BN + wn * WN;
  // gate/up: the tile's first row as a uniform base and the lanes at 32-bit
  // element offsets from it (a tile's rows hold at most 256 N elements, 512 N
  // for S0, below 2^31 with the launchers' N <= 2^22): the saving kernel then
  // keeps its addresses in registers (with 64-bit row offsets it spilled them
  // and reloaded them between the stores; training gate/up +0.7 % at the
  // Mixtral shape, bit-identical). The down kernels keep 64-bit offsets, which
  // spilled less there.
  using Off = std::conditional_t<kGateUp, uint32_t, int64_t>;
  bf16_t* const Ct = kGateUp ? C + (int64_t)t_row0 * N : C;
  bf16_t* const St = kSave && kGateUp ? S0 + (int64_t)t_row0 * N * 2 : S0;
#pragma unroll
  for (int i = 0; i < MT16; ++i) {
    const int gm = wm * WM + i * 16 + row_l;
    const int srow = t_row0 + min(gm, t_rows - 1);
    float w = 1.0f;
    if (!kGateUp && row_w != nullptr) w = bf16_bits_to_f32(row_w[srow]);  // no row weights: 1
    const Off row_off = kGateUp ? (Off)(uint32_t)(min(gm, t_rows - 1) * N + n_base) : (Off)((int64_t)srow * N + n_base);
#pragma unroll
    for (int jp = 0; jp < NJ; jp += 2) {
      // gate/up: h = bf16(u * bf16(silu(g))) per element, then transposed;
      // down: the rounded unweighted output is transposed and then scaled by
      // the row's weight (the transpose keeps each lane's row)
      bf16x4_t o[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = jp + h;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const __bf16 a = (__bf16)acc[i][j][r];
          if (kGateUp) {
            const float g = (float)a;
            const float u = (float)(__bf16)acc[i][j + NJ][r];
            const float ex = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
            const float sv = (float)(__bf16)(g * __builtin_amdgcn_rcpf(1.0f + ex));
            o[h][r] = (__bf16)(u * sv);
          } else {
            o[h][r] = a;
          }
        }
        if constexpr (kSave && kGateUp) {
          // g and u in the accumulator layout: row r, column c of h -> 2 (r N + c)
          if (gm < t_rows && n_base + j * 16 + 4 * q < N) {
            bf16x8_t gu;
#pragma unroll
            for (int r = 0; r < 4; ++r) gu[r] = (__bf16)acc[i][j][r], gu[4 + r] = (__bf16)acc[i][j + NJ][r];
            *reinterpret_cast<bf16x8_t*>(St + (Off)2 * (row_off + j * 16 + 4 * q)) = gu;
          }
        }
      }
      transpose2(o);
      // N is a multiple of 8: a lane's 8 columns are all inside the matrix or all past it
      if (gm < t_rows && n_base + jp * 16 + 8 * q < N) {
        bf16x8_t v;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = o[0][r], v[4 + r] = o[1][r];
        if constexpr (!kGateUp) {
          if constexpr (kSave) *reinterpret_cast<bf16x8_t*>(St + (row_off + jp * 16 + 8 * q)) = v;
#pragma unroll
          for (int c = 0; c < 8; ++c) v[c] = (__bf16)((float)v[c] * w);
        }
        *reinterpret_cast<bf16x8_t*>(Ct + (row_off + jp * 16 + 8 * q)) = v;
      }
    }
  }
}

// The order in which one workgroup takes its work items. Items below `dyn`
// are dealt statically: the workgroup's slot, then every G-th item. Given a
// scheduling block (`sched`, its counter cleared before the launch), the
// items from `dyn` on are claimed at run time from the counter sched[0] by
// whichever workgroups get there first, so that the compute units running at
// a higher clock take more of them (the XCDs of one part hold clocks several
// per cent apart under this load, and with a static deal the slowest one sets
// the kernel's end). Matrix-core wave 0 claims a workgroup's next item
// kClaimLead steps before the end of its current one and publishes it in the
// workgroup's ring of 8 mailbox slots (sched[kMailboxBase + 8 b ...]); every
// wave reads it when it leaves the current item, at least two barriers
// after the store (the DMA waves run up to three steps ahead of the
// matrix-core waves). -1: no item. Claiming that late needs every dynamic
// item to last more than kClaimLead steps. A claim stalls its workgroup for
// about an atomic's round trip, so claims are made only where tiles are long
// (kDynamicMinSteps): measured against the static deal, in one process with
// the builds alternating, the Mixtral-shaped GEMMs (64 and 224 steps per
// tile) gained 1.8 % (gate/up) and 0.8 % (down). At the fine-grained shape
// the 32-step gate/up tiles gained 2.3-2.7 % (1.1-1.2 % with the skewed
// router) once padding-only waves idled, and the 22-step down tiles lost
// 1.3-1.7 %.
constexpr int kMailboxBase = 64;       // int32 offset of the mailboxes in the scheduling block
constexpr int kMaxSchedGroups = 1024;  // workgroups the scheduling block has mailboxes for
constexpr int kDynamicShare = 10;      // 1 / kDynamicShare of the items are claimed at run time
constexpr int kDynamicMinSteps = 32;   // K steps per tile from which items are claimed at run time
constexpr int kClaimLead = 6;
static_assert(kClaimLead > 4 && kClaimLead < kSplitMinSteps, "claim between the DMA waves' lead and an item's end");

struct ItemSeq {
  int slot, G, m, n, dyn;
  int* mbox;  // the workgroup's 8 mailbox slots (nullptr: static deal only)
  template <int GM>
  __device__ ItemSeq(const SplitWalk<GM>& walk, int KT, int* sched)
      : slot(walk.first_slot()), G(walk.G), n(walk.items()), dyn(walk.items()), mbox(nullptr) {
    if (sched != nullptr && KT >= kDynamicMinSteps && G <= kMaxSchedGroups) {
      const int d = max(G, n - n / kDynamicShare);
      if (d < n) dyn = d, mbox = sched + kMailboxBase + 8 * (int)blockIdx.x;
    }
    m = slot < dyn ? (dyn - slot + G - 1) / G : 0;
  }
  // the workgroup's item `idx` (a mailbox read for the claimed ones)
  __device__ int id(int idx) const {
    if (idx < m) return slot + idx * G;
    if (mbox == nullptr) return -1;
    return __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(mbox + ((idx - m) & 7), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  }
  // whether the item after `idx` is claimed at run time
  __device__ bool claims_next(int idx) const { return mbox != nullptr && idx + 1 >= m; }
  // matrix-core wave 0, kClaimLead steps before the end of item `idx`:
  // claims the next item; false once a claim came back empty
  __device__ bool claim(int idx, int* sched) const {
    int c = 0;
    if (__lane_id() == 0) c = __hip_atomic_fetch_add(sched, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    c = __builtin_amdgcn_readfirstlane(c);
    const int v = dyn + c < n ? dyn + c : -1;
    if (__lane_id() == 0)
      __hip_atomic_store(mbox + ((idx + 1 - m) & 7), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the store lands in L2 before this wave's next barrier
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return v >= 0;
  }
};

// Position of a DMA wave in this workgroup's step sequence: the work item
// and K step it loads next, and that tile's global bases.
template <int BM, int BN, int GM, bool kGateUp, bool kPacked, bool kGather = false>
struct StepCursor {
  int idx, mt, nt, kt, k1, unit;  // idx: the item's place in the workgroup's order
  bool live;
  TileSrc<BM, BN, kGateUp, kPacked, kGather> src;
  __device__ void enter(const SplitWalk<GM>& walk, int logical, const int32_t* tiles, const bf16_t* A,
                        const void* const* W0, const void* const* W1, int K, int N) {
    walk.item(logical, mt, nt, kt, k1, unit);
    src.setup(tiles, A, W0, W1, K, N, mt, nt);
  }
  __device__ void start(const SplitWalk<GM>& walk, const ItemSeq& seq, const int32_t* tiles, const bf16_t* A,
                        const void* const* W0, const void* const* W1, int K, int N) {
    idx = 0, live = true;
    enter(walk, seq.id(0), tiles, A, W0, W1, K, N);
  }
  // true when the cursor moved on to the next work item
  __device__ bool advance(const SplitWalk<GM>& walk, const ItemSeq& seq, const int32_t* tiles, const bf16_t* A,
                          const void* const* W0, const void* const* W1, int K, int N) {
    if (++kt < k1) return false;
    const int nxt = seq.id(++idx);  // a claimed item was published two barriers ago
    live = nxt >= 0;
    if (live) enter(walk, nxt, tiles, A, W0, W1, K, N);
    return live;
  }
};

// kGather: A is x and the activation rows are gathered through row_src (the
// permutation's source tokens).
template <bool kGateUp, bool kPacked, bool kSave, bool kGather = false>
__global__ __launch_bounds__(StreamCfg<kGateUp>::THREADS, 1) void gemm_stream_kernel(
    const bf16_t* __restrict__ A, const int32_t* __restrict__ tiles, const void* const* __restrict__ W0,
    const void* const* __restrict__ W1, const bf16_t* __restrict__ row_w, int K, int N, int n_tiles_n,
    int capacity, bf16_t* __restrict__ C, bf16_t* __restrict__ S0, bf16_t* __restrict__ S1,
    const int32_t* __restrict__ row_src, float* __restrict__ part, int32_t* __restrict__ sched) {
  using Cfg = StreamCfg<kGateUp>;
  __shared__ __attribute__((aligned(1024))) char smem[Cfg::LDS];

  const int KT = K / kBK;  // steps per tile
  // part: partial sums of the split tail tiles (null: the tail runs whole;
  // only the down GEMMs take one); sched: the run-time claims (null: the
  // whole walk is dealt statically)
  const SplitWalk<Cfg::GM> walk(tiles, capacity, n_tiles_n, KT, !kGateUp && part != nullptr);
  const ItemSeq seq(walk, KT, sched);
  if (seq.m == 0) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;

  // Global steps g = 0, 1, ... run over this workgroup's tiles back to back.
  // Step g's activations live in A-buffer g % 2 and its weights in B-buffer
  // g % 3. Barrier X_g: every matrix-core wave has read all of step g, and
  // A(g + 1) and B(g + 1) have landed; after it the DMA waves load A(g + 2)
  // and B(g + 3) into the buffers step g held. The weights, which come from
  // HBM, thus have two steps to land, the activations one. Every wave
  // executes X_{-1} and then exactly one X_g per step.
  if (wave >= Cfg::MW) {
    // ---------------- DMA waves ----------------
    const int dw = wave - Cfg::MW;
    const uint32_t k2 = (uint32_t)K * 2u;
    StepCursor<Cfg::BM, Cfg::BN, Cfg::GM, kGateUp, kPacked, kGather> ca;  // next A step
    StepCursor<Cfg::BM, Cfg::BN, Cfg::GM, kGateUp, kPacked> cb;           // next B step
    GatherRows<Cfg::OPS> grows;
    auto load_rows = [&]() {
      if constexpr (kGather) grows.load(row_src, ca.src.row0, ca.src.rows, dw * Cfg::OPS, lane, k2);
    };
    ca.start(walk, seq, tiles, A, W0, W1, K, N);
    cb.start(walk, seq, tiles, A, W0, W1, K, N);
    load_rows();
    auto issue_a = [&](int buf) {
      const DmaLane dl(lane, ca.kt);
      char* base = smem + Cfg::A_OFF + buf * Cfg::A_BYTES;
#pragma unroll
      for (int i = 0; i < Cfg::OPS; ++i) {
        const int q = dw * Cfg::OPS + i;
        if constexpr (kGather)
          ca.src.dma_a_rows(dl, grows.off[i], q, base + q * 1024);
        else
          ca.src.dma_a(dl, q, k2, base + q * 1024);
      }
      if (ca.advance(walk, seq, tiles, A, W0, W1, K, N)) load_rows();  // the next item's rows
    };
    auto issue_b = [&](int buf) {
      const DmaLane dl(lane, cb.kt);
      char* base = smem + Cfg::B_OFF + buf * Cfg::B_BYTES;
#pragma unroll
      for (int i = 0; i < Cfg::OPS; ++i) {
        const int q = dw * Cfg::OPS + i;
        cb.src.dma_b(dl, lane, cb.kt, q, k2, base + q * 1024);
      }
      cb.advance(walk, seq, tiles, A, W0, W1, K, N);
    };
    // prologue in issue order B0, A0, B1, A1, B2 (as far as the steps exist)
    int a_iss = 0, b_iss = 0;
    issue_b(0), ++b_iss;
    issue_a(0), ++a_iss;
    if (cb.live) issue_b(1), ++b_iss;
    if (ca.live) issue_a(1), ++a_iss;
    if (cb.live) issue_b(2), ++b_iss;
    wait_groups<Cfg::OPS, 3>((a_iss - 1) + (b_iss - 1));  // A0 and B0 landed
    __builtin_amdgcn_s_barrier();                          // X_{-1}
    for (int g = 0;; ++g) {
      // A(g + 1) and B(g + 1) landed; B(g + 2), issued after A(g + 1), may stay in flight
      wait_groups<Cfg::OPS, 1>(b_iss > g + 2 ? 1 : 0);
      __builtin_amdgcn_s_barrier();  // X_g
      const bool more = ca.live;
      if (ca.live) issue_a(g & 1), ++a_iss;  // A(g + 2)
      if (cb.live) issue_b(g % 3), ++b_iss;  // B(g + 3)
      if (!more && g + 1 >= a_iss) break;    // X_g was the last step's barrier
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
  // LDS byte addresses of the lane's fragments in the current buffers: the
  // second 32-K half is the first with chunk bit 2 flipped (xor 64); row and
  // column block offsets are immediates.
  const uint32_t v_lane = frag_row * kRowBytes + ((fq ^ ((frag_row >> 1) & 7)) << 4);
  const uint32_t b_row = kGateUp ? wn * (Cfg::WN / 2) : wn * Cfg::WN;
  uint32_t vA = (uint32_t)Cfg::A_OFF + (uint32_t)(wm * Cfg::WM) * kRowBytes + v_lane;
  uint32_t vB = (uint32_t)Cfg::B_OFF + b_row * kRowBytes + v_lane;
  constexpr uint32_t kBEnd = (uint32_t)Cfg::LDS;
  auto next_b = [&](uint32_t v) -> uint32_t {
    const uint32_t n = v + Cfg::B_BYTES;
    return n >= kBEnd ? n - Cfg::B_STAGES * Cfg::B_BYTES : n;
  };
  auto rotate = [&]() {
    vA ^= (uint32_t)Cfg::A_BYTES;
    vB = next_b(vB);
    asm volatile("" : "+v"(vA), "+v"(vB));
  };
  bf16x8_t fa[AR], fb[NT16];
  f32x4_t acc[MT16][NT16];
  auto lds128 = [&](uint32_t addr) -> bf16x8_t { return *reinterpret_cast<const bf16x8_t*>(smem + addr); };
  auto rdA = [&](uint32_t base, int kh, int i) -> bf16x8_t {
    return lds128((base ^ (kh ? 64u : 0u)) + i * 16 * kRowBytes);
  };
  auto rdB = [&](uint32_t base, int kh, int j) -> bf16x8_t {
    constexpr int half = NT16 / 2;
    const int r = kGateUp ? ((j < half) ? j * 16 : Cfg::BN / 2 + (j - half) * 16) : j * 16;
    return lds128((base ^ (kh ? 64u : 0u)) + r * kRowBytes);
  };
  // one 64-K step as 16 rows of 16 (two 32-K halves x 8 row blocks) taken in
  // groups of RG rows, 4 x RG MFMAs each; A rows are prefetched PD rows ahead
  // into the ring; B fragments of the next half are reloaded right after
  // their last use; X_g sits before the first read that targets the next
  // step (only if kNext).
  constexpr int RG = Cfg::RG;
  auto step = [&](auto next_c) {
    constexpr bool kNext = decltype(next_c)::value;
    uint32_t nA = 0, nB = 0;
    static_for<16 / RG>([&](auto gg) {
      constexpr int r0 = decltype(gg)::value * RG;
      // Issue priority falls as a wave gets through the step, so that of the
      // two matrix-core waves on a SIMD the one behind takes the matrix core.
      // At equal priority the older wave issued first: it reached the step
      // barrier well ahead (~35 % of the step in per-step cycle counts), and
      // the other then issued its last rows alone, where its own fragment
      // reads left gaps. gate/up: 1 from row 0, 0 from row 8, 1 for rows 10
      // and 11, 0 from row 12; down: 1 from row 0, 0 from row 10, 1 from row
      // 12. Measured in one process, builds alternating, bit-identical, with
      // the single drop (row 8 gate/up, row 10 down): gate/up +2.1 to +2.5 %
      // (Mixtral shape), +2.7 to +3.2 % (fine-grained shape), down +2.4 to
      // +3.4 %; the later steps up and down added +0.3 to +0.7 % (Mixtral
      // shape). Drops at rows 4, 6 or 12 alone made the gathering gate/up
      // GEMM's tile changes spill; three levels (2, 1, 0) measured -0.5 to
      // -3.8 %.
      if constexpr (r0 == 0) __builtin_amdgcn_s_setprio(1);
      if constexpr (kGateUp ? (r0 == 8 || r0 == 12) : r0 == 10) __builtin_amdgcn_s_setprio(0);
      if constexpr (kGateUp ? r0 == 10 : r0 == 12) __builtin_amdgcn_s_setprio(1);
      if constexpr (r0 + PD >= 16 && r0 + PD < 16 + RG) {
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();  // X_g
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kNext) {
          nA = vA ^ (uint32_t)Cfg::A_BYTES;
          nB = next_b(vB);
        }
      }
      static_for<RG>([&](auto qq) {
        constexpr int rp = r0 + PD + decltype(qq)::value;
        if constexpr (rp < 16) {
          fa[rp % AR] = rdA(vA, rp / 8, rp % 8);
        } else if constexpr (kNext) {
          fa[rp % AR] = rdA(nA, 0, rp - 16);
        }
      });
#pragma unroll
      for (int j = 0; j < NT16; ++j) {
        static_for<RG>([&](auto qq) {
          constexpr int r = r0 + decltype(qq)::value;
          acc[r % 8][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[r % AR], acc[r % 8][j], 0, 0, 0);
        });
        if constexpr (r0 + RG == 8) fb[j] = rdB(vB, 1, j);
        if constexpr (r0 + RG == 16 && kNext) fb[j] = rdB(nB, 0, j);
      }
      // a tile's last step keeps source order: scheduled freely, its reads
      // move up and the epilogue that follows runs out of registers
      if constexpr (!kNext) __builtin_amdgcn_sched_barrier(0);
    });
  };

  lds_barrier();  // X_{-1}
  // the first step's first fragments: B of the first half and A rows 0..PD-1
#pragma unroll
  for (int j = 0; j < NT16; ++j) fb[j] = rdB(vB, 0, j);
#pragma unroll
  for (int r = 0; r < PD; ++r) fa[r % AR] = rdA(vA, 0, r);
  int mt = 0, nt = 0, k0 = 0, k1 = 0, unit = -1;
  bool claiming = wave == 0;  // matrix-core wave 0 makes the run-time claims
  // first row of this wave's half: a tile with no more rows leaves the wave
  // only padding (idle_threshold). idle_mt0: the first
  // row tile where such waves idle: every tile in GEMMs of short tiles (fewer
  // than kIdleMaxSteps K steps), else the tiles after the list's whole groups
  // of one expert (tiles[3]), which the walk reaches last.
  const int idle_row0 = __builtin_amdgcn_readfirstlane(wm * Cfg::WM);
  const int idle_mt0 = __builtin_amdgcn_readfirstlane(KT < kIdleMaxSteps ? 0 : tiles[3]);
  walk.item(seq.id(0), mt, nt, k0, k1, unit);
  for (int idx = 0;; ++idx) {
    const int claim_at = (claiming && seq.claims_next(idx)) ? k1 - kClaimLead : -1;
    const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)mt * ASTRAI_MOE_TILE_STRIDE;
    const int t_row0 = ti[1];
    const int t_rows = min(Cfg::BM, ti[2] - t_row0);
    // An expert's last tile with at most BM / 2 rows: the waves of the second
    // half hold only padding rows, so they keep the step barriers and the
    // next item's prefetch but issue no MFMAs and store nothing. Measured in
    // one process, builds alternating, bit-identical: fine-grained down GEMM
    // +6.7 %, Zipf-skewed gate/up +6.3 %. With long tiles (Mixtral shape)
    // inside the whole groups it was within +-0.4 %, and the workgroups of
    // such tiles ran ahead of the others of their XCD, which then shared
    // fewer operand strips in L2 (gate/up FETCH_SIZE +46 %, hits 78 -> 68 %):
    // long tiles idle only after the whole groups.
    // (as a row threshold: the two compares joined by && made the compiler
    // spill the prefetched fragments around the branch)
    const bool idle = idle_threshold(mt >= idle_mt0, idle_row0) >= t_rows;
    // The down kernels clear their accumulators from a zero in an SGPR:
    // cleared from 0.0f, their register allocation kept a VGPR zero that it
    // spilled across the K loop, and its reload after the epilogue made each
    // tile wait for all of the previous tile's stores (s_waitcnt vmcnt(0))
    // before its first MFMA. Measured in one process, builds alternating:
    // down +1.9 % (fine-grained shape), +1.0 % (Mixtral shape). The gate/up
    // kernels keep 0.0f: they spill nothing that way, and the SGPR zero made
    // them spill (-2.5 %, -0.7 %).
    float zero = 0.0f;
    if constexpr (!kGateUp) {
      int zs;
      asm("s_mov_b32 %0, 0" : "=s"(zs));
      zero = __builtin_bit_cast(float, zs);
    }
#pragma unroll
    for (int i = 0; i < MT16; ++i)
#pragma unroll
      for (int j = 0; j < NT16; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = zero;
    if (idle) {
      for (int kt = k0; kt < k1; ++kt) {
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();  // X_g
        __builtin_amdgcn_sched_barrier(0);
        if (kt + 1 == k1) {
          // the next item's first fragments, as the last step of a tile reads them
          const uint32_t nA = vA ^ (uint32_t)Cfg::A_BYTES, nB = next_b(vB);
#pragma unroll
          for (int r = 0; r < PD; ++r) fa[r % AR] = rdA(nA, 0, r);
#pragma unroll
          for (int j = 0; j < NT16; ++j) fb[j] = rdB(nB, 0, j);
        }
        rotate();
      }
    } else {
    // Every step, a tile's last included, prefetches the first fragments of
    // the step after it, which is the next item's first step (its data has
    // landed by X_g; after the workgroup's last step the reads return stale
    // LDS contents that nothing uses). One loop body keeps one register
    // assignment, so the accumulators do not spill at tile boundaries.
    // the K loop runs in two stretches around the claim, so that the loop
    // body itself carries nothing for it
    for (int kt = k0, stop = claim_at >= 0 ? claim_at : k1;; stop = k1) {
      for (; kt < stop; ++kt) {
        step(std::true_type{});
        rotate();
      }
      if (kt == k1) break;
      claiming = seq.claim(idx, sched);
    }
    }
    __builtin_amdgcn_sched_barrier(0);
    const int nxt = seq.id(idx + 1);
    if (kGateUp || unit < 0) {
      if (!idle)
        store_tile_direct<kGateUp, Cfg::WM, Cfg::WN, Cfg::BN, kSave>(acc, row_w, C, N, wm, wn, t_row0, t_rows, nt,
                                                                     S0, S1);
    } else {
      store_partial(acc, part, unit, wave, lane);
    }
    if (nxt < 0) break;
    walk.item(nxt, mt, nt, k0, k1, unit);
  }
}

// The epilogue of the split tail tiles (SplitWalk): workgroup (t, w), one
// wave, sums the S partials of matrix-core wave w's accumulators of tail
// tile t in slice order and stores them as that wave stores a whole tile.
// (One wave per workgroup: with a workgroup of 8 waves per tile, the 32-64
// tail tiles of the Mixtral-shaped down GEMM left most compute units idle
// and the reduce took ~45 us.) G is the streaming launch's grid; the walk is recomputed from the
// same tile list, so both kernels agree on which tiles were split.
template <bool kGateUp, bool kSave>
__global__ __launch_bounds__(64) void split_reduce_kernel(const float* __restrict__ part,
                                                           const int32_t* __restrict__ tiles, int capacity,
                                                           int n_tiles_n, int K, int G,
                                                           const bf16_t* __restrict__ row_w, bf16_t* __restrict__ C,
                                                           int N, bf16_t* __restrict__ S0) {
  using Cfg = StreamCfg<kGateUp>;
  const SplitWalk<Cfg::GM> walk(tiles, capacity, n_tiles_n, K / kBK, true, G);
  const int t = blockIdx.x;
  if (walk.S < 2 || t >= walk.total - walk.full) return;
  int mt = 0, nt = 0;
  walk.decode(walk.full + t, mt, nt);
  const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)mt * ASTRAI_MOE_TILE_STRIDE;
  const int t_row0 = ti[1];
  const int t_rows = min(Cfg::BM, ti[2] - t_row0);
  const int wave = blockIdx.y, lane = threadIdx.x;
  constexpr int MT16 = Cfg::WM / 16, NT16 = Cfg::WN / 16;
  constexpr int kUnitVecs = kSplitUnitFloats / 4;
  const f32x4_t* p = reinterpret_cast<const f32x4_t*>(part) + (int64_t)t * walk.S * kUnitVecs +
                     wave * (MT16 * NT16 * 64) + lane;
  f32x4_t acc[MT16][NT16];
#pragma unroll
  for (int i = 0; i < MT16; ++i)
#pragma unroll
    for (int j = 0; j < NT16; ++j) acc[i][j] = p[(i * NT16 + j) * 64];
  for (int s = 1; s < walk.S; ++s) {
    const f32x4_t* ps = p + (int64_t)s * kUnitVecs;
#pragma unroll
    for (int i = 0; i < MT16; ++i)
#pragma unroll
      for (int j = 0; j < NT16; ++j) acc[i][j] += ps[(i * NT16 + j) * 64];
  }
  store_tile_direct<kGateUp, Cfg::WM, Cfg::WN, Cfg::BN, kSave>(acc, row_w, C, N, wave / Cfg::WGN, wave % Cfg::WGN,
                                                               t_row0, t_rows, nt, S0, nullptr);
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

template <typename Cfg, bool kGateUp, bool kPacked, bool kGather = false>
__global__ __launch_bounds__(Cfg::THREADS, 1) void gemm_mfma_kernel(
    const bf16_t* __restrict__ A, const int32_t* __restrict__ tiles, const void* const* __restrict__ W0,
    const void* const* __restrict__ W1, const bf16_t* __restrict__ row_w, int K, int N, int n_tiles_n,
    int capacity, bf16_t* __restrict__ C, const int32_t* __restrict__ row_src) {
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

  static_assert(!kPacked || Cfg::BN == 256, "packed weights come in 256-row tiles");
  TileSrc<Cfg::BM, Cfg::BN, kGateUp, kPacked, kGather> src;
  GatherRows<Cfg::A_PER_WAVE> grows;
  // The K steps of a tile of expert e run from step (7 e) mod KT around to
  // the one before it, so the workgroups streaming different experts at the
  // same time read their weight rows at different K offsets, while the
  // column tiles of one expert still read its activation tile together (and
  // share it in L2). Starting every tile at step 0 puts the concurrent reads
  // of rows that lie a power of two apart (8 KB rows at K = 4096, experts of
  // one stacked allocation) at equal offsets, which measured 11 % slower on
  // the decode gate/up GEMM. The start depends only on the expert, so every
  // tile height sums an output in the same order.
  const int kt_n = K / kBK;
  int k_start = 0;
  auto setup_tile = [&](int mt_, int nt_) {
    src.setup(tiles, A, W0, W1, K, N, mt_, nt_);
    k_start = (tiles[ASTRAI_MOE_TILE_HEADER + (int64_t)mt_ * ASTRAI_MOE_TILE_STRIDE] * 7) % kt_n;
    if constexpr (kGather) grows.load(row_src, src.row0, src.rows, wave * Cfg::A_PER_WAVE, lane, k2);
  };
  auto issue_stage = [&](int kstep, int buf) {  // the tile's kstep-th step
    char* sa = smem + buf * Cfg::STAGE_BYTES;
    char* sb = sa + Cfg::A_BYTES;
    const int ks = kstep + k_start < kt_n ? kstep + k_start : kstep + k_start - kt_n;  // K step loaded
    const DmaLane dl(lane, ks);
#pragma unroll
    for (int i = 0; i < Cfg::A_PER_WAVE; ++i) {
      const int q = wave * Cfg::A_PER_WAVE + i;
      if constexpr (kGather)
        src.dma_a_rows(dl, grows.off[i], q, sa + q * 1024);
      else
        src.dma_a(dl, q, k2, sa + q * 1024);
    }
#pragma unroll
    for (int i = 0; i < Cfg::B_PER_WAVE; ++i) {
      const int q = wave * Cfg::B_PER_WAVE + i;
      src.dma_b(dl, lane, ks, q, k2, sb + q * 1024);
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
  setup_tile(mt, nt);
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
      setup_tile(nmt, nnt);
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
// Mid tiles: 64 x 256 outputs, 8 waves of 32 x 64 (the decode wave tile, two
// rows of waves), three stages in flight: 3 x 40 KB of stages + the waves'
// epilogue slices fit the 160 KB of LDS.
using MidCfg = TileCfg<kMfmaMidBM, 256, 3, 2, 4, 8>;
// 128-row tiles: 128 x 256 outputs, 8 waves side by side (128 x 32 each, so
// the down epilogue's per-wave 16-row slices stay small), three 48 KB stages
// in flight: 144 KB of stages + 10 KB of epilogue slices.
using Mid2Cfg = TileCfg<kMfmaMid2BM, 256, 3, 1, 8, 8>;
static_assert(StreamCfg<true>::BM == kMfmaBigBM && StreamCfg<false>::BM == kMfmaBigBM, "prefill tile height");

// Clears the run-time claim counter of a streaming launch's scheduling
// block (enqueued right before it, so the caller's workspace needs no
// initialisation and a captured graph clears it on every replay).
__global__ __launch_bounds__(64) void sched_clear_kernel(int32_t* __restrict__ sched) {
  if (threadIdx.x == 0) sched[0] = 0;
}

template <bool kGateUp, bool kPacked, bool kSave = false, bool kGather = false>
int launch_stream(const void* A, const int32_t* tiles, int64_t capacity, const void* const* W0, const void* const* W1,
                  const void* row_w, int64_t K, int64_t N, void* C, hipStream_t s, void* S0 = nullptr,
                  void* S1 = nullptr, const int32_t* row_src = nullptr, const GemmWorkspace& ws = {}) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  using Cfg = StreamCfg<kGateUp>;
  const int64_t n_tiles_n = ceil_div(N, kGateUp ? Cfg::BN / 2 : Cfg::BN);  // the last may be partial
  int64_t grid = 0;
  if (int rc = persistent_grid(capacity, n_tiles_n, &grid)) return rc;
  // run-time claims need the scheduling block and long tiles; the down
  // GEMMs' tail is split when its tiles are long and the partial sums hold a
  // unit per workgroup
  const int64_t ksteps = K / kBK;
  const bool have_ws = ws.base != nullptr && ws.bytes >= kSchedBytes && grid <= kMaxSchedGroups;
  int32_t* sched = (have_ws && ksteps >= kDynamicMinSteps) ? static_cast<int32_t*>(ws.base) : nullptr;
  float* part = (!kGateUp && have_ws && ksteps >= kSplitMinTileSteps &&
                 ws.bytes >= kSchedBytes + grid * (int64_t)sizeof(float) * kSplitUnitFloats)
                    ? reinterpret_cast<float*>(static_cast<char*>(ws.base) + kSchedBytes)
                    : nullptr;
  if (sched != nullptr) {
    hipLaunchKernelGGL(sched_clear_kernel, dim3(1), dim3(64), 0, s, sched);
    if (int rc = check_launch("sched_clear_kernel")) return rc;
  }
  hipLaunchKernelGGL((gemm_stream_kernel<kGateUp, kPacked, kSave, kGather>), dim3((unsigned)grid),
                     dim3(Cfg::THREADS), 0, s, static_cast<const bf16_t*>(A), tiles, W0, W1,
                     static_cast<const bf16_t*>(row_w), (int)K, (int)N, (int)n_tiles_n, (int)capacity,
                     static_cast<bf16_t*>(C), static_cast<bf16_t*>(S0), static_cast<bf16_t*>(S1), row_src, part,
                     sched);
  if (int rc = check_launch(kGateUp ? "gemm_stream_kernel<gate_up>" : "gemm_stream_kernel<down>")) return rc;
  if (part == nullptr) return ASTRAI_MOE_OK;
  // whether the tail was split is decided on the device (the live tile count
  // is there): at most G / 2 tail tiles, one workgroup each
  hipLaunchKernelGGL((split_reduce_kernel<kGateUp, kSave>), dim3((unsigned)((grid + 1) / 2), Cfg::MW), dim3(64), 0, s,
                     part, tiles, (int)capacity, (int)n_tiles_n, (int)K, (int)grid,
                     static_cast<const bf16_t*>(row_w), static_cast<bf16_t*>(C), (int)N, static_cast<bf16_t*>(S0));
  return check_launch("split_reduce_kernel");
}

template <typename Cfg, bool kGateUp, bool kPacked, bool kGather = false>
int launch(const void* A, const int32_t* tiles, int64_t capacity, const void* const* W0, const void* const* W1,
           const void* row_w, int64_t K, int64_t N, void* C, hipStream_t s, const int32_t* row_src = nullptr) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  const int64_t n_tiles_n = ceil_div(N, kGateUp ? Cfg::BN / 2 : Cfg::BN);  // the last may be partial
  int64_t grid = 0;
  if (int rc = persistent_grid(capacity, n_tiles_n, &grid)) return rc;
  hipLaunchKernelGGL((gemm_mfma_kernel<Cfg, kGateUp, kPacked, kGather>), dim3((unsigned)grid), dim3(Cfg::THREADS),
                     0, s, static_cast<const bf16_t*>(A), tiles, W0, W1, static_cast<const bf16_t*>(row_w), (int)K,
                     (int)N, (int)n_tiles_n, (int)capacity, static_cast<bf16_t*>(C), row_src);
  return check_launch(kGateUp ? "gemm_mfma_kernel<gate_up>" : "gemm_mfma_kernel<down>");
}

template <bool kPacked>
int gate_up_dispatch(const void* x_perm, const int32_t* tiles, int64_t capacity, const void* const* w_gate,
                     const void* const* w_up, int64_t dim, int64_t dim_ffn, int block_m, void* h, hipStream_t s,
                     const GemmWorkspace& ws) {
  if (block_m == kMfmaBigBM)
    return launch_stream<true, kPacked>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s, nullptr,
                                        nullptr, nullptr, ws);
  if (block_m == kMfmaMidBM)
    return launch<MidCfg, true, kPacked>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s);
  if (block_m == kMfmaMid2BM)
    return launch<Mid2Cfg, true, kPacked>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s);
  return launch<SmallCfg, true, kPacked>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s);
}

template <bool kPacked>
int down_dispatch(const void* h, const int32_t* tiles, int64_t capacity, const void* const* w_down,
                  const void* sorted_w, int64_t dim_ffn, int64_t dim, int block_m, void* y, hipStream_t s,
                  const GemmWorkspace& ws) {
  if (block_m == kMfmaBigBM)
    return launch_stream<false, kPacked>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s, nullptr,
                                         nullptr, nullptr, ws);
  if (block_m == kMfmaMidBM)
    return launch<MidCfg, false, kPacked>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s);
  if (block_m == kMfmaMid2BM)
    return launch<Mid2Cfg, false, kPacked>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s);
  return launch<SmallCfg, false, kPacked>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s);
}

}  // namespace

// K a multiple of the 64-K step; output columns a multiple of 8 (16-byte
// stores; the last column tile may be partial). 32-bit DMA offsets: a tile
// spans at most 256 rows of K * 2 bytes.
bool mfma_gate_up_supported(int64_t dim, int64_t dim_ffn, int block_m, const void* a, const void* c) {
  return (block_m == kMfmaBigBM || block_m == kMfmaMid2BM || block_m == kMfmaMidBM || block_m == kMfmaSmallBM) &&
         dim > 0 && dim_ffn > 0 && dim % kBK == 0 && dim_ffn % 8 == 0 && dim <= (1ll << 22) &&
         dim_ffn <= (1ll << 22) && aligned16(a) && aligned16(c);
}

bool mfma_down_supported(int64_t dim_ffn, int64_t dim, int block_m, const void* a, const void* c) {
  return (block_m == kMfmaBigBM || block_m == kMfmaMid2BM || block_m == kMfmaMidBM || block_m == kMfmaSmallBM) &&
         dim > 0 && dim_ffn > 0 && dim_ffn % kBK == 0 && dim % 8 == 0 && dim <= (1ll << 22) &&
         dim_ffn <= (1ll << 22) && aligned16(a) && aligned16(c);
}

int launch_mfma_gate_up(const void* x_perm, const int32_t* tiles, int64_t capacity, const void* const* w_gate,
                        const void* const* w_up, int64_t dim, int64_t dim_ffn, int block_m, bool packed, void* h,
                        hipStream_t s, const GemmWorkspace& ws) {
  return packed ? gate_up_dispatch<true>(x_perm, tiles, capacity, w_gate, w_gate, dim, dim_ffn, block_m, h, s, ws)
                : gate_up_dispatch<false>(x_perm, tiles, capacity, w_gate, w_up, dim, dim_ffn, block_m, h, s, ws);
}

int launch_mfma_down(const void* h, const int32_t* tiles, int64_t capacity, const void* const* w_down,
                     const void* sorted_w, int64_t dim_ffn, int64_t dim, int block_m, bool packed, void* y,
                     hipStream_t s, const GemmWorkspace& ws) {
  return packed ? down_dispatch<true>(h, tiles, capacity, w_down, sorted_w, dim_ffn, dim, block_m, y, s, ws)
                : down_dispatch<false>(h, tiles, capacity, w_down, sorted_w, dim_ffn, dim, block_m, y, s, ws);
}

int64_t gemm_workspace_bytes(bool down) {
  return kSchedBytes + (down ? (int64_t)cu_count() * (int64_t)sizeof(float) * kSplitUnitFloats : 0);
}

int launch_mfma_gate_up_save(const void* x_perm, const int32_t* tiles, int64_t capacity, const void* const* w_gate,
                             const void* const* w_up, int64_t dim, int64_t dim_ffn, void* h, void* gu,
                             hipStream_t s, const GemmWorkspace& ws) {
  return launch_stream<true, false, true>(x_perm, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s, gu,
                                          nullptr, nullptr, ws);
}

int launch_mfma_down_save(const void* h, const int32_t* tiles, int64_t capacity, const void* const* w_down,
                          const void* sorted_w, int64_t dim_ffn, int64_t dim, void* y, void* y_unweighted,
                          hipStream_t s, const GemmWorkspace& ws) {
  return launch_stream<false, false, true>(h, tiles, capacity, w_down, nullptr, sorted_w, dim_ffn, dim, y, s,
                                           y_unweighted, nullptr, nullptr, ws);
}

int launch_mfma_gate_up_gather(const void* x, const int32_t* sorted_token, const int32_t* tiles, int64_t capacity,
                               const void* const* w_gate, const void* const* w_up, int64_t dim, int64_t dim_ffn,
                               int block_m, void* h, hipStream_t s, const GemmWorkspace& ws) {
  if (block_m == kMfmaBigBM)
    return launch_stream<true, false, false, true>(x, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s,
                                                   nullptr, nullptr, sorted_token, ws);
  if (block_m == kMfmaMidBM)
    return launch<MidCfg, true, false, true>(x, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s,
                                             sorted_token);
  if (block_m == kMfmaMid2BM)
    return launch<Mid2Cfg, true, false, true>(x, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s,
                                              sorted_token);
  return launch<SmallCfg, true, false, true>(x, tiles, capacity, w_gate, w_up, nullptr, dim, dim_ffn, h, s,
                                             sorted_token);
}

int launch_pack(const void* w0, const void* w1, int64_t rows, int64_t k, bool gate_up, void* out, hipStream_t s) {
  // rows: output rows of the projection (dim_ffn for gate/up, each; dim for down)
  const int64_t n_tiles = gate_up ? rows / 128 : rows / 256;
  const int64_t units = n_tiles * (k / kBK) * 256 * 8;
  if (units == 0) return ASTRAI_MOE_OK;
  const int64_t grid = std::min<int64_t>(ceil_div(units, 256), 65536);
  if (gate_up)
    hipLaunchKernelGGL((pack_kernel<true>), dim3((unsigned)grid), dim3(256), 0, s, static_cast<const bf16_t*>(w0),
                       static_cast<const bf16_t*>(w1), n_tiles, (int)k, static_cast<uint4*>(out));
  else
    hipLaunchKernelGGL((pack_kernel<false>), dim3((unsigned)grid), dim3(256), 0, s, static_cast<const bf16_t*>(w0),
                       static_cast<const bf16_t*>(w0), n_tiles, (int)k, static_cast<uint4*>(out));
  return check_launch(gate_up ? "pack_kernel<gate_up>" : "pack_kernel<down>");
}

}  // namespace astrai_moe
