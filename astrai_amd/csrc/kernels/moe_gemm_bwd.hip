// Backward of the routed experts on CDNA4 matrix cores (gfx950): the grouped
// input-gradient (dgrad) and weight-gradient (wgrad) GEMMs of the SwiGLU
// experts, and the per-row gradient of the weighted combine.
//
// The reference layer is plain torch (astrai/model/components/mlp.py:22-25,
// 89-98) and autograd differentiates it op by op; per expert e with rows R_e:
//   dy   = dout[tok] * w                       (row_grad_kernel, also dw)
//   dh   = dy . W_down                         [R_e, F]  dgrad, W_down [D, F]
//   du   = dh * silu(g),  dg = silu'(g) * (dh * u)         (dgrad epilogue)
//   dx   = bf16(dg . W_gate) + bf16(du . W_up) [R_e, D]  two dgrad launches,
//          the second adding the first's result in its epilogue (autograd
//          rounds each linear's input gradient, then their sum)
//   dW_down = dy^T . h,  dW_gate = dg^T . x,  dW_up = du^T . x   (wgrad)
// with g, u the bf16 gate / up projections (saved interleaved, 4 columns of g
// then the same 4 of u) and h = u * silu(g) saved by the training forward.
//
// Operand layouts. The forward kernels read both operands K-contiguous. Here
// the dgrad weight operand (W_down [K = D, N = F], W_gate/W_up [K = F, N = D])
// and both wgrad operands ([K = rows, M or N]) are MN-contiguous: a stage
// holds 64 K-rows of 256 columns (512 bytes each), copied as they lie by the
// LDS DMA, and the fragments are read with ds_read_b64_tr_b16. That
// instruction works on groups of 16 lanes: source lane 4 i + q reads 4
// consecutive 16-bit values, and lane 4 q' + c of the group receives value c
// of source lanes q', 4 + q', 8 + q', 12 + q'. When lane 4 i + q of group g
// reads K-row 8 g + 4 h + i at columns 16 s + 4 q, lane j of group g receives
// K = 8 g + 4 h + 0..3 of column 16 s + j: two such reads (h = 0, 1) give
// exactly the per-lane layout of a v_mfma_f32_16x16x32_bf16 operand (index
// l % 16, K 8 (l / 16) .. + 7).
//
// MN-major swizzle: the 32-byte segment s of K-row k is stored at segment
// s ^ z(k) of its 256-byte half, z(k) = (k & 3) | ((k >> 3) & 1) << 2. The
// 32 lanes of one half-wave read rows {0..3, 8..11} + const of one segment;
// z maps them to 8 distinct 32-byte bank groups. Since z(k) depends only on
// the lane here (bits 2 and 4+ of k come from the K half and the read), a
// fragment's address is the lane's base xor (segment << 5).
//
// Schedule: the prefill kernel's (moe_gemm_mfma.hip): persistent, one
// workgroup per CU, 256 x 256 output tiles, 8 matrix-core waves of 128 x 64
// and 4 LDS-DMA waves, activations in 2 stages and the second operand in 3,
// one barrier per 64-K step, the next step's first fragments prefetched
// across tile boundaries. dgrad walks the forward's 256-row tile list; wgrad
// walks (expert, M tile, N tile) with K = the expert's rows, rows past the
// expert's end read from a zero row. Given a workspace, the dgrad_in GEMMs
// split a partial last round along K: a second launch of the same kernel
// (kTail) runs the slices into fp32 partial tiles, and
// bwd_split_reduce_kernel adds each tile's slices in order and runs its
// epilogue.
#include "mfma_tile.h"

#include <type_traits>

namespace astrai_moe {
namespace {

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));

enum class Bwd { kDgradDown, kDgradIn, kDgradInAdd, kWgrad };

// Source of K-rows past an expert's last row in wgrad (zero contribution).
__device__ __attribute__((aligned(512))) uint4 g_zero_row[32] = {};

struct BwdArgs {
  const bf16_t* a0;          // A: dy / dg / du (dgrad, K-major [rows, K]); wgrad: A [rows, M]
  const void* const* w0;     // dgrad: weight table (W_down / W_gate / W_up, each [K, N])
  const bf16_t* b_act;       // wgrad: B [rows, N]
  const int32_t* tiles;      // dgrad: 256-row tile list
  const int32_t* offsets;    // wgrad: expert row offsets [E + 1]
  const bf16_t* e0;          // dgrad down epilogue: gu [rows, 2 N]; dgrad in: addend or null
  bf16_t* c0;                // dgrad down: dg; dgrad in: dx; wgrad: dW [E, M, N]
  bf16_t* c1;                // dgrad down: du
  int K;                     // dgrad: K
  int M, N;                  // wgrad: M x N per expert; dgrad: N
  int n_tiles_m, n_tiles_n;  // column tiles (dgrad), M / N tiles (wgrad)
  int capacity;              // dgrad: tile-list capacity
  int n_experts;             // wgrad
  float* part;               // dgrad: partial sums of the split last round (null: the tail runs whole)
  int grid;                  // workgroups of the GEMM launch (the split reduce recomputes its walk)
};

struct BwdCfg {
  static constexpr int BM = 256, BN = 256, GM = 8;
  static constexpr int WGM = 2, WGN = 4, MW = 8, DW = 4;
  static constexpr int WAVES = MW + DW, THREADS = WAVES * 64;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int A_BYTES = 32768, B_BYTES = 32768;
  static constexpr int A_STAGES = 2, B_STAGES = 3;
  static constexpr int A_OFF = 0, B_OFF = A_STAGES * A_BYTES;
  static constexpr int LDS = B_OFF + B_STAGES * B_BYTES;  // 160 KB
  static constexpr int OPS = A_BYTES / 1024 / DW;         // 8 DMA ops per DMA wave per operand and step
  static constexpr int RG = 2, AR = 4, PD = 2;
  static constexpr int MN_ROW = 512;                       // bytes of one MN-major K-row (256 columns)
  static_assert(BM * 64 * 2 == A_BYTES && BN * 64 * 2 == B_BYTES, "64-K stages");
  static_assert(LDS <= 160 * 1024, "LDS");
  static_assert(3 * OPS <= 63, "vmcnt range");
  static_assert(16 % AR == 0 && 8 % RG == 0 && PD >= RG && PD + RG <= AR, "ring slots of a pair and its prefetch");
};

// A work item: tile (mt, nt) of expert e, K steps [k0, ksteps); unit >= 0:
// a slice of a split tail tile whose fp32 accumulators go to part[unit].
struct TileInfo {
  int e, mt, nt, row0, rows, k0, ksteps, unit;
};

// dgrad: the forward's tile walk over (row tile, column tile), K fixed.
// kSplit (dgrad_in): with a partial-sum buffer the last round's tiles are
// split along K as in the forward down GEMM (SplitWalk). The GEMM launch then
// walks the whole tiles (items [0, full)) and a second launch of the same
// grid the split slices (items [full, items()), at most one per workgroup),
// so that neither kernel carries both epilogues (the branch between them
// spilled the SwiGLU-backward epilogue's registers). dgrad_down keeps the
// plain walk: at the register limit already, the split walk's state cost it
// 2.5 % (same-process A/B) where its split tail gained 1 %.
template <bool kSplit>
struct RowTileWalk {
  static constexpr bool kSplitK = kSplit;  // items may start past K step 0
  std::conditional_t<kSplit, SplitWalk<BwdCfg::GM>, TileWalk<BwdCfg::GM>> w;
  const int32_t* tiles;
  int ksteps, G, begin, total;
  __device__ RowTileWalk(const BwdArgs& p, bool tail) : w(make_walk(p)), tiles(p.tiles), ksteps(p.K / kBK), G(w.G) {
    if constexpr (kSplit) {
      begin = tail ? w.full : 0;
      total = tail ? w.items() : w.full;
    } else {
      begin = 0;
      total = w.total;
    }
  }
  __device__ static decltype(w) make_walk(const BwdArgs& p) {
    if constexpr (kSplit)
      return SplitWalk<BwdCfg::GM>(p.tiles, p.capacity, p.n_tiles_n, p.K / kBK, p.part != nullptr, p.grid);
    else
      return TileWalk<BwdCfg::GM>(p.tiles, p.capacity, p.n_tiles_n);
  }
  __device__ int first_slot() const { return begin + w.first_slot(); }
  __device__ int seek(int logical, TileInfo& t) const {
    if (logical < total) {
      if constexpr (kSplit) {
        w.item(logical, t.mt, t.nt, t.k0, t.ksteps, t.unit);
      } else {
        w.decode(logical, t.mt, t.nt);
        t.k0 = 0, t.ksteps = ksteps, t.unit = -1;
      }
      const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)uniform(t.mt) * ASTRAI_MOE_TILE_STRIDE;
      t.e = load_scalar(ti);
      t.row0 = load_scalar(ti + 1);
      t.rows = min(BwdCfg::BM, load_scalar(ti + 2) - t.row0);
    }
    return logical;
  }
};

// wgrad: (expert, M tile, N tile), GM M tiles walked per N tile; experts
// without rows are skipped; K = the expert's rows in steps of 64.
struct ExpertWalk {
  static constexpr bool kSplitK = false;
  const int32_t* off;
  int MT, NT, per_e, G, total;
  __device__ ExpertWalk(const BwdArgs& p, bool)
      : off(p.offsets), MT(p.n_tiles_m), NT(p.n_tiles_n), per_e(p.n_tiles_m * p.n_tiles_n), G((int)gridDim.x),
        total(p.n_experts * p.n_tiles_m * p.n_tiles_n) {}
  __device__ int first_slot() const {
    const int bid = blockIdx.x;
    return (G % kXcds == 0) ? (bid % kXcds) * (G / kXcds) + bid / kXcds : bid;
  }
  __device__ bool decode(int logical, TileInfo& t) const {
    t.e = logical / per_e;
    const int r = logical - t.e * per_e;
    const int first_m = (r / (BwdCfg::GM * NT)) * BwdCfg::GM;
    const int gm = min(BwdCfg::GM, MT - first_m);
    const int in_group = r - first_m * NT;
    t.mt = first_m + in_group % gm;
    t.nt = in_group / gm;
    t.row0 = load_scalar(off + t.e);
    t.rows = load_scalar(off + t.e + 1) - t.row0;
    t.k0 = 0;
    t.ksteps = (t.rows + kBK - 1) / kBK;
    t.unit = -1;
    return t.rows > 0;
  }
  __device__ int seek(int logical, TileInfo& t) const {
    while (logical < total && !decode(logical, t)) logical += G;
    return logical;
  }
};

__device__ __forceinline__ int mn_swz(int k) { return (k & 3) | (((k >> 3) & 1) << 2); }

// Byte offset, within a 512-byte MN-major K-row, of what DMA lane `lane` of
// op q stores: the op fills K-rows 2 q and 2 q + 1; slot p = lane & 31 holds
// half (p & 1) of segment (p >> 1) ^ z(k).
__device__ __forceinline__ uint32_t mn_src_col(int q, int lane) {
  const int kr = 2 * q + (lane >> 5);
  const int p = lane & 31;
  return (uint32_t)((((p >> 1) ^ mn_swz(kr)) << 5) | ((p & 1) << 4));
}

// One DMA op of an MN-major stage: K-rows krow0 + 2 q + {0, 1} of `base`
// (rows at or past `valid_rows` read the zero row), columns from byte col0,
// clamped to the last 16 bytes before col_end (those columns are masked in
// the epilogue).
__device__ __forceinline__ void dma_mn(const char* base, int krow0, int valid_rows, uint32_t pitch, uint32_t col0,
                                       uint32_t col_end, int lane, int q, char* lds) {
  const int row = krow0 + 2 * q + (lane >> 5);
  const uint32_t col = min(col0 + mn_src_col(q, lane), col_end - 16u);
  const char* src = row < valid_rows ? base + (int64_t)row * pitch + col
                                     : reinterpret_cast<const char*>(g_zero_row) + (col & 511u);
  lds_dma_16(src, lds);
}

// A DMA wave's ops of one MN-major stage: groups q = dw * OPS + i. Lane
// offset i of a tile, (2 i + lane / 32) * pitch + the lane's clamped column,
// depends only on i (the swizzle z of K-row 2 q + lane / 32 does, OPS = 8),
// so a step whose 64 K-rows all lie before valid_rows issues each op as a
// uniform step base plus that 32-bit offset. Only an expert's last, partial
// step takes the per-lane zero-row select.
struct MnLanes {
  uint32_t off[BwdCfg::OPS];
  __device__ void setup(uint32_t pitch, uint32_t col0, uint32_t col_end, int lane) {
#pragma unroll
    for (int i = 0; i < BwdCfg::OPS; ++i)
      off[i] = (uint32_t)(2 * i + (lane >> 5)) * pitch + min(col0 + mn_src_col(i, lane), col_end - 16u);
  }
};
static_assert(BwdCfg::OPS == 8, "MN-major lane offsets repeat every 8 ops");

__device__ __forceinline__ void dma_mn_step(const char* base, int krow0, int valid_rows, uint32_t pitch,
                                            uint32_t col0, uint32_t col_end, const MnLanes& ml, int lane, int dw,
                                            char* stage) {
  constexpr int OPS = BwdCfg::OPS;
  if (krow0 + kBK <= valid_rows) {
    const char* sb = uniform(base + (int64_t)(krow0 + 2 * OPS * dw) * pitch);
#pragma unroll
    for (int i = 0; i < OPS; ++i) lds_dma_16(sb + ml.off[i], stage + (dw * OPS + i) * 1024);
  } else {
#pragma unroll
    for (int i = 0; i < OPS; ++i)
      dma_mn(base, krow0, valid_rows, pitch, col0, col_end, lane, dw * OPS + i, stage + (dw * OPS + i) * 1024);
  }
}

// Per-tile global bases of both operands.
template <Bwd kMode>
struct BwdSrc {
  const char* a0 = nullptr;
  const char* b0 = nullptr;
  int rows = 0;
  uint32_t a_col0 = 0, b_col0 = 0;
  MnLanes a_mn, b_mn;  // a_mn: wgrad only
  __device__ void setup(const BwdArgs& p, const TileInfo& t, int lane) {
    rows = t.rows;
    if constexpr (kMode == Bwd::kWgrad) {
      a0 = uniform(reinterpret_cast<const char*>(p.a0 + (int64_t)t.row0 * p.M));
      b0 = uniform(reinterpret_cast<const char*>(p.b_act + (int64_t)t.row0 * p.N));
      a_col0 = (uint32_t)t.mt * BwdCfg::MN_ROW;
      b_col0 = (uint32_t)t.nt * BwdCfg::MN_ROW;
      a_mn.setup((uint32_t)p.M * 2u, a_col0, (uint32_t)p.M * 2u, lane);
    } else {
      a0 = uniform(reinterpret_cast<const char*>(p.a0 + (int64_t)t.row0 * p.K));
      b0 = static_cast<const char*>(load_scalar(p.w0 + t.e));
      b_col0 = (uint32_t)t.nt * BwdCfg::MN_ROW;
    }
    b_mn.setup((uint32_t)p.N * 2u, b_col0, (uint32_t)p.N * 2u, lane);
  }
  // This DMA wave's share (groups dw * OPS ..) of step kstep's A stage: 8-row
  // groups (dgrad, K-major) or 2-K-row groups (wgrad, MN-major).
  __device__ void dma_a(const BwdArgs& p, int lane, int kstep, int dw, char* stage) const {
    if constexpr (kMode == Bwd::kWgrad) {
      dma_mn_step(a0, kstep * kBK, rows, (uint32_t)p.M * 2u, a_col0, (uint32_t)p.M * 2u, a_mn, lane, dw, stage);
    } else {
      const DmaLane dl(lane, kstep);
#pragma unroll
      for (int i = 0; i < BwdCfg::OPS; ++i) {
        const int q = dw * BwdCfg::OPS + i;
        const uint32_t row = (uint32_t)min(q * 8 + dl.row, rows - 1);
        lds_dma_16(a0 + (row * ((uint32_t)p.K * 2u) + dl.chunk(q)), stage + q * 1024);
      }
    }
  }
  // This DMA wave's share of step kstep's B stage (MN-major in every mode;
  // dgrad's weights have no rows to zero).
  __device__ void dma_b(const BwdArgs& p, int lane, int kstep, int dw, char* stage) const {
    const int valid = kMode == Bwd::kWgrad ? rows : 0x7fffffff;
    dma_mn_step(b0, kstep * kBK, valid, (uint32_t)p.N * 2u, b_col0, (uint32_t)p.N * 2u, b_mn, lane, dw, stage);
  }
};

template <Bwd kMode, typename Walk>
struct BwdCursor {
  int logical, kt;
  bool live;
  TileInfo t;
  BwdSrc<kMode> src;
  __device__ void start(const BwdArgs& p, int logical_, const TileInfo& t_, int lane) {
    logical = logical_, t = t_, kt = Walk::kSplitK ? t.k0 : 0, live = true;
    src.setup(p, t, lane);
  }
  __device__ void advance(const BwdArgs& p, const Walk& walk, int lane) {
    if (++kt == t.ksteps) {
      logical = walk.seek(logical + walk.G, t);
      live = logical < walk.total;
      if (live) kt = Walk::kSplitK ? t.k0 : 0, src.setup(p, t, lane);
    }
  }
};

__device__ __forceinline__ bf16x8_t lds_tr_pair(const char* smem, uint32_t addr) {
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(smem + addr));
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(smem + addr + 2048));
  const s16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ float sigmoid_f(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

// Epilogue of the plain GEMMs (dgrad_in, wgrad) from the accumulators (lane:
// row 16 i + l % 16, columns 16 j + 4 (l / 16) .. + 3 of the wave's block).
// The accumulators are rounded to bf16 and, per pair of 16-column tiles, go
// through the lane-group transpose, which leaves each lane 8 consecutive
// columns of its row, stored as one 16-byte piece. N is a multiple of 8, so a
// lane's 8 columns are wholly inside the matrix or wholly past its edge.
template <Bwd kMode>
__device__ __forceinline__ void bwd_epilogue(f32x4_t (&acc)[BwdCfg::WM / 16][BwdCfg::WN / 16], const BwdArgs& p,
                                             const TileInfo& t, int wm, int wn) {
  static_assert(kMode == Bwd::kDgradIn || kMode == Bwd::kWgrad, "no elementwise input");
  constexpr int MT16 = BwdCfg::WM / 16, NT16 = BwdCfg::WN / 16;
  static_assert(NT16 % 2 == 0, "tiles are transposed in pairs");
  const int el = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int row_l = el & 15;
  const int q = el >> 4;
  const int nw = t.nt * BwdCfg::BN + wn * BwdCfg::WN;  // the wave's first column
#pragma unroll
  for (int i = 0; i < MT16; ++i) {
    const int gm = wm * BwdCfg::WM + i * 16 + row_l;
    int64_t row_off;
    bool row_ok;
    if constexpr (kMode == Bwd::kWgrad) {
      const int m = t.mt * BwdCfg::BM + gm;
      row_ok = m < p.M;
      row_off = ((int64_t)t.e * p.M + min(m, p.M - 1)) * p.N;
    } else {
      row_ok = gm < t.rows;
      row_off = (int64_t)(t.row0 + min(gm, t.rows - 1)) * p.N;
    }
#pragma unroll
    for (int jp = 0; jp < NT16; jp += 2) {
      bf16x4_t e[2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) e[h][r] = (__bf16)acc[i][jp + h][r];
      transpose2(e);
      const int nn = nw + jp * 16 + 8 * q;  // the lane's 8 columns after the transpose
      if (!row_ok || nn >= p.N) continue;
      const int64_t off = row_off + nn;
      bf16x8_t o0;
#pragma unroll
      for (int c = 0; c < 8; ++c) o0[c] = e[c >> 2][c & 3];
      *reinterpret_cast<bf16x8_t*>(p.c0 + off) = o0;
    }
  }
}

// The epilogues that read an elementwise input (dgrad_down: gu; dgrad_in_add:
// the first projection's input gradient), with those loads PF row blocks
// ahead of the stores. The vector-memory counter retires loads and stores in
// issue order, so a load issued after a row block's stores cannot be consumed
// before those stores complete; here the accumulators are first rounded and
// transposed to bf16 (half their registers), then each refill of the input
// ring is issued before the stores of the row block it follows. Same rounding
// points and element order as bwd_epilogue.
template <Bwd kMode, int PF>
__device__ __forceinline__ void bwd_epilogue_pf(f32x4_t (&acc)[BwdCfg::WM / 16][BwdCfg::WN / 16], const BwdArgs& p,
                                                const TileInfo& t, int wm, int wn) {
  static_assert(kMode == Bwd::kDgradDown || kMode == Bwd::kDgradInAdd, "epilogues with an elementwise input");
  constexpr bool kSwiGlu = kMode == Bwd::kDgradDown;
  constexpr int MT16 = BwdCfg::WM / 16, NT16 = BwdCfg::WN / 16, NJ = NT16 / 2;
  constexpr int NL = kSwiGlu ? 2 : 1;  // 16-byte input loads per lane and column pair
  static_assert(NT16 % 2 == 0 && PF <= MT16, "column pairs; ring depth");
  const int el = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int row_l = el & 15;
  const int q = el >> 4;
  const int nw = t.nt * BwdCfg::BN + wn * BwdCfg::WN;
  bf16x8_t dh[MT16][NJ];  // lane: 8 consecutive columns of row block i, column pair j
#pragma unroll
  for (int i = 0; i < MT16; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      bf16x4_t e[2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) e[h][r] = (__bf16)acc[i][2 * j + h][r];
      transpose2(e);
#pragma unroll
      for (int r = 0; r < 4; ++r) dh[i][j][r] = e[0][r], dh[i][j][4 + r] = e[1][r];
    }
  // element offset of the lane's 8 columns in row block i, column pair j (clamped
  // inside the matrix for the loads; `ok`: the lane stores them)
  auto offset = [&](int i, int j, bool& ok) -> int64_t {
    const int gm = wm * BwdCfg::WM + i * 16 + row_l;
    const int nn = nw + j * 32 + 8 * q;
    ok = gm < t.rows && nn < p.N;
    return (int64_t)(t.row0 + min(gm, t.rows - 1)) * p.N + min(nn, p.N - 8);
  };
  bf16x8_t in[PF][NJ][NL];
  auto load = [&](int i, int slot) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      bool ok;
      const int64_t off = offset(i, j, ok);
#pragma unroll
      for (int l = 0; l < NL; ++l)
        in[slot][j][l] = *reinterpret_cast<const bf16x8_t*>(p.e0 + (kSwiGlu ? 2 * off + 8 * l : off));
    }
  };
#pragma unroll
  for (int b = 0; b < PF; ++b) load(b, b);
#pragma unroll
  for (int i = 0; i < MT16; ++i) {
    const int slot = i % PF;
    bf16x8_t o0[NJ], o1[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float d = (float)dh[i][j][c];
        if constexpr (kSwiGlu) {
          // gu keeps g[c..c+3], u[c..c+3] at 2 c: the lane's 8 columns are two 16-byte loads
          const bf16x8_t& gu = in[slot][j][c >> 2];
          const float g = (float)gu[c & 3];
          const float u = (float)gu[4 + (c & 3)];
          const float s = sigmoid_f(g);
          const float act = (float)(__bf16)(g * s);  // silu(g) as the forward rounded it
          o1[j][c] = (__bf16)(d * act);               // du
          const float dact = (float)(__bf16)(d * u);
          o0[j][c] = (__bf16)(dact * (s * (1.0f + g * (1.0f - s))));  // dg
        } else {
          o0[j][c] = (__bf16)(d + (float)in[slot][j][0][c]);
        }
      }
    }
    if (i + PF < MT16) load(i + PF, slot);  // before this row block's stores
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      bool ok;
      const int64_t off = offset(i, j, ok);
      if (ok) {
        if constexpr (kSwiGlu) *reinterpret_cast<bf16x8_t*>(p.c1 + off) = o1[j];
        *reinterpret_cast<bf16x8_t*>(p.c0 + off) = o0[j];
      }
    }
  }
}

template <Bwd kMode>
__device__ __forceinline__ void bwd_epilogue_any(f32x4_t (&acc)[BwdCfg::WM / 16][BwdCfg::WN / 16], const BwdArgs& p,
                                                 const TileInfo& t, int wm, int wn) {
  // input rings two (gu, 32 bytes per lane and column pair) and four row
  // blocks deep: deeper rings spilled
  if constexpr (kMode == Bwd::kDgradDown)
    bwd_epilogue_pf<kMode, 2>(acc, p, t, wm, wn);
  else if constexpr (kMode == Bwd::kDgradInAdd)
    bwd_epilogue_pf<kMode, 4>(acc, p, t, wm, wn);
  else
    bwd_epilogue<kMode>(acc, p, t, wm, wn);
}

// The epilogue of a dgrad GEMM's split tail tiles: workgroup u sums the S
// partials of tail tile u in slice order (wave w those of matrix-core wave w)
// and runs the tile's epilogue. The walk is recomputed from the same tile
// list and the GEMM launch's grid, so both kernels agree on the split.
template <Bwd kMode>
__global__ __launch_bounds__(64) void bwd_split_reduce_kernel(const BwdArgs p) {
  static_assert(kMode == Bwd::kDgradIn || kMode == Bwd::kDgradInAdd, "only dgrad_in splits its tail");
  const RowTileWalk<true> walk(p, true);
  const int u = blockIdx.x;
  if (walk.w.S < 2 || u >= walk.w.total - walk.w.full) return;
  TileInfo t;
  walk.seek(walk.w.full + u * walk.w.S, t);  // the tile's first slice
  const int wave = blockIdx.y, lane = threadIdx.x;  // one wave per (tile, matrix-core wave)
  constexpr int MT16 = BwdCfg::WM / 16, NT16 = BwdCfg::WN / 16;
  constexpr int kUnitVecs = kSplitUnitFloats / 4;
  const f32x4_t* pp = reinterpret_cast<const f32x4_t*>(p.part) + (int64_t)u * walk.w.S * kUnitVecs +
                      wave * (MT16 * NT16 * 64) + lane;
  f32x4_t acc[MT16][NT16];
#pragma unroll
  for (int i = 0; i < MT16; ++i)
#pragma unroll
    for (int j = 0; j < NT16; ++j) acc[i][j] = pp[(i * NT16 + j) * 64];
  for (int sl = 1; sl < walk.w.S; ++sl) {
    const f32x4_t* ps = pp + (int64_t)sl * kUnitVecs;
#pragma unroll
    for (int i = 0; i < MT16; ++i)
#pragma unroll
      for (int j = 0; j < NT16; ++j) acc[i][j] += ps[(i * NT16 + j) * 64];
  }
  bwd_epilogue_any<kMode>(acc, p, t, wave / BwdCfg::WGN, wave % BwdCfg::WGN);
}

// kTail: the split slices of the last round (RowTileWalk), stored as fp32
// partial sums for bwd_split_reduce_kernel; otherwise every whole tile.
template <Bwd kMode, bool kTail = false, typename Cfg = BwdCfg>
__global__ __launch_bounds__(Cfg::THREADS, 1) void gemm_bwd_kernel(const BwdArgs p) {
  constexpr bool kSplit = kMode == Bwd::kDgradIn || kMode == Bwd::kDgradInAdd;
  static_assert(!kTail || kSplit, "only dgrad_in splits its tail");
  using Walk = std::conditional_t<kMode == Bwd::kWgrad, ExpertWalk, RowTileWalk<kSplit>>;
  constexpr bool kAMn = kMode == Bwd::kWgrad;  // A operand MN-major (B always is)
  __shared__ __attribute__((aligned(1024))) char smem[Cfg::LDS];

  const Walk walk(p, kTail);
  TileInfo t;
  int logical = walk.seek(walk.first_slot(), t);
  if (logical >= walk.total) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;

  // Step protocol as in the prefill forward kernel: barrier X_g means every
  // matrix-core wave has read step g and A(g + 1), B(g + 1) have landed;
  // after it the DMA waves load A(g + 2) into A-buffer g % 2 and B(g + 3)
  // into B-buffer g % 3.
  if (wave >= Cfg::MW) {
    const int dw = wave - Cfg::MW;
    BwdCursor<kMode, Walk> ca, cb;
    ca.start(p, logical, t, lane);
    cb.start(p, logical, t, lane);
    auto issue_a = [&](int buf) {
      ca.src.dma_a(p, lane, ca.kt, dw, smem + Cfg::A_OFF + buf * Cfg::A_BYTES);
      ca.advance(p, walk, lane);
    };
    auto issue_b = [&](int buf) {
      cb.src.dma_b(p, lane, cb.kt, dw, smem + Cfg::B_OFF + buf * Cfg::B_BYTES);
      cb.advance(p, walk, lane);
    };
    int a_iss = 0, b_iss = 0;
    issue_b(0), ++b_iss;
    issue_a(0), ++a_iss;
    if (cb.live) issue_b(1), ++b_iss;
    if (ca.live) issue_a(1), ++a_iss;
    if (cb.live) issue_b(2), ++b_iss;
    wait_groups<Cfg::OPS, 3>((a_iss - 1) + (b_iss - 1));  // A0 and B0 landed
    __builtin_amdgcn_s_barrier();                          // X_{-1}
    for (int g = 0;; ++g) {
      wait_groups<Cfg::OPS, 1>(b_iss > g + 2 ? 1 : 0);
      __builtin_amdgcn_s_barrier();  // X_g
      const bool more = ca.live;
      if (ca.live) issue_a(g & 1), ++a_iss;
      if (cb.live) issue_b(g % 3), ++b_iss;
      if (!more && g + 1 >= a_iss) break;
    }
    return;
  }

  // ---------------- matrix-core waves ----------------
  const int wm = wave / Cfg::WGN;
  const int wn = wave % Cfg::WGN;
  constexpr int MT16 = Cfg::WM / 16, NT16 = Cfg::WN / 16;
  constexpr int AR = Cfg::AR, PD = Cfg::PD, RG = Cfg::RG;
  const int grp = lane >> 4;
  const int gl = lane & 15;
  // MN-major fragment bases: K-row 8 grp + (gl >> 2), bytes 8 (gl & 3) of
  // the lane's 32-byte segment, segment bits swizzled by z = z(K-row).
  const uint32_t mn_z = (uint32_t)((gl >> 2) | ((grp & 1) << 2));
  const uint32_t mn_lane = (uint32_t)(8 * grp + (gl >> 2)) * Cfg::MN_ROW + 8u * (uint32_t)(gl & 3);
  uint32_t vA, vB;
  if constexpr (kAMn) {
    vA = (uint32_t)Cfg::A_OFF + mn_lane + (uint32_t)wm * 256u + (mn_z << 5);
  } else {
    const int frag_row = lane & 15;
    const int fq = lane >> 4;
    const uint32_t v_lane = frag_row * kRowBytes + ((fq ^ ((frag_row >> 1) & 7)) << 4);
    vA = (uint32_t)Cfg::A_OFF + (uint32_t)(wm * Cfg::WM) * kRowBytes + v_lane;
  }
  vB = (uint32_t)Cfg::B_OFF + mn_lane + (uint32_t)(wn >> 1) * 256u + ((mn_z ^ (4u * (uint32_t)(wn & 1))) << 5);
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
  auto rdA = [&](uint32_t base, int kh, int i) -> bf16x8_t {
    if constexpr (kAMn) {
      return lds_tr_pair(smem, (base ^ ((uint32_t)i << 5)) + (uint32_t)kh * 32u * Cfg::MN_ROW);
    } else {
      return *reinterpret_cast<const bf16x8_t*>(smem + ((base ^ (kh ? 64u : 0u)) + i * 16 * kRowBytes));
    }
  };
  auto rdB = [&](uint32_t base, int kh, int j) -> bf16x8_t {
    return lds_tr_pair(smem, (base ^ ((uint32_t)j << 5)) + (uint32_t)kh * 32u * Cfg::MN_ROW);
  };
  auto step = [&]() {
    uint32_t nA = 0, nB = 0;
    static_for<16 / RG>([&](auto gg) {
      constexpr int r0 = decltype(gg)::value * RG;
      // Issue priority drops partway through the step, as in the forward
      // streaming GEMMs: the matrix-core wave behind on a SIMD takes the
      // matrix core, so the two reach the step barrier together. Measured in
      // one process, builds alternating, bit-identical, Mixtral shape:
      // dgrad_down +2.6 / +4.0 %, dgrad_in pair +4.0 / +4.7 %, wgrad +2.6 %
      // (fine-grained +1.8 to +3.0 %); dropping at row 8 or 12 gained less.
      if constexpr (r0 == 0) __builtin_amdgcn_s_setprio(1);
      if constexpr (r0 == 10) __builtin_amdgcn_s_setprio(0);
      if constexpr (r0 + PD >= 16 && r0 + PD < 16 + RG) {
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();  // X_g
        __builtin_amdgcn_sched_barrier(0);
        nA = vA ^ (uint32_t)Cfg::A_BYTES;
        nB = next_b(vB);
      }
      static_for<RG>([&](auto qq) {
        constexpr int rp = r0 + PD + decltype(qq)::value;
        if constexpr (rp < 16) {
          fa[rp % AR] = rdA(vA, rp / 8, rp % 8);
        } else {
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
        if constexpr (r0 + RG == 16) fb[j] = rdB(nB, 0, j);
      }
    });
  };

  lds_barrier();  // X_{-1}
#pragma unroll
  for (int j = 0; j < NT16; ++j) fb[j] = rdB(vB, 0, j);
#pragma unroll
  for (int r = 0; r < PD; ++r) fa[r % AR] = rdA(vA, 0, r);
  constexpr bool kIdleHalf = kMode == Bwd::kDgradDown;
  // first row tile where padding-only waves idle: every tile with short
  // tiles, else the tiles after the list's whole groups (as in the forward)
  const int idle_mt0 = kIdleHalf ? __builtin_amdgcn_readfirstlane(p.K / kBK < kIdleMaxSteps ? 0 : p.tiles[3]) : 0;
  while (true) {
    // dgrad_down: in an expert's last row tile of at most BM / 2 rows the
    // waves of the second half hold only padding rows; they keep the step
    // barriers and the next tile's prefetch but issue no MFMAs and store
    // nothing, as in the forward kernel (bit-identical; fine-grained shape
    // +1.9 %). In the dgrad_in pair it measured within +-1.6 %, and
    // dgrad_in_add's K loop then spilled a fragment.
    if (kIdleHalf && idle_threshold(t.mt >= idle_mt0, wm * Cfg::WM) >= t.rows) {
      for (int kt = kSplit ? t.k0 : 0; kt < t.ksteps; ++kt) {
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();  // X_g
        __builtin_amdgcn_sched_barrier(0);
        if (kt + 1 == t.ksteps) {
          const uint32_t nA = vA ^ (uint32_t)Cfg::A_BYTES, nB = next_b(vB);
#pragma unroll
          for (int j = 0; j < NT16; ++j) fb[j] = rdB(nB, 0, j);
#pragma unroll
          for (int r = 0; r < PD; ++r) fa[r % AR] = rdA(nA, 0, r);
        }
        rotate();
      }
      logical = walk.seek(logical + walk.G, t);
      if (logical >= walk.total) break;
      continue;
    }
#pragma unroll
    for (int i = 0; i < MT16; ++i)
#pragma unroll
      for (int j = 0; j < NT16; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;
    // every step, a tile's last included, prefetches the next step's first
    // fragments (the next tile's); one loop body, one register assignment
    for (int kt = kSplit ? t.k0 : 0; kt < t.ksteps; ++kt) {
      step();
      rotate();
    }
    __builtin_amdgcn_sched_barrier(0);
    // (the chain written out: through bwd_epilogue_any the compiler spilled
    // twice as much of dgrad_down)
    if constexpr (kTail)
      store_partial(acc, p.part, t.unit, wave, lane);  // the reduce runs the tile's epilogue
    else if constexpr (kMode == Bwd::kDgradDown)
      bwd_epilogue_pf<kMode, 2>(acc, p, t, wm, wn);
    else if constexpr (kMode == Bwd::kDgradInAdd)
      bwd_epilogue_pf<kMode, 4>(acc, p, t, wm, wn);
    else
      bwd_epilogue<kMode>(acc, p, t, wm, wn);
    logical = walk.seek(logical + walk.G, t);
    if (logical >= walk.total) break;
  }
}

// One wave per permuted row r (token tok = sorted_token[r], routing weight
// w): dy[r] = dout[tok] * w (bf16 product, mlp.py:97's y * w differentiated
// in y) and dw[r] = sum_d bf16(dout[tok, d] * y[r, d]) (in w), y being the
// unweighted expert output.
__global__ __launch_bounds__(256) void row_grad_kernel(const bf16_t* __restrict__ dout,
                                                       const int32_t* __restrict__ sorted_token,
                                                       const bf16_t* __restrict__ sorted_w,
                                                       const bf16_t* __restrict__ y, int64_t n_rows, int64_t dim,
                                                       bf16_t* __restrict__ dy, bf16_t* __restrict__ dw_rows) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (r >= n_rows) return;
  const int64_t tok = sorted_token[r];
  const float w = bf16_bits_to_f32(sorted_w[r]);
  const bf16x8_t* src = reinterpret_cast<const bf16x8_t*>(dout + tok * dim);
  const bf16x8_t* yr = reinterpret_cast<const bf16x8_t*>(y + r * dim);
  bf16x8_t* dst = reinterpret_cast<bf16x8_t*>(dy + r * dim);
  float acc = 0.0f;
  for (int64_t v = lane; v < dim / 8; v += 64) {
    const bf16x8_t d8 = src[v];
    const bf16x8_t y8 = yr[v];
    bf16x8_t o;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float d = (float)d8[k];
      o[k] = (__bf16)(d * w);
      acc += (float)(__bf16)(d * (float)y8[k]);
    }
    dst[v] = o;
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) acc += __shfl_xor(acc, s, 64);
  if (lane == 0) dw_rows[r] = f32_to_bf16_bits(acc);
}

// ws: the dgrad_in GEMMs' workspace (null: the last round runs whole). Its
// partial sums, one 256 KB unit per workgroup after the first kSchedBytes
// (the forward down GEMM's layout), take the split tail of tiles with at
// least kSplitMinTileSteps K steps; whether the tail is split is decided on
// the device, where the live tile count is.
template <Bwd kMode>
int launch_bwd(BwdArgs p, int64_t total, hipStream_t s, const char* name, const GemmWorkspace& ws = {}) {
  if (total == 0) return ASTRAI_MOE_OK;
  if (total >= (1ll << 31)) return fail(ASTRAI_MOE_EINVAL, "%s: %lld tiles exceed the tile-index range", name,
                                        (long long)total);
  const int64_t grid = std::min<int64_t>(total, cu_count());
  p.grid = (int)grid;
  p.part = nullptr;
  constexpr bool kSplit = kMode == Bwd::kDgradIn || kMode == Bwd::kDgradInAdd;
  if (kSplit && ws.base != nullptr && p.K / kBK >= kSplitMinTileSteps &&
      ws.bytes >= kSchedBytes + grid * (int64_t)sizeof(float) * kSplitUnitFloats)
    p.part = reinterpret_cast<float*>(static_cast<char*>(ws.base) + kSchedBytes);
  hipLaunchKernelGGL((gemm_bwd_kernel<kMode>), dim3((unsigned)grid), dim3(BwdCfg::THREADS), 0, s, p);
  if (int rc = check_launch(name)) return rc;
  if constexpr (kSplit) {
    if (p.part == nullptr) return ASTRAI_MOE_OK;
    hipLaunchKernelGGL((gemm_bwd_kernel<kMode, true>), dim3((unsigned)grid), dim3(BwdCfg::THREADS), 0, s, p);
    if (int rc = check_launch(name)) return rc;
    hipLaunchKernelGGL((bwd_split_reduce_kernel<kMode>), dim3((unsigned)((grid + 1) / 2), BwdCfg::MW), dim3(64), 0, s,
                       p);
    return check_launch("bwd_split_reduce_kernel");
  }
  return ASTRAI_MOE_OK;
}

}  // namespace

int launch_row_grad(const void* dout, const int32_t* sorted_token, const void* sorted_w, const void* y,
                    int64_t n_rows, int64_t dim, void* dy, void* dw_rows, hipStream_t s) {
  if (n_rows == 0) return ASTRAI_MOE_OK;
  hipLaunchKernelGGL(row_grad_kernel, dim3((unsigned)ceil_div(n_rows, 4)), dim3(256), 0, s,
                     static_cast<const bf16_t*>(dout), sorted_token, static_cast<const bf16_t*>(sorted_w),
                     static_cast<const bf16_t*>(y), n_rows, dim, static_cast<bf16_t*>(dy),
                     static_cast<bf16_t*>(dw_rows));
  return check_launch("row_grad_kernel");
}

int launch_dgrad_down(const void* dy, const int32_t* tiles, int64_t capacity, const void* const* w_down,
                      const void* gu, int64_t dim, int64_t dim_ffn, void* dg, void* du, hipStream_t s) {
  BwdArgs p{};
  p.a0 = static_cast<const bf16_t*>(dy);
  p.w0 = w_down;
  p.tiles = tiles;
  p.e0 = static_cast<const bf16_t*>(gu);
  p.c0 = static_cast<bf16_t*>(dg);
  p.c1 = static_cast<bf16_t*>(du);
  p.K = (int)dim;
  p.N = (int)dim_ffn;
  p.n_tiles_n = (int)ceil_div(dim_ffn, BwdCfg::BN);
  p.capacity = (int)capacity;
  return launch_bwd<Bwd::kDgradDown>(p, capacity * p.n_tiles_n, s, "gemm_bwd_kernel<dgrad_down>");
}

int launch_dgrad_in(const void* d, const int32_t* tiles, int64_t capacity, const void* const* w, int64_t k,
                    int64_t n, const void* add, void* dx, hipStream_t s, const GemmWorkspace& ws) {
  BwdArgs p{};
  p.a0 = static_cast<const bf16_t*>(d);
  p.w0 = w;
  p.tiles = tiles;
  p.e0 = static_cast<const bf16_t*>(add);
  p.c0 = static_cast<bf16_t*>(dx);
  p.K = (int)k;
  p.N = (int)n;
  p.n_tiles_n = (int)ceil_div(n, BwdCfg::BN);
  p.capacity = (int)capacity;
  if (add != nullptr)
    return launch_bwd<Bwd::kDgradInAdd>(p, capacity * p.n_tiles_n, s, "gemm_bwd_kernel<dgrad_in_add>", ws);
  return launch_bwd<Bwd::kDgradIn>(p, capacity * p.n_tiles_n, s, "gemm_bwd_kernel<dgrad_in>", ws);
}

int launch_wgrad(const void* a, const void* b, const int32_t* offsets, int n_experts, int64_t m, int64_t n,
                 void* dw, hipStream_t s) {
  BwdArgs p{};
  p.a0 = static_cast<const bf16_t*>(a);
  p.b_act = static_cast<const bf16_t*>(b);
  p.offsets = offsets;
  p.c0 = static_cast<bf16_t*>(dw);
  p.M = (int)m;
  p.N = (int)n;
  p.n_tiles_m = (int)ceil_div(m, BwdCfg::BM);
  p.n_tiles_n = (int)ceil_div(n, BwdCfg::BN);
  p.n_experts = n_experts;
  return launch_bwd<Bwd::kWgrad>(p, (int64_t)n_experts * p.n_tiles_m * p.n_tiles_n, s, "gemm_bwd_kernel<wgrad>");
}

}  // namespace astrai_moe
