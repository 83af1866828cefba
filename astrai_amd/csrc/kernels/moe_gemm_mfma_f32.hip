// fp32 grouped expert GEMMs on CDNA4 matrix cores (gfx950).
//
// Same contract as the bf16 kernels of moe_gemm_mfma.hip (reference semantics
// astrai/model/components/mlp.py:22-25, :96-97, with every rounding point an
// identity in float32): C[rows, N] = A[rows, K] . W_e[N, K]^T for every row
// tile of the device-built tile list, SiLU(gate) * up fused into the gate/up
// GEMM and the routing weight into the down GEMM.
//
// Matrix-core op: v_mfma_f32_16x16x4_f32 (2048 FLOP, full fp32 products and
// sums). Lane l supplies row l % 16 and K index l / 16 of each operand. The
// staged operands use the bf16 kernels' LDS layout unchanged: 128-byte row
// pieces (here 32 floats per K step) with 16-byte chunk c of staged row r at
// chunk c ^ ((r >> 1) & 7), filled by LDS DMA. A lane's 16-byte fragment read
// (row l % 16, chunk 4 kh + l / 16) yields four K values, which feed four
// MFMAs in a row: in MFMA s of half kh, lane group g contributes K index
// 16 kh + 4 g + s for both operands, so every product of the 16-K half is
// summed exactly once. The reads are conflict-free for the same reason as in
// the bf16 kernels (16 rows of one chunk column land on 16 bank groups).
//
// Work decomposition: 64-row tiles of the tile list (the fp32 tile height),
// BN = 64 weight rows per column tile (gate/up: 32 gate rows then the same 32
// up rows), 4 waves of 32 x 32, three 16 KB stages in flight, so a compute
// unit holds three workgroups and a wave waiting at its barrier leaves the
// matrix core to the other two. The down GEMM takes BN = 32 when 64-wide
// column tiles would leave most of those workgroup slots empty. The launch is
// persistent, round r of workgroup b taking logical tile r * G + b: with
// several workgroups per compute unit, the XCD-contiguous order of the bf16
// kernels would put a partial last round on the first XCDs only, where this
// order spreads it over all of them (measured 6-16 % faster on gate/up GEMMs
// of 1024-4096 tokens, D 512-2048; the down GEMMs within 1 %).
// Narrower tiles and more resident workgroups measured faster than 128- and
// 256-wide ones at every shape tried (up to 30 % on the down GEMM).
//
// Accumulator layout (weights as the first operand): lane l, element r of
// 16 x 16 tile (i, j) is output row 16 i + l % 16, column 16 j + 4 (l / 16) + r,
// so each lane stores 16 contiguous bytes per tile with no transpose.
#include "mfma_tile.h"

namespace astrai_moe {
namespace {

constexpr int kF32BK = kRowBytes / 4;  // 32 floats per staged row piece
constexpr int kF32BM = 64;

template <int BN_>
struct F32Cfg {
  static constexpr int BM = kF32BM, BN = BN_, STAGES = 3, WGM = 2, WGN = 2;
  static constexpr int WAVES = WGM * WGN;
  static constexpr int THREADS = WAVES * 64;
  static constexpr int WM = BM / WGM;
  static constexpr int WN = BN / WGN;
  static constexpr int A_BYTES = BM * kRowBytes;
  static constexpr int B_BYTES = BN * kRowBytes;
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int LDS_BYTES = STAGES * STAGE_BYTES;
  static constexpr int A_PER_WAVE = A_BYTES / 1024 / WAVES;
  static constexpr int B_PER_WAVE = B_BYTES / 1024 / WAVES;
  static constexpr int DMA_PER_WAVE = A_PER_WAVE + B_PER_WAVE;
  // workgroups one compute unit holds (LDS bound)
  static constexpr int PER_CU = (160 * 1024) / LDS_BYTES;
  static_assert(A_BYTES % (1024 * WAVES) == 0 && B_BYTES % (1024 * WAVES) == 0, "DMA ops split over waves");
  static_assert(WM % 16 == 0 && WN % 16 == 0, "16x16 MFMA tiles");
  static_assert(PER_CU >= 1, "LDS");
  static_assert(DMA_PER_WAVE * (STAGES - 1) <= 63, "vmcnt range");
};

template <int BN, bool kGateUp, bool kSave>
__global__ __launch_bounds__(256) void gemm_f32_mfma_kernel(
    const float* __restrict__ A, const int32_t* __restrict__ tiles, const void* const* __restrict__ W0,
    const void* const* __restrict__ W1, const float* __restrict__ row_w, int K, int N, int n_tiles_n, int capacity,
    float* __restrict__ C, float* __restrict__ S0) {
  using Cfg = F32Cfg<BN>;
  static_assert(!kGateUp || Cfg::WN % 32 == 0, "gate/up halves of 16 columns");
  constexpr int S = Cfg::STAGES;
  constexpr int DPW = Cfg::DMA_PER_WAVE;
  __shared__ __attribute__((aligned(1024))) char smem[Cfg::LDS_BYTES];

  const TileWalk<8> walk(tiles, capacity, n_tiles_n);
  int mt = 0, nt = 0;
  int logical = walk.seek((int)blockIdx.x, mt, nt);
  if (logical >= walk.total) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wm = wave / Cfg::WGN;
  const int wn = wave % Cfg::WGN;
  const uint32_t k4 = (uint32_t)K * 4u;
  const int KT = K / kF32BK;

  // ---- per-tile sources ----
  const char* a_base = nullptr;
  const char* b_base0 = nullptr;
  const char* b_base1 = nullptr;
  int row0 = 0, rows = 0;
  auto setup_tile = [&](int mt_, int nt_) {
    const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)mt_ * ASTRAI_MOE_TILE_STRIDE;
    const int e = ti[0];
    row0 = ti[1];
    rows = min(Cfg::BM, ti[2] - row0);
    a_base = reinterpret_cast<const char*>(A + (int64_t)row0 * K);
    b_base0 = reinterpret_cast<const char*>(static_cast<const float*>(W0[e]) +
                                            (int64_t)nt_ * (kGateUp ? BN / 2 : BN) * K);
    b_base1 = kGateUp ? reinterpret_cast<const char*>(static_cast<const float*>(W1[e]) + (int64_t)nt_ * (BN / 2) * K)
                      : b_base0;
  };
  // one K step into stage buffer `buf`; rows past the tile's last re-read it
  auto issue_stage = [&](int kstep, int buf) {
    char* sa = smem + buf * Cfg::STAGE_BYTES;
    char* sb = sa + Cfg::A_BYTES;
    const DmaLane dl(lane, kstep);
#pragma unroll
    for (int i = 0; i < Cfg::A_PER_WAVE; ++i) {
      const int q = wave * Cfg::A_PER_WAVE + i;
      const uint32_t row = (uint32_t)min(q * 8 + dl.row, rows - 1);
      lds_dma_16(a_base + (row * k4 + dl.chunk(q)), sa + q * 1024);
    }
#pragma unroll
    for (int i = 0; i < Cfg::B_PER_WAVE; ++i) {
      const int q = wave * Cfg::B_PER_WAVE + i;
      const int r0 = q * 8;
      const bool up = kGateUp && r0 >= BN / 2;
      const char* bb = up ? b_base1 : b_base0;
      const int rq = up ? r0 - BN / 2 : r0;
      lds_dma_16(bb + ((uint32_t)(rq + dl.row) * k4 + dl.chunk(q)), sb + q * 1024);
    }
  };

  // ---- fragment reads: lane l, row l % 16, 16-byte chunk 4 kh + l / 16 ----
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
      r = (j < half) ? wn * (Cfg::WN / 2) + j * 16 : BN / 2 + wn * (Cfg::WN / 2) + (j - half) * 16;
    } else {
      r = wn * Cfg::WN + j * 16;
    }
    b_off[j] = (r + frag_row) * kRowBytes;
  }
  f32x4_t fa[2][MT16], fb[2][NT16];
  auto read_frags = [&](int buf, int kh, int slot) {
    const char* sa = smem + buf * Cfg::STAGE_BYTES;
    const char* sb = sa + Cfg::A_BYTES;
    const int sw = ((kh * 4 + fq) ^ fsw) << 4;
#pragma unroll
    for (int i = 0; i < MT16; ++i) fa[slot][i] = *reinterpret_cast<const f32x4_t*>(sa + a_off[i] + sw);
#pragma unroll
    for (int j = 0; j < NT16; ++j) fb[slot][j] = *reinterpret_cast<const f32x4_t*>(sb + b_off[j] + sw);
  };
  f32x4_t acc[MT16][NT16];
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < MT16; ++i)
#pragma unroll
        for (int j = 0; j < NT16; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fb[slot][j][s], fa[slot][i][s], acc[i][j], 0, 0, 0);
  };

  const int row_l = lane & 15;
  const int col_l = 4 * (lane >> 4);
  while (true) {
    setup_tile(mt, nt);
#pragma unroll
    for (int s = 0; s < S; ++s)
      if (s < KT) issue_stage(s, s);
#pragma unroll
    for (int i = 0; i < MT16; ++i)
#pragma unroll
      for (int j = 0; j < NT16; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;
    wait_groups<DPW, S - 1>(min(S - 1, KT - 1));  // step 0 landed
    lds_barrier();
    read_frags(0, 0, 0);
    int buf = 0;
    for (int kt = 0; kt < KT; ++kt) {
      read_frags(buf, 1, 1);
      mfmas(0);
      const int nbuf = (buf + 1 == S) ? 0 : buf + 1;
      if (kt + 1 < KT) {
        wait_groups<DPW, S - 2>(min(S - 2, KT - 2 - kt));
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();  // step kt + 1 landed; every wave is done reading buffer `buf`
        __builtin_amdgcn_sched_barrier(0);
        read_frags(nbuf, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (kt + S < KT) issue_stage(kt + S, buf);
        __builtin_amdgcn_sched_barrier(0);
      }
      mfmas(1);
      buf = nbuf;
    }

    // ---- epilogue: 16 contiguous bytes per lane and tile ----
#pragma unroll
    for (int i = 0; i < MT16; ++i) {
      const int r = wm * Cfg::WM + i * 16 + row_l;
      if (r < rows) {
        const int64_t grow = (int64_t)row0 + r;
        if constexpr (kGateUp) {
          constexpr int NJ = NT16 / 2;
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const int n = nt * (BN / 2) + wn * (Cfg::WN / 2) + j * 16 + col_l;
            const f32x4_t g = acc[i][j], u = acc[i][j + NJ];
            f32x4_t h;
#pragma unroll
            for (int q = 0; q < 4; ++q) h[q] = u[q] * silu_f32(g[q]);
            *reinterpret_cast<f32x4_t*>(C + grow * N + n) = h;
            if constexpr (kSave) {
              // gu_index: the 4 gate values of columns n..n+3 at 2n, their up values at 2n + 4
              float* gu = S0 + grow * 2 * N + 2 * (int64_t)n;
              *reinterpret_cast<f32x4_t*>(gu) = g;
              *reinterpret_cast<f32x4_t*>(gu + 4) = u;
            }
          }
        } else {
          const float w = row_w != nullptr ? row_w[grow] : 1.0f;  // no row weights: 1
#pragma unroll
          for (int j = 0; j < NT16; ++j) {
            const int n = nt * BN + wn * Cfg::WN + j * 16 + col_l;
            const f32x4_t y = acc[i][j];
            if constexpr (kSave) *reinterpret_cast<f32x4_t*>(S0 + grow * N + n) = y;
            *reinterpret_cast<f32x4_t*>(C + grow * N + n) = y * w;
          }
        }
      }
    }

    logical = walk.seek(logical + walk.G, mt, nt);
    if (logical >= walk.total) break;
    lds_barrier();  // every wave is done with the stage buffers before the next tile's DMA
  }
}

template <int BN, bool kGateUp, bool kSave>
int launch_f32_bn(const void* A, const int32_t* tiles, int64_t capacity, const void* const* W0,
                  const void* const* W1, const void* row_w, int64_t K, int64_t N, void* C, void* S0,
                  hipStream_t s) {
  using Cfg = F32Cfg<BN>;
  const int64_t n_tiles_n = kGateUp ? N / (BN / 2) : N / BN;
  const int64_t total = capacity * n_tiles_n;
  if (total >= (1ll << 31))
    return fail(ASTRAI_MOE_EINVAL, "gemm: %lld tiles exceed the tile-index range", (long long)total);
  const int64_t grid = std::min<int64_t>(total, (int64_t)cu_count() * Cfg::PER_CU);
  hipLaunchKernelGGL((gemm_f32_mfma_kernel<BN, kGateUp, kSave>), dim3((unsigned)grid), dim3(Cfg::THREADS), 0, s,
                     static_cast<const float*>(A), tiles, W0, W1, static_cast<const float*>(row_w), (int)K, (int)N,
                     (int)n_tiles_n, (int)capacity, static_cast<float*>(C), static_cast<float*>(S0));
  return check_launch(kGateUp ? "gemm_f32_mfma_kernel<gate_up>" : "gemm_f32_mfma_kernel<down>");
}

template <bool kGateUp, bool kSave>
int launch_f32(const void* A, const int32_t* tiles, int64_t capacity, const void* const* W0, const void* const* W1,
               const void* row_w, int64_t n_rows, int n_experts, int64_t K, int64_t N, void* C, void* S0,
               hipStream_t s) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  if constexpr (!kGateUp) {
    // 32-wide down tiles when the 64-wide ones, estimated from the rows and
    // the experts' partial last tiles, would not give every compute unit two
    const int64_t row_tiles = ceil_div(n_rows, kF32BM) + n_experts / 2;
    if (row_tiles * (N / 64) < 2ll * cu_count())
      return launch_f32_bn<32, false, kSave>(A, tiles, capacity, W0, W1, row_w, K, N, C, S0, s);
  }
  return launch_f32_bn<64, kGateUp, kSave>(A, tiles, capacity, W0, W1, row_w, K, N, C, S0, s);
}

}  // namespace

bool mfma_f32_supported(int64_t k, int64_t n, bool gate_up, int block_m, const void* a, const void* c,
                        const void* s0) {
  const int64_t min_cols = gate_up ? 32 : 64;  // output columns of a column tile
  return block_m == kF32BM && k > 0 && n > 0 && k % kF32BK == 0 && n % min_cols == 0 && k <= (1ll << 22) &&
         n <= (1ll << 22) && aligned16(a) && aligned16(c) && (s0 == nullptr || aligned16(s0));
}

int launch_mfma_f32_gate_up(const void* x_perm, const int32_t* tiles, int64_t capacity, const void* const* w_gate,
                            const void* const* w_up, int64_t n_rows, int n_experts, int64_t dim, int64_t dim_ffn,
                            void* h, void* gu, hipStream_t s) {
  if (gu != nullptr)
    return launch_f32<true, true>(x_perm, tiles, capacity, w_gate, w_up, nullptr, n_rows, n_experts, dim, dim_ffn,
                                  h, gu, s);
  return launch_f32<true, false>(x_perm, tiles, capacity, w_gate, w_up, nullptr, n_rows, n_experts, dim, dim_ffn, h,
                                 nullptr, s);
}

int launch_mfma_f32_down(const void* h, const int32_t* tiles, int64_t capacity, const void* const* w_down,
                         const void* sorted_w, int64_t n_rows, int n_experts, int64_t dim_ffn, int64_t dim, void* y,
                         void* y_unweighted, hipStream_t s) {
  if (y_unweighted != nullptr)
    return launch_f32<false, true>(h, tiles, capacity, w_down, nullptr, sorted_w, n_rows, n_experts, dim_ffn, dim, y,
                                   y_unweighted, s);
  return launch_f32<false, false>(h, tiles, capacity, w_down, nullptr, sorted_w, n_rows, n_experts, dim_ffn, dim, y,
                                  nullptr, s);
}

}  // namespace astrai_moe
