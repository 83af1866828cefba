// fp32 backward of the routed experts on CDNA4 matrix cores (gfx950): the
// grouped dgrad (NN) and wgrad (TN) GEMMs of moe_gemm_generic_bwd.hip on
// v_mfma_f32_16x16x4_f32, with the same epilogues and the same contracts.
//
// Reference: torch autograd over astrai/model/components/mlp.py:22-25 and
// :97-98, per expert e with rows R_e (every rounding point the identity in
// fp32):
//   dh = dy . W_down      [R_e, F]  (NN, W_down [D, F]); du = dh silu(g),
//                                    dg = silu'(g) (dh u) in the epilogue
//   dx = dg . W_gate (+ du . W_up)   (NN twice, the second adding the first)
//   dW_down = dy^T h, dW_gate = dg^T x, dW_up = du^T x   (TN per expert)
// silu and sigmoid are evaluated as torch's float kernels do: x / (1 + exp(-x))
// and 1 / (1 + exp(-x)).
//
// Operands. A K-contiguous operand (the dgrad activations) is staged as in
// the forward fp32 kernel: 128-byte row pieces (32 K values), chunk-swizzled,
// read 16 bytes per lane, which gives a lane the four K values of four MFMAs
// in a row. An MN-contiguous operand (the dgrad weights [K, N], both wgrad
// operands [rows, M or N]) is staged as it lies, 32 K-rows of 64 or 128
// consecutive columns per stage, and read 16 bytes per lane as well: lane l
// (group g = l / 16, c = l % 16) reads, for MFMA step s, K-row 4 g + s of a
// 16-K half and columns 4 c .. 4 c + 3. Those four values feed four MFMAs of
// four different 16-column blocks: block q takes column 4 c + q for its local
// column c. A 16-lane group reads one 256-byte K-row, conflict-free, and a
// 16-K half needs four such reads for 4 x 4 MFMAs.
//
// Output layout (MN-contiguous operand as the first MFMA operand): lane l,
// element r of block q holds local row i = 4 (l / 16) + r, i.e. column
// 16 (l / 16) + 4 r + q of the 64-column block, and the row given by the
// second operand's lane l % 16. Over q = 0..3 a lane thus holds four
// consecutive columns per r: one 16-byte store each.
#include <climits>

#include "mfma_tile.h"

namespace astrai_moe {
namespace {

constexpr int kF32K = kRowBytes / 4;  // 32 K values per stage
constexpr int kF32Stages = 3;

enum class F32Nn { kDgradDown, kDgradIn, kDgradInAdd };

// Source of K-rows past an expert's last row in wgrad (zero contribution).
__device__ __attribute__((aligned(512))) uint4 g_zero_f32[32] = {};

__device__ inline float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

// One 1 KB DMA op of an MN-major stage whose K-rows hold COLS floats: K-rows
// krow0 + (1024 / (4 COLS)) o + ... of `base` (pitch bytes apart), COLS
// floats from byte col0; K-rows at or past valid_rows read zeros, columns past
// the matrix re-read its last 16 bytes (masked in the epilogue).
template <int COLS>
__device__ __forceinline__ void dma_mn_f32(const char* base, int krow0, int valid_rows, uint32_t pitch,
                                           uint32_t col0, uint32_t col_end, int lane, int o, char* lds) {
  constexpr int kLanesPerRow = COLS * 4 / 16;
  constexpr int kRowsPerOp = 64 / kLanesPerRow;
  const int row = krow0 + kRowsPerOp * o + lane / kLanesPerRow;
  const uint32_t col = min(col0 + (uint32_t)(lane % kLanesPerRow) * 16u, col_end - 16u);
  const char* src = row < valid_rows ? base + (int64_t)row * pitch + col
                                     : reinterpret_cast<const char*>(g_zero_f32) + (lane % kLanesPerRow) * 16;
  lds_dma_16(src, lds);
}

// ---------------------------------------------------------------------------
// dgrad: C[rows, N] = A[rows, K] . W_e[K, N] over the forward's 64-row tile
// list, 64-column tiles; 4 waves of 16 rows x 64 columns; three 16 KB stages,
// three workgroups per CU, persistent in plain block order.
// ---------------------------------------------------------------------------
template <F32Nn kMode>
__global__ __launch_bounds__(256) void gemm_f32_dgrad_kernel(const float* __restrict__ A,
                                                            const int32_t* __restrict__ tiles,
                                                            const void* const* __restrict__ W, const float* E0, int K,
                                                            int N, int n_tiles_n, int capacity, float* C0,
                                                            float* C1) {
  constexpr int A_BYTES = 64 * kRowBytes;  // 64 rows x 32 K
  constexpr int B_BYTES = kF32K * 256;     // 32 K-rows x 64 columns
  constexpr int STAGE = A_BYTES + B_BYTES;
  constexpr int S = kF32Stages;
  constexpr int DPW = 4;  // DMA ops per wave and stage: 2 for A, 2 for B
  __shared__ __attribute__((aligned(1024))) char smem[S * STAGE];

  const TileWalk<8> walk(tiles, capacity, n_tiles_n);
  int mt = 0, nt = 0;
  int logical = walk.seek((int)blockIdx.x, mt, nt);
  if (logical >= walk.total) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const uint32_t k4 = (uint32_t)K * 4u, n4 = (uint32_t)N * 4u;
  const int KT = K / kF32K;

  const char* a_base = nullptr;
  const char* b_base = nullptr;
  int row0 = 0, rows = 0;
  uint32_t col0 = 0;
  auto setup_tile = [&](int mt_, int nt_) {
    const int32_t* ti = tiles + ASTRAI_MOE_TILE_HEADER + (int64_t)mt_ * ASTRAI_MOE_TILE_STRIDE;
    row0 = ti[1];
    rows = min(64, ti[2] - row0);
    a_base = reinterpret_cast<const char*>(A + (int64_t)row0 * K);
    b_base = static_cast<const char*>(W[ti[0]]);
    col0 = (uint32_t)nt_ * 256u;
  };
  auto issue_stage = [&](int kstep, int buf) {
    char* sa = smem + buf * STAGE;
    char* sb = sa + A_BYTES;
    const DmaLane dl(lane, kstep);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = wave * 2 + i;
      const uint32_t row = (uint32_t)min(q * 8 + dl.row, rows - 1);  // pad rows re-read the last
      lds_dma_16(a_base + (row * k4 + dl.chunk(q)), sa + q * 1024);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int o = wave * 2 + i;
      dma_mn_f32<64>(b_base, kstep * kF32K, INT_MAX, n4, col0, n4, lane, o, sb + o * 1024);
    }
  };

  const int c = lane & 15;
  const int g = lane >> 4;
  const int a_off = (wave * 16 + c) * kRowBytes;
  const int fsw = (c >> 1) & 7;
  f32x4_t fa[2], fb[2][4];
  auto read_frags = [&](int buf, int kh, int slot) {
    const char* sa = smem + buf * STAGE;
    const char* sb = sa + A_BYTES;
    fa[slot] = *reinterpret_cast<const f32x4_t*>(sa + a_off + (((kh * 4 + g) ^ fsw) << 4));
#pragma unroll
    for (int s = 0; s < 4; ++s)
      fb[slot][s] = *reinterpret_cast<const f32x4_t*>(sb + (kh * 16 + 4 * g + s) * 256 + c * 16);
  };
  f32x4_t acc[4];
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(fb[slot][s][q], fa[slot][s], acc[q], 0, 0, 0);
  };

  while (true) {
    setup_tile(mt, nt);
#pragma unroll
    for (int s = 0; s < S; ++s)
      if (s < KT) issue_stage(s, s);
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
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

    // ---- epilogue: row wave * 16 + c, columns 16 g + 4 r .. + 3 ----
    const int rr = wave * 16 + c;
    if (rr < rows) {
      const int64_t grow = (int64_t)row0 + rr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = nt * 64 + 16 * g + 4 * r;
        if (n >= N) continue;  // N % 4 == 0: the 4 columns are all inside or all past the matrix
        const f32x4_t v = {acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
        if constexpr (kMode == F32Nn::kDgradDown) {
          // gu keeps g of columns n..n+3 at 2 n and their u at 2 n + 4
          const float* gu = E0 + grow * 2 * N + 2 * (int64_t)n;
          const f32x4_t gv = *reinterpret_cast<const f32x4_t*>(gu);
          const f32x4_t uv = *reinterpret_cast<const f32x4_t*>(gu + 4);
          f32x4_t dg, du;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const float sg = sigmoid_f32(gv[k]);
            du[k] = v[k] * (gv[k] * sg);  // dh * silu(g)
            dg[k] = (v[k] * uv[k]) * (sg * (1.0f + gv[k] * (1.0f - sg)));
          }
          *reinterpret_cast<f32x4_t*>(C1 + grow * N + n) = du;
          *reinterpret_cast<f32x4_t*>(C0 + grow * N + n) = dg;
        } else if constexpr (kMode == F32Nn::kDgradInAdd) {
          // E0 may be C0 itself: each element is read before this lane writes it
          const f32x4_t add = *reinterpret_cast<const f32x4_t*>(E0 + grow * N + n);
          *reinterpret_cast<f32x4_t*>(C0 + grow * N + n) = v + add;
        } else {
          *reinterpret_cast<f32x4_t*>(C0 + grow * N + n) = v;
        }
      }
    }

    logical = walk.seek(logical + walk.G, mt, nt);
    if (logical >= walk.total) break;
    lds_barrier();  // every wave is done with the stage buffers before the next tile's DMA
  }
}

// ---------------------------------------------------------------------------
// wgrad: dw[e] [M, N] = a[rows_e]^T . b[rows_e] for every expert with rows,
// 128 x 128 tiles, 4 waves of 64 x 64, K = the expert's rows in steps of 32
// (rows past the expert's last read zeros); three 32 KB stages, one
// workgroup per CU, persistent over (expert, M tile, N tile).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gemm_f32_wgrad_kernel(const float* __restrict__ a,
                                                            const float* __restrict__ b,
                                                            const int32_t* __restrict__ offsets, int n_experts,
                                                            int M, int N, int n_tiles_m, int n_tiles_n,
                                                            float* __restrict__ dw) {
  constexpr int OP_BYTES = kF32K * 512;  // 32 K-rows x 128 columns, per operand
  constexpr int STAGE = 2 * OP_BYTES;
  constexpr int S = kF32Stages;
  constexpr int DPW = 8;  // 4 ops per operand and wave
  __shared__ __attribute__((aligned(1024))) char smem[S * STAGE];

  const int per_e = n_tiles_m * n_tiles_n;
  const int total = n_experts * per_e;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const uint32_t m4 = (uint32_t)M * 4u, n4 = (uint32_t)N * 4u;

  const int c = lane & 15;
  const int g = lane >> 4;
  f32x4_t fa[2][4], fb[2][4];
  f32x4_t acc[4][4];

  for (int logical = (int)blockIdx.x; logical < total; logical += (int)gridDim.x) {
    const int e = logical / per_e;
    const int rem = logical - e * per_e;
    const int mt = rem / n_tiles_n, nt = rem - (rem / n_tiles_n) * n_tiles_n;
    const int r0 = offsets[e];
    const int rows = offsets[e + 1] - r0;
    if (rows <= 0) continue;  // experts without rows are not written
    const int KT = (rows + kF32K - 1) / kF32K;
    const char* a_base = reinterpret_cast<const char*>(a + (int64_t)r0 * M);
    const char* b_base = reinterpret_cast<const char*>(b + (int64_t)r0 * N);
    const uint32_t acol0 = (uint32_t)mt * 512u, bcol0 = (uint32_t)nt * 512u;

    auto issue_stage = [&](int kstep, int buf) {
      char* sa = smem + buf * STAGE;
      char* sb = sa + OP_BYTES;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int o = wave * 4 + i;
        dma_mn_f32<128>(a_base, kstep * kF32K, rows, m4, acol0, m4, lane, o, sa + o * 1024);
        dma_mn_f32<128>(b_base, kstep * kF32K, rows, n4, bcol0, n4, lane, o, sb + o * 1024);
      }
    };
    auto read_frags = [&](int buf, int kh, int slot) {
      const char* sa = smem + buf * STAGE;
      const char* sb = sa + OP_BYTES;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int krow = kh * 16 + 4 * g + s;
        fa[slot][s] = *reinterpret_cast<const f32x4_t*>(sa + krow * 512 + wm * 256 + c * 16);
        fb[slot][s] = *reinterpret_cast<const f32x4_t*>(sb + krow * 512 + wn * 256 + c * 16);
      }
    };
    auto mfmas = [&](int slot) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int qa = 0; qa < 4; ++qa)
#pragma unroll
          for (int qb = 0; qb < 4; ++qb)
            acc[qa][qb] =
                __builtin_amdgcn_mfma_f32_16x16x4f32(fb[slot][s][qb], fa[slot][s][qa], acc[qa][qb], 0, 0, 0);
    };

#pragma unroll
    for (int s = 0; s < S; ++s)
      if (s < KT) issue_stage(s, s);
#pragma unroll
    for (int qa = 0; qa < 4; ++qa)
#pragma unroll
      for (int qb = 0; qb < 4; ++qb) acc[qa][qb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
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

    // ---- epilogue: rows m = 4 c + qa, columns 16 g + 4 r .. + 3 of the wave's 64 x 64 ----
#pragma unroll
    for (int qa = 0; qa < 4; ++qa) {
      const int m = mt * 128 + wm * 64 + 4 * c + qa;
      if (m >= M) continue;
      float* out = dw + ((int64_t)e * M + m) * N;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = nt * 128 + wn * 64 + 16 * g + 4 * r;
        if (n < N)  // N % 4 == 0
          *reinterpret_cast<f32x4_t*>(out + n) = f32x4_t{acc[qa][0][r], acc[qa][1][r], acc[qa][2][r], acc[qa][3][r]};
      }
    }
    lds_barrier();  // every wave is done with the stage buffers before the next tile's DMA
  }
}

template <F32Nn kMode>
int launch_f32_dgrad(const void* a, const int32_t* tiles, int64_t capacity, const void* const* w, const void* e0,
                     int64_t k, int64_t n, void* c0, void* c1, hipStream_t s, const char* name) {
  if (capacity == 0) return ASTRAI_MOE_OK;
  const int64_t n_tiles_n = ceil_div(n, 64);
  const int64_t total = capacity * n_tiles_n;
  if (total >= (1ll << 31)) return fail(ASTRAI_MOE_EINVAL, "%s: %lld tiles exceed the tile-index range", name,
                                        (long long)total);
  const int64_t grid = std::min<int64_t>(total, 3ll * cu_count());  // three 48 KB workgroups per CU
  hipLaunchKernelGGL((gemm_f32_dgrad_kernel<kMode>), dim3((unsigned)grid), dim3(256), 0, s,
                     static_cast<const float*>(a), tiles, w, static_cast<const float*>(e0), (int)k, (int)n,
                     (int)n_tiles_n, (int)capacity, static_cast<float*>(c0), static_cast<float*>(c1));
  return check_launch(name);
}

}  // namespace

bool mfma_f32_bwd_supported(int64_t k, int64_t n, int block_m, const void* a, const void* c0, const void* c1,
                            const void* e0) {
  return block_m == 64 && k > 0 && n > 0 && k % kF32K == 0 && n % 4 == 0 && k <= (1ll << 22) &&
         n <= (1ll << 22) && aligned16(a) && aligned16(c0) && (c1 == nullptr || aligned16(c1)) &&
         (e0 == nullptr || aligned16(e0));
}

bool mfma_f32_wgrad_supported(int64_t m, int64_t n, const void* a, const void* b, const void* dw) {
  return m > 0 && n > 0 && m % 4 == 0 && n % 4 == 0 && m <= (1ll << 22) && n <= (1ll << 22) && aligned16(a) &&
         aligned16(b) && aligned16(dw);
}

int launch_mfma_f32_dgrad_down(const void* dy, const int32_t* tiles, int64_t capacity, const void* const* w_down,
                               const void* gu, int64_t dim, int64_t dim_ffn, void* dg, void* du, hipStream_t s) {
  return launch_f32_dgrad<F32Nn::kDgradDown>(dy, tiles, capacity, w_down, gu, dim, dim_ffn, dg, du, s,
                                             "gemm_f32_dgrad_kernel<dgrad_down>");
}

int launch_mfma_f32_dgrad_in(const void* d, const int32_t* tiles, int64_t capacity, const void* const* w, int64_t k,
                             int64_t n, const void* add, void* dx, hipStream_t s) {
  if (add != nullptr)
    return launch_f32_dgrad<F32Nn::kDgradInAdd>(d, tiles, capacity, w, add, k, n, dx, nullptr, s,
                                                "gemm_f32_dgrad_kernel<dgrad_in_add>");
  return launch_f32_dgrad<F32Nn::kDgradIn>(d, tiles, capacity, w, nullptr, k, n, dx, nullptr, s,
                                           "gemm_f32_dgrad_kernel<dgrad_in>");
}

int launch_mfma_f32_wgrad(const void* a, const void* b, const int32_t* offsets, int n_experts, int64_t m, int64_t n,
                          void* dw, hipStream_t s) {
  const int64_t n_tiles_m = ceil_div(m, 128), n_tiles_n = ceil_div(n, 128);
  const int64_t total = (int64_t)n_experts * n_tiles_m * n_tiles_n;
  if (total >= (1ll << 31))
    return fail(ASTRAI_MOE_EINVAL, "gemm_wgrad: %lld tiles exceed the tile-index range", (long long)total);
  const int64_t grid = std::min<int64_t>(total, cu_count());  // one 96 KB workgroup per CU
  hipLaunchKernelGGL(gemm_f32_wgrad_kernel, dim3((unsigned)grid), dim3(256), 0, s, static_cast<const float*>(a),
                     static_cast<const float*>(b), offsets, n_experts, (int)m, (int)n, (int)n_tiles_m,
                     (int)n_tiles_n, static_cast<float*>(dw));
  return check_launch("gemm_f32_wgrad_kernel");
}

}  // namespace astrai_moe
