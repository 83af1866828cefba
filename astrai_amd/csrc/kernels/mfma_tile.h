// Device helpers shared by the CDNA4 matrix-core GEMMs (gfx950): operand
// vector types, LDS DMA and its waits, the persistent XCD-aware tile walk,
// the per-lane DMA chunk choice of the 16-byte LDS swizzle and the lane-group
// transpose of the epilogues.
#pragma once

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

// Padding-only waves: a matrix-core wave whose first row is wave_row0 idles
// on a tile of `rows` valid rows iff idle_threshold(eligible, wave_row0) >=
// rows. A tile that may not idle gets -1, which no row count reaches (every
// tile has at least one row), and wave 0 (rows from 0) never idles, so the
// run-time claims it makes always happen.
__host__ __device__ constexpr int idle_threshold(bool eligible, int wave_row0) { return eligible ? wave_row0 : -1; }
static_assert(!(idle_threshold(false, 128) >= 1), "a tile that may not idle keeps every wave");
static_assert(!(idle_threshold(true, 0) >= 1), "wave 0 never idles");
static_assert(idle_threshold(true, 128) >= 128 && !(idle_threshold(true, 128) >= 129),
              "the second half idles exactly on tiles of at most 128 rows");
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

// Wave-uniform (SGPR) copies of values every lane holds alike, such as tile
// fields and weight pointers loaded at a tile boundary. Left in VGPRs, a value
// loaded on the tile-boundary path but used by every step's DMA makes the
// compiler wait for every load in flight (the LDS DMA of the stages ahead
// included) before that use, once per step.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
template <typename T>
__device__ __forceinline__ T* uniform(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(lo | (hi << 32));
}

// A load through the scalar cache (s_load), for data that nothing writes
// while the kernel runs (tile lists, expert offsets, weight-pointer tables)
// at a wave-uniform address. A vector load there would be counted by vmcnt
// like the LDS DMA, and waiting for it would drain the stages in flight.
template <typename T>
__device__ __forceinline__ T load_scalar(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
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
// logical tiles walk GM row tiles for every column tile.
//
// GM = 16 walks a group of 16 row tiles as two halves of 8 side by side: for
// each run of 4 column tiles, the first half's 8 x 4 block, then the second
// half's. With 32 workgroups per XCD, neighbouring XCDs then take the two
// halves of the same 4 column tiles at the same time, so each weight tile of
// an expert whose rows fill the group leaves HBM once (the second XCD finds
// it in the Infinity Cache) where two groups of 8 walked one after the other
// read it twice, while every XCD keeps its 8 x 4 block of tiles (12 operand
// strips per 32 tiles through its L2).
template <int GM>
struct TileWalk {
  int G, n_live, total, group_size;
  // Only the live row tiles (tiles[0] of them) enter the logical order, and
  // the last group holds just the live tiles left, so the live logical tiles
  // are exactly [0, total) and each round but the last is full. (Sizing the
  // last group by the list's capacity instead spread its live tiles over
  // several mostly empty rounds.)
  // G: the workgroups walking the list (the launch's grid unless given)
  __device__ TileWalk(const int32_t* tiles, int capacity, int n_tiles_n, int G_ = 0)
      : G(G_ > 0 ? G_ : (int)gridDim.x),
        n_live(min(tiles[0], min(tiles[2], capacity))),
        total(n_live * n_tiles_n),
        group_size(GM * n_tiles_n) {}
  __device__ int first_slot() const {
    const int bid = blockIdx.x;
    return (G % kXcds == 0) ? (bid % kXcds) * (G / kXcds) + bid / kXcds : bid;
  }
  __device__ void decode(int logical, int& mt, int& nt) const {
    const int first_m = (logical / group_size) * GM;
    const int gm = min(GM, n_live - first_m);
    const int in_group = logical - (first_m / GM) * group_size;
    if constexpr (GM == 16) {
      // runs of 4 column tiles, each the first half's block then the second's
      const int ga = min(8, gm), gb = gm - ga;
      const int n_tiles_n = group_size / GM;
      const int c = min(in_group / (gm * 4), (n_tiles_n - 1) / 4);
      const int j = in_group - c * gm * 4;
      const int wc = min(4, n_tiles_n - 4 * c);
      if (j < ga * wc) {
        mt = first_m + j % ga;
        nt = 4 * c + j / ga;
      } else {
        mt = first_m + ga + (j - ga * wc) % gb;
        nt = 4 * c + (j - ga * wc) / gb;
      }
    } else {
      mt = first_m + in_group % gm;
      nt = in_group / gm;
    }
  }
  // this workgroup's tile at `logical` (>= total: none)
  __device__ int seek(int logical, int& mt, int& nt) const {
    if (logical < total) decode(logical, mt, nt);
    return logical;
  }
};

// The persistent walk of the 256-row GEMMs, with the last round's tiles split
// along K. After R whole rounds of the G workgroups, L = total mod G tiles
// are left; run whole, they would hold L compute units for a full tile time
// while the other G - L idle (measured at the Mixtral-shaped down GEMM: 32
// tiles left after 8 rounds, 1.5 % of the work, cost 7.8 % of its time).
// When a partial-sum buffer is given and L <= G / 2, each of those tiles is
// cut into S = min(G / L, KT / kSplitMinSteps) ranges of K steps; the L * S
// work units take the last round's slots (one per workgroup), each stores its
// fp32 accumulators, and a reduce kernel (split_reduce_kernel of the forward
// down GEMM, bwd_split_reduce_kernel of the dgrad_in GEMMs) sums a tile's S
// partials in slice order and runs the tile's epilogue. Work items are indexed
// like tiles: item i < full is logical tile i, item full + u is unit u (tile
// full + u / S, slice u % S).
constexpr int kSplitMinSteps = 8;
// Tiles of fewer K steps are never split: the reduce launch and the partial
// sums' traffic (~15 us at 16 tiles) cost about what splitting a short tile
// saves (the fine-grained shape's 22-step down tiles take ~31 us).
constexpr int kSplitMinTileSteps = 64;
constexpr int kSplitUnitFloats = kMfmaBigBM * 256;  // fp32 accumulators of one 256 x 256 tile

template <int GM>
struct SplitWalk : TileWalk<GM> {
  int full, S, KT;
  __device__ SplitWalk(const int32_t* tiles, int capacity, int n_tiles_n, int KT_, bool split, int G_ = 0)
      : TileWalk<GM>(tiles, capacity, n_tiles_n, G_), full(this->total), S(1), KT(KT_) {
    if (split) {
      const int L = this->total % this->G;
      const int s = (L > 0 && 2 * L <= this->G) ? min(this->G / L, KT / kSplitMinSteps) : 1;
      if (s >= 2) S = s, full = this->total - L;
    }
  }
  __device__ int items() const { return full + (this->total - full) * S; }
  // item `i` (< items()): its tile, K steps [k0, k1) and tail unit (-1: the whole tile)
  __device__ void item(int i, int& mt, int& nt, int& k0, int& k1, int& unit) const {
    if (i < full) {
      this->decode(i, mt, nt);
      k0 = 0, k1 = KT, unit = -1;
      return;
    }
    const int u = i - full, s = u % S;
    this->decode(full + u / S, mt, nt);
    k0 = s * KT / S, k1 = (s + 1) * KT / S, unit = u;
  }
};

// A tail unit's fp32 accumulators, wave by wave in the accumulator layout:
// part[unit][wave][i][j][lane] as 16-byte vectors (one 1 KB store per wave
// and 16x16 tile).
template <int MT16, int NT16>
__device__ __forceinline__ void store_partial(const f32x4_t (&acc)[MT16][NT16], float* part, int unit, int wave,
                                              int lane) {
  f32x4_t* p = reinterpret_cast<f32x4_t*>(part) + ((int64_t)unit * 8 + wave) * (MT16 * NT16 * 64) + lane;
#pragma unroll
  for (int i = 0; i < MT16; ++i)
#pragma unroll
    for (int j = 0; j < NT16; ++j) p[(i * NT16 + j) * 64] = acc[i][j];
}

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

// ---- epilogue stores ----

typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Cross-lane exchanges of gfx950 on 8-byte values (one per lane): swap32
// trades lanes 32-63 of a for lanes 0-31 of b, swap16 trades the odd 16-lane
// rows of a (lanes 16-31, 48-63) for the even rows of b. Lane l keeps its
// l % 16 either way.
__device__ __forceinline__ void swap32(bf16x4_t& a, bf16x4_t& b) {
  const u32x2_t x = __builtin_bit_cast(u32x2_t, a), y = __builtin_bit_cast(u32x2_t, b);
  const auto r0 = __builtin_amdgcn_permlane32_swap(x[0], y[0], false, false);
  const auto r1 = __builtin_amdgcn_permlane32_swap(x[1], y[1], false, false);
  a = __builtin_bit_cast(bf16x4_t, u32x2_t{r0[0], r1[0]});
  b = __builtin_bit_cast(bf16x4_t, u32x2_t{r0[1], r1[1]});
}
__device__ __forceinline__ void swap16(bf16x4_t& a, bf16x4_t& b) {
  const u32x2_t x = __builtin_bit_cast(u32x2_t, a), y = __builtin_bit_cast(u32x2_t, b);
  const auto r0 = __builtin_amdgcn_permlane16_swap(x[0], y[0], false, false);
  const auto r1 = __builtin_amdgcn_permlane16_swap(x[1], y[1], false, false);
  a = __builtin_bit_cast(bf16x4_t, u32x2_t{r0[0], r1[0]});
  b = __builtin_bit_cast(bf16x4_t, u32x2_t{r0[1], r1[1]});
}
// e[j] of lane (row r, group q = l / 16) holds columns 16 j + 4 q .. +3 of row
// r (two 16-column tiles). Afterwards lane q holds columns 8 q .. 8 q + 7 of
// the 32 (e[0] then e[1]): one 16-byte store, and the 4 lanes of a row cover
// its 64 bytes contiguously.
__device__ __forceinline__ void transpose2(bf16x4_t (&e)[2]) {
  swap32(e[0], e[1]);
  swap16(e[0], e[1]);
}

// ---- host side of the persistent launches ----

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

}  // namespace
}  // namespace astrai_moe
