// Token permutation by expert (a counting sort keyed on expert id).
//
// Reference semantics (astrai/model/components/mlp.py:90-95): for each expert
// e in ascending order, (topk_idx == e).nonzero() lists the tokens routed to e
// in ascending token order and x[token_idx] gathers their rows. The permuted
// row order is the concatenation over experts, so it is fixed exactly:
// expert-major, token-ascending. Integer work only; results are bit-exact.
//
// Kernels:
//   range_sum_kernel     (histograms of more than kFusedScanInts counts, and
//                   more than kScanDirectRows chunks per scan thread) one
//                   workgroup per range of kRangeChunks token chunks: the
//                   range's per-expert counts.
//   block_prefix_kernel  (once a scan thread would walk more than
//                   kScanWalkRows ranges) grid (blocks of kBlockRanges
//                   ranges, groups of 256 experts): each range's counts become
//                   the inclusive prefix over its block, in place, so the
//                   block's last range holds the block's per-expert totals.
//   scan_kernel     one workgroup over the rows left (chunks, ranges or
//                   blocks: at most 32 rows per thread of an expert column;
//                   32 blocks at 262144 tokens and 1024 experts). Column sums
//                   give per-expert counts; a block-wide exclusive scan
//                   (wave64 shuffle scan + LDS for wave totals) gives expert
//                   offsets (the split partial sums of each expert column are
//                   scanned by wave shuffles, not walked by one thread); each
//                   row's base (its first slot in each expert's segment)
//                   replaces its counts in place; the GEMM row-tile list is
//                   laid out from the counts (tiles never straddle experts,
//                   empty experts get none; for rows of at least
//                   kGroupTilesMinDim elements each expert's whole groups of
//                   kTileGroup tiles come first and the rest after them) so
//                   no host synchronisation is needed.
//   For histograms of at most kFusedScanInts counts (every workload of the
//   benchmark: up to 512 chunks over 64 experts) none of these runs: each scatter
//   workgroup reads all chunk histograms itself (fused_bases) and workgroup
//   0 writes the offsets and the tile list, one launch instead of two.
//   scatter_kernel  grid (chunk, column split). A chunk's first slot in each
//                   expert's segment is its row's base; in block mode, its
//                   block's base plus the earlier ranges of its block (the
//                   prefix before its range); plus the histograms of the
//                   earlier chunks of its range. Wave 0 ranks the chunk's
//                   (token, slot) entries in order: lanes holding the same
//                   expert are found with one ballot per expert-id bit, the
//                   rank is the popcount of lower peer lanes, and an LDS
//                   counter per expert carries the running position (split 0
//                   writes the index outputs). Then all waves copy this
//                   split's columns of each token row once from x to its
//                   top_k destinations with 16-byte vector accesses. Column
//                   splits keep enough workgroups in flight when there are
//                   few tokens (decode).
#include <mutex>

#include "moe_common.h"

namespace astrai_moe {
namespace {

constexpr int kScanThreads = 1024;
constexpr int kScatterThreads = 256;
// Token chunks per scan range. The scan walks the chunks directly (one
// launch) while each of its threads has at most kScanDirectRows chunks to
// walk, and ranges of kRangeChunks chunks beyond that.
constexpr int kRangeChunks = 8;
constexpr int kScanDirectRows = 32;

// Per-expert counts of each range of kRangeChunks chunks:
// range_sum[r, e] = sum over the range's chunks c of chunk_hist[c, e].
__global__ __launch_bounds__(256) void range_sum_kernel(
    const int32_t* __restrict__ chunk_hist, int64_t n_chunks_, int n_experts,
    int32_t* __restrict__ range_sum) {
  const int64_t r = blockIdx.x;
  const int64_t c0 = r * kRangeChunks;
  const int64_t c1 = min(c0 + (int64_t)kRangeChunks, n_chunks_);
  for (int e = threadIdx.x; e < n_experts; e += 256) {
    int v = 0;
#pragma unroll
    for (int i = 0; i < kRangeChunks; ++i)
      if (c0 + i < c1) v += chunk_hist[(c0 + i) * n_experts + e];
    range_sum[r * n_experts + e] = v;
  }
}

// Ranges per block of the two-level scan, used once a scan thread would walk
// more than kScanWalkRows ranges of its expert column.
constexpr int kBlockRanges = 32;
constexpr int kScanWalkRows = 32;

// Memory row of scan row b when rows are blocks of `row_step` ranges: the
// block's last range (row_step = 1: row b itself).
__device__ __forceinline__ int64_t block_row(int64_t b, int64_t row_step, int64_t n_ranges) {
  return min((b + 1) * row_step, n_ranges) - 1;
}

// Tiles of an expert with `ntile` tiles that go to the grouped head of the
// tile list: its whole groups of kTileGroup when grouping, else none (the
// list is then in expert order). The GEMMs walk row tiles in groups of
// kTileGroup (so that the 32 workgroups of one XCD share operand strips in
// L2), and a group that straddles two experts needs both experts' weight
// strips.
__device__ __forceinline__ int grouped_tiles(int ntile, bool group) {
  return group ? ntile - ntile % kTileGroup : 0;
}
// Tiles j0 .. j1 - 1 of expert e (rows [row0, row_end)) at list positions
// slot0, slot0 + 1, ... (those below the capacity). An expert's tiles
// [0, npure) go to the grouped head at pure0 (the exclusive prefix of grouped
// tiles), the rest to the tail at n_pure + the earlier experts' leftover
// tiles, each part in expert order. (Two plain loops: a select per tile
// between the two places made the permutation ~2 us slower at 8 experts.)
__device__ __forceinline__ void write_expert_tiles(int32_t* tiles, int64_t capacity, int e, int row0, int row_end,
                                                   int block_m, int j0, int j1, int64_t slot0) {
  const int n = (int)min((int64_t)(j1 - j0), max(capacity - slot0, (int64_t)0));
  int32_t* t = tiles + ASTRAI_MOE_TILE_HEADER + slot0 * ASTRAI_MOE_TILE_STRIDE;
#pragma unroll 1
  for (int i = 0; i < n; ++i, t += ASTRAI_MOE_TILE_STRIDE) {
    t[0] = e;
    t[1] = row0 + (j0 + i) * block_m;
    t[2] = row_end;
  }
}

// Grid (blocks of kBlockRanges ranges, groups of 256 experts): each range's
// counts become the inclusive prefix over its block's ranges, in place, so
// the block's last range holds the block's per-expert totals.
__global__ __launch_bounds__(256) void block_prefix_kernel(int32_t* __restrict__ rb, int64_t n_ranges,
                                                           int n_experts) {
  const int e = (int)blockIdx.y * 256 + threadIdx.x;
  if (e >= n_experts) return;
  const int64_t r0 = (int64_t)blockIdx.x * kBlockRanges;
  const int64_t r1 = min(r0 + (int64_t)kBlockRanges, n_ranges);
  int v[kBlockRanges];
#pragma unroll
  for (int i = 0; i < kBlockRanges; ++i) v[i] = r0 + i < r1 ? rb[(r0 + i) * n_experts + e] : 0;
  int run = 0;
#pragma unroll
  for (int i = 0; i < kBlockRanges; ++i) {
    run += v[i];
    if (r0 + i < r1) rb[(r0 + i) * n_experts + e] = run;
  }
}

// Inclusive scan of `v` over the block (blockDim.x == kScanThreads).
__device__ int block_inclusive_scan(int v, int* s_wave) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  if (lane == 63) s_wave[wave] = v;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kScanThreads / 64 ? s_wave[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(w, off, 64);
      if (lane >= off) w += o;
    }
    if (lane < kScanThreads / 64) s_wave[lane] = w;
  }
  __syncthreads();
  const int r = v + (wave > 0 ? s_wave[wave - 1] : 0);
  __syncthreads();
  return r;
}

// Over `n_rows_` rows of per-expert counts: expert offsets, the tile list and
// each row's base (expert offset + counts of the earlier rows). Row b lies at
// memory row block_row(b, row_step, n_mem_rows) of `hist` (the totals of a
// block of row_step ranges); `base` may alias `hist`: every element is read
// before it is written, by the same thread. kBlocks = false: row_step is 1
// and row b is memory row b (no per-row index arithmetic).
template <bool kBlocks>
__global__ __launch_bounds__(kScanThreads) void scan_kernel(
    const int32_t* hist, int64_t n_rows_, int64_t row_step, int64_t n_mem_rows, int n_experts,
    int block_m, int64_t tile_capacity, bool group, int32_t* __restrict__ expert_offsets,
    int32_t* base, int32_t* __restrict__ tiles) {
  __shared__ int s_part[kScanThreads];
  __shared__ int s_wave[kScanThreads / 64];
  __shared__ int s_cnt[ASTRAI_MOE_MAX_EXPERTS];
  __shared__ int s_off[ASTRAI_MOE_MAX_EXPERTS];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // Threads form a [splits][ep] grid: ep = next_pow2(E) expert columns, each
  // column's rows split into `splits` contiguous runs.
  int ep = 1;
  while (ep < n_experts) ep *= 2;
  const int splits = kScanThreads / ep;
  const int e = threadIdx.x % ep;
  const int s = threadIdx.x / ep;
  const int64_t per = ceil_div(n_rows_, splits);
  const int64_t c0 = min((int64_t)s * per, n_rows_);
  const int64_t c1 = min(c0 + per, n_rows_);

  int local = 0;
  if (e < n_experts) {
#pragma unroll 8
    for (int64_t c = c0; c < c1; ++c) local += hist[(kBlocks ? block_row(c, row_step, n_mem_rows) : c) * n_experts + e];
  }
  s_part[threadIdx.x] = local;
  __syncthreads();

  // Exclusive prefix over the splits of each expert column, in parallel: one
  // wave per group of columns, lane l holding split (l % sl) of column
  // (l / sl) of its group; columns with more than 64 splits take several
  // passes with a carry. The column's total is its expert's count.
  {
    const int sl = splits < 64 ? splits : 64;
    const int cpw = 64 / sl;  // columns per wave
    if (wave < ep / cpw) {
      const int col = wave * cpw + lane / sl;
      const int j0 = lane % sl;
      const int seg_last = (lane / sl) * sl + sl - 1;
      int carry = 0;
      for (int jb = 0; jb < splits; jb += sl) {
        const int j = jb + j0;
        const int v = s_part[j * ep + col];
        int incl = v;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int o = __shfl_up(incl, off, 64);
          if (off < sl && j0 >= off) incl += o;
        }
        s_part[j * ep + col] = carry + incl - v;
        carry += __shfl(incl, seg_last, 64);
      }
      if (j0 == sl - 1 && col < n_experts) s_cnt[col] = carry;
    }
  }
  __syncthreads();

  // Expert offsets and tile starts: block scans over expert ids (rows,
  // tiles, tiles in whole groups; the last expert's thread publishes the
  // whole-group total, where the leftover tiles start).
  const int cnt = (threadIdx.x < n_experts) ? s_cnt[threadIdx.x] : 0;
  const int ntile = (cnt + block_m - 1) / block_m;
  const int npure = grouped_tiles(ntile, group);
  const int cnt_incl = block_inclusive_scan(cnt, s_wave);
  const int tile_incl = block_inclusive_scan(ntile, s_wave);
  const int pure_incl = block_inclusive_scan(npure, s_wave);
  __shared__ int s_npure;
  if (threadIdx.x == n_experts - 1) s_npure = pure_incl;
  __syncthreads();
  const int n_pure = s_npure;
  if (threadIdx.x < n_experts) {
    const int off = cnt_incl - cnt;
    const int tile0 = tile_incl - ntile, pure0 = pure_incl - npure;
    const int64_t left0 = (int64_t)n_pure + (tile0 - pure0);
    s_off[threadIdx.x] = off;
    expert_offsets[threadIdx.x] = off;
    if (threadIdx.x == n_experts - 1) {
      expert_offsets[n_experts] = cnt_incl;
      tiles[0] = tile_incl;
      tiles[1] = block_m;
      tiles[2] = (int32_t)tile_capacity;
      tiles[3] = group ? n_pure : tile_incl;
    }
    // the expert's row tiles (stores only: nothing waits on them)
    write_expert_tiles(tiles, tile_capacity, threadIdx.x, off, off + cnt, block_m, 0, npure, pure0);
    write_expert_tiles(tiles, tile_capacity, threadIdx.x, off, off + cnt, block_m, npure, ntile, left0);
  }
  __syncthreads();

  // Row bases: expert offset + tokens of that expert in earlier rows.
  if (e < n_experts) {
    int run = s_off[e] + s_part[threadIdx.x];
#pragma unroll 8
    for (int64_t c = c0; c < c1; ++c) {
      const int64_t m = kBlocks ? block_row(c, row_step, n_mem_rows) : c;
      const int v = hist[m * n_experts + e];
      base[m * n_experts + e] = run;
      run += v;
    }
  }
}

// Exclusive prefix sums over the block (blockDim.x == kScatterThreads) of N
// values per thread at once (each thread holding the sums of its own run),
// and their block totals. s_wave holds N * kScatterThreads / 64 ints.
template <int N>
__device__ void scatter_block_exclusive_scan(int (&v)[N], int* s_wave, int (&total)[N]) {
  constexpr int kW = kScatterThreads / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int inc[N];
#pragma unroll
  for (int i = 0; i < N; ++i) inc[i] = v[i];
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int o = __shfl_up(inc[i], off, 64);
      if (lane >= off) inc[i] += o;
    }
  }
  if (lane == 63) {
#pragma unroll
    for (int i = 0; i < N; ++i) s_wave[i * kW + wave] = inc[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    int before = 0;
    total[i] = 0;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      const int t = s_wave[i * kW + w];
      if (w < wave) before += t;
      total[i] += t;
    }
    v[i] = before + inc[i] - v[i];
  }
}


// The scan folded into the scatter, for histograms of at most
// kFusedScanInts counts: every workgroup reads all chunk histograms, V
// experts per load, and forms each expert's total and its count in the
// chunks before this one; an exclusive scan of the totals gives the expert
// offsets, and cnt[e] = offset + earlier count is the chunk's first slot in
// expert e's segment. Workgroup (0, 0) also writes the expert offsets and
// the GEMM tile list (as scan_kernel does). Replaces a one-workgroup launch
// whose fixed cost (~5 us) exceeded its work at these sizes.
constexpr int kFusedScanInts = 32768;

template <int V>
__device__ void fused_bases(const int32_t* __restrict__ chunk_hist, int64_t nc, int n_experts, int64_t chunk,
                            int block_m, int64_t tile_capacity, bool group, int32_t* __restrict__ expert_offsets,
                            int32_t* __restrict__ tiles, int* cnt, int* s_tot, int* s_wave) {
  const int t = threadIdx.x;
  const int cw = n_experts / V;  // V divides n_experts
  const int R = cw >= kScatterThreads ? 1 : kScatterThreads / cw;
  typedef int vint __attribute__((ext_vector_type(V)));
  // partial column sums: thread (g, col) takes rows g, g + R, ... of its column(s)
  if (t < R * cw || cw >= kScatterThreads) {
    for (int col = cw >= kScatterThreads ? t : t % cw; col < cw; col += kScatterThreads) {
      const int g = cw >= kScatterThreads ? 0 : t / cw;
      vint tot = 0, pre = 0;
#pragma unroll 16
      for (int64_t c = g; c < nc; c += R) {
        const vint h = *reinterpret_cast<const vint*>(chunk_hist + c * n_experts + col * V);
        tot += h;
        if (c < chunk) pre += h;
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        s_tot[g * n_experts + col * V + v] = tot[v];
        s_tot[(R + g) * n_experts + col * V + v] = pre[v];
      }
      if (cw < kScatterThreads) break;
    }
  }
  __syncthreads();
  // fold the R partial rows into row 0 as a tree (few experts leave R up to
  // 256: summed by one thread per expert, the rows took ~15 us)
  if (R > 1) {
    int half = 1;
    while (2 * half < R) half *= 2;
    const int g = t / cw, col = t % cw;
    for (int live = R; half > 0; live = half, half /= 2) {
      if (g < half && g + half < live) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          s_tot[g * n_experts + col * V + v] += s_tot[(g + half) * n_experts + col * V + v];
          s_tot[(R + g) * n_experts + col * V + v] += s_tot[(R + g + half) * n_experts + col * V + v];
        }
      }
      __syncthreads();
    }
  }
  // per expert: total and earlier count; thread t holds experts 4 t .. 4 t + 3
  int tot4[4], pre4[4], run = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * t + j;
    tot4[j] = pre4[j] = 0;
    if (e < n_experts) tot4[j] = s_tot[e], pre4[j] = s_tot[R * n_experts + e];
    run += tot4[j];
  }
  const bool write_list = blockIdx.x == 0 && blockIdx.y == 0;
  int ntile_run = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) ntile_run += (tot4[j] + block_m - 1) / block_m;
  // exclusive prefixes over experts of rows and tiles
  int pre[2] = {run, ntile_run}, tot[2];
  scatter_block_exclusive_scan<2>(pre, s_wave, tot);
  int off = pre[0], tile0 = pre[1];
  const int n_rows = tot[0], n_tiles = tot[1];
  // and of the tiles in whole groups, for the workgroup that writes the list
  // (uniform over the workgroup: its barriers are safe)
  int pure0 = 0, n_pure = 0;
  if (write_list && group) {
    int pure[1] = {0}, pure_tot[1];
#pragma unroll
    for (int j = 0; j < 4; ++j) pure[0] += grouped_tiles((tot4[j] + block_m - 1) / block_m, true);
    __syncthreads();  // the previous scan's reads of s_wave are done
    scatter_block_exclusive_scan<1>(pure, s_wave, pure_tot);
    pure0 = pure[0], n_pure = pure_tot[0];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * t + j;
    if (e < n_experts) {
      cnt[e] = off + pre4[j];
      if (write_list) {
        expert_offsets[e] = off;
        const int ntile = (tot4[j] + block_m - 1) / block_m;
        const int npure = grouped_tiles(ntile, group);
        write_expert_tiles(tiles, tile_capacity, e, off, off + tot4[j], block_m, 0, npure, pure0);
        write_expert_tiles(tiles, tile_capacity, e, off, off + tot4[j], block_m, npure, ntile,
                           n_pure + (tile0 - pure0));
        tile0 += ntile;
        pure0 += npure;
      }
      off += tot4[j];
    }
  }
  if (write_list && t == 0) {
    expert_offsets[n_experts] = n_rows;
    tiles[0] = n_tiles;
    tiles[1] = block_m;
    tiles[2] = (int32_t)tile_capacity;
    tiles[3] = group ? n_pure : n_tiles;
  }
  __syncthreads();
}

// kFusedV > 0: the scan is folded in (fused_bases, kFusedV experts per
// load); range_base, range_chunks, n_ranges and block_ranges are then unused.
template <typename T, bool kVec, int kFusedV = 0>
__global__ __launch_bounds__(kScatterThreads) void scatter_kernel(
    const int32_t* __restrict__ topk_idx, const T* __restrict__ topk_w,
    const int32_t* __restrict__ chunk_hist, const int32_t* __restrict__ range_base,
    int range_chunks, int64_t n_ranges, int block_ranges, const T* __restrict__ x,
    int64_t n_tokens, int n_experts, int top_k, int64_t dim,
    int32_t* __restrict__ sorted_token, T* __restrict__ sorted_w,
    int32_t* __restrict__ token_pos, T* __restrict__ x_perm,
    int block_m, int64_t tile_capacity, int32_t* __restrict__ expert_offsets,
    int32_t* __restrict__ tiles) {
  __shared__ int cnt[ASTRAI_MOE_MAX_EXPERTS];
  const bool write_index = blockIdx.y == 0;
  __shared__ int pos_l[ASTRAI_MOE_CHUNK_TOKENS * ASTRAI_MOE_MAX_TOPK];
  const int64_t chunk = blockIdx.x;
  const int64_t t0 = chunk * ASTRAI_MOE_CHUNK_TOKENS;
  const int nt = (int)min((int64_t)ASTRAI_MOE_CHUNK_TOKENS, n_tokens - t0);
  const int n_ent = nt * top_k;
  const int64_t n_rows = n_tokens * top_k;
  // The chunk's routing entries are loaded first, so that their latency
  // overlaps that of the expert bases below; they reach LDS afterwards.
  constexpr int kEnt = ASTRAI_MOE_CHUNK_TOKENS * ASTRAI_MOE_MAX_TOPK;
  constexpr int kEntPerThread = kEnt / kScatterThreads;
  static_assert(kEnt % kScatterThreads == 0, "entries per thread");
  __shared__ int s_e[kEnt];
  __shared__ T s_w[kEnt];
  int pe[kEntPerThread];
  T pw[kEntPerThread];
#pragma unroll
  for (int j = 0; j < kEntPerThread; ++j) {
    const int i = threadIdx.x + j * kScatterThreads;
    pe[j] = i < n_ent ? topk_idx[t0 * top_k + i] : -1;
    pw[j] = (i < n_ent && write_index) ? topk_w[t0 * top_k + i] : T(0);
  }
  if constexpr (kFusedV > 0) {
    __shared__ int s_tot[2 * 4 * kScatterThreads];
    __shared__ int s_wave[2 * kScatterThreads / 64];
    fused_bases<kFusedV>(chunk_hist, (int64_t)gridDim.x, n_experts, chunk, block_m, tile_capacity,
                         dim >= kGroupTilesMinDim, expert_offsets,
                         tiles, cnt, s_tot, s_wave);
  } else {
    // the chunk's first slot per expert: its range's base plus the earlier
    // chunks of the range. With blocks of ranges (block_ranges > 0) the
    // range's base is its block's base (held in the block's last range) plus
    // the earlier ranges of its block (the inclusive prefix of the range
    // before it).
    const int64_t r = chunk / range_chunks;
    const int64_t blk0 = block_ranges > 0 ? r / block_ranges * block_ranges : r;
    const int64_t brow = block_ranges > 0 ? block_row(r / block_ranges, block_ranges, n_ranges) : r;
    for (int e = threadIdx.x; e < n_experts; e += kScatterThreads) {
      int b = range_base[brow * n_experts + e];
      if (r > blk0) b += range_base[(r - 1) * n_experts + e];
      for (int64_t c = r * range_chunks; c < chunk; ++c) b += chunk_hist[c * n_experts + e];
      cnt[e] = b;
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < kEntPerThread; ++j) {
    const int i = threadIdx.x + j * kScatterThreads;
    if (i < n_ent) s_e[i] = pe[j], s_w[i] = pw[j];
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  if (threadIdx.x < 64) {
    int nbits = 0;
    while ((1 << nbits) < n_experts) ++nbits;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int base = 0; base < n_ent; base += 64) {
      const int i = base + lane;
      int e = i < n_ent ? s_e[i] : -1;
      const bool valid = e >= 0 && e < n_experts;
      uint64_t peers = __ballot(valid);
      for (int b = 0; b < nbits; ++b) {
        const bool bit = valid && ((e >> b) & 1);
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
      }
      const int rank = __popcll(peers & lt_mask);
      const int p = valid ? cnt[e] + rank : -1;
      // All reads of cnt above complete before any update below (in-order
      // LDS queue of one wave); the highest peer lane advances the counter.
      const bool last = valid && (peers >> lane) == 1ull;
      if (last) cnt[e] += __popcll(peers);
      if (i < n_ent) {
        const bool ok = valid && p >= 0 && p < n_rows;
        pos_l[i] = ok ? p : -1;
        if (write_index) {
          token_pos[t0 * top_k + i] = ok ? p : -1;
          if (ok) {
            sorted_token[p] = (int32_t)(t0 + i / top_k);
            sorted_w[p] = s_w[i];
          }
        }
      }
    }
  }
  __syncthreads();
  if (x_perm == nullptr) return;  // index outputs only (the GEMM gathers the rows itself)

  // Row copy: each token row is read once and written top_k times.
  const int wave = threadIdx.x >> 6;
  constexpr int kWaves = kScatterThreads / 64;
  const int64_t nunits = kVec ? dim * (int64_t)sizeof(T) / 16 : dim;  // 16-byte vectors or elements
  const int64_t u0 = nunits * blockIdx.y / gridDim.y;
  const int64_t u1 = nunits * (blockIdx.y + 1) / gridDim.y;
  if (kVec) {
    // 16-byte vectors; dim * sizeof(T) is a multiple of 16.
    for (int lt = wave; lt < nt; lt += kWaves) {
      const uint4* src = reinterpret_cast<const uint4*>(x + (t0 + lt) * dim);
      for (int64_t v = u0 + lane; v < u1; v += 64) {
        const uint4 val = src[v];
        for (int k = 0; k < top_k; ++k) {
          const int p = pos_l[lt * top_k + k];
          if (p >= 0) reinterpret_cast<uint4*>(x_perm + (int64_t)p * dim)[v] = val;
        }
      }
    }
  } else {
    for (int lt = wave; lt < nt; lt += kWaves) {
      const T* src = x + (t0 + lt) * dim;
      for (int64_t c = u0 + lane; c < u1; c += 64) {
        const T val = src[c];
        for (int k = 0; k < top_k; ++k) {
          const int p = pos_l[lt * top_k + k];
          if (p >= 0) x_perm[(int64_t)p * dim + c] = val;
        }
      }
    }
  }
}

// Tile list of one dense expert over n_rows rows (expert 0 owns every row),
// for running the shared experts and the standalone MLP on the grouped GEMMs;
// optionally the matching expert offsets {0, n_rows}. Built on the device so
// that a captured graph owns it like any other output of the forward.
__global__ __launch_bounds__(256) void dense_tiles_kernel(
    int64_t n_rows, int block_m, int64_t tile_capacity,
    int32_t* __restrict__ tiles, int32_t* __restrict__ offsets) {
  const int64_t n_tiles = ceil_div(n_rows, block_m);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i == 0) {
    tiles[0] = (int32_t)n_tiles;
    tiles[1] = block_m;
    tiles[2] = (int32_t)tile_capacity;
    tiles[3] = (int32_t)(n_tiles - n_tiles % kTileGroup);  // one expert: whole groups first already
    if (offsets != nullptr) {
      offsets[0] = 0;
      offsets[1] = (int32_t)n_rows;
    }
  }
  if (i < n_tiles) {
    int32_t* t = tiles + ASTRAI_MOE_TILE_HEADER + i * ASTRAI_MOE_TILE_STRIDE;
    t[0] = 0;
    t[1] = (int32_t)(i * block_m);
    t[2] = (int32_t)n_rows;
  }
}

// Chunks per row of the scan: ranges of kRangeChunks chunks (their counts
// summed into the scratch first, then scanned in place) when each scan thread
// would otherwise walk more than kScanDirectRows chunks, else the chunks.
int scan_range_chunks(int64_t n_tokens, int n_experts) {
  int ep = 1;
  while (ep < n_experts) ep *= 2;
  const int64_t rows_per_thread = ceil_div(n_chunks(n_tokens), kScanThreads / ep);
  return rows_per_thread > kScanDirectRows ? kRangeChunks : 1;
}

// int32 elements of scratch the permutation uses: one row of expert bases per
// scan row (at most n_chunks * n_experts).
int64_t permute_scratch_ints(int64_t n_tokens, int n_experts) {
  return ceil_div(n_chunks(n_tokens), scan_range_chunks(n_tokens, n_experts)) * n_experts;
}

template <typename T, bool kVec, int kFusedV>
void launch_scatter(dim3 grid, hipStream_t s, const int32_t* topk_idx, const void* topk_w, const int32_t* chunk_hist,
                    const int32_t* range_base, int range_chunks, int64_t n_ranges, int block_ranges, const void* x,
                    int64_t n_tokens, int n_experts,
                    int top_k, int64_t dim, int32_t* sorted_token, void* sorted_w, int32_t* token_pos, void* x_perm,
                    int block_m, int64_t tile_capacity, int32_t* expert_offsets, int32_t* tiles) {
  hipLaunchKernelGGL((scatter_kernel<T, kVec, kFusedV>), grid, dim3(kScatterThreads), 0, s, topk_idx,
                     static_cast<const T*>(topk_w), chunk_hist, range_base, range_chunks, n_ranges, block_ranges,
                     static_cast<const T*>(x),
                     n_tokens, n_experts, top_k, dim, sorted_token, static_cast<T*>(sorted_w), token_pos,
                     static_cast<T*>(x_perm), block_m, tile_capacity, expert_offsets, tiles);
}

template <typename T>
int launch_permute(const int32_t* topk_idx, const void* topk_w,
                   const int32_t* chunk_hist, const void* x, int64_t n_tokens,
                   int n_experts, int top_k, int64_t dim, int block_m,
                   int32_t* expert_offsets, int32_t* sorted_token,
                   void* sorted_w, int32_t* token_pos, void* x_perm,
                   int32_t* tiles, int64_t tile_capacity, int32_t* chunk_base,
                   hipStream_t s) {
  const int64_t nc = n_chunks(n_tokens);
  // small histograms: the scan is folded into the scatter (fused_bases)
  const bool fused = nc > 0 && nc * n_experts <= kFusedScanInts;
  const int range_chunks = fused ? 1 : scan_range_chunks(n_tokens, n_experts);
  const int64_t n_ranges = ceil_div(nc, range_chunks);
  int32_t* range_base = chunk_base;  // n_ranges * n_experts <= n_chunks * n_experts
  int rc = ASTRAI_MOE_OK;
  int block_ranges = 0;
  if (!fused) {
    if (range_chunks > 1) {
      hipLaunchKernelGGL(range_sum_kernel, dim3((unsigned)n_ranges), dim3(256), 0, s,
                         chunk_hist, nc, n_experts, range_base);
      if ((rc = check_launch("range_sum_kernel"))) return rc;
    }
    // two levels once a scan thread would walk more than kScanWalkRows rows
    int ep = 1;
    while (ep < n_experts) ep *= 2;
    int64_t scan_rows = n_ranges, row_step = 1;
    if (range_chunks > 1 && ceil_div(n_ranges, std::max(1, kScanThreads / ep)) > kScanWalkRows) {
      block_ranges = kBlockRanges;
      scan_rows = ceil_div(n_ranges, (int64_t)kBlockRanges);
      row_step = kBlockRanges;
      hipLaunchKernelGGL(block_prefix_kernel, dim3((unsigned)scan_rows, (unsigned)ceil_div(n_experts, 256)),
                         dim3(256), 0, s, range_base, n_ranges, n_experts);
      if ((rc = check_launch("block_prefix_kernel"))) return rc;
    }
    hipLaunchKernelGGL(block_ranges > 0 ? scan_kernel<true> : scan_kernel<false>, dim3(1), dim3(kScanThreads), 0, s,
                       range_chunks > 1 || block_ranges > 0 ? range_base : chunk_hist, scan_rows, row_step,
                       n_ranges, n_experts, block_m, tile_capacity, dim >= kGroupTilesMinDim, expert_offsets,
                       range_base, tiles);
    rc = check_launch("scan_kernel");
    if (rc || nc == 0) return rc;
  }
  const bool vec = (dim * (int64_t)sizeof(T)) % 16 == 0 &&
                   (reinterpret_cast<uintptr_t>(x) % 16) == 0 &&
                   (reinterpret_cast<uintptr_t>(x_perm) % 16) == 0;
  // Column splits: aim for >= 512 workgroups, each split >= 64 units wide.
  const int64_t nunits = vec ? dim * (int64_t)sizeof(T) / 16 : dim;
  int64_t splits = ceil_div(512, nc);
  if (splits > nunits / 64) splits = nunits / 64;
  if (splits < 1 || x_perm == nullptr) splits = 1;
  if (splits > 65535) splits = 65535;
  const dim3 grid((unsigned)nc, (unsigned)splits);
  // the fused scan reads 16-byte vectors of 4 experts where rows allow it
  const bool v4 = n_experts % 4 == 0 && reinterpret_cast<uintptr_t>(chunk_hist) % 16 == 0;
#define ASTRAI_SCATTER(VEC, FV)                                                                                       \
  launch_scatter<T, VEC, FV>(grid, s, topk_idx, topk_w, chunk_hist, range_base, range_chunks, n_ranges,            \
                             block_ranges, x, n_tokens, n_experts,                                                   \
                             top_k, dim, sorted_token, sorted_w, token_pos, x_perm, block_m, tile_capacity,          \
                             expert_offsets, tiles)
  if (!fused) {
    if (vec) ASTRAI_SCATTER(true, 0); else ASTRAI_SCATTER(false, 0);
  } else if (v4) {
    if (vec) ASTRAI_SCATTER(true, 4); else ASTRAI_SCATTER(false, 4);
  } else {
    if (vec) ASTRAI_SCATTER(true, 1); else ASTRAI_SCATTER(false, 1);
  }
#undef ASTRAI_SCATTER
  return check_launch("scatter_kernel");
}

}  // namespace
}  // namespace astrai_moe

using namespace astrai_moe;

extern "C" int64_t astrai_moe_tile_list_len(int64_t n_tokens, int n_experts,
                                            int top_k, int block_m) {
  if (n_tokens < 0 || n_experts < 1 || top_k < 1 || block_m < 1) return -1;
  const int64_t rows = n_tokens * top_k;
  int64_t cap = (rows + (int64_t)n_experts * (block_m - 1)) / block_m;
  if (cap > rows) cap = rows;
  return ASTRAI_MOE_TILE_HEADER + cap * ASTRAI_MOE_TILE_STRIDE;
}

// Scratch of astrai_moe_permute_noalloc: the scan's per-row expert bases
// (permute_scratch_ints) live here instead of in a caller-provided buffer.
// Every GPU the library runs on holds its own copy until the process ends.
// Nothing in it has to start at zero: the scan writes every element it later
// reads. Calls that overlap on one GPU (two streams, two host threads) share
// it and race.
static __device__ __align__(256) int32_t scratch[ASTRAI_MOE_NOALLOC_SCRATCH_INTS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
int32_t* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device. In host code the
// array's name is a host-side stand-in, never a device address: the address
// comes from hipGetSymbolAddress, once per device with that device current,
// and is used wherever host code needs the array (kernel arguments).
int noalloc_scratch(int32_t** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return fail(ASTRAI_MOE_ELAUNCH, "permute_noalloc: hipGetDevice: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(ASTRAI_MOE_EINVAL, "permute_noalloc: device %d beyond the %d this build tracks", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr)
      return fail(ASTRAI_MOE_ELAUNCH, "permute_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(err));
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return ASTRAI_MOE_OK;
}
}  // namespace

static int permute_impl(const char* who,
    const int32_t* topk_idx, const void* topk_w, const int32_t* chunk_hist,
    const void* x, int dtype, int64_t n_tokens, int n_experts, int top_k,
    int64_t dim, int block_m, int32_t* expert_offsets, int32_t* sorted_token,
    void* sorted_w, int32_t* token_pos, void* x_perm, int32_t* tiles,
    int64_t tiles_len, int32_t* chunk_base, bool noalloc, void* stream) {
  ASTRAI_REQUIRE(n_tokens >= 0 && n_tokens * (int64_t)top_k < (1ll << 31),
                 "%s: n_tokens * top_k must be in [0, 2^31) (got %lld)", who,
                 (long long)(n_tokens * (int64_t)top_k));
  ASTRAI_REQUIRE(n_experts >= 1 && n_experts <= ASTRAI_MOE_MAX_EXPERTS,
                 "%s: n_experts must be in [1, %d] (got %d)", who,
                 ASTRAI_MOE_MAX_EXPERTS, n_experts);
  ASTRAI_REQUIRE(top_k >= 1 && top_k <= n_experts && top_k <= ASTRAI_MOE_MAX_TOPK,
                 "%s: top_k must be in [1, min(n_experts, %d)] (got %d)", who,
                 ASTRAI_MOE_MAX_TOPK, top_k);
  ASTRAI_REQUIRE(dim >= 1, "%s: dim must be >= 1", who);
  ASTRAI_REQUIRE(block_m >= 1, "%s: block_m must be >= 1", who);
  const int64_t need = astrai_moe_tile_list_len(n_tokens, n_experts, top_k, block_m);
  ASTRAI_REQUIRE(tiles_len >= need,
                 "%s: tile list holds %lld int32, needs %lld", who,
                 (long long)tiles_len, (long long)need);
  ASTRAI_REQUIRE(topk_idx && topk_w && chunk_hist && (x || !x_perm) &&
                     expert_offsets && sorted_token && sorted_w && token_pos &&
                     tiles && (chunk_base || noalloc),
                 "%s: null buffer", who);
  if (noalloc) {
    // checked before any HIP call: a problem too large for the library's
    // scratch is refused without touching the device
    const int64_t need_scratch = permute_scratch_ints(n_tokens, n_experts);
    ASTRAI_REQUIRE(need_scratch <= ASTRAI_MOE_NOALLOC_SCRATCH_INTS,
                   "%s: %lld tokens over %d experts need %lld int32 of scratch, "
                   "the library's scratch holds %d (use astrai_moe_permute with a "
                   "caller-provided chunk_base)",
                   who, (long long)n_tokens, n_experts, (long long)need_scratch,
                   ASTRAI_MOE_NOALLOC_SCRATCH_INTS);
    if (int rc = noalloc_scratch(&chunk_base)) return rc;
  }
  const int64_t capacity =
      (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == ASTRAI_MOE_BF16)
    return launch_permute<bf16_t>(topk_idx, topk_w, chunk_hist, x, n_tokens,
                                  n_experts, top_k, dim, block_m, expert_offsets,
                                  sorted_token, sorted_w, token_pos, x_perm, tiles,
                                  capacity, chunk_base, s);
  if (dtype == ASTRAI_MOE_F32)
    return launch_permute<float>(topk_idx, topk_w, chunk_hist, x, n_tokens,
                                 n_experts, top_k, dim, block_m, expert_offsets,
                                 sorted_token, sorted_w, token_pos, x_perm, tiles,
                                 capacity, chunk_base, s);
  return fail(ASTRAI_MOE_EINVAL, "%s: unsupported dtype %d", who, dtype);
}

extern "C" int astrai_moe_permute(
    const int32_t* topk_idx, const void* topk_w, const int32_t* chunk_hist,
    const void* x, int dtype, int64_t n_tokens, int n_experts, int top_k,
    int64_t dim, int block_m, int32_t* expert_offsets, int32_t* sorted_token,
    void* sorted_w, int32_t* token_pos, void* x_perm, int32_t* tiles,
    int64_t tiles_len, int32_t* chunk_base, void* stream) {
  clear_error();
  return permute_impl("permute", topk_idx, topk_w, chunk_hist, x, dtype,
                      n_tokens, n_experts, top_k, dim, block_m, expert_offsets,
                      sorted_token, sorted_w, token_pos, x_perm, tiles,
                      tiles_len, chunk_base, false, stream);
}

extern "C" int astrai_moe_permute_noalloc(
    const int32_t* topk_idx, const void* topk_w, const int32_t* chunk_hist,
    const void* x, int dtype, int64_t n_tokens, int n_experts, int top_k,
    int64_t dim, int block_m, int32_t* expert_offsets, int32_t* sorted_token,
    void* sorted_w, int32_t* token_pos, void* x_perm, int32_t* tiles,
    int64_t tiles_len, void* stream) {
  clear_error();
  return permute_impl("permute_noalloc", topk_idx, topk_w, chunk_hist, x,
                      dtype, n_tokens, n_experts, top_k, dim, block_m,
                      expert_offsets, sorted_token, sorted_w, token_pos,
                      x_perm, tiles, tiles_len, nullptr, true, stream);
}

extern "C" int astrai_moe_dense_tiles(int64_t n_rows, int block_m,
                                      int32_t* tiles, int64_t tiles_len,
                                      int32_t* expert_offsets, void* stream) {
  clear_error();
  ASTRAI_REQUIRE(n_rows >= 0 && n_rows < (1ll << 31),
                 "dense_tiles: n_rows must be in [0, 2^31) (got %lld)",
                 (long long)n_rows);
  ASTRAI_REQUIRE(block_m >= 1, "dense_tiles: block_m must be >= 1");
  const int64_t need = astrai_moe_tile_list_len(n_rows, 1, 1, block_m);
  ASTRAI_REQUIRE(tiles_len >= need,
                 "dense_tiles: tile list holds %lld int32, needs %lld",
                 (long long)tiles_len, (long long)need);
  ASTRAI_REQUIRE(tiles != nullptr, "dense_tiles: null tile list");
  const int64_t capacity =
      (tiles_len - ASTRAI_MOE_TILE_HEADER) / ASTRAI_MOE_TILE_STRIDE;
  const int64_t n_tiles = ceil_div(n_rows, block_m);
  const int64_t grid = n_tiles > 0 ? ceil_div(n_tiles, 256) : 1;
  hipLaunchKernelGGL(dense_tiles_kernel, dim3((unsigned)grid), dim3(256), 0,
                     static_cast<hipStream_t>(stream), n_rows, block_m,
                     capacity, tiles, expert_offsets);
  return check_launch("dense_tiles_kernel");
}
