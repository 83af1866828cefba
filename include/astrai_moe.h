/*
 * astrai_moe.h — C ABI of the MI355X (gfx950) MoE expert-forward library
 * (libastrai_moe.so).
 *
 * The library replaces the routed-expert body of AstrAI's DeepSeekMoE layer,
 * astrai/model/components/mlp.py:79-100, and the combine at mlp.py:71.
 * The reference has no native code for this path: the replaced "interface" is
 * the sequence of torch calls in mlp.py, and each entry point below names the
 * lines it stands in for.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers (HBM) unless stated; sizes are elements.
 *   - Row-major, contiguous tensors. Expert weights keep the reference's
 *     nn.Linear layout [out_features, in_features] (astrai/model/components/
 *     linear.py:12) and are passed as device arrays of per-expert pointers,
 *     so the module's parameters are used in place.
 *   - dtype selects the element type of every floating-point tensor of the
 *     call: ASTRAI_MOE_F32 or ASTRAI_MOE_BF16 (bf16 stored as uint16 bits).
 *   - Work is enqueued on `stream` (a hipStream_t); nothing synchronises the
 *     host and nothing allocates device memory.
 *   - Return 0 on success, a negative ASTRAI_MOE_E* code on failure;
 *     astrai_moe_last_error() then describes the failure (per host thread).
 *   - Entry points keep no state between calls and are re-entrant; calls on
 *     different streams may run concurrently if their buffers are disjoint.
 */
#ifndef ASTRAI_MOE_H
#define ASTRAI_MOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ASTRAI_MOE_ABI_VERSION 10

/* Element types. */
#define ASTRAI_MOE_F32 0
#define ASTRAI_MOE_BF16 1

/* Status codes. */
#define ASTRAI_MOE_OK 0
#define ASTRAI_MOE_EINVAL (-1)  /* bad argument (null pointer, size, dtype) */
#define ASTRAI_MOE_ELAUNCH (-2) /* HIP reported an error at launch */

/* Tokens per routing chunk: astrai_moe_route writes one expert histogram
 * row per chunk of this many tokens, and astrai_moe_permute ranks tokens
 * chunk by chunk. */
#define ASTRAI_MOE_CHUNK_TOKENS 32

/* Limits of this build. */
#define ASTRAI_MOE_MAX_EXPERTS 1024
#define ASTRAI_MOE_MAX_TOPK 32

/* Layout of the tile list written by astrai_moe_permute and read by the two
 * grouped GEMMs (int32):
 *   tiles[0] = number of row tiles (device-written)
 *   tiles[1] = block_m (rows per tile)
 *   tiles[2] = capacity (max tiles the array holds)
 *   tiles[3] = first tile of the list's tail (see below)
 *   then per tile i: tiles[4+3i] = expert, tiles[5+3i] = first permuted row,
 *                    tiles[6+3i] = end of that expert's rows (exclusive).
 * Tiles never straddle experts, so an expert with M rows has ceil(M/block_m)
 * tiles and an expert with no rows has none. Order: for dim >= 3072, each
 * expert's first 8 * floor(n/8) tiles (n = its tile count) in expert order,
 * then, as the tail, every expert's remaining tiles in expert order (the
 * GEMMs walk row tiles in groups of 8, so that a group holds one expert's
 * tiles); tiles[3] = the number of grouped tiles. For narrower rows the
 * tiles are in expert order and tiles[3] = the tile count (no tail). The
 * 256-row GEMM kernels let padding-only waves of tiles with 48 or more K
 * steps idle only in the tail. Any order and any tiles[3] are valid inputs
 * to the GEMMs: results do not depend on them. */
#define ASTRAI_MOE_TILE_HEADER 4
#define ASTRAI_MOE_TILE_STRIDE 3

/* ABI version of the loaded library (ASTRAI_MOE_ABI_VERSION at build time). */
int astrai_moe_abi_version(void);

/* Message for the last failed call on this host thread ("" if none). */
const char* astrai_moe_last_error(void);

/* Rows per GEMM tile that the library will use for this problem. Host-side
 * policy only; no device work. Returns a positive value or a negative code. */
int astrai_moe_select_block_m(int64_t n_tokens, int n_experts, int top_k,
                              int64_t dim, int64_t dim_ffn, int dtype);

/* Number of int32 elements the tile list needs (header included). */
int64_t astrai_moe_tile_list_len(int64_t n_tokens, int n_experts, int top_k,
                                 int block_m);

/*
 * Router softmax, top-k and renormalisation.
 * Replaces mlp.py:84 (softmax(logits.float()).to(dtype)), mlp.py:86
 * (torch.topk(probs, K), largest, sorted) and mlp.py:87 (w / w.sum(-1)).
 * The router GEMM itself (mlp.py:83) stays with the caller.
 *
 *   logits     [n_tokens, n_experts]  dtype
 *   topk_idx   [n_tokens, top_k]      int32, experts by descending
 *                                     probability (ties: lower expert first)
 *   topk_w     [n_tokens, top_k]      dtype, renormalised weights
 *   chunk_hist [ceil(n_tokens/ASTRAI_MOE_CHUNK_TOKENS), n_experts] int32,
 *              routed-token count of every expert within each token chunk
 */
int astrai_moe_route(const void* logits, int dtype, int64_t n_tokens,
                     int n_experts, int top_k, int32_t* topk_idx,
                     void* topk_w, int32_t* chunk_hist, void* stream);

/*
 * Token permutation by expert.
 * Replaces mlp.py:90-95: for e = 0..E-1, (topk_idx == e).nonzero() gives the
 * tokens routed to e in ascending order, and x[token_idx] gathers their rows.
 * The permuted order is that concatenation: expert-major, token-ascending.
 *
 *   topk_idx, topk_w, chunk_hist   as written by astrai_moe_route
 *   x              [n_tokens, dim]       dtype
 *   expert_offsets [n_experts + 1]       int32, exclusive scan of counts
 *   sorted_token   [n_tokens * top_k]    int32, source token of each row
 *   sorted_w       [n_tokens * top_k]    dtype, routing weight of each row
 *   token_pos      [n_tokens * top_k]    int32, row of (token, slot)
 *   x_perm         [n_tokens * top_k, dim] dtype, x[sorted_token]; may be NULL:
 *                  then only the index outputs are written (and x may be NULL
 *                  too), for astrai_moe_gemm_gate_up_gather, which reads the
 *                  token rows of x itself
 *   tiles          astrai_moe_tile_list_len(...) int32, see layout above
 *   chunk_base     [n_chunks, n_experts] int32 scratch
 */
int astrai_moe_permute(const int32_t* topk_idx, const void* topk_w,
                       const int32_t* chunk_hist, const void* x, int dtype,
                       int64_t n_tokens, int n_experts, int top_k, int64_t dim,
                       int block_m, int32_t* expert_offsets,
                       int32_t* sorted_token, void* sorted_w,
                       int32_t* token_pos, void* x_perm, int32_t* tiles,
                       int64_t tiles_len, int32_t* chunk_base, void* stream);

/*
 * astrai_moe_permute without the chunk_base workspace, for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference.
 * Same arguments, results (bit-identical) and errors as astrai_moe_permute,
 * minus chunk_base: the scan's scratch is a fixed array inside the library,
 * ASTRAI_MOE_NOALLOC_SCRATCH_INTS int32 per GPU, held from the first call on
 * a GPU until the process ends. The call allocates nothing; the caller still
 * provides every output.
 *
 * Limit: n_experts * ceil(n_chunks / r) int32 must fit the scratch, with
 * n_chunks = ceil(n_tokens / ASTRAI_MOE_CHUNK_TOKENS) and r = 1, or r = 8 when
 * n_chunks exceeds 32 * (1024 / next_pow2(n_experts)): e.g. 262144 tokens over
 * 1024 experts, or 4 M tokens over 64. Larger problems return
 * ASTRAI_MOE_EINVAL before any device work.
 * Calls on one GPU share the scratch: calls that overlap (two streams, two
 * host threads) race and must be serialised by the caller. Nothing in the
 * scratch needs clearing between calls.
 */
#define ASTRAI_MOE_NOALLOC_SCRATCH_INTS (1 << 20)
int astrai_moe_permute_noalloc(const int32_t* topk_idx, const void* topk_w,
                               const int32_t* chunk_hist, const void* x,
                               int dtype, int64_t n_tokens, int n_experts,
                               int top_k, int64_t dim, int block_m,
                               int32_t* expert_offsets, int32_t* sorted_token,
                               void* sorted_w, int32_t* token_pos,
                               void* x_perm, int32_t* tiles, int64_t tiles_len,
                               void* stream);

/*
 * Tile list of one dense expert over n_rows rows: every row belongs to expert
 * 0, in ceil(n_rows / block_m) row tiles (layout above), and, when
 * expert_offsets is not NULL, its offsets {0, n_rows} (int32[2]). With
 * one-entry weight tables and no row weights (sorted_w = NULL) the grouped
 * GEMMs then compute mlp.py:22-25, MLP.forward, over all rows: the shared
 * experts of mlp.py:74-77 and the standalone MLP. Written on the device, so a
 * caller that captures its forward in a graph captures the list with it.
 *
 *   tiles  astrai_moe_tile_list_len(n_rows, 1, 1, block_m) int32
 */
int astrai_moe_dense_tiles(int64_t n_rows, int block_m, int32_t* tiles,
                           int64_t tiles_len, int32_t* expert_offsets,
                           void* stream);

/*
 * Grouped gate/up projection with fused SwiGLU.
 * Replaces mlp.py:22-23 (up(x) * silu(gate(x))) for every expert at once,
 * rounding to dtype where the reference does: after gate, after up, after
 * silu and after the product.
 *
 *   x_perm  [n_rows, dim]           dtype (n_rows = n_tokens * top_k)
 *   tiles   tile list from astrai_moe_permute (same block_m)
 *   w_gate, w_up  device arrays of n_experts pointers, each [dim_ffn, dim]
 *   h       [n_rows, dim_ffn]       dtype
 *   workspace  scratch of the 256-row kernel, or NULL (contents need not be
 *              initialised; calls sharing one must not overlap). With
 *              workspace_bytes >= astrai_moe_gemm_workspace_bytes(0) the
 *              last tenth of the work is handed out at run time from a
 *              counter in it, so that compute units running at a higher
 *              clock take more (the XCDs of one MI355X hold clocks several
 *              per cent apart under load); with NULL every workgroup's tiles
 *              are dealt in advance. Results do not depend on it (each tile
 *              is computed the same way by whichever workgroup takes it).
 *
 * Kernels (both GEMMs): bf16 runs on the matrix cores with block_m 32, 64,
 * 128 or 256 when K is a multiple of 64 and the output columns a multiple of
 * 8 (a partial last column tile clamps its weight rows and stores only the
 * columns inside the matrix);
 * fp32 runs on the matrix cores (v_mfma_f32_16x16x4_f32) with block_m = 64,
 * K a multiple of 32 and dim_ffn % 32 == 0 (gate/up) or dim % 64 == 0 (down);
 * every other case on a general fp32-FMA kernel. Weights whose rows are a
 * multiple of 16 bytes must start on a 16-byte boundary.
 */
int astrai_moe_gemm_gate_up(const void* x_perm, const int32_t* tiles,
                            int64_t tiles_len, const void* const* w_gate,
                            const void* const* w_up, int dtype, int64_t n_rows,
                            int n_experts, int64_t dim, int64_t dim_ffn,
                            int block_m, void* h, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * astrai_moe_gemm_gate_up reading the activation rows straight from x: row r
 * of the permuted input is x[sorted_token[r]], so the permutation need not
 * copy x (astrai_moe_permute with x_perm = NULL). Same results as
 * astrai_moe_gemm_gate_up on the copied rows (bit-identical). bf16 and the
 * matrix-core block sizes (32, 64, 128 or 256) only; x under 4 GiB.
 *
 *   x             [n_tokens, dim]   bf16
 *   sorted_token  [n_rows]          int32, from astrai_moe_permute
 */
int astrai_moe_gemm_gate_up_gather(const void* x, const int32_t* sorted_token,
                                   int64_t n_tokens, const int32_t* tiles,
                                   int64_t tiles_len, const void* const* w_gate,
                                   const void* const* w_up, int dtype,
                                   int64_t n_rows, int n_experts, int64_t dim,
                                   int64_t dim_ffn, int block_m, void* h,
                                   void* workspace,
                                   int64_t workspace_bytes, void* stream);

/*
 * Grouped down projection with the routing-weight multiply fused.
 * Replaces mlp.py:24 (down(gated)) and the product at mlp.py:97-98
 * (expert_output * weights), rounding after each as the reference does.
 *
 *   h         [n_rows, dim_ffn]   dtype
 *   w_down    device array of n_experts pointers, each [dim, dim_ffn]
 *   sorted_w  [n_rows]            dtype, from astrai_moe_permute; NULL for
 *                                 weight 1 (a dense expert: mlp.py:22-25)
 *   y         [n_rows, dim]       dtype
 *   workspace  as for astrai_moe_gemm_gate_up, plus the fp32 partial sums of
 *              the down GEMM's last round: with workspace_bytes >=
 *              astrai_moe_gemm_workspace_bytes(1) the tiles left over after
 *              the last whole round of compute units (at most half a round)
 *              are split along K over all of them and summed in a second
 *              launch, instead of holding a few units for a full tile time
 *              while the rest idle. Those tiles' fp32 sums then group K
 *              differently (within the GEMM tolerance of the whole-tile
 *              order; deterministic for one compute-unit count). Not read by
 *              other tile heights, fp32 or the general kernel.
 */
int astrai_moe_gemm_down(const void* h, const int32_t* tiles,
                         int64_t tiles_len, const void* const* w_down,
                         const void* sorted_w, int dtype, int64_t n_rows,
                         int n_experts, int64_t dim_ffn, int64_t dim,
                         int block_m, void* y, void* workspace,
                         int64_t workspace_bytes, void* stream);

/*
 * Bytes of the GEMM workspace on the current device: 64 KiB of scheduling
 * state (the run-time claim counter and a mailbox per workgroup), plus, for
 * the down GEMMs (down != 0), one 256 x 256 fp32 tile of partial sums per
 * compute unit (64 MiB on 256 compute units). The same sizes serve the
 * packed and training variants. No counterpart in the reference
 * (mlp.py:96-98 runs one F.linear per expert).
 */
int64_t astrai_moe_gemm_workspace_bytes(int down);

/*
 * Packed expert weights (bf16). No counterpart in the reference: a cached
 * copy of an expert's weight in the order the grouped GEMMs stage it, so that
 * each 64-K step of a 256-row weight tile is one contiguous 32 KB read (the
 * row-strided layout reads 128 bytes of each of 256 rows per step). Results
 * are bit-identical to the unpacked GEMMs. Measured on MI355X: the down GEMM
 * of 64 tokens over 128 experts (D 4096, F 1536, top-8) 271 -> 264 us, its
 * gate/up GEMM unchanged (~6.1 TB/s of weights either way), the 16384-token
 * Mixtral-shaped GEMMs about 1 % faster. A second copy of the weights buys
 * little, so the Python layer only uses it when asked to.
 *
 * Layout: for column tile t (256 weight rows) and K step s (64 columns), a
 * block of 256 rows x 128 bytes at byte offset (t * (K / 64) + s) * 32768;
 * row r's 16-byte chunk c sits at chunk c ^ ((r >> 1) & 7). Gate/up tiles
 * hold 128 gate rows then the same 128 up rows, so the packed gate/up of one
 * expert is 2 * dim_ffn * dim elements and the packed down dim * dim_ffn,
 * the same sizes as the unpacked weights. The packed copy goes stale when
 * the weights change; the caller repacks (the Python layer tracks each
 * parameter's version).
 *
 *   w_gate, w_up   [dim_ffn, dim] bf16, one expert    (dim_ffn % 128 == 0, dim % 64 == 0)
 *   w_down         [dim, dim_ffn] bf16, one expert    (dim % 256 == 0, dim_ffn % 64 == 0)
 *   packed         2 * dim_ffn * dim (gate/up) or dim * dim_ffn (down) bf16, 16-byte aligned
 */
int astrai_moe_pack_gate_up(const void* w_gate, const void* w_up, int dtype,
                            int64_t dim_ffn, int64_t dim, void* packed,
                            void* stream);
int astrai_moe_pack_down(const void* w_down, int dtype, int64_t dim,
                         int64_t dim_ffn, void* packed, void* stream);

/*
 * The grouped GEMMs reading packed weights: same arguments, results and
 * rounding as astrai_moe_gemm_gate_up / astrai_moe_gemm_down (bit-identical),
 * with the weight tables pointing at packed copies. bf16 and the matrix-core
 * block sizes only (block_m from astrai_moe_select_block_m being 32, 64, 128 or 256);
 * other cases return ASTRAI_MOE_EINVAL.
 */
int astrai_moe_gemm_gate_up_packed(const void* x_perm, const int32_t* tiles,
                                   int64_t tiles_len, const void* const* w_packed,
                                   int dtype, int64_t n_rows, int n_experts,
                                   int64_t dim, int64_t dim_ffn, int block_m,
                                   void* h, void* workspace,
                                   int64_t workspace_bytes, void* stream);
int astrai_moe_gemm_down_packed(const void* h, const int32_t* tiles,
                                int64_t tiles_len, const void* const* w_packed,
                                const void* sorted_w, int dtype, int64_t n_rows,
                                int n_experts, int64_t dim_ffn, int64_t dim,
                                int block_m, void* y, void* workspace,
                                int64_t workspace_bytes, void* stream);

/*
 * Weighted un-permute and combine.
 * Replaces mlp.py:89 and :98 (zeros, then index_add_ of every expert's
 * weighted rows in ascending expert order, rounding after each add),
 * mlp.py:77 (mean of the shared experts' outputs: Python sum from 0, then
 * division by n_shared, which torch evaluates as a multiply by the float
 * reciprocal) and mlp.py:71 (shared_out + routed_out).
 *
 *   y          [n_tokens * top_k, dim]  dtype, from astrai_moe_gemm_down
 *   token_pos  [n_tokens * top_k]       int32, from astrai_moe_permute
 *   row_w      [n_tokens * top_k]       dtype per permuted row (sorted_w), or
 *              NULL. Given, y holds the unweighted rows (the down GEMM run
 *              without row weights) and each is scaled by its weight and
 *              rounded before the sum, as the weighted down GEMM would: the
 *              same result, with one output fewer for a training forward
 *              that keeps the unweighted rows anyway.
 *   shared     [n_shared, n_tokens, dim] dtype: each shared expert's output
 *              (NULL when n_shared == 0: the reference's zeros_like,
 *              mlp.py:75-76)
 *   out        [n_tokens, dim]          dtype
 */
int astrai_moe_combine(const void* y, const int32_t* token_pos, const void* row_w,
                       const void* shared, int n_shared, int dtype,
                       int64_t n_tokens, int top_k, int64_t dim, void* out,
                       void* stream);

/*
 * Training: forward that keeps what the backward needs, and the backward.
 * The reference gets its gradients from torch autograd over mlp.py:22-25
 * and :89-98; these entry points compute the same quantities with grouped
 * kernels, at autograd's rounding points (identities in fp32): on the matrix
 * cores for bf16 with dim and dim_ffn multiples of 64 (tile lists built with
 * block_m = 256); for fp32 on the fp32 matrix cores with block_m = 64 where
 * the GEMM's K is a multiple of 32 and its output columns of 4 (the forward
 * GEMMs as astrai_moe_gemm_gate_up / _down choose them); on the general-shape
 * kernels for every other shape. Per expert e with permuted rows R_e:
 *
 *   forward   g = x W_gate^T, u = x W_up^T, h = u * silu(g), y = h W_down^T,
 *             out = sum over slots of y * w                    (mlp.py:22-24, :97-98)
 *   backward  dy = dout[tok] * w,  dw = sum_d dout[tok] * y    (d of y * w)
 *             du = dh * silu(g),  dg = silu'(g) * (dh * u),  dh = dy W_down
 *             dx_perm = dg W_gate + du W_up,  dx = sum over slots (astrai_moe_combine)
 *             dW_down[e] = dy^T h,  dW_gate[e] = dg^T x_perm,  dW_up[e] = du^T x_perm
 *
 * astrai_moe_gemm_gate_up_train: astrai_moe_gemm_gate_up plus gu
 *   ([n_rows, 2 dim_ffn] dtype: the rounded projections silu and the product
 *   use, in blocks of 4 columns: gu[r, 2c .. 2c+3] = g[r, c .. c+3] and
 *   gu[r, 2c+4 .. 2c+7] = u[r, c .. c+3] for c a multiple of 4; when dim_ffn
 *   is not a multiple of 4, the last block holds its w = dim_ffn % 4 columns
 *   as g then u, w values each).
 * astrai_moe_gemm_down_train: astrai_moe_gemm_down plus y_unweighted
 *   ([n_rows, dim] dtype, the rounded expert output before the routing weight).
 */
int astrai_moe_gemm_gate_up_train(const void* x_perm, const int32_t* tiles,
                                  int64_t tiles_len, const void* const* w_gate,
                                  const void* const* w_up, int dtype,
                                  int64_t n_rows, int n_experts, int64_t dim,
                                  int64_t dim_ffn, int block_m, void* h,
                                  void* gu, void* workspace,
                                  int64_t workspace_bytes, void* stream);
int astrai_moe_gemm_down_train(const void* h, const int32_t* tiles,
                               int64_t tiles_len, const void* const* w_down,
                               const void* sorted_w, int dtype, int64_t n_rows,
                               int n_experts, int64_t dim_ffn, int64_t dim,
                               int block_m, void* y, void* y_unweighted,
                               void* workspace, int64_t workspace_bytes,
                               void* stream);

/*
 * Per permuted row r (token sorted_token[r], weight sorted_w[r]):
 *   dy[r]      = dout[token] * w, rounded per element     [n_rows, dim] dtype
 *   dw_rows[r] = sum_d round(dout[token, d] * y[r, d])    [n_rows] dtype
 * (mlp.py:97's expert_output * weights, differentiated in both factors;
 * round() is the rounding to dtype, the identity in fp32).
 */
int astrai_moe_row_grad(const void* dout, const int32_t* sorted_token,
                        const void* sorted_w, const void* y_unweighted,
                        int dtype, int64_t n_rows, int64_t dim, void* dy,
                        void* dw_rows, void* stream);

/*
 * Grouped dgrad of the down projection with the SwiGLU backward fused:
 *   dh = dy . W_down[e] (W_down [dim, dim_ffn]), rounded to dtype, then
 *   du = round(dh * silu(g)), dg = round(round(dh * u) * silu'(g))
 * (the order torch autograd takes through mlp.py:23).
 *   dy [n_rows, dim], gu [n_rows, 2 dim_ffn] (from astrai_moe_gemm_gate_up_train),
 *   dg, du [n_rows, dim_ffn], all dtype.
 */
int astrai_moe_gemm_dgrad_down(const void* dy, const int32_t* tiles,
                               int64_t tiles_len, const void* const* w_down,
                               const void* gu, int dtype,
                               int64_t n_rows, int n_experts, int64_t dim,
                               int64_t dim_ffn, int block_m, void* dg, void* du,
                               void* stream);

/*
 * Grouped dgrad of the gate and up projections:
 *   dx_perm = round(round(dg . W_gate[e]) + round(du . W_up[e]))   [n_rows, dim] dtype
 * (autograd's rounding: each linear's input gradient, then their sum).
 * workspace: as the down GEMM's (astrai_moe_gemm_workspace_bytes(1) bytes,
 *   16-byte aligned, nothing to initialise; NULL / 0: none). With it, a
 *   partial last round of 256-row tiles of at least 64 K steps is split
 *   along K and the slices' fp32 sums are added in a fixed order: the same
 *   result on every call, but those tiles' sums are associated differently
 *   from the unsplit kernel's, and which tiles form the tail depends on the
 *   device's compute-unit count. Calls sharing a workspace must be ordered
 *   on one stream.
 */
int astrai_moe_gemm_dgrad_gate_up(const void* dg, const void* du,
                                  const int32_t* tiles, int64_t tiles_len,
                                  const void* const* w_gate,
                                  const void* const* w_up, int dtype,
                                  int64_t n_rows, int n_experts,
                                  int64_t dim_ffn, int64_t dim, int block_m,
                                  void* dx_perm, void* workspace,
                                  int64_t workspace_bytes, void* stream);

/*
 * Per-expert weight gradient: dw[e] = a[rows of e]^T . b[rows of e], the rows
 * of expert e being expert_offsets[e] .. expert_offsets[e + 1] - 1.
 *   a [n_rows, m], b [n_rows, n], dw [n_experts, m, n], all dtype (the
 *   matrix-core kernel for bf16 with m % 8 == 0 and n % 8 == 0, the
 *   general-shape one otherwise). Experts without rows are not written.
 * dW_down: (a, b) = (dy, h); dW_gate: (dg, x_perm); dW_up: (du, x_perm).
 */
int astrai_moe_gemm_wgrad(const void* a, const void* b,
                          const int32_t* expert_offsets, int dtype,
                          int64_t n_rows, int n_experts, int64_t m, int64_t n,
                          void* dw, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ASTRAI_MOE_H */
