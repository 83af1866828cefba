// Internal interface between the grouped-GEMM entry points (moe_gemm.hip) and
// the CDNA4 matrix-core kernels (moe_gemm_mfma.hip).
#pragma once

#include "moe_common.h"

namespace astrai_moe {

// Row-tile heights of the bf16 matrix-core kernels. The large tile serves
// prefill-sized expert loads; the small one serves decode-sized loads, where
// the work is streaming expert weights and padding rows to 256 would make the
// kernel compute-bound on empty rows.
constexpr int kMfmaBigBM = 256;
constexpr int kMfmaSmallBM = 32;
// Mid-sized expert loads (about 48-128 rows per expert): one 64-row tile per
// expert reads its weights once, where 32-row tiles would stream them twice or
// more and 256-row tiles would compute mostly padding.
constexpr int kMfmaMidBM = 64;
// Loads of up to about 128 rows per expert: one 128-row tile per expert reads
// its weights once where two 64-row tiles would stream them twice.
constexpr int kMfmaMid2BM = 128;

// Scratch of the 256-row streaming kernels (none: every work item is dealt
// statically and the tiles left over after the last whole round run whole).
// The first kSchedBytes hold the run-time work claims (a counter the launch
// clears, and one mailbox ring per workgroup); the down GEMMs' split-tail
// partial sums follow, one 256 x 256 fp32 tile per workgroup.
// gemm_workspace_bytes(down) is the size that enables both on the current
// device.
struct GemmWorkspace {
  void* base = nullptr;
  int64_t bytes = 0;
};
constexpr int64_t kSchedBytes = 65536;
int64_t gemm_workspace_bytes(bool down);

// Shape constraints of the bf16 kernels: K a multiple of 64, the output
// columns a multiple of the column tile, 16-byte aligned operands.
bool mfma_gate_up_supported(int64_t dim, int64_t dim_ffn, int block_m,
                            const void* a, const void* c);
bool mfma_down_supported(int64_t dim_ffn, int64_t dim, int block_m,
                         const void* a, const void* c);

// `packed`: the weight tables point at packed copies written by launch_pack
// (bf16, 256-row tiles of K / 64 contiguous 32 KB blocks in staged order).
int launch_mfma_gate_up(const void* x_perm, const int32_t* tiles,
                        int64_t capacity, const void* const* w_gate,
                        const void* const* w_up, int64_t dim, int64_t dim_ffn,
                        int block_m, bool packed, void* h, hipStream_t s,
                        const GemmWorkspace& ws = {});
int launch_mfma_down(const void* h, const int32_t* tiles, int64_t capacity,
                     const void* const* w_down, const void* sorted_w,
                     int64_t dim_ffn, int64_t dim, int block_m, bool packed,
                     void* y, hipStream_t s,
                     const GemmWorkspace& ws = {});

// As launch_mfma_gate_up, reading the activation rows as x[sorted_token[r]]
// (x: [n_tokens, dim]) instead of a copied x_perm.
int launch_mfma_gate_up_gather(const void* x, const int32_t* sorted_token,
                               const int32_t* tiles, int64_t capacity,
                               const void* const* w_gate,
                               const void* const* w_up, int64_t dim,
                               int64_t dim_ffn, int block_m, void* h,
                               hipStream_t s,
                        const GemmWorkspace& ws = {});

// Training forward (256-row tiles): as launch_mfma_gate_up / launch_mfma_down,
// also storing the bf16 gate and up projections (gu: [rows, 2 dim_ffn],
// blocks of 4 gate columns then the same 4 up columns) or the unweighted bf16
// expert output (y_unweighted: [rows, dim]).
int launch_mfma_gate_up_save(const void* x_perm, const int32_t* tiles,
                             int64_t capacity, const void* const* w_gate,
                             const void* const* w_up, int64_t dim,
                             int64_t dim_ffn, void* h, void* gu,
                             hipStream_t s,
                        const GemmWorkspace& ws = {});
int launch_mfma_down_save(const void* h, const int32_t* tiles,
                          int64_t capacity, const void* const* w_down,
                          const void* sorted_w, int64_t dim_ffn, int64_t dim,
                          void* y, void* y_unweighted, hipStream_t s,
                          const GemmWorkspace& ws = {});

// fp32 on the matrix cores (moe_gemm_mfma_f32.hip), 64-row tile lists, K a
// multiple of 32, output columns a multiple of 32 (gate/up) or 64 (down),
// 16-byte aligned operands. A non-null gu / y_unweighted selects the training
// forward, which also stores the gate and up projections (blocked layout of
// gu_index) or the output before the routing weight.
bool mfma_f32_supported(int64_t k, int64_t n, bool gate_up, int block_m,
                        const void* a, const void* c, const void* s0);
int launch_mfma_f32_gate_up(const void* x_perm, const int32_t* tiles,
                            int64_t capacity, const void* const* w_gate,
                            const void* const* w_up, int64_t n_rows,
                            int n_experts, int64_t dim, int64_t dim_ffn,
                            void* h, void* gu, hipStream_t s);
int launch_mfma_f32_down(const void* h, const int32_t* tiles, int64_t capacity,
                         const void* const* w_down, const void* sorted_w,
                         int64_t n_rows, int n_experts, int64_t dim_ffn,
                         int64_t dim, void* y, void* y_unweighted,
                         hipStream_t s);

// fp32 backward on the matrix cores (moe_gemm_mfma_f32_bwd.hip): the dgrad
// GEMMs over 64-row tile lists with K a multiple of 32 and N of 4, wgrad with
// M and N multiples of 4; same contracts as the general-shape ones below.
bool mfma_f32_bwd_supported(int64_t k, int64_t n, int block_m, const void* a,
                            const void* c0, const void* c1, const void* e0);
bool mfma_f32_wgrad_supported(int64_t m, int64_t n, const void* a,
                              const void* b, const void* dw);
int launch_mfma_f32_dgrad_down(const void* dy, const int32_t* tiles,
                               int64_t capacity, const void* const* w_down,
                               const void* gu, int64_t dim, int64_t dim_ffn,
                               void* dg, void* du, hipStream_t s);
int launch_mfma_f32_dgrad_in(const void* d, const int32_t* tiles,
                             int64_t capacity, const void* const* w, int64_t k,
                             int64_t n, const void* add, void* dx,
                             hipStream_t s);
int launch_mfma_f32_wgrad(const void* a, const void* b, const int32_t* offsets,
                          int n_experts, int64_t m, int64_t n, void* dw,
                          hipStream_t s);

// Backward (moe_gemm_bwd.hip), bf16, 256-row tile lists:
// dy = dout[sorted_token] * sorted_w and dw_rows = sum(dout[tok] * y) per row;
int launch_row_grad(const void* dout, const int32_t* sorted_token,
                    const void* sorted_w, const void* y, int64_t n_rows,
                    int64_t dim, void* dy, void* dw_rows, hipStream_t s);
// dg, du [rows, dim_ffn] from dy [rows, dim], W_down [dim, dim_ffn] and the
// saved interleaved gu;
int launch_dgrad_down(const void* dy, const int32_t* tiles, int64_t capacity,
                      const void* const* w_down, const void* gu, int64_t dim,
                      int64_t dim_ffn, void* dg, void* du, hipStream_t s);
// dx [rows, n] = bf16(d . W[e]) (+ add, rounded again), W[e] [k, n]; ws as
// the down GEMM's (gemm_workspace_bytes(true)): the last round's tiles split
// along K;
int launch_dgrad_in(const void* d, const int32_t* tiles, int64_t capacity,
                    const void* const* w, int64_t k, int64_t n,
                    const void* add, void* dx, hipStream_t s,
                    const GemmWorkspace& ws = {});
// dw[e] [m, n] = a[rows_e]^T . b[rows_e] for every expert with rows
// (a: [rows, m], b: [rows, n]); experts without rows are not written.
int launch_wgrad(const void* a, const void* b, const int32_t* offsets,
                 int n_experts, int64_t m, int64_t n, void* dw,
                 hipStream_t s);

// General-shape backward (moe_gemm_generic_bwd.hip): fp32 or bf16, any dim
// and dim_ffn, any row-tile height; same contracts as the matrix-core ones
// above, the saved gu in the blocked layout of gu_index.
int launch_generic_dgrad_down(int dtype, const void* dy, const int32_t* tiles,
                              int64_t capacity, const void* const* w_down,
                              const void* gu, int64_t dim, int64_t dim_ffn,
                              void* dg, void* du, hipStream_t s);
int launch_generic_dgrad_in(int dtype, const void* d, const int32_t* tiles,
                            int64_t capacity, const void* const* w, int64_t k,
                            int64_t n, const void* add, void* dx,
                            hipStream_t s);
int launch_generic_wgrad(int dtype, const void* a, const void* b,
                         const int32_t* offsets, int n_experts, int64_t m,
                         int64_t n, void* dw, hipStream_t s);
int launch_generic_row_grad(int dtype, const void* dout,
                            const int32_t* sorted_token, const void* sorted_w,
                            const void* y, int64_t n_rows, int64_t dim,
                            void* dy, void* dw_rows, hipStream_t s);

// Packs one expert's weight for the packed GEMMs: gate/up (w0 = gate, w1 =
// up, each [rows, k]) or down (w0 = [rows, k]).
int launch_pack(const void* w0, const void* w1, int64_t rows, int64_t k,
                bool gate_up, void* out, hipStream_t s);

}  // namespace astrai_moe
