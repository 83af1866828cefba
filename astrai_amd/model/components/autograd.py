"""Autograd for the MoE layer: HIP kernels forward and backward.

The reference layer is plain torch, so autograd differentiates it op by op
(``astrai/model/components/mlp.py:22-25, 64-100``). Here the forward runs on
the HIP kernels with saving epilogues (the gate and up projections ``g, u``,
``h`` and the unweighted expert output ``y``), and the backward on grouped
HIP kernels (``astrai_moe_row_grad``, ``astrai_moe_gemm_dgrad_*``,
``astrai_moe_gemm_wgrad``): bf16 with dim and dim_ffn multiples of 64 on the
matrix cores, every other shape and fp32 on the general-shape kernels.
They evaluate the formulas autograd applies to mlp.py:22-25 and :97-98 at
autograd's rounding points (per expert e: ``dy = dout[tok] * w``,
``dw = sum(dout[tok] * y)``, ``dh = dy W_down``, ``du = dh silu(g)``,
``dg = silu'(g) (dh u)``, ``dx = dg W_gate + du W_up``, ``dW_down = dy^T h``,
``dW_gate = dg^T x``, ``dW_up = du^T x``):

* ``out.index_add_(0, tok, y * w)`` (``mlp.py:98``): the gradient reaching
  expert row r is ``dout[tok(r)]``; the row's output gets ``dout * w`` and its
  routing weight gets ``sum(dout * y)`` over the model dimension;
* ``x[tok]`` (``mlp.py:95``): the per-row input gradients are summed back into
  their tokens in ascending expert order, rounding after every add, which is
  the combine kernel's contract (the reference's ``index_add_`` backward);
* experts without rows get no gradient (the reference skips them, so their
  ``.grad`` stays ``None`` there too): the forward copies the expert offsets
  to pinned host memory behind its kernels, and the backward waits on that
  copy's event, done long before, instead of on its own kernels.
"""

from __future__ import annotations

import torch
from torch import Tensor

from astrai_amd.extension import ops


class EmptyBatch(torch.autograd.Function):
    """The layer on zero tokens with shared experts (mlp.py:64-100 on an empty
    ``x``): an empty output whose gradient reaches ``x`` and the shared
    experts' weights as zeros. The reference's routed output is then a plain
    ``torch.zeros`` (every expert is skipped, mlp.py:89-94), so neither the
    router nor the routed experts get a gradient."""

    @staticmethod
    def forward(ctx, x, *params):
        ctx.param_specs = [(p.shape, p.dtype, p.device) for p in params]
        return x.new_empty(0, x.shape[1])

    @staticmethod
    def backward(ctx, dout):
        return (dout.new_zeros(0, dout.shape[1]),
                *(torch.zeros(shape, dtype=dtype, device=device) for shape, dtype, device in ctx.param_specs))


class RoutedExperts(torch.autograd.Function):
    """Routed experts and their weighted combine (mlp.py:89-100).

    ``forward(x [T, D], topk_w [T, K], topk_idx [T, K] int32, chunk_hist,
    tables, dim_ffn, *weights)`` where ``weights`` are the E gate, then the E
    up, then the E down weight tensors whose device pointers ``tables`` hold.
    Differentiable in ``x``, ``topk_w`` and every weight.
    """

    @staticmethod
    def forward(ctx, x, topk_w, topk_idx, chunk_hist, tables, dim_ffn, *weights):
        n_experts = len(weights) // 3
        dim = x.shape[1]
        tg, tu, td = tables
        route = ops.RouteResult(topk_idx, topk_w.contiguous(), chunk_hist)
        bm = ops.train_block_m(dim, dim_ffn, x.dtype)
        perm = ops.moe_permute(route, x, n_experts, bm)
        h, gu = ops.moe_gemm_gate_up_train(perm.x_perm, perm.tiles, tg, tu, n_experts, dim_ffn)
        # the down GEMM without routing weights gives the unweighted rows the
        # backward keeps; the combine applies the weights (same rounding)
        y_unw = ops.moe_gemm_down(h, perm.tiles, td, None, n_experts, dim, bm)
        out = ops.moe_combine(y_unw, perm.token_pos, row_w=perm.sorted_w)
        # which experts got rows, for the backward: copied to pinned host
        # memory now, so that the backward reads it without waiting for its
        # own kernels
        offsets_host = torch.empty(n_experts + 1, dtype=torch.int32, pin_memory=True)
        offsets_host.copy_(perm.expert_offsets, non_blocking=True)
        ctx.offsets_ready = torch.cuda.Event()
        ctx.offsets_ready.record()
        ctx.offsets_host = offsets_host
        ctx.n_experts, ctx.block_m, ctx.tables = n_experts, bm, tables
        ctx.save_for_backward(perm.x_perm, perm.sorted_token, perm.sorted_w, perm.token_pos,
                              perm.expert_offsets, perm.tiles, h, gu, y_unw, *weights)
        return out

    @staticmethod
    def backward(ctx, dout):
        dout = dout.contiguous()
        x_perm, sorted_token, sorted_w, token_pos, offsets, tiles, h, gu, y_unw, *_ = ctx.saved_tensors
        ops._tag_tiles(tiles, ctx.block_m)  # saved tensors may come back without the tag
        n_experts = ctx.n_experts
        tg, tu, td = ctx.tables
        dim = x_perm.shape[1]
        dy, dw_rows = ops.moe_row_grad(dout, sorted_token, sorted_w, y_unw)
        dg, du = ops.moe_gemm_dgrad_down(dy, tiles, td, gu, n_experts)
        dx = None
        if ctx.needs_input_grad[0]:
            dx_perm = ops.moe_gemm_dgrad_gate_up(dg, du, tiles, tg, tu, n_experts, dim)
            dx = ops.moe_combine(dx_perm, token_pos)
        dw = dw_rows[token_pos.long()] if ctx.needs_input_grad[1] else None
        none = [None] * n_experts
        g_gate, g_up, g_down = list(none), list(none), list(none)
        if any(ctx.needs_input_grad[6:]):
            d_gate = ops.moe_gemm_wgrad(dg, x_perm, offsets, n_experts)
            d_up = ops.moe_gemm_wgrad(du, x_perm, offsets, n_experts)
            d_down = ops.moe_gemm_wgrad(dy, h, offsets, n_experts)
            # experts without rows get no gradient, as in the reference; the
            # offsets were copied to the host in the forward, long done by now
            ctx.offsets_ready.synchronize()
            offs = ctx.offsets_host.tolist()
            # one call for each stack's E views (indexing them one by one cost
            # ~2 µs of host time each)
            v_gate, v_up, v_down = d_gate.unbind(0), d_up.unbind(0), d_down.unbind(0)
            for e in range(n_experts):
                if offs[e + 1] > offs[e]:
                    g_gate[e], g_up[e], g_down[e] = v_gate[e], v_up[e], v_down[e]
        return (dx, dw, None, None, None, None, *g_gate, *g_up, *g_down)


class DenseExpert(torch.autograd.Function):
    """One dense SwiGLU expert (mlp.py:22-25, the shared experts and ``MLP``):
    ``forward(x [T, D], tables, dim_ffn, w_gate, w_up, w_down)``."""

    @staticmethod
    def forward(ctx, x, tables, dim_ffn, wg, wu, wd):
        tg, tu, td = tables
        n_tokens, dim = x.shape
        ctx.tables = tables
        if n_tokens == 0:
            # torch's linear on no rows: an empty output, zero weight gradients
            ctx.save_for_backward(x, wg, wu, wd)
            ctx.empty = True
            return x.new_empty(0, dim)
        ctx.empty = False
        bm = ops.train_block_m(dim, dim_ffn, x.dtype)
        tiles, offsets = ops.dense_tiles(n_tokens, bm, x.device, with_offsets=True)
        h, gu = ops.moe_gemm_gate_up_train(x, tiles, tg, tu, 1, dim_ffn)
        out = ops.moe_gemm_down(h, tiles, td, None, 1, dim, bm)
        ctx.block_m = bm
        ctx.save_for_backward(x, tiles, offsets, h, gu, wg, wu, wd)
        return out

    @staticmethod
    def backward(ctx, dout):
        if ctx.empty:
            x, wg, wu, wd = ctx.saved_tensors
            return x.new_zeros(x.shape), None, None, torch.zeros_like(wg), torch.zeros_like(wu), torch.zeros_like(wd)
        dout = dout.contiguous()
        x, tiles, offsets, h, gu, *_ = ctx.saved_tensors
        ops._tag_tiles(tiles, ctx.block_m)  # saved tensors may come back without the tag
        tg, tu, td = ctx.tables
        dim = x.shape[1]
        dg, du = ops.moe_gemm_dgrad_down(dout, tiles, td, gu, 1)
        dx = ops.moe_gemm_dgrad_gate_up(dg, du, tiles, tg, tu, 1, dim) if ctx.needs_input_grad[0] else None
        gg = ops.moe_gemm_wgrad(dg, x, offsets, 1)[0]
        gu_w = ops.moe_gemm_wgrad(du, x, offsets, 1)[0]
        gd = ops.moe_gemm_wgrad(dout, h, offsets, 1)[0]
        return dx, None, None, gg, gu_w, gd


def routing_weights(logits: Tensor, topk_idx: Tensor, dtype: torch.dtype) -> Tensor:
    """The renormalised top-k weights as differentiable torch ops
    (mlp.py:84-87), evaluated at the route kernel's indices: the same values
    the kernel produces, with autograd's path back to the logits."""
    probs = torch.softmax(logits.float(), dim=-1).to(dtype)
    w = probs.gather(1, topk_idx.long())
    return w / w.sum(dim=-1, keepdim=True)
