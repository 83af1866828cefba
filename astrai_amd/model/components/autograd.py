"""Autograd for the MoE layer: HIP kernels forward and backward.

The reference layer is plain torch, so autograd differentiates it op by op
(``astrai/model/components/mlp.py:22-25, 64-100``). Here the forward runs on
the HIP kernels. For bf16 and the matrix-core shapes the backward runs on
grouped HIP kernels too (``astrai_moe_row_grad``, ``astrai_moe_gemm_dgrad_*``,
``astrai_moe_gemm_wgrad``): the training forward saves the gate and up
projections ``g, u`` (interleaved), ``h`` and the unweighted expert output
``y``, and the
backward evaluates the formulas autograd applies to mlp.py:22-25 and :97-98
(per expert e: ``dy = dout[tok] * w``, ``dw = sum(dout[tok] * y)``,
``dh = dy W_down``, ``du = dh silu(g)``, ``dg = silu'(g) (dh u)``,
``dx = dg W_gate + du W_up``, ``dW_down = dy^T h``, ``dW_gate = dg^T x``,
``dW_up = du^T x``). Other shapes and fp32 recompute each expert's SwiGLU
with the same torch ops as ``mlp.py:22-25`` and let autograd differentiate
them, so the gradient formulas and their rounding points are the reference's:

* ``out.index_add_(0, tok, y * w)`` (``mlp.py:98``): the gradient reaching
  expert row r is ``dout[tok(r)]``; the row's output gets ``dout * w`` and its
  routing weight gets ``sum(dout * y)`` over the model dimension;
* ``x[tok]`` (``mlp.py:95``): the per-row input gradients are summed back into
  their tokens in ascending expert order, rounding after every add, which is
  the combine kernel's contract (the reference's ``index_add_`` backward);
* experts without rows get no gradient (the reference skips them, so their
  ``.grad`` stays ``None`` there too).

In the recompute path the expert GEMMs of the backward are per-expert library
GEMMs (torch ``F.linear``); the row gather/scatter runs on the HIP kernels.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from astrai_amd.extension import ops


def _expert_forward(x: Tensor, wg: Tensor, wu: Tensor, wd: Tensor) -> Tensor:
    """``down(up(x) * silu(gate(x)))`` with mlp.py:22-25's evaluation order."""
    return F.linear(F.linear(x, wu) * F.silu(F.linear(x, wg)), wd)


def _expert_grads(x: Tensor, wg: Tensor, wu: Tensor, wd: Tensor, dz: Tensor | None, z_out: bool = False):
    """Recompute one expert on detached leaves and differentiate it."""
    with torch.enable_grad():
        leaves = [t.detach().requires_grad_(True) for t in (x, wg, wu, wd)]
        z = _expert_forward(*leaves)
    if dz is None:
        return z.detach()
    grads = torch.autograd.grad(z, leaves, dz)
    return (z.detach(), grads) if z_out else grads


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
        n_tokens, dim = x.shape
        top_k = topk_idx.shape[1]
        tg, tu, td = tables
        route = ops.RouteResult(topk_idx, topk_w.contiguous(), chunk_hist)
        ctx.n_experts = n_experts
        ctx.hip = ops.backward_supported(dim, dim_ffn, x.dtype)
        if ctx.hip:
            perm = ops.moe_permute(route, x, n_experts, ops.TRAIN_BLOCK_M)
            h, gu = ops.moe_gemm_gate_up_train(perm.x_perm, perm.tiles, tg, tu, n_experts, dim_ffn)
            y, y_unw = ops.moe_gemm_down_train(h, perm.tiles, td, perm.sorted_w, n_experts, dim)
            out = ops.moe_combine(y, perm.token_pos)
            ctx.tables = tables
            ctx.save_for_backward(perm.x_perm, perm.sorted_token, perm.sorted_w, perm.token_pos,
                                  perm.expert_offsets, perm.tiles, h, gu, y_unw, *weights)
            return out
        block_m = ops.select_block_m(n_tokens, n_experts, top_k, dim, dim_ffn, x.dtype)
        perm = ops.moe_permute(route, x, n_experts, block_m)
        h = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tg, tu, n_experts, dim_ffn, block_m)
        y = ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, n_experts, dim, block_m)
        out = ops.moe_combine(y, perm.token_pos)
        ctx.save_for_backward(perm.x_perm, perm.sorted_token, perm.sorted_w, perm.token_pos, perm.expert_offsets,
                              *weights)
        return out

    @staticmethod
    def backward(ctx, dout):
        if ctx.hip:
            return RoutedExperts._backward_hip(ctx, dout.contiguous())
        x_perm, sorted_token, sorted_w, token_pos, offsets, *weights = ctx.saved_tensors
        n_experts = ctx.n_experts
        wg, wu, wd = weights[:n_experts], weights[n_experts:2 * n_experts], weights[2 * n_experts:]
        dout = dout.contiguous()
        # gradient of index_add_'s source: the token's output gradient per permuted row
        dp = dout.index_select(0, sorted_token.long())
        dx_perm = torch.empty_like(x_perm)
        dw_rows = torch.empty(x_perm.shape[0], dtype=dout.dtype, device=dout.device)
        g_gate: list[Tensor | None] = [None] * n_experts
        g_up: list[Tensor | None] = [None] * n_experts
        g_down: list[Tensor | None] = [None] * n_experts
        bounds = offsets.tolist()  # one host sync per backward
        for e in range(n_experts):
            a, b = bounds[e], bounds[e + 1]
            if a == b:
                continue
            dp_e = dp[a:b]
            w_e = sorted_w[a:b].unsqueeze(-1)
            z, (gx, gg, gu, gd) = _expert_grads(x_perm[a:b], wg[e], wu[e], wd[e], dp_e * w_e, z_out=True)
            dw_rows[a:b] = (dp_e * z).sum(-1)
            dx_perm[a:b] = gx
            g_gate[e], g_up[e], g_down[e] = gg, gu, gd
        dx = ops.moe_combine(dx_perm, token_pos)
        dw = dw_rows[token_pos.long()]
        return (dx, dw, None, None, None, None, *g_gate, *g_up, *g_down)

    @staticmethod
    def _backward_hip(ctx, dout):
        x_perm, sorted_token, sorted_w, token_pos, offsets, tiles, h, gu, y_unw, *_ = ctx.saved_tensors
        ops._tag_tiles(tiles, ops.TRAIN_BLOCK_M)
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
            # one host sync, after every kernel is enqueued: experts without
            # rows get no gradient, as in the reference
            counts = (offsets[1:] - offsets[:-1]).tolist()
            for e, c in enumerate(counts):
                if c > 0:
                    g_gate[e], g_up[e], g_down[e] = d_gate[e], d_up[e], d_down[e]
        return (dx, dw, None, None, None, None, *g_gate, *g_up, *g_down)


class DenseExpert(torch.autograd.Function):
    """One dense SwiGLU expert (mlp.py:22-25, the shared experts and ``MLP``):
    ``forward(x [T, D], tables, dim_ffn, w_gate, w_up, w_down)``."""

    @staticmethod
    def forward(ctx, x, tables, dim_ffn, wg, wu, wd):
        tg, tu, td = tables
        n_tokens, dim = x.shape
        ctx.hip = n_tokens > 0 and ops.backward_supported(dim, dim_ffn, x.dtype)
        if ctx.hip:
            tiles, offsets = ops.dense_tiles(n_tokens, ops.TRAIN_BLOCK_M, x.device, with_offsets=True)
            h, gu = ops.moe_gemm_gate_up_train(x, tiles, tg, tu, 1, dim_ffn)
            out = ops.moe_gemm_down(h, tiles, td, None, 1, dim, ops.TRAIN_BLOCK_M)
            ctx.tables = tables
            ctx.save_for_backward(x, tiles, offsets, h, gu, wg, wu, wd)
            return out
        ctx.save_for_backward(x, wg, wu, wd)
        return ops.moe_dense_mlp(x, tg, tu, td, dim_ffn)

    @staticmethod
    def backward(ctx, dout):
        dout = dout.contiguous()
        if ctx.hip:
            x, tiles, offsets, h, gu, *_ = ctx.saved_tensors
            ops._tag_tiles(tiles, ops.TRAIN_BLOCK_M)  # saved tensors come back without the tag
            tg, tu, td = ctx.tables
            dim = x.shape[1]
            dg, du = ops.moe_gemm_dgrad_down(dout, tiles, td, gu, 1)
            dx = ops.moe_gemm_dgrad_gate_up(dg, du, tiles, tg, tu, 1, dim) if ctx.needs_input_grad[0] else None
            gg = ops.moe_gemm_wgrad(dg, x, offsets, 1)[0]
            gu = ops.moe_gemm_wgrad(du, x, offsets, 1)[0]
            gd = ops.moe_gemm_wgrad(dout, h, offsets, 1)[0]
            return dx, None, None, gg, gu, gd
        x, wg, wu, wd = ctx.saved_tensors
        gx, gg, gu, gd = _expert_grads(x, wg, wu, wd, dout)
        return gx, None, None, gg, gu, gd


def routing_weights(logits: Tensor, topk_idx: Tensor, dtype: torch.dtype) -> Tensor:
    """The renormalised top-k weights as differentiable torch ops
    (mlp.py:84-87), evaluated at the route kernel's indices: the same values
    the kernel produces, with autograd's path back to the logits."""
    probs = torch.softmax(logits.float(), dim=-1).to(dtype)
    w = probs.gather(1, topk_idx.long())
    return w / w.sum(dim=-1, keepdim=True)
