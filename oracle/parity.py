"""ORACLE — test infrastructure only. Parity of a MoE-layer forward against
the oracle (``oracle/moe_ref.py``) on the same device.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s checker legs
(the parity report next to the throughput and the CPU baseline) may import
this module; the product path (``astrai_amd``) never does.

What is compared (the reference being ``astrai/model/components/mlp.py:64-100``):

* routing (``mlp.py:84-87``): the set of top-k experts of every token and the
  renormalised weights slot by slot — bit-exact;
* permutation (``mlp.py:90-93``): the source token of every permuted row and
  the expert offsets — bit-exact (expert-major, token-ascending);
* the output, in three figures:
  - ``allclose_frac``: plain elementwise ``isclose`` at rtol 2e-2 / atol 2e-3
    (bf16) or 1e-5 / 1e-5 (fp32);
  - ``max_norm_err``: max over elements of ``|out - ref| / (atol + rtol |ref|)``
    (at most 1 means every element is within the plain tolerance);
  - ``term_bound_excess``: max over elements of
    ``|out - ref| - (k atol + rtol sum_k |y_k|)``, the same tolerance applied to
    each of the k expert terms summed into the element (at most 0 passes).
    Where expert terms cancel, the sum is small while each term carries its
    own rounding, so this is the bound that stays meaningful there.
"""

from __future__ import annotations

import torch
from torch import Tensor

from oracle import moe_ref as R


def tolerance(dtype: torch.dtype) -> tuple[float, float]:
    """(rtol, atol) of the layer output against the reference."""
    return (2e-2, 2e-3) if dtype == torch.bfloat16 else (1e-5, 1e-5)


def layer_parity(layer, x: Tensor, out: Tensor, topk_idx: Tensor | None = None, topk_w: Tensor | None = None,
                 sorted_token: Tensor | None = None, expert_offsets: Tensor | None = None) -> dict:
    """Compare ``out = layer(x)`` with the oracle evaluated on the layer's own
    parameters on x's device; optionally also the kernels' routing
    (``topk_idx [T, K]``, ``topk_w [T, K]``) and permutation
    (``sorted_token [T K]``, ``expert_offsets [E + 1]``) for the same input."""
    rtol, atol = tolerance(x.dtype)
    dim = x.shape[-1]
    x_flat = x.reshape(-1, dim)
    rw, rb, experts, shared = R.module_weights(layer)
    with torch.no_grad():
        trace = R.routed_forward(x_flat, rw, rb, experts, layer.n_activated_experts, trace=True)
        ref = R.shared_forward(x_flat, shared) + trace.out
        mag = torch.zeros(x_flat.shape, dtype=torch.float32, device=x.device)
        for item in trace.expert_out:
            if item is not None:
                tok, _, yw = item
                mag.index_add_(0, tok, yw.abs().float())
        for w in shared:
            mag += R.expert_mlp(x_flat, w).abs().float() / len(shared)
        k = layer.n_activated_experts + len(shared)
        o, r = out.reshape(x_flat.shape).float(), ref.float()
        err = (o - r).abs()
        report = {
            "rtol": rtol,
            "atol": atol,
            "allclose_frac": torch.isclose(o, r, rtol=rtol, atol=atol).float().mean().item(),
            "max_norm_err": (err / (atol + rtol * r.abs())).max().item() if err.numel() else 0.0,
            "term_bound_excess": (err - (k * atol + rtol * mag)).max().item() if err.numel() else 0.0,
            "max_abs_err": err.max().item() if err.numel() else 0.0,
            "finite": bool(torch.isfinite(o).all().item()),
        }
        if topk_idx is not None:
            same_sets = torch.equal(topk_idx.long().sort(-1).values, trace.topk_idx.sort(-1).values)
            same_w = topk_w is None or torch.equal(topk_w, trace.topk_w)
            report["routing_bit_exact"] = bool(same_sets and same_w)
        if sorted_token is not None:
            tok, _, offsets = R.permutation(trace.topk_idx, len(experts))
            same_rows = torch.equal(sorted_token.long(), tok)
            same_off = expert_offsets is None or torch.equal(expert_offsets.long(), offsets)
            report["permutation_bit_exact"] = bool(same_rows and same_off)
    return report
