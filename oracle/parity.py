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
* with ``truth_tokens``, both outputs against an fp64 truth: the layer
  evaluated from the same inputs (the same bf16 / fp32 activations and
  weights, the reference's routing, which both paths share bit for bit) with
  every intermediate kept in fp64, i.e. without the reference's rounding
  points (``mlp.py:23-24, 96-98``). For the kernels' output and for the
  reference's: the number of elements outside the plain tolerance around the
  truth (``truth_fail_kernel`` / ``truth_fail_ref``), the max normalised
  error and the RMS error. The elements where the kernels' output and the
  reference's disagree beyond the plain tolerance are where either carries
  its own bf16 roundings of cancelling expert terms; against the truth the
  two paths must fail about equally often.
"""

from __future__ import annotations

import torch
from torch import Tensor

from oracle import moe_ref as R


def tolerance(dtype: torch.dtype) -> tuple[float, float]:
    """(rtol, atol) of the layer output against the reference."""
    return (2e-2, 2e-3) if dtype == torch.bfloat16 else (1e-5, 1e-5)


def truth_forward(x_flat: Tensor, topk_idx: Tensor, topk_w: Tensor, experts, shared) -> Tensor:
    """The layer's output in fp64 from the same inputs: for every token,
    ``sum_k w_k * down(up(x) * silu(gate(x)))`` over its routed experts (the
    given routing and its renormalised weights, widened to fp64), plus the
    mean of the shared experts, with no rounding of any intermediate. The
    sum over experts runs in ascending expert order like the reference's
    ``index_add_`` (mlp.py:89-98), which in fp64 no longer changes the result
    at the tolerance in question. Returns ``[T, D]`` float64."""
    out = torch.zeros(x_flat.shape, dtype=torch.float64, device=x_flat.device)

    def mlp64(xe: Tensor, w) -> Tensor:
        g = xe @ w.gate.double().T
        u = xe @ w.up.double().T
        return (u * (g * torch.sigmoid(g))) @ w.down.double().T

    for e, w in enumerate(experts):
        tok, slot = (topk_idx.long() == e).nonzero(as_tuple=True)
        if tok.numel() == 0:
            continue
        y = mlp64(x_flat[tok].double(), w)
        out.index_add_(0, tok, y * topk_w[tok, slot].double().unsqueeze(-1))
    if len(shared):
        xs = x_flat.double()
        out += sum(mlp64(xs, w) for w in shared) / len(shared)
    return out


def truth_errors(out: Tensor, ref: Tensor, truth: Tensor, dtype: torch.dtype) -> dict:
    """Errors of the kernels' output ``out`` and the reference's ``ref``
    against the fp64 ``truth`` (all ``[T, D]``): failures of the plain
    tolerance around the truth, max normalised error and RMS error of each."""
    rtol, atol = tolerance(dtype)
    bound = atol + rtol * truth.abs()
    rep = {"truth_elements": truth.numel()}
    for name, t in (("kernel", out), ("ref", ref)):
        err = (t.double() - truth).abs()
        rep[f"truth_fail_{name}"] = int((err > bound).sum().item())
        rep[f"truth_max_norm_err_{name}"] = (err / bound).max().item() if err.numel() else 0.0
        rep[f"truth_rms_err_{name}"] = err.square().mean().sqrt().item() if err.numel() else 0.0
    return rep


def layer_parity(layer, x: Tensor, out: Tensor, topk_idx: Tensor | None = None, topk_w: Tensor | None = None,
                 sorted_token: Tensor | None = None, expert_offsets: Tensor | None = None,
                 truth_tokens: int | None = None) -> dict:
    """Compare ``out = layer(x)`` with the oracle evaluated on the layer's own
    parameters on x's device; optionally also the kernels' routing
    (``topk_idx [T, K]``, ``topk_w [T, K]``) and permutation
    (``sorted_token [T K]``, ``expert_offsets [E + 1]``) for the same input,
    and (``truth_tokens``: the first that many tokens, 0 or more than T for
    all) both outputs against the fp64 truth (``truth_errors``)."""
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
        if truth_tokens is not None:
            n = x_flat.shape[0] if truth_tokens <= 0 else min(truth_tokens, x_flat.shape[0])
            truth = truth_forward(x_flat[:n], trace.topk_idx[:n], trace.topk_w[:n], experts, shared)
            report.update(truth_errors(out.reshape(x_flat.shape)[:n], ref[:n], truth, x.dtype))
            report["truth_tokens"] = n
    return report
