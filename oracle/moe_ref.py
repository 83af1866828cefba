"""ORACLE — test infrastructure only. Restatement of AstrAI's MoE forward.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s checker legs
(the CPU baseline and the parity report, through ``oracle/parity.py``) may
import this module, and only as the checker (or, for the CPU baseline, as the
reference path being timed). The product path (``astrai_amd``) never imports
it.

What it restates: ``astrai/model/components/mlp.py:14-25`` (MLP) and
``:64-100`` (DeepSeekMoE.forward / _shared_forward / _routed_forward), with
``Linear.forward = F.linear`` (``astrai/model/components/linear.py:23-24``).
The reference's arithmetic is a composition of torch ops, so the restatement
uses the same torch ops in the same order — the order and the dtype of every
intermediate are what fix the rounding points the HIP kernels must
reproduce. It runs on any device: on the GPU it yields the reference's
results on the same device (bit-level parity targets); on the CPU it is the
reference's CPU path (the timed baseline).

Pinning (tests/test_oracle_pins.py): fp64 brute force on small inputs,
closed-form special cases (single expert, one-hot routing, uniform routing,
K = 1), a brute-force stable sort for the permutation, a rounding-point
emulation, and planted-mistake variants of this module that those checks must
reject. The reference ships no golden vectors or fixtures for this path, so
nothing else pins it.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch
import torch.nn.functional as F
from torch import Tensor


@dataclass
class ExpertWeights:
    """One SwiGLU expert in nn.Linear layout: gate/up ``[F, D]``, down ``[D, F]``."""

    gate: Tensor
    up: Tensor
    down: Tensor


def expert_mlp(x: Tensor, w: ExpertWeights) -> Tensor:
    """``down(up(x) * silu(gate(x)))`` — mlp.py:22-25 (up is evaluated first
    as in the reference's expression; each F.linear rounds to x.dtype)."""
    up = F.linear(x, w.up)
    gated = up * F.silu(F.linear(x, w.gate))
    return F.linear(gated, w.down)


def router_probs(logits: Tensor, dtype: torch.dtype) -> Tensor:
    """mlp.py:84 — fp32 softmax over experts, rounded to the activation dtype."""
    return torch.softmax(logits.float(), dim=-1).to(dtype)


def route(logits: Tensor, top_k: int, dtype: torch.dtype) -> tuple[Tensor, Tensor]:
    """mlp.py:84-87 — (renormalised top-k weights, top-k expert ids int64)."""
    probs = router_probs(logits, dtype)
    weights, idx = torch.topk(probs, top_k, dim=-1)
    weights = weights / weights.sum(dim=-1, keepdim=True)
    return weights, idx


def permutation(topk_idx: Tensor, n_experts: int) -> tuple[Tensor, Tensor, Tensor]:
    """mlp.py:90-93 — concatenation over e of ``(topk_idx == e).nonzero()``.

    Returns (token of each permuted row, slot of each row, expert offsets
    ``[E + 1]``), all int64 on topk_idx's device.
    """
    toks, slots, counts = [], [], []
    for e in range(n_experts):
        t, s = (topk_idx == e).nonzero(as_tuple=True)
        toks.append(t)
        slots.append(s)
        counts.append(t.numel())
    offsets = torch.zeros(n_experts + 1, dtype=torch.int64)
    offsets[1:] = torch.cumsum(torch.tensor(counts, dtype=torch.int64), 0)
    dev = topk_idx.device
    empty = torch.empty(0, dtype=torch.int64, device=dev)
    return (torch.cat(toks) if toks else empty, torch.cat(slots) if slots else empty, offsets.to(dev))


@dataclass
class RoutedTrace:
    """Intermediates of one routed forward, for parity checks."""

    logits: Tensor
    topk_w: Tensor
    topk_idx: Tensor
    expert_out: list  # per expert: (token_idx, slot_idx, weighted rows y*w) or None
    out: Tensor


def routed_forward(x: Tensor, router_w: Tensor, router_b: Tensor | None, experts: Sequence[ExpertWeights],
                   top_k: int, trace: bool = False):
    """mlp.py:79-100 for ``x [N, D]``."""
    n_tok, dim = x.shape
    logits = F.linear(x, router_w, router_b)
    topk_w, topk_idx = route(logits, top_k, x.dtype)
    out = torch.zeros(n_tok, dim, device=x.device, dtype=x.dtype)
    per_expert = []
    for e, w in enumerate(experts):
        tok, slot = (topk_idx == e).nonzero(as_tuple=True)
        if tok.numel() == 0:
            per_expert.append(None)
            continue
        y = expert_mlp(x[tok], w)
        yw = y * topk_w[tok, slot].unsqueeze(-1)
        out.index_add_(0, tok, yw)
        per_expert.append((tok, slot, yw) if trace else None)
    if trace:
        return RoutedTrace(logits, topk_w, topk_idx, per_expert, out)
    return out


def shared_forward(x: Tensor, shared: Sequence[ExpertWeights]) -> Tensor:
    """mlp.py:74-77 — zeros, or the mean of the shared experts (Python sum)."""
    if len(shared) == 0:
        return torch.zeros_like(x)
    return sum(expert_mlp(x, w) for w in shared) / len(shared)


def moe_forward(x: Tensor, router_w: Tensor, router_b: Tensor | None, experts: Sequence[ExpertWeights],
                shared: Sequence[ExpertWeights], top_k: int) -> Tensor:
    """mlp.py:64-72 for ``x [B, S, D]``."""
    bsz, seq_len, dim = x.shape
    x_flat = x.view(-1, dim)
    out = shared_forward(x_flat, shared) + routed_forward(x_flat, router_w, router_b, experts, top_k)
    return out.view(bsz, seq_len, dim)


def module_weights(moe) -> tuple[Tensor, Tensor | None, list[ExpertWeights], list[ExpertWeights]]:
    """Read the parameters of a DeepSeekMoE-like module (router, routed and
    shared experts with ``up/gate/down`` Linear children)."""

    def ew(m):
        return ExpertWeights(m.gate.weight.detach(), m.up.weight.detach(), m.down.weight.detach())

    rb = moe.router.bias.detach() if getattr(moe.router, "bias", None) is not None else None
    return (moe.router.weight.detach(), rb, [ew(m) for m in moe.routed_experts], [ew(m) for m in moe.shared_experts])


def module_forward(moe, x: Tensor) -> Tensor:
    """The reference forward evaluated on a module's parameters."""
    rw, rb, experts, shared = module_weights(moe)
    with torch.no_grad():
        return moe_forward(x, rw, rb, experts, shared, moe.n_activated_experts)
