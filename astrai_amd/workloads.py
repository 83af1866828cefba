"""Seeded synthetic MoE-layer workloads (shapes of the benchmark configurations).

Each workload fixes the layer shape, dtype, token count, router statistics and
seed. ``make_layer`` builds a ``DeepSeekMoE`` with ``n_shared_experts=0`` and
fills it from a seeded generator in this order: activations ``x ~ N(0, 1)``
``[B, S, D]``, router weight ``[E, D]``, then per expert gate ``[F, D]``, up
``[F, D]`` and down ``[D, F]`` weights ``~ N(0, 0.02)``, drawn in float32 and
cast to the workload dtype. Weights are drawn directly in nn.Linear
``[out, in]`` layout (i.i.d. entries, so the layout does not change the
distribution) and the expert parameters are views of one stacked tensor per
projection, so building the 2.8 GB Mixtral-shaped layer needs no extra copy.

Router statistics:
  * ``"std"``: router weight ~ N(0, router_std); with x ~ N(0, 1) the logits
    have standard deviation router_std * sqrt(D).
  * ``"zipf"``: as ``"std"`` plus a fixed per-expert router bias
    ``b_e = -zipf_scale * s * ln(rank_e)`` (log of Zipf(s) weights over a
    seeded random ranking of the experts), which concentrates tokens on the
    top-ranked experts and starves the tail.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn


@dataclass(frozen=True)
class Workload:
    name: str
    dtype: torch.dtype
    batch: int
    seq: int
    dim: int
    dim_ffn: int
    n_experts: int
    top_k: int
    seed: int
    router_std: float = 0.02
    zipf_s: float = 0.0
    zipf_scale: float = 0.0

    @property
    def n_tokens(self) -> int:
        return self.batch * self.seq

    @property
    def flops(self) -> float:
        """Algorithmic FLOPs of the expert GEMMs: 3 GEMMs of 2*D*F per routed row."""
        return 6.0 * self.n_tokens * self.top_k * self.dim * self.dim_ffn

    def describe(self) -> dict:
        return {
            "workload": self.name,
            "tokens": self.n_tokens,
            "batch": self.batch,
            "seq": self.seq,
            "dim": self.dim,
            "dim_ffn": self.dim_ffn,
            "n_experts": self.n_experts,
            "top_k": self.top_k,
            "dtype": str(self.dtype).replace("torch.", ""),
            "seed": self.seed,
        }


WORKLOADS = {
    w.name: w
    for w in [
        Workload("moe_fp32_d512_f1024_e8_k2_t1024", torch.float32, 1, 1024, 512, 1024, 8, 2, seed=0),
        Workload("moe_bf16_d2048_f1408_e64_k6_t8192", torch.bfloat16, 4, 2048, 2048, 1408, 64, 6, seed=1),
        Workload("moe_bf16_d2048_f1408_e64_k6_t8192_zipf", torch.bfloat16, 4, 2048, 2048, 1408, 64, 6, seed=2,
                 zipf_s=1.2, zipf_scale=1.2),
        Workload("moe_bf16_d4096_f14336_e8_k2_t16384", torch.bfloat16, 8, 2048, 4096, 14336, 8, 2, seed=3),
        Workload("moe_bf16_d4096_f1536_e128_k8_t64", torch.bfloat16, 64, 1, 4096, 1536, 128, 8, seed=4,
                 router_std=1.0 / 64.0),
        # batched decode / chunked prefill: 64 rows per expert on average (128-row tiles)
        Workload("moe_bf16_d4096_f1536_e128_k8_t1024", torch.bfloat16, 1024, 1, 4096, 1536, 128, 8, seed=5,
                 router_std=1.0 / 64.0),
    ]
}

# The Mixtral-shaped layer the headline throughput is quoted on.
HEADLINE = "moe_bf16_d4096_f14336_e8_k2_t16384"


def _randn(shape, gen, device, std, dtype):
    return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)


def zipf_bias(w: Workload, device) -> torch.Tensor | None:
    if w.zipf_s == 0.0:
        return None
    gen = torch.Generator().manual_seed(w.seed + 1000)
    rank = torch.randperm(w.n_experts, generator=gen) + 1
    bias = -w.zipf_scale * w.zipf_s * torch.log(rank.double())
    return bias.to(device=device, dtype=w.dtype)


def make_layer(w: Workload, device, gen_device=None, n_tokens: int | None = None):
    """Build ``(layer, x)`` for workload ``w`` on ``device``.

    ``gen_device`` selects the generator's device (default: ``device``);
    the values depend on it. ``n_tokens`` overrides the token count (rows of
    x, as ``[1, n_tokens, D]``) while keeping the workload's weights.
    """
    from astrai_amd.model.components.mlp import DeepSeekMoE

    device = torch.device(device)
    gen_device = torch.device(gen_device) if gen_device is not None else device
    gen = torch.Generator(device=gen_device).manual_seed(w.seed)
    E, D, F = w.n_experts, w.dim, w.dim_ffn
    if n_tokens is None:
        x_shape = (w.batch, w.seq, D)
    else:
        x_shape = (1, n_tokens, D)
    x = _randn(x_shape, gen, gen_device, 1.0, w.dtype).to(device)
    router = _randn((E, D), gen, gen_device, w.router_std, w.dtype).to(device)
    stacks = {}
    for name, shape in (("gate", (F, D)), ("up", (F, D)), ("down", (D, F))):
        stacks[name] = torch.empty((E, *shape), dtype=w.dtype, device=device)
    for e in range(E):
        for name in ("gate", "up", "down"):
            shape = stacks[name].shape[1:]
            stacks[name][e].copy_(_randn(shape, gen, gen_device, 0.02, w.dtype))

    with torch.device("meta"):
        layer = DeepSeekMoE(D, F, E, n_shared_experts=0, n_activated_experts=w.top_k)
    layer.router.weight = nn.Parameter(router, requires_grad=False)
    bias = zipf_bias(w, device)
    if bias is not None:
        layer.router.bias = nn.Parameter(bias, requires_grad=False)
    for e, m in enumerate(layer.routed_experts):
        m.gate.weight = nn.Parameter(stacks["gate"][e], requires_grad=False)
        m.up.weight = nn.Parameter(stacks["up"][e], requires_grad=False)
        m.down.weight = nn.Parameter(stacks["down"][e], requires_grad=False)
    return layer, x


def routing_stats(counts: torch.Tensor) -> dict:
    c = counts.double()
    mean = c.mean().item()
    return {
        "max_over_mean": (c.max().item() / mean) if mean > 0 else math.nan,
        "empty_experts": int((counts == 0).sum().item()),
        "max": int(counts.max().item()),
        "min": int(counts.min().item()),
    }
