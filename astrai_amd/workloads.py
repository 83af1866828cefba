"""Seeded synthetic MoE-layer workloads (shapes of the benchmark configurations).

Each workload fixes the layer shape, dtype, token count, router statistics and
seed. ``make_layer`` builds a ``DeepSeekMoE`` with ``n_shared_experts=0`` and
fills it from a CPU ``torch.Generator().manual_seed(seed)``, drawing in
float32 in this order, each tensor as ``torch.randn(shape)`` times its
standard deviation:

1. activations ``x [B, S, D] ~ N(0, 1)``;
2. router weight ``W_r [D, E] ~ N(0, router_std)``;
3. ``W_gate [E, D, F]``, 4. ``W_up [E, D, F]``, 5. ``W_down [E, F, D]``, all
   ``~ N(0, 0.02)``;

then casts each to the workload dtype (round to nearest even) and loads the
module as ``router.weight = W_r.T``, ``routed_experts[e].gate.weight =
W_gate[e].T``, ``.up.weight = W_up[e].T``, ``.down.weight = W_down[e].T``
(nn.Linear keeps ``[out, in]``). The fp32 workload (d512 / f1024, 8 experts,
top-2, 1024 tokens) is thus exactly "x ~ N(0,1); router weight [512, 8] and
expert weights W_gate / W_up [8, 512, 1024], W_down [8, 1024, 512] ~
N(0, 0.02); all from torch seed 0". The expert parameters are views of one
stacked tensor per projection.

Router statistics:
  * ``router_std``: with x ~ N(0, 1) the logits have standard deviation
    router_std * sqrt(D) (0.02 * sqrt(D) by default; 1 / sqrt(D) for the
    decode workloads, whose logits are ~ N(0, 1)).
  * ``zipf_s > 0``: a fixed per-expert router bias
    ``b_e = -zipf_scale * s * ln(rank_e)`` (log of Zipf(s) weights over a
    random ranking of the experts drawn from a separate CPU generator seeded
    ``seed + 1000``), which concentrates tokens on the top-ranked experts and
    starves the tail.
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
            "router_std": self.router_std,
            **({"zipf_s": self.zipf_s, "zipf_scale": self.zipf_scale} if self.zipf_s else {}),
            "generator": GENERATOR,
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


def zipf_bias(w: Workload, device) -> torch.Tensor | None:
    if w.zipf_s == 0.0:
        return None
    gen = torch.Generator().manual_seed(w.seed + 1000)
    rank = torch.randperm(w.n_experts, generator=gen) + 1
    bias = -w.zipf_scale * w.zipf_s * torch.log(rank.double())
    return bias.to(device=device, dtype=w.dtype)


GENERATOR = ("torch.Generator() on the CPU, manual_seed(seed); float32 draws in order x [B,S,D] ~ N(0,1), "
             "W_r [D,E] ~ N(0,router_std), W_gate [E,D,F], W_up [E,D,F], W_down [E,F,D] ~ N(0,0.02) (randn "
             "times the std), cast to dtype; router.weight = W_r.T, expert weights = W[e].T")


def make_layer(w: Workload, device, n_tokens: int | None = None):
    """Build ``(layer, x)`` for workload ``w`` on ``device`` (draws as in the
    module docstring). ``n_tokens`` keeps the workload's draws and takes the
    first ``n_tokens`` token rows (as ``[1, n_tokens, D]``), so the weights
    do not depend on it."""
    from astrai_amd.model.components.mlp import DeepSeekMoE

    device = torch.device(device)
    gen = torch.Generator().manual_seed(w.seed)
    E, D, F, T = w.n_experts, w.dim, w.dim_ffn, w.n_tokens
    if n_tokens is not None and not 0 <= n_tokens <= T:
        raise ValueError(f"n_tokens must be in [0, {T}] for {w.name}, got {n_tokens}")
    # one host buffer for every draw, touched once (first-touch page faults
    # of a fresh multi-GB allocation cost more than the draws)
    host = torch.zeros(max(T * D, D * E, E * D * F), dtype=torch.float32)

    def draw(shape, std):
        n = math.prod(shape)
        t = host[:n].view(shape)
        t.normal_(0.0, 1.0, generator=gen)  # torch.randn(shape, generator=gen)
        if std != 1.0:
            t.mul_(std)
        # copied off the shared buffer; the cast rounds to nearest even on either device
        return t.to(device, copy=True).to(w.dtype)

    x = draw((w.batch, w.seq, D), 1.0)
    if n_tokens is not None:
        x = x.reshape(T, D)[:n_tokens].reshape(1, n_tokens, D).clone()
    router = draw((D, E), w.router_std).t().contiguous()
    stacks = {name: draw(shape, 0.02).transpose(1, 2).contiguous()
              for name, shape in (("gate", (E, D, F)), ("up", (E, D, F)), ("down", (E, F, D)))}
    del host

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
