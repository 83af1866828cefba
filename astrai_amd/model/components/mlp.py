"""Drop-in MoE FFN layer running on the MI355X HIP kernels.

Keeps the module contract of the reference's ``astrai/model/components/
mlp.py``:

* ``FFNFactory`` with ``"mlp"`` -> ``MLP`` and ``"moe"`` -> ``DeepSeekMoE``
  (``mlp.py:10-28``), created through kwarg-filtering ``create``;
* ``DeepSeekMoE(dim, dim_ffn, n_routed_experts, n_shared_experts=1,
  n_activated_experts=2, topk_method="greedy", n_layers=1)`` with the same
  child modules and therefore the same ``state_dict`` keys:
  ``router.weight``, ``shared_experts.{i}.{up,gate,down}.weight``,
  ``routed_experts.{e}.{up,gate,down}.weight`` (``mlp.py:47-62``), and the
  same init scales;
* ``forward(x [B, S, D]) -> [B, S, D]`` in x's dtype (``mlp.py:64-72``).

The router GEMM stays ``self.router(x)`` (``F.linear``, ``mlp.py:83``), so
the logits are the reference's by construction; everything after it — softmax,
top-k, renormalisation, permutation, the expert SwiGLU GEMMs, the weighted
combine and the shared-expert mean — runs in the HIP kernels of
``astrai_amd.extension`` with the reference's rounding points.

The HIP path is the only path: inputs it cannot take (CPU tensors, dtypes
other than float32/bfloat16, experts whose ``up/gate/down`` are not bias-free
``Linear`` modules, e.g. after LoRA injection) raise instead of silently
running something else. With autograd active the forward still runs on the
kernels and so does the backward (grouped dgrad / wgrad kernels,
``autograd.py``).
"""

from __future__ import annotations

from functools import partial
from itertools import chain
from operator import attrgetter, is_not, itemgetter, methodcaller

import torch
import torch.nn as nn
from torch import Tensor

from astrai_amd.extension import ops
from astrai_amd.factory import BaseFactory
from astrai_amd.model.components.autograd import DenseExpert, EmptyBatch, RoutedExperts, routing_weights
from astrai_amd.model.components.linear import Linear


class FFNFactory(BaseFactory[nn.Module]):
    pass


def _check_gpu_input(x: Tensor, params: list[Tensor], who: str) -> None:
    if x.device.type != "cuda":
        raise RuntimeError(f"{who} runs on the HIP kernels and needs a ROCm device tensor, got {x.device}")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"{who} supports float32 and bfloat16 activations, got {x.dtype}")
    for p in params:
        if p.device != x.device or p.dtype != x.dtype:
            raise RuntimeError(f"{who}: parameters must be on {x.device} in {x.dtype}, found {p.device}/{p.dtype}")


def _needs_grad(x: Tensor, params: list[Tensor]) -> bool:
    return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in params))


def _plain_linear(m: nn.Module, who: str) -> Tensor:
    if type(m) is not Linear or m.bias is not None:
        raise RuntimeError(f"{who}: expert projections must be bias-free Linear modules, got {type(m).__name__}")
    return m.weight


@FFNFactory.register("mlp")
class MLP(nn.Module):
    """Dense SwiGLU expert ``down(up(x) * silu(gate(x)))`` (``mlp.py:14-25``)."""

    def __init__(self, dim: int, dim_ffn: int, down_init_std: float = 0.02):
        super().__init__()
        self.up = Linear(dim, dim_ffn)
        self.gate = Linear(dim, dim_ffn)
        self.down = Linear(dim_ffn, dim, init_std=down_init_std)

    def weights(self) -> tuple[Tensor, Tensor, Tensor]:
        return (
            _plain_linear(self.gate, "MLP"),
            _plain_linear(self.up, "MLP"),
            _plain_linear(self.down, "MLP"),
        )

    def _weight_tables(self, wg: Tensor, wu: Tensor, wd: Tensor) -> tuple[Tensor, Tensor, Tensor]:
        """One-entry device pointer tables of the three weights, rebuilt only
        when a weight's storage moves (a pageable host-to-device copy each)."""
        key = (wg.data_ptr(), wu.data_ptr(), wd.data_ptr())
        if getattr(self, "_table_key", None) != key:
            self._tables = tuple(ops.expert_weight_table([w], tuple(w.shape)) for w in (wg, wu, wd))
            self._table_key = key
        return self._tables

    def forward(self, x: Tensor) -> Tensor:
        wg, wu, wd = self.weights()
        _check_gpu_input(x, [wg, wu, wd], "MLP")
        lead, dim = x.shape[:-1], x.shape[-1]
        x2 = x.reshape(-1, dim).contiguous()
        tables = self._weight_tables(wg, wu, wd)
        if _needs_grad(x2, [wg, wu, wd]):
            out = DenseExpert.apply(x2, tables, wg.shape[0], wg, wu, wd)
        else:
            out = ops.moe_dense_mlp(x2, *tables, wg.shape[0])
        return out.view(*lead, dim)


_modules_of = attrgetter("_modules")
_params_of = attrgetter("_parameters")
_weight_of = itemgetter("weight")
_bias_of = methodcaller("get", "bias")
_is_set = partial(is_not, None)
_requires_grad = attrgetter("requires_grad")


class _ExpertState:
    """A DeepSeekMoE's validated expert weights (routed and shared, each as
    gate, up, down lists), their dtype and device, and the device pointer
    tables built from them; ``sig`` identifies the modules, parameter objects
    and storages they were read from."""

    __slots__ = ("sig", "ptrs", "routed", "shared", "flat", "dtype", "device", "tables")

    def __init__(self, sig, ptrs, routed, shared, flat, dtype, device, tables):
        self.sig, self.ptrs, self.routed, self.shared, self.flat = sig, ptrs, routed, shared, flat
        self.dtype, self.device, self.tables = dtype, device, tables


@FFNFactory.register("moe")
class DeepSeekMoE(nn.Module):
    def __init__(
        self,
        dim: int,
        dim_ffn: int,
        n_routed_experts: int,
        n_shared_experts: int = 1,
        n_activated_experts: int = 2,
        topk_method: str = "greedy",
        n_layers: int = 1,
    ):
        super().__init__()
        self.dim = dim
        self.n_routed_experts = n_routed_experts
        self.n_shared_experts = n_shared_experts
        self.n_activated_experts = n_activated_experts
        self.topk_method = topk_method

        self.router = Linear(dim, n_routed_experts, bias=False)
        moe_scale = 1 / max(n_shared_experts, 1) + 1 / n_activated_experts
        down_init_std = 0.02 / (2 * n_layers * moe_scale) ** 0.5
        self.shared_experts = nn.ModuleList(
            [MLP(dim, dim_ffn, down_init_std=down_init_std) for _ in range(n_shared_experts)]
        )
        self.routed_experts = nn.ModuleList(
            [MLP(dim, dim_ffn, down_init_std=down_init_std) for _ in range(n_routed_experts)]
        )
        # The experts' validated weights and their device pointer tables
        # (_current; not part of the state_dict).
        self._state: _ExpertState | None = None
        # Opt-in, inference only: keep a packed copy of the routed experts'
        # weights in the order the GEMMs stage it (ops.moe_pack_*), rebuilt
        # when a weight moves or changes (its version counter), for bf16 shapes
        # the packed GEMMs take. Same results; doubles the routed weights'
        # memory for about 1 % less GEMM time (3 % on the down GEMM of
        # decode-sized loads), so it is off by default.
        self.pack_weights = False
        self._packed: tuple | None = None

    # -- weights and their pointer tables ----------------------------------------
    def _expert_weights(self, experts: nn.ModuleList) -> tuple[list[Tensor], list[Tensor], list[Tensor]]:
        g, u, d = [], [], []
        for e in experts:
            wg, wu, wd = e.weights()
            g.append(wg)
            u.append(wu)
            d.append(wd)
        return g, u, d

    def _current(self, dtype: torch.dtype, device: torch.device) -> _ExpertState:
        """The experts' current weights and their device pointer tables.

        Reading every expert weight through ``nn.Module`` attribute lookup
        costs a few µs per expert on the host (at 128 experts ~0.6 ms per
        forward, as much as the decode step's kernels). Here the modules'
        registries (``_modules``, ``_parameters``) are read with C-level
        ``map`` calls, and the full validation (bias-free ``Linear``
        projections, one dtype and device) runs again only when a module, a
        parameter object or a weight's storage differs from the last call. The
        pointer tables are rebuilt only when a storage moved, so graphs
        captured earlier keep valid tables. Every weight must be on ``device``
        in ``dtype`` (the input's)."""
        sig = None
        try:
            lins = []
            for experts in (self.routed_experts, self.shared_experts):
                children = list(map(_modules_of, experts._modules.values()))
                lins += [list(map(itemgetter(n), children)) for n in ("gate", "up", "down")]
            flat = list(chain.from_iterable(lins))
            pdicts = list(map(_params_of, flat))
            weights = list(map(_weight_of, pdicts))
            if not any(map(_is_set, map(_bias_of, pdicts))):
                sig = (tuple(map(id, flat)), tuple(map(id, weights)), tuple(map(Tensor.data_ptr, weights)))
        except (KeyError, AttributeError, TypeError):
            sig = None
        st = self._state
        if st is not None and sig is not None and sig == st.sig and st.dtype == dtype and st.device == device:
            return st
        routed = self._expert_weights(self.routed_experts)  # raises on non-Linear or biased projections
        shared = self._expert_weights(self.shared_experts)
        flat_w = [w for ws in (*routed, *shared) for w in ws]
        for w in flat_w:
            if w.device != device or w.dtype != dtype:
                raise RuntimeError(f"DeepSeekMoE: parameters must be on {device} in {dtype}, found {w.device}/{w.dtype}")
        ptrs = tuple(w.data_ptr() for w in flat_w)
        if st is not None and st.ptrs == ptrs:
            tables = st.tables
        else:
            shape_in = tuple(routed[0][0].shape)
            shape_out = tuple(routed[2][0].shape)
            t_routed = (
                ops.expert_weight_table(routed[0], shape_in),
                ops.expert_weight_table(routed[1], shape_in),
                ops.expert_weight_table(routed[2], shape_out),
            )
            t_shared = tuple(
                tuple(ops.expert_weight_table([w], tuple(w.shape)) for w in (shared[0][i], shared[1][i], shared[2][i]))
                for i in range(len(shared[0]))
            )
            tables = (t_routed, t_shared)
        self._state = _ExpertState(sig, ptrs, routed, shared, flat_w, dtype, device, tables)
        return self._state

    def _weight_tables(self) -> tuple[Tensor, ...]:
        """(routed gate, up, down tables), per shared expert (gate, up, down),
        for the weights' own dtype and device."""
        w = self.routed_experts[0].gate.weight
        return self._current(w.dtype, w.device).tables

    def _packed_tables(self, dtype: torch.dtype, st: _ExpertState) -> tuple[Tensor, Tensor] | None:
        """Pointer tables of the packed gate/up and down copies, or None when
        this forward reads the live weights. The copies are rebuilt whenever a
        routed weight's storage or version counter changes; the cache holds a
        view of each source weight so that its storage (and address) cannot be
        reused by another tensor while the copy made from it is in use."""
        if not self.uses_packed_weights(dtype):
            return None
        g, u, d = st.routed
        srcs = [w for ws in (g, u, d) for w in ws]
        if any(w.is_inference() for w in srcs):  # no version counter to follow
            return None
        c = self._packed
        if (c is None or len(c[0]) != len(srcs)
                or any(s.data_ptr() != w.data_ptr() or v != w._version for s, v, w in zip(c[0], c[1], srcs))):
            self._packed = None  # release the stale copies before packing
            gu = [ops.moe_pack_gate_up(wg, wu) for wg, wu in zip(g, u)]
            dn = [ops.moe_pack_down(wd) for wd in d]
            self._packed = (tuple(w.detach() for w in srcs), tuple(w._version for w in srcs), gu, dn,
                            ops.expert_weight_table(gu, tuple(gu[0].shape)),
                            ops.expert_weight_table(dn, tuple(dn[0].shape)))
        return self._packed[4], self._packed[5]

    def uses_packed_weights(self, dtype: torch.dtype) -> bool:
        """Whether an inference forward in ``dtype`` reads packed weights."""
        dim_ffn = self.routed_experts[0].up.weight.shape[0]
        return self.pack_weights and ops.packed_supported(self.dim, dim_ffn, dtype)

    # -- forward ----------------------------------------------------------------
    def forward(self, x: Tensor) -> Tensor:
        bsz, seq_len, dim = x.shape
        # the reference's view (mlp.py:66), then a dense copy when the view is
        # strided (e.g. a slice of a wider buffer): the kernels take dense rows
        x_flat = x.view(-1, dim).contiguous()
        router_w = self.router.weight
        _check_gpu_input(x_flat, [router_w], "DeepSeekMoE")
        st = self._current(x_flat.dtype, x_flat.device)
        if torch.is_grad_enabled() and (x_flat.requires_grad or router_w.requires_grad
                                        or any(map(_requires_grad, st.flat))):
            return self._forward_autograd(x_flat, st).view(bsz, seq_len, dim)
        shared_out = self._shared_forward(x_flat, st)
        out = self._routed_forward(x_flat, st, shared_out)
        return out.view(bsz, seq_len, dim)

    def _shared_forward(self, x: Tensor, st: _ExpertState) -> Tensor | None:
        """Each shared expert's output stacked as ``[n_shared, T, D]``; the
        mean (``mlp.py:77``) is taken inside the combine kernel. ``None`` for
        ``n_shared_experts == 0`` (the reference's ``zeros_like``)."""
        if self.n_shared_experts == 0 or x.shape[0] == 0:
            return None
        _, t_shared = st.tables
        dim_ffn = st.shared[1][0].shape[0]
        out = torch.empty(self.n_shared_experts, x.shape[0], x.shape[1], dtype=x.dtype, device=x.device)
        # one tile list for every shared expert: they run over the same rows
        tiles = ops.dense_tiles(x.shape[0], ops.dense_block_m(x.shape[0], x.shape[1], dim_ffn, x.dtype), x.device)
        for i, (tg, tu, td) in enumerate(t_shared):
            ops.moe_dense_mlp(x, tg, tu, td, dim_ffn, out=out[i], tiles=tiles)
        return out

    def _routed_forward(self, x: Tensor, st: _ExpertState, shared: Tensor | None = None) -> Tensor:
        dim_ffn = st.routed[1][0].shape[0]
        packed_tables = self._packed_tables(x.dtype, st)
        packed = packed_tables is not None
        if packed:
            tg, td = packed_tables
            tu = tg
        else:
            tg, tu, td = st.tables[0]
        logits = self.router(x)
        return ops.moe_routed_forward(x, logits, tg, tu, td, dim_ffn, self.n_activated_experts, shared,
                                      packed=packed)

    def _forward_autograd(self, x: Tensor, st: _ExpertState) -> Tensor:
        """mlp.py:64-100 with autograd: HIP kernels forward and backward.
        Routing indices come from the route kernel; the weights are rebuilt
        from the logits with torch ops (same values) so their gradient reaches
        the router."""
        n_tokens = x.shape[0]
        if n_tokens == 0:
            # the reference's routed output is a graph-less zeros here; only
            # shared experts connect the output to x and to parameters
            if self.n_shared_experts == 0:
                return x.new_zeros(0, x.shape[1])
            return EmptyBatch.apply(x, *[w for ws in st.shared for w in ws])
        t_routed, t_shared = st.tables
        routed_w = st.routed
        dim_ffn = routed_w[0][0].shape[0]
        logits = self.router(x)
        route = ops.moe_route(logits.detach(), self.n_activated_experts)
        topk_w = routing_weights(logits, route.topk_idx, x.dtype)
        routed = RoutedExperts.apply(x, topk_w, route.topk_idx, route.chunk_hist, t_routed, dim_ffn,
                                     *routed_w[0], *routed_w[1], *routed_w[2])
        if self.n_shared_experts == 0:
            return routed
        shared_w = st.shared
        shared = sum(
            DenseExpert.apply(x, t_shared[i], dim_ffn, shared_w[0][i], shared_w[1][i], shared_w[2][i])
            for i in range(self.n_shared_experts)
        ) / self.n_shared_experts
        return shared + routed
