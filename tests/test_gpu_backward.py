"""Backward parity: gradients of DeepSeekMoE / MLP (HIP kernels forward and
backward, every shape and dtype) vs autograd through the oracle (the
reference's torch forward, mlp.py:14-25 and 64-100) with the same parameters,
input and output gradient, on the same device.

The input gradient is the reference's index_add_ order
(ascending expert) but autograd may add the router, shared and routed
contributions in another order, so everything is compared with the layer's
tolerance: elementwise |g - ref| <= atol + rtol * |ref| with atol scaled to
the tensor, >= 99.9 % of the elements passing and the worst error below 5 %
(bf16) / 1e-4 (fp32) of the largest magnitude. In bf16, atol is the larger of
1e-3 of the largest magnitude and two bf16 units in the last place at that
magnitude: an input gradient is a sum of top_k + shared + router terms, each
addition rounded to bf16 in an order autograd does not fix, so two roundings
at the largest magnitude are the resolution of the comparison (it matters on
small tensors, where a few cancelling elements are a whole permille). fp32
uses 1e-6 of the largest magnitude. Experts that receive no token must get no
gradient, as in the reference.
"""

from __future__ import annotations

import math

import pytest
import torch

from astrai_amd.model.components.mlp import MLP, DeepSeekMoE
from astrai_amd.workloads import WORKLOADS, make_layer
from oracle import moe_ref as R

pytestmark = pytest.mark.gpu


def _close(got, ref, dtype, label):
    assert got is not None and ref is not None, f"{label}: missing gradient"
    got, ref = got.float(), ref.float()
    scale = ref.abs().max().item() or 1.0
    if dtype == torch.bfloat16:
        ulp = 2.0 ** (math.floor(math.log2(scale)) - 7)  # bf16 spacing at the largest magnitude
        rtol, atol, worst_frac = 2e-2, max(1e-3 * scale, 2 * ulp), 5e-2
    else:
        rtol, atol, worst_frac = 1e-4, 1e-6 * scale, 1e-4
    err = (got - ref).abs()
    frac = (err <= atol + rtol * ref.abs()).float().mean().item()
    worst = err.max().item()
    assert frac >= 0.999, f"{label}: {frac:.5f} of elements within tolerance (max err {worst:.3e}, scale {scale:.3e})"
    assert worst <= worst_frac * scale, f"{label}: max err {worst:.3e} vs scale {scale:.3e}"


def _leaf(t):
    return t.detach().clone().requires_grad_(True)


def _oracle(layer, x, dout):
    rw = _leaf(layer.router.weight)
    rb = _leaf(layer.router.bias) if getattr(layer.router, "bias", None) is not None else None

    def ew(m):
        return R.ExpertWeights(_leaf(m.gate.weight), _leaf(m.up.weight), _leaf(m.down.weight))

    experts = [ew(m) for m in layer.routed_experts]
    shared = [ew(m) for m in layer.shared_experts]
    xl = _leaf(x)
    out = R.moe_forward(xl, rw, rb, experts, shared, layer.n_activated_experts)
    out.backward(dout)
    return out.detach(), xl.grad, rw.grad, (rb.grad if rb is not None else None), experts, shared


def _check_moe(layer, x, label, seed=0):
    g = torch.Generator(device=x.device).manual_seed(seed + 100)
    dout = torch.randn(x.shape, generator=g, device=x.device).to(x.dtype)
    ref_out, ref_dx, ref_drw, ref_drb, ref_exp, ref_shared = _oracle(layer, x, dout)
    layer.requires_grad_(True)
    layer.zero_grad(set_to_none=True)
    xl = _leaf(x)
    out = layer(xl)
    out.backward(dout)
    torch.cuda.synchronize()
    dt = x.dtype
    rtol = 2e-2 if dt == torch.bfloat16 else 1e-5
    assert torch.allclose(out.detach().float(), ref_out.float(), rtol=rtol, atol=rtol / 10) or \
        (out.detach().float() - ref_out.float()).abs().max() <= 0.05 * ref_out.float().abs().max()
    _close(xl.grad, ref_dx, dt, f"{label} dx")
    if layer.n_activated_experts == 1:
        # top-1: the renormalised weight w / w.sum() is identically 1, so the
        # router's gradient is zero in exact arithmetic and both sides hold
        # only rounding residue (in bf16 autograd rounds g / w and g w / w^2
        # apart, a bf16 unit per token; our dw rows differ from autograd's in
        # the last bit, so the residues differ): ours must be of the
        # reference's order, at most 4x its largest, or 1e-5 of dx
        floor = 1e-5 * ref_dx.float().abs().max().item()
        for name, got, ref in (("weight", layer.router.weight.grad, ref_drw),
                               ("bias", getattr(layer.router.bias, "grad", None), ref_drb)):
            if ref is not None:
                bound = max(4 * ref.float().abs().max().item(), floor)
                assert got is not None and got.float().abs().max().item() <= bound, \
                    f"{label} d router.{name}: {got.float().abs().max().item():.3e} exceeds the residue bound {bound:.3e}"
    else:
        _close(layer.router.weight.grad, ref_drw, dt, f"{label} d router.weight")
        if ref_drb is not None:
            _close(layer.router.bias.grad, ref_drb, dt, f"{label} d router.bias")
    n_none = 0
    for e, (m, r) in enumerate(zip(layer.routed_experts, ref_exp)):
        for name, got, want in (("gate", m.gate.weight.grad, r.gate.grad), ("up", m.up.weight.grad, r.up.grad),
                                ("down", m.down.weight.grad, r.down.grad)):
            if want is None:
                assert got is None, f"{label}: expert {e} has no rows but got a {name} gradient"
                n_none += 1
                continue
            _close(got, want, dt, f"{label} d expert{e}.{name}")
    for i, (m, r) in enumerate(zip(layer.shared_experts, ref_shared)):
        for name, got, want in (("gate", m.gate.weight.grad, r.gate.grad), ("up", m.up.weight.grad, r.up.grad),
                                ("down", m.down.weight.grad, r.down.grad)):
            _close(got, want, dt, f"{label} d shared{i}.{name}")
    return n_none


def _random_layer(gpu, dim, dim_ffn, n_exp, n_shared, top_k, dtype, seed=0, router_scale=1.0, bias=False):
    torch.manual_seed(seed)
    layer = DeepSeekMoE(dim, dim_ffn, n_exp, n_shared_experts=n_shared, n_activated_experts=top_k)
    for m in layer.modules():
        if hasattr(m, "reset_parameters"):
            m.reset_parameters()
    with torch.no_grad():
        layer.router.weight.mul_(router_scale)
    if bias:
        layer.router.bias = torch.nn.Parameter(torch.linspace(-1.0, 1.0, n_exp))
    return layer.to(device=gpu, dtype=dtype)


@pytest.mark.parametrize("dim,dim_ffn,n_exp,n_shared,top_k,dtype,bias", [
    (64, 128, 8, 0, 2, torch.float32, True),
    (96, 80, 6, 2, 3, torch.float32, False),
    (8, 16, 4, 1, 2, torch.bfloat16, False),   # the reference's tiny MoE test config
    (256, 512, 8, 1, 2, torch.bfloat16, False),
    (512, 256, 16, 0, 4, torch.bfloat16, True),
])
def test_moe_backward(gpu, dim, dim_ffn, n_exp, n_shared, top_k, dtype, bias):
    layer = _random_layer(gpu, dim, dim_ffn, n_exp, n_shared, top_k, dtype, bias=bias)
    g = torch.Generator(device=gpu).manual_seed(3)
    x = torch.randn(2, 61, dim, generator=g, device=gpu).to(dtype)
    _check_moe(layer, x, f"d{dim}_f{dim_ffn}_e{n_exp}_s{n_shared}_k{top_k}_{dtype}")


@pytest.mark.parametrize("dim", [120, 256])  # general-shape / matrix-core backward kernels
def test_moe_backward_empty_experts(gpu, dim):
    # a sharp router leaves most of the 32 experts without tokens
    layer = _random_layer(gpu, dim, 256, 32, 0, 2, torch.bfloat16, router_scale=40.0, bias=True)
    with torch.no_grad():
        layer.router.bias.copy_(torch.linspace(-30.0, 30.0, 32, device=gpu))
    x = torch.randn(1, 40, dim, device=gpu).to(torch.bfloat16)
    n_none = _check_moe(layer, x, "empty experts")
    assert n_none >= 3 * 10


def test_moe_backward_workload_rows(gpu):
    # the fine-grained workload's weights with 2048 tokens (256-row GEMM tiles)
    layer, x = make_layer(WORKLOADS["moe_bf16_d2048_f1408_e64_k6_t8192"], gpu, n_tokens=2048)
    _check_moe(layer, x, "d2048_f1408_e64_k6 t2048")


@pytest.mark.parametrize("dim,dim_ffn,dtype,n_shared", [
    (256, 384, torch.bfloat16, 1), (192, 320, torch.bfloat16, 2), (64, 96, torch.float32, 1),
    (256, 384, torch.bfloat16, 0),
])
def test_moe_backward_zero_tokens(gpu, dim, dim_ffn, dtype, n_shared):
    # an empty batch differentiates as autograd through the reference does: every routed expert is
    # skipped, so only shared experts connect the output to x and to parameters (zero gradients);
    # without them the output carries no graph at all
    layer = _random_layer(gpu, dim, dim_ffn, 8, n_shared, 2, dtype)
    x = torch.randn(2, 0, dim, device=gpu, dtype=dtype)
    layer.requires_grad_(True)
    layer.zero_grad(set_to_none=True)
    xl = _leaf(x)
    out = layer(xl)
    assert out.shape == x.shape
    if n_shared == 0:
        rw = _leaf(layer.router.weight)
        ref = R.moe_forward(_leaf(x), rw, None, [R.ExpertWeights(_leaf(m.gate.weight), _leaf(m.up.weight),
                                                                  _leaf(m.down.weight)) for m in layer.routed_experts],
                            [], layer.n_activated_experts)
        assert not ref.requires_grad and not out.requires_grad
        return
    dout = torch.zeros_like(x)
    ref_out, ref_dx, ref_drw, _, ref_exp, ref_shared = _oracle(layer, x, dout)
    out.backward(dout)
    torch.cuda.synchronize()
    assert xl.grad is not None and xl.grad.shape == x.shape

    def same(got, want, label):
        if want is None:
            assert got is None, f"{label}: gradient where the reference has none"
        else:
            assert got is not None and got.shape == want.shape, f"{label}: missing gradient"
            assert torch.equal(got, torch.zeros_like(got)), f"{label}: nonzero gradient from zero rows"

    same(layer.router.weight.grad, ref_drw, "router.weight")
    for group, mods, refs in (("expert", layer.routed_experts, ref_exp), ("shared", layer.shared_experts, ref_shared)):
        for i, (m, r) in enumerate(zip(mods, refs)):
            for name, got, want in (("gate", m.gate.weight.grad, r.gate.grad), ("up", m.up.weight.grad, r.up.grad),
                                    ("down", m.down.weight.grad, r.down.grad)):
                same(got, want, f"{group}{i}.{name}")


@pytest.mark.parametrize("dim,dim_ffn", [(40, 24), (192, 320), (256, 384)])  # general-shape / matrix-core kernels
def test_mlp_backward(gpu, dim, dim_ffn):
    torch.manual_seed(1)
    mlp = MLP(dim, dim_ffn).to(device=gpu, dtype=torch.bfloat16)
    for m in mlp.modules():
        if hasattr(m, "reset_parameters"):
            m.reset_parameters()
    x = torch.randn(3, 50, dim, device=gpu).to(torch.bfloat16)
    dout = torch.randn(3, 50, dim, device=gpu).to(torch.bfloat16)
    w = R.ExpertWeights(_leaf(mlp.gate.weight), _leaf(mlp.up.weight), _leaf(mlp.down.weight))
    xr = _leaf(x)
    R.expert_mlp(xr, w).backward(dout)
    xl = _leaf(x)
    mlp(xl).backward(dout)
    torch.cuda.synchronize()
    _close(xl.grad, xr.grad, torch.bfloat16, "mlp dx")
    for name, got, want in (("gate", mlp.gate.weight.grad, w.gate.grad), ("up", mlp.up.weight.grad, w.up.grad),
                            ("down", mlp.down.weight.grad, w.down.grad)):
        _close(got, want, torch.bfloat16, f"mlp d{name}")


@pytest.mark.parametrize("dim,dim_ffn,dtype", [
    (256, 256, torch.bfloat16),  # matrix-core kernels
    (40, 24, torch.bfloat16),  # general-shape kernels
    (64, 96, torch.float32),
])
def test_backward_runs_the_grouped_kernels(gpu, monkeypatch, dim, dim_ffn, dtype):
    # every shape and dtype differentiates on the grouped HIP kernels: no
    # torch recompute of the experts (no F.linear call) in the backward
    from astrai_amd.extension import ops

    calls = []
    for name in ("moe_row_grad", "moe_gemm_dgrad_down", "moe_gemm_dgrad_gate_up", "moe_gemm_wgrad"):
        fn = getattr(ops, name)
        monkeypatch.setattr(ops, name, lambda *a, _fn=fn, _n=name, **k: (calls.append(_n), _fn(*a, **k))[1])
    layer = _random_layer(gpu, dim, dim_ffn, 8, 1, 2, dtype)
    x = torch.randn(1, 300, dim, device=gpu).to(dtype).requires_grad_(True)
    out = layer(x).sum()
    linear_calls = []
    real_linear = torch.nn.functional.linear
    monkeypatch.setattr(torch.nn.functional, "linear", lambda *a, **k: (linear_calls.append(1), real_linear(*a, **k))[1])
    out.backward()
    torch.cuda.synchronize()
    # routed: row grad, 2 dgrad, 3 wgrad; shared: 2 dgrad, 3 wgrad
    assert calls.count("moe_row_grad") == 1
    assert calls.count("moe_gemm_wgrad") == 6
    assert calls.count("moe_gemm_dgrad_down") == 2 and calls.count("moe_gemm_dgrad_gate_up") == 2
    assert not linear_calls, "the backward recomputed an expert with torch"


@pytest.mark.parametrize("dim,dim_ffn,n_exp,n_shared,top_k,dtype", [
    (37, 30, 6, 1, 2, torch.bfloat16),  # dim_ffn % 4 == 2
    (13, 7, 4, 2, 3, torch.float32),  # dim_ffn % 4 == 3
    (65, 129, 8, 0, 2, torch.float32),  # dim_ffn % 4 == 1
    (24, 40, 5, 1, 5, torch.bfloat16),  # top_k == n_experts
])
def test_moe_backward_odd_shapes(gpu, dim, dim_ffn, n_exp, n_shared, top_k, dtype):
    layer = _random_layer(gpu, dim, dim_ffn, n_exp, n_shared, top_k, dtype, seed=dim)
    g = torch.Generator(device=gpu).manual_seed(dim_ffn)
    x = torch.randn(2, 45, dim, generator=g, device=gpu).to(dtype)
    _check_moe(layer, x, f"d{dim}_f{dim_ffn}_e{n_exp}_s{n_shared}_k{top_k}_{dtype}")


def test_inference_mode_has_no_graph(gpu):
    layer = _random_layer(gpu, 64, 128, 4, 1, 2, torch.bfloat16)
    x = torch.randn(1, 8, 64, device=gpu).to(torch.bfloat16)
    with torch.inference_mode():
        out = layer(x)
    assert out.grad_fn is None


def _random_bwd_configs(n, seed):
    import random

    rnd = random.Random(seed)
    out = []
    for _ in range(n):
        if rnd.random() < 0.6:  # grouped backward kernels (bf16, matrix-core shapes)
            dim, dim_ffn, dtype = 64 * rnd.randint(1, 12), 64 * rnd.randint(1, 10), torch.bfloat16
        else:  # general-shape backward kernels (also matrix-core ones where both dims are multiples of 64)
            dim, dim_ffn = 8 * rnd.randint(1, 24), 8 * rnd.randint(1, 24)
            dtype = rnd.choice([torch.bfloat16, torch.float32])
        n_exp = rnd.choice([1, 2, 4, 8, 16, 32])
        top_k = rnd.randint(1, min(n_exp, 6))
        out.append((dim, dim_ffn, n_exp, rnd.choice([0, 1, 2]), top_k, dtype, rnd.choice([3, 40, 130, 600])))
    return out


@pytest.mark.parametrize("dim,dim_ffn,n_exp,n_shared,top_k,dtype,n_tok", _random_bwd_configs(10, seed=77))
def test_moe_backward_random_shapes(gpu, dim, dim_ffn, n_exp, n_shared, top_k, dtype, n_tok):
    layer = _random_layer(gpu, dim, dim_ffn, n_exp, n_shared, top_k, dtype, seed=n_tok)
    g = torch.Generator(device=gpu).manual_seed(n_tok + dim)
    x = torch.randn(1, n_tok, dim, generator=g, device=gpu).to(dtype)
    _check_moe(layer, x, f"d{dim}_f{dim_ffn}_e{n_exp}_s{n_shared}_k{top_k}_{dtype}_t{n_tok}")
