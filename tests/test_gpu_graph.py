"""HIP-graph capture of the layer forward (serving loops replay captured
decode steps). The whole forward — router GEMM, route, permute, grouped GEMMs,
combine, and the shared experts' dense tile list — is captured on one stream
after a warm-up call (which builds the weight-pointer tables), then replayed
several times with eager work in between. Every replay must equal the eager
result bit for bit, and must match the oracle (the reference's torch forward,
mlp.py:64-100, on the same device): bit-exact routing, and the layer
tolerance per expert term plus >= 99.9 % plain allclose. A replay after the
input buffer is refilled must equal the eager result on the new input and
match the oracle on it.
"""

from __future__ import annotations

import pytest
import torch

from astrai_amd.extension import ops
from astrai_amd.model.components.mlp import DeepSeekMoE
from astrai_amd.workloads import WORKLOADS, make_layer
from oracle import parity as P

pytestmark = pytest.mark.gpu


def _layer(gpu, dim, dim_ffn, n_exp, n_shared, top_k, dtype):
    torch.manual_seed(0)
    layer = DeepSeekMoE(dim, dim_ffn, n_exp, n_shared_experts=n_shared, n_activated_experts=top_k)
    for m in layer.modules():
        if hasattr(m, "reset_parameters"):
            m.reset_parameters()
    return layer.to(device=gpu, dtype=dtype).requires_grad_(False)


def _assert_oracle(layer, x, out, label):
    logits = layer.router(x.view(-1, x.shape[-1]))
    res = ops.moe_route(logits, layer.n_activated_experts)
    rep = P.layer_parity(layer, x, out, res.topk_idx, res.topk_w)
    torch.cuda.synchronize()
    print(f"{label}: allclose={rep['allclose_frac']:.6f} worst(err-bound)={rep['term_bound_excess']:.3e}")
    assert rep["routing_bit_exact"], f"{label}: routing differs from the reference"
    assert rep["term_bound_excess"] <= 0, f"{label}: error exceeds the per-term tolerance"
    assert rep["allclose_frac"] >= 0.999, f"{label}: allclose pass fraction {rep['allclose_frac']}"


def _capture(layer, static_x):
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        layer(static_x)  # warm-up on the capture stream
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            static_out = layer(static_x)
    torch.cuda.current_stream().wait_stream(stream)
    return graph, static_out


def _check_graph(layer, x):
    static_x = x.clone()
    with torch.inference_mode():
        eager = layer(static_x)
        torch.cuda.synchronize()
        graph, static_out = _capture(layer, static_x)
        for i in range(4):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, eager), f"replay {i} differs from the eager forward"
            noise = torch.randn(1024, 1024, device=x.device) @ torch.randn(1024, 1024, device=x.device)
            del noise
        _assert_oracle(layer, static_x, static_out, "replay")
        x2 = torch.randn_like(x.float()).to(x.dtype)
        eager2 = layer(x2)
        static_x.copy_(x2)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager2), "replay on a refilled input differs from the eager forward"
        _assert_oracle(layer, static_x, static_out, "replay on a refilled input")


def test_graph_decode_workload(gpu):
    layer, x = make_layer(WORKLOADS["moe_bf16_d4096_f1536_e128_k8_t64"], gpu)
    _check_graph(layer, x)


@pytest.mark.parametrize("dim,dim_ffn,n_exp,n_shared,top_k,dtype,n_tok", [
    (256, 512, 8, 2, 2, torch.bfloat16, 300),
    (64, 128, 6, 0, 3, torch.float32, 77),
])
def test_graph_shapes(gpu, dim, dim_ffn, n_exp, n_shared, top_k, dtype, n_tok):
    layer = _layer(gpu, dim, dim_ffn, n_exp, n_shared, top_k, dtype)
    x = torch.randn(1, n_tok, dim, device=gpu).to(dtype)
    _check_graph(layer, x)


@pytest.mark.parametrize("dim,dim_ffn,n_tok", [
    (3072, 1024, 8192),  # gate/up: 48 K steps, the last tenth of ~544 tiles claimed at run time;
                         # the tile list in whole groups of one expert
    (2048, 1536, 8192),  # gate/up: 32 K steps, claims with padding-only waves idle in every tile
    (1024, 4096, 8192),  # down: 64 K steps, claims and a split last round (fp32 partials, ordered reduce)
])
def test_graph_run_time_claims_and_split_tail(gpu, dim, dim_ffn, n_tok):
    # the claim counter is cleared by a kernel of the capture on every replay,
    # and the workspace comes from the graph's own pool
    layer = _layer(gpu, dim, dim_ffn, 8, 1, 2, torch.bfloat16)
    x = torch.randn(1, n_tok, dim, device=gpu).to(torch.bfloat16)
    _check_graph(layer, x)


def test_graph_packed_weights(gpu):
    # the packed copy is built by the warm-up call, outside the capture
    layer = _layer(gpu, 512, 256, 16, 1, 4, torch.bfloat16)
    layer.pack_weights = True
    x = torch.randn(1, 200, 512, device=gpu).to(torch.bfloat16)
    _check_graph(layer, x)


def test_graph_survives_many_eager_token_counts(gpu):
    # a serving loop: decode steps replayed from a graph, eager prefills of
    # many different lengths in between. Everything the captured forward reads
    # (the shared experts' tile list included) must belong to the graph, so the
    # eager calls cannot free or rewrite it.
    layer = _layer(gpu, 256, 512, 8, 2, 2, torch.bfloat16)
    static_x = torch.randn(1, 48, 256, device=gpu).to(torch.bfloat16)
    with torch.inference_mode():
        eager = layer(static_x)
        graph, static_out = _capture(layer, static_x)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager)
        for n in range(1, 141, 2):  # 70 distinct token counts
            layer(torch.randn(1, n, 256, device=gpu).to(torch.bfloat16))
        torch.cuda.synchronize()
        for i in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, eager), f"replay {i} after the eager calls differs"
        _assert_oracle(layer, static_x, static_out, "replay after 70 eager token counts")


def test_launch_stream_is_the_current_stream(gpu):
    # every launch goes to the caller's current stream: the raw handle the
    # wrappers pass equals torch's, on the default stream and on a side stream
    t = torch.zeros(4, device=gpu)
    assert ops._stream(t) == torch.cuda.current_stream(gpu).cuda_stream
    side = torch.cuda.Stream(device=gpu)
    with torch.cuda.stream(side):
        assert ops._stream(t) == side.cuda_stream != torch.cuda.default_stream(gpu).cuda_stream
    assert ops._stream(t) == torch.cuda.current_stream(gpu).cuda_stream
