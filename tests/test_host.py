"""Host-side contract tests (CPU): factory, module contract, loader and the
C ABI (symbols exported, argument validation, host policy). No device work."""

from __future__ import annotations

import ctypes
import inspect
import re
from pathlib import Path

import pytest
import torch
import torch.nn as nn

from astrai_amd.extension import KERNEL_NAMES, is_available, loader, ops
from astrai_amd.factory import BaseFactory
from astrai_amd.model.components.linear import Linear
from astrai_amd.model.components.mlp import MLP, DeepSeekMoE, FFNFactory

HEADER = Path(__file__).resolve().parent.parent / "include" / "astrai_moe.h"


# -- factory (astrai/factory.py:45-147) ---------------------------------------


def test_factory_register_create_filters_kwargs():
    class Base(nn.Module):
        pass

    class F(BaseFactory[Base]):
        pass

    @F.register("a")
    class A(Base):
        def __init__(self, dim, scale=2):
            super().__init__()
            self.dim, self.scale = dim, scale

    obj = F.create("a", dim=3, unrelated=1, vocab_size=7)
    assert (obj.dim, obj.scale) == (3, 2)
    with pytest.raises(ValueError, match="already registered"):
        F.register("a")(A)
    with pytest.raises(ValueError, match="Unknown component"):
        F.create("b")
    with pytest.raises(TypeError):

        @F.register("c")
        class C:  # not a Base
            pass

    assert F.list_registered() == ["a"] and F.is_registered("a")


def test_ffn_factory_entries():
    assert FFNFactory.get_component_class("moe") is DeepSeekMoE
    assert FFNFactory.get_component_class("mlp") is MLP


# -- module contract (astrai/model/components/mlp.py:28-62) -------------------


def test_moe_constructor_signature_matches_reference():
    sig = inspect.signature(DeepSeekMoE.__init__)
    params = [(p.name, p.default) for p in sig.parameters.values()][1:]
    E = inspect.Parameter.empty
    assert params == [
        ("dim", E),
        ("dim_ffn", E),
        ("n_routed_experts", E),
        ("n_shared_experts", 1),
        ("n_activated_experts", 2),
        ("topk_method", "greedy"),
        ("n_layers", 1),
    ]


def test_moe_state_dict_keys_and_shapes():
    cfg = dict(dim=16, dim_ffn=24, n_routed_experts=4, n_shared_experts=2, n_activated_experts=2,
               topk_method="greedy", n_layers=3, vocab_size=100, hidden_size=16)
    m = FFNFactory.create("moe", **cfg)
    sd = m.state_dict()
    expected = {"router.weight": (4, 16)}
    for group, n in (("shared_experts", 2), ("routed_experts", 4)):
        for i in range(n):
            expected[f"{group}.{i}.up.weight"] = (24, 16)
            expected[f"{group}.{i}.gate.weight"] = (24, 16)
            expected[f"{group}.{i}.down.weight"] = (16, 24)
    assert {k: tuple(v.shape) for k, v in sd.items()} == expected
    # Same init scale as the reference: 0.02 / sqrt(2 * n_layers * moe_scale).
    moe_scale = 1 / 2 + 1 / 2
    assert m.routed_experts[0].down.init_std == pytest.approx(0.02 / (2 * 3 * moe_scale) ** 0.5)
    assert m.router.bias is None and isinstance(m.router, Linear)
    # LoRA targets the experts' Linear children by these names.
    assert {n.rsplit(".", 1)[-1] for n, mod in m.named_modules() if isinstance(mod, Linear)} == {
        "router", "up", "gate", "down"}


def test_state_dict_round_trip():
    a = DeepSeekMoE(8, 16, 3, n_shared_experts=1)
    for p in a.parameters():
        nn.init.normal_(p)
    b = DeepSeekMoE(8, 16, 3, n_shared_experts=1)
    b.load_state_dict(a.state_dict())
    for (ka, va), (kb, vb) in zip(a.state_dict().items(), b.state_dict().items()):
        assert ka == kb and torch.equal(va, vb)


def test_safetensors_checkpoint_round_trip(tmp_path):
    # the reference's checkpoints are safetensors files keyed like the module's state_dict
    from safetensors.torch import load_file, save_file

    a = DeepSeekMoE(8, 16, 3, n_shared_experts=2)
    for p in a.parameters():
        nn.init.normal_(p)
    path = tmp_path / "moe.safetensors"
    save_file(a.state_dict(), str(path))
    b = DeepSeekMoE(8, 16, 3, n_shared_experts=2)
    missing, unexpected = b.load_state_dict(load_file(str(path)))
    assert not missing and not unexpected
    for k, v in a.state_dict().items():
        assert torch.equal(v, b.state_dict()[k])


def test_cpu_input_raises_instead_of_falling_back():
    m = DeepSeekMoE(8, 16, 4, n_shared_experts=0)
    with torch.no_grad(), pytest.raises(RuntimeError, match="ROCm device"):
        m(torch.zeros(1, 2, 8))


# -- loader (astrai/extension/loader.py:14-36) --------------------------------


def test_loader_contract():
    assert KERNEL_NAMES == ["moe_route", "moe_permute", "moe_gemm_gate_up", "moe_gemm_down", "moe_combine"]
    assert loader.load_error() is None, loader.load_error()
    for name in KERNEL_NAMES:
        assert is_available(name)
        assert callable(getattr(loader.get_module(name), name))
    assert not is_available("attn_decode")
    assert loader.get_module("nope") is None


def test_single_hip_runtime_mapped():
    assert len(loader._hip_runtimes_mapped()) <= 1


def _declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(astrai_moe_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    syms = _declared_symbols()
    assert len(syms) >= 9, syms
    lib = ctypes.CDLL(str(loader.LIB_PATH))
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in astrai_moe.h but not exported"
    # ... and the loader binds every declared symbol with a signature.
    assert set(syms) == set(loader._SIGNATURES)


# -- C ABI host behaviour (validation happens before any device work) ---------


def test_abi_rejects_bad_arguments_with_message():
    lib = loader.library()
    rc = lib.astrai_moe_route(None, 1, 10, 0, 1, None, None, None, None)
    assert rc == -1 and "n_experts" in loader.last_error()
    rc = lib.astrai_moe_route(None, 1, 10, 8, 9, None, None, None, None)
    assert rc == -1 and "top_k" in loader.last_error()
    rc = lib.astrai_moe_route(1, 7, 10, 8, 2, 1, 1, 1, None)
    assert rc == -1 and "dtype" in loader.last_error()
    rc = lib.astrai_moe_permute(None, None, None, None, 1, 10, 8, 2, 16, 64, None, None, None, None, None,
                                None, 3, None, None)
    assert rc == -1 and "tile list" in loader.last_error()
    rc = lib.astrai_moe_combine(1, 1, None, None, 2, 1, 4, 2, 8, 1, None)
    assert rc == -1 and "n_shared" in loader.last_error()
    rc = lib.astrai_moe_pack_gate_up(None, None, 0, 128, 64, None, None)
    assert rc == -1 and "bf16 only" in loader.last_error()
    rc = lib.astrai_moe_pack_gate_up(None, None, 1, 100, 64, None, None)
    assert rc == -1 and "dim_ffn % 128" in loader.last_error()
    rc = lib.astrai_moe_pack_gate_up(None, None, 1, 128, 64, None, None)
    assert rc == -1 and "null buffer" in loader.last_error()
    rc = lib.astrai_moe_pack_down(None, 1, 200, 64, None, None)
    assert rc == -1 and "dim % 256" in loader.last_error()
    rc = lib.astrai_moe_pack_down(8, 1, 256, 64, 32, None)
    assert rc == -1 and "16-byte aligned" in loader.last_error()
    # training / backward entry points: every call below is refused on the host
    # (the dummy pointers are never dereferenced); fp32 and general shapes are
    # accepted, so they do not appear here with dummy pointers
    rc = lib.astrai_moe_gemm_gate_up_train(1, 1, 7, 1, 1, 7, 4, 2, 256, 128, 256, 1, 1, None, 0, None)
    assert rc == -1 and "dtype" in loader.last_error()
    rc = lib.astrai_moe_gemm_gate_up_train(1, 1, 7, 1, 1, 1, 4, 2, 256, 128, 32, 1, 1, None, 0, None)
    assert rc == -1 and "256-row tile list" in loader.last_error()
    rc = lib.astrai_moe_gemm_down_train(1, 1, 7, 1, 1, 1, 4, 2, 0, 256, 256, 1, 1, None, 0, None)
    assert rc == -1 and "dims" in loader.last_error()
    # the GEMM workspace (run-time claims, split tail): optional, aligned, size >= 0
    rc = lib.astrai_moe_gemm_gate_up(16, 16, 7, 16, 16, 1, 4, 2, 256, 256, 256, 16, 16, -1, None)
    assert rc == -1 and "negative workspace size" in loader.last_error()
    rc = lib.astrai_moe_gemm_gate_up_gather(16, 16, 2, 16, 7, 16, 16, 1, 4, 2, 256, 256, 256, 16, 8, 1 << 16, None)
    assert rc == -1 and "workspace must be 16-byte aligned" in loader.last_error()
    rc = lib.astrai_moe_gemm_gate_up_packed(16, 16, 7, 16, 1, 4, 2, 256, 256, 256, 16, 8, 1 << 16, None)
    assert rc == -1 and "workspace must be 16-byte aligned" in loader.last_error()
    rc = lib.astrai_moe_gemm_gate_up_train(16, 16, 7, 16, 16, 1, 4, 2, 256, 256, 256, 16, 16, 8, 1 << 16, None)
    assert rc == -1 and "workspace must be 16-byte aligned" in loader.last_error()
    assert lib.astrai_moe_gemm_workspace_bytes(0) == 1 << 16
    assert lib.astrai_moe_gemm_workspace_bytes(1) > lib.astrai_moe_gemm_workspace_bytes(0)
    rc = lib.astrai_moe_gemm_down(16, 16, 7, 16, 16, 1, 4, 2, 256, 256, 256, 16, 16, -1, None)
    assert rc == -1 and "negative workspace size" in loader.last_error()
    rc = lib.astrai_moe_gemm_down(16, 16, 7, 16, 16, 1, 4, 2, 256, 256, 256, 16, 8, 1 << 20, None)
    assert rc == -1 and "workspace must be 16-byte aligned" in loader.last_error()
    rc = lib.astrai_moe_gemm_down_packed(16, 16, 7, 16, 16, 1, 4, 2, 256, 256, 256, 16, 8, 1 << 20, None)
    assert rc == -1 and "workspace must be 16-byte aligned" in loader.last_error()
    rc = lib.astrai_moe_gemm_down_train(16, 16, 7, 16, 16, 1, 4, 2, 256, 256, 256, 16, 16, 8, 1 << 20, None)
    assert rc == -1 and "workspace must be 16-byte aligned" in loader.last_error()
    rc = lib.astrai_moe_gemm_dgrad_gate_up(16, 16, 16, 7, 16, 16, 1, 4, 2, 256, 256, 256, 16, 16, -1, None)
    assert rc == -1 and "negative workspace size" in loader.last_error()
    rc = lib.astrai_moe_gemm_dgrad_gate_up(16, 16, 16, 7, 16, 16, 1, 4, 2, 256, 256, 256, 16, 8, 1 << 20, None)
    assert rc == -1 and "workspace must be 16-byte aligned" in loader.last_error()
    rc = lib.astrai_moe_gemm_dgrad_down(1, 1, 7, 1, None, 1, 4, 2, 256, 128, 256, 1, 1, None)
    assert rc == -1 and "null" in loader.last_error()
    rc = lib.astrai_moe_gemm_dgrad_gate_up(1, 1, 1, 7, 1, 1, 1, 4, 2, 128, 256, 64, 1, None, 0, None)
    assert rc == -1 and "256-row tile list" in loader.last_error()
    rc = lib.astrai_moe_row_grad(1, 1, 1, 1, 1, 4, 0, 1, 1, None)
    assert rc == -1 and "dim must be" in loader.last_error()
    rc = lib.astrai_moe_row_grad(1, 1, 1, 1, 5, 4, 16, 1, 1, None)
    assert rc == -1 and "dtype" in loader.last_error()
    rc = lib.astrai_moe_gemm_wgrad(16, 16, 16, 1, 4, 2, 0, 16, 16, None)
    assert rc == -1 and "m and n" in loader.last_error()
    rc = lib.astrai_moe_gemm_wgrad(16, 16, None, 1, 4, 2, 16, 16, 16, None)
    assert rc == -1 and "null" in loader.last_error()
    assert lib.astrai_moe_gemm_wgrad(None, None, None, 1, 0, 2, 16, 16, None, None) == 0
    # Empty inputs are a valid no-op.
    assert lib.astrai_moe_route(None, 1, 0, 8, 2, None, None, None, None) == 0
    assert lib.astrai_moe_combine(None, None, None, None, 0, 1, 0, 2, 8, None, None) == 0


def test_tile_list_len_bounds_the_tile_count():
    """capacity >= sum_e ceil(M_e / block_m) for any split of T*K rows."""
    import random

    rnd = random.Random(0)
    for _ in range(200):
        n_exp = rnd.randint(1, 64)
        k = rnd.randint(1, min(8, n_exp))
        n_tok = rnd.randint(0, 5000)
        bm = rnd.choice([32, 64, 128, 256])
        rows = n_tok * k
        cuts = sorted(rnd.randint(0, rows) for _ in range(n_exp - 1))
        counts = [b - a for a, b in zip([0] + cuts, cuts + [rows])]
        need = sum(-(-c // bm) for c in counts)
        cap = (ops.tile_list_len(n_tok, n_exp, k, bm) - ops.TILE_HEADER) // ops.TILE_STRIDE
        assert cap >= need


def test_block_m_policy():
    bf = torch.bfloat16
    assert ops.select_block_m(16384, 8, 2, 4096, 14336, bf) == 256
    assert ops.select_block_m(64, 128, 8, 4096, 1536, bf) == 32
    assert ops.select_block_m(1024, 8, 2, 512, 1024, torch.float32) == 64  # the general kernel's tiles
    assert ops.select_block_m(100, 4, 2, 8, 16, bf) == 64  # shapes the MFMA kernels do not tile
    # routed, by average rows per expert: 32-row tiles below 24, 64 below 48, 128 below 128, then 256
    assert ops.select_block_m(368, 128, 8, 4096, 1536, bf) == 32  # 23 rows per expert
    assert ops.select_block_m(384, 128, 8, 4096, 1536, bf) == 64  # 24
    assert ops.select_block_m(767, 128, 8, 4096, 1536, bf) == 64  # 47
    assert ops.select_block_m(768, 128, 8, 4096, 1536, bf) == 128  # 48
    assert ops.select_block_m(1024, 128, 8, 4096, 1536, bf) == 128  # 64: the mid-sized batch workload
    assert ops.select_block_m(2047, 128, 8, 4096, 1536, bf) == 128  # 127
    assert ops.select_block_m(2048, 128, 8, 4096, 1536, bf) == 256  # 128
    assert ops.select_block_m(511, 8, 2, 4096, 14336, bf) == 128
    assert ops.select_block_m(512, 8, 2, 4096, 14336, bf) == 256
    assert ops.select_block_m(8192, 64, 6, 2048, 1408, bf) == 256  # the fine-grained workload (768 rows)
    # one dense MLP (shared experts): 32 below 96 tokens; with u = T * (F/128 + D/256): 64-row tiles
    # below u = 65536, 128 below 2.25 * 65536, then 256
    assert ops.select_block_m(95, 1, 1, 2048, 2816, bf) == 32
    assert ops.select_block_m(96, 1, 1, 2048, 2816, bf) == 64
    assert ops.select_block_m(2184, 1, 1, 2048, 2816, bf) == 64  # 30 column tiles per row tile
    assert ops.select_block_m(2185, 1, 1, 2048, 2816, bf) == 128
    assert ops.select_block_m(4915, 1, 1, 2048, 2816, bf) == 128
    assert ops.select_block_m(4916, 1, 1, 2048, 2816, bf) == 256
    assert ops.select_block_m(511, 1, 1, 4096, 14336, bf) == 64  # 128 column tiles per row tile
    assert ops.select_block_m(512, 1, 1, 4096, 14336, bf) == 128
    assert ops.select_block_m(1152, 1, 1, 4096, 14336, bf) == 256
    assert ops.select_block_m(16384, 1, 1, 2048, 2816, bf) == 256


def test_packed_weights_follow_the_matrix_core_policy():
    # matrix-core shapes (dims multiples of 64) get the matrix-core tile heights; the layer packs those of
    # them whose column tiles are whole (dim % 256, dim_ffn % 128)
    for dim, dim_ffn in [(4096, 14336), (2048, 1408), (256, 512), (512, 256), (96, 80), (8, 16), (256, 64),
                         (2880, 2880), (192, 320)]:
        for dtype in (torch.bfloat16, torch.float32):
            bm = ops.select_block_m(1024, 8, 2, dim, dim_ffn, dtype)  # 256 rows per expert: 256-row MFMA tiles
            assert ops.matrix_core_supported(dim, dim_ffn, dtype) == (bm == 256), (dim, dim_ffn, dtype)
            whole = dim % 256 == 0 and dim_ffn % 128 == 0
            assert ops.packed_supported(dim, dim_ffn, dtype) == (bm == 256 and whole), (dim, dim_ffn, dtype)
    m = DeepSeekMoE(512, 256, 4, n_shared_experts=0)
    assert not m.pack_weights and not m.uses_packed_weights(torch.bfloat16)  # opt-in
    m.pack_weights = True
    assert m.uses_packed_weights(torch.bfloat16) and not m.uses_packed_weights(torch.float32)
    assert not DeepSeekMoE(8, 16, 4, n_shared_experts=0).uses_packed_weights(torch.bfloat16)


def test_ops_validate_before_launch():
    with pytest.raises(ValueError, match="ROCm device"):
        ops.moe_route(torch.zeros(4, 8), 2)
    with pytest.raises(ValueError):
        ops.expert_weight_table([], (2, 2))


# -- weight-table arguments ---------------------------------------------------


class _NoLaunch:
    """Stands in for the library: reaching it means a wrapper let its
    arguments through to a launch."""

    def __getattr__(self, name):
        raise AssertionError(f"reached the library ({name})")

    def library(self):
        return self


def _table_wrappers(x, tiles, n_exp, dim, dim_ffn):
    """Each wrapper that takes weight tables, as ``f(gate, up, down)``."""
    rows = x.shape[0]
    h = torch.zeros(rows, dim_ffn, dtype=x.dtype)
    w = torch.ones(rows, dtype=x.dtype)
    gu = torch.zeros(rows, 2 * dim_ffn, dtype=x.dtype)
    sorted_token = torch.arange(rows, dtype=torch.int32)
    return {
        "gate_up": lambda g, u, d: ops.moe_gemm_gate_up(x, tiles, g, u, n_exp, dim_ffn, 32),
        "gate_up_packed": lambda g, u, d: ops.moe_gemm_gate_up(x, tiles, g, u, n_exp, dim_ffn, 32, packed=True),
        "gate_up_gather": lambda g, u, d: ops.moe_gemm_gate_up_gather(x, sorted_token, tiles, g, u, n_exp, dim_ffn, 32),
        "down": lambda g, u, d: ops.moe_gemm_down(h, tiles, d, w, n_exp, dim, 32),
        "down_packed": lambda g, u, d: ops.moe_gemm_down(h, tiles, d, w, n_exp, dim, 32, packed=True),
        "gate_up_train": lambda g, u, d: ops.moe_gemm_gate_up_train(x, tiles, g, u, n_exp, dim_ffn),
        "down_train": lambda g, u, d: ops.moe_gemm_down_train(h, tiles, d, w, n_exp, dim),
        "dgrad_down": lambda g, u, d: ops.moe_gemm_dgrad_down(x, tiles, d, gu, n_exp),
        "dgrad_gate_up": lambda g, u, d: ops.moe_gemm_dgrad_gate_up(h, h, tiles, g, u, n_exp, dim),
    }


def test_weight_tables_are_checked_before_any_launch(monkeypatch):
    # the kernels dereference every table entry: a weight tensor, a table of
    # the wrong length or dtype passed in a table's place must raise on the
    # host, never reach a launch (device placement relaxed to run on the CPU)
    def relaxed(t, name, ndim=None):
        if not isinstance(t, torch.Tensor) or not t.is_contiguous() or (ndim is not None and t.dim() != ndim):
            raise ValueError(name)

    monkeypatch.setattr(ops, "_require_gpu", relaxed)
    monkeypatch.setattr(ops, "_kernel", lambda name: lambda *args: _NoLaunch().__getattr__(name))
    monkeypatch.setattr(ops, "loader", _NoLaunch())
    monkeypatch.setattr(ops, "_stream", lambda t: 0)
    n_exp, dim, dim_ffn, bf = 4, 256, 128, torch.bfloat16
    x = torch.zeros(64, dim, dtype=bf)
    tiles = torch.zeros(64, dtype=torch.int32)
    good = torch.zeros(n_exp, dtype=torch.int64)
    bad = {
        "weight tensor": torch.zeros(dim_ffn, dim, dtype=bf),
        "too few entries": torch.zeros(n_exp - 1, dtype=torch.int64),
        "too many entries": torch.zeros(n_exp + 1, dtype=torch.int64),
        "int32 entries": torch.zeros(n_exp, dtype=torch.int32),
    }
    for name, call in _table_wrappers(x, tiles, n_exp, dim, dim_ffn).items():
        with pytest.raises(AssertionError, match="reached the library"):
            call(good, good, good)  # valid tables get through to the launch
        for what, t in bad.items():
            for pos in range(3):
                args = [good, good, good]
                args[pos] = t
                if (name.endswith("packed") and pos == 1) or (pos == 2) != (name.startswith("down") or name == "dgrad_down"):
                    continue  # an argument this wrapper does not read
                with pytest.raises(ValueError, match=r"^w_(gate|up|down)"):
                    call(*args)


def test_tile_list_height_is_checked_before_any_launch(monkeypatch):
    # a tile list of one height run with another would compute only part of
    # each tile and leave the rest of the output unwritten: the wrappers
    # compare the height a list was built for with their block_m
    def relaxed(t, name, ndim=None):
        if not isinstance(t, torch.Tensor) or not t.is_contiguous() or (ndim is not None and t.dim() != ndim):
            raise ValueError(name)

    monkeypatch.setattr(ops, "_require_gpu", relaxed)
    monkeypatch.setattr(ops, "_kernel", lambda name: lambda *args: _NoLaunch().__getattr__(name))
    monkeypatch.setattr(ops, "loader", _NoLaunch())
    monkeypatch.setattr(ops, "_stream", lambda t: 0)
    n_exp, dim, dim_ffn, bf = 4, 256, 128, torch.bfloat16
    x = torch.zeros(64, dim, dtype=bf)
    good = torch.zeros(n_exp, dtype=torch.int64)
    for built in (32, 64, 128, 256):
        tiles = ops._tag_tiles(torch.zeros(64, dtype=torch.int32), built)
        for name, call in _table_wrappers(x, tiles, n_exp, dim, dim_ffn).items():
            runs_at = 256 if name.endswith("train") or name.startswith("dgrad") else 32
            if built == runs_at:
                with pytest.raises(AssertionError, match="reached the library"):
                    call(good, good, good)
            else:
                with pytest.raises(ValueError, match=f"built for block_m {built}"):
                    call(good, good, good)
    # and a tile list must be an int32 list
    with pytest.raises(ValueError, match="int32 tile list"):
        ops.moe_gemm_gate_up(x, torch.zeros(64, dtype=torch.int64), good, good, n_exp, dim_ffn, 32)


def test_dense_tile_lists_are_not_cached_across_calls():
    # a graph captured with a dense expert must own its tile list: the ops
    # build one per call on the device instead of keeping a module-level cache
    # that later calls could clear and the allocator reuse
    assert not any("cache" in name for name in vars(ops) if name.startswith("_dense"))
    assert "astrai_moe_dense_tiles" in loader._SIGNATURES


def test_use_hip_ffn_swaps_the_registry_entries():
    # a registry with the reference factory's API (astrai/factory.py:45-147,
    # restated by astrai_amd.factory): register() refuses taken names, so the
    # switch writes the entries; models built afterwards get the HIP classes
    # with the reference's kwarg filtering; restore_ffn puts the old ones back
    import torch.nn as nn

    from astrai_amd.factory import BaseFactory
    from astrai_amd.integration import restore_ffn, use_hip_ffn
    from astrai_amd.model.components.mlp import MLP, DeepSeekMoE

    class FFN(BaseFactory[nn.Module]):
        pass

    @FFN.register("moe")
    class TorchMoE(nn.Module):
        def __init__(self, dim, dim_ffn, n_routed_experts, n_shared_experts=1, n_activated_experts=2):
            super().__init__()

    @FFN.register("mlp")
    class TorchMLP(nn.Module):
        def __init__(self, dim, dim_ffn):
            super().__init__()

    with pytest.raises(ValueError):
        FFN.register("moe")(DeepSeekMoE)  # why the switch writes the registry
    prev = use_hip_ffn(FFN)
    assert FFN._entries["moe"] is DeepSeekMoE and FFN._entries["mlp"] is TorchMLP
    cfg = dict(dim=64, dim_ffn=128, n_routed_experts=4, n_shared_experts=1, n_activated_experts=2, n_layers=2,
               n_heads=8, n_kv_heads=2, norm_eps=1e-5, down_init_std=0.01)  # a decoder block's whole cfg
    m = FFN.create("moe", **cfg)
    assert isinstance(m, DeepSeekMoE) and m.n_routed_experts == 4 and len(m.shared_experts) == 1
    assert "routed_experts.3.down.weight" in m.state_dict() and "router.weight" in m.state_dict()
    restore_ffn(prev, FFN)
    assert FFN._entries["moe"] is TorchMoE and FFN._entries["mlp"] is TorchMLP
    prev = use_hip_ffn(FFN, moe=False, mlp=True)
    assert FFN._entries["mlp"] is MLP and FFN._entries["moe"] is TorchMoE
    assert isinstance(FFN.create("mlp", **cfg), MLP)
    restore_ffn(prev, FFN)
    assert FFN._entries["mlp"] is TorchMLP

    class Other(BaseFactory[dict]):  # the classes must satisfy the registry's base type
        pass

    with pytest.raises(TypeError):
        use_hip_ffn(Other)
    assert "moe" not in Other._entries


def test_register_kernels_reaches_a_reference_style_loader():
    # a stand-in with the reference's discovery interface
    # (astrai/extension/loader.py:14-36): KERNEL_NAMES, _available and
    # _modules filled at import, is_available / get_module reading them, and
    # kernels imported as <package>.<name> submodules
    import importlib
    import sys
    import types

    from astrai_amd.integration import register_kernels

    pkg = types.ModuleType("fake_astrai_ext")
    pkg.__path__ = []
    ext = types.ModuleType("fake_astrai_ext.loader")
    ext.__package__ = "fake_astrai_ext"
    ext.KERNEL_NAMES = ["attn_decode"]
    ext._available = {"attn_decode": False}
    ext._modules = {"attn_decode": None}
    ext.is_available = lambda name: ext._available.get(name, False)
    ext.get_module = lambda name: ext._modules.get(name)
    sys.modules["fake_astrai_ext"], sys.modules["fake_astrai_ext.loader"] = pkg, ext
    try:
        names = register_kernels(ext)
        assert names == [n for n in loader.KERNEL_NAMES if loader.is_available(n)]
        assert loader.is_available("moe_route"), loader.load_error()  # the library loads without a GPU
        for name in names:
            assert ext.is_available(name) and name in ext.KERNEL_NAMES
            assert ext.get_module(name) is loader.get_module(name)
            assert callable(getattr(ext.get_module(name), name))
            assert importlib.import_module(f".{name}", package="fake_astrai_ext") is loader.get_module(name)
        assert ext.KERNEL_NAMES[0] == "attn_decode" and not ext.is_available("attn_decode")
        assert register_kernels(ext) == names and ext.KERNEL_NAMES.count("moe_route") == 1  # idempotent
        with pytest.raises(TypeError):
            register_kernels(types.ModuleType("not_a_loader"))
    finally:
        for key in [k for k in sys.modules if k == "fake_astrai_ext" or k.startswith("fake_astrai_ext.")]:
            del sys.modules[key]


# -- register allocation of the matrix-core GEMMs (device code compiled here) ----


def _device_kernel_metadata(src: Path, tmp_path: Path) -> dict:
    """Per-kernel register metadata of ``src``'s gfx950 device code
    (``hipcc --cuda-device-only -S``): {mangled name: {vgpr, spill}}."""
    import subprocess

    import yaml

    from astrai_amd.csrc import build as B

    out = tmp_path / (src.stem + ".s")
    cmd = [B._hipcc(), *B.HIPCC_FLAGS, f"-I{B.INCLUDE_DIR}", f"-I{B.KERNELS_DIR}", "--cuda-device-only", "-S",
           str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    text = out.read_text()
    m = re.search(r"\.amdgpu_metadata\n(.*?)\.end_amdgpu_metadata", text, re.S)
    lines = [ln for ln in m.group(1).replace("\t", "    ").split("\n") if ln.strip() not in ("---", "...")]
    meta = yaml.safe_load("\n".join(lines))
    return {k[".name"]: {"vgpr": k.get(".vgpr_count"), "spill": k.get(".vgpr_spill_count", 0)}
            for k in meta["amdhsa.kernels"]}


def test_matrix_core_gemms_keep_their_registers(tmp_path):
    """The 256-row kernels' K loops hold 128 accumulators, the operand rings
    and the addresses in 168 VGPRs: the gate/up GEMMs (plain, gathering,
    packed, and the training forward's saving one) and the dgrad_down /
    dgrad_in_add / wgrad kernels must compile without spills (a change to
    the tile loop that made the compiler spill cost the gate/up GEMM 3 % at
    the Mixtral shape)."""
    import shutil

    if shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists():
        pytest.skip("hipcc not available")
    kdir = Path(__file__).resolve().parent.parent / "astrai_amd" / "csrc" / "kernels"
    fwd = _device_kernel_metadata(kdir / "moe_gemm_mfma.hip", tmp_path)
    # gemm_stream_kernel<gate_up=true, packed, save, gather>: the inference kernels and the saving one
    gate_up = {n: v for n, v in fwd.items() if re.search(r"gemm_stream_kernelILb1ELb[01]ELb[01]ELb[01]E", n)}
    assert len(gate_up) == 4, sorted(fwd)
    for n, v in gate_up.items():
        assert v["vgpr"] <= 168 and v["spill"] == 0, (n, v)
    bwd = _device_kernel_metadata(kdir / "moe_gemm_bwd.hip", tmp_path)
    # Bwd::kDgradDown (0), kDgradInAdd (2), kWgrad (3), whole-tile launches (kTail false)
    for mode in (0, 2, 3):
        hits = {n: v for n, v in bwd.items() if f"gemm_bwd_kernelILNS0_3BwdE{mode}ELb0E" in n}
        assert len(hits) == 1, (mode, sorted(bwd))
        for n, v in hits.items():
            assert v["spill"] == 0, (n, v)
