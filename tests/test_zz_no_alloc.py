"""The permutation entry point that allocates nothing
(``astrai_moe_permute_noalloc``) against the one that takes a workspace
(``astrai_moe_permute``), both called through the C ABI.

Its outputs must equal the workspace entry point's bit for bit on every call:
calls in a row share the library's scratch, so a later call (a smaller
problem, another expert count) must not see stale contents.
Problems too large for the scratch are refused on the host, before any device
work (a CPU test).
"""

from __future__ import annotations

import pytest
import torch

from astrai_amd.extension import loader, ops

NOALLOC_SCRATCH_INTS = 1 << 20  # ASTRAI_MOE_NOALLOC_SCRATCH_INTS


def _routing(gpu, n_tok, n_exp, top_k, dtype, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    logits = (torch.randn(n_tok, n_exp, generator=g, device=gpu) * 0.5).to(dtype)
    return ops.moe_route(logits, top_k)


def _permute_noalloc(route, x, n_exp, block_m, copy_rows):
    """astrai_moe_permute_noalloc with outputs laid out as ops.moe_permute's."""
    n_tok, dim = x.shape
    top_k = route.topk_idx.shape[1]
    dev = x.device
    rows = n_tok * top_k
    tl = ops.tile_list_len(n_tok, n_exp, top_k, block_m)
    out = ops.PermuteResult(
        torch.full((n_exp + 1,), -7, dtype=torch.int32, device=dev),
        torch.full((rows,), -7, dtype=torch.int32, device=dev),
        torch.zeros(rows, dtype=x.dtype, device=dev),
        torch.full((n_tok, top_k), -7, dtype=torch.int32, device=dev),
        torch.zeros(rows, dim, dtype=x.dtype, device=dev) if copy_rows else None,
        torch.full((tl,), -7, dtype=torch.int32, device=dev),
        block_m,
    )
    rc = loader.library().astrai_moe_permute_noalloc(
        route.topk_idx.data_ptr(), route.topk_w.data_ptr(), route.chunk_hist.data_ptr(), x.data_ptr(),
        ops._DTYPE_CODES[x.dtype], n_tok, n_exp, top_k, dim, block_m, out.expert_offsets.data_ptr(),
        out.sorted_token.data_ptr(), out.sorted_w.data_ptr(), out.token_pos.data_ptr(),
        None if out.x_perm is None else out.x_perm.data_ptr(), out.tiles.data_ptr(), tl,
        torch.cuda.current_stream(dev).cuda_stream)
    assert rc == 0, loader.last_error()
    return out


@pytest.mark.gpu
def test_noalloc_permute_matches_workspace_permute(gpu):
    # (tokens, experts, top_k, dim, dtype, block_m, copy rows). Histograms of
    # more than 32768 counts (chunks of 32 tokens x experts) take the scan
    # that keeps per-range expert bases in the library's scratch (ranges of 8
    # chunks): the first case writes 157 range rows x 64 experts (rows of
    # 3072: the grouped tile order), the second
    # a smaller problem over the same experts (79 rows: it must not see the
    # first call's bases past them), the third another expert count (36 rows
    # x 128), the fourth 33 rows x 1024 scanned in two levels (blocks of 32
    # ranges). The last two are small enough for the scan folded into the
    # scatter, which needs no scratch.
    cases = [
        (40000, 64, 6, 3072, torch.bfloat16, 256, False),
        (20000, 64, 6, 128, torch.bfloat16, 256, True),
        (9000, 128, 8, 256, torch.bfloat16, 128, False),
        (8448, 1024, 2, 64, torch.bfloat16, 64, True),
        (3000, 64, 6, 512, torch.bfloat16, 64, True),
        (777, 8, 2, 96, torch.float32, 64, True),
    ]
    for i, (n_tok, n_exp, top_k, dim, dtype, block_m, copy_rows) in enumerate(cases):
        print(f"case {i}: tokens {n_tok} experts {n_exp} top_k {top_k} dim {dim} {dtype} block_m {block_m}",
              flush=True)
        route = _routing(gpu, n_tok, n_exp, top_k, dtype, seed=20 + i)
        x = torch.randn(n_tok, dim, device=gpu).to(dtype)
        want = ops.moe_permute(route, x, n_exp, block_m, copy_rows=copy_rows)
        got = _permute_noalloc(route, x, n_exp, block_m, copy_rows)
        torch.cuda.synchronize()
        for name in ("expert_offsets", "sorted_token", "sorted_w", "token_pos", "x_perm"):
            a, b = getattr(got, name), getattr(want, name)
            assert (a is None) == (b is None), name
            if a is not None:
                assert torch.equal(a, b), f"case {i}: {name} differs from astrai_moe_permute"
        # the tile list: header and live tiles (entries past the live count are
        # not written by either entry point)
        live = 4 + 3 * int(want.tiles[0].item())
        assert int(got.tiles[0].item()) == int(want.tiles[0].item()) > 0
        assert torch.equal(got.tiles[:live], want.tiles[:live]), f"case {i}: tile list differs"


def test_noalloc_permute_refuses_problems_beyond_its_scratch():
    # 2^20 tokens over 1024 experts need 4096 range rows x 1024 experts: more
    # than the scratch holds. Refused before any device work, so the dummy
    # (never dereferenced) pointers are never used.
    lib = loader.library()
    n_tok, n_exp, top_k, block_m = 1 << 20, 1024, 8, 256
    tl = ops.tile_list_len(n_tok, n_exp, top_k, block_m)
    p = 16
    rc = lib.astrai_moe_permute_noalloc(p, p, p, p, 1, n_tok, n_exp, top_k, 128, block_m, p, p, p, p, None, p, tl, None)
    assert rc == -1
    msg = loader.last_error()
    assert "scratch" in msg and str(NOALLOC_SCRATCH_INTS) in msg, msg
    # the largest problem at 1024 experts that fits: 262144 tokens (1024 range rows)
    n_ok = 262144
    assert (n_ok // 32 // 8) * n_exp == NOALLOC_SCRATCH_INTS
