"""Parity of each HIP kernel with the oracle on the same device (GPU).

Routing, permutation and combine are integer/ordering work or exact
sequences of rounded adds: they must be bit-identical to the reference's
torch ops. The grouped GEMMs are compared with torch on identical inputs at
the reference's rounding points, within rtol 2e-2 / atol 2e-3 (bf16, fp32
accumulation) or 1e-5 (fp32).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from astrai_amd.extension import ops
from astrai_amd.workloads import HEADLINE, WORKLOADS, make_layer
from oracle import moe_ref as R

pytestmark = pytest.mark.gpu

BF16_TOL = dict(rtol=2e-2, atol=2e-3)
FP32_TOL = dict(rtol=1e-5, atol=1e-5)


def _logits(gpu, n_tok, n_exp, dtype, std, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    return (torch.randn(n_tok, n_exp, generator=g, device=gpu) * std).to(dtype)


def _dense_weights(idx, w, n_exp):
    out = torch.zeros(idx.shape[0], n_exp, dtype=torch.float64, device=idx.device)
    return out.scatter(1, idx.long(), w.double())


def assert_route_exact(logits, top_k):
    dtype = logits.dtype
    w_ref, i_ref = R.route(logits, top_k, dtype)
    res = ops.moe_route(logits, top_k)
    torch.cuda.synchronize()
    n_exp = logits.shape[1]
    # Same selected set per token, same weight per (token, expert), same
    # sequence of weights (values are emitted in descending order).
    assert torch.equal(res.topk_idx.long().sort(-1).values, i_ref.sort(-1).values)
    assert torch.equal(_dense_weights(res.topk_idx, res.topk_w, n_exp), _dense_weights(i_ref, w_ref, n_exp))
    assert torch.equal(res.topk_w, w_ref)
    counts = torch.bincount(i_ref.flatten(), minlength=n_exp)
    assert torch.equal(res.chunk_hist.sum(0).long(), counts)
    return res


ROUTE_CASES = [
    # (tokens, experts, top_k, dtype, logit std)
    (1, 8, 2, torch.bfloat16, 1.0),
    (33, 8, 2, torch.float32, 1.0),
    (1000, 8, 2, torch.bfloat16, 0.9),
    (4096, 64, 6, torch.bfloat16, 0.9),
    (4096, 64, 6, torch.bfloat16, 0.01),  # near-uniform: many bf16 ties
    (2048, 128, 8, torch.bfloat16, 1.0),
    (777, 3, 2, torch.bfloat16, 0.5),
    (500, 256, 8, torch.bfloat16, 1.0),
    (300, 1024, 32, torch.float32, 2.0),
    (64, 5, 5, torch.bfloat16, 1.0),
    (256, 1, 1, torch.bfloat16, 1.0),
    (1024, 16, 1, torch.float32, 0.3),
    (262144, 64, 6, torch.bfloat16, 0.9),  # many chunks of the device-side histogram
    (100003, 32, 4, torch.float32, 1.0),  # ragged last chunk
]


@pytest.mark.parametrize("n_tok,n_exp,top_k,dtype,std", ROUTE_CASES)
def test_route_bit_exact(gpu, n_tok, n_exp, top_k, dtype, std):
    assert_route_exact(_logits(gpu, n_tok, n_exp, dtype, std, seed=n_tok * 7 + n_exp), top_k)


def test_route_crafted_ties(gpu):
    """Exactly tied logits: the lowest expert ids among the tied win."""
    logits = torch.zeros(64, 16, device=gpu, dtype=torch.bfloat16)
    logits[:, [3, 7, 9, 12]] = 1.0
    logits[1::2, 12] = 2.0
    res = assert_route_exact(logits, 3)
    assert res.topk_idx[0].tolist() == [3, 7, 9]
    assert res.topk_idx[1].tolist()[0] == 12


def _routing(gpu, n_tok, n_exp, top_k, dtype, std=1.0, seed=0):
    logits = _logits(gpu, n_tok, n_exp, dtype, std, seed)
    return ops.moe_route(logits, top_k)


PERM_CASES = [
    (1, 8, 2, 16, 256),
    (33, 8, 2, 64, 64),
    (4096, 64, 6, 2048, 256),
    (2048, 128, 8, 512, 32),
    (1000, 3, 2, 40, 64),
    (500, 1024, 4, 64, 32),
    (262144, 64, 6, 64, 256),  # 1.57 M rows: ranges scanned in blocks (two-level scan)
    (100003, 32, 4, 72, 32),  # ragged last chunk; rows copied element-wise (72 x 2 bytes is not 16-byte aligned)
    (262144, 1024, 8, 16, 256),  # two-level scan over 4 groups of 256 expert columns
    (8448, 1024, 2, 16, 64),  # 33 ranges: a last block holding a single range
    (1000, 3, 2, 4096, 64),  # rows of 4096: grouped tile order, scan folded into the scatter
    (40000, 64, 6, 3072, 256),  # rows of 3072: grouped tile order written by the scan kernel (ranges)
]


@pytest.mark.parametrize("n_tok,n_exp,top_k,dim,block_m", PERM_CASES)
def test_permute_bit_exact(gpu, n_tok, n_exp, top_k, dim, block_m):
    dtype = torch.bfloat16
    route = _routing(gpu, n_tok, n_exp, top_k, dtype, seed=n_tok + dim)
    g = torch.Generator(device=gpu).manual_seed(1)
    x = torch.randn(n_tok, dim, generator=g, device=gpu).to(dtype)
    perm = ops.moe_permute(route, x, n_exp, block_m)
    torch.cuda.synchronize()
    toks, slots, offs = R.permutation(route.topk_idx.long(), n_exp)
    assert torch.equal(perm.expert_offsets.long(), offs)
    assert torch.equal(perm.sorted_token.long(), toks)
    assert torch.equal(perm.x_perm, x[toks])
    assert torch.equal(perm.sorted_w, route.topk_w[toks, slots])
    pos = torch.empty_like(perm.token_pos)
    pos[toks, slots] = torch.arange(toks.numel(), device=gpu, dtype=torch.int32)
    assert torch.equal(perm.token_pos, pos)
    # Tile list: ceil(count / block_m) tiles per expert. Rows of 3072 or more
    # elements: every expert's whole groups of 8 tiles first (expert order),
    # then the tiles left over (expert order), tiles[3] = the number of
    # grouped tiles; narrower rows: expert order, tiles[3] = the tile count.
    tl = perm.tiles.cpu().tolist()
    counts = (offs[1:] - offs[:-1]).tolist()
    grouped, left = [], []
    for e, c in enumerate(counts):
        n = -(-c // block_m)
        n_grouped = n - n % 8 if dim >= 3072 else 0
        for j in range(n):
            (grouped if j < n_grouped else left).append([e, offs[e].item() + j * block_m, offs[e + 1].item()])
    expect = grouped + left
    assert tl[0] == len(expect) and tl[1] == block_m
    assert tl[3] == (len(grouped) if dim >= 3072 else len(expect))
    got = [tl[4 + 3 * i: 7 + 3 * i] for i in range(tl[0])]
    assert got == expect


def _experts(gpu, n_exp, dim, dim_ffn, dtype, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)

    def w(*shape):
        return (torch.randn(*shape, generator=g, device=gpu) * 0.02).to(dtype)

    return [R.ExpertWeights(w(dim_ffn, dim), w(dim_ffn, dim), w(dim, dim_ffn)) for _ in range(n_exp)]


GEMM_CASES = [
    # (tokens, experts, top_k, dim, dim_ffn, dtype): MFMA 256-row, MFMA 32-row, general kernel
    (2048, 8, 2, 1024, 1536, torch.bfloat16),
    (4096, 64, 6, 2048, 1408, torch.bfloat16),
    (64, 128, 8, 4096, 1536, torch.bfloat16),
    (300, 16, 4, 512, 256, torch.bfloat16),
    (257, 6, 2, 72, 40, torch.bfloat16),
    # one 64-K step per tile, several tiles per workgroup: every step is a
    # tile's last and prefetches the next tile's first fragments
    (16384, 4, 2, 64, 1024, torch.bfloat16),
    # partial last column tiles (dims multiples of 64, not of 128 / 256): 256-, 128- and 32-row tiles
    (2048, 8, 2, 2880, 2880, torch.bfloat16),
    (300, 16, 4, 192, 320, torch.bfloat16),
    (64, 32, 4, 704, 576, torch.bfloat16),
    (1024, 16, 4, 448, 960, torch.bfloat16),
    # fp32: matrix-core kernel (64-row tiles, K % 32 == 0) with each column-tile width, and the general kernel
    (1024, 8, 2, 512, 1024, torch.float32),  # gate/up 128-wide tiles, down 64-wide
    (4096, 16, 4, 1024, 512, torch.float32),  # 256-wide tiles for both
    (300, 16, 4, 128, 96, torch.float32),  # gate/up 64-wide (96 columns), partial row tiles, skewed experts
    (200, 4, 2, 32, 64, torch.float32),  # gate/up one K step; down 32 columns: general kernel
    (100, 5, 3, 36, 20, torch.float32),
]


@pytest.mark.parametrize("n_tok,n_exp,top_k,dim,dim_ffn,dtype", GEMM_CASES)
def test_grouped_gemms_match_torch(gpu, n_tok, n_exp, top_k, dim, dim_ffn, dtype):
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    route = _routing(gpu, n_tok, n_exp, top_k, dtype, seed=3)
    g = torch.Generator(device=gpu).manual_seed(2)
    x = torch.randn(n_tok, dim, generator=g, device=gpu).to(dtype)
    experts = _experts(gpu, n_exp, dim, dim_ffn, dtype, seed=5)
    bm = ops.select_block_m(n_tok, n_exp, top_k, dim, dim_ffn, dtype)
    perm = ops.moe_permute(route, x, n_exp, bm)
    tg = ops.expert_weight_table([e.gate for e in experts], (dim_ffn, dim))
    tu = ops.expert_weight_table([e.up for e in experts], (dim_ffn, dim))
    td = ops.expert_weight_table([e.down for e in experts], (dim, dim_ffn))
    h = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tg, tu, n_exp, dim_ffn, bm)
    y = ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, n_exp, dim, bm)
    torch.cuda.synchronize()
    offs = perm.expert_offsets.tolist()
    for e, w in enumerate(experts):
        a, b = offs[e], offs[e + 1]
        if a == b:
            continue
        xe = perm.x_perm[a:b]
        h_ref = F.linear(xe, w.up) * F.silu(F.linear(xe, w.gate))  # mlp.py:23
        torch.testing.assert_close(h[a:b], h_ref, **tol)
        # down on the kernel's own h, so the two GEMMs are checked separately
        y_ref = F.linear(h[a:b], w.down) * perm.sorted_w[a:b].unsqueeze(-1)  # mlp.py:24, :97
        torch.testing.assert_close(y[a:b], y_ref, **tol)


def test_grouped_gemms_at_the_mixtral_shape(gpu):
    """The Mixtral-shaped workload's own activations, routing and expert
    weights (D 4096, F 14336, 8 experts, top-2, 16384 tokens) through the
    kernels the layer runs there: the gate/up GEMM gathering x through the
    permutation (run-time claims engaged: 64 K steps per tile) and the down
    GEMM with its workspace (224 K steps: claims and the split tail). Every
    expert's h and y against F.linear at the reference's rounding points
    (mlp.py:23-24, :97), every element within rtol 2e-2 / atol 2e-3."""
    w = WORKLOADS[HEADLINE]
    layer, x = make_layer(w, gpu)
    E, D, Fd, K = w.n_experts, w.dim, w.dim_ffn, w.top_k
    x2 = x.view(-1, D)
    with torch.no_grad():
        route = ops.moe_route(layer.router(x2), K)
    bm = ops.select_block_m(x2.shape[0], E, K, D, Fd, x2.dtype)
    assert bm == 256
    perm = ops.moe_permute(route, x2, E, bm, copy_rows=False)
    experts = layer.routed_experts
    tg = ops.expert_weight_table([m.gate.weight for m in experts], (Fd, D))
    tu = ops.expert_weight_table([m.up.weight for m in experts], (Fd, D))
    td = ops.expert_weight_table([m.down.weight for m in experts], (D, Fd))
    h = ops.moe_gemm_gate_up_gather(x2, perm.sorted_token, perm.tiles, tg, tu, E, Fd, bm)
    y = ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, E, D, bm)
    torch.cuda.synchronize()
    offs = perm.expert_offsets.tolist()
    tok = perm.sorted_token.long()
    with torch.no_grad():
        for e, m in enumerate(experts):
            a, b = offs[e], offs[e + 1]
            assert b - a > 3000, (e, b - a)
            xe = x2[tok[a:b]]
            h_ref = F.linear(xe, m.up.weight) * F.silu(F.linear(xe, m.gate.weight))  # mlp.py:23
            torch.testing.assert_close(h[a:b], h_ref, **BF16_TOL)
            del h_ref
            y_ref = F.linear(h[a:b], m.down.weight) * perm.sorted_w[a:b].unsqueeze(-1)  # mlp.py:24, :97
            torch.testing.assert_close(y[a:b], y_ref, **BF16_TOL)
            print(f"expert {e}: {b - a} rows, h and y within tolerance on every element", flush=True)


def _tail_split(n_live, n_tiles_n, capacity, ksteps, cus):
    """Tail tiles and K slices of the 256-row down kernel's last round, as the
    kernel decides them: (L, S), S = 1 when the tail runs whole (tiles of
    fewer than 64 K steps never split)."""
    if ksteps < 64:
        return 0, 1
    grid = min(capacity * n_tiles_n, cus)
    total = n_live * n_tiles_n
    left = total % grid
    s = min(grid // left, ksteps // 8) if 0 < left and 2 * left <= grid else 1
    return (left, s) if s >= 2 else (0, 1)


@pytest.mark.parametrize("n_tok,n_exp,top_k,dim,dim_ffn,packed", [
    (8192, 8, 2, 1024, 4096, False),  # ~68 row tiles x 4 column tiles: a short last round, split 8 ways
    (8192, 8, 2, 1024, 4096, True),
    (6144, 8, 2, 2048, 1408, False),  # ~52 x 8: 22 K steps per down tile, too short to split; gate/up
                                      # 32 steps: claims
    (16384, 1, 1, 512, 4096, False),  # one expert: 64 row tiles x 2 = 128 tiles, a partial first round
    (4096, 4, 2, 256, 1024, False),  # 32 row tiles x 1 column tile
    # 32 K steps or more per tile: the last tenth of the items claimed at run time
    (16384, 8, 2, 3072, 1024, False),  # gate/up: ~132 row tiles x 8 column tiles
    (16384, 8, 2, 3072, 1024, True),
    (24576, 8, 2, 1024, 4096, False),  # down: ~196 x 4, with a split tail
    (24576, 16, 2, 512, 2048, False),  # ~200 x 2 down (32 steps: claims) / x 16 gate/up (8 steps: static)
    # skewed routers (a Zipf-like bias: hot experts, empty ones) on rows of 3072+ elements: the tile list
    # in whole groups of one expert with a tail of leftover tiles, padding-only waves idle in the tail
    pytest.param(16384, 16, 2, 3072, 1024, False, id="skewed-grouped-gate_up48"),
    pytest.param(16384, 8, 2, 3072, 4096, False, id="skewed-grouped-both64-split"),
])
def test_gemm_run_time_claims_and_split_tail(gpu, n_tok, n_exp, top_k, dim, dim_ffn, packed, request):
    """The 256-row GEMMs with their workspace (the last tenth of the tiles
    claimed at run time; the down GEMM's last round split along K, partial
    sums reduced in slice order) against the same GEMMs with every tile dealt
    in advance and run whole, and against torch at the reference's rounding
    points: gate/up bit-identical, down tiles outside the split tail
    bit-identical and the tail within the GEMM tolerance, and the train
    variants' outputs bit-identical to the inference ones."""
    dtype = torch.bfloat16
    if "skewed" in request.node.callspec.id:
        logits = _logits(gpu, n_tok, n_exp, torch.float32, 1.0, 11)
        rank = torch.randperm(n_exp, generator=torch.Generator().manual_seed(3)).to(gpu) + 1
        route = ops.moe_route((logits - 3.0 * torch.log(rank.float())).to(dtype), top_k)
    else:
        route = _routing(gpu, n_tok, n_exp, top_k, dtype, seed=11)
    g = torch.Generator(device=gpu).manual_seed(4)
    x = torch.randn(n_tok, dim, generator=g, device=gpu).to(dtype)
    experts = _experts(gpu, n_exp, dim, dim_ffn, dtype, seed=6)
    bm = 256
    perm = ops.moe_permute(route, x, n_exp, bm)
    tg = ops.expert_weight_table([e.gate for e in experts], (dim_ffn, dim))
    tu = ops.expert_weight_table([e.up for e in experts], (dim_ffn, dim))
    td = ops.expert_weight_table([e.down for e in experts], (dim, dim_ffn))
    h = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tg, tu, n_exp, dim_ffn, bm)
    h_static = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tg, tu, n_exp, dim_ffn, bm, balance=False)
    h_gather = ops.moe_gemm_gate_up_gather(x, perm.sorted_token, perm.tiles, tg, tu, n_exp, dim_ffn, bm)
    if packed:
        tpg = ops.expert_weight_table([ops.moe_pack_gate_up(e.gate, e.up) for e in experts], (2 * dim_ffn, dim))
        h_packed = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tpg, tpg, n_exp, dim_ffn, bm, packed=True)
        td = ops.expert_weight_table([ops.moe_pack_down(e.down) for e in experts], (dim, dim_ffn))
    y = ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, n_exp, dim, bm, packed=packed)
    y_whole = ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, n_exp, dim, bm, packed=packed, balance=False)
    # the same calls again: which workgroup claims a tile changes from run to
    # run, the bits may not
    h_again = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tg, tu, n_exp, dim_ffn, bm)
    h_gather_again = ops.moe_gemm_gate_up_gather(x, perm.sorted_token, perm.tiles, tg, tu, n_exp, dim_ffn, bm)
    y_again = ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, n_exp, dim, bm, packed=packed)
    torch.cuda.synchronize()
    assert torch.equal(h, h_again) and torch.equal(h, h_gather_again) and torch.equal(y, y_again)
    assert torch.equal(h, h_static) and torch.equal(h, h_gather)
    if packed:
        assert torch.equal(h, h_packed)
    tl = perm.tiles.cpu().tolist()
    n_live, capacity = tl[0], (len(tl) - 4) // 3
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    n_tiles_n = -(-dim // 256)
    left, s = _tail_split(n_live, n_tiles_n, capacity, dim_ffn // 64, cus)
    counts = (perm.expert_offsets[1:] - perm.expert_offsets[:-1]).tolist()
    print(f"{n_live} row tiles x {n_tiles_n}: {left} tail tiles split {s} ways; rows per expert {counts}; "
          f"grouped tiles {tl[3]}", flush=True)
    if "skewed" in request.node.callspec.id:
        # the case it is for: (nearly) empty experts, hot ones with whole groups, a tail with tiles of at
        # most 128 rows
        assert min(counts) <= 16 and tl[3] >= 16 and tl[3] < n_live
        tail_rows = [min(256, tl[6 + 3 * i] - tl[5 + 3 * i]) for i in range(tl[3], n_live)]
        assert min(tail_rows) <= 128, tail_rows
    # which (row tile, column tile) blocks differ between the split and whole orders
    row_tile = torch.full((h.shape[0],), -1, dtype=torch.long)
    for i in range(n_live):
        r0, end = tl[5 + 3 * i], tl[6 + 3 * i]
        row_tile[r0:min(r0 + bm, end)] = i
    diff = (y != y_whole).cpu()
    rows, cols = diff.nonzero(as_tuple=True)
    blocks = {(int(row_tile[r]), int(c) // 256) for r, c in zip(rows.tolist(), cols.tolist())}
    assert len(blocks) <= left, (len(blocks), left)
    if s == 1:
        assert torch.equal(y, y_whole)
    torch.testing.assert_close(y, y_whole, **BF16_TOL)
    offs = perm.expert_offsets.tolist()
    for e, w in enumerate(experts):
        a, b = offs[e], offs[e + 1]
        if a == b:
            continue
        y_ref = F.linear(h[a:b], w.down) * perm.sorted_w[a:b].unsqueeze(-1)  # mlp.py:24, :97
        torch.testing.assert_close(y[a:b], y_ref, **BF16_TOL)
        if "skewed" in request.node.callspec.id:
            xe = perm.x_perm[a:b]
            h_ref = (F.silu(F.linear(xe, w.gate)) * F.linear(xe, w.up))  # mlp.py:22-23
            torch.testing.assert_close(h[a:b], h_ref, **BF16_TOL)
    if not packed:
        h_tr, _ = ops.moe_gemm_gate_up_train(perm.x_perm, perm.tiles, tg, tu, n_exp, dim_ffn)
        y_tr, y_unw = ops.moe_gemm_down_train(h, perm.tiles, td, perm.sorted_w, n_exp, dim)
        torch.cuda.synchronize()
        assert torch.equal(h_tr, h) and torch.equal(y_tr, y)
        for e, w in enumerate(experts):
            a, b = offs[e], offs[e + 1]
            if a < b:
                torch.testing.assert_close(y_unw[a:b], F.linear(h[a:b], w.down), **BF16_TOL)



def test_weight_table_keeps_its_weights_alive(gpu):
    """A pointer table outliving the caller's list of weights still owns them:
    their storage is not handed to new tensors while the table lives."""
    w = [torch.randn(256, 128, device=gpu).to(torch.bfloat16) for _ in range(3)]
    ref = [t.clone() for t in w]
    table = ops.expert_weight_table(w, (256, 128))
    ptrs = {t.data_ptr() for t in w}
    del w
    junk = [torch.full((256, 128), float("nan"), device=gpu, dtype=torch.bfloat16) for _ in range(6)]
    assert not ptrs & {j.data_ptr() for j in junk}
    kept = table._astrai_weights
    assert all(torch.equal(a, b) for a, b in zip(kept, ref))
    assert [t.data_ptr() for t in kept] == table.cpu().tolist()


@pytest.mark.parametrize("n_tok,n_exp,top_k,dim,dim_ffn", [
    (2048, 8, 2, 1024, 1536),  # 256-row tiles
    (300, 16, 4, 512, 256),  # 64-row tiles
    (64, 128, 8, 4096, 1536),  # decode-sized loads, some experts empty
    (16384, 4, 2, 256, 128),  # many rows per expert, several tiles per workgroup
    (1, 8, 2, 256, 128),  # one token
    (2048, 8, 2, 2880, 2880),  # partial last column tile
])
def test_gate_up_gather_bit_identical(gpu, n_tok, n_exp, top_k, dim, dim_ffn):
    # the gate/up GEMM reading x[sorted_token] directly equals the GEMM on the
    # copied x_perm, and the index-only permutation equals the full one
    dtype = torch.bfloat16
    assert ops.gather_supported(n_tok, dim, dim_ffn, dtype)
    route = _routing(gpu, n_tok, n_exp, top_k, dtype, seed=12)
    g = torch.Generator(device=gpu).manual_seed(13)
    x = torch.randn(n_tok, dim, generator=g, device=gpu).to(dtype)
    experts = _experts(gpu, n_exp, dim, dim_ffn, dtype, seed=14)
    bm = ops.select_block_m(n_tok, n_exp, top_k, dim, dim_ffn, dtype)
    assert bm in (32, 64, 128, 256)
    perm = ops.moe_permute(route, x, n_exp, bm)
    idx = ops.moe_permute(route, x, n_exp, bm, copy_rows=False)
    assert idx.x_perm is None
    for a, b in zip(perm[:4], idx[:4]):
        assert torch.equal(a, b)
    n_live = perm.tiles[0].item()  # entries past the live tiles are never written
    assert torch.equal(perm.tiles[:4 + 3 * n_live], idx.tiles[:4 + 3 * n_live])
    tg = ops.expert_weight_table([e.gate for e in experts], (dim_ffn, dim))
    tu = ops.expert_weight_table([e.up for e in experts], (dim_ffn, dim))
    h = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tg, tu, n_exp, dim_ffn, bm)
    hg = ops.moe_gemm_gate_up_gather(x, idx.sorted_token, idx.tiles, tg, tu, n_exp, dim_ffn, bm)
    torch.cuda.synchronize()
    assert torch.equal(hg, h)


def _packed_layout(w0, w1, tile_rows):
    """Expected packed order of one expert's weight: per column tile of 256
    rows (gate/up: ``tile_rows`` = 128 gate rows then the same 128 up rows;
    down: 256 rows of ``w0``) and per 64-wide K step, a block of 256 rows x 8
    chunks of 8 elements in which row r keeps its chunk c at position
    c ^ ((r >> 1) & 7)."""
    n, k = w0.shape
    if w1 is not None:
        w = torch.cat([w0.view(n // tile_rows, tile_rows, k), w1.view(n // tile_rows, tile_rows, k)], 1)
    else:
        w = w0.view(n // tile_rows, tile_rows, k)
    nt = w.shape[0]
    blocks = w.view(nt, 256, k // 64, 8, 8).permute(0, 2, 1, 3, 4)  # [tile, kstep, row, chunk, 8]
    r = torch.arange(256, device=w0.device)[:, None]
    src_chunk = torch.arange(8, device=w0.device)[None, :] ^ ((r >> 1) & 7)
    idx = src_chunk[None, None, :, :, None].expand(nt, k // 64, 256, 8, 8)
    return blocks.gather(3, idx).reshape(-1, k)


@pytest.mark.parametrize("n_tok,n_exp,top_k,dim,dim_ffn,block_m", [
    (600, 2, 2, 1024, 65536, 256),  # down K = 65536: 128 KB weight rows, 32 MB per 256-row tile
    (300, 2, 1, 65536, 256, 256),  # gate/up K = 65536
    (64, 2, 2, 65536, 512, 32),  # the 32-row kernels at the same K
    (128, 2, 2, 65536, 512, 64),  # the 64-row kernels at the same K
])
def test_long_k_rows(gpu, n_tok, n_exp, top_k, dim, dim_ffn, block_m):
    # byte offsets within a tile grow with K (rows x K x 2 bytes, 32-bit in the
    # kernels): long rows against torch, per expert
    dtype = torch.bfloat16
    route = _routing(gpu, n_tok, n_exp, top_k, dtype, seed=31)
    g = torch.Generator(device=gpu).manual_seed(32)
    # x scaled so the gate pre-activation keeps its K = 4096 spread (std 1.3): at std 5, a one-ulp bf16 rounding
    # flip of g (fp32 sums in another order) is amplified ~6x by silu at g ~ -5, past the bf16 tolerance
    x = (torch.randn(n_tok, dim, generator=g, device=gpu) * min(1.0, (4096 / dim) ** 0.5)).to(dtype)
    experts = _experts(gpu, n_exp, dim, dim_ffn, dtype, seed=33)
    perm = ops.moe_permute(route, x, n_exp, block_m)
    tg = ops.expert_weight_table([e.gate for e in experts], (dim_ffn, dim))
    tu = ops.expert_weight_table([e.up for e in experts], (dim_ffn, dim))
    td = ops.expert_weight_table([e.down for e in experts], (dim, dim_ffn))
    h = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tg, tu, n_exp, dim_ffn, block_m)
    y = ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, n_exp, dim, block_m)
    torch.cuda.synchronize()
    offs = perm.expert_offsets.tolist()
    for e, w in enumerate(experts):
        a, b = offs[e], offs[e + 1]
        if a == b:
            continue
        # fp32 sums rounded to bf16 at the reference's rounding points (mlp.py:23-24, :97)
        xe = perm.x_perm[a:b].float()
        g = F.linear(xe, w.gate.float()).to(dtype)
        u = F.linear(xe, w.up.float()).to(dtype)
        torch.testing.assert_close(h[a:b], u * F.silu(g), **BF16_TOL)
        y_ref = F.linear(h[a:b].float(), w.down.float()).to(dtype) * perm.sorted_w[a:b].unsqueeze(-1)
        torch.testing.assert_close(y[a:b], y_ref, **BF16_TOL)


@pytest.mark.parametrize("n_tok,n_exp,top_k,dim,dim_ffn", [
    (2048, 8, 2, 1024, 1536),  # 256-row tiles
    (300, 16, 4, 512, 256),  # 32-row tiles
    (64, 128, 8, 4096, 1536),  # decode-sized loads over many experts
    (16384, 4, 2, 256, 128),  # one column tile per expert for gate/up
    (1024, 128, 8, 4096, 1536),  # 128-row tiles (64 rows per expert)
])
def test_packed_gemms_bit_identical(gpu, n_tok, n_exp, top_k, dim, dim_ffn):
    dtype = torch.bfloat16
    assert ops.packed_supported(dim, dim_ffn, dtype)
    route = _routing(gpu, n_tok, n_exp, top_k, dtype, seed=7)
    g = torch.Generator(device=gpu).manual_seed(8)
    x = torch.randn(n_tok, dim, generator=g, device=gpu).to(dtype)
    experts = _experts(gpu, n_exp, dim, dim_ffn, dtype, seed=9)
    bm = ops.select_block_m(n_tok, n_exp, top_k, dim, dim_ffn, dtype)
    perm = ops.moe_permute(route, x, n_exp, bm)
    tg = ops.expert_weight_table([e.gate for e in experts], (dim_ffn, dim))
    tu = ops.expert_weight_table([e.up for e in experts], (dim_ffn, dim))
    td = ops.expert_weight_table([e.down for e in experts], (dim, dim_ffn))
    h = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tg, tu, n_exp, dim_ffn, bm)
    y = ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, n_exp, dim, bm)
    pg = [ops.moe_pack_gate_up(e.gate, e.up) for e in experts]
    pd = [ops.moe_pack_down(e.down) for e in experts]
    for e in (0, n_exp - 1):
        assert torch.equal(pg[e], _packed_layout(experts[e].gate, experts[e].up, 128))
        assert torch.equal(pd[e], _packed_layout(experts[e].down, None, 256))
    tpg = ops.expert_weight_table(pg, (2 * dim_ffn, dim))
    tpd = ops.expert_weight_table(pd, (dim, dim_ffn))
    hp = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tpg, tpg, n_exp, dim_ffn, bm, packed=True)
    yp = ops.moe_gemm_down(h, perm.tiles, tpd, perm.sorted_w, n_exp, dim, bm, packed=True)
    torch.cuda.synchronize()
    assert torch.equal(hp, h)
    assert torch.equal(yp, y)


@pytest.mark.parametrize("n_tok,n_exp,top_k,dim,dim_ffn", [
    (64, 128, 8, 4096, 1536),  # decode shape: <= 10 rows per expert, some experts empty
    (64, 8, 2, 4096, 2048),  # few experts, many column tiles per expert
    (2048, 8, 2, 1024, 1280),  # many row tiles per expert, several tiles per workgroup
    (700, 16, 4, 2048, 768),  # ragged row tiles
    (1, 8, 2, 1024, 1024),  # one token
    (512, 8, 1, 1024, 512),  # 64 rows per expert: one 64-row tile each
    (1024, 8, 1, 1024, 512),  # 128 rows per expert: one 128-row tile each
    (900, 16, 3, 2048, 768),  # ~170 rows per expert: two 128-row tiles, ragged
])
@pytest.mark.parametrize("bm", [32, 64, 128])
def test_decode_gemms_row_strided_packed_gathered_bit_identical(gpu, n_tok, n_exp, top_k, dim, dim_ffn, bm):
    # 32-, 64- and 128-row tiles: row-strided, packed and gathered operands
    # give equal bits, the tile heights give equal bits (the same per-wave MFMA
    # sequence over K), and every expert's rows match torch
    dtype = torch.bfloat16
    route = _routing(gpu, n_tok, n_exp, top_k, dtype, seed=21)
    g = torch.Generator(device=gpu).manual_seed(22)
    x = torch.randn(n_tok, dim, generator=g, device=gpu).to(dtype)
    experts = _experts(gpu, n_exp, dim, dim_ffn, dtype, seed=23)
    perm = ops.moe_permute(route, x, n_exp, bm)
    tg = ops.expert_weight_table([e.gate for e in experts], (dim_ffn, dim))
    tu = ops.expert_weight_table([e.up for e in experts], (dim_ffn, dim))
    td = ops.expert_weight_table([e.down for e in experts], (dim, dim_ffn))
    h = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tg, tu, n_exp, dim_ffn, bm)
    hg = ops.moe_gemm_gate_up_gather(x, perm.sorted_token, perm.tiles, tg, tu, n_exp, dim_ffn, bm)
    y = ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, n_exp, dim, bm)
    pg = [ops.moe_pack_gate_up(e.gate, e.up) for e in experts]  # the tables hold pointers: keep the copies
    pd = [ops.moe_pack_down(e.down) for e in experts]
    tpg = ops.expert_weight_table(pg, (2 * dim_ffn, dim))
    tpd = ops.expert_weight_table(pd, (dim, dim_ffn))
    hp = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tpg, tpg, n_exp, dim_ffn, bm, packed=True)
    yp = ops.moe_gemm_down(h, perm.tiles, tpd, perm.sorted_w, n_exp, dim, bm, packed=True)
    if bm != 32:
        p32 = ops.moe_permute(route, x, n_exp, 32)
        h32 = ops.moe_gemm_gate_up(p32.x_perm, p32.tiles, tg, tu, n_exp, dim_ffn, 32)
        y32 = ops.moe_gemm_down(h32, p32.tiles, td, p32.sorted_w, n_exp, dim, 32)
    torch.cuda.synchronize()
    assert torch.equal(h, hp)
    assert torch.equal(hg, hp)
    assert torch.equal(y, yp)
    if bm != 32:
        assert torch.equal(p32.sorted_token, perm.sorted_token)
        assert torch.equal(h32, h)
        assert torch.equal(y32, y)
    # and against torch, per expert (first rows of the output only where rows exist)
    offs = perm.expert_offsets.tolist()
    for e in range(n_exp):
        a, b = offs[e], offs[e + 1]
        if a == b:
            continue
        w = experts[e]
        xe = perm.x_perm[a:b]
        h_ref = F.linear(xe, w.up) * F.silu(F.linear(xe, w.gate))  # mlp.py:23
        torch.testing.assert_close(h[a:b], h_ref, **BF16_TOL)
        y_ref = F.linear(h[a:b], w.down) * perm.sorted_w[a:b].unsqueeze(-1)  # mlp.py:24, :97
        torch.testing.assert_close(y[a:b], y_ref, **BF16_TOL)


@pytest.mark.parametrize("n_tok,n_exp,top_k,dim,n_shared,dtype", [
    (1000, 8, 2, 256, 0, torch.bfloat16),
    (513, 16, 5, 128, 0, torch.bfloat16),
    (100, 8, 3, 40, 2, torch.bfloat16),
    (64, 4, 4, 64, 3, torch.float32),
    (77, 8, 8, 24, 1, torch.bfloat16),
    (300, 16, 12, 256, 0, torch.bfloat16),  # top_k above 8
    (200, 4, 1, 128, 0, torch.bfloat16),
    (90, 32, 20, 64, 1, torch.float32),
])
def test_combine_bit_exact(gpu, n_tok, n_exp, top_k, dim, n_shared, dtype):
    route = _routing(gpu, n_tok, n_exp, top_k, dtype, seed=11)
    g = torch.Generator(device=gpu).manual_seed(4)
    x = torch.randn(n_tok, dim, generator=g, device=gpu).to(dtype)
    perm = ops.moe_permute(route, x, n_exp, 64)
    y = torch.randn(n_tok * top_k, dim, generator=g, device=gpu).to(dtype)
    shared = torch.randn(n_shared, n_tok, dim, generator=g, device=gpu).to(dtype) if n_shared else None
    out = ops.moe_combine(y, perm.token_pos, shared)
    # Reference sequence: zeros, index_add_ per expert ascending (mlp.py:89-98),
    # shared mean as Python sum / n (mlp.py:77), then shared + routed (:71).
    ref = torch.zeros(n_tok, dim, device=gpu, dtype=dtype)
    offs = perm.expert_offsets.tolist()
    for e in range(n_exp):
        a, b = offs[e], offs[e + 1]
        if a < b:
            ref.index_add_(0, perm.sorted_token[a:b].long(), y[a:b])
    sh = torch.zeros_like(ref) if shared is None else sum(shared[i] for i in range(n_shared)) / n_shared
    ref = sh + ref
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # unweighted rows and their routing weights: each row scaled and rounded
    # first (mlp.py:97's y * w), then the same sum
    out_w = ops.moe_combine(y, perm.token_pos, shared, row_w=perm.sorted_w)
    y_w = (y.float() * perm.sorted_w.float().unsqueeze(-1)).to(dtype)
    torch.cuda.synchronize()
    assert torch.equal(out_w, ops.moe_combine(y_w, perm.token_pos, shared))


@pytest.mark.parametrize("n_tok,dim,dim_ffn,dtype", [
    (1, 256, 128, torch.bfloat16),      # 32-row tiles
    (200, 256, 256, torch.bfloat16),    # 64-row tiles
    (3000, 2048, 2048, torch.bfloat16), # 128-row tiles
    (8192, 2048, 2048, torch.bfloat16), # 256-row tiles
    (37, 40, 24, torch.bfloat16),       # general kernel
    (129, 64, 96, torch.float32),       # general kernel, fp32
])
def test_dense_expert_tile_list_and_gemms(gpu, n_tok, dim, dim_ffn, dtype):
    # one dense expert (the shared experts, MLP; mlp.py:22-25) over all rows:
    # the device-built tile list has the layout the permutation writes, and the
    # down GEMM without row weights multiplies by nothing
    bm = ops.dense_block_m(n_tok, dim, dim_ffn, dtype)
    tiles, offsets = ops.dense_tiles(n_tok, bm, gpu, with_offsets=True)
    n = -(-n_tok // bm)
    want = [n, bm, n, n - n % 8] + [v for i in range(n) for v in (0, i * bm, n_tok)]
    torch.cuda.synchronize()
    assert tiles.tolist() == want and offsets.tolist() == [0, n_tok]
    g = torch.Generator(device=gpu).manual_seed(5)
    x = torch.randn(n_tok, dim, generator=g, device=gpu).to(dtype)
    w = R.ExpertWeights(*(torch.randn(s, generator=g, device=gpu).mul(0.05).to(dtype)
                          for s in ((dim_ffn, dim), (dim_ffn, dim), (dim, dim_ffn))))
    tg, tu, td = (ops.expert_weight_table([t], tuple(t.shape)) for t in (w.gate, w.up, w.down))
    out = ops.moe_dense_mlp(x, tg, tu, td, dim_ffn, tiles=tiles)
    h = ops.moe_gemm_gate_up(x, tiles, tg, tu, 1, dim_ffn, bm)
    ones = torch.ones(n_tok, dtype=dtype, device=gpu)
    y_ones = ops.moe_gemm_down(h, tiles, td, ones, 1, dim, bm)
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    torch.cuda.synchronize()
    assert torch.equal(out, y_ones)  # no row weights == weight 1, bit for bit
    # each GEMM against torch on the same inputs, at the reference's rounding points
    torch.testing.assert_close(h, F.linear(x, w.up) * F.silu(F.linear(x, w.gate)), **tol)  # mlp.py:23
    torch.testing.assert_close(out, F.linear(h, w.down), **tol)  # mlp.py:24
    with pytest.raises(ValueError, match="built for block_m"):
        ops.moe_gemm_gate_up(x, tiles, tg, tu, 1, dim_ffn, 256 if bm != 256 else 64)
