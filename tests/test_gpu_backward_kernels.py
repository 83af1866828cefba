"""Parity of the backward kernels (grouped dgrad / wgrad GEMMs, row gradient)
and of the training forward's saved tensors with torch on the same device.

Each kernel is checked on its own inputs against a float32 torch evaluation of
the formula torch autograd applies to mlp.py:22-25 and :97-98, at the
reference's rounding points where the kernel reproduces them exactly
(bit-exact checks) and otherwise within the layer's tolerance: elementwise
|got - ref| <= rtol |ref| + atol max|ref| with (rtol, atol) = (2e-2, 1e-3) in
bf16 and (1e-4, 1e-6) in fp32, >= 99.9 % of the elements passing and the worst
error below 5 % (bf16) / 1e-4 (fp32) of max|ref|. The cases cover both kernel
families: the matrix-core kernels (bf16, dim % 256 == 0, dim_ffn % 128 == 0)
and the general-shape ones (fp32, other shapes, dim_ffn not a multiple of 4 —
the saved projections' last block of columns then holds fewer than 4).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from astrai_amd.extension import ops

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _close(got, ref, label):
    fp32 = got.dtype == torch.float32
    rtol, atol, worst_frac = (1e-4, 1e-6, 1e-4) if fp32 else (2e-2, 1e-3, 5e-2)
    got, ref = got.float(), ref.float()
    scale = ref.abs().max().item() or 1.0
    err = (got - ref).abs()
    frac = (err <= rtol * ref.abs() + atol * scale).float().mean().item()
    worst = err.max().item()
    assert frac >= 0.999, f"{label}: {frac:.5f} within tolerance (max err {worst:.3e}, scale {scale:.3e})"
    assert worst <= worst_frac * scale, f"{label}: max err {worst:.3e} vs scale {scale:.3e}"


def _setup(gpu, n_tok, n_exp, top_k, dim, dim_ffn, skew=0.0, seed=0, dtype=BF):
    g = torch.Generator(device=gpu).manual_seed(seed)
    logits = torch.randn(n_tok, n_exp, generator=g, device=gpu)
    logits += skew * torch.log1p(torch.arange(n_exp, device=gpu, dtype=torch.float32)).neg()
    route = ops.moe_route(logits.to(dtype), top_k)
    x = torch.randn(n_tok, dim, generator=g, device=gpu).to(dtype)
    perm = ops.moe_permute(route, x, n_exp, ops.train_block_m(dim, dim_ffn, dtype))

    def w(*shape):
        return (torch.randn(*shape, generator=g, device=gpu) * 0.02).to(dtype)

    wg = [w(dim_ffn, dim) for _ in range(n_exp)]
    wu = [w(dim_ffn, dim) for _ in range(n_exp)]
    wd = [w(dim, dim_ffn) for _ in range(n_exp)]
    tables = (ops.expert_weight_table(wg, (dim_ffn, dim)), ops.expert_weight_table(wu, (dim_ffn, dim)),
              ops.expert_weight_table(wd, (dim, dim_ffn)))
    return perm, (wg, wu, wd), tables, g


CASES = [
    # (tokens, experts, top_k, dim, dim_ffn, skew, dtype): matrix-core kernels
    (2048, 8, 2, 1024, 1536, 0.0, BF),
    (300, 16, 4, 512, 384, 0.0, BF),  # partial 256-column tiles, ~75 rows per expert
    (64, 128, 8, 256, 128, 0.0, BF),  # a few rows per expert, some experts empty
    (3000, 8, 2, 256, 640, 3.0, BF),  # skewed: one expert holds most rows
    (1024, 8, 2, 704, 576, 0.0, BF),  # dims multiples of 64 only: partial last column tiles everywhere
    (300, 8, 4, 192, 320, 1.0, BF),
    # rows of 3072: the tile list in whole groups of one expert (the skew gives the hot expert several),
    # dgrad_down's 48-step tiles let padding-only waves idle in the list's tail only
    (6000, 8, 2, 3072, 512, 3.0, BF),
    # general-shape kernels
    (300, 8, 2, 40, 24, 0.0, BF),  # the reference's tiny-config scale
    (200, 4, 2, 37, 30, 0.0, BF),  # dim_ffn % 4 == 2: a 2-column last block of g/u
    (150, 6, 3, 13, 7, 0.0, torch.float32),  # dim_ffn % 4 == 3
    (257, 8, 2, 64, 129, 0.0, torch.float32),  # dim_ffn % 4 == 1
    (500, 8, 2, 256, 128, 2.0, torch.float32),  # a matrix-core shape in fp32, skewed
]


@pytest.mark.parametrize("n_tok,n_exp,top_k,dim,dim_ffn,skew,dtype", CASES)
def test_backward_kernels(gpu, n_tok, n_exp, top_k, dim, dim_ffn, skew, dtype):
    perm, (wg, wu, wd), (tg, tu, td), gen = _setup(gpu, n_tok, n_exp, top_k, dim, dim_ffn, skew, dtype=dtype)
    E = n_exp
    bm = ops.train_block_m(dim, dim_ffn, dtype)
    # training forward: h and y*w bit-identical to the inference kernels
    h, gu = ops.moe_gemm_gate_up_train(perm.x_perm, perm.tiles, tg, tu, E, dim_ffn)
    g, u = ops.gu_split(gu)
    y, y_unw = ops.moe_gemm_down_train(h, perm.tiles, td, perm.sorted_w, E, dim)
    h_inf = ops.moe_gemm_gate_up(perm.x_perm, perm.tiles, tg, tu, E, dim_ffn, bm)
    y_inf = ops.moe_gemm_down(h, perm.tiles, td, perm.sorted_w, E, dim, bm)
    torch.cuda.synchronize()
    assert torch.equal(h, h_inf) and torch.equal(y, y_inf)
    assert torch.equal(y, (y_unw.float() * perm.sorted_w.float().unsqueeze(-1)).to(dtype))

    n_tokens = n_tok
    dout = torch.randn(n_tokens, dim, generator=gen, device=gpu).to(dtype)
    dy, dw_rows = ops.moe_row_grad(dout, perm.sorted_token, perm.sorted_w, y_unw)
    dg, du = ops.moe_gemm_dgrad_down(dy, perm.tiles, td, gu, E)
    dx_perm = ops.moe_gemm_dgrad_gate_up(dg, du, perm.tiles, tg, tu, E, dim)
    dwd = ops.moe_gemm_wgrad(dy, h, perm.expert_offsets, E)
    dwg = ops.moe_gemm_wgrad(dg, perm.x_perm, perm.expert_offsets, E)
    dwu = ops.moe_gemm_wgrad(du, perm.x_perm, perm.expert_offsets, E)
    torch.cuda.synchronize()

    # row gradient: dy bit-exact (one bf16 product), dw within summation order
    dp = dout[perm.sorted_token.long()]
    assert torch.equal(dy, (dp.float() * perm.sorted_w.float().unsqueeze(-1)).to(dtype))
    dw_ref = (dp * y_unw).float().sum(-1)
    fp32 = dtype == torch.float32
    torch.testing.assert_close(dw_rows.float(), dw_ref, rtol=1e-4 if fp32 else 2e-2,
                               atol=(1e-5 if fp32 else 1e-2) * dw_ref.abs().max().item())

    offs = perm.expert_offsets.tolist()
    live = [e for e in range(E) if offs[e + 1] > offs[e]]
    assert live
    for e in live:
        a, b = offs[e], offs[e + 1]
        xe = perm.x_perm[a:b].float()
        # saved projections
        _close(g[a:b], xe @ wg[e].float().T, f"e{e} g")
        _close(u[a:b], xe @ wu[e].float().T, f"e{e} u")
        _close(y_unw[a:b], h[a:b].float() @ wd[e].float().T, f"e{e} y")
        # dgrad of down with the SwiGLU backward (rounding points of autograd over mlp.py:23)
        dh = (dy[a:b].float() @ wd[e].float()).to(dtype).float()
        gf, uf = g[a:b].float(), u[a:b].float()
        s = torch.sigmoid(gf)
        act = F.silu(gf).to(dtype).float()
        du_ref = dh * act
        dg_ref = (dh * uf).to(dtype).float() * (s * (1 + gf * (1 - s)))
        _close(du[a:b], du_ref, f"e{e} du")
        _close(dg[a:b], dg_ref, f"e{e} dg")
        # dgrad of gate/up on the kernel's own dg, du: each linear's input
        # gradient rounded, then their sum (autograd's accumulation)
        dx_ref = ((dg[a:b].float() @ wg[e].float()).to(dtype).float()
                  + (du[a:b].float() @ wu[e].float()).to(dtype).float())
        _close(dx_perm[a:b], dx_ref, f"e{e} dx_perm")
        # weight gradients
        _close(dwd[e], dy[a:b].float().T @ h[a:b].float(), f"e{e} dW_down")
        _close(dwg[e], dg[a:b].float().T @ xe, f"e{e} dW_gate")
        _close(dwu[e], du[a:b].float().T @ xe, f"e{e} dW_up")


def test_wgrad_rows_not_multiple_of_64(gpu):
    # K = an expert's rows: 1, 63, 64, 65, 127, 129 rows; the rows past the end
    # of each expert must not contribute (they read a zero row)
    counts = [1, 63, 64, 65, 0, 127, 129]
    offs = [0]
    for c in counts:
        offs.append(offs[-1] + c)
    n_rows = offs[-1]
    gen = torch.Generator(device=gpu).manual_seed(5)
    a = torch.randn(n_rows, 264, generator=gen, device=gpu).to(BF)
    b = torch.randn(n_rows, 520, generator=gen, device=gpu).to(BF)
    off_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    dw = ops.moe_gemm_wgrad(a, b, off_t, len(counts))
    torch.cuda.synchronize()
    for e, c in enumerate(counts):
        if c == 0:
            continue
        ref = a[offs[e]:offs[e + 1]].float().T @ b[offs[e]:offs[e + 1]].float()
        _close(dw[e], ref, f"expert {e} ({c} rows)")


def _tail_split(n_live, n_tiles_n, capacity, ksteps, cus):
    """(L, S): tail tiles of the last round and their K slices, as the dgrad
    kernels decide them (S = 1: the tail runs whole; tiles of fewer than 64 K
    steps never split)."""
    if ksteps < 64:
        return 0, 1
    grid = min(capacity * n_tiles_n, cus)
    left = (n_live * n_tiles_n) % grid
    s = min(grid // left, ksteps // 8) if 0 < left and 2 * left <= grid else 1
    return (left, s) if s >= 2 else (0, 1)


def _diff_blocks(a, b, tl, n_live):
    """(row tile, column tile) blocks in which a and b differ."""
    row_tile = torch.full((a.shape[0],), -1, dtype=torch.long)
    for i in range(n_live):
        r0, end = tl[5 + 3 * i], tl[6 + 3 * i]
        row_tile[r0:min(r0 + 256, end)] = i
    rows, cols = (a != b).cpu().nonzero(as_tuple=True)
    return {(int(row_tile[r]), int(c) // 256) for r, c in zip(rows.tolist(), cols.tolist())}


@pytest.mark.parametrize("n_tok,n_exp,top_k,dim,dim_ffn", [
    (4096, 8, 2, 512, 4096),  # ~35 row tiles x 2, K 4096: 70 tiles on 78 workgroups, too many to split
    (11264, 8, 2, 1024, 4096),  # ~92 x 4 = ~368 tiles on 256 workgroups: ~112 left, split 2 ways
    (16384, 8, 2, 512, 4096),  # ~132 x 2 = ~264 tiles: a short last round split 8 ways
    (18432, 8, 2, 1024, 4096),  # ~148 x 4 = ~592 tiles: 2 whole rounds, ~80 left split 3 ways
    (16384, 8, 2, 2048, 1408),  # 22 K steps: the tail runs whole
])
def test_dgrad_split_tail(gpu, n_tok, n_exp, top_k, dim, dim_ffn):
    """The dgrad_in GEMMs (dx_perm = dg . W_gate + du . W_up) with their
    workspace (a partial last round of tiles of 64+ K steps split along K, the
    slices' fp32 sums added in slice order by a reduce launch that runs the
    tile's epilogue) against the same GEMMs run whole: dx differs only inside
    the predicted tail tiles, and there within the layer's tolerance."""
    perm, weights, (tg, tu, td), gen = _setup(gpu, n_tok, n_exp, top_k, dim, dim_ffn, seed=5)
    E = n_exp
    _, gu = ops.moe_gemm_gate_up_train(perm.x_perm, perm.tiles, tg, tu, E, dim_ffn)
    dy = (torch.randn(perm.x_perm.shape[0], dim, generator=gen, device=gpu) * 0.5).to(BF)
    dg, du = ops.moe_gemm_dgrad_down(dy, perm.tiles, td, gu, E)
    dx = ops.moe_gemm_dgrad_gate_up(dg, du, perm.tiles, tg, tu, E, dim)
    dx_w = ops.moe_gemm_dgrad_gate_up(dg, du, perm.tiles, tg, tu, E, dim, balance=False)
    # the same calls again, bit for bit (the split tail's slices and their
    # ordered reduce, and the whole-tile walk, are deterministic)
    dg2, du2 = ops.moe_gemm_dgrad_down(dy, perm.tiles, td, gu, E)
    dx2 = ops.moe_gemm_dgrad_gate_up(dg, du, perm.tiles, tg, tu, E, dim)
    dx_w2 = ops.moe_gemm_dgrad_gate_up(dg, du, perm.tiles, tg, tu, E, dim, balance=False)
    torch.cuda.synchronize()
    assert torch.equal(dg, dg2) and torch.equal(du, du2)
    assert torch.equal(dx, dx2) and torch.equal(dx_w, dx_w2)
    tl = perm.tiles.cpu().tolist()
    n_live, capacity = tl[0], (len(tl) - 4) // 3
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    left, s = _tail_split(n_live, -(-dim // 256), capacity, dim_ffn // 64, cus)
    print(f"{n_live} row tiles: dgrad_in tail {left} tiles, {s} slices", flush=True)
    blocks = _diff_blocks(dx, dx_w, tl, n_live)
    assert len(blocks) <= left, (len(blocks), left)
    if s == 1:
        assert torch.equal(dx, dx_w)
    else:
        # the split path ran: reassociated fp32 sums change some bf16 roundings
        assert blocks
    _close(dx, dx_w, "dx")
    offs = perm.expert_offsets.tolist()
    wg, wu, _ = weights
    for e in range(E):
        a, b = offs[e], offs[e + 1]
        if a == b:
            continue
        ref = (dg[a:b].float() @ wg[e].float()).to(BF).float() + (du[a:b].float() @ wu[e].float()).to(BF).float()
        _close(dx[a:b], ref, f"e{e} dx")
