"""Tensor-level wrappers of the MoE HIP kernels — one function per entry point.

Each wrapper validates its arguments in Python (``ValueError`` on bad input,
as the reference's ``astrai/extension/ops.py:26-34,266-274`` does), allocates
its outputs with torch's caching allocator on the inputs' device, and enqueues
the kernel on the current stream through the C ABI (``include/astrai_moe.h``).
Nothing here synchronises with the host.

There is no torch fallback: a wrapper whose kernel is unavailable raises
``RuntimeError`` (the reference's wrappers fall back to torch,
``ops.py:180-190``; this package is the GPU path itself).

Pipeline of the routed experts (``astrai/model/components/mlp.py:79-100``):

    logits --moe_route--> (topk_idx, topk_w, chunk_hist)
           --moe_permute--> (offsets, sorted rows, tile list, x_perm)
           --moe_gemm_gate_up--> h = up(x) * silu(gate(x))
           --moe_gemm_down--> y = down(h) * w
           --moe_combine--> out
"""

from __future__ import annotations

from typing import NamedTuple, Sequence

import torch

from astrai_amd.extension import loader
from astrai_amd.extension.loader import _available, _modules

CHUNK_TOKENS = 32  # ASTRAI_MOE_CHUNK_TOKENS
MAX_EXPERTS = 1024
MAX_TOPK = 32
TILE_HEADER = 4
TILE_STRIDE = 3
# K steps (of 64) per tile from which the 256-row down-sized GEMMs split a
# partial last round along K (kSplitMinTileSteps in mfma_tile.h)
SPLIT_MIN_STEPS = 64

_DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1}


class RouteResult(NamedTuple):
    topk_idx: torch.Tensor  # [T, K] int32, descending probability
    topk_w: torch.Tensor  # [T, K] dtype, renormalised
    chunk_hist: torch.Tensor  # [ceil(T / 32), E] int32


class PermuteResult(NamedTuple):
    expert_offsets: torch.Tensor  # [E + 1] int32
    sorted_token: torch.Tensor  # [T*K] int32
    sorted_w: torch.Tensor  # [T*K] dtype
    token_pos: torch.Tensor  # [T, K] int32
    x_perm: torch.Tensor | None  # [T*K, D] dtype (None: rows not copied)
    tiles: torch.Tensor  # tile list, int32
    block_m: int


def _kernel(name: str):
    if not _available.get(name, False):
        raise RuntimeError(f"MoE HIP kernel '{name}' unavailable: {loader.load_error()}")
    return getattr(_modules[name], name)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {loader.last_error()}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    """The current stream of t's device as a raw handle (the same value as
    ``torch.cuda.current_stream(t.device).cuda_stream``, without building the
    Python stream object: ~5 µs of host time per call)."""
    if _raw_stream is not None and t.device.type == "cuda":
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def _dtype_code(t: torch.Tensor, name: str) -> int:
    code = _DTYPE_CODES.get(t.dtype)
    if code is None:
        raise ValueError(f"{name} must be float32 or bfloat16, got {t.dtype}")
    return code


def _require_gpu(t: torch.Tensor, name: str, ndim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a ROCm device, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")


def _require_table(t: torch.Tensor, name: str, n_experts: int, like: torch.Tensor) -> None:
    """A weight argument of the GEMMs is a device array of ``n_experts``
    pointers (``expert_weight_table``); the kernels dereference its entries,
    so a weight tensor passed in its place must stop here."""
    _require_gpu(t, name, 1)
    if t.dtype != torch.int64 or t.numel() != n_experts or t.device != like.device:
        raise ValueError(f"{name} must be an int64 pointer table of {n_experts} entries on {like.device} "
                         f"(expert_weight_table), got {t.dtype} shape {tuple(t.shape)} on {t.device}")


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _tag_tiles(tiles: torch.Tensor, block_m: int) -> torch.Tensor:
    """Record the row-tile height a tile list was built for. The list's own
    header holds it on the device, where the host cannot read it without a
    synchronisation; the GEMM wrappers compare this tag with their
    ``block_m``."""
    tiles._astrai_block_m = block_m
    return tiles


def _check_tiles(tiles: torch.Tensor, block_m: int, like: torch.Tensor, who: str) -> None:
    """A tile list must be a device int32 list built for this ``block_m``: a
    list of 256-row tiles run with 64-row tiles would compute only the first 64
    rows of each tile and leave the rest of the output unwritten."""
    _require_gpu(tiles, f"{who}: tiles", 1)
    if tiles.dtype != torch.int32 or tiles.device != like.device or tiles.numel() < TILE_HEADER:
        raise ValueError(f"{who}: tiles must be an int32 tile list on {like.device} "
                         f"(got {tiles.dtype}, {tiles.numel()} entries on {tiles.device})")
    built = getattr(tiles, "_astrai_block_m", None)
    if built is not None and built != block_m:
        raise ValueError(f"{who}: the tile list was built for block_m {built}, called with block_m {block_m}")


def select_block_m(n_tokens: int, n_experts: int, top_k: int, dim: int, dim_ffn: int, dtype: torch.dtype) -> int:
    """Rows per GEMM tile the kernels use for this problem (host policy)."""
    code = _DTYPE_CODES.get(dtype)
    if code is None:
        raise ValueError(f"unsupported dtype {dtype}")
    bm = loader.library().astrai_moe_select_block_m(n_tokens, n_experts, top_k, dim, dim_ffn, code)
    _check(0 if bm > 0 else bm, "select_block_m")
    return bm


def tile_list_len(n_tokens: int, n_experts: int, top_k: int, block_m: int) -> int:
    n = loader.library().astrai_moe_tile_list_len(n_tokens, n_experts, top_k, block_m)
    if n < 0:
        raise ValueError("tile_list_len: bad sizes")
    return n


def expert_weight_table(weights: Sequence[torch.Tensor], shape: tuple[int, int]) -> torch.Tensor:
    """Device array of the experts' weight pointers (int64), for the GEMMs.

    Every weight must be a contiguous ``[out, in] == shape`` tensor on one
    device with one dtype, starting on a 16-byte boundary when its rows are a
    multiple of 16 bytes; the kernels read them in place, and the table keeps
    references to them.
    """
    if len(weights) == 0:
        raise ValueError("no expert weights")
    dev, dt = weights[0].device, weights[0].dtype
    for i, w in enumerate(weights):
        _require_gpu(w, f"expert weight {i}", 2)
        if tuple(w.shape) != tuple(shape):
            raise ValueError(f"expert weight {i} has shape {tuple(w.shape)}, expected {tuple(shape)}")
        if w.device != dev or w.dtype != dt:
            raise ValueError("expert weights must share one device and dtype")
        # rows of a multiple of 16 bytes are read with 16-byte vector loads
        if (w.shape[1] * w.element_size()) % 16 == 0 and w.data_ptr() % 16 != 0:
            raise ValueError(f"expert weight {i} must start on a 16-byte boundary (its rows are read 16 bytes at a time)")
    table = torch.tensor([w.data_ptr() for w in weights], dtype=torch.int64).to(dev)
    # the table holds raw addresses: it keeps the weights alive, so that a
    # table outliving the caller's list never points at freed memory
    table._astrai_weights = tuple(weights)
    return table


def moe_route(logits: torch.Tensor, top_k: int) -> RouteResult:
    """Softmax, top-k and renormalisation of router logits (mlp.py:84-87)."""
    fn = _kernel("moe_route")
    _require_gpu(logits, "logits", 2)
    code = _dtype_code(logits, "logits")
    n_tokens, n_experts = logits.shape
    if not 1 <= n_experts <= MAX_EXPERTS:
        raise ValueError(f"n_experts must be in [1, {MAX_EXPERTS}], got {n_experts}")
    if not 1 <= top_k <= min(n_experts, MAX_TOPK):
        raise ValueError(f"top_k must be in [1, min(n_experts, {MAX_TOPK})], got {top_k}")
    dev = logits.device
    topk_idx = torch.empty(n_tokens, top_k, dtype=torch.int32, device=dev)
    topk_w = torch.empty(n_tokens, top_k, dtype=logits.dtype, device=dev)
    chunk_hist = torch.empty(-(-n_tokens // CHUNK_TOKENS), n_experts, dtype=torch.int32, device=dev)
    _check(
        fn(logits.data_ptr(), code, n_tokens, n_experts, top_k, topk_idx.data_ptr(), topk_w.data_ptr(),
           chunk_hist.data_ptr(), _stream(logits)),
        "moe_route",
    )
    return RouteResult(topk_idx, topk_w, chunk_hist)


def moe_permute(route: RouteResult, x: torch.Tensor, n_experts: int, block_m: int,
                copy_rows: bool = True) -> PermuteResult:
    """Expert-major, token-ascending permutation of the routed rows
    (mlp.py:90-95) plus the device-built GEMM tile list. ``copy_rows=False``
    writes the index outputs only (``x_perm`` is None), for
    ``moe_gemm_gate_up_gather``."""
    fn = _kernel("moe_permute")
    _require_gpu(x, "x", 2)
    code = _dtype_code(x, "x")
    topk_idx, topk_w, chunk_hist = route
    n_tokens, dim = x.shape
    if topk_idx.shape[0] != n_tokens or topk_w.shape != topk_idx.shape:
        raise ValueError("routing tensors do not match x")
    if topk_w.dtype != x.dtype:
        raise ValueError("topk_w must have x's dtype")
    top_k = topk_idx.shape[1]
    dev = x.device
    rows = n_tokens * top_k
    tl = tile_list_len(n_tokens, n_experts, top_k, block_m)
    offsets = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    sorted_token = torch.empty(rows, dtype=torch.int32, device=dev)
    sorted_w = torch.empty(rows, dtype=x.dtype, device=dev)
    token_pos = torch.empty(n_tokens, top_k, dtype=torch.int32, device=dev)
    x_perm = torch.empty(rows, dim, dtype=x.dtype, device=dev) if copy_rows else None
    tiles = torch.empty(tl, dtype=torch.int32, device=dev)
    chunk_base = torch.empty_like(chunk_hist)
    _check(
        fn(topk_idx.data_ptr(), topk_w.data_ptr(), chunk_hist.data_ptr(), x.data_ptr(), code, n_tokens, n_experts,
           top_k, dim, block_m, offsets.data_ptr(), sorted_token.data_ptr(), sorted_w.data_ptr(),
           token_pos.data_ptr(), _ptr(x_perm), tiles.data_ptr(), tl, chunk_base.data_ptr(), _stream(x)),
        "moe_permute",
    )
    return PermuteResult(offsets, sorted_token, sorted_w, token_pos, x_perm, _tag_tiles(tiles, block_m), block_m)


def _workspace(a: torch.Tensor, dim: int, dim_ffn: int, block_m: int, down: bool,
               balance: bool = True) -> tuple[torch.Tensor | None, int]:
    """Scratch of the 256-row matrix-core GEMMs (``astrai_moe_gemm_gate_up``,
    ``astrai_moe_gemm_down``): the run-time claims of the last tenth of the
    work and, for the down GEMMs, the partial sums of the split last round.
    Allocated only where that kernel runs: (tensor or None, bytes).
    ``balance=False``: none, every tile dealt in advance and run whole."""
    if not balance or block_m != 256 or a.dtype != torch.bfloat16 or not matrix_core_supported(dim, dim_ffn, a.dtype):
        return None, 0
    # the partial sums serve only tiles of SPLIT_MIN_STEPS K steps or more
    # (K = dim_ffn for the down-sized users): below that, the scheduling part
    split = down and dim_ffn // 64 >= SPLIT_MIN_STEPS
    nbytes = int(loader.library().astrai_moe_gemm_workspace_bytes(1 if split else 0))
    return torch.empty(nbytes, dtype=torch.uint8, device=a.device), nbytes


def moe_gemm_gate_up(x_perm: torch.Tensor, tiles: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                     n_experts: int, dim_ffn: int, block_m: int, packed: bool = False,
                     balance: bool = True) -> torch.Tensor:
    """h = up(x) * silu(gate(x)) over every expert's rows (mlp.py:22-23).

    ``packed``: ``w_gate`` is a table of packed gate/up copies
    (``moe_pack_gate_up``) and ``w_up`` is ignored; same results.
    ``balance``: the 256-row kernel may hand out the last tenth of its tiles
    at run time (same results; False deals every tile in advance)."""
    fn = _kernel("moe_gemm_gate_up")
    _require_gpu(x_perm, "x_perm", 2)
    code = _dtype_code(x_perm, "x_perm")
    n_rows, dim = x_perm.shape
    _check_tiles(tiles, block_m, x_perm, "moe_gemm_gate_up")
    _require_table(w_gate, "w_gate", n_experts, x_perm)
    if not packed:
        _require_table(w_up, "w_up", n_experts, x_perm)
    h = torch.empty(n_rows, dim_ffn, dtype=x_perm.dtype, device=x_perm.device)
    ws, ws_bytes = _workspace(x_perm, dim, dim_ffn, block_m, down=False, balance=balance)
    if packed:
        _check(
            loader.library().astrai_moe_gemm_gate_up_packed(
                x_perm.data_ptr(), tiles.data_ptr(), tiles.numel(), w_gate.data_ptr(), code, n_rows, n_experts, dim,
                dim_ffn, block_m, h.data_ptr(), _ptr(ws), ws_bytes, _stream(x_perm)),
            "moe_gemm_gate_up_packed",
        )
        return h
    _check(
        fn(x_perm.data_ptr(), tiles.data_ptr(), tiles.numel(), w_gate.data_ptr(), w_up.data_ptr(), code, n_rows,
           n_experts, dim, dim_ffn, block_m, h.data_ptr(), _ptr(ws), ws_bytes, _stream(x_perm)),
        "moe_gemm_gate_up",
    )
    return h


def _out_buffer(out: torch.Tensor | None, rows: int, cols: int, like: torch.Tensor) -> torch.Tensor:
    if out is None:
        return torch.empty(rows, cols, dtype=like.dtype, device=like.device)
    _require_gpu(out, "out", 2)
    if tuple(out.shape) != (rows, cols) or out.dtype != like.dtype or out.device != like.device:
        raise ValueError(f"out must be [{rows}, {cols}] {like.dtype} on {like.device}")
    return out


def matrix_core_supported(dim: int, dim_ffn: int, dtype: torch.dtype) -> bool:
    """Whether the bf16 forward GEMMs of this expert shape run on the matrix
    cores (dim and dim_ffn multiples of 64; the last column tile may be
    partial)."""
    return (dtype == torch.bfloat16 and dim % 64 == 0 and dim_ffn % 64 == 0 and 0 < dim <= 1 << 22
            and 0 < dim_ffn <= 1 << 22)


def gather_supported(n_tokens: int, dim: int, dim_ffn: int, dtype: torch.dtype) -> bool:
    """Whether ``moe_gemm_gate_up_gather`` takes this problem (bf16, the
    matrix-core shapes, x under 4 GiB)."""
    return matrix_core_supported(dim, dim_ffn, dtype) and n_tokens * dim * 2 < 1 << 32


def moe_gemm_gate_up_gather(x: torch.Tensor, sorted_token: torch.Tensor, tiles: torch.Tensor, w_gate: torch.Tensor,
                            w_up: torch.Tensor, n_experts: int, dim_ffn: int, block_m: int,
                            balance: bool = True) -> torch.Tensor:
    """``moe_gemm_gate_up`` on the permuted rows ``x[sorted_token]`` read
    straight from ``x`` (no copied ``x_perm``); bit-identical results."""
    _require_gpu(x, "x", 2)
    code = _dtype_code(x, "x")
    n_tokens, dim = x.shape
    n_rows = sorted_token.numel()
    _check_tiles(tiles, block_m, x, "moe_gemm_gate_up_gather")
    _require_table(w_gate, "w_gate", n_experts, x)
    _require_table(w_up, "w_up", n_experts, x)
    h = torch.empty(n_rows, dim_ffn, dtype=x.dtype, device=x.device)
    ws, ws_bytes = _workspace(x, dim, dim_ffn, block_m, down=False, balance=balance)
    _check(
        loader.library().astrai_moe_gemm_gate_up_gather(
            x.data_ptr(), sorted_token.data_ptr(), n_tokens, tiles.data_ptr(), tiles.numel(), w_gate.data_ptr(),
            w_up.data_ptr(), code, n_rows, n_experts, dim, dim_ffn, block_m, h.data_ptr(), _ptr(ws), ws_bytes,
            _stream(x)),
        "moe_gemm_gate_up_gather",
    )
    return h


def moe_gemm_down(h: torch.Tensor, tiles: torch.Tensor, w_down: torch.Tensor, sorted_w: torch.Tensor | None,
                  n_experts: int, dim: int, block_m: int, out: torch.Tensor | None = None,
                  packed: bool = False, balance: bool = True) -> torch.Tensor:
    """y = down(h) * routing weight over every expert's rows (mlp.py:24, :97).

    ``sorted_w`` None: no routing weight (a dense expert, mlp.py:24 alone).
    ``packed``: ``w_down`` is a table of packed copies (``moe_pack_down``).
    ``balance``: the 256-row kernel may hand out the last tenth of its tiles
    at run time and split the tiles left after its last whole round of compute
    units along K (``astrai_moe_gemm_down``); False deals every tile in
    advance and keeps each tile's single K order, whose bits do not depend on
    the device's compute-unit count."""
    fn = _kernel("moe_gemm_down")
    _require_gpu(h, "h", 2)
    code = _dtype_code(h, "h")
    n_rows, dim_ffn = h.shape
    if sorted_w is not None:
        _require_gpu(sorted_w, "sorted_w")
        if sorted_w.numel() != n_rows or sorted_w.dtype != h.dtype or sorted_w.device != h.device:
            raise ValueError("sorted_w must hold one weight of h's dtype per row")
    _check_tiles(tiles, block_m, h, "moe_gemm_down")
    _require_table(w_down, "w_down", n_experts, h)
    y = _out_buffer(out, n_rows, dim, h)
    ws, ws_bytes = _workspace(h, dim, dim_ffn, block_m, down=True, balance=balance)
    if packed:
        _check(
            loader.library().astrai_moe_gemm_down_packed(
                h.data_ptr(), tiles.data_ptr(), tiles.numel(), w_down.data_ptr(), _ptr(sorted_w), code, n_rows,
                n_experts, dim_ffn, dim, block_m, y.data_ptr(), _ptr(ws), ws_bytes, _stream(h)),
            "moe_gemm_down_packed",
        )
        return y
    _check(
        fn(h.data_ptr(), tiles.data_ptr(), tiles.numel(), w_down.data_ptr(), _ptr(sorted_w), code, n_rows,
           n_experts, dim_ffn, dim, block_m, y.data_ptr(), _ptr(ws), ws_bytes, _stream(h)),
        "moe_gemm_down",
    )
    return y


def f32_matrix_cores(dim: int, dim_ffn: int, block_m: int, dtype: torch.dtype) -> bool:
    """Whether both fp32 GEMMs of this shape run on the matrix cores
    (``gemm_f32_mfma_kernel``: 64-row tiles, dim and dim_ffn multiples of 32,
    dim a multiple of 64 for the down GEMM's column tiles)."""
    return (dtype == torch.float32 and block_m == 64 and dim % 64 == 0 and dim_ffn % 32 == 0
            and 0 < dim <= 1 << 22 and 0 < dim_ffn <= 1 << 22)


def packed_supported(dim: int, dim_ffn: int, dtype: torch.dtype) -> bool:
    """Whether the packed-weight GEMMs take this expert shape (bf16, dim a
    multiple of 256, dim_ffn a multiple of 128: whole column tiles)."""
    return (dtype == torch.bfloat16 and dim % 256 == 0 and dim_ffn % 128 == 0 and 0 < dim <= 1 << 22
            and 0 < dim_ffn <= 1 << 22)


def moe_pack_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """One expert's gate and up weights ([dim_ffn, dim] each) as one packed
    copy for the packed GEMMs: ``[2 * dim_ffn, dim]`` bf16 in staged order."""
    _require_gpu(w_gate, "w_gate", 2)
    _require_gpu(w_up, "w_up", 2)
    if w_gate.shape != w_up.shape or w_gate.dtype != w_up.dtype or w_gate.device != w_up.device:
        raise ValueError("w_gate and w_up must match in shape, dtype and device")
    code = _dtype_code(w_gate, "w_gate")
    dim_ffn, dim = w_gate.shape
    out = torch.empty(2 * dim_ffn, dim, dtype=w_gate.dtype, device=w_gate.device)
    _check(loader.library().astrai_moe_pack_gate_up(w_gate.data_ptr(), w_up.data_ptr(), code, dim_ffn, dim,
                                                    out.data_ptr(), _stream(w_gate)), "moe_pack_gate_up")
    return out


def moe_pack_down(w_down: torch.Tensor) -> torch.Tensor:
    """One expert's down weight ([dim, dim_ffn]) as a packed copy (same size)."""
    _require_gpu(w_down, "w_down", 2)
    code = _dtype_code(w_down, "w_down")
    dim, dim_ffn = w_down.shape
    out = torch.empty(dim, dim_ffn, dtype=w_down.dtype, device=w_down.device)
    _check(loader.library().astrai_moe_pack_down(w_down.data_ptr(), code, dim, dim_ffn, out.data_ptr(),
                                                 _stream(w_down)), "moe_pack_down")
    return out


def moe_combine(y: torch.Tensor, token_pos: torch.Tensor, shared: torch.Tensor | None = None,
                row_w: torch.Tensor | None = None) -> torch.Tensor:
    """out = mean(shared experts) + sum over experts (ascending) of y rows
    (mlp.py:89, :98, :77, :71). ``row_w`` (the permuted rows' routing
    weights, ``sorted_w``): y holds unweighted rows, each scaled by its
    weight and rounded before the sum (the same result as combining the
    weighted down GEMM's rows)."""
    fn = _kernel("moe_combine")
    _require_gpu(y, "y", 2)
    code = _dtype_code(y, "y")
    _require_gpu(token_pos, "token_pos", 2)
    n_tokens, top_k = token_pos.shape
    dim = y.shape[1]
    if y.shape[0] != n_tokens * top_k:
        raise ValueError("y must hold n_tokens * top_k rows")
    n_shared = 0
    if shared is not None:
        _require_gpu(shared, "shared", 3)
        if shared.shape[1:] != (n_tokens, dim) or shared.dtype != y.dtype:
            raise ValueError("shared must be [n_shared, n_tokens, dim] of y's dtype")
        n_shared = shared.shape[0]
    if row_w is not None:
        _require_gpu(row_w, "row_w", 1)
        if row_w.shape[0] != n_tokens * top_k or row_w.dtype != y.dtype:
            raise ValueError("row_w must hold n_tokens * top_k weights of y's dtype")
    out = torch.empty(n_tokens, dim, dtype=y.dtype, device=y.device)
    _check(
        fn(y.data_ptr(), token_pos.data_ptr(), _ptr(row_w), _ptr(shared), n_shared, code, n_tokens, top_k, dim,
           out.data_ptr(), _stream(y)),
        "moe_combine",
    )
    return out


def dense_tiles(n_tokens: int, block_m: int, device: torch.device,
                with_offsets: bool = False) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """Tile list of one dense expert over ``n_tokens`` rows (the shared experts
    and ``MLP``, mlp.py:22-25, on the grouped GEMMs), written on the device by
    ``astrai_moe_dense_tiles``: a fresh allocation from torch's caching
    allocator on every call, so a captured graph owns its list and no later
    call can free or rewrite it. ``with_offsets`` also returns the expert
    offsets ``{0, n_tokens}`` (int32[2]) the weight-gradient GEMM takes."""
    tl = tile_list_len(n_tokens, 1, 1, block_m)
    tiles = torch.empty(tl, dtype=torch.int32, device=device)
    offsets = torch.empty(2, dtype=torch.int32, device=device) if with_offsets else None
    _check(loader.library().astrai_moe_dense_tiles(n_tokens, block_m, tiles.data_ptr(), tl, _ptr(offsets),
                                                   torch.cuda.current_stream(device).cuda_stream), "moe_dense_tiles")
    _tag_tiles(tiles, block_m)
    return (tiles, offsets) if with_offsets else tiles


def moe_dense_mlp(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
                  dim_ffn: int, out: torch.Tensor | None = None, tiles: torch.Tensor | None = None) -> torch.Tensor:
    """One expert ``down(up(x) * silu(gate(x)))`` over all rows of x (mlp.py:22-25),
    on the grouped-GEMM kernels with one-entry weight tables. ``tiles``: a list
    from ``dense_tiles`` for these rows at ``dense_block_m``'s height (built here
    when None), so several experts over the same rows can share one."""
    n_tokens, dim = x.shape
    block_m = dense_block_m(n_tokens, dim, dim_ffn, x.dtype)
    if tiles is None:
        tiles = dense_tiles(n_tokens, block_m, x.device)
    h = moe_gemm_gate_up(x, tiles, w_gate, w_up, 1, dim_ffn, block_m)
    return moe_gemm_down(h, tiles, w_down, None, 1, dim, block_m, out=out)


def dense_block_m(n_tokens: int, dim: int, dim_ffn: int, dtype: torch.dtype) -> int:
    """Row-tile height of one dense expert over ``n_tokens`` rows."""
    return select_block_m(n_tokens, 1, 1, dim, dim_ffn, dtype)


def moe_routed_forward(x: torch.Tensor, logits: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                       w_down: torch.Tensor, dim_ffn: int, top_k: int,
                       shared: torch.Tensor | None = None, packed: bool = False) -> torch.Tensor:
    """Routed experts plus combine (mlp.py:84-100 and :71) for ``x [T, D]``
    given the router logits and the experts' weight-pointer tables (of packed
    copies with ``packed``; ``w_up`` is then ignored)."""
    n_tokens, dim = x.shape
    n_experts = logits.shape[1]
    if n_tokens == 0:
        return torch.empty(0, dim, dtype=x.dtype, device=x.device)
    block_m = select_block_m(n_tokens, n_experts, top_k, dim, dim_ffn, x.dtype)
    route = moe_route(logits, top_k)
    if not packed and gather_supported(n_tokens, dim, dim_ffn, x.dtype):
        # the gate/up GEMM reads the token rows itself: no copied x_perm
        perm = moe_permute(route, x, n_experts, block_m, copy_rows=False)
        h = moe_gemm_gate_up_gather(x, perm.sorted_token, perm.tiles, w_gate, w_up, n_experts, dim_ffn, block_m)
    else:
        perm = moe_permute(route, x, n_experts, block_m)
        h = moe_gemm_gate_up(perm.x_perm, perm.tiles, w_gate, w_up, n_experts, dim_ffn, block_m, packed=packed)
    y = moe_gemm_down(h, perm.tiles, w_down, perm.sorted_w, n_experts, dim, block_m, packed=packed)
    return moe_combine(y, perm.token_pos, shared)


# -- training: forward that keeps g, u, y and the backward kernels ------------


def backward_on_matrix_cores(dim: int, dim_ffn: int, dtype: torch.dtype) -> bool:
    """Whether training runs the matrix-core kernels for this expert shape
    (bf16, dim and dim_ffn multiples of 64; 256-row tile lists). Every other
    shape and fp32 runs the general-shape kernels."""
    return matrix_core_supported(dim, dim_ffn, dtype)


TRAIN_BLOCK_M = 256  # row-tile height of the matrix-core training kernels


def train_block_m(dim: int, dim_ffn: int, dtype: torch.dtype) -> int:
    """Row-tile height of the training forward and backward for this shape."""
    return TRAIN_BLOCK_M if backward_on_matrix_cores(dim, dim_ffn, dtype) else 64


def _lib_call(name: str, *args) -> None:
    _check(getattr(loader.library(), name)(*args), name)


def moe_gemm_gate_up_train(x_perm: torch.Tensor, tiles: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor,
                           n_experts: int, dim_ffn: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``h`` as ``moe_gemm_gate_up`` plus ``gu [rows, 2 * dim_ffn]``, the
    rounded gate and up projections the backward needs, in blocks of 4 columns
    (``gu_split`` separates them); tile list at ``train_block_m``'s height."""
    _require_gpu(x_perm, "x_perm", 2)
    code = _dtype_code(x_perm, "x_perm")
    n_rows, dim = x_perm.shape
    bm = train_block_m(dim, dim_ffn, x_perm.dtype)
    _check_tiles(tiles, bm, x_perm, "moe_gemm_gate_up_train")
    _require_table(w_gate, "w_gate", n_experts, x_perm)
    _require_table(w_up, "w_up", n_experts, x_perm)
    h = torch.empty(n_rows, dim_ffn, dtype=x_perm.dtype, device=x_perm.device)
    gu = torch.empty(n_rows, 2 * dim_ffn, dtype=x_perm.dtype, device=x_perm.device)
    ws, ws_bytes = _workspace(x_perm, dim, dim_ffn, bm, down=False)
    _lib_call("astrai_moe_gemm_gate_up_train", x_perm.data_ptr(), tiles.data_ptr(), tiles.numel(), w_gate.data_ptr(),
              w_up.data_ptr(), code, n_rows, n_experts, dim, dim_ffn, bm, h.data_ptr(), gu.data_ptr(), _ptr(ws),
              ws_bytes, _stream(x_perm))
    return h, gu


def gu_split(gu: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``(g, u)`` of the saved projections of ``moe_gemm_gate_up_train``:
    columns in blocks of 4, each block's gate values then the same columns' up
    values, the last block holding the ``dim_ffn % 4`` columns left."""
    rows, two_f = gu.shape
    f = two_f // 2
    q = f // 4
    head = gu[:, :8 * q].reshape(rows, q, 2, 4)
    g, u = head[:, :, 0, :].reshape(rows, 4 * q), head[:, :, 1, :].reshape(rows, 4 * q)
    w = f - 4 * q
    if w:
        tail = gu[:, 8 * q:]
        g, u = torch.cat([g, tail[:, :w]], 1), torch.cat([u, tail[:, w:]], 1)
    return g, u


def moe_gemm_down_train(h: torch.Tensor, tiles: torch.Tensor, w_down: torch.Tensor, sorted_w: torch.Tensor,
                        n_experts: int, dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``y * w`` as ``moe_gemm_down`` plus the unweighted expert output."""
    _require_gpu(h, "h", 2)
    code = _dtype_code(h, "h")
    n_rows, dim_ffn = h.shape
    if sorted_w.numel() != n_rows or sorted_w.dtype != h.dtype:
        raise ValueError("sorted_w must hold one weight of h's dtype per row")
    bm = train_block_m(dim, dim_ffn, h.dtype)
    _check_tiles(tiles, bm, h, "moe_gemm_down_train")
    _require_table(w_down, "w_down", n_experts, h)
    y, y_unw = (torch.empty(n_rows, dim, dtype=h.dtype, device=h.device) for _ in range(2))
    ws, ws_bytes = _workspace(h, dim, dim_ffn, bm, down=True)
    _lib_call("astrai_moe_gemm_down_train", h.data_ptr(), tiles.data_ptr(), tiles.numel(), w_down.data_ptr(),
              sorted_w.data_ptr(), code, n_rows, n_experts, dim_ffn, dim, bm, y.data_ptr(),
              y_unw.data_ptr(), _ptr(ws), ws_bytes, _stream(h))
    return y, y_unw


def moe_row_grad(dout: torch.Tensor, sorted_token: torch.Tensor, sorted_w: torch.Tensor,
                 y_unweighted: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per permuted row: ``dy = dout[token] * w`` and ``dw = sum(dout[token] * y)``
    (the two factors of mlp.py:97's ``expert_output * weights``)."""
    _require_gpu(dout, "dout", 2)
    _require_gpu(y_unweighted, "y_unweighted", 2)
    code = _dtype_code(dout, "dout")
    n_rows, dim = y_unweighted.shape
    dy = torch.empty(n_rows, dim, dtype=dout.dtype, device=dout.device)
    dw = torch.empty(n_rows, dtype=dout.dtype, device=dout.device)
    _lib_call("astrai_moe_row_grad", dout.data_ptr(), sorted_token.data_ptr(), sorted_w.data_ptr(),
              y_unweighted.data_ptr(), code, n_rows, dim, dy.data_ptr(), dw.data_ptr(), _stream(dout))
    return dy, dw


def moe_gemm_dgrad_down(dy: torch.Tensor, tiles: torch.Tensor, w_down: torch.Tensor, gu: torch.Tensor,
                        n_experts: int) -> tuple[torch.Tensor, torch.Tensor]:
    """``dh = dy . W_down`` with the SwiGLU backward fused (``gu`` from
    ``moe_gemm_gate_up_train``): returns ``(dg, du)``."""
    _require_gpu(dy, "dy", 2)
    _require_gpu(gu, "gu", 2)
    code = _dtype_code(dy, "dy")
    n_rows, dim = dy.shape
    dim_ffn = gu.shape[1] // 2
    bm = train_block_m(dim, dim_ffn, dy.dtype)
    _check_tiles(tiles, bm, dy, "moe_gemm_dgrad_down")
    _require_table(w_down, "w_down", n_experts, dy)
    dg, du = (torch.empty(n_rows, dim_ffn, dtype=dy.dtype, device=dy.device) for _ in range(2))
    _lib_call("astrai_moe_gemm_dgrad_down", dy.data_ptr(), tiles.data_ptr(), tiles.numel(), w_down.data_ptr(),
              gu.data_ptr(), code, n_rows, n_experts, dim, dim_ffn, bm, dg.data_ptr(), du.data_ptr(),
              _stream(dy))
    return dg, du


def moe_gemm_dgrad_gate_up(dg: torch.Tensor, du: torch.Tensor, tiles: torch.Tensor, w_gate: torch.Tensor,
                           w_up: torch.Tensor, n_experts: int, dim: int, balance: bool = True) -> torch.Tensor:
    """``dx_perm = dg . W_gate + du . W_up`` per expert. ``balance``: a
    partial last round of long 256-row tiles is split along K (False: every
    tile runs whole)."""
    _require_gpu(dg, "dg", 2)
    code = _dtype_code(dg, "dg")
    n_rows, dim_ffn = dg.shape
    bm = train_block_m(dim, dim_ffn, dg.dtype)
    _check_tiles(tiles, bm, dg, "moe_gemm_dgrad_gate_up")
    _require_table(w_gate, "w_gate", n_experts, dg)
    _require_table(w_up, "w_up", n_experts, dg)
    dx = torch.empty(n_rows, dim, dtype=dg.dtype, device=dg.device)
    ws, ws_bytes = _workspace(dg, dim, dim_ffn, bm, down=True, balance=balance)
    _lib_call("astrai_moe_gemm_dgrad_gate_up", dg.data_ptr(), du.data_ptr(), tiles.data_ptr(), tiles.numel(),
              w_gate.data_ptr(), w_up.data_ptr(), code, n_rows, n_experts, dim_ffn, dim, bm,
              dx.data_ptr(), _ptr(ws), ws_bytes, _stream(dg))
    return dx


def moe_gemm_wgrad(a: torch.Tensor, b: torch.Tensor, expert_offsets: torch.Tensor, n_experts: int) -> torch.Tensor:
    """``dw[e] = a[rows of e]^T . b[rows of e]`` as one ``[E, m, n]`` tensor;
    experts without rows are left unwritten."""
    _require_gpu(a, "a", 2)
    _require_gpu(b, "b", 2)
    code = _dtype_code(a, "a")
    if a.shape[0] != b.shape[0]:
        raise ValueError("a and b must have the same rows")
    n_rows, m = a.shape
    n = b.shape[1]
    dw = torch.empty(n_experts, m, n, dtype=a.dtype, device=a.device)
    _lib_call("astrai_moe_gemm_wgrad", a.data_ptr(), b.data_ptr(), expert_offsets.data_ptr(), code, n_rows,
              n_experts, m, n, dw.data_ptr(), _stream(a))
    return dw
