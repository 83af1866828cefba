"""Discovery and loading of the compiled MoE kernels.

Same contract as the reference's ``astrai/extension/loader.py:14-36``:
``KERNEL_NAMES`` lists the kernels, availability is decided once at import
(``_available``), each available kernel has a module-like handle in
``_modules`` exposing a function of the kernel's name, and ``is_available`` /
``get_module`` query them.

Difference in mechanism: the reference builds one torch extension module per
kernel; here all kernels live in one C-ABI library, ``libastrai_moe.so``
(declared in ``include/astrai_moe.h``), bound with ctypes. The library is
loaded after ``import torch`` and linked against torch's bundled HIP runtime,
so the process keeps exactly one HIP runtime (checked below) and torch's
streams and device pointers are valid in the kernels.

A kernel is unavailable when the library is missing, fails to load, has a
different ABI version or lacks the kernel's symbol; ``load_error()`` says why.
Unlike the reference there is no torch fallback behind an unavailable kernel:
the ops raise.
"""

from __future__ import annotations

import ctypes
import os
import types
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime before the library)

KERNEL_NAMES = ["moe_route", "moe_permute", "moe_gemm_gate_up", "moe_gemm_down", "moe_combine"]

ABI_VERSION = 10
LIB_PATH = Path(os.environ.get("ASTRAI_MOE_LIB", Path(__file__).resolve().parent / "libastrai_moe.so"))

_c_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int

# Entry point -> argument types (mirrors include/astrai_moe.h).
_SIGNATURES: dict[str, tuple] = {
    "astrai_moe_abi_version": (_int, []),
    "astrai_moe_last_error": (ctypes.c_char_p, []),
    "astrai_moe_select_block_m": (_int, [_i64, _int, _int, _i64, _i64, _int]),
    "astrai_moe_tile_list_len": (_i64, [_i64, _int, _int, _int]),
    "astrai_moe_dense_tiles": (_int, [_i64, _int, _vp, _i64, _vp, _vp]),
    "astrai_moe_route": (_int, [_vp, _int, _i64, _int, _int, _vp, _vp, _vp, _vp]),
    "astrai_moe_permute": (
        _int,
        [_vp, _vp, _vp, _vp, _int, _i64, _int, _int, _i64, _int, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp],
    ),
    "astrai_moe_permute_noalloc": (
        _int,
        [_vp, _vp, _vp, _vp, _int, _i64, _int, _int, _i64, _int, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp],
    ),
    "astrai_moe_gemm_gate_up": (_int, [_vp, _vp, _i64, _vp, _vp, _int, _i64, _int, _i64, _i64, _int, _vp, _vp, _i64,
                                       _vp]),
    "astrai_moe_gemm_down": (_int, [_vp, _vp, _i64, _vp, _vp, _int, _i64, _int, _i64, _i64, _int, _vp, _vp, _i64,
                                    _vp]),
    "astrai_moe_gemm_workspace_bytes": (_i64, [_int]),
    "astrai_moe_combine": (_int, [_vp, _vp, _vp, _vp, _int, _int, _i64, _int, _i64, _vp, _vp]),
    "astrai_moe_gemm_gate_up_gather": (_int, [_vp, _vp, _i64, _vp, _i64, _vp, _vp, _int, _i64, _int, _i64, _i64, _int,
                                              _vp, _vp, _i64, _vp]),
    "astrai_moe_pack_gate_up": (_int, [_vp, _vp, _int, _i64, _i64, _vp, _vp]),
    "astrai_moe_pack_down": (_int, [_vp, _int, _i64, _i64, _vp, _vp]),
    "astrai_moe_gemm_gate_up_packed": (_int, [_vp, _vp, _i64, _vp, _int, _i64, _int, _i64, _i64, _int, _vp, _vp, _i64,
                                              _vp]),
    "astrai_moe_gemm_down_packed": (_int, [_vp, _vp, _i64, _vp, _vp, _int, _i64, _int, _i64, _i64, _int, _vp, _vp,
                                           _i64, _vp]),
    "astrai_moe_gemm_gate_up_train": (_int, [_vp, _vp, _i64, _vp, _vp, _int, _i64, _int, _i64, _i64, _int, _vp, _vp,
                                             _vp, _i64, _vp]),
    "astrai_moe_gemm_down_train": (_int, [_vp, _vp, _i64, _vp, _vp, _int, _i64, _int, _i64, _i64, _int, _vp, _vp,
                                          _vp, _i64, _vp]),
    "astrai_moe_row_grad": (_int, [_vp, _vp, _vp, _vp, _int, _i64, _i64, _vp, _vp, _vp]),
    "astrai_moe_gemm_dgrad_down": (_int, [_vp, _vp, _i64, _vp, _vp, _int, _i64, _int, _i64, _i64, _int, _vp, _vp,
                                          _vp]),
    "astrai_moe_gemm_dgrad_gate_up": (_int, [_vp, _vp, _vp, _i64, _vp, _vp, _int, _i64, _int, _i64, _i64, _int, _vp,
                                             _vp, _i64, _vp]),
    "astrai_moe_gemm_wgrad": (_int, [_vp, _vp, _vp, _int, _i64, _int, _i64, _i64, _vp, _vp]),
}

_available: dict[str, bool] = {}
_modules: dict[str, object] = {}
_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def _hip_runtimes_mapped() -> set[str]:
    try:
        with open("/proc/self/maps") as f:
            return {line.split()[-1] for line in f if "libamdhip64" in line and "/" in line}
    except OSError:
        return set()


def _load() -> None:
    global _lib, _load_error
    if not LIB_PATH.exists():
        _load_error = f"{LIB_PATH} not found (build it with `python -m astrai_amd.csrc.build`)"
        return
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        _load_error = f"failed to load {LIB_PATH}: {exc}"
        return
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.astrai_moe_abi_version()
    if version != ABI_VERSION:
        _load_error = f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}"
        return
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        _load_error = f"more than one HIP runtime mapped in the process: {sorted(runtimes)}"
        return
    _lib = lib


_load()
for _name in KERNEL_NAMES:
    _fn = getattr(_lib, f"astrai_{_name}", None) if _lib is not None else None
    _available[_name] = _fn is not None
    _modules[_name] = types.SimpleNamespace(**{_name: _fn}) if _fn is not None else None


def is_available(name: str) -> bool:
    """Return ``True`` if the compiled kernel ``name`` was loaded."""
    return _available.get(name, False)


def get_module(name: str) -> object:
    """Return the loaded kernel handle for ``name``, or ``None`` if unavailable."""
    return _modules.get(name)


def library() -> ctypes.CDLL:
    """The loaded library; raises ``RuntimeError`` if it could not be loaded."""
    if _lib is None:
        raise RuntimeError(f"MoE HIP kernels unavailable: {_load_error}")
    return _lib


def load_error() -> str | None:
    """Why the library is unavailable, or ``None`` if it loaded."""
    return _load_error


def last_error() -> str:
    return library().astrai_moe_last_error().decode(errors="replace")
