"""Build registry and builder for the MoE HIP kernels (gfx950).

Mirrors the registry contract of the reference's ``csrc/build.py:34-48``:
``register(name, sources=None, **kwargs)`` records a kernel name with its
sources and flags in ``REGISTRY``. The reference turns each entry into its own
torch extension module; here every registered kernel is compiled by ``hipcc``
for gfx950 into one C-ABI shared library, ``astrai_amd/extension/
libastrai_moe.so``, whose exported ``astrai_<name>`` symbols the loader
binds by name (the signatures are declared in ``include/astrai_moe.h``).

Run ``python -m astrai_amd.csrc.build`` (or ``build()``) to compile.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

_PKG = Path(__file__).resolve().parent.parent
_REPO = _PKG.parent
KERNELS_DIR = _PKG / "csrc" / "kernels"
INCLUDE_DIR = _REPO / "include"
OUT_DIR = _PKG / "extension"
LIB_NAME = "libastrai_moe.so"

ARCH = "gfx950"
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Packed fp32 arithmetic stays off: hipcc would otherwise form v_pk_*_f32
    # from scalar float code. (The host pass warns that it does not know the
    # feature; that is harmless.)
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

REGISTRY: dict[str, dict] = {}


def register(name: str, sources: list[str] | None = None, **kwargs) -> None:
    """Record kernel ``name`` with its HIP sources and extra flags."""
    if sources is None:
        sources = [str(KERNELS_DIR / f"{name}.hip")]
    REGISTRY[name] = {
        "sources": [str(s) for s in sources],
        "hipcc_flags": [*HIPCC_FLAGS, *kwargs.pop("hipcc_flags", [])],
        "extra_link_args": kwargs.pop("extra_link_args", []),
        **kwargs,
    }


register("moe_route")
register("moe_permute")
register("moe_gemm", sources=[str(KERNELS_DIR / "moe_gemm.hip"), str(KERNELS_DIR / "moe_gemm_mfma.hip"),
                              str(KERNELS_DIR / "moe_gemm_mfma_f32.hip"), str(KERNELS_DIR / "moe_gemm_mfma_f32_bwd.hip"),
                              str(KERNELS_DIR / "moe_gemm_bwd.hip"),
                              str(KERNELS_DIR / "moe_gemm_generic_bwd.hip")])
register("moe_combine")
register("capi")

# The kernel names the Python loader binds (entry point astrai_<name>).
KERNEL_NAMES = ["moe_route", "moe_permute", "moe_gemm_gate_up", "moe_gemm_down", "moe_combine"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the MoE kernels need ROCm's hipcc to build")


def _torch_lib_dir() -> str | None:
    """Directory of the HIP runtime torch ships; linking against it keeps one
    HIP runtime in the process."""
    try:
        import torch

        d = Path(torch.__file__).resolve().parent / "lib"
        return str(d) if (d / "libamdhip64.so").exists() else None
    except Exception:
        return None


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every registered source and link ``libastrai_moe.so``."""
    hipcc = _hipcc()
    obj_dir = _PKG / "csrc" / "_build"
    obj_dir.mkdir(parents=True, exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)

    jobs_list = []
    for info in REGISTRY.values():
        for src in info["sources"]:
            obj = obj_dir / (Path(src).stem + ".o")
            cmd = [hipcc, *info["hipcc_flags"], f"-I{INCLUDE_DIR}", f"-I{KERNELS_DIR}", "-c", src, "-o", str(obj)]
            jobs_list.append((src, obj, cmd))

    def run(job):
        src, obj, cmd = job
        if verbose:
            print(" ".join(cmd), flush=True)
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{proc.stderr}")
        return obj

    n = jobs or min(len(jobs_list), os.cpu_count() or 4, 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=n) as ex:
        objs = list(ex.map(run, jobs_list))

    out = OUT_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    tlib = _torch_lib_dir()
    if tlib:
        link += [f"-L{tlib}", f"-Wl,-rpath,{tlib}"]
    for info in REGISTRY.values():
        link += info["extra_link_args"]
    if verbose:
        print(" ".join(link), flush=True)
    proc = subprocess.run(link, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
