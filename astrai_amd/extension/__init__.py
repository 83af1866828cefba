"""MoE expert-forward kernels (HIP, gfx950) behind AstrAI's extension-loading
contract.

Public API:
    - ``moe_route``        router softmax / top-k / renormalisation
    - ``moe_permute``      expert-major token permutation + GEMM tile list
    - ``moe_gemm_gate_up`` grouped gate/up projection with fused SwiGLU
    - ``moe_gemm_down``    grouped down projection with fused routing weight
    - ``moe_combine``      weighted un-permute, shared-expert mean and add
    - ``moe_routed_forward`` the five above in sequence

``is_available(name)`` and ``KERNEL_NAMES`` follow the reference's
``astrai/extension/__init__.py``.
"""

from astrai_amd.extension.loader import KERNEL_NAMES, is_available
from astrai_amd.extension.ops import (
    expert_weight_table,
    moe_combine,
    moe_dense_mlp,
    moe_gemm_down,
    moe_gemm_gate_up,
    moe_permute,
    moe_route,
    moe_routed_forward,
    select_block_m,
)

__all__ = [
    "KERNEL_NAMES",
    "is_available",
    "expert_weight_table",
    "moe_combine",
    "moe_dense_mlp",
    "moe_gemm_down",
    "moe_gemm_gate_up",
    "moe_permute",
    "moe_route",
    "moe_routed_forward",
    "select_block_m",
]
