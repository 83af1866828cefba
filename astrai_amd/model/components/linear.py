"""Linear layer with the parameter layout of the reference.

Same contract as ``astrai/model/components/linear.py:7-24``: ``weight`` is an
``nn.Parameter`` of shape ``[out_dim, in_dim]`` (allocated, not initialised),
optional zero-initialised ``bias``, ``reset_parameters`` draws
``N(0, init_std)`` weights and ``U(-1/sqrt(fan_in), 1/sqrt(fan_in))`` biases,
and ``forward`` is ``F.linear``. The MoE layer reads the expert weights of
these modules in place (the HIP kernels take their data pointers), and the
router keeps calling ``forward``.
"""

from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor


class Linear(nn.Module):
    def __init__(self, in_dim: int, out_dim: int, bias: bool = False, init_std: float = 0.02):
        super().__init__()
        self.weight = nn.Parameter(torch.empty((out_dim, in_dim)))
        self.bias = nn.Parameter(torch.zeros(out_dim)) if bias else None
        self.init_std = init_std

    def reset_parameters(self) -> None:
        nn.init.normal_(self.weight, mean=0.0, std=self.init_std)
        if self.bias is not None:
            bound = 1.0 / (self.weight.shape[1] ** 0.5)
            nn.init.uniform_(self.bias, -bound, bound)

    def forward(self, x: Tensor) -> Tensor:
        return F.linear(x, self.weight, self.bias)
