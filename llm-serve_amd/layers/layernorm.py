"""RMSNorm with the interface of the reference's llmserve/layers/layernorm.py:6-50.

``RMSNorm(hidden_size, eps)`` holds a bf16 ``weight``; ``forward(x)`` returns the normalised
activations and ``forward(x, residual)`` returns ``(normalised, new residual)`` where the new
residual is ``bf16(x + residual)``, as the reference's ``rms_forward`` / ``add_rms_forward``
do.  The computation runs in the HIP library (``w4a16_add_rmsnorm``); the projections that
consume the output can take the norm into their own call instead
(``QKVParallelLinear.forward_rmsnorm``, ``MergedColumnParallelLinear.forward_rmsnorm_silu_and_mul``).
"""
from __future__ import annotations

import torch
from torch import nn

from .quantization.awq import add_rms_norm


class RMSNorm(nn.Module):

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size, dtype=torch.bfloat16), requires_grad=False)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        return add_rms_norm(x, residual, self.weight, self.eps)
