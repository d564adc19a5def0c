"""AutoAWQ-GEMM quantization of float weights on the GPU: the drop-in for the reference's
``llmserve/quantization/awq_calibration.py`` producer functions.

* ``PackedAWQWeight``       awq_calibration.py:12-16
* ``pack_int4``             ``_pack_int4``, awq_calibration.py:19-32 (same checks and errors)
* ``quantize_awq_weight``   awq_calibration.py:35-62 (same checks and errors)

Both run in the HIP library (``w4a16_quantize``, ``w4a16_pack_int4``); the results are
bit-exact with the reference's torch arithmetic for finite weights.  Host tensors are
refused: there is no CPU path.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .._lib import lib

__all__ = ("AWQ_PACK_ORDER", "PackedAWQWeight", "pack_int4", "quantize_awq_weight")

AWQ_PACK_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
MAX_GROUP_SIZE = 128


@dataclass(frozen=True)
class PackedAWQWeight:
    qweight: torch.Tensor
    qzeros: torch.Tensor
    scales: torch.Tensor


def _require_gpu(t: torch.Tensor) -> None:
    if t.device.type != "cuda":
        raise ValueError("AWQ quantization on this backend needs GPU (HIP) tensors")


def pack_int4(values: torch.Tensor) -> torch.Tensor:
    """int values [R, C] in [0, 15] -> int32 AutoAWQ words [R, C / 8] (nibble i of word j
    holds column 8 j + AWQ_PACK_ORDER[i])."""
    if values.ndim != 2:
        raise ValueError("INT4 packing expects a 2D tensor")
    if values.shape[1] % 8 != 0:
        raise ValueError("INT4 packing requires the output dimension to be divisible by 8")
    if values.is_floating_point():
        raise TypeError("INT4 packing expects an integer tensor")
    _require_gpu(values)
    if bool(torch.any((values < 0) | (values > 15))):
        raise ValueError("INT4 values must be in [0, 15]")
    v = values.to(torch.int32).contiguous()
    if v.numel() == 0:
        return torch.empty((v.shape[0], v.shape[1] // 8), dtype=torch.int32, device=v.device)
    return lib().pack_int4(v)


def quantize_awq_weight(weight: torch.Tensor, group_size: int = 128) -> PackedAWQWeight:
    """Quantize an [out_features, in_features] weight to AutoAWQ GEMM layout
    (awq_calibration.py:35-62): per output row and group of ``group_size`` inputs,
    s = max(max - min, 1e-5) / 15, z = clamp(-round(min / s), 0, 15),
    q = clamp(round(w / s) + z, 0, 15); scales keep the weight's dtype."""
    if weight.ndim != 2:
        raise ValueError("AWQ quantization expects a two-dimensional weight tensor")
    if not weight.is_floating_point():
        raise ValueError("AWQ quantization expects a floating-point weight tensor")
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    out_features, in_features = weight.shape
    if in_features % group_size != 0:
        raise ValueError("input size must be divisible by group_size")
    if out_features % 8 != 0:
        raise ValueError("output size must be divisible by 8")
    _require_gpu(weight)
    if group_size > MAX_GROUP_SIZE:
        raise ValueError(f"this backend quantizes groups of at most {MAX_GROUP_SIZE} inputs")
    if weight.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError("AWQ quantization on this backend takes bf16, fp16 or fp32 weights")
    qweight, qzeros, scales = lib().quantize(weight.contiguous(), group_size)
    return PackedAWQWeight(qweight=qweight, qzeros=qzeros, scales=scales)
