"""The reference backend's CPU path, restated with torch CPU ops.

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``tests/`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module: the tests pin it against the numpy oracle, and the
benchmark times it on the host's cores as the CPU baseline of the W4A16 linear, because it
runs the same torch operations as the reference's own ``awq_reference_linear`` (reference =
HGinkgo/LLM-Serve, llmserve/layers/quantization/awq.py):

* ``unpack_int4``    awq.py:184-200   logical column c of a packed word sits at bit shift
                                      4 * (0, 4, 1, 5, 2, 6, 3, 7)[c % 8]; arithmetic shift,
                                      then the low 4 bits (correct for negative int32 words)
* ``dequantize``     awq.py:235-248   (bf16(q) - bf16(z)) * s in the scales' dtype, with the
                                      group rows of z and s repeated over K
* ``linear``         awq.py:251-276   matmul(x.to(W.dtype), W) on torch's CPU BLAS, then the
                                      input dtype

The unpack takes each logical column's shift directly instead of unpacking in nibble order
and gathering, which yields the same integers.
"""
from __future__ import annotations

import torch

# bit shift of logical column c within an AutoAWQ word (awq.py:8, AWQ_REVERSE_ORDER = 0,4,1,5,2,6,3,7)
_SHIFTS = torch.tensor([4 * r for r in (0, 4, 1, 5, 2, 6, 3, 7)], dtype=torch.int32)


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """int32 [R, C] AutoAWQ words -> int32 [R, 8 C] values in logical column order."""
    rows = packed.shape[0]
    vals = torch.bitwise_and(torch.bitwise_right_shift(packed.unsqueeze(-1), _SHIFTS.to(packed.device)), 0xF)
    return vals.reshape(rows, -1)


def dequantize(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """W [K, N] in the scales' dtype: (q - z) * s, each operation in that dtype."""
    dt = scales.dtype
    q = unpack_int4(qweight).to(dt)
    z = unpack_int4(qzeros).repeat_interleave(group_size, dim=0).to(dt)
    s = scales.repeat_interleave(group_size, dim=0)
    return (q - z) * s


def linear(x: torch.Tensor, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
           group_size: int) -> torch.Tensor:
    """y = x @ W in the scales' dtype on the CPU BLAS, returned in x's dtype."""
    w = dequantize(qweight, qzeros, scales, group_size)
    return torch.matmul(x.to(w.dtype), w).to(x.dtype)
