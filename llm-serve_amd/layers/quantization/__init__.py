from .awq import (
    AWQLinearMethod,
    AWQRuntimeConfig,
    awq_linear,
    dequantize_awq_gemm,
    repack_awq_qweight,
    unpack_awq_int4,
)

__all__ = (
    "AWQLinearMethod",
    "AWQRuntimeConfig",
    "awq_linear",
    "dequantize_awq_gemm",
    "repack_awq_qweight",
    "unpack_awq_int4",
)
