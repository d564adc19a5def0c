"""MI355X (gfx950) W4A16 linear layer for AutoAWQ-GEMM checkpoints.

The package directory name contains a hyphen; import it with
``importlib.import_module("llm-serve_amd")``.  Compute runs only in the HIP library
``csrc/libw4a16.so`` (C ABI in include/w4a16.h); the Python side validates arguments,
owns device memory through torch, and mirrors the reference's operator interface.
"""
from ._lib import REGIME_DECODE, REGIME_NONE, REGIME_TILE, W4A16Error, W4A16Library, lib
from .layers.quantization.awq import (
    AWQLinearMethod,
    AWQRuntimeConfig,
    FUSED_NORM_MAX_M,
    NormInput,
    add_rms_norm,
    awq_linear,
    awq_linear_residual,
    awq_linear_residual_stats,
    awq_linear_rmsnorm,
    awq_linear_rmsnorm_stats,
    awq_linear_silu_mul,
    awq_regime,
    dequantize_awq_gemm,
    repack_awq_qweight,
    unpack_awq_int4,
)

__all__ = (
    "AWQLinearMethod",
    "AWQRuntimeConfig",
    "FUSED_NORM_MAX_M",
    "NormInput",
    "REGIME_DECODE",
    "REGIME_NONE",
    "REGIME_TILE",
    "W4A16Error",
    "W4A16Library",
    "add_rms_norm",
    "awq_linear",
    "awq_linear_residual",
    "awq_linear_residual_stats",
    "awq_linear_rmsnorm",
    "awq_linear_rmsnorm_stats",
    "awq_linear_silu_mul",
    "awq_regime",
    "dequantize_awq_gemm",
    "lib",
    "repack_awq_qweight",
    "unpack_awq_int4",
)
