"""CPU oracle for the AutoAWQ-GEMM W4A16 linear path (numpy restatement).

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or, for ``cpu_baseline``, as the CPU timing subject).  The HIP product path
never calls into it; when the HIP library is missing the product raises.

What it restates (reference = HGinkgo/LLM-Serve):

* ``AWQ_PACK_ORDER`` / ``pack_awq_int4``      llmserve/quantization/awq_calibration.py:9, 19-32
                                               (test packer tests/test_awq_reference.py:7-16)
* ``AWQ_REVERSE_ORDER`` / ``unpack_awq_int4``  llmserve/layers/quantization/awq.py:8, 184-200
* ``validate_awq_tensors``                    llmserve/layers/quantization/awq.py:203-232
* ``dequantize_awq_gemm_bits``                llmserve/layers/quantization/awq.py:235-248
    W[k, n] = bf16( bf16(q[k, n]) - bf16(z[k // g, n]) ) * s[k // g, n]   (bf16 tensor ops)
  q - z is an integer in [-15, 15] and is exact in bf16; the product of that
  integer with a bf16 scale has at most 12 significant bits and is exact in fp32,
  so torch's bf16 multiply (fp32 compute, one round-to-nearest-even) equals
  ``RNE_bf16(float32(q - z) * float32(s))``.  That is what is computed here,
  bit-exactly, including signed zeros, subnormals and infinities.
* ``awq_linear_ref``                          llmserve/layers/quantization/awq.py:251-276
    y = matmul(x, W) with W from the dequant above, accumulated in fp32 (the
    reference's BLAS) or fp64 (a tighter reference for tolerance checks).
* ``silu_and_mul_ref``                        llmserve/layers/activation.py:8-11
    x, y = chunk(2, -1); silu(x) * y, evaluated in fp64 on the bf16 inputs (the
    reference's compiled kernel computes in fp32 and rounds once to bf16).
* ``awq_gate_up_silu_mul_ref``                llmserve/models/qwen3.py:126-130
    SiluAndMul(gate_up_proj(x)): the GEMM (fp64 accumulation) rounded to bf16 as the
    reference's layer returns it (or, optionally, unrounded), then ``silu_and_mul_ref``.
* ``quantize_awq_weight``                     llmserve/quantization/awq_calibration.py:35-62
    the producer side of the format, used for known-answer tests and synthetic data.
* ``add_rms_norm_ref``                        llmserve/layers/layernorm.py:16-40
    rms_forward / add_rms_forward: s = float(x) (+ float(residual)) in fp32, the new
    residual bf16(s), then bf16(float(bf16(s * rsqrt(mean(s^2) + eps))) * weight) with
    the mean in fp64 rounded to fp32, + eps in fp32 (the reference's order), the rsqrt in
    fp64, and the product s * r rounded to fp32 first, as the reference stores it.

Parity pinning (every function above is checked by tests/test_oracle.py against the
reference's own known-answer tests, hand-derived constants, torch's bf16 arithmetic
and exact rational arithmetic on small inputs).  ``f32_to_bf16_bits`` follows c10's
``round_to_nearest_even`` (canonical NaN 0x7FC0), the conversion torch applies in the
reference's bf16 arithmetic.
"""
from __future__ import annotations

import numpy as np

AWQ_PACK_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)
PACK_FACTOR = 8


# ----------------------------------------------------------------------------- bf16
def f32_to_bf16_bits(values) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest, ties to even.

    NaN maps to the canonical quiet NaN 0x7FC0 (c10::BFloat16 semantics)."""
    f = np.ascontiguousarray(np.asarray(values, dtype=np.float32))
    u = f.view(np.uint32)
    # uint32 cannot overflow here for non-NaN inputs (max 0xFF800000 + 0x8000); NaN
    # patterns may wrap but are replaced below.
    with np.errstate(over="ignore"):
        r = u + (((u >> 16) & np.uint32(1)) + np.uint32(0x7FFF))
    out = (r >> 16).astype(np.uint16)
    out[np.isnan(f)] = 0x7FC0
    return out


def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


# ------------------------------------------------------------------- pack / unpack
def pack_awq_int4(values) -> np.ndarray:
    """int values in [0, 15], shape [R, C] (C % 8 == 0) -> int32 [R, C // 8].

    Nibble i of word [r, j] holds logical column 8*j + AWQ_PACK_ORDER[i]
    (awq_calibration.py:29-32: ordered = values[..., PACK_ORDER]; sum(ordered << 4*i))."""
    v = np.asarray(values)
    if v.ndim != 2:
        raise ValueError("INT4 packing expects a 2D tensor")
    if v.shape[1] % 8 != 0:
        raise ValueError("INT4 packing requires the output dimension to be divisible by 8")
    if np.issubdtype(v.dtype, np.floating):
        raise TypeError("INT4 packing expects an integer tensor")
    if v.size and (v.min() < 0 or v.max() > 15):
        raise ValueError("INT4 values must be in [0, 15]")
    ordered = v.astype(np.int64).reshape(v.shape[0], -1, 8)[:, :, list(AWQ_PACK_ORDER)]
    shifts = np.arange(0, 32, 4, dtype=np.int64)
    packed = np.sum(ordered << shifts, axis=-1)  # int64 in [0, 2^32)
    return packed.astype(np.uint32).view(np.int32)


def unpack_awq_int4(packed) -> np.ndarray:
    """int32 [R, C] -> int32 [R, 8C] in logical column order (awq.py:184-200)."""
    p = np.asarray(packed)
    if p.ndim != 2:
        raise ValueError("packed AWQ tensor must be two-dimensional")
    if p.dtype != np.int32:
        raise ValueError("packed AWQ tensor must use int32")
    shifts = np.arange(0, 32, 4, dtype=np.int32)
    nib = (p[:, :, None] >> shifts) & 0xF  # arithmetic shift, then mask: sign-safe
    return nib[:, :, list(AWQ_REVERSE_ORDER)].reshape(p.shape[0], -1).astype(np.int32)


# ------------------------------------------------------------------ validation
def validate_awq_tensors(qweight, qzeros, scales_shape, group_size: int) -> None:
    """Shape/dtype contract of awq.py:203-232 (scales passed by shape; dtype is bf16)."""
    qweight = np.asarray(qweight)
    qzeros = np.asarray(qzeros)
    if qweight.ndim != 2 or qweight.dtype != np.int32:
        raise ValueError("qweight must be a two-dimensional int32 tensor")
    if qzeros.ndim != 2 or qzeros.dtype != np.int32:
        raise ValueError("qzeros must be a two-dimensional int32 tensor")
    if len(scales_shape) != 2:
        raise ValueError("scales must be a two-dimensional floating tensor")
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    k = qweight.shape[0]
    if k % group_size:
        raise ValueError("qweight input size must be divisible by group_size")
    groups = k // group_size
    n = qweight.shape[1] * 8
    if qzeros.shape != (groups, qweight.shape[1]):
        raise ValueError("qzeros shape must be [input_size / group_size, output_size / 8]")
    if tuple(scales_shape) != (groups, n):
        raise ValueError("scales shape must be [input_size / group_size, output_size]")


# --------------------------------------------------------------------- dequant
def dequantize_awq_gemm_f32(qweight, qzeros, scales_f32, group_size: int) -> np.ndarray:
    """Exact float32 value of (q - z) * s before the final rounding, [K, N]."""
    scales_f32 = np.asarray(scales_f32, dtype=np.float32)
    validate_awq_tensors(qweight, qzeros, scales_f32.shape, group_size)
    q = unpack_awq_int4(qweight)
    z = np.repeat(unpack_awq_int4(qzeros), group_size, axis=0)
    s = np.repeat(scales_f32, group_size, axis=0)
    d = (q - z).astype(np.float32)  # exact integer in [-15, 15]
    with np.errstate(invalid="ignore", over="ignore"):
        return d * s  # exact in fp32 for finite s (<= 12 significant bits)


def dequantize_awq_gemm_bits(qweight, qzeros, scales_bits, group_size: int, rows_per_chunk: int = 1024) -> np.ndarray:
    """bf16 bit patterns (uint16) of the dequantized weight, [K, N] (awq.py:235-248).

    Works through whole groups of rows at a time to bound temporary memory."""
    qweight = np.asarray(qweight)
    qzeros = np.asarray(qzeros)
    s = bf16_bits_to_f32(scales_bits)
    validate_awq_tensors(qweight, qzeros, s.shape, group_size)
    k, n = qweight.shape[0], qweight.shape[1] * 8
    out = np.empty((k, n), dtype=np.uint16)
    step = max(group_size, (rows_per_chunk // group_size) * group_size)
    for r0 in range(0, k, step):
        r1 = min(k, r0 + step)
        g0, g1 = r0 // group_size, r1 // group_size
        out[r0:r1] = f32_to_bf16_bits(
            dequantize_awq_gemm_f32(qweight[r0:r1], qzeros[g0:g1], s[g0:g1], group_size))
    return out


def dequantize_awq_gemm_fp(qweight, qzeros, scales, group_size: int) -> np.ndarray:
    """Dequant for a floating scales array computed in that array's own precision
    (the reference's KATs use float32 scales, awq.py:246-248 computes in scales.dtype)."""
    scales = np.asarray(scales)
    validate_awq_tensors(qweight, qzeros, scales.shape, group_size)
    q = unpack_awq_int4(qweight).astype(scales.dtype)
    z = np.repeat(unpack_awq_int4(qzeros), group_size, axis=0).astype(scales.dtype)
    return (q - z) * np.repeat(scales, group_size, axis=0)


# ---------------------------------------------------------------------- linear
def awq_linear_ref(x_bits, qweight, qzeros, scales_bits, group_size: int, accum: str = "f64") -> np.ndarray:
    """y = x @ W with x given as bf16 bits [..., K]; W = bf16 dequant (awq.py:269-276).

    Returns float32 (accum='f32': BLAS sgemm) or float64 (accum='f64') [..., N]."""
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    if x_bits.shape[-1] != np.asarray(qweight).shape[0]:
        raise ValueError("AWQ activation K must match qweight input size")
    w = bf16_bits_to_f32(dequantize_awq_gemm_bits(qweight, qzeros, scales_bits, group_size))
    x = bf16_bits_to_f32(x_bits)
    if accum == "f32":
        return np.matmul(x, w)
    if accum == "f64":
        return np.matmul(x.astype(np.float64), w.astype(np.float64))
    raise ValueError("accum must be 'f32' or 'f64'")


def awq_linear_bf16_bits(x_bits, qweight, qzeros, scales_bits, group_size: int) -> np.ndarray:
    """bf16 output bits of the reference backend: fp32-accumulated matmul, then RNE."""
    y = awq_linear_ref(x_bits, qweight, qzeros, scales_bits, group_size, accum="f32")
    return f32_to_bf16_bits(y)


# ------------------------------------------------------------------ activation
def silu_and_mul_ref(gate_up) -> np.ndarray:
    """SiluAndMul (activation.py:8-11): the last axis splits into halves x | y (first half
    x), result silu(x) * y = x / (1 + exp(-x)) * y, in float64."""
    a = np.asarray(gate_up, dtype=np.float64)
    if a.shape[-1] % 2:
        raise ValueError("SiluAndMul needs an even last dimension")
    half = a.shape[-1] // 2
    x, y = a[..., :half], a[..., half:]
    with np.errstate(over="ignore"):
        sig = 1.0 / (1.0 + np.exp(-x))
    return x * sig * y


def awq_gate_up_silu_mul_ref(x_bits, qweight, qzeros, scales_bits, group_size: int,
                             round_intermediate: bool = True) -> np.ndarray:
    """SiluAndMul(gate_up_proj(x)) (qwen3.py:126-130), float64 [..., N / 2].

    round_intermediate=True: the gate|up GEMM rounded to bf16 as the reference's layer
    returns it, then ``silu_and_mul_ref`` (the reference's two steps).  False: the same
    composition without that rounding (the exact value a fused kernel approximates)."""
    y = awq_linear_ref(x_bits, qweight, qzeros, scales_bits, group_size, accum="f64")
    if round_intermediate:
        y = bf16_bits_to_f32(f32_to_bf16_bits(y.astype(np.float32)))
    return silu_and_mul_ref(y)


# ------------------------------------------------------------------- producer
def quantize_awq_weight(weight, group_size: int = 128, out_dtype: str = "bf16"):
    """[out_features, in_features] float -> (qweight, qzeros, scales) in AutoAWQ GEMM
    layout (awq_calibration.py:35-62).  Scales are returned as bf16 bits when
    out_dtype == 'bf16', as float16 when 'f16' (RNE, as torch's .to(float16)), else as
    float32."""
    w = np.asarray(weight)
    if w.ndim != 2:
        raise ValueError("AWQ quantization expects a two-dimensional weight tensor")
    if not np.issubdtype(w.dtype, np.floating):
        raise ValueError("AWQ quantization expects a floating-point weight tensor")
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    out_f, in_f = w.shape
    if in_f % group_size != 0:
        raise ValueError("input size must be divisible by group_size")
    if out_f % 8 != 0:
        raise ValueError("output size must be divisible by 8")
    g = w.astype(np.float32).reshape(out_f, in_f // group_size, group_size)
    gmin = g.min(axis=-1)
    gmax = g.max(axis=-1)
    scales = (np.maximum(gmax - gmin, np.float32(1e-5)) / np.float32(15.0)).astype(np.float32)
    zeros = np.clip(-np.round(gmin / scales), 0, 15)
    q = np.round(g / scales[..., None]) + zeros[..., None]
    q = np.clip(q, 0, 15).astype(np.int32).reshape(out_f, in_f)
    qweight = pack_awq_int4(np.ascontiguousarray(q.T))
    qzeros = pack_awq_int4(np.ascontiguousarray(zeros.astype(np.int32).T))
    s_t = np.ascontiguousarray(scales.T)
    if out_dtype == "bf16":
        return qweight, qzeros, f32_to_bf16_bits(s_t)
    if out_dtype == "f16":
        return qweight, qzeros, s_t.astype(np.float16)
    return qweight, qzeros, s_t


# ------------------------------------------------------------- synthetic data
def add_rms_norm_ref(x_bits, residual_bits, weight_bits, eps: float):
    """(x_norm bits, residual_out bits or None, s * r in fp64) for rows of bf16 x [M, K].

    layernorm.py:28-40 (add_rms_forward) when ``residual_bits`` is given, layernorm.py:17-26
    (rms_forward) when it is None.  ``s`` = fp32 sum of the two bf16 inputs (numpy's fp32 add
    rounds to nearest even as the GPU does); the row mean of s^2 is taken in fp64 and
    rounded to fp32, eps is added in fp32 (``var + self.eps``), the reciprocal square root is
    taken in fp64; s * r is rounded to fp32 (the reference's in-place fp32 product)
    and then to bf16 (``x.to(orig_dtype)``); the product with the bf16 weight is exact in
    fp32 (two 8-bit significands), so it is rounded once, to bf16."""
    s = bf16_bits_to_f32(np.asarray(x_bits, dtype=np.uint16))
    res_out = None
    if residual_bits is not None:
        s = (s + bf16_bits_to_f32(np.asarray(residual_bits, dtype=np.uint16))).astype(np.float32)
        res_out = f32_to_bf16_bits(s)
    s64 = s.astype(np.float64)
    var = np.mean(s64 * s64, axis=-1, keepdims=True)
    var_eps = (var.astype(np.float32) + np.float32(eps)).astype(np.float64)
    normed = s64 / np.sqrt(var_eps)
    t = bf16_bits_to_f32(f32_to_bf16_bits(normed.astype(np.float32)))
    w = bf16_bits_to_f32(np.asarray(weight_bits, dtype=np.uint16))
    out = f32_to_bf16_bits((t.astype(np.float64) * w.astype(np.float64)).astype(np.float32))
    return out, res_out, normed


def make_problem(seed: int, m: int, k: int, n: int, group_size: int = 128,
                 scale_lo: float = 0.002, scale_hi: float = 0.02,
                 outlier_frac: float = 0.0, outlier_gain: float = 20.0) -> dict:
    """Seeded synthetic AWQ problem with the value distributions of the benchmark
    configs: int4 q and z uniform in {0..15} packed in AWQ order, bf16 scales uniform
    in [scale_lo, scale_hi], bf16 activations ~N(0, 1) with an optional fraction of
    input channels multiplied by ``outlier_gain``."""
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, size=(k, n), dtype=np.int64)
    z = rng.integers(0, 16, size=(k // group_size, n), dtype=np.int64)
    s = rng.uniform(scale_lo, scale_hi, size=(k // group_size, n)).astype(np.float32)
    x = rng.standard_normal(size=(m, k)).astype(np.float32)
    if outlier_frac > 0:
        count = int(round(outlier_frac * k))
        cols = rng.permutation(k)[:count]
        x[:, cols] *= np.float32(outlier_gain)
    return {
        "qweight": pack_awq_int4(q),
        "qzeros": pack_awq_int4(z),
        "scales_bits": f32_to_bf16_bits(s),
        "x_bits": f32_to_bf16_bits(x),
        "group_size": group_size,
    }


def gemm_rel_err(y, r) -> float:
    """Max elementwise relative error with an rms(r) floor on the denominator:
    max |y - r| / max(|r|, rms(r)).  Used as the bf16 GEMM tolerance metric."""
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    if r.size == 0:
        return 0.0
    rms = float(np.sqrt(np.mean(r * r)))
    denom = np.maximum(np.abs(r), rms if rms > 0 else 1.0)
    return float(np.max(np.abs(y - r) / denom))
