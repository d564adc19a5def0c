"""AutoAWQ-GEMM W4A16 linear method on MI355X: the drop-in for the reference's
``llmserve/layers/quantization/awq.py`` operator interface.

Same names, argument meaning and error behaviour as the reference:

* ``AWQRuntimeConfig`` / ``from_hf_config``        awq.py:11-67
* ``AWQLinearMethod.create_weights``               awq.py:76-113
* ``AWQLinearMethod.apply``                        awq.py:115-154
* ``AWQLinearMethod.process_weights_after_loading`` awq.py:156-181
* ``unpack_awq_int4``                              awq.py:184-200
* ``dequantize_awq_gemm``                          awq.py:235-248
* ``awq_linear`` (the reference's ``awq_cuda_linear`` / ``awq_reference_linear`` role,
  awq_cuda.py:141-185, awq.py:251-276)
* ``awq_linear_residual`` / ``AWQLinearMethod.apply_residual``: the GEMM with the residual
  add of the reference's ``add_rms_forward`` (layernorm.py:35-36) in its epilogue
* ``awq_linear_silu_mul`` / ``AWQLinearMethod.apply_silu_and_mul``: the gate|up GEMM with
  the reference's ``SiluAndMul`` (activation.py:8-11, applied at qwen3.py:126-130) fused
  into its epilogue; no reference counterpart as one call
* ``add_rms_norm``: the reference's ``RMSNorm`` forward (layernorm.py:16-50) on the HIP
  kernel; ``awq_linear_rmsnorm`` / ``AWQLinearMethod.apply_rmsnorm``: that norm in front of
  the QKV or gate_up GEMM in one library call (qwen3.py:166-173)
* ``awq_linear_residual_stats`` / ``awq_linear_rmsnorm_stats`` (``NormInput``): at decode
  sizes the same norm split between the O / down GEMM before it (residual add and row
  statistics in its epilogue) and the QKV / gate_up GEMM after it, with no launch between

There is one execution backend, the HIP library (libw4a16.so): every tensor operation
runs there and raises when the library or a GPU is missing -- nothing falls back to a CPU
path.  ``process_weights_after_loading`` reorders the ``qweight`` words once into the kernels'
group-tile layout (``awq_qweight``); ``qzeros`` and ``scales`` are consumed as stored.
"""
from __future__ import annotations

import functools
import threading
from collections.abc import Mapping
from dataclasses import dataclass

import torch
from torch import nn

from ..._lib import REGIME_DECODE, lib

AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)
EXECUTION_BACKEND = "hip"


@dataclass(frozen=True)
class AWQRuntimeConfig:
    bits: int
    group_size: int
    zero_point: bool
    version: str
    backend: str
    activation_dtype: torch.dtype
    quant_method: str = "awq"
    execution_backend: str = EXECUTION_BACKEND
    # Most tokens the engine packs into one GEMM (its Config.max_num_batched_tokens, 16384 by
    # default, config.py:11): the split-K workspace is reserved for that M at load time.
    max_batched_tokens: int = 16384

    @property
    def pack_factor(self) -> int:
        return 32 // self.bits

    @classmethod
    def from_hf_config(cls, hf_config) -> "AWQRuntimeConfig":
        raw = getattr(hf_config, "quantization_config", None)
        if not isinstance(raw, Mapping):
            raise ValueError("quantization_config must be an AWQ mapping")
        values = {
            "quant_method": str(raw.get("quant_method", "")).lower(),
            "backend": str(raw.get("backend", "")).lower(),
            "bits": raw.get("bits"),
            "group_size": raw.get("group_size"),
            "version": str(raw.get("version", "")).lower(),
            "zero_point": raw.get("zero_point"),
        }
        expected = {
            "quant_method": "awq",
            "backend": "autoawq",
            "bits": 4,
            "group_size": 128,
            "version": "gemm",
            "zero_point": True,
        }
        for field, want in expected.items():
            if values[field] != want:
                raise ValueError(f"unsupported AWQ {field}: expected {want!r}, got {values[field]!r}")
        activation_dtype = getattr(hf_config, "dtype", None)
        if activation_dtype != torch.bfloat16:
            raise ValueError(f"unsupported AWQ dtype: expected torch.bfloat16, got {activation_dtype!r}")
        return cls(
            bits=values["bits"],
            group_size=values["group_size"],
            zero_point=values["zero_point"],
            version=values["version"],
            backend=values["backend"],
            activation_dtype=activation_dtype,
            quant_method=values["quant_method"],
        )


# ------------------------------------------------------------------ workspace
class _WorkspacePool:
    """Split-K workspace shared by all layers on one device.

    One buffer per device serves every layer and every stream: kernels of one stream run in
    order, and the engine issues its layers on one stream at a time -- eagerly on its
    current stream, or under ``torch.cuda.graph(graph, pool)`` on torch's capture stream,
    which waits for the current stream before capturing and is waited for after it
    (model_runner.py:395-406).  Two GEMMs that may run at the same time on different
    streams must not share it: pass each its own ``workspace=``.  The buffer is zero-filled
    when (re)allocated and the kernels re-arm their counters to zero.  ``reserve`` (called
    by ``process_weights_after_loading`` for the largest M the engine packs) allocates
    outside the hot path, so that every later call up to that M -- on any stream, captured
    or not -- finds it big enough; ``get`` never allocates while the current stream is
    capturing a HIP graph (the allocation would become part of the graph): a request beyond
    the reservation raises there.  A buffer that is outgrown stays referenced for the life
    of the pool: a graph captured earlier may still address it, so its memory must not
    return to the allocator."""

    def __init__(self):
        self._lock = threading.Lock()
        self._buffers: dict[int, torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []

    @staticmethod
    def _key(device: torch.device) -> int:
        return device.index if device.index is not None else torch.cuda.current_device()

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor | None:
        if nbytes <= 0:
            return None
        key = self._key(device)
        with self._lock:
            buf = self._buffers.get(key)
            if buf is None or buf.numel() < nbytes:
                if torch.cuda.is_current_stream_capturing():
                    have = 0 if buf is None else buf.numel()
                    raise RuntimeError(
                        f"AWQ split-K workspace of {nbytes} bytes needed during HIP graph capture, but the "
                        f"device's workspace holds {have}: reserve it before capturing (raise "
                        f"max_batched_tokens, or call WORKSPACE.reserve)")
                if buf is not None:
                    self._retired.append(buf)
                size = max(nbytes, 2 * buf.numel() if buf is not None else 0)
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
                self._buffers[key] = buf
            return buf

    def reserve(self, device: torch.device, nbytes: int) -> None:
        self.get(device, nbytes)

    def reserved_bytes(self, device: torch.device) -> int:
        with self._lock:
            buf = self._buffers.get(self._key(device))
            return 0 if buf is None else buf.numel()


WORKSPACE = _WorkspacePool()


@functools.lru_cache(maxsize=256)
def max_workspace_bytes(k: int, n: int, max_tokens: int, group_size: int = 128) -> int:
    """Largest workspace any call with M <= max_tokens needs at this shape (the library
    evaluates its planner at every such M, so the result is kept per shape: a model loads
    the same four shapes once per layer)."""
    return lib().workspace_bytes_max(max_tokens, k, n, group_size)


# ------------------------------------------------------------- linear method
class AWQLinearMethod:

    def __init__(self, config: AWQRuntimeConfig):
        if config.execution_backend != EXECUTION_BACKEND:
            raise ValueError(
                f"unsupported AWQ execution_backend {config.execution_backend!r}: this build has a single "
                f"{EXECUTION_BACKEND!r} backend")
        self.config = config

    def create_weights(self, layer: nn.Module, input_size: int, output_size: int) -> None:
        if getattr(layer, "tp_size", 1) != 1:
            raise ValueError("AWQ tensor parallel is not supported")
        if input_size % self.config.group_size:
            raise ValueError("AWQ input size must be divisible by group_size")
        if output_size % self.config.pack_factor:
            raise ValueError("AWQ output size must be divisible by pack_factor")
        num_groups = input_size // self.config.group_size
        packed_output_size = output_size // self.config.pack_factor
        layer.qweight = nn.Parameter(torch.empty(input_size, packed_output_size, dtype=torch.int32),
                                     requires_grad=False)
        layer.qzeros = nn.Parameter(torch.empty(num_groups, packed_output_size, dtype=torch.int32),
                                    requires_grad=False)
        layer.scales = nn.Parameter(torch.empty(num_groups, output_size, dtype=self.config.activation_dtype),
                                    requires_grad=False)
        for param in (layer.qweight, layer.qzeros):
            param.output_dim = 1
            param.input_dim = 0
            param.packed_dim = 1
            param.pack_factor = self.config.pack_factor
        layer.scales.output_dim = 1
        layer.scales.input_dim = 0

    def apply_residual(self, layer: nn.Module, inputs: torch.Tensor, residual: torch.Tensor,
                       out: torch.Tensor | None = None) -> torch.Tensor:
        """``(self.apply(layer, inputs).float() + residual.float()).to(bf16)`` as one kernel:
        the residual update after O and down (qwen3.py:170-174, layernorm.py:35-36)."""
        if not hasattr(layer, "awq_qweight"):
            raise RuntimeError("AWQ HIP weights must be processed after checkpoint loading")
        return awq_linear_residual(inputs, layer.awq_qweight, layer.awq_qzeros, layer.scales, residual,
                                   group_size=self.config.group_size, out=out)

    def apply_silu_and_mul(self, layer: nn.Module, inputs: torch.Tensor) -> torch.Tensor:
        """``SiluAndMul()(self.apply(layer, inputs))`` as one kernel, for a layer whose output
        is [gate | up] of equal widths (qwen3.py:126-130)."""
        if not hasattr(layer, "awq_qweight"):
            raise RuntimeError("AWQ HIP weights must be processed after checkpoint loading")
        return awq_linear_silu_mul(inputs, layer.awq_qweight, layer.awq_qzeros, layer.scales,
                                   group_size=self.config.group_size)

    def apply_rmsnorm(self, layer: nn.Module, inputs: torch.Tensor, residual: torch.Tensor | None,
                      norm_weight: torch.Tensor, eps: float, silu_mul: bool = False):
        """``self.apply(layer, RMSNorm(inputs, residual))`` (or its SiLU(g) * u) with the
        norm in the same library call; returns ``(y, residual_out)`` (qwen3.py:166-173)."""
        if not hasattr(layer, "awq_qweight"):
            raise RuntimeError("AWQ HIP weights must be processed after checkpoint loading")
        return awq_linear_rmsnorm(inputs, residual, norm_weight, eps, layer.awq_qweight, layer.awq_qzeros,
                                  layer.scales, group_size=self.config.group_size, silu_mul=silu_mul)

    def apply_residual_stats(self, layer: nn.Module, inputs: torch.Tensor, residual: torch.Tensor,
                             residual_out: torch.Tensor | None = None):
        """The O / down projection with the residual add and the next RMSNorm's row
        statistics in its epilogue: ``(NormInput, new residual)``."""
        if not hasattr(layer, "awq_qweight"):
            raise RuntimeError("AWQ HIP weights must be processed after checkpoint loading")
        return awq_linear_residual_stats(inputs, layer.awq_qweight, layer.awq_qzeros, layer.scales, residual,
                                         group_size=self.config.group_size, residual_out=residual_out)

    def apply_rmsnorm_stats(self, layer: nn.Module, inp: NormInput, norm_weight: torch.Tensor, eps: float,
                            silu_mul: bool = False) -> torch.Tensor:
        """``self.apply(layer, RMSNorm(...))`` (or its SiLU(g) * u) from a producer's NormInput."""
        if not hasattr(layer, "awq_qweight"):
            raise RuntimeError("AWQ HIP weights must be processed after checkpoint loading")
        return awq_linear_rmsnorm_stats(inp, norm_weight, eps, layer.awq_qweight, layer.awq_qzeros, layer.scales,
                                        group_size=self.config.group_size, silu_mul=silu_mul)

    def apply(self, layer: nn.Module, inputs: torch.Tensor) -> torch.Tensor:
        if not hasattr(layer, "awq_qweight"):
            raise RuntimeError("AWQ HIP weights must be processed after checkpoint loading")
        return awq_linear(inputs, layer.awq_qweight, layer.awq_qzeros, layer.scales,
                          group_size=self.config.group_size)

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        qweight = layer.qweight.data
        if qweight.device.type != "cuda":
            raise ValueError("AWQ weights must be on a GPU (HIP) device before processing")
        _validate_awq_tensors(qweight, layer.qzeros.data, layer.scales.data, self.config.group_size)
        packed = repack_awq_qweight(qweight)
        qzeros = layer.qzeros.data.contiguous()
        k, n = qweight.shape[0], qweight.shape[1] * 8
        delattr(layer, "qweight")
        delattr(layer, "qzeros")
        layer.register_buffer("awq_qweight", packed, persistent=False)
        layer.register_buffer("awq_qzeros", qzeros, persistent=False)
        layer.awq_shape = (k, n)
        # calls up to the engine's largest packed M then never allocate (hipGraph capture,
        # tight serving loops)
        with torch.cuda.device(packed.device):
            WORKSPACE.reserve(packed.device, max_workspace_bytes(k, n, self.config.max_batched_tokens,
                                                                 self.config.group_size))


# ------------------------------------------------------------ tensor functions
def _validate_awq_tensors(qweight, qzeros, scales, group_size: int) -> None:
    """Reference contract, awq.py:203-232 (same messages)."""
    if qweight.ndim != 2 or qweight.dtype != torch.int32:
        raise ValueError("qweight must be a two-dimensional int32 tensor")
    if qzeros.ndim != 2 or qzeros.dtype != torch.int32:
        raise ValueError("qzeros must be a two-dimensional int32 tensor")
    if scales.ndim != 2 or not scales.is_floating_point():
        raise ValueError("scales must be a two-dimensional floating tensor")
    if group_size <= 0:
        raise ValueError("group_size must be positive")
    input_size = qweight.shape[0]
    if input_size % group_size:
        raise ValueError("qweight input size must be divisible by group_size")
    num_groups = input_size // group_size
    output_size = qweight.shape[1] * 8
    if qzeros.shape != (num_groups, qweight.shape[1]):
        raise ValueError("qzeros shape must be [input_size / group_size, output_size / 8]")
    if scales.shape != (num_groups, output_size):
        raise ValueError("scales shape must be [input_size / group_size, output_size]")
    if len({qweight.device, qzeros.device, scales.device}) != 1:
        raise ValueError("qweight, qzeros, and scales must share one device")


def unpack_awq_int4(packed: torch.Tensor) -> torch.Tensor:
    """int32 [R, C] -> int32 [R, 8C] in logical column order (awq.py:184-200)."""
    if packed.ndim != 2:
        raise ValueError("packed AWQ tensor must be two-dimensional")
    if packed.dtype != torch.int32:
        raise ValueError("packed AWQ tensor must use int32")
    if packed.numel() == 0:
        return torch.empty((packed.shape[0], packed.shape[1] * 8), dtype=torch.int32, device=packed.device)
    return lib().unpack_int4(packed.contiguous())


def dequantize_awq_gemm(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, *,
                        group_size: int) -> torch.Tensor:
    """bf16 W [K, N] = bf16_rne((q - z) * s), bit-exact with awq.py:235-248 for bf16 scales."""
    _validate_awq_tensors(qweight, qzeros, scales, group_size)
    if scales.dtype != torch.bfloat16:
        raise ValueError("the HIP dequant kernel takes bfloat16 scales")
    return lib().dequant(qweight.contiguous(), qzeros.contiguous(), scales.contiguous(), group_size)


def repack_awq_qweight(qweight: torch.Tensor) -> torch.Tensor:
    """AutoAWQ qweight [K, N/8] -> the kernels' group-tile layout (flat int32, same bytes)."""
    if qweight.ndim != 2 or qweight.dtype != torch.int32:
        raise ValueError("qweight must be a two-dimensional int32 tensor")
    k, n = qweight.shape[0], qweight.shape[1] * 8
    if k % 128:
        raise ValueError("qweight K must be divisible by 128")
    if n % 16:
        raise ValueError("qweight N must be divisible by 16")
    return lib().repack_qweight(qweight.contiguous())


def _aligned16(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def _prepare_linear(inputs, packed_qweight, qzeros, scales, group_size):
    """Shared argument checks of the GEMM entry points; returns (x [M, K], lead dims, K, N)."""
    if not inputs.is_floating_point():
        raise ValueError("AWQ activations must use a floating dtype")
    if inputs.dtype != scales.dtype:
        raise ValueError("AWQ activation dtype must match checkpoint scales dtype")
    if inputs.dtype != torch.bfloat16:
        raise ValueError("AWQ HIP kernels take bfloat16 activations")
    if inputs.device.type != "cuda":
        raise ValueError("AWQ HIP inputs must be GPU (HIP) tensors")
    if group_size != 128:
        raise ValueError("AWQ HIP kernels require group_size=128")
    if len({inputs.device, packed_qweight.device, qzeros.device, scales.device}) != 1:
        raise ValueError("AWQ activations and weights must share one device")
    if qzeros.dtype != torch.int32 or packed_qweight.dtype != torch.int32:
        raise ValueError("qweight and qzeros must be int32 tensors")
    n = scales.shape[1]
    k = scales.shape[0] * group_size
    if inputs.shape[-1] != k:
        raise ValueError("AWQ activation K must match qweight input size")
    if packed_qweight.numel() * 8 != k * n:
        raise ValueError("packed qweight does not match the scales shape")
    if n % 64:
        raise ValueError("AWQ HIP GEMM requires the output size to be divisible by 64")
    lead = inputs.shape[:-1]
    x = inputs.reshape(-1, k)
    if not x.is_contiguous() or not _aligned16(x):
        x = x.contiguous()
        if not _aligned16(x):
            x = x.clone()
    return x, lead, k, n


def awq_linear(inputs: torch.Tensor, packed_qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
               *, group_size: int, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """y[..., N] = inputs[..., K] @ W on the HIP kernels (bf16 in/out, fp32 accumulation).

    ``packed_qweight`` comes from ``repack_awq_qweight``; ``qzeros`` [K/128, N/8] and
    ``scales`` [K/128, N] are the AutoAWQ tensors.  Leading dimensions of ``inputs`` are
    flattened into M.  ``workspace`` (uint8, zero-filled when allocated) overrides the
    per-device shared one."""
    x, lead, k, n = _prepare_linear(inputs, packed_qweight, qzeros, scales, group_size)
    m = x.shape[0]
    y = torch.empty((m, n), dtype=inputs.dtype, device=inputs.device)
    if m == 0:
        return y.reshape(*lead, n)
    library = lib()
    if workspace is None:
        workspace = WORKSPACE.get(inputs.device, library.workspace_bytes(m, k, n, group_size))
    library.gemm(x, packed_qweight, qzeros, scales.contiguous(), y, k, n, workspace, group_size)
    return y.reshape(*lead, n)


def awq_linear_residual(inputs: torch.Tensor, packed_qweight: torch.Tensor, qzeros: torch.Tensor,
                        scales: torch.Tensor, residual: torch.Tensor, *, group_size: int,
                        out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(bf16(inputs @ W) + residual) -- the layer output rounded to bf16, then added to
    the residual in fp32 and rounded again, as the reference's add_rms_forward does
    (layernorm.py:35-36) -- in the GEMM epilogue.  ``residual`` is bf16 [..., N] on the same
    GPU; ``out`` (default: a new tensor) may be ``residual`` itself for an in-place update."""
    x, lead, k, n = _prepare_linear(inputs, packed_qweight, qzeros, scales, group_size)
    m = x.shape[0]
    if residual.dtype != torch.bfloat16 or residual.device != inputs.device:
        raise ValueError("AWQ residual must be a bfloat16 tensor on the activations' GPU")
    if residual.shape != (*lead, n):
        raise ValueError("AWQ residual shape must be the layer output shape")
    res = residual.reshape(m, n)
    if not res.is_contiguous() or not _aligned16(res):
        raise ValueError("AWQ residual must be contiguous and 16-byte aligned")
    if out is None:
        out = torch.empty_like(residual)
    if out.shape != residual.shape or out.dtype != torch.bfloat16 or not out.is_contiguous() or not _aligned16(out):
        raise ValueError("AWQ residual output must be a contiguous, 16-byte aligned bf16 tensor of the output shape")
    if m == 0:
        return out
    library = lib()
    if workspace is None:
        workspace = WORKSPACE.get(inputs.device, library.workspace_bytes(m, k, n, group_size))
    library.gemm_residual(x, packed_qweight, qzeros, scales.contiguous(), res, out.reshape(m, n), k, n, workspace,
                          group_size)
    return out


def awq_linear_silu_mul(inputs: torch.Tensor, packed_qweight: torch.Tensor, qzeros: torch.Tensor,
                        scales: torch.Tensor, *, group_size: int,
                        workspace: torch.Tensor | None = None) -> torch.Tensor:
    """SiLU(g) * u over [g | u] = inputs @ W for a gate|up weight of width N (first N/2
    columns gate, last N/2 up, as MergedColumnParallelLinear loads them): the reference's
    ``SiluAndMul`` (activation.py:8-11) applied to ``awq_linear``'s output, computed in the
    GEMM epilogue: the fp32 accumulators rounded to bf16 as that output is, then SiLU(g) * u
    in fp32, rounded once.  Returns
    [..., N/2]; N must be divisible by 128."""
    x, lead, k, n = _prepare_linear(inputs, packed_qweight, qzeros, scales, group_size)
    if n % 128:
        raise ValueError("AWQ fused SiLU * up requires the gate|up output size to be divisible by 128")
    m = x.shape[0]
    y = torch.empty((m, n // 2), dtype=inputs.dtype, device=inputs.device)
    if m == 0:
        return y.reshape(*lead, n // 2)
    library = lib()
    if workspace is None:
        workspace = WORKSPACE.get(inputs.device, library.workspace_bytes(m, k, n, group_size))
    library.gemm_silu_mul(x, packed_qweight, qzeros, scales.contiguous(), y, k, n, workspace, group_size)
    return y.reshape(*lead, n // 2)


def _norm_operands(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, strided_ok: bool = False):
    """Validated [M, K] views of the RMSNorm operands (bf16, contiguous, 16-byte aligned).
    With ``strided_ok`` (no residual) x may be a view whose rows lie at two strides (e.g.
    ``q.view(-1, heads, head_dim)`` of a split QKV output); then the first value returned is
    x itself and the row layout comes from ``_row_strides``."""
    if x.device.type != "cuda":
        raise ValueError("RMSNorm input must be on a GPU (HIP) device")
    k = x.shape[-1]
    tensors = [("input", x), ("weight", weight)] + ([("residual", residual)] if residual is not None else [])
    for name, t in tensors:
        if t.dtype != torch.bfloat16 or t.device != x.device:
            raise ValueError(f"RMSNorm {name} must be a bfloat16 tensor on the input's GPU")
        if name == "input" and strided_ok and _row_strides(x) is not None:
            continue
        if not t.is_contiguous() or not _aligned16(t):
            raise ValueError(f"RMSNorm {name} must be contiguous and 16-byte aligned")
    if weight.shape != (k,):
        raise ValueError(f"RMSNorm weight must have shape ({k},), got {tuple(weight.shape)}")
    if residual is not None and residual.shape != x.shape:
        raise ValueError("RMSNorm residual must have the input's shape")
    if k % 8 or k > 16384:
        raise ValueError(f"RMSNorm width must be a multiple of 8 and at most 16384 (got {k})")
    m = x.numel() // k if k else 0
    xv = x if strided_ok and not x.is_contiguous() else x.reshape(m, k)
    return xv, (residual.reshape(m, k) if residual is not None else None), m, k


def _row_strides(x: torch.Tensor):
    """(rows_inner, stride_outer, stride_inner) in elements when every row of x (its last
    dimension, unit stride) starts at (r // rows_inner) * stride_outer + (r % rows_inner) *
    stride_inner from x's first element with 16-byte aligned rows; None otherwise."""
    if x.stride(-1) != 1 or x.data_ptr() % 16:
        return None
    dims = [(size, stride) for size, stride in zip(x.shape[:-1], x.stride()[:-1]) if size != 1]
    # merge leading dimensions that are contiguous with each other
    merged: list[list[int]] = []
    for size, stride in dims:
        if merged and merged[-1][1] == stride * size:
            merged[-1] = [merged[-1][0] * size, stride]
        else:
            merged.append([size, stride])
    if not merged:
        return (1, 0, 0)
    if len(merged) == 1:
        rows, stride = merged[0]
        out = (rows, 0, stride)
    elif len(merged) == 2:
        (_, s_outer), (rows_inner, s_inner) = merged
        out = (rows_inner, s_outer, s_inner)
    else:
        return None
    if out[1] % 8 or out[2] % 8:
        return None
    return out


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor, eps: float,
                 *, residual_out: torch.Tensor | None = None):
    """The reference's RMSNorm forward (layernorm.py:16-50) on the HIP kernel: without a
    residual, ``bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight)``; with one, the same of
    ``s = x + residual`` (fp32) and also the new residual ``bf16(s)``, returned as
    ``(x_norm, residual_out)``.  ``residual_out`` may be ``residual`` (in place).  Without a
    residual, x may be a strided view (rows at up to two strides, unit stride inside a row),
    as q_norm / k_norm see the per-head views of the split QKV output (qwen3.py:87-94); the
    result is then a new contiguous tensor of x's shape, as the reference's is."""
    xv, rv, m, k = _norm_operands(x, residual, weight, strided_ok=residual is None)
    x_norm = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if residual is not None and residual_out is None:
        residual_out = torch.empty_like(x)
    if residual_out is not None and (residual_out.shape != x.shape or residual_out.dtype != torch.bfloat16
                                     or not residual_out.is_contiguous() or not _aligned16(residual_out)):
        raise ValueError("RMSNorm residual_out must be a contiguous, 16-byte aligned bf16 tensor of the input shape")
    if m > 0:
        if residual is None and not x.is_contiguous():
            rows_inner, s_outer, s_inner = _row_strides(x)
            lib().rmsnorm_strided(x, rows_inner, s_outer, s_inner, weight, eps, x_norm.view(m, k), m, k)
        else:
            lib().add_rmsnorm(xv, rv, weight, eps, x_norm.view(m, k),
                              residual_out.view(m, k) if residual_out is not None else None)
    return x_norm if residual is None else (x_norm, residual_out)


def awq_linear_rmsnorm(inputs: torch.Tensor, residual: torch.Tensor | None, norm_weight: torch.Tensor, eps: float,
                       packed_qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor, *,
                       group_size: int, silu_mul: bool = False, residual_out: torch.Tensor | None = None,
                       workspace: torch.Tensor | None = None):
    """The RMSNorm(+residual) in front of QKV or gate_up and the projection in one library
    call (qwen3.py:166-173 and 126-130 with layernorm.py:28-40): returns ``(y, residual_out)``
    with ``y = awq_linear(add_rms_norm(...))`` -- or, with ``silu_mul``, its SiLU(g) * u --
    and ``residual_out = bf16(inputs + residual)`` (may be ``residual`` itself).  Without a
    residual the new residual is ``inputs`` itself, as the reference's first decoder layer
    sets it (qwen3.py:166-167: ``hidden_states, residual = input_layernorm(hidden_states),
    hidden_states``).  The normalised activations go through a scratch tensor of the input's
    shape that the GEMM reads back from L2 at decode sizes."""
    xv, rv, m, k = _norm_operands(inputs, residual, norm_weight)
    lead = inputs.shape[:-1]
    _, _, k2, n = _prepare_linear(xv, packed_qweight, qzeros, scales, group_size)
    if k2 != k:
        raise ValueError("RMSNorm width and the layer's input size differ")
    if silu_mul and n % 128:
        raise ValueError("AWQ fused SiLU * up requires the gate|up output size to be divisible by 128")
    if residual is not None and residual_out is None:
        residual_out = torch.empty_like(inputs)
    if residual_out is not None and (residual_out.shape != inputs.shape or residual_out.dtype != torch.bfloat16
                                     or not residual_out.is_contiguous() or not _aligned16(residual_out)):
        raise ValueError("RMSNorm residual_out must be a contiguous, 16-byte aligned bf16 tensor of the input shape")
    n_out = n // 2 if silu_mul else n
    y = torch.empty((m, n_out), dtype=torch.bfloat16, device=inputs.device)
    if m > 0:
        library = lib()
        if workspace is None:
            workspace = WORKSPACE.get(inputs.device, library.workspace_bytes(m, k, n, group_size))
        x_norm = torch.empty((m, k), dtype=torch.bfloat16, device=inputs.device)
        library.gemm_rmsnorm(xv, rv, norm_weight, eps, x_norm,
                             residual_out.view(m, k) if residual_out is not None else None, packed_qweight,
                             qzeros, scales.contiguous(), y, n, workspace, group_size, silu_mul)
    return y.reshape(*lead, n_out), (residual_out if residual is not None else inputs)


# The RMSNorm split across two GEMMs runs in the decode kernel with its normalized rows
# staged in LDS: packed M up to this.
FUSED_NORM_MAX_M = 8


@dataclass(frozen=True)
class NormInput:
    """The input of an RMSNorm with its residual add done, as the O or down projection's
    epilogue leaves it (``awq_linear_residual_stats``): ``s`` = float(h) + float(residual) in
    fp32 [M, K], and ``ssq`` [M, K / 16] the per-row sums of s^2 over each 16-column tile."""
    s: torch.Tensor
    ssq: torch.Tensor


def awq_linear_residual_stats(inputs: torch.Tensor, packed_qweight: torch.Tensor, qzeros: torch.Tensor,
                              scales: torch.Tensor, residual: torch.Tensor, *, group_size: int,
                              residual_out: torch.Tensor | None = None, workspace: torch.Tensor | None = None):
    """The O / down projection followed by the residual add and the row statistics of the
    next RMSNorm (qwen3.py:170-174, layernorm.py:35-38), so that the norm needs no launch of
    its own: returns ``(NormInput, residual_out)`` with residual_out = bf16(h + residual)
    (``residual_out`` may be ``residual`` itself).  The projection's output h is not stored:
    the next norm reads ``NormInput.s``.  Packed M <= FUSED_NORM_MAX_M (decode sizes)."""
    x, lead, k, n = _prepare_linear(inputs, packed_qweight, qzeros, scales, group_size)
    m = x.shape[0]
    if m > FUSED_NORM_MAX_M:
        raise ValueError(f"the fused RMSNorm statistics take M <= {FUSED_NORM_MAX_M} (got {m}): use "
                         f"awq_linear_residual / awq_linear and add_rms_norm there")
    if residual.dtype != torch.bfloat16 or residual.device != inputs.device or residual.shape != (*lead, n):
        raise ValueError("AWQ residual must be a bfloat16 tensor of the layer output shape on the activations' GPU")
    res = residual.reshape(m, n)
    if not res.is_contiguous() or not _aligned16(res):
        raise ValueError("AWQ residual must be contiguous and 16-byte aligned")
    if residual_out is None:
        residual_out = torch.empty_like(residual)
    if (residual_out.shape != residual.shape or residual_out.dtype != torch.bfloat16 or not residual_out.is_contiguous()
            or not _aligned16(residual_out)):
        raise ValueError("AWQ residual output must be a contiguous, 16-byte aligned bf16 tensor of the output shape")
    s_out = torch.empty((m, n), dtype=torch.float32, device=inputs.device)
    ssq = torch.empty((m, n // 16), dtype=torch.float32, device=inputs.device)
    if m > 0:
        library = lib()
        if workspace is None:
            workspace = WORKSPACE.get(inputs.device, library.workspace_bytes(m, k, n, group_size))
        library.gemm_residual_stats(x, packed_qweight, qzeros, scales.contiguous(), res, s_out,
                                    residual_out.reshape(m, n), ssq, k, n, workspace, group_size)
    return NormInput(s_out, ssq), residual_out


def awq_linear_rmsnorm_stats(inp: NormInput, norm_weight: torch.Tensor, eps: float, packed_qweight: torch.Tensor,
                             qzeros: torch.Tensor, scales: torch.Tensor, *, group_size: int, silu_mul: bool = False,
                             x_norm: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The RMSNorm of a ``NormInput`` (the reference's rms scaling of add_rms_forward,
    layernorm.py:37-40, from the producer's sum s and row statistics) and the QKV GEMM --
    or, with ``silu_mul``, the gate|up GEMM with SiLU * up -- in one decode kernel:
    y = x_norm @ W with x_norm = bf16(float(bf16(s * rstd)) * float(norm_weight)).  The new
    residual came from the producer.  ``x_norm`` (optional, bf16 [M, K]) receives the
    normalized activations.  Packed M <= FUSED_NORM_MAX_M."""
    s, ssq = inp.s, inp.ssq
    if s.dtype != torch.float32 or s.ndim != 2 or ssq.dtype != torch.float32:
        raise ValueError("NormInput must hold fp32 s [M, K] and ssq [M, K / 16]")
    m, k = s.shape
    if ssq.shape != (m, k // 16):
        raise ValueError("NormInput ssq must be [M, K / 16]")
    if m > FUSED_NORM_MAX_M:
        raise ValueError(f"the fused RMSNorm statistics take M <= {FUSED_NORM_MAX_M} (got {m})")
    if norm_weight.dtype != torch.bfloat16 or norm_weight.shape != (k,):
        raise ValueError(f"RMSNorm weight must be a bfloat16 tensor of shape ({k},)")
    if len({s.device, ssq.device, norm_weight.device, packed_qweight.device}) != 1 or s.device.type != "cuda":
        raise ValueError("NormInput, the norm weight and the layer weights must share one GPU")
    if group_size != 128:
        raise ValueError("AWQ HIP kernels require group_size=128")
    n = scales.shape[1]
    if scales.shape[0] * group_size != k:
        raise ValueError("RMSNorm width and the layer's input size differ")
    if silu_mul and n % 128:
        raise ValueError("AWQ fused SiLU * up requires the gate|up output size to be divisible by 128")
    for t in (s, ssq, norm_weight):
        if not t.is_contiguous() or not _aligned16(t):
            raise ValueError("NormInput tensors and the norm weight must be contiguous and 16-byte aligned")
    if x_norm is not None and (x_norm.shape != (m, k) or x_norm.dtype != torch.bfloat16 or not x_norm.is_contiguous()
                               or not _aligned16(x_norm)):
        raise ValueError("x_norm must be a contiguous, 16-byte aligned bf16 [M, K] tensor")
    y = torch.empty((m, n // 2 if silu_mul else n), dtype=torch.bfloat16, device=s.device)
    if m > 0:
        library = lib()
        if workspace is None:
            workspace = WORKSPACE.get(s.device, library.workspace_bytes(m, k, n, group_size))
        library.gemm_rmsnorm_stats(s, ssq, norm_weight, eps, x_norm, packed_qweight, qzeros, scales.contiguous(), y, n,
                                   workspace, group_size, silu_mul)
    return y


def awq_regime(m: int, k: int, n: int) -> str:
    """Which kernel family ``awq_linear`` runs for this shape: 'decode' or 'tile'."""
    return "decode" if lib().regime(m, k, n) == REGIME_DECODE else "tile"
