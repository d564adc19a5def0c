"""ctypes binding of libw4a16.so, the C ABI declared in include/w4a16.h.

torch is imported first on purpose: libw4a16.so needs ``libamdhip64.so.7`` and must bind to
the HIP runtime torch already loaded (same soname), so both share one device context and
torch's streams are valid handles for the library.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc", "libw4a16.so")

REGIME_NONE = 0
REGIME_DECODE = 1
REGIME_TILE = 2

_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_c_ptr = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/w4a16.h
_SIGNATURES = {
    "w4a16_abi_version": (_c_int, []),
    "w4a16_last_error": (ctypes.c_char_p, []),
    "w4a16_unpack_int4": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_int, _c_ptr]),
    "w4a16_dequant": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_ptr]),
    "w4a16_repack_qweight": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_int, _c_ptr]),
    "w4a16_dequant_packed": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_ptr]),
    "w4a16_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "w4a16_workspace_bytes_max": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "w4a16_gemm": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_int,
                            _c_ptr, _c_size, _c_ptr]),
    "w4a16_gemm_noalloc": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_int,
                                    _c_ptr]),
    "w4a16_regime": (_c_int, [_c_int, _c_int, _c_int]),
    "w4a16_split_k": (_c_int, [_c_int, _c_int, _c_int]),
    "w4a16_plan": (_c_int, [_c_int, _c_int, _c_int, _c_int, ctypes.POINTER(ctypes.c_int)]),
    "w4a16_gemm_config": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_int,
                                   _c_int, _c_int, _c_int, _c_int, _c_int, _c_ptr, _c_size, _c_ptr]),
    "w4a16_workspace_bytes_config": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "w4a16_quantize": (_c_int, [_c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_ptr]),
    "w4a16_pack_int4": (_c_int, [_c_ptr, _c_ptr, _c_int, _c_int, _c_ptr]),
    "w4a16_gemm_residual": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int,
                                     _c_int, _c_ptr, _c_size, _c_ptr]),
    "w4a16_gemm_silu_mul": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int, _c_int,
                                     _c_ptr, _c_size, _c_ptr]),
    "w4a16_gemm_silu_mul_config": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int, _c_int, _c_int,
                                            _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_ptr, _c_size,
                                            _c_ptr]),
    "w4a16_add_rmsnorm": (_c_int, [_c_ptr, _c_ptr, _c_ptr, ctypes.c_float, _c_ptr, _c_ptr, _c_int, _c_int, _c_ptr]),
    "w4a16_rmsnorm_strided": (_c_int, [_c_ptr, _c_int, ctypes.c_int64, ctypes.c_int64, _c_ptr, ctypes.c_float,
                                       _c_ptr, _c_int, _c_int, _c_ptr]),
    "w4a16_gemm_rmsnorm": (_c_int, [_c_ptr, _c_ptr, _c_ptr, ctypes.c_float, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                    _c_ptr, _c_int, _c_int, _c_int, _c_int, _c_int, _c_ptr, _c_size, _c_ptr]),
    "w4a16_gemm_residual_stats": (_c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_int,
                                           _c_int, _c_int, _c_int, _c_ptr, _c_size, _c_ptr]),
    "w4a16_gemm_rmsnorm_stats": (_c_int, [_c_ptr, _c_ptr, _c_ptr, ctypes.c_float, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                          _c_ptr, _c_int, _c_int, _c_int, _c_int, _c_int, _c_ptr, _c_size, _c_ptr]),
}
ABI_VERSION = 5


def _ptr(t: torch.Tensor | None):
    return t.data_ptr() if t is not None else None


class W4A16Error(RuntimeError):
    """A nonzero status returned through the C ABI."""


class W4A16Library:
    """Thin typed wrapper over the C ABI.  Tensor-level methods take torch tensors on the
    GPU, allocate nothing but their outputs, and launch on the current torch stream."""

    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(
                f"W4A16 HIP library not built: {path} is missing (run __graft_entry__.build())")
        self.path = path
        self.dll = ctypes.CDLL(path)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(self.dll, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = self.dll.w4a16_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libw4a16.so ABI version {version}, expected {ABI_VERSION}")

    # ------------------------------------------------------------------ plumbing
    def last_error(self) -> str:
        return (self.dll.w4a16_last_error() or b"").decode()

    def check(self, status: int, what: str) -> None:
        if status != 0:
            raise W4A16Error(f"{what} failed (status {status}): {self.last_error()}")

    @staticmethod
    def _stream(t: torch.Tensor) -> int:
        return torch.cuda.current_stream(t.device).cuda_stream

    @staticmethod
    def _require_gpu(*tensors: torch.Tensor) -> None:
        for t in tensors:
            if t.device.type != "cuda":
                raise ValueError("W4A16 HIP kernels require GPU (HIP) tensors")

    # ------------------------------------------------------------ host queries
    def workspace_bytes(self, m: int, k: int, n: int, group_size: int = 128) -> int:
        return int(self.dll.w4a16_workspace_bytes(m, k, n, group_size))

    def workspace_bytes_max(self, m_max: int, k: int, n: int, group_size: int = 128) -> int:
        return int(self.dll.w4a16_workspace_bytes_max(m_max, k, n, group_size))

    def workspace_bytes_config(self, m: int, n: int, regime: int, p0: int, split: int) -> int:
        return int(self.dll.w4a16_workspace_bytes_config(m, n, regime, p0, split))

    def regime(self, m: int, k: int, n: int) -> int:
        return int(self.dll.w4a16_regime(m, k, n))

    def split_k(self, m: int, k: int, n: int) -> int:
        return int(self.dll.w4a16_split_k(m, k, n))

    def plan(self, m: int, k: int, n: int, entry: int = 0) -> tuple[int, int, int, int, int]:
        """(regime, p0, p1, p2, split) the entry point chooses (0 plain, 1 SiLU * up, 2 / 3
        the fused-RMSNorm consumer without / with SiLU * up, 4 the decode kernel's own plan)."""
        out = (ctypes.c_int * 5)()
        self.check(self.dll.w4a16_plan(m, k, n, entry, out), "w4a16_plan")
        return tuple(int(v) for v in out)

    # ---------------------------------------------------------- tensor methods
    def unpack_int4(self, packed: torch.Tensor) -> torch.Tensor:
        self._require_gpu(packed)
        rows, cols = packed.shape
        out = torch.empty((rows, cols * 8), dtype=torch.int32, device=packed.device)
        with torch.cuda.device(packed.device):
            self.check(self.dll.w4a16_unpack_int4(packed.data_ptr(), out.data_ptr(), rows, cols,
                                                  self._stream(packed)), "w4a16_unpack_int4")
        return out

    def dequant(self, qweight, qzeros, scales, group_size: int) -> torch.Tensor:
        self._require_gpu(qweight, qzeros, scales)
        k, n = qweight.shape[0], qweight.shape[1] * 8
        out = torch.empty((k, n), dtype=torch.bfloat16, device=qweight.device)
        with torch.cuda.device(qweight.device):
            self.check(self.dll.w4a16_dequant(qweight.data_ptr(), qzeros.data_ptr(), scales.data_ptr(),
                                              out.data_ptr(), k, n, group_size, self._stream(qweight)),
                       "w4a16_dequant")
        return out

    _DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

    def quantize(self, weight: torch.Tensor, group_size: int):
        """weight [out, in] (bf16 / fp16 / fp32, contiguous) -> (qweight [in, out/8],
        qzeros [in/g, out/8], scales [in/g, out] of weight's dtype)."""
        self._require_gpu(weight)
        out_f, in_f = weight.shape
        dev = weight.device
        qweight = torch.empty((in_f, out_f // 8), dtype=torch.int32, device=dev)
        qzeros = torch.empty((in_f // group_size, out_f // 8), dtype=torch.int32, device=dev)
        scales = torch.empty((in_f // group_size, out_f), dtype=weight.dtype, device=dev)
        with torch.cuda.device(dev):
            self.check(self.dll.w4a16_quantize(weight.data_ptr(), self._DTYPES[weight.dtype], qweight.data_ptr(),
                                               qzeros.data_ptr(), scales.data_ptr(), out_f, in_f, group_size,
                                               self._stream(weight)), "w4a16_quantize")
        return qweight, qzeros, scales

    def pack_int4(self, values: torch.Tensor) -> torch.Tensor:
        """int32 [rows, cols] -> AutoAWQ words [rows, cols/8] (low 4 bits of each value)."""
        self._require_gpu(values)
        rows, cols = values.shape
        out = torch.empty((rows, cols // 8), dtype=torch.int32, device=values.device)
        with torch.cuda.device(values.device):
            self.check(self.dll.w4a16_pack_int4(values.data_ptr(), out.data_ptr(), rows, cols,
                                                self._stream(values)), "w4a16_pack_int4")
        return out

    def repack_qweight(self, qweight: torch.Tensor) -> torch.Tensor:
        self._require_gpu(qweight)
        k, n = qweight.shape[0], qweight.shape[1] * 8
        out = torch.empty((k * n // 8,), dtype=torch.int32, device=qweight.device)
        with torch.cuda.device(qweight.device):
            self.check(self.dll.w4a16_repack_qweight(qweight.data_ptr(), out.data_ptr(), k, n,
                                                     self._stream(qweight)), "w4a16_repack_qweight")
        return out

    def dequant_packed(self, packed, qzeros, scales, k: int, n: int, group_size: int = 128) -> torch.Tensor:
        self._require_gpu(packed, qzeros, scales)
        out = torch.empty((k, n), dtype=torch.bfloat16, device=packed.device)
        with torch.cuda.device(packed.device):
            self.check(self.dll.w4a16_dequant_packed(packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(),
                                                     out.data_ptr(), k, n, group_size, self._stream(packed)),
                       "w4a16_dequant_packed")
        return out

    def gemm(self, x, packed, qzeros, scales, y, k: int, n: int, workspace: torch.Tensor | None,
             group_size: int = 128) -> torch.Tensor:
        """y[M, N] = x[M, K] @ W; every tensor already on one GPU, contiguous."""
        m = x.shape[0]
        ws_ptr = workspace.data_ptr() if workspace is not None else None
        ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
        with torch.cuda.device(x.device):
            self.check(self.dll.w4a16_gemm(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(),
                                           y.data_ptr(), m, k, n, group_size, ws_ptr, ws_len, self._stream(x)),
                       "w4a16_gemm")
        return y

    def gemm_residual(self, x, packed, qzeros, scales, residual, y, k: int, n: int,
                      workspace: torch.Tensor | None, group_size: int = 128) -> torch.Tensor:
        """y[M, N] = bf16(bf16(x @ W) + residual); residual may be y."""
        m = x.shape[0]
        ws_ptr = workspace.data_ptr() if workspace is not None else None
        ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
        with torch.cuda.device(x.device):
            self.check(self.dll.w4a16_gemm_residual(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(),
                                                    scales.data_ptr(), residual.data_ptr(), y.data_ptr(), m, k, n,
                                                    group_size, ws_ptr, ws_len, self._stream(x)),
                       "w4a16_gemm_residual")
        return y

    def gemm_silu_mul(self, x, packed, qzeros, scales, y, k: int, n: int, workspace: torch.Tensor | None,
                      group_size: int = 128) -> torch.Tensor:
        """y[M, N/2] = SiLU(g) * u, [g | u] = x[M, K] @ W for a gate|up weight of width N."""
        m = x.shape[0]
        ws_ptr = workspace.data_ptr() if workspace is not None else None
        ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
        with torch.cuda.device(x.device):
            self.check(self.dll.w4a16_gemm_silu_mul(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(),
                                                    scales.data_ptr(), y.data_ptr(), m, k, n, group_size, ws_ptr,
                                                    ws_len, self._stream(x)),
                       "w4a16_gemm_silu_mul")
        return y

    def add_rmsnorm(self, x, residual, weight, eps: float, x_norm, residual_out) -> torch.Tensor:
        """x_norm = RMSNorm(x + residual) * weight, residual_out = bf16(x + residual) (no add
        and no residual_out when residual is None); [M, K] bf16, contiguous, one GPU."""
        m, k = x.shape
        with torch.cuda.device(x.device):
            self.check(self.dll.w4a16_add_rmsnorm(x.data_ptr(), _ptr(residual), weight.data_ptr(), float(eps),
                                                  x_norm.data_ptr(), _ptr(residual_out), m, k, self._stream(x)),
                       "w4a16_add_rmsnorm")
        return x_norm

    def rmsnorm_strided(self, x, rows_inner: int, stride_outer: int, stride_inner: int, weight, eps: float,
                        x_norm, m: int, k: int) -> torch.Tensor:
        """x_norm [m, k] = RMSNorm of rows read at x + (r // rows_inner) * stride_outer +
        (r % rows_inner) * stride_inner (elements), no residual."""
        with torch.cuda.device(x.device):
            self.check(self.dll.w4a16_rmsnorm_strided(x.data_ptr(), rows_inner, stride_outer, stride_inner,
                                                      weight.data_ptr(), float(eps), x_norm.data_ptr(), m, k,
                                                      self._stream(x)),
                       "w4a16_rmsnorm_strided")
        return x_norm

    def gemm_rmsnorm(self, x, residual, weight, eps: float, x_norm, residual_out, packed, qzeros, scales, y,
                     n: int, workspace: torch.Tensor | None, group_size: int = 128,
                     silu_mul: bool = False) -> torch.Tensor:
        """The RMSNorm(+residual) prologue into x_norm, then y = x_norm @ W (or SiLU(g) * u)."""
        m, k = x.shape
        ws_ptr = workspace.data_ptr() if workspace is not None else None
        ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
        with torch.cuda.device(x.device):
            self.check(self.dll.w4a16_gemm_rmsnorm(x.data_ptr(), _ptr(residual), weight.data_ptr(), float(eps),
                                                   x_norm.data_ptr(), _ptr(residual_out), packed.data_ptr(),
                                                   qzeros.data_ptr(), scales.data_ptr(), y.data_ptr(), m, k, n,
                                                   group_size, int(silu_mul), ws_ptr, ws_len, self._stream(x)),
                       "w4a16_gemm_rmsnorm")
        return y

    def gemm_residual_stats(self, x, packed, qzeros, scales, residual, s_out, residual_out, ssq_out, k: int, n: int,
                            workspace: torch.Tensor | None, group_size: int = 128) -> None:
        """Producer half of a fused RMSNorm: s_out = float(bf16(x @ W)) + float(residual),
        residual_out = bf16(s_out), ssq_out = per-row sums of s_out^2 per 16-column tile."""
        m = x.shape[0]
        ws_ptr = workspace.data_ptr() if workspace is not None else None
        ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
        with torch.cuda.device(x.device):
            self.check(self.dll.w4a16_gemm_residual_stats(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(),
                                                          scales.data_ptr(), residual.data_ptr(), s_out.data_ptr(),
                                                          residual_out.data_ptr(), ssq_out.data_ptr(), m, k, n,
                                                          group_size, ws_ptr, ws_len, self._stream(x)),
                       "w4a16_gemm_residual_stats")

    def gemm_rmsnorm_stats(self, s, ssq, weight, eps: float, x_norm, packed, qzeros, scales, y, n: int,
                           workspace: torch.Tensor | None, group_size: int = 128, silu_mul: bool = False):
        """Consumer half: y = bf16(bf16(s * rstd) * weight) @ W (or SiLU(g) * u), rstd from ssq."""
        m, k = s.shape
        ws_ptr = workspace.data_ptr() if workspace is not None else None
        ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
        with torch.cuda.device(s.device):
            self.check(self.dll.w4a16_gemm_rmsnorm_stats(s.data_ptr(), ssq.data_ptr(), weight.data_ptr(), float(eps),
                                                         _ptr(x_norm), packed.data_ptr(), qzeros.data_ptr(),
                                                         scales.data_ptr(), y.data_ptr(), m, k, n, group_size,
                                                         int(silu_mul), ws_ptr, ws_len, self._stream(s)),
                       "w4a16_gemm_rmsnorm_stats")
        return y

    def gemm_config(self, x, packed, qzeros, scales, y, k: int, n: int, regime: int, p0: int, p1: int,
                    split: int, workspace: torch.Tensor | None, group_size: int = 128,
                    p2: int = 0, silu_mul: bool = False) -> torch.Tensor:
        m = x.shape[0]
        ws_ptr = workspace.data_ptr() if workspace is not None else None
        ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
        fn = self.dll.w4a16_gemm_silu_mul_config if silu_mul else self.dll.w4a16_gemm_config
        with torch.cuda.device(x.device):
            self.check(fn(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(), y.data_ptr(), m, k,
                          n, group_size, regime, p0, p1, p2, split, ws_ptr, ws_len, self._stream(x)),
                       "w4a16_gemm_silu_mul_config" if silu_mul else "w4a16_gemm_config")
        return y


_LOCK = threading.Lock()
_LIB: W4A16Library | None = None


def lib() -> W4A16Library:
    """The process-wide library handle (loaded on first use; raises if it is not built)."""
    global _LIB
    with _LOCK:
        if _LIB is None:
            _LIB = W4A16Library()
        return _LIB
