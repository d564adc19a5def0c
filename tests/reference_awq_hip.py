# llmserve/layers/quantization/awq_hip.py -- the "hip" execution backend of AWQLinearMethod:
# binds libw4a16.so (the MI355X W4A16 library, C ABI in include/w4a16.h) with ctypes.
# Load after `import torch`, so the library binds to the HIP runtime torch already loaded.
import ctypes
import os

import torch

_P, _I, _S, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
_lib = ctypes.CDLL(os.environ.get("W4A16_LIB", "libw4a16.so"))
_lib.w4a16_last_error.restype = ctypes.c_char_p
_lib.w4a16_repack_qweight.argtypes = [_P, _P, _I, _I, _P]
_lib.w4a16_workspace_bytes_max.argtypes = [_I, _I, _I, _I]
_lib.w4a16_workspace_bytes_max.restype = _S
_lib.w4a16_gemm.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _S, _P]
_lib.w4a16_gemm_silu_mul.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _S, _P]
_lib.w4a16_gemm_rmsnorm.argtypes = [_P, _P, _P, _F, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _S, _P]

# One split-K workspace per device, shared by every AWQ layer: the kernels of one stream run
# in order, so a single buffer serves all layers; it is sized at load time for the largest M
# the engine packs (Config.max_num_batched_tokens), so no call allocates it (graph capture
# included).  Calls on two streams at once need a buffer each.
_workspaces: dict[int, torch.Tensor] = {}


def _check(rc, what):
    if rc:
        raise RuntimeError(f"{what}: {_lib.w4a16_last_error().decode()}")


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _workspace(device):
    ws = _workspaces.get(device.index)
    return (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)


def reserve_workspace(device, k, n, max_tokens):
    need = _lib.w4a16_workspace_bytes_max(max_tokens, k, n, 128)
    have = _workspaces.get(device.index)
    if need > 0 and (have is None or have.numel() < need):
        _workspaces[device.index] = torch.zeros(need, dtype=torch.uint8, device=device)


def repack_awq_qweight_hip(qweight):  # [K, N/8] int32 -> the kernels' layout, same bytes
    k, n = qweight.shape[0], qweight.shape[1] * 8
    out = torch.empty(k * n // 8, dtype=torch.int32, device=qweight.device)
    _check(_lib.w4a16_repack_qweight(qweight.contiguous().data_ptr(), out.data_ptr(), k, n, _stream()), "repack")
    return out


def process_weights_after_loading_hip(layer, max_tokens=16384):
    """The "hip" branch of AWQLinearMethod.process_weights_after_loading (awq.py:156-181)."""
    qweight = layer.qweight.data
    k, n = qweight.shape[0], qweight.shape[1] * 8
    layer.register_buffer("awq_qweight", repack_awq_qweight_hip(qweight), persistent=False)
    layer.register_buffer("awq_qzeros", layer.qzeros.data.contiguous(), persistent=False)
    delattr(layer, "qweight")
    delattr(layer, "qzeros")
    reserve_workspace(qweight.device, k, n, max_tokens)


def awq_hip_linear(x, layer):
    """The "hip" branch of AWQLinearMethod.apply (awq.py:115-154): y = x @ W."""
    if not hasattr(layer, "awq_qweight"):
        raise RuntimeError("AWQ HIP weights must be processed after checkpoint loading")
    lead, k, n = x.shape[:-1], x.shape[-1], layer.scales.shape[1]
    x2 = x.reshape(-1, k).contiguous()
    y = torch.empty((x2.shape[0], n), dtype=x.dtype, device=x.device)
    ws, ws_bytes = _workspace(x.device)
    _check(_lib.w4a16_gemm(x2.data_ptr(), layer.awq_qweight.data_ptr(), layer.awq_qzeros.data_ptr(),
                           layer.scales.data_ptr(), y.data_ptr(), x2.shape[0], k, n, 128, ws, ws_bytes, _stream()),
           "w4a16_gemm")
    return y.reshape(*lead, n)


def awq_hip_gate_up_silu_mul(x, layer):
    """SiluAndMul()(gate_up_proj(x)) (qwen3.py:126-130) as one kernel: [..., N/2]."""
    lead, k, n = x.shape[:-1], x.shape[-1], layer.scales.shape[1]
    x2 = x.reshape(-1, k).contiguous()
    y = torch.empty((x2.shape[0], n // 2), dtype=x.dtype, device=x.device)
    ws, ws_bytes = _workspace(x.device)
    _check(_lib.w4a16_gemm_silu_mul(x2.data_ptr(), layer.awq_qweight.data_ptr(), layer.awq_qzeros.data_ptr(),
                                    layer.scales.data_ptr(), y.data_ptr(), x2.shape[0], k, n, 128, ws, ws_bytes,
                                    _stream()), "w4a16_gemm_silu_mul")
    return y.reshape(*lead, n // 2)


def awq_hip_rmsnorm_linear(h, residual, norm, layer, silu_mul=False):
    """(layer(norm(h, residual)), new residual) -- input_layernorm + qkv_proj, or
    post_attention_layernorm + gate_up_proj + SiluAndMul (qwen3.py:166-173) -- in one call.
    Without a residual the new residual is h itself, as qwen3.py:166-167 sets it."""
    k, n = h.shape[-1], layer.scales.shape[1]
    h2 = h.reshape(-1, k).contiguous()
    m = h2.shape[0]
    x_norm = torch.empty_like(h2)
    res_out = torch.empty_like(h2) if residual is not None else None
    res_in = residual.reshape(-1, k).contiguous() if residual is not None else None
    y = torch.empty((m, n // 2 if silu_mul else n), dtype=h.dtype, device=h.device)
    ws, ws_bytes = _workspace(h.device)
    _check(_lib.w4a16_gemm_rmsnorm(
        h2.data_ptr(), res_in.data_ptr() if res_in is not None else None, norm.weight.data_ptr(), norm.eps,
        x_norm.data_ptr(), res_out.data_ptr() if res_out is not None else None, layer.awq_qweight.data_ptr(),
        layer.awq_qzeros.data_ptr(), layer.scales.data_ptr(), y.data_ptr(), m, k, n, 128, int(silu_mul), ws,
        ws_bytes, _stream()), "w4a16_gemm_rmsnorm")
    new_res = res_out.reshape(h.shape) if res_out is not None else h
    return y.reshape(*h.shape[:-1], y.shape[-1]), new_res
