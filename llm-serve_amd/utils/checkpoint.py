"""One decoder layer's AWQ projections read straight from a Qwen3 AutoAWQ checkpoint
directory, merged the way the fused layers hold them (the reference's
``benchmarks/awq_linear_profile.py:29-146``).

``load_layer_projections(path, layer_id=i)`` reads ``model.safetensors.index.json``, opens only
the files that hold layer ``i``'s q/k/v/o/gate/up/down tensors, and returns the four GEMM
operands ``qkv``, ``o``, ``gate_up`` and ``down`` as AutoAWQ tensors concatenated along the
packed output dimension (q|k|v, gate|up).  The benchmark runs the kernels on these instead of
synthetic weights when given a checkpoint.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from pathlib import Path

import torch
from safetensors import safe_open

__all__ = ("AWQ_TENSOR_NAMES", "PROJECTION_COMPONENTS", "PROJECTION_NAMES", "AWQProjectionTensors",
           "load_layer_projections", "merge_projection_tensors")

PROJECTION_NAMES = ("qkv", "o", "gate_up", "down")
PROJECTION_COMPONENTS = {"qkv": ("q_proj", "k_proj", "v_proj"), "o": ("o_proj",),
                         "gate_up": ("gate_proj", "up_proj"), "down": ("down_proj",)}
AWQ_TENSOR_NAMES = ("qweight", "qzeros", "scales")
_ATTENTION = frozenset(("q_proj", "k_proj", "v_proj", "o_proj"))


@dataclass(frozen=True)
class AWQProjectionTensors:
    """AutoAWQ operands of one GEMM: qweight ``[K, N/8]``, qzeros ``[K/g, N/8]`` (int32),
    scales ``[K/g, N]`` (reference awq_linear_profile.py:37-64)."""

    name: str
    qweight: torch.Tensor
    qzeros: torch.Tensor
    scales: torch.Tensor

    @property
    def input_size(self) -> int:
        return self.qweight.shape[0]

    @property
    def output_size(self) -> int:
        return self.scales.shape[1]

    @property
    def payload_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.qweight, self.qzeros, self.scales))

    def to(self, device) -> "AWQProjectionTensors":
        return AWQProjectionTensors(self.name, self.qweight.to(device), self.qzeros.to(device),
                                    self.scales.to(device))


def merge_projection_tensors(name: str, parts) -> AWQProjectionTensors:
    """Concatenate ``(qweight, qzeros, scales)`` parts along the output dimension
    (reference awq_linear_profile.py:67-90).  Every part must share K and the group count."""
    parts = list(parts)
    if not parts:
        raise ValueError("projection must contain at least one checkpoint module")
    if len({(qw.shape[0], qz.shape[0], s.shape[0]) for qw, qz, s in parts}) != 1:
        raise ValueError("projection parts must share input/group dimensions")
    qweight, qzeros, scales = (torch.cat([p[i] for p in parts], dim=1) for i in range(3))
    merged = AWQProjectionTensors(name, qweight, qzeros, scales)
    if qweight.shape[1] * 8 != merged.output_size:
        raise ValueError("qweight packed output does not match scales")
    if qzeros.shape[1] * 8 != merged.output_size:
        raise ValueError("qzeros packed output does not match scales")
    return merged


def _module_prefix(layer_id: int, component: str) -> str:
    block = "self_attn" if component in _ATTENTION else "mlp"
    return f"model.layers.{layer_id}.{block}.{component}"


def load_layer_projections(model_path, *, layer_id: int) -> tuple[AWQProjectionTensors, ...]:
    """The four projections of layer ``layer_id``, in ``PROJECTION_NAMES`` order, on the host
    (reference awq_linear_profile.py:93-146; same errors)."""
    model_path = Path(model_path)
    index = model_path / "model.safetensors.index.json"
    if not index.is_file():
        raise ValueError("AWQ profiler requires model.safetensors.index.json")
    weight_map = json.loads(index.read_text(encoding="utf-8")).get("weight_map", {})

    wanted = [f"{_module_prefix(layer_id, c)}.{t}"
              for name in PROJECTION_NAMES for c in PROJECTION_COMPONENTS[name] for t in AWQ_TENSOR_NAMES]
    missing = [key for key in wanted if key not in weight_map]
    if missing:
        raise ValueError(f"checkpoint index is missing AWQ tensors: {missing}")

    by_file: dict[str, list[str]] = {}
    for key in wanted:
        by_file.setdefault(weight_map[key], []).append(key)
    tensors = {}
    for filename, keys in by_file.items():
        with safe_open(str(model_path / filename), framework="pt", device="cpu") as f:
            for key in keys:
                tensors[key] = f.get_tensor(key)

    return tuple(
        merge_projection_tensors(name, [tuple(tensors[f"{_module_prefix(layer_id, c)}.{t}"]
                                              for t in AWQ_TENSOR_NAMES)
                                        for c in PROJECTION_COMPONENTS[name]])
        for name in PROJECTION_NAMES)
