"""Checkpoint loading for models built from this package's Linear layers: the caller side
of the W4A16 boundary (the reference's ``llmserve/utils/loader.py:8-61``).

``load_model(model, path)`` reads every ``*.safetensors`` file under ``path`` and hands each
tensor to its parameter's ``weight_loader``.  Checkpoint names that contain a key of
``model.packed_modules_mapping`` (e.g. ``q_proj`` -> ``("qkv_proj", "q")``) are shards of a
fused layer: they are renamed and passed with their shard id, so the AutoAWQ tensors of
q/k/v (or gate/up) land side by side along the packed output dimension.  Afterwards every
parameter must have been written -- each declared shard of a fused parameter included --
or a ``RuntimeError`` names what is missing; then each AWQ module's
``process_weights_after_loading`` runs (the repack into the HIP kernels' layout).

Tensors are read on the host (safetensors, no pickle) and copied into the parameters
wherever the model lives; processing requires the model on a GPU.
"""
from __future__ import annotations

import glob
import os

import torch
from safetensors import safe_open
from torch import nn

__all__ = ("default_weight_loader", "load_model")


def default_weight_loader(param: nn.Parameter, loaded_weight: torch.Tensor) -> None:
    param.data.copy_(loaded_weight)


def _storage_key(param: torch.Tensor) -> tuple[str, int]:
    return str(param.device), param.untyped_storage().data_ptr()


def load_model(model: nn.Module, path: str, *, process_weights: bool = True) -> None:
    """Load ``path/*.safetensors`` into ``model`` (reference loader.py:12-61).

    ``process_weights=False`` stops after the loading and the completeness check (the
    reference always processes; here processing needs GPU tensors, so a model loaded on
    the host is processed after it is moved)."""
    mapping = getattr(model, "packed_modules_mapping", {})
    written: set[int] = set()
    written_storage: set[tuple[str, int]] = set()
    shards_seen: dict[int, set] = {}
    for file in sorted(glob.glob(os.path.join(path, "*.safetensors"))):
        with safe_open(file, "pt", "cpu") as f:
            for name in f.keys():
                fused = next((k for k in mapping if k in name), None)
                if fused is not None:
                    target, shard_id = mapping[fused]
                    param = model.get_parameter(name.replace(fused, target))
                    param.weight_loader(param, f.get_tensor(name), shard_id)
                    shards_seen.setdefault(id(param), set()).add(shard_id)
                else:
                    param = model.get_parameter(name)
                    getattr(param, "weight_loader", default_weight_loader)(param, f.get_tensor(name))
                written.add(id(param))
                written_storage.add(_storage_key(param))

    missing = []
    for name, param in model.named_parameters():
        expected = getattr(param, "expected_shard_ids", None)
        if expected is not None:
            missing += [f"{name}[{sid}]" for sid in expected if sid not in shards_seen.get(id(param), set())]
        elif id(param) not in written and _storage_key(param) not in written_storage:
            missing.append(name)
    if missing:
        raise RuntimeError(f"missing checkpoint parameters or shards: {missing}")

    if process_weights:
        for module in model.modules():
            method = getattr(module, "quant_method", None)
            if method is not None:
                method.process_weights_after_loading(module)
