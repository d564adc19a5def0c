"""Checkpoint loader on the CPU: AutoAWQ shards merged into fused layers, missing shards and
parameters reported, and processing refused for host tensors.

Mirrors the reference's tests/test_awq_linear_backend.py:272-367 (QKV merge, missing v
shard) and its loader contract (llmserve/utils/loader.py:38-56)."""
import importlib

import pytest
import torch
from safetensors.torch import save_file
from torch import nn


@pytest.fixture(scope="module")
def mods(pkg):
    awq = importlib.import_module("llm-serve_amd.layers.quantization.awq")
    linear = importlib.import_module("llm-serve_amd.layers.linear")
    loader = importlib.import_module("llm-serve_amd.utils.loader")
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    return linear, loader, cfg


QKV_MAPPING = {"q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"), "v_proj": ("qkv_proj", "v")}
QKV_SIZES = {"q": 16, "k": 8, "v": 8}


def qkv_model(linear, cfg, with_o=False):
    class ToyModel(nn.Module):
        packed_modules_mapping = QKV_MAPPING

        def __init__(self):
            super().__init__()
            self.qkv_proj = linear.QKVParallelLinear(hidden_size=128, head_size=8, total_num_heads=2,
                                                     total_num_kv_heads=1, quant_config=cfg)
            if with_o:
                self.o_proj = linear.RowParallelLinear(128, 64, quant_config=cfg)

    return ToyModel()


def awq_shard(out_size, value):
    return {"qweight": torch.full((128, out_size // 8), value, dtype=torch.int32),
            "qzeros": torch.full((1, out_size // 8), value + 3, dtype=torch.int32),
            "scales": torch.full((1, out_size), value + 6, dtype=torch.bfloat16)}


def write(tmp_path, tensors, name="model.safetensors"):
    save_file(tensors, str(tmp_path / name))
    return str(tmp_path)


def test_loader_merges_awq_qkv_shards(mods, tmp_path):
    linear, loader, cfg = mods
    tensors = {}
    for value, sid in enumerate(("q", "k", "v"), start=1):
        for key, t in awq_shard(QKV_SIZES[sid], value).items():
            tensors[f"{sid}_proj.{key}"] = t
    model = qkv_model(linear, cfg)
    loader.load_model(model, write(tmp_path, tensors), process_weights=False)
    for name, base in (("qweight", 1), ("qzeros", 4), ("scales", 7)):
        param = getattr(model.qkv_proj, name)
        parts = [torch.full((param.shape[0], QKV_SIZES[sid] // 8 if name != "scales" else QKV_SIZES[sid]),
                            base + i, dtype=param.dtype) for i, sid in enumerate(("q", "k", "v"))]
        assert torch.equal(param.data, torch.cat(parts, dim=1)), name


def test_loader_reads_every_file_of_a_sharded_checkpoint(mods, tmp_path):
    """q and k in one file, v in another (a checkpoint split into several safetensors)."""
    linear, loader, cfg = mods
    first, second = {}, {}
    for value, sid in enumerate(("q", "k", "v"), start=1):
        dest = second if sid == "v" else first
        for key, t in awq_shard(QKV_SIZES[sid], value).items():
            dest[f"{sid}_proj.{key}"] = t
    save_file(first, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file(second, str(tmp_path / "model-00002-of-00002.safetensors"))
    model = qkv_model(linear, cfg)
    loader.load_model(model, str(tmp_path), process_weights=False)
    assert torch.equal(model.qkv_proj.qweight.data[:, 3:], torch.full((128, 1), 3, dtype=torch.int32))


def test_loader_rejects_missing_awq_v_shard(mods, tmp_path):
    linear, loader, cfg = mods
    tensors = {}
    for value, sid in enumerate(("q", "k"), start=1):
        for key, t in awq_shard(QKV_SIZES[sid], value).items():
            tensors[f"{sid}_proj.{key}"] = t
    with pytest.raises(RuntimeError, match=r"missing.*v"):
        loader.load_model(qkv_model(linear, cfg), write(tmp_path, tensors), process_weights=False)


def test_loader_names_every_missing_shard_and_parameter(mods, tmp_path):
    linear, loader, cfg = mods
    tensors = {f"q_proj.{key}": t for key, t in awq_shard(16, 1).items()}
    tensors["o_proj.qweight"] = torch.zeros((128, 8), dtype=torch.int32)
    with pytest.raises(RuntimeError) as info:
        loader.load_model(qkv_model(linear, cfg, with_o=True), write(tmp_path, tensors), process_weights=False)
    msg = str(info.value)
    assert msg.startswith("missing checkpoint parameters or shards")
    for want in ("qkv_proj.qweight[k]", "qkv_proj.qweight[v]", "qkv_proj.scales[v]", "o_proj.qzeros",
                 "o_proj.scales"):
        assert want in msg
    assert "o_proj.qweight'" not in msg and "qkv_proj.qweight[q]" not in msg


def test_loader_merges_gate_up_by_index(mods, tmp_path):
    linear, loader, cfg = mods

    class Mlp(nn.Module):
        packed_modules_mapping = {"gate_proj": ("gate_up_proj", 0), "up_proj": ("gate_up_proj", 1)}

        def __init__(self):
            super().__init__()
            self.gate_up_proj = linear.MergedColumnParallelLinear(128, [16, 16], quant_config=cfg)
            self.down_proj = linear.RowParallelLinear(128, 16, quant_config=cfg)

    tensors = {}
    for value, name in enumerate(("gate_proj", "up_proj"), start=1):
        for key, t in awq_shard(16, value).items():
            tensors[f"mlp.{name}.{key}"] = t
    for key, t in awq_shard(16, 9).items():
        tensors[f"mlp.down_proj.{key}"] = t

    class Wrapper(nn.Module):
        packed_modules_mapping = Mlp.packed_modules_mapping

        def __init__(self):
            super().__init__()
            self.mlp = Mlp()

    model = Wrapper()
    loader.load_model(model, write(tmp_path, tensors), process_weights=False)
    assert torch.equal(model.mlp.gate_up_proj.scales.data,
                       torch.cat((torch.full((1, 16), 7.0), torch.full((1, 16), 8.0)), 1).to(torch.bfloat16))
    assert torch.equal(model.mlp.down_proj.qzeros.data, torch.full((1, 2), 12, dtype=torch.int32))


def test_loader_refuses_to_process_host_weights(mods, tmp_path):
    """Processing (the repack for the HIP kernels) runs only on GPU tensors: loading a host
    model with processing on fails loudly instead of leaving a CPU path."""
    linear, loader, cfg = mods
    tensors = {}
    for value, sid in enumerate(("q", "k", "v"), start=1):
        for key, t in awq_shard(QKV_SIZES[sid], value).items():
            tensors[f"{sid}_proj.{key}"] = t
    with pytest.raises(ValueError, match="GPU"):
        loader.load_model(qkv_model(linear, cfg), write(tmp_path, tensors))


def test_loader_unknown_checkpoint_name_is_an_error(mods, tmp_path):
    linear, loader, cfg = mods
    with pytest.raises(AttributeError):
        loader.load_model(qkv_model(linear, cfg), write(tmp_path, {"lm_head.weight": torch.zeros(2, 2)}),
                          process_weights=False)
