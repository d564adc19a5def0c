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


# ------------------------------------------------------- per-layer projection reader
# Mirrors the reference's tests/test_awq_linear_profile.py:7-56 and the index contract of
# benchmarks/awq_linear_profile.py:93-146.
@pytest.fixture(scope="module")
def ckpt(pkg):
    return importlib.import_module("llm-serve_amd.utils.checkpoint")


def test_merge_projection_tensors_uses_checkpoint_output_dimension(ckpt):
    parts = [(torch.full((128, n // 8), v, dtype=torch.int32), torch.full((1, n // 8), v + 3, dtype=torch.int32),
              torch.full((1, n), v + 6, dtype=torch.bfloat16)) for v, n in ((1, 16), (2, 8), (3, 8))]
    proj = ckpt.merge_projection_tensors("qkv", parts)
    assert proj.name == "qkv"
    assert (proj.qweight.shape, proj.qzeros.shape, proj.scales.shape) == ((128, 4), (1, 4), (1, 32))
    assert (proj.output_size, proj.input_size) == (32, 128)
    assert torch.equal(proj.qweight[:, :2], torch.full((128, 2), 1, dtype=torch.int32))
    assert torch.equal(proj.scales[:, -8:], torch.full((1, 8), 9, dtype=torch.bfloat16))
    assert proj.payload_bytes == 128 * 4 * 4 + 4 * 4 + 32 * 2


def test_merge_projection_tensors_rejects_incompatible_inputs(ckpt):
    first = (torch.zeros((128, 1), dtype=torch.int32), torch.zeros((1, 1), dtype=torch.int32),
             torch.ones((1, 8), dtype=torch.bfloat16))
    second = (torch.zeros((256, 1), dtype=torch.int32), torch.zeros((2, 1), dtype=torch.int32),
              torch.ones((2, 8), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="input/group"):
        ckpt.merge_projection_tensors("invalid", [first, second])
    with pytest.raises(ValueError, match="at least one"):
        ckpt.merge_projection_tensors("empty", [])
    with pytest.raises(ValueError, match="qweight packed output"):
        ckpt.merge_projection_tensors("bad", [(first[0], first[1], torch.ones((1, 16), dtype=torch.bfloat16))])


LAYER_SIZES = {"q_proj": (128, 32), "k_proj": (128, 16), "v_proj": (128, 16), "o_proj": (32, 128),
               "gate_proj": (128, 64), "up_proj": (128, 64), "down_proj": (64, 128)}


def write_indexed_layer(tmp_path, layer_id, drop=None):
    """A two-file checkpoint of one Qwen3 layer with its index; every tensor of component c
    holds the value ``position of c + tensor offset`` so the merge order is visible."""
    import json

    files = ({}, {})
    weight_map = {}
    for i, (comp, (k, n)) in enumerate(LAYER_SIZES.items()):
        block = "self_attn" if comp in ("q_proj", "k_proj", "v_proj", "o_proj") else "mlp"
        prefix = f"model.layers.{layer_id}.{block}.{comp}"
        for key, t in {"qweight": torch.full((k, n // 8), i, dtype=torch.int32),
                       "qzeros": torch.full((k // 32, n // 8), 10 + i, dtype=torch.int32),
                       "scales": torch.full((k // 32, n), 20 + i, dtype=torch.bfloat16)}.items():
            name = f"{prefix}.{key}"
            if name == drop:
                continue
            fname = f"model-0000{1 + i % 2}-of-00002.safetensors"
            files[i % 2][name] = t
            weight_map[name] = fname
    files[0]["model.embed_tokens.weight"] = torch.zeros(4, 4)
    weight_map["model.embed_tokens.weight"] = "model-00001-of-00002.safetensors"
    for j, f in enumerate(files):
        save_file(f, str(tmp_path / f"model-0000{1 + j}-of-00002.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    return str(tmp_path)


def test_load_layer_projections_merges_components_in_order(ckpt, tmp_path):
    projs = ckpt.load_layer_projections(write_indexed_layer(tmp_path, 3), layer_id=3)
    assert [p.name for p in projs] == ["qkv", "o", "gate_up", "down"]
    qkv, o, gate_up, down = projs
    assert qkv.qweight.shape == (128, 8) and qkv.output_size == 64 and qkv.input_size == 128
    assert qkv.qweight[0].tolist() == [0] * 4 + [1] * 2 + [2] * 2
    assert qkv.qzeros[0].tolist() == [10] * 4 + [11] * 2 + [12] * 2
    assert gate_up.scales.shape == (4, 128)
    assert gate_up.scales[0, :64].eq(24).all() and gate_up.scales[0, 64:].eq(25).all()
    assert (o.input_size, o.output_size) == (32, 128)
    assert (down.input_size, down.output_size) == (64, 128)
    assert down.qweight.eq(6).all()


def test_load_layer_projections_reports_missing_tensors(ckpt, tmp_path):
    with pytest.raises(ValueError, match="index.json"):
        ckpt.load_layer_projections(str(tmp_path), layer_id=0)
    path = write_indexed_layer(tmp_path, 0, drop="model.layers.0.mlp.up_proj.scales")
    with pytest.raises(ValueError, match=r"missing AWQ tensors: \['model.layers.0.mlp.up_proj.scales'\]"):
        ckpt.load_layer_projections(path, layer_id=0)
    with pytest.raises(ValueError, match="missing AWQ tensors"):
        ckpt.load_layer_projections(path, layer_id=1)
