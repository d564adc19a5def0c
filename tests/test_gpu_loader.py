"""End to end on the GPU: an AutoAWQ safetensors checkpoint with separate q/k/v and gate/up
shards loaded into fused layers (llmserve/utils/loader.py:12-61), processed for the HIP
kernels, and each projection's forward checked against the oracle over that projection's own
shards (tests/test_awq_linear_backend.py:238-367 covers the same path on the reference)."""
import importlib

import numpy as np
import pytest
import torch
from safetensors.torch import save_file
from torch import nn

from oracle import awq_oracle as ora
from awq_helpers import GEMM_REL_TOL, bf16_from_bits, rel_err

pytestmark = pytest.mark.gpu

HIDDEN, HEAD, HEADS, KV_HEADS, INTER = 1024, 128, 8, 2, 2048


def shard(seed, k, n):
    p = ora.make_problem(seed=seed, m=1, k=k, n=n)
    return {"qweight": p["qweight"], "qzeros": p["qzeros"], "scales_bits": p["scales_bits"]}


def to_tensors(prefix, s):
    return {f"{prefix}.qweight": torch.from_numpy(s["qweight"]),
            f"{prefix}.qzeros": torch.from_numpy(s["qzeros"]),
            f"{prefix}.scales": torch.from_numpy(s["scales_bits"].view(np.int16)).view(torch.bfloat16)}


def concat(*shards):
    return {key: np.concatenate([s[key] for s in shards], axis=1) for key in shards[0]}


def test_checkpoint_to_forward_matches_oracle(gpu_lib, tmp_path):
    linear = importlib.import_module("llm-serve_amd.layers.linear")
    awq = importlib.import_module("llm-serve_amd.layers.quantization.awq")
    loader = importlib.import_module("llm-serve_amd.utils.loader")
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)

    class Block(nn.Module):
        packed_modules_mapping = {"q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"),
                                  "v_proj": ("qkv_proj", "v"), "gate_proj": ("gate_up_proj", 0),
                                  "up_proj": ("gate_up_proj", 1)}

        def __init__(self):
            super().__init__()
            self.qkv_proj = linear.QKVParallelLinear(HIDDEN, HEAD, HEADS, KV_HEADS, quant_config=cfg)
            self.o_proj = linear.RowParallelLinear(HEADS * HEAD, HIDDEN, quant_config=cfg)
            self.gate_up_proj = linear.MergedColumnParallelLinear(HIDDEN, [INTER, INTER], quant_config=cfg)
            self.down_proj = linear.RowParallelLinear(INTER, HIDDEN, quant_config=cfg)

    shards = {"q_proj": shard(1, HIDDEN, HEADS * HEAD), "k_proj": shard(2, HIDDEN, KV_HEADS * HEAD),
              "v_proj": shard(3, HIDDEN, KV_HEADS * HEAD), "o_proj": shard(4, HEADS * HEAD, HIDDEN),
              "gate_proj": shard(5, HIDDEN, INTER), "up_proj": shard(6, HIDDEN, INTER),
              "down_proj": shard(7, INTER, HIDDEN)}
    first, second = {}, {}
    for i, (name, s) in enumerate(shards.items()):
        (first if i % 2 == 0 else second).update(to_tensors(name, s))
    save_file(first, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file(second, str(tmp_path / "model-00002-of-00002.safetensors"))

    with torch.device("cuda"):
        model = Block()
    loader.load_model(model, str(tmp_path))
    for layer in (model.qkv_proj, model.o_proj, model.gate_up_proj, model.down_proj):
        assert not hasattr(layer, "qweight") and hasattr(layer, "awq_qweight")

    expected = {"qkv_proj": concat(shards["q_proj"], shards["k_proj"], shards["v_proj"]),
                "o_proj": shards["o_proj"], "gate_up_proj": concat(shards["gate_proj"], shards["up_proj"]),
                "down_proj": shards["down_proj"]}
    rng = np.random.default_rng(0)
    for name, s in expected.items():
        layer = getattr(model, name)
        k = s["qweight"].shape[0]
        for m in (1, 16, 300):
            x_bits = ora.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
            print(f"loader forward {name} m={m} k={k}", flush=True)
            y = layer(bf16_from_bits(x_bits))
            want = ora.awq_linear_ref(x_bits, s["qweight"], s["qzeros"], s["scales_bits"], 128)
            assert y.shape == want.shape
            assert rel_err(y, want) <= GEMM_REL_TOL, (name, m)


def test_layer_projections_from_indexed_checkpoint(gpu_lib, tmp_path):
    """benchmarks/awq_linear_profile.py:93-146 path: one layer read through the safetensors
    index, merged q|k|v and gate|up, repacked on the GPU; each GEMM against the oracle; then
    the benchmark's checkpoint leg over the same directory."""
    import json
    import sys

    ckpt = importlib.import_module("llm-serve_amd.utils.checkpoint")
    awq = importlib.import_module("llm-serve_amd.layers.quantization.awq")
    hidden, q, kv, inter = 256, 256, 64, 512
    sizes = {"q_proj": (hidden, q), "k_proj": (hidden, kv), "v_proj": (hidden, kv), "o_proj": (q, hidden),
             "gate_proj": (hidden, inter), "up_proj": (hidden, inter), "down_proj": (inter, hidden)}
    shards, files, weight_map = {}, ({}, {}), {}
    for i, (comp, (k, n)) in enumerate(sizes.items()):
        shards[comp] = shard(40 + i, k, n)
        block = "self_attn" if comp in ("q_proj", "k_proj", "v_proj", "o_proj") else "mlp"
        for name, t in to_tensors(f"model.layers.2.{block}.{comp}", shards[comp]).items():
            files[i % 2][name] = t
            weight_map[name] = f"part{i % 2}.safetensors"
    for j, f in enumerate(files):
        save_file(f, str(tmp_path / f"part{j}.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))

    expected = {"qkv": concat(shards["q_proj"], shards["k_proj"], shards["v_proj"]), "o": shards["o_proj"],
                "gate_up": concat(shards["gate_proj"], shards["up_proj"]), "down": shards["down_proj"]}
    rng = np.random.default_rng(5)
    for proj in ckpt.load_layer_projections(str(tmp_path), layer_id=2):
        s = expected[proj.name]
        assert np.array_equal(proj.qweight.numpy(), s["qweight"]) and np.array_equal(proj.qzeros.numpy(), s["qzeros"])
        dev = proj.to("cuda")
        packed = awq.repack_awq_qweight(dev.qweight)
        for m in (4, 200):
            x_bits = ora.f32_to_bf16_bits(rng.standard_normal((m, proj.input_size)).astype(np.float32))
            print(f"projection {proj.name} m={m}", flush=True)
            y = awq.awq_linear(bf16_from_bits(x_bits), packed, dev.qzeros, dev.scales, group_size=128)
            want = ora.awq_linear_ref(x_bits, s["qweight"], s["qzeros"], s["scales_bits"], 128)
            assert rel_err(y, want) <= GEMM_REL_TOL, (proj.name, m)

    import os
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    if repo not in sys.path:
        sys.path.insert(0, repo)
    bench = importlib.import_module("bench")
    out = bench.checkpoint_layer(gpu_lib, torch.device("cuda"), torch.cuda.Stream(), str(tmp_path), 2, reps=2)
    assert out["layer_id"] == 2
    assert [out["projections"][name]["N"] for name in ("qkv", "o", "gate_up", "down")] == [384, 256, 1024, 256]
    assert all(out["projections"][name]["M=16"]["us"] > 0 for name in out["projections"])
