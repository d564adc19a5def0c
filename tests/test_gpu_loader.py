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
