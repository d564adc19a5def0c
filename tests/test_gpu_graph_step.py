"""A whole decode step of one Qwen3-8B decoder layer's projections captured as one HIP graph
through the layer API: QKV, O with the residual add, gate|up with the fused SiLU * up, down
with the residual add -- the four AWQ GEMMs
the reference runs per layer (qwen3.py:126-130, 168-173) and cannot capture with AWQ
(config.py:58-59, model_runner.py:342).  Replays with eager work in between must reproduce
the eager outputs bit for bit; the split-K workspace is warmed on the capture stream first,
so nothing is allocated during capture."""
import importlib

import pytest
import torch

from awq_helpers import awq_mod, random_awq_gpu, random_x_gpu

pytestmark = pytest.mark.gpu

HIDDEN, HEAD, HEADS, KV_HEADS, INTER = 4096, 128, 32, 8, 12288


def load_random(layer, seed):
    k = layer.qweight.shape[0]
    n = layer.scales.shape[1]
    qw, qz, s = random_awq_gpu(k, n, seed=seed)
    layer.qweight.data.copy_(qw)
    layer.qzeros.data.copy_(qz)
    layer.scales.data.copy_(s)
    layer.quant_method.process_weights_after_loading(layer)


@pytest.mark.parametrize("m", [1, 8, 40])
def test_decoder_layer_projections_capture_and_replay(gpu_lib, m):
    linear = importlib.import_module("llm-serve_amd.layers.linear")
    awq = awq_mod()
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    with torch.device("cuda"):
        qkv = linear.QKVParallelLinear(HIDDEN, HEAD, HEADS, KV_HEADS, quant_config=cfg)
        o = linear.RowParallelLinear(HEADS * HEAD, HIDDEN, quant_config=cfg)
        gate_up = linear.MergedColumnParallelLinear(HIDDEN, [INTER, INTER], quant_config=cfg)
        down = linear.RowParallelLinear(INTER, HIDDEN, quant_config=cfg)
    for i, layer in enumerate((qkv, o, gate_up, down)):
        load_random(layer, 90 + i)

    def step(x):
        q = qkv(x)[:, : HEADS * HEAD]
        h = o.forward_residual(q.contiguous(), x)  # residual update in the O epilogue
        return down.forward_residual(gate_up.forward_silu_and_mul(h), h)

    x = random_x_gpu(m, HIDDEN, seed=m)
    eager = step(x).clone()
    static_x = x.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step(static_x)  # sizes the split-K workspace of the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    print(f"capture decoder-layer step m={m}", flush=True)
    with torch.cuda.graph(graph, stream=stream):
        static_y = step(static_x)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_y.view(torch.int16), eager.view(torch.int16)), i
        step(random_x_gpu(m, HIDDEN, seed=100 + i))  # eager work on the same layers in between
        torch.cuda.synchronize()
    # a new input through the same graph
    static_x.copy_(random_x_gpu(m, HIDDEN, seed=7))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(static_y.view(torch.int16), step(static_x).view(torch.int16))


@pytest.mark.parametrize("m", [1, 8, 40, 300])
def test_decoder_layer_with_norms_capture_and_replay(gpu_lib, m):
    """The same layer in the reference's order with both RMSNorms (qwen3.py:166-173,
    layernorm.py:28-40): input_layernorm(h, residual) + QKV and post_attention_layernorm +
    gate|up + SiLU * up as fused norm calls, O and down plain; two outputs (hidden, residual)
    reproduced bit for bit by every replay."""
    linear = importlib.import_module("llm-serve_amd.layers.linear")
    layernorm = importlib.import_module("llm-serve_amd.layers.layernorm")
    awq = awq_mod()
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    with torch.device("cuda"):
        qkv = linear.QKVParallelLinear(HIDDEN, HEAD, HEADS, KV_HEADS, quant_config=cfg)
        o = linear.RowParallelLinear(HEADS * HEAD, HIDDEN, quant_config=cfg)
        gate_up = linear.MergedColumnParallelLinear(HIDDEN, [INTER, INTER], quant_config=cfg)
        down = linear.RowParallelLinear(INTER, HIDDEN, quant_config=cfg)
        norm1, norm2 = layernorm.RMSNorm(HIDDEN), layernorm.RMSNorm(HIDDEN)
    for i, layer in enumerate((qkv, o, gate_up, down)):
        load_random(layer, 190 + i)
    norm1.weight.copy_((1 + 0.1 * random_x_gpu(1, HIDDEN, seed=5)[0].float()).to(torch.bfloat16))
    norm2.weight.copy_((1 + 0.1 * random_x_gpu(1, HIDDEN, seed=6)[0].float()).to(torch.bfloat16))

    def step(h, res):
        q, res = qkv.forward_rmsnorm(norm1, h, res)
        a = o(q[:, : HEADS * HEAD].contiguous())
        x, res = gate_up.forward_rmsnorm_silu_and_mul(norm2, a, res)
        return down(x), res

    h, res = random_x_gpu(m, HIDDEN, seed=m), random_x_gpu(m, HIDDEN, seed=m + 1)
    eager_h, eager_res = (t.clone() for t in step(h, res))
    static_h, static_res = h.clone(), res.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step(static_h, static_res)  # sizes the split-K workspace of the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    print(f"capture decoder-layer step with norms m={m}", flush=True)
    with torch.cuda.graph(graph, stream=stream):
        out_h, out_res = step(static_h, static_res)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_h.view(torch.int16), eager_h.view(torch.int16)), i
        assert torch.equal(out_res.view(torch.int16), eager_res.view(torch.int16)), i
        step(random_x_gpu(m, HIDDEN, seed=200 + i), random_x_gpu(m, HIDDEN, seed=300 + i))
        torch.cuda.synchronize()
