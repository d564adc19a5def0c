"""The reference engine's own CUDA-graph capture loop over the AWQ layers of this package.

``ModelRunner.capture_cudagraph`` (model_runner.py:384-418) runs under inference mode; for
each batch size from the largest down it runs the model once on the current stream
(warm-up), then captures it with ``torch.cuda.graph(graph, self.graph_pool)`` -- no
``stream=`` argument, so torch captures on its own side stream -- and shares the first
graph's memory pool with every later one.  Here the model is one Qwen3-8B decoder layer's
four AWQ projections with both RMSNorms, called through the layer API the reference's
Qwen3 model calls (qwen3.py:166-173, 126-130), loaded and processed on the current stream as
``load_model`` does.  Batch sizes 512, 16 and 1 reach split-K plans on O and down (the
split-K workspace must come from the load-time reservation: capture cannot allocate), and
every replay must reproduce the eager step bit for bit."""
import importlib

import pytest
import torch

from awq_helpers import awq_mod, random_awq_gpu, random_x_gpu

pytestmark = pytest.mark.gpu

HIDDEN, HEAD, HEADS, KV_HEADS, INTER = 4096, 128, 32, 8, 12288
GRAPH_BS = (512, 16, 1)  # largest first, as model_runner.py:395 iterates reversed(graph_bs)


def _layer():
    linear = importlib.import_module("llm-serve_amd.layers.linear")
    layernorm = importlib.import_module("llm-serve_amd.layers.layernorm")
    awq = awq_mod()
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    with torch.device("cuda"):
        mods = dict(qkv=linear.QKVParallelLinear(HIDDEN, HEAD, HEADS, KV_HEADS, quant_config=cfg),
                    o=linear.RowParallelLinear(HEADS * HEAD, HIDDEN, quant_config=cfg),
                    gate_up=linear.MergedColumnParallelLinear(HIDDEN, [INTER, INTER], quant_config=cfg),
                    down=linear.RowParallelLinear(INTER, HIDDEN, quant_config=cfg),
                    norm1=layernorm.RMSNorm(HIDDEN), norm2=layernorm.RMSNorm(HIDDEN))
    for i, name in enumerate(("qkv", "o", "gate_up", "down")):
        layer = mods[name]
        qw, qz, s = random_awq_gpu(layer.qweight.shape[0], layer.scales.shape[1], seed=400 + i)
        layer.qweight.data.copy_(qw)
        layer.qzeros.data.copy_(qz)
        layer.scales.data.copy_(s)
        layer.quant_method.process_weights_after_loading(layer)  # on the current stream
    mods["norm1"].weight.copy_((1 + 0.1 * random_x_gpu(1, HIDDEN, seed=41)[0].float()).to(torch.bfloat16))
    mods["norm2"].weight.copy_((1 + 0.1 * random_x_gpu(1, HIDDEN, seed=42)[0].float()).to(torch.bfloat16))
    return mods


def _model(mods, h, res):
    """input_layernorm + qkv_proj, o_proj, post_attention_layernorm + gate_up_proj + SiluAndMul,
    down_proj (qwen3.py:166-173); attention is out of scope, so O reads the q columns."""
    q, res = mods["qkv"].forward_rmsnorm(mods["norm1"], h, res)
    a = mods["o"](q[:, : HEADS * HEAD].contiguous())
    x, res = mods["gate_up"].forward_rmsnorm_silu_and_mul(mods["norm2"], a, res)
    return mods["down"](x), res


@torch.inference_mode()
def test_reference_capture_loop_without_capture_stream(gpu_lib):
    awq = awq_mod()
    mods = _layer()
    dev = torch.device("cuda")
    # the reservation made at load covers every batch size the loop captures
    need = max(gpu_lib.workspace_bytes(bs, *shape) for bs in GRAPH_BS
               for shape in ((HIDDEN, 6144), (HIDDEN, HIDDEN), (HIDDEN, 2 * INTER), (INTER, HIDDEN)))
    assert need > 0, "some batch size must take a split-K plan, or this test checks nothing"
    assert awq.WORKSPACE.reserved_bytes(dev) >= need

    max_bs = max(GRAPH_BS)
    h_in = random_x_gpu(max_bs, HIDDEN, seed=1)
    res_in = random_x_gpu(max_bs, HIDDEN, seed=2)
    out_h = torch.zeros(max_bs, HIDDEN, dtype=torch.bfloat16, device=dev)
    out_res = torch.zeros(max_bs, HIDDEN, dtype=torch.bfloat16, device=dev)
    graphs, pool = {}, None
    for bs in GRAPH_BS:
        graph = torch.cuda.CUDAGraph()
        o_h, o_r = _model(mods, h_in[:bs], res_in[:bs])  # warm-up on the current stream
        out_h[:bs], out_res[:bs] = o_h, o_r
        print(f"engine-pattern capture bs={bs}", flush=True)
        with torch.cuda.graph(graph, pool):  # no stream=: torch's capture stream
            o_h, o_r = _model(mods, h_in[:bs], res_in[:bs])
            out_h[:bs], out_res[:bs] = o_h, o_r
        if pool is None:
            pool = graph.pool()
        graphs[bs] = graph
        torch.cuda.synchronize()

    for rep in range(2):
        for bs in GRAPH_BS:
            h_in[:bs].copy_(random_x_gpu(bs, HIDDEN, seed=10 * bs + rep))
            res_in[:bs].copy_(random_x_gpu(bs, HIDDEN, seed=10 * bs + rep + 5))
            want_h, want_res = (t.clone() for t in _model(mods, h_in[:bs], res_in[:bs]))  # eager, between replays
            torch.cuda.synchronize()
            graphs[bs].replay()
            torch.cuda.synchronize()
            assert torch.equal(out_h[:bs].view(torch.int16), want_h.view(torch.int16)), (bs, rep)
            assert torch.equal(out_res[:bs].view(torch.int16), want_res.view(torch.int16)), (bs, rep)
    assert torch.isfinite(out_h.float()).all()
