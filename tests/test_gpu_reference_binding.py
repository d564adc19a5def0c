"""The reference-side binding shown in the integration guide, run exactly as written
(tests/reference_awq_hip.py is that file; tests/test_host_api.py checks that the guide holds
it verbatim): layers processed by its process_weights_after_loading branch reserve the
shared workspace for the engine's largest packed M at load time, so chunked-prefill calls
(down at M = 512, QKV at M = 384, both split-K plans) and a HIP graph capture run without any
allocation, and agree with the reference (fp32 matmul over the oracle-pinned dequant)."""
import importlib
import os

import pytest
import torch
from torch import nn

from awq_helpers import (QWEN3_SHAPES, assert_gemm_close, assert_silu_two_step, awq_mod, random_awq_gpu,
                         random_x_gpu)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def stub(gpu_lib):
    os.environ["W4A16_LIB"] = gpu_lib.path
    return importlib.import_module("reference_awq_hip")


def awq_layer(k, n, seed):
    """A module as AWQLinearMethod.create_weights leaves it (awq.py:76-113), weights loaded."""
    qw, qz, s = random_awq_gpu(k, n, seed=seed)
    layer = nn.Module()
    layer.qweight = nn.Parameter(qw.clone(), requires_grad=False)
    layer.qzeros = nn.Parameter(qz.clone(), requires_grad=False)
    layer.scales = nn.Parameter(s, requires_grad=False)
    return layer, (qw, qz, s)


def reference(x, qw, qz, s):
    return x.float() @ awq_mod().dequantize_awq_gemm(qw, qz, s, group_size=128).float()


@pytest.mark.parametrize("shape,m", [("down", 512), ("qkv", 384), ("o", 1), ("gate_up", 16)])
def test_stub_linear_at_prefill_and_decode_sizes(stub, gpu_lib, shape, m):
    k, n = QWEN3_SHAPES[shape]
    layer, (qw, qz, s) = awq_layer(k, n, seed=400 + m)
    stub.process_weights_after_loading_hip(layer)
    assert not hasattr(layer, "qweight") and hasattr(layer, "awq_qweight")
    ws = stub._workspaces[torch.device("cuda").index or 0]
    assert ws.numel() >= gpu_lib.workspace_bytes(m, k, n)
    x = random_x_gpu(m, k, seed=m, outliers=True)
    print(f"stub {shape} m={m} split={gpu_lib.split_k(m, k, n)}", flush=True)
    assert_gemm_close(stub.awq_hip_linear(x, layer), reference(x, qw, qz, s), (shape, m))


def test_stub_fused_entries(stub, gpu_lib):
    k, n = QWEN3_SHAPES["gate_up"]
    layer, (qw, qz, s) = awq_layer(k, n, seed=31)
    stub.process_weights_after_loading_hip(layer)
    m = 384
    x = random_x_gpu(m, k, seed=3)
    assert_silu_two_step(stub.awq_hip_gate_up_silu_mul(x, layer), x,
                         awq_mod().dequantize_awq_gemm(qw, qz, s, group_size=128).float(), "gate_up silu")

    class Norm:  # RMSNorm's weight and eps (layernorm.py:6-14)
        weight = (1 + 0.1 * random_x_gpu(1, k, seed=4)[0].float()).to(torch.bfloat16)
        eps = 1e-6

    res = random_x_gpu(m, k, seed=5)
    y, new_res = stub.awq_hip_rmsnorm_linear(x, res, Norm, layer, silu_mul=True)
    xn, want_res = awq_mod().add_rms_norm(x, res, Norm.weight, Norm.eps)
    assert torch.equal(new_res.view(torch.int16), want_res.view(torch.int16))
    assert torch.equal(y.view(torch.int16), awq_mod().awq_linear_silu_mul(xn, awq_mod().repack_awq_qweight(qw), qz, s,
                                                                          group_size=128).view(torch.int16))
    y0, first_res = stub.awq_hip_rmsnorm_linear(x, None, Norm, layer)  # first layer: residual = input
    assert first_res is x and y0.shape == (m, n)


def test_stub_graph_capture_allocates_no_workspace(stub, gpu_lib):
    """A decode graph and a chunked-prefill call captured after loading: the workspace
    reserved at load covers them, and replays equal the eager results."""
    k, n = QWEN3_SHAPES["down"]
    layer, _ = awq_layer(k, n, seed=77)
    stub.process_weights_after_loading_hip(layer)
    before = {d: t.data_ptr() for d, t in stub._workspaces.items()}
    xs = [random_x_gpu(m, k, seed=m) for m in (16, 512)]
    eager = [stub.awq_hip_linear(x, layer).clone() for x in xs]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outs = [stub.awq_hip_linear(x, layer) for x in xs]
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16))
    assert {d: t.data_ptr() for d, t in stub._workspaces.items()} == before
