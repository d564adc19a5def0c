"""Host-side behaviour of the reference operator interface, on the CPU (no kernel launch).

Mirrors the reference's own CPU tests: tests/test_awq_reference.py:19-99 (config),
tests/test_awq_linear_backend.py:48-123, 209-236 (parameters, packed loaders, TP and shard
contracts) and the error contract of awq.py:203-232, 259-268."""
import importlib
from dataclasses import replace
from types import SimpleNamespace
from unittest.mock import patch

import numpy as np
import pytest
import torch

from oracle import awq_oracle as ora


@pytest.fixture(scope="module")
def awq(pkg):
    import importlib

    return importlib.import_module("llm-serve_amd.layers.quantization.awq")


@pytest.fixture(scope="module")
def linear(pkg):
    import importlib

    return importlib.import_module("llm-serve_amd.layers.linear")


def make_config(awq):
    return awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                                activation_dtype=torch.bfloat16)


BASE_QCFG = {"quant_method": "awq", "backend": "autoawq", "bits": 4, "group_size": 128, "version": "gemm",
             "zero_point": True}


def test_from_hf_config_accepts_the_pinned_format(awq):
    cfg = awq.AWQRuntimeConfig.from_hf_config(
        SimpleNamespace(dtype=torch.bfloat16, quantization_config=dict(BASE_QCFG, do_fuse=False)))
    assert (cfg.bits, cfg.group_size, cfg.pack_factor, cfg.zero_point, cfg.version, cfg.backend) == \
        (4, 128, 8, True, "gemm", "autoawq")
    assert cfg.activation_dtype == torch.bfloat16
    assert cfg.execution_backend == "hip"


@pytest.mark.parametrize("field,value", [("quant_method", "gptq"), ("backend", "llm-awq"), ("bits", 8),
                                         ("group_size", 64), ("version", "gemv"), ("zero_point", False)])
def test_from_hf_config_rejects_unsupported_layouts(awq, field, value):
    qc = dict(BASE_QCFG)
    qc[field] = value
    with pytest.raises(ValueError, match=field):
        awq.AWQRuntimeConfig.from_hf_config(SimpleNamespace(quantization_config=qc))


def test_from_hf_config_requires_metadata_and_bf16(awq):
    with pytest.raises(ValueError, match="quantization_config"):
        awq.AWQRuntimeConfig.from_hf_config(SimpleNamespace())
    with pytest.raises(ValueError, match="dtype"):
        awq.AWQRuntimeConfig.from_hf_config(SimpleNamespace(dtype=torch.float16, quantization_config=BASE_QCFG))


def test_only_the_hip_backend_exists(awq):
    with pytest.raises(ValueError, match="execution_backend"):
        awq.AWQLinearMethod(replace(make_config(awq), execution_backend="cuda"))


def test_column_linear_creates_checkpoint_native_parameters(awq, linear):
    layer = linear.ColumnParallelLinear(128, 16, quant_config=make_config(awq))
    assert not hasattr(layer, "weight")
    assert layer.qweight.shape == (128, 2) and layer.qweight.dtype == torch.int32
    assert layer.qzeros.shape == (1, 2) and layer.qzeros.dtype == torch.int32
    assert layer.scales.shape == (1, 16) and layer.scales.dtype == torch.bfloat16
    assert not layer.qweight.requires_grad
    assert layer.qweight.packed_dim == 1 and layer.qweight.pack_factor == 8
    assert layer.scales.output_dim == 1 and layer.scales.input_dim == 0


def test_merged_column_loader_slices_packed_output_dimension(awq, linear):
    layer = linear.MergedColumnParallelLinear(128, [16, 8], quant_config=make_config(awq))
    shapes = {"qweight": [(128, 2), (128, 1)], "qzeros": [(1, 2), (1, 1)], "scales": [(1, 16), (1, 8)]}
    for name, (s0, s1) in shapes.items():
        param = getattr(layer, name)
        first = torch.full(s0, 11, dtype=param.dtype)
        second = torch.full(s1, 22, dtype=param.dtype)
        param.weight_loader(param, first, 0)
        param.weight_loader(param, second, 1)
        assert torch.equal(param.data, torch.cat((first, second), dim=1))


def test_qkv_loader_slices_packed_output_dimension(awq, linear):
    layer = linear.QKVParallelLinear(hidden_size=128, head_size=8, total_num_heads=2, total_num_kv_heads=1,
                                     quant_config=make_config(awq))
    sizes = {"q": 16, "k": 8, "v": 8}
    for name in ("qweight", "qzeros", "scales"):
        param = getattr(layer, name)
        parts = []
        for value, sid in enumerate(("q", "k", "v"), start=1):
            width = sizes[sid] // 8 if name != "scales" else sizes[sid]
            loaded = torch.full((param.shape[0], width), value, dtype=param.dtype)
            param.weight_loader(param, loaded, sid)
            parts.append(loaded)
        assert torch.equal(param.data, torch.cat(parts, dim=1))


def test_row_parallel_loader_copies_full_tensor_at_world_size_one(awq, linear):
    layer = linear.RowParallelLinear(256, 64, quant_config=make_config(awq))
    qw = torch.arange(256 * 8, dtype=torch.int32).view(256, 8)
    layer.qweight.weight_loader(layer.qweight, qw)
    assert torch.equal(layer.qweight.data, qw)


def test_awq_rejects_tensor_parallel_construction(awq, linear):
    with patch.object(linear, "tp_world_size", return_value=2):
        with pytest.raises(ValueError, match="tensor parallel"):
            linear.ColumnParallelLinear(128, 16, quant_config=make_config(awq))


def test_merged_awq_rejects_unpacked_shards(awq, linear):
    with pytest.raises(ValueError, match="shard.*pack_factor"):
        linear.MergedColumnParallelLinear(128, [12, 12], quant_config=make_config(awq))
    with pytest.raises(ValueError, match="shard.*pack_factor"):
        linear.QKVParallelLinear(hidden_size=128, head_size=4, total_num_heads=4, total_num_kv_heads=1,
                                 quant_config=make_config(awq))


def test_create_weights_rejects_bad_sizes_and_bias(awq, linear):
    with pytest.raises(ValueError, match="divisible by group_size"):
        linear.ColumnParallelLinear(100, 16, quant_config=make_config(awq))
    with pytest.raises(ValueError, match="pack_factor"):
        linear.ReplicatedLinear(128, 12, quant_config=make_config(awq))
    with pytest.raises(ValueError, match="bias"):
        linear.ReplicatedLinear(128, 16, bias=True, quant_config=make_config(awq))


def test_apply_before_processing_raises(awq, linear):
    layer = linear.ColumnParallelLinear(128, 64, quant_config=make_config(awq))
    with pytest.raises(RuntimeError, match="processed"):
        layer(torch.zeros((1, 128), dtype=torch.bfloat16))


def test_process_refuses_cpu_weights(awq, linear):
    layer = linear.ColumnParallelLinear(128, 64, quant_config=make_config(awq))
    with pytest.raises(ValueError, match="GPU"):
        layer.quant_method.process_weights_after_loading(layer)


def test_tensor_functions_have_no_cpu_path(awq):
    p = ora.make_problem(seed=1, m=2, k=128, n=64)
    qw = torch.from_numpy(p["qweight"])
    qz = torch.from_numpy(p["qzeros"])
    s = torch.from_numpy(p["scales_bits"].view(np.int16)).view(torch.bfloat16)
    x = torch.from_numpy(p["x_bits"].view(np.int16)).view(torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        awq.dequantize_awq_gemm(qw, qz, s, group_size=128)
    with pytest.raises(ValueError, match="GPU"):
        awq.unpack_awq_int4(qw)
    with pytest.raises(ValueError, match="GPU"):
        awq.repack_awq_qweight(qw)
    with pytest.raises(ValueError, match="GPU"):
        awq.awq_linear(x, qw.flatten(), qz, s, group_size=128)


def test_fused_norm_functions_validate_and_have_no_cpu_path(awq):
    """The RMSNorm split across two GEMMs: no CPU path, and the NormInput contract (fp32 s
    [M, K], ssq [M, K / 16], M <= FUSED_NORM_MAX_M) is checked before any library call."""
    p = ora.make_problem(seed=2, m=2, k=128, n=64)
    qw = torch.from_numpy(p["qweight"]).flatten()
    qz = torch.from_numpy(p["qzeros"])
    s = torch.from_numpy(p["scales_bits"].view(np.int16)).view(torch.bfloat16)
    x = torch.from_numpy(p["x_bits"].view(np.int16)).view(torch.bfloat16)
    res = torch.zeros((2, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        awq.awq_linear_residual_stats(x, qw, qz, s, res, group_size=128)
    w = torch.ones(128, dtype=torch.bfloat16)
    k = 128
    assert awq.FUSED_NORM_MAX_M == 8
    good = awq.NormInput(torch.zeros((2, k)), torch.zeros((2, k // 16)))
    with pytest.raises(ValueError, match="share one GPU"):
        awq.awq_linear_rmsnorm_stats(good, w, 1e-6, qw, qz, s, group_size=128)
    with pytest.raises(ValueError, match="M <= 8"):
        awq.awq_linear_rmsnorm_stats(awq.NormInput(torch.zeros((9, k)), torch.zeros((9, k // 16))), w, 1e-6, qw, qz, s,
                                     group_size=128)
    with pytest.raises(ValueError, match="ssq must be"):
        awq.awq_linear_rmsnorm_stats(awq.NormInput(torch.zeros((2, k)), torch.zeros((2, 4))), w, 1e-6, qw, qz, s,
                                     group_size=128)
    with pytest.raises(ValueError, match="fp32"):
        awq.awq_linear_rmsnorm_stats(awq.NormInput(torch.zeros((2, k), dtype=torch.bfloat16), torch.zeros((2, 8))),
                                     w, 1e-6, qw, qz, s, group_size=128)
    with pytest.raises(ValueError, match="RMSNorm weight"):
        awq.awq_linear_rmsnorm_stats(good, w[:64], 1e-6, qw, qz, s, group_size=128)


def test_validation_messages_match_reference(awq):
    qw = torch.zeros((4, 1), dtype=torch.int32)
    qz = torch.zeros((2, 1), dtype=torch.int32)
    s = torch.ones((2, 8), dtype=torch.bfloat16)
    cases = [((qw.long(), qz, s, 2), "qweight.*int32"), ((qw, qz.long(), s, 2), "qzeros.*int32"),
             ((qw, qz, torch.ones((2, 7), dtype=torch.bfloat16), 2), "scales"),
             ((torch.zeros((5, 1), dtype=torch.int32), qz, s, 2), "divisible")]
    for (a, b, c, g), msg in cases:
        with pytest.raises(ValueError, match=msg):
            awq.dequantize_awq_gemm(a, b, c, group_size=g)


def test_linear_rejects_activation_scale_dtype_mismatch(awq):
    with pytest.raises(ValueError, match="activation dtype"):
        awq.awq_linear(torch.zeros((1, 128), dtype=torch.float16), torch.zeros(16, dtype=torch.int32),
                       torch.zeros((1, 8), dtype=torch.int32), torch.ones((1, 64), dtype=torch.bfloat16),
                       group_size=128)
    with pytest.raises(ValueError, match="floating"):
        awq.awq_linear(torch.zeros((1, 128), dtype=torch.int32), torch.zeros(16, dtype=torch.int32),
                       torch.zeros((1, 8), dtype=torch.int32), torch.ones((1, 64), dtype=torch.bfloat16),
                       group_size=128)


def test_unpack_rejects_bad_input(awq):
    with pytest.raises(ValueError, match="two-dimensional"):
        awq.unpack_awq_int4(torch.zeros(8, dtype=torch.int32))
    with pytest.raises(ValueError, match="int32"):
        awq.unpack_awq_int4(torch.zeros((1, 8), dtype=torch.int64))


# ---------------------------------------------------------------- quantizer contract
@pytest.fixture(scope="module")
def cal(pkg):
    import importlib

    return importlib.import_module("llm-serve_amd.quantization.awq_calibration")


def test_quantizer_rejects_unsupported_shapes(cal):
    """tests/test_awq_quantizer.py:74-87 (same messages), checked before any device work."""
    with pytest.raises(ValueError, match="two-dimensional"):
        cal.quantize_awq_weight(torch.zeros(8), group_size=2)
    with pytest.raises(ValueError, match="floating"):
        cal.quantize_awq_weight(torch.zeros((8, 4), dtype=torch.int32), group_size=2)
    with pytest.raises(ValueError, match="input size"):
        cal.quantize_awq_weight(torch.zeros((8, 5)), group_size=2)
    with pytest.raises(ValueError, match="output size"):
        cal.quantize_awq_weight(torch.zeros((7, 4)), group_size=2)
    with pytest.raises(ValueError, match="positive"):
        cal.quantize_awq_weight(torch.zeros((8, 4)), group_size=0)


def test_quantizer_and_packer_have_no_cpu_path(cal):
    with pytest.raises(ValueError, match="GPU"):
        cal.quantize_awq_weight(torch.zeros((8, 4)), group_size=2)
    with pytest.raises(ValueError, match="GPU"):
        cal.pack_int4(torch.zeros((2, 8), dtype=torch.int32))
    with pytest.raises(ValueError, match="2D"):
        cal.pack_int4(torch.zeros(8, dtype=torch.int32))
    with pytest.raises(ValueError, match="divisible by 8"):
        cal.pack_int4(torch.zeros((2, 6), dtype=torch.int32))
    with pytest.raises(TypeError, match="integer"):
        cal.pack_int4(torch.zeros((2, 8)))


def test_rmsnorm_module_mirrors_the_reference_interface_and_has_no_cpu_path():
    """RMSNorm(hidden_size, eps) with a bf16 weight of ones (layernorm.py:8-15); the compute
    runs only in the HIP library, so a CPU tensor is refused instead of normalised on the host."""
    layernorm = importlib.import_module("llm-serve_amd.layers.layernorm")
    awq = importlib.import_module("llm-serve_amd.layers.quantization.awq")
    norm = layernorm.RMSNorm(64, eps=1e-5)
    assert norm.eps == 1e-5 and norm.weight.shape == (64,) and norm.weight.dtype == torch.bfloat16
    assert torch.equal(norm.weight.float(), torch.ones(64))
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        norm(x)
    with pytest.raises(ValueError, match="GPU"):
        norm(x, x.clone())
    with pytest.raises(ValueError, match="GPU"):
        awq.awq_linear_rmsnorm(x, None, norm.weight, 1e-5, torch.zeros(8, dtype=torch.int32),
                               torch.zeros(1, 8, dtype=torch.int32), torch.zeros(1, 64, dtype=torch.bfloat16),
                               group_size=128)


def test_integration_stub_is_the_tested_file():
    """The integration guide's binding stub is tests/reference_awq_hip.py byte for byte, so
    the code a maintainer copies is the code tests/test_gpu_reference_binding.py runs."""
    import os
    import re

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    doc = open(os.path.join(repo, "INTEGRATION.md")).read()
    m = re.search(r"<!-- stub: tests/reference_awq_hip.py -->\n```python\n(.*?)```\n", doc, flags=re.S)
    assert m, "the integration guide has no stub block"
    assert m.group(1) == open(os.path.join(repo, "tests", "reference_awq_hip.py")).read()


def test_norm_row_strides_of_head_views(awq):
    """Row layout of strided RMSNorm inputs: the per-head views of a split q|k|v output are
    rows at two strides; contiguous leading dimensions merge; anything else is refused."""
    qkv = torch.zeros(5, 6144, dtype=torch.bfloat16)
    q, k, v = qkv.split([4096, 1024, 1024], dim=-1)
    assert awq._row_strides(q.view(-1, 32, 128)) == (32, 6144, 128)
    assert awq._row_strides(k.view(-1, 8, 128)) == (8, 6144, 128)
    assert awq._row_strides(q[:1].view(-1, 32, 128)) == (32, 0, 128)
    assert awq._row_strides(qkv.view(5, 48, 128)) == (240, 0, 128)      # contiguous: one stride
    t = torch.zeros(2, 3, 4, 136, dtype=torch.bfloat16)[:, :, :, :128]
    assert awq._row_strides(t) == (24, 0, 136)                          # padded rows: one stride
    assert awq._row_strides(torch.zeros(2, 3, 4, 136, dtype=torch.bfloat16)[:, 1:, :, :128]) == (8, 1632, 136)
    assert awq._row_strides(torch.zeros(4, 132, dtype=torch.bfloat16)[:, :128]) is None  # rows 8-byte aligned only
    assert awq._row_strides(torch.zeros(4, 128, dtype=torch.bfloat16)[:, ::2]) is None  # inner stride 2
    assert awq._row_strides(torch.zeros(2, 3, 5, 64, dtype=torch.bfloat16).permute(2, 0, 1, 3)) == (6, 64, 320)
    assert awq._row_strides(torch.zeros(2, 3, 5, 64, dtype=torch.bfloat16).permute(0, 2, 1, 3)) is None  # 3 strides


def test_runtime_config_reserves_for_the_engine_batch(awq):
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    assert cfg.max_batched_tokens == 16384  # the reference engine's max_num_batched_tokens (config.py:11)
