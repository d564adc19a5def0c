"""GPU parity of the GEMM with the residual add in its epilogue (w4a16_gemm_residual):
y = bf16(bf16(x @ W) + residual), the order of the reference's add_rms_forward
(layernorm.py:35-36) applied to the O / down output (qwen3.py:170-174).

Reference: the oracle's fp64 GEMM rounded to bf16, plus the residual in fp64, rounded to
bf16 -- compared with the GEMM tolerance (max |y - r| / max(|r|, rms(r)) <= 1e-2): the only
differences are the GEMM's fp32 summation order and its effect on the first rounding."""
import importlib

import numpy as np
import pytest
import torch

from awq_helpers import (GEMM_REL_TOL, QWEN3_SHAPES, awq_mod, bf16_from_bits, random_awq_gpu,
                         random_x_gpu, rel_err, to_gpu)
from oracle import awq_oracle as ora

pytestmark = pytest.mark.gpu


def oracle_residual(p, res_bits):
    y = ora.awq_linear_ref(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128)
    y_bf16 = ora.bf16_bits_to_f32(ora.f32_to_bf16_bits(y.astype(np.float32))).astype(np.float64)
    return y_bf16 + ora.bf16_bits_to_f32(res_bits).astype(np.float64)


@pytest.mark.parametrize("m", [1, 5, 16, 33, 64, 65, 200, 513])
def test_residual_matches_oracle_on_every_path(gpu_lib, m):
    """K = 1024, N = 512: decode without and with a K split (M <= 16 and 17..64) and the
    tile kernel without and with a K split (M > 64)."""
    k, n = 1024, 512
    p = ora.make_problem(seed=900 + m, m=m, k=k, n=n)
    res_bits = ora.f32_to_bf16_bits(np.random.default_rng(m).standard_normal((m, n)).astype(np.float32) * 4)
    t = to_gpu(p)
    awq = awq_mod()
    packed = awq.repack_awq_qweight(t["qweight"])
    res = bf16_from_bits(res_bits)
    print(f"residual m={m} regime={gpu_lib.regime(m, k, n)} split={gpu_lib.split_k(m, k, n)}", flush=True)
    y = awq.awq_linear_residual(t["x"], packed, t["qzeros"], t["scales"], res, group_size=128)
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    assert torch.equal(res, bf16_from_bits(res_bits))  # the residual is not modified
    assert rel_err(y, oracle_residual(p, res_bits)) <= GEMM_REL_TOL
    # The epilogue is exactly "round the GEMM, then add": against the plain GEMM's output
    # plus the residual, rounded once, the result is bit-identical.
    plain = awq.awq_linear(t["x"], packed, t["qzeros"], t["scales"], group_size=128)
    want = (plain.float() + res.float()).to(torch.bfloat16)
    assert torch.equal(y.view(torch.int16), want.view(torch.int16))


def test_in_place_update_equals_out_of_place(gpu_lib):
    k, n, m = 2048, 1024, 16
    qw, qz, s = random_awq_gpu(k, n, seed=3)
    awq = awq_mod()
    packed = awq.repack_awq_qweight(qw)
    x = random_x_gpu(m, k, seed=4)
    for mm in (m, 300):
        xx = random_x_gpu(mm, k, seed=mm)
        res = random_x_gpu(mm, n, seed=mm + 1)
        fresh = awq.awq_linear_residual(xx, packed, qz, s, res, group_size=128)
        inplace = res.clone()
        out = awq.awq_linear_residual(xx, packed, qz, s, inplace, group_size=128, out=inplace)
        assert out.data_ptr() == inplace.data_ptr()
        assert torch.equal(inplace.view(torch.int16), fresh.view(torch.int16)), mm
    del x


RESIDUAL_TOL = 2e-2


@pytest.mark.parametrize("shape", ["o", "down"])
def test_full_qwen3_shapes(gpu_lib, shape):
    """At the O and down shapes the result is bit-identical to the plain GEMM (itself
    checked against the reference at these shapes) plus the residual, rounded once.
    Against torch's fp32 GEMM plus the residual the bound is RESIDUAL_TOL = 2e-2: the GEMM
    is rounded to bf16 before the add (the reference's order), so where a different
    summation order flips that rounding by one bf16 ulp (2^-8 of the GEMM value) and the
    residual cancels part of it, the difference reaches about 1.2e-2 of the sum's rms."""
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=61)
    awq = awq_mod()
    packed = awq.repack_awq_qweight(qw)
    w = awq.dequantize_awq_gemm(qw, qz, s, group_size=128).float()
    for m in (1, 16, 64, 2048):
        x = random_x_gpu(m, k, seed=m)
        res = random_x_gpu(m, n, seed=m + 7)
        y = awq.awq_linear_residual(x, packed, qz, s, res, group_size=128)
        plain = awq.awq_linear(x, packed, qz, s, group_size=128)
        assert torch.equal(y.view(torch.int16), (plain.float() + res.float()).to(torch.bfloat16).view(torch.int16))
        want = (x.float() @ w).to(torch.bfloat16).float() + res.float()
        assert rel_err(y, want) <= RESIDUAL_TOL, (m, shape)


def test_row_parallel_forward_residual_and_errors(gpu_lib):
    linear = importlib.import_module("llm-serve_amd.layers.linear")
    awq = awq_mod()
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    k, n = 1024, 256
    qw, qz, s = random_awq_gpu(k, n, seed=9)
    with torch.device("cuda"):
        layer = linear.RowParallelLinear(k, n, quant_config=cfg)
    layer.qweight.weight_loader(layer.qweight, qw)
    layer.qzeros.weight_loader(layer.qzeros, qz)
    layer.scales.weight_loader(layer.scales, s)
    layer.quant_method.process_weights_after_loading(layer)
    x = random_x_gpu(6, k, seed=3).view(2, 3, k)
    res = random_x_gpu(6, n, seed=4).view(2, 3, n)
    y = layer.forward_residual(x, res)
    assert y.shape == (2, 3, n)
    assert torch.equal(y.view(torch.int16), (layer(x).float() + res.float()).to(torch.bfloat16).view(torch.int16))
    with pytest.raises(ValueError, match="shape"):
        layer.forward_residual(x, res[:, :2])
    with pytest.raises(ValueError, match="bfloat16"):
        layer.forward_residual(x, res.float())
