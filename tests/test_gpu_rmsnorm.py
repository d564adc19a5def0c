"""GPU parity of the RMSNorm(+residual) prologue (w4a16_add_rmsnorm) and of the fused
norm + projection call (w4a16_gemm_rmsnorm) in front of QKV and gate_up.

Bars: the new residual bf16(x + residual) is bit-exact with the oracle; the normalised
activations agree with the oracle bit-exactly on more than 99 % of elements and within two
bf16 ulps everywhere (the kernel sums squares in fp32 in a tree, the oracle in fp64, so
bf16(s * r) can differ by one ulp where s * r lies next to a rounding boundary; the weight
product carries that ulp of bf16(s * r) into up to two ulps of the output when the product
lands in the upper part of a lower binade); the fused call is
bit-identical to the norm followed by the plain (or SiLU * up) GEMM, and within the GEMM
tolerance (max |y - r| / max(|r|, rms(r)) <= 1e-2) of the oracle's GEMM of the oracle's
normalised activations."""
import importlib

import numpy as np
import pytest
import torch

from awq_helpers import GEMM_REL_TOL, QWEN3_SHAPES, awq_mod, bf16_from_bits, bits_of, random_awq_gpu, rel_err
from oracle import awq_oracle as ora

pytestmark = pytest.mark.gpu

EPS = 1e-6


def rand_bits(shape, seed, scale=1.0, offset=0.0):
    rng = np.random.default_rng(seed)
    return ora.f32_to_bf16_bits((offset + scale * rng.standard_normal(shape)).astype(np.float32))


def ulp_diff(a_bits, b_bits):
    return np.abs(a_bits.view(np.int16).astype(np.int32) - b_bits.view(np.int16).astype(np.int32))


@pytest.mark.parametrize("with_res", [True, False])
@pytest.mark.parametrize("m,k", [(1, 4096), (5, 4096), (64, 128), (300, 136), (3, 16384), (17, 5120), (2048, 4096)])
def test_add_rmsnorm_matches_oracle(gpu_lib, m, k, with_res):
    x_bits = rand_bits((m, k), seed=m * 7 + k, scale=2.0)
    r_bits = rand_bits((m, k), seed=m * 11 + k, scale=3.0) if with_res else None
    w_bits = rand_bits((k,), seed=k, scale=0.2, offset=1.0)
    print(f"add_rmsnorm m={m} k={k} residual={with_res}", flush=True)
    want, want_res, _ = ora.add_rms_norm_ref(x_bits, r_bits, w_bits, EPS)
    awq = awq_mod()
    x, w = bf16_from_bits(x_bits), bf16_from_bits(w_bits)
    if with_res:
        res = bf16_from_bits(r_bits)
        out, res_out = awq.add_rms_norm(x, res, w, EPS)
        assert np.array_equal(bits_of(res_out), want_res)
        assert np.array_equal(bits_of(res), r_bits)  # the input residual is not modified
    else:
        out = awq.add_rms_norm(x, None, w, EPS)
    d = ulp_diff(bits_of(out), want)
    assert d.max() <= 2 and (d == 0).mean() > 0.99, (d.max(), (d == 0).mean())
    assert np.array_equal(bits_of(x), x_bits)


def test_add_rmsnorm_special_rows(gpu_lib):
    """A constant row normalises to +-1 (times the weight), an all-zero row to zeros, and a
    row of 1e-4 to 1e-4 / sqrt(1e-8 + eps) -- the same closed forms the oracle is pinned on."""
    k = 4096
    rows = np.stack([np.full(k, 2.0), np.full(k, -0.5), np.zeros(k), np.full(k, 1e-4)]).astype(np.float32)
    x_bits = ora.f32_to_bf16_bits(rows)
    w_bits = ora.f32_to_bf16_bits(np.full(k, 2.0, np.float32))
    out = awq_mod().add_rms_norm(bf16_from_bits(x_bits), None, bf16_from_bits(w_bits), EPS)
    got = ora.bf16_bits_to_f32(bits_of(out))
    assert np.all(got[0] == 2.0) and np.all(got[1] == -2.0) and np.all(got[2] == 0.0)
    x4 = float(ora.bf16_bits_to_f32(x_bits[3, :1])[0])
    assert np.allclose(got[3], 2 * x4 / np.sqrt(x4 * x4 + EPS), rtol=2 ** -8)


def test_add_rmsnorm_in_place(gpu_lib):
    """residual_out may be the residual itself and the normalised output may replace x."""
    m, k = 33, 4096
    awq = awq_mod()
    x = bf16_from_bits(rand_bits((m, k), seed=1))
    res = bf16_from_bits(rand_bits((m, k), seed=2))
    w = bf16_from_bits(rand_bits((k,), seed=3, scale=0.1, offset=1.0))
    want, want_res = awq.add_rms_norm(x, res, w, EPS)
    awq.add_rms_norm(x, res, w, EPS, residual_out=res)
    assert torch.equal(res.view(torch.int16), want_res.view(torch.int16))
    ref = awq.add_rms_norm(x, None, w, EPS)
    awq.lib().add_rmsnorm(x, None, w, EPS, x, None)  # x_norm == x, no residual
    assert torch.equal(x.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("shape,silu", [("qkv", False), ("gate_up", True), ("gate_up", False)])
def test_fused_norm_gemm_equals_norm_then_gemm(gpu_lib, shape, silu):
    """Every regime (decode without / with a K split, the tile kernel) at the real shapes."""
    k, n = QWEN3_SHAPES[shape]
    awq = awq_mod()
    qw, qz, s = random_awq_gpu(k, n, seed=71)
    packed = awq.repack_awq_qweight(qw)
    w = bf16_from_bits(rand_bits((k,), seed=5, scale=0.1, offset=1.0))
    for m in (1, 4, 16, 33, 64, 300, 2048):
        print(f"gemm_rmsnorm {shape} silu={silu} m={m}", flush=True)
        x = bf16_from_bits(rand_bits((m, k), seed=m))
        res = bf16_from_bits(rand_bits((m, k), seed=m + 1, scale=4.0))
        y, res_out = awq.awq_linear_rmsnorm(x, res, w, EPS, packed, qz, s, group_size=128, silu_mul=silu)
        xn, want_res = awq.add_rms_norm(x, res, w, EPS)
        plain = (awq.awq_linear_silu_mul if silu else awq.awq_linear)(xn, packed, qz, s, group_size=128)
        assert y.shape == plain.shape
        assert torch.equal(y.view(torch.int16), plain.view(torch.int16)), m
        assert torch.equal(res_out.view(torch.int16), want_res.view(torch.int16)), m


@pytest.mark.parametrize("m", [1, 16, 200])
def test_fused_norm_gemm_matches_oracle(gpu_lib, m):
    """Against the oracle end to end: the oracle's add_rms_forward, then its fp64 GEMM."""
    k, n = 1024, 512
    p = ora.make_problem(seed=950 + m, m=m, k=k, n=n)
    r_bits = rand_bits((m, k), seed=m, scale=2.0)
    w_bits = rand_bits((k,), seed=k, scale=0.2, offset=1.0)
    xn_bits, res_bits, _ = ora.add_rms_norm_ref(p["x_bits"], r_bits, w_bits, EPS)
    want = ora.awq_linear_ref(xn_bits, p["qweight"], p["qzeros"], p["scales_bits"], 128)
    awq = awq_mod()
    qw = torch.from_numpy(p["qweight"]).cuda()
    qz = torch.from_numpy(p["qzeros"]).cuda()
    s = bf16_from_bits(p["scales_bits"])
    y, res_out = awq.awq_linear_rmsnorm(bf16_from_bits(p["x_bits"]), bf16_from_bits(r_bits), bf16_from_bits(w_bits),
                                        EPS, awq.repack_awq_qweight(qw), qz, s, group_size=128)
    assert np.array_equal(bits_of(res_out), res_bits)
    assert rel_err(y, want) <= GEMM_REL_TOL


def test_layer_api_with_rmsnorm_module(gpu_lib):
    linear = importlib.import_module("llm-serve_amd.layers.linear")
    layernorm = importlib.import_module("llm-serve_amd.layers.layernorm")
    awq = awq_mod()
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    k, inter = 1024, 768
    with torch.device("cuda"):
        gate_up = linear.MergedColumnParallelLinear(k, [inter, inter], quant_config=cfg)
        norm = layernorm.RMSNorm(k, eps=EPS)
    qw, qz, s = random_awq_gpu(k, 2 * inter, seed=12)
    for name, t in (("qweight", qw), ("qzeros", qz), ("scales", s)):
        param = getattr(gate_up, name)
        half = t.shape[1] // 2
        param.weight_loader(param, t[:, :half], 0)
        param.weight_loader(param, t[:, half:], 1)
    gate_up.quant_method.process_weights_after_loading(gate_up)
    norm.weight.copy_(bf16_from_bits(rand_bits((k,), seed=8, scale=0.1, offset=1.0)))
    x = bf16_from_bits(rand_bits((6, k), seed=9)).view(2, 3, k)
    res = bf16_from_bits(rand_bits((6, k), seed=10)).view(2, 3, k)
    y, new_res = gate_up.forward_rmsnorm_silu_and_mul(norm, x, res)
    xn, want_res = norm(x, res)
    assert y.shape == (2, 3, inter) and new_res.shape == (2, 3, k)
    assert torch.equal(y.view(torch.int16), gate_up.forward_silu_and_mul(xn).view(torch.int16))
    assert torch.equal(new_res.view(torch.int16), want_res.view(torch.int16))
    y2, none = gate_up.forward_rmsnorm(norm, x)
    assert none is None
    assert torch.equal(y2.view(torch.int16), gate_up(norm(x)).view(torch.int16))
    with pytest.raises(ValueError, match="weight must have shape"):
        awq.add_rms_norm(x, None, norm.weight[:-8], EPS)
    with pytest.raises(ValueError, match="residual must have"):
        norm(x, res[:1].contiguous())
