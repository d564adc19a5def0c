"""Parity at shapes other than the four Qwen3-8B projections the planner was tuned on.

Tensor-parallel shards -- the per-GPU shapes of the Qwen3-8B projections split eight ways,
QKV and gate_up column-parallel on N, O and down row-parallel on K (linear.py:14-21,
136-146, 178-196, 217-226): QKV 4096 x 768, O 512 x 4096, gate_up 4096 x 3072 and down
1536 x 4096.  One GPU shows the kernels on its share at its real shape; the all-reduce of
the row-parallel outputs lies outside this library.

The chunk sizes reach every plan these shapes take: the decode kernel's small-shape rules
(K split in four below 128 column tiles, unsplit 4-wave workgroups below 16 groups), the
mid-range tiles of 32 columns and four K slices, and the modelled tile choice beyond
M = 128.  Plain GEMMs are checked against the CPU oracle itself (awq.py:235-276, fp64
x @ W over its own dequant), the fused SiLU * up on the gate_up shard against the
reference's two steps.  The norm in front of the QKV and gate_up shards takes the same
paths as at the full shapes (the decode kernel's prologue at M <= 2, the norm kernel before
the GEMM above that, and the norm split across a producer GEMM and the shard's GEMM at
M <= 8), with the same bars (test_gpu_rmsnorm.py, test_gpu_norm_stats.py).

Larger models -- the Qwen3-14B and -32B projections, which take the larger-layer decode
rules and the mid-range cost model (below)."""
import numpy as np
import pytest
import torch

from awq_helpers import (GEMM_REL_TOL, assert_gemm_close, assert_silu_two_step, awq_mod, bf16_from_bits, bits_of, pkg,
                         random_awq_gpu, random_x_gpu, rel_err)
from oracle import awq_oracle as ora

pytestmark = pytest.mark.gpu

TP8_SHAPES = {"qkv": (4096, 768), "o": (512, 4096), "gate_up": (4096, 3072), "down": (1536, 4096)}
MS = (1, 4, 12, 24, 48, 160, 256, 384, 640, 1024, 2048)


@pytest.mark.parametrize("shape", sorted(TP8_SHAPES))
def test_tp8_shard_shapes_against_the_oracle(gpu_lib, shape):
    k, n = TP8_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=31)
    packed = awq_mod().repack_awq_qweight(qw)
    xs = [random_x_gpu(m, k, seed=50 + m, outliers=m >= 1024) for m in MS]
    ys = []
    for m, x in zip(MS, xs):
        print(f"tp8 shard {shape} {k}x{n} m={m} plan={pkg().lib().plan(m, k, n)}", flush=True)
        assert pkg().awq_regime(m, k, n) == ("decode" if m < 32 else "tile")
        ys.append(awq_mod().awq_linear(x, packed, qz, s, group_size=128))
    torch.cuda.synchronize()
    want = ora.awq_linear_ref(np.concatenate([bits_of(x) for x in xs]), qw.cpu().numpy(), qz.cpu().numpy(),
                              bits_of(s), 128)
    r0 = 0
    for m, y in zip(MS, ys):
        assert_gemm_close(y, torch.from_numpy(want[r0:r0 + m]).cuda(), (shape, m))
        r0 += m


@pytest.mark.parametrize("m", [1, 16, 48, 160, 256, 640, 2048])
def test_tp8_gate_up_shard_fused_silu_mul(gpu_lib, m):
    k, n = TP8_SHAPES["gate_up"]
    qw, qz, s = random_awq_gpu(k, n, seed=32)
    awq = awq_mod()
    packed = awq.repack_awq_qweight(qw)
    x = random_x_gpu(m, k, seed=60 + m, outliers=m >= 640)
    print(f"tp8 fused gate_up m={m} plan={pkg().lib().plan(m, k, n, 1)}", flush=True)
    y = awq.awq_linear_silu_mul(x, packed, qz, s, group_size=128)
    assert y.shape == (m, n // 2)
    assert_silu_two_step(y, x, awq.dequantize_awq_gemm(qw, qz, s, group_size=128).float(), ("gate_up/8", m))


EPS = 1e-6


def rand_bits(shape, seed, scale=1.0, offset=0.0):
    rng = np.random.default_rng(seed)
    return ora.f32_to_bf16_bits((offset + scale * rng.standard_normal(shape)).astype(np.float32))


def ulp_diff(a_bits, b_bits):
    return np.abs(a_bits.view(np.int16).astype(np.int32) - b_bits.view(np.int16).astype(np.int32))


@pytest.mark.parametrize("shape,silu", [("qkv", False), ("gate_up", True)])
def test_tp8_fused_norm_gemm_equals_norm_then_gemm(gpu_lib, shape, silu):
    """w4a16_gemm_rmsnorm on the shard: x_norm within two ulps of the oracle (> 99 % exact),
    the new residual bit-exact, the GEMM output bit-identical to the plain GEMM of x_norm."""
    k, n = TP8_SHAPES[shape]
    awq = awq_mod()
    lib = awq.lib()
    qw, qz, s = random_awq_gpu(k, n, seed=33)
    packed = awq.repack_awq_qweight(qw)
    w_bits = rand_bits((k,), seed=34, scale=0.1, offset=1.0)
    w = bf16_from_bits(w_bits)
    for m in (1, 2, 3, 16, 300):
        print(f"tp8 gemm_rmsnorm {shape} silu={silu} m={m} plan={lib.plan(m, k, n, 1 if silu else 0)}", flush=True)
        x_bits, r_bits = rand_bits((m, k), seed=m + 35), rand_bits((m, k), seed=m + 36, scale=4.0)
        x, res = bf16_from_bits(x_bits), bf16_from_bits(r_bits)
        want_xn, want_res, _ = ora.add_rms_norm_ref(x_bits, r_bits, w_bits, EPS)
        ws = torch.zeros(max(lib.workspace_bytes(m, k, n), 256), dtype=torch.uint8, device="cuda")
        xn, res_out = torch.empty_like(x), torch.empty_like(res)
        y = torch.empty((m, n // 2 if silu else n), dtype=torch.bfloat16, device="cuda")
        lib.gemm_rmsnorm(x, res, w, EPS, xn, res_out, packed, qz, s, y, n, ws, silu_mul=silu)
        assert np.array_equal(bits_of(res_out), want_res), m
        d = ulp_diff(bits_of(xn), want_xn)
        assert d.max() <= 2 and (d == 0).mean() > 0.99, (m, d.max(), (d == 0).mean())
        plain = (awq.awq_linear_silu_mul if silu else awq.awq_linear)(xn, packed, qz, s, group_size=128)
        assert torch.equal(y.view(torch.int16), plain.view(torch.int16)), m


@pytest.mark.parametrize("shape,silu", [("qkv", False), ("gate_up", True)])
def test_tp8_norm_split_across_shard_gemms(gpu_lib, shape, silu):
    """The split norm at M <= 8 with the down shard (1536 -> 4096) as the producer and the
    QKV or gate_up shard as the consumer: s and the new residual bit-exact with the plain and
    residual-epilogue GEMMs of the producer, x_norm within two ulps of the oracle's
    add_rms_forward, y within the GEMM tolerance of the plain GEMM of x_norm (> 90 %
    bit-equal) and deterministic."""
    awq = awq_mod()
    k, n = TP8_SHAPES[shape]
    kd, nd = TP8_SHAPES["down"]
    qw, qz, s = random_awq_gpu(k, n, seed=37)
    packed = awq.repack_awq_qweight(qw)
    qwd, qzd, sd = random_awq_gpu(kd, nd, seed=38)
    pd = awq.repack_awq_qweight(qwd)
    w_bits = rand_bits((k,), seed=39, scale=0.1, offset=1.0)
    w = bf16_from_bits(w_bits)
    for m in (1, 2, 3, 5, 8):
        print(f"tp8 norm split {shape} silu={silu} m={m}", flush=True)
        x = bf16_from_bits(rand_bits((m, kd), seed=m + 40))
        res = bf16_from_bits(rand_bits((m, nd), seed=m + 41, scale=4.0))
        inp, res_out = awq.awq_linear_residual_stats(x, pd, qzd, sd, res, group_size=128)
        h = awq.awq_linear(x, pd, qzd, sd, group_size=128)
        assert torch.equal(inp.s.view(torch.int32), (h.float() + res.float()).view(torch.int32)), m
        want_res_epi = awq.awq_linear_residual(x, pd, qzd, sd, res, group_size=128)
        assert torch.equal(res_out.view(torch.int16), want_res_epi.view(torch.int16)), m
        want_xn, want_res, _ = ora.add_rms_norm_ref(bits_of(h), bits_of(res), w_bits, EPS)
        assert np.array_equal(bits_of(res_out), want_res), m
        xn = torch.empty((m, k), dtype=torch.bfloat16, device="cuda")
        y = awq.awq_linear_rmsnorm_stats(inp, w, EPS, packed, qz, s, group_size=128, silu_mul=silu, x_norm=xn)
        d = ulp_diff(bits_of(xn), want_xn)
        assert d.max() <= 2 and (d == 0).mean() > 0.99, (m, d.max(), (d == 0).mean())
        plain = (awq.awq_linear_silu_mul if silu else awq.awq_linear)(xn, packed, qz, s, group_size=128)
        assert rel_err(y, plain.float()) <= GEMM_REL_TOL, m
        assert (bits_of(y) == bits_of(plain)).mean() > 0.9, m
        y2 = awq.awq_linear_rmsnorm_stats(inp, w, EPS, packed, qz, s, group_size=128, silu_mul=silu)
        assert torch.equal(y2.view(torch.int16), y.view(torch.int16)), m


# Layers larger than the tuned Qwen3-8B ones take their own decode rules and a mid-range
# cost model: the Qwen3-14B projections, every plan branch up to M = 512, against an fp32
# GEMM over the library's dequant (bit-exact with the oracle's, test_gpu_format.py) with the
# oracle itself at two row counts of the narrower layers.
Q14_SHAPES = {"qkv": (5120, 7168), "o": (5120, 5120), "gate_up": (5120, 34816), "down": (17408, 5120)}


@pytest.mark.parametrize("shape", sorted(Q14_SHAPES))
def test_larger_model_shapes(gpu_lib, shape):
    k, n = Q14_SHAPES[shape]
    awq = awq_mod()
    qw, qz, s = random_awq_gpu(k, n, seed=41)
    packed = awq.repack_awq_qweight(qw)
    w = awq.dequantize_awq_gemm(qw, qz, s, group_size=128).float()
    for m in (1, 8, 16, 24, 32, 64, 128, 256, 512):
        print(f"larger shape {shape} {k}x{n} m={m} plan={pkg().lib().plan(m, k, n)}", flush=True)
        x = random_x_gpu(m, k, seed=70 + m, outliers=m >= 256)
        y = awq.awq_linear(x, packed, qz, s, group_size=128)
        assert_gemm_close(y, x.float() @ w, (shape, m))
        if shape != "gate_up" and m in (16, 64):
            want = ora.awq_linear_ref(bits_of(x), qw.cpu().numpy(), qz.cpu().numpy(), bits_of(s), 128)
            assert_gemm_close(y, torch.from_numpy(want).cuda(), (shape, m, "oracle"))


Q32_SHAPES = {"qkv": (5120, 10240), "o": (8192, 5120), "gate_up": (5120, 51200), "down": (25600, 5120)}


@pytest.mark.parametrize("shape", sorted(Q32_SHAPES))
def test_larger_model_shapes_32b(gpu_lib, shape):
    """The Qwen3-32B projections through the same larger-layer rules (decode M = 1 .. 24,
    the mid-range model at 64 and 256), against an fp32 GEMM over the library's dequant."""
    k, n = Q32_SHAPES[shape]
    awq = awq_mod()
    qw, qz, s = random_awq_gpu(k, n, seed=42)
    packed = awq.repack_awq_qweight(qw)
    w = awq.dequantize_awq_gemm(qw, qz, s, group_size=128).float()
    for m in (1, 4, 16, 24, 64, 256):
        print(f"larger shape {shape} {k}x{n} m={m} plan={pkg().lib().plan(m, k, n)}", flush=True)
        x = random_x_gpu(m, k, seed=90 + m)
        y = awq.awq_linear(x, packed, qz, s, group_size=128)
        assert_gemm_close(y, x.float() @ w, (shape, m))


@pytest.mark.parametrize("m", [1, 16, 24, 64, 256])
def test_larger_gate_up_fused_silu_mul(gpu_lib, m):
    """The fused SiLU * up on the Qwen3-14B gate_up (5120 x 34816) through the larger-layer
    plans, against the reference's two steps."""
    k, n = Q14_SHAPES["gate_up"]
    awq = awq_mod()
    qw, qz, s = random_awq_gpu(k, n, seed=43)
    packed = awq.repack_awq_qweight(qw)
    x = random_x_gpu(m, k, seed=95 + m)
    print(f"larger fused gate_up m={m} plan={pkg().lib().plan(m, k, n, 1)}", flush=True)
    y = awq.awq_linear_silu_mul(x, packed, qz, s, group_size=128)
    assert_silu_two_step(y, x, awq.dequantize_awq_gemm(qw, qz, s, group_size=128).float(), ("gate_up 14B", m))


def test_larger_qkv_norm_paths(gpu_lib):
    """w4a16_gemm_rmsnorm (prologue at M <= 2, norm kernel + GEMM above) and the split norm
    (O 5120 x 5120 as producer) in front of the Qwen3-14B QKV (5120 x 7168)."""
    awq = awq_mod()
    lib = awq.lib()
    k, n = Q14_SHAPES["qkv"]
    qw, qz, s = random_awq_gpu(k, n, seed=44)
    packed = awq.repack_awq_qweight(qw)
    ko, no = Q14_SHAPES["o"]
    qwo, qzo, so = random_awq_gpu(ko, no, seed=45)
    po = awq.repack_awq_qweight(qwo)
    w_bits = rand_bits((k,), seed=46, scale=0.1, offset=1.0)
    w = bf16_from_bits(w_bits)
    for m in (1, 2, 3, 8, 16, 64):
        print(f"larger qkv norm m={m}", flush=True)
        x_bits, r_bits = rand_bits((m, k), seed=m + 47), rand_bits((m, k), seed=m + 48, scale=4.0)
        x, res = bf16_from_bits(x_bits), bf16_from_bits(r_bits)
        want_xn, want_res, _ = ora.add_rms_norm_ref(x_bits, r_bits, w_bits, EPS)
        ws = torch.zeros(max(lib.workspace_bytes(m, k, n), 256), dtype=torch.uint8, device="cuda")
        xn, res_out = torch.empty_like(x), torch.empty_like(res)
        y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        lib.gemm_rmsnorm(x, res, w, EPS, xn, res_out, packed, qz, s, y, n, ws, silu_mul=False)
        assert np.array_equal(bits_of(res_out), want_res), m
        d = ulp_diff(bits_of(xn), want_xn)
        assert d.max() <= 2 and (d == 0).mean() > 0.99, (m, d.max(), (d == 0).mean())
        assert torch.equal(y.view(torch.int16), awq.awq_linear(xn, packed, qz, s, group_size=128).view(torch.int16)), m
        if m <= 8:
            xo = bf16_from_bits(rand_bits((m, ko), seed=m + 49))
            inp, _ = awq.awq_linear_residual_stats(xo, po, qzo, so, res, group_size=128)
            h = awq.awq_linear(xo, po, qzo, so, group_size=128)
            want_xn2, _, _ = ora.add_rms_norm_ref(bits_of(h), r_bits, w_bits, EPS)
            xn2 = torch.empty((m, k), dtype=torch.bfloat16, device="cuda")
            y2 = awq.awq_linear_rmsnorm_stats(inp, w, EPS, packed, qz, s, group_size=128, x_norm=xn2)
            d2 = ulp_diff(bits_of(xn2), want_xn2)
            assert d2.max() <= 2 and (d2 == 0).mean() > 0.99, (m, d2.max(), (d2 == 0).mean())
            plain = awq.awq_linear(xn2, packed, qz, s, group_size=128)
            assert rel_err(y2, plain.float()) <= GEMM_REL_TOL and (bits_of(y2) == bits_of(plain)).mean() > 0.9, m


Q4_SHAPES = {"qkv": (2560, 6144), "o": (4096, 2560), "gate_up": (2560, 19456), "down": (9728, 2560)}


@pytest.mark.parametrize("shape", sorted(Q4_SHAPES))
def test_smaller_model_shapes_4b(gpu_lib, shape):
    """The Qwen3-4B projections: the 8B rules (QKV, O), the very wide / long-K rules and
    mid-range model (gate_up, down), and the one-round model beyond M = 1024 for the narrow
    ones, against an fp32 GEMM over the library's dequant."""
    k, n = Q4_SHAPES[shape]
    awq = awq_mod()
    qw, qz, s = random_awq_gpu(k, n, seed=46)
    packed = awq.repack_awq_qweight(qw)
    w = awq.dequantize_awq_gemm(qw, qz, s, group_size=128).float()
    for m in (1, 8, 16, 24, 32, 64, 256, 2048):
        print(f"smaller shape {shape} {k}x{n} m={m} plan={pkg().lib().plan(m, k, n)}", flush=True)
        x = random_x_gpu(m, k, seed=110 + m, outliers=m == 2048)
        y = awq.awq_linear(x, packed, qz, s, group_size=128)
        assert_gemm_close(y, x.float() @ w, (shape, m))
