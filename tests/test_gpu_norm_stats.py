"""GPU parity of the RMSNorm split across two decode GEMMs (w4a16_gemm_residual_stats, then
w4a16_gemm_rmsnorm_stats): the O / down projection adds the residual and leaves the fp32 sum
s and its per-tile sums of squares; the next QKV / gate_up projection normalizes s in its
fragment loads (qwen3.py:166-174, layernorm.py:28-40).

Bars: s is bit-exact with float(bf16(h)) + float(residual) for h the plain GEMM output, and
the new residual is bit-exact with the residual-epilogue GEMM (w4a16_gemm_residual); each
tile's sum of squares is within 1e-6 relative of an fp64 sum of the same 16 values; the
normalized activations are within the norm's bar of the oracle's add_rms_forward (two bf16
ulps, > 99 % exact: the kernel sums squares in fp32, the oracle in fp64); the consumer's
output is within the GEMM tolerance of the oracle's fp64 GEMM of those activations and of the
plain GEMM of the returned x_norm (the consumer may run another K split or wave count than the
plain GEMM, so its fp32 sums can round differently in the last bit; > 90 % of outputs are
bit-equal); both calls are deterministic and replay identically from a HIP graph."""
import importlib

import numpy as np
import pytest
import torch

from awq_helpers import GEMM_REL_TOL, QWEN3_SHAPES, awq_mod, bf16_from_bits, bits_of, random_awq_gpu, rel_err
from oracle import awq_oracle as ora

pytestmark = pytest.mark.gpu

EPS = 1e-6
MS = (1, 2, 3, 4, 5, 7, 8)


def rand_bits(shape, seed, scale=1.0, offset=0.0):
    rng = np.random.default_rng(seed)
    return ora.f32_to_bf16_bits((offset + scale * rng.standard_normal(shape)).astype(np.float32))


def ulp_diff(a_bits, b_bits):
    return np.abs(a_bits.view(np.int16).astype(np.int32) - b_bits.view(np.int16).astype(np.int32))


def layer(shape, seed, with_qweight=False):
    awq = awq_mod()
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=seed)
    packed = awq.repack_awq_qweight(qw)
    return (packed, qz, s, qw) if with_qweight else (packed, qz, s)


def check_producer(awq, x, packed, qz, s, res, inp, res_out):
    """s, the new residual and the tile sums of squares against the plain GEMM."""
    m = x.shape[0]
    h = awq.awq_linear(x, packed, qz, s, group_size=128)
    want_s = h.float() + res.float()
    assert torch.equal(inp.s.view(torch.int32), want_s.view(torch.int32)), m
    want_res = awq.awq_linear_residual(x, packed, qz, s, res, group_size=128)
    assert torch.equal(res_out.view(torch.int16), want_res.view(torch.int16)), m
    s64 = inp.s.double().view(m, -1, 16)
    want_ssq = (s64 * s64).sum(-1)
    d = ((inp.ssq.double() - want_ssq).abs() / want_ssq.clamp_min(1e-30)).max().item()
    assert d <= 1e-6, (m, d)
    return h


@pytest.mark.parametrize("shape", ["o", "down"])
def test_residual_stats_producer(gpu_lib, shape):
    """Every decode M of the O and down projections: s, the new residual (also in place) and
    the tile sums of squares."""
    awq = awq_mod()
    k, n = QWEN3_SHAPES[shape]
    packed, qz, s = layer(shape, seed=81)
    for m in MS:
        print(f"residual_stats {shape} m={m}", flush=True)
        x = bf16_from_bits(rand_bits((m, k), seed=m))
        res = bf16_from_bits(rand_bits((m, n), seed=m + 100, scale=3.0))
        inp, res_out = awq.awq_linear_residual_stats(x, packed, qz, s, res, group_size=128)
        assert inp.s.shape == (m, n) and inp.ssq.shape == (m, n // 16) and res_out.shape == (m, n)
        check_producer(awq, x, packed, qz, s, res, inp, res_out)
        inp2, res2 = awq.awq_linear_residual_stats(x, packed, qz, s, res, group_size=128)
        assert torch.equal(inp2.s.view(torch.int32), inp.s.view(torch.int32))
        assert torch.equal(inp2.ssq.view(torch.int32), inp.ssq.view(torch.int32))
        res_in = res.clone()
        inp3, res3 = awq.awq_linear_residual_stats(x, packed, qz, s, res_in, group_size=128, residual_out=res_in)
        assert res3 is res_in and torch.equal(res_in.view(torch.int16), res_out.view(torch.int16))
        assert torch.equal(inp3.ssq.view(torch.int32), inp.ssq.view(torch.int32))


@pytest.mark.parametrize("shape,silu", [("qkv", False), ("gate_up", True), ("gate_up", False)])
def test_rmsnorm_stats_consumer(gpu_lib, shape, silu):
    """The consumer at every decode M of QKV and gate_up (with and without SiLU * up), from a
    producer's NormInput: x_norm against the oracle's add_rms_forward of (h, residual), y
    against the oracle's GEMM of the oracle's x_norm and against the plain GEMM of x_norm."""
    awq = awq_mod()
    k, n = QWEN3_SHAPES[shape]
    packed, qz, s, qw = layer(shape, seed=82, with_qweight=True)
    po, zo, so = layer("o", seed=83)
    w_bits = rand_bits((k,), seed=7, scale=0.1, offset=1.0)
    w = bf16_from_bits(w_bits)
    for m in MS:
        print(f"rmsnorm_stats {shape} silu={silu} m={m}", flush=True)
        x = bf16_from_bits(rand_bits((m, k), seed=m + 200))
        res = bf16_from_bits(rand_bits((m, k), seed=m + 300, scale=4.0))
        inp, res_out = awq.awq_linear_residual_stats(x, po, zo, so, res, group_size=128)
        h = awq.awq_linear(x, po, zo, so, group_size=128)
        want_xn, want_res, _ = ora.add_rms_norm_ref(bits_of(h), bits_of(res), w_bits, EPS)
        assert np.array_equal(bits_of(res_out), want_res)
        xn = torch.empty((m, k), dtype=torch.bfloat16, device="cuda")
        y = awq.awq_linear_rmsnorm_stats(inp, w, EPS, packed, qz, s, group_size=128, silu_mul=silu, x_norm=xn)
        assert y.shape == (m, n // 2 if silu else n)
        d = ulp_diff(bits_of(xn), want_xn)
        assert d.max() <= 2 and (d == 0).mean() > 0.99, (m, d.max(), (d == 0).mean())
        plain = (awq.awq_linear_silu_mul if silu else awq.awq_linear)(xn, packed, qz, s, group_size=128)
        assert rel_err(y, plain.float()) <= GEMM_REL_TOL, m
        assert (bits_of(y) == bits_of(plain)).mean() > 0.9, m
        y2 = awq.awq_linear_rmsnorm_stats(inp, w, EPS, packed, qz, s, group_size=128, silu_mul=silu)
        assert torch.equal(y2.view(torch.int16), y.view(torch.int16)), m
        if not silu and m in (1, 7):
            # the oracle's fp64 GEMM of the oracle's normalized activations (the CPU GEMM at the
            # full QKV shape takes seconds: two row counts)
            want_y = ora.awq_linear_ref(want_xn, qw.cpu().numpy(), qz.cpu().numpy(), bits_of(s), 128)
            assert rel_err(y, want_y) <= GEMM_REL_TOL, m


def test_norm_stats_graph_replay(gpu_lib):
    """Producer then consumer captured in one HIP graph: every replay (with eager work and
    synchronizations between them) equals the eager result bit for bit."""
    awq = awq_mod()
    k, _ = QWEN3_SHAPES["qkv"]
    packed, qz, s = layer("qkv", seed=84)
    po, zo, so = layer("o", seed=85)
    w = bf16_from_bits(rand_bits((k,), seed=8, scale=0.1, offset=1.0))
    m = 8
    x = bf16_from_bits(rand_bits((m, k), seed=1))
    res = bf16_from_bits(rand_bits((m, k), seed=2, scale=4.0))
    inp, res_out = awq.awq_linear_residual_stats(x, po, zo, so, res, group_size=128)
    want = awq.awq_linear_rmsnorm_stats(inp, w, EPS, packed, qz, s, group_size=128)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # warm the workspace pool outside the capture
        awq.awq_linear_rmsnorm_stats(inp, w, EPS, packed, qz, s, group_size=128)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        gi, gr = awq.awq_linear_residual_stats(x, po, zo, so, res, group_size=128)
        gy = awq.awq_linear_rmsnorm_stats(gi, w, EPS, packed, qz, s, group_size=128)
    for rep in range(3):
        gy.zero_()
        gi.s.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gy.view(torch.int16), want.view(torch.int16)), rep
        assert torch.equal(gi.s.view(torch.int32), inp.s.view(torch.int32)), rep
        assert torch.equal(gr.view(torch.int16), res_out.view(torch.int16)), rep
        _ = (x.float() * 2).sum().item()  # eager work between replays


def test_norm_stats_layer_api(gpu_lib):
    """The layer methods: o_proj.forward_residual_stats, then qkv_proj.forward_rmsnorm_stats
    and gate_up.forward_rmsnorm_stats_silu_and_mul, against o_proj.forward_residual + the
    RMSNorm module + the plain projections (the new residual bit-exact, outputs within the
    GEMM tolerance); M >= 32 is refused."""
    linear = importlib.import_module("llm-serve_amd.layers.linear")
    layernorm = importlib.import_module("llm-serve_amd.layers.layernorm")
    awq = awq_mod()
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    k, inter = 1024, 768
    with torch.device("cuda"):
        o_proj = linear.RowParallelLinear(k, k, quant_config=cfg)
        qkv = linear.ColumnParallelLinear(k, 1536, quant_config=cfg)
        gate_up = linear.MergedColumnParallelLinear(k, [inter, inter], quant_config=cfg)
        norm = layernorm.RMSNorm(k, eps=EPS)
    for mod, n, seed in ((o_proj, k, 20), (qkv, 1536, 21), (gate_up, 2 * inter, 22)):
        qw, qz, s = random_awq_gpu(k, n, seed=seed)
        for name, t in (("qweight", qw), ("qzeros", qz), ("scales", s)):
            param = getattr(mod, name)
            if mod is gate_up:
                half = t.shape[1] // 2
                param.weight_loader(param, t[:, :half], 0)
                param.weight_loader(param, t[:, half:], 1)
            else:
                param.weight_loader(param, t)
        mod.quant_method.process_weights_after_loading(mod)
    norm.weight.copy_(bf16_from_bits(rand_bits((k,), seed=9, scale=0.1, offset=1.0)))
    attn = bf16_from_bits(rand_bits((6, k), seed=10)).view(2, 3, k)
    res = bf16_from_bits(rand_bits((6, k), seed=11, scale=3.0)).view(2, 3, k)
    inp, new_res = o_proj.forward_residual_stats(attn.view(6, k), res.view(6, k))
    h = o_proj(attn)
    xn, want_res = norm(h, res)
    assert torch.equal(new_res.view(torch.int16), want_res.view(6, k).view(torch.int16))
    y = qkv.forward_rmsnorm_stats(norm, inp)
    assert rel_err(y, qkv(xn).view(6, -1).float()) <= GEMM_REL_TOL
    z = gate_up.forward_rmsnorm_stats_silu_and_mul(norm, inp)
    assert rel_err(z, gate_up.forward_silu_and_mul(xn).view(6, -1).float()) <= GEMM_REL_TOL
    big = bf16_from_bits(rand_bits((9, k), seed=12))
    with pytest.raises(ValueError, match="M <= 8"):
        o_proj.forward_residual_stats(big, big)


@pytest.mark.parametrize("shape,m", [("o", 8), ("down", 3), ("down", 8)])
def test_rmsnorm_stats_consumer_split_and_long_rows(gpu_lib, shape, m):
    """Consumer plans beyond the QKV / gate_up shapes: a K split across workgroups (the O shape
    at M = 8: every split's first column block stores its K range of x_norm) and rows longer
    than 8192 (K = 12288: the tile sums beyond the first two chunks per lane are loaded after
    the ring), against the oracle's add_rms_forward and the plain GEMM of x_norm."""
    awq = awq_mod()
    lib = awq.lib()
    k, n = QWEN3_SHAPES[shape]
    print(f"rmsnorm_stats consumer {shape} m={m} plan {lib.plan(m, k, n, 2)}", flush=True)
    packed, qz, s = layer(shape, seed=86)
    w_bits = rand_bits((k,), seed=9, scale=0.1, offset=1.0)
    w = bf16_from_bits(w_bits)
    h_bits = rand_bits((m, k), seed=m + 400, scale=2.0)
    r_bits = rand_bits((m, k), seed=m + 500, scale=3.0)
    h, res = bf16_from_bits(h_bits), bf16_from_bits(r_bits)
    sv = (h.float() + res.float()).contiguous()
    ssq = (sv.double() ** 2).view(m, -1, 16).sum(-1).float().contiguous()
    xn = torch.empty((m, k), dtype=torch.bfloat16, device="cuda")
    y = awq.awq_linear_rmsnorm_stats(awq.NormInput(sv, ssq), w, EPS, packed, qz, s, group_size=128, x_norm=xn)
    want_xn, _, _ = ora.add_rms_norm_ref(h_bits, r_bits, w_bits, EPS)
    d = ulp_diff(bits_of(xn), want_xn)
    assert d.max() <= 2 and (d == 0).mean() > 0.99, (d.max(), (d == 0).mean())
    plain = awq.awq_linear(xn, packed, qz, s, group_size=128)
    assert rel_err(y, plain.float()) <= GEMM_REL_TOL
    assert (bits_of(y) == bits_of(plain)).mean() > 0.9


def test_norm_stats_empty_batch(gpu_lib):
    """M = 0: both calls return empty results and enqueue nothing."""
    awq = awq_mod()
    k, n = QWEN3_SHAPES["o"]
    packed, qz, s = layer("o", seed=87)
    x = torch.empty((0, k), dtype=torch.bfloat16, device="cuda")
    res = torch.empty((0, n), dtype=torch.bfloat16, device="cuda")
    inp, res_out = awq.awq_linear_residual_stats(x, packed, qz, s, res, group_size=128)
    assert inp.s.shape == (0, n) and inp.ssq.shape == (0, n // 16) and res_out.shape == (0, n)
    pq, zq, sq = layer("qkv", seed=88)
    w = bf16_from_bits(rand_bits((n,), seed=3, scale=0.1, offset=1.0))
    y = awq.awq_linear_rmsnorm_stats(inp, w, EPS, pq, zq, sq, group_size=128)
    assert y.shape == (0, QWEN3_SHAPES["qkv"][1])
