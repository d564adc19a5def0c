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
@pytest.mark.parametrize("m,k", [(1, 4096), (5, 4096), (64, 128), (300, 136), (3, 16384), (17, 5120), (2048, 4096),
                                 (9, 1024), (1, 520), (2, 2056), (4, 8200)])
def test_add_rmsnorm_matches_oracle(gpu_lib, m, k, with_res):
    """Short rows (K <= 512: lanes of one wave per row) and whole-workgroup rows of one, two,
    four and eight 16-byte chunks per lane, full (K = 1024, 4096, 16384) and with the last
    round of chunks partly past the row (K = 520, 2056, 5120, 8200)."""
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


@pytest.mark.parametrize("k", [4096, 136])
def test_add_rmsnorm_in_place(gpu_lib, k):
    """residual_out may be the residual itself and the normalised output may replace x
    (whole-workgroup rows and short rows)."""
    m = 33
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
    """Every regime (the decode kernel with the norm as its prologue at M <= 2, the decode
    kernel with and without a K split after the norm kernel, the tile kernel) at the real
    shapes: the call's normalised activations x_norm are within the norm's bar of the oracle
    (two ulps, > 99 % exact), its GEMM output equals the plain (or SiLU * up) GEMM of that
    x_norm bit for bit, and the new residual is bit-exact; the same with the residual updated
    in place (which always takes the norm kernel)."""
    k, n = QWEN3_SHAPES[shape]
    awq = awq_mod()
    lib = awq.lib()
    qw, qz, s = random_awq_gpu(k, n, seed=71)
    packed = awq.repack_awq_qweight(qw)
    w_bits = rand_bits((k,), seed=5, scale=0.1, offset=1.0)
    w = bf16_from_bits(w_bits)
    for m in (1, 2, 4, 5, 16, 33, 64, 300, 2048):
        print(f"gemm_rmsnorm {shape} silu={silu} m={m}", flush=True)
        x_bits, r_bits = rand_bits((m, k), seed=m), rand_bits((m, k), seed=m + 1, scale=4.0)
        x, res = bf16_from_bits(x_bits), bf16_from_bits(r_bits)
        want_xn, want_res, _ = ora.add_rms_norm_ref(x_bits, r_bits, w_bits, EPS)
        n_out = n // 2 if silu else n
        ws = torch.zeros(max(lib.workspace_bytes(m, k, n), 256), dtype=torch.uint8, device="cuda")
        for in_place in (False, True):
            res_in = res.clone()
            res_out = res_in if in_place else torch.empty_like(res)
            xn = torch.empty_like(x)
            y = torch.empty((m, n_out), dtype=torch.bfloat16, device="cuda")
            lib.gemm_rmsnorm(x, res_in, w, EPS, xn, res_out, packed, qz, s, y, n, ws, silu_mul=silu)
            assert np.array_equal(bits_of(res_out), want_res), (m, in_place)
            d = ulp_diff(bits_of(xn), want_xn)
            assert d.max() <= 2 and (d == 0).mean() > 0.99, (m, in_place, d.max(), (d == 0).mean())
            plain = (awq.awq_linear_silu_mul if silu else awq.awq_linear)(xn, packed, qz, s, group_size=128)
            assert torch.equal(y.view(torch.int16), plain.view(torch.int16)), (m, in_place)


def test_fused_norm_prologue_without_residual_and_first_layer(gpu_lib):
    """The decode prologue without a residual (the first layer's input_layernorm): x_norm
    within the bar of the oracle's rms_forward, the GEMM of it bit-identical; the layer API
    returns the input itself as the new residual."""
    k, n = QWEN3_SHAPES["qkv"]
    awq = awq_mod()
    lib = awq.lib()
    qw, qz, s = random_awq_gpu(k, n, seed=72)
    packed = awq.repack_awq_qweight(qw)
    w_bits = rand_bits((k,), seed=6, scale=0.1, offset=1.0)
    w = bf16_from_bits(w_bits)
    for m in (1, 2):
        x_bits = rand_bits((m, k), seed=40 + m, scale=2.0)
        x = bf16_from_bits(x_bits)
        xn = torch.empty_like(x)
        y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        lib.gemm_rmsnorm(x, None, w, EPS, xn, None, packed, qz, s, y, n, None)
        want_xn, _, _ = ora.add_rms_norm_ref(x_bits, None, w_bits, EPS)
        d = ulp_diff(bits_of(xn), want_xn)
        assert d.max() <= 2 and (d == 0).mean() > 0.99, (m, d.max())
        assert torch.equal(y.view(torch.int16), awq.awq_linear(xn, packed, qz, s, group_size=128).view(torch.int16))
        y2, first_res = awq.awq_linear_rmsnorm(x, None, w, EPS, packed, qz, s, group_size=128)
        assert first_res is x and torch.equal(y2.view(torch.int16), y.view(torch.int16))


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
    y2, first_res = gate_up.forward_rmsnorm(norm, x)
    assert first_res is x  # the first layer's residual is its input (qwen3.py:166-167)
    assert torch.equal(y2.view(torch.int16), gate_up(norm(x)).view(torch.int16))
    with pytest.raises(ValueError, match="weight must have shape"):
        awq.add_rms_norm(x, None, norm.weight[:-8], EPS)
    with pytest.raises(ValueError, match="residual must have"):
        norm(x, res[:1].contiguous())


@pytest.mark.parametrize("tokens", [1, 7, 64])
def test_head_norms_on_strided_qkv_views(gpu_lib, tokens):
    """q_norm / k_norm (RMSNorm(head_dim)) on q.view(-1, heads, head_dim) and
    k.view(-1, kv_heads, head_dim) of the split QKV output (qwen3.py:87-94): strided views,
    normalised in place of the reference's copy; same bar as the contiguous rows, and
    bit-identical to normalising a contiguous copy."""
    layernorm = importlib.import_module("llm-serve_amd.layers.layernorm")
    heads, kv_heads, head = 32, 8, 128
    qkv_bits = rand_bits((tokens, (heads + 2 * kv_heads) * head), seed=tokens, scale=3.0)
    qkv = bf16_from_bits(qkv_bits)
    q, k, _ = qkv.split([heads * head, kv_heads * head, kv_heads * head], dim=-1)
    with torch.device("cuda"):
        q_norm, k_norm = layernorm.RMSNorm(head, eps=EPS), layernorm.RMSNorm(head, eps=EPS)
    w_bits = rand_bits((head,), seed=1, scale=0.2, offset=1.0)
    q_norm.weight.copy_(bf16_from_bits(w_bits))
    k_norm.weight.copy_(bf16_from_bits(w_bits))
    for view, norm, nh, off in ((q.view(-1, heads, head), q_norm, heads, 0),
                                (k.view(-1, kv_heads, head), k_norm, kv_heads, heads * head)):
        assert view.is_contiguous() == (tokens == 1)  # one token's heads are contiguous
        out = norm(view)
        assert out.shape == view.shape and out.is_contiguous()
        rows = qkv_bits[:, off: off + nh * head].reshape(tokens * nh, head)
        want, _, _ = ora.add_rms_norm_ref(rows, None, w_bits, EPS)
        d = ulp_diff(bits_of(out).reshape(tokens * nh, head), want)
        assert d.max() <= 2 and (d == 0).mean() > 0.99, (d.max(), (d == 0).mean())
        assert torch.equal(out.view(torch.int16), norm(view.contiguous()).view(torch.int16))
    assert np.array_equal(bits_of(qkv), qkv_bits)  # the input is not modified


def test_strided_rows_longer_than_512(gpu_lib):
    """The strided form over rows that take a whole workgroup each: 1024-wide "heads" of a
    [tokens, 6 * 1024] tensor viewed as [tokens, 4, 1024] (row stride 6 * 1024 between
    tokens, 1024 within), against the oracle and against a contiguous copy."""
    layernorm = importlib.import_module("llm-serve_amd.layers.layernorm")
    tokens, heads, head = 5, 4, 1024
    buf_bits = rand_bits((tokens, 6 * head), seed=21, scale=2.0)
    buf = bf16_from_bits(buf_bits)
    view = buf[:, head: head + heads * head].view(tokens, heads, head)
    assert not view.is_contiguous()
    with torch.device("cuda"):
        norm = layernorm.RMSNorm(head, eps=EPS)
    w_bits = rand_bits((head,), seed=22, scale=0.2, offset=1.0)
    norm.weight.copy_(bf16_from_bits(w_bits))
    out = norm(view)
    rows = buf_bits[:, head: head + heads * head].reshape(tokens * heads, head)
    want, _, _ = ora.add_rms_norm_ref(rows, None, w_bits, EPS)
    d = ulp_diff(bits_of(out).reshape(tokens * heads, head), want)
    assert d.max() <= 2 and (d == 0).mean() > 0.99, (d.max(), (d == 0).mean())
    assert torch.equal(out.view(torch.int16), norm(view.contiguous()).view(torch.int16))
    assert np.array_equal(bits_of(buf), buf_bits)


def test_two_layer_step_from_no_residual_matches_oracle(gpu_lib):
    """Two decoder layers in the reference's order (qwen3.py:163-178) starting with
    residual=None: the first layer's residual is its input (qwen3.py:166-167), so the
    post-attention norm adds it.  Every norm's new residual is bit-exact with the oracle
    (add_rms_forward over the GPU's own inputs) and every projection within the GEMM
    tolerance of the oracle's fp64 GEMM of the GPU's input to it."""
    linear = importlib.import_module("llm-serve_amd.layers.linear")
    layernorm = importlib.import_module("llm-serve_amd.layers.layernorm")
    awq = awq_mod()
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    hidden, head, heads, kv_heads, inter = 1024, 128, 8, 2, 768
    layers = []
    for li in range(2):
        with torch.device("cuda"):
            mods = {"qkv": linear.QKVParallelLinear(hidden, head, heads, kv_heads, quant_config=cfg),
                    "o": linear.RowParallelLinear(heads * head, hidden, quant_config=cfg),
                    "gate_up": linear.MergedColumnParallelLinear(hidden, [inter, inter], quant_config=cfg),
                    "down": linear.RowParallelLinear(inter, hidden, quant_config=cfg),
                    "norm1": layernorm.RMSNorm(hidden, eps=EPS), "norm2": layernorm.RMSNorm(hidden, eps=EPS)}
        host = {}
        for i, name in enumerate(("qkv", "o", "gate_up", "down")):
            lay = mods[name]
            k, n = lay.qweight.shape[0], lay.scales.shape[1]
            p = ora.make_problem(seed=500 + 10 * li + i, m=1, k=k, n=n, scale_lo=0.001, scale_hi=0.004)
            host[name] = p
            lay.qweight.data.copy_(torch.from_numpy(p["qweight"]))
            lay.qzeros.data.copy_(torch.from_numpy(p["qzeros"]))
            lay.scales.data.copy_(bf16_from_bits(p["scales_bits"]))
            lay.quant_method.process_weights_after_loading(lay)
        for j, name in enumerate(("norm1", "norm2")):
            wb = rand_bits((hidden,), seed=60 + 2 * li + j, scale=0.1, offset=1.0)
            host[name] = wb
            mods[name].weight.copy_(bf16_from_bits(wb))
        layers.append((mods, host))

    def gemm_ref(x_bits, p):
        return ora.awq_linear_ref(x_bits, p["qweight"], p["qzeros"], p["scales_bits"], 128)

    m = 5
    h = bf16_from_bits(rand_bits((m, hidden), seed=99))
    res = None
    for li, (mods, host) in enumerate(layers):
        h_bits = bits_of(h)
        res_bits = bits_of(res) if res is not None else None
        qkv, res = mods["qkv"].forward_rmsnorm(mods["norm1"], h, res)
        xn_bits, want_res, _ = ora.add_rms_norm_ref(h_bits, res_bits, host["norm1"], EPS)
        if res_bits is None:
            assert res is h  # the first layer's residual is its input
        else:
            assert np.array_equal(bits_of(res), want_res), li
        assert rel_err(qkv, gemm_ref(xn_bits, host["qkv"])) <= GEMM_REL_TOL, ("qkv", li)
        attn = qkv[:, : heads * head].contiguous()
        a = mods["o"](attn)
        assert rel_err(a, gemm_ref(bits_of(attn), host["o"])) <= GEMM_REL_TOL, ("o", li)
        res_bits = bits_of(res)
        x, res = mods["gate_up"].forward_rmsnorm_silu_and_mul(mods["norm2"], a, res)
        xn2_bits, want_res2, _ = ora.add_rms_norm_ref(bits_of(a), res_bits, host["norm2"], EPS)
        assert np.array_equal(bits_of(res), want_res2), ("post-attention residual", li)
        gu = host["gate_up"]
        want_x = ora.awq_gate_up_silu_mul_ref(xn2_bits, gu["qweight"], gu["qzeros"], gu["scales_bits"], 128)
        assert rel_err(x, want_x) <= 1.2e-2, ("gate_up", li)  # one intermediate ulp + rounding
        h = mods["down"](x)
        assert rel_err(h, gemm_ref(bits_of(x), host["down"])) <= GEMM_REL_TOL, ("down", li)
    assert torch.isfinite(h.float()).all()


def test_workspace_reserved_at_load_and_never_grown_in_capture(gpu_lib, monkeypatch):
    """process_weights_after_loading reserves the workspace for the configured largest M; a
    request beyond the reserve while the stream captures a graph raises instead of
    allocating."""
    linear = importlib.import_module("llm-serve_amd.layers.linear")
    awq = awq_mod()
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16, max_batched_tokens=1024)
    k, n = QWEN3_SHAPES["down"]
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        with torch.device("cuda"):
            down = linear.RowParallelLinear(k, n, quant_config=cfg)
        qw, qz, s = random_awq_gpu(k, n, seed=3)
        for name, t in (("qweight", qw), ("qzeros", qz), ("scales", s)):
            getattr(down, name).data.copy_(t)
        down.quant_method.process_weights_after_loading(down)
        have = awq.WORKSPACE.reserved_bytes(torch.device("cuda"))
        assert have >= gpu_lib.workspace_bytes_max(1024, k, n) > 0
        monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
        assert awq.WORKSPACE.get(torch.device("cuda"), have) is not None  # within the reserve: no allocation
        with pytest.raises(RuntimeError, match="graph capture"):
            awq.WORKSPACE.get(torch.device("cuda"), have + 1)
