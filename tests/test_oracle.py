"""Pins the CPU oracle before any GPU result is compared against it.

Each check is independent of the oracle's own formula: hand-derived constants, the
reference's known-answer tests (tests/golden/reference_kats.json, with file:line),
torch's bf16 arithmetic (the library the reference computes with), exact rational
arithmetic on small inputs, and algebraic invariants.
"""
import json
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import awq_oracle as ora

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def hex_u32_to_i32(h):
    return np.array([int(h, 16)], dtype=np.uint64).astype(np.uint32).view(np.int32)[0]


# --------------------------------------------------------------------- format
def test_pack_order_constants_are_inverse_permutations():
    for c in range(8):
        assert ora.AWQ_PACK_ORDER[ora.AWQ_REVERSE_ORDER[c]] == c


@pytest.mark.parametrize("name", ["pack_word_0_to_7", "pack_word_8_to_15"])
def test_pack_matches_hand_derived_word(name):
    kat = kats()[name]
    packed = ora.pack_awq_int4(np.array(kat["values"]))
    assert packed.dtype == np.int32
    assert packed[0, 0] == hex_u32_to_i32(kat["packed_hex"][0])
    # unpack must restore the values, including for a word with the sign bit set
    np.testing.assert_array_equal(ora.unpack_awq_int4(packed), np.array(kat["values"]))


def test_unpack_restores_autoawq_channel_order_kat():
    kat = kats()["unpack_channel_order"]
    values = np.array(kat["values"], dtype=np.int32)
    np.testing.assert_array_equal(ora.unpack_awq_int4(ora.pack_awq_int4(values)), values)


def test_pack_nibble_positions_brute_force():
    rng = np.random.default_rng(5)
    values = rng.integers(0, 16, size=(3, 32))
    packed = ora.pack_awq_int4(values).view(np.uint32)
    for r in range(3):
        for c in range(32):
            word = int(packed[r, c // 8])
            nib = ora.AWQ_PACK_ORDER.index(c % 8)  # nibble slot that holds column c
            assert (word >> (4 * nib)) & 0xF == values[r, c]


def test_pack_rejects_out_of_range_and_shapes():
    with pytest.raises(ValueError, match="divisible by 8"):
        ora.pack_awq_int4(np.zeros((2, 7), dtype=np.int64))
    with pytest.raises(ValueError, match=r"\[0, 15\]"):
        ora.pack_awq_int4(np.full((1, 8), 16))
    with pytest.raises(TypeError):
        ora.pack_awq_int4(np.zeros((1, 8), dtype=np.float32))


# ----------------------------------------------------------------------- bf16
def test_bf16_rne_table():
    kat = kats()["bf16_rne_table"]
    f = np.array([int(h, 16) for h in kat["f32_hex"]], dtype=np.uint64).astype(np.uint32).view(np.float32)
    want = np.array([int(h, 16) for h in kat["bf16_hex"]], dtype=np.uint16)
    np.testing.assert_array_equal(ora.f32_to_bf16_bits(f), want)


def test_bf16_rne_matches_torch_on_random_bits():
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2 ** 32, size=200_000, dtype=np.uint64).astype(np.uint32)
    # force many exact ties and near-ties
    bits[:50_000] = (bits[:50_000] & 0xFFFF0000) | 0x8000
    bits[50_000:60_000] = (bits[50_000:60_000] & 0xFFFF0000) | 0x7FFF
    f = bits.view(np.float32)
    ours = ora.f32_to_bf16_bits(f)
    theirs = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    finite = ~np.isnan(f)
    np.testing.assert_array_equal(ours[finite], theirs[finite])
    # NaN stays NaN (payload is not part of the contract)
    assert np.all(np.isnan(ora.bf16_bits_to_f32(ours[~finite])))


# -------------------------------------------------------------------- dequant
def test_dequant_kat_group2_fp32():
    kat = kats()["dequant_group2_fp32"]
    qw = ora.pack_awq_int4(np.array(kat["qvalues"]))
    qz = ora.pack_awq_int4(np.array(kat["zeros"]))
    s = np.array(kat["scales"], dtype=np.float32)
    got = ora.dequantize_awq_gemm_fp(qw, qz, s, kat["group_size"])
    assert got.dtype == np.float32
    np.testing.assert_array_equal(got, np.array(kat["expected"], dtype=np.float32))
    # the bf16 path gives the same numbers (all are exact in bf16)
    bits = ora.dequantize_awq_gemm_bits(qw, qz, ora.f32_to_bf16_bits(s), kat["group_size"])
    np.testing.assert_array_equal(ora.bf16_bits_to_f32(bits), np.array(kat["expected"], dtype=np.float32))


def torch_reference_dequant_bits(qweight, qzeros, scales_bits, group_size):
    """The reference backend's arithmetic (awq.py:243-248) evaluated with torch bf16 ops."""
    q = torch.from_numpy(ora.unpack_awq_int4(qweight))
    z = torch.from_numpy(ora.unpack_awq_int4(qzeros)).repeat_interleave(group_size, dim=0)
    s = torch.from_numpy(scales_bits.view(np.int16).copy()).view(torch.bfloat16)
    s = s.repeat_interleave(group_size, dim=0)
    w = (q.to(torch.bfloat16) - z.to(torch.bfloat16)) * s
    return w.view(torch.int16).numpy().view(np.uint16)


def test_dequant_matches_torch_bf16_arithmetic_including_special_scales():
    rng = np.random.default_rng(3)
    k, n, g = 512, 64, 128
    q = rng.integers(0, 16, size=(k, n))
    z = rng.integers(0, 16, size=(k // g, n))
    q[:g, :8] = z[0, :8]  # q == z
    s = rng.uniform(0.002, 0.02, size=(k // g, n)).astype(np.float32)
    s[0, 8:16] = 0.0
    s[0, 16:24] = -0.0
    s[0, 24:32] = -0.013
    s[1, :8] = np.float32(2.0 ** -131)
    s[1, 8:16] = np.float32(2.0 ** -126)
    s[1, 16:24] = np.float32(1.0e38)
    s[1, 24:32] = np.inf
    s[2, :8] = -np.inf
    s[2, 8:16] = np.nan
    s[2, 16:24] = np.float32(3.389e38)  # near bf16 max: products overflow to inf
    qw, qz, sb = ora.pack_awq_int4(q), ora.pack_awq_int4(z), ora.f32_to_bf16_bits(s)
    ours = ora.dequantize_awq_gemm_bits(qw, qz, sb, g)
    theirs = torch_reference_dequant_bits(qw, qz, sb, g)
    nan_ours = np.isnan(ora.bf16_bits_to_f32(ours))
    nan_theirs = np.isnan(ora.bf16_bits_to_f32(theirs))
    np.testing.assert_array_equal(nan_ours, nan_theirs)
    np.testing.assert_array_equal(ours[~nan_ours], theirs[~nan_ours])
    assert nan_ours.any() and (ours == 0x8000).any() and (ours == 0x7F80).any()


def test_dequant_matches_torch_on_seeded_qwen_like_tile():
    p = ora.make_problem(seed=9, m=1, k=1024, n=512)
    ours = ora.dequantize_awq_gemm_bits(p["qweight"], p["qzeros"], p["scales_bits"], 128)
    theirs = torch_reference_dequant_bits(p["qweight"], p["qzeros"], p["scales_bits"], 128)
    np.testing.assert_array_equal(ours, theirs)


def test_dequant_invariants():
    rng = np.random.default_rng(4)
    k, n, g = 256, 32, 128
    z = rng.integers(0, 16, size=(k // g, n))
    s = ora.f32_to_bf16_bits(rng.uniform(0.002, 0.02, size=(k // g, n)))
    # q == z everywhere -> +0 exactly
    q = np.repeat(z, g, axis=0)
    w = ora.dequantize_awq_gemm_bits(ora.pack_awq_int4(q), ora.pack_awq_int4(z), s, g)
    assert np.all(w == 0)
    # power-of-two scales are exact: W == (q - z) * 2^-e
    q = rng.integers(0, 16, size=(k, n))
    s2 = ora.f32_to_bf16_bits(np.full((k // g, n), 2.0 ** -7, dtype=np.float32))
    w = ora.bf16_bits_to_f32(ora.dequantize_awq_gemm_bits(ora.pack_awq_int4(q), ora.pack_awq_int4(z), s2, g))
    np.testing.assert_array_equal(w, (q - np.repeat(z, g, axis=0)) * 2.0 ** -7)
    # changing group 1's zero point changes rows [g, 2g) only
    z2 = z.copy()
    z2[1] = (z2[1] + 3) % 16
    a = ora.dequantize_awq_gemm_bits(ora.pack_awq_int4(q), ora.pack_awq_int4(z), s, g)
    b = ora.dequantize_awq_gemm_bits(ora.pack_awq_int4(q), ora.pack_awq_int4(z2), s, g)
    assert np.array_equal(a[:g], b[:g]) and not np.array_equal(a[g:], b[g:])


def test_validation_messages_match_reference_contract():
    qw = np.zeros((4, 1), dtype=np.int32)
    qz = np.zeros((2, 1), dtype=np.int32)
    s = np.ones((2, 8), dtype=np.float32)
    with pytest.raises(ValueError, match="qweight.*int32"):
        ora.dequantize_awq_gemm_f32(qw.astype(np.int64), qz, s, 2)
    with pytest.raises(ValueError, match="qzeros.*int32"):
        ora.dequantize_awq_gemm_f32(qw, qz.astype(np.int64), s, 2)
    with pytest.raises(ValueError, match="scales"):
        ora.dequantize_awq_gemm_f32(qw, qz, np.ones((2, 7), dtype=np.float32), 2)
    with pytest.raises(ValueError, match="divisible"):
        ora.dequantize_awq_gemm_f32(np.zeros((5, 1), dtype=np.int32), qz, s, 2)


# --------------------------------------------------------------------- linear
def test_linear_kat_group2_fp32():
    kat = kats()
    d = kat["dequant_group2_fp32"]
    qw = ora.pack_awq_int4(np.array(d["qvalues"]))
    qz = ora.pack_awq_int4(np.array(d["zeros"]))
    sb = ora.f32_to_bf16_bits(np.array(d["scales"], dtype=np.float32))
    x = np.array(kat["linear_group2_fp32"]["inputs"], dtype=np.float32)
    y = ora.awq_linear_ref(ora.f32_to_bf16_bits(x), qw, qz, sb, d["group_size"], accum="f32")
    assert y.shape == (1, 2, 8)
    np.testing.assert_array_equal(y, np.array(kat["linear_group2_fp32"]["expected"], dtype=np.float32))


def exact_linear(x_bits, qweight, qzeros, scales_bits, g):
    """Brute force with Python Fractions and explicit nibble extraction."""
    qwu = np.asarray(qweight).view(np.uint32)
    qzu = np.asarray(qzeros).view(np.uint32)
    xf = ora.bf16_bits_to_f32(x_bits)
    sf = ora.bf16_bits_to_f32(scales_bits)
    m, k = xf.shape
    n = qwu.shape[1] * 8
    out = [[Fraction(0)] * n for _ in range(m)]
    for kk in range(k):
        for nn in range(n):
            slot = ora.AWQ_PACK_ORDER.index(nn % 8)
            q = (int(qwu[kk, nn // 8]) >> (4 * slot)) & 0xF
            z = (int(qzu[kk // g, nn // 8]) >> (4 * slot)) & 0xF
            wf = np.array([np.float32(q - z) * sf[kk // g, nn]], dtype=np.float32)
            w = Fraction(float(ora.bf16_bits_to_f32(ora.f32_to_bf16_bits(wf))[0]))
            for mm in range(m):
                out[mm][nn] += Fraction(float(xf[mm, kk])) * w
    return np.array([[float(v) for v in row] for row in out])


def test_linear_matches_exact_rational_brute_force():
    p = ora.make_problem(seed=21, m=3, k=256, n=16)
    want = exact_linear(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128)
    got64 = ora.awq_linear_ref(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128, accum="f64")
    got32 = ora.awq_linear_ref(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128, accum="f32")
    np.testing.assert_allclose(got64, want, rtol=1e-12, atol=1e-12)
    assert ora.gemm_rel_err(got32, want) < 1e-5


def test_linear_is_linear_in_x_and_zero_for_zero_scales():
    p = ora.make_problem(seed=22, m=4, k=256, n=64)
    x = ora.bf16_bits_to_f32(p["x_bits"])
    xa = ora.f32_to_bf16_bits(x * 2.0)  # exact scaling by 2
    ya = ora.awq_linear_ref(xa, p["qweight"], p["qzeros"], p["scales_bits"], 128)
    y = ora.awq_linear_ref(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128)
    np.testing.assert_array_equal(ya, 2.0 * y)
    zero_s = np.zeros_like(p["scales_bits"])
    assert np.all(ora.awq_linear_ref(p["x_bits"], p["qweight"], p["qzeros"], zero_s, 128) == 0)


def test_linear_rejects_k_mismatch():
    p = ora.make_problem(seed=1, m=1, k=256, n=16)
    with pytest.raises(ValueError, match="K must match"):
        ora.awq_linear_ref(p["x_bits"][:, :128], p["qweight"], p["qzeros"], p["scales_bits"], 128)


# ------------------------------------------------------------------- producer
def test_quantizer_exact_roundtrip_kat():
    kat = kats()["quantize_exact_roundtrip"]
    w = np.array(kat["weight"], dtype=np.float32)
    qw, qz, sb = ora.quantize_awq_weight(w, group_size=kat["group_size"])
    assert qw.shape == (4, 1) and qz.shape == (2, 1) and sb.shape == (2, 8)
    np.testing.assert_array_equal(ora.bf16_bits_to_f32(sb), np.array(kat["expected_scales"], dtype=np.float32))
    np.testing.assert_array_equal(ora.unpack_awq_int4(qw), np.array(kat["expected_qweight_values"]))
    np.testing.assert_array_equal(ora.unpack_awq_int4(qz), np.array(kat["expected_zero_values"]))
    restored = ora.bf16_bits_to_f32(ora.dequantize_awq_gemm_bits(qw, qz, sb, kat["group_size"])).T
    np.testing.assert_array_equal(restored, w)


def test_quantizer_matches_explicit_asymmetric_reference():
    # tests/test_awq_quantizer.py:43-72, with a numpy generator
    rng = np.random.default_rng(7)
    w = rng.standard_normal((16, 128)).astype(np.float32)
    mn, mx = w.min(axis=1, keepdims=True), w.max(axis=1, keepdims=True)
    s = np.maximum(mx - mn, 1e-5) / 15
    z = np.clip(-np.round(mn / s), 0, 15)
    expected = (np.clip(np.round(w / s) + z, 0, 15) - z) * s
    qw, qz, sb = ora.quantize_awq_weight(w, group_size=128)
    got = ora.bf16_bits_to_f32(ora.dequantize_awq_gemm_bits(qw, qz, sb, 128)).T
    np.testing.assert_allclose(got, expected, rtol=0.01, atol=0.01)


def test_quantizer_rejects_unsupported_shapes():
    with pytest.raises(ValueError, match="two-dimensional"):
        ora.quantize_awq_weight(np.zeros(8, dtype=np.float32), group_size=2)
    with pytest.raises(ValueError, match="floating"):
        ora.quantize_awq_weight(np.zeros((8, 4), dtype=np.int32), group_size=2)
    with pytest.raises(ValueError, match="input size"):
        ora.quantize_awq_weight(np.zeros((8, 5), dtype=np.float32), group_size=2)
    with pytest.raises(ValueError, match="output size"):
        ora.quantize_awq_weight(np.zeros((7, 4), dtype=np.float32), group_size=2)


# -------------------------------------------------------------- golden fixture
def test_oracle_reproduces_committed_golden_fixture():
    data = np.load(os.path.join(GOLDEN, "awq_small_seeded.npz"))
    names = sorted({k.split(".")[0] for k in data.files})
    assert {"m1", "m16", "m64", "outlier_m32", "special_scales"} <= set(names)
    for name in names:
        qw, qz, sb, xb = (data[f"{name}.{t}"] for t in ("qweight", "qzeros", "scales_bits", "x_bits"))
        np.testing.assert_array_equal(ora.dequantize_awq_gemm_bits(qw, qz, sb, 128), data[f"{name}.w_bits"])
        np.testing.assert_array_equal(ora.awq_linear_ref(xb, qw, qz, sb, 128), data[f"{name}.y_f64"])


def test_metric_floor_behaviour():
    r = np.array([1.0, -1.0, 1e-6, 0.0])
    assert ora.gemm_rel_err(r, r) == 0.0
    # rms(r) = sqrt(0.5): the two small entries are judged against that floor
    assert ora.gemm_rel_err(r + 0.01, r) == pytest.approx(0.01 / np.sqrt(0.5), rel=1e-9)


# ------------------------------------------------------------------ SiluAndMul
def test_silu_and_mul_closed_forms_and_half_order():
    """activation.py:8-11.  silu(0) = 0; silu(ln 3) = (3/4) ln 3; silu(x) - silu(-x) = x;
    the first half is the gated input (a swapped split fails the asymmetric rows)."""
    ln3 = float(np.log(3.0))
    gate_up = np.array([[0.0, ln3, 2.0, 1.0, 1.0, 5.0]])
    out = ora.silu_and_mul_ref(gate_up)
    sig2 = 1.0 / (1.0 + np.exp(-2.0))
    np.testing.assert_allclose(out, [[0.0, 0.75 * ln3, 2.0 * sig2 * 5.0]], rtol=1e-15, atol=0)
    xs = np.linspace(-8.0, 8.0, 33)
    pos = ora.silu_and_mul_ref(np.concatenate([xs, np.ones_like(xs)])[None])[0]
    neg = ora.silu_and_mul_ref(np.concatenate([-xs, np.ones_like(xs)])[None])[0]
    np.testing.assert_allclose(pos - neg, xs, rtol=1e-14, atol=1e-14)
    # saturation: silu(-inf) * u = -0, silu(+large) = x; NaN propagates
    big = ora.silu_and_mul_ref(np.array([[-1e4, 1e4, np.nan, 3.0, 2.0, 1.0]]))
    assert big[0, 0] == 0.0 and big[0, 1] == 2e4 and np.isnan(big[0, 2])
    with pytest.raises(ValueError, match="even"):
        ora.silu_and_mul_ref(np.zeros((2, 3)))


def test_silu_and_mul_matches_torch_cpu():
    """Against torch's own silu on the CPU in float64 (the library routine the reference
    calls, activation.py:11)."""
    rng = np.random.default_rng(3)
    a = rng.standard_normal((7, 64)) * 4
    t = torch.from_numpy(a)
    want = (torch.nn.functional.silu(t[:, :32]) * t[:, 32:]).numpy()
    np.testing.assert_allclose(ora.silu_and_mul_ref(a), want, rtol=1e-13, atol=1e-13)


def test_gate_up_silu_mul_composes_the_rounded_gemm():
    """qwen3.py:126-130: SiluAndMul over the gate|up GEMM output, rounded to bf16 by torch's
    own conversion (the reference's layer output dtype) or left unrounded."""
    p = ora.make_problem(seed=8, m=3, k=256, n=128)
    y = torch.from_numpy(ora.awq_linear_ref(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128))
    for rounded in (True, False):
        t = y.float().to(torch.bfloat16).double() if rounded else y
        want = (torch.nn.functional.silu(t[:, :64]) * t[:, 64:]).numpy()
        got = ora.awq_gate_up_silu_mul_ref(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128,
                                           round_intermediate=rounded)
        assert got.shape == (3, 64)
        np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-13)


def test_quantizer_ties_round_half_to_even():
    """A row with min 0 and max 15 has s = 1 exactly and z = 0, so q = round(w): the ties
    2.5, 3.5, 4.5, 13.5 go to 2, 4, 4, 14 under torch.round's half-to-even (half-up would
    give 3, 4, 5, 14)."""
    row = np.array([0.0, 15.0, 2.5, 3.5, 4.5, 13.5, 7.0, 8.0], dtype=np.float32)
    w = np.tile(row, (8, 1))  # 8 output rows, one group of 8 inputs
    qw, qz, sb = ora.quantize_awq_weight(w, group_size=8, out_dtype="f32")
    assert np.all(sb == 1.0)
    assert np.all(ora.unpack_awq_int4(qz) == 0)
    np.testing.assert_array_equal(ora.unpack_awq_int4(qw)[:, 0], [0, 15, 2, 4, 4, 14, 7, 8])


def test_quantizer_matches_torch_cpu_arithmetic():
    """The reference's steps (awq_calibration.py:50-62) evaluated by torch on the CPU -- its
    amin/amax, clamp, division and round -- bit for bit against the oracle, for fp32, bf16
    and fp16 weights (scales cast back to the weight dtype)."""
    gen = torch.Generator().manual_seed(5)
    for dtype, out in ((torch.float32, "f32"), (torch.bfloat16, "bf16"), (torch.float16, "f16")):
        w = (torch.randn((24, 256), generator=gen) * 0.05).to(dtype)
        grouped = w.to(torch.float32).reshape(24, 2, 128)
        mn, mx = grouped.amin(dim=-1), grouped.amax(dim=-1)
        s = (mx - mn).clamp(min=1e-5) / 15.0
        z = (-torch.round(mn / s)).clamp(0, 15)
        q = (torch.round(grouped / s.unsqueeze(-1)) + z.unsqueeze(-1)).clamp(0, 15).to(torch.int32).reshape(24, 256)
        qw, qz, sc = ora.quantize_awq_weight(w.float().numpy(), group_size=128, out_dtype=out)
        np.testing.assert_array_equal(ora.unpack_awq_int4(qw), q.t().numpy())
        np.testing.assert_array_equal(ora.unpack_awq_int4(qz), z.to(torch.int32).t().numpy())
        want_s = s.t().contiguous().to(dtype)
        if out == "bf16":
            np.testing.assert_array_equal(sc, want_s.view(torch.int16).numpy().view(np.uint16))
        else:
            np.testing.assert_array_equal(sc, want_s.numpy())


# --------------------------------------------------------------------- RMSNorm(+residual)
def _bits(a):
    return ora.f32_to_bf16_bits(np.asarray(a, dtype=np.float32))


def test_rms_norm_closed_forms():
    """Rows whose root mean square is known: [3, 4, 0, 0] has rms 2.5, a constant row c has
    rms |c|, and eps dominates a row of 1e-4 (1e-4 / sqrt(1e-8 + 1e-6))."""
    x = _bits([[3, 4, 0, 0], [2, 2, 2, 2], [-0.5, -0.5, -0.5, -0.5], [1e-4, 1e-4, 1e-4, 1e-4]])
    ones, twos = _bits(np.ones(4)), _bits(np.full(4, 2.0))
    out, res, normed = ora.add_rms_norm_ref(x, None, ones, 1e-6)
    assert res is None
    x32 = ora.bf16_bits_to_f32(x).astype(np.float64)
    assert np.allclose(normed[0], [1.2, 1.6, 0, 0], rtol=1e-6)
    assert np.array_equal(out[1], _bits(np.ones(4))) and np.array_equal(out[2], _bits(-np.ones(4)))
    assert np.allclose(normed[3], x32[3, 0] / np.sqrt(x32[3, 0] ** 2 + 1e-6), rtol=1e-6)
    assert abs(normed[3, 0] - 0.0995) < 1e-3
    assert np.array_equal(out[0], _bits([1.2, 1.6, 0, 0]))
    # weight 2 is exact: every output doubles, bit for bit
    out2, _, _ = ora.add_rms_norm_ref(x, None, twos, 1e-6)
    assert np.array_equal(ora.bf16_bits_to_f32(out2), 2 * ora.bf16_bits_to_f32(out))


def test_rms_norm_matches_torch_rms_norm_fp64():
    """The normalised rows (before rounding) against torch.nn.functional.rms_norm in fp64,
    and the new residual against torch's own bf16 addition."""
    rng = np.random.default_rng(5)
    x = _bits(rng.standard_normal((6, 4096)) * 3)
    r = _bits(rng.standard_normal((6, 4096)) * 5)
    w = _bits(1 + 0.1 * rng.standard_normal(4096))
    eps = 1e-6
    out, res, normed = ora.add_rms_norm_ref(x, r, w, eps)
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    rt = torch.from_numpy(r.view(np.int16)).view(torch.bfloat16)
    assert np.array_equal(res, (xt + rt).view(torch.int16).numpy().view(np.uint16))
    s = xt.double() + rt.double()
    want = torch.nn.functional.rms_norm(s, (4096,), eps=eps).numpy()
    assert np.allclose(normed, want, rtol=2e-7, atol=0)


def _torch_fp32_steps(x_bits, r_bits, w_bits, eps, round_before_weight=True):
    """The reference's steps (layernorm.py:35-40) run by torch on the CPU in fp32."""
    xt = torch.from_numpy(x_bits.view(np.int16)).view(torch.bfloat16)
    rt = torch.from_numpy(r_bits.view(np.int16)).view(torch.bfloat16)
    wt = torch.from_numpy(w_bits.view(np.int16)).view(torch.bfloat16)
    s = xt.float().add_(rt.float())
    var = s.pow(2).mean(dim=-1, keepdim=True)
    s.mul_(torch.rsqrt(var + eps))
    t = s.to(torch.bfloat16) if round_before_weight else s
    return (t * wt).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_rms_norm_agrees_with_torch_fp32_within_one_ulp():
    """torch's fp32 reduction and rsqrt are one rounding away from the oracle's fp64: the
    bf16 outputs agree exactly almost everywhere and within one bf16 ulp everywhere.  The
    same comparison fails when the oracle's intermediate bf16 rounding is taken out (a
    planted mistake), so the check sees where the roundings sit."""
    rng = np.random.default_rng(6)
    x = _bits(rng.standard_normal((8, 4096)))
    r = _bits(rng.standard_normal((8, 4096)) * 2)
    w = _bits(1 + 0.3 * rng.standard_normal(4096))
    out, _, normed = ora.add_rms_norm_ref(x, r, w, 1e-6)
    got = _torch_fp32_steps(x, r, w, 1e-6)
    ulp = np.abs(out.view(np.int16).astype(np.int32) - got.view(np.int16).astype(np.int32))
    assert ulp.max() <= 1 and (ulp == 0).mean() > 0.995
    # planted mistake: no bf16 rounding of s * r before the weight multiply
    wf = ora.bf16_bits_to_f32(w).astype(np.float64)
    wrong = ora.f32_to_bf16_bits((normed.astype(np.float32).astype(np.float64) * wf).astype(np.float32))
    assert (wrong != got).mean() > 0.05


# ------------------------------------------------- torch CPU restatement (CPU baseline)
def test_torch_cpu_backend_matches_the_numpy_oracle():
    """oracle/awq_torch_cpu.py (the CPU baseline's subject) against the numpy oracle: unpack
    and dequant bit-exact (including the KAT words and negative int32 words), the linear within
    the bf16 GEMM tolerance of the fp64 oracle, and rows independent (the reference's
    matmul over a batch equals its rows one by one, up to accumulation order)."""
    import torch
    from oracle import awq_torch_cpu as tref

    words = np.array([[0x75316420, 0xFDB9ECA8 - 2 ** 32], [-1, 0]], dtype=np.int32)
    assert np.array_equal(tref.unpack_int4(torch.from_numpy(words)).numpy(), ora.unpack_awq_int4(words))
    assert tref.unpack_int4(torch.from_numpy(words[:1, :1])).tolist() == [list(range(8))]  # round-trip KAT row
    for seed, (m, k, n) in enumerate(((3, 256, 64), (16, 512, 128))):
        p = ora.make_problem(seed=40 + seed, m=m, k=k, n=n)
        qw, qz = torch.from_numpy(p["qweight"]), torch.from_numpy(p["qzeros"])
        s = torch.from_numpy(p["scales_bits"].view(np.int16)).view(torch.bfloat16)
        x = torch.from_numpy(p["x_bits"].view(np.int16)).view(torch.bfloat16)
        w = tref.dequantize(qw, qz, s, 128)
        want_w = ora.dequantize_awq_gemm_bits(p["qweight"], p["qzeros"], p["scales_bits"], 128)
        assert np.array_equal(w.view(torch.int16).numpy().view(np.uint16), want_w)
        y = tref.linear(x, qw, qz, s, 128)
        assert y.dtype == torch.bfloat16
        want = ora.awq_linear_ref(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128)
        assert ora.gemm_rel_err(y.float().numpy(), want) <= 1e-2
