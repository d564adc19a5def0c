"""GPU parity of the format kernels: unpack, dequant (bit-exact with the oracle), repack
and the tile GEMM's in-register dequant (via w4a16_dequant_packed)."""
import json
import os

import numpy as np
import pytest
import torch

from awq_helpers import (GOLDEN, QWEN3_SHAPES, awq_mod, bf16_from_bits, bits_of, golden_cases,
                         random_awq_gpu, same_bits_nan_aware)
from oracle import awq_oracle as ora

pytestmark = pytest.mark.gpu


def kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def test_unpack_kat_and_random(gpu_lib):
    awq = awq_mod()
    values = np.array(kats()["unpack_channel_order"]["values"], dtype=np.int32)
    got = awq.unpack_awq_int4(torch.from_numpy(ora.pack_awq_int4(values)).cuda())
    np.testing.assert_array_equal(got.cpu().numpy(), values)
    rng = np.random.default_rng(2)
    words = rng.integers(-2 ** 31, 2 ** 31, size=(64, 40), dtype=np.int64).astype(np.int32)
    got = awq.unpack_awq_int4(torch.from_numpy(words).cuda())
    np.testing.assert_array_equal(got.cpu().numpy(), ora.unpack_awq_int4(words))


def test_dequant_kat_group2(gpu_lib):
    awq = awq_mod()
    kat = kats()["dequant_group2_fp32"]
    qw = torch.from_numpy(ora.pack_awq_int4(np.array(kat["qvalues"]))).cuda()
    qz = torch.from_numpy(ora.pack_awq_int4(np.array(kat["zeros"]))).cuda()
    s = torch.tensor(kat["scales"], dtype=torch.bfloat16, device="cuda")
    w = awq.dequantize_awq_gemm(qw, qz, s, group_size=kat["group_size"])
    np.testing.assert_array_equal(w.float().cpu().numpy(), np.array(kat["expected"], dtype=np.float32))


@pytest.mark.parametrize("case", sorted(golden_cases()))
def test_dequant_bit_exact_on_golden_fixtures(gpu_lib, case):
    awq = awq_mod()
    c = golden_cases()[case]
    qw = torch.from_numpy(c["qweight"]).cuda()
    qz = torch.from_numpy(c["qzeros"]).cuda()
    w = awq.dequantize_awq_gemm(qw, qz, bf16_from_bits(c["scales_bits"]), group_size=128)
    assert same_bits_nan_aware(bits_of(w), c["w_bits"])


@pytest.mark.parametrize("shape", sorted(QWEN3_SHAPES))
def test_dequant_bit_exact_full_qwen3_shapes(gpu_lib, shape):
    awq = awq_mod()
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=sorted(QWEN3_SHAPES).index(shape) + 40)
    w = awq.dequantize_awq_gemm(qw, qz, s, group_size=128)
    want = ora.dequantize_awq_gemm_bits(qw.cpu().numpy(), qz.cpu().numpy(), bits_of(s), 128)
    np.testing.assert_array_equal(bits_of(w), want)


def group_tile_layout_numpy(qweight: np.ndarray) -> np.ndarray:
    """The repacked layout restated from its definition, starting from the logical 4-bit
    values q[row, col] (the oracle's AutoAWQ unpack): per (128-row group g, 16-column tile
    t), lane l and step js hold a word whose bit 8 h + 4 (k // 2) + 16 (k % 2) carries
    q[128 g + 32 js + 8 (l // 16) + 4 h + l % 4, 16 t + 4 ((l // 4) % 4) + k]."""
    q = ora.unpack_awq_int4(qweight).astype(np.uint32)  # [K, N]
    k, n = q.shape
    out = np.zeros(k * n // 8, dtype=np.uint32)
    for g in range(k // 128):
        for t in range(n // 16):
            for lane in range(64):
                for js in range(4):
                    word = 0
                    for h in range(2):
                        for kk in range(4):
                            row = 128 * g + 32 * js + 8 * (lane // 16) + 4 * h + lane % 4
                            col = 16 * t + 4 * ((lane // 4) % 4) + kk
                            word |= int(q[row, col]) << (8 * h + 4 * (kk // 2) + 16 * (kk % 2))
                    out[((g * (n // 16) + t) * 64 + lane) * 4 + js] = word
    return out.view(np.int32)


def test_repack_matches_layout_definition(gpu_lib):
    awq = awq_mod()
    rng = np.random.default_rng(8)
    qw = rng.integers(-2 ** 31, 2 ** 31, size=(256, 8), dtype=np.int64).astype(np.int32)  # K=256, N=64
    got = awq.repack_awq_qweight(torch.from_numpy(qw).cuda()).cpu().numpy()
    np.testing.assert_array_equal(got, group_tile_layout_numpy(qw))


def test_repack_keeps_every_tiles_values(gpu_lib):
    """Each 1 KiB tile holds exactly the 2048 values of its (group, 16 columns) block."""
    awq = awq_mod()
    rng = np.random.default_rng(9)
    k, n = 512, 768
    qw = rng.integers(-2 ** 31, 2 ** 31, size=(k, n // 8), dtype=np.int64).astype(np.int32)
    got = awq.repack_awq_qweight(torch.from_numpy(qw).cuda()).cpu().numpy().view(np.uint32)
    nib = np.stack([(got >> (4 * i)) & 0xF for i in range(8)], axis=-1).reshape(k // 128, n // 16, 2048)
    q = ora.unpack_awq_int4(qw).reshape(k // 128, 128, n // 16, 16).transpose(0, 2, 1, 3).reshape(k // 128, n // 16, 2048)
    np.testing.assert_array_equal(np.sort(nib, axis=-1), np.sort(q, axis=-1))


@pytest.mark.parametrize("case", sorted(golden_cases()))
def test_tile_dequant_matches_reference_on_golden(gpu_lib, case):
    """The GEMM kernels' matrix-core dequant, read back through w4a16_dequant_packed: the
    reference's weights bit for bit (zero signs aside for non-positive scales)."""
    awq = awq_mod()
    L = gpu_lib
    c = golden_cases()[case]
    qw = torch.from_numpy(c["qweight"]).cuda()
    qz = torch.from_numpy(c["qzeros"]).cuda()
    s = bf16_from_bits(c["scales_bits"])
    k, n = qw.shape[0], qw.shape[1] * 8
    w = L.dequant_packed(awq.repack_awq_qweight(qw), qz, s, k, n)
    positive = bool(np.all(ora.bf16_bits_to_f32(c["scales_bits"]) > 0))
    got = bits_of(w)
    if positive:
        np.testing.assert_array_equal(got, c["w_bits"])
    else:
        # non-finite or huge scales are outside the in-GEMM dequant's exact range
        s32 = np.repeat(ora.bf16_bits_to_f32(c["scales_bits"]), 128, axis=0)
        ok = np.isfinite(s32) & (np.abs(s32) < 2.0 ** 123)
        assert same_bits_nan_aware(got[ok], c["w_bits"][ok], zero_sign_free=True)


@pytest.mark.parametrize("shape", ["o", "gate_up"])
def test_tile_dequant_bit_exact_full_shape(gpu_lib, shape):
    awq = awq_mod()
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=5)
    w_ref = awq.dequantize_awq_gemm(qw, qz, s, group_size=128)
    w_tile = gpu_lib.dequant_packed(awq.repack_awq_qweight(qw), qz, s, k, n)
    assert torch.equal(w_ref.view(torch.int16), w_tile.view(torch.int16))
