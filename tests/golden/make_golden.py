"""Writes the committed golden fixtures under tests/golden/.

Run from the repository root:  python tests/golden/make_golden.py

* ``reference_kats.json`` -- the known-answer inputs that the reference's own tests
  hold for this path (file:line given per entry), with expected outputs derived by
  hand from the AutoAWQ definition (they are checked again against exact rational
  arithmetic in tests/test_oracle.py).
* ``awq_small_seeded.npz`` -- seeded small problems (K=256, N=128, M in {1, 16, 64},
  plus special-scale and outlier cases) with packed inputs, bf16 bit patterns of the
  dequantized weight, and an fp64-accumulated GEMM result, produced by the oracle.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import awq_oracle as ora  # noqa: E402

KATS = {
    "unpack_channel_order": {
        "source": "tests/test_awq_reference.py:103-116",
        "values": [list(range(16)), list(reversed(range(16)))],
    },
    "pack_word_0_to_7": {
        "source": "format constant, awq_calibration.py:9 (hand-derived)",
        "values": [list(range(8))],
        "packed_hex": ["0x75316420"],
    },
    "pack_word_8_to_15": {
        "source": "format constant, awq_calibration.py:9 (hand-derived)",
        "values": [list(range(8, 16))],
        "packed_hex": ["0xfdb9eca8"],
    },
    "dequant_group2_fp32": {
        "source": "tests/test_awq_reference.py:118-156",
        "qvalues": [[1, 2, 3, 4, 5, 6, 7, 8], [8, 7, 6, 5, 4, 3, 2, 1],
                    [2, 4, 6, 8, 10, 12, 14, 15], [15, 14, 12, 10, 8, 6, 4, 2]],
        "zeros": [[1, 1, 2, 2, 3, 3, 4, 4], [4, 4, 3, 3, 2, 2, 1, 1]],
        "scales": [[0.5, 0.5, 1.0, 1.0, 1.5, 1.5, 2.0, 2.0],
                   [2.0, 2.0, 1.5, 1.5, 1.0, 1.0, 0.5, 0.5]],
        "group_size": 2,
        "expected": [[0.0, 0.5, 1.0, 2.0, 3.0, 4.5, 6.0, 8.0],
                     [3.5, 3.0, 4.0, 3.0, 1.5, 0.0, -4.0, -6.0],
                     [-4.0, 0.0, 4.5, 7.5, 8.0, 10.0, 6.5, 7.0],
                     [22.0, 20.0, 13.5, 10.5, 6.0, 4.0, 1.5, 0.5]],
    },
    "linear_group2_fp32": {
        "source": "tests/test_awq_reference.py:158-203",
        "inputs": [[[1.0, -1.0, 0.5, 2.0], [0.0, 1.0, 2.0, -1.0]]],
        "expected": [[[38.5, 37.5, 26.25, 23.75, 17.5, 17.5, 16.25, 18.5],
                      [-26.5, -17.0, -0.5, 7.5, 11.5, 16.0, 7.5, 7.5]]],
    },
    "quantize_exact_roundtrip": {
        "source": "tests/test_awq_quantizer.py:8-41",
        "weight": [[-7.0, 8.0, -14.0, 16.0]] * 8,
        "group_size": 2,
        "expected_scales": [[1.0] * 8, [2.0] * 8],
        "expected_qweight_values": [[0] * 8, [15] * 8, [0] * 8, [15] * 8],
        "expected_zero_values": [[7] * 8, [7] * 8],
    },
    "layer_forward_pattern": {
        "source": "tests/test_awq_linear_backend.py:125-148",
        "k": 128, "n": 16, "m": 4,
        "qvalues": "arange(k*n) % 16 viewed [k, n]",
        "zero": 8,
        "scales": "linspace(0.01, 0.16, 16) in bf16, one group",
    },
    "bf16_rne_table": {
        "source": "IEEE-754 round-to-nearest-even, c10 BFloat16 conversion",
        "f32_hex": ["0x3f800000", "0x3f808000", "0x3f818000", "0x3f808001", "0x3f807fff",
                    "0x7f7fffff", "0xff800000", "0x7f800000", "0x00000001", "0x00008000",
                    "0x00018000", "0x80000000", "0x7fc00001", "0xffffffff", "0x3c010000",
                    "0xbf7f8000", "0x47800000", "0x007fffff"],
        "bf16_hex": ["0x3f80", "0x3f80", "0x3f82", "0x3f81", "0x3f80",
                     "0x7f80", "0xff80", "0x7f80", "0x0000", "0x0000",
                     "0x0002", "0x8000", "0x7fc0", "0x7fc0", "0x3c01",
                     "0xbf80", "0x4780", "0x0080"],
    },
}


def seeded_cases():
    cases = {}
    for m in (1, 16, 64):
        p = ora.make_problem(seed=1000 + m, m=m, k=256, n=128)
        cases[f"m{m}"] = p
    # activation outliers (1% of input channels x20) as in the prefill config
    cases["outlier_m32"] = ora.make_problem(seed=2024, m=32, k=256, n=128, outlier_frac=0.01)
    # special scales: zero, negative, subnormal, tiny, large; q == z rows
    p = ora.make_problem(seed=77, m=8, k=256, n=128)
    s = ora.bf16_bits_to_f32(p["scales_bits"]).copy()
    s[0, 0:8] = 0.0
    s[0, 8:16] = -0.01
    s[1, 0:8] = np.float32(2.0 ** -130)  # subnormal in bf16 and fp32
    s[1, 8:16] = np.float32(2.0 ** -120)
    s[1, 16:24] = np.float32(3.0e30)
    p["scales_bits"] = ora.f32_to_bf16_bits(s)
    cases["special_scales"] = p
    return cases


def main():
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(KATS, f, indent=1)
    arrays = {}
    for name, p in seeded_cases().items():
        arrays[f"{name}.qweight"] = p["qweight"]
        arrays[f"{name}.qzeros"] = p["qzeros"]
        arrays[f"{name}.scales_bits"] = p["scales_bits"]
        arrays[f"{name}.x_bits"] = p["x_bits"]
        arrays[f"{name}.w_bits"] = ora.dequantize_awq_gemm_bits(
            p["qweight"], p["qzeros"], p["scales_bits"], p["group_size"])
        arrays[f"{name}.y_f64"] = ora.awq_linear_ref(
            p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], p["group_size"], accum="f64")
    np.savez_compressed(os.path.join(HERE, "awq_small_seeded.npz"), **arrays)
    print("wrote", sorted({k.split(".")[0] for k in arrays}))


if __name__ == "__main__":
    main()
