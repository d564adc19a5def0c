"""Shared helpers for the GPU parity tests: numpy oracle data <-> torch GPU tensors."""
import importlib
import os

import numpy as np
import torch

from oracle import awq_oracle as ora

QWEN3_SHAPES = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576), "down": (12288, 4096)}
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# The bf16 GEMM tolerance: max |y - r| / max(|r|, floor) against an fp64/fp32-accumulated
# reference over the same bf16 weights, with two floors: rms(r) (rel_err) and the stricter
# 1e-3 rms(r) (rel_err_strict: near-zero outputs are held to 1e-3 of the typical magnitude).
# Both are asserted for plain GEMM outputs (assert_gemm_close).
GEMM_REL_TOL = 1e-2
STRICT_FLOOR = 1e-3


def pkg():
    return importlib.import_module("llm-serve_amd")


def awq_mod():
    return importlib.import_module("llm-serve_amd.layers.quantization.awq")


def bf16_from_bits(bits: np.ndarray, device="cuda") -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(torch.bfloat16)
    return t.to(device)


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def to_gpu(problem: dict) -> dict:
    return {
        "qweight": torch.from_numpy(problem["qweight"]).cuda(),
        "qzeros": torch.from_numpy(problem["qzeros"]).cuda(),
        "scales": bf16_from_bits(problem["scales_bits"]),
        "x": bf16_from_bits(problem["x_bits"]),
    }


def golden_cases():
    data = np.load(os.path.join(GOLDEN, "awq_small_seeded.npz"))
    names = sorted({k.split(".")[0] for k in data.files})
    return {name: {key.split(".", 1)[1]: data[key] for key in data.files if key.startswith(name + ".")}
            for name in names}


def rel_err(y, r, floor: float = 1.0) -> float:
    """GEMM tolerance metric max |y - r| / max(|r|, floor * rms(r)) (oracle.gemm_rel_err at
    floor 1); computed on the GPU for GPU tensors."""
    if isinstance(r, torch.Tensor) and not r.is_cuda and isinstance(y, torch.Tensor) and y.is_cuda:
        r = r.cuda()
    if isinstance(r, np.ndarray) and isinstance(y, torch.Tensor) and y.is_cuda:
        r = torch.from_numpy(np.asarray(r, dtype=np.float64)).cuda()
    if isinstance(y, torch.Tensor) and isinstance(r, torch.Tensor) and y.is_cuda and r.is_cuda:
        y64, r64 = y.detach().double(), r.detach().double()
        if r64.numel() == 0:
            return 0.0
        rms = torch.sqrt(torch.mean(r64 * r64))
        fl = floor * rms if rms > 0 else torch.ones_like(rms)
        return float(torch.max((y64 - r64).abs() / torch.maximum(r64.abs(), fl)))
    y64 = y.detach().double().cpu().numpy() if isinstance(y, torch.Tensor) else np.asarray(y, dtype=np.float64)
    r64 = r.detach().double().cpu().numpy() if isinstance(r, torch.Tensor) else np.asarray(r, dtype=np.float64)
    if floor == 1.0:
        return ora.gemm_rel_err(y64, r64)
    if r64.size == 0:
        return 0.0
    rms = float(np.sqrt(np.mean(r64 * r64)))
    return float(np.max(np.abs(y64 - r64) / np.maximum(np.abs(r64), floor * rms if rms > 0 else 1.0)))


def rel_err_strict(y, r) -> float:
    """rel_err with the 1e-3 rms(r) floor."""
    return rel_err(y, r, floor=STRICT_FLOOR)


def assert_silu_two_step(f, x, w, what=None) -> None:
    """The fused SiLU(g) * u output f [M, N/2] against the reference's two steps over an fp32
    product [g | u] = x @ w (w: the bf16 dequantized gate|up weight as fp32 [K, N]): the GEMM
    output rounded to bf16, then SiLU(g) * u in fp32, rounded once.  Two GEMMs that sum in
    different orders round g or u differently where the value lies next to a bf16 rounding
    boundary, so: >= 99 % of f equals that two-step result bit for bit, and every element
    lies within one bf16 last place of the range the two steps take over every g, u within
    2^-16 sqrt(max(1, K / 4096)) (|x| @ |w|) of the fp32 product (summation-order
    differences of fp32 sums grow about as sqrt(K); at K = 4096 they are far smaller than
    2^-16).  The product is monotone in each rounded factor on such a range (SiLU's minimum
    aside, where it is flat), so the range comes from the four corners.  Where that whole
    range lies below the smallest normal float (|SiLU(g) u| < 2^-126), f may be zero: the
    kernel's fp32 arithmetic flushes subnormal results."""
    gu = x.float() @ w
    delta = (x.float().abs() @ w.abs()) * (2.0 ** -16 * max(1.0, (w.shape[0] / 4096) ** 0.5))
    n2 = gu.shape[1] // 2

    def two(sg, su):
        g = (gu[:, :n2] + sg * delta[:, :n2]).to(torch.bfloat16).double()
        u = (gu[:, n2:] + su * delta[:, n2:]).to(torch.bfloat16).double()
        return torch.nn.functional.silu(g) * u

    want = two(0.0, 0.0).to(torch.bfloat16)
    corners = torch.stack([two(sg, su) for sg in (-1.0, 1.0) for su in (-1.0, 1.0)])
    lo, hi = corners.min(0).values, corners.max(0).values
    fd = f.double()
    ulp = torch.exp2(torch.floor(torch.log2(fd.abs().clamp_min(2.0 ** -126))) - 7)
    inside = (fd >= lo - ulp) & (fd <= hi + ulp)
    inside |= (fd == 0) & (torch.maximum(lo.abs(), hi.abs()) < 2.0 ** -126)
    same = (f.view(torch.int16) == want.view(torch.int16)).float().mean().item()
    assert same >= 0.99, (what, same)
    assert bool(inside.all()), (what, int((~inside).sum()))


def assert_gemm_close(y, r, what=None) -> None:
    """A plain GEMM output against an fp32/fp64-accumulated reference over the same bf16
    weights: both floors within GEMM_REL_TOL."""
    e1, e2 = rel_err(y, r), rel_err_strict(y, r)
    assert e1 <= GEMM_REL_TOL and e2 <= GEMM_REL_TOL, (what, e1, e2)


def same_bits_nan_aware(a: np.ndarray, b: np.ndarray, zero_sign_free: bool = False) -> bool:
    fa, fb = ora.bf16_bits_to_f32(a), ora.bf16_bits_to_f32(b)
    nan_a, nan_b = np.isnan(fa), np.isnan(fb)
    if not np.array_equal(nan_a, nan_b):
        return False
    a2, b2 = a[~nan_a], b[~nan_a]
    if zero_sign_free:
        a2 = np.where((a2 & 0x7FFF) == 0, 0, a2)
        b2 = np.where((b2 & 0x7FFF) == 0, 0, b2)
    return bool(np.array_equal(a2, b2))


def random_awq_gpu(k: int, n: int, seed: int, group: int = 128, scale_lo: float = 0.002, scale_hi: float = 0.02):
    """Seeded AWQ tensors generated on the GPU: uniform random int32 words are uniform
    independent nibbles in {0..15}; scales uniform in [scale_lo, scale_hi] (bf16; the
    benchmark's [0.002, 0.02] by default)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    qweight = torch.randint(-2 ** 31, 2 ** 31 - 1, (k, n // 8), dtype=torch.int32, device="cuda", generator=g)
    qzeros = torch.randint(-2 ** 31, 2 ** 31 - 1, (k // group, n // 8), dtype=torch.int32, device="cuda",
                           generator=g)
    scales = (torch.rand((k // group, n), device="cuda", generator=g) * (scale_hi - scale_lo) + scale_lo)
    return qweight, qzeros, scales.to(torch.bfloat16)


def random_x_gpu(m: int, k: int, seed: int, outliers: bool = False) -> torch.Tensor:
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((m, k), device="cuda", generator=g)
    if outliers:
        cols = torch.randperm(k, device="cuda", generator=g)[: round(0.01 * k)]
        x[:, cols] *= 20.0
    return x.to(torch.bfloat16)


def decode_config_accepted(m: int, k: int, tn: int, depth: int, waves: int, split: int) -> bool:
    """The library's admission rules for a decode configuration, restated: activations
    staged for M <= 4 within 32 KiB; per wave, its share of the groups' scale pairs and zero
    words, staged activations and (8 or 12 waves, a ring of >= 2 groups) the prebuilt dequant
    operands, 384 bytes per tile and group; the workgroup's LDS (those slices or the
    cross-wave reduction) <= 156 KiB; accumulator + ring registers <= 176."""
    mb = (m + 15) // 16
    n_gmax = -(-(k // 128) // split)
    items = -(-n_gmax // waves)
    xl = m <= 4 and n_gmax * m * 256 <= 32 * 1024
    if waves == 12 and tn != 1:
        return False  # 12-wave workgroups hold one column tile
    pre = waves >= 8 and depth >= 2
    up = lambda v, a: -(-v // a) * a
    wave = up(up(items * tn * 32, 256) + up(items * tn * 8, 256) + (up(items * m * 256, 1024) if xl else 0)
              + (items * tn * 384 if pre else 0), 256)
    lds = max(waves * wave, waves * mb * tn * 1024)
    regs = 4 * mb * tn + depth * 4 * (tn + (0 if xl else 4 * mb))
    return lds <= 156 * 1024 and regs <= 176
