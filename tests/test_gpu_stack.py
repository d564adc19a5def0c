"""The 36-layer Qwen3-8B linear stack workload (hidden 4096, q|k|v 6144, intermediate 12288),
checked for correctness on a chained stack of four layers with independent random AWQ
weights at packed M in {1, 8, 64, 128}: per layer, the four projections with the layer's
dataflow (the benchmark's chained step; attention itself left out, O reads the first 4096
q|k|v columns):

    qkv = h @ Wqkv;  h = bf16(bf16(qkv[:, :4096] @ Wo) + h);  a = SiLU(g) * u, [g | u] = h @ Wgu;
    h = bf16(bf16(a @ Wd) + h)

The reference for every projection is composed from the oracle-pinned dequant
(dequantize_awq_gemm, bit-exact on these shapes), an fp32 matmul and the oracle's residual /
SiLU semantics, fed with the GPU's own input to that projection (so errors do not compound
through the chain):
  * QKV: both GEMM floors (max |y - r| / max(|r|, rms r) and / max(|r|, 1e-3 rms r) <= 1e-2);
  * O and down with the residual add: >= 99 % of the new hidden state is bit-exact, and
    every element lies in [bf16(bf16(o - d) + residual), bf16(bf16(o + d) + residual)] for
    o = x @ W in fp32 and d = 2^-16 (|x| @ |W|), a bound on how far another summation order
    of the same fp32 products can move o (where o lies next to a bf16 rounding boundary, the
    GPU's rounding of it may differ from the reference's, and the sum follows it);
  * gate|up with SiLU * up: against the exact composition (fp32 g and u, SiLU in fp64), the
    rms-floor GEMM tolerance.
The same four layers captured in one HIP graph replay bit-identically to the eager step, with
eager work in between the replays.  Weights use scales in [0.001, 0.004] ([0.0003, 0.0012]
for down) and the input has rms 0.25, so that the hidden state stays within 0.4 .. 3 rms
through the four layers (the benchmark's [0.002, 0.02] grows it ~5x per projection, and the
SiLU * up product squares it)."""
import numpy as np
import pytest
import torch

from awq_helpers import assert_gemm_close, assert_silu_two_step, awq_mod, random_awq_gpu

pytestmark = pytest.mark.gpu

LAYERS = 4
HIDDEN, QKV_N, INTER = 4096, 6144, 12288
SHAPES = {"qkv": (HIDDEN, QKV_N), "o": (HIDDEN, HIDDEN), "gate_up": (HIDDEN, 2 * INTER), "down": (INTER, HIDDEN)}


@pytest.fixture(scope="module")
def stack(gpu_lib):
    awq = awq_mod()
    layers = []
    for li in range(LAYERS):
        layer = {}
        for si, (name, (k, n)) in enumerate(SHAPES.items()):
            lo, hi = (0.0003, 0.0012) if name == "down" else (0.001, 0.004)
            qw, qz, s = random_awq_gpu(k, n, seed=9000 + 10 * li + si, scale_lo=lo, scale_hi=hi)
            layer[name] = (awq.repack_awq_qweight(qw), qz, s, qw)
        layers.append(layer)
    yield layers
    del layers
    torch.cuda.empty_cache()


def dequant(w):
    packed, qz, s, qw = w
    return awq_mod().dequantize_awq_gemm(qw, qz, s, group_size=128).float()


def step(layers, h, record=None):
    """One chained step over all layers, in place on h; record[li] gets each projection's
    input and output when given."""
    awq = awq_mod()
    for li, layer in enumerate(layers):
        rec = {} if record is not None else None
        packed, qz, s, _ = layer["qkv"]
        if rec is not None:
            rec["h0"] = h.clone()
        qkv = awq.awq_linear(h, packed, qz, s, group_size=128)
        attn = qkv[:, :HIDDEN].contiguous()
        packed, qz, s, _ = layer["o"]
        awq.awq_linear_residual(attn, packed, qz, s, h, group_size=128, out=h)
        if rec is not None:
            rec.update(qkv=qkv, attn=attn, h1=h.clone())
        packed, qz, s, _ = layer["gate_up"]
        act = awq.awq_linear_silu_mul(h, packed, qz, s, group_size=128)
        packed, qz, s, _ = layer["down"]
        awq.awq_linear_residual(act, packed, qz, s, h, group_size=128, out=h)
        if rec is not None:
            rec.update(act=act, h2=h.clone())
            record.append(rec)
    return h


def residual_reference(x, w, res):
    """(want, lo, hi): want = bf16(bf16(x @ W) + res) with an fp32 matmul; [lo, hi] the range
    of bf16(bf16(o) + res) over every o within the fp32 summation-order error of x @ W,
    taken as 2^-16 * (|x| @ |W|) per element (another order of the same fp32 sums differs by
    far less).  The sum is monotone in o, so the range ends come from the two extreme
    roundings of the projection output."""
    wd = dequant(w)
    o32 = x.float() @ wd
    delta = (x.float().abs() @ wd.abs()) * 2.0 ** -16
    want = (o32.to(torch.bfloat16).float() + res.float()).to(torch.bfloat16)
    lo = ((o32 - delta).to(torch.bfloat16).float() + res.float()).to(torch.bfloat16)
    hi = ((o32 + delta).to(torch.bfloat16).float() + res.float()).to(torch.bfloat16)
    return want, lo, hi


def check_residual(got, ref, what):
    """>= 99 % of the new hidden state equals the reference's rounding exactly, and every
    element lies within the range the projection output's summation order allows."""
    want, lo, hi = ref
    same = (got.view(torch.int16) == want.view(torch.int16)).float().mean().item()
    assert same >= 0.99, (what, same)
    g = got.float()
    bad = (g < lo.float()) | (g > hi.float())
    assert not bool(bad.any()), (what, int(bad.sum()))


@pytest.mark.parametrize("m", [1, 8, 64, 128])
def test_chained_stack_matches_reference_and_graph_replay(stack, gpu_lib, m):
    g = torch.Generator(device="cuda")
    g.manual_seed(77 + m)
    h_in = (0.25 * torch.randn((m, HIDDEN), device="cuda", generator=g)).to(torch.bfloat16)
    print(f"stack m={m} regimes={[awq_mod().awq_regime(m, k, n) for k, n in SHAPES.values()]}", flush=True)
    record = []
    h = step(stack, h_in.clone(), record)
    torch.cuda.synchronize()
    assert torch.isfinite(h.float()).all()
    for li, (layer, rec) in enumerate(zip(stack, record)):
        assert_gemm_close(rec["qkv"], rec["h0"].float() @ dequant(layer["qkv"]), ("qkv", li, m))
        check_residual(rec["h1"], residual_reference(rec["attn"], layer["o"], rec["h0"]), ("o", li, m))
        assert_silu_two_step(rec["act"], rec["h1"], dequant(layer["gate_up"]), ("gate_up+silu", li, m))
        check_residual(rec["h2"], residual_reference(rec["act"], layer["down"], rec["h1"]), ("down", li, m))
    # the magnitude stays in range through the chain
    rms = [float(r["h2"].float().pow(2).mean().sqrt()) for r in record]
    assert all(0.1 < v < 20 for v in rms), rms

    # the same step captured in one graph: every replay equals the eager result bit for bit
    eager = h.clone()
    static_h = h_in.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step(stack, static_h)  # warm this stream's workspace outside the capture
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step(stack, static_h)
    for i in range(3):
        static_h.copy_(h_in)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_h.view(torch.int16), eager.view(torch.int16)), (m, i)
        step(stack, 0.25 * torch.randn_like(h_in))  # eager work between the replays
        torch.cuda.synchronize()
