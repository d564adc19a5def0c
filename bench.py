"""W4A16 (AutoAWQ GEMM, group 128) linear benchmark on one MI355X.

Headline (`value`): decode-regime aggregate HBM GB/s over the Qwen3-8B projection
shapes (QKV 4096x6144, O 4096x4096, gate_up 4096x24576, down 12288x4096) at packed
M in {1, 4, 8, 16}: sum of algorithmic bytes / sum of kernel time.  One "step" is one
GEMM at each of those 16 points.  Also reported: M = 32 and 64, the chunked-prefill
TFLOP/s at M = 2048 (1% of input channels x20), and the reference backend's torch CPU path
timed on the host cores as the CPU baseline.

Method
  * Inputs are resident in HBM before timing.  Weights are random uniform int32 words
    (= uniform int4 q), zero words likewise, bf16 scales uniform in [0.002, 0.02],
    bf16 activations ~N(0, 1); weight copies rotate so that every launch of a point
    streams a different copy and the copies of one point exceed 2 x 256 MB (the
    Infinity Cache), i.e. decode bytes come from HBM.
  * Each point's launches are captured once in a HIP graph (torch.cuda.CUDAGraph) and
    replayed back to back, point after point: `steps` replays (>= 220 launches at 20 steps)
    in four blocks, each bracketed by HIP events on the replay stream, giving the average
    kernel duration with host launch overhead removed (the dispatch gap between
    back-to-back kernels, about 1 us, stays in).  Every timed region is preceded by WARM_MS
    of untimed replays of the same graph: after a host-side pause the clocks take tens of
    milliseconds of work to come back up.  The cost of alternating between the four
    projections' kernels within a decode step (up to 2 us per launch for gate_up when its
    points are interleaved with the others') is what the stack36 legs measure.
  * Algorithmic bytes per GEMM = K N / 2 + K N / 256 + K N / 64 + 2 M K + 2 M N
    (int4 weights, int32 zeros, bf16 scales, bf16 x and y); flops = 2 M N K.
  * `roofline` describes the dominant launch (the decode point with the longest
    kernel time, gate_up at M = 16): its algorithmic bytes over its event-timed
    duration, against the 8 TB/s HBM peak.  `traffic` is that launch's HBM bytes as
    measured by rocprofv3 counters (FETCH_SIZE + WRITE_SIZE, each scaled by the factor
    that makes a plain 256 MiB copy read and write 256 MiB), taken from the committed
    summary profiles/decode_gate_up_m16_traffic.txt when present.

Also reported (not part of `value`):
  * mixed_m512: the ragged continuous batch (48 decode rows + 8 x 4 verify rows + a
    432-row prefill chunk = M 512) at gate_up and down, TFLOP/s and GB/s;
  * stack36: a 36-layer Qwen3-8B-shaped stack (independent weights, 3.6 GB) stepped at
    M in {1, 8, 64, 128}: 144 GEMMs per step captured in one graph; aggregate weight
    GB/s and linear-layer time per decoded token;
  * stack36_chained: the same weights with the layer's dataflow: QKV, O on the first 4096
    QKV columns (the attention output's shape) with the residual add in its epilogue, the
    fused gate|up GEMM with SiLU * up, down with the residual add -- 144 GEMM launches and
    36 copies per step, one graph;
  * measured_ceilings: a 1 GiB device copy (read + write GB/s), plain streaming reads
    (llm-serve_amd/csrc/probe_read.hip, best of six grid sizes) of 1 GiB and of 52.3 MB
    per launch (the gate_up weight bytes, rotating over more than 2 x 256 MB) and of every
    other projection's weight bytes per launch (read_per_launch_by_shape: 13.1 MB QKV,
    8.7 MB O, 26.2 MB down), and torch.matmul (hipBLASLt) bf16 at the M = 2048 gate_up
    shape, beside the nominal peaks; `roofline.measured_frac` is the dominant launch
    against the 52.3 MB read;
  * points: every decode point's mean per-launch time, the median, min and max of its four
    timed blocks, and read_ceiling_frac: its GB/s over the plain read of its shape's weight
    bytes per launch;
  * cpu_baseline.parity_max_rel_err_vs_gpu: the oracle's output against the HIP GEMM's
    on the same inputs (the baseline's own problem);
  * fused_gate_up: the gate_up GEMM with SiLU(gate) * up in its epilogue
    (w4a16_gemm_silu_mul, [M, 12288] out) against the plain GEMM ([M, 24576] out) and
    against the reference's two steps (the plain GEMM, then torch's SiLU * up on its
    output), at M in {1, 16, 64, 512, 2048};
  * quantize: the GPU AWQ quantizer over a [24576, 4096] bf16 weight (GB/s of weight
    read + packed output written);
  * stack36_normed: stack36_chained's weights with both RMSNorms of each layer, the
    residual add in the norm prologue (the reference's order): w4a16_gemm_rmsnorm for
    input_layernorm + QKV and post_attention_layernorm + gate|up + SiLU * up (the residual
    alternating between two buffers), plain O and down -- 144 GEMM launches per step, plus 72
    norm launches where M > 2 (at M <= 2 the norm runs inside the decode kernel), one graph;
    `norm_stats` (M <= 8): the same step with each norm split across the GEMMs around it
    (O and down through w4a16_gemm_residual_stats, gate|up and QKV through
    w4a16_gemm_rmsnorm_stats) -- 144 GEMM launches and no norm launch after layer 0's;
    `policy_step_us`: the step of the per-M choice (the prologue at M = 1, the split form
    at M = 2..4, the norm kernel above);
  * rmsnorm_prologue: the norm alone, the QKV / gate|up(+SiLU * up) GEMM alone and the two
    in one w4a16_gemm_rmsnorm call at M in {1, 16, 2048};
  * tp8_shards: one GPU's share of each projection split eight ways (QKV and gate_up
    column-parallel, O and down row-parallel: 4096x768, 512x4096, 4096x3072, 1536x4096) at
    M in {1, 16, 64, 2048}, rotating weights as above; `vs_full_over_8` = (the full
    shape's time in this run / 8) / the shard's time, 1.0 for a GEMM that splits perfectly
    (the row-parallel all-reduce is not included).

Profiling mode: `--profile-point SHAPE:M` runs one point without graphs (a 256 MiB copy
for counter calibration, then --steps launches over rotating weights) so that
rocprofv3 --kernel-trace / --pmc see exactly that launch.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import platform
import statistics
import sys
import time

import torch

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

METRIC = "W4A16 GEMM HBM GB/s (M≤16) and TFLOP/s (M=2048), Qwen3-8B shapes"
SHAPES = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576), "down": (12288, 4096)}
DECODE_M = (1, 4, 8, 16)
EXTRA_DECODE_M = (32, 64)
PREFILL_M = 2048
TP8_SHAPES = {"qkv": (4096, 768), "o": (512, 4096), "gate_up": (4096, 3072), "down": (1536, 4096)}
TP8_M = (1, 16, 64, 2048)
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
CACHE_BYTES = 256 * 2 ** 20
DOMINANT = ("gate_up", 16)
TRAFFIC_FILE = os.path.join(REPO, "profiles", "decode_gate_up_m16_traffic.txt")
CALIBRATION_BYTES = 256 * 2 ** 20


def algorithmic_bytes(m: int, k: int, n: int) -> int:
    return k * n // 2 + k * n // 256 + k * n // 64 + 2 * m * k + 2 * m * n


def weight_bytes(k: int, n: int) -> int:
    return k * n // 2 + k * n // 256 + k * n // 64


class Point:
    """One (shape, M) GEMM with its rotating weight copies, captured as one HIP graph."""

    def __init__(self, lib, name, m, k, n, weights, x):
        self.name, self.m, self.k, self.n = name, m, k, n
        dev = x.device
        self.weights = weights
        self.x = x
        self.y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        ws_bytes = lib.workspace_bytes(m, k, n)
        self.ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
        self.ws_len = ws_bytes
        self.lib = lib
        self.regime = lib.regime(m, k, n)
        self.split = lib.split_k(m, k, n)
        self.graph = None

    def launch_all(self, stream_ptr):
        dll = self.lib.dll
        for packed, qzeros, scales in self.weights:
            rc = dll.w4a16_gemm(self.x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(),
                                self.y.data_ptr(), self.m, self.k, self.n, 128,
                                self.ws.data_ptr() if self.ws_len else None, self.ws_len, stream_ptr)
            if rc != 0:
                raise RuntimeError(f"w4a16_gemm failed at {self.name} M={self.m}: {self.lib.last_error()}")

    def capture(self, stream):
        with torch.cuda.stream(stream):
            self.launch_all(stream.cuda_stream)  # warm-up outside the graph
        stream.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            self.launch_all(stream.cuda_stream)

    @property
    def launches(self) -> int:
        return len(self.weights)


def make_weights(k, n, copies, dev, seed):
    """`copies` independent AWQ weight sets in the kernel layout (random words = uniform int4)."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    out = []
    for _ in range(copies):
        packed = torch.randint(-2 ** 31, 2 ** 31 - 1, (k * n // 8,), dtype=torch.int32, device=dev, generator=gen)
        qzeros = torch.randint(-2 ** 31, 2 ** 31 - 1, (k // 128, n // 8), dtype=torch.int32, device=dev,
                               generator=gen)
        scales = (torch.rand((k // 128, n), device=dev, generator=gen) * 0.018 + 0.002).to(torch.bfloat16)
        out.append((packed, qzeros, scales))
    return out


def build_points(lib, ms, dev, seed0=0, min_bytes=2 * CACHE_BYTES):
    """Decode points; the copies of one shape are shared by its M values and together
    exceed `min_bytes`, so consecutive launches never find their weights in cache."""
    points = []
    for si, (name, (k, n)) in enumerate(SHAPES.items()):
        copies = max(2, -(-min_bytes // weight_bytes(k, n)))
        weights = make_weights(k, n, copies, dev, seed0 + 7919 * si)
        for m in ms:
            gen = torch.Generator(device=dev)
            gen.manual_seed(seed0 + 1000 * si + m)
            x = torch.randn((m, k), device=dev, generator=gen).to(torch.bfloat16)
            points.append(Point(lib, name, m, k, n, weights, x))
    return points


# Untimed GPU work before each timed region.  After a host-side pause (building inputs) the
# clocks ramp up over the first tens of milliseconds of work: the first replays of the
# M=2048 gate_up GEMM take 440-540 us, later ones 390-400 us.
WARM_MS = 60.0


def warm_up(replay, min_ms: float = WARM_MS) -> None:
    """Call replay() (which enqueues GPU work) until at least min_ms of wall time has passed."""
    t0 = time.perf_counter()
    while True:
        replay()
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= min_ms:
            return


TIMED_BLOCKS = 4


def time_points(points, stream, steps, warmup):
    """Each point in turn: capture its launches (one per rotating weight copy) in a HIP
    graph, replay it `warmup` times and then for WARM_MS untimed, then `steps` times back to
    back in TIMED_BLOCKS blocks, each bracketed by HIP events on the replay stream (at 20
    steps every decode point runs >= 220 timed launches).  Returns (per-point mean ms per
    launch, total timed ms); time_points.samples holds each block's ms per launch."""
    per_point, samples, total = {}, {}, 0.0
    for p in points:
        p.capture(stream)
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                p.graph.replay()
            warm_up(p.graph.replay)
        nb = max(1, min(TIMED_BLOCKS, steps))
        counts = [steps // nb + (1 if i < steps % nb else 0) for i in range(nb)]
        events = []
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for cnt in counts:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(cnt):
                    p.graph.replay()
                e1.record(stream)
                events.append((cnt, e0, e1))
        torch.cuda.synchronize()
        block_ms = [e0.elapsed_time(e1) for _, e0, e1 in events]
        per_point[id(p)] = sum(block_ms) / (steps * p.launches)
        samples[id(p)] = [ms / (cnt * p.launches) for (cnt, _, _), ms in zip(events, block_ms)]
        total += sum(block_ms)
    time_points.samples = samples
    return per_point, total


def cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo (platform.processor() as a fallback)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(seconds_budget: float = 12.0, gpu_gemm=None) -> dict:
    """The reference backend's CPU path (oracle/awq_torch_cpu.py: the same torch ops as the
    reference's awq_reference_linear -- unpack, bf16 dequant, bf16 matmul on the CPU BLAS)
    on the host at M=16, K=N=4096 (the O projection) with torch using every host core,
    after 2 warm-up runs, repeated for about `seconds_budget` seconds; the median run is
    reported.  With gpu_gemm (a function of the problem's bit arrays returning the HIP
    GEMM's bf16 output bits), also the parity of the two results:
    max |y_gpu - y_cpu| / max(|y_cpu|, rms(y_cpu))."""
    import numpy as np

    from oracle import awq_oracle as ora
    from oracle import awq_torch_cpu as tref

    threads_before = torch.get_num_threads()
    torch.set_num_threads(os.cpu_count() or 1)
    threads = torch.get_num_threads()
    m, k, n = 16, 4096, 4096
    p = ora.make_problem(seed=0, m=m, k=k, n=n)
    qw, qz = torch.from_numpy(p["qweight"]), torch.from_numpy(p["qzeros"])
    sc = torch.from_numpy(p["scales_bits"].view(np.int16)).view(torch.bfloat16)
    x = torch.from_numpy(p["x_bits"].view(np.int16)).view(torch.bfloat16)
    run = lambda: tref.linear(x, qw, qz, sc, 128)  # noqa: E731
    for _ in range(2):
        y = run()
    y_cpu = y.double().numpy()
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or (time.perf_counter() - t_start < seconds_budget and len(times) < 1000):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    torch.set_num_threads(threads_before)
    t = statistics.median(times)
    parity = None
    if gpu_gemm is not None:
        y_gpu = ora.bf16_bits_to_f32(gpu_gemm(p)).astype("float64")
        rms = float((y_cpu ** 2).mean() ** 0.5)
        parity = round(float((abs(y_gpu - y_cpu) / (abs(y_cpu).clip(min=rms))).max()), 5)
    return {"value": round(algorithmic_bytes(m, k, n) / t / 1e9, 3), "unit": "GB/s", "cores": int(threads),
            "parity_max_rel_err_vs_gpu": parity,
            "kind": "port",
            "sample": f"reference backend's torch CPU path (unpack, bf16 dequant, bf16 matmul; "
                      f"oracle/awq_torch_cpu.py), M={m} K={k} N={n} (O proj), torch.get_num_threads()={threads}, "
                      f"median of {len(times)} runs over {time.perf_counter() - t_start:.1f} s after 2 warm-ups, "
                      f"{t * 1e3:.1f} ms/GEMM, host {cpu_model()}, os.cpu_count()={os.cpu_count()}"}


def gpu_gemm_bits(pkg, dev, prob) -> "numpy.ndarray":
    """The HIP GEMM over one problem of bit arrays (AutoAWQ tensors, bf16 bits) -> bf16 bits."""
    import numpy as np
    qw = torch.from_numpy(prob["qweight"]).to(dev)
    qz = torch.from_numpy(prob["qzeros"]).to(dev)
    sc = torch.from_numpy(prob["scales_bits"].view(np.int16)).to(dev).view(torch.bfloat16)
    x = torch.from_numpy(prob["x_bits"].view(np.int16)).to(dev).view(torch.bfloat16)
    packed = pkg.repack_awq_qweight(qw)
    y = pkg.awq_linear(x, packed, qz, sc, group_size=128)
    torch.cuda.synchronize()
    return y.view(torch.int16).cpu().numpy().view(np.uint16)


MIXED_M = 48 * 1 + 8 * 4 + 432
STACK_LAYERS = 36
STACK_M = (1, 8, 64, 128)


def time_graph(fn, stream, reps: int) -> float:
    """Capture fn() in a HIP graph on `stream`, replay it for WARM_MS untimed, then `reps`
    times between HIP events on that stream; returns ms per replay."""
    with torch.cuda.stream(stream):
        fn()
    stream.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    with torch.cuda.stream(stream):
        warm_up(g.replay)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def mixed_batch(lib, dev, stream, reps: int) -> dict:
    """48 decode rows + 8 verify sequences x 4 rows + one 432-row prefill chunk, packed into
    one [512, K] GEMM, at the gate_up and down shapes."""
    out = {}
    for si, name in enumerate(("gate_up", "down")):
        k, n = SHAPES[name]
        copies = max(2, -(-2 * CACHE_BYTES // weight_bytes(k, n)))
        gen = torch.Generator(device=dev)
        gen.manual_seed(300 + si)
        x = torch.randn((MIXED_M, k), device=dev, generator=gen).to(torch.bfloat16)
        p = Point(lib, name, MIXED_M, k, n, make_weights(k, n, copies, dev, 400 + si), x)
        ms = time_graph(lambda: p.launch_all(torch.cuda.current_stream(dev).cuda_stream), stream, reps) / p.launches
        out[name] = {"M": MIXED_M, "us": round(ms * 1e3, 2),
                     "TFLOP/s": round(2 * MIXED_M * n * k / (ms * 1e-3) / 1e12, 1),
                     "GB/s": round(algorithmic_bytes(MIXED_M, k, n) / (ms * 1e-3) / 1e9, 1),
                     "regime": "decode" if p.regime == 1 else "tile", "split": p.split}
        del p
    return out


def layer_stack(lib, dev, stream, reps: int) -> tuple[dict, dict]:
    """36 layers x (QKV, O, gate_up, down) with independent weights; one step = the 144
    GEMMs back to back on one stream at packed M.  Also returns the chained variant over
    the same weights (layer_stack_chained)."""
    layers = [{name: make_weights(k, n, 1, dev, 1000 + 4 * li + si)[0]
               for si, (name, (k, n)) in enumerate(SHAPES.items())} for li in range(STACK_LAYERS)]
    out = {}
    for m in STACK_M:
        xs = {name: torch.randn((m, k), device=dev).to(torch.bfloat16) for name, (k, n) in SHAPES.items()}
        ys = {name: torch.empty((m, n), dtype=torch.bfloat16, device=dev) for name, (k, n) in SHAPES.items()}
        ws_len = max(lib.workspace_bytes(m, k, n) for k, n in SHAPES.values())
        ws = torch.zeros(max(ws_len, 256), dtype=torch.uint8, device=dev)

        def step():
            sp = torch.cuda.current_stream(dev).cuda_stream
            for layer in layers:
                for name, (k, n) in SHAPES.items():
                    packed, qzeros, scales = layer[name]
                    rc = lib.dll.w4a16_gemm(xs[name].data_ptr(), packed.data_ptr(), qzeros.data_ptr(),
                                            scales.data_ptr(), ys[name].data_ptr(), m, k, n, 128,
                                            ws.data_ptr() if ws_len else None, ws_len, sp)
                    if rc != 0:
                        raise RuntimeError(lib.last_error())

        ms = time_graph(step, stream, reps)
        total = sum(algorithmic_bytes(m, k, n) for k, n in SHAPES.values()) * STACK_LAYERS
        out[f"M={m}"] = {"step_us": round(ms * 1e3, 1), "weight_GB/s": round(total / (ms * 1e-3) / 1e9, 1),
                         "us_per_token": round(ms * 1e3 / m, 2),
                         "regimes": sorted({"decode" if lib.regime(m, k, n) == 1 else "tile"
                                            for k, n in SHAPES.values()})}
    chained = layer_stack_chained(lib, dev, stream, reps, layers)
    normed = layer_stack_normed(lib, dev, stream, reps, layers)
    del layers
    return out, chained, normed


def layer_stack_normed(lib, dev, stream, reps: int, layers) -> dict:
    """36 layers with the reference's full dataflow around the projections (attention left
    out as in stack36_chained): input_layernorm(h, residual) + QKV as one w4a16_gemm_rmsnorm
    call, O plain, post_attention_layernorm(h, residual) + gate|up + SiLU * up as one
    w4a16_gemm_rmsnorm call, down plain -- 144 GEMM and 72 RMSNorm launches per step, one
    graph.  The residual add sits in the norm prologue here, the reference's order."""
    out = {}
    kq, nq = SHAPES["qkv"]
    ki, ni = SHAPES["gate_up"]
    for m in STACK_M:
        h = torch.randn((m, kq), device=dev).to(torch.bfloat16)
        res = torch.randn((m, kq), device=dev).to(torch.bfloat16)
        res2 = torch.empty_like(res)  # the new residual goes to the other buffer (no in-place update)
        xn = torch.empty((m, kq), dtype=torch.bfloat16, device=dev)
        nw = (1 + 0.1 * torch.randn(kq, device=dev)).to(torch.bfloat16)
        qkv = torch.empty((m, nq), dtype=torch.bfloat16, device=dev)
        attn = torch.empty((m, kq), dtype=torch.bfloat16, device=dev)
        act = torch.empty((m, ni // 2), dtype=torch.bfloat16, device=dev)
        ws_len = max(lib.workspace_bytes(m, k, n) for k, n in SHAPES.values())
        ws = torch.zeros(max(ws_len, 256), dtype=torch.uint8, device=dev)
        wsp = ws.data_ptr() if ws_len else None

        def normed(w, y, k, n, silu, r_in, r_out, sp):
            packed, qzeros, scales = w
            if lib.dll.w4a16_gemm_rmsnorm(h.data_ptr(), r_in.data_ptr(), nw.data_ptr(), 1e-6, xn.data_ptr(),
                                          r_out.data_ptr(), packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(),
                                          y.data_ptr(), m, k, n, 128, silu, wsp, ws_len, sp) != 0:
                raise RuntimeError(lib.last_error())

        def plain(x, w, k, n, sp):
            packed, qzeros, scales = w
            if lib.dll.w4a16_gemm(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(),
                                  h.data_ptr(), m, k, n, 128, wsp, ws_len, sp) != 0:
                raise RuntimeError(lib.last_error())

        def step():
            sp = torch.cuda.current_stream(dev).cuda_stream
            for layer in layers:
                normed(layer["qkv"], qkv, kq, nq, 0, res, res2, sp)
                attn.copy_(qkv[:, :kq])
                plain(attn, layer["o"], *SHAPES["o"], sp)
                normed(layer["gate_up"], act, ki, ni, 1, res2, res, sp)
                plain(act, layer["down"], *SHAPES["down"], sp)

        ms = time_graph(step, stream, reps)
        out[f"M={m}"] = {"step_us": round(ms * 1e3, 1), "us_per_token": round(ms * 1e3 / m, 2)}
        if m > 8:
            continue
        # Decode sizes: the norms split across the GEMMs around them.  O and down add the
        # residual in place and leave the fp32 sum s and its tile sums of squares; gate|up and
        # the next layer's QKV normalize s in their fragment loads.  Layer 0's QKV keeps
        # w4a16_gemm_rmsnorm (its norm input comes from outside the stack).
        s_buf = torch.empty((m, kq), dtype=torch.float32, device=dev)
        ssq = torch.empty((m, kq // 16), dtype=torch.float32, device=dev)

        def producer(x, w, k, n, sp):
            packed, qzeros, scales = w
            if lib.dll.w4a16_gemm_residual_stats(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(),
                                                 scales.data_ptr(), res2.data_ptr(), s_buf.data_ptr(),
                                                 res2.data_ptr(), ssq.data_ptr(), m, k, n, 128, wsp, ws_len,
                                                 sp) != 0:
                raise RuntimeError(lib.last_error())

        def consumer(w, y, k, n, silu, sp):
            packed, qzeros, scales = w
            if lib.dll.w4a16_gemm_rmsnorm_stats(s_buf.data_ptr(), ssq.data_ptr(), nw.data_ptr(), 1e-6, None,
                                                packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(), y.data_ptr(),
                                                m, k, n, 128, silu, wsp, ws_len, sp) != 0:
                raise RuntimeError(lib.last_error())

        def step_stats():
            sp = torch.cuda.current_stream(dev).cuda_stream
            for li, layer in enumerate(layers):
                if li == 0:
                    normed(layer["qkv"], qkv, kq, nq, 0, res, res2, sp)
                else:
                    consumer(layer["qkv"], qkv, kq, nq, 0, sp)
                attn.copy_(qkv[:, :kq])
                producer(attn, layer["o"], *SHAPES["o"], sp)
                consumer(layer["gate_up"], act, ki, ni, 1, sp)
                producer(act, layer["down"], *SHAPES["down"], sp)

        ms_s = time_graph(step_stats, stream, reps)
        out[f"M={m}"]["norm_stats"] = {"step_us": round(ms_s * 1e3, 1), "us_per_token": round(ms_s * 1e3 / m, 2)}
    # The per-M choice a model makes (the in-kernel prologue at M = 1, the split form at
    # M = 2..4, the norm kernel above): the step time of that choice.
    for key, v in out.items():
        m = int(key.split("=")[1])
        v["policy_step_us"] = v["norm_stats"]["step_us"] if 2 <= m <= 4 and "norm_stats" in v else v["step_us"]
    return out


NORM_M = (1, 16, 2048)


def norm_prologue(lib, dev, stream, reps: int) -> dict:
    """The RMSNorm(+residual) prologue alone (w4a16_add_rmsnorm, hidden 4096), the QKV and
    gate|up(+SiLU * up) GEMMs alone, and the two in one w4a16_gemm_rmsnorm call, each
    graph-replayed over rotating weight copies; `prologue_us` = fused - GEMM alone."""
    out = {}
    for name, silu in (("qkv", 0), ("gate_up", 1)):
        k, n = SHAPES[name]
        copies = max(2, -(-2 * CACHE_BYTES // weight_bytes(k, n)))
        weights = make_weights(k, n, copies, dev, 777)
        for m in NORM_M:
            x = torch.randn((m, k), device=dev).to(torch.bfloat16)
            res = torch.randn((m, k), device=dev).to(torch.bfloat16)
            res_out = torch.empty_like(res)
            xn = torch.empty_like(x)
            nw = (1 + 0.1 * torch.randn(k, device=dev)).to(torch.bfloat16)
            y = torch.empty((m, n // 2 if silu else n), dtype=torch.bfloat16, device=dev)
            ws_len = lib.workspace_bytes(m, k, n)
            ws = torch.zeros(max(ws_len, 256), dtype=torch.uint8, device=dev)
            wsp = ws.data_ptr() if ws_len else None
            gemm = lib.dll.w4a16_gemm_silu_mul if silu else lib.dll.w4a16_gemm

            def check(rc):
                if rc != 0:
                    raise RuntimeError(lib.last_error())

            def fused_step():
                sp = torch.cuda.current_stream(dev).cuda_stream
                for packed, qzeros, scales in weights:
                    check(lib.dll.w4a16_gemm_rmsnorm(x.data_ptr(), res.data_ptr(), nw.data_ptr(), 1e-6, xn.data_ptr(),
                                                     res_out.data_ptr(), packed.data_ptr(), qzeros.data_ptr(),
                                                     scales.data_ptr(), y.data_ptr(), m, k, n, 128, silu, wsp,
                                                     ws_len, sp))

            def gemm_step():
                sp = torch.cuda.current_stream(dev).cuda_stream
                for packed, qzeros, scales in weights:
                    check(gemm(xn.data_ptr(), packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(), y.data_ptr(),
                               m, k, n, 128, wsp, ws_len, sp))

            def norm_step():
                sp = torch.cuda.current_stream(dev).cuda_stream
                for _ in weights:
                    check(lib.dll.w4a16_add_rmsnorm(x.data_ptr(), res.data_ptr(), nw.data_ptr(), 1e-6, xn.data_ptr(),
                                                    res_out.data_ptr(), m, k, sp))

            f_ms = time_graph(fused_step, stream, reps) / copies
            g_ms = time_graph(gemm_step, stream, reps) / copies
            n_ms = time_graph(norm_step, stream, reps) / copies
            out[f"{name} M={m}"] = {"fused_us": round(f_ms * 1e3, 2), "gemm_us": round(g_ms * 1e3, 2),
                                    "norm_us": round(n_ms * 1e3, 2), "prologue_us": round((f_ms - g_ms) * 1e3, 2),
                                    "norm_GB/s": round(4 * m * k * 2 / (n_ms * 1e-3) / 1e9, 1)}
        del weights
    return out


def layer_stack_chained(lib, dev, stream, reps: int, layers) -> dict:
    """36 layers stepped with the layer's dataflow (attention itself left out: O reads the
    first 4096 QKV columns), O and down through w4a16_gemm_residual (in place on the hidden
    state), gate|up through w4a16_gemm_silu_mul; one graph per M."""
    out = {}
    kq, nq = SHAPES["qkv"]
    ki, ni = SHAPES["gate_up"]
    for m in STACK_M:
        h = torch.randn((m, kq), device=dev).to(torch.bfloat16)
        qkv = torch.empty((m, nq), dtype=torch.bfloat16, device=dev)
        attn = torch.empty((m, kq), dtype=torch.bfloat16, device=dev)
        act = torch.empty((m, ni // 2), dtype=torch.bfloat16, device=dev)
        ws_len = max(lib.workspace_bytes(m, k, n) for k, n in SHAPES.values())
        ws = torch.zeros(max(ws_len, 256), dtype=torch.uint8, device=dev)
        wsp = ws.data_ptr() if ws_len else None

        def call(fn, x, w, y, k, n, sp):
            packed, qzeros, scales = w
            if fn(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(), y.data_ptr(), m, k, n, 128,
                  wsp, ws_len, sp) != 0:
                raise RuntimeError(lib.last_error())

        def call_res(x, w, k, n, sp):
            packed, qzeros, scales = w
            if lib.dll.w4a16_gemm_residual(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(),
                                           h.data_ptr(), h.data_ptr(), m, k, n, 128, wsp, ws_len, sp) != 0:
                raise RuntimeError(lib.last_error())

        def step():
            sp = torch.cuda.current_stream(dev).cuda_stream
            for layer in layers:
                call(lib.dll.w4a16_gemm, h, layer["qkv"], qkv, kq, nq, sp)
                attn.copy_(qkv[:, :kq])
                call_res(attn, layer["o"], *SHAPES["o"], sp)  # h = bf16(o_proj(attn) + h), in place
                call(lib.dll.w4a16_gemm_silu_mul, h, layer["gate_up"], act, ki, ni, sp)
                call_res(act, layer["down"], *SHAPES["down"], sp)

        ms = time_graph(step, stream, reps)
        out[f"M={m}"] = {"step_us": round(ms * 1e3, 1), "us_per_token": round(ms * 1e3 / m, 2)}
    return out


def read_ceiling(dev, stream, nbytes: int, copies: int):
    """Best GB/s of a plain streaming read (csrc/probe_read.hip, libw4a16_probe.so) over
    `copies` rotating buffers of `nbytes` each, one launch per buffer, all captured in one
    graph, over a sweep of grid sizes: what a kernel reading that many bytes per launch
    gets from HBM on this GPU, launch overhead included.  None if the probe is not built."""
    import ctypes
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "llm-serve_amd", "csrc", "libw4a16_probe.so")
    if not os.path.exists(path):
        return None
    probe = ctypes.CDLL(path)
    probe.probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    nbytes -= nbytes % 16
    bufs = [torch.full((nbytes // 2,), 1.0, dtype=torch.bfloat16, device=dev) for _ in range(copies)]
    best = None
    for blocks in (512, 1024, 2048, 4096, 8192, 16384):
        sink = torch.zeros(blocks, dtype=torch.int32, device=dev)

        def run():
            sp = torch.cuda.current_stream(dev).cuda_stream
            for b in bufs:
                if probe.probe_read(b.data_ptr(), nbytes, sink.data_ptr(), blocks, sp) != 0:
                    raise RuntimeError("probe_read launch failed")

        gbs = nbytes / (time_graph(run, stream, 5) / copies * 1e-3) / 1e9
        if best is None or gbs > best[0]:
            best = (gbs, blocks)
    return best


def measured_frac(achieved_gbs: float, ceilings) -> dict:
    """The roofline kernel against the measured plain read of its own weight bytes per launch."""
    if not ceilings:
        return {}
    key = next((k for k in ceilings if k.startswith("read_") and k.endswith("MB_per_launch_GB/s")), None)
    if key is None:
        return {}
    return {"measured_peak": ceilings[key], "measured_peak_kind": key.removesuffix("_GB/s"),
            "measured_frac": round(achieved_gbs / ceilings[key], 4)}


def measured_ceilings(dev, stream) -> dict:
    """A 1 GiB device-to-device copy, read-only streams of 1 GiB and of the dominant decode
    launch's weight bytes (rotating over more than 2 x 256 MB), and a hipBLASLt bf16 GEMM at
    the prefill gate_up shape."""
    src = torch.empty(2 ** 29, dtype=torch.bfloat16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    ms = time_graph(lambda: dst.copy_(src), stream, 10)
    copy_gbs = 2 * src.numel() * 2 / (ms * 1e-3) / 1e9
    del src, dst
    read_1g = read_ceiling(dev, stream, 1 << 30, 2)
    dk, dn = SHAPES[DOMINANT[0]]
    wb = weight_bytes(dk, dn)
    read_dom = read_ceiling(dev, stream, wb, max(2, -(-2 * CACHE_BYTES // wb)))
    reads = {}
    if read_1g and read_dom:
        reads = {"read_1GiB_GB/s": round(read_1g[0], 1),
                 f"read_{wb / 1e6:.1f}MB_per_launch_GB/s": round(read_dom[0], 1),
                 "read_probe_blocks": {"1GiB": read_1g[1], f"{wb / 1e6:.1f}MB": read_dom[1]}}
        # the same probe at every projection's weight bytes per launch (decode's ceiling)
        per_shape = {}
        for name, (k, n) in SHAPES.items():
            b = weight_bytes(k, n)
            r = read_dom if name == DOMINANT[0] else read_ceiling(dev, stream, b, max(2, -(-2 * CACHE_BYTES // b)))
            per_shape[name] = {"MB": round(b / 1e6, 1), "GB/s": round(r[0], 1), "blocks": r[1]}
        reads["read_per_launch_by_shape"] = per_shape
    k, n = SHAPES["gate_up"]
    a = torch.randn((PREFILL_M, k), device=dev).to(torch.bfloat16)
    b = torch.randn((k, n), device=dev).to(torch.bfloat16)
    c = torch.empty((PREFILL_M, n), dtype=torch.bfloat16, device=dev)
    ms = time_graph(lambda: torch.matmul(a, b, out=c), stream, 10)
    return {"copy_1GiB_read+write_GB/s": round(copy_gbs, 1), **reads,
            "hipblaslt_bf16_gate_up_m2048_TFLOP/s": round(2 * PREFILL_M * n * k / (ms * 1e-3) / 1e12, 1)}


FUSED_M = (1, 16, 64, 512, 2048)


def fused_gate_up(lib, dev, stream, reps: int) -> dict:
    """Fused SiLU * up epilogue vs the plain gate_up GEMM and the two-step path, each
    graph-replayed over rotating weight copies (decode bytes come from HBM)."""
    k, n = SHAPES["gate_up"]
    copies = max(2, -(-2 * CACHE_BYTES // weight_bytes(k, n)))
    weights = make_weights(k, n, copies, dev, 4242)
    out = {}
    for m in FUSED_M:
        x = torch.randn((m, k), device=dev).to(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        yf = torch.empty((m, n // 2), dtype=torch.bfloat16, device=dev)
        ws_len = lib.workspace_bytes(m, k, n)
        ws = torch.zeros(max(ws_len, 256), dtype=torch.uint8, device=dev)
        wsp = ws.data_ptr() if ws_len else None

        def run(fn_name, dst, act=False):
            def step():
                sp = torch.cuda.current_stream(dev).cuda_stream
                for packed, qzeros, scales in weights:
                    rc = getattr(lib.dll, fn_name)(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(),
                                                   scales.data_ptr(), dst.data_ptr(), m, k, n, 128, wsp, ws_len, sp)
                    if rc != 0:
                        raise RuntimeError(lib.last_error())
                    if act:
                        torch.mul(torch.nn.functional.silu(dst[:, : n // 2]), dst[:, n // 2:], out=yf)
            return time_graph(step, stream, reps) / len(weights)

        fused_ms = run("w4a16_gemm_silu_mul", yf)
        plain_ms = run("w4a16_gemm", y)
        two_ms = run("w4a16_gemm", y, act=True)
        out[f"M={m}"] = {"fused_us": round(fused_ms * 1e3, 2), "gemm_us": round(plain_ms * 1e3, 2),
                         "two_step_us": round(two_ms * 1e3, 2),
                         "saved_vs_two_step": round(1 - fused_ms / two_ms, 4),
                         "fused_TFLOP/s": round(2 * m * n * k / (fused_ms * 1e-3) / 1e12, 1)}
    del weights
    return out


def tp8_shards(lib, dev, stream, steps: int, full_us: dict) -> dict:
    """Each projection's one-GPU share under an eight-way tensor-parallel split, timed like
    the decode points (rotating weight copies beyond the Infinity Cache; two copies at
    M = 2048), against the full shape's time from the same run divided by eight."""
    out = {}
    for si, (name, (k, n)) in enumerate(TP8_SHAPES.items()):
        copies = max(2, -(-(2 * CACHE_BYTES) // weight_bytes(k, n)))
        weights = make_weights(k, n, copies, dev, 700 + si)
        pts = []
        for m in TP8_M:
            gen = torch.Generator(device=dev)
            gen.manual_seed(800 + 10 * si + m)
            x = torch.randn((m, k), device=dev, generator=gen).to(torch.bfloat16)
            pts.append(Point(lib, name, m, k, n, weights if m < PREFILL_M else weights[:2], x))
        per_launch, _ = time_points(pts, stream, steps, 1)
        res = {"K": k, "N": n}
        for p in pts:
            ms = per_launch[id(p)]
            entry = {"us": round(ms * 1e3, 3), "split": p.split}
            if p.m < PREFILL_M:
                entry["GB/s"] = round(algorithmic_bytes(p.m, k, n) / (ms * 1e-3) / 1e9, 1)
            else:
                entry["TFLOP/s"] = round(2 * p.m * n * k / (ms * 1e-3) / 1e12, 1)
            full = full_us.get((name, p.m))
            if full:
                entry["vs_full_over_8"] = round(full / 8 / (ms * 1e3), 3)
            res[f"M={p.m}"] = entry
        out[name] = res
        del pts, weights
    return out


def quantize_throughput(lib, dev, stream, reps: int) -> dict:
    """w4a16_quantize over a [24576, 4096] bf16 weight (the gate_up projection's float
    weight): bytes = 2 per weight read + 0.5 written + scales and zeros."""
    out_f, in_f = 24576, 4096
    w = (torch.randn((out_f, in_f), device=dev) * 0.02).to(torch.bfloat16)
    qw = torch.empty((in_f, out_f // 8), dtype=torch.int32, device=dev)
    qz = torch.empty((in_f // 128, out_f // 8), dtype=torch.int32, device=dev)
    sc = torch.empty((in_f // 128, out_f), dtype=torch.bfloat16, device=dev)

    def step():
        rc = lib.dll.w4a16_quantize(w.data_ptr(), 0, qw.data_ptr(), qz.data_ptr(), sc.data_ptr(), out_f, in_f, 128,
                                    torch.cuda.current_stream(dev).cuda_stream)
        if rc != 0:
            raise RuntimeError(lib.last_error())

    ms = time_graph(step, stream, reps)
    nbytes = out_f * in_f * 2 + out_f * in_f // 2 + (in_f // 128) * out_f * (2 + 0.5)
    return {"shape": [out_f, in_f], "us": round(ms * 1e3, 1), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}


def read_traffic(path: str = TRAFFIC_FILE):
    """HBM bytes per launch recorded in the committed counter summary, or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        return None
    return None


def profile_point(lib, spec: str, steps: int, dev) -> int:
    """Counter/trace workload: one 256 MiB bf16 copy (3x) for calibration, WARM_MS of
    untimed launches, then `steps` direct launches of one decode or prefill point over
    rotating weights.  SHAPE+silu:M
    launches the fused SiLU * up GEMM of that (gate|up) shape, a trailing +norm the
    RMSNorm(+residual) prologue with it (w4a16_gemm_rmsnorm); quantize:0 launches the
    quantizer over a [24576, 4096] bf16 weight.  SHAPE:M:decode forces the decode kernel
    with its own plan (w4a16_plan entry 4) where the planner picks the tile kernel."""
    name, m, *force = spec.split(":")
    m = int(m)
    if name == "quantize":
        q = quantize_throughput(lib, dev, torch.cuda.Stream(dev), steps)
        print(json.dumps({"profile_point": spec, "launches": steps + 2, **q}))
        return 0
    normed = name.endswith("+norm")
    name = name.removesuffix("+norm")
    fused = name.endswith("+silu")
    name = name.removesuffix("+silu")
    entry = lib.dll.w4a16_gemm_silu_mul if fused else lib.dll.w4a16_gemm
    k, n = SHAPES[name]
    if normed:  # the RMSNorm(+residual) prologue and the GEMM in one w4a16_gemm_rmsnorm call
        res = torch.randn((m, k), device=dev).to(torch.bfloat16)
        res_out, xn = torch.empty_like(res), torch.empty_like(res)
        nw = (1 + 0.1 * torch.randn(k, device=dev)).to(torch.bfloat16)

        def entry(xp, pp, zp, sp_, yp, m_, k_, n_, g, wsp, wsl, stp):
            return lib.dll.w4a16_gemm_rmsnorm(xp, res.data_ptr(), nw.data_ptr(), 1e-6, xn.data_ptr(),
                                              res_out.data_ptr(), pp, zp, sp_, yp, m_, k_, n_, g, int(fused), wsp,
                                              wsl, stp)
    src = torch.ones(CALIBRATION_BYTES // 2, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    copies = max(2, -(-2 * CACHE_BYTES // weight_bytes(k, n)))
    weights = make_weights(k, n, copies, dev, 7919 * list(SHAPES).index(name))
    x = torch.randn((m, k), device=dev).to(torch.bfloat16)
    p = Point(lib, name, m, k, n, weights, x)
    stream = torch.cuda.current_stream(dev)
    if force:
        if force != ["decode"] or normed or fused:
            raise ValueError(f"unknown profile point {spec}")
        regime, p0, p1, p2, split = lib.plan(m, k, n, 4)
        p.regime, p.split = "decode", split
        ws_len = max(lib.workspace_bytes_config(m, n, regime, p0, split), 256)
        p.ws = torch.zeros(ws_len, dtype=torch.uint8, device=dev)
        p.ws_len = ws_len

        def entry(xp, pp, zp, sp_, yp, m_, k_, n_, g, wsp, wsl, stp):
            return lib.dll.w4a16_gemm_config(xp, pp, zp, sp_, yp, m_, k_, n_, g, regime, p0, p1, p2, split, wsp, wsl,
                                             stp)

    def launch_all():
        for packed, qzeros, scales in weights:
            if entry(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(), p.y.data_ptr(), m, k, n,
                     128, p.ws.data_ptr() if p.ws_len else None, p.ws_len, stream.cuda_stream) != 0:
                raise RuntimeError(lib.last_error())

    warm_up(launch_all)  # WARM_MS of the same launches first (clock ramp)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    done = 0
    while done < steps:
        for packed, qzeros, scales in weights[: steps - done]:
            rc = entry(x.data_ptr(), packed.data_ptr(), qzeros.data_ptr(), scales.data_ptr(), p.y.data_ptr(), m,
                       k, n, 128, p.ws.data_ptr() if p.ws_len else None, p.ws_len, stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(lib.last_error())
            done += 1
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    print(json.dumps({"profile_point": spec, "launches": steps, "us_per_launch_incl_gaps": round(ms * 1e3, 3),
                      "algorithmic_bytes": algorithmic_bytes(m, k, n), "regime": p.regime, "split": p.split,
                      "calibration_copy_bytes": CALIBRATION_BYTES}))
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the mixed-batch, layer-stack and ceiling legs")
    ap.add_argument("--details", action="store_true", help="print one line per point to stderr")
    ap.add_argument("--profile-point", metavar="SHAPE:M", help="profiling workload for one point (see doc)")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this path has no multi-GPU "
              f"component: each GPU runs its own layers' GEMMs)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    pkg = importlib.import_module("llm-serve_amd")
    lib = pkg.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.profile_point:
        return profile_point(lib, args.profile_point, args.steps, dev)
    stream = torch.cuda.Stream(dev)

    decode_points = build_points(lib, DECODE_M + EXTRA_DECODE_M, dev)
    per_launch, _ = time_points(decode_points, stream, args.steps, args.warmup)
    head = [p for p in decode_points if p.m in DECODE_M]
    bytes_head = sum(algorithmic_bytes(p.m, p.k, p.n) for p in head)
    ms_head = sum(per_launch[id(p)] for p in head)
    value = bytes_head / (ms_head * 1e-3) / 1e9
    dom = next(p for p in head if (p.name, p.m) == DOMINANT)
    dom_ms = per_launch[id(dom)]
    dom_gbs = algorithmic_bytes(dom.m, dom.k, dom.n) / (dom_ms * 1e-3) / 1e9
    points_out = []
    samples = time_points.samples
    for p in decode_points:
        ms = per_launch[id(p)]
        gbs = algorithmic_bytes(p.m, p.k, p.n) / (ms * 1e-3) / 1e9
        sv = samples[id(p)]
        points_out.append({"shape": p.name, "M": p.m, "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "split": p.split, "copies": p.launches,
                           "us_median": round(statistics.median(sv) * 1e3, 3),
                           "us_min": round(min(sv) * 1e3, 3), "us_max": round(max(sv) * 1e3, 3)})
        if args.details:
            print(f"decode {p.name:8s} M={p.m:3d} {ms * 1e3:8.2f} us  {gbs:8.1f} GB/s  split={p.split}",
                  file=sys.stderr)
    del decode_points

    prefill = None
    if not args.no_prefill:
        pts = []
        for si, (name, (k, n)) in enumerate(SHAPES.items()):
            gen = torch.Generator(device=dev)
            gen.manual_seed(99 + si)
            x = torch.randn((PREFILL_M, k), device=dev, generator=gen)
            cols = torch.randperm(k, device=dev, generator=gen)[: round(0.01 * k)]
            x[:, cols] *= 20.0
            pts.append(Point(lib, name, PREFILL_M, k, n, make_weights(k, n, 2, dev, 500 + si), x.to(torch.bfloat16)))
        pl, _ = time_points(pts, stream, max(5, args.steps // 2), 1)
        prefill = {}
        for p in pts:
            ms = pl[id(p)]
            tf = 2 * p.m * p.n * p.k / (ms * 1e-3) / 1e12
            prefill[p.name] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                               "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "split": p.split}
            if args.details:
                print(f"prefill {p.name:8s} M={p.m} {ms * 1e3:9.2f} us {tf:8.1f} TFLOP/s", file=sys.stderr)
        del pts

    mixed = stack = stack_chained = stack_normed = ceilings = fused = quant = norm = tp8 = None
    if not args.no_extra:
        mixed = mixed_batch(lib, dev, stream, max(3, args.steps // 4))
        stack, stack_chained, stack_normed = layer_stack(lib, dev, stream, max(2, args.steps // 10))
        ceilings = measured_ceilings(dev, stream)
        fused = fused_gate_up(lib, dev, stream, max(3, args.steps // 4))
        quant = quantize_throughput(lib, dev, stream, max(3, args.steps // 4))
        norm = norm_prologue(lib, dev, stream, max(3, args.steps // 4))
        full_us = {(pt["shape"], pt["M"]): pt["us"] for pt in points_out}
        full_us.update({(name, PREFILL_M): v["us"] for name, v in (prefill or {}).items()})
        tp8 = tp8_shards(lib, dev, stream, max(3, args.steps // 4), full_us)
        if args.details:
            print(f"mixed M={MIXED_M}: {json.dumps(mixed)}", file=sys.stderr)
            print(f"stack36: {json.dumps(stack)}", file=sys.stderr)
            print(f"stack36_chained: {json.dumps(stack_chained)}", file=sys.stderr)
            print(f"ceilings: {json.dumps(ceilings)}", file=sys.stderr)
            print(f"fused gate_up: {json.dumps(fused)}", file=sys.stderr)
            print(f"quantize: {json.dumps(quant)}", file=sys.stderr)
            print(f"stack36_normed: {json.dumps(stack_normed)}", file=sys.stderr)
            print(f"rmsnorm_prologue: {json.dumps(norm)}", file=sys.stderr)
            print(f"tp8_shards: {json.dumps(tp8)}", file=sys.stderr)

    by_shape = (ceilings or {}).get("read_per_launch_by_shape", {})
    for pt in points_out:  # each decode point against a plain read of its shape's weight bytes
        if pt["shape"] in by_shape:
            pt["read_ceiling_frac"] = round(pt["GB/s"] / by_shape[pt["shape"]]["GB/s"], 4)
    cpu = None if args.no_cpu else cpu_baseline(gpu_gemm=lambda prob: gpu_gemm_bits(pkg, dev, prob))
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_head, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "decode sweep: AWQ W4A16 GEMM, group 128, M in {1,4,8,16} x Qwen3-8B "
                               "QKV 4096x6144, O 4096x4096, gate_up 4096x24576, down 12288x4096",
                   "group_size": 128, "weights_rotated_bytes_per_point": ">= 512 MiB"},
        "roofline": {"kernel": f"decode {DOMINANT[0]} {dom.k}x{dom.n} M={DOMINANT[1]}", "bound": "hbm",
                     "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "algorithmic_bytes": algorithmic_bytes(dom.m, dom.k, dom.n),
                     "launch_us": round(dom_ms * 1e3, 3), **measured_frac(dom_gbs, ceilings)},
        "cpu_baseline": cpu,
        "prefill_m2048": prefill,
        "mixed_m512": mixed,
        "stack36": stack,
        "stack36_chained": stack_chained,
        "stack36_normed": stack_normed,
        "measured_ceilings": ceilings,
        "fused_gate_up": fused,
        "quantize": quant,
        "rmsnorm_prologue": norm,
        "tp8_shards": tp8,
        "points": points_out,
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
