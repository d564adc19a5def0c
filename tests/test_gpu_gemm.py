"""GPU parity of the W4A16 GEMM (decode split-K kernel and MFMA tile kernel).

Small sizes compare against the CPU oracle (fp64-accumulated x @ W over the reference's
bf16 weights).  Full Qwen3-8B sizes compare against the oracle itself at M = 1, 16, 64 and
2048, and at the other M against torch fp32 matmul on the GPU over the bit-exact
dequantized weights (checked separately against the oracle in test_gpu_format.py).
Tolerance: max |y - r| / max(|r|, rms(r)) <= 1e-2 (GEMM_REL_TOL), plus the reference's own
assert_close tolerances where its tests state them."""
import numpy as np
import pytest
import torch

from awq_helpers import (GEMM_REL_TOL, QWEN3_SHAPES, awq_mod, bf16_from_bits, bits_of, decode_config_accepted,
                         golden_cases, pkg, random_awq_gpu, random_x_gpu, rel_err, to_gpu, assert_gemm_close)
from oracle import awq_oracle as ora

pytestmark = pytest.mark.gpu


def hip_linear(t, packed=None, workspace=None):
    awq = awq_mod()
    packed = awq.repack_awq_qweight(t["qweight"]) if packed is None else packed
    return awq.awq_linear(t["x"], packed, t["qzeros"], t["scales"], group_size=128, workspace=workspace)


@pytest.mark.parametrize("case", sorted(golden_cases()))
def test_gemm_matches_oracle_on_golden_fixtures(gpu_lib, case):
    """Every golden case, the special-scale one included (zero, negative, bf16-subnormal,
    tiny and 3e30 scales; its outputs reach 6e32 and stay finite)."""
    c = golden_cases()[case]
    t = to_gpu({"qweight": c["qweight"], "qzeros": c["qzeros"], "scales_bits": c["scales_bits"],
                "x_bits": c["x_bits"]})
    y = hip_linear(t)
    assert y.dtype == torch.bfloat16 and y.shape == c["y_f64"].shape
    assert_gemm_close(y, c["y_f64"])
    if case == "special_scales":  # the 3e30 columns dominate rms(r): each column on its own scale too
        for j in range(y.shape[1]):
            assert rel_err(y[:, j], c["y_f64"][:, j]) <= GEMM_REL_TOL, j


def test_decode_token_counts_reference_recipe(gpu_lib):
    """tests/test_awq_cuda.py:110-155: seed 17, K=128, N=64, M in {1,4,8,16,32,65,128},
    assert_close(rtol=0.02, atol=0.05) against the reference backend."""
    rng = np.random.default_rng(17)
    k, n = 128, 64
    q = rng.integers(0, 16, size=(k, n))
    z = rng.integers(0, 16, size=(1, n))
    s = ora.f32_to_bf16_bits(rng.random((1, n)).astype(np.float32) * 0.05)
    base = {"qweight": ora.pack_awq_int4(q), "qzeros": ora.pack_awq_int4(z), "scales_bits": s}
    for m in (1, 4, 8, 16, 32, 65, 128):
        x = ora.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
        t = to_gpu(dict(base, x_bits=x))
        y = hip_linear(t)
        want = ora.bf16_bits_to_f32(ora.awq_linear_bf16_bits(x, base["qweight"], base["qzeros"], s, 128))
        torch.testing.assert_close(y.float().cpu(), torch.from_numpy(want), rtol=0.02, atol=0.05)
        assert_gemm_close(y, ora.awq_linear_ref(x, base["qweight"], base["qzeros"], s, 128))


def test_single_token_wide_gemv_reference_recipe(gpu_lib):
    """tests/test_awq_triton.py:83-113: M=1, K=128, N=16384, rtol=0.01, atol=0.02."""
    p = ora.make_problem(seed=11, m=1, k=128, n=16384, scale_lo=0.0, scale_hi=0.05)
    t = to_gpu(p)
    y = hip_linear(t)
    want = ora.bf16_bits_to_f32(ora.awq_linear_bf16_bits(p["x_bits"], p["qweight"], p["qzeros"],
                                                         p["scales_bits"], 128))
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(want), rtol=0.01, atol=0.02)


DECODE_CONFIGS = [(tn, w, d, s) for tn in (1, 2, 3, 4, 6) for w in (4, 8, 12) for d in (1, 2, 4) for s in (1, 3, 8)]


@pytest.mark.parametrize("m", [1, 3, 5, 16, 33, 64])
def test_every_decode_configuration(gpu_lib, m):
    """All column-tile / wave / depth / split combinations of the decode kernel, incl. uneven
    splits, waves with no group and prefetch rings that wrap (K = 2048: 16 groups; N = 768:
    48 column tiles, divisible by every tile count); M <= 4 runs with staged activations."""
    k, n = 2048, 768
    p = ora.make_problem(seed=100 + m, m=m, k=k, n=n)
    t = to_gpu(p)
    packed = awq_mod().repack_awq_qweight(t["qweight"])
    want = ora.awq_linear_ref(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128)
    for tn, waves, depth, split in DECODE_CONFIGS:
        if not decode_config_accepted(m, k, tn, depth, waves, split):
            continue  # rejected by the library, see test_capi
        ws_bytes = gpu_lib.workspace_bytes_config(m, n, 1, tn, split)
        ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
        y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        gpu_lib.gemm_config(t["x"], packed, t["qzeros"], t["scales"], y, k, n, 1, tn, waves, split, ws, p2=depth)
        assert_gemm_close(y, want, (tn, waves, depth, split))
        if ws_bytes:  # arrival counters (the first 64 KiB) are re-armed to zero
            assert int(torch.count_nonzero(ws[:65536])) == 0


@pytest.mark.parametrize("m", [1, 5, 40])
def test_decode_long_k_stays_within_lds(gpu_lib, m):
    """K = 65536 (512 groups): the per-wave staged scales and zeros of one workgroup would
    exceed LDS without a K split; the planner splits K until they fit."""
    k, n = 65536, 64
    p = ora.make_problem(seed=300 + m, m=m, k=k, n=n)
    t = to_gpu(p)
    y = hip_linear(t)
    assert_gemm_close(y, ora.awq_linear_ref(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128))


# (wm, tile shape code, occupancy): every compiled tile kernel (see launch_tile_cfg)
TILE_KERNELS = [(4, 1, 1), (4, 1, 2), (8, 1, 1), (4, 2, 2), (4, 3, 2), (8, 3, 2), (2, 4, 2), (4, 4, 2), (2, 5, 2),
                (4, 5, 2), (8, 5, 2), (4, 6, 1), (8, 6, 1), (2, 7, 1), (4, 7, 1), (8, 8, 2),
                (4, 9, 3), (2, 9, 3), (4, 10, 3), (8, 11, 2),
                (4, 11, 2), (6, 3, 2), (6, 8, 2), (6, 11, 2)]
# output columns of one wave per tile shape code where they are not 32 or 64 (the library
# rejects an output width that would split a wave)
WAVE_COLS = {11: 48}
TILE_CONFIGS = [(wm, shape, occ, split) for wm, shape, occ in TILE_KERNELS for split in (1, 2, 3, 4)]


@pytest.mark.parametrize("m,n", [(65, 512), (200, 768), (300, 320), (513, 256), (200, 576)])
def test_every_tile_configuration(gpu_lib, m, n):
    """Every compiled tile kernel and split: partial m-blocks (rows clamped and dropped),
    n-blocks partly past N (waves with no columns; n = 576 puts the last 384-column block of
    the 48-column-wave shape half past N), uneven K splits."""
    k = 1024
    p = ora.make_problem(seed=200 + m, m=m, k=k, n=n)
    t = to_gpu(p)
    packed = awq_mod().repack_awq_qweight(t["qweight"])
    want = ora.awq_linear_ref(p["x_bits"], p["qweight"], p["qzeros"], p["scales_bits"], 128)
    for wm, shape, occ, split in TILE_CONFIGS:
        if n % WAVE_COLS.get(shape, 1):
            continue  # rejected by the library, see test_capi
        ws_bytes = gpu_lib.workspace_bytes_config(m, n, 2, wm, split)
        ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
        y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        gpu_lib.gemm_config(t["x"], packed, t["qzeros"], t["scales"], y, k, n, 2, wm, occ, split, ws, p2=shape)
        assert_gemm_close(y, want, (wm, shape, occ, split))
        if ws_bytes:  # arrival counters (the first 64 KiB) are re-armed to zero
            assert int(torch.count_nonzero(ws[:65536])) == 0


def test_scales_and_zeros_at_word_alignment(gpu_lib):
    """The API asks only 4-byte alignment of scales and qzeros, while both kernels fetch them
    in 16-byte chunks: every tile kernel, and the planner's decode and tile plans, give the
    same bits for tensors 4 bytes past a 16-byte boundary as for aligned ones."""
    m, k, n = 200, 1024, 512
    p = ora.make_problem(seed=77, m=m, k=k, n=n)
    t = to_gpu(p)
    packed = awq_mod().repack_awq_qweight(t["qweight"])
    s_buf = torch.zeros(t["scales"].numel() + 8, dtype=torch.bfloat16, device="cuda")
    z_buf = torch.zeros(t["qzeros"].numel() + 4, dtype=torch.int32, device="cuda")
    s_off = s_buf[2:2 + t["scales"].numel()].view(t["scales"].shape)
    z_off = z_buf[1:1 + t["qzeros"].numel()].view(t["qzeros"].shape)
    s_off.copy_(t["scales"])
    z_off.copy_(t["qzeros"])
    assert s_off.data_ptr() % 16 == 4 and z_off.data_ptr() % 16 == 4
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    for wm, shape, occ in TILE_KERNELS:
        if n % WAVE_COLS.get(shape, 1):
            continue
        ys = []
        for s, z in ((t["scales"], t["qzeros"]), (s_off, z_off)):
            y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
            gpu_lib.gemm_config(t["x"], packed, z, s, y, k, n, 2, wm, occ, 1, ws, p2=shape)
            ys.append(y)
        assert torch.equal(ys[0].view(torch.int16), ys[1].view(torch.int16)), (wm, shape, occ)
    for rows in (1, 16, 200):
        x = t["x"][:rows]
        a = awq_mod().awq_linear(x, packed, t["qzeros"], t["scales"], group_size=128, workspace=ws)
        b = awq_mod().awq_linear(x, packed, z_off, s_off, group_size=128, workspace=ws)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), rows


def test_shared_workspace_across_shapes_and_m(gpu_lib):
    """One workspace reused by calls of different M and N (as the per-device pool does):
    the counters must always be found re-armed."""
    k = 4096
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    for n in (4096, 6144):
        qw, qz, s = random_awq_gpu(k, n, seed=n)
        packed = awq_mod().repack_awq_qweight(qw)
        for m in (1, 4, 16, 64, 200, 16, 1):
            x = random_x_gpu(m, k, seed=m)
            y = awq_mod().awq_linear(x, packed, qz, s, group_size=128, workspace=ws)
            assert_gemm_close(y, full_reference(x, qw, qz, s), (n, m))
    assert int(torch.count_nonzero(ws[:65536])) == 0


def test_split_k_results_are_deterministic(gpu_lib):
    k, n = 4096, 4096
    qw, qz, s = random_awq_gpu(k, n, seed=3)
    packed = awq_mod().repack_awq_qweight(qw)
    for m in (16, 300):
        x = random_x_gpu(m, k, seed=m)
        a = awq_mod().awq_linear(x, packed, qz, s, group_size=128)
        b = awq_mod().awq_linear(x, packed, qz, s, group_size=128)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def full_reference(x, qw, qz, s):
    w = awq_mod().dequantize_awq_gemm(qw, qz, s, group_size=128)
    return x.float() @ w.float()


@pytest.mark.parametrize("shape", sorted(QWEN3_SHAPES))
def test_full_qwen3_shapes_decode_sweep(gpu_lib, shape):
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=11)
    packed = awq_mod().repack_awq_qweight(qw)
    for m in (1, 4, 8, 16, 31, 32, 64):
        assert pkg().awq_regime(m, k, n) == ("decode" if m < 32 else "tile")
        x = random_x_gpu(m, k, seed=m)
        y = awq_mod().awq_linear(x, packed, qz, s, group_size=128)
        assert_gemm_close(y, full_reference(x, qw, qz, s), (m))


@pytest.mark.parametrize("shape", sorted(QWEN3_SHAPES))
def test_full_qwen3_shapes_against_the_oracle(gpu_lib, shape):
    """Full shapes against the CPU oracle itself (its own dequant, fp64 x @ W;
    awq.py:235-276): one decode launch at M = 1 and 16, a mid-M tile launch at 64 and a
    prefill chunk of 2048 rows with activation outliers, all rows through one oracle call."""
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=21)
    packed = awq_mod().repack_awq_qweight(qw)
    ms = (1, 16, 64, 2048)
    xs = [random_x_gpu(m, k, seed=40 + m, outliers=m == 2048) for m in ms]
    ys = [awq_mod().awq_linear(x, packed, qz, s, group_size=128) for x in xs]
    torch.cuda.synchronize()
    want = ora.awq_linear_ref(np.concatenate([bits_of(x) for x in xs]), qw.cpu().numpy(), qz.cpu().numpy(),
                              bits_of(s), 128)
    r0 = 0
    for m, y in zip(ms, ys):
        print(f"oracle full shape {shape} m={m} regime={pkg().awq_regime(m, k, n)}", flush=True)
        assert_gemm_close(y, torch.from_numpy(want[r0:r0 + m]).cuda(), (shape, m))
        r0 += m


@pytest.mark.parametrize("shape", sorted(QWEN3_SHAPES))
def test_full_qwen3_shapes_prefill_chunk_with_outliers(gpu_lib, shape):
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=12)
    packed = awq_mod().repack_awq_qweight(qw)
    x = random_x_gpu(2048, k, seed=7, outliers=True)
    assert pkg().awq_regime(2048, k, n) == "tile"
    y = awq_mod().awq_linear(x, packed, qz, s, group_size=128)
    assert_gemm_close(y, full_reference(x, qw, qz, s), "prefill")


@pytest.mark.parametrize("shape", sorted(QWEN3_SHAPES))
@pytest.mark.parametrize("m", [96, 128])
def test_full_qwen3_shapes_verify_and_stack_batches(gpu_lib, shape, m):
    """M = 128 (the largest batched decode step of the 36-layer stack workload) and M = 96 at the
    four full shapes, with activation outliers: the planner's mid-M plans (K split over
    workgroups and waves) against the fp32 reference over the oracle-pinned dequant."""
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=15 + m)
    packed = awq_mod().repack_awq_qweight(qw)
    x = random_x_gpu(m, k, seed=m + 3, outliers=True)
    print(f"full shape {shape} m={m} regime={pkg().awq_regime(m, k, n)} split={gpu_lib.split_k(m, k, n)}", flush=True)
    y = awq_mod().awq_linear(x, packed, qz, s, group_size=128)
    assert_gemm_close(y, full_reference(x, qw, qz, s), (shape, m))


@pytest.mark.parametrize("shape,m", [("qkv", 768), ("o", 768), ("gate_up", 256), ("down", 384), ("down", 768),
                                     ("gate_up", 31), ("gate_up", 32), ("gate_up", 48), ("gate_up", 49),
                                     ("o", 31), ("o", 32), ("o", 33), ("qkv", 33), ("down", 31), ("down", 48),
                                     ("down", 33), ("down", 257), ("qkv", 257),
                                     ("gate_up", 160), ("qkv", 160), ("o", 160), ("down", 192), ("o", 640),
                                     ("down", 640), ("qkv", 704), ("down", 896), ("gate_up", 640), ("down", 4),
                                     ("gate_up", 288), ("gate_up", 864), ("qkv", 288), ("o", 288), ("down", 288),
                                     ("qkv", 400), ("o", 513), ("o", 705)])
def test_full_qwen3_shapes_at_planner_boundaries(gpu_lib, shape, m):
    """Chunk sizes where the planner picks 128-row tiles with K split to fill one round
    (QKV / down at M = 768, gate_up at 256, down at 384), the decode / tile boundary
    (decode below M = 32, the tile kernel's 32- and 64-row plans above), the end of the mid-range plans
    (M = 257), the mid-range row blocks that follow M (96 x 256 tiles on gate_up, 32-row
    tiles on QKV / O, 64-row tiles split in K on down at M = 160 / 192), the plans above M =
    512 (96 x 256 tiles with K in two on down at 640, the best-filling narrow and wide
    tiles at QKV 704, gate_up 640, down 896 with 128 x 256 tiles and K in two), the 384-column
    tiles of 96 and 128 rows the wide layers take by useful work per round (gate_up M = 288,
    864), the 64-row tiles of narrow layers just above M = 256 (QKV 64 x 128, O 64 x 96, down
    64 x 192 with K in two at M = 288; QKV 64 x 192 at M = 400), O's 64 x 192 tiles at M =
    513 .. 704 (513, 640) and 128 x 128 tiles without a K split at 705 .. 768 (705, 768) and
    the long-K decode split at M = 4, at full shapes."""
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=14 + m)
    packed = awq_mod().repack_awq_qweight(qw)
    x = random_x_gpu(m, k, seed=m, outliers=True)
    assert pkg().awq_regime(m, k, n) == ("decode" if m < 32 else "tile")
    y = awq_mod().awq_linear(x, packed, qz, s, group_size=128)
    assert_gemm_close(y, full_reference(x, qw, qz, s), (shape, m))


@pytest.mark.parametrize("shape", ["gate_up", "down"])
def test_mixed_ragged_batch_m512(gpu_lib, shape):
    """48 decode rows + 8 x 4 verify rows + a 432-row prefill chunk packed into M = 512."""
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=13)
    x = torch.cat([random_x_gpu(48, k, 1), random_x_gpu(32, k, 2), random_x_gpu(432, k, 3, outliers=True)])
    y = awq_mod().awq_linear(x, awq_mod().repack_awq_qweight(qw), qz, s, group_size=128)
    assert_gemm_close(y, full_reference(x, qw, qz, s))
    # rows are independent: the 48 decode rows alone give the same values within rounding
    y48 = awq_mod().awq_linear(x[:48].contiguous(), awq_mod().repack_awq_qweight(qw), qz, s, group_size=128)
    assert rel_err(y48, y[:48].float()) <= GEMM_REL_TOL


@pytest.mark.parametrize("m", [0, 17, 63, 65, 100, 255, 257])
def test_ragged_m(gpu_lib, m):
    k, n = 512, 256
    qw, qz, s = random_awq_gpu(k, n, seed=m + 1)
    x = random_x_gpu(m, k, seed=m) if m else torch.empty((0, k), dtype=torch.bfloat16, device="cuda")
    y = awq_mod().awq_linear(x, awq_mod().repack_awq_qweight(qw), qz, s, group_size=128)
    assert y.shape == (m, n)
    if m:
        assert_gemm_close(y, full_reference(x, qw, qz, s))


def test_leading_dims_are_flattened(gpu_lib):
    k, n = 256, 128
    qw, qz, s = random_awq_gpu(k, n, seed=4)
    x = random_x_gpu(6, k, seed=4).view(2, 3, k)
    y = awq_mod().awq_linear(x, awq_mod().repack_awq_qweight(qw), qz, s, group_size=128)
    assert y.shape == (2, 3, n)
    assert_gemm_close(y.reshape(6, n), full_reference(x.reshape(6, k), qw, qz, s))


def test_too_small_workspace_is_an_error(gpu_lib):
    k, n, m = 12288, 4096, 16  # the down projection: split-K, so a workspace is needed
    qw, qz, s = random_awq_gpu(k, n, seed=5)
    need = gpu_lib.workspace_bytes(m, k, n)
    assert need > 0
    ws = torch.zeros(need - 256, dtype=torch.uint8, device="cuda")
    with pytest.raises(pkg().W4A16Error, match="workspace"):
        awq_mod().awq_linear(random_x_gpu(m, k, 1), awq_mod().repack_awq_qweight(qw), qz, s, group_size=128,
                             workspace=ws)


def test_zero_scales_and_q_equal_z_give_zero(gpu_lib):
    k, n = 256, 128
    qw, qz, s = random_awq_gpu(k, n, seed=6)
    packed = awq_mod().repack_awq_qweight(qw)
    for m in (8, 128):
        x = random_x_gpu(m, k, seed=1)
        y = awq_mod().awq_linear(x, packed, qz, torch.zeros_like(s), group_size=128)
        assert torch.count_nonzero(y.float()) == 0
    # q == z everywhere (every row takes its group's zero words): W == 0 exactly, so both
    # kernels multiply exact zero weights and y is exactly 0.
    q_equal_z = qz.repeat_interleave(128, dim=0).contiguous()
    packed = awq_mod().repack_awq_qweight(q_equal_z)
    for m in (8, 128):
        y = awq_mod().awq_linear(random_x_gpu(m, k, seed=2), packed, qz, s, group_size=128)
        assert torch.count_nonzero(y.float()) == 0


def test_layer_forward_matches_oracle(gpu_lib):
    """tests/test_awq_linear_backend.py:125-148 pattern (q = arange % 16, z = 8, linspace scales)
    through ColumnParallelLinear -> AWQLinearMethod.apply on the GPU."""
    import importlib

    linear = importlib.import_module("llm-serve_amd.layers.linear")
    awq = awq_mod()
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    k, n = 128, 64
    with torch.device("cuda"):
        layer = linear.ColumnParallelLinear(k, n, quant_config=cfg)
    q = np.arange(k * n).reshape(k, n) % 16
    z = np.full((1, n), 8)
    s_bits = ora.f32_to_bf16_bits(np.linspace(0.01, 0.64, n, dtype=np.float32).reshape(1, n))
    qweight, qzeros = ora.pack_awq_int4(q), ora.pack_awq_int4(z)
    layer.qweight.weight_loader(layer.qweight, torch.from_numpy(qweight).cuda())
    layer.qzeros.weight_loader(layer.qzeros, torch.from_numpy(qzeros).cuda())
    layer.scales.weight_loader(layer.scales, bf16_from_bits(s_bits))
    layer.quant_method.process_weights_after_loading(layer)
    assert not hasattr(layer, "qweight") and not hasattr(layer, "qzeros")
    for m in (4, 100):
        x_bits = ora.f32_to_bf16_bits(np.random.default_rng(m).standard_normal((m, k)).astype(np.float32))
        y = layer(bf16_from_bits(x_bits))
        want = ora.awq_linear_ref(x_bits, qweight, qzeros, s_bits, 128)
        assert_gemm_close(y, want)


def test_row_parallel_layer_forward(gpu_lib):
    import importlib

    linear = importlib.import_module("llm-serve_amd.layers.linear")
    awq = awq_mod()
    cfg = awq.AWQRuntimeConfig(bits=4, group_size=128, zero_point=True, version="gemm", backend="autoawq",
                               activation_dtype=torch.bfloat16)
    k, n = 1024, 256
    qw, qz, s = random_awq_gpu(k, n, seed=9)
    with torch.device("cuda"):
        layer = linear.RowParallelLinear(k, n, quant_config=cfg)
    layer.qweight.weight_loader(layer.qweight, qw)
    layer.qzeros.weight_loader(layer.qzeros, qz)
    layer.scales.weight_loader(layer.scales, s)
    layer.quant_method.process_weights_after_loading(layer)
    x = random_x_gpu(16, k, seed=3)
    assert_gemm_close(layer(x), full_reference(x, qw, qz, s))


def test_hip_graph_capture_replays_match_eager(gpu_lib):
    """A captured decode GEMM with a split-K reduction (counters live in the workspace)
    replayed several times, with eager work in between, matches the eager result."""
    k, n, m = 12288, 4096, 16  # the down projection
    qw, qz, s = random_awq_gpu(k, n, seed=21)
    awq = awq_mod()
    packed = awq.repack_awq_qweight(qw)
    assert gpu_lib.split_k(m, k, n) > 1
    x = random_x_gpu(m, k, seed=1)
    eager = awq.awq_linear(x, packed, qz, s, group_size=128).clone()
    static_x = x.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        awq.awq_linear(static_x, packed, qz, s, group_size=128)  # warm the per-device workspace
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        static_y = awq.awq_linear(static_x, packed, qz, s, group_size=128)
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_y.view(torch.int16), eager.view(torch.int16)), i
        _ = awq.awq_linear(random_x_gpu(m, k, seed=50 + i), packed, qz, s, group_size=128)
        torch.cuda.synchronize()


def test_activations_beyond_2gib_run_in_row_chunks(gpu_lib):
    """M x K bf16 activations of more than 2 GiB (K = 4096, M = 263000: 2.15 GB): the tile
    regime launches row chunks below 2 GiB in order; rows on both sides of the chunk
    boundary and at both ends match the reference."""
    k, n, m = 4096, 64, 263000
    fit = (2 ** 31 - 1) // (2 * k)
    assert m * k * 2 >= 2 ** 31 and m > fit
    qw, qz, s = random_awq_gpu(k, n, seed=77)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    x = torch.randn((m, k), device="cuda", dtype=torch.bfloat16, generator=g)
    print(f"2 GiB activations: m={m} k={k} n={n}", flush=True)
    y = awq_mod().awq_linear(x, awq_mod().repack_awq_qweight(qw), qz, s, group_size=128)
    assert y.shape == (m, n)
    for lo, hi in ((0, 512), (fit - 1024, fit + 1024), (m - 512, m)):
        assert_gemm_close(y[lo:hi], full_reference(x[lo:hi], qw, qz, s), (lo, hi))
    del x, y
    torch.cuda.empty_cache()
