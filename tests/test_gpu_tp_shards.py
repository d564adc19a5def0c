"""Parity at the per-GPU shapes of the Qwen3-8B projections split eight ways: QKV and
gate_up column-parallel on N, O and down row-parallel on K (linear.py:14-21, 136-146,
178-196, 217-226), i.e. QKV 4096 x 768, O 512 x 4096, gate_up 4096 x 3072 and down
1536 x 4096.  One GPU shows the kernels on its share at its real shape; the all-reduce of
the row-parallel outputs lies outside this library.

The chunk sizes reach every plan these shapes take: the decode kernel's small-shape rules
(K split in four below 128 column tiles, unsplit 4-wave workgroups below 16 groups), the
mid-range tiles of 32 columns and four K slices, and the modelled tile choice beyond
M = 128.  Plain GEMMs are checked against the CPU oracle itself (awq.py:235-276, fp64
x @ W over its own dequant), the fused SiLU * up on the gate_up shard against the
reference's two steps."""
import numpy as np
import pytest
import torch

from awq_helpers import assert_gemm_close, assert_silu_two_step, awq_mod, bits_of, pkg, random_awq_gpu, random_x_gpu
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
