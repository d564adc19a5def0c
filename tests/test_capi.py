"""C ABI checks that need no GPU: the library loads, exports every symbol the header
declares, and its host-side validation / dispatch queries behave (no kernel launches)."""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "w4a16.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(w4a16_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_surface():
    names = declared_functions()
    for required in ("w4a16_gemm", "w4a16_dequant", "w4a16_repack_qweight", "w4a16_workspace_bytes",
                     "w4a16_last_error", "w4a16_regime", "w4a16_unpack_int4"):
        assert required in names


def test_library_exports_every_declared_symbol(pkg):
    dll = pkg.lib().dll
    missing = [name for name in declared_functions() if not hasattr(dll, name)]
    assert not missing, missing


def test_binding_signatures_cover_the_header(pkg):
    from importlib import import_module

    sigs = import_module("llm-serve_amd._lib")._SIGNATURES
    assert sorted(sigs) == declared_functions()


def test_abi_version_and_empty_error(pkg):
    L = pkg.lib()
    assert L.dll.w4a16_abi_version() == 5
    assert isinstance(L.last_error(), str)


@pytest.mark.parametrize("m,k,n,group,code,msg", [
    (16, 4000, 4096, 128, 2, "K must be divisible by 128"),
    (16, 4096, 4100, 128, 2, "N must be divisible by 64"),
    (16, 4096, 4096, 64, 2, "group_size must be 128"),
    (-1, 4096, 4096, 128, 1, "M must be"),
    (16, 4096, 4096, 128, 1, "null tensor pointer"),
])
def test_gemm_rejects_bad_arguments_without_touching_the_gpu(pkg, m, k, n, group, code, msg):
    L = pkg.lib()
    rc = L.dll.w4a16_gemm(None, None, None, None, None, m, k, n, group, None, 0, None)
    assert rc == code
    assert msg in L.last_error()


def test_gemm_m_zero_is_a_noop(pkg):
    L = pkg.lib()
    assert L.dll.w4a16_gemm(None, None, None, None, None, 0, 4096, 4096, 128, None, 0, None) == 0


def test_misaligned_pointer_is_rejected(pkg):
    L = pkg.lib()
    buf = (ctypes.c_uint8 * 64)()
    base = ctypes.addressof(buf)
    p = base + (16 - base % 16) % 16 + 2  # 2 bytes past a 16-byte boundary
    rc = L.dll.w4a16_gemm(p, p, p, p, p, 16, 4096, 4096, 128, None, 0, None)
    assert rc == 3 and "aligned" in L.last_error()


def test_format_entry_points_validate_shapes(pkg):
    L = pkg.lib()
    assert L.dll.w4a16_repack_qweight(None, None, 100, 64, None) == 2
    assert L.dll.w4a16_repack_qweight(None, None, 128, 8, None) == 2
    assert L.dll.w4a16_dequant(None, None, None, None, 4, 12, 2, None) == 2  # N % 8
    assert L.dll.w4a16_dequant(None, None, None, None, 5, 8, 2, None) == 2   # K % group
    assert L.dll.w4a16_dequant_packed(None, None, None, None, 128, 64, 64, None) == 2
    assert L.dll.w4a16_unpack_int4(None, None, 0, 4, None) == 1


QWEN3 = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 24576), "down": (12288, 4096)}


def test_regime_boundary_and_split_limits(pkg):
    L = pkg.lib()
    for k, n in QWEN3.values():
        assert L.regime(0, k, n) == 0
        for m in (1, 4, 8, 16, 31, 32, 33, 48, 49, 64):
            # decode kernel below M = 32, the tile kernel from M = 32 on
            assert L.regime(m, k, n) == (1 if m < 32 else 2)
            assert 1 <= L.split_k(m, k, n) <= k // 128
        for m in (65, 128, 512, 2048, 4096):
            assert L.regime(m, k, n) == 2
            assert 1 <= L.split_k(m, k, n) <= k // 128


def test_workspace_covers_partials_and_counters(pkg):
    L = pkg.lib()
    for k, n in QWEN3.values():
        for m in (1, 16, 64, 128, 512, 2048):
            split = L.split_k(m, k, n)
            ws = L.workspace_bytes(m, k, n)
            # up to M = 8 the query also covers the fused-norm consumer's plans, which may
            # split K where the plain GEMM does not
            consumer = [L.plan(m, k, n, e)[4] for e in ((2, 3) if n % 128 == 0 else (2,))] if m <= 8 else []
            if split == 1 and all(s == 1 for s in consumer):
                assert ws == 0
            else:
                assert ws >= split * m * n * 4 + 4
    assert L.workspace_bytes(16, 4096, 4096, 64) == 0  # invalid group -> 0


def test_forced_config_validation(pkg):
    L = pkg.lib()
    f = L.dll.w4a16_gemm_config
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.addressof(buf) + (16 - ctypes.addressof(buf) % 16) % 16
    assert f(p, p, p, p, p, 128, 4096, 4096, 128, 1, 4, 4, 2, 1, None, 0, None) == 2  # decode needs M <= 64
    assert f(p, p, p, p, p, 16, 4096, 4096, 128, 1, 5, 4, 2, 1, None, 0, None) == 1  # bad tiles
    assert f(p, p, p, p, p, 16, 4096, 4096, 128, 1, 3, 4, 2, 1, None, 0, None) == 2  # 3 does not divide N/16
    assert f(p, p, p, p, p, 16, 4096, 4096, 128, 1, 4, 5, 2, 1, None, 0, None) == 1  # bad waves
    assert f(p, p, p, p, p, 16, 4096, 4096, 128, 1, 4, 4, 2, 33, None, 0, None) == 1  # split > K/128
    assert f(p, p, p, p, p, 16, 4096, 4096, 128, 1, 4, 4, 3, 1, None, 0, None) == 1  # bad depth
    assert "depth" in L.last_error()
    assert f(p, p, p, p, p, 16, 4096, 4096, 128, 1, 4, 16, 2, 1, None, 0, None) == 1  # 16 waves
    assert "waves" in L.last_error()
    assert f(p, p, p, p, p, 16, 4096, 4096, 128, 1, 4, 12, 2, 1, None, 0, None) == 1  # 12 waves, 4 column tiles
    assert "waves" in L.last_error()
    assert f(p, p, p, p, p, 64, 4096, 6144, 128, 1, 6, 8, 1, 1, None, 0, None) == 1  # 192 KiB of LDS
    assert "LDS" in L.last_error()
    assert f(p, p, p, p, p, 64, 4096, 6144, 128, 1, 3, 4, 4, 1, None, 0, None) == 1  # ring registers
    assert "registers" in L.last_error()
    assert f(p, p, p, p, p, 256, 4096, 4096, 128, 2, 12, 1, 2, 1, None, 0, None) == 1  # bad wm
    assert f(p, p, p, p, p, 256, 4096, 4096, 128, 2, 8, 4, 2, 1, None, 0, None) == 1  # bad occupancy
    assert f(p, p, p, p, p, 256, 4096, 4096, 128, 2, 2, 2, 3, 1, None, 0, None) == 1  # wm 2 x shape 3: not compiled
    assert "not compiled" in L.last_error()
    assert f(p, p, p, p, p, 256, 4096, 4096, 128, 2, 4, 2, 18, 1, None, 0, None) == 1  # bad tile shape code
    assert "shape" in L.last_error()
    assert f(p, p, p, p, p, 256, 4096, 4096, 128, 2, 8, 2, 11, 1, None, 0, None) == 2  # 48-column waves split
    assert "multiple of 48" in L.last_error()
    assert f(p, p, p, p, p, 16, 4096, 4096, 128, 7, 4, 4, 2, 1, None, 0, None) == 1  # bad regime
    # split > 1 without workspace
    assert f(p, p, p, p, p, 16, 4096, 4096, 128, 1, 4, 4, 2, 4, None, 0, None) == 4
    assert "workspace" in L.last_error()


def test_silu_mul_entry_points_validate_without_launching(pkg):
    """The fused gate|up entry points: N % 128, even decode tile counts, and the workspace
    query covering both the plain and the fused plan (no kernel launches)."""
    L = pkg.lib()
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.addressof(buf) + (16 - ctypes.addressof(buf) % 16) % 16
    g = L.dll.w4a16_gemm_silu_mul
    assert g(p, p, p, p, p, 16, 4096, 192, 128, None, 0, None) == 2  # 192 % 128
    assert "divisible by 128" in L.last_error()
    assert g(None, None, None, None, None, 0, 4096, 24576, 128, None, 0, None) == 0  # M == 0
    assert g(None, None, None, None, None, 4, 4096, 24576, 128, None, 0, None) == 1  # null pointers
    f = L.dll.w4a16_gemm_silu_mul_config
    assert f(p, p, p, p, p, 16, 4096, 4096, 128, 1, 1, 4, 2, 1, None, 0, None) == 1  # odd tile count
    assert "even" in L.last_error()
    assert f(p, p, p, p, p, 16, 4096, 4160, 128, 1, 2, 4, 2, 1, None, 0, None) == 2  # 4160 % 128
    for k, n in QWEN3.values():
        for m in (1, 4, 16, 64, 512, 2048):
            assert L.workspace_bytes(m, k, n) >= (L.split_k(m, k, n) > 1) * m * n * 4


def test_quantize_and_pack_validate_without_launching(pkg):
    L = pkg.lib()
    q = L.dll.w4a16_quantize
    assert q(None, 0, None, None, None, 0, 128, 128, None) == 1                  # sizes
    assert q(None, 5, None, None, None, 8, 128, 128, None) == 1                  # dtype
    assert "dtype" in L.last_error()
    assert q(None, 0, None, None, None, 8, 256, 256, None) == 2                  # group > 128
    assert q(None, 0, None, None, None, 8, 100, 64, None) == 2                   # in % group
    assert q(None, 0, None, None, None, 12, 128, 128, None) == 2                 # out % 8
    assert "output size" in L.last_error()
    assert q(None, 0, None, None, None, 8, 131072, 1, None) == 2                 # grid rows
    assert q(None, 2, None, None, None, 8, 128, 128, None) == 1                  # null pointers
    pk = L.dll.w4a16_pack_int4
    assert pk(None, None, 2, 12, None) == 2
    assert pk(None, None, 0, 8, None) == 1
    assert pk(None, None, 2, 8, None) == 1


def test_two_gib_limits_are_rejected_before_launch(pkg):
    """The kernels address tensors through 32-bit buffer offsets: packed weights of 2 GiB or
    more, and decode-regime activations of 2 GiB or more, are refused (tile-regime
    activations are split into row chunks instead)."""
    L = pkg.lib()
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.addressof(buf) + (16 - ctypes.addressof(buf) % 16) % 16
    assert L.dll.w4a16_gemm(p, p, p, p, p, 16, 65536, 65536, 128, None, 0, None) == 2
    assert "2 GiB" in L.last_error()
    assert L.dll.w4a16_gemm(p, p, p, p, p, 64, 1 << 24, 64, 128, None, 0, None) == 2
    assert "2 GiB" in L.last_error()


def test_residual_entry_point_validates_without_launching(pkg):
    L = pkg.lib()
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.addressof(buf) + (16 - ctypes.addressof(buf) % 16) % 16
    f = L.dll.w4a16_gemm_residual
    assert f(p, p, p, p, None, p, 16, 4096, 4096, 128, None, 0, None) == 1
    assert "residual" in L.last_error()
    assert f(p, p, p, p, p + 2, p, 16, 4096, 4096, 128, None, 0, None) == 3
    assert f(p, p, p, p, p, p, 16, 4096, 4100, 128, None, 0, None) == 2
    assert f(None, None, None, None, None, None, 0, 4096, 4096, 128, None, 0, None) == 0


def test_rmsnorm_entry_points_validate_without_launching(pkg):
    L = pkg.lib()
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.addressof(buf) + (16 - ctypes.addressof(buf) % 16) % 16
    q = p + 32  # a second, distinct aligned address
    norm = L.dll.w4a16_add_rmsnorm
    # (x, residual, weight, eps, x_norm, residual_out, M, K, stream)
    assert norm(p, None, p, 1e-6, p, None, 0, 4096, None) == 0  # M == 0: nothing enqueued
    assert norm(p, None, p, 1e-6, p, None, 4, 4100, None) == 2 and "multiple of 8" in L.last_error()
    assert norm(p, None, p, 1e-6, p, None, 4, 16392, None) == 2
    assert norm(p, p, p, 1e-6, p, None, 4, 4096, None) == 1 and "both" in L.last_error()
    assert norm(p, p, p, 1e-6, q, q, 4, 4096, None) == 1 and "different" in L.last_error()
    assert norm(p, None, p, -1.0, p, None, 4, 4096, None) == 1 and "eps" in L.last_error()
    assert norm(p, None, p, float("nan"), p, None, 4, 4096, None) == 1
    assert norm(p + 2, None, p, 1e-6, p, None, 4, 4096, None) == 3
    assert norm(None, None, p, 1e-6, p, None, 4, 4096, None) == 1
    fused = L.dll.w4a16_gemm_rmsnorm
    # (x, residual, weight, eps, x_norm, residual_out, packed, qzeros, scales, y, M, K, N, group,
    #  silu_mul, workspace, workspace_bytes, stream)
    # validation never dereferences a pointer: y gets an address far from the other operands
    y = p + (1 << 30)
    assert fused(p, None, p, 1e-6, p, None, p, p, p, y, 0, 4096, 4096, 128, 0, None, 0, None) == 0
    assert fused(p, None, p, 1e-6, p, None, p, p, p, y, 4, 4096, 4096, 128, 2, None, 0, None) == 1
    assert fused(p, None, p, 1e-6, p, None, p, p, p, y, 4, 4096, 4160, 128, 1, None, 0, None) == 2
    assert fused(p, None, p, 1e-6, p, None, p, p, p, y, 4, 4096, 4096, 64, 0, None, 0, None) == 2
    # y overlapping an input or a norm output: rejected (x_norm here starts inside y's range)
    assert fused(p, None, p, 1e-6, y + 4096, None, p, p, p, y, 4, 4096, 4096, 128, 0, None, 0, None) == 1
    assert "overlap" in L.last_error()
    assert fused(p, None, p, 1e-6, p, None, p, p, p, p + 4096, 4, 4096, 4096, 128, 0, None, 0, None) == 1
    # a planned K split needs the workspace: reported before the norm is enqueued
    m, k, n = 32, 4096, 4096
    assert L.split_k(m, k, n) > 1
    assert fused(p, None, p, 1e-6, p, None, p, p, p, y, m, k, n, 128, 0, None, 0, None) == 4


def test_norm_stats_entry_points_validate_without_launching(pkg):
    """The RMSNorm split across two decode GEMMs: every case below fails validation (or is
    M = 0) before anything is enqueued."""
    L = pkg.lib()
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.addressof(buf) + (16 - ctypes.addressof(buf) % 16) % 16
    far = p + (1 << 30)
    prod = L.dll.w4a16_gemm_residual_stats
    # (x, packed, qzeros, scales, residual, s_out, residual_out, ssq_out, M, K, N, group, ws, ws_bytes, stream)
    assert prod(p, p, p, p, p, far, p, far + (1 << 28), 0, 4096, 4096, 128, None, 0, None) == 0
    assert prod(p, p, p, p, p, far, p, far + (1 << 28), 9, 4096, 4096, 128, None, 0, None) == 2
    assert "M <= 8" in L.last_error()
    assert prod(p, p, p, p, None, far, p, far + (1 << 28), 8, 4096, 4096, 128, None, 0, None) == 1
    assert prod(p, p, p, p, p, far, p, far + (1 << 28) + 4, 8, 4096, 4096, 128, None, 0, None) == 3
    # s_out over the residual, ssq_out inside s_out: rejected
    assert prod(p, p, p, p, p, p, far, far + (1 << 28), 8, 4096, 4096, 128, None, 0, None) == 1
    assert "overlap" in L.last_error()
    assert prod(p, p, p, p, p, far, p, far + 64, 8, 4096, 4096, 128, None, 0, None) == 1
    cons = L.dll.w4a16_gemm_rmsnorm_stats
    # (s, ssq, weight, eps, x_norm, packed, qzeros, scales, y, M, K, N, group, silu_mul, ws, ws_bytes, stream)
    assert cons(p, p, p, 1e-6, None, p, p, p, far, 0, 4096, 4096, 128, 0, None, 0, None) == 0
    assert cons(p, p, p, 1e-6, None, p, p, p, far, 8, 4096, 4096, 128, 2, None, 0, None) == 1
    assert cons(p, p, p, 1e-6, None, p, p, p, far, 9, 4096, 4096, 128, 0, None, 0, None) == 2
    assert cons(p, None, p, 1e-6, None, p, p, p, far, 8, 4096, 4096, 128, 0, None, 0, None) == 1
    assert cons(p, p, p, -1.0, None, p, p, p, far, 8, 4096, 4096, 128, 0, None, 0, None) == 1
    assert cons(p, p + 4, p, 1e-6, None, p, p, p, far, 8, 4096, 4096, 128, 0, None, 0, None) == 3
    assert cons(p, p, p, 1e-6, None, p, p, p, p + 4096, 8, 4096, 4096, 128, 0, None, 0, None) == 1
    assert "overlap" in L.last_error()


def test_plan_introspection(pkg):
    """w4a16_plan reports what the entry points run: the planner's regime and split, the
    decode kernel's own plan where the tile kernel is chosen, and refuses what no entry does."""
    L = pkg.lib()
    for m, k, n in ((1, 4096, 6144), (16, 12288, 4096), (48, 4096, 4096), (2048, 4096, 24576)):
        r = L.plan(m, k, n)
        assert r[0] == L.regime(m, k, n) and r[4] == L.split_k(m, k, n)
    assert L.plan(48, 4096, 4096, 4)[0] == pkg.REGIME_DECODE
    for m in (1, 4, 8):
        for entry in (2, 3):
            assert L.plan(m, 4096, 24576, entry)[0] == pkg.REGIME_DECODE
    out = (ctypes.c_int * 5)()
    assert L.dll.w4a16_plan(9, 4096, 4096, 2, out) == 2
    assert L.dll.w4a16_plan(65, 4096, 4096, 4, out) == 2
    assert L.dll.w4a16_plan(8, 4096, 4096, 5, out) == 1
    assert L.dll.w4a16_plan(8, 4096, 4160, 1, out) == 2
    assert L.dll.w4a16_plan(8, 4096, 4096, 0, None) == 1


def test_workspace_bytes_max_covers_every_m(pkg):
    """w4a16_workspace_bytes_max(M_max, K, N) is the largest per-call need up to M_max, for the
    plain and the fused plans alike, at every Qwen3-8B shape."""
    L = pkg.lib()
    for k, n in ((4096, 6144), (4096, 4096), (4096, 24576), (12288, 4096)):
        for m_max in (1, 16, 64, 600):
            want = max(L.workspace_bytes(m, k, n) for m in range(1, m_max + 1))
            assert L.workspace_bytes_max(m_max, k, n) == want, (k, n, m_max)
    # the engine default (16384 tokens) covers chunked prefill: more than any decode-only size
    assert L.workspace_bytes_max(16384, 12288, 4096) >= L.workspace_bytes_max(64, 12288, 4096)
    assert L.workspace_bytes_max(16384, 12288, 4096) >= L.workspace_bytes(512, 12288, 4096) > 0
    assert L.workspace_bytes_max(0, 4096, 4096) == 0
    assert L.workspace_bytes_max(64, 4096, 4100) == 0


def test_rmsnorm_strided_validates_without_launching(pkg):
    L = pkg.lib()
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.addressof(buf) + (16 - ctypes.addressof(buf) % 16) % 16
    f = L.dll.w4a16_rmsnorm_strided
    # (x, rows_inner, stride_outer, stride_inner, weight, eps, x_norm, M, K, stream)
    assert f(p, 32, 6144, 128, p, 1e-6, p, 0, 128, None) == 0  # M == 0: nothing enqueued
    assert f(p, 32, 6144, 130, p, 1e-6, p, 64, 128, None) == 3 and "multiples of 8" in L.last_error()
    assert f(p, 0, 6144, 128, p, 1e-6, p, 64, 128, None) == 1
    assert f(p, 32, -8, 128, p, 1e-6, p, 64, 128, None) == 1
    assert f(p, 32, 6144, 128, p, 1e-6, p, 64, 132, None) == 2
    assert f(p + 2, 32, 6144, 128, p, 1e-6, p, 64, 128, None) == 3


def test_plan_errors_come_before_anything_is_enqueued(pkg):
    """w4a16_gemm_rmsnorm runs every plan check (workspace size and alignment) before the norm
    is enqueued: with host pointers a launch would fault, so a clean error code proves no
    launch was attempted."""
    L = pkg.lib()
    buf = (ctypes.c_uint8 * 1024)()
    base = ctypes.addressof(buf)
    p = base + (256 - base % 256) % 256 if (256 - base % 256) % 256 + 512 <= 1024 else base
    m, k, n = 32, 4096, 4096
    need = L.workspace_bytes(m, k, n)
    assert need > 0
    fused = L.dll.w4a16_gemm_rmsnorm
    args = (p, None, p, 1e-6, p, None, p, p, p, p + (1 << 30), m, k, n, 128, 0)  # y apart from the inputs
    assert fused(*args, p, need - 1, None) == 4 and "workspace" in L.last_error()
    assert fused(*args, p + 16, need, None) == 3 and "256-byte" in L.last_error()


def test_noalloc_scratch_covers_every_planned_workspace(pkg):
    """w4a16_gemm_noalloc's 48 MiB scratch holds the largest workspace the planner asks for at
    the Qwen3-8B shapes for every M up to the engine's 16384 tokens."""
    L = pkg.lib()
    for k, n in ((4096, 6144), (4096, 4096), (4096, 24576), (12288, 4096)):
        assert L.workspace_bytes_max(16384, k, n) <= 48 << 20, (k, n)


def test_every_plan_passes_the_configuration_checks(pkg):
    """Every plan the planner emits -- plain and fused SiLU * up, decode and tile regimes --
    for the Qwen3-8B projections, their eight-way tensor-parallel shards, the Qwen3-4B, -14B
    and -32B projections and seeded random layer shapes, at chunk sizes across every
    planner boundary, passes the library's own configuration checks (shape, tiles, waves,
    depth, LDS, registers), and its workspace is covered by w4a16_workspace_bytes (plain) or
    w4a16_workspace_bytes_max (both).  Without a GPU a valid configuration stops at the
    launch (W4A16_ERR_LAUNCH); any other status is a planner or workspace-query bug.  The
    pointers are dummies, so on a machine with a GPU the test is skipped."""
    import random

    import torch

    if torch.cuda.is_available():
        pytest.skip("dummy pointers: the configuration calls would launch on a real GPU")
    L = pkg.lib()
    buf = (ctypes.c_uint8 * 1024)()
    p = ctypes.addressof(buf) + (256 - ctypes.addressof(buf) % 256) % 256  # the workspace is 256-byte aligned
    shapes = [(4096, 6144), (4096, 4096), (4096, 24576), (12288, 4096),
              (4096, 768), (512, 4096), (4096, 3072), (1536, 4096),
              (2560, 6144), (4096, 2560), (2560, 19456), (9728, 2560),
              (5120, 7168), (5120, 5120), (5120, 34816), (17408, 5120),
              (5120, 10240), (8192, 5120), (5120, 51200), (25600, 5120)]
    rng = random.Random(5)
    shapes += [(128 * rng.randint(2, 200), 128 * rng.randint(2, 400)) for _ in range(12)]
    ms = list(range(1, 34)) + [40, 48, 49, 64, 65, 96, 128, 129, 160, 192, 256, 257, 288, 320, 321, 384, 448, 512,
                               513, 640, 704, 705, 768, 769, 1024, 1025, 1152, 1536, 2048, 2049, 3072, 4096]
    bad = []
    for k, n in shapes:
        ws_max = L.workspace_bytes_max(max(ms), k, n)
        for m in ms:
            for entry, fn in ((0, L.dll.w4a16_gemm_config), (1, L.dll.w4a16_gemm_silu_mul_config)):
                if entry == 1 and n % 128:
                    continue
                plan = L.plan(m, k, n, entry)
                ws = L.workspace_bytes(m, k, n) if entry == 0 else ws_max
                rc = fn(p, p, p, p, p, m, k, n, 128, *plan, p if ws else None, ws, None)
                if rc != 5:
                    bad.append((k, n, m, entry, plan, rc, L.last_error()[:80]))
    assert not bad, bad[:10]
