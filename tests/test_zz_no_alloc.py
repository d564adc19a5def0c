"""w4a16_gemm_noalloc, the allocation-free entry point, through the C ABI: its outputs equal
w4a16_gemm's (same kernels and plan, caller workspace) bit for bit, on two calls in a row
with the second smaller, at split-K plans of the decode and tile kernels and a plan without a
split; nothing is allocated by the library (neither the torch allocator's reserved bytes nor the
device's free bytes change across the calls once the outputs exist and each plan has run once).
The first call on a device sets up the library's scratch and is refused under graph capture."""
import ctypes

import pytest
import torch

from awq_helpers import QWEN3_SHAPES, awq_mod, random_awq_gpu, random_x_gpu

pytestmark = pytest.mark.gpu


def c_gemm(lib, fn, x, w, y, k, n, ws=None):
    packed, qz, s = w
    m = x.shape[0]
    stream = torch.cuda.current_stream().cuda_stream
    args = [x.data_ptr(), packed.data_ptr(), qz.data_ptr(), s.data_ptr(), y.data_ptr(), m, k, n, 128]
    if fn == "w4a16_gemm":
        args += [ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0]
    rc = getattr(lib.dll, fn)(*args, ctypes.c_void_p(stream))
    assert rc == 0, (fn, m, k, n, lib.last_error())


def test_first_noalloc_call_under_capture_is_refused(gpu_lib):
    """Runs first in this file: no w4a16_gemm_noalloc call has set up the scratch yet in a
    process that runs this file alone or after the other tests (none of them calls it).
    Under capture the set-up is refused before anything is enqueued, and the capture ends
    cleanly; an eager call then sets it up."""
    k, n = QWEN3_SHAPES["down"]
    qw, qz, s = random_awq_gpu(k, n, seed=60)
    w = (awq_mod().repack_awq_qweight(qw), qz, s)
    x = random_x_gpu(16, k, seed=4)
    assert gpu_lib.split_k(16, k, n) > 1  # the call needs the scratch
    y = torch.empty((16, n), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    print("noalloc first call under capture", flush=True)
    rc = []
    with torch.cuda.graph(graph, stream=stream):
        packed, qz_, s_ = w
        rc.append(gpu_lib.dll.w4a16_gemm_noalloc(x.data_ptr(), packed.data_ptr(), qz_.data_ptr(), s_.data_ptr(),
                                                 y.data_ptr(), 16, k, n, 128, ctypes.c_void_p(stream.cuda_stream)))
        msg = gpu_lib.last_error()
    assert rc == [5] and "must not be captured" in msg, (rc, msg)
    torch.cuda.synchronize()
    c_gemm(gpu_lib, "w4a16_gemm_noalloc", x, w, y, k, n)  # eager: sets it up
    ref = torch.empty_like(y)
    ws = torch.zeros(gpu_lib.workspace_bytes(16, k, n), dtype=torch.uint8, device="cuda")
    c_gemm(gpu_lib, "w4a16_gemm", x, w, ref, k, n, ws)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("shape,ms", [("down", (512, 16)), ("qkv", (384, 64)), ("o", (1024, 8)),
                                      ("gate_up", (64, 1))])
def test_noalloc_matches_gemm_on_two_calls(gpu_lib, shape, ms):
    k, n = QWEN3_SHAPES[shape]
    qw, qz, s = random_awq_gpu(k, n, seed=61)
    w = (awq_mod().repack_awq_qweight(qw), qz, s)
    xs = [random_x_gpu(m, k, seed=m) for m in ms]
    want = []
    for x in xs:
        ws_bytes = gpu_lib.workspace_bytes(x.shape[0], k, n)
        ws = torch.zeros(max(ws_bytes, 256), dtype=torch.uint8, device="cuda") if ws_bytes else None
        y = torch.empty((x.shape[0], n), dtype=torch.bfloat16, device="cuda")
        c_gemm(gpu_lib, "w4a16_gemm", x, w, y, k, n, ws)
        want.append(y)
    # two repetitions of the two calls, each into its own output; only the library calls sit
    # inside the measured window (torch's own temporaries, e.g. of torch.equal, would not)
    outs = [[torch.empty((x.shape[0], n), dtype=torch.bfloat16, device="cuda") for x in xs] for _ in range(2)]
    torch.cuda.synchronize()
    print(f"noalloc {shape} M={ms} splits={[gpu_lib.split_k(x.shape[0], k, n) for x in xs]}", flush=True)
    for x, y in zip(xs, outs[0]):
        c_gemm(gpu_lib, "w4a16_gemm_noalloc", x, w, y, k, n)
    torch.cuda.synchronize()
    # every plan has run once: a library allocation would now show as less free device memory
    reserved, free = torch.cuda.memory_reserved(), torch.cuda.mem_get_info()[0]
    for x, y in zip(xs, outs[1]):
        c_gemm(gpu_lib, "w4a16_gemm_noalloc", x, w, y, k, n)
    torch.cuda.synchronize()
    assert torch.cuda.memory_reserved() == reserved
    assert torch.cuda.mem_get_info()[0] == free
    for rep in range(2):
        for x, y, ref in zip(xs, outs[rep], want):
            assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), (shape, x.shape[0], rep)


def test_noalloc_rejects_bad_arguments_before_launch(gpu_lib):
    f = gpu_lib.dll.w4a16_gemm_noalloc
    assert f(None, None, None, None, None, 0, 4096, 4096, 128, None) == 0  # M == 0: nothing to do
    assert f(None, None, None, None, None, 16, 4096, 4100, 128, None) == 2
    assert f(None, None, None, None, None, 16, 4096, 4096, 64, None) == 2
    assert f(None, None, None, None, None, 16, 4096, 4096, 128, None) == 1


def test_noalloc_under_graph_capture(gpu_lib):
    """Captured after a first eager call (the set-up on this device is done then), replayed
    several times with eager work in between: every replay equals w4a16_gemm's result."""
    k, n = QWEN3_SHAPES["down"]
    qw, qz, s = random_awq_gpu(k, n, seed=62)
    w = (awq_mod().repack_awq_qweight(qw), qz, s)
    x = random_x_gpu(16, k, seed=3)
    ws = torch.zeros(gpu_lib.workspace_bytes(16, k, n), dtype=torch.uint8, device="cuda")
    ref = torch.empty((16, n), dtype=torch.bfloat16, device="cuda")
    c_gemm(gpu_lib, "w4a16_gemm", x, w, ref, k, n, ws)
    y = torch.empty_like(ref)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        c_gemm(gpu_lib, "w4a16_gemm_noalloc", x, w, y, k, n)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        c_gemm(gpu_lib, "w4a16_gemm_noalloc", x, w, y, k, n)
    for i in range(3):
        y.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), i
        other = torch.empty_like(ref)
        c_gemm(gpu_lib, "w4a16_gemm_noalloc", random_x_gpu(16, k, seed=10 + i), w, other, k, n)
        torch.cuda.synchronize()
