// Measurement helper for bench.py, built as its own libw4a16_probe.so (not part of the
// W4A16 library or its C ABI): a plain streaming read of a device buffer, 16 bytes per
// lane and load, UNROLL independent loads in flight per lane, grid-stride.  It measures what
// HBM delivers to a kernel that reads a given number of bytes per launch.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kUnroll = 4;

__global__ __launch_bounds__(kThreads) void read_kernel(const u32x4_t* __restrict__ p, size_t n,
                                                        uint32_t* __restrict__ sink, uint32_t key) {
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kUnroll - 1) * stride < n; i += kUnroll * stride) {
    u32x4_t v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = p[i + u * stride];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n; i += stride) {
    const u32x4_t v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  // The loaded data decides whether anything is stored (practically never), so no load
  // can be dropped and the kernel writes nothing in the normal case.
  if (acc == key) sink[blockIdx.x] = acc;
}

}  // namespace

// Reads `bytes` (a multiple of 16) at p with `blocks` workgroups of 256 threads; sink holds
// at least `blocks` words.  Returns the launch status (0 = hipSuccess).
extern "C" int probe_read(const void* p, size_t bytes, uint32_t* sink, int blocks, void* stream) {
  if (!p || !sink || blocks < 1 || bytes % 16) return static_cast<int>(hipErrorInvalidValue);
  read_kernel<<<blocks, kThreads, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const u32x4_t*>(p), bytes / 16,
                                                                        sink, 0x9E3779B9u);
  return static_cast<int>(hipGetLastError());
}
