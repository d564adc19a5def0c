// RMSNorm with the optional residual add in front of it: the normalisation that feeds
// the QKV and gate_up projections of every decoder layer.  One workgroup per row.
//
// Per row of K elements, in the reference's order (layernorm.py:17-40):
//   s  = float(x) + float(residual)            (fp32; s = float(x) without a residual)
//   residual_out = bf16(s)
//   r  = rsqrt(mean(s * s) + eps)               (fp32 sum of squares; rsqrt in fp64)
//   x_norm = bf16(float(bf16(s * r)) * float(weight))
// s stays in registers between the two passes (K <= kNormMaxK), so residual_out may be
// residual or x, and x_norm may be x: every element is read by the thread that writes it,
// before it writes it.  HBM-bound: 4K bytes read and 4K written per row with a residual,
// 2K + 2K without (the weight row is L2-resident after the first workgroups).
#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormChunks = kNormMaxK / (8 * kNormThreads);  // 16-byte chunks per thread

template <bool RES>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(const uint16_t* x, const uint16_t* residual,
                                                                    const uint16_t* __restrict__ weight,
                                                                    uint16_t* x_norm, uint16_t* residual_out, int K,
                                                                    float eps) {
  const size_t row = static_cast<size_t>(blockIdx.x) * K;
  const int chunks = K >> 3;
  float s[kNormChunks][8];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    if (c < chunks) {
      unpack_bf16x8(*reinterpret_cast<const uint4*>(x + row + 8 * c), s[j]);
      if constexpr (RES) {
        float r[8];
        unpack_bf16x8(*reinterpret_cast<const uint4*>(residual + row + 8 * c), r);
#pragma unroll
        for (int i = 0; i < 8; ++i) s[j][i] += r[i];
        *reinterpret_cast<uint4*>(residual_out + row + 8 * c) = pack_bf16x8(s[j]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += s[j][i] * s[j][i];
    }
  }
  __shared__ float part[kNormThreads / 64];
  ss = wave_sum64(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float var = ((part[0] + part[1]) + (part[2] + part[3])) / static_cast<float>(K);
  const float rstd = rsqrt_rn(var + eps);
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    if (c < chunks) {
      *reinterpret_cast<uint4*>(x_norm + row + 8 * c) =
          rms_scale_bf16x8(s[j], rstd, *reinterpret_cast<const uint4*>(weight + 8 * c));
    }
  }
}

}  // namespace

hipError_t launch_add_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                              uint16_t* x_norm, uint16_t* residual_out, int M, int K, float eps,
                              hipStream_t stream) {
  if (M <= 0) return hipSuccess;
  if (residual)
    add_rmsnorm_kernel<true><<<M, kNormThreads, 0, stream>>>(x, residual, weight, x_norm, residual_out, K, eps);
  else
    add_rmsnorm_kernel<false><<<M, kNormThreads, 0, stream>>>(x, nullptr, weight, x_norm, nullptr, K, eps);
  return hipGetLastError();
}

}  // namespace w4a16
