// RMSNorm with the optional residual add in front of it: the normalisation that feeds
// the QKV and gate_up projections of every decoder layer.  One workgroup per row.
//
// Per row of K elements, in the reference's order (layernorm.py:17-40):
//   s  = float(x) + float(residual)            (fp32; s = float(x) without a residual)
//   residual_out = bf16(s)
//   r  = rsqrt(mean(s * s) + eps)               (fp32 sum of squares; rsqrt correctly rounded)
//   x_norm = bf16(float(bf16(s * r)) * float(weight))
// s stays in registers between the two passes (K <= kNormMaxK), so residual_out may be
// residual or x, and x_norm may be x: every element is read by the thread that writes it,
// before it writes it.  HBM-bound: 4K bytes read and 4K written per row with a residual,
// 2K + 2K without (the weight row is L2-resident after the first workgroups).
#include <math.h>

#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormChunks = kNormMaxK / (8 * kNormThreads);  // 16-byte chunks per thread

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ void unpack8(uint4 v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

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
      unpack8(*reinterpret_cast<const uint4*>(x + row + 8 * c), s[j]);
      if constexpr (RES) {
        float r[8];
        unpack8(*reinterpret_cast<const uint4*>(residual + row + 8 * c), r);
#pragma unroll
        for (int i = 0; i < 8; ++i) s[j][i] += r[i];
        *reinterpret_cast<uint4*>(residual_out + row + 8 * c) = pack8(s[j]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += s[j][i] * s[j][i];
    }
  }
  __shared__ float part[kNormThreads / 64];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float var = ((part[0] + part[1]) + (part[2] + part[3])) / static_cast<float>(K);
  // One correctly rounded reciprocal square root per row (fp64 costs nothing here).
  const float rstd = static_cast<float>(1.0 / sqrt(static_cast<double>(var + eps)));
#pragma unroll
  for (int j = 0; j < kNormChunks; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    if (c < chunks) {
      float t[8], w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) t[i] = s[j][i] * rstd;
      unpack8(pack8(t), t);  // bf16(s * r): the reference's x.to(orig_dtype)
      unpack8(*reinterpret_cast<const uint4*>(weight + 8 * c), w);
#pragma unroll
      for (int i = 0; i < 8; ++i) t[i] *= w[i];  // exact in fp32 (two 8-bit significands)
      *reinterpret_cast<uint4*>(x_norm + row + 8 * c) = pack8(t);
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
