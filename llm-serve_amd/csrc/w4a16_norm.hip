// RMSNorm with the optional residual add in front of it: the normalisation that feeds
// the QKV and gate_up projections of every decoder layer, and the per-head q_norm / k_norm
// applied to strided views of the QKV output.
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
//
// LPR lanes work on one row, each on 16-byte chunks: rows of K > 512 take a whole
// 256-lane workgroup (sum of squares: wave shuffles, then four partial sums through LDS);
// shorter rows (the 128-wide heads) take LPR = 8 .. 64 lanes of one wave, 256 / LPR rows per
// workgroup, reduced by shuffles inside the lane group.  Row r of x starts at element
// (r / rows_inner) * stride_outer + (r % rows_inner) * stride_inner; residual, residual_out
// and x_norm are contiguous [M, K].
#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

constexpr int kNormThreads = 256;

template <bool RES, int LPR>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(const uint16_t* x, const uint16_t* residual,
                                                                    const uint16_t* __restrict__ weight,
                                                                    uint16_t* x_norm, uint16_t* residual_out, int M,
                                                                    int K, int rows_inner, int64_t stride_outer,
                                                                    int64_t stride_inner, float eps) {
  constexpr int kRows = kNormThreads / LPR;             // rows per workgroup
  // 16-byte chunks per lane: up to 8 for whole-workgroup rows, one for shorter rows (the
  // launcher picks LPR >= K / 8 for them).
  constexpr int kChunks = LPR == kNormThreads ? kNormMaxK / (8 * kNormThreads) : 1;
  const int sub = threadIdx.x / LPR;
  const int l = threadIdx.x % LPR;
  const int r = blockIdx.x * kRows + sub;
  const bool live = r < M;  // uniform over the lanes of a row
  const int64_t xrow = live ? static_cast<int64_t>(r / rows_inner) * stride_outer +
                                  static_cast<int64_t>(r % rows_inner) * stride_inner
                            : 0;
  const size_t row = static_cast<size_t>(live ? r : 0) * K;
  const int chunks = K >> 3;
  // The weight chunks are loaded first, so that they arrive during the sum of squares
  // instead of after it.
  uint4 wv[kChunks];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c = l + j * LPR;
    if (live && c < chunks) wv[j] = *reinterpret_cast<const uint4*>(weight + 8 * c);
  }
  float s[kChunks][8];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c = l + j * LPR;
    if (live && c < chunks) {
      unpack_bf16x8(*reinterpret_cast<const uint4*>(x + xrow + 8 * c), s[j]);
      if constexpr (RES) {
        float rr[8];
        unpack_bf16x8(*reinterpret_cast<const uint4*>(residual + row + 8 * c), rr);
#pragma unroll
        for (int i = 0; i < 8; ++i) s[j][i] += rr[i];
        *reinterpret_cast<uint4*>(residual_out + row + 8 * c) = pack_bf16x8(s[j]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += s[j][i] * s[j][i];
    }
  }
  float total;
  if constexpr (LPR == kNormThreads) {
    __shared__ float part[kNormThreads / 64];
    ss = wave_sum64(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    total = (part[0] + part[1]) + (part[2] + part[3]);
  } else {
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    total = ss;
  }
  const float rstd = rsqrt_rn(total / static_cast<float>(K) + eps);
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c = l + j * LPR;
    if (live && c < chunks) {
      *reinterpret_cast<uint4*>(x_norm + row + 8 * c) = rms_scale_bf16x8(s[j], rstd, wv[j]);
    }
  }
}

template <bool RES, int LPR>
hipError_t launch_lpr(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, uint16_t* x_norm,
                      uint16_t* residual_out, int M, int K, int rows_inner, int64_t stride_outer,
                      int64_t stride_inner, float eps, hipStream_t stream) {
  constexpr int kRows = kNormThreads / LPR;
  add_rmsnorm_kernel<RES, LPR><<<(M + kRows - 1) / kRows, kNormThreads, 0, stream>>>(
      x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer, stride_inner, eps);
  return hipGetLastError();
}

template <bool RES>
hipError_t launch_rows(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, uint16_t* x_norm,
                       uint16_t* residual_out, int M, int K, int rows_inner, int64_t stride_outer,
                       int64_t stride_inner, float eps, hipStream_t stream) {
  const int chunks = K / 8;
  if (chunks <= 8)
    return launch_lpr<RES, 8>(x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer,
                              stride_inner, eps, stream);
  if (chunks <= 16)
    return launch_lpr<RES, 16>(x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer,
                               stride_inner, eps, stream);
  if (chunks <= 32)
    return launch_lpr<RES, 32>(x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer,
                               stride_inner, eps, stream);
  if (chunks <= 64)
    return launch_lpr<RES, 64>(x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer,
                               stride_inner, eps, stream);
  return launch_lpr<RES, kNormThreads>(x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer,
                                       stride_inner, eps, stream);
}

}  // namespace

hipError_t launch_add_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                              uint16_t* x_norm, uint16_t* residual_out, int M, int K, float eps,
                              hipStream_t stream) {
  if (M <= 0) return hipSuccess;
  if (residual) return launch_rows<true>(x, residual, weight, x_norm, residual_out, M, K, M, 0, K, eps, stream);
  return launch_rows<false>(x, nullptr, weight, x_norm, nullptr, M, K, M, 0, K, eps, stream);
}

hipError_t launch_rmsnorm_strided(const uint16_t* x, int rows_inner, int64_t stride_outer, int64_t stride_inner,
                                  const uint16_t* weight, uint16_t* x_norm, int M, int K, float eps,
                                  hipStream_t stream) {
  if (M <= 0) return hipSuccess;
  return launch_rows<false>(x, nullptr, weight, x_norm, nullptr, M, K, rows_inner, stride_outer, stride_inner, eps,
                            stream);
}

}  // namespace w4a16
