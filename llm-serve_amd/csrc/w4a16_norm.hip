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
// and the value it writes depends on what it read.  HBM-bound: 4K bytes read and 4K
// written per row with a residual, 2K + 2K without (the weight row is L2-resident after
// the first workgroups).
//
// Lanes work on 16-byte chunks: rows of K > 512 take a whole 256-lane workgroup (sum of
// squares: wave shuffles, then four partial sums through LDS); shorter rows (the 128-wide
// heads) take 8 .. 64 lanes of one wave, reduced by shuffles.  Row r of x starts at element
// (r / rows_inner) * stride_outer + (r % rows_inner) * stride_inner; residual, residual_out
// and x_norm are contiguous [M, K].
#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {
namespace {

constexpr int kNormThreads = 256;

// Rows of K <= 512: LPR = 8 .. 64 lanes of one wave per row (LPR >= K / 8), 256 / LPR rows per
// workgroup, one 16-byte chunk per lane, reduced by shuffles inside the lane group.
template <bool RES, int LPR>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_rows_kernel(
    const uint16_t* x, const uint16_t* residual, const uint16_t* __restrict__ weight, uint16_t* x_norm,
    uint16_t* residual_out, int M, int K, int rows_inner, int64_t stride_outer, int64_t stride_inner, float eps) {
  constexpr int kRows = kNormThreads / LPR;  // rows per workgroup
  const int c = threadIdx.x % LPR;           // the lane's chunk of its row
  const int r = blockIdx.x * kRows + static_cast<int>(threadIdx.x / LPR);
  const bool on = r < M && c < (K >> 3);
  const int64_t xrow = on ? static_cast<int64_t>(r / rows_inner) * stride_outer +
                                static_cast<int64_t>(r % rows_inner) * stride_inner
                          : 0;
  const size_t row = static_cast<size_t>(on ? r : 0) * K;
  // The weight chunk is loaded first, so that it arrives during the sum of squares.
  uint4 wv{};
  float s[8] = {};
  if (on) {
    wv = *reinterpret_cast<const uint4*>(weight + 8 * c);
    unpack_bf16x8(*reinterpret_cast<const uint4*>(x + xrow + 8 * c), s);
    if constexpr (RES) {
      float rr[8];
      unpack_bf16x8(*reinterpret_cast<const uint4*>(residual + row + 8 * c), rr);
#pragma unroll
      for (int i = 0; i < 8; ++i) s[i] += rr[i];
      *reinterpret_cast<uint4*>(residual_out + row + 8 * c) = pack_bf16x8(s);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += s[i] * s[i];
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  const float rstd = rsqrt_rn(ss / static_cast<float>(K) + eps);
  if (on) *reinterpret_cast<uint4*>(x_norm + row + 8 * c) = rms_scale_bf16x8(s, rstd, wv);
}

// Rows of K > 512: one 256-lane workgroup per row, C = K / 2048 rounded up to 1, 2, 4 or 8
// 16-byte chunks per lane.  Every load of the row is an unconditional buffer load over the
// row (chunks past K read zeros without a memory access), all issued before the first use,
// so a row costs one memory round trip; the stores follow the reduction (stores past the
// row are dropped).  The row comes from blockIdx alone, so the buffer descriptors are
// uniform over the workgroup.
template <bool RES, int C>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(
    const uint16_t* x, const uint16_t* residual, const uint16_t* __restrict__ weight, uint16_t* x_norm,
    uint16_t* residual_out, int K, int rows_inner, int64_t stride_outer, int64_t stride_inner, float eps) {
  const int l = threadIdx.x;
  const int r = blockIdx.x;  // the grid has one workgroup per row
  const int64_t xrow = static_cast<int64_t>(r / rows_inner) * stride_outer +
                       static_cast<int64_t>(r % rows_inner) * stride_inner;
  const size_t row = static_cast<size_t>(r) * K;
  const uint32_t row_bytes = static_cast<uint32_t>(K) * 2u;
  const auto xb = make_buffer(x + xrow, row_bytes);
  const auto rb = make_buffer(RES ? residual + row : x, RES ? row_bytes : 0u);
  const auto wb = make_buffer(weight, row_bytes);
  uint4 wv[C], xv[C], rv[C];
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const uint32_t off = static_cast<uint32_t>(l + j * kNormThreads) * 16u;
    wv[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wb, off, 0, 0));
    xv[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xb, off, 0, 0));
    if constexpr (RES) rv[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
  }
  float s[C][8];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < C; ++j) {
    unpack_bf16x8(xv[j], s[j]);
    if constexpr (RES) {
      float rr[8];
      unpack_bf16x8(rv[j], rr);
#pragma unroll
      for (int i = 0; i < 8; ++i) s[j][i] += rr[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += s[j][i] * s[j][i];
  }
  __shared__ float part[kNormThreads / 64];
  ss = wave_sum64(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float rstd = rsqrt_rn(total / static_cast<float>(K) + eps);
  const auto ob = make_buffer(x_norm + row, row_bytes);
  const auto nb = make_buffer(RES ? residual_out + row : x_norm, RES ? row_bytes : 0u);
#pragma unroll
  for (int j = 0; j < C; ++j) {
    const uint32_t off = static_cast<uint32_t>(l + j * kNormThreads) * 16u;
    if constexpr (RES)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, pack_bf16x8(s[j])), nb, off, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, rms_scale_bf16x8(s[j], rstd, wv[j])), ob,
                                           off, 0, 0);
  }
}

template <bool RES, int LPR>
hipError_t launch_lpr(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, uint16_t* x_norm,
                      uint16_t* residual_out, int M, int K, int rows_inner, int64_t stride_outer,
                      int64_t stride_inner, float eps, hipStream_t stream) {
  constexpr int kRows = kNormThreads / LPR;
  add_rmsnorm_rows_kernel<RES, LPR><<<(M + kRows - 1) / kRows, kNormThreads, 0, stream>>>(
      x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer, stride_inner, eps);
  return hipGetLastError();
}

template <bool RES, int C>
hipError_t launch_whole(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, uint16_t* x_norm,
                        uint16_t* residual_out, int M, int K, int rows_inner, int64_t stride_outer,
                        int64_t stride_inner, float eps, hipStream_t stream) {
  add_rmsnorm_kernel<RES, C><<<M, kNormThreads, 0, stream>>>(x, residual, weight, x_norm, residual_out, K,
                                                            rows_inner, stride_outer, stride_inner, eps);
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
  static_assert(kNormMaxK == 8 * 8 * kNormThreads, "whole-workgroup rows hold at most 8 chunks per lane");
  if (chunks <= kNormThreads)
    return launch_whole<RES, 1>(x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer,
                                 stride_inner, eps, stream);
  if (chunks <= 2 * kNormThreads)
    return launch_whole<RES, 2>(x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer,
                                 stride_inner, eps, stream);
  if (chunks <= 4 * kNormThreads)
    return launch_whole<RES, 4>(x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer,
                                 stride_inner, eps, stream);
  return launch_whole<RES, 8>(x, residual, weight, x_norm, residual_out, M, K, rows_inner, stride_outer,
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
