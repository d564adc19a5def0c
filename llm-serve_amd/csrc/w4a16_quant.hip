// Producer side of the AutoAWQ format on the GPU: group-wise asymmetric int4 quantization
// of a float weight and the AWQ-order int4 packer (the reference's quantize_awq_weight and
// _pack_int4, llmserve/quantization/awq_calibration.py:19-62).  HBM-bound byte/integer work:
// the weight is read once and 0.5 byte per weight (plus scales and zeros) is written.
//
// quantize_kernel: one workgroup per (64 output features, one group of gs <= 128 inputs).
// The 64 x gs slice of W [out, in] (rows of gs contiguous values) is read coalesced into LDS
// as fp32 (at most 33 KiB); four threads per row reduce its min and max; the row's scale and
// zero follow the reference's fp32 arithmetic exactly
//   s = max(max - min, 1e-5) / 15      z = clamp(-rint(min / s), 0, 15)
//   q = clamp(rint(w / s) + z, 0, 15)  (rint = round half to even, as torch.round;
//                                        / is the correctly rounded IEEE division)
// and the transposed AutoAWQ words qweight[k, o / 8] are written 8 consecutive words (32
// bytes) per input row k.
#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {

constexpr int kQuantRows = 64;  // output features per workgroup
constexpr int kQuantThreads = 256;

__device__ __forceinline__ float load_weight(const uint16_t* p, int dtype, size_t i) {
  const uint16_t b = p[i];
  if (dtype == kDtypeF16) return static_cast<float>(__builtin_bit_cast(_Float16, b));
  return bf16_bits_to_f32(b);
}

__global__ __launch_bounds__(kQuantThreads) void quantize_kernel(const void* __restrict__ weight, int dtype,
                                                                 uint32_t* __restrict__ qweight,
                                                                 uint32_t* __restrict__ qzeros,
                                                                 void* __restrict__ scales, int out_f, int in_f,
                                                                 int gs, bool vec) {
  extern __shared__ float tile[];  // [kQuantRows][gs + 1]
  __shared__ float row_s[kQuantRows];
  __shared__ float row_z[kQuantRows];
  const int pitch = gs + 1;  // odd pitch: the eight rows one packed word reads sit in distinct banks
  const int o0 = blockIdx.x * kQuantRows;
  const int g = blockIdx.y;
  const int rows = out_f - o0 < kQuantRows ? out_f - o0 : kQuantRows;  // a multiple of 8
  const int tid = threadIdx.x;

  if (vec) {
    // 16-byte loads: 8 values of a 16-bit type or 4 floats per load (gs a multiple of
    // either, weight 16-byte aligned; checked on the host).
    const int per = dtype == kDtypeF32 ? 4 : 8;
    const int cpr = gs / per;  // chunks per row
    for (int e = tid; e < rows * cpr; e += kQuantThreads) {
      const int r = e / cpr;
      const int c = (e - r * cpr) * per;
      const size_t i = static_cast<size_t>(o0 + r) * in_f + static_cast<size_t>(g) * gs + c;
      float* dst = tile + r * pitch + c;
      if (dtype == kDtypeF32) {
        const float4 v = *reinterpret_cast<const float4*>(static_cast<const float*>(weight) + i);
        dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(weight) + i);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const uint16_t lo = static_cast<uint16_t>(w[h] & 0xFFFFu), hi = static_cast<uint16_t>(w[h] >> 16);
          dst[2 * h] = dtype == kDtypeF16 ? static_cast<float>(__builtin_bit_cast(_Float16, lo)) : bf16_bits_to_f32(lo);
          dst[2 * h + 1] = dtype == kDtypeF16 ? static_cast<float>(__builtin_bit_cast(_Float16, hi)) : bf16_bits_to_f32(hi);
        }
      }
    }
  } else {
    for (int e = tid; e < rows * gs; e += kQuantThreads) {
      const int r = e / gs;
      const int c = e - r * gs;
      const size_t i = static_cast<size_t>(o0 + r) * in_f + static_cast<size_t>(g) * gs + c;
      tile[r * pitch + c] = dtype == kDtypeF32 ? static_cast<const float*>(weight)[i]
                                               : load_weight(static_cast<const uint16_t*>(weight), dtype, i);
    }
  }
  __syncthreads();

  // Min and max of row r = tid / 4 over its quarter of the group; NaN propagates as in
  // torch's amin / amax.
  static_assert(kQuantThreads == 4 * kQuantRows, "four threads per row");
  {
    const int r = tid >> 2;
    const int h = tid & 3;
    const int part = (gs + 3) >> 2;
    const int c_end = (h + 1) * part < gs ? (h + 1) * part : gs;
    float mn = __builtin_inff(), mx = -__builtin_inff();
    if (r < rows) {
      for (int c = h * part; c < c_end; ++c) {
        const float v = tile[r * pitch + c];
        mn = (v < mn || v != v) ? v : mn;
        mx = (v > mx || v != v) ? v : mx;
      }
    }
#pragma unroll
    for (int d = 1; d <= 2; d <<= 1) {
      const float mn2 = __shfl_xor(mn, d);
      const float mx2 = __shfl_xor(mx, d);
      mn = (mn2 < mn || mn2 != mn2) ? mn2 : mn;
      mx = (mx2 > mx || mx2 != mx2) ? mx2 : mx;
    }
    if (h == 0 && r < rows) {
      float d = mx - mn;
      d = d < 1e-5f ? 1e-5f : d;  // torch clamp(min=): NaN stays NaN
      const float s = d / 15.0f;
      float z = -__builtin_rintf(mn / s);
      z = z < 0.f ? 0.f : (z > 15.f ? 15.f : z);
      row_s[r] = s;
      row_z[r] = z;
      const size_t si = static_cast<size_t>(g) * out_f + o0 + r;
      if (dtype == kDtypeF32) static_cast<float*>(scales)[si] = s;
      else if (dtype == kDtypeF16) static_cast<_Float16*>(scales)[si] = static_cast<_Float16>(s);
      else static_cast<uint16_t*>(scales)[si] = f32_to_bf16_bits(s);
    }
  }
  __syncthreads();

  const int W = rows / 8;     // packed words per input row in this workgroup
  const int C8 = out_f / 8;   // packed words per input row
  if (tid < W) {
    uint32_t word = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) word |= (static_cast<uint32_t>(row_z[8 * tid + c]) & 0xFu) << awq_shift(c);
    qzeros[static_cast<size_t>(g) * C8 + o0 / 8 + tid] = word;
  }
  for (int e = tid; e < gs * W; e += kQuantThreads) {
    const int k = e / W;
    const int j = e - k * W;
    uint32_t word = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int r = 8 * j + c;
      float q = __builtin_rintf(tile[r * pitch + k] / row_s[r]) + row_z[r];
      q = q < 0.f ? 0.f : (q > 15.f ? 15.f : q);
      word |= (static_cast<uint32_t>(q) & 0xFu) << awq_shift(c);
    }
    qweight[(static_cast<size_t>(g) * gs + k) * C8 + o0 / 8 + j] = word;
  }
}

// Fast path for GS in {32, 64, 128} (the same arithmetic, bit for bit): each of the four
// threads of a row holds its GS / 4 consecutive values in registers (16-byte loads), the
// row's min and max come from two lane shuffles, and only the 4-bit codes go through LDS
// (one byte each, rows padded to GS + 4 bytes so that the eight rows one packed word
// gathers sit in different banks) for the transposed packing.
template <int GS, int DTYPE>
__global__ __launch_bounds__(kQuantThreads) void quantize_rows_kernel(const void* __restrict__ weight,
                                                                      uint32_t* __restrict__ qweight,
                                                                      uint32_t* __restrict__ qzeros,
                                                                      void* __restrict__ scales, int out_f, int in_f) {
  constexpr int PART = GS / 4;       // values per thread
  constexpr int QP = GS + 4;         // LDS row pitch of the codes, bytes
  constexpr int PER = DTYPE == kDtypeF32 ? 4 : 8;  // values per 16-byte load
  static_assert(PART % PER == 0, "a thread's values must split into 16-byte loads");
  __shared__ __attribute__((aligned(16))) uint8_t codes[kQuantRows * QP];
  __shared__ float row_z[kQuantRows];
  const int o0 = blockIdx.x * kQuantRows;
  const int g = blockIdx.y;
  const int rows = out_f - o0 < kQuantRows ? out_f - o0 : kQuantRows;  // a multiple of 8
  const int tid = threadIdx.x;
  const int r = tid >> 2;  // the four threads of row r are adjacent lanes of one wave
  const int h = tid & 3;
  const bool live = r < rows;

  float v[PART];
  const size_t base = static_cast<size_t>(o0 + (live ? r : 0)) * in_f + static_cast<size_t>(g) * GS + h * PART;
#pragma unroll
  for (int c = 0; c < PART; c += PER) {
    if constexpr (DTYPE == kDtypeF32) {
      const float4 w = live ? *reinterpret_cast<const float4*>(static_cast<const float*>(weight) + base + c)
                            : float4{0.f, 0.f, 0.f, 0.f};
      v[c] = w.x; v[c + 1] = w.y; v[c + 2] = w.z; v[c + 3] = w.w;
    } else {
      const uint4 w = live ? *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(weight) + base + c)
                           : uint4{0u, 0u, 0u, 0u};
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t lo = static_cast<uint16_t>(ww[e] & 0xFFFFu), hi = static_cast<uint16_t>(ww[e] >> 16);
        if constexpr (DTYPE == kDtypeF16) {
          v[c + 2 * e] = static_cast<float>(__builtin_bit_cast(_Float16, lo));
          v[c + 2 * e + 1] = static_cast<float>(__builtin_bit_cast(_Float16, hi));
        } else {
          v[c + 2 * e] = bf16_bits_to_f32(lo);
          v[c + 2 * e + 1] = bf16_bits_to_f32(hi);
        }
      }
    }
  }
  // Row min and max (NaN propagates as in torch's amin / amax).
  float mn = v[0], mx = v[0];
#pragma unroll
  for (int c = 1; c < PART; ++c) {
    mn = (v[c] < mn || v[c] != v[c]) ? v[c] : mn;
    mx = (v[c] > mx || v[c] != v[c]) ? v[c] : mx;
  }
#pragma unroll
  for (int d = 1; d <= 2; d <<= 1) {
    const float mn2 = __shfl_xor(mn, d);
    const float mx2 = __shfl_xor(mx, d);
    mn = (mn2 < mn || mn2 != mn2) ? mn2 : mn;
    mx = (mx2 > mx || mx2 != mx2) ? mx2 : mx;
  }
  float dd = mx - mn;
  dd = dd < 1e-5f ? 1e-5f : dd;  // torch clamp(min=): NaN stays NaN
  const float s = dd / 15.0f;
  float z = -__builtin_rintf(mn / s);
  z = z < 0.f ? 0.f : (z > 15.f ? 15.f : z);
  if (live) {
    uint32_t packed[PART / 4];
#pragma unroll
    for (int c = 0; c < PART; c += 4) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float q = __builtin_rintf(v[c + e] / s) + z;
        q = q < 0.f ? 0.f : (q > 15.f ? 15.f : q);
        word |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * e);
      }
      packed[c / 4] = word;
    }
    uint32_t* dst = reinterpret_cast<uint32_t*>(codes + r * QP + h * PART);
#pragma unroll
    for (int c = 0; c < PART / 4; ++c) dst[c] = packed[c];
    if (h == 0) {
      row_z[r] = z;
      const size_t si = static_cast<size_t>(g) * out_f + o0 + r;
      if constexpr (DTYPE == kDtypeF32) static_cast<float*>(scales)[si] = s;
      else if constexpr (DTYPE == kDtypeF16) static_cast<_Float16*>(scales)[si] = static_cast<_Float16>(s);
      else static_cast<uint16_t*>(scales)[si] = f32_to_bf16_bits(s);
    }
  }
  __syncthreads();

  const int W = rows / 8;    // packed words per input row in this workgroup
  const int C8 = out_f / 8;  // packed words per input row
  if (tid < W) {
    uint32_t word = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) word |= (static_cast<uint32_t>(row_z[8 * tid + c]) & 0xFu) << awq_shift(c);
    qzeros[static_cast<size_t>(g) * C8 + o0 / 8 + tid] = word;
  }
  for (int e = tid; e < GS * W; e += kQuantThreads) {
    const int k = e / W;
    const int j = e - k * W;
    uint32_t word = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c) word |= (static_cast<uint32_t>(codes[(8 * j + c) * QP + k]) & 0xFu) << awq_shift(c);
    qweight[(static_cast<size_t>(g) * GS + k) * C8 + o0 / 8 + j] = word;
  }
}

// One thread per packed word: out[r, c8] = sum_c (v[r, 8 c8 + c] & 15) << awq_shift(c).
__global__ __launch_bounds__(256) void pack_int4_kernel(const int32_t* __restrict__ values,
                                                        uint32_t* __restrict__ packed, int rows, int c8) {
  const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<size_t>(rows) * c8) return;
  const int4* src = reinterpret_cast<const int4*>(values + idx * 8);
  const int4 a = src[0], b = src[1];
  const int v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t word = 0;
#pragma unroll
  for (int c = 0; c < 8; ++c) word |= (static_cast<uint32_t>(v[c]) & 0xFu) << awq_shift(c);
  packed[idx] = word;
}

size_t quantize_lds_bytes(int group_size) {
  return static_cast<size_t>(kQuantRows) * (group_size + 1) * sizeof(float);
}

template <int GS>
static hipError_t launch_quantize_rows(const void* weight, int dtype, uint32_t* qweight, uint32_t* qzeros,
                                       void* scales, int out_f, int in_f, dim3 grid, hipStream_t stream) {
  switch (dtype) {
    case kDtypeF32:
      quantize_rows_kernel<GS, kDtypeF32><<<grid, kQuantThreads, 0, stream>>>(weight, qweight, qzeros, scales, out_f, in_f);
      break;
    case kDtypeF16:
      quantize_rows_kernel<GS, kDtypeF16><<<grid, kQuantThreads, 0, stream>>>(weight, qweight, qzeros, scales, out_f, in_f);
      break;
    default:
      quantize_rows_kernel<GS, kDtypeBF16><<<grid, kQuantThreads, 0, stream>>>(weight, qweight, qzeros, scales, out_f, in_f);
  }
  return hipGetLastError();
}

hipError_t launch_quantize(const void* weight, int dtype, uint32_t* qweight, uint32_t* qzeros, void* scales,
                           int out_f, int in_f, int group_size, hipStream_t stream) {
  const dim3 grid((out_f + kQuantRows - 1) / kQuantRows, in_f / group_size);
  // Fast path: 16-byte aligned weight (every row segment a thread loads is then aligned).
  if (reinterpret_cast<uintptr_t>(weight) % 16 == 0) {
    switch (group_size) {
      case 128: return launch_quantize_rows<128>(weight, dtype, qweight, qzeros, scales, out_f, in_f, grid, stream);
      case 64: return launch_quantize_rows<64>(weight, dtype, qweight, qzeros, scales, out_f, in_f, grid, stream);
      case 32: return launch_quantize_rows<32>(weight, dtype, qweight, qzeros, scales, out_f, in_f, grid, stream);
      default: break;
    }
  }
  const bool vec = reinterpret_cast<uintptr_t>(weight) % 16 == 0 && group_size % (dtype == kDtypeF32 ? 4 : 8) == 0;
  quantize_kernel<<<grid, kQuantThreads, quantize_lds_bytes(group_size), stream>>>(
      weight, dtype, qweight, qzeros, scales, out_f, in_f, group_size, vec);
  return hipGetLastError();
}

hipError_t launch_pack_int4(const int32_t* values, uint32_t* packed, int rows, int cols, hipStream_t stream) {
  const size_t words = static_cast<size_t>(rows) * (cols / 8);
  const unsigned blocks = static_cast<unsigned>((words + 255) / 256);
  pack_int4_kernel<<<blocks, 256, 0, stream>>>(values, packed, rows, cols / 8);
  return hipGetLastError();
}

}  // namespace w4a16
