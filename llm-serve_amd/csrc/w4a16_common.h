// Device helpers shared by the W4A16 kernels (gfx950 / CDNA4, wave64).
//
// Fragment layout ("K8 words"): the GEMM kernels consume the weights as one 32-bit word
// per (8 consecutive k, 1 column n), arranged so that a wavefront's 64 lanes load a
// whole 1 KiB block -- (128-row group g, 16-column tile t) -- with one 16-byte load each:
//   word index  ((g * NT + t) * 64 + lane) * 4 + j,   NT = N / 16
//   column      n = 16 t + lane % 16
//   rows        k = 128 g + 32 j + 8 (lane / 16) + i,  i = 0..7
//   value i     at bit offset 4 * (0,4,1,5,2,6,3,7)[i]  (AutoAWQ's nibble order, along K)
// This is exactly the B-operand fragment of v_mfma_f32_16x16x32_bf16 for k-step j:
// lane l supplies column l % 16 and k = 8 (l / 16) .. +7 of the 32-deep step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a16 {

constexpr int kGroup = 128;       // quantization group (rows of K per scale / zero)
constexpr int kTileN = 16;        // columns per MFMA tile
constexpr int kBlockWords = 256;  // words per (group, column tile) block = 1 KiB

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Bit offset of logical column c (0..7) inside an AutoAWQ word: 4 * (0,4,1,5,2,6,3,7)[c].
// The same offsets place value i of a K8 word.
__device__ __forceinline__ int awq_shift(int c) { return ((c & 1) << 4) | ((c >> 1) << 2); }

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even float pair -> packed bf16 pair (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2_t v = {lo, hi};
  bf16x2_t b = __builtin_convertvector(v, bf16x2_t);
  return __builtin_bit_cast(uint32_t, b);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
  return static_cast<uint16_t>(pack_bf16x2(v, 0.0f) & 0xFFFFu);
}

// (x & mask) | bias in one VALU op; mask comes from an SGPR, bias from a VGPR (CDNA VOP3
// encodings cannot carry literal constants).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t bias) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(bias));
  return r;
}

// K8 word -> bf16 fragment holding (128 + q_i), i = 0..7, exactly: bf16 0x4300 is 128.0
// with a unit last place, so OR-ing a nibble into the low mantissa bits adds it.
// 7 VALU ops per 8 values.
__device__ __forceinline__ bf16x8_t unpack_biased(uint32_t w, uint32_t bias_v) {
  const uint32_t m = 0x000F000Fu;
  u32x4_t r;
  r[0] = and_or(w, m, bias_v);
  r[1] = and_or(w >> 4, m, bias_v);
  r[2] = and_or(w >> 8, m, bias_v);
  r[3] = and_or(w >> 12, m, bias_v);
  return __builtin_bit_cast(bf16x8_t, r);
}

// In-register dequant used by the MFMA tile GEMM: W = fma(q, s, -(z*s)).  z*s and q*s
// carry at most 12 significant bits, so for every finite scale with |s| < 2^123 the fma
// yields the exact (q - z) * s and the bf16 rounding gives the reference's bits
// (bf16_rne((q - z) * s), computed by the reference as float(q - z) * s), with one
// exception: a zero weight is always +0, where the reference has -0 when (q - z) * s is a
// negative zero (s <= 0).  AutoAWQ scales are (max - min) / 15 > 0, so for checkpoints the
// weights are identical; the standalone dequant kernel keeps the reference's arithmetic
// order for every scale.
struct DequantScale {
  float s;
  float nzs;  // -(z * s), exact
};

__device__ __forceinline__ DequantScale make_dequant_scale(float s, uint32_t z) {
  DequantScale d;
  d.s = s;
  d.nzs = -(static_cast<float>(z) * s);
  return d;
}

// K8 word -> bf16 fragment of bf16_rne((q_i - z) * s) (see DequantScale):
// 3 (split) + 8 (cvt_f32_ubyte) + 8 (fma) + 4 (cvt_pk_bf16) VALU ops per 8 values.
__device__ __forceinline__ bf16x8_t dequant_k8(uint32_t w, const DequantScale& d) {
  // The masks go through opaque asm so the compiler keeps one v_cvt_f32_ubyteN per value
  // instead of re-deriving a v_bfe_u32 for each nibble.
  uint32_t lo, hi;
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(lo) : "v"(w));         // bytes: i = 0, 4, 1, 5
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(hi) : "v"(w >> 4));    // bytes: i = 2, 6, 3, 7
  float q[8];
  q[0] = static_cast<float>(lo & 0xFFu);
  q[4] = static_cast<float>((lo >> 8) & 0xFFu);
  q[1] = static_cast<float>((lo >> 16) & 0xFFu);
  q[5] = static_cast<float>(lo >> 24);
  q[2] = static_cast<float>(hi & 0xFFu);
  q[6] = static_cast<float>((hi >> 8) & 0xFFu);
  q[3] = static_cast<float>((hi >> 16) & 0xFFu);
  q[7] = static_cast<float>(hi >> 24);
  float f[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = __builtin_fmaf(q[i], d.s, d.nzs);
  u32x4_t r;
  r[0] = pack_bf16x2(f[0], f[1]);
  r[1] = pack_bf16x2(f[2], f[3]);
  r[2] = pack_bf16x2(f[4], f[5]);
  r[3] = pack_bf16x2(f[6], f[7]);
  return __builtin_bit_cast(bf16x8_t, r);
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Index of the calling wave within its workgroup, as a wave-uniform (scalar) value so
// that branches on it stay scalar branches.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Zero point of column n in group g from the AutoAWQ qzeros tensor [G, N/8].
__device__ __forceinline__ uint32_t load_zero(const uint32_t* __restrict__ qzeros, int g, int N, int n) {
  const uint32_t w = qzeros[static_cast<size_t>(g) * (N >> 3) + (n >> 3)];
  return (w >> awq_shift(n & 7)) & 0xFu;
}

}  // namespace w4a16
