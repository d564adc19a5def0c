// Device helpers shared by the W4A16 kernels (gfx950 / CDNA4, wave64).
//
// Weight layout ("group tiles").  One 1 KiB tile per (128-row group g, 16-column tile
// t): 64 lanes x 4 words, one 32-bit word per lane per 32-row step js, so a wavefront
// fetches a tile with one 16-byte load per lane:
//   word index   ((g * (N / 16) + t) * 64 + lane) * 4 + js
//   word bits    nibble of (row, column) at bit 8 h + 4 (k / 2) + 16 (k % 2), h = 0..1,
//                k = 0..3, with
//   row          128 g + 32 js + 8 (lane / 16) + 4 h + lane % 4
//   column       16 t + 4 ((lane / 4) % 4) + k
// The nibbles are AutoAWQ's unchanged 4-bit values; only their placement differs.
//
// Dequant on the matrix cores.  For step js, lane l's word unpacks -- one v_and_or_b32 per
// two values -- into the exact bf16 values (128 + q): words r_s = ((w >> 4 s) & 0x000F000F)
// | 0x43004300, s = 0..3, so {r_0, r_1} holds k = 0..3 of half h = 0 and {r_2, r_3} those of
// h = 1.  That is the A operand of v_mfma_f32_4x4x4bf16_1k, whose 16 blocks b = l / 4 each
// multiply a 4 x 4 A (lane 4 b + i holds row i) by a 4 x 4 B (lane 4 b + j holds column j).
// With B the diagonal of the block's 4 column scales and the accumulator input
// C = -(128 + z) s, block b returns (128 + q) s - (128 + z) s = (q - z) s, exact in fp32
// (every product has <= 16 significant bits and the result is representable), and
// v_cvt_pk_bf16_f32 rounds it like the reference.  Output register i of lane l (column
// j = l % 4 of block b) is weight row 8 (l / 16) + 4 h + i of column 4 (b % 4) + j = l % 16,
// so the two half-steps give the 8 consecutive rows 8 (l / 16) .. +7 of column l % 16:
// exactly the B fragment of the main v_mfma_f32_16x16x32_bf16, whose A fragment is then the
// plain 16-byte activation load x[row][8 (lane / 16) .. +7].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a16 {

constexpr int kGroup = 128;      // quantization group (rows of K per scale / zero)
// Element types of a float weight given to the quantizer (W4A16_DTYPE_* in w4a16.h).
constexpr int kDtypeBF16 = 0;
constexpr int kDtypeF16 = 1;
constexpr int kDtypeF32 = 2;
constexpr int kTileCols = 16;    // columns of one layout tile
constexpr int kTileWords = 256;  // words of one (group, 16-column) tile = 1 KiB

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

// Bit offset of logical column c (0..7) inside an AutoAWQ word: 4 * (0,4,1,5,2,6,3,7)[c].
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

// Eight bf16 values (one 16-byte chunk) to fp32 and back (round to nearest even).
__device__ __forceinline__ void unpack_bf16x8(uint4 v, float (&f)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

__device__ __forceinline__ uint4 pack_bf16x8(const float (&f)[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

// One DPP move of v between the lanes of each row of 16 (every source lane active).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over each row of 16 lanes, every lane of the row getting the total, by DPP moves in
// registers (a shuffle through the LDS crossbar costs a round trip per step): neighbours
// (quad_perm 1,0,3,2), pairs of them (quad_perm 2,3,0,1), quads (mirror within 8 lanes),
// halves (mirror within 16).  Each step adds the same two partial sums on both lanes, in
// either order, which fp32 addition ignores, so every lane holds the same bits:
// (((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7))) + (...).  All 64 lanes must be active.
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  return v;
}

// Sum over the 64 lanes of a wave, every lane getting the same total: the four row sums,
// then (row 0 + row 2) + (row 1 + row 3).  All 64 lanes must be active.
__device__ __forceinline__ float wave_sum64(float v) {
  v = row_sum16(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r2) + (r1 + r3);
}

// 1 / sqrt(v) for the RMSNorm row scale, evaluated in fp64 and rounded once to fp32 (within
// half an fp32 ulp but for fp64's own rounding); once per row, so fp64 costs nothing.
__device__ __forceinline__ float rsqrt_rn(float v) {
  return static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(v)));
}

// RMSNorm scaling of one chunk of s (fp32, the residual sum): bf16(float(bf16(s * rstd)) *
// weight), the reference's x.to(orig_dtype).mul_(self.weight); the weight product is exact
// in fp32 (two 8-bit significands) and rounded once.
__device__ __forceinline__ uint4 rms_scale_bf16x8(const float (&s)[8], float rstd, const float (&w)[8]) {
  float t[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) t[i] = s[i] * rstd;
  unpack_bf16x8(pack_bf16x8(t), t);
#pragma unroll
  for (int i = 0; i < 8; ++i) t[i] *= w[i];
  return pack_bf16x8(t);
}

__device__ __forceinline__ uint4 rms_scale_bf16x8(const float (&s)[8], float rstd, uint4 weight) {
  float w[8];
  unpack_bf16x8(weight, w);
  return rms_scale_bf16x8(s, rstd, w);
}

// Residual epilogue: eight bf16 GEMM outputs plus eight bf16 residuals, added in fp32 and
// rounded once more -- the reference's order (the layer's bf16 output, then
// x.float() + residual.float() rounded back to bf16).
__device__ __forceinline__ uint4 add_bf16x8(uint4 v, uint4 r) {
  const uint32_t vv[4] = {v.x, v.y, v.z, v.w}, rr[4] = {r.x, r.y, r.z, r.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = pack_bf16x2(bf16_bits_to_f32(vv[e] & 0xFFFFu) + bf16_bits_to_f32(rr[e] & 0xFFFFu),
                       bf16_bits_to_f32(vv[e] >> 16) + bf16_bits_to_f32(rr[e] >> 16));
  return uint4{o[0], o[1], o[2], o[3]};
}

__device__ __forceinline__ uint16_t add_bf16(uint16_t v, uint16_t r) {
  return f32_to_bf16_bits(bf16_bits_to_f32(v) + bf16_bits_to_f32(r));
}

// SiLU(g) * u = g / (1 + e^-g) * u in fp32 for the fused gate/up epilogue, e^-g as
// 2^(-g log2 e) on the hardware exp2 and the quotient by the hardware reciprocal (about
// 1 ulp each, far below the bf16 rounding of the result).  Below g = -44 the reciprocal of
// 1 + e^-g approaches the subnormal range, where it flushes to zero, and below g = -88.7
// e^-g itself overflows, although g u / (1 + e^-g) is still a normal float down to about
// g = -95 (g = -88, u = 15: -8.1e-36): there the quotient is formed as
// g / (2^-64 + 2^(-g log2 e - 64)) * u * 2^-64.  Results below the smallest normal float
// flush to zero.  g -> -inf gives -0, g -> +inf gives g u; NaN propagates.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float t = -g * 1.44269504088896341f;
  const bool low = t > 64.0f;
  const float e = __builtin_amdgcn_exp2f(low ? t - 64.0f : t);
  const float sc = low ? 0x1p-64f : 1.0f;
  return g * __builtin_amdgcn_rcpf(sc + e) * u * sc;
}

// The fused gate/up epilogue from the fp32 accumulators, in the reference's two steps: g and
// u rounded to bf16 first (the gate_up layer's output dtype), then SiLU(g) * u in fp32 and
// one rounding of the result (its SiluAndMul, a compiled pointwise kernel, keeps the
// expression in fp32).
__device__ __forceinline__ float silu_mul_of_bf16(float g, float u) {
  const uint32_t p = pack_bf16x2(g, u);
  return silu_mul(bf16_bits_to_f32(p & 0xFFFFu), __uint_as_float(p & 0xFFFF0000u));
}

// The two constants of the nibble unpack, held in registers: mask 0x000F000F in an SGPR,
// bias 0x43004300 (the bf16 pair (128, 128)) in a VGPR.  Built once per kernel.  The empty
// asm statements emit nothing; they only hide the values from constant folding, so that
// (x & mask) | bias selects to a single v_and_or_b32 (gfx9 VOP3 encodings cannot carry
// literal constants, and with literals the compiler splits it into v_and + v_or).  The
// v_and_or_b32 itself must stay compiler-generated: inline-asm VALU instructions are not
// seen by the compiler's MFMA hazard tracking.
struct NibbleConsts {
  uint32_t mask;
  uint32_t bias;
};

__device__ __forceinline__ NibbleConsts nibble_consts() {
  uint32_t mask = 0x000F000Fu;
  uint32_t bias = 0x43004300u;
  asm volatile("" : "+s"(mask));
  asm volatile("" : "+v"(bias));
  return NibbleConsts{mask, bias};
}

// Tile word -> the two A operands (half-steps h = 0, 1) of the 4x4x4 dequant MFMAs, each
// four exact bf16 values (128 + q): bf16 0x4300 is 128.0 with a unit last place, so OR-ing
// a nibble into the low mantissa bits adds it.  7 VALU ops per 8 values.
__device__ __forceinline__ void unpack_biased(s16x4_t (&a)[2], uint32_t w, const NibbleConsts& k) {
  u32x2_t h0, h1;
  h0[0] = (w & k.mask) | k.bias;
  h0[1] = ((w >> 4) & k.mask) | k.bias;
  h1[0] = ((w >> 8) & k.mask) | k.bias;
  h1[1] = ((w >> 12) & k.mask) | k.bias;
  a[0] = __builtin_bit_cast(s16x4_t, h0);
  a[1] = __builtin_bit_cast(s16x4_t, h1);
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Split-K exchange between workgroups.
//
// Partial sums travel as lane-major 16-byte fragments written and read with the
// device-coherent cache policy sc1 (coherent across XCDs), so no L2-wide write-back or
// invalidate is needed -- a release/acquire fence at agent scope would emit both
// (buffer_wbl2 / buffer_inv) for every workgroup.  Ordering comes from the hardware: each
// writer waits for its fragment stores to complete (s_waitcnt vmcnt(0)) before one lane
// increments the arrival counter with a relaxed agent-scope atomic, and the last arriver
// issues its fragment loads only after that increment has returned.  Plain buffer
// operations rather than atomic loads let the reducer issue many loads before one wait.
constexpr int kCoherentPolicy = 16;        // buffer-op cache policy bits: sc1
constexpr int kRawBufferWord3 = 0x00020000;  // raw (untyped) buffer, 32-bit data format

// Offset used for "fetch nothing": >= every descriptor's size (tensors are < 2 GiB, checked
// on the host).
constexpr uint32_t kOutOfRange = 0x80000000u;

// Buffer descriptor over `bytes` bytes at p: loads past the end return zeros without a
// memory access, stores past the end are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_buffer(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), static_cast<short>(0), static_cast<int>(bytes),
                                           kRawBufferWord3);
}

__device__ __forceinline__ void store_fragment(__amdgpu_buffer_rsrc_t r, uint32_t offset, f32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, offset, 0, kCoherentPolicy);
}

__device__ __forceinline__ f32x4_t load_fragment(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
  return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, kCoherentPolicy));
}

// Arrival count before this workgroup's increment.
__device__ __forceinline__ int arrive(int* counter) {
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void rearm(int* counter) {
  __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Index of the calling wave within its workgroup, as a wave-uniform (scalar) value so
// that branches on it stay scalar branches.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Zero point of column n in group g from the AutoAWQ qzeros tensor [G, N/8].
__device__ __forceinline__ uint32_t load_zero(const uint32_t* __restrict__ qzeros, int g, int N, int n) {
  const uint32_t w = qzeros[static_cast<size_t>(g) * (N >> 3) + (n >> 3)];
  return (w >> awq_shift(n & 7)) & 0xFu;
}

// ---------------------------------------------------------------------------
// Matrix-core dequant (see the layout note at the top of this file).

// MFMA operands that scale one lane's column c = 16 t + lane % 16 of a tile: the diagonal
// B element (lane 4 b + j carries s in element j = lane % 4, zeros elsewhere) and the
// accumulator input -(128 + z) s.  `s_pair` is the aligned 32-bit word of bf16 scales
// holding columns c & ~1 and c | 1, so the lane's scale sits in half c % 2 == lane % 2 --
// where element j = lane % 4 of the diagonal wants it.
struct TileScale {
  s16x4_t diag;
  f32x4_t cin;
};

// Byte selectors of v_perm_b32 over (0, s_pair) for the lane's scale (bytes 0-1 for an even
// column, 2-3 for an odd one): kept in its own half (the diagonal element), moved to the high
// half (its fp32 value), or zero.  They depend on the lane only, so loops hoist them.
__device__ __forceinline__ TileScale make_tile_scale(uint32_t s_pair, uint32_t z, int lane) {
  TileScale t;
  const bool hi = (lane & 1) != 0;
  const bool upper = (lane & 2) != 0;  // element j in 32-bit register j / 2
  constexpr uint32_t kZero = 0x0C0C0C0Cu;
  const uint32_t sel_own = hi ? 0x03020C0Cu : 0x0C0C0100u;
  const uint32_t sel_f32 = hi ? 0x03020C0Cu : 0x01000C0Cu;
  u32x2_t d;
  d[0] = __builtin_amdgcn_perm(0u, s_pair, upper ? kZero : sel_own);
  d[1] = __builtin_amdgcn_perm(0u, s_pair, upper ? sel_own : kZero);
  t.diag = __builtin_bit_cast(s16x4_t, d);
  // 128 + z (z < 16) is exact in fp32 as 0x43000000 | z << 16; the product has 16 significant
  // bits at most, so it is exact too.
  const float c = -(__uint_as_float(0x43000000u | (z << 16)) * __uint_as_float(__builtin_amdgcn_perm(0u, s_pair, sel_f32)));
  t.cin = f32x4_t{c, c, c, c};
  return t;
}

__device__ __forceinline__ f32x4_t mfma4(s16x4_t a, s16x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 0, 0, 0);
}

// One tile word of step js -> the B fragment of the main MFMA for the lane's column,
// bf16_rne((q - z) s) for rows 8 (lane / 16) .. +7.  2 scaling MFMAs, 7 + 4 VALU ops, in two
// phases: the unpack and the scaling MFMAs (dequant_scale), then the rounding to bf16
// (dequant_pack), which a caller may place after other matrix work so that it does not wait
// for the scaling MFMAs' results.
struct ScaledStep {
  f32x4_t d0, d1;
};

__device__ __forceinline__ ScaledStep dequant_scale(uint32_t w, const TileScale& ts, const NibbleConsts& k) {
  s16x4_t a[2];
  unpack_biased(a, w, k);
  return ScaledStep{mfma4(a[0], ts.diag, ts.cin), mfma4(a[1], ts.diag, ts.cin)};
}

__device__ __forceinline__ bf16x8_t dequant_pack(const ScaledStep& d) {
  u32x4_t r;
  r[0] = pack_bf16x2(d.d0[0], d.d0[1]);
  r[1] = pack_bf16x2(d.d0[2], d.d0[3]);
  r[2] = pack_bf16x2(d.d1[0], d.d1[1]);
  r[3] = pack_bf16x2(d.d1[2], d.d1[3]);
  return __builtin_bit_cast(bf16x8_t, r);
}

__device__ __forceinline__ bf16x8_t dequant_step(uint32_t w, const TileScale& ts, const NibbleConsts& k) {
  return dequant_pack(dequant_scale(w, ts, k));
}

// Word offset of lane `lane`'s 4 words in tile (g, t) of the group-tile layout
// (NT = N / 16 tiles per group row).
__device__ __forceinline__ size_t tile_word(int g, int t, int NT, int lane) {
  return ((static_cast<size_t>(g) * NT + t) * 64 + lane) * 4;
}

}  // namespace w4a16
