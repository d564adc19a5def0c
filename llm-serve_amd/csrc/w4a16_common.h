// Device helpers shared by the W4A16 kernels (gfx950 / CDNA4, wave64).
//
// Weight layout ("group blocks").  The kernels read the AutoAWQ words unchanged -- each
// holds 8 consecutive columns of one row, column c at bit 4 * (0,4,1,5,2,6,3,7)[c] --
// but in an order that lets a wavefront fetch one (128-row group g, 32-column block b)
// block of 2 KiB as two 16-byte loads per lane:
//   word index  ((g * (N / 32) + b) * 64 + lane) * 8 + 2 js + h,  js = 0..3, h = 0..1
//   row         k = 128 g + 32 js + 8 ((lane % 16) / 4) + 4 h + lane % 4
//   column word 4 b + lane / 16          (columns 32 b + 8 (lane / 16) .. +7)
//
// Dequant on the matrix cores.  For a 32-row step js, lane l's word h unpacks -- one
// v_and_or_b32 per two values -- into the exact bf16 values (128 + q) of its 8 columns,
// which is the A operand of v_mfma_f32_16x16x32_bf16 (16 rows x 32 columns).  With B the
// 32 x 16 diagonal carrying s for the 16 columns of output tile u and the accumulator
// input C = -(128 + z) s, the MFMA returns (128 + q) s - (128 + z) s = (q - z) s, exact in
// fp32 (every product has <= 16 significant bits and the result is representable), and
// v_cvt_pk_bf16_f32 rounds it like the reference.  Output row i of the MFMA fed by half h
// is weight row 8 (i / 4) + 4 h + i % 4, so a lane's results for h = 0 and 1 are the 8
// consecutive rows k = 8 (lane / 16) .. +7 of its column lane % 16: exactly the B fragment
// of the main v_mfma_f32_16x16x32_bf16, whose A fragment is then the plain 16-byte
// activation load x[row][8 (lane / 16) .. +7].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a16 {

constexpr int kGroup = 128;      // quantization group (rows of K per scale / zero)
constexpr int kBlockCols = 32;   // columns of one layout block
constexpr int kBlockWords = 512; // words of one (group, 32-column) block = 2 KiB

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

// AutoAWQ word -> bf16 fragment holding (128 + q_i), i = 0..7, exactly: bf16 0x4300 is
// 128.0 with a unit last place, so OR-ing a nibble into the low mantissa bits adds it.
// Element 2 j + h holds the nibble at bit 4 j + 16 h.  7 VALU ops per 8 values.
__device__ __forceinline__ bf16x8_t unpack_biased(uint32_t w, const NibbleConsts& k) {
  u32x4_t r;
  r[0] = (w & k.mask) | k.bias;
  r[1] = ((w >> 4) & k.mask) | k.bias;
  r[2] = ((w >> 8) & k.mask) | k.bias;
  r[3] = ((w >> 12) & k.mask) | k.bias;
  return __builtin_bit_cast(bf16x8_t, r);
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Split-K exchange between workgroups.
//
// Partial sums travel as relaxed agent-scope atomic stores and loads, which CDNA
// performs coherently across XCDs (sc1 accesses), so no L2-wide write-back or
// invalidate is needed -- a release/acquire fence at agent scope would emit both
// (buffer_wbl2 / buffer_inv) for every workgroup.  Ordering comes from the hardware:
// each writer's partial stores complete (the workgroup barrier waits for vmcnt(0))
// before one lane increments the arrival counter, and the last arriver issues its
// partial loads only after that increment has returned.
__device__ __forceinline__ void store_partial(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float load_partial(float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// MFMA operands that scale one 16-column output tile u of a 32-column block: the
// diagonal B (lane l carries s in element l % 8 iff lane / 16 == 2 u + (l / 8) % 2, i.e.
// where its inner column 8 (l / 16) + l % 8 equals output column 16 u + l % 16) and the
// accumulator input -(128 + z) s.  s and z are those of the lane's own output column c;
// `s_pair` is the aligned 32-bit word of bf16 scales holding columns c & ~1 and c | 1, so
// the lane's scale sits in half c % 2 == lane % 2 -- where the diagonal wants it.
struct TileScale {
  bf16x8_t diag;
  f32x4_t cin;
};

__device__ __forceinline__ TileScale make_tile_scale(uint32_t s_pair, uint32_t z, int u, int lane) {
  TileScale t;
  const bool hi = (lane & 1) != 0;
  const uint32_t mine = s_pair & (hi ? 0xFFFF0000u : 0x0000FFFFu);
  const bool active = (lane >> 4) == 2 * u + ((lane >> 3) & 1);
  const uint32_t val = active ? mine : 0u;
  const int slot = (lane & 7) >> 1;
  u32x4_t d;
  d[0] = slot == 0 ? val : 0u;
  d[1] = slot == 1 ? val : 0u;
  d[2] = slot == 2 ? val : 0u;
  d[3] = slot == 3 ? val : 0u;
  t.diag = __builtin_bit_cast(bf16x8_t, d);
  const float c = -((128.0f + static_cast<float>(z)) * __uint_as_float(hi ? mine : (mine << 16)));
  t.cin = f32x4_t{c, c, c, c};
  return t;
}

__device__ __forceinline__ uint32_t pack_pair(float a, float b) { return pack_bf16x2(a, b); }

// Two AutoAWQ words (h = 0, 1) of one 32-row step of a 32-column block -> the B fragments
// of its two 16-column tiles, bf16_rne((q - z) s).  4 scaling MFMAs, 14 + 8 VALU ops.
__device__ __forceinline__ void dequant_block(bf16x8_t (&frag)[2], uint32_t w0, uint32_t w1, const TileScale (&ts)[2],
                                              const NibbleConsts& k) {
  const bf16x8_t a0 = unpack_biased(w0, k);
  const bf16x8_t a1 = unpack_biased(w1, k);
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const f32x4_t d0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, ts[u].diag, ts[u].cin, 0, 0, 0);
    const f32x4_t d1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, ts[u].diag, ts[u].cin, 0, 0, 0);
    u32x4_t r;
    r[0] = pack_pair(d0[0], d0[1]);
    r[1] = pack_pair(d0[2], d0[3]);
    r[2] = pack_pair(d1[0], d1[1]);
    r[3] = pack_pair(d1[2], d1[3]);
    frag[u] = __builtin_bit_cast(bf16x8_t, r);
  }
}

// Word offset of lane `lane`'s 8 words in block (g, b) of the group-block layout.
__device__ __forceinline__ size_t block_word(int g, int b, int NB, int lane) {
  return ((static_cast<size_t>(g) * NB + b) * 64 + lane) * 8;
}

}  // namespace w4a16
