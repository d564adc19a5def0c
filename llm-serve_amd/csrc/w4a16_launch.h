// Host-side launchers, one per kernel family; each translation unit that defines a
// kernel also defines its launcher, so no relocatable device code is needed.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace w4a16 {

hipError_t launch_unpack(const uint32_t* packed, int32_t* out, int rows, int cols, hipStream_t stream);
hipError_t launch_dequant(const uint32_t* qweight, const uint32_t* qzeros, const uint16_t* scales,
                          uint16_t* w_out, int K, int N, int group_size, hipStream_t stream);
hipError_t launch_repack(const uint32_t* qweight, uint32_t* packed, int K, int N, hipStream_t stream);
hipError_t launch_dequant_packed(const uint32_t* packed, const uint32_t* qzeros, const uint16_t* scales,
                                 uint16_t* w_out, int K, int N, hipStream_t stream);

// Quantizer and packer (producer side of the format).  quantize: W [out_f, in_f] of element
// type dtype (kDtype*) -> qweight [in_f, out_f / 8], qzeros [in_f / group_size, out_f / 8],
// scales [in_f / group_size, out_f] of type dtype; out_f % 8 == 0, 1 <= group_size <= 128
// dividing in_f.  pack: int32 [rows, cols] (cols % 8 == 0, values masked to 4 bits) ->
// [rows, cols / 8] AutoAWQ words.
hipError_t launch_quantize(const void* weight, int dtype, uint32_t* qweight, uint32_t* qzeros, void* scales,
                           int out_f, int in_f, int group_size, hipStream_t stream);
hipError_t launch_pack_int4(const int32_t* values, uint32_t* packed, int rows, int cols, hipStream_t stream);

// Split-K decode kernel, M <= 64.  tn in {1, 2, 3, 4, 6} 16-column tiles per workgroup (tn
// divides N / 16), depth in {1, 2, 4} groups in flight per wave, waves in {4, 8},
// 1 <= split <= K / 128, decode_config_fits() and decode_lds_bytes() <= kDecodeMaxLds.
// `partials` holds the split-K fp32 fragments and `counters` N / (16 tn) ints (both unused
// when split == 1).
// LDS of one decode workgroup: a gfx950 CU has 160 KiB; the kernel's static LDS must fit
// beside the dynamic part (a launch past the total is not rejected by the runtime: it faults).
constexpr size_t kDecodeMaxLds = 156 * 1024;
constexpr size_t kDecodeMaxStagedX = 32 * 1024;  // activations staged in LDS (M <= 4 only)

// Whether the activations of an (M, K, split) problem are staged in LDS.
bool decode_stages_x(int M, int K, int split);
// Register staging of a decode wave's scale words, zero words and (staged rows) activation
// chunks: at most this many 64-lane loads of each per launch (one-tile workgroups with
// prebuilt dequant operands: one scale and one zero word per (group, column) entry, at most
// kStageE loads of each).
constexpr int kStageS = 3;
constexpr int kStageZ = 1;
constexpr int kStageX = 4;
constexpr int kStageE = 4;
// ns: the fused-norm consumer (DecodeRowStats), which stages its normalized rows (M <= 8, at
// most 4 groups per wave).
bool decode_stage_fits(int M, int K, int tn, int waves, int depth, int split, bool ns = false);
// Whether a decode configuration builds its dequant operands once per wave in LDS
// (8 waves and a ring at least two groups deep) instead of per tile and group.
constexpr bool decode_prebuilt_scales(int waves, int depth) { return waves >= 8 && depth >= 2; }
// LDS bytes of a decode workgroup: staged scales, zeros (and activations, and prebuilt
// dequant operands), or the cross-wave reduction, whichever is larger.
size_t decode_lds_bytes(int M, int K, int tn, int waves, int depth, int split, bool ns = false);

// Register budget of a decode configuration (16-row activation blocks mb, tiles tn, ring
// depth, activations staged or not): fp32 accumulators plus the ring of in-flight loads,
// in 32-bit registers per lane, at most 176.  Configurations beyond it are not compiled.
constexpr int decode_ring_regs(int mb, int tn, int depth, bool xl) {
  return 4 * mb * tn + depth * 4 * (tn + (xl ? 0 : 4 * mb));
}
constexpr bool decode_config_fits(int mb, int tn, int depth, bool xl) {
  return decode_ring_regs(mb, tn, depth, xl) <= 176;
}

// RMSNorm(+residual) prologue of a decode GEMM whose activations are staged in LDS: the
// GEMM input is x_norm = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * w), s = x + res (fp32; s = x
// without res), computed by every workgroup from its staged rows; the first workgroup also
// writes res_out = bf16(s) (when res is given) and x_out = x_norm.  None of res_out, x_out
// may alias x or res.
struct DecodeNorm {
  const uint16_t* res;  // [M, K] residual or null
  const uint16_t* w;    // [K] norm weight
  uint16_t* res_out;    // [M, K] new residual (null iff res is null)
  uint16_t* x_out;      // [M, K] normalized activations
  float eps;
};

// An RMSNorm split across two decode GEMMs (M <= 8), so that no separate norm launch sits
// between them.  The producer -- the O or down projection, whose output h feeds the norm --
// adds the residual in its epilogue as the reference's add_rms_forward does, s =
// float(bf16(h)) + float(res) in fp32, and writes s (s_out, fp32 [M, N]), the new residual
// bf16(s) (res_out, [M, N]; may be res itself) and, per row, the sum of s^2 over each
// 16-column tile (ssq_out, [M, N / 16]).  The consumer -- the QKV or gate|up projection
// behind the norm -- reads s (s_in, [M, K]) and the tile sums (ssq_in, [M, K / 16]), sums
// each row's in a fixed order to rstd = 1 / sqrt(mean(s^2) + eps), and stages x_norm =
// bf16(bf16(s * rstd) * w) (w: the norm weight, [K]) in LDS as its activations; the
// workgroups of its first column block also store x_norm (x_out, [M, K], may be null).
struct DecodeRowStats {
  float* s_out;
  uint16_t* res_out;
  float* ssq_out;
  const float* s_in;
  const float* ssq_in;
  const uint16_t* w;
  float eps;
  uint16_t* x_out;
};

// LDS bytes of a decode workgroup that also runs the norm prologue (the same layout as
// without it: the prologue works from registers and writes the activation slice), or 0 if
// the configuration cannot run it (M > 2, activations not staged, a K split, or more than
// four groups per wave).
size_t decode_norm_lds_bytes(int M, int K, int tn, int waves, int depth, int split);

// up_tiles: 0 for the plain GEMM (y is [M, N]); N / 32 for the fused SiLU(gate) * up of a
// gate|up weight (tn even, N % 128 == 0, y is [M, N / 2]).  res: null, or a bf16 [M, N]
// residual added in the epilogue (plain GEMM only; may be y itself).  norm: null, or the
// prologue above (requires decode_norm_lds_bytes(...) in (0, kDecodeMaxLds]).
// rs: null, or the producer half (s_out set: plain GEMM with res) or the consumer half (s_in
// set: x is then unused, M < 32) of a fused RMSNorm.
hipError_t launch_decode_cfg(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                             const uint16_t* scales, uint16_t* y, const uint16_t* res, float* partials,
                             int* counters, int M, int K, int N, int tn, int depth, int waves, int split, int up_tiles,
                             const DecodeNorm* norm, hipStream_t stream, const DecodeRowStats* rs = nullptr);

// LDS-tiled MFMA GEMM.  A tile shape code selects the wave grid: wk K slices of nwm waves
// along M x nwn along N, each wave owning tw 16-column layout tiles and 16 wm rows, so the
// workgroup tile is (16 wm nwm) x (16 tw nwn) and has nwm nwn wk waves.  Codes: 1 (or 0) =
// {tw 4, 1 x 4}, 2 = {tw 4, 2 x 4}, 3 = {tw 2, 1 x 8}, 4 = {tw 2, 1 x 2, 4 slices},
// 5 = {tw 2, 1 x 4, 2 slices}, 6 = {tw 2, 1 x 2, 2 slices}, 7 = {tw 2, 1 x 1, 4 slices},
// 8 = {tw 4, 1 x 8}, 9 = {tw 2, 1 x 3, 4 slices}, 10 = {tw 2, 1 x 6, 2 slices},
// 11 = {tw 3, 1 x 8} (plain GEMM only: the fused product pairs tiles within a wave).
constexpr int kTileShapeMax = 11;
struct TileShape {
  int tw, nwm, nwn, wk;
};
TileShape tile_shape(int shape);
// Whether (wm, shape, occ) is compiled; occ = waves per SIMD the register allocation targets.
// Compiled (wm, shape, occ): (4,1,1), (4,1,2), (8,1,1), (4,2,2), (4,3,2), (8,3,2), (2,4,2),
// (4,4,2), (2,5,2), (4,5,2), (8,5,2), (4,6,1), (8,6,1), (2,7,1), (4,7,1), (8,8,2), (4,9,3),
// (2,9,3), (4,10,3), (8,11,2), (4,11,2), (6,3,2), (6,8,2), (6,11,2).
bool tile_config_compiled(int wm, int shape, int occ);
// `partials` holds the split-K fp32 fragments and `counters` one int per output tile (both
// unused when split == 1).  up_tiles and res as for the decode kernel (N % 128 == 0 when
// fused; res 16-byte aligned).
hipError_t launch_tile_cfg(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                           const uint16_t* scales, uint16_t* y, const uint16_t* res, float* partials, int* counters,
                           int M, int K, int N, int wm, int shape, int occ, int split, int up_tiles,
                           hipStream_t stream);

// RMSNorm of each row of x [M, K] (after adding residual [M, K] when it is not null, which
// then also writes residual_out = bf16(x + residual)); K % 8 == 0, K <= kNormMaxK, every
// pointer 16-byte aligned; residual_out may be residual or x, x_norm may be x.
constexpr int kNormMaxK = 16384;
hipError_t launch_add_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                              uint16_t* x_norm, uint16_t* residual_out, int M, int K, float eps,
                              hipStream_t stream);
// RMSNorm without a residual of rows read through two strides: row r of x starts at element
// (r / rows_inner) * stride_outer + (r % rows_inner) * stride_inner (multiples of 8, x 16-byte
// aligned); x_norm is contiguous [M, K].
hipError_t launch_rmsnorm_strided(const uint16_t* x, int rows_inner, int64_t stride_outer, int64_t stride_inner,
                                  const uint16_t* weight, uint16_t* x_norm, int M, int K, float eps,
                                  hipStream_t stream);

}  // namespace w4a16
