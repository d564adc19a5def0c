// Format kernels: AutoAWQ unpack, bit-exact dequant, and the repack into the group-tile
// layout described in w4a16_common.h.  All are HBM-bound byte/integer work.
#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {

// One thread per packed word: out[r, 8c + col] for col = 0..7 (two 16-byte stores).
__global__ __launch_bounds__(256) void unpack_int4_kernel(const uint32_t* __restrict__ packed,
                                                          int32_t* __restrict__ out, int rows, int cols) {
  const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t total = static_cast<size_t>(rows) * cols;
  if (idx >= total) return;
  const uint32_t w = packed[idx];
  int32_t v[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) v[c] = static_cast<int32_t>((w >> awq_shift(c)) & 0xFu);
  int4* dst = reinterpret_cast<int4*>(out + idx * 8);
  dst[0] = make_int4(v[0], v[1], v[2], v[3]);
  dst[1] = make_int4(v[4], v[5], v[6], v[7]);
}

// One thread per qweight word [k, c8]: W[k, 8 c8 + col] = bf16_rne((q - z) * s).  The
// product is formed exactly as the reference does (float(q - z) * s, one rounding), so
// every scale value -- zero, negative, subnormal, inf, NaN -- gives the reference's bits
// (NaN payloads aside).
__global__ __launch_bounds__(256) void dequant_awq_kernel(const uint32_t* __restrict__ qweight,
                                                          const uint32_t* __restrict__ qzeros,
                                                          const uint16_t* __restrict__ scales,
                                                          uint16_t* __restrict__ w_out, int K, int N,
                                                          int group_size) {
  const int C8 = N >> 3;
  const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<size_t>(K) * C8) return;
  const int k = static_cast<int>(idx / C8);
  const int c8 = static_cast<int>(idx - static_cast<size_t>(k) * C8);
  const int g = k / group_size;
  const uint32_t w = qweight[idx];
  const uint32_t zw = qzeros[static_cast<size_t>(g) * C8 + c8];
  const uint4 sv = *reinterpret_cast<const uint4*>(scales + static_cast<size_t>(g) * N + 8 * c8);
  const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
  uint32_t outw[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float f[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = 2 * p + h;
      const int sh = awq_shift(c);
      const int q = static_cast<int>((w >> sh) & 0xFu);
      const int z = static_cast<int>((zw >> sh) & 0xFu);
      const float s = bf16_bits_to_f32(h ? (sw[p] >> 16) : (sw[p] & 0xFFFFu));
      f[h] = static_cast<float>(q - z) * s;
    }
    outw[p] = pack_bf16x2(f[0], f[1]);
  }
  *reinterpret_cast<uint4*>(w_out + idx * 8) = make_uint4(outw[0], outw[1], outw[2], outw[3]);
}

// One thread per output word of the group-tile layout (see w4a16_common.h): gathers the
// 8 nibbles it holds from two AutoAWQ words (rows r and r + 4, the same 4 columns).
// Writes are coalesced; this runs once per weight at load time.
__global__ __launch_bounds__(256) void repack_kernel(const uint32_t* __restrict__ qweight,
                                                     uint32_t* __restrict__ packed, int K, int N) {
  const size_t idx = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const size_t total = static_cast<size_t>(K) * (N >> 3);
  if (idx >= total) return;
  const int NT = N / kTileCols;
  const int js = static_cast<int>(idx & 3);
  const int lane = static_cast<int>((idx >> 2) & 63);
  const size_t tile = idx >> 8;
  const int g = static_cast<int>(tile / NT);
  const int t = static_cast<int>(tile - static_cast<size_t>(g) * NT);
  const int col0 = kTileCols * t + 4 * ((lane >> 2) & 3);  // 4 columns of one AutoAWQ word
  uint32_t out = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = kGroup * g + 32 * js + 8 * (lane >> 4) + 4 * h + (lane & 3);
    const uint32_t src = qweight[static_cast<size_t>(row) * (N >> 3) + (col0 >> 3)];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t q = (src >> awq_shift((col0 + k) & 7)) & 0xFu;
      out |= q << (8 * h + 4 * (k >> 1) + 16 * (k & 1));
    }
  }
  packed[idx] = out;
}

// One wave per (group, 16-column tile): the MFMA GEMMs' dequant (dequant_step) run on the
// tile, with every lane writing the 8 rows x 1 column it produces per step.  Exists to check
// that path bit for bit against the reference.
__global__ __launch_bounds__(256) void dequant_packed_kernel(const uint4* __restrict__ packed,
                                                             const uint32_t* __restrict__ qzeros,
                                                             const uint16_t* __restrict__ scales,
                                                             uint16_t* __restrict__ w_out, int K, int N) {
  const int NT = N / kTileCols;
  const int lane = threadIdx.x & 63;
  const size_t tile = static_cast<size_t>(blockIdx.x) * (blockDim.x >> 6) + wave_id();
  const size_t ntiles = static_cast<size_t>(K / kGroup) * NT;
  if (tile >= ntiles) return;  // whole wave exits together
  const int g = static_cast<int>(tile / NT);
  const int t = static_cast<int>(tile - static_cast<size_t>(g) * NT);
  const uint4 v = packed[tile * 64 + lane];
  const uint32_t words[4] = {v.x, v.y, v.z, v.w};
  const int col = kTileCols * t + (lane & 15);
  const uint32_t s_pair = reinterpret_cast<const uint32_t*>(scales)[(static_cast<size_t>(g) * N + col) >> 1];
  const TileScale ts = make_tile_scale(s_pair, load_zero(qzeros, g, N, col), lane);
  const NibbleConsts nib = nibble_consts();
#pragma unroll
  for (int js = 0; js < 4; ++js) {
    const u32x4_t f = __builtin_bit_cast(u32x4_t, dequant_step(words[js], ts, nib));
    const int k0 = kGroup * g + 32 * js + 8 * (lane >> 4);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      w_out[static_cast<size_t>(k0 + e) * N + col] = static_cast<uint16_t>(f[e >> 1] >> (16 * (e & 1)));
  }
}

static inline unsigned blocks_for(size_t threads, unsigned per_block) {
  return static_cast<unsigned>((threads + per_block - 1) / per_block);
}

hipError_t launch_unpack(const uint32_t* packed, int32_t* out, int rows, int cols, hipStream_t stream) {
  const size_t n = static_cast<size_t>(rows) * cols;
  unpack_int4_kernel<<<blocks_for(n, 256), 256, 0, stream>>>(packed, out, rows, cols);
  return hipGetLastError();
}

hipError_t launch_dequant(const uint32_t* qweight, const uint32_t* qzeros, const uint16_t* scales,
                          uint16_t* w_out, int K, int N, int group_size, hipStream_t stream) {
  const size_t n = static_cast<size_t>(K) * (N >> 3);
  dequant_awq_kernel<<<blocks_for(n, 256), 256, 0, stream>>>(qweight, qzeros, scales, w_out, K, N, group_size);
  return hipGetLastError();
}

hipError_t launch_repack(const uint32_t* qweight, uint32_t* packed, int K, int N, hipStream_t stream) {
  const size_t n = static_cast<size_t>(K) * (N >> 3);
  repack_kernel<<<blocks_for(n, 256), 256, 0, stream>>>(qweight, packed, K, N);
  return hipGetLastError();
}

hipError_t launch_dequant_packed(const uint32_t* packed, const uint32_t* qzeros, const uint16_t* scales,
                                 uint16_t* w_out, int K, int N, hipStream_t stream) {
  const size_t waves = static_cast<size_t>(K / kGroup) * (N / kTileCols);
  dequant_packed_kernel<<<blocks_for(waves, 4), 256, 0, stream>>>(
      reinterpret_cast<const uint4*>(packed), qzeros, scales, w_out, K, N);
  return hipGetLastError();
}

}  // namespace w4a16
