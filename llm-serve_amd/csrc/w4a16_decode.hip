// Decode / speculative-verify regime (M <= 64): HBM-bound split-K kernel.
//
// Each wave streams (128-row group, 16-column tile) weight tiles (1 KiB, one 16-byte load
// per lane), dequantizes them on the matrix cores (dequant_step: the reference's
// bf16_rne((q - z) s) weights) and multiplies them with up to four 16-row activation
// fragments by v_mfma_f32_16x16x32_bf16, accumulating in fp32.  The output is the
// reference's matmul over the reference's bf16 weights up to fp32 summation order.
//
// Work split.  A workgroup owns TN 16-column tiles and one K range (blockIdx.y of
// `split`); its W waves take interleaved 128-row groups of that range, are reduced
// through LDS in a fixed order, and with split > 1 the workgroups exchange fp32 partials
// (store_fragment / arrive / load_fragment): the last one to finish a column block sums
// them in split order, writes bf16 and re-arms the counter.  Results are deterministic.
#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {

struct DecodeArgs {
  const uint16_t* x;
  const uint32_t* packed;
  const uint32_t* qzeros;
  const uint16_t* scales;
  uint16_t* y;
  float* partials;
  int* counters;
  int M, K, N, split;
};

// Everything one wave needs for one 128-row group: one 16-byte weight load per tile, the
// raw scale-pair and zero words of its TN output columns, and the MB x 4 activation
// fragments.  Loaded DEPTH groups ahead of use; decoded only when consumed.
template <int MB, int TN>
struct DecodeStage {
  u32x4_t w[TN];
  uint32_t s[TN];
  uint32_t zw[TN];
  u32x4_t a[MB][4];
};

// Buffer descriptors of the four inputs.  Every load of the decode kernel is an
// unconditional buffer load: a lane or a group with nothing to fetch (activation row >= M,
// group past the workgroup's K range) uses kOutOfRange, which the hardware answers with
// zeros and no memory access.  With no branch around any load the compiler's wait counts
// are exact, so the DEPTH groups in flight really overlap.
struct DecodeSources {
  __amdgpu_buffer_rsrc_t x, w, s, z;
};

// Byte offsets that do not depend on the group: per activation fragment row (or
// kOutOfRange for rows >= M), and per block of the lane's weight words.
template <int MB>
struct DecodeOffsets {
  uint32_t x_row[MB];  // (row K + 8 (lane / 16)) * 2, or kOutOfRange
};

template <int MB, int TN>
__device__ __forceinline__ void load_decode_stage(DecodeStage<MB, TN>& st, const DecodeSources& src,
                                                  const DecodeOffsets<MB>& off, int g, bool valid, int N, int cb,
                                                  int lane) {
  const int NT = N / kTileCols;
  const int c = lane & 15;
  const uint32_t oob = valid ? 0u : kOutOfRange;
#pragma unroll
  for (int tt = 0; tt < TN; ++tt) {
    const int t = cb * TN + tt;
    const uint32_t wo = (valid ? static_cast<uint32_t>(tile_word(g, t, NT, lane)) * 4u : 0u) | oob;
    st.w[tt] = __builtin_amdgcn_raw_buffer_load_b128(src.w, wo, 0, 0);
    const int col = kTileCols * t + c;
    st.s[tt] = __builtin_amdgcn_raw_buffer_load_b32(src.s, oob | (static_cast<uint32_t>(g * N + (col & ~1)) * 2u), 0, 0);
    st.zw[tt] = __builtin_amdgcn_raw_buffer_load_b32(src.z, oob | (static_cast<uint32_t>(g * (N >> 3) + (col >> 3)) * 4u),
                                                     0, 0);
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const uint32_t xo = (off.x_row[mb] | oob) + static_cast<uint32_t>(kGroup * g) * 2u;
#pragma unroll
    for (int j = 0; j < 4; ++j) st.a[mb][j] = __builtin_amdgcn_raw_buffer_load_b128(src.x, xo + 64u * j, 0, 0);
  }
}

template <int MB, int TN>
__device__ __forceinline__ void compute_decode_stage(f32x4_t (&acc)[MB][TN], const DecodeStage<MB, TN>& st,
                                                     const NibbleConsts& nib, int lane) {
  const int zshift = awq_shift(lane & 7);
  TileScale ts[TN];
#pragma unroll
  for (int tt = 0; tt < TN; ++tt) ts[tt] = make_tile_scale(st.s[tt], (st.zw[tt] >> zshift) & 0xFu, lane);
#pragma unroll
  for (int js = 0; js < 4; ++js) {
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) {
      const bf16x8_t frag = dequant_step(st.w[tt][js], ts[tt], nib);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        acc[mb][tt] = mfma16(__builtin_bit_cast(bf16x8_t, st.a[mb][js]), frag, acc[mb][tt]);
    }
  }
}

template <int MB, int TN, int DEPTH, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void decode_kernel(const uint16_t* __restrict__ x,
                                                            const uint32_t* __restrict__ packed,
                                                            const uint32_t* __restrict__ qzeros,
                                                            const uint16_t* __restrict__ scales,
                                                            uint16_t* __restrict__ y, float* __restrict__ partials,
                                                            int* __restrict__ counters, int M, int K, int N,
                                                            int split) {
  extern __shared__ f32x4_t red[];  // [W][MB][TN][64]
  __shared__ int is_last;
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  constexpr int W = WAVES;
  const int G = K / kGroup;
  const int cb = blockIdx.x;
  const int sidx = blockIdx.y;
  const int g_begin = (G * sidx) / split;
  const int g_end = (G * (sidx + 1)) / split;
  const int col0 = cb * (16 * TN) + (lane & 15);  // this lane's column in tile 0

  DecodeSources src;
  src.x = make_buffer(x, static_cast<uint32_t>(M) * K * 2u);
  src.w = make_buffer(packed, static_cast<uint32_t>(K) * (N / 2));
  src.s = make_buffer(scales, static_cast<uint32_t>(G) * N * 2u);
  src.z = make_buffer(qzeros, static_cast<uint32_t>(G) * (N / 8) * 4u);
  DecodeOffsets<MB> off;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = 16 * mb + (lane & 15);
    off.x_row[mb] = row < M ? static_cast<uint32_t>(row * K + 8 * (lane >> 4)) * 2u : kOutOfRange;
  }

  f32x4_t acc[MB][TN];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) acc[mb][tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Depth-DEPTH ring over the wave's groups g0 + i W (g0 = g_begin + wave): group i is
  // loaded while group i - DEPTH is being consumed.  The first trip only loads (its
  // compute guards are all false), so the loop is the only place loads are issued and
  // each stage's wait is "all but the DEPTH - 1 younger stages".  Loads are issued
  // whether or not the group exists (out-of-range ones fetch nothing): no branch encloses
  // a load, and the scheduling barriers keep each stage's loads together and in order.
  DecodeStage<MB, TN> ring[DEPTH];
  const int g0 = g_begin + wave;
  const NibbleConsts nib = nibble_consts();
  for (int base = g0 - DEPTH * W; base < g_end; base += DEPTH * W) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int g = base + d * W;
      if (g >= g0 && g < g_end) compute_decode_stage<MB, TN>(acc, ring[d], nib, lane);
      const int gn = g + DEPTH * W;
      __builtin_amdgcn_sched_barrier(0);
      load_decode_stage<MB, TN>(ring[d], src, off, gn, gn < g_end, N, cb, lane);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Reduce the W waves' partial sums in wave order.
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) red[((wave * MB + mb) * TN + tt) * 64 + lane] = acc[mb][tt];
  __syncthreads();

  // Output (mb, tt) pairs are spread over the waves; p is a compile-time index so the
  // register arrays stay in registers.
  constexpr int kPairs = MB * TN;
  f32x4_t out[kPairs];
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    if (p % W != wave) continue;
    f32x4_t v = red[p * 64 + lane];
#pragma unroll
    for (int w = 1; w < W; ++w) v += red[(w * kPairs + p) * 64 + lane];
    out[p] = v;
  }

  if (split == 1) {
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      if (p % W != wave) continue;
      const int n = col0 + 16 * (p % TN);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * (p / TN) + 4 * (lane >> 4) + i;
        if (row < M) y[static_cast<size_t>(row) * N + n] = f32_to_bf16_bits(out[p][i]);
      }
    }
    return;
  }

  // Split K: every workgroup stores its fp32 fragments (lane-major, 1 KiB per output pair)
  // into partials[sidx][cb]; the last to arrive sums all splits in split order.
  const int nwg = gridDim.x;
  const __amdgpu_buffer_rsrc_t rp = make_buffer(partials, static_cast<uint32_t>(split) * nwg * kPairs * 1024u);
  const uint32_t lane_off = static_cast<uint32_t>(lane) * 16u;
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    if (p % W != wave) continue;
    store_fragment(rp, ((static_cast<uint32_t>(sidx) * nwg + cb) * kPairs + p) * 1024u + lane_off, out[p]);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) is_last = (arrive(&counters[cb]) == split - 1);
  __syncthreads();
  if (!is_last) return;
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    if (p % W != wave) continue;
    f32x4_t v = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < split; s0 += 4) {
      f32x4_t part[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)  // splits past `split` lie past the buffer: zeros, no access
        part[u] = load_fragment(rp, ((static_cast<uint32_t>(s0 + u) * nwg + cb) * kPairs + p) * 1024u + lane_off);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (s0 + u < split) v += (s0 + u == sidx) ? out[p] : part[u];
    }
    const int n = col0 + 16 * (p % TN);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * (p / TN) + 4 * (lane >> 4) + i;
      if (row < M) y[static_cast<size_t>(row) * N + n] = f32_to_bf16_bits(v[i]);
    }
  }
  if (threadIdx.x == 0) rearm(&counters[cb]);
}

template <int MB, int TN, int DEPTH, int WAVES>
static hipError_t launch_decode_t(const DecodeArgs& a, hipStream_t stream) {
  // Configurations whose cross-wave reduction exceeds 64 KiB of LDS are rejected by the
  // API before launch; they are not instantiated.
  if constexpr (WAVES * MB * TN > 64) {
    return hipErrorInvalidValue;
  } else {
  const dim3 grid(a.N / (kTileCols * TN), a.split);
  const size_t lds = static_cast<size_t>(WAVES) * MB * TN * 64 * sizeof(f32x4_t);
  decode_kernel<MB, TN, DEPTH, WAVES><<<grid, 64 * WAVES, lds, stream>>>(
      a.x, a.packed, a.qzeros, a.scales, a.y, a.partials, a.counters, a.M, a.K, a.N, a.split);
  return hipGetLastError();
  }
}

template <int MB, int TN, int DEPTH>
static hipError_t launch_decode_w(const DecodeArgs& a, int waves, hipStream_t stream) {
  switch (waves) {
    case 4: return launch_decode_t<MB, TN, DEPTH, 4>(a, stream);
    case 8: return launch_decode_t<MB, TN, DEPTH, 8>(a, stream);
    default: return launch_decode_t<MB, TN, DEPTH, 16>(a, stream);
  }
}

template <int MB, int TN>
static hipError_t launch_decode_d(const DecodeArgs& a, int depth, int waves, hipStream_t stream) {
  switch (depth) {
    case 1: return launch_decode_w<MB, TN, 1>(a, waves, stream);
    case 2: return launch_decode_w<MB, TN, 2>(a, waves, stream);
    default: return launch_decode_w<MB, TN, 4>(a, waves, stream);
  }
}

template <int MB>
static hipError_t launch_decode_m(const DecodeArgs& a, int tn, int depth, int waves, hipStream_t stream) {
  switch (tn) {
    case 1: return launch_decode_d<MB, 1>(a, depth, waves, stream);
    case 2: return launch_decode_d<MB, 2>(a, depth, waves, stream);
    case 3: return launch_decode_d<MB, 3>(a, depth, waves, stream);
    default: return launch_decode_d<MB, 4>(a, depth, waves, stream);
  }
}

hipError_t launch_decode_cfg(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                             const uint16_t* scales, uint16_t* y, float* partials, int* counters, int M, int K,
                             int N, int tn, int depth, int waves, int split, hipStream_t stream) {
  const DecodeArgs a{x, packed, qzeros, scales, y, partials, counters, M, K, N, split};
  switch ((M + 15) / 16) {
    case 1: return launch_decode_m<1>(a, tn, depth, waves, stream);
    case 2: return launch_decode_m<2>(a, tn, depth, waves, stream);
    case 3: return launch_decode_m<3>(a, tn, depth, waves, stream);
    default: return launch_decode_m<4>(a, tn, depth, waves, stream);
  }
}

}  // namespace w4a16
