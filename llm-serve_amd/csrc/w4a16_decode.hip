// Decode / speculative-verify regime (M <= 64): HBM-bound split-K kernel.
//
// Each lane dequantizes its weights in registers exactly as the reference does --
// bf16_rne((q - z) s), see dequant_k8 -- and feeds them to v_mfma_f32_16x16x32_bf16
// against up to four 16-row activation fragments, accumulating in fp32.  The output is
// therefore the reference's matmul over the reference's bf16 weights, up to fp32
// summation order.
//
// Work split.  A workgroup owns TN 16-column tiles (16 TN columns) and one K range
// (blockIdx.y of `split`); its W waves take interleaved 128-row groups of that range and
// are reduced through LDS in a fixed order.  With split > 1 the workgroups write fp32
// partials; the last one to finish a column block (atomic arrival counter) sums them in
// split order and writes bf16, then re-arms the counter to zero.  Results are therefore
// deterministic run to run.
#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {

template <int MB, int TN, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void decode_kernel(const uint16_t* __restrict__ x,
                                                      const uint4* __restrict__ packed,
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
  const int NT = N >> 4;
  const int G = K / kGroup;
  const int cb = blockIdx.x;
  const int sidx = blockIdx.y;
  const int g_begin = (G * sidx) / split;
  const int g_end = (G * (sidx + 1)) / split;
  const int col0 = cb * (16 * TN) + (lane & 15);  // this lane's column in tile 0
  const f32x4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  const u32x4_t zero_u = {0u, 0u, 0u, 0u};
  const bf16x8_t zero_a = __builtin_bit_cast(bf16x8_t, zero_u);

  f32x4_t acc[MB][TN];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) acc[mb][tt] = zero4;

  // One-group-ahead prefetch of the HBM stream (weights, scales, zeros).
  uint4 bw[TN];
  float sc[TN];
  uint32_t zz[TN];
  int g = g_begin + wave;
  if (g < g_end) {
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) {
      const int n = col0 + 16 * tt;
      bw[tt] = packed[(static_cast<size_t>(g) * NT + cb * TN + tt) * 64 + lane];
      sc[tt] = bf16_bits_to_f32(scales[static_cast<size_t>(g) * N + n]);
      zz[tt] = load_zero(qzeros, g, N, n);
    }
  }
  for (; g < g_end; g += W) {
    const int gn = g + W;
    uint4 bw_n[TN];
    float sc_n[TN];
    uint32_t zz_n[TN];
    if (gn < g_end) {
#pragma unroll
      for (int tt = 0; tt < TN; ++tt) {
        const int n = col0 + 16 * tt;
        bw_n[tt] = packed[(static_cast<size_t>(gn) * NT + cb * TN + tt) * 64 + lane];
        sc_n[tt] = bf16_bits_to_f32(scales[static_cast<size_t>(gn) * N + n]);
        zz_n[tt] = load_zero(qzeros, gn, N, n);
      }
    }
    // Activation fragments: row 16 mb + lane % 16, k = 128 g + 32 j + 8 (lane / 16) .. +7.
    bf16x8_t a[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int row = 16 * mb + (lane & 15);
      const bf16x8_t* src = reinterpret_cast<const bf16x8_t*>(
          x + static_cast<size_t>(row) * K + kGroup * g + 8 * (lane >> 4));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (row < M) {
          a[mb][j] = src[4 * j];
        } else {
          a[mb][j] = zero_a;
        }
      }
    }
    DequantScale d[TN];
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) d[tt] = make_dequant_scale(sc[tt], zz[tt]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int tt = 0; tt < TN; ++tt) {
        const uint32_t wj = j == 0 ? bw[tt].x : j == 1 ? bw[tt].y : j == 2 ? bw[tt].z : bw[tt].w;
        const bf16x8_t b = dequant_k8(wj, d[tt]);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb][tt] = mfma16(a[mb][j], b, acc[mb][tt]);
      }
    }
    if (gn < g_end) {
#pragma unroll
      for (int tt = 0; tt < TN; ++tt) {
        bw[tt] = bw_n[tt];
        sc[tt] = sc_n[tt];
        zz[tt] = zz_n[tt];
      }
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

#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    if (p % W != wave) continue;
    const int n = col0 + 16 * (p % TN);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * (p / TN) + 4 * (lane >> 4) + i;
      if (row < M) partials[(static_cast<size_t>(sidx) * M + row) * N + n] = out[p][i];
    }
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int arrived = __hip_atomic_fetch_add(&counters[cb], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (arrived == split - 1);
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    if (p % W != wave) continue;
    const int n = col0 + 16 * (p % TN);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * (p / TN) + 4 * (lane >> 4) + i;
      if (row < M) {
        float v = 0.0f;
        for (int s = 0; s < split; ++s)
          v += (s == sidx) ? out[p][i] : partials[(static_cast<size_t>(s) * M + row) * N + n];
        y[static_cast<size_t>(row) * N + n] = f32_to_bf16_bits(v);
      }
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(&counters[cb], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int MB, int TN, int WAVES>
static hipError_t launch_decode_t(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                                  const uint16_t* scales, uint16_t* y, float* partials, int* counters, int M,
                                  int K, int N, int split, hipStream_t stream) {
  const dim3 grid(N / (16 * TN), split);
  const size_t lds = static_cast<size_t>(WAVES) * MB * TN * 64 * sizeof(f32x4_t);
  decode_kernel<MB, TN, WAVES><<<grid, 64 * WAVES, lds, stream>>>(
      x, reinterpret_cast<const uint4*>(packed), qzeros, scales, y, partials, counters, M, K, N, split);
  return hipGetLastError();
}

template <int MB, int TN>
static hipError_t launch_decode_w(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                                  const uint16_t* scales, uint16_t* y, float* partials, int* counters, int M,
                                  int K, int N, int waves, int split, hipStream_t stream) {
  switch (waves) {
    case 4: return launch_decode_t<MB, TN, 4>(x, packed, qzeros, scales, y, partials, counters, M, K, N, split, stream);
    case 8: return launch_decode_t<MB, TN, 8>(x, packed, qzeros, scales, y, partials, counters, M, K, N, split, stream);
    default: return launch_decode_t<MB, TN, 16>(x, packed, qzeros, scales, y, partials, counters, M, K, N, split, stream);
  }
}

template <int MB>
static hipError_t launch_decode_m(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                                  const uint16_t* scales, uint16_t* y, float* partials, int* counters, int M,
                                  int K, int N, int tn, int waves, int split, hipStream_t stream) {
  switch (tn) {
    case 1: return launch_decode_w<MB, 1>(x, packed, qzeros, scales, y, partials, counters, M, K, N, waves, split, stream);
    case 2: return launch_decode_w<MB, 2>(x, packed, qzeros, scales, y, partials, counters, M, K, N, waves, split, stream);
    default: return launch_decode_w<MB, 4>(x, packed, qzeros, scales, y, partials, counters, M, K, N, waves, split, stream);
  }
}

// tn in {1, 2, 4} column tiles per workgroup, waves in {4, 8, 16}, 1 <= split <= K / 128.
hipError_t launch_decode_cfg(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                             const uint16_t* scales, uint16_t* y, float* partials, int* counters, int M, int K,
                             int N, int tn, int waves, int split, hipStream_t stream) {
  switch ((M + 15) / 16) {
    case 1: return launch_decode_m<1>(x, packed, qzeros, scales, y, partials, counters, M, K, N, tn, waves, split, stream);
    case 2: return launch_decode_m<2>(x, packed, qzeros, scales, y, partials, counters, M, K, N, tn, waves, split, stream);
    case 3: return launch_decode_m<3>(x, packed, qzeros, scales, y, partials, counters, M, K, N, tn, waves, split, stream);
    default: return launch_decode_m<4>(x, packed, qzeros, scales, y, partials, counters, M, K, N, tn, waves, split, stream);
  }
}

}  // namespace w4a16
