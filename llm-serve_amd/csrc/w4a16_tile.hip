// Chunked-prefill / mixed-batch regime (M > 64): LDS-tiled bf16 MFMA GEMM with the int4
// weights dequantized in registers.
//
// Workgroup = 4 waves, output tile BM x 256 (BM = 16 WM).  Wave w owns columns
// [64 w, 64 w + 64) of the tile and all BM rows: 4 x WM accumulator tiles of
// v_mfma_f32_16x16x32_bf16.  Because a wave's columns belong to it alone, each weight is
// dequantized exactly once per workgroup, on the matrix cores straight from its 16-byte
// loads into MFMA B fragments -- bf16_rne((q - z) s), the reference's weights, see
// dequant_step -- with no LDS round trip.  The activation tile (BM rows x one 128-deep
// group) is shared by all four waves through LDS: it is brought in by direct-to-LDS 16-byte
// buffer loads in a three-stage ring (two groups in flight while one is computed), in a
// row-major layout whose 16-byte chunks are XOR-swizzled by (row & 7) so the A-fragment
// reads are conflict-free.  The weights, scales and zeros of those groups travel in a
// matching ring of registers.
//
// Grid: one workgroup per (m-block, n-block, k-split), enumerated XCD-major so the ~32
// workgroups resident on one XCD cover a few n-blocks x all m-blocks and share their
// operands in that XCD's L2.  With split > 1 the workgroups write fp32 partials and the
// last to arrive at a tile (atomic counter) sums them in split order; the counter is
// re-armed to zero.
#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {

constexpr int kTileWaves = 4;
constexpr int kTileBN = 256;
constexpr int kARowBytes = kGroup * 2;  // one activation row of a stage

typedef __attribute__((address_space(3))) void lds_void_t;

// Issue the direct-to-LDS loads of activation rows [row0, row0 + BM) x group g into `stage`.
// Instruction i of wave w fills rows 16 i + 4 w .. +3 (1 KiB); lane -> (row, physical chunk).
// An invalid group (past the workgroup's K range) fetches nothing.
template <int WM>
__device__ __forceinline__ void issue_a_stage(__amdgpu_buffer_rsrc_t rx, uint8_t* stage, int row0, int M, int K,
                                              int g, bool valid, int wave, int lane) {
  const int p = lane & 15;
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int r = 16 * i + 4 * wave + (lane >> 4);
    const int c = p ^ (r & 7);
    int row = row0 + r;
    row = row < M ? row : M - 1;  // rows past M load a valid row; their outputs are dropped
    const uint32_t off =
        valid ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(K) + kGroup * g + 8u * c) * 2u : kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(stage + (16 * i + 4 * wave) * kARowBytes), 16, off,
                                             0, 0, 0);
  }
}

// Raw loads of one group for a wave's 64 columns (four 16-column layout tiles): one
// 16-byte weight load per tile, and the scale-pair and zero words of the lane's column in
// each tile.  Decoding waits until the group is consumed.  An invalid group (past the K
// range, or a wave whose columns lie past N) fetches nothing.
struct BGroup {
  u32x4_t w[4];
  uint32_t s[4];   // bf16 scale pair holding the lane's column
  uint32_t zw[4];  // AutoAWQ zero word holding the lane's column
};
constexpr int kBLoads = 12;  // buffer loads per BGroup

struct BSources {
  __amdgpu_buffer_rsrc_t w, s, z;
};

__device__ __forceinline__ void load_b_group(BGroup& b, const BSources& src, int g, bool valid, int N, int t0,
                                             int lane) {
  const int NT = N / kTileCols;
  const int c = lane & 15;
  const uint32_t oob = valid ? 0u : kOutOfRange;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int t = t0 + tt;
    const uint32_t wo = valid ? static_cast<uint32_t>(tile_word(g, t, NT, lane)) * 4u : kOutOfRange;
    b.w[tt] = __builtin_amdgcn_raw_buffer_load_b128(src.w, wo, 0, 0);
    const int col = kTileCols * t + c;
    b.s[tt] = __builtin_amdgcn_raw_buffer_load_b32(src.s, oob | (static_cast<uint32_t>(g * N + (col & ~1)) * 2u), 0, 0);
    b.zw[tt] = __builtin_amdgcn_raw_buffer_load_b32(src.z, oob | (static_cast<uint32_t>(g * (N >> 3) + (col >> 3)) * 4u),
                                                    0, 0);
  }
}

// One 128-deep group: per 32-row step, the matrix-core dequant of the wave's 4 weight
// tiles (8 scaling MFMAs), then WM x 4 main MFMAs against the LDS activation tile.
template <int WM>
__device__ __forceinline__ void mma_group(f32x4_t (&acc)[WM][4], const uint8_t* stage, const BGroup& b,
                                          const NibbleConsts& nib, int lane) {
  const int arow = lane & 15;
  const int zshift = awq_shift(lane & 7);
  TileScale ts[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) ts[tt] = make_tile_scale(b.s[tt], (b.zw[tt] >> zshift) & 0xFu, lane);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    bf16x8_t bf[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      bf[tt] = dequant_step(b.w[tt][j], ts[tt], nib);
    }
    const int pchunk = (4 * j + (lane >> 4)) ^ (lane & 7);
    const uint8_t* base = stage + arow * kARowBytes + pchunk * 16;
#pragma unroll
    for (int mt = 0; mt < WM; ++mt) {
      const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(base + mt * 16 * kARowBytes);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) acc[mt][tt] = mfma16(a, bf[tt], acc[mt][tt]);
    }
  }
}

// OCC = waves per SIMD the register allocation must allow (1 or 2).
template <int WM, int OCC>
__global__ __launch_bounds__(256, OCC) void tile_kernel(const uint16_t* __restrict__ x,
                                                      const uint32_t* __restrict__ packed,
                                                      const uint32_t* __restrict__ qzeros,
                                                      const uint16_t* __restrict__ scales,
                                                      uint16_t* __restrict__ y, float* __restrict__ partials,
                                                      int* __restrict__ counters, int M, int K, int N, int split,
                                                      int m_blocks, int n_blocks) {
  constexpr int BM = 16 * WM;
  constexpr int kStage = BM * kARowBytes;
  constexpr int S = WM >= 16 ? 2 : 3;  // pipeline stages (LDS: S * kStage bytes)
  __shared__ __attribute__((aligned(1024))) uint8_t stages[S][kStage];
  __shared__ int is_last;

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int G = K / kGroup;

  // XCD-major enumeration: consecutive blockIdx go to different XCDs (round-robin), so
  // undo that and give each XCD a contiguous run of logical tiles (m fastest).
  const int total = m_blocks * n_blocks * split;
  const int b = blockIdx.x;
  const int per = total >> 3, rem = total & 7, xcd = b & 7, idx = b >> 3;
  const int L = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int mbk = L % m_blocks;
  const int rest = L / m_blocks;
  const int nbk = rest % n_blocks;
  const int sidx = rest / n_blocks;
  const int g_begin = (G * sidx) / split;
  const int g_end = (G * (sidx + 1)) / split;
  const int row0 = mbk * BM;
  const int col_w = nbk * kTileBN + 64 * wave;  // first column of this wave
  const int t0 = col_w / kTileCols;
  const bool active = col_w < N;  // wave-uniform: the last n-block may be partly past N

  f32x4_t acc[WM][4];
#pragma unroll
  for (int mt = 0; mt < WM; ++mt)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) acc[mt][tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // S-stage ring over the workgroup's groups: item i (group g_begin + i) lives in LDS stage
  // and register slot i % S.  Step i waits for every outstanding load (items i .. i + S - 2:
  // direct-to-LDS loads may complete out of order with the register loads issued after
  // them, so a partial count would not cover item i's stage), passes one barrier -- after
  // which every wave has finished item i - 1, whose slot is refilled with item i + S - 1 --
  // and computes item i while items i + 1 .. i + S - 1 are in flight.  The first trip only
  // issues loads.
  const NibbleConsts nib = nibble_consts();
  const __amdgpu_buffer_rsrc_t rx = make_buffer(x, static_cast<uint32_t>(M) * K * 2u);
  const BSources bsrc{make_buffer(packed, static_cast<uint32_t>(K) * (N / 2)),
                      make_buffer(scales, static_cast<uint32_t>(G) * N * 2u),
                      make_buffer(qzeros, static_cast<uint32_t>(G) * (N / 8) * 4u)};
  constexpr int kWaitAll = 0x0F70;  // vmcnt(0); expcnt and lgkmcnt not waited for
  const int n_items = g_end - g_begin;
  BGroup ring[S];
  for (int base = -S; base < n_items; base += S) {
#pragma unroll
    for (int d = 0; d < S; ++d) {
      const int i = base + d;
      const bool live = i >= 0 && i < n_items;
      if (live) {
        __builtin_amdgcn_s_waitcnt(kWaitAll);  // item i's LDS and register loads have landed
        __syncthreads();
      }
      const int ds = (d + S - 1) % S;  // a constant once the loop is unrolled
      const int j = i + S - 1;
      const bool valid = j >= 0 && j < n_items;
      __builtin_amdgcn_sched_barrier(0);
      // Past the last item nothing is issued: no barrier separates those steps from other
      // waves still reading stage ds (item n_items - 1), and an out-of-range direct-to-LDS
      // load may still write its zeros there.  No later step waits on these loads.
      if (i < n_items) {
        issue_a_stage<WM>(rx, stages[ds], row0, M, K, g_begin + j, valid, wave, lane);
        load_b_group(ring[ds], bsrc, g_begin + j, valid && active, N, t0, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (live && active) mma_group<WM>(acc, stages[d], ring[d], nib, lane);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // trailing (empty) loads, before the stages are reused
  __syncthreads();

  if (split > 1) {
    // Every workgroup stores its fp32 fragments (lane-major, 1 KiB per 16 x 16 MFMA tile)
    // into partials[sidx][tile][wave]; the last to arrive sums all splits in split order,
    // 8 fragments at a time so that the loads of a chunk share one wait.
    const int ntiles = m_blocks * n_blocks;
    const int tile = mbk * n_blocks + nbk;
    constexpr int kFrags = WM * 4;
    const __amdgpu_buffer_rsrc_t rp =
        make_buffer(partials, static_cast<uint32_t>(split) * ntiles * kTileWaves * kFrags * 1024u);
    const uint32_t lane_off = static_cast<uint32_t>(lane) * 16u;
    auto frag_off = [&](int sp, int f) {
      return (((static_cast<uint32_t>(sp) * ntiles + tile) * kTileWaves + wave) * kFrags + f) * 1024u + lane_off;
    };
#pragma unroll
    for (int f = 0; f < kFrags; ++f) store_fragment(rp, frag_off(sidx, f), acc[f / 4][f % 4]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) is_last = (arrive(&counters[tile]) == split - 1);
    __syncthreads();
    if (!is_last) return;
#pragma unroll
    for (int c = 0; c < kFrags; c += 8) {
      f32x4_t tot[8];
#pragma unroll
      for (int f = 0; f < 8; ++f) tot[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      for (int sp = 0; sp < split; ++sp) {
        if (sp == sidx) {
#pragma unroll
          for (int f = 0; f < 8; ++f) tot[f] += acc[(c + f) / 4][(c + f) % 4];
        } else {
          f32x4_t part[8];
#pragma unroll
          for (int f = 0; f < 8; ++f) part[f] = load_fragment(rp, frag_off(sp, c + f));
#pragma unroll
          for (int f = 0; f < 8; ++f) tot[f] += part[f];
        }
      }
#pragma unroll
      for (int f = 0; f < 8; ++f) acc[(c + f) / 4][(c + f) % 4] = tot[f];
    }
    if (threadIdx.x == 0) rearm(&counters[tile]);
  }

  if (!active) return;
  // Epilogue: bf16 through LDS (row-major BM x 64 per wave, 16-byte chunks swizzled by
  // row & 7), then 16-byte coalesced stores.  The stages are free after the last barrier.
  uint8_t* ep = &stages[0][0] + wave * (BM * 128);
#pragma unroll
  for (int mt = 0; mt < WM; ++mt)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * mt + 4 * (lane >> 4) + i;
        const int c = 16 * tt + (lane & 15);
        const int off = r * 128 + (((c >> 3) ^ (r & 7)) << 4) + ((c & 7) << 1);
        *reinterpret_cast<uint16_t*>(ep + off) = f32_to_bf16_bits(acc[mt][tt][i]);
      }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
#pragma unroll 4
  for (int round = 0; round < BM / 8; ++round) {
    const int r = 8 * round + (lane >> 3);
    const int q = lane & 7;
    const uint4 v = *reinterpret_cast<const uint4*>(ep + r * 128 + ((q ^ (r & 7)) << 4));
    const int row = row0 + r;
    if (row < M) *reinterpret_cast<uint4*>(y + static_cast<size_t>(row) * N + col_w + 8 * q) = v;
  }
}

template <int WM, int OCC>
static hipError_t launch_tile_t(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                                const uint16_t* scales, uint16_t* y, float* partials, int* counters, int M, int K,
                                int N, int split, hipStream_t stream) {
  const int m_blocks = (M + 16 * WM - 1) / (16 * WM);
  const int n_blocks = (N + kTileBN - 1) / kTileBN;
  const unsigned grid = static_cast<unsigned>(m_blocks * n_blocks * split);
  tile_kernel<WM, OCC><<<grid, 64 * kTileWaves, 0, stream>>>(x, packed, qzeros, scales, y, partials, counters, M,
                                                             K, N, split, m_blocks, n_blocks);
  return hipGetLastError();
}

hipError_t launch_tile_cfg(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                           const uint16_t* scales, uint16_t* y, float* partials, int* counters, int M, int K,
                           int N, int wm, int occ, int split, hipStream_t stream) {
  if (wm == 4) {
    if (occ == 2) return launch_tile_t<4, 2>(x, packed, qzeros, scales, y, partials, counters, M, K, N, split, stream);
    return launch_tile_t<4, 1>(x, packed, qzeros, scales, y, partials, counters, M, K, N, split, stream);
  }
  if (wm == 8) {
    if (occ == 2) return launch_tile_t<8, 2>(x, packed, qzeros, scales, y, partials, counters, M, K, N, split, stream);
    return launch_tile_t<8, 1>(x, packed, qzeros, scales, y, partials, counters, M, K, N, split, stream);
  }
  return launch_tile_t<16, 1>(x, packed, qzeros, scales, y, partials, counters, M, K, N, split, stream);
}

}  // namespace w4a16
