// Chunked-prefill / mixed-batch regime (M > 64, and M > 48 for N >= 16384): LDS-tiled bf16
// MFMA GEMM with the int4 weights dequantized in registers.
//
// Workgroup = NWM x NWN waves, output tile BM x BN (BM = 16 WM NWM, BN = 16 TW NWN).  Wave
// (wm, wn) owns TW 16-column layout tiles (columns [16 TW wn, 16 TW (wn + 1)) of the tile)
// and rows [16 WM wm, 16 WM (wm + 1)): WM x TW accumulator tiles of
// v_mfma_f32_16x16x32_bf16.  Each wave dequantizes its own columns on the matrix cores
// straight from its 16-byte loads into MFMA B fragments -- bf16_rne((q - z) s), the
// reference's weights, see dequant_step -- with no LDS round trip, so a weight is
// dequantized NWM times per workgroup and used for 16 WM rows each time: the dequant work
// per main MFMA falls as 1 / WM whatever TW is.  The activation tile (BM rows x one 128-deep
// group) is shared by all waves through LDS: it is brought in by direct-to-LDS 16-byte
// buffer loads, one or two groups per batch with the next batch in flight while one is
// computed, in a row-major layout whose sixteen 16-byte chunks per row are XOR-swizzled by
// (row & 15): the 16 lanes reading one fragment chunk (16 consecutive rows) then hit 16
// different chunk positions, i.e. all 64 LDS banks once.  The scales and zero words of the
// workgroup's columns for those groups are staged beside them (two direct-to-LDS loads per
// group for the whole workgroup, issue_sz_stage), and the weights travel in a matching ring
// of registers.
//
// K split inside the workgroup (WK > 1, for short and mid-sized M on narrow layers): the
// workgroup's waves form WK slices of NWM x NWN waves; slice k computes the groups k, k + WK,
// ... of each load batch (P = WK groups per batch, staged together), so narrow column blocks
// still keep 8 waves busy and share each group's activation stage among the NWM x NWN waves
// of a slice.  After the K loop the slices' fp32 tiles are summed through LDS in slice order
// by slice 0, which alone takes part in the split-K exchange and the epilogue.
//
// Grid: one workgroup per (m-block, n-block, k-split), enumerated XCD-major so the
// workgroups resident on one XCD cover a few n-blocks x all m-blocks and share their
// operands in that XCD's L2.  With split > 1 the workgroups write fp32 partials and the
// last to arrive at a tile (atomic counter) sums them in split order; the counter is
// re-armed to zero.
#include <type_traits>

#include "w4a16_common.h"
#include "w4a16_launch.h"
#include "w4a16_mma.h"

namespace w4a16 {

typedef __attribute__((address_space(3))) void lds_void_t;

// Issue the direct-to-LDS loads of activation rows [row0, row0 + BM) x group g into `stage`
// (NW waves, NI instructions each).  Instruction i of wave w fills rows 4 (NW i + w) .. +3
// (1 KiB); lane -> (row, physical chunk).  When the BM / 4 row quads do not split evenly over
// the waves, the instructions past them fetch nothing into `spare` (1 KiB of LDS no one
// reads), so that every wave issues the same NI loads.  g is a group of the activations
// (callers clamp a prefetch past their K range to its last group); the group's part of the
// offset is the instruction's scalar offset, the lane's part the same for every group, and
// their sum stays inside the activations (rows past M read row M - 1).
template <int NI, int NW, int BM>
__device__ __forceinline__ void issue_a_stage(__amdgpu_buffer_rsrc_t rx, uint8_t* stage, uint8_t* spare, int row0,
                                              int M, int K, int g, int wave, int lane) {
  const int p = lane & 15;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int quad = NW * i + wave;
    const bool in = NI * NW * 4 == BM || quad < BM / 4;  // wave-uniform
    const int r = 4 * quad + (lane >> 4);
    const int c = p ^ (r & 15);
    int row = row0 + r;
    row = row < M ? row : M - 1;  // rows past M load a valid row; their outputs are dropped
    const uint32_t off = in ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(K) + 8u * c) * 2u : kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(in ? stage + quad * 4 * kARowBytes : spare), 16, off,
                                             static_cast<int>(static_cast<uint32_t>(g) * kGroup * 2u), 0, 0);
  }
}

// Groups per load batch: with a K split inside the workgroup, one per slice (WK); otherwise
// two when four BM-row activation stages fit in 128 KiB of LDS and the register ring of four
// groups fits the occupancy (always for 32-column waves), else one.
constexpr int tile_batch(int bm, int tw, int occ, int wk) {
  return wk > 1 ? wk : (4 * bm * kARowBytes <= 128 * 1024 && (tw == 2 || occ == 1) ? 2 : 1);
}

// OCC = waves per SIMD the register allocation must allow (1, 2 or 3; 8-wave workgroups
// always put two waves on every SIMD, 12-wave ones three).  WK = K slices inside the
// workgroup.
template <int WM, int TW, int NWM, int NWN, int OCC, int WK>
__global__ __launch_bounds__(64 * NWM * NWN * WK, OCC) void tile_kernel(const uint16_t* __restrict__ x,
                                                                   const uint32_t* __restrict__ packed,
                                                                   const uint32_t* __restrict__ qzeros,
                                                                   const uint16_t* __restrict__ scales,
                                                                   uint16_t* y, const uint16_t* res,
                                                                   float* __restrict__ partials,
                                                                   int* __restrict__ counters, int M, int K, int N,
                                                                   int split, int m_blocks, int n_blocks,
                                                                   int up_tiles) {
  constexpr int NWG = NWM * NWN;  // waves of one K slice
  constexpr int NW = NWG * WK;    // waves per workgroup
  constexpr int BM = 16 * WM * NWM;
  constexpr int BN = 16 * TW * NWN;
  constexpr int NI = (BM / 4 + NW - 1) / NW;  // activation-stage instructions per wave
  static_assert(BM % 4 == 0, "activation stages hold whole row quads");
  static_assert(NW >= 2, "a group's scale and zero loads are issued by two waves");
  constexpr int kStage = BM * kARowBytes;
  constexpr int P = tile_batch(BM, TW, OCC, WK);  // groups per load batch
  constexpr int S = 2 * P;                        // LDS stages: two batches
  constexpr int PW = P / WK;                      // groups of a batch each wave computes
  static_assert(PW * WK == P && S <= 8, "load batches hold whole slices, at most 8 stages");
  // One LDS object per stage: the compiler then knows that a direct-to-LDS load into one
  // stage does not alias the reads of another, and does not wait for the loads just issued
  // (the next batch's stages) before reading the current one.
  __shared__ __attribute__((aligned(1024))) uint8_t stage0[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t stage1[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t stage2[S > 2 ? kStage : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t stage3[S > 3 ? kStage : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t stage4[S > 4 ? kStage : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t stage5[S > 5 ? kStage : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t stage6[S > 6 ? kStage : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t stage7[S > 7 ? kStage : 16];
  auto stage = [&](int st) -> uint8_t* {
    return st == 0 ? stage0 : st == 1 ? stage1 : st == 2 ? stage2 : st == 3 ? stage3
         : st == 4 ? stage4 : st == 5 ? stage5 : st == 6 ? stage6 : stage7;
  };
  // Scales and zero words of stage i's group in LDS (kStageSZ), or in the register ring.
  constexpr bool kStageSZ = WK <= 2;
  __shared__ __attribute__((aligned(16))) uint8_t sz_stage[kStageSZ ? S : 1][kStageSZ ? kSzStageBytes : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t spare[NI * NW * 4 == BM ? 16 : 1024];  // uneven stage issue
  __shared__ int is_last;

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int wk = wave / NWG;       // K slice of the wave
  const int wave_in = wave % NWG;  // wave within its slice
  const int wn = wave_in % NWN;    // column slice of the wave
  const int wm = wave_in / NWN;    // row slice of the wave
  const int G = K / kGroup;

  const TileCoord tc = tile_coord(blockIdx.x, m_blocks, n_blocks, split);
  const int sidx = tc.sidx, mbk = tc.mbk, nbk = tc.nbk;
  const int g_begin = (G * sidx) / split;
  const int g_end = (G * (sidx + 1)) / split;
  const int row0 = mbk * BM;
  // Plain: the wave computes output columns [col_w, col_w + 16 TW) = layout tiles t0 + tt.
  // Fused SiLU(gate) * up (up_tiles = N / 32), even TW: output columns [col_w, col_w + 8 TW)
  // of the [M, N / 2] result, from gate tiles t0 + tt and up tiles t0 + up_tiles + tt,
  // tt < TW / 2 -- the two halves of the wave's tiles.  Odd TW pairs waves instead: wave
  // wn < NWN / 2 holds the gate tiles t0 .. t0 + TW - 1 of output columns
  // [col_w, col_w + 16 TW) and wave wn + NWN / 2 the up tiles of the same columns; the
  // epilogue meets them in LDS.
  constexpr bool kCross = TW % 2 == 1;
  static_assert(!kCross || (NWN % 2 == 0 && NWM == 1 && WK == 1), "waves pair up along N in one slice");
  const bool act = up_tiles != 0;
  const bool up_wave = kCross && act && wn >= NWN / 2;
  const int gw = up_wave ? wn - NWN / 2 : wn;
  const int n_out = act ? N / 2 : N;
  const int col_w = !act ? nbk * BN + 16 * TW * wn
                  : kCross ? nbk * (BN / 2) + 16 * TW * gw : nbk * (BN / 2) + 8 * TW * wn;  // first output column
  const int t0 = col_w / kTileCols + (up_wave ? up_tiles : 0);
  const int dt = act && !kCross ? up_tiles - TW / 2 : 0;
  const bool active = col_w < n_out;  // wave-uniform (n_out % 64 == 0): the last n-block may be partly past it
  // The workgroup's two column ranges of BN / 2 (scale and zero staging).
  const int cs0 = act ? nbk * (BN / 2) : nbk * BN;
  const int cs1 = act ? cs0 + up_tiles * kTileCols : cs0 + BN / 2;
  const SzOffsets<TW, BN> szo(act, wn, lane);
  const AOffsets<WM> ao(wm, lane);

  f32x4_t acc[WM][TW];
#pragma unroll
  for (int mt = 0; mt < WM; ++mt)
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) acc[mt][tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Batched pipeline over the workgroup's groups (item i = group g_begin + i).  Items travel
  // in batches of P: batch b (items b .. b + P - 1) lives in LDS stages P h .. P h + P - 1,
  // h = (b / P) % 2; a wave of slice wk computes items b + wk + WK j (j < PW) of the batch,
  // whose weights sit in its register slots PW h + j.  At the start of batch b every wave
  // waits for all of its outstanding loads (direct-to-LDS loads may complete out of order
  // with the register loads issued after them, so only a full wait covers them) and passes
  // one barrier -- after which batch b's data is visible and every wave has finished batch
  // b - P -- then issues batch b + P into the other half and computes batch b.  Each load
  // therefore has a batch of compute to land, and there is one wait and one barrier per
  // batch.
  const NibbleConsts nib = nibble_consts();
  const __amdgpu_buffer_rsrc_t rx = make_buffer(x, static_cast<uint32_t>(M) * K * 2u);
  const BSources bsrc{make_buffer(packed, static_cast<uint32_t>(K) * (N / 2)),
                      make_buffer(scales, static_cast<uint32_t>(G) * N * 2u),
                      make_buffer(qzeros, static_cast<uint32_t>(G) * (N / 8) * 4u)};
  constexpr int kWaitAll = 0x0F70;  // vmcnt(0); expcnt and lgkmcnt not waited for
  const int n_items = g_end - g_begin;
  BGroup<TW> ring[2 * PW];
  // A prefetch past the workgroup's last item reloads that item's group (never consumed);
  // ranges are never empty (split <= K / 128).
  auto group_of = [&](int item) { return g_begin + (item < n_items ? item : n_items - 1); };
  auto issue = [&](int half, int b) {  // batch starting at item b into half `half`
#pragma unroll
    for (int q = 0; q < P; ++q) {
      issue_a_stage<NI, NW, BM>(rx, stage(half * P + q), spare, row0, M, K, group_of(b + q), wave, lane);
      // the group's scale and zero instructions go to waves 2q and 2q + 1 (mod NW)
      if (kStageSZ && (wave == (2 * q) % NW || wave == (2 * q + 1) % NW))
        issue_sz_stage<BN>(bsrc, sz_stage[kStageSZ ? half * P + q : 0], group_of(b + q), N, cs0, cs1,
                           wave == (2 * q) % NW ? 0 : 1, lane);
    }
#pragma unroll
    for (int j = 0; j < PW; ++j) {
      const int item = b + wk + WK * j;
      load_b_group<TW, !kStageSZ>(ring[half * PW + j], bsrc, group_of(item), active, N, t0, dt, lane);
    }
  };
  issue(0, 0);
  for (int b0 = 0; b0 < n_items; b0 += 2 * P) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // two batches per trip, so every stage index is a constant
      const int b = b0 + h * P;
      // Past the last item nothing is waited for or issued: no barrier would separate
      // those loads from other waves still reading the other half, and an out-of-range
      // direct-to-LDS load may still write its zeros there.
      if (b < n_items) {
        __builtin_amdgcn_s_waitcnt(kWaitAll);  // batch b's LDS and register loads have landed
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kStageSZ) {
#pragma unroll
          for (int j = 0; j < PW; ++j)  // the wave's groups of the batch: items b + wk + WK j
            read_group_scales<TW, BN>(ring[h * PW + j].sc, sz_stage[h * P + wk + WK * j], szo);
          __builtin_amdgcn_sched_barrier(0);
        }
        // nothing past the last item (the full wait at the next batch would wait for it)
        if (b + P < n_items) issue(1 - h, b + P);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < P; ++q) {
          // q is a constant, so the stage is a known LDS object; the slice test is uniform
          if (q % WK == wk && b + q < n_items && active)
            mma_group<WM, TW>(acc, stage(h * P + q), ao, ring[h * PW + q / WK], nib, lane);
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // trailing (empty) loads, before the stages are reused
  __syncthreads();

  TileOut out{y, res, partials, counters, M, N, n_out, split, sidx, mbk * n_blocks + nbk, m_blocks * n_blocks,
              row0 + wm * 16 * WM, col_w, act, active};
  finish_tile<WM, TW, NWG, WK, S, kStage>(acc, stage, &is_last, out, wave_in, wk, lane);
}

template <int WM, int TW, int NWM, int NWN, int OCC, int WK>
static hipError_t launch_tile_t(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                                const uint16_t* scales, uint16_t* y, const uint16_t* res, float* partials,
                                int* counters, int M, int K, int N, int split, int up_tiles, hipStream_t stream) {
  constexpr int BM = 16 * WM * NWM;
  constexpr int BN = 16 * TW * NWN;
  const int m_blocks = (M + BM - 1) / BM;
  const int n_blocks = (N + BN - 1) / BN;
  const unsigned grid = static_cast<unsigned>(m_blocks * n_blocks * split);
  tile_kernel<WM, TW, NWM, NWN, OCC, WK><<<grid, 64 * NWM * NWN * WK, 0, stream>>>(
      x, packed, qzeros, scales, y, res, partials, counters, M, K, N, split, m_blocks, n_blocks, up_tiles);
  return hipGetLastError();
}

TileShape tile_shape(int shape) {
  switch (shape) {
    case 2: return TileShape{4, 2, 4, 1};  // 8 waves: 2 along M x 4 along N, 64 columns each
    case 3: return TileShape{2, 1, 8, 1};  // 8 waves along N, 32 columns each
    case 4: return TileShape{2, 1, 2, 4};  // 8 waves: 4 K slices x 2 along N, 32 columns each
    case 5: return TileShape{2, 1, 4, 2};  // 8 waves: 2 K slices x 4 along N, 32 columns each
    case 6: return TileShape{2, 1, 2, 2};  // 4 waves: 2 K slices x 2 along N, 32 columns each
    case 7: return TileShape{2, 1, 1, 4};  // 4 waves: 4 K slices x 32 columns
    case 8: return TileShape{4, 1, 8, 1};  // 8 waves along N, 64 columns each
    case 9: return TileShape{2, 1, 3, 4};   // 12 waves: 4 K slices x 3 along N, 32 columns each
    case 10: return TileShape{2, 1, 6, 2};  // 12 waves: 2 K slices x 6 along N, 32 columns each
    case 11: return TileShape{3, 1, 8, 1};  // 8 waves along N, 48 columns each (plain GEMM only)
    default: return TileShape{4, 1, 4, 1};  // 4 waves along N, 64 columns each
  }
}

// The compiled (wm, tile shape, occupancy) combinations, in one list for the launcher and
// for tile_config_compiled: X(WM, TW, NWM, NWN, OCC, WK).
#define W4A16_TILE_CONFIGS(X)                                                                 \
  X(4, 4, 1, 4, 1, 1) X(4, 4, 1, 4, 2, 1) X(8, 4, 1, 4, 1, 1) X(4, 4, 2, 4, 2, 1) X(4, 2, 1, 8, 2, 1)  \
  X(8, 2, 1, 8, 2, 1)                                                                         \
  X(2, 2, 1, 2, 2, 4) X(4, 2, 1, 2, 2, 4) X(2, 2, 1, 4, 2, 2) X(4, 2, 1, 4, 2, 2) X(8, 2, 1, 4, 2, 2)  \
  X(4, 2, 1, 2, 1, 2) X(8, 2, 1, 2, 1, 2) X(2, 2, 1, 1, 1, 4) X(4, 2, 1, 1, 1, 4) X(8, 4, 1, 8, 2, 1) X(4, 2, 1, 3, 3, 4) X(2, 2, 1, 3, 3, 4) \
  X(4, 2, 1, 6, 3, 2) X(8, 3, 1, 8, 2, 1) X(4, 3, 1, 8, 2, 1) X(6, 2, 1, 8, 2, 1) X(6, 4, 1, 8, 2, 1) X(6, 3, 1, 8, 2, 1)

bool tile_config_compiled(int wm, int shape, int occ) {
  const TileShape ts = tile_shape(shape);
#define W4A16_TILE_MATCH(WM_, TW_, NWM_, NWN_, OCC_, WK_) \
  if (wm == WM_ && ts.tw == TW_ && ts.nwm == NWM_ && ts.nwn == NWN_ && occ == OCC_ && ts.wk == WK_) return true;
  W4A16_TILE_CONFIGS(W4A16_TILE_MATCH)
#undef W4A16_TILE_MATCH
  return false;
}

hipError_t launch_tile_cfg(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                           const uint16_t* scales, uint16_t* y, const uint16_t* res, float* partials, int* counters,
                           int M, int K, int N, int wm, int shape, int occ, int split, int up_tiles,
                           hipStream_t stream) {
  const TileShape ts = tile_shape(shape);
#define W4A16_TILE_LAUNCH(WM_, TW_, NWM_, NWN_, OCC_, WK_)                                                       \
  if (wm == WM_ && ts.tw == TW_ && ts.nwm == NWM_ && ts.nwn == NWN_ && occ == OCC_ && ts.wk == WK_)              \
    return launch_tile_t<WM_, TW_, NWM_, NWN_, OCC_, WK_>(x, packed, qzeros, scales, y, res, partials, counters, M, \
                                                          K, N, split, up_tiles, stream);
  W4A16_TILE_CONFIGS(W4A16_TILE_LAUNCH)
#undef W4A16_TILE_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace w4a16
