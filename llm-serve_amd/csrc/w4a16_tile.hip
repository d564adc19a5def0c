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
// different chunk positions, i.e. all 64 LDS banks once.  The weights, scales and zeros of
// those groups travel in a matching ring of registers.
//
// Grid: one workgroup per (m-block, n-block, k-split), enumerated XCD-major so the
// workgroups resident on one XCD cover a few n-blocks x all m-blocks and share their
// operands in that XCD's L2.  With split > 1 the workgroups write fp32 partials and the
// last to arrive at a tile (atomic counter) sums them in split order; the counter is
// re-armed to zero.
#include <type_traits>

#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {

constexpr int kARowBytes = kGroup * 2;  // one activation row of a stage

typedef __attribute__((address_space(3))) void lds_void_t;

// Issue the direct-to-LDS loads of activation rows [row0, row0 + 4 NI NW) x group g into
// `stage` (NW waves, NI instructions each).  Instruction i of wave w fills rows
// 4 (NW i + w) .. +3 (1 KiB); lane -> (row, physical chunk).  An invalid group (past the
// workgroup's K range) fetches nothing.
template <int NI, int NW>
__device__ __forceinline__ void issue_a_stage(__amdgpu_buffer_rsrc_t rx, uint8_t* stage, int row0, int M, int K,
                                              int g, bool valid, int wave, int lane) {
  const int p = lane & 15;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int r = 4 * (NW * i + wave) + (lane >> 4);
    const int c = p ^ (r & 15);
    int row = row0 + r;
    row = row < M ? row : M - 1;  // rows past M load a valid row; their outputs are dropped
    const uint32_t off =
        valid ? (static_cast<uint32_t>(row) * static_cast<uint32_t>(K) + kGroup * g + 8u * c) * 2u : kOutOfRange;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(stage + 4 * (NW * i + wave) * kARowBytes), 16, off,
                                             0, 0, 0);
  }
}

// Raw loads of one group for a wave's TW layout tiles: one 16-byte weight load per tile,
// and the scale-pair and zero words of the lane's column in each tile.  Decoding waits
// until the group is consumed.  An invalid group (past the K range, or a wave whose columns
// lie past N) fetches nothing.
template <int TW>
struct BGroup {
  u32x4_t w[TW];
  uint32_t s[TW];   // bf16 scale pair holding the lane's column
  uint32_t zw[TW];  // AutoAWQ zero word holding the lane's column
};

struct BSources {
  __amdgpu_buffer_rsrc_t w, s, z;
};

// The wave's tiles are t0 + tt, plus dt for tt >= TW / 2 (dt = 0 for the plain GEMM; for
// the fused gate/up product the second half are the up tiles of the first half's gate tiles).
template <int TW>
__device__ __forceinline__ void load_b_group(BGroup<TW>& b, const BSources& src, int g, bool valid, int N, int t0,
                                             int dt, int lane) {
  const int NT = N / kTileCols;
  const int c = lane & 15;
  const uint32_t oob = valid ? 0u : kOutOfRange;
#pragma unroll
  for (int tt = 0; tt < TW; ++tt) {
    const int t = t0 + tt + (tt >= TW / 2 ? dt : 0);
    const uint32_t wo = valid ? static_cast<uint32_t>(tile_word(g, t, NT, lane)) * 4u : kOutOfRange;
    b.w[tt] = __builtin_amdgcn_raw_buffer_load_b128(src.w, wo, 0, 0);
    const int col = kTileCols * t + c;
    b.s[tt] = __builtin_amdgcn_raw_buffer_load_b32(src.s, oob | (static_cast<uint32_t>(g * N + (col & ~1)) * 2u), 0, 0);
    b.zw[tt] = __builtin_amdgcn_raw_buffer_load_b32(src.z, oob | (static_cast<uint32_t>(g * (N >> 3) + (col >> 3)) * 4u),
                                                    0, 0);
  }
}

// One 128-deep group: per 32-row step, the matrix-core dequant of the wave's TW weight
// tiles (2 TW scaling MFMAs), then WM x TW main MFMAs against the wave's 16 WM rows of the
// LDS activation tile (`stage` points at the first of them).  Software-pipelined: step
// j + 1's fragments are read and its weights dequantized while step j's main MFMAs run, so
// the VALU dequant of one step can hide under the matrix work of the previous one.  The
// order within a step is left to the compiler: explicit scheduling groups (one main MFMA,
// then two VALU and one LDS read) measured 1.3-2.5 % slower on MI355X at M = 512 and 2048.
template <int WM, int TW>
__device__ __forceinline__ void mma_group(f32x4_t (&acc)[WM][TW], const uint8_t* stage, const BGroup<TW>& b,
                                          const NibbleConsts& nib, int lane) {
  const int arow = lane & 15;
  const int zshift = awq_shift(lane & 7);
  TileScale ts[TW];
#pragma unroll
  for (int tt = 0; tt < TW; ++tt) ts[tt] = make_tile_scale(b.s[tt], (b.zw[tt] >> zshift) & 0xFu, lane);
  auto read_a = [&](bf16x8_t (&a)[WM], int j) {
    const int pchunk = (4 * j + (lane >> 4)) ^ (lane & 15);  // row & 15 == lane & 15
    const uint8_t* base = stage + arow * kARowBytes + pchunk * 16;
#pragma unroll
    for (int mt = 0; mt < WM; ++mt) a[mt] = *reinterpret_cast<const bf16x8_t*>(base + mt * 16 * kARowBytes);
  };
  auto dequant = [&](bf16x8_t (&bf)[TW], int j) {
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) bf[tt] = dequant_step(b.w[tt][j], ts[tt], nib);
  };
  if constexpr (WM * TW > 16) {
    // Large wave tiles: no register double-buffering (the accumulators fill the AGPRs);
    // the WM x TW independent MFMAs of a step leave the scheduler enough work to overlap.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bf16x8_t a[WM];
      bf16x8_t bf[TW];
      read_a(a, j);
      dequant(bf, j);
#pragma unroll
      for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) acc[mt][tt] = mfma16(a[mt], bf[tt], acc[mt][tt]);
    }
    return;
  }
  bf16x8_t a[2][WM];
  bf16x8_t bf[2][TW];
  read_a(a[0], 0);
  dequant(bf[0], 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = j & 1;
    if (j < 3) {
      read_a(a[c ^ 1], j + 1);
      dequant(bf[c ^ 1], j + 1);
    }
    // 128-row waves raise their issue priority while they issue the step's main MFMAs, so
    // that the SIMD's other wave (in its dequant or LDS reads) does not starve the matrix
    // pipe: measured on MI355X 2-3 % faster at M = 2048 (gate_up, down, O), while the
    // 64-row configurations ran 3-4 % slower with it.
    if constexpr (WM >= 8) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
      for (int tt = 0; tt < TW; ++tt) acc[mt][tt] = mfma16(a[c][mt], bf[c][tt], acc[mt][tt]);
    if constexpr (WM >= 8) __builtin_amdgcn_s_setprio(0);
  }
}

// Groups per load batch: two when four BM-row activation stages fit in 128 KiB of LDS and
// the register ring of four groups fits the occupancy (always for 32-column waves), else one.
constexpr int tile_batch(int bm, int tw, int occ) {
  return 4 * bm * kARowBytes <= 128 * 1024 && (tw == 2 || occ == 1) ? 2 : 1;
}

// OCC = waves per SIMD the register allocation must allow (1 or 2; 8-wave workgroups
// always put two waves on every SIMD).
template <int WM, int TW, int NWM, int NWN, int OCC>
__global__ __launch_bounds__(64 * NWM * NWN, OCC) void tile_kernel(const uint16_t* __restrict__ x,
                                                                   const uint32_t* __restrict__ packed,
                                                                   const uint32_t* __restrict__ qzeros,
                                                                   const uint16_t* __restrict__ scales,
                                                                   uint16_t* y, const uint16_t* res,
                                                                   float* __restrict__ partials,
                                                                   int* __restrict__ counters, int M, int K, int N,
                                                                   int split, int m_blocks, int n_blocks,
                                                                   int up_tiles) {
  constexpr int NW = NWM * NWN;  // waves per workgroup
  constexpr int BM = 16 * WM * NWM;
  constexpr int BN = 16 * TW * NWN;
  constexpr int NI = BM / (4 * NW);  // activation-stage instructions per wave
  static_assert(NI * 4 * NW == BM, "the activation stage must split evenly over the waves");
  constexpr int kStage = BM * kARowBytes;
  constexpr int P = tile_batch(BM, TW, OCC);  // groups per load batch
  constexpr int S = 2 * P;                    // LDS stages and register slots: two batches
  // One LDS object per stage: the compiler then knows that a direct-to-LDS load into one
  // stage does not alias the reads of another, and does not wait for the loads just issued
  // (the next batch's stages) before reading the current one.
  __shared__ __attribute__((aligned(1024))) uint8_t stage0[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t stage1[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t stage2[S > 2 ? kStage : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t stage3[S > 3 ? kStage : 16];
  auto stage = [&](int st) -> uint8_t* { return st == 0 ? stage0 : st == 1 ? stage1 : st == 2 ? stage2 : stage3; };
  __shared__ int is_last;

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int wn = wave % NWN;  // column slice of the wave
  const int wm = wave / NWN;  // row slice of the wave
  const int G = K / kGroup;

  // XCD-major enumeration: consecutive blockIdx go to different XCDs (round-robin), so
  // undo that and give each XCD a contiguous run of logical tiles.  Within a K split the
  // logical tiles run in groups of kGroupM m-blocks: m fastest inside a group, then n, so an
  // XCD works on few m-blocks across many n-blocks at a time -- their activation rows stay
  // in its L2 while the weights stream past (instead of every n-block re-fetching all rows).
  constexpr int kGroupM = 4;
  const int total = m_blocks * n_blocks * split;
  const int b = blockIdx.x;
  const int per = total >> 3, rem = total & 7, xcd = b & 7, idx = b >> 3;
  const int L = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int tiles = m_blocks * n_blocks;
  const int sidx = L / tiles;
  const int Lt = L - sidx * tiles;
  const int grp = Lt / (kGroupM * n_blocks);
  const int in_grp = Lt - grp * (kGroupM * n_blocks);
  const int gm = m_blocks - grp * kGroupM < kGroupM ? m_blocks - grp * kGroupM : kGroupM;
  const int mbk = grp * kGroupM + in_grp % gm;
  const int nbk = in_grp / gm;
  const int g_begin = (G * sidx) / split;
  const int g_end = (G * (sidx + 1)) / split;
  const int row0 = mbk * BM;
  // Plain: the wave computes output columns [col_w, col_w + 16 TW) = layout tiles t0 + tt.
  // Fused SiLU(gate) * up (up_tiles = N / 32): output columns [col_w, col_w + 8 TW) of the
  // [M, N / 2] result, from gate tiles t0 + tt and up tiles t0 + up_tiles + tt, tt < TW / 2.
  static_assert(TW % 2 == 0, "the fused product pairs the two halves of a wave's tiles");
  const bool act = up_tiles != 0;
  const int n_out = act ? N / 2 : N;
  const int col_w = act ? nbk * (BN / 2) + 8 * TW * wn : nbk * BN + 16 * TW * wn;  // first output column
  const int t0 = col_w / kTileCols;
  const int dt = act ? up_tiles - TW / 2 : 0;
  const bool active = col_w < n_out;  // wave-uniform (n_out % 64 == 0): the last n-block may be partly past it

  f32x4_t acc[WM][TW];
#pragma unroll
  for (int mt = 0; mt < WM; ++mt)
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) acc[mt][tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Batched pipeline over the workgroup's groups (item i = group g_begin + i).  Items travel
  // in batches of P: batch b (items b .. b + P - 1) lives in LDS stages and register slots
  // P h .. P h + P - 1, h = (b / P) % 2.  At the start of batch b every wave waits for all of
  // its outstanding loads (direct-to-LDS loads may complete out of order with the register
  // loads issued after them, so only a full wait covers them) and passes one barrier --
  // after which batch b's data is visible and every wave has finished batch b - P -- then
  // issues batch b + P into the other half and computes batch b.  Each load therefore has P
  // groups of compute to land, and there is one wait and one barrier per P groups.
  const NibbleConsts nib = nibble_consts();
  const __amdgpu_buffer_rsrc_t rx = make_buffer(x, static_cast<uint32_t>(M) * K * 2u);
  const BSources bsrc{make_buffer(packed, static_cast<uint32_t>(K) * (N / 2)),
                      make_buffer(scales, static_cast<uint32_t>(G) * N * 2u),
                      make_buffer(qzeros, static_cast<uint32_t>(G) * (N / 8) * 4u)};
  constexpr int kWaitAll = 0x0F70;  // vmcnt(0); expcnt and lgkmcnt not waited for
  const int n_items = g_end - g_begin;
  BGroup<TW> ring[S];
  auto issue = [&](int slot, int item) {
    const bool valid = item < n_items;
    issue_a_stage<NI, NW>(rx, stage(slot), row0, M, K, g_begin + item, valid, wave, lane);
    load_b_group<TW>(ring[slot], bsrc, g_begin + item, valid && active, N, t0, dt, lane);
  };
#pragma unroll
  for (int q = 0; q < P; ++q) issue(q, q);
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
#pragma unroll
        for (int q = 0; q < P; ++q) issue((1 - h) * P + q, b + P + q);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < P; ++q)
          if (b + q < n_items && active)
            mma_group<WM, TW>(acc, stage(h * P + q) + wm * 16 * WM * kARowBytes, ring[h * P + q], nib, lane);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // trailing (empty) loads, before the stages are reused
  __syncthreads();

  if (split > 1) {
    // Every workgroup stores its fp32 fragments (lane-major, 1 KiB per 16 x 16 MFMA tile)
    // into partials[sidx][tile][wave]; the last to arrive sums all splits in split order,
    // KC fragments at a time so that the loads of a chunk share one wait.
    const int ntiles = m_blocks * n_blocks;
    const int tile = mbk * n_blocks + nbk;
    constexpr int kFrags = WM * TW;
    constexpr int KC = kFrags % 8 == 0 ? 8 : 4;
    static_assert(kFrags % KC == 0, "fragments must split into chunks");
    const __amdgpu_buffer_rsrc_t rp =
        make_buffer(partials, static_cast<uint32_t>(split) * ntiles * NW * kFrags * 1024u);
    const uint32_t lane_off = static_cast<uint32_t>(lane) * 16u;
    auto frag_off = [&](int sp, int f) {
      return (((static_cast<uint32_t>(sp) * ntiles + tile) * NW + wave) * kFrags + f) * 1024u + lane_off;
    };
#pragma unroll
    for (int f = 0; f < kFrags; ++f) store_fragment(rp, frag_off(sidx, f), acc[f / TW][f % TW]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) is_last = (arrive(&counters[tile]) == split - 1);
    __syncthreads();
    if (!is_last) return;
#pragma unroll
    for (int c = 0; c < kFrags; c += KC) {
      f32x4_t tot[KC];
#pragma unroll
      for (int f = 0; f < KC; ++f) tot[f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      for (int sp = 0; sp < split; ++sp) {
        if (sp == sidx) {
#pragma unroll
          for (int f = 0; f < KC; ++f) tot[f] += acc[(c + f) / TW][(c + f) % TW];
        } else {
          f32x4_t part[KC];
#pragma unroll
          for (int f = 0; f < KC; ++f) part[f] = load_fragment(rp, frag_off(sp, c + f));
#pragma unroll
          for (int f = 0; f < KC; ++f) tot[f] += part[f];
        }
      }
#pragma unroll
      for (int f = 0; f < KC; ++f) acc[(c + f) / TW][(c + f) % TW] = tot[f];
    }
    if (threadIdx.x == 0) rearm(&counters[tile]);
  }

  if (!active) return;
  // Epilogue: bf16 through LDS (row-major 16 WM rows x the wave's output columns: rows of
  // CPR 16-byte chunks swizzled by row), then 16-byte coalesced stores.  The stages are free
  // after the last barrier.
  constexpr int WR = 16 * WM;  // rows of a wave
  constexpr int kStageRows = kStage / (WR * 32 * TW);
  static_assert(kStageRows >= 1 && kStageRows * S >= NW, "epilogue staging exceeds the stages");
  uint8_t* ep = stage(wave / kStageRows) + (wave % kStageRows) * (WR * 32 * TW);
  auto store_rows = [&](auto cpr_tag) {
    constexpr int CPR = decltype(cpr_tag)::value;
    constexpr int PITCH = 16 * CPR;
    constexpr int kRowsPerRound = 64 / CPR;
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
#pragma unroll 4
    for (int round = 0; round < WR / kRowsPerRound; ++round) {
      const int r = kRowsPerRound * round + lane / CPR;
      const int q = lane % CPR;
      const uint4 v = *reinterpret_cast<const uint4*>(ep + r * PITCH + ((q ^ (r % CPR)) << 4));
      const int row = row0 + wm * WR + r;
      if (row < M) {
        const size_t off = static_cast<size_t>(row) * n_out + col_w + 8 * q;
        *reinterpret_cast<uint4*>(y + off) = res ? add_bf16x8(v, *reinterpret_cast<const uint4*>(res + off)) : v;
      }
    }
  };
  if (!act) {
    constexpr int CPR = 2 * TW;  // 16-byte chunks per row
    constexpr int PITCH = 16 * CPR;
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
      for (int tt = 0; tt < TW; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * mt + 4 * (lane >> 4) + i;
          const int c = 16 * tt + (lane & 15);
          const int off = r * PITCH + (((c >> 3) ^ (r % CPR)) << 4) + ((c & 7) << 1);
          *reinterpret_cast<uint16_t*>(ep + off) = f32_to_bf16_bits(acc[mt][tt][i]);
        }
    store_rows(std::integral_constant<int, CPR>{});
  } else {
    constexpr int H = TW / 2;
    constexpr int CPR = TW;  // half the columns
    constexpr int PITCH = 16 * CPR;
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
      for (int tt = 0; tt < H; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * mt + 4 * (lane >> 4) + i;
          const int c = 16 * tt + (lane & 15);
          const int off = r * PITCH + (((c >> 3) ^ (r % CPR)) << 4) + ((c & 7) << 1);
          *reinterpret_cast<uint16_t*>(ep + off) = f32_to_bf16_bits(silu_mul(acc[mt][tt][i], acc[mt][tt + H][i]));
        }
    store_rows(std::integral_constant<int, CPR>{});
  }
}

template <int WM, int TW, int NWM, int NWN, int OCC>
static hipError_t launch_tile_t(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                                const uint16_t* scales, uint16_t* y, const uint16_t* res, float* partials,
                                int* counters, int M, int K, int N, int split, int up_tiles, hipStream_t stream) {
  constexpr int BM = 16 * WM * NWM;
  constexpr int BN = 16 * TW * NWN;
  const int m_blocks = (M + BM - 1) / BM;
  const int n_blocks = (N + BN - 1) / BN;
  const unsigned grid = static_cast<unsigned>(m_blocks * n_blocks * split);
  tile_kernel<WM, TW, NWM, NWN, OCC><<<grid, 64 * NWM * NWN, 0, stream>>>(
      x, packed, qzeros, scales, y, res, partials, counters, M, K, N, split, m_blocks, n_blocks, up_tiles);
  return hipGetLastError();
}

TileShape tile_shape(int shape) {
  switch (shape) {
    case 2: return TileShape{4, 2, 4};  // 8 waves: 2 along M x 4 along N, 64 columns each
    case 3: return TileShape{2, 1, 8};  // 8 waves along N, 32 columns each
    default: return TileShape{4, 1, 4};  // 4 waves along N, 64 columns each
  }
}

// The compiled (wm, tile shape, occupancy) combinations, in one list for the launcher and
// for tile_config_compiled.
#define W4A16_TILE_CONFIGS(X)                                                                 \
  X(4, 4, 1, 4, 1) X(4, 4, 1, 4, 2) X(8, 4, 1, 4, 1) X(4, 4, 2, 4, 2) X(4, 2, 1, 8, 2) X(8, 2, 1, 8, 2)

bool tile_config_compiled(int wm, int shape, int occ) {
  const TileShape ts = tile_shape(shape);
#define W4A16_TILE_MATCH(WM_, TW_, NWM_, NWN_, OCC_) \
  if (wm == WM_ && ts.tw == TW_ && ts.nwm == NWM_ && ts.nwn == NWN_ && occ == OCC_) return true;
  W4A16_TILE_CONFIGS(W4A16_TILE_MATCH)
#undef W4A16_TILE_MATCH
  return false;
}

hipError_t launch_tile_cfg(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                           const uint16_t* scales, uint16_t* y, const uint16_t* res, float* partials, int* counters,
                           int M, int K, int N, int wm, int shape, int occ, int split, int up_tiles,
                           hipStream_t stream) {
  const TileShape ts = tile_shape(shape);
#define W4A16_TILE_LAUNCH(WM_, TW_, NWM_, NWN_, OCC_)                                                           \
  if (wm == WM_ && ts.tw == TW_ && ts.nwm == NWM_ && ts.nwn == NWN_ && occ == OCC_)                            \
    return launch_tile_t<WM_, TW_, NWM_, NWN_, OCC_>(x, packed, qzeros, scales, y, res, partials, counters, M, K, N, \
                                                     split, up_tiles, stream);
  W4A16_TILE_CONFIGS(W4A16_TILE_LAUNCH)
#undef W4A16_TILE_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace w4a16
