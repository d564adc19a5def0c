// Pieces of the LDS-staged GEMM kernel (tile_kernel): the raw loads of one 128-deep group of
// a wave's weight tiles, the MFMA work of one group against an activation stage in LDS, the
// workgroup-to-tile mapping and the output side (slice sum, split-K exchange, epilogue).
//
// Activation stage layout: BM rows x one 128-deep group, row-major (256 bytes per row), the
// sixteen 16-byte chunks of row r stored at chunk position c ^ (r & 15): the 16 lanes reading
// one fragment chunk (16 consecutive rows) then hit 16 different chunk positions, i.e. all
// 64 LDS banks once.
#pragma once

#include <type_traits>
#include <utility>

#include "w4a16_common.h"

namespace w4a16 {

constexpr int kARowBytes = kGroup * 2;  // one activation row of a stage

// Workgroup -> (K split, m-block, n-block).  XCD-major enumeration: consecutive blockIdx go
// to different XCDs (round-robin), so undo that and give each XCD a contiguous run of
// logical tiles.  Within a K split the logical tiles run in groups of kGroupM m-blocks: m
// fastest inside a group, then n, so an XCD works on few m-blocks across many n-blocks at a
// time -- their activation rows stay in its L2 while the weights stream past (instead of
// every n-block re-fetching all rows).
struct TileCoord {
  int sidx, mbk, nbk;
};

__device__ __forceinline__ TileCoord tile_coord(int b, int m_blocks, int n_blocks, int split) {
  constexpr int kGroupM = 4;
  const int total = m_blocks * n_blocks * split;
  const int per = total >> 3, rem = total & 7, xcd = b & 7, idx = b >> 3;
  const int L = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int tiles = m_blocks * n_blocks;
  const int sidx = L / tiles;
  const int Lt = L - sidx * tiles;
  const int grp = Lt / (kGroupM * n_blocks);
  const int in_grp = Lt - grp * (kGroupM * n_blocks);
  const int gm = m_blocks - grp * kGroupM < kGroupM ? m_blocks - grp * kGroupM : kGroupM;
  return TileCoord{sidx, grp * kGroupM + in_grp % gm, in_grp / gm};
}

// The scale pair word and the AutoAWQ zero word holding the lane's column, per tile of a
// wave, for one group.
template <int TW>
struct GroupScales {
  uint32_t s[TW], zw[TW];
};

// Raw loads of one group for a wave's TW layout tiles: one 16-byte weight load per tile,
// and (LOAD_SC) the scale-pair and zero words of the lane's column in each tile -- else those
// come from the workgroup's LDS stage (issue_sz_stage, read_group_scales).  Decoding waits
// until the group is consumed.  A wave whose columns lie past N fetches nothing.
template <int TW>
struct BGroup {
  u32x4_t w[TW];
  GroupScales<TW> sc;
};

struct BSources {
  __amdgpu_buffer_rsrc_t w, s, z;
};

// The wave's tiles are t0 + tt, plus dt for tt >= TW / 2 (dt = 0 for the plain GEMM; for
// the fused gate/up product the second half are the up tiles of the first half's gate tiles).
// g is a group of the weights (callers clamp a prefetch past their range to its last group);
// an inactive wave (columns past N) fetches nothing.  The group's part of each offset is the
// instruction's scalar offset and the lane's part is the same for every group, so the loop
// spends no vector instructions on addresses; every lane offset plus its group offset stays
// inside its buffer (the wave's tiles lie below N / 16).
template <int TW, bool LOAD_SC>
__device__ __forceinline__ void load_b_group(BGroup<TW>& b, const BSources& src, int g, bool active, int N, int t0,
                                             int dt, int lane) {
  const int NT = N / kTileCols;
  const int c = lane & 15;
  const uint32_t oob = active ? 0u : kOutOfRange;
#pragma unroll
  for (int tt = 0; tt < TW; ++tt) {
    const int t = t0 + tt + (tt >= TW / 2 ? dt : 0);
    const uint32_t wo = oob | (static_cast<uint32_t>(t * 64 + lane) * 16u);
    b.w[tt] = __builtin_amdgcn_raw_buffer_load_b128(src.w, wo, static_cast<int>(static_cast<uint32_t>(g) * NT * 1024u),
                                                     0);
    if constexpr (LOAD_SC) {
      const int col = kTileCols * t + c;
      b.sc.s[tt] = __builtin_amdgcn_raw_buffer_load_b32(src.s, oob | (static_cast<uint32_t>(col & ~1) * 2u),
                                                        static_cast<int>(static_cast<uint32_t>(g) * N * 2u), 0);
      b.sc.zw[tt] = __builtin_amdgcn_raw_buffer_load_b32(src.z, oob | (static_cast<uint32_t>(col >> 3) * 4u),
                                                         static_cast<int>(static_cast<uint32_t>(g) * (N >> 3) * 4u), 0);
    }
  }
}

// Scale and zero staging of a tile workgroup.  Per group, the workgroup's BN columns are two
// ranges of BN / 2 columns starting at cs0 and cs1: the gate and up halves of the fused
// product, or the two halves of a plain column block.  Their bf16 scales (BN / 8 chunks of
// 16 bytes, range 0 first) go to bytes [0, 2 BN) of the group's LDS stage and their zero
// words (kSzZeroChunks 16-byte chunks of 32 columns per range) to bytes [1024, 2048), each
// by one direct-to-LDS load instruction per group for the whole workgroup -- in place of
// two 4-byte loads per tile and wave, which cost the prefill kernel 16 % of its time.  (With
// four K slices, each stage serves only two waves, and the per-wave loads measured faster.)
constexpr int kSzStageBytes = 2048;
constexpr int kSzZeroBase = 1024;
template <int BN>
constexpr int sz_zero_chunks() { return (BN + 63) / 64; }

// Instruction `which` (0: scales, 1: zero words) of group g's stage, on the lanes that have
// a chunk.  g is a group of the weights (callers clamp a prefetch past their K range to its
// last group): its part of the offset is the instruction's scalar offset, the lane's part
// (the column) the same for every group.
template <int BN>
__device__ __forceinline__ void issue_sz_stage(const BSources& src, uint8_t* sz, int g, int N, int cs0, int cs1,
                                               int which, int lane) {
  typedef __attribute__((address_space(3))) void lds_void_t;
  static_assert(BN % 32 == 0 && BN / 8 <= 64, "one instruction holds the scales of the column block");
  if (which == 0) {
    constexpr int kHalf = BN / 16;  // 16-byte chunks of one range
    const int r = lane >= kHalf;
    const int col = (r ? cs1 : cs0) + 8 * (lane - r * kHalf);
    if (lane < 2 * kHalf)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src.s, (lds_void_t*)sz, 16, static_cast<uint32_t>(col) * 2u,
                                               static_cast<int>(static_cast<uint32_t>(g) * N * 2u), 0, 0);
  } else {
    constexpr int kZc = sz_zero_chunks<BN>();
    const int r = lane >= kZc;
    const int col = (r ? cs1 : cs0) + 32 * (lane - r * kZc);
    if (lane < 2 * kZc)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(src.z, (lds_void_t*)(sz + kSzZeroBase), 16,
                                               static_cast<uint32_t>(col >> 3) * 4u,
                                               static_cast<int>(static_cast<uint32_t>(g) * (N >> 3) * 4u), 0, 0);
  }
}

// LDS byte offsets, within a group's scale/zero stage, of the scale pair word and the zero
// word holding the lane's column of each of the wave's tiles.  Plain: the wave's columns are
// [16 TW wn, 16 TW (wn + 1)) of the block; fused, even TW: gate columns [8 TW wn, 8 TW (wn + 1))
// of range 0 and the same up columns of range 1; fused, odd TW: columns [16 TW v, 16 TW (v + 1))
// of range 0 for the first half of the waves (v = wn) and of range 1 for the second.
template <int TW, int BN>
struct SzOffsets {
  uint32_t s[TW], z[TW];
  __device__ __forceinline__ SzOffsets(bool act, int wn, int lane) {
    const int c = lane & 15;
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) {
      int r, u;
      if (act && TW % 2 == 1) {  // waves pair up: wn < NWN / 2 gate, the others up
        constexpr int kHalfWaves = BN / (32 * TW);
        r = wn >= kHalfWaves;
        u = 16 * TW * (wn - r * kHalfWaves) + 16 * tt;
      } else if (act) {
        r = tt >= TW / 2;
        u = 8 * TW * wn + 16 * (tt - r * (TW / 2));
      } else {
        const int p = 16 * TW * wn + 16 * tt;
        r = p >= BN / 2;
        u = p - r * (BN / 2);
      }
      s[tt] = static_cast<uint32_t>(BN * r + 2 * u + 2 * (c & ~1));
      z[tt] = static_cast<uint32_t>(kSzZeroBase + 16 * sz_zero_chunks<BN>() * r + 4 * (u >> 3) + 4 * (c >> 3));
    }
  }
};

// The scale pair and zero words of the lane's columns in one group's stage.  Read right
// after the batch barrier, ahead of the next batch's load issue, so that their latency is
// not on the path into the group's first dequant.
template <int TW, int BN>
__device__ __forceinline__ void read_group_scales(GroupScales<TW>& gs, const uint8_t* sz, const SzOffsets<TW, BN>& szo) {
#pragma unroll
  for (int tt = 0; tt < TW; ++tt) {
    gs.s[tt] = *reinterpret_cast<const uint32_t*>(sz + szo.s[tt]);
    gs.zw[tt] = *reinterpret_cast<const uint32_t*>(sz + szo.z[tt]);
  }
}

// Lane byte offsets, within an activation stage, of the wave's first fragment of each of a
// group's four 32-deep steps: row 16 WM wm + (lane & 15), the step's physical chunk.  The
// stage's own address is then a constant, which the LDS reads carry in their offset field.
template <int WM>
struct AOffsets {
  uint32_t o[4];
  __device__ __forceinline__ AOffsets(int wm, int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pchunk = (4 * j + (lane >> 4)) ^ (lane & 15);  // row & 15 == lane & 15
      o[j] = static_cast<uint32_t>((16 * WM * wm + (lane & 15)) * kARowBytes + pchunk * 16);
    }
  }
};

// One 128-deep group: per 32-row step, the matrix-core dequant of the wave's TW weight
// tiles (2 TW scaling MFMAs), then WM x TW main MFMAs against the wave's 16 WM rows of the
// LDS activation tile (`stage` is the activation stage, `ao` the lane's offsets of the
// wave's rows in it).  Software-pipelined: step j + 1's fragments are read and its weights
// dequantized while step j's main MFMAs run, so the VALU dequant of one step can hide under
// the matrix work of the previous one.  The
// order within a step is left to the compiler (except the split of the dequant for wave
// tiles of 96 and 128 rows, below): explicit scheduling groups (one main MFMA, then two VALU
// and one LDS read) measured 1.3-2.5 % slower on MI355X at M = 512 and 2048, and with 32-
// and 64-row wave tiles (the LDS reads, then one MFMA and one to three VALU at a time)
// 1-7 % slower at M = 48 - 256.
template <int WM, int TW>
__device__ __forceinline__ void mma_group(f32x4_t (&acc)[WM][TW], const uint8_t* stage, const AOffsets<WM>& ao,
                                          const BGroup<TW>& b, const NibbleConsts& nib, int lane) {
  const int zshift = awq_shift(lane & 7);
  TileScale ts[TW];
#pragma unroll
  for (int tt = 0; tt < TW; ++tt) ts[tt] = make_tile_scale(b.sc.s[tt], (b.sc.zw[tt] >> zshift) & 0xFu, lane);
  auto read_a = [&](bf16x8_t (&a)[WM], int j) {
    const uint8_t* base = stage + ao.o[j];
#pragma unroll
    for (int mt = 0; mt < WM; ++mt) a[mt] = *reinterpret_cast<const bf16x8_t*>(base + mt * 16 * kARowBytes);
  };
  // A step's dequant issues every tile's scaling MFMAs before the first rounding reads one
  // (tile by tile, each rounding waits on the MFMA just issued: 0.3-2.3 % slower at M >= 128).
  auto dequant = [&](bf16x8_t (&bf)[TW], int j) {
    ScaledStep sd[TW];
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) sd[tt] = dequant_scale(b.w[tt][j], ts[tt], nib);
#pragma unroll
    for (int tt = 0; tt < TW; ++tt) bf[tt] = dequant_pack(sd[tt]);
  };
  if constexpr (WM * TW > 16) {
    // Large wave tiles: no register double-buffering (the 128 x 64 tile's accumulators
    // take half of the 256 registers a wave has at two waves per SIMD, and the kernel uses
    // 250 of them); the WM x TW independent MFMAs of a step leave the scheduler enough
    // work to overlap.
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
    if constexpr (WM >= 6) {
      // Step j + 1's unpack, scaling MFMAs and fragment reads, free to interleave with step
      // j's main MFMAs; step j + 1's rounding to bf16 only after them, when its inputs are
      // ready, so that it does not hold back the main MFMAs queued behind it.  Measured on
      // MI355X 1-3.7 % faster with 96- and 128-row wave tiles (M = 256 - 2048), and 1-3 %
      // slower with 32- and 64-row ones, which keep the compiler's order.  (Raising the
      // wave's issue priority over the main MFMAs, which helped the unphased order at
      // M = 2048, no longer does.)
      ScaledStep sd[TW];
      if (j < 3) {
        read_a(a[c ^ 1], j + 1);
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) sd[tt] = dequant_scale(b.w[tt][j + 1], ts[tt], nib);
      }
#pragma unroll
      for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) acc[mt][tt] = mfma16(a[c][mt], bf[c][tt], acc[mt][tt]);
      __builtin_amdgcn_sched_barrier(0);
      if (j < 3) {
#pragma unroll
        for (int tt = 0; tt < TW; ++tt) bf[c ^ 1][tt] = dequant_pack(sd[tt]);
      }
      continue;
    }
    if (j < 3) {
      read_a(a[c ^ 1], j + 1);
      dequant(bf[c ^ 1], j + 1);
    }
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
      for (int tt = 0; tt < TW; ++tt) acc[mt][tt] = mfma16(a[c][mt], bf[c][tt], acc[mt][tt]);
  }
}

// The output side of a tile workgroup.
struct TileOut {
  uint16_t* y;
  const uint16_t* res;  // residual added in the epilogue (may be y), or null
  float* partials;      // split-K fp32 fragments
  int* counters;        // split-K arrival counters, one per output tile
  int M, N, n_out, split, sidx, tile, ntiles;
  int row_w;            // first output row of the wave
  int col_w;            // first output column of the wave
  bool act;             // fused SiLU(gate) * up: y is [M, N / 2]
  bool active;          // the wave has output columns (col_w < n_out)
};

// f(std::integral_constant<int, i>{}) for i = 0 .. N - 1, unrolled at compile time.
template <int N, class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

// The fused SiLU(gate) * up epilogue of wave layouts with an odd tile count (TW = 3): wave
// v < NWG / 2 holds the gate values and wave v + NWG / 2 the up values of output columns
// [col_w, col_w + 16 TW).  In row passes every wave rounds its values to bf16 into its own LDS
// region (rows of 2 TW 16-byte chunks, chunk q of row r at (q + r) % (2 TW)); after a barrier
// each gate wave reads both operands of a chunk, forms SiLU(g) * u in fp32 (g and u being the
// bf16 layer outputs, as in the reference's two steps) and stores the rounded chunk.  Every
// wave of the workgroup passes the barriers, those without columns too.
template <int WM, int TW, int NWG, int S, int kStage, class StageFn>
__device__ __forceinline__ void cross_silu_epilogue(const f32x4_t (&acc)[WM][TW], StageFn stage, const TileOut& o,
                                                    int wave_in, int lane) {
  constexpr int WR = 16 * WM;
  constexpr int CPR = 2 * TW;  // 16-byte chunks per row
  constexpr int PITCH = 16 * CPR;
  // the fewest row passes (dividing WM) whose NWG regions fit the stages
  constexpr int kP = [] {
    for (int p = 1; p <= WM; ++p)
      if (WM % p == 0 && (kStage / ((WR / p) * PITCH)) * S >= NWG) return p;
    return 0;
  }();
  static_assert(kP > 0, "the paired epilogue's regions exceed the stages");
  constexpr int MP = WM / kP;  // 16-row tiles per pass
  constexpr int RP = 16 * MP;  // rows per pass
  constexpr int kRegion = RP * PITCH;
  constexpr int kPerStage = kStage / kRegion;
  constexpr int kHalf = NWG / 2;
  constexpr int kRowsPerRound = 64 / CPR;
  // wave v's region, the stage chosen among compile-time addresses
  auto region = [&](int v) -> uint8_t* {
    uint8_t* r = stage(0) + (v % kPerStage) * kRegion;
    static_for<(NWG + kPerStage - 1) / kPerStage>([&](auto i_tag) {
      constexpr int i = decltype(i_tag)::value;
      if (i > 0 && v / kPerStage == i) r = stage(i) + (v % kPerStage) * kRegion;
    });
    return r;
  };
  const bool gate = wave_in < kHalf;
  uint8_t* own = region(wave_in);
  uint8_t* partner = region(gate ? wave_in + kHalf : wave_in);
#pragma unroll
  for (int part = 0; part < kP; ++part) {
    if (o.active) {
#pragma unroll
      for (int ml = 0; ml < MP; ++ml)
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 16 * ml + 4 * (lane >> 4) + i;
            const int c = 16 * t + (lane & 15);
            const int off = r * PITCH + ((((c >> 3) + r) % CPR) << 4) + ((c & 7) << 1);
            *reinterpret_cast<uint16_t*>(own + off) = f32_to_bf16_bits(acc[part * MP + ml][t][i]);
          }
    }
    __syncthreads();
    if (gate && o.active) {
#pragma unroll 4
      for (int round = 0; round < (RP + kRowsPerRound - 1) / kRowsPerRound; ++round) {
        const int r = kRowsPerRound * round + lane / CPR;
        const int q = lane % CPR;
        const int row = o.row_w + RP * part + r;
        if (lane < kRowsPerRound * CPR && r < RP && row < o.M) {
          const int pos = r * PITCH + (((q + r) % CPR) << 4);
          float g[8], u[8];
          unpack_bf16x8(*reinterpret_cast<const uint4*>(own + pos), g);
          unpack_bf16x8(*reinterpret_cast<const uint4*>(partner + pos), u);
#pragma unroll
          for (int k = 0; k < 8; ++k) g[k] = silu_mul(g[k], u[k]);
          *reinterpret_cast<uint4*>(o.y + static_cast<size_t>(row) * o.n_out + o.col_w + 8 * q) = pack_bf16x8(g);
        }
      }
    }
    __syncthreads();  // the regions are read before the next pass writes them
  }
}

// After the K loop: the sum of the workgroup's K slices (WK > 1), the split-K exchange
// between workgroups (split > 1) and the epilogue.  stage(i), i < S, is LDS region i of
// kStage bytes; all of them are free here.  Every wave of the workgroup calls this (the
// barriers count them all); only slice 0 holds results afterwards.
template <int WM, int TW, int NWG, int WK, int S, int kStage, class StageFn>
__device__ __forceinline__ void finish_tile(f32x4_t (&acc)[WM][TW], StageFn stage, int* is_last_lds,
                                            const TileOut& o, int wave_in, int wk, int lane) {
  if constexpr (WK > 1) {
    // Sum the slices' tiles in slice order: slices 1 .. WK - 1 park theirs in the stages
    // (lane-major fragments, 1 KiB each), slice 0 adds them to its own.  Parking slot
    // (k2 - 1) kFragsW + f holds fragment f of every wave of slice k2, wave-major, so its
    // stage and offset are compile-time constants once the slice is known (a uniform switch):
    // only the wave's index within its slice is added at run time.  (A stage chosen at run
    // time compiles to a chain of scalar compares, which all waves of a CU queue for on its
    // shared scalar unit: 1.4 us of the O M=64 launch on MI355X.)
    constexpr int kFragsW = WM * TW;
    constexpr int kSlotBytes = NWG * 1024;
    constexpr int kSlotsPerStage = kStage / kSlotBytes;
    static_assert(kSlotsPerStage >= 1 && (WK - 1) * kFragsW <= S * kSlotsPerStage, "slice tiles exceed the stages");
    const uint32_t lane_off = static_cast<uint32_t>(wave_in) * 1024u + static_cast<uint32_t>(lane) * 16u;
    auto slot_ptr = [&](auto slot_tag) -> f32x4_t* {
      constexpr int slot = decltype(slot_tag)::value;
      return reinterpret_cast<f32x4_t*>(stage(slot / kSlotsPerStage) + (slot % kSlotsPerStage) * kSlotBytes + lane_off);
    };
    auto park_slice = [&](auto k2_tag) {
      constexpr int k2 = decltype(k2_tag)::value;
      static_for<kFragsW>([&](auto f_tag) {
        constexpr int f = decltype(f_tag)::value;
        *slot_ptr(std::integral_constant<int, (k2 - 1) * kFragsW + f>{}) = acc[f / TW][f % TW];
      });
    };
    if (wk > 0) {
      static_for<WK - 1>([&](auto i_tag) {
        constexpr int k2 = decltype(i_tag)::value + 1;
        if (wk == k2) park_slice(std::integral_constant<int, k2>{});
      });
    }
    __syncthreads();
    if (wk == 0) {
      static_for<WK - 1>([&](auto i_tag) {
        constexpr int k2 = decltype(i_tag)::value + 1;
        static_for<kFragsW>([&](auto f_tag) {
          constexpr int f = decltype(f_tag)::value;
          acc[f / TW][f % TW] += *slot_ptr(std::integral_constant<int, (k2 - 1) * kFragsW + f>{});
        });
      });
    }
    __syncthreads();
  }

  if (o.split > 1) {
    // Every workgroup stores its fp32 fragments (lane-major, 1 KiB per 16 x 16 MFMA tile)
    // into partials[sidx][tile][wave of slice 0]; the last to arrive sums all splits in
    // split order, KC fragments at a time so that the loads of a chunk share one wait.  Only
    // slice 0 holds results; the other slices take part in the barriers alone.
    const int ntiles = o.ntiles;
    const int tile = o.tile;
    const int split = o.split, sidx = o.sidx;
    float* partials = o.partials;
    int* counters = o.counters;
    constexpr int kFrags = WM * TW;
    constexpr int KC = kFrags % 8 == 0 ? 8 : kFrags % 4 == 0 ? 4 : 2;
    static_assert(kFrags % KC == 0, "fragments must split into chunks");
    const __amdgpu_buffer_rsrc_t rp =
        make_buffer(partials, static_cast<uint32_t>(split) * ntiles * NWG * kFrags * 1024u);
    const uint32_t lane_off = static_cast<uint32_t>(lane) * 16u;
    auto frag_off = [&](int sp, int f) {
      return (((static_cast<uint32_t>(sp) * ntiles + tile) * NWG + wave_in) * kFrags + f) * 1024u + lane_off;
    };
    if (wk == 0) {
#pragma unroll
      for (int f = 0; f < kFrags; ++f) store_fragment(rp, frag_off(sidx, f), acc[f / TW][f % TW]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) *is_last_lds = (arrive(&counters[tile]) == split - 1);
    __syncthreads();
    if (!*is_last_lds || wk != 0) return;
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

  if constexpr (TW % 2 == 1) {
    if (o.act) {  // uniform: waves paired along N (WK == 1)
      cross_silu_epilogue<WM, TW, NWG, S, kStage>(acc, stage, o, wave_in, lane);
      return;
    }
  }
  if (!o.active || wk != 0) return;
  // Epilogue (slice 0): bf16 through LDS (row-major 16 WM rows x the wave's output columns:
  // rows of CPR 16-byte chunks swizzled by row), then 16-byte coalesced stores.  The stages
  // are free after the last barrier.  When they cannot hold every wave's columns at once, a
  // wave writes and stores its columns in two passes through half the space (wave-local).
  constexpr int WR = 16 * WM;  // rows of a wave
  constexpr int kFull = WR * 32 * TW;
  constexpr int kParts = (kStage / kFull) * S >= NWG ? 1 : 2;
  constexpr int kRegion = kFull / kParts;
  constexpr int kStageRows = kStage / kRegion;
  static_assert(kStageRows >= 1 && kStageRows * S >= NWG, "epilogue staging exceeds the stages");
  // the wave's region: stage wave_in / kStageRows, chosen with compile-time stage addresses
  uint8_t* ep = stage(0) + (wave_in % kStageRows) * kRegion;
  if constexpr (kStageRows < NWG) {
    static_for<(NWG + kStageRows - 1) / kStageRows>([&](auto i_tag) {
      constexpr int i = decltype(i_tag)::value;
      if (i > 0 && wave_in / kStageRows == i) ep = stage(i) + (wave_in % kStageRows) * kRegion;
    });
  }
  auto store_rows = [&](auto cpr_tag, int col0) {
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
      const int row = o.row_w + r;
      if (row < o.M) {
        const size_t off = static_cast<size_t>(row) * o.n_out + col0 + 8 * q;
        *reinterpret_cast<uint4*>(o.y + off) = o.res ? add_bf16x8(v, *reinterpret_cast<const uint4*>(o.res + off)) : v;
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // the region's reads are done before the next pass writes it
    __builtin_amdgcn_wave_barrier();
  };
  if constexpr ((TW & (TW - 1)) != 0) {
    // Three tiles per wave (48 columns; the fused product never has an odd count): whole
    // 96-byte row segments per store, the passes taking row ranges instead of column
    // ranges.  (A 32-byte piece per pass left every 64-byte block to two partial writes:
    // 1.7x the output bytes at QKV M=2048.)  Chunks rotate by row, (q + r) % CPR, since CPR
    // is not a power of two; 10 rows of 6 chunks per store round, lanes 60..63 idle.
    static_assert(WM % kParts == 0, "row passes of whole 16-row tiles");
    constexpr int CPR = 2 * TW;
    constexpr int PITCH = 16 * CPR;
    constexpr int MP = WM / kParts;  // 16-row tiles per pass
    constexpr int RP = 16 * MP;      // rows per pass: RP * PITCH == kRegion
    static_assert(RP * PITCH <= kRegion, "a row pass exceeds the wave's region");
    constexpr int kRowsPerRound = 64 / CPR;
#pragma unroll
    for (int part = 0; part < kParts; ++part) {
#pragma unroll
      for (int ml = 0; ml < MP; ++ml)
#pragma unroll
        for (int t = 0; t < TW; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 16 * ml + 4 * (lane >> 4) + i;
            const int c = 16 * t + (lane & 15);
            const int off = r * PITCH + ((((c >> 3) + r) % CPR) << 4) + ((c & 7) << 1);
            *reinterpret_cast<uint16_t*>(ep + off) = f32_to_bf16_bits(acc[part * MP + ml][t][i]);
          }
      __builtin_amdgcn_s_waitcnt(0);
      __builtin_amdgcn_wave_barrier();
#pragma unroll 4
      for (int round = 0; round < (RP + kRowsPerRound - 1) / kRowsPerRound; ++round) {
        const int r = kRowsPerRound * round + lane / CPR;
        const int q = lane % CPR;
        if (lane < kRowsPerRound * CPR && r < RP) {
          const uint4 v = *reinterpret_cast<const uint4*>(ep + r * PITCH + (((q + r) % CPR) << 4));
          const int row = o.row_w + RP * part + r;
          if (row < o.M) {
            const size_t off = static_cast<size_t>(row) * o.n_out + o.col_w + 8 * q;
            *reinterpret_cast<uint4*>(o.y + off) =
                o.res ? add_bf16x8(v, *reinterpret_cast<const uint4*>(o.res + off)) : v;
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0);  // the region's reads are done before the next pass writes it
      __builtin_amdgcn_wave_barrier();
    }
  } else if (!o.act) {
    constexpr int TP0 = TW / kParts;
    constexpr int TP = TP0 & -TP0;  // tiles per pass: a power of two, so that rows are whole lane groups
    constexpr int CPR = 2 * TP;     // 16-byte chunks per row
    constexpr int PITCH = 16 * CPR;
#pragma unroll
    for (int part = 0; part < TW / TP; ++part) {
#pragma unroll
      for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int t = 0; t < TP; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 16 * mt + 4 * (lane >> 4) + i;
            const int c = 16 * t + (lane & 15);
            const int off = r * PITCH + (((c >> 3) ^ (r % CPR)) << 4) + ((c & 7) << 1);
            *reinterpret_cast<uint16_t*>(ep + off) = f32_to_bf16_bits(acc[mt][part * TP + t][i]);
          }
      store_rows(std::integral_constant<int, CPR>{}, o.col_w + 16 * TP * part);
    }
  } else if constexpr (TW % 2 == 0) {  // the fused product pairs the two halves of a wave's tiles
    constexpr int H = TW / 2;
    constexpr int TP0 = (H % kParts == 0) ? H / kParts : H;
    constexpr int TP = TP0 & -TP0;  // gate tiles per pass (a power of two)
    constexpr int NP = H / TP;
    constexpr int CPR = 2 * TP;
    constexpr int PITCH = 16 * CPR;
#pragma unroll
    for (int part = 0; part < NP; ++part) {
#pragma unroll
      for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int t = 0; t < TP; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 16 * mt + 4 * (lane >> 4) + i;
            const int c = 16 * t + (lane & 15);
            const int off = r * PITCH + (((c >> 3) ^ (r % CPR)) << 4) + ((c & 7) << 1);
            const int tt = part * TP + t;
            *reinterpret_cast<uint16_t*>(ep + off) = f32_to_bf16_bits(silu_mul_of_bf16(acc[mt][tt][i], acc[mt][tt + H][i]));
          }
      store_rows(std::integral_constant<int, CPR>{}, o.col_w + 16 * TP * part);
    }
  }
}

}  // namespace w4a16
