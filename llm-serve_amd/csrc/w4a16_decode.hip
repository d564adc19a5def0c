// Decode / speculative-verify regime (M <= 64; the planner sends wide layers to the tile
// kernel above M = 48): HBM-bound split-K kernel.
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
//
// Memory traffic.  The weight stream is the only per-group global load of a wave: each
// wave copies the scales and zero words of its own groups and tiles (2.5 bytes per column
// and group) into a private slice of LDS once, at the start, by direct-to-LDS buffer loads
// with every lane busy, and so the activation rows of its groups when they are small (XL:
// M <= 4 rows and at most kDecodeMaxStagedX bytes per workgroup).  Small per-lane loads of
// scales, zeros and partly used activation rows issued per group cost memory-pipeline time
// out of proportion to their bytes; staging removes them from the streaming loop, whose
// vector-memory instructions are then the TN weight loads per group (plus the activation
// fragments when they are not staged).  The slices are private, so no barrier delays the
// start of the stream: a wave waits only for its own loads.
//
// RMSNorm prologue (NR = M <= 2 rows, with staged activations and no K split): each lane
// loads its share of the wave's activation rows, residual rows and norm-weight slices into
// registers before the ring's weight loads are issued, and the norm runs while those are in
// flight: per-row sums of squares of s = x + res, exchanged between the waves through LDS
// (one barrier that waits for LDS only, summed in wave order), then x_norm = bf16(bf16(s *
// rstd) * w) is written into the wave's activation slice in the staged layout; the first
// workgroup also writes the new residual and the normalized rows.  The row statistic needs
// the whole row, which a workgroup without a K split reads anyway, so the norm costs no
// kernel launch and no round trip of x_norm -- but every workgroup repeats it, on its
// critical path: measured on MI355X it adds 1.4 - 1.9 us to the Qwen3-8B QKV / gate|up
// GEMMs at M = 1, against about 3 us for the separate norm kernel.
#include <atomic>

#include "w4a16_common.h"
#include "w4a16_launch.h"

namespace w4a16 {

typedef __attribute__((address_space(3))) void lds_void_t;

struct DecodeArgs {
  DecodeRowStats rs;  // fused RMSNorm across two GEMMs (see DecodeRowStats), or all null
  const uint16_t* x;
  const uint32_t* packed;
  const uint32_t* qzeros;
  const uint16_t* scales;
  uint16_t* y;
  const uint16_t* res;  // residual added to y (may be y itself), or null
  float* partials;
  int* counters;
  int M, K, N, split;
  int up_tiles;  // 0: plain GEMM; else fused SiLU(gate) * up with up tiles this far past gate
  DecodeNorm norm;  // used by the NORM kernels only
};

// LDS layout of the staged operands.  A wave owns at most `items` groups (its groups
// gi = wave + i W of the workgroup's K range); its slice holds, per item i, scale pairs
// [items][TN * 8] words and zero words [items][TN * 2], then (XL) activations
// [items][M][128] bf16 with 16-byte chunks swizzled by row, then (pre) the dequant operands
// built from the scales and zeros: C inputs [items][TN][16 columns] x 16 bytes and
// diagonals [items][TN][16] x 8 bytes.  Region sizes are rounded so that the last
// 64-lane store of a region (4 or 16 bytes per lane) stays in it.  The cross-wave reduction
// reuses the same memory after the streaming loop.
struct DecodeLds {
  uint32_t s_off, z_off, x_off, c_off, d_off, wave_bytes, staged, reduce, total;
};

__host__ __device__ constexpr uint32_t round_up(uint32_t v, uint32_t a) { return (v + a - 1) / a * a; }

__host__ __device__ inline DecodeLds decode_lds_layout(int M, int K, int tn, int waves, int split, bool xl,
                                                      bool pre) {
  const int G = K / kGroup;
  const uint32_t n_gmax = static_cast<uint32_t>((G + split - 1) / split);
  const uint32_t items = (n_gmax + waves - 1) / waves;
  DecodeLds l{};
  l.s_off = 0;
  l.z_off = round_up(items * tn * 8u * 4u, 256u);
  l.x_off = l.z_off + round_up(items * tn * 2u * 4u, 256u);
  l.c_off = l.x_off + (xl ? round_up(items * static_cast<uint32_t>(M) * 256u, 1024u) : 0u);
  l.d_off = l.c_off + (pre ? items * tn * 16u * 16u : 0u);
  l.wave_bytes = round_up(l.d_off + (pre ? items * tn * 16u * 8u : 0u), 256u);
  l.staged = l.wave_bytes * static_cast<uint32_t>(waves);
  l.reduce = static_cast<uint32_t>(waves) * ((M + 15) / 16) * tn * 1024u;
  l.total = l.staged > l.reduce ? l.staged : l.reduce;
  return l;
}

// Launch constants, the same for every wave, computed once on the host: the LDS layout,
// the buffer sizes, the K split's group ranges and a multiplier for dividing by M.  (Every
// wave runs its own copy of whatever scalar set-up the kernel does, and the scalar unit is
// shared by the waves of a CU: at decode sizes, with 8 - 24 waves per CU, the divisions
// and layout arithmetic this replaces kept the weight stream from starting for 1 - 3 us.)
struct DecodeGeom {
  uint32_t z_off, x_off, c_off, d_off, wave_bytes;  // LDS layout (s_off = 0)
  uint32_t x_bytes, w_bytes, s_bytes, z_bytes;      // buffer sizes
  int G;                                            // 128-row groups of K
  int gq, gr;      // split s covers gq groups (gq + 1 for s < gr), starting at s gq + min(s, gr)
  uint32_t m_mul;  // ceil(2^16 / M): v / M == (v * m_mul) >> 16 for 0 <= v < 2^12
};

inline DecodeGeom decode_geom(int M, int K, int N, int tn, int waves, int split, bool xl, bool pre) {
  const DecodeLds l = decode_lds_layout(M, K, tn, waves, split, xl, pre);
  const int G = K / kGroup;
  DecodeGeom g{};
  g.z_off = l.z_off;
  g.x_off = l.x_off;
  g.c_off = l.c_off;
  g.d_off = l.d_off;
  g.wave_bytes = l.wave_bytes;
  g.x_bytes = static_cast<uint32_t>(M) * K * 2u;
  g.w_bytes = static_cast<uint32_t>(K) * (N / 2);
  g.s_bytes = static_cast<uint32_t>(G) * N * 2u;
  g.z_bytes = static_cast<uint32_t>(G) * (N / 8) * 4u;
  g.G = G;
  g.gq = G / split;
  g.gr = G % split;
  g.m_mul = (65536u + static_cast<uint32_t>(M) - 1u) / static_cast<uint32_t>(M);
  return g;
}

// Column tiles of a workgroup.  Plain: tiles tb + tt, tt < TN.  Fused gate/up (TN even,
// H = TN / 2): gate tiles tb + tt for tt < H and their up tiles tb + up_tiles + tt - H, i.e.
// tile tb + tt + dt for tt >= H with dt = up_tiles - H (dt = 0 plain).
template <int TN>
__device__ __forceinline__ int decode_tile(int tb, int dt, int tt) {
  return tb + tt + (tt >= TN / 2 ? dt : 0);
}

// Everything one wave loads from global memory for one 128-row group: one 16-byte weight
// load per tile and, when the activations are not staged, the MB x 4 activation fragments.
// Loaded DEPTH groups ahead of use; decoded only when consumed.
template <int MB, int TN, bool XL>
struct DecodeStage {
  u32x4_t w[TN];
  u32x4_t a[XL ? 1 : MB][4];
};

// Buffer descriptors of the four inputs.  Every global load of the decode kernel is an
// unconditional buffer load: a lane or a group with nothing to fetch (activation row >= M,
// group past the workgroup's K range) uses kOutOfRange, which the hardware answers with
// zeros and no memory access.  With no branch around any load the compiler's wait counts
// are exact, so the DEPTH groups in flight really overlap.
struct DecodeSources {
  __amdgpu_buffer_rsrc_t x, w, s, z;
};

template <int MB, int TN, bool XL>
__device__ __forceinline__ void load_decode_stage(DecodeStage<MB, TN, XL>& st, const DecodeSources& src,
                                                  const uint32_t (&x_row)[MB], int g, bool valid, int N, int tb,
                                                  int dt, int lane) {
  const int NT = N / kTileCols;
  const uint32_t oob = valid ? 0u : kOutOfRange;
#pragma unroll
  for (int tt = 0; tt < TN; ++tt) {
    const int t = decode_tile<TN>(tb, dt, tt);
    const uint32_t wo = (valid ? static_cast<uint32_t>(tile_word(g, t, NT, lane)) * 4u : 0u) | oob;
    st.w[tt] = __builtin_amdgcn_raw_buffer_load_b128(src.w, wo, 0, 0);
  }
  if constexpr (!XL) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const uint32_t xo = (x_row[mb] | oob) + static_cast<uint32_t>(kGroup * g) * 2u;
#pragma unroll
      for (int j = 0; j < 4; ++j) st.a[mb][j] = __builtin_amdgcn_raw_buffer_load_b128(src.x, xo + 64u * j, 0, 0);
    }
  }
}

// Multiply-accumulate one group: the dequant operands (built from the staged scales and
// zeros, or with PRE read prebuilt) and, with XL, the activation fragments come from the
// wave's LDS slice `wl`; i is the group's item index within the wave.
template <int MB, int TN, bool XL, bool PRE>
__device__ __forceinline__ void compute_decode_stage(f32x4_t (&acc)[MB][TN], const DecodeStage<MB, TN, XL>& st,
                                                     const uint8_t* wl, const DecodeLds& lay, int i, int M,
                                                     const NibbleConsts& nib, int lane) {
  const int c = lane & 15;
  TileScale ts[TN];
  if constexpr (PRE) {
    const f32x4_t* lc = reinterpret_cast<const f32x4_t*>(wl + lay.c_off) + i * (TN * 16) + c;
    const s16x4_t* ld = reinterpret_cast<const s16x4_t*>(wl + lay.d_off) + i * (TN * 16) + c;
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) {
      ts[tt].cin = lc[tt * 16];
      ts[tt].diag = ld[tt * 16];
    }
  } else {
    const uint32_t* ls = reinterpret_cast<const uint32_t*>(wl + lay.s_off) + i * (TN * 8) + (c >> 1);
    const uint32_t* lz = reinterpret_cast<const uint32_t*>(wl + lay.z_off) + i * (TN * 2) + (c >> 3);
    const int zshift = awq_shift(lane & 7);
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) ts[tt] = make_tile_scale(ls[tt * 8], (lz[tt * 2] >> zshift) & 0xFu, lane);
  }
  u32x4_t a[MB][4];
  if constexpr (XL) {
    // Rows >= M read row M - 1: their outputs are never stored.
    const int r = (c < M ? c : M - 1);
    const uint8_t* lx = wl + lay.x_off + (i * M + r) * 256;
#pragma unroll
    for (int js = 0; js < 4; ++js)
      a[0][js] = *reinterpret_cast<const u32x4_t*>(lx + ((((js << 2) | (lane >> 4)) ^ (r & 15)) << 4));
  } else {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int js = 0; js < 4; ++js) a[mb][js] = st.a[mb][js];
  }
  // Per 32-row step: every tile's unpack and scaling MFMAs first, then each tile's rounding
  // to bf16 and main MFMAs, so that a rounding does not wait on the scaling MFMA issued just
  // before it (the tile-by-tile order measured 3-5 % slower for gate_up at M = 8 and 16).
#pragma unroll
  for (int js = 0; js < 4; ++js) {
    ScaledStep sd[TN];
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) sd[tt] = dequant_scale(st.w[tt][js], ts[tt], nib);
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) {
      const bf16x8_t frag = dequant_pack(sd[tt]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        acc[mb][tt] = mfma16(__builtin_bit_cast(bf16x8_t, a[mb][js]), frag, acc[mb][tt]);
    }
  }
}

// Staging of the scale pairs, zero words and (XL) activation rows of the wave's items
// (groups g_first + i W, i < n_items) into its LDS slice `wl`, in two steps around the issue
// of the weight ring: load_staged() issues ordinary register loads (64 consecutive words or
// 16-byte chunks per instruction, every lane busy; lanes past the end fetch nothing),
// store_staged() writes them to the slice once they have arrived.  (Direct-to-LDS loads, the
// obvious alternative, cost 0.35 - 1.5 us of issue time per launch at the Qwen3-8B decode
// shapes on MI355X, growing with the waves per CU; register loads issue at once.)  At most
// kStageS x 64 scale words, kStageZ x 64 zero words and kStageX x 64 activation chunks
// per wave (decode_stage_fits()).  With NORM the activation slice is written by the norm
// prologue instead.
// Prebuilt dequant operands (PRE) of one-tile workgroups come straight from one scale and
// one zero word per lane and (item, column) entry -- the words of its own entry -- with no
// round trip of the raw words through LDS: measured on MI355X 2-4 % faster for QKV and O at
// M <= 4.  With more tiles the entries outnumber the contiguous words several times, and
// the extra loads cost more than the round trip (gate_up M=1 +6 %, down M=4 +8 %).
template <int TN, bool PRE>
constexpr bool direct_entries() {
  return PRE && TN == 1;
}

template <int TN, bool XL, bool PRE>
struct StagedRegs {
  uint32_t s[direct_entries<TN, PRE>() ? kStageE : kStageS];  // scale words: contiguous, or per entry
  uint32_t z[direct_entries<TN, PRE>() ? kStageE : kStageZ];  // zero words, likewise
  u32x4_t x[XL ? kStageX : 1];
};

template <int TN, bool XL, int W, bool NORM, bool PRE>
__device__ __forceinline__ void load_staged(StagedRegs<TN, XL, PRE>& st, const DecodeSources& src, int M, int K, int N,
                                            int tb, int dt, int g_first, int n_items, int lane, uint32_t m_mul) {
  if constexpr (direct_entries<TN, PRE>()) {
    // entry e = (item, column c) of the single tile: the words holding column c's scale and zero
    const int entries = n_items * 16;
#pragma unroll
    for (int u = 0; u < kStageE; ++u) {
      if (u == 0 || 64 * u < entries) {  // uniform
        const int e = 64 * u + lane;
        const int col = kTileCols * tb + (e & 15);
        const int g = g_first + (e >> 4) * W;
        const bool ok = e < entries;
        st.s[u] = __builtin_amdgcn_raw_buffer_load_b32(
            src.s, ok ? static_cast<uint32_t>(g * N + (col & ~1)) * 2u : kOutOfRange, 0, 0);
        st.z[u] = __builtin_amdgcn_raw_buffer_load_b32(
            src.z, ok ? static_cast<uint32_t>(g * (N >> 3) + (col >> 3)) * 4u : kOutOfRange, 0, 0);
      }
    }
  } else {
    constexpr int kSW = TN * 8;  // scale-pair words per group (8 per tile)
    constexpr int kZW = TN * 2;  // zero words per group (2 per tile)
    const int s_words = n_items * kSW;
#pragma unroll
    for (int u = 0; u < kStageS; ++u) {
      if (u == 0 || 64 * u < s_words) {  // uniform
        const int w = 64 * u + lane;
        const int i = w / kSW;
        const int j = w - i * kSW;
        const int sj = tb * 8 + j + (j >= (TN / 2) * 8 ? dt * 8 : 0);
        const uint32_t off =
            w < s_words ? static_cast<uint32_t>((g_first + i * W) * (N >> 1) + sj) * 4u : kOutOfRange;
        st.s[u] = __builtin_amdgcn_raw_buffer_load_b32(src.s, off, 0, 0);
      }
    }
    const int z_words = n_items * kZW;
#pragma unroll
    for (int u = 0; u < kStageZ; ++u) {
      if (u == 0 || 64 * u < z_words) {
        const int w = 64 * u + lane;
        const int i = w / kZW;
        const int j = w - i * kZW;
        const int zj = tb * 2 + j + (j >= (TN / 2) * 2 ? dt * 2 : 0);
        const uint32_t off =
            w < z_words ? static_cast<uint32_t>((g_first + i * W) * (N >> 3) + zj) * 4u : kOutOfRange;
        st.z[u] = __builtin_amdgcn_raw_buffer_load_b32(src.z, off, 0, 0);
      }
    }
  }
  if constexpr (XL && !NORM) {
    // LDS chunk C = (i M + r) 16 + cc holds global chunk cc ^ (r & 15) of row r of item i's
    // group: the 16 rows of one fragment read then sit in 16 different chunk positions,
    // i.e. on all 64 banks once.
    const int chunks = n_items * M * 16;
#pragma unroll
    for (int u = 0; u < kStageX; ++u) {
      if (u == 0 || 64 * u < chunks) {
        const int C = 64 * u + lane;
        const int im = C >> 4;  // < 2^12: a workgroup stages at most 32 KiB of 256-byte row slices
        const int i = static_cast<int>((static_cast<uint32_t>(im) * m_mul) >> 16);
        const int r = im - i * M;
        const int cc = (C & 15) ^ (r & 15);
        const uint32_t off =
            C < chunks
                ? (static_cast<uint32_t>(r) * K + static_cast<uint32_t>(g_first + i * W) * kGroup) * 2u + cc * 16u
                : kOutOfRange;
        st.x[u] = __builtin_amdgcn_raw_buffer_load_b128(src.x, off, 0, 0);
      }
    }
  }
}

// Dequant operands of every (item, tile, column) entry of the wave, built once instead of
// per tile and group in the loop (make_tile_scale depends on the lane only through lane % 4,
// which equals the entry's column % 4 for every lane that later reads entry c).  It saves
// about 12 VALU instructions per tile and group but puts an LDS round trip before the first
// group: measured on MI355X it pays with 8 waves and a ring at least two groups deep
// (gate_up M=16 -4 %), and costs 2-8 % with 4 waves or a one-group ring, where that
// latency is not hidden.  From the staged raw words in LDS:
template <int TN>
__device__ __forceinline__ void build_tile_scales(uint8_t* wl, const DecodeLds& lay, int n_items, int lane) {
  const uint32_t* ls = reinterpret_cast<const uint32_t*>(wl + lay.s_off);
  const uint32_t* lz = reinterpret_cast<const uint32_t*>(wl + lay.z_off);
  f32x4_t* lc = reinterpret_cast<f32x4_t*>(wl + lay.c_off);
  s16x4_t* ld = reinterpret_cast<s16x4_t*>(wl + lay.d_off);
  const int entries = n_items * TN * 16;
  for (int e = lane; e < entries; e += 64) {
    const int c = e & 15;
    const int it = e >> 4;  // item * TN + tile
    const uint32_t z = (lz[it * 2 + (c >> 3)] >> awq_shift(c & 7)) & 0xFu;
    const TileScale t = make_tile_scale(ls[it * 8 + (c >> 1)], z, c);
    lc[e] = t.cin;
    ld[e] = t.diag;
  }
}

// Lanes past a region's end write into its rounding (every region is a multiple of 64
// words or 64 chunks).  With PRE the dequant operands are built here: from the lane's own
// entry words (direct_entries), or from the raw words once they are in LDS.
template <int TN, bool XL, bool NORM, bool PRE>
__device__ __forceinline__ void store_staged(const StagedRegs<TN, XL, PRE>& st, uint8_t* wl, const DecodeLds& lay, int M,
                                             int n_items, int lane) {
  if constexpr (direct_entries<TN, PRE>()) {
    const int entries = n_items * 16;
#pragma unroll
    for (int u = 0; u < kStageE; ++u) {
      const int e = 64 * u + lane;
      if ((u == 0 || 64 * u < entries) && e < entries) {
        const int c = e & 15;
        const TileScale t = make_tile_scale(st.s[u], (st.z[u] >> awq_shift(c & 7)) & 0xFu, c);
        reinterpret_cast<f32x4_t*>(wl + lay.c_off)[e] = t.cin;
        reinterpret_cast<s16x4_t*>(wl + lay.d_off)[e] = t.diag;
      }
    }
  } else {
    const int s_words = n_items * TN * 8;
#pragma unroll
    for (int u = 0; u < kStageS; ++u)
      if (u == 0 || 64 * u < s_words) reinterpret_cast<uint32_t*>(wl + lay.s_off)[64 * u + lane] = st.s[u];
    const int z_words = n_items * TN * 2;
#pragma unroll
    for (int u = 0; u < kStageZ; ++u)
      if (u == 0 || 64 * u < z_words) reinterpret_cast<uint32_t*>(wl + lay.z_off)[64 * u + lane] = st.z[u];
    if constexpr (PRE) build_tile_scales<TN>(wl, lay, n_items, lane);
  }
  if constexpr (XL && !NORM) {
    const int chunks = n_items * M * 16;
#pragma unroll
    for (int u = 0; u < kStageX; ++u)
      if (u == 0 || 64 * u < chunks) reinterpret_cast<u32x4_t*>(wl + lay.x_off)[64 * u + lane] = st.x[u];
  }
}

// Operands of the RMSNorm prologue held by one lane: lane l works on item i = l / 16 of the
// wave (at most kNormItems items; lanes past n_items idle) at staged chunk position p = l % 16
// of each of the M <= 4 rows, i.e. on row r's 16-byte chunk c = p ^ r of the item's group --
// the chunk the staged layout keeps at position p -- so the wave's 64 lanes cover its four
// items and each lane does M chunks.
constexpr int kNormItems = 4;
// Rows of the prologue: NR = M registers' worth each (at M >= 3 the extra loads and registers
// made the one-launch form slower than the norm kernel plus the GEMM on MI355X).
constexpr int kNormMaxRows = 2;
template <int NR>  // rows held: M <= NR
struct NormRegs {
  u32x4_t x[NR], r[NR], w[NR];
};

__device__ __forceinline__ uint4 as_uint4(u32x4_t v) { return make_uint4(v[0], v[1], v[2], v[3]); }

// Issues the lane's activation, residual (a null residual: a zero-length buffer, which
// loads zeros) and weight chunks; rows past M and items past n_items fetch nothing.
template <int W, int NR>
__device__ __forceinline__ void load_norm_operands(NormRegs<NR>& nr, const DecodeSources& src,
                                                   __amdgpu_buffer_rsrc_t rres, __amdgpu_buffer_rsrc_t rw, int M, int K,
                                                   int g_first, int n_items, int lane) {
  const int i = lane >> 4;
  const int p = lane & 15;
  const uint32_t g0 = static_cast<uint32_t>(g_first + i * W) * kGroup;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const bool ok = r < M && i < n_items;
    const uint32_t col = (g0 + 8u * static_cast<uint32_t>(p ^ r)) * 2u;
    const uint32_t xo = ok ? static_cast<uint32_t>(r) * K * 2u + col : kOutOfRange;
    nr.x[r] = __builtin_amdgcn_raw_buffer_load_b128(src.x, xo, 0, 0);
    nr.r[r] = __builtin_amdgcn_raw_buffer_load_b128(rres, xo, 0, 0);
    nr.w[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? col : kOutOfRange, 0, 0);
  }
}

// The prologue proper: s = x + res in fp32 (s = x without a residual); per row, the sum of
// s^2 over the lane's chunk, over the wave's 64 lanes (xor shuffles) to part[wave][row], a
// workgroup barrier on LDS alone (the weight loads in flight are not waited for), the row
// scale from the sum over the waves in wave order, then x_norm written into the wave's
// activation slice; the writer workgroup also stores res_out = bf16(s) and x_out = x_norm.
// Every workgroup computes the same values in the same order.
template <int W, int NR>
__device__ __forceinline__ void norm_rows(const NormRegs<NR>& nr, uint8_t* wl, const DecodeLds& lay, float (*part)[4],
                                          int wave, int lane, int M, int K, int g_first, int n_items, bool writer,
                                          const DecodeNorm& nrm) {
  const int i = lane >> 4;
  const int p = lane & 15;
  const bool live = i < n_items;
  const bool has_res = nrm.res != nullptr;
  float sv[NR][8];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if (r < M) {
      unpack_bf16x8(as_uint4(nr.x[r]), sv[r]);
      if (has_res) {
        float rv[8];
        unpack_bf16x8(as_uint4(nr.r[r]), rv);
#pragma unroll
        for (int q = 0; q < 8; ++q) sv[r][q] += rv[q];
      }
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) ss += sv[r][q] * sv[r][q];
      ss = wave_sum64(ss);
      if (lane == 0) part[wave][r] = ss;
    }
  }
  // Only LDS needs ordering here: a workgroup-scope fence on the local address space waits
  // for LDS operations alone, so the barrier leaves the ring's loads in flight.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  const size_t g0 = static_cast<size_t>(g_first + i * W) * kGroup;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if (r < M) {
      float t = 0.f;
      for (int w = 0; w < W; ++w) t += part[w][r];
      const float rstd = rsqrt_rn(t / static_cast<float>(K) + nrm.eps);
      if (live) {
        const uint4 out = rms_scale_bf16x8(sv[r], rstd, as_uint4(nr.w[r]));
        *reinterpret_cast<uint4*>(wl + lay.x_off + (i * M + r) * 256 + p * 16) = out;
        if (writer) {
          const size_t off = static_cast<size_t>(r) * K + g0 + 8 * (p ^ r);
          *reinterpret_cast<uint4*>(nrm.x_out + off) = out;
          if (has_res) *reinterpret_cast<uint4*>(nrm.res_out + off) = pack_bf16x8(sv[r]);
        }
      }
    }
  }
}

// Consumer of the fused RMSNorm statistics (NSR > 0: room for NSR >= M rows, M <= 8, staged
// activations): the producer GEMM left s = float(h) + float(residual) in fp32 and, per row, the
// sums of s^2 over each 16-column tile (DecodeRowStats).  Lane l works on item i = l / 16 of
// its wave and on the group's global chunk p = l % 16 (8 columns) of every row, so it loads the
// norm weight's chunk once and two 16-byte fp32 halves per row; row r's chunk p goes to staged
// position p ^ r, the layout the staged-activation loop reads.  Only the M real rows are
// normalized, once per workgroup and group (the loop's 16-row fragments would redo it for
// every padded row).
template <int NSR>
struct NsRegs {
  u32x4_t s[NSR][2];
  u32x4_t w;
};

template <int W, int NSR>
__device__ __forceinline__ void load_ns_operands(NsRegs<NSR>& ns, __amdgpu_buffer_rsrc_t rsum,
                                                 __amdgpu_buffer_rsrc_t rw, int M, int K, int g_first, int n_items,
                                                 int lane) {
  const int i = lane >> 4;
  const bool live = i < n_items;
  const uint32_t col = static_cast<uint32_t>(g_first + i * W) * kGroup + 8u * static_cast<uint32_t>(lane & 15);
  ns.w = __builtin_amdgcn_raw_buffer_load_b128(rw, live ? col * 2u : kOutOfRange, 0, 0);
  // Rows past M issue nothing (a uniform branch): an out-of-range load still occupies the
  // CU's address unit, shared by all its waves.
#pragma unroll
  for (int r = 0; r < NSR; ++r) {
    if (r < M) {
      const uint32_t off = (static_cast<uint32_t>(r) * K + col) * 4u;
      ns.s[r][0] = __builtin_amdgcn_raw_buffer_load_b128(rsum, live ? off : kOutOfRange, 0, 0);
      ns.s[r][1] = __builtin_amdgcn_raw_buffer_load_b128(rsum, live ? off + 16u : kOutOfRange, 0, 0);
    }
  }
}

// The per-row tile sums of s^2 a wave reduces: rows wave + j W (j < kRows), at most two 16-byte
// chunks of four tile sums per lane and row (K <= 8192; longer rows load the rest later).
template <int W>
struct NsStats {
  static constexpr int kRows = (8 + W - 1) / W;
  u32x4_t q[kRows][2];
};

template <int W>
__device__ __forceinline__ void load_ns_stats(NsStats<W>& st, __amdgpu_buffer_rsrc_t rq, int M, int tiles_k, int wave,
                                              int lane) {
#pragma unroll
  for (int j = 0; j < NsStats<W>::kRows; ++j) {
    const int r = wave + j * W;
    if (r < M) {  // wave-uniform
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c0 = 4 * lane + 256 * h;
        st.q[j][h] = __builtin_amdgcn_raw_buffer_load_b128(
            rq, c0 < tiles_k ? static_cast<uint32_t>(r * tiles_k + c0) * 4u : kOutOfRange, 0, 0);
      }
    }
  }
}

// Row scales into row_rstd[r]: each lane sums its tile sums in chunk order (four at a time),
// then the wave sums its lanes (xor butterfly) -- the same order in every workgroup, whatever
// the wave count -- and 1 / rms = rsqrt(sum / K + eps).
template <int W>
__device__ __forceinline__ void ns_row_scales(const NsStats<W>& st, __amdgpu_buffer_rsrc_t rq, float* row_rstd, int M,
                                              int K, int tiles_k, float eps, int wave, int lane) {
#pragma unroll
  for (int j = 0; j < NsStats<W>::kRows; ++j) {
    const int r = wave + j * W;
    if (r < M) {  // wave-uniform
      float t = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x4_t v = st.q[j][h];
        t += (__uint_as_float(v[0]) + __uint_as_float(v[1])) + (__uint_as_float(v[2]) + __uint_as_float(v[3]));
      }
      for (int c0 = 4 * lane + 512; c0 < tiles_k; c0 += 256) {
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rq, static_cast<uint32_t>(r * tiles_k + c0) * 4u, 0, 0);
        t += (__uint_as_float(v[0]) + __uint_as_float(v[1])) + (__uint_as_float(v[2]) + __uint_as_float(v[3]));
      }
      t = wave_sum64(t);
      if (lane == 0) row_rstd[r] = rsqrt_rn(t / static_cast<float>(K) + eps);
    }
  }
}

// x_norm = bf16(bf16(s * rstd) * w) of the lane's chunk of every row into the wave's staged
// activation slice; the writer workgroup also stores it to x_out.
template <int W, int NSR>
__device__ __forceinline__ void ns_rows(const NsRegs<NSR>& ns, const float* row_rstd, uint8_t* wl, const DecodeLds& lay,
                                        int M, int K, int g_first, int n_items, int lane, uint16_t* x_out) {
  const int i = lane >> 4;
  const int p = lane & 15;
  if (i >= n_items) return;
  float w[8];
  unpack_bf16x8(as_uint4(ns.w), w);
  const size_t col = static_cast<size_t>(g_first + i * W) * kGroup + 8 * p;
#pragma unroll
  for (int r = 0; r < NSR; ++r) {
    if (r < M) {
      float sv[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sv[q] = __uint_as_float(ns.s[r][0][q]);
        sv[4 + q] = __uint_as_float(ns.s[r][1][q]);
      }
      const uint4 out = rms_scale_bf16x8(sv, row_rstd[r], w);
      *reinterpret_cast<uint4*>(wl + lay.x_off + (i * M + r) * 256 + ((p ^ r) & 15) * 16) = out;
      if (x_out != nullptr) *reinterpret_cast<uint4*>(x_out + static_cast<size_t>(r) * K + col) = out;
    }
  }
}

// FN, the fused RMSNorm split across two GEMMs (DecodeRowStats): 0 none, 1..8 the consumer
// with room for FN rows, -1 the producer.  A compile-time mode, so that the plain kernels carry
// none of it (the producer's epilogue behind a run-time test cost the plain decode GEMMs 2 %).
template <int MB, int TN, int DEPTH, int WAVES, bool XL, int NR, int FN>
__global__ __launch_bounds__(64 * WAVES) void decode_kernel(const uint16_t* __restrict__ x,
                                                            const uint32_t* __restrict__ packed,
                                                            const uint32_t* __restrict__ qzeros,
                                                            const uint16_t* __restrict__ scales,
                                                            uint16_t* y, const uint16_t* res,
                                                            float* __restrict__ partials,
                                                            int* __restrict__ counters, int M, int K, int N,
                                                            int split, int up_tiles, DecodeGeom geo, DecodeNorm nrm,
                                                            DecodeRowStats rs) {
  constexpr bool NORM = NR > 0;
  constexpr bool NS = FN > 0;
  constexpr bool PROD = FN < 0;
  constexpr int NSR = NS ? FN : 1;
  static_assert(!NORM || (XL && MB == 1), "the norm prologue works on staged rows (M <= 4)");
  static_assert(!NS || (XL && MB == 1 && !NORM && FN <= 8), "the fused-norm consumer stages its rows (M <= 8)");
  static_assert(!PROD || (MB == 1 && !NORM), "the fused-norm producer runs at M <= 8");
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  __shared__ int is_last;
  __shared__ float norm_part[NORM ? WAVES : 1][4];
  __shared__ float row_rstd[NS ? 8 : 1];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  constexpr int W = WAVES;
  const int cb = blockIdx.x;
  const int sidx = blockIdx.y;
  const int g_begin = sidx * geo.gq + (sidx < geo.gr ? sidx : geo.gr);
  const int nG = geo.gq + (sidx < geo.gr ? 1 : 0);
  // Fused SiLU(gate) * up (TN even): the workgroup's H gate tiles are output tiles
  // cb H .. cb H + H - 1 of the [M, N / 2] result.
  constexpr int H = TN / 2;
  const bool act = TN % 2 == 0 && up_tiles != 0;
  const int tb = act ? cb * H : cb * TN;
  const int dt = act ? up_tiles - H : 0;
  constexpr bool kPre = decode_prebuilt_scales(WAVES, DEPTH);
  const DecodeLds lay{0u, geo.z_off, geo.x_off, geo.c_off, geo.d_off, geo.wave_bytes, 0u, 0u, 0u};

  DecodeSources src;
  src.x = make_buffer(x, geo.x_bytes);
  src.w = make_buffer(packed, geo.w_bytes);
  src.s = make_buffer(scales, geo.s_bytes);
  src.z = make_buffer(qzeros, geo.z_bytes);
  uint32_t x_row[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = 16 * mb + (lane & 15);
    x_row[mb] = row < M ? static_cast<uint32_t>(row * K + 8 * (lane >> 4)) * 2u : kOutOfRange;
  }

  f32x4_t acc[MB][TN];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) acc[mb][tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // The wave's groups: gi = wave + i W of the K range, i < n_items.
  const int n_items = nG > wave ? (nG - wave + W - 1) / W : 0;
  uint8_t* wl = lds + wave * lay.wave_bytes;
  StagedRegs<TN, XL, kPre> staged;
  load_staged<TN, XL, W, NORM || NS, kPre>(staged, src, M, K, N, tb, dt, g_begin + wave, n_items, lane, geo.m_mul);
  // Residual epilogues: when every wave owns at most one output pair (pair p belongs to wave
  // p), the wave loads its pair's residual values now, ahead of the ring, so their latency
  // (the previous kernel wrote them) hides behind the stream instead of ending the kernel.
  constexpr bool kResPre = MB * TN <= WAVES;
  uint32_t res_pre[2] = {0u, 0u};  // rows 16 mb + 4 (lane / 16) + i, i < 4, two bf16 per word
  if (kResPre && res != nullptr && up_tiles == 0 && wave < MB * TN) {
    const int mb = wave / TN, tt = wave % TN;
    const size_t n = 16 * static_cast<size_t>(tb + tt) + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * mb + 4 * (lane >> 4) + i;
      const uint32_t v = row < M ? res[static_cast<size_t>(row) * N + n] : 0u;
      res_pre[i >> 1] |= v << (16 * (i & 1));
    }
  }
  // The residual of output pair p (owned by this wave), row i of the lane's four, at idx.
  auto res_bits = [&](int p, int i, size_t idx) -> uint16_t {
    (void)p;
    if constexpr (kResPre) return static_cast<uint16_t>(res_pre[i >> 1] >> (16 * (i & 1)));
    return res[idx];
  };
  NormRegs<(NR > 0 ? NR : 1)> nr;
  if constexpr (NORM)
    load_norm_operands<W>(nr, src, make_buffer(nrm.res, nrm.res ? geo.x_bytes : 0u),
                          make_buffer(nrm.w, static_cast<uint32_t>(K) * 2u), M, K, g_begin + wave, n_items, lane);
  // NS: the rows of s (M x K fp32: twice the bf16 activation bytes) and the tile sums of s^2
  NsRegs<NSR> nsr;
  NsStats<W> nss;
  const int tiles_k = K / kTileCols;
  const __amdgpu_buffer_rsrc_t rq = make_buffer(NS ? rs.ssq_in : nullptr, NS ? static_cast<uint32_t>(M) * tiles_k * 4u : 0u);
  if constexpr (NS) {
    load_ns_operands<W>(nsr, make_buffer(rs.s_in, geo.x_bytes * 2u), make_buffer(rs.w, static_cast<uint32_t>(K) * 2u),
                        M, K, g_begin + wave, n_items, lane);
    load_ns_stats<W>(nss, rq, M, tiles_k, wave, lane);
  }
  __builtin_amdgcn_sched_barrier(0);  // the staging loads stay ahead of the ring's

  // Depth-DEPTH ring over the wave's items: item i is loaded while item i - DEPTH is being
  // consumed.  The ring is filled first; then every load is issued whether or not its item
  // exists (out-of-range ones fetch nothing), so no branch encloses a load and the
  // scheduling barriers keep each item's loads together and in order.
  DecodeStage<MB, TN, XL> ring[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d)
    load_decode_stage<MB, TN, XL>(ring[d], src, x_row, g_begin + wave + d * W, d < n_items, N, tb, dt, lane);
  // The staged operands go to LDS as soon as they arrive (the ring's loads stay in flight:
  // the compiler waits for each register load individually), then the norm prologue works
  // from its registers and writes the activation slice.
  store_staged<TN, XL, NORM || NS, kPre>(staged, wl, lay, M, n_items, lane);
  if constexpr (NORM)
    norm_rows<W>(nr, wl, lay, norm_part, wave, lane, M, K, g_begin + wave, n_items, blockIdx.x == 0 && sidx == 0, nrm);
  if constexpr (NS) {
    // Row scales (wave w takes rows w, w + W, ...), shared through LDS by one barrier that
    // orders LDS alone (the ring's loads stay in flight); then each wave normalizes its items'
    // rows into its own slice, which only it reads.  The first column block's workgroups
    // store x_norm (each its own K range).
    ns_row_scales<W>(nss, rq, row_rstd, M, K, tiles_k, rs.eps, wave, lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    ns_rows<W>(nsr, row_rstd, wl, lay, M, K, g_begin + wave, n_items, lane, blockIdx.x == 0 ? rs.x_out : nullptr);
  }

  const NibbleConsts nib = nibble_consts();
  for (int base = 0; base < n_items; base += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int i = base + d;
      if (i < n_items) compute_decode_stage<MB, TN, XL, kPre>(acc, ring[d], wl, lay, i, M, nib, lane);
      const int in = i + DEPTH;
      __builtin_amdgcn_sched_barrier(0);
      load_decode_stage<MB, TN, XL>(ring[d], src, x_row, g_begin + wave + in * W, in < n_items, N, tb, dt, lane);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Reduce the W waves' partial sums in wave order (through the staging memory, once every
  // wave has finished reading it).
  f32x4_t* red = reinterpret_cast<f32x4_t*>(lds);  // [W][MB][TN][64]
  __syncthreads();
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int tt = 0; tt < TN; ++tt) red[((wave * MB + mb) * TN + tt) * 64 + lane] = acc[mb][tt];
  __syncthreads();

  // Output (mb, tt) pairs are spread over the waves; p is a compile-time index so the
  // register arrays stay in registers.  Fused, a gate pair and its up pair (tt and tt + H)
  // belong to the same wave.
  constexpr int kPairs = MB * TN;
  auto owner = [&](int p) {
    return (act ? (p / TN) * H + (p % TN) % (H > 0 ? H : 1) : p) % W;
  };
  f32x4_t out[kPairs];
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    if (owner(p) != wave) continue;
    f32x4_t v = red[p * 64 + lane];
#pragma unroll
    for (int w = 1; w < W; ++w) v += red[(w * kPairs + p) * 64 + lane];
    out[p] = v;
  }

  if (split > 1) {
    // Split K: every workgroup stores its fp32 fragments (lane-major, 1 KiB per output
    // pair) into partials[sidx][cb]; the last to arrive sums all splits in split order.
    const int nwg = gridDim.x;
    const __amdgpu_buffer_rsrc_t rp = make_buffer(partials, static_cast<uint32_t>(split) * nwg * kPairs * 1024u);
    const uint32_t lane_off = static_cast<uint32_t>(lane) * 16u;
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      if (owner(p) != wave) continue;
      store_fragment(rp, ((static_cast<uint32_t>(sidx) * nwg + cb) * kPairs + p) * 1024u + lane_off, out[p]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) is_last = (arrive(&counters[cb]) == split - 1);
    __syncthreads();
    if (!is_last) return;
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      if (owner(p) != wave) continue;
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
      out[p] = v;
    }
    if (threadIdx.x == 0) rearm(&counters[cb]);
  }

  const int c = lane & 15;
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    if (owner(p) != wave) continue;
    const int mb = p / TN, tt = p % TN;
    if (PROD) {  // compile-time
      // Producer of a fused RMSNorm: s = float(bf16(o)) + float(res) in fp32, the new
      // residual bf16(s), and per row the sum of s^2 over this 16-column tile (the 16 lanes
      // of each row quad -- one DPP row -- hold its 16 columns).
      const int n = 16 * (tb + tt) + c;
      float ss[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mb + 4 * (lane >> 4) + i;
        ss[i] = 0.f;
        if (row < M) {
          const size_t idx = static_cast<size_t>(row) * N + n;
          const float sv = bf16_bits_to_f32(f32_to_bf16_bits(out[p][i])) + bf16_bits_to_f32(res_bits(p, i, idx));
          rs.s_out[idx] = sv;
          rs.res_out[idx] = f32_to_bf16_bits(sv);
          ss[i] = sv * sv;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) ss[i] = row_sum16(ss[i]);
      if (c == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * mb + 4 * (lane >> 4) + i;
          if (row < M) rs.ssq_out[static_cast<size_t>(row) * (N / kTileCols) + tb + tt] = ss[i];
        }
      }
    } else if (!act) {
      const int n = 16 * (tb + tt) + c;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mb + 4 * (lane >> 4) + i;
        if (row < M) {
          const size_t idx = static_cast<size_t>(row) * N + n;
          const uint16_t b = f32_to_bf16_bits(out[p][i]);
          y[idx] = res ? add_bf16(b, res_bits(p, i, idx)) : b;
        }
      }
    } else if constexpr (H > 0) {
      if (tt < H) {
        const int n = 16 * (tb + tt) + c;  // output column of the [M, N / 2] result
        const f32x4_t u = out[p + H < kPairs ? p + H : p];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * mb + 4 * (lane >> 4) + i;
          if (row < M)
            y[static_cast<size_t>(row) * (N >> 1) + n] = f32_to_bf16_bits(silu_mul_of_bf16(out[p][i], u[i]));
        }
      }
    }
  }
}

bool decode_stages_x(int M, int K, int split) {
  const int G = K / kGroup;
  const size_t n_gmax = static_cast<size_t>((G + split - 1) / split);
  // Staging the activations pays for M <= 4 only: measured on MI355X over the Qwen3-8B
  // shapes, staging them for M = 5..16 (up to 128 KiB per workgroup) gave no gain.
  return M <= 4 && n_gmax * M * 256 <= kDecodeMaxStagedX;
}

bool decode_stage_fits(int M, int K, int tn, int waves, int depth, int split, bool ns) {
  const int G = K / kGroup;
  const int items = ((G + split - 1) / split + waves - 1) / waves;
  if (ns && (M > 8 || items > kNormItems)) return false;  // the consumer's lane map: 4 items x 16 chunks
  const bool sz = (tn == 1 && decode_prebuilt_scales(waves, depth))
                      ? items * 16 <= 64 * kStageE
                      : items * tn * 8 <= 64 * kStageS && items * tn * 2 <= 64 * kStageZ;
  return sz && (ns || !decode_stages_x(M, K, split) || items * M * 16 <= 64 * kStageX);
}

size_t decode_lds_bytes(int M, int K, int tn, int waves, int depth, int split, bool ns) {
  return decode_lds_layout(M, K, tn, waves, split, ns || decode_stages_x(M, K, split),
                           decode_prebuilt_scales(waves, depth))
      .total;
}

size_t decode_norm_lds_bytes(int M, int K, int tn, int waves, int depth, int split) {
  const int G = K / kGroup;
  if (M > kNormMaxRows || split != 1 || !decode_stages_x(M, K, split) || (G + waves - 1) / waves > kNormItems)
    return 0;
  return decode_lds_layout(M, K, tn, waves, split, true, decode_prebuilt_scales(waves, depth)).total;
}

constexpr int kMaxDevices = 64;

template <int MB, int TN, int DEPTH, int WAVES, bool XL, int NR = 0, int FN = 0>
static hipError_t launch_decode_t(const DecodeArgs& a, hipStream_t stream) {
  if constexpr (!decode_config_fits(MB, TN, DEPTH, XL)) {
    return hipErrorInvalidValue;  // rejected by the API before launch; not compiled
  } else {
  const dim3 grid(a.N / (kTileCols * TN), a.split);
  constexpr bool kPre = decode_prebuilt_scales(WAVES, DEPTH);
  const size_t lds = decode_lds_layout(a.M, a.K, TN, WAVES, a.split, XL, kPre).total;
  const DecodeGeom geo = decode_geom(a.M, a.K, a.N, TN, WAVES, a.split, XL, kPre);
  if (lds > kDecodeMaxLds || !decode_stage_fits(a.M, a.K, TN, WAVES, DEPTH, a.split, FN > 0) ||
      a.M > (FN > 0 ? FN : FN < 0 ? 8 : 64))
    return hipErrorInvalidValue;  // checked by the API before launch
  if (lds > 64 * 1024) {
    // Dynamic LDS beyond 64 KiB must be allowed per kernel, once per device (a repeated
    // call from a racing thread is harmless).  A failed call returns before the launch: a
    // launch that asks for more LDS than allowed is not rejected by the runtime.
    static std::atomic<bool> raised[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    if (!raised[dev].load(std::memory_order_acquire)) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(decode_kernel<MB, TN, DEPTH, WAVES, XL, NR, FN>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               static_cast<int>(kDecodeMaxLds));
      if (e != hipSuccess) return e;
      raised[dev].store(true, std::memory_order_release);
    }
  }
  decode_kernel<MB, TN, DEPTH, WAVES, XL, NR, FN><<<grid, 64 * WAVES, lds, stream>>>(
      a.x, a.packed, a.qzeros, a.scales, a.y, a.res, a.partials, a.counters, a.M, a.K, a.N, a.split, a.up_tiles,
      geo, a.norm, a.rs);
  return hipGetLastError();
  }
}

template <int MB, int TN, int DEPTH, int WAVES>
static hipError_t launch_decode_x(const DecodeArgs& a, bool norm, hipStream_t stream) {
  if (a.rs.s_out != nullptr) {  // fused-norm producer: the plain plan's kernel with its epilogue, M <= 8
    if constexpr (MB == 1) {
      if (decode_stages_x(a.M, a.K, a.split)) return launch_decode_t<1, TN, DEPTH, WAVES, true, 0, -1>(a, stream);
      return launch_decode_t<1, TN, DEPTH, WAVES, false, 0, -1>(a, stream);
    }
    return hipErrorInvalidValue;  // checked by the API
  }
  if (a.rs.s_in != nullptr) {  // fused-norm consumer: M <= 8, staged rows, at most 8 waves, 2 groups in flight
    if constexpr (MB == 1 && WAVES <= 8 && DEPTH <= 2) {
      // rows held in registers: as few as M allows (the plain kernel's occupancy at M <= 2)
      if (a.M <= 1) return launch_decode_t<1, TN, DEPTH, WAVES, true, 0, 1>(a, stream);
      if (a.M <= 2) return launch_decode_t<1, TN, DEPTH, WAVES, true, 0, 2>(a, stream);
      if (a.M <= 4) return launch_decode_t<1, TN, DEPTH, WAVES, true, 0, 4>(a, stream);
      return launch_decode_t<1, TN, DEPTH, WAVES, true, 0, 8>(a, stream);
    }
    return hipErrorInvalidValue;  // checked by the API
  }
  if constexpr (MB == 1) {
    if (decode_stages_x(a.M, a.K, a.split)) {
      if (norm) {
        if (a.M == 1) return launch_decode_t<MB, TN, DEPTH, WAVES, true, 1>(a, stream);
        if (a.M == 2) return launch_decode_t<MB, TN, DEPTH, WAVES, true, 2>(a, stream);
        return hipErrorInvalidValue;  // M <= kNormMaxRows (checked by the API)
      }
      return launch_decode_t<MB, TN, DEPTH, WAVES, true>(a, stream);
    }
  }
  if (norm) return hipErrorInvalidValue;  // the prologue needs staged rows (checked by the API)
  return launch_decode_t<MB, TN, DEPTH, WAVES, false>(a, stream);
}

template <int MB, int TN, int DEPTH>
static hipError_t launch_decode_w(const DecodeArgs& a, int waves, bool norm, hipStream_t stream) {
  switch (waves) {
    case 4: return launch_decode_x<MB, TN, DEPTH, 4>(a, norm, stream);
    case 12:  // one-tile workgroups only (checked by the API)
      if constexpr (TN == 1) return launch_decode_x<MB, TN, DEPTH, 12>(a, norm, stream);
      return hipErrorInvalidValue;
    default: return launch_decode_x<MB, TN, DEPTH, 8>(a, norm, stream);
  }
}

template <int MB, int TN>
static hipError_t launch_decode_d(const DecodeArgs& a, int depth, int waves, bool norm, hipStream_t stream) {
  switch (depth) {
    case 1: return launch_decode_w<MB, TN, 1>(a, waves, norm, stream);
    case 2: return launch_decode_w<MB, TN, 2>(a, waves, norm, stream);
    default: return launch_decode_w<MB, TN, 4>(a, waves, norm, stream);
  }
}

template <int MB>
static hipError_t launch_decode_m(const DecodeArgs& a, int tn, int depth, int waves, bool norm, hipStream_t stream) {
  switch (tn) {
    case 1: return launch_decode_d<MB, 1>(a, depth, waves, norm, stream);
    case 2: return launch_decode_d<MB, 2>(a, depth, waves, norm, stream);
    case 3: return launch_decode_d<MB, 3>(a, depth, waves, norm, stream);
    case 4: return launch_decode_d<MB, 4>(a, depth, waves, norm, stream);
    default: return launch_decode_d<MB, 6>(a, depth, waves, norm, stream);
  }
}

hipError_t launch_decode_cfg(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                             const uint16_t* scales, uint16_t* y, const uint16_t* res, float* partials,
                             int* counters, int M, int K, int N, int tn, int depth, int waves, int split, int up_tiles,
                             const DecodeNorm* norm, hipStream_t stream, const DecodeRowStats* rs) {
  const DecodeArgs a{rs ? *rs : DecodeRowStats{}, x, packed, qzeros, scales, y, res, partials, counters, M, K, N,
                     split, up_tiles, norm ? *norm : DecodeNorm{}};
  switch ((M + 15) / 16) {
    case 1: return launch_decode_m<1>(a, tn, depth, waves, norm != nullptr, stream);
    case 2: return launch_decode_m<2>(a, tn, depth, waves, norm != nullptr, stream);
    case 3: return launch_decode_m<3>(a, tn, depth, waves, norm != nullptr, stream);
    default: return launch_decode_m<4>(a, tn, depth, waves, norm != nullptr, stream);
  }
}

}  // namespace w4a16
