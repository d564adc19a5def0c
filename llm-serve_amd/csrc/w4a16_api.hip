// extern "C" entry points of libw4a16.so (declared in include/w4a16.h): argument
// validation, kernel choice, workspace layout and thread-local error text.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "../../include/w4a16.h"
#include "w4a16_common.h"
#include "w4a16_launch.h"

// Split-K workspace of w4a16_gemm_noalloc (see scratch_for_current_device below).
constexpr size_t kScratchBytes = size_t(48) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_error[0] = '\0';
  return W4A16_OK;
}

int check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(W4A16_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Whether the byte ranges [a, a + na) and [b, b + nb) share a byte (a null pointer: no range).
bool overlap(const void* a, size_t na, const void* b, size_t nb) {
  if (!a || !b || na == 0 || nb == 0) return false;
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + nb && pb < pa + na;
}

constexpr int kDecodeMaxM = 64;
// The fused RMSNorm across two GEMMs (w4a16_gemm_residual_stats, w4a16_gemm_rmsnorm_stats)
// runs in the decode kernel, whose consumer stages its normalized rows in LDS.  Measured on
// MI355X at the Qwen3-8B shapes, the pair (producer + consumer) beats the residual GEMM
// plus w4a16_gemm_rmsnorm by 0.3 - 3.4 us per norm for M = 2..8; at M = 16 the consumer's
// fp32 row reads (every column block reads all of s) cost more than the norm launch saves.
constexpr int kRowStatsMaxM = 8;
// Both GEMM kernels address their inputs through buffer descriptors with 32-bit byte
// offsets and use offsets >= 2^31 as "fetch nothing".
constexpr size_t kMaxTensorBytes = size_t(1) << 31;

// Kernel configuration for one GEMM problem.
struct GemmPlan {
  int regime;  // w4a16_regime_id
  int p0;      // decode: column tiles per workgroup; tile: wm (16-row tiles per wave)
  int p1;      // decode: waves per workgroup; tile: waves per SIMD the registers allow
  int p2;      // decode: groups in flight per wave; tile: tile shape code (w4a16::tile_shape)
  int split;   // K splits (1 = none)
};

int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Tile regime: rows and columns of the workgroup tile.
int tile_bm(const GemmPlan& p) { return 16 * p.p0 * w4a16::tile_shape(p.p2).nwm; }
int tile_bn(const GemmPlan& p) {
  const w4a16::TileShape t = w4a16::tile_shape(p.p2);
  return 16 * t.tw * t.nwn;
}

// The four Qwen3-8B projections (K x N) the rule sets below were tuned on.
bool tuned_shape(int K, int N) {
  return (K == 4096 && (N == 6144 || N == 4096 || N == 24576)) || (K == 12288 && N == 4096);
}

// Layers at least as large as the tuned ones in both dimensions, other than those four:
// their own rules (decode) and cost model (mid range), from sweeps of the Qwen3-14B and
// Qwen3-32B projections.
bool larger_shape(int K, int N) { return K >= 4096 && N >= 4096 && !tuned_shape(K, N); }

// Layers narrower or shorter than the tuned ones (tensor-parallel shards, small models):
// their own small-grid rules, and a one-round tile cost model above M = 128.
bool smaller_shape(int K, int N) { return N < 4096 || K < 4096; }

// Untuned layers that are very wide (N >= 16384) or long (K >= 8192) also take the larger
// layers' mid-range cost model, and the very wide ones their decode rules (Qwen3-4B gate_up
// 2560 x 19456 and down 9728 x 2560 at M = 32 .. 256: 81.2 / 64.6 us, the best
// configurations, against 89.7 / 76.5 us by the tuned rules; gate_up decode at M = 8 / 16:
// 10.8 / 12.1 against 12.0 / 14.5 us).
bool wide_or_long_shape(int K, int N) { return !tuned_shape(K, N) && (N >= 16384 || K >= 8192); }

// Decode regime, chosen from a sweep of every configuration on MI355X over the Qwen3-8B
// projection shapes (tn 16-column tiles per workgroup, waves, depth = groups in flight per
// wave, split = K splits).  The activation traffic per weight byte falls as tn grows (each
// workgroup reads its K range of x once), the grid shrinks with it, and the exchange of
// split-K partials costs an extra pass over M x N fp32:
//  * wide layers (N >= 16384): 32-column workgroups up to M = 2 (768 for gate_up), 48 up
//    to M = 8, 96 beyond (fewer, wider workgroups: every wave repeats the kernel's scalar
//    set-up, so the grid's wave count is a fixed cost), one group in flight per wave at
//    M > 24 (gate_up+SiLU M = 32: 19.0 against 19.6 us with two, plain 18.4 against 19.7);
//  * medium layers (4096 < N < 16384): 16 columns at M = 1, 32 up to M = 8, then 48 with K
//    in two;
//  * narrow layers (N <= 4096), K < 8192: 16 columns up to M = 16 (one workgroup per CU for
//    N = 4096; 12 waves up to M = 4 -- O M = 1 / 2 / 4: 4.58 / 4.84 / 5.20 us against 4.78 /
//    4.96 / 5.37 us with 8 --, one group each in flight at M = 3, 4 -- O M = 3 / 4: 4.97 /
//    5.05 against 5.13 / 5.19 us with two --, from M = 5 on 4 waves with four groups each in
//    flight), then 64 columns with K in four;
//  * narrow layers below the tuned sizes (the tensor-parallel shards of these layers): fewer
//    than 128 column tiles split K in four from M = 9 on (QKV / 8 = 4096 x 768 at M = 16 /
//    24: 6.0 / 6.4 us against 6.7 / 7.9 us unsplit), fewer than 16 groups stay unsplit in
//    one-tile workgroups of 4 waves (O / 8 = 512 x 4096 at M = 24: 3.9 against 7.2 us);
//    no workgroup has more waves than groups, nor a wave a deeper ring than its groups;
//  * narrow layers with long K: 16 columns at M = 1 (12 waves, four groups each in flight:
//    down 8.3 - 8.6 us against 8.7 - 8.9 us with 8), 32 with K in two up to M = 8 (down
//    M = 4: 9.96 us against 10.27 us with K in four), then 64 columns with K in four.
GemmPlan plan_decode(int M, int K, int N) {
  const int G = K / w4a16::kGroup;
  const int MB = (M + 15) / 16;
  const int T = N / 16;
  int tn = 2, waves = 8, depth = 2, split = 1;
  if (larger_shape(K, N) || (N >= 16384 && wide_or_long_shape(K, N))) {
    // K split s0 so that a workgroup covers more than 4096 of K (K = 8192 unsplit, 17408 and
    // 25600 in four).  Very wide (>= 1024 column tiles) or long-K (s0 >= 4) layers: 32
    // columns and one group in flight up to M = 8, then 64 columns (K split twice as often
    // for long K; 4 waves above M = 16 on wide ones).  Others: 32 columns at M = 1, then 64
    // where that still gives >= 160 workgroups (else 32), 4 waves for 32 columns at
    // 8 < M <= 16 (64 columns with K in two for K >= 8192), and 64 columns with one group
    // in flight beyond.  Sweeps of the Qwen3-14B and -32B projections (QKV 5120 x 7168 /
    // 10240, O 5120 x 5120 / 8192 x 5120, gate_up 5120 x 34816 / 51200, down 17408 / 25600
    // x 5120) at M = 1, 4, 8, 16, 24: within 0.9 % / 1.6 % of the best configurations in
    // total (331.0 / 414.0 against 377.5 / 437.8 us for the rules of the tuned shapes).
    int s0 = 1;
    while (K / (2 * s0) > 4096) s0 *= 2;
    const bool wide = T >= 1024, longk = s0 >= 4;
    const int tn_m = T / 4 >= 160 ? 4 : 2;
    split = s0;
    if (wide || longk) {
      depth = 1;
      if (M <= 8) tn = 2;
      else if (M > 16 && wide) { tn = 4; waves = 4; split = (G >= 32 ? 2 : 1) * s0; }  // 4B gate_up M = 24: 16.8 / 18.7 us
      else { tn = 4; split = wide ? s0 : 2 * s0; }
    } else if (M <= 1) {
      tn = 2;
    } else if (M <= 8) {
      tn = tn_m;
    } else if (M <= 16) {
      tn = tn_m;
      if (tn_m == 2 && K >= 8192) { tn = 4; split = 2 * s0; }  // O 8192 x 5120: 11.4 against 14.0 us
      else if (tn_m == 2) waves = 4;
    } else {
      tn = 4;
      depth = 1;
      if (tn_m == 2) split = 2 * s0;
    }
  } else if (N >= 16384) {
    if (M <= 2) tn = 2;
    else if (M <= 8) tn = 3;
    else if (M <= 24) tn = 6;
    else { tn = 6; depth = 1; }
  } else if (N > 4096) {
    if (M <= 1) tn = 1;
    else if (M <= 8) tn = 2;
    else { tn = 3; depth = 1; split = 2; if (M > 32) waves = 4; }
  } else if (K < 8192) {
    if (M <= 4) { tn = 1; waves = 12; if (M > 2) depth = 1; }
    else if (M <= 16) { tn = 1; waves = 4; depth = 4; }
    else { tn = 4; depth = 1; split = 4; }
    // Narrow layers smaller than the tuned shapes (tensor-parallel shards and the like):
    // fewer than 128 column tiles split K in four from M = 9 on, so that the grid still
    // covers the CUs; fewer than 16 groups keep one-tile workgroups of 4 waves unsplit.
    if (M > 8 && T < 128 && G >= 16) { tn = 1; waves = 4; depth = 2; split = 4; }
    else if (M > 16 && G < 16) { tn = 1; waves = 4; depth = 2; split = 1; }
  } else {
    if (M <= 1) { tn = 1; depth = 4; waves = 12; }
    else if (M <= 8) { tn = 2; split = 2; }
    else { tn = 4; depth = 1; split = 4; if (M > 32) waves = 4; }
  }
  if (split > G) split = G;
  // No more waves than a workgroup has groups (at least one per SIMD), and no deeper ring
  // than a wave has groups.
  const int per_wg = ceil_div(G, split);
  while (waves > 4 && waves > per_wg) waves -= 4;
  while (depth > 1 && depth > ceil_div(per_wg, waves)) depth /= 2;
  const bool xl = w4a16::decode_stages_x(M, K, split);
  // Other shapes: the widest tile count <= tn that divides N / 16 and fits the registers.
  while (depth > 1 && !w4a16::decode_config_fits(MB, tn, depth, xl)) depth /= 2;
  while (tn > 1 && (T % tn != 0 || tn == 5 || !w4a16::decode_config_fits(MB, tn, depth, xl))) --tn;
  // Very long K: split it until the staged operands of a workgroup fit in LDS and a wave's
  // staging loads fit its registers.
  while ((w4a16::decode_lds_bytes(M, K, tn, waves, depth, split) > w4a16::kDecodeMaxLds ||
          !w4a16::decode_stage_fits(M, K, tn, waves, depth, split)) &&
         split < G)
    split = split * 2 > G ? G : split * 2;
  return GemmPlan{W4A16_REGIME_DECODE, tn, waves, depth, split};
}

// Tile plans for layers narrower (N < 4096) or shorter (K < 4096) than the shapes the rules
// below were tuned on -- tensor-parallel shards and small models -- from a cost model: one
// round of workgroups takes alpha + beta * K / 1024 us per tile (least-squares fits over
// sweeps of the Qwen3-8B layers split eight ways, 4096 x 768, 512 x 4096, 4096 x 3072 and
// 1536 x 4096, at M = 160 .. 2048; every fit within 6 %), and a plan costs its rounds of 256
// workgroups times that.  Over those sweeps the model's choice is within 1 % of the best
// configuration at M > 128 (533.9 against 628.8 us in total for the rules below) where its
// grid has at least 144 workgroups; below that, K split over the same tile fills the grid
// (QKV / 8 at M = 160 .. 320: 8.7 - 9.4 us, within 1 % of the best configuration).  Used up
// to M = 2048 (beyond M = 1024 for widths below 4096 only: wider layers fill rounds with the
// rules' 384- and 512-column tiles, which the model leaves out -- Qwen3-4B QKV 2560 x 6144
// at M = 2048: 58.8 us on 128 x 384 tiles against 69.6 us on the model's 64 x 96).
struct ModelTile {
  int wm, shape, occ, bm, bn;
  double alpha, beta;
};
constexpr ModelTile kModelTiles[] = {
    {8, 3, 2, 128, 256, 8.97, 12.05}, {6, 3, 2, 96, 256, 5.67, 10.31}, {4, 3, 2, 64, 256, 5.23, 8.05},
    {8, 5, 2, 128, 128, 6.10, 6.87},  {4, 10, 3, 64, 192, 5.39, 6.22}, {4, 5, 2, 64, 128, 4.58, 4.68},
    {4, 9, 3, 64, 96, 5.33, 3.69},    {4, 4, 2, 64, 64, 4.69, 2.80},   {2, 5, 2, 32, 128, 3.87, 3.42},
    {2, 9, 3, 32, 96, 4.46, 2.58},    {2, 4, 2, 32, 64, 4.00, 1.85}};


// The cheapest modelled tile; when its grid has fewer than 144 workgroups, K split in powers
// of two (at least 8 groups per split) while the grid stays within one round (QKV / 8 at
// M = 352: 132 workgroups unsplit 11.1 us, 264 split in two 15.1 us).
GemmPlan model_tile(int M, int K, int N) {
  const int G = K / w4a16::kGroup;
  const ModelTile* best = nullptr;
  double best_cost = 0.0;
  int best_grid = 0;
  for (const ModelTile& c : kModelTiles) {
    const int t = ceil_div(M, c.bm) * ceil_div(N, c.bn);
    const double cost = ceil_div(t, 256) * (c.alpha + c.beta * K / 1024.0);
    if (!best || cost < best_cost - 1e-9) best = &c, best_cost = cost, best_grid = t;
  }
  int split = 1;
  while (best_grid * split < 144 && best_grid * split * 2 <= 256 && G / (2 * split) >= 8) split *= 2;
  return GemmPlan{W4A16_REGIME_TILE, best->wm, best->occ, best->shape, split};
}

// Mid-range (M <= 256) plans for layers larger than the tuned ones: every modelled tile with
// K split s in {1, 2, 3, 4, 6, 8} (at least 4 groups per split), costed as its rounds of 256
// workgroups times alpha + beta * K / s / 1024, plus for s > 1 the exchange of partials,
// (-0.31 + 0.59 A + 0.19 (s - 1) A) us per round for A = the tile's area / 4096 (least
// squares over every split configuration of the Qwen3-14B and tensor-parallel sweeps).  On
// the Qwen3-14B sweep at M = 32 .. 256 it comes within 3.6 % of the best configuration in
// total (740.7 against 715.2 us), where the tuned rules took 897.0 us.
GemmPlan model_tile_split(int M, int K, int N) {
  const int G = K / w4a16::kGroup;
  const ModelTile* best = nullptr;
  int best_split = 1;
  double best_cost = 0.0;
  for (const ModelTile& c : kModelTiles) {
    for (int sp : {1, 2, 3, 4, 6, 8}) {
      if (G / sp < 4) continue;
      const int t = ceil_div(M, c.bm) * ceil_div(N, c.bn) * sp;
      const double rounds = ceil_div(t, 256);
      const double area = c.bm * c.bn / 4096.0;
      double cost = rounds * (c.alpha + c.beta * K / (1024.0 * sp));
      if (sp > 1) cost += rounds * (-0.31 + 0.59 * area + 0.19 * (sp - 1) * area);
      if (!best || cost < best_cost - 1e-9) best = &c, best_split = sp, best_cost = cost;
    }
  }
  return GemmPlan{W4A16_REGIME_TILE, best->wm, best->occ, best->shape, best_split};
}

// Tile regime, chosen from sweeps of every tile configuration on MI355X over the Qwen3-8B
// shapes at M = 32 .. 2048.  Wave layouts (w4a16::tile_shape): shape 3 = 8 waves side by side
// along N (32 columns each), one workgroup per CU; shape 1 = 4 waves (64 columns each), two
// workgroups per CU; shapes 4 and 5 = 8 waves as 4 K slices x 2 along N (64 columns) or 2 K
// slices x 4 along N (128 columns), the slices summed through LDS.
//
// Up to M = 256 (the mid range: speculative-verify and small mixed batches, the 36-layer
// stack's batched decode steps) narrow column blocks with the K split over the waves of a
// workgroup keep the grid at one round of 144 .. 256 workgroups with little or no split-K
// exchange between workgroups; short rows blocks (32 rows) re-dequantize the weights per
// row block but read each activation stage once per 64 columns:
//  * wide layers (N >= 16384): 64-row tiles of 128 columns up to M = 64, then 128-row
//    tiles of 128 columns, then (M > 128) 96- or 128-row tiles of 256 columns, K not split;
//  * long K (>= 8192): 32-row tiles up to M = 64 (64 columns up to M = 32, then 128),
//    then 64 rows of 128 columns, K split until the grid has 144 workgroups;
//  * otherwise 32-row tiles of 64 columns up to M = 64 (up to M = 128 for N <= 4096), then
//    64-row tiles (128 columns above M = 128 when N > 4096); K split in powers of two only
//    until the grid has 144 workgroups, with >= 8 groups per split.
// Measured against the best of every configuration at M = 32, 48, 64, 96, 128, 192, 256: within
// 6 % at every point, 1.6 % in total (e.g. O M=128: 12.9 us, from 20.5 us with the 64-row
// tiles of 256 columns used before; QKV M=64: 12.7 vs 16.1 us for the decode kernel).
GemmPlan plan_mid(int M, int K, int N) {
  const int G = K / w4a16::kGroup;
  if (larger_shape(K, N) || wide_or_long_shape(K, N)) return model_tile_split(M, K, N);
  if (M > 128 && N < 16384 && smaller_shape(K, N)) {
    return model_tile(M, K, N);
  }
  // Layers whose width is a multiple of 96 columns (QKV: 6144) above M = 64: 12-wave
  // workgroups of 96 columns (shape 9: 4 K slices x 3 waves along N, three waves per SIMD),
  // 32-row tiles up to M = 128 and 64-row tiles beyond, when that grid has >= 192
  // workgroups (QKV M = 72 .. 128: 16.4 - 16.5 us against 17.9 - 18.1 us; M = 176 .. 256:
  // 22.9 - 23.2 against 24.7 - 24.9 us).
  // Above M = 128, 32-row tiles while they fill one round: of 128 columns on QKV-width layers
  // (shape 5; QKV M = 160: 19.0 us against 22.9 us for 64 x 96 tiles), of 96 columns on
  // narrow ones (shape 9; O M = 160: 16.4 against 17.9 us for 64 x 64 tiles) -- 64-row tiles
  // would compute 192 rows for 160.
  // Both need a grid of 192 .. 256 workgroups; where both qualify (narrow layers whose width
  // is a multiple of 96, such as gate_up / 8 = 4096 x 3072) the larger grid wins (M = 256:
  // 15.0 against 17.5 us).
  if (N < 16384 && K < 8192 && M > 128) {
    const int t5 = N % 96 == 0 ? ceil_div(M, 32) * ceil_div(N, 128) : 0;
    const int t9 = N <= 4096 ? ceil_div(M, 32) * ceil_div(N, 96) : 0;
    const bool ok5 = t5 >= 192 && t5 <= 256, ok9 = t9 >= 192 && t9 <= 256;
    if (ok9 && (!ok5 || t9 > t5)) return GemmPlan{W4A16_REGIME_TILE, 2, 3, 9, 1};
    if (ok5) return GemmPlan{W4A16_REGIME_TILE, 2, 2, 5, 1};
  }
  if (N < 16384 && K < 8192 && N % 96 == 0 && M > 64) {
    const int wm9 = M <= 128 ? 2 : 4;
    if (ceil_div(M, 16 * wm9) * (N / 96) >= 192) return GemmPlan{W4A16_REGIME_TILE, wm9, 3, 9, 1};
  }
  int wm, shape, split = 1;
  // Wide layers at 64 < M <= 128: 12-wave workgroups of 64 rows x 192 columns (shape 10:
  // 2 K slices x 6 waves along N, three waves per SIMD), one round of 256 workgroups for
  // gate_up (34.2 - 35.6 us against 37.9 - 39.2 us for 128 x 128 tiles on 192 workgroups).
  if (N >= 16384 && M > 64 && M <= 128 && N % 192 == 0) return GemmPlan{W4A16_REGIME_TILE, 4, 3, 10, 1};
  // Wide layers above M = 128: 96 x 256 tiles while they fill one round (gate_up M = 160 /
  // 192: 51.1 / 52.1 us against 60.7 / 61.3 us for 128 x 256 tiles, which compute 256 rows).
  if (N >= 16384 && M > 128 && ceil_div(M, 96) * ceil_div(N, 256) <= 256) return GemmPlan{W4A16_REGIME_TILE, 6, 2, 3, 1};
  // Wide layers up to M = 64: 12-wave workgroups of 96 columns (shape 9: 4 K slices x 3 waves
  // along N), one round of 256 workgroups for gate_up, 32-row tiles up to M = 32 and 64-row
  // ones beyond (gate_up M = 32 / 48 / 64: 16.9 / 21.0 / 21.4 us against 18.9 / 23.6 / 24.0 us
  // for 128-column tiles of 2 K slices).
  if (N >= 16384 && M <= 64 && N % 96 == 0) return GemmPlan{W4A16_REGIME_TILE, M <= 32 ? 2 : 4, 3, 9, 1};
  if (N >= 16384) {
    if (M <= 64) { wm = 4; shape = 5; }
    else { wm = 8; shape = M <= 128 ? 5 : 3; }
  } else if (K >= 8192) {
    // 64-row tiles from M = 33 up to M = 256 (down M = 48 / 64: 16.4 / 17.4 us in 4 K slices
    // against 17.7 / 17.7 us for two 32-row blocks; M = 160 / 192: 37.0 / 37.3 us against
    // 37.6 / 38.3 us with 128-row tiles split in four)
    wm = M <= 32 ? 2 : 4;
    shape = M <= 64 ? 4 : 5;
  } else {
    wm = (M <= 64 || (M <= 128 && N <= 4096)) ? 2 : 4;
    shape = (M > 128 && N > 4096) ? 5 : 4;
    // Layers smaller than the tuned shapes: 32-row tiles when 64-row ones leave fewer than
    // 144 workgroups (QKV / 8 = 4096 x 768 at M = 256: 9.3 against 10.8 us, K split in two
    // instead of four).
    if (wm == 4 && ceil_div(M, 64) * ceil_div(N, 16 * w4a16::tile_shape(shape).tw * w4a16::tile_shape(shape).nwn) < 144)
      wm = 2;
  }
  const w4a16::TileShape ts = w4a16::tile_shape(shape);
  int tiles = ceil_div(M, 16 * wm * ts.nwm) * ceil_div(N, 16 * ts.tw * ts.nwn);
  if (N < 16384)
    while (tiles * split < 144 && G / (2 * split) >= 8) split *= 2;
  // Still fewer than 144 workgroups (few columns, or K too short to split): 32-column
  // workgroups of four K slices, four waves (shape 7) double the grid (O / 8 = 512 x 4096
  // at M = 32 / 64: 4.4 against 4.9 us; down / 8 = 1536 x 4096: 6.2 against 7.1 / 6.9 us;
  // QKV / 8 at M = 32 / 64: 7.6 / 7.9 against 8.0 / 8.1 us with K in four).
  if (K < 8192 && N < 16384 && shape == 4 && tiles * split < 144) return GemmPlan{W4A16_REGIME_TILE, wm, 1, 7, split};
  return GemmPlan{W4A16_REGIME_TILE, wm, 2, shape, split};
}

// Tile candidates of the fill score below: rows x columns of one workgroup's tile, and the
// measured efficiency of the tile relative to 128 x 512 tiles (the same work in 128 x 256,
// 96 x 512, 96 x 256 and 128 x 128 tiles takes 1 / 0.955, 1 / 0.91, 1 / 0.87 and 1 / 0.73
// the time).  Wide layers choose among the first four; narrow layers, whose 512-column
// tiles leave too few workgroups, among 256 and 128 columns.
struct TileCand {
  int wm, shape, bm, bn;
  double eff;
};
constexpr TileCand kWideTiles[] = {{8, 8, 128, 512, 1.0}, {8, 3, 128, 256, 0.955}, {6, 8, 96, 512, 0.91}, {6, 3, 96, 256, 0.87}};
constexpr TileCand kNarrowTiles[] = {{8, 3, 128, 256, 0.955}, {6, 3, 96, 256, 0.87}, {8, 5, 128, 128, 0.73}};
// Plain GEMMs on narrow widths that are multiples of 384 also weigh 384-column tiles (shape
// 11: 128 x 384 at 0.93, 96 x 384 at 0.89 of 128 x 512); on these layers (QKV) 128 x 256
// tiles measure 0.86 (M = 4096: 198.0 against 184.5 us for 128 x 384 at full rounds).
constexpr TileCand kNarrow384Tiles[] = {{8, 8, 128, 512, 1.0}, {8, 11, 128, 384, 0.93}, {6, 8, 96, 512, 0.91},
                                        {6, 11, 96, 384, 0.89}, {6, 3, 96, 256, 0.87}, {8, 3, 128, 256, 0.86}};

// Wide layers whose width is a multiple of 384 columns, for 256 < M <= 1024: 128 / 96 rows x
// 512 / 384 / 256 columns, with efficiencies from whole rounds of the gate_up shape relative
// to a 128 x 512 round (111 us at M = 2048): 128 x 384 0.94 (M = 1536 / 1024 / 512: 260 /
// 181 / 90 us), 96 x 384 0.855 (M = 768 / 384: 146.5 / 72.8 us), 128 x 256 0.907 (M = 960:
// 183.7 us), 96 x 256 0.815 (M = 768: 153.4 us).
constexpr TileCand kWide384Tiles[] = {{8, 8, 128, 512, 1.0},    {8, 11, 128, 384, 0.94}, {6, 8, 96, 512, 0.91},
                                      {6, 11, 96, 384, 0.855}, {8, 3, 128, 256, 0.907}, {6, 3, 96, 256, 0.815}};

// The candidate that does the most useful work per round of 256 workgroups: its efficiency
// times the M x N outputs over the rows x columns its rounds compute, so that rows padded
// past M count against a tile (96-row tiles of a short chunk waste less than 128-row ones).
// Ties go to the earlier tile.
template <size_t C>
GemmPlan most_useful_tile(int M, int N, const TileCand (&cands)[C]) {
  const TileCand* best = &cands[0];
  double best_score = 0.0;
  for (const TileCand& c : cands) {
    const int t = ceil_div(M, c.bm) * ceil_div(N, c.bn);
    const double score = c.eff * M * N / (ceil_div(t, 256) * 256.0 * c.bm * c.bn);
    if (score > best_score + 1e-9) best = &c, best_score = score;
  }
  return GemmPlan{W4A16_REGIME_TILE, best->wm, 2, best->shape, 1};
}

// The candidate whose grid fills its last round of 256 workgroups best, weighted by its
// efficiency; ties go to the earlier (larger) tile.  Regime NONE when no candidate fills
// half its last round.
template <size_t C>
GemmPlan best_filling_tile(int M, int N, const TileCand (&cands)[C]) {
  const TileCand* best = nullptr;
  double best_score = 0.0;
  for (const TileCand& c : cands) {
    const int t = ceil_div(M, c.bm) * ceil_div(N, c.bn);
    const double score = c.eff * t / (ceil_div(t, 256) * 256.0);
    if (score > best_score + 1e-9) best = &c, best_score = score;
  }
  if (best_score < 0.5) return GemmPlan{W4A16_REGIME_NONE, 0, 0, 0, 1};
  return GemmPlan{W4A16_REGIME_TILE, best->wm, 2, best->shape, 1};
}

// 256 < M <= 1024 (chunked-prefill chunks and mixed batches).  Wide layers: below M = 384,
// 64-row tiles of 256 columns, two workgroups per CU (shape 1); from M = 384 on, the
// best-filling wide tile (fused gate_up M = 384 / 448 / 512 / 640 / 768 / 896: 87.7 / 94.9 /
// 106.5 / 116.8 / 161.6 / 186.6 us against 106.4 / 108.0 / 115.4 / 146.7 / 174.8 / 189.3 us
// with 64-row tiles up to M = 768 and 128 x 256 beyond).  Narrow layers above M = 512: 96 x
// 256 tiles with K split in two where that grid fills one round (O / down M = 640: 34.1 /
// 78.9 us against 37.7 / 99.5 us), 128 x 256 tiles with K split in two for long K where
// that grid fills three quarters of a round or more (down M = 832 / 1024: 96.0 / 102.1
// against 100.2 / 105.3 us), else the best-filling narrow tile (QKV M = 704 / 896 / 960:
// 49.8 / 52.3 / 52.6 against 54.4 / 56.3 / 57.5 us), except that QKV-width layers keep 64 x
// 384 tiles when 128 x 256 tiles would fill more than half a round and 96-row tiles do not
// win.  Up to M = 512: 128-row tiles unless they leave too few workgroups: 256 columns
// (shape 3) when that grid alone has >= 144 workgroups, else 128 columns (shape 5, 2 K
// slices), K split in two or more for long K while the grid is below 144 workgroups;
// short-K narrow layers switch to 64-row tiles of 128 columns instead of splitting K.  From
// sweeps of every tile configuration at M = 320 ... 1024.  `fused`: narrow layers leave out
// the 384-column tiles (their fused form pairs waves; measured on wide layers only).
GemmPlan plan_large(int M, int K, int N, bool fused) {
  const int G = K / w4a16::kGroup;
  if (N < 16384 && smaller_shape(K, N)) {
    return model_tile(M, K, N);
  }
  // Plain GEMMs on widths that are multiples of 384 columns: 128 x 384 tiles (shape 11, 8
  // waves of 48) where they fill one round on wide layers (gate_up M = 384 / 512: 86.6 / 96.1
  // us against 104.0 / 112.6 us), 64 x 384 tiles on QKV-width layers once 128 x 256 tiles
  // would fill a round (QKV M = 768 / 1024: 54.7 / 59.4 us against 60.5 / 61.1 us).
  const bool w384 = !fused && N % 384 == 0;
  // Wide layers of such widths, the fused product too (its 384-column waves pair gate and up
  // waves), by useful work per round (gate_up M = 288 / 384 / 672 / 768 / 864 / 960: 66.5 /
  // 72.8 / 135.0 / 146.5 / 163.1 / 174.2 us against 79.9 / 81.2 / 145.9 / 153.4 / 175.6 /
  // 183.7 us by round fill; the fused gate_up M = 384 / 512 / 768 / 1024: 73.0 / 90.0 /
  // 147.3 / 179.3 against 83.7 / 101.5 / 152.9 / 188.3 us).
  if (N >= 16384 && N % 384 == 0) return most_useful_tile(M, N, kWide384Tiles);
  // Narrow layers just above M = 256: 64-row tiles, five row blocks (320 rows computed
  // instead of three 128-row blocks' 384), the width chosen for a grid of 192 .. 256: long K
  // 64 x 192 tiles with K in two (down M = 272 / 320: 46.9 / 47.0 against 51.3 / 51.5 us),
  // else 64 x 128 (QKV M = 272 / 320: 24.2 / 24.8 against 32.8 / 33.1 us) or 64 x 96 tiles
  // (O: 20.1 / 20.5 against 23.1 / 23.0 us).  Above that, for short K, 64 x 192 tiles while
  // their grid fills 192 .. 255 workgroups of a round (QKV M = 336 .. 448: 30.3 / 32.2 against
  // 33.6 / 33.7 us at M = 384 / 448; O M = 513 .. 704: 29.5 / 31.3 against 31.3 / 35.0 us at
  // M = 528 / 704), then 128 x 128 tiles while theirs fills 192 .. 256 (O M = 736 / 768: 33.7 /
  // 33.8 against 34.7 / 35.2 us).
  if (N < 16384 && M <= 320) {
    const int mb = ceil_div(M, 64);
    if (K >= 8192 && mb * ceil_div(N, 192) * 2 <= 256) return GemmPlan{W4A16_REGIME_TILE, 4, 3, 10, 2};
    if (K < 8192 && N % 128 == 0 && mb * (N / 128) >= 192 && mb * (N / 128) <= 256)
      return GemmPlan{W4A16_REGIME_TILE, 4, 2, 5, 1};
    if (K < 8192 && mb * ceil_div(N, 96) >= 192 && mb * ceil_div(N, 96) <= 256)
      return GemmPlan{W4A16_REGIME_TILE, 4, 3, 9, 1};
  }
  if (N < 16384 && K < 8192) {
    const int t10 = ceil_div(M, 64) * ceil_div(N, 192);
    if (t10 >= 192 && t10 < 256) return GemmPlan{W4A16_REGIME_TILE, 4, 3, 10, 1};
    const int t5 = ceil_div(M, 128) * ceil_div(N, 128);
    if (t5 >= 192 && t5 <= 256) return GemmPlan{W4A16_REGIME_TILE, 8, 2, 5, 1};
  }
  if (N >= 16384 && M < 384) return GemmPlan{W4A16_REGIME_TILE, 4, 2, 1, 1};
  if (N >= 16384) {
    const GemmPlan p = best_filling_tile(M, N, kWideTiles);
    if (p.regime == W4A16_REGIME_TILE) return p;
  }
  const int t3 = ceil_div(M, 128) * ceil_div(N, 256);
  if (N < 16384 && M > 512) {
    if (ceil_div(M, 96) * ceil_div(N, 256) * 2 <= 256 && G >= 32) return GemmPlan{W4A16_REGIME_TILE, 6, 2, 3, 2};
    if (K >= 8192 && t3 * 2 >= 192 && t3 * 2 <= 256) return GemmPlan{W4A16_REGIME_TILE, 8, 2, 3, 2};
    const GemmPlan p = best_filling_tile(M, N, kNarrowTiles);
    if (p.regime == W4A16_REGIME_TILE) return w384 && t3 >= 144 && p.p0 != 6 ? GemmPlan{W4A16_REGIME_TILE, 4, 2, 11, 1} : p;
  }
  if (t3 >= 144 && N < 16384 && w384) return GemmPlan{W4A16_REGIME_TILE, 4, 2, 11, 1};
  if (t3 >= 144) return GemmPlan{W4A16_REGIME_TILE, 8, 2, 3, 1};
  const int t5 = ceil_div(M, 128) * ceil_div(N, 128);
  if (t5 >= 144) return GemmPlan{W4A16_REGIME_TILE, 8, 2, 5, 1};
  int split = 1;
  if (K >= 8192) {
    while (t5 * split < 144 && G / (2 * split) >= 16) split *= 2;
    return GemmPlan{W4A16_REGIME_TILE, 8, 2, 5, split};
  }
  const int t4 = ceil_div(M, 64) * ceil_div(N, 128);
  while (t4 * split < 144 && G / (2 * split) >= 8) split *= 2;
  return GemmPlan{W4A16_REGIME_TILE, 4, 2, 5, split};
}

// Beyond M = 1024 (whole prefill chunks): 128 x 512 tiles (shape 8: 8 waves of 128 x 64)
// on wide layers from four rounds of workgroups on -- every activation row is then re-read
// from L2 by half as many workgroups as with 256 columns (gate_up M=2048: 4.7 % faster,
// bit-identical); else the best-filling of four tile sizes (below); for small grids, K split
// in two or four over 128 x 256 tiles, or 64-row tiles of 256 columns, two workgroups per
// CU (shape 1).  Split-K partials are reduced by the last workgroup of each tile.
GemmPlan plan_tile(int M, int K, int N, bool fused) {
  if (M <= 256) return plan_mid(M, K, N);
  if (M <= 1024) return plan_large(M, K, N, fused);
  const int G = K / w4a16::kGroup;
  if (M <= 2048 && N < 4096 && smaller_shape(K, N)) {
    return model_tile(M, K, N);
  }
  // Plain GEMMs on widths that are multiples of 384 columns: on narrow layers the best-filling
  // of the 384-, 512- and 256-column tiles of 96 or 128 rows (QKV M = 1536 / 2048 / 3072 on
  // 384-column tiles: 76.8 / 95.4 / 151.0 us against 85.9 / 110.6 / 171.9 us; M = 5120 /
  // 8192 on 128 x 512 tiles: 220.4 / 339.2 us against 275.6 / 365.4 us on 384 columns); on
  // wide ones 128 x 384 tiles where they fill two or three rounds (gate_up M = 1536: 277.8
  // against 301.7 us).
  const int t11 = ceil_div(M, 128) * (N / 384);
  if (!fused && N % 384 == 0 && N < 16384) {
    const GemmPlan p = best_filling_tile(M, N, kNarrow384Tiles);
    if (p.regime == W4A16_REGIME_TILE) return p;
  }
  if (N % 384 == 0 && N >= 16384 && t11 % 256 == 0 && t11 < 1024) return GemmPlan{W4A16_REGIME_TILE, 8, 2, 11, 1};
  const int t9 = ceil_div(M, 128) * ceil_div(N, 512);
  if (N >= 16384 && t9 >= 1024) return GemmPlan{W4A16_REGIME_TILE, 8, 2, 8, 1};
  // Otherwise the best-filling tile (above).  From sweeps at M = 1280 ... 4096: O and down
  // at M = 1280 / 2304 / 3584 50.9 / 88.0 / 110.0 and 140.6 / 249.8 / 310.0 us against 60.8
  // / 104.7 / 136.4 and 169.5 / 297.6 / 389.2 us with 128-row tiles only; the fused gate_up
  // at M = 1280 / 1536 / 1792 222.8 / 280.3 / 326.4 against 268.7 / 301.5 / 369.5 us.
  const GemmPlan best = best_filling_tile(M, N, kWideTiles);
  if (best.regime == W4A16_REGIME_TILE) return best;
  // Small grids: K split in two or four over 128 x 256 tiles, or 64-row tiles.
  const int t8 = ceil_div(M, 128) * ceil_div(N, 256);
  int s8 = 1;
  while (s8 < 4 && t8 * s8 * 2 <= 256 && 16 * s8 * 2 <= G) s8 *= 2;
  if (t8 * s8 >= 144 && t8 * s8 <= 256) return GemmPlan{W4A16_REGIME_TILE, 8, 2, 3, s8};
  return GemmPlan{W4A16_REGIME_TILE, 4, 2, 1, 1};
}

// Regime: the decode kernel below M = 32, the tile kernel from M = 32 on, where its 32-row
// tiles beat the decode kernel on every Qwen3-8B shape (M = 32: QKV 9.80 / 9.87, O 8.90 /
// 9.04, gate_up 16.88 / 17.63, down 13.29 / 13.72 us; M = 48: gate_up 21.02 / 22.50 us).
GemmPlan plan(int M, int K, int N, bool fused = false) {
  if (M == 0) return GemmPlan{W4A16_REGIME_NONE, 0, 0, 0, 1};
  if (M >= 32) return plan_tile(M, K, N, fused);
  return plan_decode(M, K, N);
}

// The fused SiLU(gate) * up product of a gate|up weight [K, N] runs the plain GEMM's plan,
// except where the pairing of gate and up values constrains it: narrow layers leave out
// the 384-column tiles (with three tiles per wave the product pairs gate and up waves, which
// the wide layers' rules take), and in the decode regime an odd tile count tn becomes 2 tn
// (measured best for tn = 3 at M = 3..8), or the largest even count below that divides
// N / 16 and fits the registers (the LDS check may then split K further).
GemmPlan plan_silu_mul(int M, int K, int N) {
  GemmPlan p = plan(M, K, N, true);
  if (p.regime != W4A16_REGIME_DECODE || p.p0 % 2 == 0) return p;
  const int G = K / w4a16::kGroup;
  const int MB = (M + 15) / 16;
  const int T = N / 16;
  const bool xl = w4a16::decode_stages_x(M, K, p.split);
  int tn = 2 * p.p0;
  while (tn > 2 && (T % tn != 0 || !w4a16::decode_config_fits(MB, tn, 1, xl))) tn -= 2;
  while (p.p2 > 1 && !w4a16::decode_config_fits(MB, tn, p.p2, xl)) p.p2 /= 2;
  p.p0 = tn;
  if (p.p1 == 12) p.p1 = 8;  // 12-wave workgroups hold one column tile
  while ((w4a16::decode_lds_bytes(M, K, tn, p.p1, p.p2, p.split) > w4a16::kDecodeMaxLds ||
          !w4a16::decode_stage_fits(M, K, tn, p.p1, p.p2, p.split)) &&
         p.split < G)
    p.split = p.split * 2 > G ? G : p.split * 2;
  return p;
}

// Workspace layout: [arrival counters: kCounterBytes][fp32 partials: split * M * N].
// The counters sit at a fixed offset so that a workspace shared by calls of different
// shapes always presents zeroed counters (every kernel re-arms the ones it used).
constexpr size_t kCounterBytes = 64 * 1024;
constexpr size_t kMaxCounters = kCounterBytes / sizeof(int);

size_t counters_needed(const GemmPlan& p, int M, int N) {
  if (p.regime == W4A16_REGIME_DECODE) return static_cast<size_t>(N / 16);
  return static_cast<size_t>(ceil_div(M, tile_bm(p))) * ceil_div(N, tile_bn(p));
}

// fp32 partial tiles: split x (M padded to the kernel's row block) x (N padded to its
// column block), stored as lane-major 16-byte fragments.
size_t partial_bytes(const GemmPlan& p, int M, int N) {
  if (p.regime == W4A16_REGIME_DECODE)
    return static_cast<size_t>(p.split) * (16 * ceil_div(M, 16)) * N * sizeof(float);
  const int bm = tile_bm(p), bn = tile_bn(p);
  return static_cast<size_t>(p.split) * (bm * ceil_div(M, bm)) * (bn * ceil_div(N, bn)) * sizeof(float);
}

// The consumer of the fused RMSNorm statistics (w4a16_gemm_rmsnorm_stats, M <= 8) runs the
// plain (or SiLU * up) decode plan with its normalized rows staged in LDS: at most 8 waves
// and two groups in flight per wave (the compiled consumer kernels), and K split further
// where the staged rows exceed LDS or a wave would hold more than four groups.
GemmPlan plan_norm_stats(int M, int K, int N, bool silu_mul) {
  GemmPlan p = silu_mul ? plan_silu_mul(M, K, N) : plan(M, K, N);
  if (p.regime != W4A16_REGIME_DECODE) return p;
  const int G = K / w4a16::kGroup;
  if (p.p1 > 8) p.p1 = 8;
  if (p.p2 > 2) p.p2 = 2;
  while ((w4a16::decode_lds_bytes(M, K, p.p0, p.p1, p.p2, p.split, true) > w4a16::kDecodeMaxLds ||
          !w4a16::decode_stage_fits(M, K, p.p0, p.p1, p.p2, p.split, true)) &&
         p.split < G)
    p.split = p.split * 2 > G ? G : p.split * 2;
  return p;
}

size_t workspace_for(const GemmPlan& p, int M, int N) {
  if (p.regime == W4A16_REGIME_NONE || p.split <= 1) return 0;
  return kCounterBytes + partial_bytes(p, M, N);
}

int validate_gemm(const void* x, const void* packed, const void* qzeros, const void* scales, const void* y, int M,
                  int K, int N, int group_size, bool silu_mul = false) {
  if (M < 0 || K <= 0 || N <= 0) return fail(W4A16_ERR_ARG, "M must be >= 0 and K, N positive (got M=%d K=%d N=%d)", M, K, N);
  if (group_size != w4a16::kGroup)
    return fail(W4A16_ERR_SHAPE, "group_size must be 128 (got %d)", group_size);
  if (K % w4a16::kGroup) return fail(W4A16_ERR_SHAPE, "K must be divisible by 128 (got %d)", K);
  if (N % 64) return fail(W4A16_ERR_SHAPE, "N must be divisible by 64 (got %d)", N);
  if (silu_mul && N % 128)
    return fail(W4A16_ERR_SHAPE, "the gate|up width N must be divisible by 128 (got %d)", N);
  if (static_cast<size_t>(K) * N / 2 >= kMaxTensorBytes)
    return fail(W4A16_ERR_SHAPE, "packed weights of K=%d N=%d exceed 2 GiB", K, N);
  if (static_cast<size_t>(M) * K * 2 >= kMaxTensorBytes && M <= kDecodeMaxM)
    return fail(W4A16_ERR_SHAPE, "activations of M=%d K=%d exceed 2 GiB", M, K);
  if (M == 0) return ok();
  if (!x || !packed || !qzeros || !scales || !y) return fail(W4A16_ERR_ARG, "null tensor pointer");
  if (!aligned(x, 16) || !aligned(packed, 16) || !aligned(y, 16))
    return fail(W4A16_ERR_ALIGN, "x, packed qweight and y must be 16-byte aligned");
  if (!aligned(qzeros, 4) || !aligned(scales, 4))
    return fail(W4A16_ERR_ALIGN, "qzeros and scales must be 4-byte aligned");
  return ok();
}

// Every check a planned GEMM can fail on after argument validation: workspace size and
// alignment, partial and counter limits of a K split, and the tile kernel's row chunks.
// Callers run it before enqueueing anything, so a failing call leaves no work behind.
int check_plan(const GemmPlan& p, int M, int K, int N, const void* workspace, size_t workspace_bytes) {
  if (p.regime == W4A16_REGIME_NONE) return ok();
  const size_t need = workspace_for(p, M, N);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(W4A16_ERR_WORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if (need > 0 && !aligned(workspace, 256)) return fail(W4A16_ERR_ALIGN, "workspace must be 256-byte aligned");
  if (need > 0 && partial_bytes(p, M, N) >= kMaxTensorBytes)
    return fail(W4A16_ERR_SHAPE, "split-K partials of %zu bytes exceed 2 GiB", partial_bytes(p, M, N));
  if (need > 0 && counters_needed(p, M, N) > kMaxCounters)
    return fail(W4A16_ERR_SHAPE, "split-K needs %zu arrival counters (limit %zu)", counters_needed(p, M, N),
                kMaxCounters);
  if (p.regime == W4A16_REGIME_TILE && (kMaxTensorBytes - 1) / (2 * static_cast<size_t>(K)) < static_cast<size_t>(tile_bm(p)))
    return fail(W4A16_ERR_SHAPE, "K=%d is too long for one %d-row tile below 2 GiB", K, tile_bm(p));
  return ok();
}

// up_tiles: 0 for the plain GEMM, N / 32 for the fused SiLU(gate) * up (y is [M, N / 2]).
// res: null, or a bf16 [M, N] residual added in the epilogue (plain GEMM; may be y).
// norm: the decode kernel's RMSNorm prologue (decode regime with staged rows only), or null.
int run_plan(const GemmPlan& p, const uint16_t* x, const int32_t* packed, const int32_t* qzeros,
             const uint16_t* scales, uint16_t* y, int M, int K, int N, void* workspace, size_t workspace_bytes,
             hipStream_t stream, int up_tiles = 0, const uint16_t* res = nullptr,
             const w4a16::DecodeNorm* norm = nullptr, const w4a16::DecodeRowStats* rs = nullptr) {
  if (p.regime == W4A16_REGIME_NONE) return ok();
  const int c = check_plan(p, M, K, N, workspace, workspace_bytes);
  if (c != W4A16_OK) return c;
  const size_t need = workspace_for(p, M, N);
  int* counters = need ? static_cast<int*>(workspace) : nullptr;
  float* partials = need ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes) : nullptr;
  const uint32_t* pk = reinterpret_cast<const uint32_t*>(packed);
  const uint32_t* qz = reinterpret_cast<const uint32_t*>(qzeros);
  if (p.regime == W4A16_REGIME_DECODE)
    return check_launch(w4a16::launch_decode_cfg(x, pk, qz, scales, y, res, partials, counters, M, K, N, p.p0,
                                                 p.p2, p.p1, p.split, up_tiles, norm, stream, rs),
                        "decode");
  // The tile kernel addresses the activations through a buffer descriptor (32-bit byte
  // offsets, >= 2^31 meaning "fetch nothing"): rows go in chunks of < 2 GiB of activations,
  // one launch each, in order on the stream (each launch re-arms the counters it used).
  const int bm = tile_bm(p);
  const size_t n_out = up_tiles ? N / 2 : N;
  const size_t fit = (kMaxTensorBytes - 1) / (2 * static_cast<size_t>(K));
  const int chunk = fit >= static_cast<size_t>(M) ? M : static_cast<int>(fit / bm) * bm;  // > 0: check_plan
  for (int r0 = 0; r0 < M; r0 += chunk) {
    const int mc = M - r0 < chunk ? M - r0 : chunk;
    const int rc = check_launch(w4a16::launch_tile_cfg(x + static_cast<size_t>(r0) * K, pk, qz, scales,
                                                       y + static_cast<size_t>(r0) * n_out,
                                                       res ? res + static_cast<size_t>(r0) * N : nullptr, partials,
                                                       counters, mc, K, N, p.p0, p.p2, p.p1, p.split, up_tiles, stream),
                                "tile");
    if (rc != W4A16_OK) return rc;
  }
  return ok();
}

// Arguments of the residual-add + RMSNorm prologue (w4a16_add_rmsnorm, w4a16_gemm_rmsnorm).
int validate_norm(const void* x, const void* residual, const void* weight, float eps, const void* x_norm,
                  const void* residual_out, int M, int K) {
  if (M < 0 || K <= 0) return fail(W4A16_ERR_ARG, "M must be >= 0 and K positive (got M=%d K=%d)", M, K);
  if (K % 8 || K > w4a16::kNormMaxK)
    return fail(W4A16_ERR_SHAPE, "the RMSNorm width K must be a multiple of 8 and at most %d (got %d)",
                w4a16::kNormMaxK, K);
  if (!(eps >= 0.0f) || eps > 1.0f) return fail(W4A16_ERR_ARG, "eps must be in [0, 1] (got %g)", eps);
  if (!x || !weight || !x_norm) return fail(W4A16_ERR_ARG, "null tensor pointer");
  if ((residual == nullptr) != (residual_out == nullptr))
    return fail(W4A16_ERR_ARG, "residual and residual_out must both be given or both be null");
  if (residual_out && residual_out == x_norm)
    return fail(W4A16_ERR_ARG, "x_norm and residual_out must be different buffers");
  if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(x_norm, 16) || !aligned(residual, 16) ||
      !aligned(residual_out, 16))
    return fail(W4A16_ERR_ALIGN, "x, residual, weight, x_norm and residual_out must be 16-byte aligned");
  return ok();
}

// ---------------------------------------------------------------------------
// Library-owned split-K workspace of w4a16_gemm_noalloc, for callers that cannot allocate
// device memory.  `scratch` is a device array of the code object: each GPU the library
// runs on holds its own copy, at its own address, until the process ends.  In host code the
// name is only a stand-in for the symbol; its device address comes from hipGetSymbolAddress
// on each device (with that device current) and is the only thing host code passes on.
// Layout as any workspace: arrival counters in the first kCounterBytes, then fp32 partials.
// The counters start at zero (cleared once per device on first use by a fill kernel on the
// caller's stream) and every kernel re-arms the ones it used; calls that overlap on one GPU
// share the array and race.
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kScratchDevices];  // per device; null until set up

__global__ void clear_words(uint32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// Device address of the current device's scratch, set up on the first call on that device
// (symbol lookup, then the counters cleared on `stream`).  Returns a W4A16 status.
int scratch_for_current_device(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices)
    return fail(W4A16_ERR_LAUNCH, "no current HIP device (or device index >= %d)", kScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    // The clear must run now: captured into a graph, it would only run at the graph's
    // replays, and eager calls before that would find the counters uncleared.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const hipError_t ce = hipStreamIsCapturing(stream, &cap);
    if (ce != hipSuccess || cap != hipStreamCaptureStatusNone)
      return fail(W4A16_ERR_LAUNCH,
                  "the first w4a16_gemm_noalloc call on device %d sets up the library scratch and must not be "
                  "captured into a graph: make one call outside capture first",
                  dev);
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(W4A16_ERR_LAUNCH, "hipGetSymbolAddress of the library scratch failed on device %d: %s", dev,
                  hipGetErrorString(e));
    // hipLaunchKernel returns this launch's own status (hipGetLastError after a <<<>>> launch
    // would also report an earlier, unrelated error of the thread).
    uint32_t* words = static_cast<uint32_t*>(ptr);
    int n_words = static_cast<int>(kCounterBytes / 4);
    void* args[] = {&words, &n_words};
    const hipError_t le =
        hipLaunchKernel(reinterpret_cast<const void*>(clear_words), dim3(16), dim3(256), args, 0, stream);
    if (le != hipSuccess)
      return fail(W4A16_ERR_LAUNCH, "clearing the library scratch failed on device %d: %s", dev, hipGetErrorString(le));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return ok();
}

}  // namespace

extern "C" {

int w4a16_gemm_noalloc(const uint16_t* x, const int32_t* packed, const int32_t* qzeros, const uint16_t* scales,
                       uint16_t* y, int M, int K, int N, int group_size, void* stream) {
  const int v = validate_gemm(x, packed, qzeros, scales, y, M, K, N, group_size);
  if (v != W4A16_OK) return v;
  if (M == 0) return ok();
  const GemmPlan p = plan(M, K, N);
  const size_t need = workspace_for(p, M, N);
  if (need > kScratchBytes)
    return fail(W4A16_ERR_WORKSPACE,
                "M=%d K=%d N=%d needs %zu bytes of split-K workspace; w4a16_gemm_noalloc holds %zu (use w4a16_gemm "
                "with a caller workspace)",
                M, K, N, need, kScratchBytes);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if (need > 0) {
    const int r = scratch_for_current_device(s, &ws);
    if (r != W4A16_OK) return r;
  }
  return run_plan(p, x, packed, qzeros, scales, y, M, K, N, ws, need > 0 ? kScratchBytes : 0, s);
}

int w4a16_add_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, float eps,
                      uint16_t* x_norm, uint16_t* residual_out, int M, int K, void* stream) {
  const int v = validate_norm(x, residual, weight, eps, x_norm, residual_out, M, K);
  if (v != W4A16_OK) return v;
  if (M == 0) return ok();
  return check_launch(w4a16::launch_add_rmsnorm(x, residual, weight, x_norm, residual_out, M, K, eps,
                                                static_cast<hipStream_t>(stream)),
                      "add_rmsnorm");
}

int w4a16_rmsnorm_strided(const uint16_t* x, int rows_inner, int64_t stride_outer, int64_t stride_inner,
                          const uint16_t* weight, float eps, uint16_t* x_norm, int M, int K, void* stream) {
  int v = validate_norm(x, nullptr, weight, eps, x_norm, nullptr, M, K);
  if (v != W4A16_OK) return v;
  if (M == 0) return ok();
  if (rows_inner <= 0 || stride_outer < 0 || stride_inner < 0)
    return fail(W4A16_ERR_ARG, "rows_inner must be positive and the strides non-negative");
  if (stride_outer % 8 || stride_inner % 8)
    return fail(W4A16_ERR_ALIGN, "row strides must be multiples of 8 elements (16 bytes)");
  const int64_t last = static_cast<int64_t>((M - 1) / rows_inner) * stride_outer +
                       static_cast<int64_t>((M - 1) % rows_inner) * stride_inner + K;
  if (last >= (int64_t(1) << 40)) return fail(W4A16_ERR_SHAPE, "strided rows span too far");
  return check_launch(w4a16::launch_rmsnorm_strided(x, rows_inner, stride_outer, stride_inner, weight, x_norm, M, K,
                                                    eps, static_cast<hipStream_t>(stream)),
                      "rmsnorm_strided");
}

int w4a16_gemm_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* norm_weight, float eps,
                       uint16_t* x_norm, uint16_t* residual_out, const int32_t* packed, const int32_t* qzeros,
                       const uint16_t* scales, uint16_t* y, int M, int K, int N, int group_size, int silu_mul,
                       void* workspace, size_t workspace_bytes, void* stream) {
  int v = validate_norm(x, residual, norm_weight, eps, x_norm, residual_out, M, K);
  if (v != W4A16_OK) return v;
  if (silu_mul != 0 && silu_mul != 1) return fail(W4A16_ERR_ARG, "silu_mul must be 0 or 1 (got %d)", silu_mul);
  v = validate_gemm(x_norm, packed, qzeros, scales, y, M, K, N, group_size, silu_mul != 0);
  if (v != W4A16_OK) return v;
  if (M == 0) return ok();
  // y is written while the inputs and the norm's outputs are still being read (by other
  // workgroups, or by the GEMM that follows the norm kernel): it must overlap none of them.
  const size_t row_bytes = static_cast<size_t>(M) * K * 2;
  const size_t y_bytes = static_cast<size_t>(M) * (silu_mul ? N / 2 : N) * 2;
  if (overlap(y, y_bytes, x, row_bytes) || overlap(y, y_bytes, residual, row_bytes) ||
      overlap(y, y_bytes, x_norm, row_bytes) || overlap(y, y_bytes, residual_out, row_bytes))
    return fail(W4A16_ERR_ARG, "y must not overlap x, residual, x_norm or residual_out");
  // Every check that could fail the GEMM runs before the prologue is enqueued.
  GemmPlan p = silu_mul ? plan_silu_mul(M, K, N) : plan(M, K, N);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int up_tiles = silu_mul ? N / 32 : 0;
  // A decode plan with M <= 2 rows staged in LDS, no K split and at most 4 groups per wave
  // (M = 1, 2 at the Qwen3-8B QKV and gate|up shapes) takes the norm as a prologue of the
  // GEMM kernel: one launch, and x_norm is written once by the first workgroup, never read
  // back.  Its outputs must not overlap the inputs (other workgroups still read x and
  // residual while the first one writes).
  const bool disjoint = !overlap(x_norm, row_bytes, x, row_bytes) && !overlap(x_norm, row_bytes, residual, row_bytes) &&
                        !overlap(residual_out, row_bytes, x, row_bytes) &&
                        !overlap(residual_out, row_bytes, residual, row_bytes);
  if (p.regime == W4A16_REGIME_DECODE && disjoint) {
    // With the norm as a prologue every workgroup repeats it, so one-tile 8-wave plans at
    // M = 1 take two tiles per workgroup when they divide N (half the workgroups: QKV 7.23
    // against 7.44 us).
    GemmPlan q = p;
    if (M == 1 && q.p0 == 1 && q.p1 == 8 && (N / 16) % 2 == 0 &&
        w4a16::decode_config_fits(1, 2, q.p2, w4a16::decode_stages_x(M, K, q.split)) &&
        w4a16::decode_stage_fits(M, K, 2, q.p1, q.p2, q.split) &&
        w4a16::decode_norm_lds_bytes(M, K, 2, q.p1, q.p2, q.split) > 0)
      q.p0 = 2;
    const size_t lds = w4a16::decode_norm_lds_bytes(M, K, q.p0, q.p1, q.p2, q.split);
    if (lds > 0 && lds <= w4a16::kDecodeMaxLds) {
      v = check_plan(q, M, K, N, workspace, workspace_bytes);
      if (v != W4A16_OK) return v;
      const w4a16::DecodeNorm nrm{residual, norm_weight, residual_out, x_norm, eps};
      return run_plan(q, x, packed, qzeros, scales, y, M, K, N, workspace, workspace_bytes, s, up_tiles, nullptr,
                      &nrm);
    }
  }
  v = check_plan(p, M, K, N, workspace, workspace_bytes);
  if (v != W4A16_OK) return v;
  // Otherwise the norm kernel writes x_norm and the GEMM reads it back (from L2 at decode sizes).
  v = check_launch(w4a16::launch_add_rmsnorm(x, residual, norm_weight, x_norm, residual_out, M, K, eps, s),
                   "add_rmsnorm");
  if (v != W4A16_OK) return v;
  return run_plan(p, x_norm, packed, qzeros, scales, y, M, K, N, workspace, workspace_bytes, s, up_tiles);
}

int w4a16_abi_version(void) { return W4A16_ABI_VERSION; }

const char* w4a16_last_error(void) { return g_error; }

int w4a16_unpack_int4(const int32_t* packed, int32_t* out, int rows, int cols, void* stream) {
  if (rows <= 0 || cols <= 0) return fail(W4A16_ERR_ARG, "rows and cols must be positive");
  if (!packed || !out) return fail(W4A16_ERR_ARG, "null tensor pointer");
  if (!aligned(packed, 4) || !aligned(out, 16)) return fail(W4A16_ERR_ALIGN, "out must be 16-byte aligned");
  return check_launch(w4a16::launch_unpack(reinterpret_cast<const uint32_t*>(packed), out, rows, cols,
                                           static_cast<hipStream_t>(stream)),
                      "unpack");
}

int w4a16_dequant(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales, uint16_t* w_out, int K,
                  int N, int group_size, void* stream) {
  if (K <= 0 || N <= 0) return fail(W4A16_ERR_ARG, "K and N must be positive");
  if (group_size <= 0) return fail(W4A16_ERR_SHAPE, "group_size must be positive");
  if (K % group_size) return fail(W4A16_ERR_SHAPE, "K must be divisible by group_size");
  if (N % 8) return fail(W4A16_ERR_SHAPE, "N must be divisible by 8");
  if (!qweight || !qzeros || !scales || !w_out) return fail(W4A16_ERR_ARG, "null tensor pointer");
  if (!aligned(scales, 16) || !aligned(w_out, 16) || !aligned(qweight, 4) || !aligned(qzeros, 4))
    return fail(W4A16_ERR_ALIGN, "scales and w_out must be 16-byte aligned");
  return check_launch(w4a16::launch_dequant(reinterpret_cast<const uint32_t*>(qweight),
                                            reinterpret_cast<const uint32_t*>(qzeros), scales, w_out, K, N,
                                            group_size, static_cast<hipStream_t>(stream)),
                      "dequant");
}

int w4a16_repack_qweight(const int32_t* qweight, int32_t* packed, int K, int N, void* stream) {
  if (K <= 0 || N <= 0) return fail(W4A16_ERR_ARG, "K and N must be positive");
  if (K % w4a16::kGroup) return fail(W4A16_ERR_SHAPE, "K must be divisible by 128 (got %d)", K);
  if (N % 16) return fail(W4A16_ERR_SHAPE, "N must be divisible by 16 (got %d)", N);
  if (!qweight || !packed) return fail(W4A16_ERR_ARG, "null tensor pointer");
  if (!aligned(qweight, 4) || !aligned(packed, 16)) return fail(W4A16_ERR_ALIGN, "packed must be 16-byte aligned");
  return check_launch(w4a16::launch_repack(reinterpret_cast<const uint32_t*>(qweight),
                                           reinterpret_cast<uint32_t*>(packed), K, N,
                                           static_cast<hipStream_t>(stream)),
                      "repack");
}

int w4a16_dequant_packed(const int32_t* packed, const int32_t* qzeros, const uint16_t* scales, uint16_t* w_out,
                         int K, int N, int group_size, void* stream) {
  if (K <= 0 || N <= 0) return fail(W4A16_ERR_ARG, "K and N must be positive");
  if (group_size != w4a16::kGroup) return fail(W4A16_ERR_SHAPE, "group_size must be 128 (got %d)", group_size);
  if (K % w4a16::kGroup) return fail(W4A16_ERR_SHAPE, "K must be divisible by 128 (got %d)", K);
  if (N % 16) return fail(W4A16_ERR_SHAPE, "N must be divisible by 16 (got %d)", N);
  if (!packed || !qzeros || !scales || !w_out) return fail(W4A16_ERR_ARG, "null tensor pointer");
  if (!aligned(packed, 16) || !aligned(w_out, 2) || !aligned(scales, 4) || !aligned(qzeros, 4))
    return fail(W4A16_ERR_ALIGN, "packed must be 16-byte and scales, qzeros 4-byte aligned");
  return check_launch(w4a16::launch_dequant_packed(reinterpret_cast<const uint32_t*>(packed),
                                                   reinterpret_cast<const uint32_t*>(qzeros), scales, w_out, K, N,
                                                   static_cast<hipStream_t>(stream)),
                      "dequant_packed");
}

int w4a16_quantize(const void* weight, int dtype, int32_t* qweight, int32_t* qzeros, void* scales,
                   int out_features, int in_features, int group_size, void* stream) {
  static_assert(W4A16_DTYPE_BF16 == w4a16::kDtypeBF16 && W4A16_DTYPE_F16 == w4a16::kDtypeF16 &&
                    W4A16_DTYPE_F32 == w4a16::kDtypeF32,
                "dtype codes");
  if (out_features <= 0 || in_features <= 0) return fail(W4A16_ERR_ARG, "out_features and in_features must be positive");
  if (dtype != W4A16_DTYPE_BF16 && dtype != W4A16_DTYPE_F16 && dtype != W4A16_DTYPE_F32)
    return fail(W4A16_ERR_ARG, "unknown weight dtype %d", dtype);
  if (group_size < 1 || group_size > 128)
    return fail(W4A16_ERR_SHAPE, "group_size must be in [1, 128] (got %d)", group_size);
  if (in_features % group_size) return fail(W4A16_ERR_SHAPE, "input size must be divisible by group_size");
  if (out_features % 8) return fail(W4A16_ERR_SHAPE, "output size must be divisible by 8");
  if (in_features / group_size > 65535) return fail(W4A16_ERR_SHAPE, "more than 65535 groups per row");
  if (!weight || !qweight || !qzeros || !scales) return fail(W4A16_ERR_ARG, "null tensor pointer");
  const size_t elem = dtype == W4A16_DTYPE_F32 ? 4 : 2;
  if (!aligned(weight, elem) || !aligned(scales, elem) || !aligned(qweight, 4) || !aligned(qzeros, 4))
    return fail(W4A16_ERR_ALIGN, "weight and scales must be aligned to their element size");
  return check_launch(w4a16::launch_quantize(weight, dtype, reinterpret_cast<uint32_t*>(qweight),
                                             reinterpret_cast<uint32_t*>(qzeros), scales, out_features,
                                             in_features, group_size, static_cast<hipStream_t>(stream)),
                      "quantize");
}

int w4a16_pack_int4(const int32_t* values, int32_t* packed, int rows, int cols, void* stream) {
  if (rows <= 0 || cols <= 0) return fail(W4A16_ERR_ARG, "rows and cols must be positive");
  if (cols % 8) return fail(W4A16_ERR_SHAPE, "INT4 packing requires the output dimension to be divisible by 8");
  if (!values || !packed) return fail(W4A16_ERR_ARG, "null tensor pointer");
  if (!aligned(values, 16) || !aligned(packed, 4)) return fail(W4A16_ERR_ALIGN, "values must be 16-byte aligned");
  return check_launch(w4a16::launch_pack_int4(values, reinterpret_cast<uint32_t*>(packed), rows, cols,
                                              static_cast<hipStream_t>(stream)),
                      "pack_int4");
}

size_t w4a16_workspace_bytes(int M, int K, int N, int group_size) {
  if (M <= 0 || K <= 0 || N <= 0 || group_size != w4a16::kGroup || K % w4a16::kGroup || N % 64) return 0;
  // the largest of every entry point's plan at this shape: plain, SiLU * up and, below
  // M = 32, the fused RMSNorm consumer's variants of both
  size_t most = workspace_for(plan(M, K, N), M, N);
  const auto take = [&](const GemmPlan& q) {
    const size_t b = workspace_for(q, M, N);
    most = b > most ? b : most;
  };
  if (N % 128 == 0) take(plan_silu_mul(M, K, N));
  if (M <= kRowStatsMaxM) {
    take(plan_norm_stats(M, K, N, false));
    if (N % 128 == 0) take(plan_norm_stats(M, K, N, true));
  }
  return most;
}

// The maximum runs the planner at every M <= M_max; a model asks for it once per layer with
// the same few shapes, so recent answers are kept (a small table, replaced round-robin).
size_t w4a16_workspace_bytes_max(int M_max, int K, int N, int group_size) {
  struct Entry {
    int m_max, k, n, group;
    size_t bytes;
  };
  static std::mutex mu;
  static Entry cache[16];
  static int used = 0, next = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < used; ++i)
      if (cache[i].m_max == M_max && cache[i].k == K && cache[i].n == N && cache[i].group == group_size)
        return cache[i].bytes;
  }
  size_t most = 0;
  for (int m = 1; m <= M_max; ++m) {
    const size_t b = w4a16_workspace_bytes(m, K, N, group_size);
    most = b > most ? b : most;
  }
  std::lock_guard<std::mutex> lock(mu);
  cache[next] = Entry{M_max, K, N, group_size, most};
  next = (next + 1) % 16;
  used = used < 16 ? used + 1 : 16;
  return most;
}

int w4a16_regime(int M, int K, int N) {
  if (M < 0 || K <= 0 || N <= 0) return W4A16_REGIME_NONE;
  return plan(M, K, N).regime;
}

int w4a16_split_k(int M, int K, int N) {
  if (M <= 0 || K <= 0 || N <= 0 || K % w4a16::kGroup) return 1;
  return plan(M, K, N).split;
}

int w4a16_plan(int M, int K, int N, int entry, int* out) {
  if (!out) return fail(W4A16_ERR_ARG, "null output pointer");
  if (M <= 0 || K <= 0 || N <= 0 || K % w4a16::kGroup || N % 64)
    return fail(W4A16_ERR_SHAPE, "no plan for M=%d K=%d N=%d", M, K, N);
  if (entry < 0 || entry > 4) return fail(W4A16_ERR_ARG, "entry must be 0..4 (got %d)", entry);
  if (entry == 4 && M > kDecodeMaxM) return fail(W4A16_ERR_SHAPE, "decode kernel needs M <= 64 (got %d)", M);
  if (entry & 1 && N % 128) return fail(W4A16_ERR_SHAPE, "the gate|up width N must be divisible by 128 (got %d)", N);
  if ((entry == 2 || entry == 3) && M > kRowStatsMaxM)
    return fail(W4A16_ERR_SHAPE, "the fused RMSNorm statistics take M <= %d (got %d)", kRowStatsMaxM, M);
  const GemmPlan p = entry == 0   ? plan(M, K, N)
                     : entry == 1 ? plan_silu_mul(M, K, N)
                     : entry == 4 ? plan_decode(M, K, N)
                                  : plan_norm_stats(M, K, N, entry == 3);
  out[0] = p.regime;
  out[1] = p.p0;
  out[2] = p.p1;
  out[3] = p.p2;
  out[4] = p.split;
  return ok();
}

int w4a16_gemm(const uint16_t* x, const int32_t* packed, const int32_t* qzeros, const uint16_t* scales, uint16_t* y,
               int M, int K, int N, int group_size, void* workspace, size_t workspace_bytes, void* stream) {
  const int v = validate_gemm(x, packed, qzeros, scales, y, M, K, N, group_size);
  if (v != W4A16_OK) return v;
  return run_plan(plan(M, K, N), x, packed, qzeros, scales, y, M, K, N, workspace, workspace_bytes,
                  static_cast<hipStream_t>(stream));
}

int w4a16_gemm_residual(const uint16_t* x, const int32_t* packed, const int32_t* qzeros, const uint16_t* scales,
                        const uint16_t* residual, uint16_t* y, int M, int K, int N, int group_size, void* workspace,
                        size_t workspace_bytes, void* stream) {
  const int v = validate_gemm(x, packed, qzeros, scales, y, M, K, N, group_size);
  if (v != W4A16_OK) return v;
  if (M == 0) return ok();
  if (!residual) return fail(W4A16_ERR_ARG, "null residual pointer");
  if (!aligned(residual, 16)) return fail(W4A16_ERR_ALIGN, "residual must be 16-byte aligned");
  return run_plan(plan(M, K, N), x, packed, qzeros, scales, y, M, K, N, workspace, workspace_bytes,
                  static_cast<hipStream_t>(stream), 0, residual);
}

int w4a16_gemm_residual_stats(const uint16_t* x, const int32_t* packed, const int32_t* qzeros, const uint16_t* scales,
                              const uint16_t* residual, float* s_out, uint16_t* residual_out, float* ssq_out, int M,
                              int K, int N, int group_size, void* workspace, size_t workspace_bytes, void* stream) {
  const int v = validate_gemm(x, packed, qzeros, scales, residual_out, M, K, N, group_size);
  if (v != W4A16_OK) return v;
  if (M == 0) return ok();
  if (M > kRowStatsMaxM)
    return fail(W4A16_ERR_SHAPE, "the fused RMSNorm statistics take M <= %d (got %d)", kRowStatsMaxM, M);
  if (!residual || !s_out || !ssq_out) return fail(W4A16_ERR_ARG, "null residual, s_out or ssq_out pointer");
  if (!aligned(residual, 16) || !aligned(s_out, 16) || !aligned(ssq_out, 16))
    return fail(W4A16_ERR_ALIGN, "residual, s_out and ssq_out must be 16-byte aligned");
  const size_t rb = static_cast<size_t>(M) * N * 2, sb = static_cast<size_t>(M) * N * 4;
  const size_t qb = static_cast<size_t>(M) * (N / 16) * 4, xb = static_cast<size_t>(M) * K * 2;
  if ((residual_out != residual && overlap(residual_out, rb, residual, rb)) || overlap(s_out, sb, residual, rb) ||
      overlap(s_out, sb, residual_out, rb) || overlap(ssq_out, qb, s_out, sb) || overlap(ssq_out, qb, residual, rb) ||
      overlap(ssq_out, qb, residual_out, rb) || overlap(s_out, sb, x, xb) || overlap(residual_out, rb, x, xb) ||
      overlap(ssq_out, qb, x, xb))
    return fail(W4A16_ERR_ARG, "s_out, residual_out and ssq_out must not overlap each other or the inputs "
                               "(residual_out may be residual itself)");
  const GemmPlan p = plan(M, K, N);  // the decode kernel (M <= 8)
  const w4a16::DecodeRowStats rs{s_out, residual_out, ssq_out, nullptr, nullptr, nullptr, 0.f, nullptr};
  return run_plan(p, x, packed, qzeros, scales, residual_out, M, K, N, workspace, workspace_bytes,
                  static_cast<hipStream_t>(stream), 0, residual, nullptr, &rs);
}

int w4a16_gemm_rmsnorm_stats(const float* s, const float* ssq, const uint16_t* norm_weight, float eps,
                             uint16_t* x_norm, const int32_t* packed, const int32_t* qzeros, const uint16_t* scales,
                             uint16_t* y, int M, int K, int N, int group_size, int silu_mul, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (silu_mul != 0 && silu_mul != 1) return fail(W4A16_ERR_ARG, "silu_mul must be 0 or 1 (got %d)", silu_mul);
  // s is checked as the GEMM input (its alignment); its fp32 rows are 4 K bytes
  const int v = validate_gemm(reinterpret_cast<const uint16_t*>(s), packed, qzeros, scales, y, M, K, N, group_size,
                              silu_mul != 0);
  if (v != W4A16_OK) return v;
  if (M == 0) return ok();
  if (M > kRowStatsMaxM)
    return fail(W4A16_ERR_SHAPE, "the fused RMSNorm statistics take M <= %d (got %d)", kRowStatsMaxM, M);
  if (static_cast<size_t>(M) * K * 4 >= kMaxTensorBytes)
    return fail(W4A16_ERR_SHAPE, "fp32 activations of M=%d K=%d exceed 2 GiB", M, K);
  if (!ssq || !norm_weight) return fail(W4A16_ERR_ARG, "null ssq or norm_weight pointer");
  if (!aligned(ssq, 16) || !aligned(norm_weight, 16) || !aligned(x_norm, 16))
    return fail(W4A16_ERR_ALIGN, "ssq, norm_weight and x_norm must be 16-byte aligned");
  if (!(eps >= 0.0f) || eps > 1.0f) return fail(W4A16_ERR_ARG, "eps must be in [0, 1] (got %g)", eps);
  const size_t yb = static_cast<size_t>(M) * (silu_mul ? N / 2 : N) * 2;
  if (overlap(y, yb, s, static_cast<size_t>(M) * K * 4) || overlap(y, yb, ssq, static_cast<size_t>(M) * (K / 16) * 4) ||
      overlap(y, yb, x_norm, static_cast<size_t>(M) * K * 2) || overlap(y, yb, norm_weight, static_cast<size_t>(K) * 2))
    return fail(W4A16_ERR_ARG, "y must not overlap s, ssq, norm_weight or x_norm");
  const GemmPlan p = plan_norm_stats(M, K, N, silu_mul != 0);
  const int c = check_plan(p, M, K, N, workspace, workspace_bytes);
  if (c != W4A16_OK) return c;
  const w4a16::DecodeRowStats rs{nullptr, nullptr, nullptr, s, ssq, norm_weight, eps, x_norm};
  return run_plan(p, reinterpret_cast<const uint16_t*>(s), packed, qzeros, scales, y, M, K, N, workspace,
                  workspace_bytes, static_cast<hipStream_t>(stream), silu_mul ? N / 32 : 0, nullptr, nullptr, &rs);
}

int w4a16_gemm_silu_mul(const uint16_t* x, const int32_t* packed, const int32_t* qzeros, const uint16_t* scales,
                        uint16_t* y, int M, int K, int N, int group_size, void* workspace, size_t workspace_bytes,
                        void* stream) {
  const int v = validate_gemm(x, packed, qzeros, scales, y, M, K, N, group_size, true);
  if (v != W4A16_OK) return v;
  return run_plan(plan_silu_mul(M, K, N), x, packed, qzeros, scales, y, M, K, N, workspace, workspace_bytes,
                  static_cast<hipStream_t>(stream), N / 32);
}

}  // extern "C"

namespace {

int gemm_config_impl(const uint16_t* x, const int32_t* packed, const int32_t* qzeros, const uint16_t* scales,
                     uint16_t* y, int M, int K, int N, int group_size, int regime, int p0, int p1, int p2, int split,
                     void* workspace, size_t workspace_bytes, void* stream, bool silu_mul) {
  const int v = validate_gemm(x, packed, qzeros, scales, y, M, K, N, group_size, silu_mul);
  if (v != W4A16_OK) return v;
  if (M == 0) return ok();
  const int G = K / w4a16::kGroup;
  GemmPlan p{regime, p0, p1, p2, split};
  if (split < 1 || split > G) return fail(W4A16_ERR_ARG, "split must be in [1, K/128] (got %d)", split);
  if (regime == W4A16_REGIME_DECODE) {
    if (M > kDecodeMaxM) return fail(W4A16_ERR_SHAPE, "decode kernel needs M <= 64 (got %d)", M);
    if (p0 < 1 || p0 > 6 || p0 == 5) return fail(W4A16_ERR_ARG, "decode column tiles must be 1, 2, 3, 4 or 6");
    if ((N / 16) % p0) return fail(W4A16_ERR_SHAPE, "N / 16 = %d is not a multiple of %d column tiles", N / 16, p0);
    if (silu_mul && p0 % 2)
      return fail(W4A16_ERR_ARG, "the fused SiLU * up product needs an even decode column tile count");
    if (p1 != 4 && p1 != 8 && !(p1 == 12 && p0 == 1))
      return fail(W4A16_ERR_ARG, "decode waves must be 4 or 8, or 12 with one column tile");
    if (p2 != 1 && p2 != 2 && p2 != 4) return fail(W4A16_ERR_ARG, "decode depth must be 1, 2 or 4");
    if (w4a16::decode_lds_bytes(M, K, p0, p1, p2, split) > w4a16::kDecodeMaxLds)
      return fail(W4A16_ERR_ARG, "decode configuration needs %zu bytes of LDS (limit %zu)",
                  w4a16::decode_lds_bytes(M, K, p0, p1, p2, split), w4a16::kDecodeMaxLds);
    if (!w4a16::decode_stage_fits(M, K, p0, p1, p2, split))
      return fail(W4A16_ERR_ARG, "decode configuration stages more scale, zero or activation words per wave than "
                  "its registers hold (split K further)");
    if (!w4a16::decode_config_fits((M + 15) / 16, p0, p2, w4a16::decode_stages_x(M, K, split)))
      return fail(W4A16_ERR_ARG, "decode configuration needs %d ring and accumulator registers per lane (limit 176)",
                  w4a16::decode_ring_regs((M + 15) / 16, p0, p2, w4a16::decode_stages_x(M, K, split)));
  } else if (regime == W4A16_REGIME_TILE) {
    if (p0 != 2 && p0 != 4 && p0 != 6 && p0 != 8) return fail(W4A16_ERR_ARG, "tile wm must be 2, 4, 6 or 8");
    if (p2 < 0 || p2 > w4a16::kTileShapeMax)
      return fail(W4A16_ERR_ARG, "tile shape code must be 0..%d", w4a16::kTileShapeMax);
    // The fused product pairs a wave's gate and up tiles (even tile counts) or, with an odd
    // count, two waves of one K slice along N.
    const w4a16::TileShape ts = w4a16::tile_shape(p2);
    const bool paired_waves = silu_mul && ts.tw % 2;
    if (paired_waves && (ts.nwn % 2 || ts.nwm != 1 || ts.wk != 1))
      return fail(W4A16_ERR_ARG, "the fused SiLU * up product cannot pair the waves of tile wave layout %d", p2);
    // A wave's output columns must lie wholly inside or wholly past the output width (true for
    // every layout of 32 or 64 columns per wave whenever N % 64 == 0).
    const int wave_cols = (silu_mul && !paired_waves ? 8 : 16) * ts.tw;
    if ((silu_mul ? N / 2 : N) % wave_cols)
      return fail(W4A16_ERR_SHAPE, "tile wave layout %d needs an output width that is a multiple of %d (got %d)", p2,
                  wave_cols, silu_mul ? N / 2 : N);
    if (p1 < 1 || p1 > 3) return fail(W4A16_ERR_ARG, "tile occupancy must be 1, 2 or 3");
    if (!w4a16::tile_config_compiled(p0, p2, p1))
      return fail(W4A16_ERR_ARG, "tile configuration wm %d, shape %d, occupancy %d is not compiled", p0, p2, p1);
  } else {
    return fail(W4A16_ERR_ARG, "unknown regime %d", regime);
  }
  return run_plan(p, x, packed, qzeros, scales, y, M, K, N, workspace, workspace_bytes,
                  static_cast<hipStream_t>(stream), silu_mul ? N / 32 : 0);
}

}  // namespace

extern "C" {

int w4a16_gemm_config(const uint16_t* x, const int32_t* packed, const int32_t* qzeros, const uint16_t* scales,
                      uint16_t* y, int M, int K, int N, int group_size, int regime, int p0, int p1, int p2,
                      int split, void* workspace, size_t workspace_bytes, void* stream) {
  return gemm_config_impl(x, packed, qzeros, scales, y, M, K, N, group_size, regime, p0, p1, p2, split, workspace,
                          workspace_bytes, stream, false);
}

int w4a16_gemm_silu_mul_config(const uint16_t* x, const int32_t* packed, const int32_t* qzeros,
                               const uint16_t* scales, uint16_t* y, int M, int K, int N, int group_size, int regime,
                               int p0, int p1, int p2, int split, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return gemm_config_impl(x, packed, qzeros, scales, y, M, K, N, group_size, regime, p0, p1, p2, split, workspace,
                          workspace_bytes, stream, true);
}

size_t w4a16_workspace_bytes_config(int M, int N, int regime, int p0, int split) {
  if (M <= 0 || N <= 0) return 0;
  // Tile regime: enough for every tile shape (taller or wider tiles pad more).
  size_t most = workspace_for(GemmPlan{regime, p0, 0, 1, split}, M, N);
  if (regime != W4A16_REGIME_TILE) return most;
  for (int shape = 2; shape <= w4a16::kTileShapeMax; ++shape) {
    const size_t b = workspace_for(GemmPlan{regime, p0, 0, shape, split}, M, N);
    most = b > most ? b : most;
  }
  return most;
}

}  // extern "C"
