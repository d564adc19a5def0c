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

// Split-K decode kernel, M <= 64.  tn in {1, 2, 3, 4} 16-column tiles per workgroup (tn
// divides N / 16), depth in
// {1, 2, 4} groups in flight per wave, waves in {4, 8, 16}, 1 <= split <= K / 128.
// `partials` holds the split-K fp32 fragments and `counters` N / (16 tn) ints (both unused
// when split == 1).
hipError_t launch_decode_cfg(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                             const uint16_t* scales, uint16_t* y, float* partials, int* counters, int M, int K,
                             int N, int tn, int depth, int waves, int split, hipStream_t stream);

// LDS-tiled MFMA GEMM: workgroup tile (16 wm) x 256, wm in {4, 8, 16}; occ in {1, 2} waves
// per SIMD the register allocation targets (wm 16: 1 only).  `partials` holds the split-K
// fp32 fragments and `counters` one int per output tile (both unused when split == 1).
hipError_t launch_tile_cfg(const uint16_t* x, const uint32_t* packed, const uint32_t* qzeros,
                           const uint16_t* scales, uint16_t* y, float* partials, int* counters, int M, int K,
                           int N, int wm, int occ, int split, hipStream_t stream);

}  // namespace w4a16
