/*
 * w4a16.h -- C ABI of the MI355X (gfx950) W4A16 linear library (libw4a16.so).
 *
 * Weight format consumed: AutoAWQ "GEMM" version, 4-bit, zero point, group 128:
 *   qweight int32 [K, N/8]   nibble i of word [k, j] holds column 8j + (0,2,4,6,1,3,5,7)[i]
 *   qzeros  int32 [K/128, N/8] same nibble order
 *   scales  bf16  [K/128, N]
 *   W[k, n] = bf16_rne( (q[k, n] - z[k/128, n]) * s[k/128, n] )
 * Activations x bf16 [M, K] row-major, output y bf16 [M, N] row-major.
 *
 * Conventions
 *   - Every tensor pointer is a device pointer owned by the caller; the library never
 *     allocates.  bf16 data is passed as uint16_t bit patterns.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Calls only enqueue
 *     work; nothing synchronises the host.
 *   - Return 0 on success, otherwise a W4A16_ERR_* code; w4a16_last_error() then gives a
 *     thread-local message.  No C++ exception crosses this boundary.
 *
 * Reference interfaces replaced (HGinkgo/LLM-Serve):
 *   pybind module of llmserve/layers/quantization/csrc/awq_w4a16.cu:375-379
 *     (repack_qweight, reorder_qzeros, linear) and its Python wrappers in
 *     llmserve/layers/quantization/awq_cuda.py:17-185, plus the reference backend
 *     functions of llmserve/layers/quantization/awq.py:184-276.
 */
#ifndef W4A16_H_
#define W4A16_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4A16_ABI_VERSION 5

enum w4a16_status {
  W4A16_OK = 0,
  W4A16_ERR_ARG = 1,       /* null pointer or non-positive size */
  W4A16_ERR_SHAPE = 2,     /* K / N / group contract violated */
  W4A16_ERR_ALIGN = 3,     /* a pointer is not aligned as the kernel requires */
  W4A16_ERR_WORKSPACE = 4, /* workspace missing or smaller than w4a16_workspace_bytes */
  W4A16_ERR_LAUNCH = 5     /* hipGetLastError() reported a launch failure */
};

/* Kernel families reported by w4a16_regime(). */
/* Element type of a float weight given to w4a16_quantize (its scales get the same type). */
enum w4a16_dtype {
  W4A16_DTYPE_BF16 = 0,
  W4A16_DTYPE_F16 = 1,
  W4A16_DTYPE_F32 = 2
};

enum w4a16_regime_id {
  W4A16_REGIME_NONE = 0,   /* M == 0: nothing to launch */
  W4A16_REGIME_DECODE = 1, /* M < 32: split-K, HBM-bound kernel */
  W4A16_REGIME_TILE = 2    /* larger M: LDS-tiled bf16 MFMA GEMM */
};

/* ABI version of the loaded library (W4A16_ABI_VERSION). No reference counterpart. */
int w4a16_abi_version(void);

/* Thread-local text of the last error on this thread ("" if none).
 * Replaces the TORCH_CHECK messages of awq_w4a16.cu:249-334. */
const char* w4a16_last_error(void);

/* Unpack int32 [R, C] AWQ words into int32 [R, 8C] in logical column order.
 * Replaces unpack_awq_int4 (awq.py:184-200).  Requires R, C > 0. */
int w4a16_unpack_int4(const int32_t* packed, int32_t* out, int rows, int cols, void* stream);

/* Dequantize the AutoAWQ tensors into bf16 W [K, N], bit-exact with the reference.
 * Replaces dequantize_awq_gemm (awq.py:235-248).  Any group_size > 0 dividing K; N % 8 == 0. */
int w4a16_dequant(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                  uint16_t* w_out, int K, int N, int group_size, void* stream);

/* Rearrange qweight [K, N/8] into the group-tile layout consumed by w4a16_gemm (same
 * 4-bit values, same byte size K*N/2).  One 1 KiB tile per (128-row group g, 16-column
 * tile t); word [((g*(N/16) + t)*64 + lane)*4 + js] holds, at bit 8h + 4(k/2) + 16(k%2),
 * the value of row 128g + 32js + 8(lane/16) + 4h + lane%4 and column
 * 16t + 4((lane/4)%4) + k, for h = 0..1 and k = 0..3.  K % 128 == 0, N % 16 == 0.
 * Replaces repack_qweight (awq_w4a16.cu:81-109, 256-272) / repack_awq_qweight_cuda
 * (awq_cuda.py:129-132).  qzeros need no reorder: the kernels read them as stored, so
 * reorder_qzeros (awq_w4a16.cu:111-118, 274-286) has no counterpart. */
int w4a16_repack_qweight(const int32_t* qweight, int32_t* packed, int K, int N, void* stream);

/* Dequantize from the repacked layout through the GEMM kernels' matrix-core dequant
 * (same bits as w4a16_dequant for every finite scale with |s| < 2^123, zero signs aside);
 * exists to verify that path bit-exactly.  K % 128 == 0, N % 16 == 0.  No reference
 * counterpart beyond dequantize_awq_gemm (awq.py:235-248). */
int w4a16_dequant_packed(const int32_t* packed, const int32_t* qzeros, const uint16_t* scales,
                         uint16_t* w_out, int K, int N, int group_size, void* stream);

/* Group-wise asymmetric int4 quantization of weight [out_features, in_features] (row-major,
 * element type dtype) into the AutoAWQ GEMM layout: qweight [in_features, out_features/8],
 * qzeros [in_features/group_size, out_features/8] (int32), scales
 * [in_features/group_size, out_features] of type dtype.  Per (output row, group):
 * s = max(max - min, 1e-5) / 15, z = clamp(-round(min / s), 0, 15),
 * q = clamp(round(w / s) + z, 0, 15) in fp32, round half to even -- bit-exact with the
 * reference for finite weights.  out_features % 8 == 0, 1 <= group_size <= 128 dividing
 * in_features, in_features / group_size <= 65535; weight 2- or 4-byte aligned by type.
 * Replaces quantize_awq_weight (awq_calibration.py:35-62). */
int w4a16_quantize(const void* weight, int dtype, int32_t* qweight, int32_t* qzeros, void* scales,
                   int out_features, int in_features, int group_size, void* stream);

/* Pack int32 values [rows, cols] (cols % 8 == 0; each value's low 4 bits) into AutoAWQ words
 * [rows, cols/8]: nibble i of word [r, j] holds column 8j + (0,2,4,6,1,3,5,7)[i].  values
 * 16-byte aligned.  Range checks on the values stay with the caller.
 * Replaces _pack_int4 (awq_calibration.py:19-32). */
int w4a16_pack_int4(const int32_t* values, int32_t* packed, int rows, int cols, void* stream);

/* Bytes of workspace w4a16_gemm needs for this problem (0 = none), and, when N % 128 == 0,
 * w4a16_gemm_silu_mul too (the larger of the two).  The workspace must be
 * zero-filled once when first allocated; the kernels leave its counter words at zero.
 * Two GEMMs in flight at the same time must not share one workspace.
 * Replaces the workspace sizing of awq.py:168-180 and awq_cuda.py:157-176. */
size_t w4a16_workspace_bytes(int M, int K, int N, int group_size);

/* The largest w4a16_workspace_bytes(M, K, N, group_size) over 1 <= M <= M_max: one buffer of
 * this size, allocated and zero-filled at load time, serves every call with M <= M_max at
 * this shape (e.g. M_max = the engine's max_num_batched_tokens, 16384 by default), so the
 * GEMM calls never allocate.  0 for M_max < 1 or an invalid shape.
 * Replaces the load-time workspace allocation of process_weights_after_loading
 * (awq.py:168-180), which the reference sizes for its M <= 16 split-K kernel only. */
size_t w4a16_workspace_bytes_max(int M_max, int K, int N, int group_size);

/* y[M, N] = x[M, K] @ W with W given as (packed, qzeros, scales); bf16 in and out, fp32
 * accumulation.  M >= 0 (M == 0 is a no-op), K % 128 == 0, N % 64 == 0, group_size == 128,
 * K * N / 2 < 2^31 bytes of packed weights; x, packed, y 16-byte and qzeros, scales 4-byte
 * aligned.
 * Replaces linear (awq_w4a16.cu:288-371) / awq_cuda_linear (awq_cuda.py:141-185) and the
 * reference backend awq_reference_linear (awq.py:251-276). */
int w4a16_gemm(const uint16_t* x, const int32_t* packed, const int32_t* qzeros,
               const uint16_t* scales, uint16_t* y, int M, int K, int N, int group_size,
               void* workspace, size_t workspace_bytes, void* stream);

/* w4a16_gemm for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation): no workspace argument; the split-K
 * workspace is a 48 MiB device array of the library itself, one per GPU, held until the
 * process ends, set up on the first call on each device (symbol lookup, its counters
 * cleared by a kernel on `stream`): that first call must not be under graph capture
 * (W4A16_ERR_LAUNCH, nothing enqueued); later calls may be.  Allocates nothing.  Problems whose plan needs more
 * than 48 MiB of workspace (w4a16_workspace_bytes) are rejected with W4A16_ERR_WORKSPACE
 * before anything is enqueued (every Qwen3-8B projection at M <= 16384 fits).  Calls that
 * overlap on one GPU (two streams at once) share the array and race: serialize them.
 * Arguments, limits and results otherwise as w4a16_gemm (same kernels, same bits).
 * No counterpart in the reference: an allocation-free entry for the callers above. */
int w4a16_gemm_noalloc(const uint16_t* x, const int32_t* packed, const int32_t* qzeros,
                       const uint16_t* scales, uint16_t* y, int M, int K, int N, int group_size,
                       void* stream);

/* y[M, N] = bf16(bf16(x[M, K] @ W) + residual[M, N]): the GEMM with the residual add that
 * follows the O and down projections (the reference's add_rms_forward: x.float() +
 * residual.float() then bf16, layernorm.py:35-36) done in the epilogue.  residual may be y itself
 * (in place); 16-byte aligned.  Otherwise as w4a16_gemm; same workspace.  Replaces
 * o_proj / down_proj followed by that add (qwen3.py:170-174). */
int w4a16_gemm_residual(const uint16_t* x, const int32_t* packed, const int32_t* qzeros,
                        const uint16_t* scales, const uint16_t* residual, uint16_t* y, int M, int K,
                        int N, int group_size, void* workspace, size_t workspace_bytes, void* stream);

/* y[M, N/2] = SiLU(g) * u with [g | u] = x[M, K] @ W for a gate|up weight W [K, N] whose
 * first N/2 columns are the gate projection and last N/2 the up projection (the layout of
 * MergedColumnParallelLinear's gate_up_proj); g and u are rounded to bf16 as that layer
 * returns them, and SiLU(g) * u is computed in fp32 and rounded once, the reference's two
 * steps in one kernel.  Same arguments and limits as w4a16_gemm, plus N % 128 == 0; y is
 * [M, N/2], 16-byte aligned; workspace from w4a16_workspace_bytes(M, K, N, 128).
 * Replaces gate_up_proj followed by SiluAndMul (qwen3.py:126-130, activation.py:8-11):
 * the [M, N] gate|up intermediate is never written. */
int w4a16_gemm_silu_mul(const uint16_t* x, const int32_t* packed, const int32_t* qzeros,
                        const uint16_t* scales, uint16_t* y, int M, int K, int N, int group_size,
                        void* workspace, size_t workspace_bytes, void* stream);

/* RMSNorm of each row of x [M, K], with the residual add in front when residual is not NULL:
 *   s = float(x) + float(residual)  (s = float(x) without a residual), in fp32;
 *   residual_out = bf16(s);
 *   x_norm = bf16(float(bf16(s * rsqrt(mean(s * s) + eps))) * float(weight)).
 * weight is bf16 [K].  residual and residual_out are both given or both NULL; residual_out
 * may be residual or x (in place), x_norm may be x, x_norm != residual_out.  K % 8 == 0,
 * K <= 16384, every pointer 16-byte aligned, 0 <= eps <= 1.  rsqrt is evaluated in fp64
 * and the sum of squares is an fp32 tree sum, so bf16(s * r) can differ from another fp32
 * implementation by one bf16 ulp where s * r lies next to a rounding boundary (up to two
 * ulps of x_norm after the weight product).
 * Replaces RMSNorm.rms_forward / add_rms_forward (layernorm.py:16-40). */
int w4a16_add_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* weight, float eps,
                      uint16_t* x_norm, uint16_t* residual_out, int M, int K, void* stream);

/* RMSNorm without a residual (as w4a16_add_rmsnorm with residual == NULL) of rows read
 * through two strides: row r of x starts at element
 * (r / rows_inner) * stride_outer + (r % rows_inner) * stride_inner; x_norm is contiguous
 * [M, K].  Strides are multiples of 8 elements, x 16-byte aligned; other limits as
 * w4a16_add_rmsnorm.  Rows of K <= 512 share a wave (8 .. 64 lanes per row).
 * Replaces RMSNorm.rms_forward (layernorm.py:16-25) on a non-contiguous view: q_norm and
 * k_norm over q.view(-1, heads, head_dim) of the split QKV output (qwen3.py:87-94). */
int w4a16_rmsnorm_strided(const uint16_t* x, int rows_inner, int64_t stride_outer, int64_t stride_inner,
                          const uint16_t* weight, float eps, uint16_t* x_norm, int M, int K, void* stream);

/* The RMSNorm(+residual) prologue of w4a16_add_rmsnorm followed, on the same stream and in
 * the same call, by w4a16_gemm (silu_mul == 0) or w4a16_gemm_silu_mul (silu_mul == 1) of
 * x_norm: y = x_norm @ W, or SiLU(g) * u of it.  x_norm [M, K] (a caller buffer) and
 * residual_out receive the norm's outputs.  At M <= 2 on decode plans without a K split
 * (the Qwen3-8B QKV and gate|up shapes) and with x_norm / residual_out overlapping neither x
 * nor residual, the norm runs inside the GEMM kernel (one launch); otherwise the norm kernel
 * writes x_norm and the GEMM reads it back (from L2 at decode sizes).  Arguments as for
 * those two calls; y must overlap none of x, residual, x_norm and residual_out
 * (W4A16_ERR_ARG).  The workspace is w4a16_workspace_bytes(M, K, N, 128).  Argument, shape
 * and workspace errors are reported before anything is enqueued.
 * Replaces input_layernorm / post_attention_layernorm followed by qkv_proj / gate_up_proj
 * (qwen3.py:166-173 with layernorm.py:28-40, qwen3.py:126-130). */
int w4a16_gemm_rmsnorm(const uint16_t* x, const uint16_t* residual, const uint16_t* norm_weight, float eps,
                       uint16_t* x_norm, uint16_t* residual_out, const int32_t* packed,
                       const int32_t* qzeros, const uint16_t* scales, uint16_t* y, int M, int K, int N,
                       int group_size, int silu_mul, void* workspace, size_t workspace_bytes,
                       void* stream);

/* The RMSNorm that follows the O or down projection, split across that GEMM and the next
 * one so that no norm launch sits between them (decode sizes, 0 <= M <= 8; M > 8 is
 * W4A16_ERR_SHAPE: use w4a16_gemm_residual / w4a16_gemm and w4a16_gemm_rmsnorm there).
 * Producer: h = bf16(x[M, K] @ W) is added to residual [M, N] in fp32 in the epilogue, as
 * the reference's add_rms_forward does (layernorm.py:35-36): s_out[M, N] (fp32) =
 * float(h) + float(residual), residual_out = bf16(s_out) (may be residual itself, in place),
 * and ssq_out[M, N / 16] (fp32) holds, per row, the sum of s^2 over each 16-column tile.  h
 * itself is not stored.  x, W, workspace as w4a16_gemm; every pointer 16-byte aligned; the
 * outputs overlap neither each other (but for residual_out == residual) nor the inputs.
 * Replaces o_proj / down_proj followed by the residual add and the sum of squares of the
 * next RMSNorm (qwen3.py:170-174 with layernorm.py:35-38). */
int w4a16_gemm_residual_stats(const uint16_t* x, const int32_t* packed, const int32_t* qzeros,
                              const uint16_t* scales, const uint16_t* residual, float* s_out,
                              uint16_t* residual_out, float* ssq_out, int M, int K, int N,
                              int group_size, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Consumer of w4a16_gemm_residual_stats: the norm's scaling and the QKV GEMM (silu_mul == 0)
 * or the gate|up GEMM with SiLU * up (silu_mul == 1) in one decode kernel, whose workgroups
 * normalize the M rows of their K range once into LDS.  s [M, K] and
 * ssq [M, K / 16] are the producer's s_out and ssq_out (K its N); per row, rstd =
 * 1 / sqrt(sum(ssq) / K + eps) with the K / 16 tile sums added in a fixed order (rsqrt in
 * fp64, rounded once), then x_norm = bf16(float(bf16(s * rstd)) * float(norm_weight)) and
 * y = x_norm @ W (or SiLU(g) * u of it).  x_norm (may be NULL) receives the normalized
 * activations.  The sum of squares is added in another order than w4a16_add_rmsnorm's, so
 * x_norm can differ from it by one bf16 unit where s * rstd lies next to a rounding
 * boundary.  0 <= M <= 8, eps in [0, 1], every pointer 16-byte aligned; y overlaps none of
 * the inputs; workspace as w4a16_gemm (w4a16_workspace_bytes(M, K, N, 128) suffices).
 * Replaces post_attention_layernorm / input_layernorm followed by gate_up_proj / qkv_proj
 * (qwen3.py:166-173 with layernorm.py:28-40). */
int w4a16_gemm_rmsnorm_stats(const float* s, const float* ssq, const uint16_t* norm_weight, float eps,
                             uint16_t* x_norm, const int32_t* packed, const int32_t* qzeros,
                             const uint16_t* scales, uint16_t* y, int M, int K, int N, int group_size,
                             int silu_mul, void* workspace, size_t workspace_bytes, void* stream);

/* Kernel family w4a16_gemm launches for (M, K, N): a w4a16_regime_id.
 * Replaces the dispatch rule of select_awq_cuda_split_k (awq_cuda.py:17-26) and
 * AWQLinearMethod.apply (awq.py:115-154) as the thing a caller can query. */
int w4a16_regime(int M, int K, int N);

/* Number of K splits w4a16_gemm uses for (M, K, N) (1 = no cross-workgroup reduction).
 * Counterpart of select_awq_cuda_split_k (awq_cuda.py:17-26). */
int w4a16_split_k(int M, int K, int N);

/* The kernel configuration an entry point chooses for (M, K, N), written to out[5] as
 * {regime, p0, p1, p2, split} in w4a16_gemm_config's terms.  entry: 0 = w4a16_gemm (and
 * w4a16_gemm_residual, w4a16_gemm_residual_stats), 1 = w4a16_gemm_silu_mul, 2 and 3 =
 * w4a16_gemm_rmsnorm_stats without and with silu_mul (M <= 8), 4 = the decode kernel's own
 * plan (M <= 64), which w4a16_gemm runs below M = 32.  No reference counterpart: an
 * introspection hook for tuning and benchmarks. */
int w4a16_plan(int M, int K, int N, int entry, int* out);

/* w4a16_gemm with the kernel configuration forced instead of chosen: regime
 * W4A16_REGIME_DECODE (p0 = 16-column tiles per workgroup in {1,2,3,4,6} dividing N/16,
 * p1 = waves per workgroup in {4,8} (or 12 with p0 = 1), p2 = 128-row groups in flight per
 * wave in {1,2,4}, M <= 64; configurations whose LDS exceeds 156 KiB or whose accumulators and load ring
 * exceed 176 registers per lane are rejected) or W4A16_REGIME_TILE (p0 = 16-row tiles per
 * wave in {2,4,6,8}, p1 = waves per SIMD the register allocation targets, p2 = wave layout: 0 or 1 =
 * 4 waves of 64 columns, 2 = 2 x 4 waves of 64 columns, 3 = 8 waves of 32 columns,
 * 4 = 4 K slices x 2 waves of 32 columns, 5 = 2 K slices x 4 waves of 32 columns,
 * 6 = 2 K slices x 2 waves of 32 columns, 7 = 4 K slices x 1 wave of 32 columns,
 * 9 = 4 K slices x 3 waves of 32 columns, 10 = 2 K slices x 6 waves of 32 columns, the K
 * slices of a workgroup summed through LDS, 8 = 8 waves of 64 columns, 11 = 8 waves of 48
 * columns (plain GEMM only, N a multiple of 48); the compiled (p0, p2, p1) are (4,1,1),
 * (4,1,2), (8,1,1), (4,2,2), (4,3,2), (8,3,2), (2,4,2), (4,4,2), (2,5,2), (4,5,2), (8,5,2),
 * (4,6,1), (8,6,1), (2,7,1), (4,7,1), (8,8,2), (4,9,3), (2,9,3), (4,10,3), (8,11,2),
 * (4,11,2), (6,3,2), (6,8,2), (6,11,2));
 * 1 <= split <= K/128.  No reference counterpart: a tuning and testing hook (it exercises
 * every split-K reduction path at small sizes). */
int w4a16_gemm_config(const uint16_t* x, const int32_t* packed, const int32_t* qzeros,
                      const uint16_t* scales, uint16_t* y, int M, int K, int N, int group_size,
                      int regime, int p0, int p1, int p2, int split, void* workspace,
                      size_t workspace_bytes, void* stream);

/* w4a16_gemm_silu_mul with the kernel configuration forced, as w4a16_gemm_config (decode
 * p0 must be even).  No reference counterpart: a testing hook. */
int w4a16_gemm_silu_mul_config(const uint16_t* x, const int32_t* packed, const int32_t* qzeros,
                               const uint16_t* scales, uint16_t* y, int M, int K, int N,
                               int group_size, int regime, int p0, int p1, int p2, int split,
                               void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes w4a16_gemm_config needs for that configuration (for the tile regime,
 * enough for every wave layout).  No reference counterpart. */
size_t w4a16_workspace_bytes_config(int M, int N, int regime, int p0, int split);

#ifdef __cplusplus
}
#endif

#endif /* W4A16_H_ */
