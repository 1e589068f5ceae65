/*
 * fluxbin_amd -- C ABI of the MI355X (gfx950) W3 packed-LUT batch-1 decode path.
 *
 * Plain C types only: device pointers are passed as void* / typed pointers, the
 * HIP stream as an opaque void* (a hipStream_t; NULL = the default stream).
 * Every entry point is asynchronous on that stream, allocates nothing and never
 * synchronises, so all of them may be captured into a HIP graph.  Return value:
 * FX_OK, or an FX_E* code with a message available from fx_last_error() (per
 * calling thread).
 *
 * dtype codes: FX_F32 = 0, FX_F16 = 1, FX_BF16 = 2.
 *
 * Payload (maxiu188-afk/Marlin_Style_Fluxbin gptq_deployment.py:199-227, with two
 * extensions: optional per-group zero-points, fp16 or bf16 scales):
 *   planes  uint8 [G,3,O,16], 16-byte aligned; K = 128 * G
 *   scales  fp16|bf16 [G,O]
 *   zeros   uint8 [G,O] or NULL (NULL: every zero-point is 4)
 *   perm    int16 [K] or NULL (NULL: identity)
 * Activations x are [M,K] fp16|bf16 row-major; outputs [M,O] in the same dtype.
 */
#ifndef FLUXBIN_AMD_H
#define FLUXBIN_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FX_OK 0
#define FX_EINVAL 1
#define FX_EHIP 2

#define FX_F32 0
#define FX_F16 1
#define FX_BF16 2

#define FX_ARITH_STRUCTURAL 0  /* fp32 s*(q-z) grouped dot */
#define FX_ARITH_DECODED_BF16 1 /* + per-weight bf16 rounding of s*(q-z) (bf16 scales, zero 3 or 4) */

/* ABI version of this header (bumped on any signature change). */
int fx_abi_version(void);
/* Last error message of the calling thread ("" if none). */
const char *fx_last_error(void);

/*
 * Reference: csrc/w3_lut.cu:251-260 (inline_main / inline_main_bf16_weight),
 * bound through w3_lut_deployment.py:100-126.  Writes fp32 partial sums
 * partial[s, m, o] for the ceil(G/groups_per_split) K splits; row_tile in
 * {256,512,1024} selects rows per workgroup.  For M = 1 the partial buffer is
 * the reference's fp32 [splits, O] workspace.
 */
int fx_w3_inline_main(const void *x, int x_dtype, const uint8_t *planes, const void *scales,
                      int scale_dtype, const uint8_t *zeros, const int16_t *perm,
                      float *partial, int M, int O, int K, int groups_per_split,
                      int row_tile, int arithmetic, void *stream);

/*
 * Reference: csrc/w3_lut.cu:262-284 (finish), w3_lut_deployment.py:129-135.
 * out[m, o] = sum_s partial[s, m, o] (sequential in s), cast to out_dtype.
 */
int fx_w3_finish(const float *partial, void *out, int out_dtype, int splits, int M, int O,
                 void *stream);

/*
 * Reference: csrc/w3_lut.cu:286-332 (m1_out), w3_lut_deployment.py:138-171.
 * With one split the workspace is not touched and one kernel writes out;
 * otherwise inline_main + finish through the fp32 workspace [splits, M, O].
 */
int fx_w3_m1_out(const void *x, int x_dtype, const uint8_t *planes, const void *scales,
                 int scale_dtype, const uint8_t *zeros, const int16_t *perm, float *workspace,
                 void *out, int M, int O, int K, int groups_per_split, int row_tile,
                 int arithmetic, void *stream);

/*
 * Fast path used by PackedW3Linear and its prepared decode binding
 * (w3_lut_deployment.py:250-359 in the reference).  structural arithmetic: the
 * gfx950 MFMA kernel -- codes dequantized in registers to bf16/fp16 subnormal
 * MFMA operands against exact power-of-two-scaled activations, fp32
 * accumulation, K split over the waves of a workgroup; one launch per call,
 * plus a stream-ordered finish launch when the output has fewer 16-row tiles
 * than CUs and K is also split over workgroups.  decoded_bf16 arithmetic: the
 * LUT kernel plus finish.  Tiling comes from (M, O, K) and the CU count.
 * workspace: fx_w3_gemv_workspace_bytes(M, O, K) bytes, 256-byte aligned, no
 * initial contents required; NULL is accepted when that size is 0.  Calls that
 * share a workspace must be ordered on one stream.
 */
size_t fx_w3_gemv_workspace_bytes(int M, int O, int K);
int fx_w3_gemv(const void *x, int x_dtype, const uint8_t *planes, const void *scales,
               int scale_dtype, const uint8_t *zeros, const int16_t *perm, void *workspace,
               size_t workspace_bytes, void *out, int M, int O, int K, int arithmetic,
               void *stream);
/* Structural MFMA path with an explicit tiling (benchmark sweeps): waves per
 * workgroup in {4,8}, 4-group batches kept in flight per wave in {1,2},
 * groups per K split (rounded up to a multiple of 4, clamped to the padded group
 * count), 16-row tiles per wave in {1,2}. */
size_t fx_w3_gemv_config_workspace_bytes(int M, int O, int K, int waves, int prefetch,
                                         int groups_per_split, int tiles);
int fx_w3_gemv_config(const void *x, int x_dtype, const uint8_t *planes, const void *scales,
                      int scale_dtype, const uint8_t *zeros, const int16_t *perm,
                      void *workspace, size_t workspace_bytes, void *out, int M, int O, int K,
                      int waves, int prefetch, int groups_per_split, int tiles, void *stream);

/*
 * Reference: restore_planar_w3 (gptq_deployment.py:247-260), the dequantize
 * step of the dense fallback (w3_lut_deployment.py:327-333).  weight [O,K] in
 * weight_dtype: round_weight_dtype(round_scale_dtype(s * (q - z))).
 */
int fx_w3_restore(const uint8_t *planes, const void *scales, int scale_dtype,
                  const uint8_t *zeros, const int16_t *perm, void *weight, int weight_dtype,
                  int O, int K, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FLUXBIN_AMD_H */
