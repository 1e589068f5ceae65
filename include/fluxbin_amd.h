/*
 * fluxbin_amd -- C ABI of the MI355X (gfx950) W3 packed-LUT batch-1 decode path.
 *
 * Plain C types only: device pointers are passed as void* / typed pointers, the
 * HIP stream as an opaque void* (a hipStream_t; NULL = the default stream).
 * Every entry point is asynchronous on that stream, allocates nothing and never
 * synchronises, so all of them may be captured into a HIP graph.  Return value:
 * FX_OK, or an FX_E* code with a message available from fx_last_error() (per
 * calling thread).  Host threads may call concurrently on their own streams (a
 * call's state lives in its arguments) with one exception: fx_w3_gemv_noalloc's
 * calls share a per-GPU scratch array and must not overlap on one GPU.
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

/* Payload formats of the one-row decode GEMVs: the reference's planar layout, or
 * the library's field layout (fx_w3_planes_to_fields) or fp6 layout
 * (fx_w3_planes_to_fp6), both in the same sorted column order. */
#define FX_W3_PLANAR 0
#define FX_W3_FIELDS 1
#define FX_W3_FP6 2

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
/* fx_w3_gemv without a workspace argument.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The K-split partials that
 * fx_w3_gemv keeps in the caller's workspace live in a 4 MiB array of the library,
 * one per GPU, held until the process ends; its device address is resolved on the
 * first call on each device.  Calls whose fx_w3_gemv_workspace_bytes(M, O, K)
 * exceeds 4 MiB fail with FX_EINVAL.  The array keeps the last call's contents and
 * every call overwrites what it reads, so nothing needs clearing; calls that
 * overlap on one GPU (different streams, or host threads) race on it and must be
 * serialised by the caller.  Same kernels and results as fx_w3_gemv. */
int fx_w3_gemv_noalloc(const void *x, int x_dtype, const uint8_t *planes, const void *scales,
                       int scale_dtype, const uint8_t *zeros, const int16_t *perm, void *out, int M,
                       int O, int K, int arithmetic, void *stream);
/* Fused gate|up projection and SwiGLU of a Qwen3 MLP for one activation row.  No
 * single reference entry point: it replaces the reference's two PackedW3Linear
 * calls (gate_proj, up_proj; w3_lut_deployment.py:250-359) followed by HF
 * Qwen3MLP's act_fn(gate) * up, with bit-identical results.  The payload's O rows
 * interleave the two projections (row 2r = gate row r, row 2r+1 = up row r, in
 * planes, scales and zero-points alike); out receives O / 2 values
 * round(round(silu(round(g))) * round(u)) in x's dtype, each round an RNE cast
 * to that dtype.  Structural MFMA arithmetic, one launch, no workspace. */
int fx_w3_gemv_swiglu(const void *x, int x_dtype, const uint8_t *planes, const void *scales,
                      int scale_dtype, const uint8_t *zeros, const int16_t *perm, const int16_t *out_index,
                      void *out, int O, int K, int payload_format, void *stream);
/* The decoder layer's residual stream threaded through its W3 GEMVs (one
 * activation row, structural MFMA arithmetic).  No single reference entry point: together they
 * replace HF Qwen3DecoderLayer's residual adds and Qwen3RMSNorm (as the reference
 * patches them, fused_modules.py:30-63) around the PackedW3Linear calls
 * (w3_lut_deployment.py:250-359).
 * fx_w3_gemv_residual: out = round(residual + round(x @ W.T)) -- out may alias
 * residual -- and tile_sumsq[t] = sum of out^2 over rows [16 t, 16 t + 16),
 * ceil(O / 16) floats.
 * fx_w3_gemv_rmsnormed: h is such an out (K = its O) and tile_sumsq its tile
 * sums (n_tiles = ceil(K / 16), K <= 4096); the GEMV reads
 * x = round(norm_weight * round(h * rsqrt(sum(tile_sumsq) / K + eps))), the
 * RMSNorm of h, summing the tile sums in a fixed order; swiglu != 0 reads the
 * row-interleaved gate|up payload of fx_w3_gemv_swiglu.  It takes no permutation:
 * with a column-permuted payload, h and norm_weight come in the payload's sorted
 * column order (h[k] = residual[perm[k]], norm_weight[k] = w[perm[k]]); the
 * tile sums are order-free.
 * Column order for permuted consumers (the reference's desc_act payloads carry
 * perm = argsort(g_idx), gptq_deployment.py:199-227): out_index (int16, NULL =
 * none) names where each output value goes, so the producer writes the next
 * GEMV's activations in that GEMV's sorted order and it reads them contiguously.
 * fx_w3_gemv_residual: out row o is also written to sorted_out[out_index[o]]
 * (both NULL or both set; sorted_out [O] must not alias out or residual).
 * fx_w3_gemv_swiglu / fx_w3_gemv_rmsnormed (swiglu = 1 only): SwiGLU value r goes
 * to out[out_index[r]] instead of out[r].  With out_index the inverse of the next
 * GEMV's perm, that GEMV's result is bit-identical to the same GEMV given the
 * row-ordered activation and the perm.  Entries outside [0, outputs) are not
 * written.
 * payload_format (all): FX_W3_PLANAR, FX_W3_FIELDS with `planes` holding the
 * field layout, or FX_W3_FP6 with `planes` holding the fp6 layout (bf16
 * activations, no perm, O % 16 == 0, K % 512 == 0). */
int fx_w3_gemv_residual(const void *x, int x_dtype, const uint8_t *planes, const void *scales,
                        int scale_dtype, const uint8_t *zeros, const int16_t *perm, const void *residual,
                        void *out, float *tile_sumsq, const int16_t *out_index, void *sorted_out, int O, int K,
                        int payload_format, void *stream);
int fx_w3_gemv_rmsnormed(const void *h, int x_dtype, const uint8_t *planes, const void *scales,
                         int scale_dtype, const uint8_t *zeros, const float *tile_sumsq, int n_tiles,
                         const void *norm_weight, float eps, const int16_t *out_index, void *out, int O, int K,
                         int swiglu, int payload_format, void *stream);
/* A strided batch of one-row structural GEMVs in one launch: no reference
 * counterpart (the reference runs one PackedW3Linear call per payload).  Payload
 * p (0 <= p < batch) reads x + p * x_stride, planes + p * planes_stride (bytes),
 * scales + p * scales_stride, zeros + p * zeros_stride (elements; zeros NULL =
 * every zero-point 4) and writes out + p * out_stride: out_p [1, O] = x_p [1, K] @
 * W_p.T, each bit-identical to the same payload's single call of the same format
 * (fx_w3_gemv's one-split plan, or fx_w3_gemv_fields).  Identity column order; with
 * batch > 1, O / 16 a multiple of 8 and each stride at least one payload / row.
 * For the same-shape Linears of many layers, and to measure the kernel without
 * the per-launch cost. */
int fx_w3_gemv_strided_batched(const void *x, int x_dtype, long long x_stride, const uint8_t *planes,
                               long long planes_stride, const void *scales, int scale_dtype,
                               long long scales_stride, const uint8_t *zeros, long long zeros_stride, void *out,
                               long long out_stride, int batch, int O, int K, int payload_format, void *stream);
/* The field layout: no reference counterpart; a bind-time repack of the
 * reference's planar payload (gptq_deployment.py:199-244 layout, same sorted
 * column order, same [G, 3, O, 16] byte shape, three bits per code) whose
 * dequantization costs half the instructions.  The codes of sorted columns
 * 32 w + t (t < 32) of a (group, row) sit in little-endian word w (bytes 4 w ..)
 * of its three 16-byte member rows: i = t / 2, h = t % 2; for i < 15 the code
 * occupies bits [16 h + 3 f, +3) of member i / 5 (f = i % 5); for i = 15 its
 * bit k occupies bit 15 + 16 h of member k.  fields must not alias planes;
 * both 16-byte aligned. */
int fx_w3_planes_to_fields(const uint8_t *planes, uint8_t *fields, int O, int K, void *stream);
/* One-row structural GEMV on the field layout (identity column order, one
 * launch, no workspace): out [1, O] = x [1, K] @ W.T as fx_w3_gemv's structural
 * arithmetic (fp32 accumulation of exact products; the sum order differs). */
int fx_w3_gemv_fields(const void *x, int x_dtype, const uint8_t *fields, const void *scales, int scale_dtype,
                      const uint8_t *zeros, void *out, int O, int K, void *stream);
/* No reference counterpart: a second bind-time repack of the planes, for
 * gfx950's v_mfma_scale_f32_16x16x128_f8f6f4 with fp6 e2m3 weight operands (a
 * field with zero sign and exponent bits and the code in its mantissa is exactly
 * q / 8).  Same byte count as the planes, ordered [K / 512, O, k-block (4),
 * group slot (4), 3 words]: field e of A lane block kb multiplies group column
 * 32 (2 (kb % 2) + e / 16) + 16 (kb / 2) + e % 16, and the three words expand
 * into the six fp6 registers with two masks, two shift-and-masks and one
 * register that takes bits 29, 30 from bits 1, 2 of the third word (M0 =
 * 0xC71C71C7 for registers 0, 3; M1 = 0x71C71C71 for 1, 4; M2 = 0x1C71C71C for
 * 2, 5, of the first words shifted right by one).  K a multiple of 512; fp6
 * must not alias planes; both 16-byte aligned. */
int fx_w3_planes_to_fp6(const uint8_t *planes, uint8_t *fp6, int O, int K, void *stream);
/* One-row structural GEMV on the fp6 layout: out [1, O] = x [1, K] @ W.T with x
 * bf16 in sorted column order, each group's activations split into two fp8 e4m3
 * digits (exact down to 2^-10 of the group's max|x|), one scaled matrix
 * instruction per group and 16-row tile, fp32 accumulation.  O a multiple of
 * 16, K of 512. */
int fx_w3_gemv_fp6(const void *x, int x_dtype, const uint8_t *fp6, const void *scales, int scale_dtype,
                   const uint8_t *zeros, void *out, int O, int K, void *stream);
/* Field-layout GEMV of M <= 8 activation rows (no single counterpart: the
 * small-M route of w3_lut_deployment.py:327-333 on the bind-time field layout):
 * out [M, O] = x [M, K] @ W.T, structural arithmetic.  One row is
 * fx_w3_gemv_fields; more run the M-row kernel in one launch (a workgroup of
 * several row tiles stages each batch of all its rows once for them; one of a
 * single tile restages per batch, wave by wave), with each batch's products
 * summed in batch order, so every plan of fx_w3_fields_plan gives the same
 * bits.  For M > 1: K a multiple of 512 and at most 16384 under the default
 * plans, O a multiple of 16. */
int fx_w3_gemv_fields_rows(const void *x, int x_dtype, const uint8_t *fields, const void *scales, int scale_dtype,
                           const uint8_t *zeros, void *out, int M, int O, int K, void *stream);
/* Field-layout plans (no counterpart in the reference: benchmark sweeps and the
 * plan-independence tests).  Every field-layout launch of the calling thread
 * (fx_w3_gemv_fields, the FX_W3_FIELDS forms of fx_w3_gemv_swiglu / _residual /
 * _rmsnormed and fx_w3_gemv_strided_batched) runs the given plan until the next
 * call: tiles > 0 the shared-staging kernel with tiles 16-row tiles x parts K
 * parts per workgroup, prefetch batches (512 columns) in flight and stage staged
 * batches per wave -- one of (1,8,1,1) (1,8,3,3) (2,4,2,1) (3,4,2,1) (4,2,4,1),
 * or (1,12,2,2) (1,16,2,2) for fx_w3_gemv_fields_rows only, else FX_EINVAL, and
 * a launch whose shape the plan cannot run (O % 16, K % 512, more batches than
 * it stages, an M-row-only plan on one row) fails with FX_EINVAL; tiles <= 0 the
 * one-tile kernel (fx_w3_gemv_fields_rows: its default plans), the default.
 * Every plan gives the same bits.  Thread-local state. */
int fx_w3_fields_plan(int tiles, int parts, int prefetch, int stage);
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
 * weight_dtype: round_weight_dtype(round_scale_dtype(s * (q - z))); sorted
 * column s of row o lands at weight[o, perm[s]].  perm NULL is the identity
 * order (row-ordered 16-byte stores; pass NULL when the order is known to be
 * the identity); a permutation stages whole rows in LDS and needs K <= 32768.
 * perm entries outside [0, K) are skipped and a column that no entry names is
 * zero.
 */
int fx_w3_restore(const uint8_t *planes, const void *scales, int scale_dtype,
                  const uint8_t *zeros, const int16_t *perm, void *weight, int weight_dtype,
                  int O, int K, void *stream);

/*
 * Reference: rms_norm_reference / fused_rms_norm_forward (fused_modules.py:30-63),
 * i.e. stock Qwen3RMSNorm.forward (transformers modeling_qwen3.py), optionally
 * fused with the decoder layer's residual add.  x, residual, out, residual_out are
 * [rows, hidden] row-major, weight [hidden], all in dtype, 16-byte aligned,
 * hidden % 8 == 0.  With residual (non-NULL): s = round(x + residual) is written
 * to residual_out, then out = round(weight * round(s * rsqrt(mean(s^2) + eps)));
 * without: the same on x.  out may alias x; residual_out may alias x or
 * residual.
 */
int fx_rmsnorm(const void *x, const void *residual, const void *weight, void *out,
               void *residual_out, int rows, int hidden, float eps, int dtype, void *stream);

#define FX_ROPE_NONE 0
#define FX_ROPE_STOCK 1 /* HF apply_rotary_pos_emb: round(round(y*cos) + round(rot(y)*sin)) */
#define FX_ROPE_FUSED 2 /* fused_apply_rotary_pos_emb (addcmul): round(round(y*cos) + rot(y)*sin) */

/*
 * Reference: per-head q_norm / k_norm (Qwen3RMSNorm over head_dim) followed by
 * apply_rotary_pos_emb (modeling_qwen3.py) or fused_apply_rotary_pos_emb
 * (fused_modules.py:66-85), for up to 4 tensors in one launch.  Tensor i has
 * batch x heads[i] x seq rows of head_dim contiguous elements; strides[6i..6i+2]
 * are its input element strides (batch, head, position), strides[6i+3..6i+5] its
 * output strides (e.g. a KV cache slot).  weights[i] NULL: no norm; rope[i] 0: no
 * rotation (a strided copy).  cos/sin rows are at batch*cos_strides[0] +
 * position*cos_strides[1] (+ position[0]*head_dim when the device scalar
 * `position` is given, for graph-replayed decode).  Outputs must not overlap
 * inputs of another tensor.
 */
int fx_head_norm_rope(int ntensors, const void *const *inputs, void *const *outputs,
                      const void *const *weights, const int *heads, const int *rope,
                      const long long *strides, int batch, int seq, int head_dim,
                      const void *cos, const void *sin, const long long *cos_strides,
                      const int *position, float eps, int rope_mode, int dtype, void *stream);

/* Attention plan of the calling thread (no counterpart in the reference: sweeps
 * and tests): keys_per_thread 1, 2 or 4 and head_groups 1, 2 or 4 (query heads of
 * a KV head split over that many 256-thread groups of the split workgroup); 0
 * keeps the default for either.  Applies to fx_decode_attention(_rope) until the
 * next call.  Thread-local state. */
int fx_decode_attention_plan(int keys_per_thread, int head_groups);
/*
 * Decode attention of one token over a static KV cache: the attention the
 * reference's decode runs inside stock HF Qwen3Attention (static_decode.py:73-81:
 * StaticCache + boolean mask, SDPA).  q [n_q_heads, head_dim]; caches
 * [n_kv_heads, max_len, head_dim]; query head h reads KV head h / (n_q_heads /
 * n_kv_heads) at slots 0..position (later slots are never read); fp32 scores
 * scaled by `scale`, fp32 softmax and accumulation, out [n_q_heads, head_dim]
 * rounded to dtype.  One launch over key chunks and a second that combines
 * their partials (one launch when one chunk covers the context), through
 * `workspace` (fx_decode_attention_workspace_bytes bytes, 16-byte aligned, no
 * initial contents needed).  Calls that share a workspace must not overlap.
 * head_dim in {64, 128, 256}.  out_index (int16 [n_q_heads * head_dim], NULL =
 * none): value i of the output goes to out[out_index[i]] (the o projection's
 * sorted column order when its payload carries a permutation; entries outside
 * the output are not written).
 */
size_t fx_decode_attention_workspace_bytes(int n_q_heads, int max_len, int head_dim);
int fx_decode_attention(const void *q, const void *k_cache, const void *v_cache, void *workspace,
                        size_t workspace_bytes, const int16_t *out_index, void *out, int n_q_heads,
                        int n_kv_heads, int max_len, int head_dim, int position, float scale, int dtype,
                        void *stream);
/*
 * Decode attention with the per-head q/k RMSNorm + RoPE folded in: no single
 * reference entry point; it replaces HF Qwen3Attention's q_norm / k_norm,
 * apply_rotary_pos_emb (stock or the reference's fused_apply_rotary_pos_emb,
 * fused_modules.py:66-85), the KV-cache update at `position` and the attention
 * of fx_decode_attention.  q [Hq, D], k and v [Hk, D] are the raw projections of
 * the current token; q_norm_weight / k_norm_weight [D]; cos / sin the RoPE rows
 * [D] of `position`.  The key (normalised, rotated) and value of `position` are
 * written into k_cache / v_cache and used; rounding points as fx_head_norm_rope
 * (the per-head sum of squares may differ from it in the last bit).
 */
int fx_decode_attention_rope(const void *q, const void *k, const void *v, const void *q_norm_weight,
                             const void *k_norm_weight, const void *cos, const void *sin, float eps,
                             int rope_mode, void *k_cache, void *v_cache, void *workspace,
                             size_t workspace_bytes, const int16_t *out_index, void *out, int n_q_heads,
                             int n_kv_heads, int max_len, int head_dim, int position, float scale, int dtype,
                             void *stream);

/*
 * Qwen3MLP activation (transformers modeling_qwen3.py, run by the reference's
 * decode): out = round(round(silu(gate)) * up) elementwise over n values.
 */
int fx_silu_mul(const void *gate, const void *up, void *out, int n, int dtype, void *stream);

/*
 * End of a greedy decode step: the final RMSNorm, the LM head and
 * the argmax that the reference's decode runs as model.norm, lm_head and
 * logits.argmax(-1, keepdim=True) (static_decode.py:67-76).
 *   x = round(norm_weight * round(hidden * rsqrt(mean(hidden^2) + eps)))
 *       (norm_weight NULL: x = hidden, already normalised)
 *   logits[v] = round(weight[v, :] . x), fp32 accumulation, v < vocab
 *   *prediction = argmax of the rounded logits: the first index of the maximum,
 *                 a NaN above every number (torch.argmax)
 * hidden / norm_weight [hidden_size], weight [vocab, hidden_size] row-major,
 * logits [vocab], all in `dtype`; hidden_size a multiple of 512 up to 8192;
 * hidden, norm_weight, weight 16-byte aligned, logits 2-byte aligned.  The
 * normalised x is bit-identical to fx_rmsnorm's.  Two launches: the streaming
 * kernel leaves each workgroup's best logit in `workspace`
 * (fx_lm_head_argmax_workspace_bytes, 16-byte aligned, no initial contents
 * needed) and a one-workgroup launch merges them into *prediction.  Calls sharing
 * a workspace must not overlap.
 */
size_t fx_lm_head_argmax_workspace_bytes(void);
int fx_lm_head_argmax(const void *hidden, const void *norm_weight, float eps, const void *weight, void *logits,
                      long long *prediction, void *workspace, size_t workspace_bytes, int vocab,
                      int hidden_size, int dtype, void *stream);
/*
 * fx_lm_head_argmax's two launches one at a time (no reference counterpart: the
 * decode chain splits them so the merge can ride in the next step's first
 * launch).  fx_lm_head_logits: the streaming launch (logits, and the
 * per-workgroup maxima left in `workspace`).  fx_lm_head_merge: their merge into
 * *prediction; `vocab` must be the one the streaming call was given (it fixes
 * how many maxima there are).  Together bit-identical to fx_lm_head_argmax.
 */
int fx_lm_head_logits(const void *hidden, const void *norm_weight, float eps, const void *weight, void *logits,
                      void *workspace, size_t workspace_bytes, int vocab, int hidden_size, int dtype, void *stream);
int fx_lm_head_merge(void *workspace, size_t workspace_bytes, int vocab, long long *prediction, void *stream);

/*
 * Start of a decode step (no single reference counterpart: it replaces the
 * embedding lookup of the step's token and the first decoder layer's
 * input RMSNorm statistics, static_decode.py:67-76 / HF Qwen3Model.forward).  One
 * workgroup: out [hidden] = table[*token] (row-major [vocab, hidden], bit copy),
 * tile_sumsq [hidden / 16] = per 16-element tile the fp32 sum of squares, the
 * partials fx_w3_gemv_rmsnormed reads; a token outside [0, vocab) writes NaNs.
 * prediction non-null: also merges the previous step's fx_lm_head_logits maxima
 * (lm_workspace, lm_vocab) into *prediction, as fx_lm_head_merge does.  hidden a
 * multiple of 16; table and out 16-byte aligned, token 8-byte aligned.
 * out_index (int16 [hidden], 16-byte aligned) and sorted_out [hidden], both NULL
 * or both set: element i of the row is also written to sorted_out[out_index[i]]
 * (the first layer's q|k|v sorted column order, as fx_w3_gemv_residual's).
 */
int fx_decode_embed(const long long *token, const void *table, int vocab, int hidden, void *out, float *tile_sumsq,
                    const int16_t *out_index, void *sorted_out, void *lm_workspace, size_t lm_workspace_bytes,
                    int lm_vocab, long long *prediction, int dtype, void *stream);

/*
 * Two-base binary-basis GEMV, rank-one format with salient columns, batch 1:
 * the benchmark's config-4 form of the reference's two-base M=1 GEMV
 * (deployment.py:168-179 m1_out -> csrc/m1_v5.cu:26-104 lut_m1; same
 * contract: caller-owned output and workspace, current stream, no allocation,
 * fp32 accumulation, x [1, K] contiguous):
 *   y[o] = s_r[o] * (a1[o] * (B1[o,:] . u) + a2[o] * (B2[o,:] . u))
 *          + sum_j salient[o, j] * x[salient_idx[j]],   u[k] = t_c[k] * x[k]
 * planes uint8 [K/128, O, 2, 16] (16-byte aligned): sign bit (1 = +1) of column
 * 128 g + k of base b, row o at bit k >> 4 of byte k & 15 of planes[g][o][b];
 * coef fp16 [2, O] (a1, a2); srow fp16 [O]; tcol fp16 [K]; salient bf16
 * [O, n_salient] and salient_idx int32 [n_salient], n_salient <= 32 (both may
 * be null when n_salient == 0; indices outside [0, K) contribute nothing).  x / out fp16 or
 * bf16 (x_dtype), x and tcol 16-byte aligned.  Workspace: fp32 partials when K
 * is split over workgroups (fx_two_base_gemv_workspace_bytes, may be 0).
 */
size_t fx_two_base_gemv_workspace_bytes(int O, int K);
int fx_two_base_gemv(const void *x, int x_dtype, const uint8_t *planes, const void *coef,
                     const void *srow, const void *tcol, const void *salient,
                     const int32_t *salient_idx, int n_salient, void *workspace,
                     size_t workspace_bytes, void *out, int O, int K, void *stream);
/* Same with an explicit tiling: `tiles` 16-row tiles per workgroup, waves =
 * tiles * (waves per tile along K), prefetch = batches of sign loads in flight;
 * (tiles, waves/tiles, prefetch) in (1,4,1|2) (1,8,1|2) (2,4,1|2) (3,4,1|2)
 * (4,4,2) (2,8,2).  groups_per_split is rounded up to a multiple of 4 and capped
 * at what one workgroup stages (96 groups, 16 per wave). */
size_t fx_two_base_gemv_config_workspace_bytes(int O, int K, int waves, int prefetch,
                                               int groups_per_split, int tiles);
int fx_two_base_gemv_config(const void *x, int x_dtype, const uint8_t *planes, const void *coef,
                            const void *srow, const void *tcol, const void *salient,
                            const int32_t *salient_idx, int n_salient, void *workspace,
                            size_t workspace_bytes, void *out, int O, int K, int waves,
                            int prefetch, int groups_per_split, int tiles, void *stream);

/*
 * Two-base hybrid g128/s8 GEMV over the reference's planar deployment layout,
 * batch 1: deployment.py:168-179 m1_out with a v5_p* kernel (csrc/m1_v5.cu:26-112,
 * PLANAR_CODES) -- caller-owned output and workspace, current stream, no
 * allocation, x [1, K] contiguous:
 *   y[o] = sum_g sum_b rows[g,o,b] * (B_b[o,g,:] . (x_g * columns[g,:,b]))
 *        + sum_g sum_b sparse_rows[g,o,b] * (R_b[o,g,:] . (x[128g + indices[g,:]] * sparse_columns[g,:,b]))
 * codes uint8 [G, O, 2, 16] (bit j of byte c of base b = column 8c + j, 1 = +1),
 * rows / sparse_rows fp32 [G, O, 2], columns fp32 [G, 128, 2], indices int16
 * [G, 8] (0..127), sparse_codes uint8 [G, O, 2, 1], sparse_columns fp32 [G, 8, 2]
 * (convert_artifact, deployment.py:84-103).  The workspace bounds the K split:
 * the kernel uses at most workspace_bytes / (4 O) splits (the reference's fp32
 * [splits, O] workspace fits), and none when the output is wide enough.
 */
size_t fx_hybrid_gemv_workspace_bytes(int O, int K);
int fx_hybrid_gemv(const void *x, int x_dtype, const uint8_t *codes, const float *rows,
                   const float *columns, const int16_t *indices, const uint8_t *sparse_codes,
                   const float *sparse_rows, const float *sparse_columns, void *workspace,
                   size_t workspace_bytes, void *out, int O, int K, void *stream);
/*
 * fx_hybrid_gemv over n_segments (1..4) layouts that read the same activation,
 * in one launch: no single reference entry point; it replaces the reference
 * decode's separate m1_out calls for q_proj, k_proj, v_proj (or gate_proj,
 * up_proj) (deployment.py:168-179) and gives each row the bits of its own
 * fx_hybrid_gemv call when both split K over the same number of workgroups (the
 * decode shapes); otherwise the rows' fp32 partials are summed in another order.
 * codes, rows, sparse_codes and sparse_rows are the
 * segments' arrays concatenated along O ([G, O_total, ...]); columns, indices
 * and sparse_columns hold one pointer per segment (its [G, 128, 2], [G, 8],
 * [G, 8, 2] arrays); segment_rows[s] is segment s's row count, a multiple of 16
 * when n_segments > 1; out [O_total], O_total = sum of segment_rows (<= 65536).
 * Workspace as fx_hybrid_gemv_workspace_bytes(O_total, K).
 */
int fx_hybrid_gemv_segments(const void *x, int x_dtype, int n_segments, const int *segment_rows,
                            const uint8_t *codes, const float *rows, const float *const *columns,
                            const int16_t *const *indices, const uint8_t *sparse_codes, const float *sparse_rows,
                            const float *const *sparse_columns, void *workspace, size_t workspace_bytes, void *out,
                            int K, void *stream);
/*
 * fx_hybrid_gemv with the decoder layer's residual add folded in (no single
 * reference entry point: it replaces m1_out for o_proj / down_proj plus the
 * following add of HF Qwen3DecoderLayer): out = round(residual + round(y)) in
 * x_dtype (residual may alias out) and tile_sumsq[i] = the fp32 sum of out^2 over
 * rows 16i .. 16i+15, the partials the next fx_hybrid_gemv_segments_rmsnormed
 * reads.  swiglu != 0 (down_proj, replacing also the SwiGLU of Qwen3MLP): x holds
 * gate | up, 2K values, and the GEMV reads round(round(silu(gate)) * up), bit for
 * bit what fx_silu_mul writes.  One K split (no workspace): fails when K needs more.
 */
int fx_hybrid_gemv_residual(const void *x, int x_dtype, const uint8_t *codes, const float *rows,
                            const float *columns, const int16_t *indices, const uint8_t *sparse_codes,
                            const float *sparse_rows, const float *sparse_columns, const void *residual, void *out,
                            float *tile_sumsq, int O, int K, int swiglu, void *stream);
/*
 * fx_hybrid_gemv_segments of RMSNorm(h): no single reference entry point; it
 * replaces the input_layernorm / post_attention_layernorm of HF Qwen3DecoderLayer
 * plus the projections' m1_out calls.  The kernel normalises h [K] on the fly as
 * Qwen3RMSNorm does, x = round(w * round(h * rsqrt(sum(tile_sumsq) / K + eps))),
 * from n_tiles = ceil(K / 16) partial sums of h^2 (fx_hybrid_gemv_residual's or
 * fx_decode_embed's), norm_weight [K] 16-byte aligned, K <= 4096.
 */
int fx_hybrid_gemv_segments_rmsnormed(const void *h, int x_dtype, int n_segments, const int *segment_rows,
                                      const uint8_t *codes, const float *rows, const float *const *columns,
                                      const int16_t *const *indices, const uint8_t *sparse_codes,
                                      const float *sparse_rows, const float *const *sparse_columns,
                                      const float *tile_sumsq, int n_tiles, const void *norm_weight, float eps,
                                      void *workspace, size_t workspace_bytes, void *out, int K, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FLUXBIN_AMD_H */
