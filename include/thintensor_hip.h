/*
 * thintensor_hip.h — C ABI of the MI355X (gfx950) decode kernels.
 *
 * Each entry point replaces one operator of the reference's kernel backend
 * (`TritonDecodeBackend`, thinruntime/triton_kernels.py) and keeps its argument
 * meaning: destination-passing, packed layouts unchanged, row/expert strides given
 * explicitly, expert and token indices read from device memory.  Every call is
 * asynchronous on `stream` (a hipStream_t), allocates nothing, never synchronises,
 * and is safe to record into a HIP graph.
 *
 * Conventions
 *   - pointers are device pointers; sizes and strides are element counts unless the
 *     name ends in `_bytes`;
 *   - dtype codes: TT_F16, TT_BF16 (activations), TT_F32 (outputs / scales);
 *   - expert_indices arrays of the selected-expert operators hold int32 or int64
 *     ids (index_bytes 4 or 8), as the reference's kernels load whichever integer
 *     tensor the runtime passes (triton_kernels.py:439, 886, 956, 1157, 1240);
 *   - return value: TT_OK, or a negative code with a message in tt_last_error().
 *
 * Numerics: binary32 accumulation with a fixed, documented reduction order (see
 * the kernel sources), outputs rounded to nearest even.  Results are bit-for-bit
 * reproducible on the CPU.
 */
#ifndef THINTENSOR_HIP_H
#define THINTENSOR_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TT_OK 0
#define TT_ERR_INVALID (-1)     /* shape / dtype / stride / alignment contract violated */
#define TT_ERR_UNSUPPORTED (-2) /* valid for the reference, not provided by this build */
#define TT_ERR_HIP (-3)         /* HIP runtime reported an error at launch */

#define TT_F16 0
#define TT_BF16 1
#define TT_F32 2
#define TT_W_FP8 3   /* weight format code: float8_e4m3fn (scaled GEMVs, tt_split_k_matvec) */
#define TT_W_INT8 4  /* weight format code: int8 (the same entry points) */

/* Library version and last error (thread-local message of the last failing call). */
int tt_version(void);
const char* tt_last_error(void);

/* Lanes per output row used by the GEMV kernels for a K axis of `chunks` 32-element
 * chunks whose quantisation groups span `group_chunks` chunks (1 for per-row or
 * per-block scales).  Part of the documented reduction order; returns 0 if no
 * valid choice exists. */
int tt_gemv_lanes_per_row(int64_t chunks, int64_t group_chunks);

/* ---------------------------------------------------------------- GEMV family */

/* y[n] = sum_g s[n,g] * sum_{k in g} (c[n,k] - 8) x[k]            (affine == 0)
 * y[n] = sum_g (s[n,g] * sum_{k in g} c[n,k] x[k] + m[n,g] * sum_{k in g} x[k]) (affine)
 * packed: uint8 [rows, cols/2] (row stride w_row_bytes), k = 2b in the low nibble of
 * byte b, k = 2b+1 in the high nibble (== uint32 little-endian, 8 codes per word).
 * scales: fp16/fp32 [rows, groups] or [rows, groups, 2] (s, m) with element strides.
 * group_size >= cols means one scale per row.
 * Replaces TritonDecodeBackend.int4_scaled_matvec (triton_kernels.py:4597-4743;
 * kernels :1439-1652). */
int tt_int4_scaled_matvec(const void* packed, int64_t w_row_bytes,
                          const void* scales, int scale_dtype, int64_t s_row, int64_t s_group,
                          int64_t s_pair, int affine,
                          const void* x, int x_dtype, void* out, int out_dtype,
                          int64_t rows, int64_t cols, int64_t group_size, void* stream);

/* Two or three int4 matrices with a shared input written to one concatenated
 * output (QKV / gate-up in one launch).  All matrices share cols, group_size,
 * scale dtype and affine flag.
 * Replaces TritonDecodeBackend.multi_int4_scaled_matvec (triton_kernels.py:5066-5117). */
int tt_multi_int4_scaled_matvec(int count, const void* const* packed, const int64_t* w_row_bytes,
                                const void* const* scales, int scale_dtype, const int64_t* s_row,
                                const int64_t* s_group, int64_t s_pair, int affine,
                                const int64_t* rows, const void* x, int x_dtype,
                                void* out, int out_dtype, int64_t cols, int64_t group_size,
                                void* stream);

/* y[n] = (sum_k w[n,k] x[k]) * s[n], w [rows, cols] float8_e4m3fn (w_format TT_W_FP8) or
 * int8 (TT_W_INT8), s fp32 or fp16 [rows].  Replaces TritonDecodeBackend.scaled_matvec
 * for per-row scales (triton_kernels.py:4452-4595; kernels :539-592, :2990-3019, which
 * read either byte format). */
int tt_scaled_matvec(const void* weight, int w_format, int64_t w_row_bytes, const void* scales, int scale_dtype,
                     const void* x, int x_dtype, void* out, int out_dtype,
                     int64_t rows, int64_t cols, void* stream);

/* y[n] = sum_k w[n,k] x[k], w fp16/bf16 [rows, cols] (row stride in elements).
 * Replaces TritonDecodeBackend.matvec (triton_kernels.py:3701-3771). */
int tt_matvec(const void* weight, int w_dtype, int64_t w_row, const void* x, int x_dtype,
              void* out, int out_dtype, int64_t rows, int64_t cols, void* stream);

/* Two or three dense matrices, one launch, concatenated output.
 * Replaces TritonDecodeBackend.multi_matvec (triton_kernels.py:4978-5064). */
int tt_multi_matvec(int count, const void* const* weights, int w_dtype, const int64_t* w_row,
                    const int64_t* rows, const void* x, int x_dtype, void* out, int out_dtype,
                    int64_t cols, void* stream);

/* out[s, n] = sum_k e2m1(blocks[E_s, n, k/32, (k%32)/2]) * 2^(scales[E_s, n, k/32] - 127) * x_s[k]
 * with E_s = expert_indices[s] read on the device; x is [cols] (x_slot == 0) or
 * [selected, cols].  Element 2j of a block byte is the low nibble.
 * Replaces TritonDecodeBackend.mxfp4_selected_matvec (triton_kernels.py:3847-3911;
 * kernel :416-481). */
int tt_mxfp4_selected_matvec(const void* blocks, int64_t b_expert_bytes, int64_t b_row_bytes,
                             const void* scales, int64_t s_expert, int64_t s_row,
                             const void* x, int x_dtype, int64_t x_slot,
                             const void* expert_indices, int index_bytes, int64_t selected,
                             void* out, int out_dtype, int64_t out_slot,
                             int64_t rows, int64_t cols, void* stream);

/* Q1/Q2 experts with E8M0 block scales (32 elements per block):
 * q2 code c (byte i/4, bits 2(i%4)) -> {-1.5,-0.5,0.5,1.5}[c]; q1 bit (byte i/8,
 * bit i%8) -> +1 / -1; times 2^(e-127).
 * Replaces TritonDecodeBackend.mxfp_lowbit_selected_matvec
 * (triton_kernels.py:4132-4176; kernel :1137-1210). */
int tt_mxfp_lowbit_selected_matvec(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                   const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                   const void* x, int x_dtype, int64_t x_slot,
                                   const void* expert_indices, int index_bytes, int64_t selected,
                                   void* out, int out_dtype, int64_t out_slot,
                                   int64_t rows, int64_t cols, void* stream);

/* Ternary experts ({-a, 0, +a} per 32-element group), rows of w_row_bytes bytes:
 * bytes [0, ceil(cols/5)) hold five base-3 digits per byte (column k: byte k/5,
 * digit (b / 3^(k%5)) % 3; digit 1 = 0, 0 = negative, 2 = positive); the next
 * ceil(3*cols/32/8) bytes hold a 3-bit selector m per group at bit 3g, |w| =
 * e2m1(m + 1); scales are E8M0 [E, rows, cols/32] (w = (digit-1)*|w|*2^(e-127)).
 * `experts` = E; w_total_bytes / s_total_bytes bound every read.  Selected ids
 * outside [0, E) produce NaN rows.  Summation order (binary32): per group, the
 * column-order fma chain of digit*x minus the column-order sum of x; per 160-column
 * chunk, the groups' scaled sums in order; per row, the chunks in order.
 * Replaces TritonDecodeBackend.mxfp_ternary_selected_tensorcore_matvec
 * (triton_kernels.py:4057-4130; kernel :1022-1133; packer gpu_runtime.py:494-583). */
int tt_mxfp_ternary_selected_matvec(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                    int64_t w_total_bytes, const void* scales, int64_t s_expert,
                                    int64_t s_row, int64_t s_total_bytes, int64_t experts,
                                    const void* x, int x_dtype, int64_t x_slot,
                                    const void* expert_indices, int index_bytes, int64_t selected,
                                    void* out, int out_dtype, int64_t out_slot,
                                    int64_t rows, int64_t cols, void* stream);

/* Sparse residual sidecar: out[m] = out[m] + sum_k values[m,k] * x[indices[m,k]]
 * (values fp16/bf16/fp32 with element strides vm, vk; indices int16, int32 or int64,
 * index_bytes 2, 4 or 8, strides im, ik; int16 is the reference runtime's sidecar
 * layout, gpu_runtime.py:6468, and is sign-extended).  One wave per row: lane l sums
 * terms l, l+64, ... in order, then a butterfly over 64 lanes; an index outside
 * [0, cols) makes the row's correction NaN.
 * Replaces TritonDecodeBackend.sparse_residual_matvec (triton_kernels.py:5429-5456;
 * kernel :2335-2374). */
int tt_sparse_residual_matvec(const void* values, int value_dtype, int64_t vm, int64_t vk,
                              const void* indices, int index_bytes, int64_t im, int64_t ik,
                              const void* x, int x_dtype, void* out, int out_dtype,
                              int64_t rows, int64_t terms, int64_t cols, void* stream);

/* Binary residual sidecar: out[m] = out[m] + sum_k (bit ? +1 : -1) * scale[m, k/32] * x[k],
 * sign bit k at byte k/8 (row stride bm bytes), bit k%8.  One wave per row: lane l
 * owns 32-column groups l, l+64, ...; per group the column-order sum of +-x times
 * the scale, then a butterfly over 64 lanes.
 * Replaces TritonDecodeBackend.binary_residual_matvec (triton_kernels.py:5458-5487;
 * kernel :2377-2419). */
int tt_binary_residual_matvec(const void* packed_signs, int64_t bm, const void* scales, int scale_dtype,
                              int64_t sm, const void* x, int x_dtype, void* out, int out_dtype,
                              int64_t rows, int64_t cols, void* stream);

/* Fused gate/up GEMV on interleaved rows (2i gate, 2i+1 up) + gpt-oss SwiGLU;
 * bits 1/2 = E8M0 low-bit experts (bf16 rounding), bits 4 = MXFP4 blocks (rounding
 * in the activation dtype, the reference's unfused MXFP4 chain):
 * g = bf16(bf16(dot) + bias), u likewise; g = min(g, L); u = clamp(u, -L, L);
 * out = (u + 1) * g / (1 + exp(-alpha g)).  bias [E, 2I] (nullable).
 * Replaces TritonDecodeBackend.mxfp_lowbit_selected_swiglu
 * (triton_kernels.py:4178-4235; kernel :1214-1343). */
int tt_mxfp_lowbit_selected_swiglu(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                   const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                   const void* x, int x_dtype, int64_t x_slot,
                                   const void* expert_indices, int index_bytes, int64_t selected,
                                   const void* bias, int bias_dtype, int64_t bias_expert,
                                   float alpha, float limit,
                                   void* out, int out_dtype, int64_t out_slot,
                                   int64_t activation_rows, int64_t cols, void* stream);

/* out[n] = sum_s score_s * bf16(bf16(dot_s(n)) + bias[E_s, n]), summed in slot order.
 * Replaces TritonDecodeBackend.mxfp_lowbit_weighted_down
 * (triton_kernels.py:4237-4285; kernel :1347-1435). */
int tt_mxfp_lowbit_weighted_down(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                 const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                 const void* x, int x_dtype, int64_t x_slot,
                                 const void* expert_indices, int index_bytes, const void* router_scores,
                                 int score_dtype, int64_t selected,
                                 const void* bias, int bias_dtype, int64_t bias_expert,
                                 void* out, int out_dtype, int64_t rows, int64_t cols, void* stream);

/* out[t] = W x[t] (+ bias) for m activation rows (x rows x_row elements apart, out rows
 * out_row apart), fp16/bf16 dense W; each row equals tt_multi_matvec_bias on that row
 * alone.  No reference counterpart: it serves the batched decode of independent
 * sequences (the reference decodes one token per step). */
int tt_matvec_bias_rows(const void* weight, int w_dtype, int64_t w_row, const void* bias, const void* x,
                        int x_dtype, int64_t x_row, void* out, int out_dtype, int64_t out_row, int64_t m,
                        int64_t rows, int64_t cols, void* stream);

/* Several tokens at once, each with `selected` experts (no reference counterpart: the
 * reference decodes one token per step; these serve the batched decode of independent
 * sequences).  Token t's activation vector is x + t * x_token; its slots are
 * t * selected ... in expert_indices and in out (out_slot elements apart).  Each slot's
 * values equal tt_mxfp_lowbit_selected_swiglu on that token alone. */
int tt_mxfp_lowbit_selected_swiglu_tokens(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                          const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                          const void* x, int x_dtype, int64_t x_token,
                                          const void* expert_indices, int index_bytes, int64_t selected,
                                          const void* bias, int bias_dtype, int64_t bias_expert,
                                          float alpha, float limit, void* out, int out_dtype,
                                          int64_t out_slot, int64_t activation_rows, int64_t cols,
                                          int64_t tokens, void* stream);

/* Token t sums its `selected` slots (x rows t * selected ..., x_slot elements apart;
 * expert_indices and router_scores entries t * selected ...) into out + t * out_token;
 * each token's output equals tt_mxfp_lowbit_weighted_down on that token alone.  No
 * reference counterpart (batched decode of independent sequences). */
int tt_mxfp_lowbit_weighted_down_tokens(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                        const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                        const void* x, int x_dtype, int64_t x_slot,
                                        const void* expert_indices, int index_bytes, const void* router_scores,
                                        int score_dtype, int64_t selected, const void* bias, int bias_dtype,
                                        int64_t bias_expert, void* out, int out_dtype, int64_t out_token,
                                        int64_t rows, int64_t cols, int64_t tokens, void* stream);

/* Affine low-bit GEMV with fp16 (scale, zero) per group: w = (c - z) * s,
 * evaluated as sum_g fmaf(X_g, -(z_g s_g), S_g s_g).  bits 2: c in [0,3]
 * (byte i/4, bits 2(i%4)); bits 1: c in {0,1} (byte i/8, bit i%8).
 * No reference kernel: the dense-page analogue of the reference's affine int4
 * form (triton_kernels.py:1633-1649) for the ultra-low-bit layouts. */
int tt_lowbit_affine_matvec(const void* packed, int64_t w_row_bytes, const void* scale_zero,
                            int64_t s_row, int64_t s_group, int bits,
                            const void* x, int x_dtype, void* out, int out_dtype,
                            int64_t rows, int64_t cols, int64_t group_size, void* stream);

/* Selected-expert int4 GEMV: packed uint8 [E, rows, cols/2], scales [E, rows, groups].
 * Replaces TritonDecodeBackend.int4_selected_matvec (triton_kernels.py:4745-4805;
 * kernel :1656-1724). */
int tt_int4_selected_matvec(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                            const void* scales, int scale_dtype, int64_t s_expert, int64_t s_row,
                            int64_t s_group, const void* x, int x_dtype, int64_t x_slot,
                            const void* expert_indices, int index_bytes, int64_t selected,
                            void* out, int out_dtype, int64_t out_slot,
                            int64_t rows, int64_t cols, int64_t group_size, void* stream);

/* fp8 / int8 GEMV with per-block scales: y[m] = sum_b s[m*s_row + b*s_block] *
 * sum_{k in block b} w[m,k] x[k], blocks of `block` columns (a power of two; the last may
 * be partial; a block as wide as the row is the per-row-scale GEMV).  Blocks of 32 to
 * 2048 columns; w_format TT_W_FP8 or TT_W_INT8.  Replaces the block-scaled branch of
 * TritonDecodeBackend.scaled_matvec (triton_kernels.py:4465-4497; kernel :3113-3152). */
int tt_block_scaled_matvec(const void* weight, int w_format, int64_t w_row_bytes, const void* scales,
                           int scale_dtype, int64_t s_row, int64_t s_block, int64_t block, const void* x,
                           int x_dtype, void* out, int out_dtype, int64_t rows, int64_t cols, void* stream);

/* One to three fp8 or int8 matrices (one w_format for all) with per-row scales (scale i
 * of matrix j at scales[j][i * s_stride[j]]) over one activation vector; outputs
 * concatenated in matrix order.  Replaces TritonDecodeBackend.multi_scaled_tensorcore_matvec
 * (triton_kernels.py:5119-5180; kernel :1958-2071, IS_FP8 selecting the byte format). */
int tt_multi_scaled_matvec(int count, const void* const* weights, int w_format, const int64_t* w_row_bytes,
                           const void* const* scales, int scale_dtype, const int64_t* s_stride,
                           const int64_t* rows, const void* x, int x_dtype, void* out, int out_dtype,
                           int64_t cols, void* stream);

/* Split-K GEMV: K cut into split_k (2, 4 or 8) slices of whole 32-column chunks; binary32
 * row sums of each slice go to partials[s * rows + m] (caller scratch of split_k * rows
 * floats), then y = ((0 + p_0) + p_1 + ...) * scale (scales nullable).  w_format TT_F16,
 * TT_BF16, TT_W_FP8 or TT_W_INT8.  Replaces TritonDecodeBackend.split_k_matvec
 * (triton_kernels.py:3773-3845; kernels :3023-3100). */
int tt_split_k_matvec(const void* weight, int w_format, int64_t w_row_bytes, const void* scales, int scale_dtype,
                      const void* x, int x_dtype, void* out, int out_dtype, int64_t rows, int64_t cols,
                      int split_k, float* partials, int64_t partials_capacity, void* stream);

/* Fused fp8 / int8 gate/up GEMV + SiLU: out[m] = silu(g) * u with
 * g = bf16((W_g[m] . x) * s_g[m]) and u = bf16((W_u[m] . x) * s_u[m]) (bfloat16 rounding
 * whatever the activation dtype); both matrices in w_format TT_W_FP8 or TT_W_INT8.  Each
 * dot product has the reduction order of tt_scaled_matvec.  Replaces
 * TritonDecodeBackend.fused_scaled_gate_up_silu (triton_kernels.py:4346-4436; kernels
 * :3243-3350). */
int tt_scaled_gate_up_silu(const void* gate_weight, int64_t wg_row_bytes, const void* gate_scales,
                           int64_t sg_stride, const void* up_weight, int64_t wu_row_bytes, const void* up_scales,
                           int64_t su_stride, int w_format, int scale_dtype, const void* x, int x_dtype,
                           void* out, int out_dtype, int64_t rows, int64_t cols, void* stream);

/* Greedy lm_head: logits = round(W x) (stored when `logits` is non-null), token =
 * first index of the maximum rounded logit (NaN counts as the maximum, +0 == -0),
 * written as int64 to out_idx and the value to out_val (nullable).  `partials` is
 * caller scratch of tt_matvec_argmax_partials(rows, cols) uint64 entries.
 * Replaces TritonDecodeBackend.matvec_argmax_tensor and its two-stage / persistent
 * variants (triton_kernels.py:5365-5398, 5516-5625; kernels :2222-2285, :2456-2558). */
int64_t tt_matvec_argmax_partials(int64_t rows, int64_t cols);
int tt_matvec_argmax(const void* weight, int w_dtype, int64_t w_row, const void* x, int x_dtype,
                     void* logits, int logits_dtype, int64_t rows, int64_t cols, uint64_t* partials,
                     int64_t partials_capacity, int64_t* out_idx, float* out_val, void* stream);

/* No-allocation greedy lm_head: tt_matvec_argmax with its argmax partials in a
 * library-owned device array of TT_NOALLOC_ARGMAX_KEYS uint64 keys (64 KiB per GPU,
 * held until the process ends) instead of caller scratch; it calls no hipMalloc or
 * hipFree.  Every shape tt_matvec_argmax accepts fits.  Calls that overlap on one GPU
 * share the array and race; serialize them (one stream, or events).
 * No counterpart in the reference: it is for callers that cannot allocate device
 * memory (HIP graph capture, tight serving loops, harnesses that forbid allocation). */
#define TT_NOALLOC_ARGMAX_KEYS 8192
int tt_matvec_argmax_noalloc(const void* weight, int w_dtype, int64_t w_row, const void* x, int x_dtype,
                             void* logits, int logits_dtype, int64_t rows, int64_t cols, int64_t* out_idx,
                             float* out_val, void* stream);

/* tt_multi_matvec with a per-matrix bias (nullable entries) fused into the
 * epilogue: out = round(round(dot) + bias), identical to the runtime's GEMV followed
 * by its in-place bias add (gpu_runtime.py:9100-9114, 9213-9221). */
int tt_multi_matvec_bias(int count, const void* const* weights, int w_dtype, const int64_t* w_row,
                         const int64_t* rows, const void* const* biases, const void* x, int x_dtype,
                         void* out, int out_dtype, int64_t cols, void* stream);

/* ---------------------------------------------------------------- norms / elementwise */

/* out = x * (1 / sqrt(mean(x^2) + eps)) * (w + weight_offset)
 * Replaces TritonDecodeBackend.rms_norm (triton_kernels.py:5632-5644; kernel :2562-2577). */
int tt_rms_norm(const void* x, int x_dtype, const void* weight, int w_dtype, void* out, int out_dtype,
                int64_t n, float eps, float weight_offset, void* stream);

/* residual_out = bf16(left + right); out = residual * rsqrt(mean(residual^2) + eps) * w
 * Replaces TritonDecodeBackend.add_rms_norm (triton_kernels.py:5646-5667; kernel :2581-2614). */
int tt_add_rms_norm(const void* left, const void* right, void* residual_out, int x_dtype,
                    const void* weight, int w_dtype, void* out, int out_dtype, int64_t n, float eps,
                    void* stream);

/* For each of `rows` rows (row stride `row` for left/right/sum_out, `out_row` for out):
 * sum_out = left + right rounded to x_dtype, then out = rms_norm(sum_out) * weight --
 * tt_add followed by tt_rms_norm (weight offset 0) per row, bit for bit, in one launch.
 * The batched form of TritonDecodeBackend.add + rms_norm (triton_kernels.py:5862-5873,
 * 5632-5644) at the end of a batched decode step.  n a multiple of 8 up to 4096,
 * 16-byte aligned rows. */
int tt_add_then_rms_norm_rows(const void* left, const void* right, void* sum_out, int x_dtype, int64_t row,
                              const void* weight, int w_dtype, void* out, int out_dtype, int64_t out_row, int64_t rows,
                              int64_t n, float eps, void* stream);

/* out = a + b.  Replaces TritonDecodeBackend.add (triton_kernels.py:5862-5873). */
int tt_add(const void* a, const void* b, void* out, int dtype, int64_t n, void* stream);

/* out = silu(gate) * up.  Replaces TritonDecodeBackend.silu_mul (triton_kernels.py:5751-5762). */
int tt_silu_mul(const void* gate, const void* up, void* out, int dtype, int64_t n, void* stream);

/* gpt-oss SwiGLU on interleaved gate/up rows [rows, 2n] -> [rows, n].
 * Replaces TritonDecodeBackend.interleaved_swiglu (triton_kernels.py:5764-5782). */
int tt_interleaved_swiglu(const void* gate_up, int64_t in_row, void* out, int64_t out_row, int dtype,
                          int64_t rows, int64_t n, float alpha, float limit, void* stream);

/* out[n] = sum_e experts[e, n] * scores[e] in expert order.
 * Replaces TritonDecodeBackend.weighted_expert_sum (triton_kernels.py:5784-5801). */
int tt_weighted_expert_sum(const void* experts, int dtype, int64_t stride, int64_t count,
                           const void* scores, int score_dtype, void* out, int64_t width, void* stream);

/* In-place RoPE of q [heads, D] and k [kv_heads, D] with cos/sin rows taken from a
 * [table_rows, D/2] table at the position read from position_dev (if non-null) or
 * `position`; a device position outside the table leaves q and k unchanged.  Replaces TritonDecodeBackend.rope_qk_inplace
 * (triton_kernels.py:5689-5714; kernel :2638-2687), with the position on the device. */
int tt_rope_qk_inplace(void* q, void* k, int dtype, const void* cos_table, const void* sin_table,
                       int64_t table_row, int64_t table_rows, const int32_t* position_dev, int64_t position,
                       int64_t heads, int64_t kv_heads, int64_t head_dim, void* stream);

/* Per-head RMSNorm: out[h*D + i] = (x * (1 / sqrt(mean_h(x^2) + eps))) * w[i], heads of
 * head_dim <= 512.  Replaces TritonDecodeBackend.head_rms_norm (triton_kernels.py:
 * 5669-5687; kernel :2618-2634). */
int tt_head_rms_norm(const void* x, int dtype, const void* weight, int w_dtype, void* out, int64_t heads,
                     int64_t head_dim, float eps, void* stream);

/* Per-head RMSNorm then RoPE in place on q heads and k heads: a' = a * (inv * w[i]),
 * b' = b * (inv * w[i + half]), then (a' c - b' s, b' c + a' s) in binary32 with cos/sin
 * taken from a table row (device or host position, as tt_rope_qk_inplace); head_dim <= 512.
 * Replaces TritonDecodeBackend.qk_head_rmsnorm_rope_inplace (triton_kernels.py:5716-5749;
 * kernel :2691-2757). */
int tt_qk_head_rmsnorm_rope_inplace(void* q, void* k, int dtype, const void* q_weight, const void* k_weight,
                                    int w_dtype, const void* cos_table, const void* sin_table, int64_t table_row,
                                    int64_t table_rows, const int32_t* position_dev, int64_t position, int64_t heads,
                                    int64_t kv_heads, int64_t head_dim, float eps, void* stream);

/* out = embed[token] with the token read from token_dev (int64) if non-null; a device
 * token outside [0, vocab) leaves out unchanged.
 * Replaces the runtime's embedding row copy (gpu_runtime.py:11396-11427). */
int tt_embedding(const void* embed, int64_t row_stride, int64_t vocab, const int64_t* token_dev, int64_t token,
                 void* out, int64_t n, void* stream);

/* keys[h, pos, :] = k[h, :]; values[h, pos, :] = v[h, :] (16-bit elements); a device
 * position outside [0, capacity) writes nothing.
 * Replaces PagedKVCache.append for a flat cache (gpu_runtime.py:4132-4229). */
int tt_kv_append(const void* k, const void* v, void* keys, void* values, int64_t stride_head,
                 int64_t stride_token, const int32_t* position_dev, int64_t position, int64_t capacity,
                 int64_t kv_heads, int64_t head_dim, void* stream);

/* position_dev[0] += step (keeps graph replays moving along the sequence). */
int tt_advance_position(int32_t* position_dev, int32_t step, void* stream);

/* history[position - base] = token, all read on the device (token log of graph
 * replays); indices outside [0, capacity) are skipped. */
int tt_record_token(const int64_t* token_dev, const int32_t* position_dev, const int32_t* base_dev,
                    int64_t* history, int32_t capacity, void* stream);

/* Batched token log of a decode batch: history[r * history_row + position - base] =
 * tokens[r] for r < count (indices outside [0, capacity) skipped), then position +=
 * step -- tt_record_token per row followed by tt_advance_position, in one launch.
 * No reference counterpart (graph-replay helper of the batched decoder). */
int tt_record_tokens_advance(const int64_t* tokens_dev, int32_t count, int32_t* position_dev, const int32_t* base_dev,
                             int64_t* history, int64_t history_row, int32_t capacity, int32_t step, void* stream);

/* ---------------------------------------------------------------- attention / router */

/* Floats of scratch tt_single_token_gqa_attention needs.  The scratch must be
 * zero-filled before its first use (its head holds arrival counters that every call
 * leaves at zero); calls sharing one scratch must be ordered (same stream). */
int tt_attention_scratch_floats(int64_t heads, int64_t max_tokens, int64_t head_dim);

/* Single-token GQA attention over keys/values [kv_heads, tokens, D] (strides in
 * elements) with optional sinks [heads]; the token count is `tokens`, or
 * tokens_dev[0] + tokens when tokens_dev (int32) is non-null (a decode step passes its
 * position and 1).  max_tokens bounds the count (it sizes the scratch).  out [heads, D].
 * Replaces TritonDecodeBackend.single_token_gqa_attention and
 * split_single_token_gqa_attention (triton_kernels.py:5228-5363; kernels :15-245). */
int tt_single_token_gqa_attention(const void* q, const void* keys, const void* values, int dtype,
                                  int64_t k_head, int64_t k_tok, int64_t v_head, int64_t v_tok,
                                  const void* sinks, int sink_dtype, const int32_t* tokens_dev,
                                  int64_t tokens, int64_t max_tokens, int64_t heads, int64_t kv_heads,
                                  int64_t head_dim, float* scratch, int64_t scratch_floats, void* out,
                                  void* stream);

/* Attention then o_proj in two launches, the decode step's single_token_gqa_attention
 * followed by the o_proj int4_scaled_matvec (triton_kernels.py:5228-5278, then the
 * o_proj matvec of gpu_runtime.py's layer loop).  The first call stores the chunk
 * partials into the attention scratch only (head_dim-64 caches of whole 64-token
 * chunks, 1/2/4/8 query heads per KV head, no sinks); the second combines them into the
 * activation -- the bits tt_single_token_gqa_attention writes to `out` -- and runs the
 * int4 group-128 GEMV (fp16 scales [rows, cols/128] with strides s_row, s_group) over it:
 * out [rows] = W [rows, heads*64] x combined.  attn_out (optional) receives the
 * combined activation.  At most 32 query heads; same scratch, token count and capacity
 * in both calls, on one stream. */
int tt_single_token_gqa_attention_partials(const void* q, const void* keys, const void* values, int dtype,
                                           int64_t k_head, int64_t k_tok, int64_t v_head, int64_t v_tok,
                                           const int32_t* tokens_dev, int64_t tokens, int64_t max_tokens,
                                           int64_t heads, int64_t kv_heads, int64_t head_dim, float* scratch,
                                           int64_t scratch_floats, void* stream);
int tt_attention_combine_int4_matvec(const float* scratch, int64_t scratch_floats, const int32_t* tokens_dev,
                                     int64_t tokens, int64_t max_tokens, int64_t heads, int64_t head_dim, int dtype,
                                     const void* packed, int64_t w_row_bytes, const void* scales, int64_t s_row,
                                     int64_t s_group, void* attn_out, void* out, int64_t rows, void* stream);

/* Router GEMV + bias + top-k + softmax (E <= 128), logits rounded through bf16.
 * Replaces TritonDecodeBackend.moe_router_matvec_topk (triton_kernels.py:5826-5860;
 * kernel :2855-2921). */
int tt_moe_router_matvec_topk(const void* weight, int w_dtype, int64_t w_row, const void* hidden,
                              int x_dtype, int64_t hidden_size, const void* bias, int bias_dtype,
                              int64_t experts, int64_t top_k, int renormalize, int32_t* indices_out,
                              void* scores_out, int score_dtype, void* stream);

/* add_rms_norm followed by moe_router_matvec_topk on its output, in one launch when
 * experts <= 32, hidden_size <= 4096 and the activations, norm weight and norm output share
 * an fp16/bf16 dtype (otherwise the two operators run one after the other).  Outputs and
 * bits are those of tt_add_rms_norm then tt_moe_router_matvec_topk(hidden = norm_out).
 * `tokens` rows at once: left/right/residual_out/norm_out [tokens, hidden_size],
 * indices/scores [tokens, top_k], all contiguous.
 * Fuses the reference's add_rms_norm (triton_kernels.py:5646-5667) and
 * moe_router_matvec_topk (:5826-5860) as its MoE layer calls them back to back
 * (gpu_runtime.py:9465-9513); the reference has no single entry point for the pair.
 * With a workspace of tt_norm_router_workspace_bytes(tokens) bytes, zero-filled before
 * its first use, each token's router rows are spread over ceil(experts / 4)
 * workgroups and the last one to finish takes the top-k (it leaves the workspace
 * zeroed; calls sharing one workspace must be ordered); without one, a single
 * workgroup per token does everything.  Same bits either way. */
int64_t tt_norm_router_workspace_bytes(int64_t tokens);
int tt_add_rms_norm_router_topk(const void* left, const void* right, void* residual_out, int x_dtype,
                                const void* norm_weight, int norm_w_dtype, void* norm_out, int norm_dtype,
                                int64_t hidden_size, float eps, const void* weight, int w_dtype, int64_t w_row,
                                const void* bias, int bias_dtype, int64_t experts, int64_t top_k, int renormalize,
                                int32_t* indices_out, void* scores_out, int score_dtype, int64_t tokens,
                                void* workspace, int64_t workspace_bytes, void* stream);

/* tt_add_rms_norm_router_topk without the top-k: residual_out and norm_out as there, and
 * logits_out[t * experts + e] the router logit it ranks (bf16-rounded dot product, plus the
 * bias rounded again), in one launch of ceil(experts / 4) workgroups per token with no
 * arrival count.  The decode step's SwiGLU then runs the top-k on these logits
 * (tt_mxfp_lowbit_selected_swiglu_router).  experts <= 32, hidden_size <= 4096.  Serves
 * the same reference call pair as tt_add_rms_norm_router_topk (gpu_runtime.py:9465-9513). */
int tt_add_rms_norm_router_logits(const void* left, const void* right, void* residual_out, int x_dtype,
                                  const void* norm_weight, int norm_w_dtype, void* norm_out, int norm_dtype,
                                  int64_t hidden_size, float eps, const void* weight, int w_dtype, int64_t w_row,
                                  const void* bias, int bias_dtype, int64_t experts, float* logits_out,
                                  int64_t tokens, void* stream);

/* tt_mxfp_lowbit_selected_swiglu_tokens with the router's top-k folded in: router_logits
 * [tokens, experts] fp32 as tt_add_rms_norm_router_logits writes them.  Every wave runs
 * the top-k + softmax of its token (tt_moe_router_topk's selection and scores, bit for
 * bit) and takes its slot's expert; slot t * selected + k is token t's k-th choice.  The
 * slots' experts and scores (renormalized over the selected experts or not, score_dtype
 * fp16/bf16/fp32) also go to indices_out / scores_out [tokens, selected] for the
 * weighted-down.  experts <= 128, rows of at most four rounds of lanes and 8192 columns.
 * Replaces the reference's moe_router_matvec_topk + mxfp_lowbit_selected_swiglu pair
 * (triton_kernels.py:5826-5860, 4178-4235) as gpu_runtime.py:9465-9513 calls it. */
int tt_mxfp_lowbit_selected_swiglu_router(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                          const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                          const void* x, int x_dtype, int64_t x_token,
                                          const float* router_logits, int64_t experts, int64_t selected,
                                          int renormalize, int32_t* indices_out, void* scores_out,
                                          int score_dtype, const void* bias, int bias_dtype,
                                          int64_t bias_expert, float alpha, float limit, void* out,
                                          int out_dtype, int64_t out_slot, int64_t activation_rows,
                                          int64_t cols, int64_t tokens, void* stream);

/* Top-k + softmax on given logits, any expert count up to 65536 (one wave up to 128
 * experts, one workgroup above; above 128 experts top_k is at most 4096).  The
 * runtime calls it exactly when the router has more than 128 rows
 * (gpu_runtime.py:9474-9496).  Replaces TritonDecodeBackend.moe_router_topk
 * (triton_kernels.py:5803-5824; kernel :2821-2851). */
int tt_moe_router_topk(const void* logits, int logits_dtype, int64_t experts, int64_t top_k, int renormalize,
                       int32_t* indices_out, void* scores_out, int score_dtype, void* stream);

/* ---------------------------------------------------------------- batched small-M GEMM
 *
 * y[m] = W x[m] for M activation rows x [M, x_row] (fp16), y [M, out_row] (fp16).
 * The reference has no batched variant (its kernels take one activation vector and
 * its tensor-core variants broadcast it, triton_kernels.py:596-638); these extend
 * TritonDecodeBackend.int4_scaled_matvec (:4597-4743) and scaled_matvec (:4452-4595)
 * to M rows.  Small M (int4: M < 4, fp8: M < 16) runs the GEMV engine on up to four
 * rows per launch (row m equals the single-row operator bit for bit); from there (up
 * to 64) an MFMA kernel runs whose fp32 sums follow the hardware's order (tolerance
 * parity).  cols must be a multiple of 256 up to 8192.  The MFMA path is one launch
 * with no workspace: one workgroup per CU owns a block of weight rows for every
 * activation row, its four waves split K, and their fp32 tiles are summed in a fixed
 * order inside the workgroup, so the result is the same from run to run.
 * tt_batched_workspace_floats returns 0 and the workspace arguments are accepted and
 * unused (kept for callers written against a workspace-taking build). */
int64_t tt_batched_workspace_floats(int64_t m, int64_t rows, int64_t cols);
int tt_int4_batched_matvec(const void* packed, int64_t w_row_bytes, const void* scales_f16, int64_t s_row,
                           const void* x, int64_t x_row, void* out, int64_t out_row, int64_t m, int64_t rows,
                           int64_t cols, int64_t group_size, float* workspace, int64_t workspace_floats,
                           void* stream);
/* fp8-e4m3 rows with an fp32 scale per output row (applied to the fp32 sum). */
int tt_scaled_batched_matvec(const void* weight, int64_t w_row_bytes, const float* scales, const void* x,
                             int64_t x_row, void* out, int64_t out_row, int64_t m, int64_t rows, int64_t cols,
                             float* workspace, int64_t workspace_floats, void* stream);

/* Greedy lm_head for M activation rows: out_idx[m] = first index of the maximum of
 * round(W x[m]) (the tt_matvec_argmax semantics per row), logits [M, logits_row]
 * stored when non-null.  `partials` needs tt_matvec_argmax_batched_partials(m, rows,
 * cols) entries.  Extends matvec_argmax_tensor (triton_kernels.py:5365-5398) to M
 * rows. */
int64_t tt_matvec_argmax_batched_partials(int64_t m, int64_t rows, int64_t cols);
int tt_matvec_argmax_batched(const void* weight, int64_t w_row, const void* x, int64_t x_row, int64_t m,
                             void* logits, int64_t logits_row, int64_t rows, int64_t cols, uint64_t* partials,
                             int64_t partials_capacity, int64_t* out_idx, float* out_val, void* stream);

/* ---------------------------------------------------------------- fused decode-step GEMVs
 *
 * One launch of the GEMV engine with the neighbouring decode-step operators folded
 * in.  These have no single counterpart in the reference: they fuse, per launch,
 * operators the reference issues back to back in _forward_token_triton
 * (gpu_runtime.py:11429-11726) and _forward_token_moe (:8968-9908), with each
 * operator's own rounding points, so the outputs equal the unfused sequence bit for
 * bit:
 *   prologue  TT_PRO_ADD_NORM:   add_rms_norm (triton_kernels.py:5646-5667) producing
 *                                the GEMV input (residual_out written once);
 *             TT_PRO_EMBED_NORM: embedding row copy + rms_norm (gpu_runtime.py:11396-11427,
 *                                triton_kernels.py:5632-5644);
 *             TT_PRO_ADD_RMS_NORM: add (:5862-5873) then rms_norm, the final norm of the MoE
 *                                step (gpu_runtime.py:9338-9349);
 *   segments  TT_SEG_ROPE_OUT / TT_SEG_ROPE_CACHE: rope_qk_inplace (:5689-5714) on the q / k
 *                                rows, k then stored to the cache at the device position
 *                                like the KV append (gpu_runtime.py:4132-4229);
 *             TT_SEG_CACHE:      v rows stored to the cache at the position;
 *             TT_SEG_SILU:       silu_mul (:5751-5762) of the gate and up rows;
 *             TT_SEG_PLAIN:      the GEMV output (+ bias, as multi_matvec_bias).
 * Weight formats: TT_FMT_INT4_G (symmetric int4, fp16 scales, group 128) and
 * TT_FMT_DENSE (fp16 / bf16 rows).  Activations and outputs use act_dtype. */
#define TT_FMT_INT4_G 0
#define TT_FMT_DENSE 1
#define TT_PRO_LOAD 0
#define TT_PRO_ADD_NORM 1
#define TT_PRO_EMBED_NORM 2
#define TT_PRO_ADD_RMS_NORM 3
#define TT_SEG_PLAIN 0
#define TT_SEG_ROPE_OUT 1
#define TT_SEG_ROPE_CACHE 2
#define TT_SEG_CACHE 3
#define TT_SEG_SILU 4

typedef struct tt_fused_segment {
  const void* weight;      /* int4: uint8 [rows, cols/2]; dense: [rows, cols] */
  const void* weight2;     /* TT_SEG_SILU: the up-projection rows, same layout */
  int64_t w_row_bytes;
  const void* scales;      /* int4: fp16 [rows, cols/group] */
  const void* scales2;     /* TT_SEG_SILU: scales of weight2 */
  int64_t s_row;           /* scale elements between rows */
  void* out;               /* output vector, or this layer's cache [kv_heads, capacity, head_dim] */
  const void* bias;        /* TT_FMT_DENSE only; nullable */
  int64_t rows;            /* output rows (TT_SEG_SILU: activation rows) */
  int32_t kind;            /* TT_SEG_* */
  int32_t reserved;
} tt_fused_segment;

typedef struct tt_fused_gemv {
  int32_t weight_format;   /* TT_FMT_* */
  int32_t weight_dtype;    /* TT_FMT_DENSE: TT_F16 / TT_BF16 */
  int64_t group_size;      /* TT_FMT_INT4_G */
  int32_t act_dtype;       /* TT_F16 / TT_BF16 */
  int32_t prologue;        /* TT_PRO_* */
  int64_t cols;
  const void* x;           /* TT_PRO_LOAD */
  const void* left;        /* TT_PRO_ADD_NORM: residual = bf16(left + right); TT_PRO_ADD_RMS_NORM: round(left + right) */
  const void* right;
  const void* embed;       /* TT_PRO_EMBED_NORM: residual = embed[token[0]] (token clamped to [0, vocab)) */
  int64_t embed_row;
  int64_t vocab;
  const int64_t* token;
  const void* norm_weight; /* RMSNorm weight [cols], act_dtype */
  float eps;
  int32_t count;           /* segments, 1 to 3 */
  void* residual_out;      /* nullable */
  tt_fused_segment seg[3];
  const int32_t* position; /* device position for RoPE / cache segments */
  int64_t capacity;        /* cache tokens */
  int64_t cache_head;      /* elements between KV heads of one layer's cache */
  const void* cos_table;   /* [table_rows, table_row], act_dtype */
  const void* sin_table;
  int64_t table_row;
  int64_t table_rows;
  int64_t head_dim;
  /* Several tokens (independent sequences at one shared position) in one launch; 0 or 1
   * = one.  Token t reads x / left / right / embed row token[t] and writes residual_out
   * at + t * token_x elements, TT_SEG_PLAIN / ROPE_OUT / SILU outputs at + t * token_out
   * and ROPE_CACHE / CACHE outputs at + t * token_cache.  Each token's values equal the
   * one-token launch's.  Not for the lm_head. */
  int64_t tokens;
  int64_t token_x;
  int64_t token_out;
  int64_t token_cache;
} tt_fused_gemv;

int tt_fused_gemv_run(const tt_fused_gemv* desc, void* stream);

/* sizeof(tt_fused_segment) and sizeof(tt_fused_gemv), so bindings can check their layout. */
int tt_fused_struct_sizes(int64_t* segment_size, int64_t* desc_size);

/* Fused greedy lm_head: the prologue of `desc` builds the input, seg[0] (TT_FMT_DENSE,
 * TT_SEG_PLAIN, out = logits or null) is the lm_head, the token is chosen as by
 * tt_matvec_argmax, and then, when position is non-null, the step's bookkeeping
 * runs in the same finishing kernel: history[position - base] = token (skipped
 * outside [0, history_len)) and position += 1 -- the sequence record_token +
 * advance_position of a decode step.  `partials` needs
 * tt_matvec_argmax_partials(rows, cols) entries. */
int tt_fused_lm_head_argmax(const tt_fused_gemv* desc, uint64_t* partials, int64_t partials_capacity,
                            int64_t* out_idx, float* out_val, int32_t* position, const int32_t* base,
                            int64_t* history, int32_t history_len, void* stream);

/* Memory-floor reference (measurement utility; no counterpart in the reference): a
 * pure streaming read of `bytes` (a multiple of 16) in contiguous spans of bytes_per_wave
 * (a multiple of 2048) per wave, one 32-bit word stored per wave into `out`
 * (tt_stream_read_waves(bytes, bytes_per_wave) words).  Used to time the fastest
 * single launch that moves a given number of bytes. */
int64_t tt_stream_read_waves(int64_t bytes, int64_t bytes_per_wave);
int tt_stream_read(const void* data, int64_t bytes, int64_t bytes_per_wave, void* out, int64_t out_words,
                   void* stream);

/* ---------------------------------------------------------------- load-time quantizers
 * Device-side packers of the layouts the GEMV kernels read.  Sources are row-major
 * [rows, cols] fp16/bf16/fp32 (src_row elements between rows); outputs are contiguous.
 * Group sums are taken in binary64 in a fixed lane order and rounded once, so results
 * agree with the reference's binary32 torch sums except at near-ties that the
 * reference's own summation order decides. */

#define TT_Q4_LSQ 0          /* quantize_to_int4_cpu: amax/7, one least-squares refit, codes [-8,7]+8, fp16 scales [rows, groups] */
#define TT_Q4_LSQ_AFFINE 1   /* quantize_to_int4_cpu, THINTENSOR_AFFINE_INT4=1: min/max line, 2 refits + final refit, codes [0,15], fp16 [rows, groups, 2] */
#define TT_Q4_ROWS 2         /* _quantize_int4_rows: amax/7, codes [-7,7]+8, fp32 scales [rows, groups] */
#define TT_Q4_ROWS_AFFINE 3  /* _quantize_int4_rows affine: min/max line, codes [0,15], fp32 [rows, groups, 2] */

/* Grouped INT4 (two codes per byte, even column in the low nibble) for group sizes
 * 32..512 (powers of two); importance [cols] (binary32 max(rms^2, 1e-8)) only with
 * TT_Q4_LSQ_AFFINE.  gptq_factors (nullable; TT_Q4_LSQ_AFFINE with groups of 32 only):
 * device fp32 [groups, 32, 32], per group the upper Cholesky factor U of the inverse
 * damped input covariance; after the affine fit two GPTQ passes requantize the group
 * column by column, spreading each column's error (divided by U[c][c]) over the later
 * columns along row c of U, with one refit of the line between the passes.  Replaces
 * quantize_to_int4_cpu (gpu_runtime.py:91-304) and
 * ThinGpuCausalLMRuntime._quantize_int4_rows (gpu_runtime.py:6609-6700). */
int tt_quantize_int4(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t src_row,
                     int64_t group_size, int mode, const float* importance, const float* gptq_factors,
                     uint8_t* packed, void* scales, void* stream);

/* float8_e4m3fn rows with fp32 scales max(amax, 1e-12)/448 per row (block == 0, scales
 * [rows]) or per block of columns (scales [rows, ceil(cols/block)]).  via_bf16 rounds the
 * source and x/scale through bfloat16 first.  Replaces
 * ThinGpuCausalLMRuntime._quantize_fp8_rows (gpu_runtime.py:6551-6607) and
 * quantize_to_fp8_via_gpu (:40-88). */
int tt_quantize_fp8_rows(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t src_row,
                         int64_t block, int via_bf16, uint8_t* out, float* scales, void* stream);

/* Native MXFP4 rows: packed [rows, cols/2] nibbles and E8M0 scales [rows, cols/32];
 * optional Walsh-Hadamard blocks of `transform` (0 or 32..512) with sign flips `signs`
 * [cols] (source dtype), and the binary-residual error criterion.  Replaces
 * ThinGpuCausalLMRuntime._quantize_mxfp4_rows (gpu_runtime.py:6702-6812). */
int tt_quantize_mxfp4_rows(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t src_row,
                           int64_t transform, const void* signs, int binary_residual, uint8_t* packed,
                           uint8_t* scales, void* stream);

/* MXFP4 groups (blocks [n, 16] bytes, E8M0 scales [n]) to Q2 ([n, 8]) or Q1 ([n, 4])
 * groups with the MSE-chosen exponent offset.  Replaces quantize_mxfp4_to_lowbit_cpu
 * (gpu_runtime.py:306-395). */
int tt_requantize_mxfp4_lowbit(const uint8_t* blocks, const uint8_t* scales, int64_t n_groups, int bits,
                               uint8_t* out, uint8_t* out_scales, void* stream);

/* Dense rows to Q2/Q1 E8M0 groups: out [rows, cols/32, 8 or 4], scales [rows, cols/32].
 * Replaces quantize_dense_to_mxfp_lowbit_cpu (gpu_runtime.py:398-491). */
int tt_quantize_dense_lowbit(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t src_row,
                             int bits, uint8_t* out, uint8_t* out_scales, void* stream);

/* MXFP4 rows (blocks [rows, groups, 16]) to the ternary layout [rows, ceil(32 groups/5)
 * + ceil(3 groups/8)] (five base-3 digits per byte, then 3-bit magnitude selectors);
 * the E8M0 scales are kept as they are.  Rows up to 16384 columns.  Replaces
 * quantize_mxfp4_to_ternary_cpu (gpu_runtime.py:494-583). */
int tt_pack_mxfp4_ternary(const uint8_t* blocks, int64_t rows, int64_t groups, uint8_t* out, void* stream);

/* ---------------------------------------------------------------- .thin archives
 * Memory-mapped reader of ThinTensor v0 archives (header, JSON manifest, page table,
 * payload).  Replaces the binary parsing and checks of ThinArchive
 * (thinruntime/archive.py:99-208, 248-254; format src/archive.rs:14-41, 583-662) with
 * the same messages; the manifest JSON and its page index stay with the caller.  The
 * validation comes in the reference's order: tt_archive_open (header),
 * tt_archive_parse_pages (page table, data_off), tt_archive_check_overlaps. */
typedef struct tt_archive tt_archive;

typedef struct {
  uint32_t header_len, version;
  uint64_t manifest_off, manifest_len, page_table_off, page_count, data_off;
  uint8_t archive_hash[32];
  uint64_t file_size;
  const uint8_t* manifest; /* manifest_len bytes inside the mapping */
} tt_archive_info;

typedef struct {
  const char* id; /* id_len bytes of UTF-8 inside the mapping (not terminated) */
  int64_t id_len;
  uint64_t offset, stored_size, raw_size;
  uint32_t flags;
  uint8_t checksum[32];
} tt_archive_record;

int tt_archive_open(const char* path, tt_archive** out);
int tt_archive_parse_pages(tt_archive* archive);
int tt_archive_check_overlaps(const tt_archive* archive);
int tt_archive_get_info(const tt_archive* archive, tt_archive_info* out);
int tt_archive_get_record(const tt_archive* archive, int64_t index, tt_archive_record* out);
/* Index of the page table record named id, or -1. */
int64_t tt_archive_find(const tt_archive* archive, const char* id, int64_t id_len);
/* Base address of the read-only mapping (file offset 0); valid until tt_archive_close. */
const uint8_t* tt_archive_data(const tt_archive* archive);
/* Copy file bytes [offset, offset + nbytes) to device memory `dst` on `stream` through
 * two 32 MiB pinned staging buffers (allocated on first use for the current device).
 * Returns once the last chunk is queued; calls on one archive are serialized. */
int tt_archive_upload(tt_archive* archive, int64_t offset, int64_t nbytes, void* dst, void* stream);
int tt_archive_close(tt_archive* archive);

#ifdef __cplusplus
}
#endif

#endif /* THINTENSOR_HIP_H */
