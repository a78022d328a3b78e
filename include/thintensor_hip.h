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

/* y[n] = (sum_k w[n,k] x[k]) * s[n], w float8_e4m3fn [rows, cols], s fp32 or fp16 [rows].
 * Replaces TritonDecodeBackend.scaled_matvec for per-row scales
 * (triton_kernels.py:4452-4595; kernels :539-592, :2990-3019). */
int tt_scaled_matvec(const void* weight, int64_t w_row_bytes, const void* scales, int scale_dtype,
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
                             const int32_t* expert_indices, int64_t selected,
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
                                   const int32_t* expert_indices, int64_t selected,
                                   void* out, int out_dtype, int64_t out_slot,
                                   int64_t rows, int64_t cols, void* stream);

/* Fused gate/up GEMV on interleaved rows (2i gate, 2i+1 up) + gpt-oss SwiGLU:
 * g = bf16(bf16(dot) + bias), u likewise; g = min(g, L); u = clamp(u, -L, L);
 * out = (u + 1) * g / (1 + exp(-alpha g)).  bias [E, 2I] (nullable).
 * Replaces TritonDecodeBackend.mxfp_lowbit_selected_swiglu
 * (triton_kernels.py:4178-4235; kernel :1214-1343). */
int tt_mxfp_lowbit_selected_swiglu(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                   const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                   const void* x, int x_dtype, int64_t x_slot,
                                   const int32_t* expert_indices, int64_t selected,
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
                                 const int32_t* expert_indices, const void* router_scores,
                                 int score_dtype, int64_t selected,
                                 const void* bias, int bias_dtype, int64_t bias_expert,
                                 void* out, int out_dtype, int64_t rows, int64_t cols, void* stream);

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
                            const int32_t* expert_indices, int64_t selected,
                            void* out, int out_dtype, int64_t out_slot,
                            int64_t rows, int64_t cols, int64_t group_size, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* THINTENSOR_HIP_H */
