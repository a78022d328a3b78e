// Decode-step elementwise and normalisation operators for gfx950:
// rms_norm, add_rms_norm, add, silu_mul, interleaved_swiglu, weighted_expert_sum,
// rope_qk_inplace, embedding row copy and KV-cache append.  Token ids and token
// positions can be read from device memory so a whole decode step can be replayed
// from a HIP graph.
#include "tt_abi_internal.h"
#include "tt_common.h"

#include <type_traits>

namespace tt {

// ---------------------------------------------------------------- RMSNorm
// out_i = (x_i * (1 / sqrt(mean(x^2) + eps))) * (w_i + offset) (triton_kernels.py:
// 2562-2577), add_rms_norm with the residual rounded through bfloat16 (:2581-2614).  The
// sum of squares follows the piece partition of tt_common.h (8-element pieces, piece p to
// thread p % 256).  With whole aligned pieces (vec) a thread holds its pieces in
// registers, every load issued before the first use; otherwise it reads element by
// element in the same partition.

template <typename XT, typename WT, typename OT>
__global__ __launch_bounds__(256) void rms_norm_kernel(const void* x, const void* w, void* out, int n, float eps,
                                                       float offset, int vec) {
  __shared__ float red[4];
  const int np = (n + 7) >> 3;
  const int t = threadIdx.x;
  if (vec && np <= 256 * kNormPieces) {
    uint4 xr[kNormPieces];
#pragma unroll
    for (int k = 0; k < kNormPieces; k++) {
      const int p = t + 256 * k;
      xr[k] = reinterpret_cast<const uint4*>(x)[p < np ? p : np - 1];
    }
    __builtin_amdgcn_sched_barrier(0);
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormPieces; k++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float v = piece_f32<XT>(xr[k], e);
        if (8 * (t + 256 * k) + e < n) s = __builtin_fmaf(v, v, s);
      }
    const float total = block_sum256(s, red);
    const float inv = 1.0f / __builtin_sqrtf(total / (float)n + eps);
#pragma unroll
    for (int k = 0; k < kNormPieces; k++) {
      const int p = t + 256 * k;
      if (p < np) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int i = 8 * p + e;
          if (i < n) store<OT>(reinterpret_cast<OT*>(out) + i, (piece_f32<XT>(xr[k], e) * inv) * (ld<WT>(w, i) + offset));
        }
      }
    }
    return;
  }
  float s = 0.0f;
  for (int p = t; p < np; p += 256)
    for (int i = 8 * p; i < 8 * p + 8 && i < n; i++) {
      const float v = ld<XT>(x, i);
      s = __builtin_fmaf(v, v, s);
    }
  const float total = block_sum256(s, red);
  const float inv = 1.0f / __builtin_sqrtf(total / (float)n + eps);
  for (int p = t; p < np; p += 256)
    for (int i = 8 * p; i < 8 * p + 8 && i < n; i++)
      store<OT>(reinterpret_cast<OT*>(out) + i, (ld<XT>(x, i) * inv) * (ld<WT>(w, i) + offset));
}

// residual = bf16(left + right) (stored in the activation dtype); the RMS is taken over
// the rounded residual.
template <typename XT, typename WT, typename OT>
__global__ __launch_bounds__(256) void add_rms_norm_kernel(const void* left, const void* right, void* residual_out,
                                                           const void* w, void* out, int n, float eps, int vec) {
  __shared__ float red[4];
  const int np = (n + 7) >> 3;
  const int t = threadIdx.x;
  if (vec && np <= 256 * kNormPieces) {
    uint4 lr[kNormPieces], rr[kNormPieces];
#pragma unroll
    for (int k = 0; k < kNormPieces; k++) {
      const int p = t + 256 * k;
      const int pc = p < np ? p : np - 1;
      lr[k] = reinterpret_cast<const uint4*>(left)[pc];
      rr[k] = reinterpret_cast<const uint4*>(right)[pc];
    }
    __builtin_amdgcn_sched_barrier(0);
    float res[kNormPieces][8];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormPieces; k++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        res[k][e] = round_bf16(piece_f32<XT>(lr[k], e) + piece_f32<XT>(rr[k], e));
        if (8 * (t + 256 * k) + e < n) s = __builtin_fmaf(res[k][e], res[k][e], s);
      }
    const float total = block_sum256(s, red);
    const float inv = 1.0f / __builtin_sqrtf(total / (float)n + eps);
#pragma unroll
    for (int k = 0; k < kNormPieces; k++) {
      const int p = t + 256 * k;
      if (p < np) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int i = 8 * p + e;
          if (i < n) {
            store<XT>(reinterpret_cast<XT*>(residual_out) + i, res[k][e]);
            store<OT>(reinterpret_cast<OT*>(out) + i, (res[k][e] * inv) * ld<WT>(w, i));
          }
        }
      }
    }
    return;
  }
  float s = 0.0f;
  for (int p = t; p < np; p += 256)
    for (int i = 8 * p; i < 8 * p + 8 && i < n; i++) {
      const float r = round_bf16(ld<XT>(left, i) + ld<XT>(right, i));
      s = __builtin_fmaf(r, r, s);
    }
  const float total = block_sum256(s, red);
  const float inv = 1.0f / __builtin_sqrtf(total / (float)n + eps);
  for (int p = t; p < np; p += 256)
    for (int i = 8 * p; i < 8 * p + 8 && i < n; i++) {
      const float r = round_bf16(ld<XT>(left, i) + ld<XT>(right, i));
      store<XT>(reinterpret_cast<XT*>(residual_out) + i, r);
      store<OT>(reinterpret_cast<OT*>(out) + i, (r * inv) * ld<WT>(w, i));
    }
}

// Rows of a decode batch, one workgroup per row: sum_r = a_r + b_r rounded to the
// activation dtype (add_kernel's rounding), out_r = rms_norm(sum_r) * w (rms_norm_kernel's
// piece partition and reduction, weight offset 0).  Whole aligned pieces only.
template <typename XT, typename WT, typename OT>
__global__ __launch_bounds__(256) void add_then_rms_norm_rows_kernel(const void* a, const void* b, void* sum,
                                                                     const void* w, void* out, int n, int64_t row,
                                                                     int64_t out_row, float eps) {
  __shared__ float red[4];
  const int np = n >> 3;
  const int t = threadIdx.x;
  const int64_t off = (int64_t)blockIdx.x * row;
  const uint4* ap = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a) + off);
  const uint4* bp = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(b) + off);
  uint4 ar[kNormPieces], br[kNormPieces];
#pragma unroll
  for (int k = 0; k < kNormPieces; k++) {
    const int p = t + 256 * k;
    const int pc = p < np ? p : np - 1;
    ar[k] = ap[pc];
    br[k] = bp[pc];
  }
  __builtin_amdgcn_sched_barrier(0);
  float r[kNormPieces][8];
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < kNormPieces; k++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      r[k][e] = round_to<XT>(piece_f32<XT>(ar[k], e) + piece_f32<XT>(br[k], e));
      if (t + 256 * k < np) s = __builtin_fmaf(r[k][e], r[k][e], s);
    }
  const float total = block_sum256(s, red);
  const float inv = 1.0f / __builtin_sqrtf(total / (float)n + eps);
  XT* so = reinterpret_cast<XT*>(sum) + off;
  OT* oo = reinterpret_cast<OT*>(out) + (int64_t)blockIdx.x * out_row;
#pragma unroll
  for (int k = 0; k < kNormPieces; k++) {
    const int p = t + 256 * k;
    if (p < np) {
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int i = 8 * p + e;
        store<XT>(so + i, r[k][e]);
        store<OT>(oo + i, (r[k][e] * inv) * ld<WT>(w, i));
      }
    }
  }
}

// ---------------------------------------------------------------- elementwise
template <typename T>
__global__ void add_kernel(const void* a, const void* b, void* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) store<T>(reinterpret_cast<T*>(out) + i, ld<T>(a, i) + ld<T>(b, i));
}

// silu(g) * u = (g / (1 + exp(-g))) * u (triton_kernels.py:2761-2774)
template <typename T>
__global__ void silu_mul_kernel(const void* g, const void* u, void* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    store<T>(reinterpret_cast<T*>(out) + i, silu_mul_val(ld<T>(g, i), ld<T>(u, i)));
  }
}

// gpt-oss SwiGLU on interleaved [.., 2n] gate/up (triton_kernels.py:2778-2793)
template <typename T>
__global__ void interleaved_swiglu_kernel(const void* gu, void* out, int n, int64_t in_row, int64_t out_row,
                                          float alpha, float limit) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int r = blockIdx.y;
  if (i < n) {
    float g = ld<T>(gu, r * in_row + 2 * (int64_t)i);
    float u = ld<T>(gu, r * in_row + 2 * (int64_t)i + 1);
    g = fminf(g, limit);
    u = fmaxf(fminf(u, limit), -limit);
    const float num = (u + 1.0f) * g;
    const float den = 1.0f + exp_f32(-g * alpha);
    store<T>(reinterpret_cast<T*>(out) + r * out_row + i, num / den);
  }
}

// out[n] = sum_e fma(experts[e, n], scores[e], .) in expert order (triton_kernels.py:2797-2817)
template <typename T, typename ST>
__global__ void weighted_expert_sum_kernel(const void* ex, const void* scores, void* out, int width, int count,
                                           int64_t stride) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < width) {
    float acc = 0.0f;
    for (int e = 0; e < count; e++) acc = __builtin_fmaf(ld<T>(ex, e * stride + i), ld<ST>(scores, e), acc);
    store<T>(reinterpret_cast<T*>(out) + i, acc);
  }
}

// ---------------------------------------------------------------- RoPE
// q1' = r(r(q1 c) - r(q2 s)), q2' = r(r(q2 c) + r(q1 s)) with r() rounding to the
// activation dtype, as the reference's torch RoPE path (gpu_runtime.py:8696-8705).
// cos/sin rows come from a table indexed by the token position, which may be read
// from device memory (pos_dev) so graph replays advance with the position.
template <typename T>
__global__ void rope_kernel(void* q, void* k, const void* cos_t, const void* sin_t, int64_t table_row, int64_t table_rows,
                            const int32_t* pos_dev, int pos, int heads, int kv_heads, int head_dim) {
  const int half = head_dim >> 1;
  const int64_t p = pos_dev ? (int64_t)pos_dev[0] : (int64_t)pos;
  if (p < 0 || p >= table_rows) return;
  const int total = (heads + kv_heads) * half;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int h = idx / half, i = idx - h * half;
  T* base = h < heads ? reinterpret_cast<T*>(q) + (int64_t)h * head_dim : reinterpret_cast<T*>(k) + (int64_t)(h - heads) * head_dim;
  const float c = ld<T>(cos_t, p * table_row + i);
  const float s = ld<T>(sin_t, p * table_row + i);
  float o1, o2;
  rope_pair<T>(to_f32(base[i]), to_f32(base[i + half]), c, s, o1, o2);
  store<T>(base + i, o1);
  store<T>(base + i + half, o2);
}

// ---------------------------------------------------------------- per-head RMSNorm
// One wave per head (head_dim <= 512): lane l holds elements l, l + 64, ...; the sum of
// squares is an fma chain per lane in that order, then the 64-lane xor butterfly;
// out = (x * (1 / sqrt(sum / head_dim + eps))) * w (triton_kernels.py:2618-2634).
constexpr int kHeadHeld = 8;

template <typename T, typename WT>
__global__ __launch_bounds__(256) void head_rms_norm_kernel(const void* x, const void* w, void* out, int heads, int D,
                                                            float eps) {
  const int head = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (head >= heads) return;   // whole waves
  const T* xh = reinterpret_cast<const T*>(x) + (int64_t)head * D;
  float v[kHeadHeld];
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < kHeadHeld; k++) {
    const int i = lane + 64 * k;
    v[k] = i < D ? to_f32(xh[i]) : 0.0f;
    if (i < D) s = __builtin_fmaf(v[k], v[k], s);
  }
  s = xor_sum(s, 1, 64);
  const float inv = 1.0f / __builtin_sqrtf(s / (float)D + eps);
  T* oh = reinterpret_cast<T*>(out) + (int64_t)head * D;
#pragma unroll
  for (int k = 0; k < kHeadHeld; k++) {
    const int i = lane + 64 * k;
    if (i < D) store<T>(oh + i, (v[k] * inv) * ld<WT>(w, i));
  }
}

// Per-head RMSNorm then RoPE, in place on q heads then k heads (triton_kernels.py:
// 2691-2757): one wave per head, lane l holds the pairs (i, i + half) for i = l, l + 64,
// ...; sum of squares per lane: fma(a, a, .) then fma(b, b, .) per pair, then the 64-lane
// butterfly; a' = a * (inv * w[i]), b' = b * (inv * w[i + half]); the rotation is binary32
// (a' c - b' s, b' c + a' s, cos/sin read from the activation-dtype table), rounded once
// by the store.
constexpr int kPairHeld = 4;

template <typename T, typename WT>
__global__ __launch_bounds__(256) void qk_head_norm_rope_kernel(void* q, void* k, const void* qw, const void* kw,
                                                                const void* cos_t, const void* sin_t,
                                                                int64_t table_row, int64_t table_rows,
                                                                const int32_t* pos_dev, int pos, int heads,
                                                                int kv_heads, int D, float eps) {
  const int hh = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (hh >= heads + kv_heads) return;   // whole waves
  const int64_t p = pos_dev ? (int64_t)pos_dev[0] : (int64_t)pos;
  if (p < 0 || p >= table_rows) return;
  const bool is_q = hh < heads;
  T* base = is_q ? reinterpret_cast<T*>(q) + (int64_t)hh * D : reinterpret_cast<T*>(k) + (int64_t)(hh - heads) * D;
  const void* w = is_q ? qw : kw;
  const int half = D >> 1;
  float a[kPairHeld], b[kPairHeld];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kPairHeld; j++) {
    const int i = lane + 64 * j;
    const bool ok = i < half;
    a[j] = ok ? to_f32(base[i]) : 0.0f;
    b[j] = ok ? to_f32(base[i + half]) : 0.0f;
    if (ok) {
      s = __builtin_fmaf(a[j], a[j], s);
      s = __builtin_fmaf(b[j], b[j], s);
    }
  }
  s = xor_sum(s, 1, 64);
  const float inv = 1.0f / __builtin_sqrtf(s / (float)D + eps);
#pragma unroll
  for (int j = 0; j < kPairHeld; j++) {
    const int i = lane + 64 * j;
    if (i < half) {
      const float an = a[j] * (inv * ld<WT>(w, i));
      const float bn = b[j] * (inv * ld<WT>(w, i + half));
      const float c = ld<T>(cos_t, p * table_row + i), sn = ld<T>(sin_t, p * table_row + i);
      store<T>(base + i, an * c - bn * sn);
      store<T>(base + i + half, bn * c + an * sn);
    }
  }
}

// ---------------------------------------------------------------- embedding / KV
// out = embed[token] (row copy), token read from device memory when token_dev is set.
__global__ void embed_kernel(const uint16_t* embed, int64_t row, int64_t vocab, const int64_t* token_dev, int64_t token,
                             uint16_t* out, int n) {
  const int64_t t = token_dev ? token_dev[0] : token;
  if (t < 0 || t >= vocab) return;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = embed[t * row + i];
}

// keys[h, pos, :] = k[h, :], values[h, pos, :] = v[h, :]
__global__ void kv_append_kernel(const uint16_t* k, const uint16_t* v, uint16_t* keys, uint16_t* values,
                                 int64_t stride_h, int64_t stride_t, const int32_t* pos_dev, int pos, int64_t capacity,
                                 int kv_heads, int head_dim) {
  const int64_t p = pos_dev ? (int64_t)pos_dev[0] : (int64_t)pos;
  if (p < 0 || p >= capacity) return;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= kv_heads * head_dim) return;
  const int h = idx / head_dim, d = idx - h * head_dim;
  keys[h * stride_h + p * stride_t + d] = k[idx];
  values[h * stride_h + p * stride_t + d] = v[idx];
}

__global__ void advance_position_kernel(int32_t* pos, int32_t step) {
  if (threadIdx.x == 0) pos[0] += step;
}

// history[pos - base] = token (all read on the device)
__global__ void record_token_kernel(const int64_t* token, const int32_t* pos, const int32_t* base, int64_t* history,
                                    int32_t capacity) {
  if (threadIdx.x == 0) {
    const int32_t i = pos[0] - base[0];
    if (i >= 0 && i < capacity) history[i] = token[0];
  }
}

// history[r * history_row + pos - base] = tokens[r] for the rows of a batch, then
// pos += step once every row has read it.
__global__ void record_tokens_advance_kernel(const int64_t* tokens, int32_t count, int32_t* pos, const int32_t* base,
                                             int64_t* history, int64_t history_row, int32_t capacity, int32_t step) {
  const int32_t i = pos[0] - base[0];
  for (int r = threadIdx.x; r < count; r += blockDim.x)
    if (i >= 0 && i < capacity) history[(int64_t)r * history_row + i] = tokens[r];
  __syncthreads();
  if (threadIdx.x == 0) pos[0] = pos[0] + step;
}

template <typename Fn> static int with_act(int code, Fn&& f) {
  if (code == TT_F16) return f(f16_t{});
  if (code == TT_BF16) return f(bf16_t{});
  set_error("activation dtype must be fp16 or bf16 (got %d)", code);
  return TT_ERR_INVALID;
}
template <typename Fn> static int with_any(int code, Fn&& f) {
  if (code == TT_F16) return f(f16_t{});
  if (code == TT_BF16) return f(bf16_t{});
  if (code == TT_F32) return f(float{});
  set_error("unsupported dtype code %d", code);
  return TT_ERR_INVALID;
}

}  // namespace tt

using namespace tt;

extern "C" int tt_rms_norm(const void* x, int x_dtype, const void* weight, int w_dtype, void* out, int out_dtype,
                           int64_t n, float eps, float weight_offset, void* stream) {
  TT_REQUIRE(x && weight && out && n > 0 && n <= (1 << 24), "rms_norm: bad arguments");
  return with_act(x_dtype, [&](auto xt) {
    using XT = decltype(xt);
    return with_any(w_dtype, [&](auto wt) {
      using WT = decltype(wt);
      return with_any(out_dtype, [&](auto ot) {
        using OT = decltype(ot);
        const int vec = n % 8 == 0 && aligned(x, 16);
        hipLaunchKernelGGL((rms_norm_kernel<XT, WT, OT>), dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), x,
                           weight, out, (int)n, eps, weight_offset, vec);
        return check_launch("rms_norm");
      });
    });
  });
}

extern "C" int tt_add_rms_norm(const void* left, const void* right, void* residual_out, int x_dtype,
                               const void* weight, int w_dtype, void* out, int out_dtype, int64_t n, float eps,
                               void* stream) {
  TT_REQUIRE(left && right && residual_out && weight && out && n > 0 && n <= (1 << 24), "add_rms_norm: bad arguments");
  return with_act(x_dtype, [&](auto xt) {
    using XT = decltype(xt);
    return with_any(w_dtype, [&](auto wt) {
      using WT = decltype(wt);
      return with_any(out_dtype, [&](auto ot) {
        using OT = decltype(ot);
        const int vec = n % 8 == 0 && aligned(left, 16) && aligned(right, 16);
        hipLaunchKernelGGL((add_rms_norm_kernel<XT, WT, OT>), dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream),
                           left, right, residual_out, weight, out, (int)n, eps, vec);
        return check_launch("add_rms_norm");
      });
    });
  });
}

extern "C" int tt_add_then_rms_norm_rows(const void* left, const void* right, void* sum_out, int x_dtype, int64_t row,
                                         const void* weight, int w_dtype, void* out, int out_dtype, int64_t out_row,
                                         int64_t rows, int64_t n, float eps, void* stream) {
  const char* what = "add_then_rms_norm_rows";
  TT_REQUIRE(left && right && sum_out && weight && out && rows >= 1 && rows <= 65535, "%s: bad arguments", what);
  TT_REQUIRE(n > 0 && n % 8 == 0 && n <= 8 * 256 * kNormPieces, "%s: n must be a multiple of 8 up to %d", what,
             8 * 256 * kNormPieces);
  TT_REQUIRE(aligned(left, 16) && aligned(right, 16) && aligned(sum_out, 16) && row % 8 == 0 && row >= n &&
                 out_row >= n,
             "%s: 16-byte aligned rows required", what);
  return with_act(x_dtype, [&](auto xt) {
    using XT = decltype(xt);
    return with_any(w_dtype, [&](auto wt) {
      using WT = decltype(wt);
      return with_any(out_dtype, [&](auto ot) {
        using OT = decltype(ot);
        hipLaunchKernelGGL((add_then_rms_norm_rows_kernel<XT, WT, OT>), dim3((unsigned)rows), dim3(256), 0,
                           static_cast<hipStream_t>(stream), left, right, sum_out, weight, out, (int)n, row, out_row,
                           eps);
        return check_launch(what);
      });
    });
  });
}

extern "C" int tt_add(const void* a, const void* b, void* out, int dtype, int64_t n, void* stream) {
  TT_REQUIRE(a && b && out && n > 0 && n < (1LL << 31), "add: bad arguments");
  return with_any(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL((add_kernel<T>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       a, b, out, (int)n);
    return check_launch("add");
  });
}

extern "C" int tt_silu_mul(const void* gate, const void* up, void* out, int dtype, int64_t n, void* stream) {
  TT_REQUIRE(gate && up && out && n > 0 && n < (1LL << 31), "silu_mul: bad arguments");
  return with_any(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL((silu_mul_kernel<T>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), gate, up, out, (int)n);
    return check_launch("silu_mul");
  });
}

extern "C" int tt_interleaved_swiglu(const void* gate_up, int64_t in_row, void* out, int64_t out_row, int dtype,
                                     int64_t rows, int64_t n, float alpha, float limit, void* stream) {
  TT_REQUIRE(gate_up && out && n > 0 && rows > 0 && rows <= 65535, "interleaved_swiglu: bad arguments");
  return with_any(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL((interleaved_swiglu_kernel<T>), dim3((unsigned)((n + 255) / 256), (unsigned)rows), dim3(256), 0,
                       static_cast<hipStream_t>(stream), gate_up, out, (int)n, in_row, out_row, alpha, limit);
    return check_launch("interleaved_swiglu");
  });
}

extern "C" int tt_weighted_expert_sum(const void* experts, int dtype, int64_t stride, int64_t count,
                                      const void* scores, int score_dtype, void* out, int64_t width, void* stream) {
  TT_REQUIRE(experts && scores && out && width > 0 && count > 0, "weighted_expert_sum: bad arguments");
  return with_any(dtype, [&](auto t) {
    using T = decltype(t);
    return with_any(score_dtype, [&](auto st) {
      using ST = decltype(st);
      hipLaunchKernelGGL((weighted_expert_sum_kernel<T, ST>), dim3((unsigned)((width + 255) / 256)), dim3(256), 0,
                         static_cast<hipStream_t>(stream), experts, scores, out, (int)width, (int)count, stride);
      return check_launch("weighted_expert_sum");
    });
  });
}

extern "C" int tt_rope_qk_inplace(void* q, void* k, int dtype, const void* cos_table, const void* sin_table,
                                  int64_t table_row, int64_t table_rows, const int32_t* position_dev, int64_t position,
                                  int64_t heads, int64_t kv_heads, int64_t head_dim, void* stream) {
  TT_REQUIRE(q && k && cos_table && sin_table && head_dim > 0 && head_dim % 2 == 0, "rope: RoPE head_dim must be even");
  TT_REQUIRE(heads > 0 && kv_heads >= 0, "rope: bad head counts");
  TT_REQUIRE(table_rows > 0 && (position_dev != nullptr || (position >= 0 && position < table_rows)),
             "rope: position outside the cos/sin table");
  const int total = (int)((heads + kv_heads) * (head_dim / 2));
  return with_act(dtype, [&](auto t) {
    using T = decltype(t);
    hipLaunchKernelGGL((rope_kernel<T>), dim3((total + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream), q, k,
                       cos_table, sin_table, table_row, table_rows, position_dev, (int)position, (int)heads, (int)kv_heads,
                       (int)head_dim);
    return check_launch("rope_qk_inplace");
  });
}

extern "C" int tt_head_rms_norm(const void* x, int dtype, const void* weight, int w_dtype, void* out, int64_t heads,
                                int64_t head_dim, float eps, void* stream) {
  TT_REQUIRE(x && weight && out && heads > 0, "head_rms_norm: bad arguments");
  TT_UNSUPPORTED(head_dim > 0 && head_dim <= 64 * kHeadHeld, "head_rms_norm: head_dim up to %d", 64 * kHeadHeld);
  return with_act(dtype, [&](auto t) {
    using T = decltype(t);
    return with_any(w_dtype, [&](auto wt) {
      using WT = decltype(wt);
      hipLaunchKernelGGL((head_rms_norm_kernel<T, WT>), dim3((unsigned)((heads + 3) / 4)), dim3(256), 0,
                         static_cast<hipStream_t>(stream), x, weight, out, (int)heads, (int)head_dim, eps);
      return check_launch("head_rms_norm");
    });
  });
}

extern "C" int tt_qk_head_rmsnorm_rope_inplace(void* q, void* k, int dtype, const void* q_weight, const void* k_weight,
                                               int w_dtype, const void* cos_table, const void* sin_table,
                                               int64_t table_row, int64_t table_rows, const int32_t* position_dev,
                                               int64_t position, int64_t heads, int64_t kv_heads, int64_t head_dim,
                                               float eps, void* stream) {
  const char* what = "qk_head_rmsnorm_rope_inplace";
  TT_REQUIRE(q && k && q_weight && k_weight && cos_table && sin_table, "%s: null pointer", what);
  TT_REQUIRE(head_dim > 0 && head_dim % 2 == 0, "%s: RoPE head_dim must be even, got %lld", what, (long long)head_dim);
  TT_UNSUPPORTED(head_dim <= 128 * kPairHeld, "%s: head_dim up to %d", what, 128 * kPairHeld);
  TT_REQUIRE(heads > 0 && kv_heads >= 0, "%s: bad head counts", what);
  TT_REQUIRE(table_rows > 0 && (position_dev != nullptr || (position >= 0 && position < table_rows)),
             "%s: position outside the cos/sin table", what);
  return with_act(dtype, [&](auto t) {
    using T = decltype(t);
    return with_any(w_dtype, [&](auto wt) {
      using WT = decltype(wt);
      hipLaunchKernelGGL((qk_head_norm_rope_kernel<T, WT>), dim3((unsigned)((heads + kv_heads + 3) / 4)), dim3(256), 0,
                         static_cast<hipStream_t>(stream), q, k, q_weight, k_weight, cos_table, sin_table, table_row,
                         table_rows, position_dev, (int)position, (int)heads, (int)kv_heads, (int)head_dim, eps);
      return check_launch(what);
    });
  });
}

extern "C" int tt_embedding(const void* embed, int64_t row_stride, int64_t vocab, const int64_t* token_dev,
                            int64_t token, void* out, int64_t n, void* stream) {
  TT_REQUIRE(embed && out && n > 0 && vocab > 0, "embedding: bad arguments");
  TT_REQUIRE(token_dev != nullptr || (token >= 0 && token < vocab), "embedding: token id out of range");
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((n + 255) / 256 < 64 ? (n + 255) / 256 : 64)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(embed), row_stride, vocab, token_dev, token,
                     static_cast<uint16_t*>(out), (int)n);
  return check_launch("embedding");
}

extern "C" int tt_kv_append(const void* k, const void* v, void* keys, void* values, int64_t stride_head,
                            int64_t stride_token, const int32_t* position_dev, int64_t position, int64_t capacity,
                            int64_t kv_heads, int64_t head_dim, void* stream) {
  TT_REQUIRE(k && v && keys && values && kv_heads > 0 && head_dim > 0 && capacity > 0, "kv_append: bad arguments");
  TT_REQUIRE(position_dev != nullptr || (position >= 0 && position < capacity), "kv_append: position beyond the cache");
  const int total = (int)(kv_heads * head_dim);
  hipLaunchKernelGGL(kv_append_kernel, dim3((total + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), static_cast<uint16_t*>(keys),
                     static_cast<uint16_t*>(values), stride_head, stride_token, position_dev, (int)position, capacity,
                     (int)kv_heads, (int)head_dim);
  return check_launch("kv_append");
}

extern "C" int tt_advance_position(int32_t* position_dev, int32_t step, void* stream) {
  TT_REQUIRE(position_dev != nullptr, "advance_position: null pointer");
  hipLaunchKernelGGL(advance_position_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), position_dev, step);
  return check_launch("advance_position");
}

extern "C" int tt_record_token(const int64_t* token_dev, const int32_t* position_dev, const int32_t* base_dev,
                               int64_t* history, int32_t capacity, void* stream) {
  TT_REQUIRE(token_dev && position_dev && base_dev && history && capacity > 0, "record_token: bad arguments");
  hipLaunchKernelGGL(record_token_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), token_dev, position_dev,
                     base_dev, history, capacity);
  return check_launch("record_token");
}

extern "C" int tt_record_tokens_advance(const int64_t* tokens_dev, int32_t count, int32_t* position_dev,
                                        const int32_t* base_dev, int64_t* history, int64_t history_row,
                                        int32_t capacity, int32_t step, void* stream) {
  TT_REQUIRE(tokens_dev && position_dev && base_dev && history && count >= 1 && capacity > 0 && history_row >= capacity,
             "record_tokens_advance: bad arguments");
  hipLaunchKernelGGL(record_tokens_advance_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), tokens_dev,
                     count, position_dev, base_dev, history, history_row, capacity, step);
  return check_launch("record_tokens_advance");
}
