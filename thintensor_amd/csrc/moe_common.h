// Shared parameter blocks and helpers of the fused MoE expert kernels: gate/up GEMV + gpt-oss SwiGLU on interleaved rows and
// down GEMV + router-weighted sum, for E8M0 block-scaled formats (q1, q2, MXFP4).
// Expert ids and router scores are read on the device (no host synchronisation).
//
// RT is the precision the reference rounds the GEMV results and bias sums through:
// bfloat16 for the reference's fused low-bit kernels (triton_kernels.py:1319-1333,
// 1421-1434), the activation dtype for the MXFP4 chain that the reference runs as
// separate kernels plus torch adds (gpu_runtime.py:9647-9704, 9855-9903).
#pragma once

#include "gemv_impl.h"
#include "tt_topk.h"

#include <type_traits>

namespace tt {

struct SwigluParams {
  const uint8_t* w; int64_t w_expert, w_row;
  const uint8_t* s; int64_t s_expert, s_row;
  const void* x; int64_t x_slot;
  const void* experts; int ishift;   // expert ids, int32 (ishift 0) or int64 (1)
  const void* bias; int64_t bias_expert;
  float alpha, limit;
  void* out; int64_t out_slot;
  int act_rows, cols;
  int x_div;   // slots sharing one activation vector: slot s reads x + (s / x_div) * x_slot
  // router logits [tokens, n_exp] (float) instead of expert ids: slot s is token s / top_k's
  // (s % top_k)-th choice, and row block 0 writes each slot's expert and score to idx_out /
  // score_out (score_dtype) for the weighted-down after it
  const float* logits;
  int n_exp, top_k, renorm, score_dtype;
  int32_t* idx_out;
  void* score_out;
};

template <typename BT> __device__ __forceinline__ float ld_bias(const void* b, int64_t i) {
  return to_f32(reinterpret_cast<const BT*>(b)[i]);
}


struct DownParams {
  const uint8_t* w; int64_t w_expert, w_row;
  const uint8_t* s; int64_t s_expert, s_row;
  const void* x; int64_t x_slot;
  const void* experts; int ishift;   // expert ids, int32 (ishift 0) or int64 (1)
  const void* scores;
  const void* bias; int64_t bias_expert;
  void* out;
  int rows, cols, slots;          // slots per token
  int bias_dtype, score_dtype;   // storage codes (TT_F16 / TT_BF16 / TT_F32)
  int64_t out_token;             // elements between tokens' outputs (token = blockIdx.y)
  int tokens;                    // tokens, each with `slots` selected experts
};

// One element of a small vector (bias, router scores) whose storage type is a runtime
// code: these are read once per row and slot, so a branch is cheaper than one more
// template dimension.
__device__ __forceinline__ float ld_typed(const void* p, int dtype, int64_t i) {
  if (dtype == TT_F32) return reinterpret_cast<const float*>(p)[i];
  const uint16_t b = reinterpret_cast<const uint16_t*>(p)[i];
  return dtype == TT_BF16 ? to_f32(bf16_t{b}) : to_f32(f16_t{b});
}


// ld_typed in two 16-bit halves requested without a branch on the dtype (both loads stay
// inside the array for every dtype: a 16-bit array reads element i twice) and converted
// where the value is used, so a kernel can request it long before it needs it.
struct TypedBits { uint16_t lo, hi; };
__device__ __forceinline__ TypedBits ld_typed_bits(const void* p, int dtype, int64_t i) {
  const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
  const bool wide = dtype == TT_F32;
  const int64_t k = wide ? 2 * i : i;
  return TypedBits{h[k], h[wide ? k + 1 : k]};
}
__device__ __forceinline__ float typed_f32(TypedBits b, int dtype) {
  if (dtype == TT_F32) return __builtin_bit_cast(float, (uint32_t)b.lo | ((uint32_t)b.hi << 16));
  return dtype == TT_BF16 ? to_f32(bf16_t{b.lo}) : to_f32(f16_t{b.lo});
}

// Expert of SwiGLU slot `slot`: from the index list, or -- with router logits -- the
// (slot % top_k)-th choice of this wave's own top-k over its token's logits
// (wave_topk_expert: the router's selection, bit for bit).  The token's logits stay in
// lg0 / lg1 (expert e in lane e % 64 of lg(e / 64)) for swiglu_publish.
struct SlotRoute {
  int64_t e;
  float lg0, lg1;
};
__device__ __forceinline__ SlotRoute swiglu_slot_route(const SwigluParams& P, int slot) {
  if (P.logits == nullptr) return SlotRoute{load_expert(P.experts, P.ishift, slot), 0.0f, 0.0f};
  const int lane = lane_id();
  const int tk = slot / P.top_k, k = slot - tk * P.top_k;
  const float* lg = P.logits + (int64_t)tk * P.n_exp;
  const float lg0 = lg[lane < P.n_exp ? lane : 0];
  const float lg1 = lg[lane + 64 < P.n_exp ? lane + 64 : 0];
  return SlotRoute{wave_topk_expert(lg0, lg1, P.n_exp, k), lg0, lg1};
}

// With router logits: the slot's expert id and router score (wave_topk_lanes, the
// router's selection and softmax bit for bit) to idx_out / score_out.  One wave per slot
// calls it, after its weight loads are issued, so the softmax is off every wave's path to
// its first weight request.
__device__ __forceinline__ void swiglu_publish(const SwigluParams& P, int slot, float lg0, float lg1) {
  if (P.logits == nullptr) return;
  const int lane = lane_id();
  const int k = slot % P.top_k;
  const TopkLanes r = wave_topk_lanes(lg0, lg1, P.n_exp, P.top_k, P.renorm != 0);
  if (lane == (k & 63)) {
    P.idx_out[slot] = k < 64 ? r.idx0 : r.idx1;
    const float sc = k < 64 ? r.score0 : r.score1;
    if (P.score_dtype == TT_F32) reinterpret_cast<float*>(P.score_out)[slot] = sc;
    else if (P.score_dtype == TT_BF16) store<bf16_t>(reinterpret_cast<bf16_t*>(P.score_out) + slot, sc);
    else store<f16_t>(reinterpret_cast<f16_t*>(P.score_out) + slot, sc);
  }
}

template <typename T> struct DT;
template <> struct DT<f16_t> { static constexpr int code = TT_F16; };
template <> struct DT<bf16_t> { static constexpr int code = TT_BF16; };
template <> struct DT<float> { static constexpr int code = TT_F32; };

// Calls f.template operator()<T>() for the storage type matching `code`.
template <typename Fn> static int with_type(int code, Fn&& f) {
  switch (code) {
    case TT_F16: return f(f16_t{});
    case TT_BF16: return f(bf16_t{});
    case TT_F32: return f(float{});
  }
  set_error("unsupported dtype code %d", code);
  return TT_ERR_INVALID;
}

static Fmt fmt_for_bits(int bits) { return bits == 2 ? Fmt::kQ2E8 : (bits == 1 ? Fmt::kQ1E8 : Fmt::kMxfp4); }

}  // namespace tt
