// MoE router for gfx950: router GEMV + bias + top-k + softmax in one launch
// (triton_kernels.py:2855-2921), and top-k + softmax on given logits
// (triton_kernels.py:2821-2851).
//
//   logit_e = bf16(dot_e) (+ bias_e, rounded to bf16 again) -- the reference rounds
//             through bfloat16 whatever the activation dtype;
//   dot_e   = GEMV row in the library order with 64 lanes per row;
//   top-k   = iterated argmax, lowest index on ties;
//   score_i = exp(v_i - max_all) / D, D summed in slot order over the selected
//             experts (renormalize) or in expert order over all experts.
// Indices are written as int32 and stay on the device.
#include "tt_abi_internal.h"
#include "tt_common.h"
#include "tt_gemv.h"

#include <type_traits>

namespace tt {

template <typename T> __device__ __forceinline__ float ldv(const void* p, int64_t i) {
  return to_f32(reinterpret_cast<const T*>(p)[i]);
}

// Ordered key of a router logit: larger value wins, equal values (+0 == -0) go to
// the lowest expert index.  NaN never wins through the key (see wave_topk).
__device__ __forceinline__ uint64_t topk_key(float v, uint32_t e) {
  uint32_t b = __builtin_bit_cast(uint32_t, v);
  if ((b & 0x7fffffffu) == 0) b = 0;
  const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - e);
}

__device__ __forceinline__ float lane_value(float a, float b, int i) {
  return i < 64 ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), i))
                : __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, b), i - 64));
}

// Top-k + softmax over E <= 128 logits held by one wave (expert e in lane e % 64,
// register e / 64).  Same result as scanning the experts in order for each slot:
// the first untaken expert starts the scan and a later one replaces it only when
// strictly greater -- so a NaN at the first untaken position is selected, any other
// NaN never is, and equal values keep the lowest index.  The denominator is summed
// sequentially in slot order (renormalize) or expert order, each term
// exp(v - max) with max the NaN-ignoring maximum over all experts.
template <typename OT>
__device__ void wave_topk(float lg0, float lg1, int E, int top_k, bool renorm, int32_t* idx_out, OT* score_out) {
  const int lane = lane_id();
  const bool v0 = lane < E, v1 = lane + 64 < E;
  float m = __builtin_bit_cast(float, 0xff800000u);
  if (v0) m = fmaxf(m, lg0);
  if (v1) m = fmaxf(m, lg1);
  m = fmaxf(m, xor_partner<1>(m));
  m = fmaxf(m, xor_partner<2>(m));
  m = fmaxf(m, xor_partner<4>(m));
  m = fmaxf(m, xor_partner<8>(m));
  m = fmaxf(m, xor_partner<16>(m));
  m = fmaxf(m, xor_partner<32>(m));
  bool t0 = !v0, t1 = !v1;
  float sel0 = 0.0f, sel1 = 0.0f;
  for (int s = 0; s < top_k; s++) {
    uint64_t k = 0, f = 0;
    if (!t0) {
      f = 0xffffffffu - (uint32_t)lane;
      if (!__builtin_isnan(lg0)) k = topk_key(lg0, lane);
    }
    if (!t1) {
      if (f == 0) f = 0xffffffffu - (uint32_t)(lane + 64);
      if (!__builtin_isnan(lg1)) {
        const uint64_t k1 = topk_key(lg1, lane + 64);
        k = k1 > k ? k1 : k;
      }
    }
    k = wave_max_u64(k);
    f = wave_max_u64(f);
    const int first = __builtin_amdgcn_readfirstlane((int)(0xffffffffu - (uint32_t)f));
    const float fv = lane_value(lg0, lg1, first);
    int bi = first;
    if (!__builtin_isnan(fv)) bi = __builtin_amdgcn_readfirstlane((int)(0xffffffffu - (uint32_t)k));
    const float bv = lane_value(lg0, lg1, bi);
    if (lane == bi) t0 = true;
    if (lane + 64 == bi) t1 = true;
    if (lane == (s & 63)) {
      if (s < 64) sel0 = bv;
      else sel1 = bv;
    }
    if (lane == 0) idx_out[s] = bi;
  }
  const float e0 = exp_f32(sel0 - m), e1 = exp_f32(sel1 - m);
  float den = 0.0f;
  if (renorm) {
    for (int s = 0; s < top_k; s++) den = den + lane_value(e0, e1, s);
  } else {
    const float a0 = exp_f32(lg0 - m), a1 = exp_f32(lg1 - m);
    for (int e = 0; e < E; e++) den = den + lane_value(a0, a1, e);
  }
  if (lane < top_k) store<OT>(score_out + lane, e0 / den);
  if (lane + 64 < top_k) store<OT>(score_out + lane + 64, e1 / den);
}

// Rows of E <= 32 experts with H <= 4096 (two rounds of 64 lanes): every wave requests
// the weights of both of its experts and the activation chunks of both rounds before
// the first wait (chunk indices clamped, contributions masked), then reduces as the
// general loop below does.
template <typename WT, typename XT, typename BT>
__device__ __forceinline__ void router_rows_held(const void* w, int64_t w_row, const void* x, int H, const void* bias,
                                                 int E, int wave, int lane, float (&lg)[2]) {
  constexpr Fmt F = std::is_same_v<WT, bf16_t> ? Fmt::kBF16W : Fmt::kF16W;
  const int nchunks = H >> 5;
  Raw<64> wr[2][2], xr[2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    int j = r * 64 + lane;
    j = j < nchunks ? j : nchunks - 1;
    xr[r] = load_raw<64>(reinterpret_cast<const uint8_t*>(x) + (int64_t)32 * j * 2);
#pragma unroll
    for (int k = 0; k < 2; k++) {
      int e = wave + 16 * k;
      e = e < E ? e : E - 1;
      wr[k][r] = load_raw<64>(reinterpret_cast<const uint8_t*>(w) + ((int64_t)e * w_row + 32 * j) * 2);
    }
  }
  BT braw[2];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int e = wave + 16 * k;
    if (bias != nullptr) braw[k] = reinterpret_cast<const BT*>(bias)[e < E ? e : E - 1];
  }
  __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the first use
#pragma unroll
  for (int k = 0; k < 2; k++) {
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const bool cv = r * 64 + lane < nchunks;
      const float p = chunk_dot<F, XT>(wr[k][r], xr[r].w);
      if (r == 0 || (nchunks > 64)) acc = acc + (cv ? p : 0.0f);
    }
    // logit = bf16(dot) (+ bias, rounded to bf16 again)
    float v = round_bf16(xor_sum(acc, 1, 64));
    if (bias != nullptr) v = round_bf16(v + to_f32(braw[k]));
    lg[k] = v;
  }
}

template <typename WT, typename XT, typename BT, typename OT>
__global__ __launch_bounds__(1024) void router_kernel(const void* w, int64_t w_row, const void* x, int H, const void* bias,
                                                      int E, int top_k, int renorm, int32_t* idx_out, void* score_out) {
  __shared__ float logits[128];
  constexpr Fmt F = std::is_same_v<WT, bf16_t> ? Fmt::kBF16W : Fmt::kF16W;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int nchunks = H >> 5;
  const int rounds = (nchunks + 63) / 64;
  if (E <= 32 && nchunks <= 128 && nwaves == 16) {
    float lg[2];
    router_rows_held<WT, XT, BT>(w, w_row, x, H, bias, E, wave, lane, lg);
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int e = wave + 16 * k;
      if (e < E && lane == 0) logits[e] = lg[k];
    }
    __syncthreads();
    if (wave == 0) {
      const float l0 = lane < E ? logits[lane] : 0.0f;
      wave_topk<OT>(l0, 0.0f, E, top_k, renorm != 0, idx_out, reinterpret_cast<OT*>(score_out));
    }
    return;
  }
  for (int e = wave; e < E; e += nwaves) {
    float acc = 0.0f;
    for (int r = 0; r < rounds; r++) {
      const int j = r * 64 + lane;
      float p = 0.0f;
      if (j < nchunks) {
        const Raw<64> wr = load_raw<64>(reinterpret_cast<const uint8_t*>(w) + ((int64_t)e * w_row + 32 * j) * 2);
        const Raw<64> xr = load_raw<64>(reinterpret_cast<const uint8_t*>(x) + (int64_t)32 * j * 2);
        p = chunk_dot<F, XT>(wr, xr.w);
      }
      acc = acc + p;
    }
    acc = xor_sum(acc, 1, 64);
    float lg = round_bf16(acc);
    if (bias != nullptr) lg = round_bf16(lg + ldv<BT>(bias, e));
    if (lane == 0) logits[e] = lg;
  }
  __syncthreads();
  if (wave == 0) {
    const float l0 = lane < E ? logits[lane] : 0.0f;
    const float l1 = lane + 64 < E ? logits[lane + 64] : 0.0f;
    wave_topk<OT>(l0, l1, E, top_k, renorm != 0, idx_out, reinterpret_cast<OT*>(score_out));
  }
}

template <typename LT, typename OT>
__global__ __launch_bounds__(64) void topk_kernel(const void* logits_in, int E, int top_k, int renorm, int32_t* idx_out,
                                                  void* score_out) {
  const int lane = lane_id();
  const float l0 = lane < E ? ldv<LT>(logits_in, lane) : 0.0f;
  const float l1 = lane + 64 < E ? ldv<LT>(logits_in, lane + 64) : 0.0f;
  wave_topk<OT>(l0, l1, E, top_k, renorm != 0, idx_out, reinterpret_cast<OT*>(score_out));
}

template <typename Fn> static int dt3(int code, Fn&& f) {
  if (code == TT_F16) return f(f16_t{});
  if (code == TT_BF16) return f(bf16_t{});
  if (code == TT_F32) return f(float{});
  set_error("unsupported dtype code %d", code);
  return TT_ERR_INVALID;
}

}  // namespace tt

using namespace tt;

extern "C" int tt_moe_router_matvec_topk(const void* weight, int w_dtype, int64_t w_row, const void* hidden,
                                         int x_dtype, int64_t hidden_size, const void* bias, int bias_dtype,
                                         int64_t experts, int64_t top_k, int renormalize, int32_t* indices_out,
                                         void* scores_out, int score_dtype, void* stream) {
  const char* what = "moe_router_matvec_topk";
  TT_REQUIRE(experts > 0 && experts <= 128, "%s: fused router supports at most 128 experts", what);
  TT_REQUIRE(top_k > 0 && top_k <= experts, "%s: top_k must be in [1, experts]", what);
  TT_REQUIRE(hidden_size > 0 && hidden_size % 32 == 0, "%s: hidden size must be a multiple of 32", what);
  TT_REQUIRE(weight && hidden && indices_out && scores_out, "%s: null pointer", what);
  TT_REQUIRE(aligned(weight, 16) && aligned(hidden, 16) && w_row % 8 == 0, "%s: weight rows and hidden must be 16-byte aligned", what);
  const int bdt = bias ? bias_dtype : TT_F32;
  return dt3(w_dtype, [&](auto wt) {
    using WT = decltype(wt);
    return dt3(x_dtype, [&](auto xt) {
      using XT = decltype(xt);
      return dt3(bdt, [&](auto bt) {
        using BT = decltype(bt);
        return dt3(score_dtype, [&](auto ot) {
          using OT = decltype(ot);
          if constexpr (std::is_same_v<WT, float> || std::is_same_v<XT, float>) {
            set_error("%s: router weight and hidden must be fp16 or bf16", what);
            return TT_ERR_UNSUPPORTED;
          } else {
            hipLaunchKernelGGL((router_kernel<WT, XT, BT, OT>), dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                               weight, w_row, hidden, (int)hidden_size, bias, (int)experts, (int)top_k, renormalize,
                               indices_out, scores_out);
            return check_launch(what);
          }
        });
      });
    });
  });
}

extern "C" int tt_moe_router_topk(const void* logits, int logits_dtype, int64_t experts, int64_t top_k, int renormalize,
                                  int32_t* indices_out, void* scores_out, int score_dtype, void* stream) {
  const char* what = "moe_router_topk";
  TT_REQUIRE(experts > 0 && experts <= 128 && top_k > 0 && top_k <= experts, "%s: bad expert counts", what);
  TT_REQUIRE(logits && indices_out && scores_out, "%s: null pointer", what);
  return dt3(logits_dtype, [&](auto lt) {
    using LT = decltype(lt);
    return dt3(score_dtype, [&](auto ot) {
      using OT = decltype(ot);
      hipLaunchKernelGGL((topk_kernel<LT, OT>), dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), logits,
                         (int)experts, (int)top_k, renormalize, indices_out, scores_out);
      return check_launch(what);
    });
  });
}
