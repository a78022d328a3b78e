// Fused per-row-scaled gate/up GEMV + SiLU for gfx950 (float8_e4m3fn or int8 weights):
//
//   out[m] = silu(g) * u,  g = bf16((W_g[m] . x) * s_g[m]),  u = bf16((W_u[m] . x) * s_u[m])
//
// with silu(g) = g / (1 + e^-g) in binary32 and the two projections rounded through
// bfloat16 whatever the activation dtype (triton_kernels.py:3243-3350, wrapper
// :4346-4436).
//
// Gate row m and up row m are the two rows of one lane group of LPR lanes, LPR chosen by
// the single-matrix lanes-per-row rule, so each dot product has exactly the reduction
// order of scaled_matvec (tt_gemv.h: 32-element chunks, chunk j on lane j % LPR in round
// j / LPR, fma chains from +0, round sums, lane butterfly; the row scale multiplies the
// row sum).  After the reduction lane 0 of the group holds g and lane 1 holds u; one
// cross-lane move brings u to lane 0, which stores the product.  The activation vector
// is staged once per workgroup in LDS.
#include <type_traits>

#include "gemv_impl.h"

namespace tt {
namespace {

struct GateUpParams {
  const uint8_t* wg;   // gate weights [rows, cols], wg_row bytes between rows
  const uint8_t* wu;   // up weights
  const void* sg;      // per-row scales, sg_stride / su_stride elements apart
  const void* su;
  const void* x;       // [cols], 16-byte aligned
  void* out;           // [rows]
  int64_t wg_row, wu_row, sg_stride, su_stride;
  int rows, cols;
};

template <Fmt F, typename XT, typename OT, typename ST, int LPR>
__global__ __launch_bounds__(256) void gate_up_silu_kernel(const GateUpParams P) {
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr int SUBS = 64 / LPR;
  extern __shared__ uint32_t xs_lds[];
  const int lane = threadIdx.x & 63;
  const int sub = lane / LPR;
  const int l = lane % LPR;
  const int nchunks = P.cols >> 5;
  const int rounds = (nchunks + LPR - 1) / LPR;
  const int wave = threadIdx.x >> 6;
  const int m = (int)(blockIdx.x * 4 + wave) * SUBS + sub;
  const bool live = m < P.rows;
  const int mc = live ? m : P.rows - 1;
  const uint8_t* wrow[2] = {P.wg + (int64_t)mc * P.wg_row, P.wu + (int64_t)mc * P.wu_row};

  // round 0's weights are requested before the activation copy
  auto fetch = [&](int r, Raw<B>* w) {
    int j = r * LPR + l;
    j = j < nchunks ? j : nchunks - 1;
    w[0] = load_raw<B>(wrow[0] + (int64_t)j * B);
    w[1] = load_raw<B>(wrow[1] + (int64_t)j * B);
  };
  Raw<B> cur[2];
  fetch(0, cur);
  // the scale of the row this lane finishes (lane bit 0: gate or up)
  const float scale = (l & 1) ? to_f32(reinterpret_cast<const ST*>(P.su)[(int64_t)mc * P.su_stride])
                              : to_f32(reinterpret_cast<const ST*>(P.sg)[(int64_t)mc * P.sg_stride]);

  const int xn = P.cols >> 3;   // 16-byte pieces
  for (int i = threadIdx.x; i < xn; i += 256)
    reinterpret_cast<uint4*>(xs_lds)[i] = reinterpret_cast<const uint4*>(P.x)[i];
  lds_barrier();

  float acc[2] = {0.0f, 0.0f};
  for (int r = 0; r < rounds; r++) {
    Raw<B> nxt[2];
    const bool more = r + 1 < rounds;
    if (more) fetch(r + 1, nxt);
    const int j = r * LPR + l;
    const bool cv = j < nchunks;
    uint32_t xw[16];
    const uint4* xp = reinterpret_cast<const uint4*>(xs_lds + (cv ? j : 0) * 16);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint4 v = xp[q];
      xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
    }
    float p[2];
    chunk_dot_rows<F, XT, 2>(cur, xw, p);
    acc[0] = acc[0] + (cv ? p[0] : 0.0f);
    acc[1] = acc[1] + (cv ? p[1] : 0.0f);
    if (more) {
      cur[0] = nxt[0];
      cur[1] = nxt[1];
    }
  }
  // lane bit 0 splits the two rows (reduce-scatter), the other bits are butterflies
  reduce_range<2, 1, LPR>(acc);
  const float v = round_bf16(acc[0] * scale);
  const float up = xor_partner<1>(v);
  if (live && l == 0) store<OT>(reinterpret_cast<OT*>(P.out) + m, silu_mul_val(v, up));
}

}  // namespace
}  // namespace tt

using namespace tt;

extern "C" int tt_scaled_gate_up_silu(const void* gate_weight, int64_t wg_row_bytes, const void* gate_scales,
                                      int64_t sg_stride, const void* up_weight, int64_t wu_row_bytes,
                                      const void* up_scales, int64_t su_stride, int w_format, int scale_dtype,
                                      const void* x, int x_dtype, void* out, int out_dtype, int64_t rows,
                                      int64_t cols, void* stream) {
  const char* what = "fused_scaled_gate_up_silu";
  TT_REQUIRE(w_format == TT_W_FP8 || w_format == TT_W_INT8, "%s: weights must be float8_e4m3fn or int8 (format %d)",
             what, w_format);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: scales must be fp16 or fp32", what);
  TT_REQUIRE(gate_weight && up_weight && aligned(gate_weight, 16) && aligned(up_weight, 16) && wg_row_bytes % 16 == 0 &&
                 wu_row_bytes % 16 == 0 && wg_row_bytes >= cols && wu_row_bytes >= cols,
             "%s: weights must be 16-byte aligned rows", what);
  TT_REQUIRE(gate_scales && up_scales && sg_stride >= 1 && su_stride >= 1, "%s: bad scales", what);
  TT_REQUIRE(x && aligned(x, 16) && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  TT_REQUIRE(cols > 0 && cols % 32 == 0 && cols <= 32768, "%s: cols must be a positive multiple of 32 up to 32768",
             what);
  GateUpParams P{static_cast<const uint8_t*>(gate_weight), static_cast<const uint8_t*>(up_weight), gate_scales,
                 up_scales, x, out, wg_row_bytes, wu_row_bytes, sg_stride, su_stride, (int)rows, (int)cols};
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t lds = (size_t)cols * 2;
  auto launch = [&](auto fmt, auto xt, auto ot, auto sdt) -> int {
    constexpr Fmt F = decltype(fmt)::value;
    using XT = decltype(xt);
    using OT = decltype(ot);
    using ST = decltype(sdt);
    const int per_block = 4 * (64 / lpr);
    const dim3 grid((unsigned)((rows + per_block - 1) / per_block));
    switch (lpr) {
      case 64: hipLaunchKernelGGL((gate_up_silu_kernel<F, XT, OT, ST, 64>), grid, dim3(256), lds, st, P); break;
      case 32: hipLaunchKernelGGL((gate_up_silu_kernel<F, XT, OT, ST, 32>), grid, dim3(256), lds, st, P); break;
      case 16: hipLaunchKernelGGL((gate_up_silu_kernel<F, XT, OT, ST, 16>), grid, dim3(256), lds, st, P); break;
      default: set_error("%s: invalid lanes per row %d", what, lpr); return TT_ERR_INVALID;
    }
    return check_launch(what);
  };
  auto go = [&](auto xt, auto ot, auto sdt) -> int {
    if (w_format == TT_W_INT8) return launch(std::integral_constant<Fmt, Fmt::kInt8>{}, xt, ot, sdt);
    return launch(std::integral_constant<Fmt, Fmt::kFp8>{}, xt, ot, sdt);
  };
  auto by_scale = [&](auto xt, auto ot) { return scale_dtype == TT_F16 ? go(xt, ot, f16_t{}) : go(xt, ot, float{}); };
  if (x_dtype == TT_F16) {
    if (out_dtype == TT_F16) return by_scale(f16_t{}, f16_t{});
    if (out_dtype == TT_F32) return by_scale(f16_t{}, float{});
  } else {
    if (out_dtype == TT_BF16) return by_scale(bf16_t{}, bf16_t{});
    if (out_dtype == TT_F32) return by_scale(bf16_t{}, float{});
  }
  set_error("%s: output must match the activation dtype or be fp32", what);
  return TT_ERR_UNSUPPORTED;
}
