// E8M0 block-scaled (MXFP4, q1, q2) and affine low-bit GEMV entry points.
#include "gemv_lean.h"

using namespace tt;

namespace {

int selected_e8(const char* what, Fmt fmt, const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                const void* scales, int64_t s_expert, int64_t s_row, const void* x, int x_dtype, int64_t x_slot,
                const void* experts, int index_bytes, int64_t selected, void* out, int out_dtype, int64_t out_slot, int64_t rows,
                int64_t cols, void* stream) {
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(selected >= 1 && selected <= 65535 && experts != nullptr, "%s: need 1..65535 selected experts", what);
  int ishift;
  TT_REQUIRE(index_shift(index_bytes, &ishift), "%s: expert indices must be int32 or int64", what);
  const int align = fmt == Fmt::kMxfp4 ? 16 : (fmt == Fmt::kQ2E8 ? 8 : 4);
  TT_REQUIRE(packed && aligned(packed, align) && w_row_bytes % align == 0 && w_expert_bytes % align == 0,
             "%s: packed weights must be %d-byte aligned", what, align);
  TT_REQUIRE(scales && x && aligned(x, 16) && (x_slot % 8) == 0 && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L;
  bool row_mode;
  int rc = tt::plan_groups(what, cols, cols, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, 1, out, (int)rows};
  P.x = x;
  P.x_slot = x_slot;
  P.experts = experts;
  P.ishift = ishift;
  P.w_expert = w_expert_bytes;
  P.s_expert = s_expert;
  P.out_slot = out_slot;
  P.cols = (int)cols;
  const int Lg = 1;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int slots = (int)selected;
  if (x_dtype == out_dtype && lean_fits(rows, w_row_bytes, s_row, cols)) {
    LeanParams L{};
    L.w = static_cast<const uint8_t*>(packed);
    L.s = scales;
    L.x = x;
    L.out = out;
    L.experts = experts;
    L.ishift = ishift;
    L.w_expert = w_expert_bytes;
    L.s_expert = s_expert;
    L.x_slot = x_slot;
    L.out_slot = out_slot;
    L.w_row = (uint32_t)w_row_bytes;
    L.s_row = (uint32_t)s_row;
    L.rows = (int)rows;
    L.cols = (int)cols;
    switch (fmt) {
      case Fmt::kMxfp4: return lean_launch<Fmt::kMxfp4, SMode::kBlockE8, uint8_t, 1>(x_dtype, lpr, L, slots, st, what);
      case Fmt::kQ2E8: return lean_launch<Fmt::kQ2E8, SMode::kBlockE8, uint8_t, 1>(x_dtype, lpr, L, slots, st, what);
      case Fmt::kQ1E8: return lean_launch<Fmt::kQ1E8, SMode::kBlockE8, uint8_t, 1>(x_dtype, lpr, L, slots, st, what);
      default: break;
    }
  }
  switch (fmt) {
    case Fmt::kMxfp4: return launch_types<Fmt::kMxfp4, SMode::kBlockE8, uint8_t, 4>(x_dtype, out_dtype, Lg, lpr, P, slots, st, what);
    case Fmt::kQ2E8: return launch_types<Fmt::kQ2E8, SMode::kBlockE8, uint8_t, 4>(x_dtype, out_dtype, Lg, lpr, P, slots, st, what);
    case Fmt::kQ1E8: return launch_types<Fmt::kQ1E8, SMode::kBlockE8, uint8_t, 4>(x_dtype, out_dtype, Lg, lpr, P, slots, st, what);
    default: break;
  }
  set_error("%s: bad format", what);
  return TT_ERR_INVALID;
}

// Grouped affine Q2 / Q1 with 64-element groups, whole groups per lane load.
//
// Same arithmetic as the documented GEMV order (tt_gemv.h) with LPR lanes per row and
// L = 2 chunks per group: the two chunks of group g sit in lanes 2(g mod P), +1 of the
// contract (P = LPR / 2 "pair lanes") in round g div P, so S_g = p_2g + p_2g+1,
// X_g = x_2g + x_2g+1, t_g = fmaf(X_g, -(z_g s_g), S_g s_g) and pair lane p keeps
// A_p = ((+0 + t_round0) + t_round1) + ...; the row is the lane-index tree over the A_p.
// Here one lane holds VP adjacent pair lanes (one group is 16 bytes of Q2, 8 of Q1)
// with one accumulator each; the first tree level over them is taken in
// the lane and the rest over the row's Q = P / VP lanes, so the bits are those of the
// contract.  Chunk x sums (sequential from +0) are computed once per workgroup; x sits
// in LDS with 16-byte piece k of group g at slot 9g + k: one pad piece per group puts
// the row's lanes, which read consecutive groups, on distinct banks, and a lane's pieces
// are immediate offsets from one address.
struct Aff16Params {
  const uint8_t* w;
  const uint16_t* s;      // fp16 (scale, zero) pairs
  const void* x;
  void* out;
  uint32_t w_row, s_row, s_grp;
  int rows, cols;
};

// RPL rows per lane (rows lane / Q and lane / Q + 64 / (Q * RPL) ... of the wave's block
// share each activation read and give the lane RPL * 2 independent fma chains per group).
// ALL: the row's rounds all fit the PF-round ring (the host checks), so they are consumed
// in one straight pass with no refill loop (a loop with conditional refills kept more
// registers live, too many for the whole 17920-row grid to be resident at once).
constexpr int kAffXPieces = 4;   // 16-byte activation pieces per thread requested up front
template <int BITS, typename XT, typename OT, int P, int VP, int RPL, int PF, bool ALL>
__global__ __launch_bounds__(256) void affine16_kernel(const Aff16Params A) {
  constexpr int Q = P / VP;                 // lanes per row
  constexpr int RG = 64 / Q;                // row groups per wave
  constexpr int RPW = RG * RPL;             // rows per wave
  constexpr int GB = 8 * BITS;              // bytes per 64-element group
  constexpr int LB = GB * VP;               // bytes per lane per round (16 or 8)
  constexpr Fmt F = BITS == 2 ? Fmt::kQ2Aff : Fmt::kQ1Aff;
  constexpr int CB = FmtInfo<F>::kBytes;    // bytes per 32-element chunk
  extern __shared__ uint4 x_lds[];          // cols / 8 pieces, then cols / 32 floats
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int q = lane % Q;
  const int row0 = (int)(blockIdx.x * 4 + wave) * RPW + lane / Q;
  int row[RPL], rc[RPL];
  bool live[RPL];
#pragma unroll
  for (int i = 0; i < RPL; i++) {
    row[i] = row0 + i * RG;
    live[i] = row[i] < A.rows;
    rc[i] = live[i] ? row[i] : A.rows - 1;
  }
  const int G = A.cols >> 6;
  const int rounds = (G + P - 1) / P;

  struct Rnd {
    uint32_t w[RPL][LB / 4];
    uint16_t s[RPL][VP], z[RPL][VP];
  };
  auto fetch = [&](int r, Rnd& d) {
    int g0 = r * P + q * VP;
    g0 = g0 < G ? g0 : G - VP;              // past the last group: re-read it (unused)
#pragma unroll
    for (int i = 0; i < RPL; i++) {
      const uint8_t* wp = A.w + (size_t)rc[i] * A.w_row + (uint32_t)g0 * GB;
      if constexpr (LB == 16) {
        const uint4 v = *reinterpret_cast<const uint4*>(wp);
        d.w[i][0] = v.x; d.w[i][1] = v.y; d.w[i][2] = v.z; d.w[i][3] = v.w;
      } else {
        const uint2 v = *reinterpret_cast<const uint2*>(wp);
        d.w[i][0] = v.x; d.w[i][1] = v.y;
      }
      const uint16_t* sp = A.s + (size_t)rc[i] * A.s_row;
#pragma unroll
      for (int v = 0; v < VP; v++) {
        const uint32_t o = (uint32_t)(g0 + v) * A.s_grp;
        d.s[i][v] = sp[o];
        d.z[i][v] = sp[o + 1];
      }
    }
  };
  // the activation pieces first (clamped; native 4-vectors: an array of the uint4
  // struct type is kept in scratch memory), then the weight rounds
  typedef uint32_t piece_t __attribute__((ext_vector_type(4)));
  const int xn = A.cols >> 3;
  const piece_t* xg = reinterpret_cast<const piece_t*>(A.x);
  piece_t xr[kAffXPieces];
#pragma unroll
  for (int k = 0; k < kAffXPieces; k++) {
    const int i = (int)threadIdx.x + 256 * k;
    xr[k] = xg[i < xn ? i : xn - 1];
  }
  Rnd ring[PF];
#pragma unroll
  for (int k = 0; k < PF; k++) fetch(k, ring[k]);
  __builtin_amdgcn_sched_barrier(0);

  // x into LDS (padded pieces), then the chunk sums
  piece_t* xl = reinterpret_cast<piece_t*>(x_lds);
#pragma unroll
  for (int k = 0; k < kAffXPieces; k++) {
    const int i = (int)threadIdx.x + 256 * k;
    if (i < xn) xl[9 * (i >> 3) + (i & 7)] = xr[k];
  }
  for (int i = (int)threadIdx.x + 256 * kAffXPieces; i < xn; i += 256) xl[9 * (i >> 3) + (i & 7)] = xg[i];
  __syncthreads();
  float* xsum = reinterpret_cast<float*>(x_lds + xn + (A.cols >> 6));
  for (int c = threadIdx.x; c < (A.cols >> 5); c += 256) {
    const int g = c >> 1;
    float t = 0.0f;
#pragma unroll
    for (int k4 = 0; k4 < 4; k4++) {
      const int k = 4 * (c & 1) + k4;
      const uint4 v = x_lds[9 * g + k];
      const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; e++) t = t + ((e & 1) ? hi_f32<XT>(wd[e >> 1]) : lo_f32<XT>(wd[e >> 1]));
    }
    xsum[c] = t;
  }
  __syncthreads();

  float acc[RPL][VP];
#pragma unroll
  for (int i = 0; i < RPL; i++)
#pragma unroll
    for (int v = 0; v < VP; v++) acc[i][v] = 0.0f;
  auto consume = [&](const Rnd& c, int r) {
#pragma unroll
    for (int v = 0; v < VP; v++) {
      const int g = r * P + q * VP + v;
      const bool gv = g < G;
      const int gc = gv ? g : G - 1;
      float pch[RPL][2];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        // chunk 2g + h: its 32 activations (pieces 4h .. 4h+3 of the group), then the
        // weight bytes of each row
        uint32_t xw[16];
#pragma unroll
        for (int k4 = 0; k4 < 4; k4++) {
          const int k = 4 * h + k4;
          const uint4 xv4 = x_lds[9 * gc + k];
          xw[4 * k4] = xv4.x; xw[4 * k4 + 1] = xv4.y; xw[4 * k4 + 2] = xv4.z; xw[4 * k4 + 3] = xv4.w;
        }
        Raw<CB> raw[RPL];
#pragma unroll
        for (int i = 0; i < RPL; i++)
#pragma unroll
          for (int u = 0; u < CB / 4; u++) raw[i].w[u] = c.w[i][(v * 2 + h) * (CB / 4) + u];
        float p[RPL];
        chunk_dot_rows<F, XT, RPL>(raw, xw, p);
#pragma unroll
        for (int i = 0; i < RPL; i++) pch[i][h] = p[i];
      }
      const float X = xsum[2 * gc] + xsum[2 * gc + 1];
#pragma unroll
      for (int i = 0; i < RPL; i++) {
        const float S = pch[i][0] + pch[i][1];
        const float sk = (float)__builtin_bit_cast(_Float16, c.s[i][v]);
        const float m = -((float)__builtin_bit_cast(_Float16, c.z[i][v]) * sk);
        const float t = __builtin_fmaf(X, m, S * sk);
        acc[i][v] = acc[i][v] + (gv ? t : 0.0f);
      }
    }
  };
  if constexpr (ALL) {
    // rounds past the last re-read the last group and add +0
#pragma unroll
    for (int k = 0; k < PF; k++) consume(ring[k], k);
  } else {
    for (int r0 = 0; r0 < rounds; r0 += PF) {
#pragma unroll
      for (int k = 0; k < PF; k++) {
        if (r0 + k < rounds) {
          consume(ring[k], r0 + k);
          if (r0 + k + PF < rounds) fetch(r0 + k + PF, ring[k]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RPL; i++) {
    float a = acc[i][0];
    if constexpr (VP == 2) a = acc[i][0] + acc[i][1];
    a = xor_sum(a, 1, Q);
    if (live[i] && q == 0) store<OT>(reinterpret_cast<OT*>(A.out) + row[i], a);
  }
}

// Measured at the cfg2 shapes: one group and one row per lane was the fastest of
// {VP 1, 2} x {rows per lane 1, 2} for both formats.
// Launches of several workgroups per CU request five rounds up front (17920 x 5120: q2
// 14.26 -> 14.01 us, q1 12.81 -> 12.42 us); one-round launches keep two (five there:
// q2 5120 x 5120 7.41 -> 7.70 us).
constexpr int kAffVP = 1, kAffRPL = 1, kAffPF = 2, kAffPFBig = 5;
constexpr int64_t kAffBigRows = 16384;

template <int BITS, typename XT, int P, int VP, int RPL>
int launch_affine16(const Aff16Params& A, hipStream_t st, const char* what) {
  constexpr int RPW = 64 / (P / VP) * RPL;
  const int64_t waves = ((int64_t)A.rows + RPW - 1) / RPW;
  const dim3 grid((unsigned)((waves + 3) / 4));
  const size_t lds = (size_t)A.cols * 2 + (size_t)(A.cols / 64) * 16 + (size_t)(A.cols / 32) * 4;
  const int rounds = (A.cols / 64 + P - 1) / P;
  if (A.rows >= kAffBigRows && rounds <= kAffPFBig)
    hipLaunchKernelGGL((affine16_kernel<BITS, XT, XT, P, VP, RPL, kAffPFBig, true>), grid, dim3(256), lds, st, A);
  else if (A.rows >= kAffBigRows)
    hipLaunchKernelGGL((affine16_kernel<BITS, XT, XT, P, VP, RPL, kAffPFBig, false>), grid, dim3(256), lds, st, A);
  else
    hipLaunchKernelGGL((affine16_kernel<BITS, XT, XT, P, VP, RPL, kAffPF, false>), grid, dim3(256), lds, st, A);
  return check_launch(what);
}

template <int BITS, typename XT>
int affine16_by_lpr(int lpr, const Aff16Params& A, hipStream_t st, const char* what) {
  constexpr int VP = kAffVP;
  constexpr int RPL = kAffRPL;
  switch (lpr) {
    case 64: return launch_affine16<BITS, XT, 32, VP, RPL>(A, st, what);
    case 32: return launch_affine16<BITS, XT, 16, VP, RPL>(A, st, what);
    default: return launch_affine16<BITS, XT, 8, VP, RPL>(A, st, what);
  }
}

}  // namespace

extern "C" int tt_mxfp4_selected_matvec(const void* blocks, int64_t b_expert_bytes, int64_t b_row_bytes,
                                        const void* scales, int64_t s_expert, int64_t s_row, const void* x,
                                        int x_dtype, int64_t x_slot, const void* expert_indices, int index_bytes, int64_t selected,
                                        void* out, int out_dtype, int64_t out_slot, int64_t rows, int64_t cols,
                                        void* stream) {
  return selected_e8("mxfp4_selected_matvec", Fmt::kMxfp4, blocks, b_expert_bytes, b_row_bytes, scales, s_expert,
                     s_row, x, x_dtype, x_slot, expert_indices, index_bytes, selected, out, out_dtype, out_slot, rows, cols, stream);
}

extern "C" int tt_mxfp_lowbit_selected_matvec(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                              const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                              const void* x, int x_dtype, int64_t x_slot,
                                              const void* expert_indices, int index_bytes, int64_t selected, void* out,
                                              int out_dtype, int64_t out_slot, int64_t rows, int64_t cols,
                                              void* stream) {
  if (bits != 1 && bits != 2) {
    set_error("mxfp_lowbit_selected_matvec: low-bit expert weights must be packed Q1 or Q2");
    return TT_ERR_INVALID;
  }
  return selected_e8("mxfp_lowbit_selected_matvec", bits == 2 ? Fmt::kQ2E8 : Fmt::kQ1E8, packed, w_expert_bytes,
                     w_row_bytes, scales, s_expert, s_row, x, x_dtype, x_slot, expert_indices, index_bytes, selected, out,
                     out_dtype, out_slot, rows, cols, stream);
}

extern "C" int tt_lowbit_affine_matvec(const void* packed, int64_t w_row_bytes, const void* scale_zero, int64_t s_row,
                                       int64_t s_group, int bits, const void* x, int x_dtype, void* out,
                                       int out_dtype, int64_t rows, int64_t cols, int64_t group_size, void* stream) {
  const char* what = "lowbit_affine_matvec";
  TT_REQUIRE(bits == 1 || bits == 2, "%s: bits must be 1 or 2", what);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  const int align = bits == 2 ? 8 : 4;
  TT_REQUIRE(packed && aligned(packed, align) && w_row_bytes % align == 0 && w_row_bytes * 8 >= cols * bits,
             "%s: packed rows must be %d-byte aligned", what, align);
  TT_REQUIRE(scale_zero && x && aligned(x, 16) && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L;
  bool row_mode;
  int rc = tt::plan_groups(what, cols, group_size, &L, &row_mode);
  if (rc) return rc;
  TT_UNSUPPORTED(!row_mode, "%s: group_size must be smaller than cols", what);
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scale_zero, s_row, s_group, out, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  const int Lg = L;
  P.s_pair = 1;
  P.aff_zero = 1;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, L);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // 64-element groups, 16-byte rows, every lane's share a whole number of 16-byte loads
  const int vp = kAffVP;
  if (x_dtype == out_dtype && Lg == 2 && aligned(packed, 16) && w_row_bytes % 16 == 0 &&
      (cols / 64) % vp == 0 && lpr / 2 >= vp && lean_fits(rows, w_row_bytes, 2 * s_row, cols) && s_group >= 2 &&
      s_group * (cols / group_size) < (1LL << 30)) {
    Aff16Params A{static_cast<const uint8_t*>(packed), static_cast<const uint16_t*>(scale_zero), x, out,
                  (uint32_t)w_row_bytes, (uint32_t)s_row, (uint32_t)s_group, (int)rows, (int)cols};
    if (bits == 2)
      return x_dtype == TT_F16 ? affine16_by_lpr<2, f16_t>(lpr, A, st, what) : affine16_by_lpr<2, bf16_t>(lpr, A, st, what);
    return x_dtype == TT_F16 ? affine16_by_lpr<1, f16_t>(lpr, A, st, what) : affine16_by_lpr<1, bf16_t>(lpr, A, st, what);
  }
  if (x_dtype == out_dtype && lean_group_ok(Lg) && lean_fits(rows, w_row_bytes, 2 * s_row, cols) && s_group >= 0 &&
      s_group * (cols / group_size) < (1LL << 30)) {
    LeanParams Q{};
    Q.w = static_cast<const uint8_t*>(packed);
    Q.s = scale_zero;
    Q.x = x;
    Q.out = out;
    Q.s_pair = 1;
    Q.aff_zero = 1;
    Q.w_row = (uint32_t)w_row_bytes;
    Q.s_row = (uint32_t)s_row;
    Q.s_grp = (uint32_t)s_group;
    Q.rows = (int)rows;
    Q.cols = (int)cols;
    if (bits == 2) return lean_launch_group<Fmt::kQ2Aff, SMode::kGroupAff, f16_t>(Lg, x_dtype, lpr, Q, 1, st, what);
    return lean_launch_group<Fmt::kQ1Aff, SMode::kGroupAff, f16_t>(Lg, x_dtype, lpr, Q, 1, st, what);
  }
  if (bits == 2) return launch_types<Fmt::kQ2Aff, SMode::kGroupAff, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  return launch_types<Fmt::kQ1Aff, SMode::kGroupAff, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
}
