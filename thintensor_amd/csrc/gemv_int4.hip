// int4 GEMV entry points (dense, multi-matrix, selected expert).
#include "gemv_lean.h"

using namespace tt;

namespace {

// Symmetric int4, fp16 group-128 scales: the single-matrix GEMV of the decode hot path.
// Same reduction order as gemv_kernel (chunk j on lane j mod LPR in round j div LPR,
// group butterflies over 4 lanes, scaled sums accumulated in round order, row
// butterfly over the remaining lane bits), without its segment / expert / epilogue
// machinery: one batch of ROWS * (64 / LPR) rows per wave and a short argument list.
// Row bases are wave-uniform scalars and every per-lane offset is 32-bit (the host
// keeps each operand under 4 GiB), so addressing costs almost no vector work.  The
// weight, scale and activation loads of round 0 are issued before the first wait;
// later rounds are fetched one ahead.  Activation staging XM: 0 = one copy per
// workgroup in LDS behind a barrier; 1 = each lane reads its chunk from global memory;
// 2 = each wave stages the whole vector in its own LDS slice with coalesced loads
// (no workgroup barrier; a wave's LDS accesses complete in order); 3 = the activation is
// the combine of single-token attention chunk partials (CombineSrc), built in LDS by the
// workgroup behind a barrier.
//
// Chunk partials of a head_dim-64 attention (the scratch layout of
// tt_single_token_gqa_attention): per query head h and chunk c, the chunk maximum m,
// the sum l of exp(s - m) and the 64 weighted sums o.
struct CombineSrc {
  const float* pm;
  const float* pl;
  const float* po;
  const int32_t* tokens_dev;   // device token count (null: `tokens` is the count)
  int tokens, max_tokens, max_chunks;
  uint16_t* xout;              // optional: workgroup 0 writes the combined activation here
};
constexpr int kCombineChunks = 12;   // chunks whose partials are requested with the first weights (48 loads: with
                                     // the weights under the 63 loads a wave can have outstanding)

template <typename XT, int LPR, int ROWS, int XM, int PFR>
__global__ __launch_bounds__(256) void int4g128_kernel(const uint8_t* __restrict__ W, uint32_t w_row,
                                                       const f16_t* __restrict__ S, uint32_t s_row, uint32_t s_grp,
                                                       const uint16_t* __restrict__ x, XT* __restrict__ y, int rows,
                                                       int cols, CombineSrc C) {
  constexpr int L = 4;                       // 32-element chunks per group of 128
  constexpr int SUBS = 64 / LPR;
  constexpr int NVG = ROWS / L > 0 ? ROWS / L : 1;
  constexpr int GLEV = log2c(L) < log2c(ROWS) ? log2c(L) : log2c(ROWS);
  constexpr int kXR = 4;                     // 16-byte activation pieces per thread via registers
  extern __shared__ uint32_t xs_lds[];
  const int lane = threadIdx.x & 63;
  const int sub = lane / LPR;
  const int l = lane % LPR;
  const int nchunks = cols >> 5;
  const int rounds = (nchunks + LPR - 1) / LPR;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int row0 = (int)(blockIdx.x * 4 + wave) * (ROWS * SUBS);   // wave-uniform

  // activation pieces for LDS (clamped indices: duplicates of the last piece, no branch)
  const int xn = cols >> 3;
  uint4 xreg[kXR];
  uint32_t xidx[kXR];
  constexpr bool XG = XM == 1;
  constexpr int kXW = 4;                     // pieces per lane when a wave stages its own copy
  uint4 xwreg[kXW];
  uint32_t xwidx[kXW];
  if constexpr (XM == 0) {
#pragma unroll
    for (int k = 0; k < kXR; k++) {
      const int idx = threadIdx.x + 256 * k;
      xidx[k] = idx < xn ? idx : xn - 1;
      xreg[k] = reinterpret_cast<const uint4*>(x)[xidx[k]];
    }
  } else if constexpr (XM == 2) {
#pragma unroll
    for (int k = 0; k < kXW; k++) {
      const int idx = lane + 64 * k;
      xwidx[k] = idx < xn ? idx : xn - 1;
      xwreg[k] = reinterpret_cast<const uint4*>(x)[xwidx[k]];
    }
  }
  // XM 3: thread p builds piece p of the activation (head p / 8, dimensions 8 (p mod 8)
  // .. +7; the host keeps cols <= 2048).  The partials of the first kCombineChunks chunks
  // of the scratch (values past the active count are unused) and the token count are
  // requested before the weights; the activation is rounded to XT.
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr int kCB = XM == 3 ? kCombineChunks : 1;
  float cm[kCB], cl[kCB];
  f32x4 co[kCB][2];
  int ctok = 0;
  const int cp = (int)threadIdx.x < xn ? (int)threadIdx.x : xn - 1;
  const float* cpm = nullptr;
  const float* cpl = nullptr;
  const f32x4* cpo = nullptr;
  if constexpr (XM == 3) {
    const int h = cp >> 3;
    cpm = C.pm + (int64_t)h * C.max_chunks;
    cpl = C.pl + (int64_t)h * C.max_chunks;
    cpo = reinterpret_cast<const f32x4*>(C.po + (int64_t)h * C.max_chunks * 64 + 8 * (cp & 7));
    // chunks past the scratch re-read its last chunk (values unused: the active count
    // never exceeds the scratch, which holds at least one chunk).  The loads are
    // unconditional: a load under a branch leaves a copy at the join that waits for it,
    // and that wait would hold back every later load by a memory round trip.
#pragma unroll
    for (int u = 0; u < kCB; u++) {
      const int uc = u < C.max_chunks ? u : C.max_chunks - 1;
      cm[u] = cpm[uc];
      cl[u] = cpl[uc];
      co[u][0] = cpo[uc * 16];
      co[u][1] = cpo[uc * 16 + 1];
    }
    ctok = C.tokens_dev ? C.tokens_dev[0] + C.tokens : C.tokens;
  }

  // weights: row i of lane group `sub` is row0 + i * SUBS + sub (clamped to the last row)
  const uint8_t* wrow[ROWS];
  bool rv[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    const int r0 = row0 + i * SUBS;                       // lane group 0's row (uniform)
    const int rc = r0 < rows - 1 ? r0 : rows - 1;
    wrow[i] = W + (size_t)rc * w_row;
    rv[i] = r0 + sub < rows;
  }
  // per-lane part: sub * w_row for the lane's group (0 when one row spans the wave),
  // clamped so the last rows never step past the matrix
  uint32_t wlane[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    const int r0 = row0 + i * SUBS;
    const int rc = r0 < rows - 1 ? r0 : rows - 1;
    const int rl = r0 + sub < rows ? r0 + sub : rows - 1;
    wlane[i] = SUBS == 1 ? 0u : (uint32_t)(rl - rc) * w_row;
  }
  // scales: value k of this lane belongs to batch row rs_row(l, GLEV, k) * SUBS + sub
  const f16_t* sbase = S + (size_t)(row0 < rows ? row0 : rows - 1) * s_row;
  uint32_t soff[NVG];
  bool sv[NVG];
#pragma unroll
  for (int k = 0; k < NVG; k++) {
    const int r = row0 + rs_row<ROWS>(l, GLEV, k) * SUBS + sub;
    sv[k] = r < rows;
    soff[k] = (uint32_t)((sv[k] ? r : rows - 1) - (row0 < rows ? row0 : rows - 1)) * s_row;
  }
  auto fetch = [&](int r, Raw<16>* w, f16_t* sc, uint4* xc) {
    uint32_t j = (uint32_t)(r * LPR + l);
    j = j < (uint32_t)nchunks ? j : (uint32_t)nchunks - 1;
#pragma unroll
    for (int i = 0; i < ROWS; i++) w[i] = load_raw<16>(wrow[i] + (wlane[i] + j * 16u));
    if constexpr (XG) {
#pragma unroll
      for (int q = 0; q < 4; q++) xc[q] = *reinterpret_cast<const uint4*>(x + (j * 32u + 8u * q));
    }
#pragma unroll
    for (int k = 0; k < NVG; k++) sc[k] = sbase[soff[k] + (j >> 2) * s_grp];
  };
  // PFR > 1: rounds are requested PFR at a time (rounds past the last re-read its chunk,
  // unused), for shapes with few waves and several rounds per row
  Raw<16> wc[PFR][ROWS];
  f16_t sc[PFR][NVG];
  uint4 xc[PFR][4];
#pragma unroll
  for (int k = 0; k < PFR; k++) fetch(k, wc[k], sc[k], xc[k]);

  uint32_t* xs = xs_lds;                     // this wave's activation copy
  if constexpr (XM == 0) {
    uint4* xl = reinterpret_cast<uint4*>(xs_lds);
#pragma unroll
    for (int k = 0; k < kXR; k++) xl[xidx[k]] = xreg[k];
    for (int idx = threadIdx.x + 256 * kXR; idx < xn; idx += 256) xl[idx] = reinterpret_cast<const uint4*>(x)[idx];
    lds_barrier();
  } else if constexpr (XM == 2) {
    xs = xs_lds + wave * (cols >> 1);
    uint4* xl = reinterpret_cast<uint4*>(xs);
#pragma unroll
    for (int k = 0; k < kXW; k++) xl[xwidx[k]] = xwreg[k];
    for (int idx = lane + 64 * kXW; idx < xn; idx += 64) xl[idx] = reinterpret_cast<const uint4*>(x)[idx];
  } else if constexpr (XM == 3) {
    // the combine of single_token_gqa_attention: M = the maximum of the active chunks'
    // maxima, then in chunk order e = exp(m_c - M), den = fma(l_c, e, den),
    // acc = fma(o_c, e, acc); the activation is acc / den rounded to fp16
    const int T_act = min(ctok, C.max_tokens);
    const int nc = T_act > 0 ? (T_act + 63) / 64 : 0;
    float M = __builtin_bit_cast(float, 0xff800000u);
#pragma unroll
    for (int u = 0; u < kCB; u++)
      if (u < nc) M = fmaxf(M, cm[u]);
    for (int c = kCB; c < nc; c++) M = fmaxf(M, cpm[c]);
    float den = 0.0f;
    float acc[8];
#pragma unroll
    for (int k = 0; k < 8; k++) acc[k] = 0.0f;
    auto fold = [&](float m, float lc, f32x4 o0, f32x4 o1) {
      const float ec = exp_f32(m - M);
      den = __builtin_fmaf(lc, ec, den);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        acc[k] = __builtin_fmaf(o0[k], ec, acc[k]);
        acc[4 + k] = __builtin_fmaf(o1[k], ec, acc[4 + k]);
      }
    };
#pragma unroll
    for (int u = 0; u < kCB; u++)
      if (u < nc) fold(cm[u], cl[u], co[u][0], co[u][1]);
    for (int c = kCB; c < nc; c++) fold(cpm[c], cpl[c], cpo[c * 16], cpo[c * 16 + 1]);
    uint32_t pk[4];
#pragma unroll
    for (int k = 0; k < 4; k++)
      pk[k] = bits16<XT>(acc[2 * k] / den) | (bits16<XT>(acc[2 * k + 1] / den) << 16);
    const uint4 piece{pk[0], pk[1], pk[2], pk[3]};
    if ((int)threadIdx.x < xn) {
      reinterpret_cast<uint4*>(xs_lds)[threadIdx.x] = piece;
      if (C.xout != nullptr && blockIdx.x == 0) reinterpret_cast<uint4*>(C.xout)[threadIdx.x] = piece;
    }
    lds_barrier();
  }

  float acc[NVG];
#pragma unroll
  for (int k = 0; k < NVG; k++) acc[k] = 0.0f;
  auto consume = [&](const Raw<16>* w, const f16_t* sk, const uint4* xk, int r) {
    const int j = r * LPR + l;
    const bool cv = j < nchunks;
    uint32_t xw[16];
    {
      const uint4* xp = reinterpret_cast<const uint4*>(xs + (cv ? j : 0) * 16);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint4 v = XG ? xk[q] : xp[q];
        xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
      }
    }
    float p[ROWS];
    chunk_dot_rows<Fmt::kInt4Sym, XT, ROWS>(w, xw, p);
#pragma unroll
    for (int i = 0; i < ROWS; i++) p[i] = (cv && rv[i]) ? p[i] : 0.0f;
    reduce_range<ROWS, 1, L>(p);
#pragma unroll
    for (int k = 0; k < NVG; k++) {
      const float t = p[k] * to_f32(sk[k]);
      acc[k] = acc[k] + ((cv && sv[k]) ? t : 0.0f);
    }
  };
  if constexpr (PFR == 1) {
    // do-while: the host guarantees one round (cols >= 32), and no loop-entry test keeps
    // every argument load in the one scalar batch at the top
    int r = 0;
    do {
      Raw<16> wn[ROWS];
      f16_t sn[NVG];
      uint4 xnx[4];
      const bool more = r + 1 < rounds;
      if (more) fetch(r + 1, wn, sn, xnx);
      consume(wc[0], sc[0], xc[0], r);
      if (more) {
#pragma unroll
        for (int i = 0; i < ROWS; i++) wc[0][i] = wn[i];
#pragma unroll
        for (int k = 0; k < NVG; k++) sc[0][k] = sn[k];
        if constexpr (XG) {
#pragma unroll
          for (int q = 0; q < 4; q++) xc[0][q] = xnx[q];
        }
      }
    } while (++r < rounds);
  } else {
    for (int r0 = 0;;) {
#pragma unroll
      for (int k = 0; k < PFR; k++)
        if (r0 + k < rounds) consume(wc[k], sc[k], xc[k], r0 + k);
      r0 += PFR;
      if (r0 >= rounds) break;
#pragma unroll
      for (int k = 0; k < PFR; k++) fetch(r0 + k, wc[k], sc[k], xc[k]);
    }
  }
  reduce_range<NVG, L, LPR>(acc);
  const int frow = row0 + rs_row<ROWS>(l, log2c(ROWS), 0) * SUBS + sub;
  if ((l >> log2c(ROWS)) == 0 && frow < rows) store<XT>(y + frow, acc[0]);
}

// Activation staging mode (see int4g128_kernel).
inline int int4g128_x_mode(int64_t rows, int64_t cols, int lpr) { return cols / 32 <= lpr ? 1 : 0; }

template <typename XT, int LPR>
int launch_int4g128_lpr(int rpw, const void* W, int64_t w_row, const void* S, int64_t s_row, int64_t s_grp,
                        const void* x, void* y, int rows, int cols, hipStream_t st, const CombineSrc* combine = nullptr) {
  const int per_wave = rpw * (64 / LPR);
  const int64_t waves = ((int64_t)rows + per_wave - 1) / per_wave;
  const dim3 grid((unsigned)((waves + 3) / 4));
  const auto* w = static_cast<const uint8_t*>(W);
  const auto* s = static_cast<const f16_t*>(S);
  const auto* xv = static_cast<const uint16_t*>(x);
  auto* yv = static_cast<XT*>(y);
  const int xm = combine ? 3 : int4g128_x_mode(rows, cols, LPR);
  const size_t lds = xm == 1 ? 0 : (size_t)cols * 2 * (xm == 2 ? 4 : 1);
  const CombineSrc cmb = combine ? *combine : CombineSrc{};
  const uint32_t wr = (uint32_t)w_row, sr = (uint32_t)s_row, sg = (uint32_t)s_grp;
  const int rounds = (cols / 32 + LPR - 1) / LPR;
  // several rounds per row and few rows per wave: rounds requested PFR at a time -- five
  // rows of five rounds in one pass (17920 x 5120 at two rows per wave: 14.6 -> 13.1 us),
  // two of the four rounds of a one-row wave (2048 x 8192: 5.39 -> 5.17 us), else four
#define TT_INT4G_LAUNCH(R, M)                                                                                  \
  do {                                                                                                        \
    if (rounds == 5 && R <= 2)                                                                                \
      hipLaunchKernelGGL((int4g128_kernel<XT, LPR, R, M, 5>), grid, dim3(256), lds, st, w, wr, s, sr, sg, xv, yv, \
                         rows, cols, cmb);                                                                    \
    else if (rounds == 4 && R == 1)                                                                           \
      hipLaunchKernelGGL((int4g128_kernel<XT, LPR, R, M, 2>), grid, dim3(256), lds, st, w, wr, s, sr, sg, xv, yv, \
                         rows, cols, cmb);                                                                    \
    else if (rounds > 1 && R <= 2)                                                                            \
      hipLaunchKernelGGL((int4g128_kernel<XT, LPR, R, M, 4>), grid, dim3(256), lds, st, w, wr, s, sr, sg, xv, yv, \
                         rows, cols, cmb);                                                                    \
    else                                                                                                      \
      hipLaunchKernelGGL((int4g128_kernel<XT, LPR, R, M, 1>), grid, dim3(256), lds, st, w, wr, s, sr, sg, xv, yv, \
                         rows, cols, cmb);                                                                    \
  } while (0)
#define TT_INT4G_MODES(R)                                                                                  \
  if (xm == 1) TT_INT4G_LAUNCH(R, 1); else if (xm == 2) TT_INT4G_LAUNCH(R, 2); else if (xm == 3) TT_INT4G_LAUNCH(R, 3); \
  else TT_INT4G_LAUNCH(R, 0);
  if (rpw == 4) { TT_INT4G_MODES(4) }
  else if (rpw == 2) { TT_INT4G_MODES(2) }
  else { TT_INT4G_MODES(1) }
#undef TT_INT4G_MODES
#undef TT_INT4G_LAUNCH
  return check_launch("int4_scaled_matvec");
}

// Rows per wave of the single-matrix path: enough waves to cover the chip several
// times over before a wave takes more than one row.  Rows of several rounds take four
// rows per wave from half the lane groups, except rows of five rounds, which take two
// with all five rounds in flight (17920 x 5120: 15.5 us at one row, 14.6 at four, 13.1 at
// two in one pass); rows of several rounds stay at one row per wave up to 2048 lane
// groups (2048 x 8192: 5.43 -> 5.17 us); single-round rows of 8192 x 2048 are faster at
// two.  Rows per wave never change the bits (the oracle's order has no such parameter).
inline int int4g128_rows_per_wave(int64_t rows, int64_t cols, int lpr) {
  const int64_t groups = rows * lpr / 64;   // lane groups needed at one row each
  const int64_t rounds = (cols / 32 + lpr - 1) / lpr;
  const bool multi_round = rounds > 1;
  if (multi_round && rounds == 5 && groups >= 8192) return 2;
  if (groups >= 16384 || (multi_round && groups >= 8192)) return 4;
  if (multi_round && groups <= 2048) return 1;
  if (groups >= 2048) return 2;
  return 1;
}

// The lean kernel addresses each operand with 32-bit offsets.
inline bool int4g128_fits(int64_t rows, int64_t w_row, int64_t s_row, int64_t s_grp, int64_t cols) {
  const int64_t lim = (int64_t)1 << 31;
  return w_row > 0 && s_row >= 0 && s_grp >= 0 && rows * w_row < lim && (rows * s_row + cols / 128 * s_grp) * 2 < lim &&
         cols * 2 < lim;
}

template <typename XT>
int launch_int4g128(int lpr, const void* W, int64_t w_row, const void* S, int64_t s_row, int64_t s_grp, const void* x,
                    void* y, int rows, int cols, hipStream_t st) {
  const int rpw = int4g128_rows_per_wave(rows, cols, lpr);
  if (lpr == 64) return launch_int4g128_lpr<XT, 64>(rpw, W, w_row, S, s_row, s_grp, x, y, rows, cols, st);
  if (lpr == 32) return launch_int4g128_lpr<XT, 32>(rpw, W, w_row, S, s_row, s_grp, x, y, rows, cols, st);
  return launch_int4g128_lpr<XT, 16>(rpw, W, w_row, S, s_row, s_grp, x, y, rows, cols, st);
}

}  // namespace


extern "C" int tt_gemv_lanes_per_row(int64_t chunks, int64_t group_chunks) {
  if (chunks <= 0) return 0;
  int best = 0;
  double best_util = -1.0;
  const int cand[3] = {64, 32, 16};
  for (int c : cand) {
    if (group_chunks > 1 && (c % group_chunks) != 0) continue;
    const int64_t r = (chunks + c - 1) / c;
    const double util = (double)chunks / (double)(r * c);
    if (util > best_util + 1e-12) { best = c; best_util = util; }
  }
  return best;
}


extern "C" int tt_int4_scaled_matvec(const void* packed, int64_t w_row_bytes, const void* scales, int scale_dtype,
                                     int64_t s_row, int64_t s_group, int64_t s_pair, int affine, const void* x,
                                     int x_dtype, void* out, int out_dtype, int64_t rows, int64_t cols,
                                     int64_t group_size, void* stream) {
  const int64_t rows_arr[1] = {rows};
  const void* p_arr[1] = {packed};
  const int64_t wr_arr[1] = {w_row_bytes};
  const void* s_arr[1] = {scales};
  const int64_t sr_arr[1] = {s_row};
  const int64_t sg_arr[1] = {s_group};
  return tt_multi_int4_scaled_matvec(1, p_arr, wr_arr, s_arr, scale_dtype, sr_arr, sg_arr, s_pair, affine, rows_arr, x,
                                     x_dtype, out, out_dtype, cols, group_size, stream);
}

extern "C" int tt_multi_int4_scaled_matvec(int count, const void* const* packed, const int64_t* w_row_bytes,
                                           const void* const* scales, int scale_dtype, const int64_t* s_row,
                                           const int64_t* s_group, int64_t s_pair, int affine, const int64_t* rows,
                                           const void* x, int x_dtype, void* out, int out_dtype, int64_t cols,
                                           int64_t group_size, void* stream) {
  const char* what = "int4_scaled_matvec";
  TT_REQUIRE(count >= 1 && count <= 3, "%s: supports one to three matrices (got %d)", what, count);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: scales must be fp16 or fp32", what);
  TT_REQUIRE(x != nullptr && out != nullptr && aligned(x, 16), "%s: x must be a 16-byte aligned device pointer", what);
  int L = 1;
  bool row_mode = false;
  int rc = tt::plan_groups(what, cols, group_size, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = count;
  int64_t acc_rows = 0;
  const size_t osz = out_dtype == TT_F32 ? 4 : 2;
  for (int i = 0; i < count; i++) {
    TT_REQUIRE(rows[i] > 0, "%s: rows must be positive", what);
    TT_REQUIRE(packed[i] != nullptr && aligned(packed[i], 16) && w_row_bytes[i] % 16 == 0 && w_row_bytes[i] >= cols / 2,
               "%s: packed weights must be 16-byte aligned with a row stride >= cols/2 that is a multiple of 16", what);
    TT_REQUIRE(scales[i] != nullptr, "%s: scales missing", what);
    P.seg[i].w = static_cast<const uint8_t*>(packed[i]);
    P.seg[i].w_row = w_row_bytes[i];
    P.seg[i].s = scales[i];
    P.seg[i].s_row = s_row[i];
    P.seg[i].s_grp = s_group[i];
    P.seg[i].out = static_cast<char*>(out) + acc_rows * osz;
    P.seg[i].rows = (int)rows[i];
    acc_rows += rows[i];
  }
  TT_REQUIRE(acc_rows < (1LL << 30), "%s: too many rows", what);
  P.x = x;
  P.cols = (int)cols;
  const int Lg = L;
  P.s_pair = s_pair;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, row_mode ? 1 : L);
  TT_UNSUPPORTED(lpr > 0, "%s: no lane mapping for cols %lld / group %lld", what, (long long)cols, (long long)group_size);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (affine) {
    TT_UNSUPPORTED(!row_mode, "%s: affine int4 needs group_size < cols", what);
    if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Aff, SMode::kGroupAff, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
    return launch_types<Fmt::kInt4Aff, SMode::kGroupAff, float, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  }
  if (row_mode) {
    if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
    return launch_types<Fmt::kInt4Sym, SMode::kRow, float, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  }
  if (count == 1 && !affine && !row_mode && scale_dtype == TT_F16 && x_dtype == out_dtype && lean_group_ok(Lg) &&
      lean_fits(rows[0], w_row_bytes[0], 2 * s_row[0], cols) && s_group[0] >= 0 && s_group[0] * (cols / group_size) < (1LL << 30)) {
    // one matrix, symmetric, fp16 group scales: the lean single-matrix kernels (a
    // dedicated one for group 128, the decode hot path)
    if (Lg == 4 && int4g128_fits(rows[0], w_row_bytes[0], s_row[0], s_group[0], cols)) {
      if (x_dtype == TT_F16)
        return launch_int4g128<f16_t>(lpr, packed[0], w_row_bytes[0], scales[0], s_row[0], s_group[0], x, out,
                                      (int)rows[0], (int)cols, st);
      return launch_int4g128<bf16_t>(lpr, packed[0], w_row_bytes[0], scales[0], s_row[0], s_group[0], x, out,
                                     (int)rows[0], (int)cols, st);
    }
    LeanParams L{};
    L.w = static_cast<const uint8_t*>(packed[0]);
    L.s = scales[0];
    L.x = x;
    L.out = out;
    L.w_row = (uint32_t)w_row_bytes[0];
    L.s_row = (uint32_t)s_row[0];
    L.s_grp = (uint32_t)s_group[0];
    L.rows = (int)rows[0];
    L.cols = (int)cols;
    return lean_launch_group<Fmt::kInt4Sym, SMode::kGroup, f16_t>(Lg, x_dtype, lpr, L, 1, st, what);
  }
  if (scale_dtype == TT_F16 && Lg == 4 && x_dtype == out_dtype) {
    // the decode hot path (group 128, fp16 scales): launch shape chosen from the matrix
    int rpw, pf;
    int4_shape(acc_rows, (int)((cols / 32 + lpr - 1) / lpr), false, &rpw, &pf);
    if (x_dtype == TT_F16) return launch_int4_g128<f16_t, f16_t, Pro::kLoad, false>(lpr, rpw, pf, P, st, what);
    return launch_int4_g128<bf16_t, bf16_t, Pro::kLoad, false>(lpr, rpw, pf, P, st, what);
  }
  if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kGroup, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  return launch_types<Fmt::kInt4Sym, SMode::kGroup, float, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
}

extern "C" int tt_attention_combine_int4_matvec(const float* scratch, int64_t scratch_floats, const int32_t* tokens_dev,
                                                int64_t tokens, int64_t max_tokens, int64_t heads, int64_t head_dim,
                                                int dtype, const void* packed, int64_t w_row_bytes, const void* scales,
                                                int64_t s_row, int64_t s_group, void* attn_out, void* out, int64_t rows,
                                                void* stream) {
  const char* what = "attention_combine_int4_matvec";
  TT_REQUIRE(scratch && packed && scales && out, "%s: null pointer", what);
  TT_REQUIRE(dtype == TT_F16 || dtype == TT_BF16, "%s: activation dtype must be fp16 or bf16", what);
  TT_REQUIRE(tokens_dev != nullptr || (tokens > 0 && tokens <= max_tokens), "%s: attention requires at least one KV token", what);
  TT_REQUIRE(tokens_dev == nullptr || (tokens >= 0 && tokens <= 1), "%s: device token count offset must be 0 or 1", what);
  TT_UNSUPPORTED(head_dim == 64 && heads > 0 && heads * head_dim <= 2048,
                 "%s: combines head_dim-64 attention of at most 32 query heads", what);
  TT_REQUIRE(max_tokens > 0 && max_tokens % 64 == 0, "%s: capacity must be a whole number of 64-token chunks", what);
  const int64_t cols = heads * head_dim, chunks = max_tokens / 64;
  TT_REQUIRE(scratch_floats >= kAttnCounters + heads * chunks * (2 + head_dim), "%s: scratch too small", what);
  TT_REQUIRE(rows > 0 && packed && aligned(packed, 16) && w_row_bytes % 16 == 0 && w_row_bytes >= cols / 2,
             "%s: packed weights must be 16-byte aligned with a row stride >= cols/2 that is a multiple of 16", what);
  TT_REQUIRE(attn_out == nullptr || aligned(attn_out, 16), "%s: attention output must be 16-byte aligned", what);
  TT_REQUIRE(int4g128_fits(rows, w_row_bytes, s_row, s_group, cols) && s_row >= 0 && s_group >= 0,
             "%s: operands too large for 32-bit offsets", what);
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 4);
  TT_UNSUPPORTED(lpr > 0, "%s: no lane mapping for cols %lld", what, (long long)cols);
  // the partials follow the arrival counters of the attention scratch
  const float* part = scratch + kAttnCounters;
  CombineSrc C{};
  C.pm = part;
  C.pl = part + heads * chunks;
  C.po = part + 2 * heads * chunks;
  C.tokens_dev = tokens_dev;
  C.tokens = (int)tokens;
  C.max_tokens = (int)max_tokens;
  C.max_chunks = (int)chunks;
  C.xout = static_cast<uint16_t*>(attn_out);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int rpw = int4g128_rows_per_wave(rows, cols, lpr);
  auto go = [&](auto t) -> int {
    using XT = decltype(t);
    if (lpr == 64) return launch_int4g128_lpr<XT, 64>(rpw, packed, w_row_bytes, scales, s_row, s_group, nullptr, out, (int)rows, (int)cols, st, &C);
    if (lpr == 32) return launch_int4g128_lpr<XT, 32>(rpw, packed, w_row_bytes, scales, s_row, s_group, nullptr, out, (int)rows, (int)cols, st, &C);
    return launch_int4g128_lpr<XT, 16>(rpw, packed, w_row_bytes, scales, s_row, s_group, nullptr, out, (int)rows, (int)cols, st, &C);
  };
  if (dtype == TT_F16) return go(f16_t{});
  return go(bf16_t{});
}

extern "C" int tt_int4_selected_matvec(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                       const void* scales, int scale_dtype, int64_t s_expert, int64_t s_row,
                                       int64_t s_group, const void* x, int x_dtype, int64_t x_slot,
                                       const void* expert_indices, int index_bytes, int64_t selected, void* out, int out_dtype,
                                       int64_t out_slot, int64_t rows, int64_t cols, int64_t group_size,
                                       void* stream) {
  const char* what = "int4_selected_matvec";
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: scales must be fp16 or fp32", what);
  TT_REQUIRE(selected >= 1 && selected <= 65535 && expert_indices != nullptr, "%s: need 1..65535 selected experts", what);
  int ishift;
  TT_REQUIRE(index_shift(index_bytes, &ishift), "%s: expert indices must be int32 or int64", what);
  TT_REQUIRE(packed && aligned(packed, 16) && w_row_bytes % 16 == 0 && w_expert_bytes % 16 == 0,
             "%s: packed weights must be 16-byte aligned", what);
  TT_REQUIRE(x && aligned(x, 16) && (x_slot % 8) == 0, "%s: x must be 16-byte aligned (slot stride a multiple of 8)", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L = 1;
  bool row_mode = false;
  int rc = tt::plan_groups(what, cols, group_size, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, s_group, out, (int)rows};
  P.x = x;
  P.x_slot = x_slot;
  P.experts = expert_indices;
  P.ishift = ishift;
  P.w_expert = w_expert_bytes;
  P.s_expert = s_expert;
  P.out_slot = out_slot;
  P.cols = (int)cols;
  const int Lg = L;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, row_mode ? 1 : L);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!row_mode && scale_dtype == TT_F16 && x_dtype == out_dtype && lean_group_ok(Lg) &&
      lean_fits(rows, w_row_bytes, 2 * s_row, cols) && s_group >= 0 && s_group * (cols / group_size) < (1LL << 30)) {
    LeanParams Q{};
    Q.w = static_cast<const uint8_t*>(packed);
    Q.s = scales;
    Q.x = x;
    Q.out = out;
    Q.experts = expert_indices;
    Q.ishift = ishift;
    Q.w_expert = w_expert_bytes;
    Q.s_expert = s_expert;
    Q.x_slot = x_slot;
    Q.out_slot = out_slot;
    Q.w_row = (uint32_t)w_row_bytes;
    Q.s_row = (uint32_t)s_row;
    Q.s_grp = (uint32_t)s_group;
    Q.rows = (int)rows;
    Q.cols = (int)cols;
    return lean_launch_group<Fmt::kInt4Sym, SMode::kGroup, f16_t>(Lg, x_dtype, lpr, Q, (int)selected, st, what);
  }
  if (row_mode) {
    if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, (int)selected, st, what);
    return launch_types<Fmt::kInt4Sym, SMode::kRow, float, 4>(x_dtype, out_dtype, Lg, lpr, P, (int)selected, st, what);
  }
  if (scale_dtype == TT_F16) return launch_types<Fmt::kInt4Sym, SMode::kGroup, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, (int)selected, st, what);
  return launch_types<Fmt::kInt4Sym, SMode::kGroup, float, 4>(x_dtype, out_dtype, Lg, lpr, P, (int)selected, st, what);
}

