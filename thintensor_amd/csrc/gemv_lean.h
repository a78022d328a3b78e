// Lean single-matrix dequant GEMV for gfx950: the reduction order of gemv_kernel
// (gemv_impl.h, documented in tt_gemv.h) without its multi-segment, persistent-loop
// and epilogue machinery.
//
//   * one batch of ROWS * (64 / LPR) rows per wave, one wave per batch;
//   * a short argument block read in one scalar batch; row bases are wave-uniform
//     scalars, per-lane offsets are 32-bit (the host keeps each operand under 2 GiB);
//   * round 0's weight, metadata and activation loads are all issued before the first
//     wait, later rounds are fetched one ahead;
//   * the activation chunk comes from global memory per lane (XM = 1, one round per
//     row) or from a per-workgroup LDS copy behind one barrier (XM = 0).
// Optional device-side expert selection (blockIdx.y = slot) covers the
// selected-expert entry points.
#pragma once

#include "gemv_impl.h"

namespace tt {

struct LeanParams {
  const uint8_t* w;         // weights (expert 0)
  const void* s;            // scales / exponents (expert 0), nullptr for SMode::kNone
  const void* x;            // activations (slot 0)
  void* out;                // output (slot 0)
  const void* bias;         // optional, output dtype
  const void* experts;      // expert id per slot (int32 or int64), nullptr: dense
  int64_t w_expert, s_expert, x_slot, out_slot;
  int64_t s_pair;           // affine: element offset of the second value of a pair
  uint32_t w_row;           // bytes between rows
  uint32_t s_row, s_grp;    // scale element strides
  int rows, cols, aff_zero;
  int ishift;               // log2 of the expert id size in 32-bit words
};

template <Fmt F, SMode SM, typename XT, typename OT, typename ST, int LPR, int ROWS, int L, int XM, bool EXP,
          int PFR = 1>
__global__ __launch_bounds__(256) void lean_gemv_kernel(const LeanParams P) {
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr bool kGroup = SM == SMode::kGroup || SM == SMode::kGroupAff;
  constexpr int LG = kGroup ? L : 1;
  constexpr int SUBS = 64 / LPR;
  constexpr int NVG = kGroup ? (ROWS / LG > 0 ? ROWS / LG : 1) : ROWS;   // accumulators per lane
  constexpr int GLEV = kGroup ? (log2c(LG) < log2c(ROWS) ? log2c(LG) : log2c(ROWS)) : 0;
  constexpr int NS = kGroup ? NVG : 0;                                     // scale values per round
  constexpr int kXR = 4;
  static_assert(ROWS <= LPR && LG <= LPR, "batch rows and groups must fit the lane group");
  extern __shared__ uint32_t xs_lds[];

  const int lane = threadIdx.x & 63;
  const int sub = lane / LPR;
  const int l = lane % LPR;
  const int rows = P.rows, cols = P.cols;
  const int nchunks = cols >> 5;
  const int rounds = (nchunks + LPR - 1) / LPR;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int row0 = (int)(blockIdx.x * 4 + wave) * (ROWS * SUBS);   // wave-uniform
  const int slot = blockIdx.y;
  const uint8_t* W = P.w;
  const ST* S = reinterpret_cast<const ST*>(P.s);
  if constexpr (EXP) {   // compile-time, so the argument loads stay in one scalar batch
    const int64_t e = load_expert(P.experts, P.ishift, slot);
    W += e * P.w_expert;
    S += e * P.s_expert;
  }
  const uint16_t* x = reinterpret_cast<const uint16_t*>(P.x) + (int64_t)slot * P.x_slot;

  // activation pieces for the LDS copies (clamped indices: duplicates, no branch)
  const int xn = cols >> 3;
  uint4 xreg[kXR];
  uint32_t xidx[kXR];
  if constexpr (XM == 0) {
#pragma unroll
    for (int k = 0; k < kXR; k++) {
      const int idx = (int)threadIdx.x + 256 * k;
      xidx[k] = idx < xn ? idx : xn - 1;
      xreg[k] = reinterpret_cast<const uint4*>(x)[xidx[k]];
    }
  }

  // row i of lane group `sub` is row0 + i * SUBS + sub, clamped to the last row
  const int rlast = rows - 1;
  const uint8_t* wrow[ROWS];
  uint32_t wlane[ROWS];
  bool rv[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    const int r0 = row0 + i * SUBS;
    const int rc = r0 < rlast ? r0 : rlast;
    const int rl = r0 + sub < rlast ? r0 + sub : rlast;
    wrow[i] = W + (size_t)rc * P.w_row;
    wlane[i] = SUBS == 1 ? 0u : (uint32_t)(rl - rc) * P.w_row;
    rv[i] = r0 + sub < rows;
  }
  const int rbase = row0 < rlast ? row0 : rlast;
  const ST* sbase = SM == SMode::kNone ? S : S + (size_t)rbase * P.s_row;
  uint32_t soff[NS > 0 ? NS : 1];
  bool sv[NS > 0 ? NS : 1];
  if constexpr (kGroup) {
#pragma unroll
    for (int k = 0; k < NS; k++) {
      const int r = row0 + rs_row<ROWS>(l, GLEV, k) * SUBS + sub;
      sv[k] = r < rows;
      soff[k] = (uint32_t)((sv[k] ? r : rlast) - rbase) * P.s_row;
    }
  }
  uint32_t eoff[ROWS];   // block-exponent row offsets
  if constexpr (SM == SMode::kBlockE8) {
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      const int r = row0 + i * SUBS + sub;
      eoff[i] = (uint32_t)((r < rows ? r : rlast) - rbase) * P.s_row;
    }
  }
  // the row scale of the row this lane stores, loaded up front
  const int frow = row0 + rs_row<ROWS>(l, log2c(ROWS), 0) * SUBS + sub;
  const bool fstore = (l >> log2c(ROWS)) == 0;
  ST rscale{};
  if constexpr (SM == SMode::kRow) rscale = sbase[(uint32_t)((frow < rows ? frow : rlast) - rbase) * P.s_row];

  struct Round {
    Raw<B> w[ROWS];
    ST s[NS > 0 ? NS : 1], m[NS > 0 ? NS : 1];
    uint8_t e[SM == SMode::kBlockE8 ? ROWS : 1];
    uint4 xc[XM == 1 ? 4 : 1];
  };
  auto fetch = [&](int r, Round& d) {
    uint32_t j = (uint32_t)(r * LPR + l);
    j = j < (uint32_t)nchunks ? j : (uint32_t)nchunks - 1;
#pragma unroll
    for (int i = 0; i < ROWS; i++) d.w[i] = load_raw<B>(wrow[i] + (wlane[i] + j * (uint32_t)B));
    if constexpr (XM == 1) {
#pragma unroll
      for (int q = 0; q < 4; q++) d.xc[q] = *reinterpret_cast<const uint4*>(x + (j * 32u + 8u * q));
    }
    if constexpr (kGroup) {
#pragma unroll
      for (int k = 0; k < NS; k++) {
        const uint32_t off = soff[k] + (j / (uint32_t)LG) * P.s_grp;
        d.s[k] = sbase[off];
        if constexpr (SM == SMode::kGroupAff) d.m[k] = sbase[off + (uint32_t)P.s_pair];
      }
    }
    if constexpr (SM == SMode::kBlockE8) {
#pragma unroll
      for (int i = 0; i < ROWS; i++) d.e[i] = reinterpret_cast<const uint8_t*>(sbase)[eoff[i] + j];
    }
  };
  // PFR > 1: rounds requested PFR at a time (past the last they re-read its chunk, unused)
  Round ring[PFR];
#pragma unroll
  for (int k = 0; k < PFR; k++) fetch(k, ring[k]);

  const uint32_t* xs = xs_lds;
  if constexpr (XM == 0) {
    uint4* xl = reinterpret_cast<uint4*>(xs_lds);
#pragma unroll
    for (int k = 0; k < kXR; k++) xl[xidx[k]] = xreg[k];
    for (int idx = threadIdx.x + 256 * kXR; idx < xn; idx += 256) xl[idx] = reinterpret_cast<const uint4*>(x)[idx];
    lds_barrier();
  }

  float acc[NVG];
#pragma unroll
  for (int k = 0; k < NVG; k++) acc[k] = 0.0f;
  auto consume = [&](const Round& c, int r) {
    const int j = r * LPR + l;
    const bool cv = j < nchunks;
    uint32_t xw[16];
    {
      const uint4* xp = reinterpret_cast<const uint4*>(xs + (cv ? j : 0) * 16);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint4 v = XM == 1 ? c.xc[q] : xp[q];
        xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
      }
    }
    float p[ROWS];
    chunk_dot_rows<F, XT, ROWS>(c.w, xw, p);
#pragma unroll
    for (int i = 0; i < ROWS; i++) p[i] = (cv && rv[i]) ? p[i] : 0.0f;
    if constexpr (SM == SMode::kNone || SM == SMode::kRow) {
#pragma unroll
      for (int i = 0; i < ROWS; i++) acc[i] = acc[i] + p[i];
    } else if constexpr (SM == SMode::kBlockE8) {
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        const float t = p[i] * pow2i((int)c.e[i] - 127);
        acc[i] = acc[i] + ((cv && rv[i]) ? t : 0.0f);
      }
    } else {
      float xsum = 0.0f;
      if constexpr (SM == SMode::kGroupAff) {
#pragma unroll
        for (int e = 0; e < 32; e++) xsum = xsum + xv<XT>(xw, e);
        xsum = cv ? xsum : 0.0f;
        reduce_range<1, 1, LG>(&xsum);
      }
      reduce_range<ROWS, 1, LG>(p);
#pragma unroll
      for (int k = 0; k < NVG; k++) {
        const float sk = to_f32(c.s[k]);
        float t;
        if constexpr (SM == SMode::kGroupAff) {
          float m = to_f32(c.m[k]);
          if (P.aff_zero) m = -(m * sk);
          t = __builtin_fmaf(xsum, m, p[k] * sk);
        } else {
          t = p[k] * sk;
        }
        // a group counts when its first chunk is in range (a ragged last group of a
        // block-scaled matrix keeps its partial sum on every lane of the group)
        const bool gv = (j & ~(LG - 1)) < nchunks;
        acc[k] = acc[k] + ((gv && sv[k]) ? t : 0.0f);
      }
    }
  };
  if constexpr (PFR == 1) {
    int r = 0;
    do {   // the host guarantees one round (cols >= 32)
      Round nxt;
      const bool more = r + 1 < rounds;
      if (more) fetch(r + 1, nxt);
      consume(ring[0], r);
      if (more) ring[0] = nxt;
    } while (++r < rounds);
  } else {
    for (int r0 = 0;;) {
#pragma unroll
      for (int k = 0; k < PFR; k++)
        if (r0 + k < rounds) consume(ring[k], r0 + k);
      r0 += PFR;
      if (r0 >= rounds) break;
#pragma unroll
      for (int k = 0; k < PFR; k++) fetch(r0 + k, ring[k]);
    }
  }

  if constexpr (kGroup) reduce_range<NVG, LG, LPR>(acc);
  else reduce_range<ROWS, 1, LPR>(acc);
  float v = acc[0];
  const bool ok = fstore && frow < rows;
  if constexpr (SM == SMode::kRow) v = v * to_f32(rscale);
  if (ok) {
    OT* out = reinterpret_cast<OT*>(P.out) + (int64_t)slot * P.out_slot;
    if (P.bias != nullptr) v = round_to<OT>(v) + to_f32(reinterpret_cast<const OT*>(P.bias)[frow]);
    store<OT>(out + frow, v);
  }
}

// ------------------------------------------------------------------ dispatch

// Rows per wave: enough waves to cover the chip several times over before a wave
// takes more than one row (measured on the int4 g128 shapes of the decode step).
inline int lean_rows_per_wave(int64_t rows, int lpr, int slots) {
  const int64_t groups = rows * lpr / 64 * slots;
  if (groups >= 16384) return 4;
  if (groups >= 2048) return 2;
  return 1;
}

// Activation staging: per-lane global reads when a row takes one round, one LDS copy
// per workgroup otherwise.
inline int lean_x_mode(int64_t cols, int lpr) { return cols / 32 <= lpr ? 1 : 0; }

// Whether the lean kernel can address the operands with 32-bit offsets.
inline bool lean_fits(int64_t rows, int64_t w_row, int64_t s_row_bytes, int64_t cols) {
  const int64_t lim = (int64_t)1 << 31;
  return rows > 0 && w_row > 0 && rows * w_row < lim && rows * s_row_bytes < lim && cols * 2 < lim && cols <= 32768;
}

template <Fmt F, SMode SM, typename XT, typename OT, typename ST, int LPR, int L>
int lean_launch_lpr(const LeanParams& P, int slots, hipStream_t st, const char* what) {
  int rpw = lean_rows_per_wave(P.rows, LPR, slots);
  // dense rows of two rounds, one slot, under 4096 lane groups (the gpt-oss o_proj, 2880 x
  // 4096): one row per wave, twice the waves (decode 742.7 -> 747.3 tok/s; four rows 740.0)
  if (SM == SMode::kNone && slots == 1 && rpw == 2 && (P.cols / 32 + LPR - 1) / LPR == 2 &&
      (int64_t)P.rows * LPR / 64 < 4096)
    rpw = 1;
  const int xm = lean_x_mode(P.cols, LPR);
  const int per_wave = rpw * (64 / LPR);
  const int64_t waves = ((int64_t)P.rows + per_wave - 1) / per_wave;
  const dim3 grid((unsigned)((waves + 3) / 4), (unsigned)slots);
  const size_t lds = xm == 1 ? 0 : (size_t)P.cols * 2;
  // dense rows of two rounds, up to two rows per wave: both rounds requested at once
  constexpr bool kDense2 = SM == SMode::kNone;
  const bool two = kDense2 && rpw <= 2 && (P.cols / 32 + LPR - 1) / LPR == 2;
  // rows of three to five rounds, up to two rows per wave: every round requested at once
  // (same bits; 17920 x 5120 fp8 20.9 -> 19.2 us, 5120 x 5120 fp8 9.9 -> 8.5 us, 17920 x 3072
  // fp8 13.8 -> 12.6 us at three rounds ahead; five ahead for four rounds re-reads one chunk)
  const int lrounds = (P.cols / 32 + LPR - 1) / LPR;
  const int ahead = rpw <= 2 && lrounds >= 3 && lrounds <= 5 ? (lrounds == 3 ? 3 : 5) : 0;
#define TT_LEAN(R, M)                                                                                     \
  if (P.experts != nullptr)                                                                               \
    hipLaunchKernelGGL((lean_gemv_kernel<F, SM, XT, OT, ST, LPR, R, L, M, true>), grid, dim3(256), lds, st, P); \
  else if (ahead == 3)                                                                                    \
    hipLaunchKernelGGL((lean_gemv_kernel<F, SM, XT, OT, ST, LPR, R, L, M, false, 3>), grid, dim3(256), lds, st, P); \
  else if (ahead == 5)                                                                                    \
    hipLaunchKernelGGL((lean_gemv_kernel<F, SM, XT, OT, ST, LPR, R, L, M, false, 5>), grid, dim3(256), lds, st, P); \
  else if (two)                                                                                           \
    hipLaunchKernelGGL((lean_gemv_kernel<F, SM, XT, OT, ST, LPR, R, L, M, false, kDense2 ? 2 : 1>), grid,  \
                       dim3(256), lds, st, P);                                                            \
  else                                                                                                    \
    hipLaunchKernelGGL((lean_gemv_kernel<F, SM, XT, OT, ST, LPR, R, L, M, false>), grid, dim3(256), lds, st, P)
#define TT_LEAN_X(R) \
  if (xm == 1) { TT_LEAN(R, 1); } else { TT_LEAN(R, 0); }
  if (rpw == 4) { TT_LEAN_X(4) }
  else if (rpw == 2) { TT_LEAN_X(2) }
  else { TT_LEAN_X(1) }
#undef TT_LEAN_X
#undef TT_LEAN
  return check_launch(what);
}

template <Fmt F, SMode SM, typename XT, typename OT, typename ST, int L>
int lean_launch_l(int lpr, const LeanParams& P, int slots, hipStream_t st, const char* what) {
  switch (lpr) {
    case 64: return lean_launch_lpr<F, SM, XT, OT, ST, 64, L>(P, slots, st, what);
    case 32:
      if constexpr (L <= 32) return lean_launch_lpr<F, SM, XT, OT, ST, 32, L>(P, slots, st, what);
      break;
    case 16:
      if constexpr (L <= 16) return lean_launch_lpr<F, SM, XT, OT, ST, 16, L>(P, slots, st, what);
      break;
    default: break;
  }
  set_error("%s: invalid lanes per row %d for a %d-chunk group", what, lpr, L);
  return TT_ERR_INVALID;
}

// Activation dtype == output dtype (fp16 or bf16); other pairs use gemv_kernel.
template <Fmt F, SMode SM, typename ST, int L>
int lean_launch(int x_dtype, int lpr, const LeanParams& P, int slots, hipStream_t st, const char* what) {
  if (x_dtype == TT_F16) return lean_launch_l<F, SM, f16_t, f16_t, ST, L>(lpr, P, slots, st, what);
  return lean_launch_l<F, SM, bf16_t, bf16_t, ST, L>(lpr, P, slots, st, what);
}

// Group sizes of 32, 64 and 128 elements (L = 1, 2, 4 chunks).
inline bool lean_group_ok(int L) { return L == 1 || L == 2 || L == 4; }

template <Fmt F, SMode SM, typename ST>
int lean_launch_group(int L, int x_dtype, int lpr, const LeanParams& P, int slots, hipStream_t st, const char* what) {
  switch (L) {
    case 1: return lean_launch<F, SM, ST, 1>(x_dtype, lpr, P, slots, st, what);
    case 2: return lean_launch<F, SM, ST, 2>(x_dtype, lpr, P, slots, st, what);
    case 4: return lean_launch<F, SM, ST, 4>(x_dtype, lpr, P, slots, st, what);
  }
  set_error("%s: unsupported group of %d chunks", what, L);
  return TT_ERR_UNSUPPORTED;
}

}  // namespace tt
