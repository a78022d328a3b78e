// Fused MoE down kernels: down GEMV of the selected experts + router-weighted sum in
// slot order (E8M0 block-scaled q1, q2, MXFP4); expert ids and scores are read on the device.
#include "moe_common.h"

namespace tt {

// One block owns RB = RPW * (64 / LPR) output rows.  Its four waves split the
// selected slots (wave w computes slots w, w + 4, ...), each slot's row values
// v = round(dot) (+ bias, rounded again) go to LDS, and after the barrier lane t of
// the block combines row t in slot order: c = fma(v_s, score_s, c) from +0.
template <Fmt F, typename XT, typename OT, typename RT, int LPR, int RPW>
__global__ __launch_bounds__(256) void weighted_down_kernel(DownParams P) {
  extern __shared__ uint32_t xs_lds[];
  constexpr int SUBS = 64 / LPR;
  constexpr int RB = RPW * SUBS;
  const int words = P.cols >> 1;
  float* vals = reinterpret_cast<float*>(xs_lds + P.slots * words);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int sub = lane / LPR, l = lane % LPR;
  const int nchunks = P.cols >> 5;
  const int row0 = blockIdx.x * RB;
  int row[RPW];
  bool rv[RPW];
#pragma unroll
  for (int i = 0; i < RPW; i++) {
    row[i] = row0 + i * SUBS + sub;
    rv[i] = row[i] < P.rows;
  }
  const uint8_t* wrow[RPW];
  const uint8_t* srow[RPW];
  int64_t e = 0;
  auto point = [&](int s) {
    e = load_expert(P.experts, P.ishift, (int64_t)blockIdx.y * P.slots + s);
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      wrow[i] = P.w + e * P.w_expert + (int64_t)row[i] * P.w_row;
      srow[i] = P.s + e * P.s_expert + (int64_t)row[i] * P.s_row;
    }
  };
  E8Round<F, RPW> cur;
  int s = wave;
  if (s < P.slots) {
    point(s);
    e8_fetch<F, LPR, RPW>(cur, 0, l, nchunks, wrow, srow, rv);
  }
  for (int t = 0; t < P.slots; t++) {
    const uint32_t* xg = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(P.x) +
                                                           ((int64_t)blockIdx.y * P.slots + t) * P.x_slot);
    for (int i = threadIdx.x; i < words; i += blockDim.x) xs_lds[t * words + i] = xg[i];
  }
  __syncthreads();
  for (; s < P.slots; s += nwaves) {
    if (s != wave) {
      point(s);
      e8_fetch<F, LPR, RPW>(cur, 0, l, nchunks, wrow, srow, rv);
    }
    float dot[RPW];
    e8_rows_dot<F, XT, LPR, RPW>(cur, wrow, srow, rv, xs_lds + s * words, nchunks, l, dot);
#pragma unroll
    for (int i = 0; i < RPW; i++) {
      if (l != i || !rv[i]) continue;
      float v = round_to<RT>(dot[i]);
      if (P.bias != nullptr) v = round_to<RT>(v + ld_typed(P.bias, P.bias_dtype, e * P.bias_expert + row[i]));
      vals[s * RB + i * SUBS + sub] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x < RB && row0 + (int)threadIdx.x < P.rows) {
    float c = 0.0f;
    for (int t = 0; t < P.slots; t++)
      c = __builtin_fmaf(vals[t * RB + threadIdx.x], ld_typed(P.scores, P.score_dtype, (int64_t)blockIdx.y * P.slots + t), c);
    store<OT>(reinterpret_cast<OT*>(P.out) + (int64_t)blockIdx.y * P.out_token + row0 + threadIdx.x, c);
  }
}

// ------------------------------------------------------------------ lean variants
// Same arithmetic as swiglu_kernel / weighted_down_kernel, laid out like the lean GEMV
// (gemv_lean.h): one batch per wave, every load of a round issued before its first
// use, the next round in flight while one is consumed, and the cross-row work done in
// registers after one reduce-scatter.

// Weighted down: every wave computes its ROWS rows (per lane group) for all S selected
// slots; after the reduction the lane holding a row folds the slots in slot order:
// c = fma(v_s, score_s, c) from +0.  The grid is small (one row per lane group), so
// latency is hidden inside each wave: the slots' activations are requested first
// (into registers, then LDS), then R rounds of every slot's weights at once.
template <Fmt F, typename XT, typename OT, typename RT, int LPR, int ROWS, int S>
__global__ __launch_bounds__(256) void down_lean_kernel(const DownParams P) {
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr int SUBS = 64 / LPR;
  constexpr int R = 16 / (S * ROWS) < 1 ? 1 : (16 / (S * ROWS) > 4 ? 4 : 16 / (S * ROWS));   // rounds in flight
  constexpr int kXR = 4;   // 16-byte activation pieces per thread per register array (two arrays)
  extern __shared__ uint32_t xs_lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int sub = lane / LPR, l = lane % LPR;
  const int nchunks = P.cols >> 5;
  const int rounds = (nchunks + LPR - 1) / LPR;
  const int words = P.cols >> 1;
  const int n0 = (int)(blockIdx.x * 4 + wave) * (ROWS * SUBS);

  // activations: piece idx of the LDS copy (slot t at piece t * xn) is piece idx - t * xn
  // of slot t; the first 256 * 2 * kXR pieces through registers, indices clamped
  const int tok = blockIdx.y;   // token: its S slots' activations, experts and scores
  const uint16_t* xtok = reinterpret_cast<const uint16_t*>(P.x) + (int64_t)tok * S * P.x_slot;
  const int xn = P.cols >> 3;
  const int xtotal = xn * S;
  // (two arrays of four: one array of eight is kept in scratch memory by the compiler)
  uint4 xra[kXR], xrb[kXR];
  int xidx[2 * kXR];
  auto xload = [&](int k) -> uint4 {
    const int idx = threadIdx.x + 256 * k;
    xidx[k] = idx < xtotal ? idx : xtotal - 1;
    int t = 0;
#pragma unroll
    for (int q = 1; q < S; q++) t += xidx[k] >= q * xn ? 1 : 0;
    const uint4* xg = reinterpret_cast<const uint4*>(xtok + (int64_t)t * P.x_slot);
    return xg[xidx[k] - t * xn];
  };
#pragma unroll
  for (int k = 0; k < kXR; k++) xra[k] = xload(k);
#pragma unroll
  for (int k = 0; k < kXR; k++) xrb[k] = xload(kXR + k);

  int64_t e[S];
#pragma unroll
  for (int s = 0; s < S; s++) e[s] = load_expert(P.experts, P.ishift, (int64_t)tok * S + s);
  const uint8_t* wrow[S][ROWS];
  const uint8_t* srow[S][ROWS];
  bool rv[ROWS];
  int rcl[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    const int n = n0 + i * SUBS + sub;
    rv[i] = n < P.rows;
    rcl[i] = rv[i] ? n : P.rows - 1;
  }
#pragma unroll
  for (int s = 0; s < S; s++)
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      wrow[s][i] = P.w + e[s] * P.w_expert + (int64_t)rcl[i] * P.w_row;
      srow[s][i] = P.s + e[s] * P.s_expert + (int64_t)rcl[i] * P.s_row;
    }
  struct Round {
    Raw<B> w[S][ROWS];
    uint8_t ex[S][ROWS];
  };
  // rounds past the last clamp to the last chunk (re-reads, results unused)
  auto fetch = [&](int r, Round& d) {
    uint32_t j = (uint32_t)(r * LPR + l);
    j = j < (uint32_t)nchunks ? j : (uint32_t)nchunks - 1;
#pragma unroll
    for (int s = 0; s < S; s++)
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        d.w[s][i] = load_raw<B>(wrow[s][i] + j * (uint32_t)B);
        d.ex[s][i] = srow[s][i][j];
      }
  };
  Round d[R];
#pragma unroll
  for (int k = 0; k < R; k++) fetch(k, d[k]);
  __builtin_amdgcn_sched_barrier(0);
  {
    uint4* xl = reinterpret_cast<uint4*>(xs_lds);
#pragma unroll
    for (int k = 0; k < kXR; k++) xl[xidx[k]] = xra[k];
#pragma unroll
    for (int k = 0; k < kXR; k++) xl[xidx[kXR + k]] = xrb[k];
    for (int idx = threadIdx.x + 256 * 2 * kXR; idx < xtotal; idx += 256) {
      int t = 0;
#pragma unroll
      for (int q = 1; q < S; q++) t += idx >= q * xn ? 1 : 0;
      xl[idx] = reinterpret_cast<const uint4*>(xtok + (int64_t)t * P.x_slot)[idx - t * xn];
    }
  }
  lds_barrier();

  float acc[S][ROWS];
#pragma unroll
  for (int s = 0; s < S; s++)
#pragma unroll
    for (int i = 0; i < ROWS; i++) acc[s][i] = 0.0f;
  auto consume = [&](const Round& c, int r) {
    const int j = r * LPR + l;
    const bool cv = j < nchunks;
#pragma unroll
    for (int s = 0; s < S; s++) {
      uint32_t xw[16];
      const uint4* xp = reinterpret_cast<const uint4*>(xs_lds + s * words + (cv ? j : 0) * 16);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint4 v = xp[q];
        xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
      }
      float p[ROWS];
      chunk_dot_rows<F, XT, ROWS>(c.w[s], xw, p);
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        const float t = p[i] * pow2i((int)c.ex[s][i] - 127);
        acc[s][i] = acc[s][i] + ((cv && rv[i]) ? t : 0.0f);
      }
    }
  };
  for (int r0 = 0;;) {
#pragma unroll
    for (int k = 0; k < R; k++)
      if (r0 + k < rounds) consume(d[k], r0 + k);
    r0 += R;
    if (r0 >= rounds) break;
#pragma unroll
    for (int k = 0; k < R; k++) fetch(r0 + k, d[k]);
  }
#pragma unroll
  for (int s = 0; s < S; s++) reduce_range<ROWS, 1, LPR>(acc[s]);
  const int n = n0 + rs_row<ROWS>(l, log2c(ROWS), 0) * SUBS + sub;
  if ((l >> log2c(ROWS)) != 0 || n >= P.rows) return;
  float c = 0.0f;
#pragma unroll
  for (int s = 0; s < S; s++) {
    float v = round_to<RT>(acc[s][0]);
    if (P.bias != nullptr) v = round_to<RT>(v + ld_typed(P.bias, P.bias_dtype, e[s] * P.bias_expert + n));
    c = __builtin_fmaf(v, ld_typed(P.scores, P.score_dtype, tok * S + s), c);
  }
  store<OT>(reinterpret_cast<OT*>(P.out) + (int64_t)tok * P.out_token + n, c);
}

constexpr int kDownSlotRounds = 4;   // rounds of a row per lane group (all in flight)
constexpr int kDownSlotPieces = 6;   // 16-byte activation pieces per lane (cols <= 3072)

// Weighted down with one wave per (row block, slot): wave s of a workgroup computes slot
// s's values of the workgroup's ROWS * SUBS rows (ROWS rows per lane group;
// down_lean_kernel's chunk order, lane reduction and rounding).  Each wave stages its own
// slot's activation in its own LDS region (no workgroup barrier before the dot
// products) while every round of its weights, the bias and the router scores are in
// flight.  The rounded row values meet in LDS and thread g folds row g's slots in slot
// order: c = fma(v_s, score_s, c) from +0, the same bits as down_lean_kernel.  S times
// the waves of down_lean_kernel for the same work, few registers per wave, so the whole
// grid at the gpt-oss shape is resident at once: one memory phase, not two generations.
template <Fmt F, typename XT, typename OT, typename RT, int LPR, int S, int ROWS>
__global__ __launch_bounds__(64 * S) void down_slot_kernel(const DownParams P) {
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr int SUBS = 64 / LPR;
  constexpr int RB = ROWS * SUBS;        // rows of the workgroup (row i * SUBS + sub of lane group sub)
  constexpr int R = kDownSlotRounds;
  extern __shared__ uint4 xs_pieces[];   // [S][cols / 8]
  __shared__ float vals[S][RB];
  const int lane = threadIdx.x & 63;
  const int s = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int sub = lane / LPR, l = lane % LPR;
  const int nchunks = P.cols >> 5;
  const int xn = P.cols >> 3;
  const int tok = blockIdx.y;
  const int row0 = blockIdx.x * RB;
  int n[ROWS], ncl[ROWS];
  bool rv[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    n[i] = row0 + i * SUBS + sub;
    rv[i] = n[i] < P.rows;
    ncl[i] = rv[i] ? n[i] : P.rows - 1;
  }
  // this slot's activation pieces first (they do not wait for the expert id), clamped
  const uint4* xg = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(P.x) +
                                                   ((int64_t)tok * S + s) * P.x_slot);
  // (native 4-vectors: an array of the uint4 struct type is kept in scratch memory)
  typedef uint32_t piece_t __attribute__((ext_vector_type(4)));
  const piece_t* xgp = reinterpret_cast<const piece_t*>(xg);
  piece_t xr[kDownSlotPieces];
#pragma unroll
  for (int k = 0; k < kDownSlotPieces; k++) {
    const int i = lane + 64 * k;
    xr[k] = xgp[i < xn ? i : xn - 1];
  }
  const int64_t e = load_expert(P.experts, P.ishift, (int64_t)tok * S + s);
  const uint8_t* wrow[ROWS];
  const uint8_t* srow[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    wrow[i] = P.w + e * P.w_expert + (int64_t)ncl[i] * P.w_row;
    srow[i] = P.s + e * P.s_expert + (int64_t)ncl[i] * P.s_row;
  }
  // every round of the rows (rounds past the last clamp to the last chunk: re-reads,
  // results unused)
  Raw<B> w[R][ROWS];
  uint8_t ex[R][ROWS];
#pragma unroll
  for (int k = 0; k < R; k++) {
    uint32_t j = (uint32_t)(k * LPR + l);
    j = j < (uint32_t)nchunks ? j : (uint32_t)nchunks - 1;
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      w[k][i] = load_raw<B>(wrow[i] + j * (uint32_t)B);
      ex[k][i] = srow[i][j];
    }
  }
  // the epilogue's biases and router scores (a null bias reads score 0 instead, unused)
  const bool has_bias = P.bias != nullptr;
  TypedBits braw[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++)
    braw[i] = ld_typed_bits(has_bias ? P.bias : P.scores, has_bias ? P.bias_dtype : P.score_dtype,
                            has_bias ? e * P.bias_expert + ncl[i] : 0);
  TypedBits sraw[S];
#pragma unroll
  for (int t = 0; t < S; t++) sraw[t] = ld_typed_bits(P.scores, P.score_dtype, (int64_t)tok * S + t);
  __builtin_amdgcn_sched_barrier(0);
  uint4* xl = xs_pieces + s * xn;
#pragma unroll
  for (int k = 0; k < kDownSlotPieces; k++) {
    const int i = lane + 64 * k;
    if (i < xn) reinterpret_cast<piece_t*>(xl)[i] = xr[k];
  }
  // the wave reads only its own pieces: its LDS operations run in order
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  float acc[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) acc[i] = 0.0f;
  // every round is computed (a round past the last one adds +0): a round guarded by a
  // branch had its loads sunk into the branch
#pragma unroll
  for (int k = 0; k < R; k++) {
    const int j = k * LPR + l;
    const bool cv = j < nchunks;
    uint32_t xw[16];
    const uint4* xp = xl + (cv ? j : 0) * 4;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint4 v = xp[q];
      xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
    }
    float p[ROWS];
    chunk_dot_rows<F, XT, ROWS>(w[k], xw, p);
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      const float t = p[i] * pow2i((int)ex[k][i] - 127);
      acc[i] = acc[i] + ((cv && rv[i]) ? t : 0.0f);
    }
  }
  // each row's lane sum is the butterfly over the lane group's bits (the reduce-scatter
  // levels pair the same lanes), so ROWS does not change the bits
  reduce_range<ROWS, 1, LPR>(acc);
  if ((l >> log2c(ROWS)) == 0) {
    const int i = rs_row<ROWS>(l, log2c(ROWS), 0);
    float v = round_to<RT>(acc[0]);
    TypedBits bb = braw[0];
#pragma unroll
    for (int r = 1; r < ROWS; r++)
      if (i == r) bb = braw[r];
    if (has_bias) v = round_to<RT>(v + typed_f32(bb, P.bias_dtype));
    vals[s][i * SUBS + sub] = v;
  }
  __syncthreads();
  if (threadIdx.x < RB) {
    const int nn = row0 + (int)threadIdx.x;
    if (nn < P.rows) {
      float c = 0.0f;
#pragma unroll
      for (int t = 0; t < S; t++) c = __builtin_fmaf(vals[t][threadIdx.x], typed_f32(sraw[t], P.score_dtype), c);
      store<OT>(reinterpret_cast<OT*>(P.out) + (int64_t)tok * P.out_token + nn, c);
    }
  }
}

// ------------------------------------------------------------------ dispatch

// One row per lane group for one token (the grid is then resident at once); four for a
// batch of tokens, where each wave's staged activation then serves four times the rows
// (gpt-oss, eight tokens: bs=8 decode 2,087 -> 2,170 tok/s with two rows, 2,186 -> 2,205
// with four against two).
template <Fmt F, typename XT, typename OT, typename RT, int LPR, int S>
static int launch_down_slot(const DownParams& P, hipStream_t st) {
  constexpr int SUBS = 64 / LPR;
  if (P.tokens > 1) {
    hipLaunchKernelGGL((down_slot_kernel<F, XT, OT, RT, LPR, S, 4>),
                       dim3((unsigned)((P.rows + 4 * SUBS - 1) / (4 * SUBS)), P.tokens), dim3(64 * S),
                       (size_t)P.cols * 2 * S, st, P);
    return check_launch("mxfp_lowbit_weighted_down");
  }
  hipLaunchKernelGGL((down_slot_kernel<F, XT, OT, RT, LPR, S, 1>), dim3((unsigned)((P.rows + SUBS - 1) / SUBS), P.tokens),
                     dim3(64 * S), (size_t)P.cols * 2 * S, st, P);
  return check_launch("mxfp_lowbit_weighted_down");
}

template <Fmt F, typename XT, typename OT, typename RT, int LPR, int S>
static int launch_down_lean(const DownParams& P, hipStream_t st) {
  constexpr int SUBS = 64 / LPR;
  const int64_t waves = ((int64_t)P.rows + SUBS - 1) / SUBS;   // one row per lane group
  hipLaunchKernelGGL((down_lean_kernel<F, XT, OT, RT, LPR, 1, S>), dim3((unsigned)((waves + 3) / 4), P.tokens), dim3(256),
                     (size_t)P.cols * 2 * S, st, P);
  return check_launch("mxfp_lowbit_weighted_down");
}

template <Fmt F, typename XT, typename OT, typename RT, int LPR>
static int launch_down_lean_s(const DownParams& P, hipStream_t st) {
  if ((P.cols / 32 + LPR - 1) / LPR <= kDownSlotRounds && P.cols / 8 <= 64 * kDownSlotPieces) {
    switch (P.slots) {
      case 1: return launch_down_slot<F, XT, OT, RT, LPR, 1>(P, st);
      case 2: return launch_down_slot<F, XT, OT, RT, LPR, 2>(P, st);
      case 4: return launch_down_slot<F, XT, OT, RT, LPR, 4>(P, st);
      default: return launch_down_slot<F, XT, OT, RT, LPR, 8>(P, st);
    }
  }
  switch (P.slots) {
    case 1: return launch_down_lean<F, XT, OT, RT, LPR, 1>(P, st);
    case 2: return launch_down_lean<F, XT, OT, RT, LPR, 2>(P, st);
    case 4: return launch_down_lean<F, XT, OT, RT, LPR, 4>(P, st);
    default: return launch_down_lean<F, XT, OT, RT, LPR, 8>(P, st);
  }
}

template <Fmt F, typename XT, typename OT, typename RT>
static int launch_down(const DownParams& P, int lpr, hipStream_t st) {
  if ((P.slots == 1 || P.slots == 2 || P.slots == 4 || P.slots == 8) && P.cols % 8 == 0 &&
      (int64_t)P.cols * 2 * P.slots <= 65536 && P.x_slot % 8 == 0) {
    if (lpr == 64) return launch_down_lean_s<F, XT, OT, RT, 64>(P, st);
    if (lpr == 32) return launch_down_lean_s<F, XT, OT, RT, 32>(P, st);
    if (lpr == 16) return launch_down_lean_s<F, XT, OT, RT, 16>(P, st);
  }
  auto go = [&](auto kern, int rb) {
    const size_t lds = (size_t)P.cols * 2 * P.slots + (size_t)rb * 4 * P.slots;
    const int blocks = (P.rows + rb - 1) / rb;
    hipLaunchKernelGGL(kern, dim3(blocks, P.tokens), dim3(256), lds, st, P);
    return check_launch("mxfp_lowbit_weighted_down");
  };
  switch (lpr) {
    case 64: return go(weighted_down_kernel<F, XT, OT, RT, 64, 4>, 4);
    case 32: return go(weighted_down_kernel<F, XT, OT, RT, 32, 4>, 8);
    default: return go(weighted_down_kernel<F, XT, OT, RT, 16, 4>, 16);
  }
}

template <typename XT, typename RT>
static int down_dispatch(Fmt fmt, int out_dtype, const DownParams& P, int lpr, hipStream_t st) {
  return with_type(out_dtype, [&](auto ot) -> int {
    using OT = decltype(ot);
    if constexpr (std::is_same_v<OT, float> || std::is_same_v<OT, XT>) {
      switch (fmt) {
        case Fmt::kQ2E8: return launch_down<Fmt::kQ2E8, XT, OT, RT>(P, lpr, st);
        case Fmt::kQ1E8: return launch_down<Fmt::kQ1E8, XT, OT, RT>(P, lpr, st);
        default: return launch_down<Fmt::kMxfp4, XT, OT, RT>(P, lpr, st);
      }
    } else {
      set_error("weighted_down: output dtype must match the activation dtype or be fp32");
      return TT_ERR_UNSUPPORTED;
    }
  });
}

}  // namespace tt

using namespace tt;

static int weighted_down_impl(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                            const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                            const void* x, int x_dtype, int64_t x_slot,
                                            const void* expert_indices, int index_bytes, const void* router_scores,
                                            int score_dtype, int64_t selected, const void* bias, int bias_dtype,
                                            int64_t bias_expert, void* out, int out_dtype, int64_t rows,
                                            int64_t cols, int64_t tokens, int64_t out_token, void* stream) {
  const char* what = "mxfp_lowbit_weighted_down";
  TT_REQUIRE(tokens >= 1 && tokens <= 65535, "%s: bad token count", what);
  TT_REQUIRE(bits == 1 || bits == 2 || bits == 4, "%s: fused down requires packed Q1, Q2 or MXFP4 experts", what);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(cols > 0 && cols % 32 == 0, "%s: cols must be a multiple of 32", what);
  TT_REQUIRE(selected >= 1 && selected * (2 * cols + 64) <= 65536,
             "%s: selected activations and row values must fit 64 KiB of LDS", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  const int align = bits == 4 ? 16 : (bits == 2 ? 8 : 4);
  TT_REQUIRE(packed && aligned(packed, align) && w_row_bytes % align == 0 && w_expert_bytes % align == 0,
             "%s: packed weights must be %d-byte aligned", what, align);
  TT_REQUIRE(scales && x && aligned(x, 4) && x_slot % 2 == 0 && out && expert_indices && router_scores,
             "%s: null or misaligned pointer", what);
  TT_REQUIRE(valid_out_dtype(score_dtype), "%s: bad score dtype", what);
  int ishift;
  TT_REQUIRE(index_shift(index_bytes, &ishift), "%s: expert indices must be int32 or int64", what);
  if (bias) TT_REQUIRE(valid_out_dtype(bias_dtype), "%s: bad bias dtype", what);
  DownParams P{static_cast<const uint8_t*>(packed), w_expert_bytes, w_row_bytes,
               static_cast<const uint8_t*>(scales), s_expert, s_row, x, x_slot, expert_indices, ishift, router_scores, bias,
               bias_expert, out, (int)rows, (int)cols, (int)selected, bias ? bias_dtype : TT_F32, score_dtype, out_token,
               (int)tokens};
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const Fmt fmt = fmt_for_bits(bits);
  if (x_dtype == TT_F16) {
    if (bits == 4) return down_dispatch<f16_t, f16_t>(fmt, out_dtype, P, lpr, st);
    return down_dispatch<f16_t, bf16_t>(fmt, out_dtype, P, lpr, st);
  }
  return down_dispatch<bf16_t, bf16_t>(fmt, out_dtype, P, lpr, st);
}

extern "C" int tt_mxfp_lowbit_weighted_down(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                            const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                            const void* x, int x_dtype, int64_t x_slot,
                                            const void* expert_indices, int index_bytes, const void* router_scores,
                                            int score_dtype, int64_t selected, const void* bias, int bias_dtype,
                                            int64_t bias_expert, void* out, int out_dtype, int64_t rows,
                                            int64_t cols, void* stream) {
  return weighted_down_impl(packed, w_expert_bytes, w_row_bytes, scales, s_expert, s_row, bits, x, x_dtype, x_slot,
                            expert_indices, index_bytes, router_scores, score_dtype, selected, bias, bias_dtype, bias_expert, out,
                            out_dtype, rows, cols, 1, 0, stream);
}

extern "C" int tt_mxfp_lowbit_weighted_down_tokens(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                                   const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                                   const void* x, int x_dtype, int64_t x_slot,
                                                   const void* expert_indices, int index_bytes, const void* router_scores,
                                                   int score_dtype, int64_t selected, const void* bias, int bias_dtype,
                                                   int64_t bias_expert, void* out, int out_dtype, int64_t out_token,
                                                   int64_t rows, int64_t cols, int64_t tokens, void* stream) {
  return weighted_down_impl(packed, w_expert_bytes, w_row_bytes, scales, s_expert, s_row, bits, x, x_dtype, x_slot,
                            expert_indices, index_bytes, router_scores, score_dtype, selected, bias, bias_dtype, bias_expert, out,
                            out_dtype, rows, cols, tokens, out_token, stream);
}
