// Fused MoE gate/up kernels: gate/up GEMV + gpt-oss SwiGLU on interleaved rows of the
// selected experts (E8M0 block-scaled q1, q2, MXFP4); expert ids are read on the device.
#include "moe_common.h"

namespace tt {

// gate/up rows 2a and 2a+1 of the selected expert; APW activation rows per wave pass.
template <Fmt F, typename XT, typename OT, typename RT, typename BT, int LPR, int APW>
__global__ __launch_bounds__(256) void swiglu_kernel(SwigluParams P) {
  extern __shared__ uint32_t xs_lds[];
  constexpr int SUBS = 64 / LPR;
  const int slot = blockIdx.y;
  const int64_t e = load_expert(P.experts, P.ishift, slot);
  const uint8_t* wexp = P.w + e * P.w_expert;
  const uint8_t* sexp = P.s + e * P.s_expert;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, l = lane % LPR;
  const int nchunks = P.cols >> 5;
  const int per_iter = APW * SUBS;
  const int waves_total = gridDim.x * (blockDim.x >> 6);
  bool staged = false;
  for (int base = (blockIdx.x * (blockDim.x >> 6) + wave) * per_iter;; base += waves_total * per_iter) {
    const bool active = base < P.act_rows;
    const uint8_t* wrow[2 * APW];
    const uint8_t* srow[2 * APW];
    bool rv[2 * APW];
    int act[APW];
#pragma unroll
    for (int i = 0; i < APW; i++) {
      act[i] = base + i * SUBS + sub;
      const bool v = act[i] < P.act_rows;
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int64_t row = 2 * (int64_t)act[i] + h;
        rv[2 * i + h] = v;
        wrow[2 * i + h] = wexp + row * P.w_row;
        srow[2 * i + h] = sexp + row * P.s_row;
      }
    }
    E8Round<F, 2 * APW> cur;
    if (active) e8_fetch<F, LPR, 2 * APW>(cur, 0, l, nchunks, wrow, srow, rv);
    if (!staged) {
      const uint32_t* xg = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(P.x) + (int64_t)(slot / P.x_div) * P.x_slot);
      for (int i = threadIdx.x; i < (P.cols >> 1); i += blockDim.x) xs_lds[i] = xg[i];
      __syncthreads();
      staged = true;
    }
    if (!active) break;
    float dot[2 * APW];
    e8_rows_dot<F, XT, LPR, 2 * APW>(cur, wrow, srow, rv, xs_lds, nchunks, l, dot);
#pragma unroll
    for (int i = 0; i < APW; i++) {
      if (!rv[2 * i] || l != i) continue;
      float g = round_to<RT>(dot[2 * i]);
      float u = round_to<RT>(dot[2 * i + 1]);
      if (P.bias != nullptr) {
        const int64_t bb = e * P.bias_expert + 2 * (int64_t)act[i];
        g = round_to<RT>(g + ld_bias<BT>(P.bias, bb));
        u = round_to<RT>(u + ld_bias<BT>(P.bias, bb + 1));
      }
      g = fminf(g, P.limit);
      u = fmaxf(fminf(u, P.limit), -P.limit);
      const float num = (u + 1.0f) * g;
      const float den = 1.0f + exp_f32(-g * P.alpha);
      store<OT>(reinterpret_cast<OT*>(P.out) + (int64_t)slot * P.out_slot + act[i], num / den);
    }
  }
}

// ------------------------------------------------------------------ lean variants
// Same arithmetic as swiglu_kernel / weighted_down_kernel, laid out like the lean GEMV
// (gemv_lean.h): one batch per wave, every load of a round issued before its first
// use, the next round in flight while one is consumed, and the cross-row work done in
// registers after one reduce-scatter.

// SwiGLU: a lane group's batch is APL activation rows, i.e. 2 * APL weight rows with
// gate row 2a and up row 2a + 1 adjacent, so after the reduction the gate value and its
// up partner sit on lanes that one cross-lane move connects.
template <Fmt F, typename XT, typename OT, typename RT, typename BT, int LPR, int ROWS>
__global__ __launch_bounds__(256) void swiglu_lean_kernel(const SwigluParams P) {
  static_assert(ROWS >= 2 && ROWS % 2 == 0, "gate/up pairs");
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr int SUBS = 64 / LPR;
  constexpr int APL = ROWS / 2;
  extern __shared__ uint32_t xs_lds[];
  const int slot = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int sub = lane / LPR, l = lane % LPR;
  const int nchunks = P.cols >> 5;
  const int rounds = (nchunks + LPR - 1) / LPR;
  const int a0 = (int)(blockIdx.x * 4 + wave) * (APL * SUBS);
  // the slot's activations go to LDS (loads first, clamped indices)
  const int xn = P.cols >> 3;
  const uint4* xg = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(P.x) + (int64_t)(slot / P.x_div) * P.x_slot);
  uint4 xreg[4];
  int xidx[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int idx = threadIdx.x + 256 * k;
    xidx[k] = idx < xn ? idx : xn - 1;
    xreg[k] = xg[xidx[k]];
  }
  const int64_t e = load_expert(P.experts, P.ishift, slot);
  const uint8_t* wexp = P.w + e * P.w_expert;
  const uint8_t* sexp = P.s + e * P.s_expert;
  const uint8_t* wrow[ROWS];
  const uint8_t* srow[ROWS];
  bool rv[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) {
    const int a = a0 + (i >> 1) * SUBS + sub;
    rv[i] = a < P.act_rows;
    const int64_t row = 2 * (int64_t)(rv[i] ? a : P.act_rows - 1) + (i & 1);
    wrow[i] = wexp + row * P.w_row;
    srow[i] = sexp + row * P.s_row;
  }
  struct Round {
    Raw<B> w[ROWS];
    uint8_t ex[ROWS];
  };
  auto fetch = [&](int r, Round& d) {
    uint32_t j = (uint32_t)(r * LPR + l);
    j = j < (uint32_t)nchunks ? j : (uint32_t)nchunks - 1;
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      d.w[i] = load_raw<B>(wrow[i] + j * (uint32_t)B);
      d.ex[i] = srow[i][j];
    }
  };
  // R rounds in flight at once (rounds past the last re-read its chunk; unused): the
  // grid is small, so latency is hidden inside each wave
  constexpr int R = 16 / ROWS > 4 ? 4 : 16 / ROWS;
  Round d[R];
#pragma unroll
  for (int k = 0; k < R; k++) fetch(k, d[k]);
  uint4* xl = reinterpret_cast<uint4*>(xs_lds);
#pragma unroll
  for (int k = 0; k < 4; k++) xl[xidx[k]] = xreg[k];
  for (int idx = threadIdx.x + 1024; idx < xn; idx += 256) xl[idx] = xg[idx];
  lds_barrier();

  float acc[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) acc[i] = 0.0f;
  auto consume = [&](const Round& c, int r) {
    const int j = r * LPR + l;
    const bool cv = j < nchunks;
    uint32_t xw[16];
    const uint4* xp = reinterpret_cast<const uint4*>(xs_lds + (cv ? j : 0) * 16);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint4 v = xp[q];
      xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
    }
    float p[ROWS];
    chunk_dot_rows<F, XT, ROWS>(c.w, xw, p);
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      const float t = p[i] * pow2i((int)c.ex[i] - 127);
      acc[i] = acc[i] + ((cv && rv[i]) ? t : 0.0f);
    }
  };
  for (int r0 = 0;;) {   // cols >= 32: at least one round
#pragma unroll
    for (int k = 0; k < R; k++)
      if (r0 + k < rounds) consume(d[k], r0 + k);
    r0 += R;
    if (r0 >= rounds) break;
#pragma unroll
    for (int k = 0; k < R; k++) fetch(r0 + k, d[k]);
  }
  reduce_range<ROWS, 1, LPR>(acc);
  const float v = acc[0];
  const float pv = xor_partner<ROWS / 2>(v);   // the other row of the gate/up pair
  const int br = rs_row<ROWS>(l, log2c(ROWS), 0);
  if ((l >> log2c(ROWS)) != 0 || (br & 1) != 0) return;
  const int a = a0 + (br >> 1) * SUBS + sub;
  if (a >= P.act_rows) return;
  float g = round_to<RT>(v);
  float u = round_to<RT>(pv);
  if (P.bias != nullptr) {
    const int64_t bb = e * P.bias_expert + 2 * (int64_t)a;
    g = round_to<RT>(g + ld_bias<BT>(P.bias, bb));
    u = round_to<RT>(u + ld_bias<BT>(P.bias, bb + 1));
  }
  g = fminf(g, P.limit);
  u = fmaxf(fminf(u, P.limit), -P.limit);
  const float num = (u + 1.0f) * g;
  const float den = 1.0f + exp_f32(-g * P.alpha);
  store<OT>(reinterpret_cast<OT*>(P.out) + (int64_t)slot * P.out_slot + a, num / den);
}

// swiglu_lean_kernel with KB consecutive row blocks per workgroup (ROWS = 2, rows of at
// most three rounds): the slot's activations are staged once, and block k + 1's weight
// rounds are in flight while block k computes, so a workgroup waits for memory once per
// launch rather than once per block and the grid has KB times fewer workgroups.  Each
// row's arithmetic is swiglu_lean_kernel's (same chunk partition, fma order, reduction
// and epilogue), so the bits are the same.
template <Fmt F, typename XT, typename OT, typename RT, typename BT, int LPR, int KB>
__global__ __launch_bounds__(256) void swiglu_lean_multi_kernel(const SwigluParams P, int nblocks) {
  constexpr int ROWS = 2;
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr int SUBS = 64 / LPR;
  constexpr int R = 3;   // rounds per row (the host checks)
  extern __shared__ uint32_t xs_lds[];
  const int slot = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int sub = lane / LPR, l = lane % LPR;
  const int nchunks = P.cols >> 5;
  const int rounds = (nchunks + LPR - 1) / LPR;
  const int xn = P.cols >> 3;
  // (native 4-vectors: an array of the uint4 struct type is kept in scratch memory)
  typedef uint32_t piece_t __attribute__((ext_vector_type(4)));
  const piece_t* xg = reinterpret_cast<const piece_t*>(reinterpret_cast<const uint16_t*>(P.x) + (int64_t)(slot / P.x_div) * P.x_slot);
  piece_t xreg[4];
  int xidx[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int idx = threadIdx.x + 256 * k;
    xidx[k] = idx < xn ? idx : xn - 1;
    xreg[k] = xg[xidx[k]];
  }
  const SlotRoute route = swiglu_slot_route(P, slot);
  const int64_t e = route.e;
  const uint8_t* wexp = P.w + e * P.w_expert;
  const uint8_t* sexp = P.s + e * P.s_expert;
  struct Round {
    Raw<B> w[ROWS];
    uint8_t ex[ROWS];
  };
  // activation row of block kb for this lane, clamped, and the block's rows
  auto block_row = [&](int kb) -> int {
    const int bx = (int)blockIdx.x * KB + kb;
    return (bx * 4 + wave) * SUBS + sub;
  };
  auto fetch_block = [&](int kb, Round* d) {
    const int a = block_row(kb);
    const int ac = a < P.act_rows ? a : P.act_rows - 1;
    const uint8_t* w0 = wexp + 2 * (int64_t)ac * P.w_row;
    const uint8_t* s0 = sexp + 2 * (int64_t)ac * P.s_row;
#pragma unroll
    for (int r = 0; r < R; r++) {
      uint32_t j = (uint32_t)(r * LPR + l);
      j = j < (uint32_t)nchunks ? j : (uint32_t)nchunks - 1;
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        d[r].w[i] = load_raw<B>(w0 + i * P.w_row + j * (uint32_t)B);
        d[r].ex[i] = s0[i * P.s_row + j];
      }
    }
  };
  Round d[2][R];
  fetch_block(0, d[0]);
  if (blockIdx.x == 0 && wave == 0) swiglu_publish(P, slot, route.lg0, route.lg1);
  piece_t* xl = reinterpret_cast<piece_t*>(xs_lds);
#pragma unroll
  for (int k = 0; k < 4; k++) xl[xidx[k]] = xreg[k];
  for (int idx = threadIdx.x + 1024; idx < xn; idx += 256) xl[idx] = xg[idx];
  lds_barrier();

  // every block's fetch and every round's arithmetic is unconditional (a block past the
  // last reads clamped rows and stores nothing, a round past the last adds +0): a fetch
  // or round under a branch had its loads sunk to their use
  (void)nblocks;
#pragma unroll
  for (int kb = 0; kb < KB; kb++) {
    if (kb + 1 < KB) fetch_block(kb + 1, d[(kb + 1) & 1]);
    const Round* c = d[kb & 1];
    const int a = block_row(kb);
    const bool av = a < P.act_rows;
    float acc[ROWS];
#pragma unroll
    for (int i = 0; i < ROWS; i++) acc[i] = 0.0f;
#pragma unroll
    for (int r = 0; r < R; r++) {
      {
        const int j = r * LPR + l;
        const bool cv = j < nchunks;
        uint32_t xw[16];
        const uint4* xp = reinterpret_cast<const uint4*>(xs_lds + (cv ? j : 0) * 16);
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const uint4 v = xp[q];
          xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
        }
        float p[ROWS];
        chunk_dot_rows<F, XT, ROWS>(c[r].w, xw, p);
#pragma unroll
        for (int i = 0; i < ROWS; i++) {
          const float t = p[i] * pow2i((int)c[r].ex[i] - 127);
          acc[i] = acc[i] + ((cv && av) ? t : 0.0f);
        }
      }
    }
    reduce_range<ROWS, 1, LPR>(acc);
    const float v = acc[0];
    const float pv = xor_partner<ROWS / 2>(v);   // the other row of the gate/up pair
    const int br = rs_row<ROWS>(l, log2c(ROWS), 0);
    if ((l >> log2c(ROWS)) == 0 && (br & 1) == 0 && av) {
      float g = round_to<RT>(v);
      float u = round_to<RT>(pv);
      if (P.bias != nullptr) {
        const int64_t bb = e * P.bias_expert + 2 * (int64_t)a;
        g = round_to<RT>(g + ld_bias<BT>(P.bias, bb));
        u = round_to<RT>(u + ld_bias<BT>(P.bias, bb + 1));
      }
      g = fminf(g, P.limit);
      u = fmaxf(fminf(u, P.limit), -P.limit);
      const float num = (u + 1.0f) * g;
      const float den = 1.0f + exp_f32(-g * P.alpha);
      store<OT>(reinterpret_cast<OT*>(P.out) + (int64_t)slot * P.out_slot + a, num / den);
    }
  }
}

constexpr int kSwigluSlotRounds = 4;   // rounds of a row per lane group (all in flight)
constexpr int kSwigluSlotPieces = 4;   // 16-byte activation pieces per thread (cols <= 8192)

// swiglu_lean_kernel (ROWS = 2) for rows of at most kSwigluSlotRounds rounds, with no
// refill loop: the slot's activation pieces, then every round of the wave's gate/up
// rows and their biases are requested before the first wait, and every round is
// computed (a round past the last adds +0), so no load is sunk into a branch and the
// wave needs few registers: at the gpt-oss shape the whole grid is resident at once.
// Same chunk partition, fma order, reduction and epilogue as swiglu_lean_kernel.
template <Fmt F, typename XT, typename OT, typename RT, typename BT, int LPR>
__global__ __launch_bounds__(256) void swiglu_slot_kernel(const SwigluParams P) {
  constexpr int ROWS = 2;
  constexpr int B = FmtInfo<F>::kBytes;
  constexpr int SUBS = 64 / LPR;
  constexpr int R = kSwigluSlotRounds;
  extern __shared__ uint32_t xs_lds[];
  const int slot = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int sub = lane / LPR, l = lane % LPR;
  const int nchunks = P.cols >> 5;
  const int a = (int)(blockIdx.x * 4 + wave) * SUBS + sub;   // this lane group's activation row
  const bool av = a < P.act_rows;
  const int ac = av ? a : P.act_rows - 1;
  // the slot's activations go to LDS (loads first, clamped indices; native 4-vectors:
  // an array of the uint4 struct type is kept in scratch memory)
  typedef uint32_t piece_t __attribute__((ext_vector_type(4)));
  const int xn = P.cols >> 3;
  const piece_t* xg = reinterpret_cast<const piece_t*>(reinterpret_cast<const uint16_t*>(P.x) +
                                                       (int64_t)(slot / P.x_div) * P.x_slot);
  piece_t xr[kSwigluSlotPieces];
#pragma unroll
  for (int k = 0; k < kSwigluSlotPieces; k++) {
    const int i = (int)threadIdx.x + 256 * k;
    xr[k] = xg[i < xn ? i : xn - 1];
  }
  const SlotRoute route = swiglu_slot_route(P, slot);
  const int64_t e = route.e;
  const uint8_t* w0 = P.w + e * P.w_expert + 2 * (int64_t)ac * P.w_row;
  const uint8_t* s0 = P.s + e * P.s_expert + 2 * (int64_t)ac * P.s_row;
  Raw<B> w[R][ROWS];
  uint8_t ex[R][ROWS];
#pragma unroll
  for (int k = 0; k < R; k++) {
    uint32_t j = (uint32_t)(k * LPR + l);
    j = j < (uint32_t)nchunks ? j : (uint32_t)nchunks - 1;
#pragma unroll
    for (int i = 0; i < ROWS; i++) {
      w[k][i] = load_raw<B>(w0 + i * P.w_row + j * (uint32_t)B);
      ex[k][i] = s0[i * P.s_row + j];
    }
  }
  // gate and up biases (a null bias reads the activation instead, unused)
  const bool has_bias = P.bias != nullptr;
  const int64_t bb = has_bias ? e * P.bias_expert + 2 * (int64_t)ac : 0;
  const BT* bp = reinterpret_cast<const BT*>(has_bias ? P.bias : P.x);
  const BT bg = bp[bb], bu = bp[has_bias ? bb + 1 : bb];
  __builtin_amdgcn_sched_barrier(0);
  if (blockIdx.x == 0 && wave == 0) swiglu_publish(P, slot, route.lg0, route.lg1);
  piece_t* xl = reinterpret_cast<piece_t*>(xs_lds);
#pragma unroll
  for (int k = 0; k < kSwigluSlotPieces; k++) {
    const int i = (int)threadIdx.x + 256 * k;
    if (i < xn) xl[i] = xr[k];
  }
  lds_barrier();

  float acc[ROWS] = {0.0f, 0.0f};
#pragma unroll
  for (int k = 0; k < R; k++) {
    const int j = k * LPR + l;
    const bool cv = j < nchunks;
    uint32_t xw[16];
    const uint4* xp = reinterpret_cast<const uint4*>(xs_lds + (cv ? j : 0) * 16);
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
      acc[i] = acc[i] + ((cv && av) ? t : 0.0f);
    }
  }
  reduce_range<ROWS, 1, LPR>(acc);
  const float v = acc[0];
  const float pv = xor_partner<1>(v);   // the other row of the gate/up pair
  if (l != 0 || !av) return;
  float g = round_to<RT>(v);
  float u = round_to<RT>(pv);
  if (has_bias) {
    g = round_to<RT>(g + to_f32(bg));
    u = round_to<RT>(u + to_f32(bu));
  }
  g = fminf(g, P.limit);
  u = fmaxf(fminf(u, P.limit), -P.limit);
  const float num = (u + 1.0f) * g;
  const float den = 1.0f + exp_f32(-g * P.alpha);
  store<OT>(reinterpret_cast<OT*>(P.out) + (int64_t)slot * P.out_slot + a, num / den);
}

// ------------------------------------------------------------------ dispatch

// Row blocks per workgroup of swiglu_lean_multi_kernel: 2 once the one-block grid would
// be several generations of workgroups deep, 1 (swiglu_lean_kernel) otherwise.
constexpr int kSwigluMultiBlocks = 2;
constexpr int64_t kSwigluMultiMinWorkgroups = 4096;

template <Fmt F, typename XT, typename OT, typename RT, typename BT, int LPR>
static int launch_swiglu_lean(const SwigluParams& P, int slots, hipStream_t st) {
  constexpr int SUBS = 64 / LPR;
  const int per_wave = SUBS;   // one activation row (two weight rows) per lane group
  const int64_t waves = ((int64_t)P.act_rows + per_wave - 1) / per_wave;
  const int64_t nblocks = (waves + 3) / 4;
  const int rounds = (P.cols / 32 + LPR - 1) / LPR;
  if (rounds <= 3 && nblocks * slots >= kSwigluMultiMinWorkgroups) {
    constexpr int KB = kSwigluMultiBlocks;
    // a multiple of 8 workgroups per slot, so that the workgroups of one row block for
    // every slot sit on the same XCD (slots sharing an expert share its L2 lines)
    const int64_t groups = ((nblocks + KB - 1) / KB + 7) / 8 * 8;
    hipLaunchKernelGGL((swiglu_lean_multi_kernel<F, XT, OT, RT, BT, LPR, KB>), dim3((unsigned)groups, slots), dim3(256),
                       (size_t)P.cols * 2, st, P, (int)nblocks);
    return check_launch("mxfp_lowbit_selected_swiglu");
  }
  if (rounds <= kSwigluSlotRounds && P.cols / 8 <= 256 * kSwigluSlotPieces) {
    hipLaunchKernelGGL((swiglu_slot_kernel<F, XT, OT, RT, BT, LPR>), dim3((unsigned)((waves + 3) / 4), slots),
                       dim3(256), (size_t)P.cols * 2, st, P);
    return check_launch("mxfp_lowbit_selected_swiglu");
  }
  hipLaunchKernelGGL((swiglu_lean_kernel<F, XT, OT, RT, BT, LPR, 2>), dim3((unsigned)((waves + 3) / 4), slots),
                     dim3(256), (size_t)P.cols * 2, st, P);
  return check_launch("mxfp_lowbit_selected_swiglu");
}

template <Fmt F, typename XT, typename OT, typename RT, typename BT>
static int launch_swiglu(const SwigluParams& P, int lpr, int slots, hipStream_t st) {
  if (P.cols <= 8192) {
    if (lpr == 64) return launch_swiglu_lean<F, XT, OT, RT, BT, 64>(P, slots, st);
    if (lpr == 32) return launch_swiglu_lean<F, XT, OT, RT, BT, 32>(P, slots, st);
    if (lpr == 16) return launch_swiglu_lean<F, XT, OT, RT, BT, 16>(P, slots, st);
  }
  const size_t lds = (size_t)P.cols * 2;
  auto go = [&](auto kern, int subs) {
    constexpr int APW = 2;
    const int per_block = 4 * APW * subs;
    const int blocks = (P.act_rows + per_block - 1) / per_block;
    hipLaunchKernelGGL(kern, dim3(blocks, slots), dim3(256), lds, st, P);
    return check_launch("mxfp_lowbit_selected_swiglu");
  };
  switch (lpr) {
    case 64: return go(swiglu_kernel<F, XT, OT, RT, BT, 64, 2>, 1);
    case 32: return go(swiglu_kernel<F, XT, OT, RT, BT, 32, 2>, 2);
    default: return go(swiglu_kernel<F, XT, OT, RT, BT, 16, 2>, 4);
  }
}

template <typename XT, typename RT>
static int swiglu_dispatch(Fmt fmt, int out_dtype, int bias_dtype, const SwigluParams& P, int lpr, int slots, hipStream_t st) {
  return with_type(out_dtype, [&](auto ot) -> int {
    using OT = decltype(ot);
    if constexpr (std::is_same_v<OT, float> || std::is_same_v<OT, XT>) {
      return with_type(bias_dtype, [&](auto bt) -> int {
        using BT = decltype(bt);
        switch (fmt) {
          case Fmt::kQ2E8: return launch_swiglu<Fmt::kQ2E8, XT, OT, RT, BT>(P, lpr, slots, st);
          case Fmt::kQ1E8: return launch_swiglu<Fmt::kQ1E8, XT, OT, RT, BT>(P, lpr, slots, st);
          default: return launch_swiglu<Fmt::kMxfp4, XT, OT, RT, BT>(P, lpr, slots, st);
        }
      });
    } else {
      set_error("swiglu: output dtype must match the activation dtype or be fp32");
      return TT_ERR_UNSUPPORTED;
    }
  });
}

}  // namespace tt

using namespace tt;

// Router-logits mode (logits != nullptr): slot s is token s / selected's (s % selected)-th
// choice of the top-k over its n_exp logits, computed in the kernel; the slots' experts
// and scores go to idx_out / score_out.
struct SwigluRouter {
  const float* logits;
  int64_t n_exp;
  int renorm;
  int32_t* idx_out;
  void* score_out;
  int score_dtype;
};

static int selected_swiglu_impl(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                              const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                              const void* x, int x_dtype, int64_t x_slot,
                                              const void* expert_indices, int index_bytes, int64_t selected, const void* bias,
                                              int bias_dtype, int64_t bias_expert, float alpha, float limit,
                                              void* out, int out_dtype, int64_t out_slot, int64_t activation_rows,
                                              int64_t cols, int64_t tokens, void* stream,
                                              const SwigluRouter* router = nullptr) {
  const char* what = router ? "mxfp_lowbit_selected_swiglu_router" : "mxfp_lowbit_selected_swiglu";
  TT_REQUIRE(tokens >= 1 && tokens * selected <= 65535, "%s: bad token count", what);
  TT_REQUIRE(bits == 1 || bits == 2 || bits == 4, "%s: fused SwiGLU requires packed Q1, Q2 or MXFP4 experts", what);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(cols > 0 && cols % 32 == 0 && cols <= 32768, "%s: cols must be a multiple of 32 up to 32768", what);
  TT_REQUIRE(activation_rows > 0 && activation_rows < (1 << 29), "%s: bad activation rows", what);
  int ishift = 0;
  if (router) {
    TT_REQUIRE(router->logits && router->idx_out && router->score_out && aligned(router->logits, 4),
               "%s: null or misaligned router buffers", what);
    TT_REQUIRE(router->n_exp >= 1 && router->n_exp <= 128 && selected >= 1 && selected <= router->n_exp,
               "%s: need 1..128 experts and 1..experts selected", what);
    TT_REQUIRE(valid_out_dtype(router->score_dtype), "%s: bad score dtype", what);
    const int lpr0 = tt_gemv_lanes_per_row(cols / 32, 1);
    TT_UNSUPPORTED(cols <= 8192 && (cols / 32 + lpr0 - 1) / lpr0 <= kSwigluSlotRounds,
                   "%s: rows of at most %d rounds and 8192 columns", what, kSwigluSlotRounds);
  } else {
    TT_REQUIRE(selected >= 1 && selected <= 65535 && expert_indices, "%s: need selected experts", what);
    TT_REQUIRE(index_shift(index_bytes, &ishift), "%s: expert indices must be int32 or int64", what);
  }
  const int align = bits == 4 ? 16 : (bits == 2 ? 8 : 4);
  TT_REQUIRE(packed && aligned(packed, align) && w_row_bytes % align == 0 && w_expert_bytes % align == 0,
             "%s: packed weights must be %d-byte aligned", what, align);
  TT_REQUIRE(scales && x && aligned(x, 4) && x_slot % 2 == 0 && out, "%s: null or misaligned pointer", what);
  if (bias) TT_REQUIRE(valid_out_dtype(bias_dtype), "%s: bad bias dtype", what);
  SwigluParams P{static_cast<const uint8_t*>(packed), w_expert_bytes, w_row_bytes,
                 static_cast<const uint8_t*>(scales), s_expert, s_row, x, x_slot, expert_indices, ishift, bias, bias_expert,
                 alpha, limit, out, out_slot, (int)activation_rows, (int)cols, tokens > 1 ? (int)selected : 1};
  if (router) {
    P.x_div = (int)selected;   // slot s reads token s / selected's activation
    P.logits = router->logits;
    P.n_exp = (int)router->n_exp;
    P.top_k = (int)selected;
    P.renorm = router->renorm;
    P.score_dtype = router->score_dtype;
    P.idx_out = router->idx_out;
    P.score_out = router->score_out;
  }
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const Fmt fmt = fmt_for_bits(bits);
  const int bdt = bias ? bias_dtype : TT_F32;
  if (x_dtype == TT_F16) {
    if (bits == 4) return swiglu_dispatch<f16_t, f16_t>(fmt, out_dtype, bdt, P, lpr, (int)(tokens * selected), st);
    return swiglu_dispatch<f16_t, bf16_t>(fmt, out_dtype, bdt, P, lpr, (int)(tokens * selected), st);
  }
  return swiglu_dispatch<bf16_t, bf16_t>(fmt, out_dtype, bdt, P, lpr, (int)(tokens * selected), st);
}

// bits: 1 or 2 (E8M0 q1/q2, bf16 rounding), 4 (MXFP4, rounding in the activation dtype).
extern "C" int tt_mxfp_lowbit_selected_swiglu(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                              const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                              const void* x, int x_dtype, int64_t x_slot,
                                              const void* expert_indices, int index_bytes, int64_t selected, const void* bias,
                                              int bias_dtype, int64_t bias_expert, float alpha, float limit,
                                              void* out, int out_dtype, int64_t out_slot, int64_t activation_rows,
                                              int64_t cols, void* stream) {
  return selected_swiglu_impl(packed, w_expert_bytes, w_row_bytes, scales, s_expert, s_row, bits, x, x_dtype, x_slot,
                              expert_indices, index_bytes, selected, bias, bias_dtype, bias_expert, alpha, limit, out, out_dtype,
                              out_slot, activation_rows, cols, 1, stream);
}

extern "C" int tt_mxfp_lowbit_selected_swiglu_tokens(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                                     const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                                     const void* x, int x_dtype, int64_t x_token,
                                                     const void* expert_indices, int index_bytes, int64_t selected,
                                                     const void* bias, int bias_dtype, int64_t bias_expert,
                                                     float alpha, float limit, void* out, int out_dtype,
                                                     int64_t out_slot, int64_t activation_rows, int64_t cols,
                                                     int64_t tokens, void* stream) {
  return selected_swiglu_impl(packed, w_expert_bytes, w_row_bytes, scales, s_expert, s_row, bits, x, x_dtype, x_token,
                              expert_indices, index_bytes, selected, bias, bias_dtype, bias_expert, alpha, limit, out, out_dtype,
                              out_slot, activation_rows, cols, tokens, stream);
}

// The decode step's SwiGLU with the router's top-k folded in: router_logits [tokens,
// experts] as tt_add_rms_norm_router_logits writes them; every wave runs the top-k +
// softmax of its token (the selection and scores of tt_moe_router_topk, bit for bit) and
// takes its slot's expert; the slots' experts and scores (renormalized over the selected
// experts or not) go to indices_out / scores_out [tokens, selected] for the weighted-down.
// Rows of at most four rounds of lanes and 8192 columns.
extern "C" int tt_mxfp_lowbit_selected_swiglu_router(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                                     const void* scales, int64_t s_expert, int64_t s_row, int bits,
                                                     const void* x, int x_dtype, int64_t x_token,
                                                     const float* router_logits, int64_t experts, int64_t selected,
                                                     int renormalize, int32_t* indices_out, void* scores_out,
                                                     int score_dtype, const void* bias, int bias_dtype,
                                                     int64_t bias_expert, float alpha, float limit, void* out,
                                                     int out_dtype, int64_t out_slot, int64_t activation_rows,
                                                     int64_t cols, int64_t tokens, void* stream) {
  const SwigluRouter R{router_logits, experts, renormalize, indices_out, scores_out, score_dtype};
  return selected_swiglu_impl(packed, w_expert_bytes, w_row_bytes, scales, s_expert, s_row, bits, x, x_dtype, x_token,
                              nullptr, 4, selected, bias, bias_dtype, bias_expert, alpha, limit, out, out_dtype, out_slot,
                              activation_rows, cols, tokens, stream, &R);
}
