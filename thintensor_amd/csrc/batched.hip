// Batched small-M dequant GEMM: y[m] = W x[m] for M activation rows.
//
//   * M below the MFMA threshold (int4: 4, fp8: 16): the GEMV engine with up to four
//     activation rows per wave (every weight word decoded once, one fma chain per
//     activation row), so row m equals the single-row GEMV bit for bit (one int4 row
//     goes to the single-row kernel itself);
//   * from the threshold (int4 M >= 4, where the engine's per-row fma chains make it
//     VALU-bound; fp8 M >= 16): MFMA (mfma_ksplit_kernel below): one workgroup per CU
//     owns a block of weight rows for all M (<= 64) activation rows, its four waves
//     split K, each reads its weight and activation fragments straight into MFMA
//     operand registers, and the waves' fp32 tiles are summed in a fixed order at the
//     end.  MFMA sums products in a hardware-defined order, so this path matches the
//     dequantise-then-matmul reference to the stated tolerance, not bit for bit.
//   * the M-row lm_head argmax runs the GEMV engine with eight activation rows per
//     launch and one argmax key per (wave, row); a finishing kernel picks each row's
//     token, as tt_matvec_argmax does for one row;
//   * the M-row dense GEMV + bias of a batched decode step (tt_matvec_bias_rows, fp16)
//     runs the same engine with eight rows per launch: each weight load feeds every
//     row's fma chain, the bits per row those of the single-row operator.
#include "gemv_impl.h"

#include <type_traits>

using namespace tt;

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

enum class WFmt : int { kInt4G128 = 0, kFp8Row = 1 };

// Bytes of one weight row a lane reads per pipeline step and steps in flight per wave
// of mfma_ksplit_kernel (measured on the MI355X: 32-byte reads and more steps in flight
// gained nothing), and waves per SIMD of both MFMA kernels (two or four were slower).
#define TT_KS_LB1 16   // one activation tile
#define TT_KS_LB 16    // two or four activation tiles
#define TT_KS_D1 2
#define TT_KS_D 2
#define TT_KS_WPE 1
template <int MT> constexpr int ks_lane_bytes() { return MT == 1 ? TT_KS_LB1 : TT_KS_LB; }
template <int MT> constexpr int ks_depth() { return MT == 1 ? TT_KS_D1 : TT_KS_D; }
// K columns per pipeline step: a lane reads LB bytes of one weight row, a quarter of
// the step's columns (int4: 2 LB columns, fp8: LB).
template <WFmt W, int MT> constexpr int step_cols() {
  return W == WFmt::kInt4G128 ? 8 * ks_lane_bytes<MT>() : 4 * ks_lane_bytes<MT>();
}
constexpr int kMaxNT = 6;     // 16-row tiles per workgroup

struct MfmaParams {
  const uint8_t* w;
  int64_t w_row;        // bytes between weight rows
  const void* s;        // int4: fp16 [N, K/128] (s_row elements between rows); fp8: fp32 [N]
  int64_t s_row;
  const uint16_t* x;    // fp16 [M, x_row]
  int64_t x_row;
  uint16_t* out;        // fp16 [M, out_row]
  int64_t out_row;
  int m, n, k;
  int rt;               // weight rows per 16-row MFMA tile (<= 16; rows past rt are padding)
  int steps;            // K / step_cols
};

// A operand of MFMA q: 8 weights (one 32-bit word of int4 codes, two of fp8) as fp16.
//   int4: (c - 8) * s rounded once to fp16 (the dequantised weight), in the order the
//         nibble decode yields them: columns 0 4 1 5 2 6 3 7 of the word (the
//         activations are permuted to the same order);
//   fp8:  the exact fp16 value of each byte in column order (the row scale multiplies
//         the fp32 sum).
template <WFmt W>
__device__ __forceinline__ h8 a_operand(const uint32_t* wd, int q, h2 s2) {
  h8 a;
  if constexpr (W == WFmt::kInt4G128) {
    h2 p0, p1, p2, p3;
    nib_pairs(wd[q], 8.0f, p0, p1, p2, p3);   // exact c - 8
    p0 = p0 * s2; p1 = p1 * s2; p2 = p2 * s2; p3 = p3 * s2;
    a[0] = p0[0]; a[1] = p0[1]; a[2] = p1[0]; a[3] = p1[1];
    a[4] = p2[0]; a[5] = p2[1]; a[6] = p3[0]; a[7] = p3[1];
  } else {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const h2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(wd[2 * q + h], 1.0f, false);
      const h2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(wd[2 * q + h], 1.0f, true);
      a[4 * h + 0] = lo[0]; a[4 * h + 1] = lo[1]; a[4 * h + 2] = hi[0]; a[4 * h + 3] = hi[1];
    }
  }
  return a;
}

// Eight consecutive activations (x0 .. x7 in four dwords) reordered to the int4
// operand order x0 x4 x1 x5 x2 x6 x3 x7.
__device__ __forceinline__ uint4 nib_order(uint4 v) {
  return (uint4){__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                 __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
}

// f(integral_constant<I>) for I = B .. E-1, unrolled at compile time.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// y[m][n] = sum_k W[n][k] x[m][k] on v_mfma_f32_16x16x32_f16, the weights as the A
// operand (rows n) and the activations as the B operand (columns m).
//
//   * Workgroup b owns NT tiles of rt weight rows each (rows b NT rt ..), every
//     activation row (MT tiles of 16) and the whole K axis; the host picks NT and rt so
//     that the blocks cover N with one workgroup per CU (17920 rows on 256 CUs: five
//     tiles of 14 rows).  Rows past rt in a tile are padding: their lanes load a
//     duplicate of the tile's last row and their outputs are not stored.
//   * The four waves split K: wave w takes steps [w S / 4, (w + 1) S / 4).  In a step,
//     lane l reads LB bytes of weight row l % 16 of every tile (columns of quarter l / 16
//     of the step) and the matching activation columns of row l % 16 of every
//     activation tile, straight into MFMA operand registers: no LDS staging, and no
//     operand is read twice inside the workgroup (the activations come from L2; every
//     workgroup reads all of x once).  Each activation fragment feeds NT MFMAs and each
//     dequantised weight fragment MT.
//   * D steps of loads are in flight per wave (the weights and activations of step
//     i + D requested right after step i computes; vector loads complete in issue
//     order, so both streams get the same lead).
//   * At the end the waves' fp32 tiles are summed through LDS in a fixed order,
//     w0 + (w1 + (w2 + w3)), times the fp8 row scale, and stored as fp16: one launch,
//     no workspace, and a result independent of timing.
// MFMA sums products in a hardware-defined order, so this path matches the
// dequantise-then-matmul reference to the stated tolerance, not bit for bit.
template <WFmt W, int MT, int NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TT_KS_WPE, TT_KS_WPE)))
void mfma_ksplit_kernel(MfmaParams P) {
  constexpr bool kI4 = W == WFmt::kInt4G128;
  constexpr int LB = ks_lane_bytes<MT>();
  constexpr int D = ks_depth<MT>();
  constexpr int kSC = step_cols<W, MT>();
  constexpr int kLC = kSC / 4;             // columns per lane and step
  constexpr int kNQ = kLC / 8;             // MFMAs per (tile, activation tile) and step
  constexpr int kRB = kI4 ? kSC / 2 : kSC; // weight bytes per row and step
  constexpr int kWV = LB / 16;             // 16-byte weight loads per tile and step
  constexpr int kXV = kLC / 8;             // 16-byte activation loads per activation tile and step
  static_assert(kRB == 4 * LB, "a lane reads a quarter of the step's row bytes");
  __shared__ float red[NT * MT * 4 * 64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int r = lane & 15, q4 = lane >> 4;
  const int s0 = wave * P.steps / 4;
  const int cnt = (wave + 1) * P.steps / 4 - s0;
  const int rt = P.rt;
  const int64_t row0 = (int64_t)blockIdx.x * NT * rt;

  const uint8_t* wp[NT];
  const uint16_t* sp[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    int64_t row = row0 + t * rt + (r < rt ? r : rt - 1);
    row = row < P.n ? row : P.n - 1;
    wp[t] = P.w + row * P.w_row + (int64_t)s0 * kRB + q4 * LB;
    // int4: the lane's columns lie in group (step * kSC + q4 * kLC) / 128
    if constexpr (kI4) sp[t] = static_cast<const uint16_t*>(P.s) + row * P.s_row + (s0 * kSC + q4 * kLC) / 128;
  }
  const uint16_t* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const int m = 16 * mt + r < P.m ? 16 * mt + r : P.m - 1;
    xp[mt] = P.x + (int64_t)m * P.x_row + (int64_t)s0 * kSC + q4 * kLC;
  }
  // fp8: the row scales of the lane's output rows, requested first (clamped rows: every
  // load unconditional, so none of them waits in the epilogue)
  float rs[kI4 ? 1 : NT][4];
  if constexpr (!kI4) {
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        int64_t row = row0 + t * rt + (4 * q4 + i < rt ? 4 * q4 + i : rt - 1);
        row = row < P.n ? row : P.n - 1;
        rs[t][i] = static_cast<const float*>(P.s)[row];
      }
  }

  uint4 wr[D][NT][kWV];
  uint16_t sr[D][NT];
  uint4 xr[D][MT][kXV];
  auto load = [&](auto uc, int i) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int t = 0; t < NT; t++) {
#pragma unroll
      for (int v = 0; v < kWV; v++) wr[u][t][v] = *reinterpret_cast<const uint4*>(wp[t] + (int64_t)i * kRB + 16 * v);
      if constexpr (kI4) sr[u][t] = sp[t][i * kSC / 128];
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int v = 0; v < kXV; v++) xr[u][mt][v] = *reinterpret_cast<const uint4*>(xp[mt] + (int64_t)i * kSC + 8 * v);
  };

  f4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[t][mt] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    h2 s2[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if constexpr (kI4) {
        const _Float16 sv = __builtin_bit_cast(_Float16, sr[u][t]);
        s2[t] = (h2){sv, sv};
      } else {
        s2[t] = (h2){};
      }
    }
#pragma unroll
    for (int q = 0; q < kNQ; q++) {
      h8 b[MT];
#pragma unroll
      for (int mt = 0; mt < MT; mt++) b[mt] = __builtin_bit_cast(h8, kI4 ? nib_order(xr[u][mt][q]) : xr[u][mt][q]);
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const uint32_t* wd = reinterpret_cast<const uint32_t*>(&wr[u][t][0]);
        const h8 a = a_operand<W>(wd, q, s2[t]);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[mt], acc[t][mt], 0, 0, 0);
      }
    }
  };

  // Every load in the pipeline is unconditional (steps past the range repeat the last
  // one, a cache hit), so the outstanding-load count is the same on every path and
  // each wait leaves the later steps' loads in flight.
  if (cnt > 0) {
    static_for<0, D>([&](auto uc) __attribute__((always_inline)) {
      load(uc, decltype(uc)::value < cnt ? decltype(uc)::value : cnt - 1);
    });
    int i0 = 0;
    for (; i0 + D <= cnt; i0 += D) {
      static_for<0, D>([&](auto uc) __attribute__((always_inline)) {
        compute(uc);
        const int nxt = i0 + decltype(uc)::value + D;
        load(uc, nxt < cnt ? nxt : cnt - 1);
      });
    }
    static_for<0, D - 1>([&](auto uc) __attribute__((always_inline)) {
      if (i0 + decltype(uc)::value < cnt) compute(uc);
    });
  }

  // waves 3, 2, 1 leave running sums in LDS (the same lane and register positions in
  // every wave hold the same output element); wave 0 adds its own and stores
#pragma unroll
  for (int w = 3; w >= 1; w--) {
    if (wave == w) {
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float* p = red + ((t * MT + mt) * 4 + i) * 64 + lane;
            *p = w == 3 ? acc[t][mt][i] : acc[t][mt][i] + *p;
          }
    }
    __syncthreads();
  }
  if (wave != 0) return;
  // lane holds rows 4 q4 + i of tile t, activation row 16 mt + r
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int tr = 4 * q4 + i;
      const int64_t row = row0 + t * rt + tr;
      if (tr >= rt || row >= P.n) continue;
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        const int m = 16 * mt + r;
        if (m >= P.m) continue;
        float v = acc[t][mt][i] + red[((t * MT + mt) * 4 + i) * 64 + lane];
        if constexpr (!kI4) v = v * rs[t][i];
        P.out[(int64_t)m * P.out_row + row] = f32_to_f16_bits(v);
      }
    }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32x4 nib_order4(u32x4 v) {
  return (u32x4){__builtin_amdgcn_perm(v[2], v[0], 0x05040100u), __builtin_amdgcn_perm(v[2], v[0], 0x07060302u),
                 __builtin_amdgcn_perm(v[3], v[1], 0x05040100u), __builtin_amdgcn_perm(v[3], v[1], 0x07060302u)};
}

// ---------------------------------------------------------------- MFMA, LDS-staged operands
// The same block / K-split decomposition as mfma_ksplit_kernel, with both operands
// loaded coalesced and transposed through a per-wave LDS buffer instead of straight
// into operand registers.  A direct load in MFMA layout gives the 16 lanes of a pass
// 16 different rows, which the address unit serves one row at a time; here every quad
// of lanes reads 64 contiguous bytes of one row into registers (D steps ahead), the
// wave writes a step's pieces to its LDS buffer (swizzled so that the fragment reads
// are free of bank conflicts, up to two-way for the int4 weights) and reads its MFMA
// fragments back.  A wave's LDS reads and writes execute in order, so the buffer needs
// no barrier; the waves share nothing until the final sum.
//
// A step covers 64 columns of K.  Per wave and step: the weight rows of the NT tiles
// (int4: 32 bytes a row, fp8: 64) and 64 columns of every activation row; lane
// (r = l % 16, q4 = l / 16) owns columns [16 q4, 16 q4 + 16) of the step, MFMA q of the
// step (q = 0, 1) the eight columns 16 q4 + 8 q ..  Steps past a wave's range repeat its
// last step, so every load is unconditional.
// steps in flight per wave (one activation tile / more)
#define TT_LDS_D1 3
#define TT_LDS_D 2
template <WFmt W, int MT, int NT> struct LdsGeom {
  static constexpr bool kI4 = W == WFmt::kInt4G128;
  static constexpr int kSC = 64;                        // K columns per step
  static constexpr int kWRB = kI4 ? 32 : 64;            // weight bytes per row and step
  static constexpr int kWP = NT * 16 * kWRB / 16;       // 16-byte weight pieces per step
  static constexpr int kWI = (kWP + 63) / 64;           // weight loads per lane and step
  static constexpr int kXI = 2 * MT;                    // activation loads per lane and step
  static constexpr int kBuf = (kWI + kXI) * 1024;       // LDS bytes per wave
  static constexpr int D = MT == 1 ? TT_LDS_D1 : TT_LDS_D;
  static constexpr int kRed = NT * MT * 4 * 64 * 4;     // bytes of the cross-wave sum
  static constexpr int kLds = (4 * kBuf > kRed ? 4 * kBuf : kRed);
};

template <WFmt W, int MT, int NT, int WV = 4>
__global__ __launch_bounds__(64 * WV) void mfma_lds_kernel(MfmaParams P) {
  using G = LdsGeom<W, MT, NT>;
  constexpr bool kI4 = G::kI4;
  constexpr int D = G::D;
  constexpr int kLds = WV * G::kBuf > G::kRed ? WV * G::kBuf : G::kRed;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int r = lane & 15, q4 = lane >> 4;
  const int s0 = wave * P.steps / WV;
  const int cnt = (wave + 1) * P.steps / WV - s0;
  const int rt = P.rt;
  const int64_t row0 = (int64_t)blockIdx.x * NT * rt;
  // the wave's buffer as an LDS-space pointer: stores through it cannot alias the
  // private arrays (a generic pointer would force them into scratch memory)
  typedef __attribute__((address_space(3))) uint8_t lds_u8;
  lds_u8* const buf = reinterpret_cast<lds_u8*>(reinterpret_cast<uintptr_t>(lds)) + wave * G::kBuf;

  // ---- load sources (step 0 of the wave; + i * step bytes) and LDS destinations
  // weights: piece f = v * 64 + lane of the step's block (rows of all tiles in order)
  const uint8_t* wsrc[G::kWI];
  int wdst[G::kWI];
#pragma unroll
  for (int v = 0; v < G::kWI; v++) {
    const int f0 = v * 64 + lane;
    const int f = f0 < G::kWP ? f0 : G::kWP - 1;        // the last load's spare lanes repeat a piece
    int R, c, pc;
    if constexpr (kI4) {              // 32-byte rows: two pieces, swapped on row bit 2
      R = f >> 1;
      c = f & 1;
      pc = c ^ ((R >> 2) & 1);
    } else {                          // 64-byte rows: four pieces, xor-swizzled on row bits 1-2
      R = f >> 2;
      c = f & 3;
      pc = c ^ ((R >> 1) & 3);
    }
    const int t = R >> 4, rr = R & 15;
    int64_t row = row0 + t * rt + (rr < rt ? rr : rt - 1);
    row = row < P.n ? row : P.n - 1;
    wsrc[v] = P.w + row * P.w_row + (int64_t)s0 * G::kWRB + 16 * c;
    wdst[v] = R * G::kWRB + 16 * pc;
  }
  // activations: load v = 2 mt + h covers rows 8 h .. 8 h + 7 of tile mt, eight 16-byte
  // pieces a row, xor-swizzled on the row's low three bits
  const uint16_t* xsrc[G::kXI];
  int xdst[G::kXI];
#pragma unroll
  for (int v = 0; v < G::kXI; v++) {
    const int mt = v >> 1;
    const int rr = 8 * (v & 1) + (lane >> 3);
    const int c = lane & 7;
    const int m = 16 * mt + rr < P.m ? 16 * mt + rr : P.m - 1;
    xsrc[v] = P.x + (int64_t)m * P.x_row + (int64_t)s0 * G::kSC + 8 * c;
    xdst[v] = G::kWI * 1024 + mt * 2048 + rr * 128 + 16 * (c ^ (rr & 7));
  }
  // int4 group scale of the lane's row in every tile (group (s0 + i) / 2 at step i)
  const uint16_t* sp[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    int64_t row = row0 + t * rt + (r < rt ? r : rt - 1);
    row = row < P.n ? row : P.n - 1;
    if constexpr (kI4) sp[t] = static_cast<const uint16_t*>(P.s) + row * P.s_row;
    else sp[t] = nullptr;
  }
  float rs[kI4 ? 1 : NT][4];
  if constexpr (!kI4) {
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        int64_t row = row0 + t * rt + (4 * q4 + i < rt ? 4 * q4 + i : rt - 1);
        row = row < P.n ? row : P.n - 1;
        rs[t][i] = static_cast<const float*>(P.s)[row];
      }
  }

  u32x4 wst[D][G::kWI], xst[D][G::kXI];
  uint16_t sr[D][NT];
  auto issue = [&](auto uc, int i) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int v = 0; v < G::kWI; v++) wst[u][v] = *reinterpret_cast<const u32x4*>(wsrc[v] + (int64_t)i * G::kWRB);
#pragma unroll
    for (int v = 0; v < G::kXI; v++) xst[u][v] = *reinterpret_cast<const u32x4*>(xsrc[v] + (int64_t)i * G::kSC);
    if constexpr (kI4) {
#pragma unroll
      for (int t = 0; t < NT; t++) sr[u][t] = sp[t][(s0 + i) >> 1];
    }
  };

  f4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[t][mt] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

  // fragment offsets in the buffer
  const int wfrag = kI4 ? r * 32 + 16 * ((q4 >> 1) ^ ((r >> 2) & 1)) + 8 * (q4 & 1)
                        : r * 64 + 16 * (q4 ^ ((r >> 1) & 3));
  const int xfrag0 = G::kWI * 1024 + r * 128 + 16 * ((2 * q4) ^ (r & 7));
  const int xfrag1 = G::kWI * 1024 + r * 128 + 16 * ((2 * q4 + 1) ^ (r & 7));

  auto compute = [&](auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int v = 0; v < G::kWI; v++) *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(buf + wdst[v]) = wst[u][v];
#pragma unroll
    for (int v = 0; v < G::kXI; v++) *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(buf + xdst[v]) = xst[u][v];
    uint32_t wd[NT][4];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if constexpr (kI4) {
        const u32x2 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x2*>(buf + t * 512 + wfrag);
        wd[t][0] = v[0]; wd[t][1] = v[1]; wd[t][2] = 0; wd[t][3] = 0;
      } else {
        const u32x4 v = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(buf + t * 1024 + wfrag);
        wd[t][0] = v[0]; wd[t][1] = v[1]; wd[t][2] = v[2]; wd[t][3] = v[3];
      }
    }
    u32x4 xf[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      xf[mt][0] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(buf + mt * 2048 + xfrag0);
      xf[mt][1] = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(buf + mt * 2048 + xfrag1);
    }
    h2 s2[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if constexpr (kI4) {
        const _Float16 sv = __builtin_bit_cast(_Float16, sr[u][t]);
        s2[t] = (h2){sv, sv};
      } else {
        s2[t] = (h2){};
      }
    }
    // every operand of the step is formed before the first MFMA: a VALU write to a
    // register that an issued MFMA still reads waits for that MFMA, so operand
    // registers are not reused inside the step
    h8 bo[2][MT], ao[2][NT];
#pragma unroll
    for (int q = 0; q < 2; q++) {
#pragma unroll
      for (int mt = 0; mt < MT; mt++) bo[q][mt] = __builtin_bit_cast(h8, kI4 ? nib_order4(xf[mt][q]) : xf[mt][q]);
#pragma unroll
      for (int t = 0; t < NT; t++) ao[q][t] = a_operand<W>(wd[t], q, s2[t]);
    }
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
          acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ao[q][t], bo[q][mt], acc[t][mt], 0, 0, 0);
  };

  if (cnt > 0) {
    static_for<0, D>([&](auto uc) __attribute__((always_inline)) {
      issue(uc, decltype(uc)::value < cnt ? decltype(uc)::value : cnt - 1);
    });
    int i0 = 0;
    for (; i0 + D <= cnt; i0 += D) {
      static_for<0, D>([&](auto uc) __attribute__((always_inline)) {
        compute(uc);
        const int nxt = i0 + decltype(uc)::value + D;
        issue(uc, nxt < cnt ? nxt : cnt - 1);
      });
    }
    static_for<0, D - 1>([&](auto uc) __attribute__((always_inline)) {
      if (i0 + decltype(uc)::value < cnt) compute(uc);
    });
  }
  __syncthreads();   // every wave is done with its buffer: the sum reuses the space

  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int w = WV - 1; w >= 1; w--) {
    if (wave == w) {
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float* p = red + ((t * MT + mt) * 4 + i) * 64 + lane;
            *p = w == WV - 1 ? acc[t][mt][i] : acc[t][mt][i] + *p;
          }
    }
    __syncthreads();
  }
  if (wave != 0) return;
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int tr = 4 * q4 + i;
      const int64_t row = row0 + t * rt + tr;
      if (tr >= rt || row >= P.n) continue;
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        const int m = 16 * mt + r;
        if (m >= P.m) continue;
        float v = acc[t][mt][i] + red[((t * MT + mt) * 4 + i) * 64 + lane];
        if constexpr (!kI4) v = v * rs[t][i];
        P.out[(int64_t)m * P.out_row + row] = f32_to_f16_bits(v);
      }
    }
}

inline int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int c = 0;
    cus[dev] = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0 ? c : 256;
  }
  return cus[dev];
}

// Tiles per workgroup (nt <= kMaxNT) and rows per tile (rt <= 16): the fewest rows per
// workgroup that cover N with one workgroup per CU, cut into as few tiles as hold them.
struct MfmaPlan {
  int nt, rt;
  int64_t blocks;
};
inline MfmaPlan mfma_plan(int64_t n, int cus) {
  const int64_t per = (n + cus - 1) / cus;
  MfmaPlan p;
  p.nt = (int)std::min<int64_t>(kMaxNT, std::max<int64_t>(1, (per + 15) / 16));
  p.rt = (int)std::min<int64_t>(16, (per + p.nt - 1) / p.nt);
  p.blocks = (n + (int64_t)p.nt * p.rt - 1) / ((int64_t)p.nt * p.rt);
  return p;
}

// Four waves per workgroup: eight (each with half the K steps, two waves per SIMD)
// measured slower at 17920 x 5120 (int4 M = 64 39.5 -> 41.2 us, fp8 M = 16 26.7 -> 28.1 us).
template <WFmt W, int MT, int NT>
int launch_lds(const MfmaParams& P, const dim3& grid, hipStream_t st) {
  constexpr int WV = 4;
  hipLaunchKernelGGL((mfma_lds_kernel<W, MT, NT, WV>), grid, dim3(64 * WV), 0, st, P);
  return TT_OK;
}

// int4 with one activation tile runs the register-direct kernel (its per-step VALU
// work, not the address unit, bounds it: 22.8 against 24.4 us at 17920 x 5120, M = 16);
// everything else the LDS-staged one (int4 M = 64: 44.3 -> 40.8 us, fp8 M = 16 / 64:
// 31.2 -> 26.7 / 47.7 -> 40.9 us).
template <WFmt W, int MT> constexpr bool use_lds_kernel() { return !(W == WFmt::kInt4G128 && MT == 1); }

template <WFmt W, int MT>
int launch_mfma_mt(const MfmaParams& P, int nt, const dim3& grid, hipStream_t st) {
  if constexpr (use_lds_kernel<W, MT>()) {
    switch (nt) {
      case 1: return launch_lds<W, MT, 1>(P, grid, st);
      case 2: return launch_lds<W, MT, 2>(P, grid, st);
      case 3: return launch_lds<W, MT, 3>(P, grid, st);
      case 4: return launch_lds<W, MT, 4>(P, grid, st);
      case 5: return launch_lds<W, MT, 5>(P, grid, st);
      default: return launch_lds<W, MT, 6>(P, grid, st);
    }
  } else {
    switch (nt) {
      case 1: hipLaunchKernelGGL((mfma_ksplit_kernel<W, MT, 1>), grid, dim3(256), 0, st, P); break;
      case 2: hipLaunchKernelGGL((mfma_ksplit_kernel<W, MT, 2>), grid, dim3(256), 0, st, P); break;
      case 3: hipLaunchKernelGGL((mfma_ksplit_kernel<W, MT, 3>), grid, dim3(256), 0, st, P); break;
      case 4: hipLaunchKernelGGL((mfma_ksplit_kernel<W, MT, 4>), grid, dim3(256), 0, st, P); break;
      case 5: hipLaunchKernelGGL((mfma_ksplit_kernel<W, MT, 5>), grid, dim3(256), 0, st, P); break;
      default: hipLaunchKernelGGL((mfma_ksplit_kernel<W, MT, 6>), grid, dim3(256), 0, st, P); break;
    }
  }
  return TT_OK;
}

template <WFmt W>
int launch_mfma(MfmaParams P, hipStream_t st, const char* what) {
  const MfmaPlan plan = mfma_plan(P.n, device_cus() * TT_KS_WPE);
  const int mt = (P.m + 15) / 16;
  const int sc = mt == 1 ? (use_lds_kernel<W, 1>() ? 64 : step_cols<W, 1>()) : (use_lds_kernel<W, 4>() ? 64 : step_cols<W, 4>());
  P.rt = plan.rt;
  P.steps = P.k / sc;
  TT_REQUIRE(P.steps >= 1 && P.steps * sc == P.k, "%s: K must be a multiple of %d on the MFMA path", what, sc);
  TT_REQUIRE(plan.blocks >= 1 && plan.blocks < (1LL << 31), "%s: bad MFMA grid", what);
  const dim3 grid((unsigned)plan.blocks);
  int rc;
  if (mt == 1) rc = launch_mfma_mt<W, 1>(P, plan.nt, grid, st);
  else if (mt == 2) rc = launch_mfma_mt<W, 2>(P, plan.nt, grid, st);
  else rc = launch_mfma_mt<W, 4>(P, plan.nt, grid, st);
  return rc ? rc : check_launch(what);
}

// Up to four activation rows per GEMV launch, eight with M8 (the dense decode-step
// GEMVs, whose fp16 weights are the largest reads of a batched step); VALU, bit-exact
// per row.
template <Fmt F, SMode SM, typename ST, int ROWS, int L, bool AM, bool M8 = AM>
int launch_rows(GemvParams P, int64_t m_total, int64_t x_row, int64_t out_row, int lpr, hipStream_t st,
                const char* what, int64_t partial_stride) {
  P.x_slot = x_row;
  P.out_slot = out_row;
  const uint16_t* x0 = static_cast<const uint16_t*>(P.x);
  uint8_t* out0 = static_cast<uint8_t*>(P.seg[0].out);
  uint64_t* part0 = P.am_partials;
  for (int64_t m0 = 0; m0 < m_total;) {
    const int64_t left = m_total - m0;
    const int mr = (M8 && left >= 8) ? 8 : (left >= 4 ? 4 : (left >= 2 ? 2 : 1));
    GemvParams Q = P;
    Q.x = x0 + m0 * x_row;
    if (out0) Q.seg[0].out = out0 + m0 * out_row * 2;
    if (AM) Q.am_partials = part0 + m0 * partial_stride;
    int rc;
    switch (mr) {
      case 8:
        if constexpr (M8) rc = launch_lpr<F, SM, f16_t, f16_t, ST, ROWS, L, Pro::kLoad, false, 1, 8>(lpr, Q, 1, st, what);
        else rc = TT_ERR_INVALID;
        break;
      case 4: rc = launch_lpr<F, SM, f16_t, f16_t, ST, ROWS, L, Pro::kLoad, false, 1, 4>(lpr, Q, 1, st, what); break;
      case 2: rc = launch_lpr<F, SM, f16_t, f16_t, ST, ROWS, L, Pro::kLoad, false, 1, 2>(lpr, Q, 1, st, what); break;
      default: rc = launch_lpr<F, SM, f16_t, f16_t, ST, ROWS, L, Pro::kLoad, false, 1, 1>(lpr, Q, 1, st, what); break;
    }
    if (rc) return rc;
    m0 += mr;
  }
  return TT_OK;
}

// Token of each activation row.  Rows go to GEMV launches of eight (then four, two
// and one for the tail); the launch holding rows m0 .. m0 + mr - 1 writes the key of
// (wave w, row r) at partials[m0 * per + w * mr + r].
__global__ __launch_bounds__(256) void argmax_rows_kernel(const uint64_t* partials, int64_t per, int64_t m_total,
                                                          int64_t* out_idx, float* out_val) {
  const int64_t m = blockIdx.x;
  int64_t b = m_total / 8 * 8, rem = m_total - b;
  int64_t m0, mr;
  if (m < b) {
    m0 = m / 8 * 8;
    mr = 8;
  } else {
    if (rem >= 4 && m >= b + 4) {
      b += 4;
      rem -= 4;
    }
    if (rem >= 4) {
      m0 = b;
      mr = 4;
    } else if (rem >= 2 && m < b + 2) {
      m0 = b;
      mr = 2;
    } else {
      m0 = m;
      mr = 1;
    }
  }
  const uint64_t* base = partials + m0 * per + (m - m0);
  __shared__ uint64_t red[256];
  uint64_t best = 0;
  // eight independent loads in flight per thread and step
  for (int64_t i0 = threadIdx.x; i0 < per; i0 += 256 * 8) {
    uint64_t k[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int64_t i = i0 + 256 * u;
      k[u] = i < per ? base[i * mr] : 0;
    }
#pragma unroll
    for (int u = 0; u < 8; u++) best = k[u] > best ? k[u] : best;
  }
  red[threadIdx.x] = best;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] = red[threadIdx.x + s] > red[threadIdx.x] ? red[threadIdx.x + s] : red[threadIdx.x];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const uint64_t k = red[0];
    const uint32_t o = (uint32_t)(k >> 32);
    const uint32_t bits = o == 0xffffffffu ? 0x7fc00000u : ((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
    out_idx[m] = (int64_t)(0xffffffffu - (uint32_t)k);
    if (out_val) out_val[m] = __builtin_bit_cast(float, bits);
  }
}

}  // namespace

namespace tt {
int dense_bias_rows_f16(const void* weight, int64_t w_row, const void* bias, const void* x, int64_t x_row, void* out,
                        int64_t out_row, int64_t m, int64_t rows, int64_t cols, hipStream_t st) {
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight), w_row * 2, nullptr, 0, 0, out, (int)rows};
  P.seg[0].bias = bias;
  P.x = x;
  P.cols = (int)cols;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  return launch_rows<Fmt::kF16W, SMode::kNone, float, 2, 1, false, true>(P, m, x_row, out_row, lpr, st,
                                                                         "matvec_bias_rows", 0);
}
}  // namespace tt

// Smallest M that runs on MFMA (tolerance parity from there; bit-exact GEMV below).
constexpr int kInt4MfmaMin = 4;
constexpr int kFp8MfmaMin = 16;

// The MFMA path sums its partial tiles inside the workgroup: no workspace (the
// workspace arguments of the batched entry points are accepted and unused).
extern "C" int64_t tt_batched_workspace_floats(int64_t m, int64_t rows, int64_t cols) {
  (void)m;
  (void)rows;
  (void)cols;
  return 0;
}

extern "C" int tt_int4_batched_matvec(const void* packed, int64_t w_row_bytes, const void* scales, int64_t s_row,
                                      const void* x, int64_t x_row, void* out, int64_t out_row, int64_t m,
                                      int64_t rows, int64_t cols, int64_t group_size, float* workspace,
                                      int64_t workspace_floats, void* stream) {
  const char* what = "int4_batched_matvec";
  TT_UNSUPPORTED(group_size == 128, "%s: batched int4 uses group size 128", what);
  TT_REQUIRE(cols > 0 && cols % 256 == 0 && cols <= 8192, "%s: cols must be a multiple of 256 up to 8192", what);
  TT_REQUIRE(m >= 1 && m <= 64, "%s: 1 to 64 activation rows", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 28), "%s: bad rows", what);
  TT_REQUIRE(packed && aligned(packed, 16) && w_row_bytes % 16 == 0 && w_row_bytes >= cols / 2,
             "%s: packed weights must be 16-byte aligned rows", what);
  TT_REQUIRE(scales && x && out && aligned(x, 16) && x_row % 8 == 0 && x_row >= cols && out_row >= rows,
             "%s: null or misaligned pointer / bad row strides", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)workspace;
  (void)workspace_floats;
  if (m >= kInt4MfmaMin) {
    TT_REQUIRE(aligned(scales, 2) && s_row >= cols / 128, "%s: fp16 scales [rows, cols / 128] expected", what);
    MfmaParams P{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, static_cast<const uint16_t*>(x),
                 x_row, static_cast<uint16_t*>(out), out_row, (int)m, (int)rows, (int)cols};
    return launch_mfma<WFmt::kInt4G128>(P, st, what);
  }
  if (m == 1)   // one row: the single-row GEMV itself (its lean int4 kernel)
    return tt_int4_scaled_matvec(packed, w_row_bytes, scales, TT_F16, s_row, 1, 0, 0, x, TT_F16, out, TT_F16, rows, cols,
                                 group_size, stream);
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, 1, out, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 4);
  return launch_rows<Fmt::kInt4Sym, SMode::kGroup, f16_t, 2, 4, false>(P, m, x_row, out_row, lpr, st, what, 0);
}

extern "C" int tt_scaled_batched_matvec(const void* weight, int64_t w_row_bytes, const float* scales, const void* x,
                                        int64_t x_row, void* out, int64_t out_row, int64_t m, int64_t rows,
                                        int64_t cols, float* workspace, int64_t workspace_floats, void* stream) {
  const char* what = "scaled_batched_matvec";
  TT_REQUIRE(cols > 0 && cols % 256 == 0 && cols <= 8192, "%s: cols must be a multiple of 256 up to 8192", what);
  TT_REQUIRE(m >= 1 && m <= 64, "%s: 1 to 64 activation rows", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 28), "%s: bad rows", what);
  TT_REQUIRE(weight && aligned(weight, 16) && w_row_bytes % 16 == 0 && w_row_bytes >= cols,
             "%s: fp8 weights must be 16-byte aligned rows", what);
  TT_REQUIRE(scales && x && out && aligned(x, 16) && x_row % 8 == 0 && x_row >= cols && out_row >= rows,
             "%s: null or misaligned pointer / bad row strides", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)workspace;
  (void)workspace_floats;
  if (m >= kFp8MfmaMin) {
    MfmaParams P{static_cast<const uint8_t*>(weight), w_row_bytes, scales, 1, static_cast<const uint16_t*>(x), x_row,
                 static_cast<uint16_t*>(out), out_row, (int)m, (int)rows, (int)cols};
    return launch_mfma<WFmt::kFp8Row>(P, st, what);
  }
  if (m == 1)   // one row: the single-row GEMV itself (its lean kernel; the same bits as a row of the engine)
    return tt_scaled_matvec(weight, TT_W_FP8, w_row_bytes, scales, TT_F32, x, TT_F16, out, TT_F16, rows, cols, stream);
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight), w_row_bytes, scales, 1, 0, out, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  return launch_rows<Fmt::kFp8, SMode::kRow, float, 2, 1, false>(P, m, x_row, out_row, lpr, st, what, 0);
}

extern "C" int64_t tt_matvec_argmax_batched_partials(int64_t m, int64_t rows, int64_t cols) {
  return m * tt_matvec_argmax_partials(rows, cols);
}

extern "C" int tt_matvec_argmax_batched(const void* weight, int64_t w_row, const void* x, int64_t x_row, int64_t m,
                                        void* logits, int64_t logits_row, int64_t rows, int64_t cols,
                                        uint64_t* partials, int64_t partials_capacity, int64_t* out_idx,
                                        float* out_val, void* stream) {
  const char* what = "matvec_argmax_batched";
  TT_REQUIRE(m >= 1 && m <= 1024, "%s: 1 to 1024 activation rows", what);
  TT_REQUIRE(weight && aligned(weight, 16) && (w_row * 2) % 16 == 0 && w_row >= cols, "%s: bad weight layout", what);
  TT_REQUIRE(x && aligned(x, 16) && x_row % 8 == 0 && x_row >= cols && partials && out_idx,
             "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1LL << 31) && cols > 0 && cols % 32 == 0 && cols <= 8192, "%s: bad shape", what);
  TT_REQUIRE(logits == nullptr || logits_row >= rows, "%s: bad logits stride", what);
  const int64_t per = tt_matvec_argmax_partials(rows, cols);
  TT_REQUIRE(partials_capacity >= m * per, "%s: partials buffer needs %lld entries", what, (long long)(m * per));
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight), w_row * 2, nullptr, 0, 0, logits, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  P.am_partials = partials;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = launch_rows<Fmt::kF16W, SMode::kNone, float, 2, 1, true>(P, m, x_row, logits ? logits_row : 0, lpr, st,
                                                                    what, per);
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3((unsigned)m), dim3(256), 0, st, partials, per, m, out_idx, out_val);
  return check_launch(what);
}
