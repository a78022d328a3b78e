// Batched small-M dequant GEMM: y[m] = W x[m] for M activation rows.
//
//   * M below the MFMA threshold (int4: 4, fp8: 16): the GEMV engine with up to four
//     activation rows per wave (every weight word decoded once, one fma chain per
//     activation row), so row m equals the single-row GEMV bit for bit (one int4 row
//     goes to the single-row kernel itself);
//   * from the threshold (int4 M >= 4, where the engine's per-row fma chains make it
//     VALU-bound; fp8 M >= 16): MFMA, rows past M clamped to the last one.  The four
//     waves of a workgroup own a 64-row block (16 rows each) and all M (<= 64, in
//     tiles of 16) activation rows; per quantisation
//     group of 128 columns each wave issues four v_mfma_f32_16x16x32_f16 with the
//     dequantised weights as the A operand (int4: code times group scale, rounded
//     to fp16; fp8: exact) and the activations (staged in LDS per 256-column slice)
//     as the B operand; fp8's row scale multiplies the fp32 sum.  The (block, slice)
//     units are split evenly over a grid of two workgroups per CU (stream-K), and
//     blocks split between workgroups are summed in a fixed order by a second
//     kernel.  MFMA sums products in a hardware-defined order, so this path matches
//     the dequantise-then-matmul reference to the stated tolerance, not bit for bit.
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

constexpr int kSlice = 256;   // columns of x staged in LDS per step (two int4 groups)
constexpr int kMaxSlices = 8192 / kSlice;

// LDS position (in 16-byte pieces) of activation row 16 t + i, columns 128 gs +
// 32 g + 8 q + [0, 8) of a staged slice.  The B operand of (gs, q, t) is one read of
// 64 consecutive pieces, lane 16 g + i taking piece i ^ (4 q + g) of its 16: any
// group of lanes the LDS serves together reads distinct banks, and so do the 16
// consecutive lanes of a store (one row, 16 pieces = 16 distinct (q, g)).
__device__ __forceinline__ int x_piece(int t, int gs, int q, int g, int i) {
  return ((t * (kSlice / 128) + gs) * 4 + q) * 64 + g * 16 + (i ^ (4 * q + g));
}

enum class WFmt : int { kInt4G128 = 0, kFp8Row = 1 };

struct MfmaParams {
  const uint8_t* w;
  int64_t w_row;        // bytes between weight rows
  const void* s;        // int4: fp16 [N, K/128] (s_row elements between rows); fp8: fp32 [N]
  int64_t s_row;
  const uint16_t* x;    // fp16 [M, x_row]
  int64_t x_row;
  uint16_t* out;        // fp16 [M, out_row]
  int64_t out_row;
  float* ws;            // fp32 partial tiles [2 * grid][16 MT][64] of blocks shared by workgroups
  int m, n, k;
  int spb;              // 256-column slices per 64-row block
  int64_t units;        // blocks * spb
  int grid;             // workgroups
  int ws_row_scale;     // fold: multiply by the fp8 row scale
};

// Weights of one 128-column group for this lane: row n0 + lane % 16, columns
// 128 g + 32 (lane / 16) + [0, 32).
template <WFmt W>
struct WChunk {
  uint32_t w[W == WFmt::kInt4G128 ? 4 : 8];
};

// p: this lane's 32 columns of the group (int4: 16 bytes, fp8: 32 bytes).
template <WFmt W>
__device__ __forceinline__ WChunk<W> load_chunk(const uint8_t* p) {
  WChunk<W> c;
  if constexpr (W == WFmt::kInt4G128) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    c.w[0] = v.x; c.w[1] = v.y; c.w[2] = v.z; c.w[3] = v.w;
  } else {
    const uint4 a = reinterpret_cast<const uint4*>(p)[0], b = reinterpret_cast<const uint4*>(p)[1];
    c.w[0] = a.x; c.w[1] = a.y; c.w[2] = a.z; c.w[3] = a.w;
    c.w[4] = b.x; c.w[5] = b.y; c.w[6] = b.z; c.w[7] = b.w;
  }
  return c;
}

// A operand of step q: the 8 weights of word q of this lane's 32 columns as fp16.
//   int4: (c - 8) * s rounded once to fp16 (the dequantised weight), in the order
//         the nibble decode yields them: k = 0, 4, 1, 5, 2, 6, 3, 7 of the word (the
//         activations are staged in LDS in the same order, so the products pair up);
//   fp8:  the exact fp16 value of each byte, natural order (row scale at the end).
template <WFmt W>
__device__ __forceinline__ h8 a_operand(const WChunk<W>& c, int q, h2 s2) {
  h8 a;
  if constexpr (W == WFmt::kInt4G128) {
    h2 p0, p1, p2, p3;
    nib_pairs(c.w[q], 8.0f, p0, p1, p2, p3);   // exact c - 8
    p0 = p0 * s2; p1 = p1 * s2; p2 = p2 * s2; p3 = p3 * s2;
    a[0] = p0[0]; a[1] = p0[1]; a[2] = p1[0]; a[3] = p1[1];
    a[4] = p2[0]; a[5] = p2[1]; a[6] = p3[0]; a[7] = p3[1];
  } else {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const h2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c.w[2 * q + h], 1.0f, false);
      const h2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c.w[2 * q + h], 1.0f, true);
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

// Workgroups per CU (one wave per SIMD each) and pipeline depth (units in flight)
// per activation tile count.  Two units in flight per workgroup already keep ~16 MB
// of loads in flight over the chip; deeper pipelines only lengthen the start, when
// every workgroup's first unit waits behind the whole initial burst (measured at
// 17920 x 5120, M = 16: depth 8 -> 2 takes 28.0 -> 23.9 us).
#ifndef TT_MFMA_TUNE
template <int MT> constexpr int mfma_per_cu() { return 2; }
template <bool I4, int MT> constexpr int mfma_depth() { return MT <= 3 ? 2 : (I4 ? 3 : 2); }
#endif

// Stream-K over (64-row block, 256-column slice) units: unit u is block u / spb,
// slice u % spb; workgroup w owns units [w T / G, (w + 1) T / G) of T, so every
// workgroup gets the same work (within one unit) whatever the block count, and the
// grid is exactly the workgroups the chip holds at once.
__device__ __host__ __forceinline__ int64_t unit_begin(int64_t w, int64_t units, int64_t grid) {
  return w * units / grid;
}
// The workgroup whose range holds unit u.
__device__ __forceinline__ int64_t unit_owner(int64_t u, int64_t units, int64_t grid) {
  return ((u + 1) * grid - 1) / units;
}

template <WFmt W, int MT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(mfma_per_cu<MT>()))) void mfma_gemm_kernel(MfmaParams P) {
  // Software pipeline of depth D units, held in registers:
  //   * the weights (and int4 group scales) and the activations of unit i are both
  //     requested D units before i computes (vector loads complete in issue order,
  //     so a load issued later than another can never be waited for earlier: both
  //     streams get the same lead);
  //   * the activations of unit i + 1 go from registers to one of two LDS buffers at
  //     the end of unit i;
  //   * barriers order LDS only, so the global loads stay in flight across them;
  //   * the pipeline runs on across block boundaries: at the last unit of a block
  //     (or of the workgroup's range) the tile is written out and the accumulators
  //     restart.  A block that lies inside one workgroup's range is stored as fp16;
  //     a block shared by several workgroups leaves one fp32 partial tile per
  //     workgroup, summed in workgroup order by mfma_fold_kernel.
  // int4 weights enter the MFMA already scaled (fp16), so every product of a row
  // accumulates into one fp32 tile; with a single activation tile the accumulation
  // alternates between two tiles (summed at the end) to halve the dependency chain.
  constexpr bool kI4 = W == WFmt::kInt4G128;
  constexpr int kAhead = mfma_depth<kI4, MT>();
  constexpr int NA = MT == 1 ? 2 : 1;                  // accumulator tiles per activation tile
  constexpr int XS = MT * 16 * kSlice;                 // halves per buffer
  constexpr int XV = MT * 16 * kSlice / 8 / 256;       // 16-byte pieces per thread per slice
  constexpr int GPS = kSlice / 128;                    // quantisation groups per slice
  __shared__ __attribute__((aligned(16))) uint16_t xs[2 * XS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int spb = P.spb;
  const int64_t u0 = unit_begin(blockIdx.x, P.units, P.grid);
  const int count = (int)(unit_begin(blockIdx.x + 1, P.units, P.grid) - u0);
  const int first_block = (int)(u0 / spb);
  // cursors: the unit computed (cb, cs) and the unit loaded next (lb, ls, li);
  // loads past the range repeat its last unit, so every load is unconditional and
  // the compiler keeps exact outstanding-load counts across the unrolled pipeline
  int cb = first_block, cs = (int)(u0 - (int64_t)first_block * spb);
  int lb = cb, ls = cs, li = 0;
  // load pointers of the lane: weight row of block lb at slice ls (and its group
  // scales); stepped by one slice per unit, recomputed at block changes
  constexpr int kSliceBytes = kI4 ? kSlice / 2 : kSlice;
  const int lane_col = (kI4 ? 16 : 32) * g;
  const uint8_t* wp;
  const uint16_t* sp;
  auto row_ptrs = [&]() __attribute__((always_inline)) {
    int row = lb * 64 + wave * 16 + (lane & 15);
    row = row < P.n ? row : P.n - 1;
    wp = P.w + (int64_t)row * P.w_row + ls * kSliceBytes + lane_col;
    if constexpr (kI4) sp = static_cast<const uint16_t*>(P.s) + (int64_t)row * P.s_row + ls * GPS;
  };
  row_ptrs();
  auto advance_load = [&]() __attribute__((always_inline)) {
    if (li < count - 1) {
      li++;
      if (++ls == spb) {
        ls = 0;
        lb++;
        row_ptrs();
      } else {
        wp += kSliceBytes;
        if constexpr (kI4) sp += GPS;
      }
    }
  };
  // activation slot u: xq_even / xq_odd[(u / 2) * XV + v] (two arrays: smaller
  // private arrays are the ones the compiler keeps in registers)
  uint4 xq_even[(kAhead + 1) / 2 * XV], xq_odd[(kAhead + 1) / 2 * XV];
  const uint16_t* xb[XV];                              // row min(r, m - 1), columns 8 c8 .. of slice 0
#pragma unroll
  for (int v = 0; v < XV; v++) {
    const int i = threadIdx.x + 256 * v;
    int r = i / (kSlice / 8);
    const int c8 = i - r * (kSlice / 8);
    r = r < P.m ? r : P.m - 1;
    xb[v] = P.x + (int64_t)r * P.x_row + 8 * c8;
  }
  auto load_x = [&](int sl, auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int v = 0; v < XV; v++) {
      const uint4 t = *reinterpret_cast<const uint4*>(xb[v] + sl * kSlice);
      if constexpr ((u & 1) == 0) xq_even[u / 2 * XV + v] = t;
      else xq_odd[u / 2 * XV + v] = t;
    }
  };
  auto store_x = [&](int buf, auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int v = 0; v < XV; v++) {
      const int i = threadIdx.x + 256 * v;
      const int r = i / (kSlice / 8), c8 = i - r * (kSlice / 8);
      uint4 t = (u & 1) == 0 ? xq_even[u / 2 * XV + v] : xq_odd[u / 2 * XV + v];
      if constexpr (kI4) t = nib_order(t);
      const int cc = c8 & 15;
      *reinterpret_cast<uint4*>(xs + buf * XS + 8 * x_piece(r >> 4, c8 >> 4, cc & 3, cc >> 2, r & 15)) = t;
    }
  };
  WChunk<W> ring[kAhead][GPS];
  uint32_t sring[kI4 ? kAhead : 1];                    // int4: the row's two group scales (fp16 pair)
  auto load_unit = [&](auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int gs = 0; gs < GPS; gs++) ring[u][gs] = load_chunk<W>(wp + gs * (kSliceBytes / GPS));
    if constexpr (kI4) sring[u] = *reinterpret_cast<const uint32_t*>(sp);
    load_x(ls, uc);
  };
  f4 acc[NA][MT];
#pragma unroll
  for (int j = 0; j < NA; j++)
#pragma unroll
    for (int t = 0; t < MT; t++) acc[j][t] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
  // prologue: units 0 .. kAhead - 1 in the order every step issues its loads (the
  // wait for unit i + 1's activations is then as shallow in the first loop
  // iteration as in later ones, and the first store waits for unit 0 only)
  static_for<0, kAhead>([&](auto uc) __attribute__((always_inline)) {
    load_unit(uc);
    advance_load();
  });
  store_x(0, std::integral_constant<int, 0>{});
  lds_barrier();

  // lane holds output rows b * 64 + wave * 16 + 4 g + i of activation row 16 t + lane % 16
  auto flush = [&](int b) __attribute__((always_inline)) {
    if constexpr (NA == 2) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        acc[0][0][i] = acc[0][0][i] + acc[1][0][i];
        acc[1][0][i] = 0.0f;
      }
    }
    const int64_t bu = (int64_t)b * spb;
    const int r0 = b * 64 + wave * 16 + 4 * g;
    if (bu >= u0 && bu + spb <= u0 + count) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = r0 + i;
        if (r >= P.n) continue;
        float rs = 1.0f;
        if constexpr (W == WFmt::kFp8Row) rs = reinterpret_cast<const float*>(P.s)[r];
#pragma unroll
        for (int t = 0; t < MT; t++) {
          const int m = 16 * t + (lane & 15);
          if (m < P.m) {
            const float v = W == WFmt::kFp8Row ? acc[0][t][i] * rs : acc[0][t][i];
            P.out[(int64_t)m * P.out_row + r] = f32_to_f16_bits(v);
          }
        }
      }
    } else {
      // partial tile [16 MT][64] in slot 2 w + (0: the range's first block, 1: its last)
      float* tile = P.ws + (int64_t)(2 * blockIdx.x + (b == first_block ? 0 : 1)) * (16 * MT * 64);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int t = 0; t < MT; t++) tile[(16 * t + (lane & 15)) * 64 + wave * 16 + 4 * g + i] = acc[0][t][i];
    }
#pragma unroll
    for (int t = 0; t < MT; t++) acc[0][t] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
  };

  auto step = [&](int i, auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    const uint16_t* xl = xs + (i & 1) * XS;
    // this lane's row scales of the unit's two groups, as (s, s) pairs
    h2 s2[GPS];
    if constexpr (kI4) {
      const h2 sp = __builtin_bit_cast(h2, sring[u]);
#pragma unroll
      for (int gs = 0; gs < GPS; gs++) s2[gs] = (h2){sp[gs], sp[gs]};
    }
    // B operands of a group are read from LDS together, the next group's while the
    // current one's MFMAs run
    h8 bb[GPS][4][MT];
    auto read_b = [&](int gs) __attribute__((always_inline)) {
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int t = 0; t < MT; t++)
          bb[gs][q][t] = *reinterpret_cast<const h8*>(xl + 8 * x_piece(t, gs, q, g, lane & 15));
    };
    read_b(0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int gs = 0; gs < GPS; gs++) {
      if (gs + 1 < GPS) read_b(gs + 1);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const h8 a = a_operand<W>(ring[u][gs], q, kI4 ? s2[gs] : (h2){});
#pragma unroll
        for (int t = 0; t < MT; t++) {
          f4& d = acc[NA == 2 ? (q & 1) : 0][t];
          d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bb[gs][q][t], d, 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (cs == spb - 1 || i == count - 1) flush(cb);
    if (++cs == spb) { cs = 0; cb++; }
    load_unit(uc);                                                   // slot u held unit i, stored a step ago
    advance_load();
    store_x((i + 1) & 1, std::integral_constant<int, (u + 1) % kAhead>{});  // unit i + 1
    lds_barrier();
  };
  int i0 = 0;
  for (; i0 + kAhead <= count; i0 += kAhead)
    static_for<0, kAhead>([&](auto uc) __attribute__((always_inline)) { step(i0 + decltype(uc)::value, uc); });
  // tail: fewer than kAhead units, still with static ring slots
  static_for<0, kAhead - 1>([&](auto uc) __attribute__((always_inline)) {
    if (i0 + decltype(uc)::value < count) step(i0 + decltype(uc)::value, uc);
  });
}

// out[m][n] of the blocks that several workgroups share: the partial tiles summed in
// workgroup order (((+0 + first) + second) + ...) [times the fp8 row scale], so the
// result does not depend on which workgroup finished first.  Workgroup w of this
// kernel takes the block holding unit_begin(w) when w is the first range boundary
// inside that block.
__global__ __launch_bounds__(256) void mfma_fold_kernel(MfmaParams P, int mp) {
  const int64_t w = (int64_t)blockIdx.x + 1;
  const int spb = P.spb;
  const int64_t uw = unit_begin(w, P.units, P.grid);
  const int64_t b = uw / spb, bu = b * spb;
  if (uw == bu || unit_begin(w - 1, P.units, P.grid) > bu) return;
  // partial tiles of the block in workgroup order: workgroups w - 1 .. last
  __shared__ int slot[kMaxSlices + 1];
  const int n_slots = (int)(unit_owner(bu + spb - 1, P.units, P.grid) - (w - 1) + 1);
  if (threadIdx.x < n_slots) {
    const int64_t o = w - 1 + threadIdx.x;
    slot[threadIdx.x] = (int)(2 * o + (b == unit_begin(o, P.units, P.grid) / spb ? 0 : 1));
  }
  __syncthreads();
  const float* rsc = P.ws_row_scale ? reinterpret_cast<const float*>(P.s) : nullptr;
  // kE elements per thread and step with every partial of up to kJ slots requested before
  // the first sum (one memory round trip per step instead of one per element and slot);
  // slots past kJ (blocks shared by more workgroups) are added one at a time after them
  constexpr int kE = 4, kJ = 4;
  for (int e0 = threadIdx.x; e0 < mp * 64; e0 += 256 * kE) {
    float p[kJ][kE];
#pragma unroll
    for (int j = 0; j < kJ; j++)
#pragma unroll
      for (int u = 0; u < kE; u++) {
        const int e = e0 + 256 * u;
        p[j][u] = (j < n_slots && e < mp * 64) ? P.ws[((int64_t)slot[j] * mp + (e >> 6)) * 64 + (e & 63)] : 0.0f;
      }
#pragma unroll
    for (int u = 0; u < kE; u++) {
      const int e = e0 + 256 * u;
      const int mi = e >> 6, c = e & 63;
      const int64_t r = b * 64 + c;
      if (e >= mp * 64 || mi >= P.m || r >= P.n) continue;
      float v = 0.0f;
#pragma unroll
      for (int j = 0; j < kJ; j++)
        if (j < n_slots) v = v + p[j][u];
      for (int j = kJ; j < n_slots; j++) v = v + P.ws[((int64_t)slot[j] * mp + mi) * 64 + c];
      if (rsc) v = v * rsc[r];
      P.out[(int64_t)mi * P.out_row + r] = f32_to_f16_bits(v);
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

// Workgroups of the stream-K grid: the workgroups the chip holds at once, at most
// one per unit.
inline int64_t mfma_grid(int64_t units, int mt) {
  static constexpr int per_cu[4] = {mfma_per_cu<1>(), mfma_per_cu<2>(), mfma_per_cu<3>(), mfma_per_cu<4>()};
  return std::min<int64_t>((int64_t)per_cu[mt - 1] * device_cus(), units);
}

inline int64_t mfma_ws_floats(int64_t m, int64_t rows, int64_t cols) {
  const int mt = (int)((m + 15) / 16);
  const int64_t units = (rows + 63) / 64 * (cols / kSlice);
  return 2 * mfma_grid(units, mt) * 16 * mt * 64;
}

template <WFmt W>
int launch_mfma(MfmaParams P, float* ws, int64_t ws_floats, hipStream_t st, const char* what) {
  const int mt = (P.m + 15) / 16;
  P.spb = P.k / kSlice;
  P.units = (int64_t)((P.n + 63) / 64) * P.spb;
  P.grid = (int)mfma_grid(P.units, mt);
  TT_REQUIRE(P.spb >= 1 && P.units >= 1 && P.grid >= 1, "%s: bad MFMA grid", what);
  TT_REQUIRE(ws != nullptr && ws_floats >= mfma_ws_floats(P.m, P.n, P.k),
             "%s: workspace of tt_batched_workspace_floats(m, rows, cols) floats required on the MFMA path", what);
  P.ws = ws;
  P.ws_row_scale = W == WFmt::kFp8Row ? 1 : 0;
  const dim3 grid((unsigned)P.grid);
  switch (mt) {
    case 1: hipLaunchKernelGGL((mfma_gemm_kernel<W, 1>), grid, dim3(256), 0, st, P); break;
    case 2: hipLaunchKernelGGL((mfma_gemm_kernel<W, 2>), grid, dim3(256), 0, st, P); break;
    case 3: hipLaunchKernelGGL((mfma_gemm_kernel<W, 3>), grid, dim3(256), 0, st, P); break;
    default: hipLaunchKernelGGL((mfma_gemm_kernel<W, 4>), grid, dim3(256), 0, st, P); break;
  }
  int rc = check_launch(what);
  if (rc || P.grid == 1) return rc;
  hipLaunchKernelGGL(mfma_fold_kernel, dim3((unsigned)(P.grid - 1)), dim3(256), 0, st, P, 16 * mt);
  return check_launch(what);
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

extern "C" int64_t tt_batched_workspace_floats(int64_t m, int64_t rows, int64_t cols) {
  if (m < kInt4MfmaMin || m > 64 || rows <= 0 || cols < kSlice) return 0;
  return mfma_ws_floats(m, rows, cols);
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
  if (m >= kInt4MfmaMin) {
    TT_REQUIRE(aligned(scales, 4) && s_row % 2 == 0, "%s: m >= 4 reads scale pairs: 4-byte aligned scales, even row stride",
               what);
    MfmaParams P{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, static_cast<const uint16_t*>(x),
                 x_row, static_cast<uint16_t*>(out), out_row, nullptr, (int)m, (int)rows, (int)cols};
    return launch_mfma<WFmt::kInt4G128>(P, workspace, workspace_floats, st, what);
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
  if (m >= kFp8MfmaMin) {
    MfmaParams P{static_cast<const uint8_t*>(weight), w_row_bytes, scales, 1, static_cast<const uint16_t*>(x), x_row,
                 static_cast<uint16_t*>(out), out_row, nullptr, (int)m, (int)rows, (int)cols};
    return launch_mfma<WFmt::kFp8Row>(P, workspace, workspace_floats, st, what);
  }
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
