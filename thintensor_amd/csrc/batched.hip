// Batched small-M dequant GEMM: y[m] = W x[m] for M activation rows.
//
//   * M < 16: the GEMV engine with up to four activation rows per wave (every
//     weight word decoded once, one fma chain per activation row), so row m equals
//     the single-row GEMV bit for bit;
//   * M >= 16: MFMA.  Each wave owns 16 output rows and all M (<= 64, in tiles of
//     16) activation rows; per quantisation group of 128 columns it issues four
//     v_mfma_f32_16x16x32_f16 with the dequantised weights as the A operand and the
//     activations (staged in LDS per 256-column slice) as the B operand, then scales
//     the group's fp32 tile (int4) or accumulates it (fp8, row scale at the end).
//     MFMA sums products in a hardware-defined order, so this path matches the
//     dequantise-then-matmul reference to the stated tolerance, not bit for bit.
//   * the M-row lm_head argmax runs the GEMV engine with four activation rows per
//     launch and one argmax key per (wave, row); a finishing kernel picks each row's
//     token, as tt_matvec_argmax does for one row.
#include "gemv_impl.h"

#include <type_traits>

using namespace tt;

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kSlice = 256;   // columns of x staged in LDS per step (two int4 groups)
// LDS row pitch of a staged slice, in halves: 16 bytes of padding per row put the 16
// rows that one B-operand read touches in 16 different 4-bank groups (an unpadded
// 512-byte pitch maps them all to the same banks).
constexpr int kPitch = kSlice + 8;

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
  int m, n, k;
};

// Weights of one 128-column group for this lane: row n0 + lane % 16, columns
// 128 g + 32 (lane / 16) + [0, 32).
template <WFmt W>
struct WChunk {
  uint32_t w[W == WFmt::kInt4G128 ? 4 : 8];
};

template <WFmt W>
__device__ __forceinline__ WChunk<W> load_chunk(const MfmaParams& P, int row, int grp, int lane) {
  WChunk<W> c;
  if constexpr (W == WFmt::kInt4G128) {
    const uint4 v = *reinterpret_cast<const uint4*>(P.w + (int64_t)row * P.w_row + (int64_t)grp * 64 + 16 * (lane >> 4));
    c.w[0] = v.x; c.w[1] = v.y; c.w[2] = v.z; c.w[3] = v.w;
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(P.w + (int64_t)row * P.w_row + (int64_t)grp * 128 + 32 * (lane >> 4));
    const uint4 a = p[0], b = p[1];
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

constexpr int kMaxGroups = 8192 / 128;   // int4 scale groups per row (cols <= 8192)

// f(integral_constant<I>) for I = B .. E-1, unrolled at compile time.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Pipeline depth (slices in flight) per activation tile count: as deep as two
// workgroups per CU (256 registers per wave) allow.
template <bool I4, int MT> constexpr int mfma_depth() { return MT == 1 ? 8 : (MT == 2 ? 4 : (I4 ? 4 : 2)); }

template <WFmt W, int MT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void mfma_gemm_kernel(MfmaParams P) {
  // Software pipeline of depth D slices, held in registers:
  //   * the weights and the activations of slice s are both requested D slices
  //     before s computes (vector loads complete in issue order, so a load issued
  //     later than another can never be waited for earlier: both streams get the same
  //     lead);
  //   * the activations of slice s + 1 go from registers to one of two LDS buffers at
  //     the end of slice s;
  //   * the workgroup's int4 group scales are staged in LDS once ([row][group]);
  //   * barriers order LDS only, so the global loads stay in flight across them.
  // int4 weights enter the MFMA already scaled (fp16), so every product of a row
  // accumulates into one fp32 tile; with a single activation tile the accumulation
  // alternates between two tiles (summed at the end) to halve the dependency chain.
  constexpr bool kI4 = W == WFmt::kInt4G128;
  constexpr int kAhead = mfma_depth<kI4, MT>();
  constexpr int NA = MT == 1 ? 2 : 1;                  // accumulator tiles per activation tile
  constexpr int XS = MT * 16 * kPitch;                 // halves per buffer
  constexpr int XV = MT * 16 * kSlice / 8 / 256;       // 16-byte pieces per thread per slice
  constexpr int GPS = kSlice / 128;                    // quantisation groups per slice
  __shared__ __attribute__((aligned(16))) uint16_t xs[2 * XS];
  __shared__ __attribute__((aligned(16))) uint16_t scl[kI4 ? kMaxGroups * 64 : 4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb = blockIdx.x * 64;
  const int n0 = nb + wave * 16;
  const int arow = n0 + (lane & 15);                 // weight row this lane loads (A operand)
  const int lrow = arow < P.n ? arow : P.n - 1;
  const int g = lane >> 4;
  const int slices = P.k / kSlice;
  const int groups = P.k / 128;
  // Every load below is unconditional (indices are clamped) so the compiler keeps
  // exact outstanding-load counts across the unrolled pipeline; rows of x past m and
  // slices past the end are loaded again, and only feed outputs that are not stored.
  // activation slot u: xq_even / xq_odd[(u / 2) * XV + v] (two arrays: smaller
  // private arrays are the ones the compiler keeps in registers)
  uint4 xq_even[kAhead / 2 * XV], xq_odd[kAhead / 2 * XV];
  auto load_x = [&](int sl, auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
#pragma unroll
    for (int v = 0; v < XV; v++) {
      const int i = threadIdx.x + 256 * v;
      int r = i / (kSlice / 8);
      const int c8 = i - r * (kSlice / 8);
      r = r < P.m ? r : P.m - 1;
      const uint4 t = *reinterpret_cast<const uint4*>(P.x + (int64_t)r * P.x_row + (int64_t)sl * kSlice + 8 * c8);
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
      *reinterpret_cast<uint4*>(xs + buf * XS + r * kPitch + 8 * c8) = t;
    }
  };
  f4 acc[NA][MT];
#pragma unroll
  for (int j = 0; j < NA; j++)
#pragma unroll
    for (int t = 0; t < MT; t++) acc[j][t] = (f4){0.0f, 0.0f, 0.0f, 0.0f};
  WChunk<W> ring[kAhead][GPS];
#pragma unroll
  for (int u = 0; u < kAhead; u++)
#pragma unroll
    for (int gs = 0; gs < GPS; gs++) ring[u][gs] = load_chunk<W>(P, lrow, (u < slices ? u : slices - 1) * GPS + gs, lane);
  static_for<0, kAhead>([&](auto uc) __attribute__((always_inline)) {
    load_x(decltype(uc)::value < slices ? decltype(uc)::value : slices - 1, uc);
  });
  if constexpr (kI4) {
    // thread t stages row t / 4, groups t % 4 + 4 j, into scl[row * groups + group]
    const int r = threadIdx.x >> 2;
    const int row = nb + r < P.n ? nb + r : P.n - 1;
    const uint16_t* sg = reinterpret_cast<const uint16_t*>(P.s) + (int64_t)row * P.s_row;
    uint16_t sv[kMaxGroups / 4];
#pragma unroll
    for (int j = 0; j < kMaxGroups / 4; j++) {
      const int gi = (threadIdx.x & 3) + 4 * j;
      sv[j] = sg[gi < groups ? gi : groups - 1];
    }
#pragma unroll
    for (int j = 0; j < kMaxGroups / 4; j++) {
      const int gi = (threadIdx.x & 3) + 4 * j;
      if (gi < groups) scl[r * groups + gi] = sv[j];
    }
  }
  store_x(0, std::integral_constant<int, 0>{});
  lds_barrier();

  const uint16_t* my_scl = scl + (wave * 16 + (lane & 15)) * groups;
  auto step = [&](int sl, auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    const uint16_t* xl = xs + (u & 1) * XS;
    // this lane's row scales of the slice's two groups, as (s, s) pairs
    h2 s2[GPS];
    if constexpr (kI4) {
#pragma unroll
      for (int gs = 0; gs < GPS; gs++) {
        const _Float16 sc = __builtin_bit_cast(_Float16, my_scl[sl * GPS + gs]);
        s2[gs] = (h2){sc, sc};
      }
    }
    // B operands of a group are read from LDS together, the next group's while the
    // current one's MFMAs run (with one wave per SIMD nothing else hides LDS latency)
    h8 bb[GPS][4][MT];
    auto read_b = [&](int gs) __attribute__((always_inline)) {
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int t = 0; t < MT; t++)
          bb[gs][q][t] = *reinterpret_cast<const h8*>(xl + (16 * t + (lane & 15)) * kPitch + 128 * gs + 32 * g + 8 * q);
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
    const int nx = sl + kAhead < slices ? sl + kAhead : slices - 1;
#pragma unroll
    for (int gs = 0; gs < GPS; gs++) ring[u][gs] = load_chunk<W>(P, lrow, nx * GPS + gs, lane);
    load_x(nx, uc);                                                  // slot u held slice sl, stored a step ago
    store_x((u + 1) & 1, std::integral_constant<int, (u + 1) % kAhead>{});  // slice sl + 1
    lds_barrier();
  };
  int s0 = 0;
  for (; s0 + kAhead <= slices; s0 += kAhead)
    static_for<0, kAhead>([&](auto uc) __attribute__((always_inline)) { step(s0 + decltype(uc)::value, uc); });
  // tail: fewer than kAhead slices, still with static ring slots
  static_for<0, kAhead - 1>([&](auto uc) __attribute__((always_inline)) {
    if (s0 + decltype(uc)::value < slices) step(s0 + decltype(uc)::value, uc);
  });
  if constexpr (NA == 2) {
#pragma unroll
    for (int i = 0; i < 4; i++) acc[0][0][i] = acc[0][0][i] + acc[1][0][i];
  }
  // out[m][n]: lane holds rows n0 + 4g + i of activation row 16t + lane % 16
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = n0 + 4 * g + i;
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
}

template <WFmt W>
int launch_mfma(const MfmaParams& P, hipStream_t st, const char* what) {
  const int blocks = (P.n + 63) / 64;
  const int mt = (P.m + 15) / 16;
  switch (mt) {
    case 1: hipLaunchKernelGGL((mfma_gemm_kernel<W, 1>), dim3(blocks), dim3(256), 0, st, P); break;
    case 2: hipLaunchKernelGGL((mfma_gemm_kernel<W, 2>), dim3(blocks), dim3(256), 0, st, P); break;
    case 3: hipLaunchKernelGGL((mfma_gemm_kernel<W, 3>), dim3(blocks), dim3(256), 0, st, P); break;
    default: hipLaunchKernelGGL((mfma_gemm_kernel<W, 4>), dim3(blocks), dim3(256), 0, st, P); break;
  }
  return check_launch(what);
}

// Up to four activation rows per GEMV launch (VALU, bit-exact per row).
template <Fmt F, SMode SM, typename ST, int ROWS, int L, bool AM>
int launch_rows(GemvParams P, int64_t m_total, int64_t x_row, int64_t out_row, int lpr, hipStream_t st,
                const char* what, int64_t partial_stride) {
  P.x_slot = x_row;
  P.out_slot = out_row;
  const uint16_t* x0 = static_cast<const uint16_t*>(P.x);
  uint8_t* out0 = static_cast<uint8_t*>(P.seg[0].out);
  uint64_t* part0 = P.am_partials;
  for (int64_t m0 = 0; m0 < m_total;) {
    const int64_t left = m_total - m0;
    const int mr = left >= 4 ? 4 : (left >= 2 ? 2 : 1);
    GemvParams Q = P;
    Q.x = x0 + m0 * x_row;
    if (out0) Q.seg[0].out = out0 + m0 * out_row * 2;
    if (AM) Q.am_partials = part0 + m0 * partial_stride;
    int rc;
    switch (mr) {
      case 4: rc = launch_lpr<F, SM, f16_t, f16_t, ST, ROWS, L, Pro::kLoad, false, 1, 4>(lpr, Q, 1, st, what); break;
      case 2: rc = launch_lpr<F, SM, f16_t, f16_t, ST, ROWS, L, Pro::kLoad, false, 1, 2>(lpr, Q, 1, st, what); break;
      default: rc = launch_lpr<F, SM, f16_t, f16_t, ST, ROWS, L, Pro::kLoad, false, 1, 1>(lpr, Q, 1, st, what); break;
    }
    if (rc) return rc;
    m0 += mr;
  }
  return TT_OK;
}

// Token of each activation row.  Rows go to GEMV launches of four (then two, then
// one for the tail); the launch holding rows m0 .. m0 + mr - 1 writes the key of
// (wave w, row r) at partials[m0 * per + w * mr + r].
__global__ __launch_bounds__(256) void argmax_rows_kernel(const uint64_t* partials, int64_t per, int64_t m_total,
                                                          int64_t* out_idx, float* out_val) {
  const int64_t m = blockIdx.x;
  const int64_t full = m_total / 4 * 4;
  int64_t m0, mr;
  if (m < full) {
    m0 = m / 4 * 4;
    mr = 4;
  } else if (m_total - full >= 2 && m < full + 2) {
    m0 = full;
    mr = 2;
  } else {
    m0 = m;
    mr = 1;
  }
  const uint64_t* base = partials + m0 * per + (m - m0);
  __shared__ uint64_t red[256];
  uint64_t best = 0;
  for (int64_t i = threadIdx.x; i < per; i += 256) {
    const uint64_t k = base[i * mr];
    best = k > best ? k : best;
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

extern "C" int tt_int4_batched_matvec(const void* packed, int64_t w_row_bytes, const void* scales, int64_t s_row,
                                      const void* x, int64_t x_row, void* out, int64_t out_row, int64_t m,
                                      int64_t rows, int64_t cols, int64_t group_size, void* stream) {
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
  if (m >= 16) {
    MfmaParams P{static_cast<const uint8_t*>(packed), w_row_bytes, scales, s_row, static_cast<const uint16_t*>(x),
                 x_row, static_cast<uint16_t*>(out), out_row, (int)m, (int)rows, (int)cols};
    return launch_mfma<WFmt::kInt4G128>(P, st, what);
  }
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
                                        int64_t cols, void* stream) {
  const char* what = "scaled_batched_matvec";
  TT_REQUIRE(cols > 0 && cols % 256 == 0 && cols <= 8192, "%s: cols must be a multiple of 256 up to 8192", what);
  TT_REQUIRE(m >= 1 && m <= 64, "%s: 1 to 64 activation rows", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 28), "%s: bad rows", what);
  TT_REQUIRE(weight && aligned(weight, 16) && w_row_bytes % 16 == 0 && w_row_bytes >= cols,
             "%s: fp8 weights must be 16-byte aligned rows", what);
  TT_REQUIRE(scales && x && out && aligned(x, 16) && x_row % 8 == 0 && x_row >= cols && out_row >= rows,
             "%s: null or misaligned pointer / bad row strides", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (m >= 16) {
    MfmaParams P{static_cast<const uint8_t*>(weight), w_row_bytes, scales, 1, static_cast<const uint16_t*>(x), x_row,
                 static_cast<uint16_t*>(out), out_row, (int)m, (int)rows, (int)cols};
    return launch_mfma<WFmt::kFp8Row>(P, st, what);
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
