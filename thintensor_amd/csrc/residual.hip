// Residual sidecar corrections for gfx950: out[m] += correction[m], read-modify-write of
// a GEMV output already in `out` (triton_kernels.py:2335-2419, 5429-5487).
//
//   * sparse:  correction = sum_k values[m, k] * x[indices[m, k]]  (k < terms);
//   * binary:  correction = sum_k (bit(m, k) ? +1 : -1) * scale[m, k / 32] * x[k], sign
//              bit k of row m at byte k / 8, bit k % 8 (LSB first).
//
// One wave per row.  Fixed summation order (binary32, reproduced by the CPU oracle):
//   * sparse: lane l sums terms l, l + 64, ... as acc + v * x (separately rounded
//     product and sum); the row is the xor butterfly over the 64 lanes (lane bits in
//     increasing order); out = round(out + correction);
//   * binary: lane l owns 32-column groups l, l + 64, ...; per group p = column-order sum
//     of +-x (exact terms), acc = acc + scale * p; butterfly over 64 lanes; then as above.
// An index outside [0, cols) makes its row's correction NaN (no out-of-range read).
#include "tt_abi_internal.h"
#include "tt_common.h"

namespace tt {
namespace {

struct SparseParams {
  const void* values;       // [rows, terms] (vm, vk element strides)
  const void* indices;      // [rows, terms] int16, int32 or int64 (im, ik element strides)
  const void* x;            // [cols]
  void* out;                // [rows], read and written
  int64_t vm, vk, im, ik;
  int rows, terms, cols;
};

template <typename VT, typename IT, typename XT, typename OT>
__global__ __launch_bounds__(256) void sparse_residual_kernel(SparseParams P) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const bool live = row < P.rows;
  const int lrow = live ? row : P.rows - 1;
  const VT* v = reinterpret_cast<const VT*>(P.values) + (int64_t)lrow * P.vm;
  const IT* ix = reinterpret_cast<const IT*>(P.indices) + (int64_t)lrow * P.im;
  const XT* x = reinterpret_cast<const XT*>(P.x);
  float acc = 0.0f;
  bool bad = false;
  for (int k = lane; k < P.terms; k += 64) {
    const int64_t i = (int64_t)ix[k * P.ik];
    const bool ok = i >= 0 && i < P.cols;
    bad |= !ok;
    const float xv = to_f32(x[ok ? i : 0]);
    acc = acc + to_f32(v[k * P.vk]) * xv;
  }
  acc = xor_sum(acc, 1, 64);
  // any lane's bad index poisons the row
  if (__ballot(bad)) acc = __builtin_nanf("");
  if (live && lane == 0) {
    OT* o = reinterpret_cast<OT*>(P.out) + row;
    store(o, to_f32(*o) + acc);
  }
}

struct BinaryParams {
  const uint8_t* signs;     // [rows, cols / 8] bytes, row stride bm bytes
  const void* scales;       // [rows, cols / 32], row stride sm elements
  const void* x;            // [cols], 16-byte aligned
  void* out;
  int64_t bm, sm;
  int rows, cols;
};

template <typename ST, typename XT, typename OT>
__global__ __launch_bounds__(256) void binary_residual_kernel(BinaryParams P) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const bool live = row < P.rows;
  const int lrow = live ? row : P.rows - 1;
  const uint8_t* sg = P.signs + (int64_t)lrow * P.bm;
  const ST* sc = reinterpret_cast<const ST*>(P.scales) + (int64_t)lrow * P.sm;
  const uint4* xv = reinterpret_cast<const uint4*>(P.x);
  const int groups = P.cols / 32;
  float acc = 0.0f;
  for (int g = lane; g < groups; g += 64) {
    const uint32_t bits = *reinterpret_cast<const uint32_t*>(sg + 4 * g);
    uint4 xq[4];
#pragma unroll
    for (int q = 0; q < 4; q++) xq[q] = xv[4 * g + q];
    const float s = to_f32(sc[g]);
    float p = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t w[4] = {xq[q].x, xq[q].y, xq[q].z, xq[q].w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int k = 8 * q + 2 * j;
        const float a = lo_f32<XT>(w[j]), b = hi_f32<XT>(w[j]);
        p = p + (((bits >> k) & 1u) ? a : -a);
        p = p + (((bits >> (k + 1)) & 1u) ? b : -b);
      }
    }
    acc = acc + s * p;
  }
  acc = xor_sum(acc, 1, 64);
  if (live && lane == 0) {
    OT* o = reinterpret_cast<OT*>(P.out) + row;
    store(o, to_f32(*o) + acc);
  }
}

template <typename A, typename B, typename C, typename F>
int with_out(int out_dtype, F&& f) {
  switch (out_dtype) {
    case TT_F16: return f(A{}, B{}, C{}, f16_t{});
    case TT_BF16: return f(A{}, B{}, C{}, bf16_t{});
    default: return f(A{}, B{}, C{}, float{});
  }
}

}  // namespace
}  // namespace tt

using namespace tt;

extern "C" int tt_sparse_residual_matvec(const void* values, int value_dtype, int64_t vm, int64_t vk,
                                         const void* indices, int index_bytes, int64_t im, int64_t ik,
                                         const void* x, int x_dtype, void* out, int out_dtype, int64_t rows,
                                         int64_t terms, int64_t cols, void* stream) {
  const char* what = "sparse_residual_matvec";
  TT_REQUIRE(valid_out_dtype(value_dtype) && valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype),
             "%s: bad dtype codes", what);
  TT_REQUIRE(index_bytes == 2 || index_bytes == 4 || index_bytes == 8, "%s: indices must be int16, int32 or int64",
             what);
  TT_REQUIRE(rows >= 0 && rows < (1LL << 31) && terms >= 0 && terms < (1LL << 31) && cols > 0 && cols < (1LL << 31),
             "%s: bad shape", what);
  TT_REQUIRE(values && indices && x && out, "%s: null pointer", what);
  if (rows == 0) return TT_OK;
  SparseParams P{values, indices, x, out, vm, vk, im, ik, (int)rows, (int)terms, (int)cols};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((rows + 3) / 4));
  auto go = [&](auto vt, auto it, auto xt, auto ot) {
    hipLaunchKernelGGL((sparse_residual_kernel<decltype(vt), decltype(it), decltype(xt), decltype(ot)>), grid,
                       dim3(256), 0, st, P);
    return check_launch(what);
  };
  auto by_x = [&](auto vt, auto it) {
    return x_dtype == TT_F16 ? with_out<decltype(vt), decltype(it), f16_t>(out_dtype, go)
                             : with_out<decltype(vt), decltype(it), bf16_t>(out_dtype, go);
  };
  // int16 indices (the reference runtime's sidecar layout, gpu_runtime.py:6468) are
  // sign-extended, so a negative stored index takes the out-of-range NaN rule
  auto by_i = [&](auto vt) {
    if (index_bytes == 2) return by_x(vt, int16_t{});
    return index_bytes == 4 ? by_x(vt, int32_t{}) : by_x(vt, int64_t{});
  };
  switch (value_dtype) {
    case TT_F16: return by_i(f16_t{});
    case TT_BF16: return by_i(bf16_t{});
    default: return by_i(float{});
  }
}

extern "C" int tt_binary_residual_matvec(const void* packed_signs, int64_t bm, const void* scales, int scale_dtype,
                                         int64_t sm, const void* x, int x_dtype, void* out, int out_dtype,
                                         int64_t rows, int64_t cols, void* stream) {
  const char* what = "binary_residual_matvec";
  TT_REQUIRE(valid_out_dtype(scale_dtype) && valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype),
             "%s: bad dtype codes", what);
  TT_UNSUPPORTED(cols > 0 && cols % 32 == 0 && cols < (1LL << 31), "%s: cols must be a positive multiple of 32", what);
  TT_REQUIRE(rows >= 0 && rows < (1LL << 31), "%s: bad rows", what);
  TT_REQUIRE(packed_signs && scales && x && out && aligned(packed_signs, 4) && bm % 4 == 0 && bm >= cols / 8 &&
                 sm >= cols / 32 && aligned(x, 16),
             "%s: null or misaligned pointer / bad row strides", what);
  if (rows == 0) return TT_OK;
  BinaryParams P{static_cast<const uint8_t*>(packed_signs), scales, x, out, bm, sm, (int)rows, (int)cols};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((rows + 3) / 4));
  auto go = [&](auto s, auto xt, auto, auto ot) {
    hipLaunchKernelGGL((binary_residual_kernel<decltype(s), decltype(xt), decltype(ot)>), grid, dim3(256), 0, st, P);
    return check_launch(what);
  };
  auto by_x = [&](auto s) {
    return x_dtype == TT_F16 ? with_out<decltype(s), f16_t, int>(out_dtype, go)
                             : with_out<decltype(s), bf16_t, int>(out_dtype, go);
  };
  switch (scale_dtype) {
    case TT_F16: return by_x(f16_t{});
    case TT_BF16: return by_x(bf16_t{});
    default: return by_x(float{});
  }
}
