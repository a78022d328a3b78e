// fp16/bf16 and fp8 GEMV entry points.
#include <mutex>

#include "gemv_lean.h"

using namespace tt;

// Byte-per-element weight formats of the scaled GEMVs: TT_W_FP8 (float8_e4m3fn) or
// TT_W_INT8 (two's-complement int8); both decode exactly to binary32.
static bool scaled_format_ok(int w_format) { return w_format == TT_W_FP8 || w_format == TT_W_INT8; }

// fp8 or int8 weights with one scale per row, scales s_stride elements apart.
template <Fmt F>
static int scaled_matvec_fmt(const void* weight, int64_t w_row_bytes, const void* scales, int scale_dtype,
                             int64_t s_stride, const void* x, int x_dtype, void* out, int out_dtype, int64_t rows,
                             int64_t cols, void* stream) {
  const char* what = "scaled_matvec";
  TT_REQUIRE(s_stride >= 1 && s_stride < (1LL << 31), "%s: bad scale stride", what);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: scales must be fp16 or fp32", what);
  TT_REQUIRE(weight && aligned(weight, 16) && w_row_bytes % 16 == 0 && w_row_bytes >= cols,
             "%s: weights must be 16-byte aligned rows", what);
  TT_REQUIRE(x && aligned(x, 16) && scales && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L;
  bool row_mode;
  int rc = tt::plan_groups(what, cols, cols, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight), w_row_bytes, scales, s_stride, 0, out, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  const int Lg = 1;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (scale_dtype == TT_F32 && x_dtype == out_dtype && lean_fits(rows, w_row_bytes, 4 * s_stride, cols)) {
    LeanParams L{};
    L.w = static_cast<const uint8_t*>(weight);
    L.s = scales;
    L.x = x;
    L.out = out;
    L.w_row = (uint32_t)w_row_bytes;
    L.s_row = (uint32_t)s_stride;
    L.rows = (int)rows;
    L.cols = (int)cols;
    return lean_launch<F, SMode::kRow, float, 1>(x_dtype, lpr, L, 1, st, what);
  }
  if (scale_dtype == TT_F16) return launch_types<F, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  return launch_types<F, SMode::kRow, float, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
}

static int scaled_matvec_impl(const void* weight, int w_format, int64_t w_row_bytes, const void* scales,
                              int scale_dtype, int64_t s_stride, const void* x, int x_dtype, void* out, int out_dtype,
                              int64_t rows, int64_t cols, void* stream) {
  TT_REQUIRE(scaled_format_ok(w_format), "scaled_matvec: weights must be float8_e4m3fn or int8 (format %d)", w_format);
  if (w_format == TT_W_INT8)
    return scaled_matvec_fmt<Fmt::kInt8>(weight, w_row_bytes, scales, scale_dtype, s_stride, x, x_dtype, out,
                                         out_dtype, rows, cols, stream);
  return scaled_matvec_fmt<Fmt::kFp8>(weight, w_row_bytes, scales, scale_dtype, s_stride, x, x_dtype, out, out_dtype,
                                      rows, cols, stream);
}

extern "C" int tt_scaled_matvec(const void* weight, int w_format, int64_t w_row_bytes, const void* scales,
                                int scale_dtype, const void* x, int x_dtype, void* out, int out_dtype, int64_t rows,
                                int64_t cols, void* stream) {
  return scaled_matvec_impl(weight, w_format, w_row_bytes, scales, scale_dtype, 1, x, x_dtype, out, out_dtype, rows,
                            cols, stream);
}

extern "C" int tt_multi_matvec_bias(int count, const void* const* weights, int w_dtype, const int64_t* w_row,
                                    const int64_t* rows, const void* const* biases, const void* x, int x_dtype,
                                    void* out, int out_dtype, int64_t cols, void* stream) {
  const char* what = "matvec";
  TT_REQUIRE(count >= 1 && count <= 3, "%s: supports one to three matrices", what);
  TT_REQUIRE(w_dtype == TT_F16 || w_dtype == TT_BF16, "%s: weights must be fp16 or bf16", what);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(x && aligned(x, 16) && out, "%s: null or misaligned pointer", what);
  int L;
  bool row_mode;
  int rc = tt::plan_groups(what, cols, cols, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = count;
  int64_t acc_rows = 0;
  const size_t osz = out_dtype == TT_F32 ? 4 : 2;
  for (int i = 0; i < count; i++) {
    TT_REQUIRE(rows[i] > 0, "%s: rows must be positive", what);
    TT_REQUIRE(weights[i] && aligned(weights[i], 16) && (w_row[i] * 2) % 16 == 0 && w_row[i] >= cols,
               "%s: weights must be 16-byte aligned with a row stride that is a multiple of 8 elements", what);
    P.seg[i] = Seg{static_cast<const uint8_t*>(weights[i]), w_row[i] * 2, nullptr, 0, 0,
                   static_cast<char*>(out) + acc_rows * osz, (int)rows[i], 0, biases ? biases[i] : nullptr};
    acc_rows += rows[i];
  }
  TT_REQUIRE(acc_rows < (1LL << 30), "%s: too many rows", what);
  P.x = x;
  P.cols = (int)cols;
  const int Lg = 1;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (count == 1 && x_dtype == out_dtype && lean_fits(rows[0], w_row[0] * 2, 0, cols)) {
    LeanParams L{};
    L.w = static_cast<const uint8_t*>(weights[0]);
    L.x = x;
    L.out = out;
    L.bias = biases ? biases[0] : nullptr;
    L.w_row = (uint32_t)(w_row[0] * 2);
    L.rows = (int)rows[0];
    L.cols = (int)cols;
    if (w_dtype == TT_F16) return lean_launch<Fmt::kF16W, SMode::kNone, float, 1>(x_dtype, lpr, L, 1, st, what);
    return lean_launch<Fmt::kBF16W, SMode::kNone, float, 1>(x_dtype, lpr, L, 1, st, what);
  }
  if (w_dtype == TT_F16) return launch_types<Fmt::kF16W, SMode::kNone, float, 2>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  return launch_types<Fmt::kBF16W, SMode::kNone, float, 2>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
}

extern "C" int tt_matvec_bias_rows(const void* weight, int w_dtype, int64_t w_row, const void* bias, const void* x,
                                   int x_dtype, int64_t x_row, void* out, int out_dtype, int64_t out_row, int64_t m,
                                   int64_t rows, int64_t cols, void* stream) {
  const char* what = "matvec_bias_rows";
  TT_REQUIRE(m >= 1 && m <= 65535, "%s: 1 to 65535 activation rows", what);
  TT_REQUIRE(weight && x && out && rows > 0 && cols > 0 && cols % 32 == 0, "%s: bad arguments", what);
  TT_REQUIRE(w_dtype == TT_F16 || w_dtype == TT_BF16, "%s: weights must be fp16 or bf16", what);
  const int64_t xsz = x_dtype == TT_F32 ? 4 : 2, osz = out_dtype == TT_F32 ? 4 : 2;
  const bool one_launch = m > 1 && x_dtype == out_dtype && x_dtype != TT_F32 && aligned(weight, 16) &&
                          (w_row * 2) % 16 == 0 && w_row >= cols && aligned(x, 16) && x_row % 8 == 0 &&
                          x_row >= cols && out_row >= rows && lean_fits(rows, w_row * 2, 0, cols);
  if (!one_launch) {
    // the single-row operator per activation row
    for (int64_t t = 0; t < m; t++) {
      const void* w_arr[1] = {weight};
      const int64_t wr[1] = {w_row};
      const int64_t r[1] = {rows};
      const void* b_arr[1] = {bias};
      const int rc = tt_multi_matvec_bias(1, w_arr, w_dtype, wr, r, b_arr, static_cast<const char*>(x) + t * x_row * xsz,
                                          x_dtype, static_cast<char*>(out) + t * out_row * osz, out_dtype, cols, stream);
      if (rc != TT_OK) return rc;
    }
    return TT_OK;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (w_dtype == TT_F16 && x_dtype == TT_F16 && cols <= 4096)   // eight activation rows in 64 KB of LDS
    return dense_bias_rows_f16(weight, w_row, bias, x, x_row, out, out_row, m, rows, cols, st);
  // rows of the batch are slots of the lean kernel (blockIdx.y), each with its own
  // activation and output row; the arithmetic per row is the single-row kernel's
  LeanParams L{};
  L.w = static_cast<const uint8_t*>(weight);
  L.x = x;
  L.out = out;
  L.bias = bias;
  L.x_slot = x_row;
  L.out_slot = out_row;
  L.w_row = (uint32_t)(w_row * 2);
  L.rows = (int)rows;
  L.cols = (int)cols;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  if (w_dtype == TT_F16) return lean_launch<Fmt::kF16W, SMode::kNone, float, 1>(x_dtype, lpr, L, (int)m, st, what);
  return lean_launch<Fmt::kBF16W, SMode::kNone, float, 1>(x_dtype, lpr, L, (int)m, st, what);
}

extern "C" int tt_multi_matvec(int count, const void* const* weights, int w_dtype, const int64_t* w_row,
                               const int64_t* rows, const void* x, int x_dtype, void* out, int out_dtype,
                               int64_t cols, void* stream) {
  return tt_multi_matvec_bias(count, weights, w_dtype, w_row, rows, nullptr, x, x_dtype, out, out_dtype, cols, stream);
}

extern "C" int tt_matvec(const void* weight, int w_dtype, int64_t w_row, const void* x, int x_dtype, void* out,
                         int out_dtype, int64_t rows, int64_t cols, void* stream) {
  const void* w_arr[1] = {weight};
  const int64_t wr[1] = {w_row};
  const int64_t r[1] = {rows};
  return tt_multi_matvec(1, w_arr, w_dtype, wr, r, x, x_dtype, out, out_dtype, cols, stream);
}


namespace {

__global__ __launch_bounds__(256) void argmax_finish_kernel(const uint64_t* partials, int n, int64_t* out_idx,
                                                            float* out_val) {
  __shared__ uint64_t red[4];
  const uint64_t k = block_max_u64(partials, n, red);
  if (threadIdx.x == 0) {
    const uint32_t o = (uint32_t)(k >> 32);
    const uint32_t bits = o == 0xffffffffu ? 0x7fc00000u : ((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
    out_idx[0] = (int64_t)(0xffffffffu - (uint32_t)k);
    if (out_val) out_val[0] = __builtin_bit_cast(float, bits);
  }
}

}  // namespace

// Number of uint64 partials tt_matvec_argmax needs for a matrix of `rows` x `cols`.
extern "C" int64_t tt_matvec_argmax_partials(int64_t rows, int64_t cols) {
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  if (lpr <= 0 || rows <= 0) return 0;
  const int64_t per_iter = 2 * (64 / lpr);
  const int64_t batches = (rows + per_iter - 1) / per_iter;
  int64_t blocks = (batches + 3) / 4;
  if (blocks < 1) blocks = 1;
  if (blocks > kMaxGemvBlocks) blocks = kMaxGemvBlocks;
  return 4 * blocks;
}

// Greedy lm_head: logits = round(W x) (optionally stored), token = first index of
// the maximum rounded logit, written as int64 to out_idx (and the value to out_val).
extern "C" int tt_matvec_argmax(const void* weight, int w_dtype, int64_t w_row, const void* x, int x_dtype,
                                void* logits, int logits_dtype, int64_t rows, int64_t cols, uint64_t* partials,
                                int64_t partials_capacity, int64_t* out_idx, float* out_val, void* stream) {
  const char* what = "matvec_argmax";
  TT_REQUIRE(w_dtype == TT_F16 || w_dtype == TT_BF16, "%s: weights must be fp16 or bf16", what);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(logits_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(weight && aligned(weight, 16) && (w_row * 2) % 16 == 0 && w_row >= cols, "%s: bad weight layout", what);
  TT_REQUIRE(x && aligned(x, 16) && partials && out_idx, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1LL << 31), "%s: bad rows", what);
  int L;
  bool row_mode;
  int rc = tt::plan_groups(what, cols, cols, &L, &row_mode);
  if (rc) return rc;
  const int64_t need = tt_matvec_argmax_partials(rows, cols);
  TT_REQUIRE(partials_capacity >= need, "%s: partials buffer needs %lld entries", what, (long long)need);
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight), w_row * 2, nullptr, 0, 0, logits, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  P.am_partials = partials;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int Lg = 1;
  if (w_dtype == TT_F16) rc = launch_types<Fmt::kF16W, SMode::kNone, float, 2>(x_dtype, logits_dtype, Lg, lpr, P, 1, st, what);
  else rc = launch_types<Fmt::kBF16W, SMode::kNone, float, 2>(x_dtype, logits_dtype, Lg, lpr, P, 1, st, what);
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_finish_kernel, dim3(1), dim3(256), 0, st, partials, (int)need, out_idx, out_val);
  return check_launch(what);
}

// ------------------------------------------------------------------ no-allocation lm_head
//
// tt_matvec_argmax with its argmax partials in a file-scope device array instead of a
// caller workspace, for callers that cannot allocate device memory.  The array holds
// kNoAllocArgmaxKeys keys (64 KiB), the most any shape can ask for: the grid is capped at
// kMaxGemvBlocks workgroups of four waves and every wave writes its key in each call, so
// nothing needs clearing between calls.  Each GPU holds its own copy until the process
// ends; calls that overlap on one GPU share it and race.

namespace {

constexpr int kNoAllocArgmaxKeys = TT_NOALLOC_ARGMAX_KEYS;
static_assert(kNoAllocArgmaxKeys >= kMaxGemvWaves, "argmax scratch must hold one key per wave of the largest grid");

static __device__ __align__(256) uint64_t scratch[kNoAllocArgmaxKeys];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
uint64_t* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device, resolved once per device with that
// device current (each GPU holds its own copy at its own address).
int scratch_for_current_device(const char* what, uint64_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  TT_REQUIRE(e == hipSuccess && dev >= 0 && dev < kMaxScratchDevices, "%s: no usable current device", what);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev, hipGetErrorString(e));
      return TT_ERR_HIP;
    }
    g_scratch_ptr[dev] = static_cast<uint64_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return TT_OK;
}

}  // namespace

extern "C" int tt_matvec_argmax_noalloc(const void* weight, int w_dtype, int64_t w_row, const void* x, int x_dtype,
                                        void* logits, int logits_dtype, int64_t rows, int64_t cols, int64_t* out_idx,
                                        float* out_val, void* stream) {
  const char* what = "matvec_argmax_noalloc";
  TT_REQUIRE(rows > 0 && rows < (1LL << 31) && cols > 0, "%s: bad shape", what);
  const int64_t need = tt_matvec_argmax_partials(rows, cols);
  TT_REQUIRE(need <= kNoAllocArgmaxKeys, "%s: %lld argmax partials exceed the %d-key scratch", what, (long long)need,
             kNoAllocArgmaxKeys);
  uint64_t* ptr = nullptr;
  int rc = scratch_for_current_device(what, &ptr);
  if (rc) return rc;
  return tt_matvec_argmax(weight, w_dtype, w_row, x, x_dtype, logits, logits_dtype, rows, cols, ptr,
                          kNoAllocArgmaxKeys, out_idx, out_val, stream);
}

// ------------------------------------------------------------------ fp8 with block scales
//
// y[m] = sum_b s[m, b] * sum_{k in block b} w[m, k] x[k], blocks of `block` columns (a
// power of two; the last one may be partial) (triton_kernels.py:3113-3152, wrapper
// :4465-4497).  A block is a group of block / 32 chunks in the group-scale reduction
// order; a block as wide as the row is the per-row-scale GEMV.

template <Fmt F>
static int block_scaled_fmt(const void* weight, int w_format, int64_t w_row_bytes, const void* scales, int scale_dtype,
                            int64_t s_row, int64_t s_block, int64_t block, const void* x, int x_dtype, void* out,
                            int out_dtype, int64_t rows, int64_t cols, void* stream) {
  const char* what = "block_scaled_matvec";
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: scales must be fp16 or fp32", what);
  TT_REQUIRE(weight && aligned(weight, 16) && w_row_bytes % 16 == 0 && w_row_bytes >= cols,
             "%s: weights must be 16-byte aligned rows", what);
  TT_REQUIRE(x && aligned(x, 16) && scales && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  TT_REQUIRE(cols > 0 && cols % 32 == 0 && cols <= 32768, "%s: cols must be a positive multiple of 32 up to 32768",
             what);
  TT_REQUIRE(block > 0 && (block & (block - 1)) == 0, "%s: the scale block must be a power of two", what);
  TT_REQUIRE(s_row >= (cols + block - 1) / block || block >= cols, "%s: scale rows too short", what);
  if (block >= cols)   // one block per row: the per-row-scale GEMV (s_row is the row stride)
    return scaled_matvec_impl(weight, w_format, w_row_bytes, scales, scale_dtype, s_row, x, x_dtype, out, out_dtype,
                              rows, cols, stream);
  TT_UNSUPPORTED(block >= 32 && block <= 2048, "%s: scale blocks of %lld columns (32 to 2048 supported)", what,
                 (long long)block);
  const int L = (int)(block / 32);
  const int lpr = tt_gemv_lanes_per_row(cols / 32, L);
  TT_REQUIRE(lpr > 0, "%s: no lane layout for blocks of %lld columns", what, (long long)block);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (scale_dtype == TT_F32 && x_dtype == out_dtype && lean_group_ok(L) &&
      lean_fits(rows, w_row_bytes, 4 * s_row, cols) && s_row < (1LL << 31) && s_block < (1LL << 31)) {
    LeanParams Lp{};
    Lp.w = static_cast<const uint8_t*>(weight);
    Lp.s = scales;
    Lp.x = x;
    Lp.out = out;
    Lp.w_row = (uint32_t)w_row_bytes;
    Lp.s_row = (uint32_t)s_row;
    Lp.s_grp = (uint32_t)s_block;
    Lp.rows = (int)rows;
    Lp.cols = (int)cols;
    return lean_launch_group<F, SMode::kGroup, float>(L, x_dtype, lpr, Lp, 1, st, what);
  }
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight), w_row_bytes, scales, s_row, s_block, out, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  if (scale_dtype == TT_F16)
    return launch_types<F, SMode::kGroup, f16_t, 2>(x_dtype, out_dtype, L, lpr, P, 1, st, what);
  return launch_types<F, SMode::kGroup, float, 2>(x_dtype, out_dtype, L, lpr, P, 1, st, what);
}

extern "C" int tt_block_scaled_matvec(const void* weight, int w_format, int64_t w_row_bytes, const void* scales,
                                      int scale_dtype, int64_t s_row, int64_t s_block, int64_t block, const void* x,
                                      int x_dtype, void* out, int out_dtype, int64_t rows, int64_t cols,
                                      void* stream) {
  TT_REQUIRE(scaled_format_ok(w_format), "block_scaled_matvec: weights must be float8_e4m3fn or int8 (format %d)",
             w_format);
  if (w_format == TT_W_INT8)
    return block_scaled_fmt<Fmt::kInt8>(weight, w_format, w_row_bytes, scales, scale_dtype, s_row, s_block, block, x,
                                        x_dtype, out, out_dtype, rows, cols, stream);
  return block_scaled_fmt<Fmt::kFp8>(weight, w_format, w_row_bytes, scales, scale_dtype, s_row, s_block, block, x,
                                     x_dtype, out, out_dtype, rows, cols, stream);
}

// ------------------------------------------------------------------ several fp8 matrices

// Two or three fp8 matrices with per-row scales over one activation vector, outputs
// concatenated in matrix order (triton_kernels.py:1958-2071, wrapper :5119-5180).  Each
// row has the single-matrix reduction order.
extern "C" int tt_multi_scaled_matvec(int count, const void* const* weights, int w_format,
                                      const int64_t* w_row_bytes, const void* const* scales, int scale_dtype,
                                      const int64_t* s_stride, const int64_t* rows, const void* x, int x_dtype,
                                      void* out, int out_dtype, int64_t cols, void* stream) {
  const char* what = "multi_scaled_matvec";
  TT_REQUIRE(count >= 1 && count <= 3, "%s: supports one to three matrices", what);
  TT_REQUIRE(scaled_format_ok(w_format), "%s: weights must be float8_e4m3fn or int8 (format %d)", what, w_format);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: scales must be fp16 or fp32", what);
  TT_REQUIRE(x && aligned(x, 16) && out && weights && scales && rows && w_row_bytes && s_stride,
             "%s: null or misaligned pointer", what);
  int L;
  bool row_mode;
  int rc = tt::plan_groups(what, cols, cols, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = count;
  int64_t acc_rows = 0;
  const size_t osz = out_dtype == TT_F32 ? 4 : 2;
  for (int i = 0; i < count; i++) {
    TT_REQUIRE(rows[i] > 0 && weights[i] && scales[i], "%s: matrix %d is empty or null", what, i);
    TT_REQUIRE(aligned(weights[i], 16) && w_row_bytes[i] % 16 == 0 && w_row_bytes[i] >= cols,
               "%s: weights must be 16-byte aligned rows", what);
    TT_REQUIRE(s_stride[i] >= 1, "%s: bad scale stride", what);
    P.seg[i] = Seg{static_cast<const uint8_t*>(weights[i]), w_row_bytes[i], scales[i], s_stride[i], 0,
                   static_cast<char*>(out) + acc_rows * osz, (int)rows[i]};
    acc_rows += rows[i];
  }
  TT_REQUIRE(acc_rows < (1LL << 30), "%s: too many rows", what);
  P.x = x;
  P.cols = (int)cols;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (w_format == TT_W_INT8) {
    if (scale_dtype == TT_F16)
      return launch_types<Fmt::kInt8, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, 1, lpr, P, 1, st, what);
    return launch_types<Fmt::kInt8, SMode::kRow, float, 4>(x_dtype, out_dtype, 1, lpr, P, 1, st, what);
  }
  if (scale_dtype == TT_F16) return launch_types<Fmt::kFp8, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, 1, lpr, P, 1, st, what);
  return launch_types<Fmt::kFp8, SMode::kRow, float, 4>(x_dtype, out_dtype, 1, lpr, P, 1, st, what);
}

// ------------------------------------------------------------------ split-K

namespace {

// y[m] = (((0 + p_0[m]) + p_1[m]) + ...) * s[m], binary32, splits in order.
template <typename OT, typename ST>
__global__ __launch_bounds__(256) void split_k_reduce_kernel(const float* partials, int splits, int rows,
                                                             const void* scales, void* out) {
  const int m = blockIdx.x * 256 + threadIdx.x;
  if (m >= rows) return;
  float acc = 0.0f;
  for (int s = 0; s < splits; s++) acc = acc + partials[(int64_t)s * rows + m];
  if (scales != nullptr) acc = acc * to_f32(reinterpret_cast<const ST*>(scales)[m]);
  store<OT>(reinterpret_cast<OT*>(out) + m, acc);
}

template <Fmt F>
int split_k_partials(const void* weight, int64_t w_row_bytes, const void* x, int x_dtype, float* partials,
                     int64_t rows, int64_t col0, int64_t width, int slots, int64_t slot_cols, int64_t slot0,
                     hipStream_t st, const char* what) {
  constexpr int B = FmtInfo<F>::kBytes;
  const int64_t xsz = 2, wsz = B / 32;   // bytes per activation / weight element
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight) + col0 * wsz, w_row_bytes, nullptr, 0, 0,
                 partials + slot0 * rows, (int)rows};
  P.x = static_cast<const char*>(x) + col0 * xsz;
  P.x_slot = slot_cols;
  P.w_slot = slot_cols * wsz;
  P.out_slot = rows;
  P.cols = (int)width;
  const int lpr = tt_gemv_lanes_per_row(width / 32, 1);
  return launch_types<F, SMode::kNone, float, 4>(x_dtype, TT_F32, 1, lpr, P, slots, st, what);
}

}  // namespace

// Split-K GEMV (triton_kernels.py:3023-3100, wrapper :3773-3845): the K axis is cut into
// `split_k` slices of q = ceil(K / 32 / split_k) whole 32-column chunks (the last slice
// may be shorter or empty); slice s writes its binary32 row sums to partials[s, :] in the
// single-matrix reduction order of its width, then one kernel adds the slices in order
// and applies the optional per-row scale.  w_format: TT_F16 / TT_BF16 dense, or
// TT_W_FP8 / TT_W_INT8 (float8_e4m3fn / int8, then `scales` are the per-row fp32/fp16
// scales).
extern "C" int tt_split_k_matvec(const void* weight, int w_format, int64_t w_row_bytes, const void* scales,
                                 int scale_dtype, const void* x, int x_dtype, void* out, int out_dtype, int64_t rows,
                                 int64_t cols, int split_k, float* partials, int64_t partials_capacity, void* stream) {
  const char* what = "split_k_matvec";
  TT_REQUIRE(split_k == 2 || split_k == 4 || split_k == 8, "%s: split_k must be 2, 4, or 8", what);
  TT_REQUIRE(w_format == TT_F16 || w_format == TT_BF16 || scaled_format_ok(w_format), "%s: bad weight format", what);
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scales == nullptr || scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: bad scale dtype", what);
  TT_REQUIRE(weight && aligned(weight, 16) && w_row_bytes % 16 == 0 && x && aligned(x, 16) && out && partials,
             "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  TT_REQUIRE(cols > 0 && cols % 32 == 0 && cols <= 32768, "%s: cols must be a positive multiple of 32 up to 32768",
             what);
  TT_REQUIRE(partials_capacity >= split_k * rows, "%s: partials need %lld floats", what, (long long)(split_k * rows));
  const int64_t nchunks = cols / 32;
  const int64_t q = (nchunks + split_k - 1) / split_k;
  const int64_t full = nchunks / q;                   // slices of q chunks
  const int64_t rem = nchunks - full * q;             // chunks of the last, shorter slice
  const int used = (int)(full + (rem > 0 ? 1 : 0));   // slices that own columns
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto partial = [&](int64_t col0, int64_t width, int slots, int64_t slot0) {
    if (w_format == TT_F16)
      return split_k_partials<Fmt::kF16W>(weight, w_row_bytes, x, x_dtype, partials, rows, col0, width, slots,
                                         width, slot0, st, what);
    if (w_format == TT_BF16)
      return split_k_partials<Fmt::kBF16W>(weight, w_row_bytes, x, x_dtype, partials, rows, col0, width, slots,
                                          width, slot0, st, what);
    if (w_format == TT_W_INT8)
      return split_k_partials<Fmt::kInt8>(weight, w_row_bytes, x, x_dtype, partials, rows, col0, width, slots, width,
                                          slot0, st, what);
    return split_k_partials<Fmt::kFp8>(weight, w_row_bytes, x, x_dtype, partials, rows, col0, width, slots, width,
                                       slot0, st, what);
  };
  int rc = partial(0, q * 32, (int)full, 0);
  if (rc == TT_OK && rem > 0) rc = partial(full * q * 32, rem * 32, 1, full);
  if (rc) return rc;
  const dim3 grid((unsigned)((rows + 255) / 256));
  auto reduce = [&](auto ot, auto sdt) {
    hipLaunchKernelGGL((split_k_reduce_kernel<decltype(ot), decltype(sdt)>), grid, dim3(256), 0, st, partials, used,
                       (int)rows, scales, out);
    return check_launch(what);
  };
  auto by_out = [&](auto sdt) {
    if (out_dtype == TT_F16) return reduce(f16_t{}, sdt);
    if (out_dtype == TT_BF16) return reduce(bf16_t{}, sdt);
    return reduce(float{}, sdt);
  };
  return scale_dtype == TT_F16 && scales != nullptr ? by_out(f16_t{}) : by_out(float{});
}
