// fp16/bf16 and fp8 GEMV entry points.
#include <mutex>

#include "gemv_lean.h"

using namespace tt;

extern "C" int tt_scaled_matvec(const void* weight, int64_t w_row_bytes, const void* scales, int scale_dtype,
                                const void* x, int x_dtype, void* out, int out_dtype, int64_t rows, int64_t cols,
                                void* stream) {
  const char* what = "scaled_matvec";
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(scale_dtype == TT_F16 || scale_dtype == TT_F32, "%s: scales must be fp16 or fp32", what);
  TT_REQUIRE(weight && aligned(weight, 16) && w_row_bytes % 16 == 0 && w_row_bytes >= cols, "%s: fp8 weights must be 16-byte aligned rows", what);
  TT_REQUIRE(x && aligned(x, 16) && scales && out, "%s: null or misaligned pointer", what);
  TT_REQUIRE(rows > 0 && rows < (1 << 30), "%s: bad rows", what);
  int L;
  bool row_mode;
  int rc = tt::plan_groups(what, cols, cols, &L, &row_mode);
  if (rc) return rc;
  GemvParams P{};
  P.nseg = 1;
  P.seg[0] = Seg{static_cast<const uint8_t*>(weight), w_row_bytes, scales, 1, 0, out, (int)rows};
  P.x = x;
  P.cols = (int)cols;
  const int Lg = 1;
  const int lpr = tt_gemv_lanes_per_row(cols / 32, 1);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (scale_dtype == TT_F32 && x_dtype == out_dtype && lean_fits(rows, w_row_bytes, 4, cols)) {
    LeanParams L{};
    L.w = static_cast<const uint8_t*>(weight);
    L.s = scales;
    L.x = x;
    L.out = out;
    L.w_row = (uint32_t)w_row_bytes;
    L.s_row = 1;
    L.rows = (int)rows;
    L.cols = (int)cols;
    return lean_launch<Fmt::kFp8, SMode::kRow, float, 1>(x_dtype, lpr, L, 1, st, what);
  }
  if (scale_dtype == TT_F16) return launch_types<Fmt::kFp8, SMode::kRow, f16_t, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
  return launch_types<Fmt::kFp8, SMode::kRow, float, 4>(x_dtype, out_dtype, Lg, lpr, P, 1, st, what);
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
  hipStream_t st = static_cast<hipStream_t>(stream);
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
