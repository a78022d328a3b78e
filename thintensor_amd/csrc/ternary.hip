// Ternary selected-expert GEMV for gfx950: grouped {-a, 0, +a} expert weights.
//
// Packed row layout (one row of one expert, row_bytes apart; the reference's packer
// gpu_runtime.py:494-583, read by triton_kernels.py:1022-1133):
//   * bytes [0, T), T = ceil(cols / 5): five base-3 digits per byte, column k at byte
//     k / 5, digit k % 5 (digit i of byte b is (b / 3^i) % 3; digit 1 means 0, digit 0
//     the negative and digit 2 the positive magnitude);
//   * bytes [T, T + ceil(3 G / 8)), G = cols / 32: a 3-bit magnitude selector m per
//     32-column group g at bit 3 g (LSB first, crossing bytes): |w| = e2m1(m + 1), i.e.
//     {0.5, 1, 1.5, 2, 3, 4, 6} for m = 0..6 and 0 for m = 7 (e2m1 code 8 is -0);
//   * E8M0 scales [E, rows, G] as a separate tensor: w = (digit - 1) * |w| * 2^(e - 127).
//
// Work split.  Five groups are exactly 32 digit bytes (lcm(5, 32) = 160 columns), so a
// lane owns whole 160-column chunks: 32 digit bytes, a 15-bit field of magnitude
// selectors and five scale bytes.  L lanes share a row (L = the smallest power of two
// >= chunks, at most 64; lanes loop over chunks j, j + L, ...), 64 / L rows per wave,
// and a workgroup walks kIter row sets per wave so the activation vector staged in
// LDS (as fp32) is reused over 4 * kIter * 64 / L rows.  Rows are not 4-byte aligned
// (row_bytes is arbitrary), so each lane reads aligned dwords that cover its bytes and
// shifts them into place; dwords that would cross the end of a buffer are assembled
// from byte loads instead.
//
// Fixed summation order (a CPU restatement reproduces every bit):
//   p_g = sum over the group's 32 columns in column order of (digit - 1) * x   (fp32);
//   acc = acc + (|w|_g * 2^(e_g - 127)) * p_g over the lane's groups in column order;
//   row = butterfly over the L lanes (lane bits in increasing order), stored rounded
//   to the output dtype.
// The reference contracts the same products on tensor cores in hardware order; this
// order is held to the dequantise-then-matmul tolerance against it.
#include "tt_abi_internal.h"
#include "tt_common.h"

namespace tt {
namespace {

constexpr int kChunk = 160;                   // columns per lane step
constexpr int kMaxCols = 8192;
constexpr int kMaxChunks = (kMaxCols + kChunk - 1) / kChunk;
constexpr int kIter = 4;                      // row sets per wave

struct TernParams {
  const uint8_t* w;         // [E, rows, row_bytes]
  const uint8_t* w_end;     // one past the last readable weight byte
  const uint8_t* s;         // E8M0 [E, rows, G]
  const uint8_t* s_end;
  const void* x;            // [cols] or [selected, cols]
  const int32_t* experts;
  void* out;                // [selected, out_slot]
  int64_t w_expert, w_row;  // bytes
  int64_t s_expert, s_row;  // bytes
  int64_t x_slot, out_slot; // elements
  int64_t n_experts;
  int rows, cols, tbytes, groups, chunks, L;
};

// Dword at a 4-byte aligned address; bytes at or past `end` read as zero.
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* a4, const uint8_t* end) {
  if (a4 + 4 <= end) return *reinterpret_cast<const uint32_t*>(a4);
  uint32_t v = 0;
#pragma unroll
  for (int i = 0; i < 4; i++)
    if (a4 + i < end) v |= (uint32_t)a4[i] << (8 * i);
  return v;
}

// 64 bits starting at byte address a (any alignment; at most 3 + 8 bytes are touched).
__device__ __forceinline__ uint64_t ld_u64_at(const uint8_t* a, const uint8_t* end) {
  const uint8_t* a4 = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(a) & ~(uintptr_t)3);
  const uint32_t sh = (uint32_t)(a - a4);
  const uint32_t d0 = ld_u32(a4, end), d1 = ld_u32(a4 + 4, end), d2 = ld_u32(a4 + 8, end);
  const uint32_t lo = __builtin_amdgcn_alignbyte(d1, d0, sh);
  const uint32_t hi = __builtin_amdgcn_alignbyte(d2, d1, sh);
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

// |w| * 2 for selector m: {1, 2, 3, 4, 6, 8, 12, 0}.
__device__ __forceinline__ float magnitude(uint32_t m) { return (float)((0x0C864321u >> (4 * m)) & 15u) * 0.5f; }

template <typename XT, typename OT>
__global__ __launch_bounds__(256) void ternary_selected_kernel(TernParams P) {
  __shared__ __attribute__((aligned(16))) float xs[kMaxChunks * kChunk];
  const int slot = blockIdx.y;
  const int64_t e = P.experts[slot];
  const bool valid_expert = e >= 0 && e < P.n_experts;
  // stage the slot's activations as fp32 (zero past cols, up to whole chunks)
  const XT* xv = reinterpret_cast<const XT*>(P.x) + (int64_t)slot * P.x_slot;
  const int padded = P.chunks * kChunk;
  for (int i = threadIdx.x; i < padded; i += 256) xs[i] = i < P.cols ? to_f32(xv[i]) : 0.0f;
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int L = P.L;
  const int per_wave = 64 / L;
  const int r_in = lane / L, j0 = lane % L;
  OT* out = reinterpret_cast<OT*>(P.out) + (int64_t)slot * P.out_slot;
  const int wg_rows = 4 * kIter * per_wave;
  for (int it = 0; it < kIter; it++) {
    const int row = blockIdx.x * wg_rows + (it * 4 + wave) * per_wave + r_in;
    const int lrow = row < P.rows ? row : P.rows - 1;
    float acc = 0.0f;
    if (valid_expert) {
      const uint8_t* wrow = P.w + e * P.w_expert + (int64_t)lrow * P.w_row;
      const uint8_t* srow = P.s + e * P.s_expert + (int64_t)lrow * P.s_row;
      for (int c = j0; c < P.chunks; c += L) {
        // 32 digit bytes at wrow + 32 c: nine aligned dwords, shifted into eight words
        const uint8_t* a = wrow + 32 * c;
        const uint8_t* a4 = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(a) & ~(uintptr_t)3);
        const uint32_t sh = (uint32_t)(a - a4);
        uint32_t d[9];
#pragma unroll
        for (int i = 0; i < 9; i++) d[i] = ld_u32(a4 + 4 * i, P.w_end);
        uint32_t wd[8];
#pragma unroll
        for (int i = 0; i < 8; i++) wd[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
        // magnitude selectors of groups 5c .. 5c+4: bits 15 c .. 15 c + 14 of the sidecar
        const int mbit = 15 * c;
        const uint64_t mw = ld_u64_at(wrow + P.tbytes + (mbit >> 3), P.w_end);
        const uint32_t mfield = (uint32_t)(mw >> (mbit & 7)) & 0x7fffu;
        const uint64_t sw = ld_u64_at(srow + 5 * c, P.s_end);
        const float* xc = xs + kChunk * c;
        float p[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int b = 0; b < 32; b++) {
          uint32_t q = (wd[b >> 2] >> (8 * (b & 3))) & 0xffu;
#pragma unroll
          for (int i = 0; i < 5; i++) {
            const uint32_t q3 = (q * 171u) >> 9;   // q / 3 for q < 256
            const int digit = (int)(q - 3u * q3);
            q = q3;
            const int t = 5 * b + i;
            p[t / 32] = p[t / 32] + (float)(digit - 1) * xc[t];
          }
        }
#pragma unroll
        for (int g = 0; g < 5; g++) {
          if (5 * c + g < P.groups) {
            const uint32_t m = (mfield >> (3 * g)) & 7u;
            const int ex = (int)((sw >> (8 * g)) & 0xffu);
            const float v = magnitude(m) * pow2i(ex - 127);
            acc = acc + v * p[g];
          }
        }
      }
    }
    acc = xor_sum(acc, 1, L);
    if (j0 == 0 && row < P.rows) store(out + row, valid_expert ? acc : __builtin_nanf(""));
  }
}

int lanes_for(int chunks) {
  int L = 1;
  while (L < chunks && L < 64) L <<= 1;
  return L;
}

template <typename XT>
int launch_out(int out_dtype, const TernParams& P, dim3 grid, hipStream_t st) {
  switch (out_dtype) {
    case TT_F16: hipLaunchKernelGGL((ternary_selected_kernel<XT, f16_t>), grid, dim3(256), 0, st, P); break;
    case TT_BF16: hipLaunchKernelGGL((ternary_selected_kernel<XT, bf16_t>), grid, dim3(256), 0, st, P); break;
    default: hipLaunchKernelGGL((ternary_selected_kernel<XT, float>), grid, dim3(256), 0, st, P); break;
  }
  return check_launch("mxfp_ternary_selected_matvec");
}

}  // namespace
}  // namespace tt

using namespace tt;

extern "C" int tt_ternary_lanes_per_row(int64_t cols) {
  if (cols <= 0) return 1;
  return lanes_for((int)((cols + kChunk - 1) / kChunk));
}

extern "C" int tt_mxfp_ternary_selected_matvec(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                               int64_t w_total_bytes, const void* scales, int64_t s_expert,
                                               int64_t s_row, int64_t s_total_bytes, int64_t experts,
                                               const void* x, int x_dtype, int64_t x_slot,
                                               const int32_t* expert_indices, int64_t selected, void* out,
                                               int out_dtype, int64_t out_slot, int64_t rows, int64_t cols,
                                               void* stream) {
  const char* what = "mxfp_ternary_selected_matvec";
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(cols > 0 && cols % 32 == 0, "%s: cols must be a positive multiple of 32", what);
  TT_UNSUPPORTED(cols <= kMaxCols, "%s: cols above %d are not supported", what, kMaxCols);
  TT_REQUIRE(rows > 0 && rows < (1 << 30) && experts >= 1, "%s: bad rows / experts", what);
  TT_REQUIRE(selected >= 1 && selected <= 65535 && expert_indices, "%s: need 1..65535 selected experts", what);
  const int64_t groups = cols / 32, tbytes = (cols + 4) / 5, mbytes = (groups * 3 + 7) / 8;
  TT_REQUIRE(w_row_bytes >= tbytes + mbytes && w_expert_bytes >= rows * w_row_bytes &&
                 w_total_bytes >= (experts - 1) * w_expert_bytes + rows * w_row_bytes,
             "%s: weight rows must hold %lld digit and %lld selector bytes", what, (long long)tbytes,
             (long long)mbytes);
  TT_REQUIRE(s_row >= groups && s_expert >= rows * s_row && s_total_bytes >= (experts - 1) * s_expert + rows * s_row,
             "%s: scale rows must hold %lld groups", what, (long long)groups);
  TT_REQUIRE(packed && scales && aligned(packed, 4) && aligned(scales, 4),
             "%s: packed weights and scales must be 4-byte aligned", what);
  TT_REQUIRE(x && out && x_slot >= 0 && (selected == 1 || out_slot >= rows), "%s: null pointer or bad strides", what);
  TernParams P{};
  P.w = static_cast<const uint8_t*>(packed);
  P.w_end = P.w + w_total_bytes;
  P.s = static_cast<const uint8_t*>(scales);
  P.s_end = P.s + s_total_bytes;
  P.x = x;
  P.experts = expert_indices;
  P.out = out;
  P.w_expert = w_expert_bytes;
  P.w_row = w_row_bytes;
  P.s_expert = s_expert;
  P.s_row = s_row;
  P.x_slot = x_slot;
  P.out_slot = out_slot;
  P.n_experts = experts;
  P.rows = (int)rows;
  P.cols = (int)cols;
  P.tbytes = (int)tbytes;
  P.groups = (int)groups;
  P.chunks = (int)((cols + kChunk - 1) / kChunk);
  P.L = lanes_for(P.chunks);
  const int wg_rows = 4 * kIter * (64 / P.L);
  const dim3 grid((unsigned)((rows + wg_rows - 1) / wg_rows), (unsigned)selected);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return x_dtype == TT_F16 ? launch_out<f16_t>(out_dtype, P, grid, st) : launch_out<bf16_t>(out_dtype, P, grid, st);
}
