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
// Work split.  Five groups are exactly 32 digit bytes (lcm(5, 32) = 160 columns), so
// the unit of work is an item = (two consecutive rows, 160-column chunk): per row 32
// digit bytes, a 15-bit field of magnitude selectors and five scale bytes.  A workgroup
// of 128 threads owns `rpw` rows of one selected slot and hands its items to its
// threads in turn; every activation read from LDS feeds both rows' chains.  The slot's
// activations are staged once per workgroup in LDS as fp32, together with the group
// sums of x and a 256-entry table that expands a digit byte into its five digits as
// bytes (read back with v_cvt_f32_ubyte).  Rows are not 4-byte aligned (row_bytes is
// arbitrary), so each item reads aligned dwords that cover its bytes and shifts them
// into place (reads are clamped to each buffer's last aligned dword).
//
// Fixed summation order (a CPU restatement reproduces every bit), all binary32:
//   A_g = sum over the group's 32 columns in order of digit * x   (fma chain, exact
//         products), B_g = sum of the group's x in order, p_g = A_g - B_g
//         (so p_g sums (digit - 1) * x);
//   chunk = sum over the chunk's groups in order of (|w|_g * 2^(e_g - 127)) * p_g;
//   row = sum of the row's chunks in order, stored rounded to the output dtype.
// The reference contracts the same products on tensor cores in hardware order; this
// order is held to the dequantise-then-matmul tolerance against it.
#include "tt_abi_internal.h"
#include "tt_common.h"

namespace tt {
namespace {

constexpr int kChunk = 160;                   // columns per item
// LDS floats per chunk of staged activations: 160 plus a 16-byte pad.  Neighbouring
// threads take neighbouring chunks, so at a stride of 160 floats every lane of a wave
// read the same one or two banks (bank-conflict cycles 8x the LDS-active cycles);
// 164 spreads the chunks over the banks and keeps 16-byte alignment (gate/up
// 17.6 -> 15.5 us, down 12.7 -> 11.6 us; 161 floats, unaligned, was slower).
constexpr int kXS = 164;
constexpr int kMaxCols = 8192;
constexpr int kThreads = 128;
// Measured at the gpt-oss expert shapes (gate/up 5760 x 2880, down 2880 x 2880, four
// slots): two rows per item with one item's loads in flight (21.2 / 13.5 us) beat one row
// per item with two (24.2 / 15.2 us), three (23.9 / 15.8 us), and four rows per item
// (24.8 / 21.3 us: occupancy 2).  The activation reads from LDS are the main cost; an
// item's reads feed every row of the item.  One item per thread (rows per workgroup from
// the chunk count, no item loop) took gate/up to 17.7 us (16 rows per workgroup made 144
// items, a second loop pass with its own memory round trip for 16 threads) and down to
// 13.1 us; requesting the items' words before the activation staging was slower (20.1 /
// 14.5 us).
constexpr int kRowsPerItem = 2;
constexpr int kBatch = 1;                     // items whose loads are in flight together

struct TernParams {
  const uint8_t* w;         // [E, rows, row_bytes]
  const uint8_t* w_end;     // one past the last readable weight byte
  const uint8_t* s;         // E8M0 [E, rows, G]
  const uint8_t* s_end;
  const void* x;            // [cols] or [selected, cols]
  const void* experts;   // int32 (ishift 0) or int64 (ishift 1) ids
  int ishift;
  void* out;                // [selected, out_slot]
  int64_t w_expert, w_row;  // bytes
  int64_t s_expert, s_row;  // bytes
  int64_t x_slot, out_slot; // elements
  int64_t n_experts;
  int rows, cols, tbytes, groups, chunks, rpw;
};

// Aligned dword at a4, or the buffer's last aligned dword if a4 lies past it.  An
// aligned dword that holds at least one byte of the buffer lies in the same memory
// page as that byte, so this read cannot fault; its bytes past the buffer's end only
// feed groups past `groups`, whose sums are never used.
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* a4, const uint8_t* last4) {
  return *reinterpret_cast<const uint32_t*>(a4 < last4 ? a4 : last4);
}

// Round down to 4 bytes by pointer arithmetic (keeps the global address space).
__device__ __forceinline__ const uint8_t* align4(const uint8_t* a) {
  return a - (reinterpret_cast<uintptr_t>(a) & 3u);
}

// |w| * 2 for selector m: {1, 2, 3, 4, 6, 8, 12, 0}.
__device__ __forceinline__ float magnitude(uint32_t m) { return (float)((0x0C864321u >> (4 * m)) & 15u) * 0.5f; }

// One row's share of an item.
struct ItemRow {
  uint32_t d[9];   // dwords covering the 32 digit bytes
  uint32_t m[3];   // dwords covering the selector field
  uint32_t s[3];   // dwords covering the five scale bytes
  uint32_t shd, shm, shs;
};

// RP rows per item: the item's activation reads from LDS feed the fma chains of RP
// rows (each chain in the single-row order).
template <typename XT, typename OT, int RP>
__global__ __launch_bounds__(kThreads) void ternary_selected_kernel(TernParams P) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float* xs = smem;                                     // chunks * kXS (zero past cols, pads unused)
  float* bsum = xs + P.chunks * kXS;                    // chunks * 5 group sums
  float* part = bsum + P.chunks * 5 + ((P.chunks * 5) & 1);   // rpw * chunks item sums (8-byte aligned end)
  uint2* dlut = reinterpret_cast<uint2*>(part + P.rpw * P.chunks + ((P.rpw * P.chunks) & 1));
  const int slot = blockIdx.y;
  const int row0 = blockIdx.x * P.rpw;
  const int nrows = P.rows - row0 < P.rpw ? P.rows - row0 : P.rpw;
  OT* out = reinterpret_cast<OT*>(P.out) + (int64_t)slot * P.out_slot + row0;
  const int64_t e = load_expert(P.experts, P.ishift, slot);
  const XT* xv = reinterpret_cast<const XT*>(P.x) + (int64_t)slot * P.x_slot;
  // 16-byte activation loads, four per thread in flight (cols is a multiple of 32 and
  // the slot's row is 16-byte aligned), then zeros up to whole chunks.  The first four
  // go out with the expert id, before the id is tested.
  const int nvec = P.cols / 8;
  uint4 t0[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const int v = (int)threadIdx.x + u * kThreads < nvec ? (int)threadIdx.x + u * kThreads : nvec - 1;
    t0[u] = reinterpret_cast<const uint4*>(xv)[v];
  }
  if (e < 0 || e >= P.n_experts) {                      // uniform over the workgroup
    for (int r = threadIdx.x; r < nrows; r += kThreads) store(out + r, __builtin_nanf(""));
    return;
  }
  for (int v0 = threadIdx.x; v0 < nvec; v0 += 4 * kThreads) {
    uint4 t[4];
    if (v0 == (int)threadIdx.x) {
#pragma unroll
      for (int u = 0; u < 4; u++) t[u] = t0[u];
    } else {
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int v = v0 + u * kThreads < nvec ? v0 + u * kThreads : nvec - 1;
        t[u] = reinterpret_cast<const uint4*>(xv)[v];
      }
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int v = v0 + u * kThreads;
      if (v < nvec) {
        const uint32_t wv[4] = {t[u].x, t[u].y, t[u].z, t[u].w};
        const int pv = (8 * v / kChunk) * kXS + 8 * v % kChunk;   // eight columns never cross a chunk
#pragma unroll
        for (int j = 0; j < 4; j++) {
          xs[pv + 2 * j] = lo_f32<XT>(wv[j]);
          xs[pv + 2 * j + 1] = hi_f32<XT>(wv[j]);
        }
      }
    }
  }
  const int padded = P.chunks * kChunk;
  for (int i = P.cols + threadIdx.x; i < padded; i += kThreads) xs[(i / kChunk) * kXS + i % kChunk] = 0.0f;
  for (int b = threadIdx.x; b < 256; b += kThreads) {
    uint32_t q = (uint32_t)b, lo = 0, hi = 0;
    for (int i = 0; i < 5; i++) {
      const uint32_t q3 = q / 3u, dg = q - 3u * q3;
      if (i < 4) lo |= dg << (8 * i);
      else hi = dg;
      q = q3;
    }
    dlut[b] = make_uint2(lo, hi);
  }
  __syncthreads();
  for (int g = threadIdx.x; g < P.chunks * 5; g += kThreads) {
    float b = 0.0f;
    const float* xg = xs + (g / 5) * kXS + 32 * (g % 5);
    for (int k = 0; k < 32; k++) b = b + xg[k];
    bsum[g] = b;
  }
  __syncthreads();
  // this thread's item (the host keeps a workgroup's items within its threads)
  const uint8_t* wlast = align4(P.w_end - 1);
  const uint8_t* slast = align4(P.s_end - 1);
  const uint8_t* wexp = P.w + e * P.w_expert;
  const uint8_t* sexp = P.s + e * P.s_expert;
  // items: (RP consecutive rows, chunk); the last item's missing rows read the last row
  const int rgroups = (nrows + RP - 1) / RP;
  const int items = rgroups * P.chunks;
  const int base = threadIdx.x;
  ItemRow it[kBatch][RP];
  int mbit[kBatch];
#pragma unroll
  for (int u = 0; u < kBatch; u++) {
    int item = base + u * kThreads;
    item = item < items ? item : items - 1;
    const int rg = item / P.chunks, c = item - rg * P.chunks;
    const int mb = 15 * c;
    mbit[u] = mb & 7;
#pragma unroll
    for (int k = 0; k < RP; k++) {
      const int r = RP * rg + k < nrows ? RP * rg + k : nrows - 1;
      ItemRow& ir = it[u][k];
      const uint8_t* wrow = wexp + (int64_t)(row0 + r) * P.w_row;
      const uint8_t* a = wrow + 32 * c;
      const uint8_t* a4 = align4(a);
      ir.shd = (uint32_t)(a - a4);
#pragma unroll
      for (int i = 0; i < 9; i++) ir.d[i] = ld_u32(a4 + 4 * i, wlast);
      const uint8_t* ma = wrow + P.tbytes + (mb >> 3);
      const uint8_t* ma4 = align4(ma);
      ir.shm = (uint32_t)(ma - ma4);
#pragma unroll
      for (int i = 0; i < 3; i++) ir.m[i] = ld_u32(ma4 + 4 * i, wlast);
      const uint8_t* sa = sexp + (int64_t)(row0 + r) * P.s_row + 5 * c;
      const uint8_t* sa4 = align4(sa);
      ir.shs = (uint32_t)(sa - sa4);
#pragma unroll
      for (int i = 0; i < 3; i++) ir.s[i] = ld_u32(sa4 + 4 * i, slast);
    }
  }

  {
#pragma unroll
    for (int u = 0; u < kBatch; u++) {
      const int item = base + u * kThreads;
      if (item >= items) break;
      const int rg = item / P.chunks, c = item - rg * P.chunks;
      const float* xc = xs + kXS * c;
      float A[RP][5];
#pragma unroll
      for (int k = 0; k < RP; k++)
#pragma unroll
        for (int g = 0; g < 5; g++) A[k][g] = 0.0f;
#pragma unroll
      for (int wi = 0; wi < 8; wi++) {
        uint32_t word[RP];
#pragma unroll
        for (int k = 0; k < RP; k++)
          word[k] = __builtin_amdgcn_alignbyte(it[u][k].d[wi + 1], it[u][k].d[wi], it[u][k].shd);
#pragma unroll
        for (int bi = 0; bi < 4; bi++) {
          const int b = 4 * wi + bi;
          uint2 ent[RP];
#pragma unroll
          for (int k = 0; k < RP; k++) ent[k] = dlut[(word[k] >> (8 * bi)) & 0xffu];
#pragma unroll
          for (int i = 0; i < 5; i++) {
            const int t = 5 * b + i;
            const float xt = xc[t];
#pragma unroll
            for (int k = 0; k < RP; k++) {
              const uint32_t src = i < 4 ? ent[k].x : ent[k].y;
              const float dg = (float)((src >> (8 * (i & 3))) & 0xffu);
              A[k][t / 32] = __builtin_fmaf(dg, xt, A[k][t / 32]);
            }
          }
        }
        // finish each word's fma chains before the next word's table and activation
        // reads (bounds the registers that hold LDS results; without it the compiler
        // issues every read of the item first and keeps all 160 activations live)
#pragma unroll
        for (int k = 0; k < RP; k++)
          asm volatile("" : "+v"(A[k][0]), "+v"(A[k][1]), "+v"(A[k][2]), "+v"(A[k][3]), "+v"(A[k][4])::"memory");
      }
#pragma unroll
      for (int k = 0; k < RP; k++) {
        if (RP * rg + k >= nrows) break;
        const ItemRow& ir = it[u][k];
        const uint32_t mlo = __builtin_amdgcn_alignbyte(ir.m[1], ir.m[0], ir.shm);
        const uint32_t mhi = __builtin_amdgcn_alignbyte(ir.m[2], ir.m[1], ir.shm);
        const uint32_t mfield = (uint32_t)((((uint64_t)mhi << 32) | mlo) >> mbit[u]) & 0x7fffu;
        const uint32_t slo = __builtin_amdgcn_alignbyte(ir.s[1], ir.s[0], ir.shs);
        const uint32_t shi = __builtin_amdgcn_alignbyte(ir.s[2], ir.s[1], ir.shs);
        float chunk = 0.0f;
#pragma unroll
        for (int g = 0; g < 5; g++) {
          if (5 * c + g < P.groups) {
            const uint32_t m = (mfield >> (3 * g)) & 7u;
            const int ex = (int)(((g < 4 ? slo : shi) >> (8 * (g & 3))) & 0xffu);
            const float v = magnitude(m) * pow2i(ex - 127);
            const float p = A[k][g] - bsum[5 * c + g];
            chunk = chunk + v * p;
          }
        }
        part[(RP * rg + k) * P.chunks + c] = chunk;
      }
    }
  }
  __syncthreads();
  for (int r = threadIdx.x; r < nrows; r += kThreads) {
    float acc = 0.0f;
    for (int c = 0; c < P.chunks; c++) acc = acc + part[r * P.chunks + c];
    store(out + r, acc);
  }
}

// Rows per workgroup: one thread per item (RP rows x one 160-column chunk), as many
// items as the threads hold (the kernel takes item = thread); fewer rows only while the
// grid has less than one workgroup per CU.  (gpt-oss down, 2880 rows x 4 slots: 14 rows,
// 824 workgroups, 12.8 us, against 8 rows, 1440 workgroups with 56 idle threads each,
// 13.1 us.)
int rows_per_wg(int64_t rows, int64_t selected, int chunks) {
  int rpw = kRowsPerItem * (kThreads / chunks);
  if (rpw > 32) rpw = 32;
  while (rpw > kRowsPerItem && ((rows + rpw - 1) / rpw) * selected < 256) {
    rpw = rpw / 2 / kRowsPerItem * kRowsPerItem;
    if (rpw < kRowsPerItem) rpw = kRowsPerItem;
  }
  return rpw;
}

size_t lds_bytes(int chunks, int rpw) {
  const int a = chunks * 5, b = rpw * chunks;
  return sizeof(float) * ((size_t)chunks * kXS + a + (a & 1) + b + (b & 1)) + 256 * sizeof(uint2);
}

template <typename XT>
int launch_out(int out_dtype, const TernParams& P, dim3 grid, size_t lds, hipStream_t st) {
  constexpr int RP = kRowsPerItem;
  switch (out_dtype) {
    case TT_F16: hipLaunchKernelGGL((ternary_selected_kernel<XT, f16_t, RP>), grid, dim3(kThreads), lds, st, P); break;
    case TT_BF16: hipLaunchKernelGGL((ternary_selected_kernel<XT, bf16_t, RP>), grid, dim3(kThreads), lds, st, P); break;
    default: hipLaunchKernelGGL((ternary_selected_kernel<XT, float, RP>), grid, dim3(kThreads), lds, st, P); break;
  }
  return check_launch("mxfp_ternary_selected_matvec");
}

}  // namespace
}  // namespace tt

using namespace tt;

extern "C" int tt_mxfp_ternary_selected_matvec(const void* packed, int64_t w_expert_bytes, int64_t w_row_bytes,
                                               int64_t w_total_bytes, const void* scales, int64_t s_expert,
                                               int64_t s_row, int64_t s_total_bytes, int64_t experts,
                                               const void* x, int x_dtype, int64_t x_slot,
                                               const void* expert_indices, int index_bytes, int64_t selected, void* out,
                                               int out_dtype, int64_t out_slot, int64_t rows, int64_t cols,
                                               void* stream) {
  const char* what = "mxfp_ternary_selected_matvec";
  TT_REQUIRE(valid_act_dtype(x_dtype) && valid_out_dtype(out_dtype), "%s: bad dtype codes", what);
  TT_REQUIRE(cols > 0 && cols % 32 == 0, "%s: cols must be a positive multiple of 32", what);
  TT_UNSUPPORTED(cols <= kMaxCols, "%s: cols above %d are not supported", what, kMaxCols);
  TT_REQUIRE(rows > 0 && rows < (1 << 30) && experts >= 1, "%s: bad rows / experts", what);
  TT_REQUIRE(selected >= 1 && selected <= 65535 && expert_indices, "%s: need 1..65535 selected experts", what);
  int ishift;
  TT_REQUIRE(index_shift(index_bytes, &ishift), "%s: expert indices must be int32 or int64", what);
  const int64_t groups = cols / 32, tbytes = (cols + 4) / 5, mbytes = (groups * 3 + 7) / 8;
  TT_REQUIRE(w_row_bytes >= tbytes + mbytes && w_expert_bytes >= rows * w_row_bytes &&
                 w_total_bytes >= (experts - 1) * w_expert_bytes + rows * w_row_bytes,
             "%s: weight rows must hold %lld digit and %lld selector bytes", what, (long long)tbytes,
             (long long)mbytes);
  TT_REQUIRE(s_row >= groups && s_expert >= rows * s_row && s_total_bytes >= (experts - 1) * s_expert + rows * s_row,
             "%s: scale rows must hold %lld groups", what, (long long)groups);
  TT_REQUIRE(w_total_bytes >= 4 && s_total_bytes >= 4, "%s: weight and scale buffers must hold 4 bytes or more", what);
  TT_REQUIRE(packed && scales && aligned(packed, 4) && aligned(scales, 4),
             "%s: packed weights and scales must be 4-byte aligned", what);
  TT_REQUIRE(x && out && aligned(x, 16) && x_slot >= 0 && x_slot % 8 == 0 && (selected == 1 || out_slot >= rows),
             "%s: null or misaligned pointer / bad strides", what);
  TernParams P{};
  P.w = static_cast<const uint8_t*>(packed);
  P.w_end = P.w + w_total_bytes;
  P.s = static_cast<const uint8_t*>(scales);
  P.s_end = P.s + s_total_bytes;
  P.x = x;
  P.experts = expert_indices;
  P.ishift = ishift;
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
  P.rpw = rows_per_wg(rows, selected, P.chunks);
  TT_REQUIRE(P.rpw >= kRowsPerItem && (P.rpw + kRowsPerItem - 1) / kRowsPerItem * P.chunks <= kThreads,
             "%s: a workgroup's items must fit its %d threads", what, kThreads);
  const size_t lds = lds_bytes(P.chunks, P.rpw);
  const dim3 grid((unsigned)((rows + P.rpw - 1) / P.rpw), (unsigned)selected);
  hipStream_t st = static_cast<hipStream_t>(stream);
  return x_dtype == TT_F16 ? launch_out<f16_t>(out_dtype, P, grid, lds, st)
                           : launch_out<bf16_t>(out_dtype, P, grid, lds, st);
}
