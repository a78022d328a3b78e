// Single-token GQA decode attention (fp16/bf16 KV) for gfx950, split over the KV
// sequence.  Semantics follow the reference kernel (triton_kernels.py:15-109):
// softmax(q.k * head_dim^-0.5) v in binary32 with an optional per-head sink that
// joins the softmax denominator but carries no value.
//
// Order of evaluation (restated in oracle/tt_oracle.c):
//   * the KV sequence is cut into chunks of 64 tokens; one wave handles one
//     (kv_head, chunk) for all query heads of that KV head;
//   * score_t = (fma chain over d ascending of q_d k_td) * scale;
//   * chunk max m_c (order free), p_t = exp(score_t - m_c), l_c = butterfly sum of p
//     over the 64 token lanes, o_c[d] = fma chain over the chunk's tokens ascending;
//   * combine in chunk order: M = max(sink, m_c...), den starts at exp(sink - M)
//     (or 0), den = fma(l_c, e_c, den), acc_d = fma(o_c[d], e_c, acc_d) with
//     e_c = exp(m_c - M); out_d = acc_d / den.
// The active token count may be read from device memory (count = tokens_dev[0] +
// tokens, so a decode step can pass its position and 1) so graph replays follow the
// growing cache; chunks past the count exit without work.  The count is clamped to
// max_tokens so a runaway device counter can never read past the cache.
//
// Contiguous head_dim-64 caches use kernels that issue every load before the first
// wait: the chunk wave requests its K row, V column and query rows before the active
// count is known (all rows up to the capacity are in bounds), and the combine wave
// requests the chunk metadata and up to 32 chunks of partial outputs at once.
#include "tt_abi_internal.h"
#include "tt_common.h"

namespace tt {

constexpr int kChunk = 64;

struct AttnParams {
  const void* q;          // [heads, D]
  const void* keys;       // [kv_heads, tokens, D] with strides
  const void* values;
  int64_t k_head, k_tok, v_head, v_tok;
  const void* sinks;      // [heads] or null
  const int32_t* tokens_dev;
  int tokens;
  float* part_m;          // [heads, max_chunks]
  float* part_l;
  float* part_o;          // [heads, max_chunks, D]
  int heads, kv_heads, head_dim, max_chunks, max_tokens;
  float scale;
  void* out;              // [heads, D]
};

// DC: head_dim known at compile time (0: runtime head_dim, scalar loads).  With DC
// set and contiguous rows (token stride DC), the K row of a lane is read with
// 128-bit loads and the V column of the chunk is loaded in full before the weighted
// sum, so each phase waits for memory once.
template <typename T, int G, int DC>
__device__ void attn_chunk(const AttnParams& P, int kvh, int c, int T_act) {
  const int D = DC ? DC : P.head_dim;
  const int lane = threadIdx.x;
  __shared__ float q_s[G * 256];
  __shared__ float p_s[G * kChunk];
  const int h0 = kvh * G;
  for (int i = lane; i < G * D; i += 64) q_s[i] = to_f32(reinterpret_cast<const T*>(P.q)[(int64_t)h0 * D + i]);
  __syncthreads();
  // phase 1: lane = token
  const int t = c * kChunk + lane;
  const bool valid = t < T_act;
  const int nt = min(kChunk, T_act - c * kChunk);
  float sc[G];
#pragma unroll
  for (int g = 0; g < G; g++) sc[g] = 0.0f;
  // V column requested together with K when the registers allow it (G <= 4)
  constexpr bool kVEarly = DC == 64 && G <= 4;
  float vv[DC == 64 ? kChunk : 1];
  if constexpr (DC != 0) {
    // contiguous rows, capacity a whole number of chunks: every row of the chunk is in
    // bounds, rows past the count are read and masked
    const uint4* krow = reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(P.keys) + kvh * P.k_head + (int64_t)t * DC);
    uint4 kr[DC / 8];
#pragma unroll
    for (int i = 0; i < DC / 8; i++) kr[i] = krow[i];
    if constexpr (kVEarly) {
      // the chunk's V column (lane = dimension) is requested together with K
      const T* vcol = reinterpret_cast<const T*>(P.values) + kvh * P.v_head + (int64_t)(c * kChunk) * DC + lane;
#pragma unroll
      for (int tt = 0; tt < kChunk; tt++) vv[tt] = to_f32(vcol[tt * DC]);
    }
#pragma unroll
    for (int i = 0; i < DC / 8; i++) {
      const uint32_t kw[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float kv = (e & 1) ? hi_f32<T>(kw[e >> 1]) : lo_f32<T>(kw[e >> 1]);
#pragma unroll
        for (int g = 0; g < G; g++) sc[g] = __builtin_fmaf(q_s[g * DC + 8 * i + e], kv, sc[g]);
      }
    }
  } else {
    const T* krow = reinterpret_cast<const T*>(P.keys) + kvh * P.k_head + (int64_t)(valid ? t : 0) * P.k_tok;
    for (int d = 0; d < D; d++) {
      const float kv = to_f32(krow[d]);
#pragma unroll
      for (int g = 0; g < G; g++) sc[g] = __builtin_fmaf(q_s[g * D + d], kv, sc[g]);
    }
  }
  const float ninf = __builtin_bit_cast(float, 0xff800000u);
#pragma unroll
  for (int g = 0; g < G; g++) {
    float s = valid ? sc[g] * P.scale : ninf;
    float m = s;
    // chunk max (order-independent)
    m = fmaxf(m, xor_partner<1>(m));
    m = fmaxf(m, xor_partner<2>(m));
    m = fmaxf(m, xor_partner<4>(m));
    m = fmaxf(m, xor_partner<8>(m));
    m = fmaxf(m, xor_partner<16>(m));
    m = fmaxf(m, xor_partner<32>(m));
    const float p = valid ? exp_f32(s - m) : 0.0f;
    const float l = xor_sum(p, 1, 64);
    p_s[g * kChunk + lane] = p;
    if (lane == 0) {
      P.part_m[(int64_t)(h0 + g) * P.max_chunks + c] = m;
      P.part_l[(int64_t)(h0 + g) * P.max_chunks + c] = l;
    }
  }
  __syncthreads();
  // phase 2: lane = dimension, o = fma chain over the chunk's tokens ascending
  if constexpr (DC == 64) {
    if constexpr (!kVEarly) {
      const T* vcol = reinterpret_cast<const T*>(P.values) + kvh * P.v_head + (int64_t)(c * kChunk) * DC + lane;
#pragma unroll
      for (int tt = 0; tt < kChunk; tt++) vv[tt] = to_f32(vcol[tt * DC]);
    }
    float o[G];
#pragma unroll
    for (int g = 0; g < G; g++) o[g] = 0.0f;
    // tokens past the count add fma(0, 0, o) == o (p is 0 there and o is never -0)
#pragma unroll
    for (int tt = 0; tt < kChunk; tt++) {
      const float v = tt < nt ? vv[tt] : 0.0f;
#pragma unroll
      for (int g = 0; g < G; g++) o[g] = __builtin_fmaf(p_s[g * kChunk + tt], v, o[g]);
    }
#pragma unroll
    for (int g = 0; g < G; g++) P.part_o[((int64_t)(h0 + g) * P.max_chunks + c) * DC + lane] = o[g];
  } else {
    for (int d = lane; d < D; d += 64) {
      float o[G];
#pragma unroll
      for (int g = 0; g < G; g++) o[g] = 0.0f;
      const T* vcol = reinterpret_cast<const T*>(P.values) + kvh * P.v_head + (int64_t)(c * kChunk) * P.v_tok + d;
      for (int tt = 0; tt < nt; tt++) {
        const float vv = to_f32(vcol[(int64_t)tt * P.v_tok]);
#pragma unroll
        for (int g = 0; g < G; g++) o[g] = __builtin_fmaf(p_s[g * kChunk + tt], vv, o[g]);
      }
#pragma unroll
      for (int g = 0; g < G; g++) P.part_o[((int64_t)(h0 + g) * P.max_chunks + c) * D + d] = o[g];
    }
  }
}

template <typename T, int G, int DC>
__global__ __launch_bounds__(64) void attn_partial_kernel(AttnParams P) {
  const int kvh = blockIdx.y;
  const int c = blockIdx.x;
  const int T_act = min(P.tokens_dev ? P.tokens_dev[0] + P.tokens : P.tokens, P.max_tokens);
  if (c * kChunk < T_act) attn_chunk<T, G, DC>(P, kvh, c, T_act);
}

// Combine of one head, same arithmetic as the sequential description above: the
// chunk metadata is loaded one chunk per lane, exp(m_c - M) is evaluated per lane and
// the chunk-order folds read it back lane by lane.  One wave.
template <typename T, typename SKT>
__device__ void combine_head(const AttnParams& P, int h, int lane) {
  const int T_act = min(P.tokens_dev ? P.tokens_dev[0] + P.tokens : P.tokens, P.max_tokens);
  const int nc = T_act > 0 ? (T_act + kChunk - 1) / kChunk : 0;
  const float* pm = P.part_m + (int64_t)h * P.max_chunks;
  const float* pl = P.part_l + (int64_t)h * P.max_chunks;
  const float ninf = __builtin_bit_cast(float, 0xff800000u);
  float M = ninf;
  const bool has_sink = P.sinks != nullptr;
  float sink = 0.0f;
  if (has_sink) {
    sink = to_f32(reinterpret_cast<const SKT*>(P.sinks)[h]);
    M = sink;
  }
  // the maximum ignores NaN and does not depend on the order
  for (int c0 = 0; c0 < nc; c0 += 64) {
    float m = c0 + lane < nc ? pm[c0 + lane] : ninf;
    m = fmaxf(m, xor_partner<1>(m));
    m = fmaxf(m, xor_partner<2>(m));
    m = fmaxf(m, xor_partner<4>(m));
    m = fmaxf(m, xor_partner<8>(m));
    m = fmaxf(m, xor_partner<16>(m));
    m = fmaxf(m, xor_partner<32>(m));
    M = fmaxf(M, m);
  }
  float den = has_sink ? exp_f32(sink - M) : 0.0f;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int D = P.head_dim;
  for (int c0 = 0; c0 < nc; c0 += 64) {
    const int n = min(64, nc - c0);
    const float e = c0 + lane < nc ? exp_f32(pm[c0 + lane] - M) : 0.0f;
    const float l = c0 + lane < nc ? pl[c0 + lane] : 0.0f;
    for (int c1 = 0; c1 < n; c1 += 8) {
      // partials of eight chunks are loaded before they are folded in chunk order
      float po[8][4];
#pragma unroll
      for (int u = 0; u < 8; u++) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int d = lane + 64 * q;
          po[u][q] = (c1 + u < n && d < D) ? P.part_o[((int64_t)h * P.max_chunks + c0 + c1 + u) * D + d] : 0.0f;
        }
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        if (c1 + u < n) {
          const int c = c1 + u;
          const float ec = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), c));
          const float lc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l), c));
          den = __builtin_fmaf(lc, ec, den);
#pragma unroll
          for (int q = 0; q < 4; q++) acc[q] = __builtin_fmaf(po[u][q], ec, acc[q]);
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int d = lane + 64 * q;
    if (d < D) store<T>(reinterpret_cast<T*>(P.out) + (int64_t)h * D + d, acc[q] / den);
  }
}

template <typename T, typename SKT>
__global__ __launch_bounds__(64) void attn_combine_kernel(AttnParams P) {
  combine_head<T, SKT>(P, blockIdx.x, threadIdx.x);
}

// Chunk partials for contiguous head_dim-64 caches whose capacity is a whole number
// of chunks (every row of every chunk is in bounds, so all loads are issued before the
// active count is known).  Same arithmetic as attn_chunk.
template <typename T, int G>
__global__ __launch_bounds__(64) void attn_partial64_kernel(AttnParams P) {
  constexpr int D = 64;
  const int kvh = blockIdx.y;
  const int c = blockIdx.x;
  const int lane = threadIdx.x;
  const int h0 = kvh * G;
  __shared__ float q_s[G * D];
  __shared__ float p_s[G * kChunk];
  // K row of this lane's token, the chunk's V column (lane = dimension), query rows
  const int t = c * kChunk + lane;
  const uint4* krow = reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(P.keys) + kvh * P.k_head + (int64_t)t * D);
  uint4 kr[D / 8];
#pragma unroll
  for (int i = 0; i < D / 8; i++) kr[i] = krow[i];
  const T* vcol = reinterpret_cast<const T*>(P.values) + kvh * P.v_head + (int64_t)(c * kChunk) * D + lane;
  T vraw[kChunk];
#pragma unroll
  for (int tt = 0; tt < kChunk; tt++) vraw[tt] = vcol[tt * D];
  T qraw[G];
#pragma unroll
  for (int g = 0; g < G; g++) qraw[g] = reinterpret_cast<const T*>(P.q)[(int64_t)h0 * D + g * D + lane];
  const int T_act = min(P.tokens_dev ? P.tokens_dev[0] + P.tokens : P.tokens, P.max_tokens);
  if (c * kChunk >= T_act) return;
  const bool valid = t < T_act;
  const int nt = min(kChunk, T_act - c * kChunk);
#pragma unroll
  for (int g = 0; g < G; g++) q_s[g * D + lane] = to_f32(qraw[g]);
  __syncthreads();
  float sc[G];
#pragma unroll
  for (int g = 0; g < G; g++) sc[g] = 0.0f;
#pragma unroll
  for (int i = 0; i < D / 8; i++) {
    const uint32_t kw[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float kv = (e & 1) ? hi_f32<T>(kw[e >> 1]) : lo_f32<T>(kw[e >> 1]);
#pragma unroll
      for (int g = 0; g < G; g++) sc[g] = __builtin_fmaf(q_s[g * D + 8 * i + e], kv, sc[g]);
    }
  }
  const float ninf = __builtin_bit_cast(float, 0xff800000u);
#pragma unroll
  for (int g = 0; g < G; g++) {
    const float s = valid ? sc[g] * P.scale : ninf;
    float m = s;
    m = fmaxf(m, xor_partner<1>(m));
    m = fmaxf(m, xor_partner<2>(m));
    m = fmaxf(m, xor_partner<4>(m));
    m = fmaxf(m, xor_partner<8>(m));
    m = fmaxf(m, xor_partner<16>(m));
    m = fmaxf(m, xor_partner<32>(m));
    const float p = valid ? exp_f32(s - m) : 0.0f;
    const float l = xor_sum(p, 1, 64);
    p_s[g * kChunk + lane] = p;
    if (lane == 0) {
      P.part_m[(int64_t)(h0 + g) * P.max_chunks + c] = m;
      P.part_l[(int64_t)(h0 + g) * P.max_chunks + c] = l;
    }
  }
  __syncthreads();
  float o[G];
#pragma unroll
  for (int g = 0; g < G; g++) o[g] = 0.0f;
#pragma unroll
  for (int tt = 0; tt < kChunk; tt++) {
    const float v = tt < nt ? to_f32(vraw[tt]) : 0.0f;
#pragma unroll
    for (int g = 0; g < G; g++) o[g] = __builtin_fmaf(p_s[g * kChunk + tt], v, o[g]);
  }
#pragma unroll
  for (int g = 0; g < G; g++) P.part_o[((int64_t)(h0 + g) * P.max_chunks + c) * D + lane] = o[g];
}

// Combine of one head of dimension 64 (lane = dimension), the arithmetic of
// combine_head; the chunk metadata and the partial outputs of up to kBlk chunks are
// requested together before the maximum is formed.
template <typename T, typename SKT>
__global__ __launch_bounds__(64) void attn_combine64_kernel(AttnParams P) {
  constexpr int D = 64, kBlk = 32;
  const int h = blockIdx.x;
  const int lane = threadIdx.x;
  const int T_act = min(P.tokens_dev ? P.tokens_dev[0] + P.tokens : P.tokens, P.max_tokens);
  const int nc = T_act > 0 ? (T_act + kChunk - 1) / kChunk : 0;
  const float* pm = P.part_m + (int64_t)h * P.max_chunks;
  const float* pl = P.part_l + (int64_t)h * P.max_chunks;
  const float* po = P.part_o + (int64_t)h * P.max_chunks * D + lane;
  const int last = P.max_chunks - 1;
  // first block of every operand, clamped to the scratch (values past nc are unused)
  float mv = pm[lane < last ? lane : last];
  float lv = pl[lane < last ? lane : last];
  float ov[kBlk];
#pragma unroll
  for (int u = 0; u < kBlk; u++) ov[u] = po[(int64_t)(u < last ? u : last) * D];
  const float ninf = __builtin_bit_cast(float, 0xff800000u);
  const bool has_sink = P.sinks != nullptr;
  const float sink = has_sink ? to_f32(reinterpret_cast<const SKT*>(P.sinks)[h]) : 0.0f;
  float M = has_sink ? sink : ninf;
  for (int c0 = 0; c0 < nc; c0 += 64) {
    float m = c0 + lane < nc ? (c0 == 0 ? mv : pm[c0 + lane]) : ninf;
    m = fmaxf(m, xor_partner<1>(m));
    m = fmaxf(m, xor_partner<2>(m));
    m = fmaxf(m, xor_partner<4>(m));
    m = fmaxf(m, xor_partner<8>(m));
    m = fmaxf(m, xor_partner<16>(m));
    m = fmaxf(m, xor_partner<32>(m));
    M = fmaxf(M, m);
  }
  float den = has_sink ? exp_f32(sink - M) : 0.0f;
  float acc = 0.0f;
  for (int c0 = 0; c0 < nc; c0 += 64) {
    const int n = min(64, nc - c0);
    const float e = c0 + lane < nc ? exp_f32((c0 == 0 ? mv : pm[c0 + lane]) - M) : 0.0f;
    const float l = c0 + lane < nc ? (c0 == 0 ? lv : pl[c0 + lane]) : 0.0f;
    for (int c1 = 0; c1 < n; c1 += kBlk) {
      if (c0 + c1 > 0) {
#pragma unroll
        for (int u = 0; u < kBlk; u++) {
          const int cc = c0 + c1 + u;
          ov[u] = po[(int64_t)(cc < last ? cc : last) * D];
        }
      }
#pragma unroll
      for (int u = 0; u < kBlk; u++) {
        if (c1 + u < n) {
          const float ec = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), c1 + u));
          const float lc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l), c1 + u));
          den = __builtin_fmaf(lc, ec, den);
          acc = __builtin_fmaf(ov[u], ec, acc);
        }
      }
    }
  }
  store<T>(reinterpret_cast<T*>(P.out) + (int64_t)h * D + lane, acc / den);
}

// One workgroup per query head (contiguous head_dim-64 caches, whole-chunk capacity):
// its kHeadWaves waves compute the head's chunk partials (chunk c on wave c mod
// kHeadWaves) into LDS with the arithmetic of attn_partial64_kernel, and after one
// barrier wave 0 combines them in chunk order with the arithmetic of
// attn_combine64_kernel -- one launch, no communication between workgroups.
//
// Memory path: a wave requests its chunk's K and V blocks as sixteen fully coalesced
// 16-byte loads per lane (each instruction covers 1 KB of consecutive bytes) and
// transposes them through its own 8 KB LDS slice: K first (token r's piece d at slot
// 8r + (d xor (r mod 8)), so the row reads of the score phase are free of bank
// conflicts), then V in the same slice for the weighted sum.  The next chunk's blocks
// are requested before the softmax so the value phase hides them.
// Workgroups are dealt to the XCDs round-robin by id, so the query heads of one KV head
// get ids congruent mod 8 (when the head counts allow it) and read its K/V rows through
// one L2.
constexpr int kHeadWaves = 12;
constexpr int kHeadMaxChunks = 192;   // LDS partials: 66 floats per chunk
constexpr int kXcds = 8;

// A chunk's K and V blocks (64 tokens x 64 dims, 8 KB each) as 16-byte pieces
// i * 64 + lane: token 8i + lane / 8, dimensions 8 (lane mod 8) .. +7.
struct ChunkPieces {
  uint4 k[8], v[8];
};

__device__ __forceinline__ ChunkPieces load_chunk(const uint4* kbase, const uint4* vbase, int c, int lane) {
  const uint4* kblk = kbase + (int64_t)c * (kChunk * 64 / 8);
  const uint4* vblk = vbase + (int64_t)c * (kChunk * 64 / 8);
  ChunkPieces r;
#pragma unroll
  for (int i = 0; i < 8; i++) r.k[i] = kblk[i * 64 + lane];
#pragma unroll
  for (int i = 0; i < 8; i++) r.v[i] = vblk[i * 64 + lane];
  return r;
}

template <typename T, typename SKT>
__global__ __launch_bounds__(64 * kHeadWaves) void attn_head_kernel(AttnParams P) {
  constexpr int D = 64;
  const int G = P.heads / P.kv_heads;
  int h = blockIdx.x;
  if (P.heads % kXcds == 0 && P.kv_heads % kXcds == 0) {
    // workgroup w runs on XCD w mod 8; its slot j = w / 8 on that XCD names
    // (KV head 8 * (j / G) + w mod 8, query head j mod G of that group)
    const int x = h % kXcds, j = h / kXcds;
    h = ((j / G) * kXcds + x) * G + j % G;
  }
  const int kvh = h / G;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  __shared__ float q_s[D];
  __shared__ float p_s[kHeadWaves][kChunk];
  __shared__ uint4 kv_s[kHeadWaves][kChunk * D / 8];
  __shared__ float pm_s[kHeadMaxChunks], pl_s[kHeadMaxChunks];
  __shared__ float po_s[kHeadMaxChunks][D];
  const float ninf = __builtin_bit_cast(float, 0xff800000u);
  const uint4* kbase = reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(P.keys) + kvh * P.k_head);
  const uint4* vbase = reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(P.values) + kvh * P.v_head);
  // first chunk of this wave: every load is issued before the active count is known
  // (chunks below max_chunks are inside the capacity)
  const int c_first = wave;
  ChunkPieces cur;
  if (c_first < P.max_chunks) cur = load_chunk(kbase, vbase, c_first, lane);
  const T qraw = reinterpret_cast<const T*>(P.q)[(int64_t)h * D + lane];
  const int T_act = min(P.tokens_dev ? P.tokens_dev[0] + P.tokens : P.tokens, P.max_tokens);
  const int nc = T_act > 0 ? (T_act + kChunk - 1) / kChunk : 0;
  if (wave == 0) q_s[lane] = to_f32(qraw);
  __syncthreads();

  float* p_w = p_s[wave];
  uint4* kv_w = kv_s[wave];
  for (int c = c_first; c < nc; c += kHeadWaves) {
    const int t = c * kChunk + lane;
    const bool valid = t < T_act;
    const int nt = min(kChunk, T_act - c * kChunk);
    // K block into the slice, then this lane's token row back out of it
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int r = i * 8 + (lane >> 3);
      const uint4 k = cur.k[i];
      kv_w[r * 8 + ((lane & 7) ^ (r & 7))] = uint4{k.x, k.y, k.z, k.w};
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the K stores are done
    __builtin_amdgcn_wave_barrier();
    uint32_t krow[8][4];
#pragma unroll
    for (int d = 0; d < 8; d++) {
      const uint4 k = kv_w[lane * 8 + (d ^ (lane & 7))];
      krow[d][0] = k.x; krow[d][1] = k.y; krow[d][2] = k.z; krow[d][3] = k.w;
    }
    // V pieces of tokens past the count are staged as zeros: the weighted sum then adds
    // fma(0, 0, o) == o for them (p is 0 there and o is never -0).  The wave's LDS
    // operations complete in order, so these stores follow the row reads above.
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const uint32_t keep = i * 8 + (lane >> 3) < nt ? ~0u : 0u;
      kv_w[i * 64 + lane] = uint4{cur.v[i].x & keep, cur.v[i].y & keep, cur.v[i].z & keep, cur.v[i].w & keep};
    }
    // score: fma chain over d ascending, lane = token
    float sc = 0.0f;
#pragma unroll
    for (int i = 0; i < D / 8; i++) {
      if ((i & 3) == 0) asm volatile("" : "+v"(sc)::"memory");   // 32 query values live per step
      const uint32_t* kw = krow[i];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float kv = (e & 1) ? hi_f32<T>(kw[e >> 1]) : lo_f32<T>(kw[e >> 1]);
        sc = __builtin_fmaf(q_s[8 * i + e], kv, sc);
      }
    }
    // the next chunk of this wave is requested while this one finishes
    if (c + kHeadWaves < nc) cur = load_chunk(kbase, vbase, c + kHeadWaves, lane);
    const float s = valid ? sc * P.scale : ninf;
    float m = s;
    m = fmaxf(m, xor_partner<1>(m));
    m = fmaxf(m, xor_partner<2>(m));
    m = fmaxf(m, xor_partner<4>(m));
    m = fmaxf(m, xor_partner<8>(m));
    m = fmaxf(m, xor_partner<16>(m));
    m = fmaxf(m, xor_partner<32>(m));
    const float p = valid ? exp_f32(s - m) : 0.0f;
    const float l = xor_sum(p, 1, 64);
    p_w[lane] = p;
    if (lane == 0) {
      pm_s[c] = m;
      pl_s[c] = l;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's p and V stores done
    __builtin_amdgcn_wave_barrier();
    // weighted values: lane = dimension, fma chain over the chunk's tokens ascending
    const T* vs = reinterpret_cast<const T*>(kv_w);
    float o = 0.0f;
#pragma unroll
    for (int tt = 0; tt < kChunk; tt++) {
      if ((tt & 31) == 0) asm volatile("" : "+v"(o)::"memory");   // 32 tokens live per step
      o = __builtin_fmaf(p_w[tt], to_f32(vs[tt * D + lane]), o);
    }
    po_s[c][lane] = o;
    __builtin_amdgcn_s_waitcnt(0xc07f);   // reads of the wave's LDS slices done before reuse
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  if (wave != 0) return;

  // combine in chunk order (the arithmetic of combine_head)
  const bool has_sink = P.sinks != nullptr;
  const float sink = has_sink ? to_f32(reinterpret_cast<const SKT*>(P.sinks)[h]) : 0.0f;
  float M = has_sink ? sink : ninf;
  for (int c0 = 0; c0 < nc; c0 += 64) {
    float mm = c0 + lane < nc ? pm_s[c0 + lane] : ninf;
    mm = fmaxf(mm, xor_partner<1>(mm));
    mm = fmaxf(mm, xor_partner<2>(mm));
    mm = fmaxf(mm, xor_partner<4>(mm));
    mm = fmaxf(mm, xor_partner<8>(mm));
    mm = fmaxf(mm, xor_partner<16>(mm));
    mm = fmaxf(mm, xor_partner<32>(mm));
    M = fmaxf(M, mm);
  }
  float den = has_sink ? exp_f32(sink - M) : 0.0f;
  float acc = 0.0f;
  for (int c0 = 0; c0 < nc; c0 += 64) {
    const int n = min(64, nc - c0);
    const float e = c0 + lane < nc ? exp_f32(pm_s[c0 + lane] - M) : 0.0f;
    const float lv = c0 + lane < nc ? pl_s[c0 + lane] : 0.0f;
    for (int u = 0; u < n; u++) {
      const float ec = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), u));
      const float lc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv), u));
      den = __builtin_fmaf(lc, ec, den);
      acc = __builtin_fmaf(po_s[c0 + u][lane], ec, acc);
    }
  }
  store<T>(reinterpret_cast<T*>(P.out) + (int64_t)h * D + lane, acc / den);
}

// One workgroup per (KV head, chunk) with one wave per query head of that KV head
// (contiguous head_dim-64 caches, whole-chunk capacity): the chunk's K and V blocks are
// read once per KV head -- each CU moves 16 KB instead of a whole sequence -- staged in
// LDS (K swizzled as in attn_head_kernel, V rows of tokens past the count zeroed), and
// wave g computes the chunk partial of query head G kvh + g with the arithmetic of
// attn_partial64_kernel.  The partials go to the scratch with device-scope atomic stores;
// the workgroup counts itself in its KV head's arrival counter once its stores have
// completed, and the last of the head's active chunks combines every query head of the
// KV head in chunk order (the arithmetic of attn_combine64_kernel, partials read with
// device-scope atomic loads) and resets the counter to zero.  No workgroup waits for
// another.  Same bits as attn_head_kernel.
__device__ __forceinline__ void st_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T, typename SKT, int G, int CPW = 1, bool COMBINE = true>
__global__ __launch_bounds__(64 * G) void attn_kvchunk_kernel(AttnParams P, int* counters) {
  // CPW chunks per workgroup (1 or 2): with 2, both chunks' K and V pieces are requested
  // up front and the chunks are computed one after the other through the same LDS, which
  // halves the grid when it is several generations of workgroups deep; every chunk's
  // partial is computed exactly as with one chunk per workgroup
  static_assert(CPW == 1 || CPW == 2, "one or two chunks per workgroup");
  constexpr int D = 64;
  const int c0 = blockIdx.x * CPW, kvh = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int h = kvh * G + wave;
  constexpr int nthr = 64 * G;
  __shared__ uint4 ks[kChunk * D / 8], vs_s[kChunk * D / 8];
  __shared__ float q_s[G][D];
  __shared__ float p_s[G][kChunk];
  __shared__ int last;
  const float ninf = __builtin_bit_cast(float, 0xff800000u);
  // every load before the active count is known (chunks below max_chunks are inside
  // the capacity; a second chunk past them is clamped to the last one, values unused):
  // K and V pieces of the chunks, this wave's query row
  constexpr int kPer = kChunk * D / 8 / nthr;   // 16-byte pieces per thread
  // (native 4-vectors: arrays of the uint4 struct type are kept in scratch memory here)
  typedef uint32_t piece_t __attribute__((ext_vector_type(4)));
  piece_t kr[kPer], vr[kPer], kr1[kPer], vr1[kPer];
  auto load_chunk = [&](int c, piece_t (&kk)[kPer], piece_t (&vv)[kPer]) {
    const piece_t* kblk = reinterpret_cast<const piece_t*>(reinterpret_cast<const T*>(P.keys) + kvh * P.k_head) +
                          (int64_t)c * (kChunk * D / 8);
    const piece_t* vblk = reinterpret_cast<const piece_t*>(reinterpret_cast<const T*>(P.values) + kvh * P.v_head) +
                          (int64_t)c * (kChunk * D / 8);
#pragma unroll
    for (int j = 0; j < kPer; j++) {
      kk[j] = kblk[(int)threadIdx.x + nthr * j];
      vv[j] = vblk[(int)threadIdx.x + nthr * j];
    }
  };
  load_chunk(c0, kr, vr);
  if constexpr (CPW == 2) load_chunk(c0 + 1 < P.max_chunks ? c0 + 1 : P.max_chunks - 1, kr1, vr1);
  const T qraw = reinterpret_cast<const T*>(P.q)[(int64_t)h * D + lane];
  const int T_act = min(P.tokens_dev ? P.tokens_dev[0] + P.tokens : P.tokens, P.max_tokens);
  const int nc = T_act > 0 ? (T_act + kChunk - 1) / kChunk : 0;
  if (c0 >= nc) return;
  const int done = min(CPW, nc - c0);   // active chunks of this workgroup
  q_s[wave][lane] = to_f32(qraw);

#pragma unroll
  for (int cc = 0; cc < CPW; cc++) {
    if (cc >= done) break;   // uniform
    const int c = c0 + cc;
    if (cc > 0) __syncthreads();   // the previous chunk's LDS reads are done
    const int nt = min(kChunk, T_act - c * kChunk);
    auto stage = [&](const piece_t (&kk)[kPer], const piece_t (&vv)[kPer]) {
#pragma unroll
      for (int j = 0; j < kPer; j++) {
        const int pidx = (int)threadIdx.x + nthr * j;
        const int r = pidx >> 3, col = pidx & 7;
        reinterpret_cast<piece_t*>(ks)[r * 8 + (col ^ (r & 7))] = kk[j];
        const uint32_t keep = r < nt ? ~0u : 0u;
        reinterpret_cast<piece_t*>(vs_s)[pidx] = vv[j] & keep;
      }
    };
    if (cc == 0) stage(kr, vr);
    else stage(kr1, vr1);
    __syncthreads();

    // ---- chunk partial of query head h (lane = token, then lane = dimension)
    const int t = c * kChunk + lane;
    const bool valid = t < T_act;
    uint32_t krow[8][4];
#pragma unroll
    for (int d = 0; d < 8; d++) {
      const uint4 k = ks[lane * 8 + (d ^ (lane & 7))];
      krow[d][0] = k.x; krow[d][1] = k.y; krow[d][2] = k.z; krow[d][3] = k.w;
    }
    const float* qw = q_s[wave];
    float sc = 0.0f;
#pragma unroll
    for (int i = 0; i < D / 8; i++) {
      if ((i & 3) == 0) asm volatile("" : "+v"(sc)::"memory");
      const uint32_t* kw = krow[i];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float kv = (e & 1) ? hi_f32<T>(kw[e >> 1]) : lo_f32<T>(kw[e >> 1]);
        sc = __builtin_fmaf(qw[8 * i + e], kv, sc);
      }
    }
    const float s = valid ? sc * P.scale : ninf;
    float m = s;
    m = fmaxf(m, xor_partner<1>(m));
    m = fmaxf(m, xor_partner<2>(m));
    m = fmaxf(m, xor_partner<4>(m));
    m = fmaxf(m, xor_partner<8>(m));
    m = fmaxf(m, xor_partner<16>(m));
    m = fmaxf(m, xor_partner<32>(m));
    const float p = valid ? exp_f32(s - m) : 0.0f;
    const float l = xor_sum(p, 1, 64);
    float* p_w = p_s[wave];
    p_w[lane] = p;
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's p stores done
    __builtin_amdgcn_wave_barrier();
    const T* vsp = reinterpret_cast<const T*>(vs_s);
    float o = 0.0f;
#pragma unroll
    for (int tt = 0; tt < kChunk; tt++) {
      if ((tt & 31) == 0) asm volatile("" : "+v"(o)::"memory");
      o = __builtin_fmaf(p_w[tt], to_f32(vsp[tt * D + lane]), o);
    }
    const int64_t slot = (int64_t)h * P.max_chunks + c;
    if (lane == 0) {
      st_dev(P.part_m + slot, m);
      st_dev(P.part_l + slot, l);
    }
    st_dev(P.part_o + slot * D + lane, o);
  }
  // without COMBINE the partials are the result: the kernel that consumes them runs after
  // this one on the stream
  if constexpr (!COMBINE) return;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(counters + kvh, done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nc - done;
  __syncthreads();
  if (!last) return;

  // ---- combine of query head h in chunk order (attn_combine64_kernel's arithmetic); the
  // first 64 chunks' (m, l) and the first kBlk chunks' partial rows are requested together
  // with the sink, one round trip, before the maximum is formed
  constexpr int kBlk = 32;
  const float* pm = P.part_m + (int64_t)h * P.max_chunks;
  const float* pl = P.part_l + (int64_t)h * P.max_chunks;
  const float* po = P.part_o + (int64_t)h * P.max_chunks * D + lane;
  const bool has_sink = P.sinks != nullptr;
  const float m0 = lane < nc ? ld_dev(pm + lane) : ninf;
  const float l0 = lane < nc ? ld_dev(pl + lane) : 0.0f;
  float ov0[kBlk];
#pragma unroll
  for (int u = 0; u < kBlk; u++) ov0[u] = u < nc ? ld_dev(po + (int64_t)u * D) : 0.0f;
  const float sink = has_sink ? to_f32(reinterpret_cast<const SKT*>(P.sinks)[h]) : 0.0f;
  float M = has_sink ? sink : ninf;
  for (int c0 = 0; c0 < nc; c0 += 64) {
    float mm = c0 == 0 ? m0 : (c0 + lane < nc ? ld_dev(pm + c0 + lane) : ninf);
    mm = fmaxf(mm, xor_partner<1>(mm));
    mm = fmaxf(mm, xor_partner<2>(mm));
    mm = fmaxf(mm, xor_partner<4>(mm));
    mm = fmaxf(mm, xor_partner<8>(mm));
    mm = fmaxf(mm, xor_partner<16>(mm));
    mm = fmaxf(mm, xor_partner<32>(mm));
    M = fmaxf(M, mm);
  }
  float den = has_sink ? exp_f32(sink - M) : 0.0f;
  float acc = 0.0f;
  for (int c0 = 0; c0 < nc; c0 += 64) {
    const int n = min(64, nc - c0);
    const float e = c0 + lane < nc ? exp_f32((c0 == 0 ? m0 : ld_dev(pm + c0 + lane)) - M) : 0.0f;
    const float lv = c0 + lane < nc ? (c0 == 0 ? l0 : ld_dev(pl + c0 + lane)) : 0.0f;
    for (int c1 = 0; c1 < n; c1 += kBlk) {
      float ov[kBlk];
      if (c0 == 0 && c1 == 0) {
#pragma unroll
        for (int u = 0; u < kBlk; u++) ov[u] = ov0[u];
      } else {
#pragma unroll
        for (int u = 0; u < kBlk; u++) {
          const int cc = c0 + c1 + u;
          ov[u] = cc < nc ? ld_dev(po + (int64_t)cc * D) : 0.0f;
        }
      }
#pragma unroll
      for (int u = 0; u < kBlk; u++) {
        if (c1 + u < n) {
          const float ec = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), c1 + u));
          const float lc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv), c1 + u));
          den = __builtin_fmaf(lc, ec, den);
          acc = __builtin_fmaf(ov[u], ec, acc);
        }
      }
    }
  }
  store<T>(reinterpret_cast<T*>(P.out) + (int64_t)h * D + lane, acc / den);
  if (threadIdx.x == 0) __hip_atomic_store(counters + kvh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Two chunks per workgroup once the one-chunk grid holds more workgroups than this.
constexpr int64_t kAttnPairMinWorkgroups = 1024;

template <typename T, int G>
static int launch_attn(const AttnParams& P, int sink_dtype, bool contiguous64, int* counters, hipStream_t st) {
  if constexpr (G <= 8) {
    if (contiguous64 && counters != nullptr) {
      const dim3 block(64 * G);
      if ((int64_t)P.max_chunks * P.kv_heads > kAttnPairMinWorkgroups) {
        const dim3 grid((unsigned)((P.max_chunks + 1) / 2), (unsigned)P.kv_heads);
        switch (sink_dtype) {
          case TT_BF16: hipLaunchKernelGGL((attn_kvchunk_kernel<T, bf16_t, G, 2>), grid, block, 0, st, P, counters); break;
          case TT_F32: hipLaunchKernelGGL((attn_kvchunk_kernel<T, float, G, 2>), grid, block, 0, st, P, counters); break;
          default: hipLaunchKernelGGL((attn_kvchunk_kernel<T, f16_t, G, 2>), grid, block, 0, st, P, counters); break;
        }
        return check_launch("gqa_attention");
      }
      const dim3 grid((unsigned)P.max_chunks, (unsigned)P.kv_heads);
      switch (sink_dtype) {
        case TT_BF16: hipLaunchKernelGGL((attn_kvchunk_kernel<T, bf16_t, G>), grid, block, 0, st, P, counters); break;
        case TT_F32: hipLaunchKernelGGL((attn_kvchunk_kernel<T, float, G>), grid, block, 0, st, P, counters); break;
        default: hipLaunchKernelGGL((attn_kvchunk_kernel<T, f16_t, G>), grid, block, 0, st, P, counters); break;
      }
      return check_launch("gqa_attention");
    }
  }
  if (contiguous64 && P.max_chunks <= kHeadMaxChunks) {
    switch (sink_dtype) {
      case TT_BF16: hipLaunchKernelGGL((attn_head_kernel<T, bf16_t>), dim3(P.heads), dim3(64 * kHeadWaves), 0, st, P); break;
      case TT_F32: hipLaunchKernelGGL((attn_head_kernel<T, float>), dim3(P.heads), dim3(64 * kHeadWaves), 0, st, P); break;
      default: hipLaunchKernelGGL((attn_head_kernel<T, f16_t>), dim3(P.heads), dim3(64 * kHeadWaves), 0, st, P); break;
    }
    return check_launch("gqa_attention");
  }
  if (contiguous64) {
    hipLaunchKernelGGL((attn_partial64_kernel<T, G>), dim3(P.max_chunks, P.kv_heads), dim3(64), 0, st, P);
    int rc = check_launch("gqa_attention");
    if (rc) return rc;
    switch (sink_dtype) {
      case TT_BF16: hipLaunchKernelGGL((attn_combine64_kernel<T, bf16_t>), dim3(P.heads), dim3(64), 0, st, P); break;
      case TT_F32: hipLaunchKernelGGL((attn_combine64_kernel<T, float>), dim3(P.heads), dim3(64), 0, st, P); break;
      default: hipLaunchKernelGGL((attn_combine64_kernel<T, f16_t>), dim3(P.heads), dim3(64), 0, st, P); break;
    }
    return check_launch("gqa_attention");
  }
  if (contiguous64)
    hipLaunchKernelGGL((attn_partial_kernel<T, G, 64>), dim3(P.max_chunks, P.kv_heads), dim3(64), 0, st, P);
  else
    hipLaunchKernelGGL((attn_partial_kernel<T, G, 0>), dim3(P.max_chunks, P.kv_heads), dim3(64), 0, st, P);
  int rc = check_launch("gqa_attention");
  if (rc) return rc;
  switch (sink_dtype) {
    case TT_BF16: hipLaunchKernelGGL((attn_combine_kernel<T, bf16_t>), dim3(P.heads), dim3(64), 0, st, P); break;
    case TT_F32: hipLaunchKernelGGL((attn_combine_kernel<T, float>), dim3(P.heads), dim3(64), 0, st, P); break;
    default: hipLaunchKernelGGL((attn_combine_kernel<T, f16_t>), dim3(P.heads), dim3(64), 0, st, P); break;
  }
  return check_launch("gqa_attention");
}

}  // namespace tt

using namespace tt;


extern "C" int tt_attention_scratch_floats(int64_t heads, int64_t max_tokens, int64_t head_dim) {
  const int64_t chunks = (max_tokens + kChunk - 1) / kChunk;
  return (int)(kAttnCounters + heads * chunks * (2 + head_dim));
}

// Chunk partials only (contiguous head_dim-64 caches, whole-chunk capacity, no sinks):
// the one-launch kernel without its arrival count and combine, for a consumer that
// combines the partials itself (tt_attention_combine_int4_matvec).
template <typename T, int G>
static int launch_attn_partials(const AttnParams& P, hipStream_t st) {
  const dim3 block(64 * G);
  if ((int64_t)P.max_chunks * P.kv_heads > kAttnPairMinWorkgroups)
    hipLaunchKernelGGL((attn_kvchunk_kernel<T, f16_t, G, 2, false>), dim3((unsigned)((P.max_chunks + 1) / 2), (unsigned)P.kv_heads),
                       block, 0, st, P, nullptr);
  else
    hipLaunchKernelGGL((attn_kvchunk_kernel<T, f16_t, G, 1, false>), dim3((unsigned)P.max_chunks, (unsigned)P.kv_heads), block,
                       0, st, P, nullptr);
  return check_launch("gqa_attention_partials");
}

extern "C" int tt_single_token_gqa_attention_partials(const void* q, const void* keys, const void* values, int dtype,
                                                      int64_t k_head, int64_t k_tok, int64_t v_head, int64_t v_tok,
                                                      const int32_t* tokens_dev, int64_t tokens, int64_t max_tokens,
                                                      int64_t heads, int64_t kv_heads, int64_t head_dim, float* scratch,
                                                      int64_t scratch_floats, void* stream) {
  const char* what = "single_token_gqa_attention_partials";
  TT_REQUIRE(q && keys && values && scratch, "%s: null pointer", what);
  TT_REQUIRE(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "%s: heads must be a multiple of kv_heads", what);
  TT_REQUIRE(tokens_dev != nullptr || (tokens > 0 && tokens <= max_tokens), "%s: attention requires at least one KV token", what);
  TT_REQUIRE(tokens_dev == nullptr || (tokens >= 0 && tokens <= 1), "%s: device token count offset must be 0 or 1", what);
  TT_REQUIRE(max_tokens > 0 && kv_heads <= 65535, "%s: bad max_tokens / kv_heads", what);
  const int64_t chunks = (max_tokens + kChunk - 1) / kChunk;
  TT_REQUIRE(chunks <= 65535, "%s: sequence too long", what);
  TT_REQUIRE(scratch_floats >= kAttnCounters + heads * chunks * (2 + head_dim), "%s: scratch too small", what);
  const int64_t G = heads / kv_heads;
  TT_UNSUPPORTED(head_dim == 64 && k_tok == 64 && v_tok == 64 && max_tokens % kChunk == 0 && aligned(keys, 16) &&
                     aligned(values, 16) && k_head % 8 == 0 && v_head % 8 == 0 && (G == 1 || G == 2 || G == 4 || G == 8),
                 "%s: needs contiguous head_dim-64 caches whose capacity is a multiple of %d tokens and 1, 2, 4 or 8 "
                 "query heads per KV head", what, kChunk);
  AttnParams P{};
  P.q = q; P.keys = keys; P.values = values;
  P.k_head = k_head; P.k_tok = k_tok; P.v_head = v_head; P.v_tok = v_tok;
  P.sinks = nullptr; P.tokens_dev = tokens_dev; P.tokens = (int)tokens;
  scratch += kAttnCounters;
  P.part_m = scratch;
  P.part_l = scratch + heads * chunks;
  P.part_o = scratch + 2 * heads * chunks;
  P.heads = (int)heads; P.kv_heads = (int)kv_heads; P.head_dim = (int)head_dim; P.max_chunks = (int)chunks;
  P.max_tokens = (int)max_tokens;
  P.scale = (float)(1.0 / __builtin_sqrt((double)head_dim));
  P.out = nullptr;
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto by_g = [&](auto t) -> int {
    using T = decltype(t);
    switch (G) {
      case 1: return launch_attn_partials<T, 1>(P, st);
      case 2: return launch_attn_partials<T, 2>(P, st);
      case 4: return launch_attn_partials<T, 4>(P, st);
      default: return launch_attn_partials<T, 8>(P, st);
    }
  };
  if (dtype == TT_F16) return by_g(f16_t{});
  if (dtype == TT_BF16) return by_g(bf16_t{});
  set_error("%s: KV dtype must be fp16 or bf16", what);
  return TT_ERR_INVALID;
}

extern "C" int tt_single_token_gqa_attention(const void* q, const void* keys, const void* values, int dtype,
                                             int64_t k_head, int64_t k_tok, int64_t v_head, int64_t v_tok,
                                             const void* sinks, int sink_dtype, const int32_t* tokens_dev,
                                             int64_t tokens, int64_t max_tokens, int64_t heads, int64_t kv_heads,
                                             int64_t head_dim, float* scratch, int64_t scratch_floats, void* out,
                                             void* stream) {
  const char* what = "single_token_gqa_attention";
  TT_REQUIRE(q && keys && values && out && scratch, "%s: null pointer", what);
  TT_REQUIRE(head_dim > 0 && head_dim <= 256, "%s: fused single-token attention supports head_dim <= 256", what);
  TT_REQUIRE(heads > 0 && kv_heads > 0 && heads % kv_heads == 0, "%s: heads must be a multiple of kv_heads", what);
  TT_REQUIRE(tokens_dev != nullptr || (tokens > 0 && tokens <= max_tokens), "%s: attention requires at least one KV token", what);
  TT_REQUIRE(tokens_dev == nullptr || (tokens >= 0 && tokens <= 1), "%s: device token count offset must be 0 or 1", what);
  TT_REQUIRE(max_tokens > 0, "%s: bad max_tokens", what);
  const int64_t chunks = (max_tokens + kChunk - 1) / kChunk;
  TT_REQUIRE(scratch_floats >= kAttnCounters + heads * chunks * (2 + head_dim), "%s: scratch too small", what);
  int* counters = kv_heads <= kAttnCounters ? reinterpret_cast<int*>(scratch) : nullptr;
  scratch += kAttnCounters;
  TT_REQUIRE(chunks <= 65535 && kv_heads <= 65535, "%s: sequence too long", what);
  AttnParams P{};
  P.q = q; P.keys = keys; P.values = values;
  P.k_head = k_head; P.k_tok = k_tok; P.v_head = v_head; P.v_tok = v_tok;
  P.sinks = sinks; P.tokens_dev = tokens_dev; P.tokens = (int)tokens;
  P.part_m = scratch;
  P.part_l = scratch + heads * chunks;
  P.part_o = scratch + 2 * heads * chunks;
  P.heads = (int)heads; P.kv_heads = (int)kv_heads; P.head_dim = (int)head_dim; P.max_chunks = (int)chunks;
  P.max_tokens = (int)max_tokens;
  P.scale = (float)(1.0 / __builtin_sqrt((double)head_dim));
  P.out = out;
  const int G = (int)(heads / kv_heads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // 128-bit K loads and whole-chunk V loads need contiguous 64-wide rows and a
  // capacity that is a whole number of chunks
  const bool c64 = head_dim == 64 && k_tok == 64 && v_tok == 64 && max_tokens % kChunk == 0 && aligned(keys, 16) &&
                   k_head % 8 == 0 && v_head % 8 == 0 && heads / kv_heads <= 8;
  auto by_g = [&](auto t) -> int {
    using T = decltype(t);
    switch (G) {
      case 1: return launch_attn<T, 1>(P, sink_dtype, c64, counters, st);
      case 2: return launch_attn<T, 2>(P, sink_dtype, c64, counters, st);
      case 4: return launch_attn<T, 4>(P, sink_dtype, c64, counters, st);
      case 8: return launch_attn<T, 8>(P, sink_dtype, c64, counters, st);
      case 16: return launch_attn<T, 16>(P, sink_dtype, c64, counters, st);
    }
    set_error("%s: query heads per KV head must be 1, 2, 4, 8 or 16 (got %d)", what, G);
    return TT_ERR_UNSUPPORTED;
  };
  if (dtype == TT_F16) return by_g(f16_t{});
  if (dtype == TT_BF16) return by_g(bf16_t{});
  set_error("%s: KV dtype must be fp16 or bf16", what);
  return TT_ERR_INVALID;
}
