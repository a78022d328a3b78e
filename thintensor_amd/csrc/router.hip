// MoE router for gfx950: router GEMV + bias + top-k + softmax in one launch
// (triton_kernels.py:2855-2921), and top-k + softmax on given logits
// (triton_kernels.py:2821-2851).
//
//   logit_e = bf16(dot_e) (+ bias_e, rounded to bf16 again) -- the reference rounds
//             through bfloat16 whatever the activation dtype;
//   dot_e   = GEMV row in the library order with 64 lanes per row;
//   top-k   = iterated argmax, lowest index on ties;
//   score_i = exp(v_i - max_all) / D, D summed in slot order over the selected
//             experts (renormalize) or in expert order over all experts.
// Indices are written as int32 and stay on the device.
#include "tt_abi_internal.h"
#include "tt_common.h"
#include "tt_gemv.h"
#include "tt_topk.h"

#include <type_traits>

namespace tt {

template <typename T> __device__ __forceinline__ float ldv(const void* p, int64_t i) {
  return to_f32(reinterpret_cast<const T*>(p)[i]);
}

// Top-k + softmax of one wave's logits (wave_topk_lanes), written out: slot s's expert
// to idx_out[s] and its score to score_out[s].
template <typename OT>
__device__ void wave_topk(float lg0, float lg1, int E, int top_k, bool renorm, int32_t* idx_out, OT* score_out) {
  const int lane = lane_id();
  const TopkLanes r = wave_topk_lanes(lg0, lg1, E, top_k, renorm);
  if (lane < top_k) {
    idx_out[lane] = r.idx0;
    store<OT>(score_out + lane, r.score0);
  }
  if (lane + 64 < top_k) {
    idx_out[lane + 64] = r.idx1;
    store<OT>(score_out + lane + 64, r.score1);
  }
}

// Rows of E <= 32 experts with H <= 4096 (two rounds of 64 lanes): every wave requests
// the weights of both of its experts and the activation chunks of both rounds before
// the first wait (chunk indices clamped, contributions masked), then reduces as the
// general loop below does.
template <typename WT, typename XT, typename BT>
__device__ __forceinline__ void router_rows_held(const void* w, int64_t w_row, const void* x, int H, const void* bias,
                                                 int E, int wave, int lane, float (&lg)[2]) {
  constexpr Fmt F = std::is_same_v<WT, bf16_t> ? Fmt::kBF16W : Fmt::kF16W;
  const int nchunks = H >> 5;
  Raw<64> wr[2][2], xr[2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    int j = r * 64 + lane;
    j = j < nchunks ? j : nchunks - 1;
    xr[r] = load_raw<64>(reinterpret_cast<const uint8_t*>(x) + (int64_t)32 * j * 2);
#pragma unroll
    for (int k = 0; k < 2; k++) {
      int e = wave + 16 * k;
      e = e < E ? e : E - 1;
      wr[k][r] = load_raw<64>(reinterpret_cast<const uint8_t*>(w) + ((int64_t)e * w_row + 32 * j) * 2);
    }
  }
  BT braw[2];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int e = wave + 16 * k;
    if (bias != nullptr) braw[k] = reinterpret_cast<const BT*>(bias)[e < E ? e : E - 1];
  }
  __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the first use
#pragma unroll
  for (int k = 0; k < 2; k++) {
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const bool cv = r * 64 + lane < nchunks;
      const float p = chunk_dot<F, XT>(wr[k][r], xr[r].w);
      if (r == 0 || (nchunks > 64)) acc = acc + (cv ? p : 0.0f);
    }
    // logit = bf16(dot) (+ bias, rounded to bf16 again)
    float v = round_bf16(xor_sum(acc, 1, 64));
    if (bias != nullptr) v = round_bf16(v + to_f32(braw[k]));
    lg[k] = v;
  }
}

template <typename WT, typename XT, typename BT, typename OT>
__global__ __launch_bounds__(1024) void router_kernel(const void* w, int64_t w_row, const void* x, int H, const void* bias,
                                                      int E, int top_k, int renorm, int32_t* idx_out, void* score_out) {
  __shared__ float logits[128];
  constexpr Fmt F = std::is_same_v<WT, bf16_t> ? Fmt::kBF16W : Fmt::kF16W;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int nchunks = H >> 5;
  const int rounds = (nchunks + 63) / 64;
  if (E <= 32 && nchunks <= 128 && nwaves == 16) {
    float lg[2];
    router_rows_held<WT, XT, BT>(w, w_row, x, H, bias, E, wave, lane, lg);
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int e = wave + 16 * k;
      if (e < E && lane == 0) logits[e] = lg[k];
    }
    __syncthreads();
    if (wave == 0) {
      const float l0 = lane < E ? logits[lane] : 0.0f;
      wave_topk<OT>(l0, 0.0f, E, top_k, renorm != 0, idx_out, reinterpret_cast<OT*>(score_out));
    }
    return;
  }
  for (int e = wave; e < E; e += nwaves) {
    float acc = 0.0f;
    for (int r = 0; r < rounds; r++) {
      const int j = r * 64 + lane;
      float p = 0.0f;
      if (j < nchunks) {
        const Raw<64> wr = load_raw<64>(reinterpret_cast<const uint8_t*>(w) + ((int64_t)e * w_row + 32 * j) * 2);
        const Raw<64> xr = load_raw<64>(reinterpret_cast<const uint8_t*>(x) + (int64_t)32 * j * 2);
        p = chunk_dot<F, XT>(wr, xr.w);
      }
      acc = acc + p;
    }
    acc = xor_sum(acc, 1, 64);
    float lg = round_bf16(acc);
    if (bias != nullptr) lg = round_bf16(lg + ldv<BT>(bias, e));
    if (lane == 0) logits[e] = lg;
  }
  __syncthreads();
  if (wave == 0) {
    const float l0 = lane < E ? logits[lane] : 0.0f;
    const float l1 = lane + 64 < E ? logits[lane + 64] : 0.0f;
    wave_topk<OT>(l0, l1, E, top_k, renorm != 0, idx_out, reinterpret_cast<OT*>(score_out));
  }
}

// add+RMSNorm and the router on its output in one workgroup (E <= 32, H <= 4096, one
// activation dtype).  Every wave requests the weight rows of its two experts (wave and
// wave + 16) and their bias right after the norm inputs (16-byte pieces staged through
// LDS); waves 0-3 form the residual and the normalized vector with the thread
// partition, reduction order and rounding points of add_rms_norm_kernel (ops.hip)
// while the weights are still arriving.  The normalized vector is stored
// (norm_out, residual_out) and kept in LDS, from which the router rows read their
// activations.  Same bits as tt_add_rms_norm followed by tt_moe_router_matvec_topk on
// norm_out.
struct NormRouterParams {
  const void* left;
  const void* right;
  void* residual_out;
  const void* norm_w;
  void* norm_out;
  const void* w;       // router weight [E, H], row stride w_row elements
  const void* bias;    // [E] or nullptr
  int32_t* idx_out;
  void* score_out;
  int64_t w_row;
  float eps;
  int H, E, top_k, renorm;
  float* logits_out;   // split kernel only: when set, the logits [tokens, E] go here and the top-k is left to the caller
};

constexpr int kNormRouterExperts = 32;   // 16 waves x 2 experts

template <typename WT, typename XT, typename BT, typename OT>
__global__ __launch_bounds__(1024) void norm_router_kernel(const NormRouterParams P) {
  constexpr Fmt F = std::is_same_v<WT, bf16_t> ? Fmt::kBF16W : Fmt::kF16W;
  __shared__ float red[4];
  __shared__ float logits[kNormRouterExperts];
  __shared__ uint4 xs[4096 / 8];   // normalized vector, XT bits
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int n = P.H;
  const int nchunks = n >> 5;
  const bool norm_wave = wave < 4;
  // token blockIdx.x of a [tokens, H] batch (one workgroup per token)
  const int64_t tok = blockIdx.x;
  const XT* const left = reinterpret_cast<const XT*>(P.left) + tok * n;
  const XT* const right = reinterpret_cast<const XT*>(P.right) + tok * n;
  XT* const residual_out = reinterpret_cast<XT*>(P.residual_out) + tok * n;
  XT* const norm_out = reinterpret_cast<XT*>(P.norm_out) + tok * n;
  int32_t* const idx_out = P.idx_out + tok * P.top_k;
  OT* const score_out = reinterpret_cast<OT*>(P.score_out) + tok * P.top_k;

  // ---- every load before the first wait: the norm inputs as 16-byte pieces (threads
  // 0-511, one piece of each vector; n <= 4096), then this wave's router rows and bias
  __shared__ uint4 raw_a[512], raw_b[512], raw_w[512];   // left, right, norm weight (raw bits)
  static_assert(kNormPieces * 256 == 512, "the staging buffers hold whole vectors");
  const int nq = n >> 3;
  // every thread loads (threads past the vector repeat its last piece), so no branch
  // separates these loads from the weight loads below
  const int q = (int)threadIdx.x < nq ? (int)threadIdx.x : nq - 1;
  const uint4 in_a = reinterpret_cast<const uint4*>(left)[q];
  const uint4 in_b = reinterpret_cast<const uint4*>(right)[q];
  const uint4 in_w = reinterpret_cast<const uint4*>(P.norm_w)[q];
  Raw<64> wr[2][2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    int j = r * 64 + lane;
    j = j < nchunks ? j : nchunks - 1;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      int e = wave + 16 * k;
      e = e < P.E ? e : P.E - 1;
      wr[k][r] = load_raw<64>(reinterpret_cast<const uint8_t*>(P.w) + ((int64_t)e * P.w_row + 32 * j) * 2);
    }
  }
  // bias loads without a branch: with no bias they read (and discard) the first elements
  // of the weight matrix, which holds at least E * H >= 2E halves
  const BT* bsrc = reinterpret_cast<const BT*>(P.bias != nullptr ? P.bias : P.w);
  BT braw[2];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int e = wave + 16 * k;
    braw[k] = bsrc[e < P.E ? e : P.E - 1];
  }
  __builtin_amdgcn_sched_barrier(0);
  if ((int)threadIdx.x < nq) {
    raw_a[threadIdx.x] = in_a;
    raw_b[threadIdx.x] = in_b;
    raw_w[threadIdx.x] = in_w;
  }
  __syncthreads();

  // ---- add + RMSNorm in add_rms_norm_kernel's piece partition and order: thread t of
  // waves 0-3 takes pieces t, t + 256 of 8 elements, fma chain in element order, wave
  // butterfly, (w0 + w1) + (w2 + w3)
  const int t = threadIdx.x;
  float res[kNormPieces][8];
  if (norm_wave) {
    uint4 pa[kNormPieces], pb[kNormPieces];
#pragma unroll
    for (int k = 0; k < kNormPieces; k++) {
      const int pi = t + 256 * k;
      const int pc = pi < nq ? pi : nq - 1;
      pa[k] = raw_a[pc];
      pb[k] = raw_b[pc];
    }
    __builtin_amdgcn_sched_barrier(0);   // every LDS read issued before the first use
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormPieces; k++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        res[k][e] = round_bf16(piece_f32<XT>(pa[k], e) + piece_f32<XT>(pb[k], e));
        if (8 * (t + 256 * k) + e < n) ss = __builtin_fmaf(res[k][e], res[k][e], ss);
      }
    ss = xor_sum(ss, 1, 64);
    if (lane == 0) red[wave] = ss;
  }
  __syncthreads();
  if (norm_wave) {
    const float total = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / __builtin_sqrtf(total / (float)n + P.eps);
#pragma unroll
    for (int k = 0; k < kNormPieces; k++) {
      const int pi = t + 256 * k;
      if (pi < nq) {
        const uint4 wv = raw_w[pi];
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = (res[k][e] * inv) * piece_f32<XT>(wv, e);
        const uint4 op = pack_piece<XT>(o);
        reinterpret_cast<uint4*>(residual_out)[pi] = pack_piece<XT>(res[k]);
        reinterpret_cast<uint4*>(norm_out)[pi] = op;
        xs[pi] = op;
      }
    }
  }
  __syncthreads();

  // ---- router rows (router_rows_held's arithmetic) on the normalized vector from LDS
  float acc[2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    int j = r * 64 + lane;
    j = j < nchunks ? j : nchunks - 1;
    Raw<64> xr;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint4 v = xs[j * 4 + q];
      xr.w[4 * q] = v.x;
      xr.w[4 * q + 1] = v.y;
      xr.w[4 * q + 2] = v.z;
      xr.w[4 * q + 3] = v.w;
    }
    const bool cv = r * 64 + lane < nchunks;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const float p = chunk_dot<F, XT>(wr[k][r], xr.w);
      if (r == 0) acc[k] = 0.0f + (cv ? p : 0.0f);
      else if (nchunks > 64) acc[k] = acc[k] + (cv ? p : 0.0f);
    }
  }
#pragma unroll
  for (int k = 0; k < 2; k++) {
    float v = round_bf16(xor_sum(acc[k], 1, 64));
    if (P.bias != nullptr) v = round_bf16(v + to_f32(braw[k]));
    const int e = wave + 16 * k;
    if (e < P.E && lane == 0) logits[e] = v;
  }
  __syncthreads();
  if (wave == 0) {
    const float l0 = lane < P.E ? logits[lane] : 0.0f;
    wave_topk<OT>(l0, 0.0f, P.E, P.top_k, P.renorm != 0, idx_out, score_out);
  }
}

// The same operator over ceil(E / 4) workgroups of four waves per token: every
// workgroup forms the residual and the normalized vector itself (the norm inputs are a
// few KB; same partition, order and rounding as add_rms_norm_kernel, so every copy has
// the same bits) while its waves' router rows arrive, wave w of workgroup g computes
// expert 4 g + w, and the workgroup stores its logits in the token's workspace slot
// and counts itself in the slot's arrival counter.  The last workgroup to arrive reads
// the E logits, takes the top-k and resets the counter to zero; no workgroup waits for
// another.  Logits and counters use device-scope atomic loads and stores, coherent
// across the XCDs' caches; a workgroup's logit stores have completed (vector memory
// counter drained) before it counts itself.  Workgroup 0 stores residual_out and
// norm_out.  Same bits as norm_router_kernel.
constexpr int kNormRouterSlot = 64;   // ints per token: counter at 0, logits at 32 + e

template <typename WT, typename XT, typename BT, typename OT>
__global__ __launch_bounds__(256) void norm_router_split_kernel(const NormRouterParams P, int* ws) {
  constexpr Fmt F = std::is_same_v<WT, bf16_t> ? Fmt::kBF16W : Fmt::kF16W;
  __shared__ float red[4];
  __shared__ int last;
  __shared__ uint4 xs[4096 / 8];   // normalized vector, XT bits
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int n = P.H;
  const int nchunks = n >> 5;
  const int64_t tok = blockIdx.y;
  const XT* const left = reinterpret_cast<const XT*>(P.left) + tok * n;
  const XT* const right = reinterpret_cast<const XT*>(P.right) + tok * n;
  int* const slot = ws + tok * kNormRouterSlot;

  // ---- every load before the first wait: the norm inputs (kNormPieces 16-byte pieces
  // of each vector per thread), then this wave's router row and bias
  const int nq = n >> 3;
  const int t = threadIdx.x;
  uint4 pa[kNormPieces], pb[kNormPieces], pw[kNormPieces];
#pragma unroll
  for (int k = 0; k < kNormPieces; k++) {
    const int pi = t + 256 * k;
    const int pc = pi < nq ? pi : nq - 1;
    pa[k] = reinterpret_cast<const uint4*>(left)[pc];
    pb[k] = reinterpret_cast<const uint4*>(right)[pc];
    pw[k] = reinterpret_cast<const uint4*>(P.norm_w)[pc];
  }
  const int e = 4 * blockIdx.x + wave;
  const int er = e < P.E ? e : P.E - 1;
  Raw<64> wr[2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    int j = r * 64 + lane;
    j = j < nchunks ? j : nchunks - 1;
    wr[r] = load_raw<64>(reinterpret_cast<const uint8_t*>(P.w) + ((int64_t)er * P.w_row + 32 * j) * 2);
  }
  const BT* bsrc = reinterpret_cast<const BT*>(P.bias != nullptr ? P.bias : P.w);
  const BT braw = bsrc[er];
  __builtin_amdgcn_sched_barrier(0);

  // ---- add + RMSNorm in add_rms_norm_kernel's partition and order
  float res[kNormPieces][8];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < kNormPieces; k++)
#pragma unroll
    for (int c = 0; c < 8; c++) {
      res[k][c] = round_bf16(piece_f32<XT>(pa[k], c) + piece_f32<XT>(pb[k], c));
      if (8 * (t + 256 * k) + c < n) ss = __builtin_fmaf(res[k][c], res[k][c], ss);
    }
  ss = xor_sum(ss, 1, 64);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / __builtin_sqrtf(total / (float)n + P.eps);
  XT* const residual_out = reinterpret_cast<XT*>(P.residual_out) + tok * n;
  XT* const norm_out = reinterpret_cast<XT*>(P.norm_out) + tok * n;
#pragma unroll
  for (int k = 0; k < kNormPieces; k++) {
    const int pi = t + 256 * k;
    if (pi < nq) {
      float o[8];
#pragma unroll
      for (int c = 0; c < 8; c++) o[c] = (res[k][c] * inv) * piece_f32<XT>(pw[k], c);
      const uint4 op = pack_piece<XT>(o);
      if (blockIdx.x == 0) {
        reinterpret_cast<uint4*>(residual_out)[pi] = pack_piece<XT>(res[k]);
        reinterpret_cast<uint4*>(norm_out)[pi] = op;
      }
      xs[pi] = op;
    }
  }
  __syncthreads();

  // ---- this wave's router row (router_rows_held's arithmetic) on the vector in LDS
  float acc = 0.0f;
#pragma unroll
  for (int r = 0; r < 2; r++) {
    int j = r * 64 + lane;
    j = j < nchunks ? j : nchunks - 1;
    Raw<64> xr;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint4 v = xs[j * 4 + q];
      xr.w[4 * q] = v.x;
      xr.w[4 * q + 1] = v.y;
      xr.w[4 * q + 2] = v.z;
      xr.w[4 * q + 3] = v.w;
    }
    const bool cv = r * 64 + lane < nchunks;
    const float p = chunk_dot<F, XT>(wr[r], xr.w);
    if (r == 0) acc = 0.0f + (cv ? p : 0.0f);
    else if (nchunks > 64) acc = acc + (cv ? p : 0.0f);
  }
  float v = round_bf16(xor_sum(acc, 1, 64));
  if (P.bias != nullptr) v = round_bf16(v + to_f32(braw));
  if (P.logits_out != nullptr) {
    // logits only: the kernel that consumes them runs the top-k (wave_topk_lanes) itself
    if (e < P.E && lane == 0) P.logits_out[tok * P.E + e] = v;
    return;
  }
  if (e < P.E && lane == 0)
    __hip_atomic_store(reinterpret_cast<float*>(slot) + 32 + e, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(slot, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int)gridDim.x - 1;
  __syncthreads();
  if (!last || wave != 0) return;
  const float l0 = lane < P.E
                       ? __hip_atomic_load(reinterpret_cast<float*>(slot) + 32 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                       : 0.0f;
  wave_topk<OT>(l0, 0.0f, P.E, P.top_k, P.renorm != 0, P.idx_out + tok * P.top_k,
                reinterpret_cast<OT*>(P.score_out) + tok * P.top_k);
  if (lane == 0) __hip_atomic_store(slot, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename LT, typename OT>
__global__ __launch_bounds__(64) void topk_kernel(const void* logits_in, int E, int top_k, int renorm, int32_t* idx_out,
                                                  void* score_out) {
  const int lane = lane_id();
  const float l0 = lane < E ? ldv<LT>(logits_in, lane) : 0.0f;
  const float l1 = lane + 64 < E ? ldv<LT>(logits_in, lane + 64) : 0.0f;
  wave_topk<OT>(l0, l1, E, top_k, renorm != 0, idx_out, reinterpret_cast<OT*>(score_out));
}

// Top-k + softmax over 128 < E <= kTopkMaxExperts logits in one 256-thread workgroup:
// the reference kernel has no expert cap (triton_kernels.py:2821-2851) and the runtime
// calls it exactly when the router has more than 128 rows (gpu_runtime.py:9474-9496).
// Same selection rule and summation order as wave_topk: slot s takes the first untaken
// expert when its logit is NaN, otherwise the untaken expert of the largest non-NaN key
// (lowest index among equal values); taken experts are bits of an LDS mask.  The logits
// are re-read on every slot (cache hits after the first pass).  The denominator is summed
// sequentially in slot order (renormalize) or in expert order by wave 0.
constexpr int kTopkMaxExperts = 65536;
constexpr int kTopkMaxSlots = 4096;

template <typename LT, typename OT>
__global__ __launch_bounds__(256) void topk_block_kernel(const void* logits_in, int E, int top_k, int renorm,
                                                         int32_t* idx_out, void* score_out) {
  __shared__ uint32_t taken[kTopkMaxExperts / 32];
  __shared__ float sel_v[kTopkMaxSlots];
  __shared__ uint64_t red_k[4];
  __shared__ uint32_t red_f[4];
  __shared__ float red_m[4];
  const int t = threadIdx.x, lane = lane_id(), wave = t >> 6;
  for (int i = t; i < (E + 31) / 32; i += 256) taken[i] = 0u;
  float m = __builtin_bit_cast(float, 0xff800000u);
  for (int e = t; e < E; e += 256) m = fmaxf(m, ldv<LT>(logits_in, e));
  m = fmaxf(m, xor_partner<1>(m));
  m = fmaxf(m, xor_partner<2>(m));
  m = fmaxf(m, xor_partner<4>(m));
  m = fmaxf(m, xor_partner<8>(m));
  m = fmaxf(m, xor_partner<16>(m));
  m = fmaxf(m, xor_partner<32>(m));
  if (lane == 0) red_m[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
  float den = 0.0f;
  for (int s = 0; s < top_k; s++) {
    uint64_t k = 0;
    uint64_t f = 0;
    for (int e = t; e < E; e += 256) {
      if (taken[e >> 5] & (1u << (e & 31))) continue;
      const uint64_t fe = 0xffffffffu - (uint32_t)e;
      f = fe > f ? fe : f;
      const float v = ldv<LT>(logits_in, e);
      if (!__builtin_isnan(v)) {
        const uint64_t key = topk_key(v, (uint32_t)e);
        k = key > k ? key : k;
      }
    }
    k = wave_max_u64(k);
    f = wave_max_u64(f);
    if (lane == 0) {
      red_k[wave] = k;
      red_f[wave] = (uint32_t)f;
    }
    __syncthreads();
    k = red_k[0];
    uint32_t fb = red_f[0];
#pragma unroll
    for (int w = 1; w < 4; w++) {
      k = red_k[w] > k ? red_k[w] : k;
      fb = red_f[w] > fb ? red_f[w] : fb;
    }
    const int first = (int)(0xffffffffu - fb);
    const float fv = ldv<LT>(logits_in, first);
    const int bi = __builtin_isnan(fv) ? first : (int)(0xffffffffu - (uint32_t)k);
    const float bv = ldv<LT>(logits_in, bi);
    if (renorm) den = den + exp_f32(bv - m);
    if (t == 0) {
      idx_out[s] = bi;
      sel_v[s] = bv;
      taken[bi >> 5] |= 1u << (bi & 31);
    }
    __syncthreads();
  }
  if (!renorm) {
    if (wave == 0) {
      for (int b = 0; b < E; b += 64) {
        const float a = b + lane < E ? exp_f32(ldv<LT>(logits_in, b + lane) - m) : 0.0f;
        const int n = E - b < 64 ? E - b : 64;
        for (int j = 0; j < n; j++) den = den + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), j));
      }
      if (lane == 0) red_m[0] = den;
    }
    __syncthreads();
    den = red_m[0];
  }
  for (int s = t; s < top_k; s += 256) store<OT>(reinterpret_cast<OT*>(score_out) + s, exp_f32(sel_v[s] - m) / den);
}

template <typename Fn> static int dt3(int code, Fn&& f) {
  if (code == TT_F16) return f(f16_t{});
  if (code == TT_BF16) return f(bf16_t{});
  if (code == TT_F32) return f(float{});
  set_error("unsupported dtype code %d", code);
  return TT_ERR_INVALID;
}

}  // namespace tt

using namespace tt;

extern "C" int tt_moe_router_matvec_topk(const void* weight, int w_dtype, int64_t w_row, const void* hidden,
                                         int x_dtype, int64_t hidden_size, const void* bias, int bias_dtype,
                                         int64_t experts, int64_t top_k, int renormalize, int32_t* indices_out,
                                         void* scores_out, int score_dtype, void* stream) {
  const char* what = "moe_router_matvec_topk";
  TT_REQUIRE(experts > 0 && experts <= 128, "%s: fused router supports at most 128 experts", what);
  TT_REQUIRE(top_k > 0 && top_k <= experts, "%s: top_k must be in [1, experts]", what);
  TT_REQUIRE(hidden_size > 0 && hidden_size % 32 == 0, "%s: hidden size must be a multiple of 32", what);
  TT_REQUIRE(weight && hidden && indices_out && scores_out, "%s: null pointer", what);
  TT_REQUIRE(aligned(weight, 16) && aligned(hidden, 16) && w_row % 8 == 0, "%s: weight rows and hidden must be 16-byte aligned", what);
  const int bdt = bias ? bias_dtype : TT_F32;
  return dt3(w_dtype, [&](auto wt) {
    using WT = decltype(wt);
    return dt3(x_dtype, [&](auto xt) {
      using XT = decltype(xt);
      return dt3(bdt, [&](auto bt) {
        using BT = decltype(bt);
        return dt3(score_dtype, [&](auto ot) {
          using OT = decltype(ot);
          if constexpr (std::is_same_v<WT, float> || std::is_same_v<XT, float>) {
            set_error("%s: router weight and hidden must be fp16 or bf16", what);
            return TT_ERR_UNSUPPORTED;
          } else {
            hipLaunchKernelGGL((router_kernel<WT, XT, BT, OT>), dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                               weight, w_row, hidden, (int)hidden_size, bias, (int)experts, (int)top_k, renormalize,
                               indices_out, scores_out);
            return check_launch(what);
          }
        });
      });
    });
  });
}

extern "C" int tt_moe_router_topk(const void* logits, int logits_dtype, int64_t experts, int64_t top_k, int renormalize,
                                  int32_t* indices_out, void* scores_out, int score_dtype, void* stream) {
  const char* what = "moe_router_topk";
  TT_REQUIRE(experts > 0 && top_k > 0 && top_k <= experts, "%s: bad expert counts", what);
  TT_UNSUPPORTED(experts <= kTopkMaxExperts && (experts <= 128 || top_k <= kTopkMaxSlots),
                 "%s: at most %d experts and, above 128 experts, %d slots", what, kTopkMaxExperts, kTopkMaxSlots);
  TT_REQUIRE(logits && indices_out && scores_out, "%s: null pointer", what);
  return dt3(logits_dtype, [&](auto lt) {
    using LT = decltype(lt);
    return dt3(score_dtype, [&](auto ot) {
      using OT = decltype(ot);
      if (experts <= 128)
        hipLaunchKernelGGL((topk_kernel<LT, OT>), dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), logits,
                           (int)experts, (int)top_k, renormalize, indices_out, scores_out);
      else
        hipLaunchKernelGGL((topk_block_kernel<LT, OT>), dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream),
                           logits, (int)experts, (int)top_k, renormalize, indices_out, scores_out);
      return check_launch(what);
    });
  });
}

extern "C" int64_t tt_norm_router_workspace_bytes(int64_t tokens) {
  return tokens > 0 ? tokens * kNormRouterSlot * (int64_t)sizeof(int) : 0;
}

extern "C" int tt_add_rms_norm_router_topk(const void* left, const void* right, void* residual_out, int x_dtype,
                                           const void* norm_weight, int norm_w_dtype, void* norm_out, int norm_dtype,
                                           int64_t hidden_size, float eps, const void* weight, int w_dtype,
                                           int64_t w_row, const void* bias, int bias_dtype, int64_t experts,
                                           int64_t top_k, int renormalize, int32_t* indices_out, void* scores_out,
                                           int score_dtype, int64_t tokens, void* workspace, int64_t workspace_bytes,
                                           void* stream) {
  const char* what = "add_rms_norm_router_topk";
  TT_REQUIRE(tokens >= 1 && tokens <= 65535, "%s: bad token count", what);
  TT_REQUIRE(left && right && residual_out && norm_weight && norm_out, "%s: null pointer", what);
  const bool one_launch = experts <= kNormRouterExperts && hidden_size <= 4096 && hidden_size % 32 == 0 && hidden_size > 0 &&
                          x_dtype != TT_F32 && norm_w_dtype == x_dtype && norm_dtype == x_dtype &&
                          (w_dtype == TT_F16 || w_dtype == TT_BF16) && weight && indices_out && scores_out &&
                          aligned(weight, 16) && w_row % 8 == 0 && experts > 0 && top_k > 0 && top_k <= experts &&
                          aligned(left, 16) && aligned(right, 16) && aligned(residual_out, 16) &&
                          aligned(norm_weight, 16) && aligned(norm_out, 16);
  if (!one_launch) {
    // the two operators per token, each with its own checks
    const int64_t xs = hidden_size * (x_dtype == TT_F32 ? 4 : 2), ns = hidden_size * (norm_dtype == TT_F32 ? 4 : 2);
    const int64_t ss = top_k * (score_dtype == TT_F32 ? 4 : 2);
    for (int64_t t = 0; t < tokens; t++) {
      auto at = [t](const void* p, int64_t bytes) { return static_cast<const char*>(p) + t * bytes; };
      int rc = tt_add_rms_norm(at(left, xs), at(right, xs), const_cast<char*>(at(residual_out, xs)), x_dtype, norm_weight,
                               norm_w_dtype, const_cast<char*>(at(norm_out, ns)), norm_dtype, hidden_size, eps, stream);
      if (rc != TT_OK) return rc;
      rc = tt_moe_router_matvec_topk(weight, w_dtype, w_row, at(norm_out, ns), norm_dtype, hidden_size, bias, bias_dtype,
                                     experts, top_k, renormalize, indices_out + t * top_k,
                                     const_cast<char*>(at(scores_out, ss)), score_dtype, stream);
      if (rc != TT_OK) return rc;
    }
    return TT_OK;
  }
  NormRouterParams P;
  P.left = left; P.right = right; P.residual_out = residual_out; P.norm_w = norm_weight; P.norm_out = norm_out;
  P.w = weight; P.bias = bias; P.idx_out = indices_out; P.score_out = scores_out; P.w_row = w_row; P.eps = eps;
  P.H = (int)hidden_size; P.E = (int)experts; P.top_k = (int)top_k; P.renorm = renormalize;
  P.logits_out = nullptr;
  const int bdt = bias ? bias_dtype : TT_F32;
  return dt3(w_dtype, [&](auto wt) {
    using WT = decltype(wt);
    return dt3(x_dtype, [&](auto xt) {
      using XT = decltype(xt);
      return dt3(bdt, [&](auto bt) {
        using BT = decltype(bt);
        return dt3(score_dtype, [&](auto ot) {
          using OT = decltype(ot);
          if constexpr (std::is_same_v<WT, float> || std::is_same_v<XT, float>) {
            set_error("%s: unsupported dtypes", what);
            return TT_ERR_UNSUPPORTED;
          } else {
            if (workspace != nullptr && workspace_bytes >= tt_norm_router_workspace_bytes(tokens) &&
                aligned(workspace, 4)) {
              hipLaunchKernelGGL((norm_router_split_kernel<WT, XT, BT, OT>), dim3((unsigned)((experts + 3) / 4),
                                 (unsigned)tokens), dim3(256), 0, static_cast<hipStream_t>(stream), P,
                                 static_cast<int*>(workspace));
            } else {
              hipLaunchKernelGGL((norm_router_kernel<WT, XT, BT, OT>), dim3((unsigned)tokens), dim3(1024), 0,
                                 static_cast<hipStream_t>(stream), P);
            }
            return check_launch(what);
          }
        });
      });
    });
  });
}

// add_rms_norm + router logits, one launch of ceil(experts / 4) workgroups per token with
// no finishing step: logits_out[t * experts + e] is the logit tt_add_rms_norm_router_topk
// ranks (bf16-rounded dot, plus the bias rounded again); the decode step's SwiGLU kernel
// runs the top-k on them (tt_mxfp_lowbit_selected_swiglu_router).
extern "C" int tt_add_rms_norm_router_logits(const void* left, const void* right, void* residual_out, int x_dtype,
                                             const void* norm_weight, int norm_w_dtype, void* norm_out, int norm_dtype,
                                             int64_t hidden_size, float eps, const void* weight, int w_dtype,
                                             int64_t w_row, const void* bias, int bias_dtype, int64_t experts,
                                             float* logits_out, int64_t tokens, void* stream) {
  const char* what = "add_rms_norm_router_logits";
  TT_REQUIRE(tokens >= 1 && tokens <= 65535, "%s: bad token count", what);
  TT_REQUIRE(left && right && residual_out && norm_weight && norm_out && weight && logits_out, "%s: null pointer", what);
  TT_UNSUPPORTED(experts >= 1 && experts <= kNormRouterExperts && hidden_size > 0 && hidden_size <= 4096 &&
                     hidden_size % 32 == 0,
                 "%s: 1..%d experts and hidden sizes up to 4096 (multiples of 32)", what, kNormRouterExperts);
  TT_REQUIRE(x_dtype != TT_F32 && norm_w_dtype == x_dtype && norm_dtype == x_dtype && (w_dtype == TT_F16 || w_dtype == TT_BF16),
             "%s: fp16 or bf16 vectors of one dtype and an fp16 or bf16 router", what);
  TT_REQUIRE(aligned(weight, 16) && w_row % 8 == 0 && w_row >= hidden_size && aligned(left, 16) && aligned(right, 16) &&
                 aligned(residual_out, 16) && aligned(norm_weight, 16) && aligned(norm_out, 16) && aligned(logits_out, 4),
             "%s: misaligned pointer or bad row stride", what);
  NormRouterParams P;
  P.left = left; P.right = right; P.residual_out = residual_out; P.norm_w = norm_weight; P.norm_out = norm_out;
  P.w = weight; P.bias = bias; P.idx_out = nullptr; P.score_out = nullptr; P.w_row = w_row; P.eps = eps;
  P.H = (int)hidden_size; P.E = (int)experts; P.top_k = 1; P.renorm = 0;
  P.logits_out = logits_out;
  const int bdt = bias ? bias_dtype : TT_F32;
  if (bias) TT_REQUIRE(bias_dtype == TT_F16 || bias_dtype == TT_BF16 || bias_dtype == TT_F32, "%s: bad bias dtype", what);
  return dt3(w_dtype, [&](auto wt) {
    using WT = decltype(wt);
    return dt3(x_dtype, [&](auto xt) {
      using XT = decltype(xt);
      return dt3(bdt, [&](auto bt) {
        using BT = decltype(bt);
        if constexpr (std::is_same_v<WT, float> || std::is_same_v<XT, float>) {
          set_error("%s: unsupported dtypes", what);
          return TT_ERR_UNSUPPORTED;
        } else {
          hipLaunchKernelGGL((norm_router_split_kernel<WT, XT, BT, float>), dim3((unsigned)((experts + 3) / 4),
                             (unsigned)tokens), dim3(256), 0, static_cast<hipStream_t>(stream), P, nullptr);
          return check_launch(what);
        }
      });
    });
  });
}
