// Shared device helpers for the ThinTensor decode kernels on gfx950 (CDNA4, wave64).
//
// Numerics contract used by every kernel in this library:
//   * only IEEE-754 binary32 operations with a single rounding are used for
//     accumulation: fmaf, +, *, correctly rounded / and sqrt.  No v_dot2 (its
//     internal accumulator truncates and cannot be reproduced on a CPU), no packed
//     fp32, no approximate transcendental instructions.
//   * every reduction has a fixed order that does not depend on the launch shape
//     beyond the documented "lanes per row" parameter, so a CPU restatement can
//     reproduce each output bit for bit.
//   * fp16/bf16 stores round to nearest even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tt {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

struct f16_t { uint16_t bits; };
struct bf16_t { uint16_t bits; };

__device__ __forceinline__ float to_f32(f16_t v) { return (float)__builtin_bit_cast(_Float16, v.bits); }
__device__ __forceinline__ float to_f32(bf16_t v) { return __builtin_bit_cast(float, (uint32_t)v.bits << 16); }
__device__ __forceinline__ float to_f32(float v) { return v; }

// A binary32 value pinned in a register.  Every conversion to fp16 goes through it:
// otherwise the compiler may fold the product or sum that feeds the conversion into one
// mixed-precision fma with an fp16 result (v_fma_mixlo_f16), which rounds once, straight
// to fp16, where the reference rounds to binary32 first and then to fp16 (the two
// differ when the binary32 rounding lands on an fp16 halfway point).
__device__ __forceinline__ float pin_f32(float f) {
  asm("" : "+v"(f));
  return f;
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)pin_f32(f)); }
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
// Round a binary32 value to bfloat16 and back (used where the reference rounds
// through bfloat16 regardless of the activation dtype).
__device__ __forceinline__ float round_bf16(float f) { return __builtin_bit_cast(float, (uint32_t)f32_to_bf16_bits(f) << 16); }
__device__ __forceinline__ float round_f16(float f) { return (float)(_Float16)pin_f32(f); }

template <typename T> struct Store;
template <> struct Store<f16_t> { __device__ static void st(f16_t* p, float v) { p->bits = f32_to_f16_bits(v); } };
template <> struct Store<bf16_t> { __device__ static void st(bf16_t* p, float v) { p->bits = f32_to_bf16_bits(v); } };
template <> struct Store<float> { __device__ static void st(float* p, float v) { *p = v; } };
template <typename T> __device__ __forceinline__ void store(T* p, float v) { Store<T>::st(p, v); }

// A wave-uniform pointer pinned to scalar registers.  A per-lane choice between two such
// pointers then compiles to a select; without it the compiler may instead turn the choice
// into a vector load of whichever kernel argument the lane picked, which queues behind
// every load issued before it.
template <typename T> __device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  // through the global address space, so that loads from it stay global (not flat) loads
  typedef __attribute__((address_space(1))) T GlobalT;
  return (T*)reinterpret_cast<GlobalT*>(((uint64_t)hi << 32) | lo);
}

// Round a value to the storage precision of T and return it as float.
template <typename T> __device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<f16_t>(float v) { return round_f16(v); }
template <> __device__ __forceinline__ float round_to<bf16_t>(float v) { return round_bf16(v); }
template <> __device__ __forceinline__ float round_to<float>(float v) { return v; }

// Two 16-bit activations packed in one 32-bit register -> binary32.
template <typename XT> __device__ __forceinline__ float lo_f32(uint32_t w);
template <typename XT> __device__ __forceinline__ float hi_f32(uint32_t w);
template <> __device__ __forceinline__ float lo_f32<f16_t>(uint32_t w) { return (float)__builtin_bit_cast(h2, w)[0]; }
template <> __device__ __forceinline__ float hi_f32<f16_t>(uint32_t w) { return (float)__builtin_bit_cast(h2, w)[1]; }
template <> __device__ __forceinline__ float lo_f32<bf16_t>(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
template <> __device__ __forceinline__ float hi_f32<bf16_t>(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// Exact xor partner: value of lane (lane ^ M) for M in {1,2,4,8,16,32}, for any
// lane values.  1 and 2 use DPP quad_perm, 4 two bank-masked DPP row shifts, 8 DPP
// row_ror:8 (== xor 8 inside a 16-lane row), 16 and 32 the gfx950 permlane swaps.
template <int M>
__device__ __forceinline__ float xor_partner(float v) {
  const int iv = __builtin_bit_cast(int, v);
  if constexpr (M == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false));
  else if constexpr (M == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false));
  else if constexpr (M == 4) {
    // banks 0,2 (lanes 0-3, 8-11 of each row) read lane+4 (row_shl:4); banks 1,3 read lane-4 (row_shr:4)
    int t = __builtin_amdgcn_update_dpp(iv, iv, 0x104, 0xF, 0x5, false);
    t = __builtin_amdgcn_update_dpp(t, iv, 0x114, 0xF, 0xA, false);
    return __builtin_bit_cast(float, t);
  } else if constexpr (M == 8) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x128, 0xF, 0xF, false));
  else if constexpr (M == 16) {
    auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 16) ? r[0] : r[1]);
  } else {
    auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
  }
}

// One butterfly level on lane bit M: v_i <- v_i + v_{i^M}.  IEEE addition is
// commutative, so lanes i and i^M produce identical bits.
template <int M> __device__ __forceinline__ float bfly(float v) { return v + xor_partner<M>(v); }

// Butterfly sum over lane bits [m_begin, m_end) (wave-uniform powers of two), levels
// in increasing order: every participating lane ends with
// T(a[0..n)) = T(a[0..n/2)) + T(a[n/2..n)).  All 64 lanes must be active.
__device__ __forceinline__ float xor_sum(float v, int m_begin, int m_end) {
  if (m_begin <= 1 && m_end > 1) v = bfly<1>(v);
  if (m_begin <= 2 && m_end > 2) v = bfly<2>(v);
  if (m_begin <= 4 && m_end > 4) v = bfly<4>(v);
  if (m_begin <= 8 && m_end > 8) v = bfly<8>(v);
  if (m_begin <= 16 && m_end > 16) v = bfly<16>(v);
  if (m_begin <= 32 && m_end > 32) v = bfly<32>(v);
  return v;
}

// Reduce-scatter level on lane bit M for NV per-lane values (one per row): lanes
// with bit M clear keep values [0, NV/2), lanes with it set keep [NV/2, NV); each
// kept value becomes own + partner's value of the same row.  The additions are the
// butterfly's additions for that row, only spread over fewer lanes.
template <int NV, int M>
__device__ __forceinline__ void rs_level(const float* in, float* out) {
  const bool hi = (threadIdx.x & M) != 0;
#pragma unroll
  for (int i = 0; i < NV / 2; i++) {
    const float keep = hi ? in[NV / 2 + i] : in[i];
    const float give = hi ? in[i] : in[NV / 2 + i];
    out[i] = keep + xor_partner<M>(give);
  }
}

// exp(x) for binary32, reproducible bit for bit on the CPU: Cody-Waite reduction
// x = n*ln2 + r (two-constant split), degree-7 Taylor polynomial of e^r in Horner
// form with fmaf, then an exact scaling by 2^n.  Relative error < 2 ulp on
// [-87, 88]; inputs below -87.3 return 0, above 88.7 return +inf.
__device__ __forceinline__ float exp_f32(float x) {
  if (x != x) return x;
  if (x < -0x1.5d589ep+6f) return 0.0f;
  if (x > 0x1.62e42ep+6f) return __builtin_bit_cast(float, 0x7f800000u);
  const float log2e = 0x1.715476p+0f;
  float n = __builtin_rintf(x * log2e);
  float r = __builtin_fmaf(n, -0x1.62e4p-1f, x);       // ln2 high part (n*hi is exact)
  r = __builtin_fmaf(n, -0x1.7f7d1cp-20f, r);    // ln2 low part
  float p = 0x1.a01a02p-13f;                    // 1/7!
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);    // 1/6!
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);     // 1/5!
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);     // 1/4!
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);     // 1/3!
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  // scale by 2^ni in two exact steps so that ni in [-126, 128] never overflows the
  // exponent field of an intermediate.
  int n1 = ni / 2, n2 = ni - n1;
  p = p * __builtin_bit_cast(float, (uint32_t)(n1 + 127) << 23);
  p = p * __builtin_bit_cast(float, (uint32_t)(n2 + 127) << 23);
  return p;
}

// 2^e for an integer e in [-149, 127], built exactly (subnormal below -126).
__device__ __forceinline__ float pow2i(int e) {
  if (e >= -126) return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23);
  return __builtin_bit_cast(float, 1u << (e + 149));
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Expert id of slot s from an index array of int32 (ishift 0) or int64 (ishift 1)
// elements, as the reference's kernels load whichever integer type they are given.
// Both 32-bit words are requested at once from addresses that depend only on the
// arguments (for int32 the second load repeats the first word, so nothing past the
// array is read); an int64 id keeps its high word, so an out-of-range id stays out
// of range.
__device__ __forceinline__ int64_t load_expert(const void* p, int ishift, int64_t s) {
  const int32_t* q = reinterpret_cast<const int32_t*>(p) + (s << ishift);
  const uint32_t lo = (uint32_t)q[0];
  const int32_t hi = q[ishift];
  return ishift ? (int64_t)(((uint64_t)(uint32_t)hi << 32) | lo) : (int64_t)(int32_t)lo;
}

// Maximum of a 64-bit key over the wave (every lane gets the result).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#define TT_MAXSTEP(M)                                                                                     \
  {                                                                                                       \
    const uint32_t hi = __builtin_bit_cast(uint32_t, xor_partner<M>(__builtin_bit_cast(float, (uint32_t)(k >> 32)))); \
    const uint32_t lo = __builtin_bit_cast(uint32_t, xor_partner<M>(__builtin_bit_cast(float, (uint32_t)k)));         \
    const uint64_t o = ((uint64_t)hi << 32) | lo;                                                         \
    k = o > k ? o : k;                                                                                    \
  }

  TT_MAXSTEP(1) TT_MAXSTEP(2) TT_MAXSTEP(4) TT_MAXSTEP(8) TT_MAXSTEP(16) TT_MAXSTEP(32)
#undef TT_MAXSTEP
  return k;
}

// Maximum of n >= 1 uint64 keys over a 256-thread block: eight loads per thread are in
// flight at a time (indices past n repeat the last key), then a wave maximum and one
// barrier.  Every thread returns the result.  The maximum is exact, so its order does
// not matter.
__device__ __forceinline__ uint64_t block_max_u64(const uint64_t* p, int n, uint64_t* red4) {
  uint64_t best = 0;
  for (int i0 = 0; i0 < n; i0 += 256 * 8) {
    uint64_t v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int i = i0 + (int)threadIdx.x + 256 * k;
      v[k] = p[i < n ? i : n - 1];
    }
#pragma unroll
    for (int k = 0; k < 8; k++) best = v[k] > best ? v[k] : best;
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = best;
  __syncthreads();
  uint64_t m = red4[0];
  m = red4[1] > m ? red4[1] : m;
  m = red4[2] > m ? red4[2] : m;
  m = red4[3] > m ? red4[3] : m;
  return m;
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also waits for
// every outstanding global load of the wave, which would drain a register prefetch
// pipeline at each barrier; this one leaves those loads in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <typename T> __device__ __forceinline__ float ld(const void* p, int64_t i) {
  return to_f32(reinterpret_cast<const T*>(p)[i]);
}

// Block-wide sum of a 256-thread workgroup in a fixed order: thread partials are
// reduced with the wave butterfly, then the four wave sums as (w0 + w1) + (w2 + w3).
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = xor_sum(v, 1, 64);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

// Residual element of add+RMSNorm: the reference rounds left + right through
// bfloat16 whatever the activation dtype (triton_kernels.py:2603-2606).
template <typename XT>
__device__ __forceinline__ float norm_residual(const void* left, const void* right, int64_t i) {
  return round_bf16(ld<XT>(left, i) + ld<XT>(right, i));
}

// RoPE on one (first-half, second-half) pair with rounding to T after every product
// and sum, as the reference's torch path (gpu_runtime.py:8696-8705):
// o1 = r(r(a c) - r(b s)), o2 = r(r(b c) + r(a s)); the caller's store rounds o1, o2.
template <typename T>
__device__ __forceinline__ void rope_pair(float a, float b, float c, float s, float& o1, float& o2) {
  const float ac = round_to<T>(a * c), bs = round_to<T>(b * s);
  const float bc = round_to<T>(b * c), as = round_to<T>(a * s);
  o1 = ac - bs;
  o2 = bc + as;
}

// ---------------------------------------------------------------- RMSNorm partition
// Every RMSNorm in the library (the standalone kernels and the fused prologues) cuts the
// vector into pieces of 8 elements (16 bytes of a 16-bit type); piece p belongs to thread
// p % 256 of the normalizing threads, and a thread's sum of squares is an fma chain over
// its elements in increasing index order, followed by block_sum256.  One 16-byte load
// brings a whole piece, and all implementations give the same bits.
constexpr int kNormPieces = 2;   // pieces per thread held in registers: vectors up to 4096

// element e (0..7) of a piece of a 16-bit type, as binary32
template <typename T>
__device__ __forceinline__ float piece_f32(const uint4& v, int e) {
  const uint32_t w = e < 2 ? v.x : (e < 4 ? v.y : (e < 6 ? v.z : v.w));
  return (e & 1) ? hi_f32<T>(w) : lo_f32<T>(w);
}

template <typename T> __device__ __forceinline__ uint32_t bits16(float v);
template <> __device__ __forceinline__ uint32_t bits16<f16_t>(float v) { return f32_to_f16_bits(v); }
template <> __device__ __forceinline__ uint32_t bits16<bf16_t>(float v) { return f32_to_bf16_bits(v); }

// eight binary32 values rounded to a 16-bit type and packed as one piece (as store<T>
// rounds them one at a time)
template <typename T>
__device__ __forceinline__ uint4 pack_piece(const float* v) {
  uint4 r;
  r.x = bits16<T>(v[0]) | (bits16<T>(v[1]) << 16);
  r.y = bits16<T>(v[2]) | (bits16<T>(v[3]) << 16);
  r.z = bits16<T>(v[4]) | (bits16<T>(v[5]) << 16);
  r.w = bits16<T>(v[6]) | (bits16<T>(v[7]) << 16);
  return r;
}

// silu(g) * u = (g / (1 + exp(-g))) * u in binary32 (triton_kernels.py:2761-2774).
__device__ __forceinline__ float silu_mul_val(float g, float u) { return (g / (1.0f + exp_f32(-g))) * u; }

}  // namespace tt
