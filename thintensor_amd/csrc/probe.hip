// Memory-floor reference for the GEMV rooflines: a pure streaming read.
//
// Each wave reads its own contiguous span of `bytes_per_wave` bytes with 16-byte loads
// (64 lanes x 16 B = 1 KiB per load, two loads in flight per lane), folds the words into
// one value and stores a single 32-bit word per wave (any kernel that produces output
// pays for at least that).  At a given byte count it is the fastest a single launch can
// move data on this part, so a GEMV of the same bytes is compared against it.
#include "tt_abi_internal.h"
#include "tt_common.h"

namespace tt {
namespace {

// The grid holds whole workgroups of four waves; waves at or past `waves` (the last
// workgroup's padding) return at once, so out[] is written for wave < waves only.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, int64_t units,
                                                          int units_per_wave, int64_t waves,
                                                          uint32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wave >= waves) return;   // wave-uniform
  const int64_t base = wave * units_per_wave;
  uint32_t acc = 0;
  for (int u = 0; u < units_per_wave; u += 128) {
    int64_t i0 = base + u + lane, i1 = i0 + 64;
    i0 = i0 < units ? i0 : units - 1;   // clamped: re-reads of the last unit, in bounds
    i1 = i1 < units ? i1 : units - 1;
    const uint4 a = p[i0], b = p[i1];
    acc ^= (a.x + a.y + a.z + a.w) ^ (b.x + b.y + b.z + b.w);
  }
  for (int m = 1; m < 64; m <<= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m);
  if (lane == 0) out[wave] = acc;
}

}  // namespace
}  // namespace tt

using namespace tt;

extern "C" int64_t tt_stream_read_waves(int64_t bytes, int64_t bytes_per_wave) {
  if (bytes <= 0 || bytes_per_wave <= 0) return 0;
  return (bytes + bytes_per_wave - 1) / bytes_per_wave;
}

extern "C" int tt_stream_read(const void* data, int64_t bytes, int64_t bytes_per_wave, void* out, int64_t out_words,
                              void* stream) {
  const char* what = "stream_read";
  TT_REQUIRE(data && out && aligned(data, 16), "%s: null or misaligned pointer", what);
  TT_REQUIRE(bytes > 0 && bytes % 16 == 0, "%s: bytes must be a positive multiple of 16", what);
  TT_REQUIRE(bytes_per_wave >= 2048 && bytes_per_wave % 2048 == 0 && bytes_per_wave < (1LL << 31),
             "%s: bytes_per_wave must be a multiple of 2048", what);
  const int64_t waves = tt_stream_read_waves(bytes, bytes_per_wave);
  TT_REQUIRE(out_words >= waves, "%s: out needs %lld words", what, (long long)waves);
  const dim3 grid((unsigned)((waves + 3) / 4));
  hipLaunchKernelGGL(stream_read_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(data), bytes / 16, (int)(bytes_per_wave / 16), waves,
                     static_cast<uint32_t*>(out));
  return check_launch(what);
}
