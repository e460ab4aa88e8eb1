// Shared device helpers for the diffrast HIP kernels (gfx950, wave64).
//
// All sources are compiled with -ffp-contract=off: every float operation written here is one
// IEEE-rounded operation, in the order written, and '/' is correctly rounded. The visibility,
// resolve and interpolate kernels rely on that to repeat the reference backend's arithmetic
// (src/diffrast/backends/reference.py) bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/diffrast_hip.h"

#define DR_WAVE 64

namespace dr {

// Status of the launches made so far on this thread.
inline int launch_status() {
  hipError_t err = hipGetLastError();
  return err == hipSuccess ? DR_OK : DR_ERR_HIP;
}

inline int blocks_for(int64_t n, int threads) { return (int)((n + threads - 1) / threads); }

// Pixel-centre NDC coordinate of column (or row) i of an image `size` pixels across:
// (2 i + 1) / size - 1, rounded as float32 (reference.py:268-271).
__device__ __forceinline__ float pixel_centre(int i, int size) {
  return (float)(2 * i + 1) / (float)size - 1.0f;
}

// 64-bit visibility key: order-preserving depth bits above the triangle row. -0 and +0 map
// to the same key, so equal depths are ordered by triangle row alone.
__device__ __forceinline__ uint64_t depth_key(float depth, uint32_t tri) {
  if (depth == 0.0f) depth = 0.0f;
  uint32_t bits = __float_as_uint(depth);
  uint32_t ordered = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return ((uint64_t)ordered << 32) | (uint64_t)tri;
}

constexpr uint64_t kEmptyKey = ~0ull;

__device__ __forceinline__ float4 load4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ void store4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// Hardware fp32 atomic add (the buffers are ordinary coarse-grained device memory).
__device__ __forceinline__ void atomic_add(float* p, float v) { unsafeAtomicAdd(p, v); }

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Sum of v over the lanes of the wave whose bit is set in `mask`, valid in every lane.
__device__ __forceinline__ float wave_masked_sum(float v, uint64_t mask) {
  float x = ((mask >> lane_id()) & 1ull) ? v : 0.0f;
#pragma unroll
  for (int offset = 32; offset >= 1; offset >>= 1) x += __shfl_xor(x, offset);
  return x;
}

// Scatter helper. Lanes whose `key` (>= 0) is equal target the same addresses; up to `rounds`
// groups of them are merged, leader first: group(same_mask, leader) is called by every lane of
// the wave (it sums values with wave_masked_sum and lets the leader write). Lanes left over,
// and every lane once a round finds nothing to merge, call direct() on their own.
template <typename Group, typename Direct>
__device__ __forceinline__ void wave_grouped(int64_t key, int rounds, Group group,
                                             Direct direct) {
  uint64_t pending = __ballot(key >= 0);
  for (int r = 0; r < rounds && pending; ++r) {
    const int leader = __ffsll((unsigned long long)pending) - 1;
    const int64_t lead_key = __shfl(key, leader);
    const uint64_t same = __ballot(key == lead_key) & pending;
    if (__popcll(same) == 1) break;
    group(same, leader);
    pending &= ~same;
  }
  if ((pending >> lane_id()) & 1ull) direct();
}

// wave_grouped for a fixed number of values per lane: add(values) is called with the merged
// sums by a group's leader and with its own values by a lane left over.
template <int N, typename Add>
__device__ __forceinline__ void wave_merged_scatter(int64_t key, const float (&vals)[N],
                                                    int rounds, Add add) {
  wave_grouped(
      key, rounds,
      [&](uint64_t same, int leader) {
        float sums[N];
#pragma unroll
        for (int i = 0; i < N; ++i) sums[i] = wave_masked_sum(vals[i], same);
        if (lane_id() == leader) add(sums);
      },
      [&]() { add(vals); });
}

}  // namespace dr
