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


// ---- workgroup tiling ---------------------------------------------------------------------

// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X, each with its own L2.
// This maps dispatch order to work order so that XCD k gets the k-th contiguous eighth of the
// work items: neighbouring tiles, which gather the same vertices and texels, share an L2.
__device__ __forceinline__ int64_t xcd_order(int64_t block, int64_t blocks) {
  constexpr int kXcds = 8;
  if (blocks < kXcds) return block;
  const int64_t per = blocks / kXcds, extra = blocks % kXcds;
  const int64_t xcd = block % kXcds, slot = block / kXcds;
  // XCDs < extra own per + 1 items, the others per.
  const int64_t start = xcd * per + (xcd < extra ? xcd : extra);
  const int64_t own = per + (xcd < extra ? 1 : 0);
  return slot < own ? start + slot : block;  // the tail beyond own items keeps its order
}

// A 16 x 16 pixel tile of image b per 256-thread workgroup; (x, y) of this thread.
struct TilePixel {
  int b, x, y;
  bool inside;
  int64_t pixel;
};

__device__ __forceinline__ TilePixel tile_pixel(int batch, int height, int width) {
  const int tiles_x = (width + 15) / 16, tiles_y = (height + 15) / 16;
  const int64_t blocks = (int64_t)batch * tiles_x * tiles_y;
  const int64_t tile = xcd_order(blockIdx.x, blocks);
  TilePixel p;
  p.b = (int)(tile / ((int64_t)tiles_x * tiles_y));
  const int in_image = (int)(tile - (int64_t)p.b * tiles_x * tiles_y);
  p.x = (in_image % tiles_x) * 16 + (int)(threadIdx.x & 15);
  p.y = (in_image / tiles_x) * 16 + (int)(threadIdx.x >> 4);
  p.inside = p.x < width && p.y < height;
  p.pixel = ((int64_t)p.b * height + p.y) * width + p.x;
  return p;
}

inline int64_t tile_blocks(int batch, int height, int width) {
  return (int64_t)batch * ((width + 15) / 16) * ((height + 15) / 16);
}

// ---- workgroup scatter table --------------------------------------------------------------

// Accumulates gradient rows in LDS before they reach global memory. A row is CH floats at
// dst + key * stride; a workgroup adds its rows here (open addressing on the key, LDS float
// atomics), then flush() writes each distinct row once, CH consecutive lanes per row, so that
// the global atomics are few and each row's are coalesced. Rows that find no free slot within
// kProbe steps go straight to global memory. Keys must be < 0xffffffff.
template <int SLOTS, int CH>
struct ScatterTable {
  static constexpr uint32_t kEmpty = 0xffffffffu;
  static constexpr int kProbe = 32;
  uint32_t keys[SLOTS];
  float vals[SLOTS * CH];

  __device__ __forceinline__ void clear() {
    for (int i = threadIdx.x; i < SLOTS; i += blockDim.x) keys[i] = kEmpty;
    for (int i = threadIdx.x; i < SLOTS * CH; i += blockDim.x) vals[i] = 0.0f;
  }

  __device__ __forceinline__ static uint32_t hash(uint32_t k) {
    k ^= k >> 16;
    k *= 0x7feb352du;
    k ^= k >> 15;
    return k;
  }

  // Adds n (<= CH) values of row `key`; returns false if the table had no room.
  __device__ __forceinline__ bool add(uint32_t key, const float* v, int n) {
    uint32_t slot = hash(key) & (SLOTS - 1);
    for (int probe = 0; probe < kProbe; ++probe) {
      const uint32_t seen = atomicCAS(keys + slot, kEmpty, key);
      if (seen == kEmpty || seen == key) {
        for (int c = 0; c < n; ++c)
          if (v[c] != 0.0f) atomicAdd(vals + slot * CH + c, v[c]);
        return true;
      }
      slot = (slot + 1) & (SLOTS - 1);
    }
    return false;
  }

  // Adds a row from every lane that has one (key != kEmpty). When every such lane of the wave
  // has the same key, the wave sums first and one lane adds, which keeps a hot row from
  // serialising 64 LDS atomics. Rows without room are added to global memory directly.
  __device__ __forceinline__ void add_wave(uint32_t key, const float* v, int n, float* dst,
                                           int64_t stride) {
    const uint64_t live = __ballot(key != kEmpty);
    if (live == 0) return;
    const int first = __ffsll((unsigned long long)live) - 1;
    const uint32_t lead = __shfl(key, first);
    if (__ballot(key == lead) == live && __popcll(live) > 1) {
      float sums[CH];
      for (int c = 0; c < n; ++c) sums[c] = wave_masked_sum(v[c], live);
      if (lane_id() == first && !add(lead, sums, n))
        for (int c = 0; c < n; ++c)
          if (sums[c] != 0.0f) atomic_add(dst + (int64_t)lead * stride + c, sums[c]);
      return;
    }
    if (key != kEmpty && !add(key, v, n))
      for (int c = 0; c < n; ++c)
        if (v[c] != 0.0f) atomic_add(dst + (int64_t)key * stride + c, v[c]);
  }

  // Writes the accumulated rows; call after a barrier that follows every add.
  __device__ __forceinline__ void flush(float* dst, int64_t stride, int n) {
    for (int i = threadIdx.x; i < SLOTS * CH; i += blockDim.x) {
      const int slot = i / CH, c = i - slot * CH;
      const uint32_t key = keys[slot];
      if (key == kEmpty || c >= n) continue;
      const float v = vals[i];
      if (v != 0.0f) atomic_add(dst + (int64_t)key * stride + c, v);
    }
  }
};

}  // namespace dr
