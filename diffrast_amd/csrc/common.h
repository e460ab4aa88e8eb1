// Shared device helpers for the diffrast HIP kernels (gfx950, wave64).
//
// All sources are compiled with -ffp-contract=off: every float operation written here is one
// IEEE-rounded operation, in the order written, and '/' is correctly rounded. The visibility,
// resolve and interpolate kernels rely on that to repeat the reference backend's arithmetic
// (src/diffrast/backends/reference.py) bit for bit.
#pragma once

#include <type_traits>

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

// N consecutive floats at p with the widest loads their alignment allows (16 bytes for N a
// multiple of 4, 8 bytes for N = 2); false, with nothing loaded, when p is not so aligned. Gathers
// of whole rows this way cost one memory instruction per 16 bytes instead of one per channel.
template <int N>
__device__ __forceinline__ bool load_wide(const float* p, float (&v)[N]) {
  if constexpr (N % 4 == 0) {
    if (reinterpret_cast<uintptr_t>(p) & 15u) return false;
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const float4 q = reinterpret_cast<const float4*>(p)[i];
      v[4 * i] = q.x;
      v[4 * i + 1] = q.y;
      v[4 * i + 2] = q.z;
      v[4 * i + 3] = q.w;
    }
    return true;
  } else if constexpr (N == 2) {
    if (reinterpret_cast<uintptr_t>(p) & 7u) return false;
    const float2 q = *reinterpret_cast<const float2*>(p);
    v[0] = q.x;
    v[1] = q.y;
    return true;
  }
  return false;
}

template <int N>
__device__ __forceinline__ bool store_wide(float* p, const float (&v)[N]) {
  if constexpr (N % 4 == 0) {
    if (reinterpret_cast<uintptr_t>(p) & 15u) return false;
#pragma unroll
    for (int i = 0; i < N / 4; ++i)
      reinterpret_cast<float4*>(p)[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    return true;
  } else if constexpr (N == 2) {
    if (reinterpret_cast<uintptr_t>(p) & 7u) return false;
    *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
    return true;
  }
  return false;
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Launches of kernels templated on NC channels per group: 1-4 as they are, more in groups of 4.
template <typename F>
int channel_groups(int channels, F f) {
  switch (channels) {
    case 1: return f(std::integral_constant<int, 1>());
    case 2: return f(std::integral_constant<int, 2>());
    case 3: return f(std::integral_constant<int, 3>());
    default: return f(std::integral_constant<int, 4>());
  }
}

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


// ---- sums over runs of lanes ----------------------------------------------------------------

// The value of lane - S of the same 16-lane row, 0 in the row's first S lanes (DPP row_shr).
template <int S>
__device__ __forceinline__ float row_shr(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + S, 0xf, 0xf, true));
}
template <int S>
__device__ __forceinline__ uint32_t row_shr(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x110 + S, 0xf, 0xf, true);
}
// The value of lane + S of the same 16-lane row, 0 in the row's last S lanes (DPP row_shl).
template <int S>
__device__ __forceinline__ uint32_t row_shl(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x100 + S, 0xf, 0xf, true);
}

// Wave-wide scans with DPP moves only (no LDS permute, no lane-address registers): row_shr
// steps within each 16-lane row, then row_bcast:15 (rows 1 and 3 take the last lane of the
// row before) and row_bcast:31 (rows 2 and 3 take lane 31). Lanes a move does not reach get 0,
// the identity of both sum and unsigned max.
__device__ __forceinline__ uint32_t bcast15(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);
}
__device__ __forceinline__ uint32_t bcast31(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);
}
// The value of the previous lane of the wave (0 in lane 0): DPP wave_shr:1.
__device__ __forceinline__ uint32_t wave_shr1(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x138, 0xf, 0xf, true);
}

__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v) {
  v += row_shr<1>(v);
  v += row_shr<2>(v);
  v += row_shr<4>(v);
  v += row_shr<8>(v);
  v += bcast15(v);
  v += bcast31(v);
  return v;
}

__device__ __forceinline__ uint32_t wave_inclusive_max(uint32_t v) {
  v = max(v, row_shr<1>(v));
  v = max(v, row_shr<2>(v));
  v = max(v, row_shr<4>(v));
  v = max(v, row_shr<8>(v));
  v = max(v, bcast15(v));
  v = max(v, bcast31(v));
  return v;
}

template <int S>
__device__ __forceinline__ uint64_t row_shr64(uint64_t v) {
  return (uint64_t)row_shr<S>((uint32_t)(v >> 32)) << 32 | row_shr<S>((uint32_t)v);
}

// Largest value over the wave, in every lane.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  uint64_t o;
  o = row_shr64<1>(v);
  v = o > v ? o : v;
  o = row_shr64<2>(v);
  v = o > v ? o : v;
  o = row_shr64<4>(v);
  v = o > v ? o : v;
  o = row_shr64<8>(v);
  v = o > v ? o : v;
  o = (uint64_t)bcast15((uint32_t)(v >> 32)) << 32 | bcast15((uint32_t)v);
  v = o > v ? o : v;
  o = (uint64_t)bcast31((uint32_t)(v >> 32)) << 32 | bcast31((uint32_t)v);
  v = o > v ? o : v;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), DR_WAVE - 1);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)v, DR_WAVE - 1);
  return (uint64_t)hi << 32 | lo;
}

template <int S, int N>
__device__ __forceinline__ void run_step(float (&v)[N], bool take) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float y = row_shr<S>(v[i]);
    v[i] += take ? y : 0.0f;
  }
}

// Segmented sums over runs of consecutive lanes of a 16-lane row that hold the same key (a
// tile row of pixels showing one triangle): afterwards the last lane of each run holds in v
// the sum over the run. Returns true in those lanes. Every lane of the wave must be active.
template <int N>
__device__ __forceinline__ bool row_run_sums(uint32_t key, float (&v)[N]) {
  const int lane = lane_id();
  const int pos = lane & 15;
  // Both neighbours are read in every lane (a DPP read from an inactive lane yields 0).
  const uint32_t left = row_shr<1>(key), right = row_shl<1>(key);
  const bool head = (pos == 0) | (left != key);
  const bool last = (pos == 15) | (right != key);
  const uint64_t heads = __ballot(head);
  const int start = 63 - __clzll(heads & ((2ull << lane) - 1ull));  // first lane of the run
  // A step adds nothing unless some lane sits at least that far into its run: the lanes at
  // position >= 1, 2, 4 and 8, as masks of the wave (runs never cross a row: its first lane is
  // a head), end the scan early where the runs are short.
  const uint64_t at1 = ~heads;
  if (at1 == 0) return last;
  run_step<1>(v, lane - 1 >= start);
  const uint64_t at2 = at1 & (at1 << 1);
  if (at2 == 0) return last;
  run_step<2>(v, lane - 2 >= start);
  const uint64_t at4 = at2 & (at2 << 2);
  if (at4 == 0) return last;
  run_step<4>(v, lane - 4 >= start);
  if ((at4 & (at4 << 4)) == 0) return last;
  run_step<8>(v, lane - 8 >= start);
  return last;
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

// xcd_order within consecutive groups of 8 * K blocks: each XCD takes a contiguous run of K
// blocks of every group, so neighbouring work shares an L2 while the groups still run roughly
// in order (the last, partial group keeps dispatch order).
__device__ __forceinline__ int64_t xcd_order_grouped(int64_t block, int64_t blocks, int k) {
  constexpr int kXcds = 8;
  const int64_t group_size = (int64_t)kXcds * k;
  const int64_t group = block / group_size;
  if ((group + 1) * group_size > blocks) return block;
  const int64_t r = block - group * group_size;
  return group * group_size + (r % kXcds) * k + r / kXcds;
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

// The pixels of a thread in the gather kernels (resolve, interpolate), in one of two layouts.
// Rows: PPT pixels 256 apart in pixel order, so every wave reads and writes runs of 64
// consecutive pixels; best when what the pixels gather (index rows, vertices, attributes) stays
// in the L2s anyway, or when the pass is bound by its writes. Tiles: a TW x (256 / TW) PPT tile
// per workgroup, the tiles in XCD order, pixel j at (x, y0 + 256 / TW j); the pixels of a
// triangle and of its neighbours, which share vertices, then gather into one XCD's L2 rather
// than one per image row, which pays when the gathered data outgrows an L2.
template <int PPT>
struct PixelSlots {
  int64_t pixel[PPT];
  int b[PPT], x[PPT], y[PPT];
  bool inside[PPT];
};

template <int PPT, bool TILES, int TW = 16>
__device__ __forceinline__ PixelSlots<PPT> pixel_slots(int batch, int height, int width) {
  static_assert(TW > 0 && 256 % TW == 0, "the tile width must divide the 256 threads");
  PixelSlots<PPT> s;
  if constexpr (TILES) {
    constexpr int TR = 256 / TW;  // rows of the workgroup per pixel slot
    const int tiles_x = (width + TW - 1) / TW, tiles_y = (height + TR * PPT - 1) / (TR * PPT);
    const int64_t tile = xcd_order(blockIdx.x, (int64_t)batch * tiles_x * tiles_y);
    const int b = (int)(tile / ((int64_t)tiles_x * tiles_y));
    const int in_image = (int)(tile - (int64_t)b * tiles_x * tiles_y);
    const int x = (in_image % tiles_x) * TW + (int)(threadIdx.x % TW);
    const int y0 = (in_image / tiles_x) * TR * PPT + (int)(threadIdx.x / TW);
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      s.b[j] = b;
      s.x[j] = x;
      s.y[j] = y0 + TR * j;
      s.inside[j] = x < width && s.y[j] < height;
      s.pixel[j] = ((int64_t)b * height + s.y[j]) * width + x;
    }
  } else {
    const int64_t image_pixels = (int64_t)height * width;
    const int64_t total = (int64_t)batch * image_pixels;
    const int64_t first = (int64_t)blockIdx.x * blockDim.x * PPT + threadIdx.x;
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int64_t pixel = first + (int64_t)j * blockDim.x;
      s.pixel[j] = pixel;
      s.inside[j] = pixel < total;
      s.b[j] = pixel < 0xffffffffLL && image_pixels < 0xffffffffLL
                   ? (int)((uint32_t)pixel / (uint32_t)image_pixels)
                   : (int)(pixel / image_pixels);
      const int64_t in_image = pixel - (int64_t)s.b[j] * image_pixels;
      s.y[j] = (int)(in_image / width);
      s.x[j] = (int)(in_image - (int64_t)s.y[j] * width);
    }
  }
  return s;
}

template <int PPT, bool TILES, int TW = 16>
inline int64_t pixel_slot_blocks(int batch, int height, int width) {
  constexpr int TR = 256 / TW;
  if (TILES)
    return (int64_t)batch * ((width + TW - 1) / TW) * ((height + TR * PPT - 1) / (TR * PPT));
  return blocks_for((int64_t)batch * height * width, 256 * PPT);
}

// Whether a gather kernel takes the tile layout: when the mesh data one image's pixels gather
// is larger than an XCD's 4 MiB L2.
inline bool gather_tiles(int64_t gathered_bytes) { return gathered_bytes > (int64_t)4 << 20; }

// ---- workgroup scatter table --------------------------------------------------------------

// Fixed-point scale of one accumulation pass of a workgroup. LDS float atomics are slow on
// gfx950 (one lane per clock per CU), 64-bit integer ones an order of magnitude faster, so the
// row table accumulates value * 2^shift as 64-bit integers. With every value a lane gives at
// most M in magnitude, M < 2^(e + 1), shift = 44 - e keeps each value below 2^45 and a wave's
// sum of up to 64 of them (add_wave) below 2^51, the range of to_fixed(); any 2^11 such adds stay
// below 2^62. The rounding of each value is at most 2^-45 M, far below float32 accumulation. A
// non-finite value anywhere in the pass sends the whole pass to global float atomics instead.
// Largest magnitude among n values, +inf if any is not finite.
__device__ __forceinline__ float max_magnitude(const float* v, int n) {
  float m = 0.0f;
  bool bad = false;
  for (int i = 0; i < n; ++i) {
    bad = bad || !isfinite(v[i]);
    m = fmaxf(m, fabsf(v[i]));
  }
  return bad ? __int_as_float(0x7f800000) : m;
}

struct FixedPass {
  double scale;  // 2^shift
  double inv;    // 2^-shift
  bool direct;   // no table: values go straight to global memory
};

// round(v * scale), to nearest even. |v * scale| < 2^51 here, so adding 1.5 * 2^52 leaves that
// integer in the low bits of the double (every value of [2^52, 2^53) is an integer), and the
// product itself is exact (scale is a power of two): one fused multiply-add and a subtraction.
__device__ __forceinline__ long long to_fixed(float v, const FixedPass& f) {
  const double magic = 6755399441055744.0;  // 1.5 * 2^52
  const double y = __fma_rn((double)v, f.scale, magic);
  return __double_as_longlong(y) - __double_as_longlong(magic);
}

__device__ __forceinline__ float from_fixed(long long x, const FixedPass& f) {
  return (float)((double)x * f.inv);
}

// Accumulates gradient rows in LDS before they reach global memory. A row is CH floats at
// dst + key * stride. Lanes add rows here: open addressing on the key, where a plain read finds
// a key already present and a compare-and-swap claims a free slot, which then joins the list
// of used slots; values add as 64-bit fixed point (FixedPass). flush() adds each used row to
// global memory once, CH consecutive lanes per row, and zeroes it, so clearing and flushing
// cost what the workgroup touched, not the table size. A key that finds no slot within kProbe
// steps goes straight to global memory. Keys must be < 0xffffffff.
template <int SLOTS, int CH>
struct RowTable {
  static constexpr uint32_t kEmpty = 0xffffffffu;
  static constexpr int kProbe = 16;
  static_assert((SLOTS & (SLOTS - 1)) == 0 && CH % 2 == 0 && SLOTS <= 65536,
                "power-of-two slots (at most 2^16), even CH");
  uint32_t keys[SLOTS];
  long long vals[CH * SLOTS];  // channel-major: lanes adding to different rows hit different banks
  // The slots in use, in 16 bits: a 512 x 4 table then needs 19.5 KB of LDS, under the 20 KB
  // that lets eight workgroups share a CU.
  uint16_t used[SLOTS];
  uint32_t count;
  float wave_max[256 / DR_WAVE];
  int wave_bad[256 / DR_WAVE];

  // Empties the table. Every thread of the workgroup calls it; begin() orders it before adds.
  __device__ __forceinline__ void init() {
    for (int i = threadIdx.x; i < SLOTS; i += blockDim.x) keys[i] = kEmpty;
    longlong2* v2 = reinterpret_cast<longlong2*>(vals);
    for (int i = threadIdx.x; i < SLOTS * CH / 2; i += blockDim.x) v2[i] = make_longlong2(0, 0);
    if (threadIdx.x == 0) count = 0u;
  }

  // Starts a pass: every thread gives the largest magnitude it will add (NaN or inf for a
  // non-finite value). Contains a barrier, which also orders init() or reset() before the adds.
  __device__ __forceinline__ FixedPass begin(float lane_max) {
    const bool bad = !isfinite(lane_max);
    float m = bad ? 0.0f : lane_max;
#pragma unroll
    for (int d = 1; d < DR_WAVE; d <<= 1) m = fmaxf(m, __shfl_xor(m, d));
    const bool wave_bad_now = __ballot(bad) != 0;
    if (lane_id() == 0) {
      wave_max[threadIdx.x / DR_WAVE] = m;
      wave_bad[threadIdx.x / DR_WAVE] = wave_bad_now;
    }
    __syncthreads();
    float M = 0.0f;
    bool any_bad = false;
#pragma unroll
    for (int w = 0; w < 256 / DR_WAVE; ++w) {
      M = fmaxf(M, wave_max[w]);
      any_bad = any_bad || wave_bad[w];
    }
    FixedPass f;
    f.direct = any_bad;
    int e = 0;
    if (M > 0.0f) e = ilogbf(M);
    f.scale = ldexp(1.0, 44 - e);
    f.inv = ldexp(1.0, e - 44);
    return f;
  }

  __device__ __forceinline__ static uint32_t hash(uint32_t k) {
    k ^= k >> 16;
    k *= 0x7feb352du;
    k ^= k >> 15;
    return k;
  }

  // Slot of `key`, claimed if new; -1 if none within kProbe steps.
  __device__ __forceinline__ int slot_of(uint32_t key) {
    uint32_t slot = hash(key) & (SLOTS - 1);
    for (int probe = 0; probe < kProbe; ++probe) {
      uint32_t seen =
          __hip_atomic_load(keys + slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (seen == key) return (int)slot;
      if (seen == kEmpty) {
        seen = atomicCAS(keys + slot, kEmpty, key);
        if (seen == kEmpty) {
          used[atomicAdd(&count, 1u)] = (uint16_t)slot;
          return (int)slot;
        }
        if (seen == key) return (int)slot;
      }
      slot = (slot + 1) & (SLOTS - 1);
    }
    return -1;
  }

  // Adds n (<= CH) values of row `key`; false if the table had no room (or the pass is direct).
  __device__ __forceinline__ bool add(uint32_t key, const float* v, int n, const FixedPass& f) {
    if (f.direct) return false;
    const int slot = slot_of(key);
    if (slot < 0) return false;
    unsigned long long* col = reinterpret_cast<unsigned long long*>(vals + slot);
#pragma unroll
    for (int c = 0; c < CH; ++c)
      if (c < n) atomicAdd(col + c * SLOTS, (unsigned long long)to_fixed(v[c], f));
    return true;
  }

  // Adds a row to the table, or to global memory if the table has no room.
  __device__ __forceinline__ void add_or_global(uint32_t key, const float* v, int n, float* dst,
                                                int64_t stride, const FixedPass& f) {
    if (!add(key, v, n, f))
      for (int c = 0; c < n; ++c)
        if (v[c] != 0.0f) atomic_add(dst + (int64_t)key * stride + c, v[c]);
  }

  // Adds a row from every lane that has one (key != kEmpty). When every such lane of the wave
  // has the same key, the wave sums first and one lane adds, which keeps a hot row from
  // serialising 64 LDS atomics.
  __device__ __forceinline__ void add_wave(uint32_t key, const float* v, int n, float* dst,
                                           int64_t stride, const FixedPass& f) {
    const uint64_t live = __ballot(key != kEmpty);
    if (live == 0) return;
    const int first = __ffsll((unsigned long long)live) - 1;
    const uint32_t lead = __shfl(key, first);
    if (__ballot(key == lead) == live && __popcll(live) > 1) {
      float sums[CH];
      for (int c = 0; c < n; ++c) sums[c] = wave_masked_sum(v[c], live);
      if (lane_id() == first) add_or_global(lead, sums, n, dst, stride, f);
      return;
    }
    if (key != kEmpty) add_or_global(key, v, n, dst, stride, f);
  }

  // Adds the used rows to global memory and zeroes them; call after a barrier that follows
  // every add. Lanes take (row, channel) pairs, a power of two >= n lanes per row.
  __device__ __forceinline__ void flush(float* dst, int64_t stride, int n, const FixedPass& f) {
    const int shift = n <= 1 ? 0 : (n <= 2 ? 1 : (n <= 4 ? 2 : 3));
    const uint32_t rows = count;
    for (uint32_t i = threadIdx.x; i < (rows << shift); i += blockDim.x) {
      const int c = (int)(i & ((1u << shift) - 1u));
      if (c >= n) continue;
      const uint32_t slot = used[i >> shift];
      long long* p = vals + c * SLOTS + slot;
      const long long x = *p;
      if (x != 0) atomic_add(dst + (int64_t)keys[slot] * stride + c, from_fixed(x, f));
      *p = 0;
    }
  }

  // Empties the table again after flush() for another pass; call after a barrier that follows
  // the flush. Contains its own barriers.
  __device__ __forceinline__ void reset() {
    const uint32_t rows = count;
    for (uint32_t i = threadIdx.x; i < rows; i += blockDim.x) keys[used[i]] = kEmpty;
    __syncthreads();
    if (threadIdx.x == 0) count = 0u;
    __syncthreads();
  }
};

}  // namespace dr
