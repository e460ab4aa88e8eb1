// Rasterize for gfx950: visibility as 64-bit (depth, triangle) keys, then resolve.
//
// Visibility decides, per pixel, the nearest triangle that covers the pixel centre, with the
// coverage test of the reference backend (src/diffrast/backends/reference.py:293-365) and its
// tie-break (lower triangle row on equal depth, reference.py:368-397). The result does not
// depend on the order in which triangles are processed -- a key is (depth, row) and merging
// takes the minimum -- which leaves the processing order free for the hardware's sake:
//
// 1. Order. For a large instanced mesh, triangles are bucket-sorted by the Morton code of their
//    centroid in the first view's clip space (an affine image of world space, so neighbours in
//    the order are neighbours on screen in every view). Meshes such as subdivided spheres list
//    children of one face far apart; in this order a workgroup's triangles cover a compact
//    patch of the screen, which makes the binning below aggregate well.
// 2. Setup: one thread per triangle instance culls it (a non-finite coordinate, or every w <= 0:
//    the interpolated w is then never positive) and bounds its pixels. Boxes of at most
//    small_pixels() pixel centres are rasterized right away (64-bit atomic min per covered
//    pixel); the others are binned into 16x16 tiles. Per-tile counts gather in an LDS table of
//    the workgroup before one global atomic per distinct tile.
// 3. A three-phase scan turns tile counts into list offsets; the bin pass reserves each
//    workgroup's share of a tile's list with one global atomic and fills it. Each tile has one
//    list per depth slab (the triangle's nearest vertex within the image's depth span), so a
//    tile's entries run near to far.
// 4. One 256-thread workgroup per tile with entries (heavy tiles first, each XCD on its own
//    share of the tiles) holds the tile's keys in LDS and walks its entries 256 at a time:
//    triangles entirely behind the tile's farthest key are skipped; the others are staged in
//    LDS with, per tile row, the span of columns their pixel centres may cover (a bound proved
//    against the coverage test in coverage.h), and the pixels of those spans are tested as one
//    flat list of work items (every lane busy whatever the span lengths), merging into the
//    tile's keys (64-bit min). The workgroup alone owns the tile: one plain store per pixel at
//    the end.
//
// The resolve kernels turn keys into rast / rast_db (reference.py:69-114) and carry gradients
// back to the vertices.
#include <mutex>

#include "common.h"
#include "coverage.h"

namespace dr {
namespace {

constexpr int kTile = 16;            // tile edge in pixels; a tile is one 256-thread workgroup
constexpr int kChunk = 256;          // triangles per tile work item
constexpr int kWorkClasses = 128;    // tile work classes: none, then 32 entries each (heavy-first order)
constexpr int kWindow = 1024;        // work items per map of the tile kernel (256 threads x 4)
static_assert(kWindow == 4 * 256, "the map scan gives each thread four entries");
// Bounding boxes up to this many pixel centres skip binning: a device atomic per covered pixel
// against a record, tile entries and the tile pass's per-tile work. Many views of one dense
// mesh keep few (1.31 M triangles, 8 x 1024^2: 8 is best, 16 costs 26 us, 64 far more in
// atomics); range mode, where every image draws its own small item and most tiles hold few
// triangles, keeps many (256 items of 5120 triangles at 512^2, 4 layers: visibility 3.08 ms
// with 16, 2.38 with 64).
constexpr int kSmallPixelsDense = 8;
constexpr int kSmallPixelsRanges = 64;
constexpr int kScanBlock = 1024;     // elements per scan block (256 threads x 4)
constexpr int kOrderBuckets = 4096;  // Morton buckets (12 bits of a 30-bit code)
constexpr int kOrderMinTris = 8192;  // smaller meshes keep their own order
constexpr int kTileSlots = 1024;     // LDS table of a workgroup's tiles
constexpr int kRecord = 4;           // float4 per binned triangle record (one 64-byte line)
constexpr int kDepthSlabs = 16;      // tile lists per tile, by the triangle's nearest depth
                                     // (dense views; range mode keeps one list per tile)
constexpr int kRangeParts = 64;      // workgroups per image in the depth span reduction
constexpr int kXcdShares = 8;        // XCDs of an MI355X: workgroup b runs on XCD b mod 8

struct Workspace {
  float4* records;           // binned triangles, kRecord float4 each: the three clip-space
                             // vertices, then the bits of (image, row, tx0 | tx1 << 16,
                             // ty0 | ty1 << 16)
  uint4* record_bins;        // per record slot, what the bin pass reads (16 bytes, not the
                             // record's 64): tx0 | tx1 << 16, ty0 | ty1 << 16, the list of tile
                             // (0, 0) of its image and slab, and the bits of its triangle's
                             // depth_lower_bound, which the bin pass copies into the entries
  // Tile lists: list tile * slabs + slab holds the binned triangles of that tile whose
  // nearest depth falls in depth slab `slab` of their image, so a tile's entries are one range
  // that runs near to far.
  uint32_t* list_counts;     // [lists + 1]
  uint32_t* list_offsets;    // [lists + 1] exclusive prefix of list_counts
  uint32_t* list_cursor;     // [lists + 1] fill positions of the bin pass
  uint32_t* chunk_offsets;   // [lists + 1] exclusive prefix of ceil(count / kChunk)
  uint32_t* depth_range;     // [depth_ranges][2] order-preserving bits of the nearest and
                             // farthest vertex depth of an image (one when pos is shared)
  uint32_t* range_parts;     // [depth_ranges][kRangeParts][2] partial spans
  uint2* block_sums;         // [scan blocks] (entries, chunks)
  uint32_t* counters;        // [0] setup workgroups, [1] entries, [2] tile pass
                             // workgroups, [3] busy tiles
  uint32_t* block_records;   // [record_blocks] binned triangles of each setup workgroup
  uint32_t* tile_order;      // [tiles] tile pass order: heavy tiles first within each XCD's share
  uint8_t* tile_class;       // [tiles] work class of each tile (entries / 32, capped)
  uint32_t* class_counts;    // [8][kWorkClasses] tiles per (XCD share, class)
  uint32_t* class_cursor;    // [8][kWorkClasses] fill positions of the placement pass
  uint32_t* share_info;      // [16] busy tiles of each XCD share, then where they start in the order
  float* px;                 // [width] pixel-centre x per column
  float* py;                 // [height] pixel-centre y per row
  int4* order;               // [num_tri] processing order (instanced meshes only): the vertex
                             // rows of each triangle and its row of tri
  float4* centroids;         // [num_tri] clip-space centroids in the first view
  uint32_t* bucket_counts;   // [kOrderBuckets]
  uint32_t* bucket_cursor;   // [kOrderBuckets]
  uint32_t* bounds;          // [6] order-preserving bits of min x, y, z and max x, y, z
  uint32_t* bound_parts;     // [centroid workgroups][6] the same per workgroup
  bool ordered;
  int tiles_x, tiles_y;
  int64_t tiles;
  int64_t lists;
  int depth_ranges;
  int scan_blocks;
  int record_blocks;          // setup workgroups; each owns 256 record slots
  int slabs;                  // tile lists per tile: kDepthSlabs, or 1 in range mode
  size_t bytes;
};

size_t align_up(size_t v) { return (v + 255) & ~size_t(255); }

int small_pixels(const DrRasterGeometry& g) {
  return g.ranges != nullptr ? kSmallPixelsRanges : kSmallPixelsDense;
}

bool use_order(const DrRasterGeometry& g) {
  return g.ranges == nullptr && g.num_tri >= kOrderMinTris;
}

Workspace layout(const DrRasterGeometry& g, char* base) {
  Workspace w{};
  w.tiles_x = (g.width + kTile - 1) / kTile;
  w.tiles_y = (g.height + kTile - 1) / kTile;
  w.tiles = (int64_t)g.batch * w.tiles_x * w.tiles_y;
  // Range mode keeps one list per tile: its items' triangles mostly take the small-triangle path,
  // so the near-to-far slabs gain its tile pass nothing, while their lists (clears, scans) and
  // the depth span they need cost 0.2 ms per step of four layers of 256 items at 512 x 512.
  w.slabs = g.ranges != nullptr ? 1 : kDepthSlabs;
  w.lists = w.tiles * w.slabs;
  w.scan_blocks = (int)((w.lists + 1 + kScanBlock - 1) / kScanBlock);
  w.depth_ranges = (g.ranges == nullptr && g.pos_batch_stride != 0) ? std::max(g.batch, 1) : 1;
  w.ordered = use_order(g);
  w.record_blocks = std::max(blocks_for(g.num_instances, 256), 1);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off = align_up(off + bytes);
    return p;
  };
  w.counters = (uint32_t*)take(16);
  w.list_counts = (uint32_t*)take(sizeof(uint32_t) * (w.lists + 1));
  w.list_offsets = (uint32_t*)take(sizeof(uint32_t) * (w.lists + 1));
  w.list_cursor = (uint32_t*)take(sizeof(uint32_t) * (w.lists + 1));
  w.chunk_offsets = (uint32_t*)take(sizeof(uint32_t) * (w.lists + 1));
  w.depth_range = (uint32_t*)take(sizeof(uint32_t) * 2 * w.depth_ranges);
  w.range_parts = (uint32_t*)take(sizeof(uint32_t) * 2 * kRangeParts * w.depth_ranges);
  w.block_sums = (uint2*)take(sizeof(uint2) * (w.scan_blocks + 1));
  w.block_records = (uint32_t*)take(sizeof(uint32_t) * w.record_blocks);
  w.tile_order = (uint32_t*)take(sizeof(uint32_t) * w.tiles);
  w.tile_class = (uint8_t*)take(w.tiles);
  w.class_counts = (uint32_t*)take(sizeof(uint32_t) * 8 * kWorkClasses);
  w.class_cursor = (uint32_t*)take(sizeof(uint32_t) * 8 * kWorkClasses);
  w.share_info = (uint32_t*)take(sizeof(uint32_t) * 16);
  w.px = (float*)take(sizeof(float) * g.width);
  w.py = (float*)take(sizeof(float) * g.height);
  if (w.ordered) {
    w.order = (int4*)take(sizeof(int4) * g.num_tri);
    w.centroids = (float4*)take(sizeof(float4) * g.num_tri);
    w.bucket_counts = (uint32_t*)take(sizeof(uint32_t) * kOrderBuckets);
    w.bucket_cursor = (uint32_t*)take(sizeof(uint32_t) * kOrderBuckets);
    w.bounds = (uint32_t*)take(sizeof(uint32_t) * 8);
    w.bound_parts = (uint32_t*)take(sizeof(uint32_t) * 6 * (size_t)blocks_for(g.num_tri, 256));
  }
  w.records = (float4*)take(sizeof(float4) * kRecord * 256 * (size_t)w.record_blocks);
  w.record_bins = (uint4*)take(sizeof(uint4) * 256 * (size_t)w.record_blocks);
  w.bytes = off;
  if (w.ordered && g.order != nullptr) w.order = (int4*)g.order;
  return w;
}

// ---- geometry helpers -------------------------------------------------------------------

// (image, triangle row) of triangle instance i.
__device__ __forceinline__ void instance(const DrRasterGeometry& g, int64_t i, int& b, int& t) {
  if (g.ranges == nullptr) {
    b = (int)(i / g.num_tri);
    t = (int)(i - (int64_t)b * g.num_tri);
    return;
  }
  // The item of the wave's first instance by a binary search on wave-uniform values (scalar
  // loads), then each lane steps forward over the few items its wave spans.
  const uint32_t first_lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)i);
  const uint32_t first_hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(i >> 32));
  const int64_t first = (int64_t)((uint64_t)first_hi << 32 | first_lo);  // the first active lane's
  int lo = 0, hi = g.batch;  // largest b with range_prefix[b] <= first
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if (g.range_prefix[mid] <= first) lo = mid; else hi = mid;
  }
  while (lo + 1 < g.batch && g.range_prefix[lo + 1] <= i) ++lo;
  b = lo;
  t = g.ranges[2 * b] + (int)(i - g.range_prefix[b]);
}

__device__ __forceinline__ void load_vertices(const DrRasterGeometry& g, int b, const int (&v)[3],
                                              Tri& T) {
  const float* base = g.pos + (int64_t)b * g.pos_batch_stride;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    float4 p = load4(base + 4 * (int64_t)v[k]);
    T.x[k] = p.x;
    T.y[k] = p.y;
    T.z[k] = p.z;
    T.w[k] = p.w;
  }
  T.reach_x = reach(T.x, T.w);
  T.reach_y = reach(T.y, T.w);
}

__device__ __forceinline__ void load_tri(const DrRasterGeometry& g, int b, int t, Tri& T,
                                         int (&v)[3]) {
  const int32_t* row = g.tri + 3 * (int64_t)t;
  v[0] = row[0];
  v[1] = row[1];
  v[2] = row[2];
  load_vertices(g, b, v, T);
}

__device__ __forceinline__ bool finite_tri(const Tri& T) {
  bool ok = true;
#pragma unroll
  for (int k = 0; k < 3; ++k)
    ok = ok && isfinite(T.x[k]) && isfinite(T.y[k]) && isfinite(T.z[k]) && isfinite(T.w[k]);
  return ok;
}

// Pixel-centre range [lo, hi] along one axis that may be covered, or lo > hi for none.
// p(n) = (n + 1) * size / 2 - 1/2 is the continuous pixel index of NDC coordinate n; the
// margin covers the float32 error of the projection and of the pixel centres, which grows
// with the image size.
__device__ __forceinline__ void axis_range(float n0, float n1, float n2, int size, int& lo,
                                           int& hi) {
  const float half = 0.5f * (float)size;
  const float p0 = (n0 + 1.0f) * half - 0.5f;
  const float p1 = (n1 + 1.0f) * half - 0.5f;
  const float p2 = (n2 + 1.0f) * half - 0.5f;
  const float margin = 0.015625f + 4e-6f * (float)size;
  float a = fminf(fminf(p0, p1), p2) - margin;
  float c = fmaxf(fmaxf(p0, p1), p2) + margin;
  a = fmaxf(a, -1.0f);
  c = fminf(c, (float)size);
  lo = max((int)ceilf(a), 0);
  hi = min((int)floorf(c), size - 1);
}

// Reciprocal of w (w > 0) through the hardware's approximate reciprocal, within 1 ulp: enough
// for bounds that carry margins far wider than that (boxes, depth bounds and slabs); 0 when it
// does not give a finite value, for the caller to divide instead.
__device__ __forceinline__ float approx_rcp(float w) {
  const float r = __builtin_amdgcn_rcpf(w);
  return isfinite(r) ? r : 0.0f;
}

// x / w and y / w of the vertices (every w > 0), with approx_rcp where it serves.
__device__ __forceinline__ void ndc(const Tri& T, float (&nx)[3], float (&ny)[3]) {
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float r = approx_rcp(T.w[k]);
    nx[k] = T.x[k] * r;
    ny[k] = T.y[k] * r;
    if (r == 0.0f || !isfinite(nx[k]) || !isfinite(ny[k])) {
      nx[k] = T.x[k] / T.w[k];
      ny[k] = T.y[k] / T.w[k];
    }
  }
}

// z / w of the vertices (every w > 0), likewise.
__device__ __forceinline__ void vertex_depths(const Tri& T, float (&d)[3]) {
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float r = approx_rcp(T.w[k]);
    d[k] = T.z[k] * r;
    if (r == 0.0f || !isfinite(d[k])) d[k] = T.z[k] / T.w[k];
  }
}

// A lower bound of the triangle's depth at any pixel it covers (-inf when it crosses the camera
// plane). The depth computed at a covered pixel is a convex combination of the vertex depths
// z_k / w_k up to a few float32 roundings (~6 * 2^-24 of the largest |z_k / w_k|); the margin
// is 1e-5 of it. approx_rcp's error (2^-22 relative) is far inside the margin.
__device__ __forceinline__ float depth_lower_bound(const Tri& T) {
  if (!(T.w[0] > 0.0f && T.w[1] > 0.0f && T.w[2] > 0.0f)) return -__int_as_float(0x7f800000);
  float d[3];
  vertex_depths(T, d);
  const float nearest = fminf(fminf(d[0], d[1]), d[2]);
  const float scale = fmaxf(fmaxf(fabsf(d[0]), fabsf(d[1])), fabsf(d[2]));
  return nearest - 1e-5f * scale;
}

// Box [x_lo, x_hi] x [y_lo, y_hi] of the pixel centres a triangle may cover; empty (lo > hi)
// for a culled triangle. A triangle crossing the camera plane may cover any pixel.
__device__ __forceinline__ void candidate_box(const DrRasterGeometry& g, const Tri& T, int& x_lo,
                                              int& x_hi, int& y_lo, int& y_hi) {
  x_lo = y_lo = 0;
  x_hi = y_hi = -1;
  const bool any_front = T.w[0] > 0.0f || T.w[1] > 0.0f || T.w[2] > 0.0f;
  if (!finite_tri(T) || !any_front) return;
  if (T.w[0] > 0.0f && T.w[1] > 0.0f && T.w[2] > 0.0f) {
    float nx[3], ny[3];
    ndc(T, nx, ny);
    axis_range(nx[0], nx[1], nx[2], g.width, x_lo, x_hi);
    axis_range(ny[0], ny[1], ny[2], g.height, y_lo, y_hi);
  } else {
    x_hi = g.width - 1;
    y_hi = g.height - 1;
  }
}

// The depth a key holds (depth_key's inverse on the upper 32 bits).
__device__ __forceinline__ float key_depth(uint64_t key) {
  const uint32_t ordered = (uint32_t)(key >> 32);
  return __uint_as_float((ordered & 0x80000000u) ? (ordered & 0x7fffffffu) : ~ordered);
}

// The largest of v over the lanes of each 16-lane row, in the row's last lane.
__device__ __forceinline__ uint64_t row_max_u64(uint64_t v) {
  uint64_t o = row_shr64<1>(v);
  v = o > v ? o : v;
  o = row_shr64<2>(v);
  v = o > v ? o : v;
  o = row_shr64<4>(v);
  v = o > v ? o : v;
  o = row_shr64<8>(v);
  return o > v ? o : v;
}

// Merges a key into the key buffer, unless the previous layer rules it out. The atomic
// returns nothing, so a thread never waits on it.
__device__ __forceinline__ void merge_key(uint64_t* keys, const uint64_t* prev, int64_t pixel,
                                          uint64_t key) {
  if (prev != nullptr && key <= prev[pixel]) return;
  atomicMin((unsigned long long*)(keys + pixel), (unsigned long long)key);
}

// ---- workgroup table of tiles -------------------------------------------------------------

// Counts (and, in the bin pass, list reservations) per distinct tile of a workgroup, in LDS.
// A tile whose key finds no free slot within kProbe steps is handled with global atomics; the
// same key always meets the same fate within one pass, so counts and reservations agree.
struct TileTable {
  static constexpr uint32_t kEmpty = 0xffffffffu;
  static constexpr int kProbe = 32;
  uint32_t key[kTileSlots];
  uint32_t count[kTileSlots];
  uint32_t base[kTileSlots];

  __device__ __forceinline__ void clear() {
    for (int i = threadIdx.x; i < kTileSlots; i += blockDim.x) {
      key[i] = kEmpty;
      count[i] = 0u;
    }
  }
  __device__ __forceinline__ static uint32_t hash(uint32_t k) {
    k ^= k >> 16;
    k *= 0x7feb352du;
    k ^= k >> 15;
    return k & (kTileSlots - 1);
  }
  __device__ __forceinline__ int insert(uint32_t k) {
    uint32_t slot = hash(k);
    for (int probe = 0; probe < kProbe; ++probe) {
      const uint32_t seen = atomicCAS(key + slot, kEmpty, k);
      if (seen == kEmpty || seen == k) return (int)slot;
      slot = (slot + 1) & (kTileSlots - 1);
    }
    return -1;
  }
  __device__ __forceinline__ int find(uint32_t k) const {
    uint32_t slot = hash(k);
    for (int probe = 0; probe < kProbe; ++probe) {
      const uint32_t seen = key[slot];
      if (seen == k) return (int)slot;
      if (seen == kEmpty) return -1;
      slot = (slot + 1) & (kTileSlots - 1);
    }
    return -1;
  }
};

// ---- kernels: fills and pixel centres -----------------------------------------------------

// Everything a visibility call starts from, in one launch: the key buffer emptied, the list
// counts, counters and class (and bucket) counts zeroed, the pixel centres tabulated.
__global__ void raster_prepare(uint64_t* keys, int64_t pixels, Workspace ws, int width,
                               int height) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t i = t; i < pixels; i += stride) keys[i] = kEmptyKey;
  for (int64_t i = t; i < ws.lists + 1; i += stride) ws.list_counts[i] = 0u;
  for (int64_t i = t; i < kXcdShares * kWorkClasses; i += stride) ws.class_counts[i] = 0u;
  if (ws.ordered)
    for (int64_t i = t; i < kOrderBuckets; i += stride) ws.bucket_counts[i] = 0u;
  if (t < 4) ws.counters[t] = t == 0 ? (uint32_t)ws.record_blocks : 0u;
  for (int64_t i = t; i < width; i += stride) ws.px[i] = pixel_centre((int)i, width);
  for (int64_t i = t; i < height; i += stride) ws.py[i] = pixel_centre((int)i, height);
}

// ---- kernels: triangle order --------------------------------------------------------------

__device__ __forceinline__ uint32_t ordered_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_ordered_bits(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

// Centroid of every triangle in the first view, and per workgroup the bounds of the finite
// ones (order-preserving bits: min x, y, z, then max x, y, z).
__global__ __launch_bounds__(256) void order_centroids(DrRasterGeometry g, Workspace ws) {
  __shared__ uint32_t s_part[256 / DR_WAVE][6];
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t b[6] = {0xffffffffu, 0xffffffffu, 0xffffffffu, 0u, 0u, 0u};
  if (t < g.num_tri) {
    const int32_t* row = g.tri + 3 * (int64_t)t;
    float c[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const float4 p = load4(g.pos + 4 * (int64_t)row[k]);
      c[0] += p.x;
      c[1] += p.y;
      c[2] += p.z;
    }
    ws.centroids[t] = make_float4(c[0], c[1], c[2], 0.0f);
    if (isfinite(c[0]) && isfinite(c[1]) && isfinite(c[2])) {
#pragma unroll
      for (int k = 0; k < 3; ++k) b[k] = b[3 + k] = ordered_bits(c[k]);
    }
  }
#pragma unroll
  for (int d = 1; d < DR_WAVE; d <<= 1)
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      b[k] = min(b[k], (uint32_t)__shfl_xor(b[k], d));
      b[3 + k] = max(b[3 + k], (uint32_t)__shfl_xor(b[3 + k], d));
    }
  if (lane_id() == 0)
#pragma unroll
    for (int k = 0; k < 6; ++k) s_part[threadIdx.x / DR_WAVE][k] = b[k];
  __syncthreads();
  if (threadIdx.x < 6) {
    const int k = threadIdx.x;
    uint32_t v = s_part[0][k];
    for (int w = 1; w < 256 / DR_WAVE; ++w) v = k < 3 ? min(v, s_part[w][k]) : max(v, s_part[w][k]);
    ws.bound_parts[6 * blockIdx.x + k] = v;
  }
}

// The bounds over all workgroups' parts (one workgroup).
__global__ __launch_bounds__(256) void order_bounds(Workspace ws, int parts) {
  __shared__ uint32_t s_part[256 / DR_WAVE][6];
  uint32_t b[6] = {0xffffffffu, 0xffffffffu, 0xffffffffu, 0u, 0u, 0u};
  for (int i = threadIdx.x; i < parts; i += blockDim.x)
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const uint32_t v = ws.bound_parts[6 * i + k];
      b[k] = k < 3 ? min(b[k], v) : max(b[k], v);
    }
#pragma unroll
  for (int d = 1; d < DR_WAVE; d <<= 1)
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      b[k] = min(b[k], (uint32_t)__shfl_xor(b[k], d));
      b[3 + k] = max(b[3 + k], (uint32_t)__shfl_xor(b[3 + k], d));
    }
  if (lane_id() == 0)
#pragma unroll
    for (int k = 0; k < 6; ++k) s_part[threadIdx.x / DR_WAVE][k] = b[k];
  __syncthreads();
  if (threadIdx.x < 6) {
    const int k = threadIdx.x;
    uint32_t v = s_part[0][k];
    for (int w = 1; w < 256 / DR_WAVE; ++w) v = k < 3 ? min(v, s_part[w][k]) : max(v, s_part[w][k]);
    ws.bounds[k] = v;
  }
}

__device__ __forceinline__ uint32_t spread10(uint32_t v) {
  v &= 1023u;
  v = (v | (v << 16)) & 0x030000FFu;
  v = (v | (v << 8)) & 0x0300F00Fu;
  v = (v | (v << 4)) & 0x030C30C3u;
  v = (v | (v << 2)) & 0x09249249u;
  return v;
}

// Morton bucket (top 12 bits of a 30-bit code) of a triangle's centroid c.
__device__ __forceinline__ uint32_t order_bucket(const Workspace& ws, float4 c) {
  const float cc[3] = {c.x, c.y, c.z};
  uint32_t q[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float lo = from_ordered_bits(ws.bounds[k]), hi = from_ordered_bits(ws.bounds[3 + k]);
    const float range = hi - lo;
    float u = range > 0.0f ? (cc[k] - lo) / range : 0.0f;
    u = isfinite(u) ? fminf(fmaxf(u, 0.0f), 1.0f) : 0.0f;
    q[k] = min((uint32_t)(u * 1024.0f), 1023u);
  }
  const uint32_t code = (spread10(q[0]) << 2) | (spread10(q[1]) << 1) | spread10(q[2]);
  return code >> 18;
}

// The bucket passes give each workgroup 4096 triangles (16 per thread), so that clearing and
// flushing its LDS histogram of kOrderBuckets counts is paid once per 4096 triangles.
constexpr int kOrderPerThread = 16;

__global__ __launch_bounds__(256) void order_count(DrRasterGeometry g, Workspace ws) {
  __shared__ uint32_t hist[kOrderBuckets];
  for (int i = threadIdx.x; i < kOrderBuckets; i += blockDim.x) hist[i] = 0u;
  __syncthreads();
  // The thread's centroids are all loaded before the first is used (a clamped index past the
  // end, not a branch, so nothing separates the loads).
  const int64_t first = (int64_t)blockIdx.x * blockDim.x * kOrderPerThread;
  float4 c[kOrderPerThread];
#pragma unroll
  for (int i = 0; i < kOrderPerThread; ++i) {
    const int64_t t = first + (int64_t)i * blockDim.x + threadIdx.x;
    c[i] = ws.centroids[t < g.num_tri ? t : g.num_tri - 1];
  }
#pragma unroll
  for (int i = 0; i < kOrderPerThread; ++i) {
    const int64_t t = first + (int64_t)i * blockDim.x + threadIdx.x;
    if (t >= g.num_tri) continue;
    const uint32_t bucket = order_bucket(ws, c[i]);
    ws.centroids[t].w = __uint_as_float(bucket);  // for order_place
    atomicAdd(hist + bucket, 1u);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kOrderBuckets; i += blockDim.x)
    if (hist[i]) atomicAdd(ws.bucket_counts + i, hist[i]);
}

// Exclusive scan of the bucket counts into the bucket cursors (one workgroup).
__global__ __launch_bounds__(256) void order_scan(Workspace ws) {
  __shared__ uint32_t part[256];
  constexpr int kPer = kOrderBuckets / 256;
  uint32_t local[kPer], sum = 0;
  for (int k = 0; k < kPer; ++k) {
    local[k] = ws.bucket_counts[threadIdx.x * kPer + k];
    sum += local[k];
  }
  part[threadIdx.x] = sum;
  __syncthreads();
  for (int d = 1; d < 256; d <<= 1) {
    const uint32_t v = threadIdx.x >= (unsigned)d ? part[threadIdx.x - d] : 0u;
    __syncthreads();
    part[threadIdx.x] += v;
    __syncthreads();
  }
  uint32_t run = part[threadIdx.x] - sum;
  for (int k = 0; k < kPer; ++k) {
    ws.bucket_cursor[threadIdx.x * kPer + k] = run;
    run += local[k];
  }
}

__global__ __launch_bounds__(256) void order_place(DrRasterGeometry g, Workspace ws) {
  __shared__ uint32_t hist[kOrderBuckets];
  __shared__ uint32_t base[kOrderBuckets];
  for (int i = threadIdx.x; i < kOrderBuckets; i += blockDim.x) hist[i] = 0u;
  __syncthreads();
  // The thread's buckets, all loaded before the first is used (clamped index past the end).
  const int64_t first = (int64_t)blockIdx.x * blockDim.x * kOrderPerThread;
  uint32_t bucket[kOrderPerThread];
#pragma unroll
  for (int i = 0; i < kOrderPerThread; ++i) {
    const int64_t t = first + (int64_t)i * blockDim.x + threadIdx.x;
    bucket[i] = __float_as_uint(ws.centroids[t < g.num_tri ? t : g.num_tri - 1].w);
  }
#pragma unroll
  for (int i = 0; i < kOrderPerThread; ++i) {
    const int64_t t = first + (int64_t)i * blockDim.x + threadIdx.x;
    if (t < g.num_tri) atomicAdd(hist + bucket[i], 1u);
  }
  __syncthreads();
  // The reservations: each thread's buckets' atomics are all issued before it waits for any.
  constexpr int kBucketsPerThread = kOrderBuckets / 256;
  uint32_t reserved[kBucketsPerThread];
#pragma unroll
  for (int k = 0; k < kBucketsPerThread; ++k) {
    const int i = threadIdx.x + k * 256;
    reserved[k] = hist[i] ? atomicAdd(ws.bucket_cursor + i, hist[i]) : 0u;
  }
#pragma unroll
  for (int k = 0; k < kBucketsPerThread; ++k) {
    const int i = threadIdx.x + k * 256;
    base[i] = reserved[k];
    hist[i] = 0u;
  }
  __syncthreads();
  // The index rows, a quarter of the thread's triangles at a time, loaded before their use.
  constexpr int kQuarter = kOrderPerThread / 4;
#pragma unroll
  for (int q = 0; q < kOrderPerThread; q += kQuarter) {
    int32_t rows[kQuarter][3];
#pragma unroll
    for (int i = 0; i < kQuarter; ++i) {
      const int64_t t = first + (int64_t)(q + i) * blockDim.x + threadIdx.x;
      const int32_t* row = g.tri + 3 * (t < g.num_tri ? t : g.num_tri - 1);
      rows[i][0] = row[0];
      rows[i][1] = row[1];
      rows[i][2] = row[2];
    }
#pragma unroll
    for (int i = 0; i < kQuarter; ++i) {
      const int64_t t = first + (int64_t)(q + i) * blockDim.x + threadIdx.x;
      if (t >= g.num_tri) continue;
      const uint32_t b = bucket[q + i];
      ws.order[base[b] + atomicAdd(hist + b, 1u)] =
          make_int4(rows[i][0], rows[i][1], rows[i][2], (int)t);
    }
  }
}

// ---- kernels: depth range ----------------------------------------------------------------

// Nearest and farthest depth z / w, clipped to [-1, 1], of the vertices in front of the camera,
// per image (or once when pos is shared): the span the depth slabs divide. Each of
// kRangeParts workgroups of 1024 threads per image reduces a share of its vertices to a partial
// span (1024 threads: enough waves to keep the loads in flight with 64 workgroups per image); a
// second pass merges the partial spans (no atomics on a handful of addresses).
__global__ __launch_bounds__(1024) void raster_depth_range(DrRasterGeometry g, Workspace ws) {
  __shared__ uint32_t s_lo[1024 / DR_WAVE], s_hi[1024 / DR_WAVE];
  const int image = blockIdx.x / kRangeParts, part = blockIdx.x % kRangeParts;
  const float* P = g.pos + (int64_t)image * g.pos_batch_stride;
  // Four vertices per thread and step, loaded before any is used; the span only places
  // triangles in depth slabs (an ordering), so the hardware reciprocal serves for z / w.
  uint32_t lo = 0xffffffffu, hi = 0u;
  const int step = kRangeParts * blockDim.x;
  for (int v0 = part * blockDim.x + threadIdx.x; v0 < g.num_vertices; v0 += 4 * step) {
    float4 p[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int v = v0 + u * step;
      p[u] = v < g.num_vertices ? load4(P + 4 * (int64_t)v) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float d = p[u].z * __builtin_amdgcn_rcpf(p[u].w);
      if (p[u].w > 0.0f && isfinite(d)) {
        const uint32_t bits = ordered_bits(fminf(fmaxf(d, -1.0f), 1.0f));
        lo = min(lo, bits);
        hi = max(hi, bits);
      }
    }
  }
#pragma unroll
  for (int d = 1; d < DR_WAVE; d <<= 1) {
    lo = min(lo, (uint32_t)__shfl_xor(lo, d));
    hi = max(hi, (uint32_t)__shfl_xor(hi, d));
  }
  if (lane_id() == 0) {
    s_lo[threadIdx.x / DR_WAVE] = lo;
    s_hi[threadIdx.x / DR_WAVE] = hi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 1024 / DR_WAVE; ++w) {
      lo = min(lo, s_lo[w]);
      hi = max(hi, s_hi[w]);
    }
    ws.range_parts[2 * blockIdx.x] = lo;
    ws.range_parts[2 * blockIdx.x + 1] = hi;
  }
}

__global__ __launch_bounds__(kRangeParts) void raster_depth_range_merge(Workspace ws) {
  const int image = blockIdx.x;
  uint32_t lo = ws.range_parts[2 * (image * kRangeParts + threadIdx.x)];
  uint32_t hi = ws.range_parts[2 * (image * kRangeParts + threadIdx.x) + 1];
#pragma unroll
  for (int d = 1; d < kRangeParts; d <<= 1) {
    lo = min(lo, (uint32_t)__shfl_xor(lo, d));
    hi = max(hi, (uint32_t)__shfl_xor(hi, d));
  }
  if (threadIdx.x == 0) {
    ws.depth_range[2 * image] = lo;
    ws.depth_range[2 * image + 1] = hi;
  }
}

// Depth slab of a binned triangle: its nearest vertex depth's place in the image's depth span
// (order-preserving bits of its nearest and farthest depth, from ws.depth_range). Triangles that
// cross the camera plane, or have a vertex depth beyond [-1, 1], go first (slab 0): in slab
// s >= 1 every triangle's depth_lower_bound is at least slab_floor(span, s, slabs).
__device__ __forceinline__ int depth_slab(uint2 span, const Tri& T, int slabs) {
  if (slabs == 1 || !(T.w[0] > 0.0f && T.w[1] > 0.0f && T.w[2] > 0.0f)) return 0;
  float d[3];
  vertex_depths(T, d);
  if (!(fmaxf(fmaxf(fabsf(d[0]), fabsf(d[1])), fabsf(d[2])) <= 1.0f)) return 0;
  const float nearest = fminf(fminf(d[0], d[1]), d[2]);
  const float lo = from_ordered_bits(span.x);
  const float hi = from_ordered_bits(span.y);
  const float f = (nearest - lo) / (hi - lo) * (float)slabs;
  if (!(hi > lo) || !isfinite(f)) return 0;
  return min(max((int)f, 0), slabs - 1);
}

// A lower bound of depth_lower_bound over the triangles of slab s >= 1 (depth_slab). Such a
// triangle has all w > 0, every vertex depth within [-1, 1] and f = fl(fl(fl(nearest - lo) /
// fl(hi - lo)) * slabs) >= s, so nearest >= lo + s (hi - lo) / slabs * (1 - 3 * 2^-24) (three
// roundings of relative error at most 2^-24; the product by slabs, a power of two, is exact);
// its bound fl(nearest - fl(1e-5 * scale)) with scale <= 1 is then above nearest - 1.0001e-5 -
// 2^-23. Evaluated in double (exact for these float operands up to 2^-50 relative) with that
// slack widened to 2e-5 + 2^-20.
__device__ __forceinline__ double slab_floor(uint2 span, int s, int slabs) {
  const double lo = (double)from_ordered_bits(span.x);
  const double hi = (double)from_ordered_bits(span.y);
  return lo + (double)s * (hi - lo) / (double)slabs * (1.0 - 4.0 / 16777216.0) - 2e-5 -
         1.0 / 1048576.0;
}

// ---- kernels: setup, scan, bin, tiles -----------------------------------------------------

// Splits work item p of a box bw pixels wide (bw <= 64, p < 64) into (dx, dy). The float
// quotient (p + 1/2) / bw lies at least 1/128 away from an integer, far more than the error of
// the approximate reciprocal (2^-22 relative, below 2^-15 here), so the truncation is exact.
__device__ __forceinline__ void box_cell(int p, int bw, int& dx, int& dy) {
  dy = (int)(((float)p + 0.5f) * __builtin_amdgcn_rcpf((float)bw));
  dx = p - dy * bw;
}

// Packs a box of at most 16 x 16 pixels: x0 | (w - 1) << 8 | y0 << 16 | (h - 1) << 24.
__device__ __forceinline__ uint32_t pack_box(int x0, int w, int y0, int h) {
  return (uint32_t)x0 | ((uint32_t)(w - 1) << 8) | ((uint32_t)y0 << 16) |
         ((uint32_t)(h - 1) << 24);
}

// Small triangles of a workgroup staged for the wave that rasterizes them.
struct SmallStage {
  float4 tri[256][4];  // the three vertices, then (reach_x, reach_y, row bits, image bits)
  uint2 box[256];      // (x0 | (w - 1) << 20, y0 | (h - 1) << 20), w * h <= small_pixels()
  int start[256];      // first work item of each lane's triangle within its wave
  uint8_t mark[256 / DR_WAVE][DR_WAVE];  // per wave: lane + 1 at the first item of its triangle
};

// One thread per triangle instance. A small triangle's pixels become work items of its wave
// (lane j owns items start[j] .. start[j + 1] - 1), which the wave's lanes take in steps of 64;
// the others are binned, their per-tile counts gathered in the workgroup's tile table.
__global__ __launch_bounds__(256) void raster_setup_kernel(DrRasterGeometry g,
                                                           const uint64_t* prev, uint64_t* keys,
                                                           Workspace ws, int small_limit) {
  __shared__ union {
    SmallStage small;
    TileTable table;
  } lds;
  __shared__ int s_wave_binned[256 / DR_WAVE];
  const int64_t block = xcd_order(blockIdx.x, gridDim.x);
  const int64_t i = block * blockDim.x + threadIdx.x;
  bool binned = false;
  int area = 0;
  uint2 span = make_uint2(0u, 0u);  // the image's depth span, for a binned triangle's slab
  int b = 0, t = 0, x_lo = 0, x_hi = -1, y_lo = 0, y_hi = -1;
  Tri T;
  if (i < g.num_instances) {
    int v[3];
    if (ws.ordered) {  // the ordered triangle carries its vertex rows: one load fewer in line
      b = (int)(i / g.num_tri);
      const int4 o = ws.order[i - (int64_t)b * g.num_tri];
      v[0] = o.x;
      v[1] = o.y;
      v[2] = o.z;
      t = o.w;
      load_vertices(g, b, v, T);
    } else {
      instance(g, i, b, t);
      load_tri(g, b, t, T, v);
    }
    // Loaded now and used after the small triangles' work, which hides the load's latency.
    if (ws.slabs > 1) span = reinterpret_cast<const uint2*>(ws.depth_range)[ws.depth_ranges > 1 ? b : 0];
    candidate_box(g, T, x_lo, x_hi, y_lo, y_hi);
    if (x_lo <= x_hi && y_lo <= y_hi) {
      const int64_t count = (int64_t)(x_hi - x_lo + 1) * (y_hi - y_lo + 1);
      if (count <= small_limit) {
        area = (int)count;
        SmallStage& st = lds.small;
#pragma unroll
        for (int k = 0; k < 3; ++k)
          st.tri[threadIdx.x][k] = make_float4(T.x[k], T.y[k], T.z[k], T.w[k]);
        st.tri[threadIdx.x][3] = make_float4(T.reach_x, T.reach_y, __int_as_float(t),
                                             __int_as_float(b));
        st.box[threadIdx.x] = make_uint2((uint32_t)x_lo | ((uint32_t)(x_hi - x_lo) << 20),
                                         (uint32_t)y_lo | ((uint32_t)(y_hi - y_lo) << 20));
      } else {
        binned = true;
      }
    }
  }
  // Small triangles: exclusive prefix of the areas over the wave, then the wave's items, 64
  // per round. An item's triangle (lane) is found by marks: the lane whose first item falls in
  // the round marks that place with lane + 1, and a max-scan over the round (marks grow with
  // the lane) gives each item the last mark at or before it, or the last triangle of the
  // rounds before.
  const int lane = lane_id();
  const int wave_base = threadIdx.x - lane;
  const int incl = (int)wave_inclusive_sum((uint32_t)area);
  const int total = __builtin_amdgcn_readlane(incl, DR_WAVE - 1);
  const int first_item = incl - area;
  lds.small.start[threadIdx.x] = first_item;
  uint8_t* mark = lds.small.mark[threadIdx.x / DR_WAVE];
  __syncthreads();
  uint32_t carry = 0u;
  // Pixel centres (2 i + 1) / size - 1: for a power-of-two size the quotient is the exact
  // product with 1 / size (2 i + 1 < 2^24), so three instructions give pixel_centre()'s bits
  // without the table's dependent load; other sizes read the table.
  const bool pow2 = (g.width & (g.width - 1)) == 0 && (g.height & (g.height - 1)) == 0;
  const float inv_w = 1.0f / (float)g.width, inv_h = 1.0f / (float)g.height;
  for (int round = 0; round < total; round += DR_WAVE) {  // uniform over the wave
    mark[lane] = 0;
    if (area > 0 && first_item >= round && first_item < round + DR_WAVE)
      mark[first_item - round] = (uint8_t)(lane + 1);
    // Lanes read marks other lanes of the wave wrote: the fences keep the compiler from
    // answering the read from this lane's own store.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint32_t owner_mark = max(wave_inclusive_max((uint32_t)mark[lane]), carry);
    carry = (uint32_t)__builtin_amdgcn_readlane((int)owner_mark, DR_WAVE - 1);
    const int item = round + lane;
    if (item >= total) continue;
    const int j = (int)owner_mark - 1;
    const int* start = lds.small.start + wave_base;
    const int owner = wave_base + j;
    const float4 v0 = lds.small.tri[owner][0], v1 = lds.small.tri[owner][1];
    const float4 v2 = lds.small.tri[owner][2], extra = lds.small.tri[owner][3];
    const uint2 box = lds.small.box[owner];
    int dx, dy;
    box_cell(item - start[j], (int)(box.x >> 20) + 1, dx, dy);
    const int x = (int)(box.x & 0xfffffu) + dx, y = (int)(box.y & 0xfffffu) + dy;
    const float X[3] = {v0.x, v1.x, v2.x}, Y[3] = {v0.y, v1.y, v2.y};
    const float Z[3] = {v0.z, v1.z, v2.z}, Wv[3] = {v0.w, v1.w, v2.w};
    float cx, cy;
    if (pow2) {  // uniform
      cx = (float)(2 * x + 1) * inv_w - 1.0f;
      cy = (float)(2 * y + 1) * inv_h - 1.0f;
    } else {
      cx = ws.px[x];
      cy = ws.py[y];
    }
    float depth;
    if (covers(X, Y, Z, Wv, extra.x, extra.y, cx, cy, depth)) {
      const int64_t pixel = ((int64_t)__float_as_int(extra.w) * g.height + y) * g.width + x;
      merge_key(keys, prev, pixel, depth_key(depth, (uint32_t)__float_as_int(extra.z)));
    }
  }
  // Binned triangles go to this workgroup's record slots, compacted in thread order.
  const int wave = threadIdx.x / DR_WAVE;
  const uint64_t mask = __ballot(binned);
  if (lane == 0) s_wave_binned[wave] = __popcll(mask);
  __syncthreads();  // the stage's memory becomes the tile table
  lds.table.clear();
  int before = 0, block_binned = 0;
#pragma unroll
  for (int w = 0; w < 256 / DR_WAVE; ++w) {
    before += w < wave ? s_wave_binned[w] : 0;
    block_binned += s_wave_binned[w];
  }
  if (threadIdx.x == 0) ws.block_records[block] = (uint32_t)block_binned;
  __syncthreads();
  TileTable& table = lds.table;

  {
    if (binned) {
      const uint32_t rec = (uint32_t)(block * 256 + before) +
                           (uint32_t)__popcll(mask & ((1ull << lane) - 1ull));
      const int tx0 = x_lo / kTile, tx1 = x_hi / kTile, ty0 = y_lo / kTile, ty1 = y_hi / kTile;
      const int slab = depth_slab(span, T, ws.slabs);
      float4* out = ws.records + (size_t)rec * kRecord;
#pragma unroll
      for (int k = 0; k < 3; ++k) out[k] = make_float4(T.x[k], T.y[k], T.z[k], T.w[k]);
      const uint32_t tx_range = (uint32_t)tx0 | ((uint32_t)tx1 << 16);
      const uint32_t ty_range = (uint32_t)ty0 | ((uint32_t)ty1 << 16);
      out[3] = make_float4(__int_as_float(b), __int_as_float(t | (slab << 24)),
                           __uint_as_float(tx_range), __uint_as_float(ty_range));
      const uint32_t list0 = (uint32_t)b * ws.tiles_x * ws.tiles_y * ws.slabs + (uint32_t)slab;
      ws.record_bins[rec] =
          make_uint4(tx_range, ty_range, list0, __float_as_uint(depth_lower_bound(T)));
      for (int ty = ty0; ty <= ty1; ++ty)
        for (int tx = tx0; tx <= tx1; ++tx) {
          const uint32_t list = list0 + (uint32_t)(ty * ws.tiles_x + tx) * ws.slabs;
          const int slot = table.insert(list);
          if (slot >= 0)
            atomicAdd(table.count + slot, 1u);
          else
            atomicAdd(ws.list_counts + list, 1u);
        }
    }
  }
  __syncthreads();
  for (int s = threadIdx.x; s < kTileSlots; s += blockDim.x)
    if (table.key[s] != TileTable::kEmpty) atomicAdd(ws.list_counts + table.key[s], table.count[s]);
}

// Inclusive scan of (entries, chunks) pairs over the 256 threads of a block.
__device__ __forceinline__ uint2 block_inclusive_scan(uint2 v, uint2* lds) {
  const int lane = lane_id();
  const int wave = threadIdx.x / DR_WAVE;
#pragma unroll
  for (int d = 1; d < DR_WAVE; d <<= 1) {
    uint32_t ax = __shfl_up(v.x, d), ay = __shfl_up(v.y, d);
    if (lane >= d) {
      v.x += ax;
      v.y += ay;
    }
  }
  if (lane == DR_WAVE - 1) lds[wave] = v;
  __syncthreads();
  uint2 offset = make_uint2(0, 0);
  for (int k = 0; k < wave; ++k) {
    offset.x += lds[k].x;
    offset.y += lds[k].y;
  }
  __syncthreads();
  return make_uint2(v.x + offset.x, v.y + offset.y);
}

__device__ __forceinline__ uint2 scan_item(const uint32_t* counts, int64_t i, int64_t n) {
  uint32_t c = i < n ? counts[i] : 0u;
  return make_uint2(c, (c + kChunk - 1) / kChunk);
}

// Phase 1: per-block totals.
__global__ __launch_bounds__(256) void raster_scan_reduce(const uint32_t* counts, int64_t n,
                                                          uint2* block_sums) {
  __shared__ uint2 lds[4];
  const int64_t base = (int64_t)blockIdx.x * kScanBlock + threadIdx.x * 4;
  uint2 s = make_uint2(0, 0);
  for (int k = 0; k < 4; ++k) {
    uint2 v = scan_item(counts, base + k, n);
    s.x += v.x;
    s.y += v.y;
  }
  uint2 total = block_inclusive_scan(s, lds);
  if (threadIdx.x == 255) block_sums[blockIdx.x] = total;
}

// Phase 2: exclusive scan of the block totals in one block; totals go to the counters.
__global__ __launch_bounds__(256) void raster_scan_blocks(uint2* block_sums, int blocks,
                                                          uint32_t* counters) {
  __shared__ uint2 lds[4];
  __shared__ uint2 step_total;
  uint2 carry = make_uint2(0, 0);
  for (int start = 0; start < blocks; start += 256) {
    const int i = start + threadIdx.x;
    const uint2 v = i < blocks ? block_sums[i] : make_uint2(0, 0);
    const uint2 inc = block_inclusive_scan(v, lds);
    if (i < blocks) block_sums[i] = make_uint2(carry.x + inc.x - v.x, carry.y + inc.y - v.y);
    if (threadIdx.x == 255) step_total = inc;
    __syncthreads();
    carry.x += step_total.x;
    carry.y += step_total.y;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    counters[1] = carry.x;
  }
}

// Phase 3: exclusive offsets per tile (and the totals at index n).
__global__ __launch_bounds__(256) void raster_scan_apply(const uint32_t* counts, int64_t n,
                                                         const uint2* block_sums,
                                                         uint32_t* offsets, uint32_t* cursor,
                                                         uint32_t* chunk_offsets) {
  __shared__ uint2 lds[4];
  const int64_t base = (int64_t)blockIdx.x * kScanBlock + threadIdx.x * 4;
  uint2 items[4];
  uint2 s = make_uint2(0, 0);
  for (int k = 0; k < 4; ++k) {
    items[k] = scan_item(counts, base + k, n);
    s.x += items[k].x;
    s.y += items[k].y;
  }
  uint2 inc = block_inclusive_scan(s, lds);
  uint2 run = make_uint2(block_sums[blockIdx.x].x + inc.x - s.x,
                         block_sums[blockIdx.x].y + inc.y - s.y);
  for (int k = 0; k < 4; ++k) {
    const int64_t i = base + k;
    if (i <= n) {
      offsets[i] = run.x;
      chunk_offsets[i] = run.y;
      if (i < n) cursor[i] = run.x;
    }
    run.x += items[k].x;
    run.y += items[k].y;
  }
}

// Fills the per-tile lists: the workgroup counts its records per tile in LDS, reserves its
// share of each tile's list with one global atomic, then writes the entries. A workgroup takes
// the records of kBinBlocks consecutive setup workgroups (neighbours in the processing order,
// so they share tiles): fewer reservations, and fewer workgroups waiting on their round trip
// (bin pass 186 -> 163 us at 8 x 1024^2 with two; 172 us with four).
constexpr int kBinBlocks = 2;

__global__ __launch_bounds__(256) void raster_bin_kernel(Workspace ws, uint2* entries,
                                                         uint32_t capacity) {
  // Entries beyond the buffer's capacity: the pass is left to a later launch with a larger
  // buffer (the cursors stay untouched, so that launch places every entry).
  if (ws.counters[1] > capacity) return;  // uniform over the grid
  __shared__ TileTable table;
  table.clear();
  __syncthreads();
  // This thread's record of each of the workgroup's setup workgroups: tile range, first list,
  // and the triangle's depth bound, which each entry carries so that the tile pass can skip a
  // triangle behind every key of its tile without reading its record.
  int tx0[kBinBlocks], tx1[kBinBlocks], ty0[kBinBlocks], ty1[kBinBlocks];
  uint32_t list0[kBinBlocks], bound_bits[kBinBlocks], rec[kBinBlocks];
#pragma unroll
  for (int q = 0; q < kBinBlocks; ++q) {
    const int block = (int)blockIdx.x * kBinBlocks + q;
    tx0[q] = ty0[q] = 0;
    tx1[q] = ty1[q] = -1;
    list0[q] = bound_bits[q] = 0u;
    rec[q] = (uint32_t)block * 256u + threadIdx.x;
    if (block < ws.record_blocks && threadIdx.x < ws.block_records[block]) {
      const uint4 info = ws.record_bins[rec[q]];
      tx0[q] = (int)(info.x & 0xffffu);
      tx1[q] = (int)(info.x >> 16);
      ty0[q] = (int)(info.y & 0xffffu);
      ty1[q] = (int)(info.y >> 16);
      list0[q] = info.z;
      bound_bits[q] = info.w;
    }
  }
#pragma unroll
  for (int q = 0; q < kBinBlocks; ++q)
    for (int ty = ty0[q]; ty <= ty1[q]; ++ty)
      for (int tx = tx0[q]; tx <= tx1[q]; ++tx) {
        const int slot = table.insert(list0[q] + (uint32_t)(ty * ws.tiles_x + tx) * ws.slabs);
        if (slot >= 0) atomicAdd(table.count + slot, 1u);
      }
  __syncthreads();
  // The reservations: each thread's slots' atomics are all issued before it waits for any.
  constexpr int kSlotsPerThread = kTileSlots / 256;
  uint32_t reserved[kSlotsPerThread];
#pragma unroll
  for (int k = 0; k < kSlotsPerThread; ++k) {
    const int s = threadIdx.x + k * 256;
    reserved[k] = 0u;
    if (table.key[s] != TileTable::kEmpty)
      reserved[k] = atomicAdd(ws.list_cursor + table.key[s], table.count[s]);
  }
#pragma unroll
  for (int k = 0; k < kSlotsPerThread; ++k) {
    const int s = threadIdx.x + k * 256;
    table.base[s] = reserved[k];
    table.count[s] = 0u;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kBinBlocks; ++q)
    for (int ty = ty0[q]; ty <= ty1[q]; ++ty)
      for (int tx = tx0[q]; tx <= tx1[q]; ++tx) {
        const uint32_t list = list0[q] + (uint32_t)(ty * ws.tiles_x + tx) * ws.slabs;
        const int slot = table.find(list);
        const uint32_t at = slot >= 0 ? table.base[slot] + atomicAdd(table.count + slot, 1u)
                                      : atomicAdd(ws.list_cursor + list, 1u);
        entries[at] = make_uint2(rec[q], bound_bits[q]);
      }
}

static int bin_grid(const Workspace& ws) {
  return (ws.record_blocks + kBinBlocks - 1) / kBinBlocks;
}

// ---- tile order: heavy tiles first within each XCD's share -----------------------------------
//
// The tile pass takes tiles in this order: the busy tiles in their XCD shares' order (so that
// XCD k, which takes the k-th eighth of the workgroups under xcd_order, gets about share k),
// within a share the tiles with the most binned triangles first, so that the longest
// workgroups do not start last. A counting sort by entry count in kWorkClasses
// classes of 32 entries, in three passes over the tiles (classes and their counts, the class
// cursors, placement); workgroups aggregate in LDS before touching global counters. The order
// within a class is free: tiles are independent.

// The XCD share of tile i under xcd_order, and the first tile of share k.
__device__ __forceinline__ int xcd_share(int64_t i, int64_t tiles) {
  if (tiles < kXcdShares) return (int)i;
  const int64_t per = tiles / kXcdShares, extra = tiles % kXcdShares;
  const int64_t big = extra * (per + 1);
  return i < big ? (int)(i / (per + 1)) : (int)(extra + (i - big) / per);
}
__device__ __forceinline__ int64_t share_start(int k, int64_t tiles) {
  if (tiles < kXcdShares) return k;
  const int64_t per = tiles / kXcdShares, extra = tiles % kXcdShares;
  return k * per + (k < extra ? k : extra);
}

// Pass 1, one thread per tile: its class (kept for pass 3), the class counts of each share and
// the number of tiles with binned triangles (counters[3], the tile pass's busy workgroups).
__global__ __launch_bounds__(256) void raster_tile_classes(Workspace ws) {
  __shared__ uint32_t hist[kXcdShares * kWorkClasses];
  __shared__ uint32_t busy;
  for (int i = threadIdx.x; i < kXcdShares * kWorkClasses; i += blockDim.x) hist[i] = 0u;
  if (threadIdx.x == 0) busy = 0u;
  __syncthreads();
  const int64_t tile = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  bool has = false;
  if (tile < ws.tiles) {
    const uint32_t n =
        ws.list_offsets[(tile + 1) * ws.slabs] - ws.list_offsets[tile * ws.slabs];
    // Class 0: no entries; then one class per 32 entries, the last one open-ended.
    const int c = n == 0 ? 0 : (int)min((n >> 5) + 1, (uint32_t)(kWorkClasses - 1));
    ws.tile_class[tile] = (uint8_t)c;
    atomicAdd(hist + xcd_share(tile, ws.tiles) * kWorkClasses + c, 1u);
    has = n > 0;
  }
  const uint64_t mask = __ballot(has);
  if (lane_id() == 0 && mask != 0) atomicAdd(&busy, (uint32_t)__popcll(mask));
  __syncthreads();
  for (int i = threadIdx.x; i < kXcdShares * kWorkClasses; i += blockDim.x)
    if (hist[i]) atomicAdd(ws.class_counts + i, hist[i]);
  if (threadIdx.x == 0 && busy) atomicAdd(ws.counters + 3, busy);
}

// Pass 2, one workgroup: first position of each class. The busy tiles come first, share by
// share, heaviest class first within a share; the tiles without entries follow, so that the
// tile pass launches one workgroup per busy tile. The classes' offsets are a scan over 32
// threads per share (a serial walk over the 128 classes, writing each cursor twice, took 10 us).
__global__ __launch_bounds__(256) void raster_tile_cursors(Workspace ws) {
  static_assert(kXcdShares * 32 == 256 && kWorkClasses == 4 * 32,
                "32 threads per share, 4 classes each");
  __shared__ uint32_t busy[kXcdShares], idle[kXcdShares];
  // Thread t takes share k = t / 32 and its classes 127 - 4s .. 124 - 4s (s = t % 32), heaviest
  // first; class 0 (no entries) is counted apart.
  const int k = threadIdx.x / 32, s = threadIdx.x % 32;
  uint32_t v[4], local = 0u;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = kWorkClasses - 1 - 4 * s - q;
    v[q] = c >= 1 ? ws.class_counts[k * kWorkClasses + c] : 0u;
    local += v[q];
  }
  // Exclusive prefix of the share's classes in that order: a wave holds two shares (lanes 0-31
  // and 32-63), so the upper half drops the lower half's total.
  const uint32_t incl = wave_inclusive_sum(local);
  const uint32_t lower = (uint32_t)__builtin_amdgcn_readlane((int)incl, 31);
  const uint32_t share_incl = lane_id() >= 32 ? incl - lower : incl;
  if (s == 31) {
    busy[k] = share_incl;
    idle[k] = ws.class_counts[k * kWorkClasses];
  }
  __syncthreads();
  uint32_t first = 0u, idle_first = 0u, widest = 0u;
#pragma unroll
  for (int j = 0; j < kXcdShares; ++j) {
    first += j < k ? busy[j] : 0u;
    idle_first += busy[j] + (j < k ? idle[j] : 0u);
    widest = max(widest, busy[j]);
  }
  uint32_t at = first + share_incl - local;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = kWorkClasses - 1 - 4 * s - q;
    if (c >= 1) ws.class_cursor[k * kWorkClasses + c] = at;
    at += v[q];
  }
  if (s == 0) {
    ws.class_cursor[k * kWorkClasses] = idle_first;
    ws.share_info[k] = busy[k];
    ws.share_info[kXcdShares + k] = first;
    if (k == 0) ws.counters[2] = kXcdShares * widest;  // the tile pass's workgroups
  }
}

// Pass 3, one thread per tile: its place in the order.
__global__ __launch_bounds__(256) void raster_tile_place(Workspace ws) {
  __shared__ uint32_t hist[kXcdShares * kWorkClasses];
  __shared__ uint32_t base[kXcdShares * kWorkClasses];
  for (int i = threadIdx.x; i < kXcdShares * kWorkClasses; i += blockDim.x) hist[i] = 0u;
  __syncthreads();
  const int64_t tile = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int slot = 0;
  if (tile < ws.tiles) {
    slot = xcd_share(tile, ws.tiles) * kWorkClasses + ws.tile_class[tile];
    atomicAdd(hist + slot, 1u);
  }
  __syncthreads();
  constexpr int kClassesPerThread = kXcdShares * kWorkClasses / 256;
  uint32_t reserved[kClassesPerThread];
#pragma unroll
  for (int k = 0; k < kClassesPerThread; ++k) {
    const int i = threadIdx.x + k * 256;
    reserved[k] = hist[i] ? atomicAdd(ws.class_cursor + i, hist[i]) : 0u;
  }
#pragma unroll
  for (int k = 0; k < kClassesPerThread; ++k) {
    const int i = threadIdx.x + k * 256;
    base[i] = reserved[k];
    hist[i] = 0u;
  }
  __syncthreads();
  if (tile < ws.tiles) ws.tile_order[base[slot] + atomicAdd(hist + slot, 1u)] = (uint32_t)tile;
}

// One workgroup per tile: the tile's keys stay in LDS while it walks the tile's binned
// triangles near to far (its depth-slab lists are one range of the entry array), kChunk at a
// time. Each chunk is staged in LDS together with, per row of the tile, the columns its pixel
// centres may cover (row_bounds(); the whole row of the box for a triangle without spans). The
// pixels of all those row spans form one list of work items, which the 256 threads walk in
// steps of 256, so every lane has a pixel to test whatever the span lengths. The list is mapped
// kWindow items at a time: each triangle writes (its first item, itself) at its first item of
// the window, a max-scan over the window carries that to the triangle's other items, and an
// item finds its pixel by a binary search over its triangle's spans. Hits merge into the keys
// in LDS (64-bit min). Before each chunk the tile's farthest key
// bounds what can still win: triangles entirely behind it are skipped, and so are single pixels
// that already hold a nearer key. The improved keys are stored once at the end.
template <bool kLoop>
__device__ __forceinline__ void tile_pass(const DrRasterGeometry& g, const uint64_t* prev,
                                          uint64_t* keys, const Workspace& ws,
                                          const uint2* entries, uint32_t capacity) {
  // Per staged triangle: the three vertices, (reach_x, reach_y) and its row of tri.
  __shared__ float4 s_tri[kChunk][3];
  __shared__ float2 s_reach[kChunk];
  __shared__ uint32_t s_row[kChunk];
  // Per staged triangle, its row spans that hold work items, in row order: items before the
  // span << 8 | first column << 4 | row (a triangle has at most 256 items in a tile, so the
  // count before a span fits 8 bits); and how many there are.
  __shared__ uint16_t s_span[kChunk][kTile];
  __shared__ uint8_t s_spans[kChunk];
  // Work item -> (first item of its triangle in the window) << 20 | triangle << 12 |
  // (the triangle's first item - the window's + 2048).
  __shared__ uint4 s_map[kWindow / 4];
  __shared__ int s_wave_sum[256 / DR_WAVE];
  __shared__ uint32_t s_wave_max[256 / DR_WAVE];
  __shared__ unsigned long long s_key[kTile * kTile];
  __shared__ float s_px[kTile], s_py[kTile];
  __shared__ uint64_t s_far[256 / DR_WAVE];
  __shared__ float s_row_far[kTile];  // the depth of the farthest key of each tile row (NaN: empty)
  __shared__ float s_bound[kChunk];  // lower bound of each staged triangle's depth
  __shared__ float s_floor[DR_WAVE];  // per depth slab: a lower bound of its triangles' bounds

  // Workgroups are dispatched round-robin over the 8 XCDs: XCD k runs the busy tiles of share
  // k (for a batch of 8 images, one image), so the records that neighbouring tiles share stay in
  // one L2, heaviest first. The grid is a multiple of 8 and workgroup b takes slot b / 8 of its
  // share; with kLoop also slots b / 8 + grid / 8, b / 8 + 2 grid / 8, ..., so that a grid
  // sized before the shares were known still covers every tile. (The loop costs registers, so
  // it is compiled only for that.)
  const int share = (int)(blockIdx.x % kXcdShares);
  // Lists that did not fit the entry buffer were not binned: nothing to read (the overflow
  // pass rasterizes the binned triangles instead).
  if (ws.counters[1] > capacity) return;  // uniform over the grid
  const uint32_t busy = ws.share_info[share];
  const uint32_t stride = gridDim.x / kXcdShares;
  for (uint32_t slot = blockIdx.x / kXcdShares; slot < busy; slot += stride) {
  const uint32_t tile = ws.tile_order[ws.share_info[kXcdShares + share] + slot];
  const uint32_t begin = ws.list_offsets[(size_t)tile * ws.slabs];
  const uint32_t end = ws.list_offsets[(size_t)(tile + 1) * ws.slabs];
  if (begin == end) {  // uniform over the workgroup
    if (!kLoop) break;
    continue;
  }

  // This thread's entry of the next chunk, read ahead: (record, depth bound).
  uint2 next = begin + threadIdx.x < end ? entries[begin + threadIdx.x] : make_uint2(0u, 0u);

  const int per_image = ws.tiles_x * ws.tiles_y;
  const int b = (int)(tile / per_image);
  const int tile_in_image = (int)(tile - (uint32_t)b * per_image);
  const int tile_x0 = (tile_in_image % ws.tiles_x) * kTile;
  const int tile_y0 = (tile_in_image / ws.tiles_x) * kTile;

  // This thread's pixel of the tile and its key so far (from the small-triangle pass).
  const int x = tile_x0 + (threadIdx.x % kTile), y = tile_y0 + (threadIdx.x / kTile);
  const bool inside = x < g.width && y < g.height;
  const int64_t tile_pixel0 = ((int64_t)b * g.height + tile_y0) * g.width + tile_x0;
  s_key[threadIdx.x] =
      inside ? keys[tile_pixel0 + (int64_t)(threadIdx.x / kTile) * g.width + threadIdx.x % kTile]
             : kEmptyKey;
  if (threadIdx.x < kTile && tile_x0 + (int)threadIdx.x < g.width)
    s_px[threadIdx.x] = ws.px[tile_x0 + threadIdx.x];
  if (threadIdx.x >= 32 && threadIdx.x < 32 + kTile && tile_y0 + (int)threadIdx.x - 32 < g.height)
    s_py[threadIdx.x - 32] = ws.py[tile_y0 + threadIdx.x - 32];
  const int lane = lane_id();
  const int wave = threadIdx.x / DR_WAVE;

  // The depth of the tile's farthest key when the previous chunk began (+inf while a pixel is
  // empty). Keys only get nearer, so an entry whose bound lies beyond it lies beyond the
  // farthest key of its own chunk too: it is dropped before its record is read.
  float stale_far = __int_as_float(0x7f800000);
  // s_floor[s] (1 <= s < slabs) is the floor of slab s's depth bounds, rounded down to float:
  // once the tile's farthest key lies before it, slab s and every farther one are behind every
  // key of the tile, and the walk ends at the slab's first entry. (The previous tile's last
  // chunk ended with a barrier, so the table is free.)
  const bool by_slab = ws.slabs > 1 && ws.slabs <= DR_WAVE;
  if (by_slab && threadIdx.x >= 1 && (int)threadIdx.x < ws.slabs) {
    const uint2 span = reinterpret_cast<const uint2*>(ws.depth_range)[ws.depth_ranges > 1 ? b : 0];
    s_floor[threadIdx.x] = __double2float_rd(slab_floor(span, threadIdx.x, ws.slabs));
  }
  uint32_t stop = end;
  for (uint32_t at = begin; at < stop; at += kChunk) {
    const uint32_t end = stop;
    const int n = (int)min(end - at, (uint32_t)kChunk);
    // A lower bound of the entry's triangle's depth at any pixel it covers.
    const float bound = __uint_as_float(next.y);
    const bool staged = (int)threadIdx.x < n && !(bound > stale_far);
    Tri T = {};
    uint32_t tri_row = 0u;
    if (staged) {
      const float4* rec = ws.records + (size_t)next.x * kRecord;
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const float4 v = rec[k];
        T.x[k] = v.x;
        T.y[k] = v.y;
        T.z[k] = v.z;
        T.w[k] = v.w;
      }
      tri_row = __float_as_uint(rec[3].y);  // masked where it is stored, not waited for here
    }
    if (at + kChunk + threadIdx.x < end) next = entries[at + kChunk + threadIdx.x];

    // The farthest key of the tile so far (pixels outside the image count as nearest). A
    // triangle whose depth bound lies beyond it (depth_lower_bound: the nearest vertex depth
    // less the rounding of the depth) cannot win any pixel of the tile and is skipped; the same
    // bound skips single pixels that already hold a nearer key. Equal depths are never skipped.
    __syncthreads();  // the previous chunk's merges (and the set-up above) are done
    const uint64_t own_key = inside ? s_key[threadIdx.x] : 0ull;
    const uint64_t row_far = row_max_u64(own_key);  // a wave holds four rows of the tile
    if ((lane & (kTile - 1)) == kTile - 1) s_row_far[threadIdx.x / kTile] = key_depth(row_far);
    uint64_t far_key = wave_max_u64(own_key);
    if (lane == 0) s_far[wave] = far_key;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 256 / DR_WAVE; ++w) far_key = s_far[w] > far_key ? s_far[w] : far_key;
    const bool cull = far_key != kEmptyKey;
    const float far_depth = key_depth(far_key);
    // (Uniform over the workgroup: kept in scalar registers.)
    stale_far = __uint_as_float(__builtin_amdgcn_readfirstlane(
        __float_as_uint(cull ? far_depth : __int_as_float(0x7f800000))));
    if (cull && by_slab) {
      const uint64_t behind_slabs =
          __ballot(lane >= 1 && lane < ws.slabs && s_floor[lane] > far_depth);  // uniform
      if (behind_slabs != 0) {
        const int first = __ffsll((unsigned long long)behind_slabs) - 1;
        stop = __builtin_amdgcn_readfirstlane(
            min(stop, ws.list_offsets[(size_t)tile * ws.slabs + first]));
      }
    }

    int items = 0;
    // A staged triangle behind the farthest key as it is now makes no items: nothing of it is
    // kept.
    if (staged && !(cull && bound > far_depth)) {
#pragma unroll
      for (int k = 0; k < 3; ++k)
        s_tri[threadIdx.x][k] = make_float4(T.x[k], T.y[k], T.z[k], T.w[k]);
      T.reach_x = reach(T.x, T.w);
      T.reach_y = reach(T.y, T.w);
      int x_lo, x_hi, y_lo, y_hi;
      candidate_box(g, T, x_lo, x_hi, y_lo, y_hi);
      const int bx0 = max(x_lo - tile_x0, 0), bx1 = min(x_hi - tile_x0, kTile - 1);
      const int by0 = max(y_lo - tile_y0, 0), by1 = min(y_hi - tile_y0, kTile - 1);
      s_bound[threadIdx.x] = bound;
      s_reach[threadIdx.x] = make_float2(T.reach_x, T.reach_y);
      asm volatile("" : "+v"(tri_row));  // keeps the mask (and the wait for the load) here
      s_row[threadIdx.x] = tri_row & 0xffffffu;
      if (bx0 <= bx1 && by0 <= by1) {
        // (A triangle without spans gets bounds that constrain nothing: its box's whole rows.)
        RowSpans se;
        // (The tile's column origin as an opaque scalar: hoisted out of the chunk loop as a
        // double, it would be spilled at the 96-VGPR budget.)
        int x0 = tile_x0;
        asm volatile("" : "+s"(x0));
        span_setup(T.x, T.y, T.w, T.reach_x, T.reach_y, g.width, x0, se);
        const float fx0 = (float)bx0, fx1 = (float)bx1;
        uint16_t* out = s_span[threadIdx.x];
        uint32_t code = (uint32_t)by0;  // items so far << 8 | row
        for (int r = by0; r <= by1; ++r, ++code) {
          float lo = fx0, hi = fx1;
          row_bounds(se, s_py[r], lo, hi);
          // Every pixel of the row already holds a key nearer than the triangle can reach (an
          // empty key reads as NaN and never compares greater).
          if (bound > s_row_far[r]) hi = -__int_as_float(0x7f800000);
          if (lo <= hi) {  // then 0 <= lo <= hi <= 15, integers
            *out++ = (uint16_t)(code | (uint32_t)lo << 4);
            code += ((uint32_t)(hi - lo) + 1u) << 8;
          }
        }
        s_spans[threadIdx.x] = (uint8_t)(out - s_span[threadIdx.x]);
        items = (int)(code >> 8);
      }
    }
    // Exclusive prefix of the item counts over the workgroup.
    const int incl = (int)wave_inclusive_sum((uint32_t)items);
    if (lane == DR_WAVE - 1) s_wave_sum[wave] = incl;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < 256 / DR_WAVE; ++w) {
      const int v = s_wave_sum[w];
      before += w < wave ? v : 0;
      total += v;
    }
    const int tri_first = before + incl - items;

    for (int base = 0; base < total; base += kWindow) {
      s_map[threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);
      __syncthreads();
      // Mark the first item in the window of each triangle that reaches into it. Its first
      // item overall is within 256 items of the window (-256 < tri_first - base < kWindow).
      if (items > 0 && tri_first < base + kWindow && tri_first + items > base) {
        const int pos = max(tri_first, base) - base;
        reinterpret_cast<uint32_t*>(s_map)[pos] =
            (uint32_t)pos << 20 | threadIdx.x << 12 | (uint32_t)(tri_first - base + 2048);
      }
      __syncthreads();
      // Inclusive max-scan of the window (each mark exceeds every mark before it).
      uint4 m = s_map[threadIdx.x];
      m.y = max(m.y, m.x);
      m.z = max(m.z, m.y);
      m.w = max(m.w, m.z);
      const uint32_t run = wave_inclusive_max(m.w);
      if (lane == DR_WAVE - 1) s_wave_max[wave] = run;
      uint32_t carry = wave_shr1(run);
      __syncthreads();
#pragma unroll
      for (int w = 0; w < 256 / DR_WAVE; ++w)
        carry = w < wave ? max(carry, s_wave_max[w]) : carry;
      m.x = max(m.x, carry);
      m.y = max(m.y, carry);
      m.z = max(m.z, carry);
      m.w = max(m.w, carry);
      s_map[threadIdx.x] = m;
      __syncthreads();

      const int count = min(total - base, kWindow);
      for (int i = threadIdx.x; i < count; i += 256) {
        const uint32_t v = reinterpret_cast<const uint32_t*>(s_map)[i];
        const int j = (int)((v >> 12) & 0xffu);
        // The item's place among its triangle's items, then its span: the last one that
        // starts at or before it (binary search over the triangle's at most 16 spans).
        const int li = i + 2048 - (int)(v & 0xfffu);
        const int held = s_spans[j];
        uint32_t e = s_span[j][0];
        int at_span = 0;
#pragma unroll
        for (int step = kTile / 2; step >= 1; step >>= 1) {
          if (at_span + step < held) {
            const uint32_t c = s_span[j][at_span + step];
            if ((int)(c >> 8) <= li) {
              at_span += step;
              e = c;
            }
          }
        }
        const int p = (int)(e & 15u) * kTile + (int)((e >> 4) & 15u) + li - (int)(e >> 8);
        // Early depth test: the pixel already holds a nearer key (NaN for an empty one).
        if (s_bound[j] > key_depth(s_key[p])) continue;
        const float4 v0 = s_tri[j][0], v1 = s_tri[j][1], v2 = s_tri[j][2];
        const float2 rc = s_reach[j];
        const float X[3] = {v0.x, v1.x, v2.x}, Y[3] = {v0.y, v1.y, v2.y};
        const float Z[3] = {v0.z, v1.z, v2.z}, Wv[3] = {v0.w, v1.w, v2.w};
        const int lx = p & (kTile - 1), ly = p / kTile;
        float depth;
        if (covers(X, Y, Z, Wv, rc.x, rc.y, s_px[lx], s_py[ly], depth)) {
          const uint64_t key = depth_key(depth, s_row[j]);
          // Peeling: only keys after the previous layer's (read where a candidate needs it).
          if (prev == nullptr || key > prev[tile_pixel0 + (int64_t)ly * g.width + lx])
            atomicMin(s_key + p, (unsigned long long)key);
        }
      }
      __syncthreads();
    }
  }
  __syncthreads();
  // This workgroup alone writes the tile's keys.
  if (inside)
    keys[tile_pixel0 + (int64_t)(threadIdx.x / kTile) * g.width + threadIdx.x % kTile] =
        s_key[threadIdx.x];
  if (!kLoop) break;
  __syncthreads();  // the next tile's set-up reuses the LDS
  }
}

// The tile pass's two kernels. Without the loop over tiles it fits five waves per SIMD, as many
// as its LDS allows, when the compiler keeps it to 96 VGPRs (it needs a few more otherwise, and
// four waves are ~12 % slower); the looping kernel would spill at that budget and keeps its own.
template <bool kLoop>
__global__ void raster_tile_kernel(DrRasterGeometry g, const uint64_t* prev, uint64_t* keys,
                                   Workspace ws, const uint2* entries, uint32_t capacity);

template <>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5))) void
raster_tile_kernel<false>(DrRasterGeometry g, const uint64_t* prev, uint64_t* keys, Workspace ws,
                          const uint2* entries, uint32_t capacity) {
  tile_pass<false>(g, prev, keys, ws, entries, capacity);
}

template <>
__global__ __launch_bounds__(256) void raster_tile_kernel<true>(DrRasterGeometry g,
                                                                const uint64_t* prev,
                                                                uint64_t* keys, Workspace ws,
                                                                const uint2* entries,
                                                                uint32_t capacity) {
  tile_pass<true>(g, prev, keys, ws, entries, capacity);
}

// Visibility of the binned triangles when their tile lists did not fit the entry buffer (the
// bin and tile passes then returned without work): each workgroup takes the records of every
// gridDim.x-th setup workgroup, one triangle at a time, and its 256 threads test the pixel centres of the
// triangle's box, merging hits into the keys with 64-bit atomic min. The result is the same as
// the tile pass's; the work is not (no spans, no depth culling, one atomic per hit).
__global__ __launch_bounds__(256) void raster_overflow_kernel(DrRasterGeometry g,
                                                              const uint64_t* prev,
                                                              uint64_t* keys, Workspace ws,
                                                              uint32_t capacity) {
  if (ws.counters[1] <= capacity) return;  // uniform over the grid: the lists fitted
  for (int block = blockIdx.x; block < ws.record_blocks; block += gridDim.x) {
  const uint32_t count = ws.block_records[block];
  for (uint32_t j = 0; j < count; ++j) {
    const float4* rec = ws.records + ((size_t)block * 256 + j) * kRecord;
    Tri T;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const float4 v = rec[k];
      T.x[k] = v.x;
      T.y[k] = v.y;
      T.z[k] = v.z;
      T.w[k] = v.w;
    }
    const float4 meta = rec[3];
    const int b = __float_as_int(meta.x);
    const uint32_t row = __float_as_uint(meta.y) & 0xffffffu;
    T.reach_x = reach(T.x, T.w);
    T.reach_y = reach(T.y, T.w);
    int x_lo, x_hi, y_lo, y_hi;
    candidate_box(g, T, x_lo, x_hi, y_lo, y_hi);
    if (x_lo > x_hi || y_lo > y_hi) continue;  // uniform: every thread read the same record
    const int bw = x_hi - x_lo + 1;
    const int64_t area = (int64_t)bw * (y_hi - y_lo + 1);
    for (int64_t p = threadIdx.x; p < area; p += blockDim.x) {
      const int y = y_lo + (int)(p / bw), x = x_lo + (int)(p % bw);
      float depth;
      if (covers(T.x, T.y, T.z, T.w, T.reach_x, T.reach_y, ws.px[x], ws.py[y], depth)) {
        const int64_t pixel = ((int64_t)b * g.height + y) * g.width + x;
        merge_key(keys, prev, pixel, depth_key(depth, row));
      }
    }
  }
  }
}

// ---- resolve ----------------------------------------------------------------------------

// Per-pixel quantities of the visible triangle, in the reference's operation order
// (reference.py:84-111 with _edge_functions / _edge_derivatives, reference.py:274-290).
struct Resolved {
  float a[3], c[3], e[3], area, b[3], num, den, depth, dex[3], dey[3], sum_dx, sum_dy;
  float db_dx[3], db_dy[3];
  float inv_area, inv_den;  // 1 / area and 1 / den (the backward pass's quotients)
};

// With kExact (the forward pass) every quotient is the reference's correctly rounded division;
// otherwise (the backward pass, whose gradients are compared to 1e-4) the quotients by area and
// depth denominator multiply by their reciprocals, within 2 ulp.
template <bool kExact = true>
__device__ __forceinline__ void resolve_pixel(const Tri& T, float px, float py, Resolved& R) {
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    R.a[k] = T.x[k] - px * T.w[k];
    R.c[k] = T.y[k] - py * T.w[k];
  }
  R.e[0] = R.a[1] * R.c[2] - R.a[2] * R.c[1];
  R.e[1] = R.a[2] * R.c[0] - R.a[0] * R.c[2];
  R.e[2] = R.a[0] * R.c[1] - R.a[1] * R.c[0];
  R.area = R.e[0] + R.e[1] + R.e[2];
  R.inv_area = 1.0f / R.area;
#pragma unroll
  for (int k = 0; k < 3; ++k) R.b[k] = kExact ? R.e[k] / R.area : R.e[k] * R.inv_area;
  R.num = R.b[0] * T.z[0] + R.b[1] * T.z[1] + R.b[2] * T.z[2];
  R.den = R.b[0] * T.w[0] + R.b[1] * T.w[1] + R.b[2] * T.w[2];
  R.inv_den = 1.0f / R.den;
  R.depth = kExact ? R.num / R.den : R.num * R.inv_den;
  // d e / d px = c x w and d e / d py = w x a.
  R.dex[0] = R.c[1] * T.w[2] - R.c[2] * T.w[1];
  R.dex[1] = R.c[2] * T.w[0] - R.c[0] * T.w[2];
  R.dex[2] = R.c[0] * T.w[1] - R.c[1] * T.w[0];
  R.dey[0] = T.w[1] * R.a[2] - T.w[2] * R.a[1];
  R.dey[1] = T.w[2] * R.a[0] - T.w[0] * R.a[2];
  R.dey[2] = T.w[0] * R.a[1] - T.w[1] * R.a[0];
  R.sum_dx = R.dex[0] + R.dex[1] + R.dex[2];
  R.sum_dy = R.dey[0] + R.dey[1] + R.dey[2];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float nx = R.dex[k] - R.b[k] * R.sum_dx, ny = R.dey[k] - R.b[k] * R.sum_dy;
    R.db_dx[k] = kExact ? nx / R.area : nx * R.inv_area;
    R.db_dy[k] = kExact ? ny / R.area : ny * R.inv_area;
  }
}

// Four pixels per thread, in rows or tiles (pixel_slots); their loads go out level by level
// (keys, index rows, vertices) so that a thread waits once per level for all four.
template <bool TILES>
__global__ __launch_bounds__(256) void resolve_fwd_kernel(DrRasterGeometry g,
                                                          const uint64_t* keys, float* rast,
                                                          float* rast_db, float scale_x,
                                                          float scale_y) {
  constexpr int kPixels = 4;
  const PixelSlots<kPixels> s = pixel_slots<kPixels, TILES>(g.batch, g.height, g.width);
  const int64_t* pixel = s.pixel;
  uint64_t key[kPixels];
#pragma unroll
  for (int j = 0; j < kPixels; ++j) key[j] = s.inside[j] ? keys[pixel[j]] : kEmptyKey;
  // The pixels' index rows, then their vertices, each level's loads issued together: in a wave
  // with any covered pixel every lane reads (triangle 0 of image 0 for an empty one), with no
  // branch between the pixels.
  int v[kPixels][3];
  int b[kPixels];
  bool covered = false;
#pragma unroll
  for (int j = 0; j < kPixels; ++j) {
    const bool hit = key[j] != kEmptyKey;
    covered = covered || hit;
    b[j] = hit ? s.b[j] : 0;
    v[j][0] = v[j][1] = v[j][2] = 0;
  }
  Tri T[kPixels];
  if (__any(covered)) {  // then tri has rows
#pragma unroll
    for (int j = 0; j < kPixels; ++j) {
      const int32_t* row = g.tri + 3 * (int64_t)(key[j] != kEmptyKey ? (uint32_t)key[j] : 0u);
      v[j][0] = row[0];
      v[j][1] = row[1];
      v[j][2] = row[2];
    }
#pragma unroll
    for (int j = 0; j < kPixels; ++j) load_vertices(g, b[j], v[j], T[j]);
  }
#pragma unroll
  for (int j = 0; j < kPixels; ++j) {
    if (!s.inside[j]) continue;
    if (key[j] == kEmptyKey) {
      store4(rast + 4 * pixel[j], make_float4(0.f, 0.f, 0.f, 0.f));
      if (rast_db) store4(rast_db + 4 * pixel[j], make_float4(0.f, 0.f, 0.f, 0.f));
      continue;
    }
    const int t = (int)(uint32_t)key[j];
    Resolved R;
    resolve_pixel(T[j], pixel_centre(s.x[j], g.width), pixel_centre(s.y[j], g.height), R);
    store4(rast + 4 * pixel[j], make_float4(R.b[0], R.b[1], R.depth, (float)(t + 1)));
    if (rast_db)
      store4(rast_db + 4 * pixel[j], make_float4(R.db_dx[0] * scale_x, R.db_dy[0] * scale_y,
                                                 R.db_dx[1] * scale_x, R.db_dy[1] * scale_y));
  }
}

__device__ __forceinline__ void cross3(const float* u, const float* v, float* out) {
  out[0] = u[1] * v[2] - u[2] * v[1];
  out[1] = u[2] * v[0] - u[0] * v[2];
  out[2] = u[0] * v[1] - u[1] * v[0];
}

// Reverse mode of resolve_pixel for the gradient of (b0, b1, depth) and, optionally, rast_db.
// For u x v with upstream G: grad u = v x G, grad v = G x u. Vertex gradients (x, y, z, w)
// gather in the workgroup's scatter table, keyed by vertex row of pos, before the atomics.
__global__ __launch_bounds__(256) void resolve_bwd_kernel(
    DrRasterGeometry g, const uint64_t* keys, const float* grad_rast, const float* grad_db,
    float* grad_pos, float scale_x, float scale_y) {
  using Table = RowTable<512, 4>;
  __shared__ Table table;
  table.init();
  const TilePixel tp = tile_pixel(g.batch, g.height, g.width);
  const int64_t pixel = tp.pixel;
  float vals[3][4];
  uint32_t rows[3] = {Table::kEmpty, Table::kEmpty, Table::kEmpty};
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int c = 0; c < 4; ++c) vals[k][c] = 0.0f;
  const uint64_t key = tp.inside ? keys[pixel] : kEmptyKey;
  if (key != kEmptyKey) {
    const int t = (int)(uint32_t)key;
    const int b = tp.b;
    Tri T;
    int v[3];
    load_tri(g, b, t, T, v);
    const float px = pixel_centre(tp.x, g.width), py = pixel_centre(tp.y, g.height);
    Resolved R;
    resolve_pixel<false>(T, px, py, R);
    const float4 gr = load4(grad_rast + 4 * pixel);
    float gb[3] = {gr.x, gr.y, 0.0f};
    float gw[3] = {0.f, 0.f, 0.f}, gz[3];
    // depth = num / den
    const float g_num = gr.z * R.inv_den;
    const float g_den = -gr.z * R.depth * R.inv_den;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      gb[k] += g_num * T.z[k] + g_den * T.w[k];
      gz[k] = g_num * R.b[k];
      gw[k] = g_den * R.b[k];
    }
    float g_area = 0.0f;
    float g_dex[3] = {0.f, 0.f, 0.f}, g_dey[3] = {0.f, 0.f, 0.f};
    if (grad_db != nullptr) {
      const float4 gd = load4(grad_db + 4 * pixel);
      const float gx[3] = {gd.x * scale_x, gd.z * scale_x, 0.0f};
      const float gy[3] = {gd.y * scale_y, gd.w * scale_y, 0.0f};
      // db_dx_k = (dex_k - b_k Sx) / area, Sx = sum dex.
      float dot_x = 0.f, dot_y = 0.f;
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        dot_x += gx[k] * R.b[k];
        dot_y += gy[k] * R.b[k];
        gb[k] -= (gx[k] * R.sum_dx + gy[k] * R.sum_dy) * R.inv_area;
        g_area -= (gx[k] * R.db_dx[k] + gy[k] * R.db_dy[k]) * R.inv_area;
      }
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        g_dex[k] = (gx[k] - dot_x) * R.inv_area;
        g_dey[k] = (gy[k] - dot_y) * R.inv_area;
      }
    }
    // b_k = e_k / area
    float dot_b = 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) dot_b += gb[k] * R.b[k];
    g_area -= dot_b * R.inv_area;
    float ge[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) ge[k] = gb[k] * R.inv_area + g_area;
    // e = a x c; dex = c x w; dey = w x a.
    float ga[3], gc[3], tmp[3];
    cross3(R.c, ge, ga);
    cross3(ge, R.a, gc);
    cross3(T.w, g_dex, tmp);  // grad c from dex = c x w
    for (int k = 0; k < 3; ++k) gc[k] += tmp[k];
    cross3(g_dex, R.c, tmp);  // grad w from dex
    for (int k = 0; k < 3; ++k) gw[k] += tmp[k];
    cross3(R.a, g_dey, tmp);  // grad w from dey = w x a
    for (int k = 0; k < 3; ++k) gw[k] += tmp[k];
    cross3(g_dey, T.w, tmp);  // grad a from dey
    for (int k = 0; k < 3; ++k) ga[k] += tmp[k];
    // a = x - px w, c = y - py w
    const int64_t row0 = g.pos_batch_stride != 0 ? (int64_t)b * (g.pos_batch_stride / 4) : 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      vals[k][0] = ga[k];
      vals[k][1] = gc[k];
      vals[k][2] = gz[k];
      vals[k][3] = gw[k] - px * ga[k] - py * gc[k];
      rows[k] = (uint32_t)(row0 + v[k]);
    }
  }
  // Pixels of a tile row that show one triangle are summed first; each run then makes one
  // table update per vertex.
  float run[12];
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int c = 0; c < 4; ++c) run[4 * k + c] = vals[k][c];
  const bool last = row_run_sums(key != kEmptyKey ? (uint32_t)key : 0xffffffffu, run);
  const bool adds = last && key != kEmptyKey;
  const FixedPass f = table.begin(adds ? max_magnitude(run, 12) : 0.0f);
  if (adds) {
#pragma unroll
    for (int k = 0; k < 3; ++k) table.add_or_global(rows[k], run + 4 * k, 4, grad_pos, 4, f);
  }
  __syncthreads();
  table.flush(grad_pos, 4, 4, f);
}

}  // namespace
}  // namespace dr

using namespace dr;

static bool valid_geometry(const DrRasterGeometry* g) {
  if (!g || g->batch < 0 || g->num_tri < 0 || g->height <= 0 || g->width <= 0) return false;
  if ((g->batch > 0 && g->num_tri > 0) && (!g->pos || !g->tri)) return false;
  if (g->ranges && !g->range_prefix) return false;
  if (g->num_tri > (1 << 24) || g->num_instances < 0 || g->num_vertices < 0) return false;
  // Per-image vertex arrays hold pos_batch_stride / 4 vertices.
  if (g->pos_batch_stride != 0 && g->pos_batch_stride < 4 * (int64_t)g->num_vertices) return false;
  // Tile coordinates are stored in 16 bits.
  if ((g->width + 15) / 16 > 0xffff || (g->height + 15) / 16 > 0xffff) return false;
  return true;
}

extern "C" int dr_raster_workspace_size(const DrRasterGeometry* g, size_t* bytes) {
  if (!valid_geometry(g) || !bytes) return DR_ERR_ARGUMENT;
  *bytes = layout(*g, nullptr).bytes;
  return DR_OK;
}

// The tile pass's grid when the busy tiles are not known yet: 8 x the largest share of tiles
// (its workgroups beyond a share's busy tiles return at once).
static int64_t tile_grid_bound(const Workspace& ws) {
  return ws.tiles < kXcdShares ? kXcdShares
                               : kXcdShares * ((ws.tiles + kXcdShares - 1) / kXcdShares);
}

// The order passes, into ws.order (after raster_prepare has zeroed the bucket counts).
static void queue_order(const DrRasterGeometry& g, const Workspace& ws, hipStream_t s) {
  const int tri_blocks = blocks_for(g.num_tri, 256);
  order_centroids<<<tri_blocks, 256, 0, s>>>(g, ws);
  order_bounds<<<1, 256, 0, s>>>(ws, tri_blocks);
  const int bucket_blocks = blocks_for(g.num_tri, 256 * kOrderPerThread);
  order_count<<<bucket_blocks, 256, 0, s>>>(g, ws);
  order_scan<<<1, 256, 0, s>>>(ws);
  order_place<<<bucket_blocks, 256, 0, s>>>(g, ws);
}

extern "C" int dr_raster_order_size(const DrRasterGeometry* g, size_t* bytes) {
  if (!valid_geometry(g) || !bytes) return DR_ERR_ARGUMENT;
  *bytes = use_order(*g) ? sizeof(int4) * (size_t)g->num_tri : 0;
  return DR_OK;
}

extern "C" int dr_raster_order(const DrRasterGeometry* g, void* order, size_t order_bytes,
                               void* workspace, size_t workspace_bytes, void* stream) {
  size_t need = 0;
  const int status = dr_raster_order_size(g, &need);
  if (status != DR_OK || need == 0) return status;
  if (!order || order_bytes < need) return DR_ERR_CAPACITY;
  DrRasterGeometry own = *g;
  own.order = nullptr;
  Workspace ws = layout(own, (char*)workspace);
  if (!workspace || workspace_bytes < ws.bytes) return DR_ERR_CAPACITY;
  ws.order = (int4*)order;
  hipStream_t s = (hipStream_t)stream;
  // raster_prepare with no pixels: the bucket counts (and the other counts) zeroed.
  raster_prepare<<<(int)std::min<int64_t>(blocks_for(ws.lists + 1, 256), 65536), 256, 0, s>>>(
      nullptr, 0, ws, g->width, g->height);
  queue_order(own, ws, s);
  return launch_status();
}

// Queues the first part of the visibility and the copy of its counts to host_counts.
static int queue_visibility_start(const DrRasterGeometry* g, const uint64_t* prev_keys,
                                  uint64_t* keys, void* workspace, size_t workspace_bytes,
                                  uint32_t* host_counts, hipStream_t s) {
  const int64_t pixels = (int64_t)g->batch * g->height * g->width;
  if (pixels == 0) return DR_OK;
  Workspace ws = layout(*g, (char*)workspace);
  if (!workspace || workspace_bytes < ws.bytes) return DR_ERR_CAPACITY;
  // Record slots (256 per setup workgroup) and tiles are indexed with 32 bits.
  if (g->num_instances > ((int64_t)1 << 32) - 512 || ws.lists >= ((int64_t)1 << 32) - 1)
    return DR_ERR_ARGUMENT;
  const int64_t fill_items = std::max<int64_t>(pixels, ws.lists + 1);
  raster_prepare<<<(int)std::min<int64_t>(blocks_for(fill_items, 256), 65536), 256, 0, s>>>(
      keys, pixels, ws, g->width, g->height);
  if (g->num_instances > 0) {
    if (ws.ordered && g->order == nullptr) queue_order(*g, ws, s);
    if (ws.slabs > 1) {  // the depth span places binned triangles in slabs
      raster_depth_range<<<ws.depth_ranges * kRangeParts, 1024, 0, s>>>(*g, ws);
      raster_depth_range_merge<<<ws.depth_ranges, kRangeParts, 0, s>>>(ws);
    }
    raster_setup_kernel<<<blocks_for(g->num_instances, 256), 256, 0, s>>>(*g, prev_keys, keys,
                                                                          ws, small_pixels(*g));
    raster_scan_reduce<<<ws.scan_blocks, 256, 0, s>>>(ws.list_counts, ws.lists, ws.block_sums);
    raster_scan_blocks<<<1, 256, 0, s>>>(ws.block_sums, ws.scan_blocks, ws.counters);
    raster_scan_apply<<<ws.scan_blocks, 256, 0, s>>>(ws.list_counts, ws.lists, ws.block_sums,
                                                     ws.list_offsets, ws.list_cursor,
                                                     ws.chunk_offsets);
    const int tile_blocks = blocks_for(ws.tiles, 256);
    raster_tile_classes<<<tile_blocks, 256, 0, s>>>(ws);
    raster_tile_cursors<<<1, 256, 0, s>>>(ws);
    raster_tile_place<<<tile_blocks, 256, 0, s>>>(ws);
  }
  const int status = launch_status();
  if (status != DR_OK) return status;
  if (host_counts != nullptr &&
      hipMemcpyAsync(host_counts, ws.counters, 4 * sizeof(uint32_t), hipMemcpyDeviceToHost, s) !=
          hipSuccess)
    return DR_ERR_HIP;
  return DR_OK;
}

// Up to this many workgroups, a tile pass without a requested grid launches one workgroup per
// tile (the idle ones return at once, ~0.2 us per thousand) rather than the looping kernel.
constexpr int64_t kPlainTileGrid = 1 << 16;

// Launches the tile pass so that it covers every busy tile whatever `requested` is. A grid of
// at least one workgroup per tile (`requested` 0 or at least that, and then at most
// kPlainTileGrid workgroups) runs the plain kernel, one tile per workgroup. Any smaller grid
// runs the looping kernel: `requested` workgroups (0: one per tile), rounded up to a multiple
// of 8 and kept below 2^24, each taking every (grid / 8)-th busy tile of its XCD share. So a
// grid sized before the busy tiles were known, or sized wrongly by a caller, loses no tile.
static void launch_tile_pass(const DrRasterGeometry& g, const uint64_t* prev, uint64_t* keys,
                             const Workspace& ws, const uint2* entries, uint32_t capacity,
                             uint32_t requested, hipStream_t s) {
  const int64_t bound = tile_grid_bound(ws);
  const int64_t limit = ((int64_t)1 << 24) - kXcdShares;
  const bool full = requested == 0 || (int64_t)requested >= bound;
  if (full && bound <= kPlainTileGrid) {
    raster_tile_kernel<false><<<(int)bound, 256, 0, s>>>(g, prev, keys, ws, entries, capacity);
    return;
  }
  int64_t grid = full ? bound : ((int64_t)requested + kXcdShares - 1) / kXcdShares * kXcdShares;
  grid = std::min(std::min(std::max<int64_t>(grid, kXcdShares), bound), limit);
  raster_tile_kernel<true><<<(int)grid, 256, 0, s>>>(g, prev, keys, ws, entries, capacity);
}

// The overflow pass's grid: it walks the setup workgroups' records with a grid stride, so that
// it costs little when there is nothing to do.
static int overflow_grid(const Workspace& ws) { return std::min(ws.record_blocks, 2048); }

// The whole visibility, queued: the first part, then the bin and tile passes with an entry
// buffer of `capacity` entries, then the overflow pass, which rasterizes the binned triangles
// itself when the lists turned out larger than the buffer (the device decides; nothing waits
// for the host).
static int queue_visibility(const DrRasterGeometry* g, const uint64_t* prev_keys,
                            uint64_t* keys, void* workspace, size_t workspace_bytes,
                            uint2* entries, uint32_t capacity, uint32_t tile_groups,
                            uint32_t* host_counts, hipStream_t s) {
  const int status = queue_visibility_start(g, prev_keys, keys, workspace, workspace_bytes,
                                            host_counts, s);
  if (status != DR_OK) return status;
  if ((int64_t)g->batch * g->height * g->width == 0 || g->num_instances == 0) return DR_OK;
  Workspace ws = layout(*g, (char*)workspace);
  if (capacity > 0) {
    raster_bin_kernel<<<bin_grid(ws), 256, 0, s>>>(ws, entries, capacity);
    launch_tile_pass(*g, prev_keys, keys, ws, entries, capacity, tile_groups, s);
  }
  raster_overflow_kernel<<<overflow_grid(ws), 256, 0, s>>>(*g, prev_keys, keys, ws, capacity);
  return launch_status();
}

extern "C" int dr_raster_visibility_overflow(const DrRasterGeometry* g,
                                             const uint64_t* prev_keys, uint64_t* keys,
                                             void* workspace, size_t workspace_bytes,
                                             uint32_t entry_capacity, void* stream) {
  if (!valid_geometry(g)) return DR_ERR_ARGUMENT;
  if ((int64_t)g->batch * g->height * g->width == 0 || g->num_instances == 0) return DR_OK;
  if (!keys) return DR_ERR_ARGUMENT;
  Workspace ws = layout(*g, (char*)workspace);
  if (!workspace || workspace_bytes < ws.bytes) return DR_ERR_CAPACITY;
  raster_overflow_kernel<<<overflow_grid(ws), 256, 0, (hipStream_t)stream>>>(
      *g, prev_keys, keys, ws, entry_capacity);
  return launch_status();
}

// ---- the allocation-free visibility ---------------------------------------------------------
//
// One static device buffer holds the workspace and the tile entries of
// dr_raster_visibility_static, for callers that cannot allocate. Each GPU that runs it holds its
// own copy for the life of the process. Host code never passes the array's name to a kernel (on
// the host it is only a stand-in for the symbol): its device address, per device, comes from
// hipGetSymbolAddress on the first call with that device current.
constexpr size_t kScratchBytes = (size_t)64 << 20;
constexpr size_t kScratchMinEntries = 4096;  // the workspace leaves room for at least these
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex scratch_mutex;
static void* scratch_address[kMaxDevices] = {};

static int scratch_of_current_device(void** address) {
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess) return DR_ERR_HIP;
  if (device < 0 || device >= kMaxDevices) return DR_ERR_ARGUMENT;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_address[device] == nullptr) {
    void* found = nullptr;
    if (hipGetSymbolAddress(&found, HIP_SYMBOL(scratch)) != hipSuccess || found == nullptr)
      return DR_ERR_HIP;
    scratch_address[device] = found;
  }
  *address = scratch_address[device];
  return DR_OK;
}

extern "C" int dr_raster_visibility_static(const DrRasterGeometry* g,
                                           const uint64_t* prev_keys, uint64_t* keys,
                                           void* stream) {
  if (!valid_geometry(g)) return DR_ERR_ARGUMENT;
  const size_t workspace_bytes = layout(*g, nullptr).bytes;  // a multiple of 256
  if (workspace_bytes + kScratchMinEntries * sizeof(uint2) > kScratchBytes)
    return DR_ERR_SCRATCH;
  void* base = nullptr;
  const int status = scratch_of_current_device(&base);
  if (status != DR_OK) return status;
  uint2* entries = (uint2*)((char*)base + workspace_bytes);
  const size_t capacity =
      std::min<size_t>((kScratchBytes - workspace_bytes) / sizeof(uint2), 0xffffffffu);
  // Everything the passes read is set up by raster_prepare at the start of the call (keys,
  // list counts, counters), so what the previous call left in the buffer does not matter.
  return queue_visibility(g, prev_keys, keys, base, workspace_bytes, entries,
                          (uint32_t)capacity, 0, nullptr, (hipStream_t)stream);
}

extern "C" int dr_raster_visibility(const DrRasterGeometry* g, const uint64_t* prev_keys,
                                    uint64_t* keys, void* workspace, size_t workspace_bytes,
                                    void* entries, uint32_t entry_capacity,
                                    uint32_t tile_groups, uint32_t* host_counts, void* stream) {
  if (!valid_geometry(g) || (entry_capacity > 0 && !entries)) return DR_ERR_ARGUMENT;
  if (host_counts) host_counts[0] = host_counts[1] = host_counts[2] = host_counts[3] = 0;
  return queue_visibility(g, prev_keys, keys, workspace, workspace_bytes, (uint2*)entries,
                          entry_capacity, tile_groups, host_counts, (hipStream_t)stream);
}

extern "C" int dr_raster_visibility_start(const DrRasterGeometry* g, const uint64_t* prev_keys,
                                          uint64_t* keys, void* workspace,
                                          size_t workspace_bytes, uint32_t* host_counts,
                                          void* stream) {
  if (!valid_geometry(g)) return DR_ERR_ARGUMENT;
  if (host_counts) host_counts[0] = host_counts[1] = host_counts[2] = host_counts[3] = 0;
  return queue_visibility_start(g, prev_keys, keys, workspace, workspace_bytes, host_counts,
                                (hipStream_t)stream);
}

extern "C" int dr_raster_visibility_begin(const DrRasterGeometry* g, const uint64_t* prev_keys,
                                          uint64_t* keys, void* workspace,
                                          size_t workspace_bytes, uint32_t counts[4],
                                          void* stream) {
  if (!valid_geometry(g) || !counts) return DR_ERR_ARGUMENT;
  counts[0] = counts[1] = counts[2] = counts[3] = 0;
  // The counts come back through pinned host memory (one small buffer per host thread, kept
  // for the life of the process): a copy into pageable memory is staged and slower to return.
  static thread_local uint32_t* host = nullptr;
  if (host == nullptr && hipHostMalloc((void**)&host, 4 * sizeof(uint32_t)) != hipSuccess) {
    host = nullptr;
    return DR_ERR_HIP;
  }
  host[0] = host[1] = host[2] = host[3] = 0;
  hipStream_t s = (hipStream_t)stream;
  const int status = queue_visibility_start(g, prev_keys, keys, workspace, workspace_bytes,
                                            host, s);
  if (status != DR_OK) return status;
  if (hipStreamSynchronize(s) != hipSuccess) return DR_ERR_HIP;
  for (int i = 0; i < 4; ++i) counts[i] = host[i];
  return DR_OK;
}

extern "C" int dr_raster_visibility_bin(const DrRasterGeometry* g, void* workspace,
                                        size_t workspace_bytes, void* entries,
                                        const uint32_t counts[4], void* stream) {
  if (!valid_geometry(g) || !counts) return DR_ERR_ARGUMENT;
  // Nothing was binned without pixels or triangles (and the workspace was not prepared).
  if (counts[1] == 0 || g->batch == 0 || g->num_instances == 0) return DR_OK;
  if (!entries) return DR_ERR_ARGUMENT;
  Workspace ws = layout(*g, (char*)workspace);
  if (!workspace || workspace_bytes < ws.bytes) return DR_ERR_CAPACITY;
  hipStream_t s = (hipStream_t)stream;
  raster_bin_kernel<<<bin_grid(ws), 256, 0, s>>>(ws, (uint2*)entries, counts[1]);
  return launch_status();
}

extern "C" int dr_raster_visibility_tiles(const DrRasterGeometry* g, const uint64_t* prev_keys,
                                          uint64_t* keys, void* workspace,
                                          size_t workspace_bytes, const void* entries,
                                          const uint32_t counts[4], void* stream) {
  if (!valid_geometry(g) || !counts) return DR_ERR_ARGUMENT;
  if (counts[1] == 0 || g->batch == 0 || g->num_instances == 0) return DR_OK;
  if (!entries || !keys) return DR_ERR_ARGUMENT;
  Workspace ws = layout(*g, (char*)workspace);
  if (!workspace || workspace_bytes < ws.bytes) return DR_ERR_CAPACITY;
  launch_tile_pass(*g, prev_keys, keys, ws, (const uint2*)entries, counts[1], counts[2],
                   (hipStream_t)stream);
  return launch_status();
}

static void resolve_scales(const DrRasterGeometry* g, float& sx, float& sy) {
  // The reference multiplies by the Python float 2 / size, which PyTorch rounds to float32.
  sx = (float)(2.0 / (double)g->width);
  sy = (float)(2.0 / (double)g->height);
}

extern "C" int dr_resolve_forward(const DrRasterGeometry* g, const uint64_t* keys, float* rast,
                                  float* rast_db, void* stream) {
  if (!valid_geometry(g) || !rast) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)g->batch * g->height * g->width;
  if (pixels == 0) return DR_OK;
  float sx, sy;
  resolve_scales(g, sx, sy);
  // The index rows and vertices one image's pixels may gather: a range item draws its own
  // triangles only; a closed mesh has about half a vertex per triangle.
  const int64_t image_tris = g->ranges != nullptr ? g->num_tri / std::max(g->batch, 1) : g->num_tri;
  const hipStream_t st = (hipStream_t)stream;
  if (gather_tiles(20 * image_tris))
    resolve_fwd_kernel<true><<<pixel_slot_blocks<4, true>(g->batch, g->height, g->width), 256, 0,
                               st>>>(*g, keys, rast, rast_db, sx, sy);
  else
    resolve_fwd_kernel<false><<<pixel_slot_blocks<4, false>(g->batch, g->height, g->width), 256,
                                0, st>>>(*g, keys, rast, rast_db, sx, sy);
  return launch_status();
}

extern "C" int dr_resolve_backward(const DrRasterGeometry* g, const uint64_t* keys,
                                   const float* grad_rast, const float* grad_rast_db,
                                   float* grad_pos, void* stream) {
  if (!valid_geometry(g) || !grad_rast || !grad_pos) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)g->batch * g->height * g->width;
  if (pixels == 0) return DR_OK;
  float sx, sy;
  resolve_scales(g, sx, sy);
  if ((int64_t)g->batch * (g->pos_batch_stride / 4) >= 0xffffffffLL) return DR_ERR_ARGUMENT;
  resolve_bwd_kernel<<<tile_blocks(g->batch, g->height, g->width), 256, 0,
                       (hipStream_t)stream>>>(
      *g, keys, grad_rast, grad_rast_db, grad_pos, sx, sy);
  return launch_status();
}
