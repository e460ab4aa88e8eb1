// Antialias for gfx950: edge adjacency, silhouette classification, and analytic blending of
// colours across silhouette edges with its gradient.
//
// Adjacency (reference.py:768-787) is built once per index buffer with an open-addressing
// hash table keyed on the sorted vertex pair of each edge: one 64-bit compare-and-swap claims
// a slot, a counter numbers the edges that share it, and a second pass reads off the partner
// edge of every edge used by exactly two triangles. The result does not depend on the order
// of insertion. The silhouette mask (reference.py:790-814) packs the three edge flags of a
// triangle into one byte per (image, triangle).
//
// Blending (reference.py:202-265, 675-765): for each pair of horizontally or vertically
// adjacent pixels showing different triangles, each pixel's triangle is tested at the other
// centre; the crossing t of its exit edge is found by linear interpolation of the edge
// functions, the nearer triangle owns the edge, and the pixel on t's side takes |t - 0.5| of
// the other's colour. aa_pairs_kernel evaluates every pair once (each pixel its right and
// lower pair) into a compact record -- t and (active, owner, edge) bits -- that the rest
// reuses: aa_blend_kernel gathers a pixel's four pairs into its output, and aa_bwd_kernel
// gathers the colour gradient the same way and sends the position gradient of each active
// pair (two vertices; x, y and w) through the workgroup's scatter table. No pass needs a
// colour atomic.
#include <algorithm>

#include "common.h"

namespace dr {
namespace {

constexpr uint64_t kEmptySlot = ~0ull;
constexpr float kEdgeTie = 4.76837158203125e-07f;   // 4 * float32 epsilon (reference.py:35)
constexpr float kAxisTie = 1.00010001659393310546875f;  // float32(1 + 1e-4) (reference.py:32)

// ---- adjacency --------------------------------------------------------------------------

struct HashTable {
  uint64_t* keys;
  uint32_t* counts;
  int32_t* edges;  // two edge numbers per slot
  uint64_t mask;
  size_t bytes;
};

HashTable hash_layout(int32_t num_tri, char* base) {
  uint64_t capacity = 1024;
  while (capacity < 2ull * 3ull * (uint64_t)num_tri) capacity <<= 1;
  HashTable h{};
  h.mask = capacity - 1;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off = (off + bytes + 255) & ~size_t(255);
    return p;
  };
  h.keys = (uint64_t*)take(8 * capacity);
  h.counts = (uint32_t*)take(4 * capacity);
  h.edges = (int32_t*)take(8 * capacity);
  h.bytes = off;
  return h;
}

__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdull;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ull;
  x ^= x >> 33;
  return x;
}

__device__ __forceinline__ uint64_t edge_key(const int32_t* tri, int64_t e) {
  const int64_t t = e / 3;
  const int k = (int)(e - 3 * t);
  const uint32_t a = (uint32_t)tri[3 * t + (k + 1) % 3];
  const uint32_t b = (uint32_t)tri[3 * t + (k + 2) % 3];
  const uint32_t lo = min(a, b), hi = max(a, b);
  return ((uint64_t)lo << 32) | hi;
}

__global__ void edge_hash_clear(HashTable h) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i > h.mask) return;
  h.keys[i] = kEmptySlot;
  h.counts[i] = 0u;
}

__global__ __launch_bounds__(256) void edge_hash_insert(const int32_t* tri, int64_t num_edges,
                                                   HashTable h) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= num_edges) return;
  const uint64_t key = edge_key(tri, e);
  uint64_t slot = mix64(key) & h.mask;
  for (uint64_t probe = 0; probe <= h.mask; ++probe) {
    const unsigned long long seen =
        atomicCAS((unsigned long long*)(h.keys + slot), (unsigned long long)kEmptySlot,
                  (unsigned long long)key);
    if (seen == kEmptySlot || seen == key) {
      const uint32_t n = atomicAdd(h.counts + slot, 1u);
      if (n < 2) h.edges[2 * slot + n] = (int32_t)e;
      return;
    }
    slot = (slot + 1) & h.mask;
  }
}

__global__ __launch_bounds__(256) void edge_hash_partner(const int32_t* tri, int64_t num_edges,
                                                    HashTable h, int32_t* neighbours) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= num_edges) return;
  const uint64_t key = edge_key(tri, e);
  uint64_t slot = mix64(key) & h.mask;
  int32_t partner = -1;
  for (uint64_t probe = 0; probe <= h.mask; ++probe) {
    const uint64_t k = h.keys[slot];
    if (k == key) {
      if (h.counts[slot] == 2u) {
        const int32_t a = h.edges[2 * slot], b = h.edges[2 * slot + 1];
        partner = (a == (int32_t)e) ? b : a;
      }
      break;
    }
    if (k == kEmptySlot) break;
    slot = (slot + 1) & h.mask;
  }
  neighbours[e] = partner;
}

// ---- silhouettes ------------------------------------------------------------------------

struct XYW {
  float x, y, w;
};

__device__ __forceinline__ XYW load_xyw(const float* pos, int v) {
  const float4 p = load4(pos + 4 * (int64_t)v);
  return {p.x, p.y, p.w};
}

// Sign of det[start, end, p] * w_p in homogeneous (x, y, w) (reference.py:802-809).
__device__ __forceinline__ float side(const float (&line)[3], const XYW& p) {
  const float d = line[0] * p.x + line[1] * p.y + line[2] * p.w;
  const float v = d * p.w;
  return v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f);
}

// Marks the triangles that rast shows (only their silhouette bits are ever read).
constexpr uint8_t kShown = 0x80;

// Zeroes n bytes: 16-byte stores over the aligned body, single bytes before and after it.
__global__ void aa_clear_mask(uint8_t* mask, int64_t n) {
  const int64_t head = std::min<int64_t>(n, (int64_t)((16u - ((uintptr_t)mask & 15u)) & 15u));
  const int64_t body = (n - head) / 16;
  const int64_t tail = head + body * 16;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < head) mask[t] = 0;
  if (t < n - tail) mask[tail + t] = 0;
  uint4* wide = reinterpret_cast<uint4*>(mask + head);
  for (int64_t i = t; i < body; i += (int64_t)gridDim.x * blockDim.x)
    wide[i] = make_uint4(0u, 0u, 0u, 0u);
}

__global__ __launch_bounds__(256) void aa_mark_shown(const float* rast, int64_t image_pixels,
                                                     int64_t pixels, int num_tri, int pos_batch,
                                                     uint8_t* mask) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= pixels) return;
  const float id = rintf(rast[4 * i + 3]);
  if (!(id >= 1.0f && id <= (float)num_tri)) return;
  const int64_t row = pos_batch > 1 ? i / image_pixels : 0;
  mask[row * num_tri + (int64_t)id - 1] = kShown;
}

// Silhouette bits of a triangle with vertex rows v in positions P, given the partner edge of
// each of its edges (-1: none) and the vertex opposite each partner edge (tri[partner]): bit k
// when edge k has no partner or both triangles lie on one side of it.
__device__ __forceinline__ uint8_t fold_bits(const float* P, const int (&v)[3],
                                             const int (&partner)[3], const int (&opposite)[3]) {
  const XYW p[3] = {load_xyw(P, v[0]), load_xyw(P, v[1]), load_xyw(P, v[2])};
  const XYW q[3] = {load_xyw(P, opposite[0]), load_xyw(P, opposite[1]),
                    load_xyw(P, opposite[2])};
  uint8_t bits = 0;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    if (partner[k] < 0) {
      bits |= (uint8_t)(1u << k);
      continue;
    }
    const XYW& s = p[(k + 1) % 3];
    const XYW& e = p[(k + 2) % 3];
    // The reference takes this cross product with torch.linalg.cross, whose CPU kernel rounds
    // each component as one fused multiply-add of the first product with the rounded second
    // (u_i v_j - u_j v_i = fma(u_i, v_j, -(u_j v_i)); checked bit for bit on a million random
    // float32 triples). A fold is classified by the sign of what follows, so near-degenerate
    // (edge-on) triangles at a silhouette need the same rounding.
    const float line[3] = {__builtin_fmaf(s.y, e.w, -(s.w * e.y)),
                           __builtin_fmaf(s.w, e.x, -(s.x * e.w)),
                           __builtin_fmaf(s.x, e.y, -(s.y * e.x))};
    if (side(line, p[k]) * side(line, q[k]) > 0.0f) bits |= (uint8_t)(1u << k);
  }
  return bits;
}

// The partner edges of triangle t and the vertices opposite them (row 0 where there is none).
__device__ __forceinline__ void partners(const int32_t* tri, const int32_t* nbr, int t,
                                         int (&v)[3], int (&partner)[3], int (&opposite)[3]) {
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    v[k] = tri[3 * t + k];
    partner[k] = nbr[3 * t + k];
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) opposite[k] = partner[k] >= 0 ? tri[partner[k]] : 0;
}

// Silhouette bits of (pos batch, triangle) i.
__device__ __forceinline__ void silhouette_bits(const float* pos, int64_t stride,
                                                const int32_t* tri, int num_tri,
                                                const int32_t* nbr, int64_t i, uint8_t* mask) {
  const int b = (int)(i / num_tri);
  const int t = (int)(i - (int64_t)b * num_tri);
  int v[3], partner[3], opposite[3];
  partners(tri, nbr, t, v, partner, opposite);
  mask[i] = fold_bits(pos + (int64_t)b * stride, v, partner, opposite);
}

// Silhouette bits of every (pos batch, triangle).
__global__ __launch_bounds__(256) void aa_silhouette_kernel(const float* pos, int64_t stride,
                                                            int pos_batch, const int32_t* tri,
                                                            int num_tri, const int32_t* nbr,
                                                            uint8_t* mask) {
  const int64_t n = (int64_t)pos_batch * num_tri;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    silhouette_bits(pos, stride, tri, num_tri, nbr, i, mask);
}

// Silhouette bits of the marked (pos batch, triangle) entries only (the others stay 0): one
// thread per triangle, over the batch entries it is marked in. Its index row, partners and
// opposite vertices are read once for every entry, together with the marks of eight entries at
// a time, so that a thread waits for two rounds of loads and then one per entry it is marked
// in, not three per (entry, triangle) in turn: the pass is bound by the latency of its gathers.
__global__ __launch_bounds__(256) void aa_silhouette_shown_kernel(const float* pos,
                                                                  int64_t stride, int pos_batch,
                                                                  const int32_t* tri,
                                                                  int num_tri, const int32_t* nbr,
                                                                  uint8_t* mask) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= num_tri) return;
  int v[3], partner[3], opposite[3];
  bool rows = false;
  constexpr int kGroup = 8;
  for (int b0 = 0; b0 < pos_batch; b0 += kGroup) {
    uint8_t marks[kGroup];
#pragma unroll
    for (int j = 0; j < kGroup; ++j)
      marks[j] = b0 + j < pos_batch ? mask[(int64_t)(b0 + j) * num_tri + t] : 0;
    if (!rows) {
      partners(tri, nbr, t, v, partner, opposite);  // issued before the marks are waited for
      rows = true;
    }
    uint32_t shown = 0u;
#pragma unroll
    for (int j = 0; j < kGroup; ++j) shown |= (marks[j] == kShown ? 1u : 0u) << j;
    while (shown != 0u) {
      const int j = __ffs(shown) - 1;
      shown &= shown - 1u;
      const int64_t b = b0 + j;
      mask[b * num_tri + t] = fold_bits(pos + b * stride, v, partner, opposite);
    }
  }
}

// ---- crossings --------------------------------------------------------------------------

// a[k] for a k known only at run time, as selects: indexing a register array with it would
// move the array to scratch memory.
template <typename V>
__device__ __forceinline__ V pick3(const V (&a)[3], int k) {
  return k == 0 ? a[0] : (k == 1 ? a[1] : a[2]);
}

struct Triangle {
  int v[3];
  float x[3], y[3], w[3];
};

struct Crossing {
  bool found;
  float t;
  int edge;
};

// Exit of the triangle shown at the source centre along the segment to the destination
// centre (reference.py:675-727), without its gradient.
__device__ __forceinline__ Crossing crossing(const Triangle& T, uint8_t sil, bool horizontal,
                                             int width, int height, float sx, float sy, float dx,
                                             float dy) {
  Crossing out{false, 0.0f, 0};
  float e_src[3], e_dst[3], slack[3];
  float as[3], cs[3], ad[3], cd[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    as[k] = T.x[k] - sx * T.w[k];
    cs[k] = T.y[k] - sy * T.w[k];
    ad[k] = T.x[k] - dx * T.w[k];
    cd[k] = T.y[k] - dy * T.w[k];
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int i = (k + 1) % 3, j = (k + 2) % 3;
    e_src[k] = as[i] * cs[j] - as[j] * cs[i];
    e_dst[k] = ad[i] * cd[j] - ad[j] * cd[i];
    // Rounding bound of the edge function at the destination (reference.py:730-746).
    const float rxi = fabsf(T.x[i]) + fabsf(T.w[i]), rxj = fabsf(T.x[j]) + fabsf(T.w[j]);
    const float ryi = fabsf(T.y[i]) + fabsf(T.w[i]), ryj = fabsf(T.y[j]) + fabsf(T.w[j]);
    const float terms = (rxi + fabsf(ad[i])) * fabsf(cd[j]) + (rxj + fabsf(ad[j])) * fabsf(cd[i]) +
                        ryj * fabsf(ad[i]) + ryi * fabsf(ad[j]);
    slack[k] = terms * kEdgeTie;
  }
  const float sign = (e_src[0] + e_src[1] + e_src[2]) < 0.0f ? -1.0f : 1.0f;
  bool any = false;
  float best = __int_as_float(0x7f800000);  // +inf
  int edge = 0;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float span = e_src[k] - e_dst[k];
    const bool crossed = (e_dst[k] * sign <= slack[k]) && (span * sign > 2.0f * slack[k]);
    if (crossed) {
      any = true;
      const float t = e_src[k] / span;
      if (t < best) {
        best = t;
        edge = k;
      }
    }
  }
  if (!any || !((sil >> edge) & 1u)) return out;
  // The axis whose pixel pairs handle this edge (reference.py:749-765).
  const int i = (edge + 1) % 3, j = (edge + 2) % 3;
  const float xi = pick3(T.x, i), yi = pick3(T.y, i), wi = pick3(T.w, i);
  const float xj = pick3(T.x, j), yj = pick3(T.y, j), wj = pick3(T.w, j);
  const float steep = fabsf(wj * yi - wi * yj) * (float)height * kAxisTie;
  const float flat = fabsf(xj * wi - xi * wj) * (float)width;
  const bool along = horizontal ? (steep >= flat) : (flat > steep);
  if (!along) return out;
  out.found = true;
  out.t = best;
  out.edge = edge;
  return out;
}

// The two vertices i, j of a triangle's edge: rows and x, y, w.
struct EdgeVerts {
  int vi, vj;
  float xi, yi, wi, xj, yj, wj;
};

// d t / d (x, y, w) of the edge's two vertices, t = e_s / (e_s - e_d) with
// e = a_i c_j - a_j c_i, a = x - px w, c = y - py w. Order: x_i, y_i, w_i, x_j, y_j, w_j.
__device__ __forceinline__ void crossing_grad(const EdgeVerts& E, float sx, float sy,
                                              float dx, float dy, float (&g)[6]) {
  const float xi = E.xi, yi = E.yi, wi = E.wi, xj = E.xj, yj = E.yj, wj = E.wj;
  const float asi = xi - sx * wi, csi = yi - sy * wi;
  const float asj = xj - sx * wj, csj = yj - sy * wj;
  const float adi = xi - dx * wi, cdi = yi - dy * wi;
  const float adj = xj - dx * wj, cdj = yj - dy * wj;
  const float es = asi * csj - asj * csi;
  const float ed = adi * cdj - adj * cdi;
  const float span = es - ed;
  const float inv = 1.0f / (span * span);  // one division (the quotients within two ulp)
  const float dt_des = -ed * inv;
  const float dt_ded = es * inv;
  // d e / d(x_i, y_i, w_i, x_j, y_j, w_j) at a centre (px, py) with a, c there.
  auto de = [](float ai, float ci, float aj, float cj, float px, float py, float (&d)[6]) {
    d[0] = cj;
    d[1] = -aj;
    d[2] = -px * cj + py * aj;
    d[3] = -ci;
    d[4] = ai;
    d[5] = px * ci - py * ai;
  };
  float ds[6], dd[6];
  de(asi, csi, asj, csj, sx, sy, ds);
  de(adi, cdi, adj, cdj, dx, dy, dd);
#pragma unroll
  for (int k = 0; k < 6; ++k) g[k] = dt_des * ds[k] + dt_ded * dd[k];
}

__device__ __forceinline__ int pixel_tri(const DrAntialiasArgs& a, int64_t pixel, float& depth) {
  const float4 r = load4(a.rast + 4 * pixel);
  depth = r.z;
  const float id = rintf(r.w);
  // Ids past the end of tri are background (reference.py:228-230).
  return (id >= 1.0f && id <= (float)a.num_tri) ? (int)id - 1 : -1;
}

// The vertex rows of triangle t.
__device__ __forceinline__ void load_rows(const DrAntialiasArgs& a, int t, int (&v)[3]) {
#pragma unroll
  for (int k = 0; k < 3; ++k) v[k] = a.tri[3 * (int64_t)t + k];
}

// x, y and w of the vertices in rows v of image b's positions.
__device__ __forceinline__ void load_vertices(const DrAntialiasArgs& a, int b, const int (&v)[3],
                                              Triangle& T) {
  const float* P = a.pos + (int64_t)b * a.pos_batch_stride;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    T.v[k] = v[k];
    const float4 p = load4(P + 4 * (int64_t)v[k]);
    T.x[k] = p.x;
    T.y[k] = p.y;
    T.w[k] = p.w;
  }
}

__device__ __forceinline__ void load_triangle(const DrAntialiasArgs& a, int b, int t,
                                              Triangle& T) {
  int v[3];
  load_rows(a, t, v);
  load_vertices(a, b, v, T);
}

// Rows and vertices of edge `edge` of triangle t: its vertices (edge + 1) mod 3 and
// (edge + 2) mod 3, the only two the crossing's gradient needs.
__device__ __forceinline__ void load_edge(const DrAntialiasArgs& a, int b, int t, int edge,
                                          EdgeVerts& E) {
  const int32_t* row = a.tri + 3 * (int64_t)t;
  E.vi = row[edge == 2 ? 0 : edge + 1];
  E.vj = row[edge == 0 ? 2 : edge - 1];
  const float* P = a.pos + (int64_t)b * a.pos_batch_stride;
  const float4 pi = load4(P + 4 * (int64_t)E.vi), pj = load4(P + 4 * (int64_t)E.vj);
  E.xi = pi.x;
  E.yi = pi.y;
  E.wi = pi.w;
  E.xj = pj.x;
  E.yj = pj.y;
  E.wj = pj.w;
}

// Pair record bits: the pair is active, the first pixel's triangle owns the edge, edge index.
constexpr uint8_t kActive = 0x8, kOwnerFirst = 0x4;

// Record bits and t of the pair (p, q) from the crossings found from each side
// (reference.py:238-258): the nearer triangle owns the edge, p's on a depth tie.
__device__ __forceinline__ uint8_t pair_record(const Crossing& from_p, const Crossing& from_q,
                                               float depth_p, float depth_q, float& t) {
  const bool use_p = from_p.found && (!from_q.found || depth_p <= depth_q);
  const bool use_q = from_q.found && !use_p;
  t = 0.0f;
  if (!use_p && !use_q) return 0;
  t = use_p ? from_p.t : 1.0f - from_q.t;
  return (uint8_t)(kActive | (use_p ? kOwnerFirst : 0) | (use_p ? from_p.edge : from_q.edge));
}

// Triangle index of a rast pixel from its (z, w) pair, and its depth; -1 for background.
__device__ __forceinline__ int zw_tri(const DrAntialiasArgs& a, float2 zw, float& depth) {
  depth = zw.x;
  const float id = rintf(zw.y);
  // Ids past the end of tri are background (reference.py:228-230).
  return (id >= 1.0f && id <= (float)a.num_tri) ? (int)id - 1 : -1;
}

// The 16 x 16 tile of a pixel, numbered as tile_pixel() numbers workgroups before xcd_order.
__device__ __forceinline__ int64_t tile_of(const DrAntialiasArgs& a, const TilePixel& tp) {
  const int tiles_x = (a.width + 15) / 16, tiles_y = (a.height + 15) / 16;
  return ((int64_t)tp.b * tiles_y + tp.y / 16) * tiles_x + tp.x / 16;
}

// The activity flags (aa_pairs_kernel) of tp's tile and of the tiles to its left and above,
// whose last column and row hold records that its pixels read. A tile without an active pair
// has no records written: its pixels' pairs are all inactive. Uniform over the workgroup.
struct TileFlags {
  bool own, left, up;
  __device__ __forceinline__ bool any() const { return own || left || up; }
};

__device__ __forceinline__ TileFlags tile_flags(const DrAntialiasArgs& a, const TilePixel& tp,
                                                const uint8_t* tile_active) {
  if (tile_active == nullptr) return {true, true, true};  // dense: every record written
  const int tiles_x = (a.width + 15) / 16;
  const int64_t t = tile_of(a, tp);
  TileFlags f;
  f.own = tile_active[t] != 0;
  f.left = tp.x >= 16 && tile_active[t - 1] != 0;
  f.up = tp.y >= 16 && tile_active[t - tiles_x] != 0;
  return f;
}

// Copies the workgroup's 16 x 16 tile of [.., C] values from src to dst, row by row, 16 bytes
// per thread where the rows allow (a tile row is 16 C consecutive floats): every thread of the
// workgroup takes part, inside the image or not.
__device__ __forceinline__ void copy_tile(const DrAntialiasArgs& a, const TilePixel& tp,
                                          const float* __restrict__ src,
                                          float* __restrict__ dst) {
  const int C = a.channels;
  const int x0 = tp.x & ~15, y0 = tp.y & ~15;
  const int rows = min(16, a.height - y0), row_floats = min(16, a.width - x0) * C;
  const int64_t first = (((int64_t)tp.b * a.height + y0) * a.width + x0) * C;
  const int64_t stride = (int64_t)a.width * C;
  const bool wide = row_floats % 4 == 0 && stride % 4 == 0 && first % 4 == 0 &&
                    ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) == 0;
  if (wide) {  // uniform
    const int per_row = row_floats / 4;
    for (int i = threadIdx.x; i < rows * per_row; i += blockDim.x) {
      const int r = i / per_row;
      const int64_t at = first + r * stride + 4 * (i - r * per_row);
      store4(dst + at, load4(src + at));
    }
  } else {
    for (int i = threadIdx.x; i < rows * row_floats; i += blockDim.x) {
      const int r = i / row_floats;
      const int64_t at = first + r * stride + (i - r * row_floats);
      dst[at] = src[at];
    }
  }
}

// Every pixel evaluates the pairs it forms with its right and lower neighbours, once. The
// loads go level by level over the (at most three) triangles involved -- ids, silhouette bits,
// index rows, vertices -- so that each level's loads are in flight together: a wave where any
// pixel needs a triangle reads all three for every lane, lanes that need fewer reading
// triangle 0 in their place (one cached line). A pair of pixels showing one triangle, or two
// triangles without silhouette edges, is inactive.
// The pixel's records: crossings (t_right, t_down) and bits (right, down).
__device__ __forceinline__ void pixel_pairs_of(const DrAntialiasArgs& a, const TilePixel& tp,
                                               float2& pair_t, uchar2& pair_bits) {
  const bool has_right = tp.x + 1 < a.width, has_down = tp.y + 1 < a.height;
  const float* zw = a.rast + 4 * tp.pixel + 2;
  const float2 zw_p = *reinterpret_cast<const float2*>(zw);
  const float2 zw_r = *reinterpret_cast<const float2*>(zw + (has_right ? 4 : 0));
  const float2 zw_d = *reinterpret_cast<const float2*>(zw + (has_down ? 4 * (int64_t)a.width : 0));
  float depth, depth_r, depth_d;
  const int id = zw_tri(a, zw_p, depth);
  const int id_r = zw_tri(a, zw_r, depth_r);
  const int id_d = zw_tri(a, zw_d, depth_d);
  const bool live_r = id != id_r, live_d = id != id_d;
  const uint8_t* sil = a.silhouette + (int64_t)tp.b * a.silhouette_batch_stride;
  const uint8_t sil_p = (live_r || live_d) && id >= 0 ? sil[id] : 0;
  const uint8_t sil_r = live_r && id_r >= 0 ? sil[id_r] : 0;
  const uint8_t sil_d = live_d && id_d >= 0 ? sil[id_d] : 0;
  // A triangle is read where it has silhouette edges and its pixel is in a live pair.
  const bool need_p = sil_p != 0, need_r = sil_r != 0, need_d = sil_d != 0;
  float t_right = 0.f, t_down = 0.f;
  uint8_t right = 0, down = 0;
  if (__any(need_p || need_r || need_d)) {  // then num_tri >= 1: triangle 0 exists
    int rows_p[3], rows_r[3], rows_d[3];
    load_rows(a, need_p ? id : 0, rows_p);
    load_rows(a, need_r ? id_r : 0, rows_r);
    load_rows(a, need_d ? id_d : 0, rows_d);
    Triangle Tp, Tr, Td;
    load_vertices(a, tp.b, rows_p, Tp);
    load_vertices(a, tp.b, rows_r, Tr);
    load_vertices(a, tp.b, rows_d, Td);
    const float px = pixel_centre(tp.x, a.width), py = pixel_centre(tp.y, a.height);
    if (live_r && (need_p || need_r)) {
      const float qx = pixel_centre(tp.x + 1, a.width);
      const Crossing none{false, 0.f, 0};
      const Crossing from_p =
          need_p ? crossing(Tp, sil_p, true, a.width, a.height, px, py, qx, py) : none;
      const Crossing from_q =
          need_r ? crossing(Tr, sil_r, true, a.width, a.height, qx, py, px, py) : none;
      right = pair_record(from_p, from_q, depth, depth_r, t_right);
    }
    if (live_d && (need_p || need_d)) {
      const float qy = pixel_centre(tp.y + 1, a.height);
      const Crossing none{false, 0.f, 0};
      const Crossing from_p =
          need_p ? crossing(Tp, sil_p, false, a.width, a.height, px, py, px, qy) : none;
      const Crossing from_q =
          need_d ? crossing(Td, sil_d, false, a.width, a.height, px, qy, px, py) : none;
      down = pair_record(from_p, from_q, depth, depth_d, t_down);
    }
  }
  pair_t = make_float2(t_right, t_down);
  pair_bits = make_uchar2(right, down);
}

// One workgroup per tile: the tile's flag (any active pair) and, only in a flagged tile, every
// pixel's pair records. The blend and the backward pass treat the records of unflagged tiles as
// inactive without reading them, and copy colour and gradient where no record they read is
// active. Without flags (tile_active NULL: dense images, where nearly every tile has an active
// pair and the flags' loads would only add a round trip) every record is written.
__global__ __launch_bounds__(256) void aa_pairs_kernel(DrAntialiasArgs a, float2* pair_t,
                                                       uchar2* pair_bits,
                                                       uint8_t* tile_active) {
  __shared__ int s_active;
  if (threadIdx.x == 0) s_active = 0;
  __syncthreads();
  const TilePixel tp = tile_pixel(a.batch, a.height, a.width);
  float2 t = make_float2(0.f, 0.f);
  uchar2 bits = make_uchar2(0, 0);
  if (tp.inside) pixel_pairs_of(a, tp, t, bits);
  if ((bits.x | bits.y) & kActive) s_active = 1;  // any order: every writer stores 1
  __syncthreads();
  const bool active = tile_active == nullptr || s_active != 0;
  if (threadIdx.x == 0 && tile_active != nullptr) tile_active[tile_of(a, tp)] = (uint8_t)active;
  if (active && tp.inside) {
    pair_t[tp.pixel] = t;
    pair_bits[tp.pixel] = bits;
  }
}

// The four pairs of a pixel as (active, t, other pixel, this pixel is the first).
struct PixelPairs {
  bool active[4];
  float t[4];
  int64_t other[4];
  bool first[4];
};

__device__ __forceinline__ PixelPairs pixel_pairs(const DrAntialiasArgs& a, const TilePixel& tp,
                                                  const float2* pair_t,
                                                  const uchar2* pair_bits, TileFlags f) {
  PixelPairs P;
  const float2 own_t = pair_t[tp.pixel];
  const uchar2 own_b = pair_bits[tp.pixel];
  // Records of an unflagged tile were never written (whatever they read is ignored).
  const bool left_ok = (tp.x & 15) ? f.own : f.left, up_ok = (tp.y & 15) ? f.own : f.up;
  P.active[0] = f.own && (own_b.x & kActive);
  P.t[0] = own_t.x;
  P.other[0] = tp.pixel + 1;
  P.first[0] = true;
  P.active[1] = f.own && (own_b.y & kActive);
  P.t[1] = own_t.y;
  P.other[1] = tp.pixel + a.width;
  P.first[1] = true;
  // The left and upper neighbours' records, read with the pixel's own (a pixel on the first
  // column or row reads its own record there and ignores it): no branch between the loads.
  const int64_t left = tp.x > 0 ? tp.pixel - 1 : tp.pixel;
  const int64_t up = tp.y > 0 ? tp.pixel - a.width : tp.pixel;
  const uchar2 left_b = pair_bits[left], up_b = pair_bits[up];
  const float2 left_t = pair_t[left], up_t = pair_t[up];
  P.active[2] = tp.x > 0 && left_ok && (left_b.x & kActive);
  P.t[2] = left_t.x;
  P.other[2] = tp.pixel - 1;
  P.first[2] = false;
  P.active[3] = tp.y > 0 && up_ok && (up_b.y & kActive);
  P.t[3] = up_t.y;
  P.other[3] = tp.pixel - a.width;
  P.first[3] = false;
  return P;
}

// Channels [c0, c0 + n) of a pixel whose first channel is at p (n <= N; 0 past n): the widest
// loads the alignment allows, all issued together.
template <int N>
__device__ __forceinline__ void load_group(const float* p, int n, float (&v)[N]) {
  if constexpr (N == 4) {
    if (n == 4 && load_wide<4>(p, v)) return;
  } else if constexpr (N == 2) {
    if (n == 2 && load_wide<2>(p, v)) return;
  }
#pragma unroll
  for (int c = 0; c < N; ++c) v[c] = c < n ? p[c] : 0.0f;
}

template <int N>
__device__ __forceinline__ void store_group(float* p, int n, const float (&v)[N]) {
  if constexpr (N == 4 || N == 2) {
    if (n == N && store_wide<N>(p, v)) return;
  }
#pragma unroll
  for (int c = 0; c < N; ++c)
    if (c < n) p[c] = v[c];
}

// out = colour + |t - 0.5| of the neighbour's colour on the side of each crossing
// (reference.py:253-264). A pixel takes (0.5 - t) of its pair partner when it is the first
// pixel and t < 0.5, and (t - 0.5) when it is the second and t >= 0.5.
// NC channels per group: the channel count for 1 to 4 channels (whole-pixel loads and stores),
// 4 with a loop over groups for more.
template <int NC, bool SPARSE>
__global__ __launch_bounds__(256) void aa_blend_kernel(DrAntialiasArgs a, const float2* pair_t,
                                                       const uchar2* pair_bits,
                                                       const uint8_t* tile_active, float* out) {
  const TilePixel tp = tile_pixel(a.batch, a.height, a.width);
  const int C = a.channels;
  const TileFlags flags = SPARSE ? tile_flags(a, tp, tile_active) : TileFlags{true, true, true};
  if (SPARSE && !flags.any()) {  // uniform: no pair moves colour here
    copy_tile(a, tp, a.color, out);
    return;
  }
  if (!tp.inside) return;
  const PixelPairs P = pixel_pairs(a, tp, pair_t, pair_bits, flags);
  float weight[4];
  bool any = false;
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const float t = P.t[n];
    const bool takes = P.active[n] && (P.first[n] ? t < 0.5f : t >= 0.5f);
    weight[n] = takes ? (P.first[n] ? 0.5f - t : t - 0.5f) : 0.0f;
    any = any || takes;
  }
  const float* color = a.color + tp.pixel * C;
  float* o = out + tp.pixel * C;
  for (int c0 = 0; c0 < C; c0 += NC) {
    const int n = min(NC, C - c0);
    float own[NC], v[NC];
    load_group<NC>(color + c0, n, own);
#pragma unroll
    for (int c = 0; c < NC; ++c) v[c] = own[c];
    if (any) {
      // Every neighbour that lends colour is read before any is used.
      float other[4][NC];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (weight[k] != 0.0f) {
          load_group<NC>(a.color + P.other[k] * C + c0, n, other[k]);
        } else {
#pragma unroll
          for (int c = 0; c < NC; ++c) other[k][c] = own[c];
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (weight[k] == 0.0f) continue;
#pragma unroll
        for (int c = 0; c < NC; ++c) v[c] += weight[k] * (other[k][c] - own[c]);
      }
    }
    store_group<NC>(o + c0, n, v);
  }
}

// Colour gradient (a gather over the same pairs) and position gradient of each active pair,
// written by its first pixel through the workgroup's scatter table (rows of pos: x, y, z, w).
template <int NC, bool SPARSE>
__global__ __launch_bounds__(256) void aa_bwd_kernel(DrAntialiasArgs a, const float2* pair_t,
                                                     const uchar2* pair_bits,
                                                     const uint8_t* tile_active,
                                                     const float* grad_out, float* grad_color,
                                                     float* grad_pos) {
  using Table = RowTable<512, 4>;
  __shared__ Table table;
  if (!SPARSE) table.init();
  const TilePixel tp = tile_pixel(a.batch, a.height, a.width);
  const int C = a.channels;
  const TileFlags flags = SPARSE ? tile_flags(a, tp, tile_active) : TileFlags{true, true, true};
  if (SPARSE && !flags.any()) {  // uniform: the gradient passes through
    if (grad_color) copy_tile(a, tp, grad_out, grad_color);
    return;
  }
  if (SPARSE) table.init();
  uint32_t rows[4] = {Table::kEmpty, Table::kEmpty, Table::kEmpty, Table::kEmpty};
  float vals[4][4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int c = 0; c < 4; ++c) vals[k][c] = 0.0f;
  if (tp.inside) {
    const PixelPairs P = pixel_pairs(a, tp, pair_t, pair_bits, flags);
    const float* g = grad_out + tp.pixel * C;
    if (grad_color) {
      for (int c0 = 0; c0 < C; c0 += NC) {
        const int n = min(NC, C - c0);
        float gv[NC], v[NC];
        load_group<NC>(g + c0, n, gv);
#pragma unroll
        for (int c = 0; c < NC; ++c) v[c] = gv[c];
        // Every active neighbour's gradient is read before any is used.
        float g2s[4][NC];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (P.active[k]) {
            load_group<NC>(grad_out + P.other[k] * C + c0, n, g2s[k]);
          } else {
#pragma unroll
            for (int c = 0; c < NC; ++c) g2s[k][c] = 0.0f;
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (!P.active[k]) continue;
          const float t = P.t[k];
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            if (P.first[k]) {
              v[c] += t < 0.5f ? -(0.5f - t) * gv[c] : (t - 0.5f) * g2s[k][c];
            } else {
              v[c] += t < 0.5f ? (0.5f - t) * g2s[k][c] : -(t - 0.5f) * gv[c];
            }
          }
        }
        store_group<NC>(grad_color + tp.pixel * C + c0, n, v);
      }
    }
    if (grad_pos) {
      const uchar2 bits = flags.own ? pair_bits[tp.pixel] : make_uchar2(0, 0);
      const int pos_b = a.pos_batch_stride != 0 ? tp.b : 0;
      const int64_t row0 = (int64_t)pos_b * (a.pos_batch_stride / 4);
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const uint8_t info = n == 0 ? bits.x : bits.y;
        if (!(info & kActive)) continue;
        const float t = P.t[n];
        const int64_t q = P.other[n];
        const float* cP = a.color + tp.pixel * C;
        const float* cQ = a.color + q * C;
        const float* g2 = grad_out + q * C;
        float g_t = 0.0f;
        for (int c0 = 0; c0 < C; c0 += NC) {
          const int m = min(NC, C - c0);
          float vP[NC], vQ[NC], vg[NC];
          load_group<NC>(cP + c0, m, vP);
          load_group<NC>(cQ + c0, m, vQ);
          load_group<NC>((t < 0.5f ? g : g2) + c0, m, vg);
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            if (t < 0.5f)
              g_t -= vg[c] * (vQ[c] - vP[c]);
            else
              g_t += vg[c] * (vP[c] - vQ[c]);
          }
        }
        const bool owner_first = info & kOwnerFirst;
        g_t *= owner_first ? a.boost : -a.boost;  // t = 1 - t_q when the second pixel owns it
        if (g_t == 0.0f) continue;
        const int qx = tp.x + (n == 0 ? 1 : 0), qy = tp.y + (n == 0 ? 0 : 1);
        const float px = pixel_centre(tp.x, a.width), py = pixel_centre(tp.y, a.height);
        const float qcx = pixel_centre(qx, a.width), qcy = pixel_centre(qy, a.height);
        float depth;
        const int owner = pixel_tri(a, owner_first ? tp.pixel : q, depth);
        EdgeVerts E;
        load_edge(a, tp.b, owner, info & 3, E);
        float d[6];
        crossing_grad(E, owner_first ? px : qcx, owner_first ? py : qcy,
                      owner_first ? qcx : px, owner_first ? qcy : py, d);
        const int vi = E.vi, vj = E.vj;
        rows[2 * n] = (uint32_t)(row0 + vi);
        rows[2 * n + 1] = (uint32_t)(row0 + vj);
        vals[2 * n][0] = g_t * d[0];
        vals[2 * n][1] = g_t * d[1];
        vals[2 * n][3] = g_t * d[2];
        vals[2 * n + 1][0] = g_t * d[3];
        vals[2 * n + 1][1] = g_t * d[4];
        vals[2 * n + 1][3] = g_t * d[5];
      }
    }
  }
  if (grad_pos == nullptr) return;  // uniform over the workgroup
  float lane_max = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (rows[k] != Table::kEmpty) lane_max = fmaxf(lane_max, max_magnitude(vals[k], 4));
  const FixedPass f = table.begin(lane_max);
#pragma unroll
  for (int k = 0; k < 4; ++k) table.add_wave(rows[k], vals[k], 4, grad_pos, 4, f);
  __syncthreads();
  table.flush(grad_pos, 4, 4, f);
}

bool valid_args(const DrAntialiasArgs* a) {
  if (!a || !a->color || !a->rast || !a->pos || !a->tri || !a->silhouette) return false;
  if (a->batch < 0 || a->height <= 0 || a->width <= 0 || a->channels < 0 || a->num_tri < 0)
    return false;
  return true;
}

}  // namespace
}  // namespace dr

using namespace dr;

extern "C" int dr_edge_hash_workspace_size(int32_t num_tri, size_t* bytes) {
  if (num_tri < 0 || !bytes) return DR_ERR_ARGUMENT;
  *bytes = hash_layout(num_tri, nullptr).bytes;
  return DR_OK;
}

extern "C" int dr_edge_neighbours(const int32_t* tri, int32_t num_tri, void* workspace,
                                  size_t workspace_bytes, int32_t* neighbours, void* stream) {
  if (num_tri < 0 || num_tri > (1 << 24)) return DR_ERR_ARGUMENT;
  if (num_tri == 0) return DR_OK;
  if (!tri || !neighbours) return DR_ERR_ARGUMENT;
  HashTable h = hash_layout(num_tri, (char*)workspace);
  if (!workspace || workspace_bytes < h.bytes) return DR_ERR_CAPACITY;
  hipStream_t s = (hipStream_t)stream;
  const int64_t edges = 3 * (int64_t)num_tri;
  edge_hash_clear<<<blocks_for((int64_t)h.mask + 1, 256), 256, 0, s>>>(h);
  edge_hash_insert<<<blocks_for(edges, 256), 256, 0, s>>>(tri, edges, h);
  edge_hash_partner<<<blocks_for(edges, 256), 256, 0, s>>>(tri, edges, h, neighbours);
  return launch_status();
}

extern "C" int dr_silhouette_mask(const float* pos, int64_t pos_batch_stride, int32_t pos_batch,
                                  const int32_t* tri, int32_t num_tri, const int32_t* neighbours,
                                  const float* rast, int32_t batch, int32_t height, int32_t width,
                                  uint8_t* mask, void* stream) {
  if (pos_batch < 0 || num_tri < 0) return DR_ERR_ARGUMENT;
  const int64_t n = (int64_t)pos_batch * num_tri;
  if (n == 0) return DR_OK;
  if (!pos || !tri || !neighbours || !mask) return DR_ERR_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  if (rast != nullptr) {
    if (batch < 0 || height <= 0 || width <= 0) return DR_ERR_ARGUMENT;
    if (pos_batch > 1 && pos_batch != batch) return DR_ERR_ARGUMENT;
    const int64_t image_pixels = (int64_t)height * width, pixels = image_pixels * batch;
    aa_clear_mask<<<(int)std::min<int64_t>(blocks_for(n / 16 + 16, 256), 65536), 256, 0, s>>>(
        mask, n);
    if (pixels > 0)
      aa_mark_shown<<<blocks_for(pixels, 256), 256, 0, s>>>(rast, image_pixels, pixels, num_tri,
                                                           pos_batch, mask);
  }
  if (rast != nullptr)
    aa_silhouette_shown_kernel<<<blocks_for(num_tri, 256), 256, 0, s>>>(
        pos, pos_batch_stride, pos_batch, tri, num_tri, neighbours, mask);
  else
    aa_silhouette_kernel<<<(int)std::min<int64_t>(blocks_for(n, 256), 4096), 256, 0, s>>>(
        pos, pos_batch_stride, pos_batch, tri, num_tri, neighbours, mask);
  return launch_status();
}

extern "C" int dr_antialias_workspace_size(const DrAntialiasArgs* a, size_t* bytes) {
  if (!valid_args(a) || !bytes) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  *bytes = (size_t)pixels * (sizeof(float2) + sizeof(uchar2)) +
           (size_t)tile_blocks(a->batch, a->height, a->width);
  return DR_OK;
}

// Whether the pair records are sparse enough for tile flags: as for the silhouettes, when
// the (pos batch, triangle) pairs are fewer than a sixth of the pixels (small meshes in large
// images, range mode); dense views of one mesh fill nearly every tile with active pairs.
static bool sparse_pairs(const DrAntialiasArgs* a) {
  const int64_t pos_batch = a->pos_batch_stride != 0 ? a->batch : 1;
  return 6 * pos_batch * (int64_t)a->num_tri <= (int64_t)a->batch * a->height * a->width;
}

// The pair records: crossings, then bits, then one activity flag per 16 x 16 tile.
static void pair_buffers(const DrAntialiasArgs* a, void* pairs, float2*& t, uchar2*& bits,
                         uint8_t*& tiles) {
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  t = (float2*)pairs;
  bits = (uchar2*)((char*)pairs + pixels * sizeof(float2));
  tiles = (uint8_t*)((char*)pairs + pixels * (sizeof(float2) + sizeof(uchar2)));
}

extern "C" int dr_antialias_forward(const DrAntialiasArgs* a, void* pairs, size_t pairs_bytes,
                                    float* out, void* stream) {
  if (!valid_args(a) || !out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  size_t need = 0;
  dr_antialias_workspace_size(a, &need);
  if (!pairs || pairs_bytes < need) return DR_ERR_CAPACITY;
  float2* t;
  uchar2* bits;
  uint8_t* tiles;
  pair_buffers(a, pairs, t, bits, tiles);
  const bool sparse = sparse_pairs(a);
  if (!sparse) tiles = nullptr;
  const int64_t blocks = tile_blocks(a->batch, a->height, a->width);
  aa_pairs_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(*a, t, bits, tiles);
  if (a->channels <= 0) return launch_status();
  return channel_groups(a->channels, [&](auto nc) {
    constexpr int NC = decltype(nc)::value;
    if (sparse)
      aa_blend_kernel<NC, true><<<blocks, 256, 0, (hipStream_t)stream>>>(*a, t, bits, tiles, out);
    else
      aa_blend_kernel<NC, false><<<blocks, 256, 0, (hipStream_t)stream>>>(*a, t, bits, tiles, out);
    return launch_status();
  });
}

extern "C" int dr_antialias_backward(const DrAntialiasArgs* a, const void* pairs,
                                     size_t pairs_bytes, const float* grad_out,
                                     float* grad_color, float* grad_pos, void* stream) {
  if (!valid_args(a) || !grad_out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  size_t need = 0;
  dr_antialias_workspace_size(a, &need);
  if (!pairs || pairs_bytes < need) return DR_ERR_CAPACITY;
  if (grad_pos && (int64_t)a->batch * (a->pos_batch_stride / 4) >= 0xffffffffLL)
    return DR_ERR_ARGUMENT;
  float2* t;
  uchar2* bits;
  uint8_t* tiles;
  pair_buffers(a, (void*)pairs, t, bits, tiles);
  const bool sparse = sparse_pairs(a);
  if (!sparse) tiles = nullptr;
  const int64_t blocks = tile_blocks(a->batch, a->height, a->width);
  return channel_groups(a->channels, [&](auto nc) {
    constexpr int NC = decltype(nc)::value;
    if (sparse)
      aa_bwd_kernel<NC, true><<<blocks, 256, 0, (hipStream_t)stream>>>(
          *a, t, bits, tiles, grad_out, grad_color, grad_pos);
    else
      aa_bwd_kernel<NC, false><<<blocks, 256, 0, (hipStream_t)stream>>>(
          *a, t, bits, tiles, grad_out, grad_color, grad_pos);
    return launch_status();
  });
}
