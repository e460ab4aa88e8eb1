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
// the other's colour. The forward kernel is a gather: every pixel evaluates the (at most four)
// pairs it belongs to and writes its own output, so no atomics are needed. The backward kernel
// gathers the colour gradient the same way and scatters the position gradient of each active
// pair (two vertices, x, y and w) with atomics from the pair's first pixel.
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

__global__ __launch_bounds__(256) void aa_silhouette_kernel(const float* pos, int64_t stride,
                                                         int pos_batch, const int32_t* tri,
                                                         int num_tri, const int32_t* nbr,
                                                         uint8_t* mask) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)pos_batch * num_tri) return;
  const int b = (int)(i / num_tri);
  const int t = (int)(i - (int64_t)b * num_tri);
  const float* P = pos + (int64_t)b * stride;
  const int v[3] = {tri[3 * t], tri[3 * t + 1], tri[3 * t + 2]};
  uint8_t bits = 0;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int partner = nbr[3 * t + k];
    if (partner < 0) {
      bits |= (uint8_t)(1u << k);
      continue;
    }
    const XYW s = load_xyw(P, v[(k + 1) % 3]), e = load_xyw(P, v[(k + 2) % 3]);
    const float line[3] = {s.y * e.w - s.w * e.y, s.w * e.x - s.x * e.w, s.x * e.y - s.y * e.x};
    const XYW mine = load_xyw(P, v[k]);
    const XYW theirs = load_xyw(P, tri[partner]);  // vertex opposite the partner edge
    if (side(line, mine) * side(line, theirs) > 0.0f) bits |= (uint8_t)(1u << k);
  }
  mask[i] = bits;
}

// ---- crossings --------------------------------------------------------------------------

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
  const float steep = fabsf(T.w[j] * T.y[i] - T.w[i] * T.y[j]) * (float)height * kAxisTie;
  const float flat = fabsf(T.x[j] * T.w[i] - T.x[i] * T.w[j]) * (float)width;
  const bool along = horizontal ? (steep >= flat) : (flat > steep);
  if (!along) return out;
  out.found = true;
  out.t = best;
  out.edge = edge;
  return out;
}

// d t / d (x, y, w) of the two vertices of `edge`, t = e_s / (e_s - e_d) with
// e = a_i c_j - a_j c_i, a = x - px w, c = y - py w. Order: x_i, y_i, w_i, x_j, y_j, w_j.
__device__ __forceinline__ void crossing_grad(const Triangle& T, int edge, float sx, float sy,
                                              float dx, float dy, float (&g)[6]) {
  const int i = (edge + 1) % 3, j = (edge + 2) % 3;
  const float asi = T.x[i] - sx * T.w[i], csi = T.y[i] - sy * T.w[i];
  const float asj = T.x[j] - sx * T.w[j], csj = T.y[j] - sy * T.w[j];
  const float adi = T.x[i] - dx * T.w[i], cdi = T.y[i] - dy * T.w[i];
  const float adj = T.x[j] - dx * T.w[j], cdj = T.y[j] - dy * T.w[j];
  const float es = asi * csj - asj * csi;
  const float ed = adi * cdj - adj * cdi;
  const float span = es - ed;
  const float dt_des = -ed / (span * span);
  const float dt_ded = es / (span * span);
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

struct AAContext {
  const DrAntialiasArgs* a;
};

__device__ __forceinline__ int pixel_tri(const DrAntialiasArgs& a, int64_t pixel, float& depth) {
  const float4 r = load4(a.rast + 4 * pixel);
  depth = r.z;
  const float id = rintf(r.w);
  // Ids past the end of tri are background (reference.py:228-230).
  return (id >= 1.0f && id <= (float)a.num_tri) ? (int)id - 1 : -1;
}

__device__ __forceinline__ void load_triangle(const DrAntialiasArgs& a, int b, int t,
                                              Triangle& T) {
  const float* P = a.pos + (int64_t)b * a.pos_batch_stride;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    T.v[k] = a.tri[3 * (int64_t)t + k];
    const float4 p = load4(P + 4 * (int64_t)T.v[k]);
    T.x[k] = p.x;
    T.y[k] = p.y;
    T.w[k] = p.w;
  }
}

struct Pair {
  bool active;
  bool use_p;      // the first pixel's triangle owns the edge (else the second's)
  float t;         // crossing from the first pixel, in [0, 1]
  int edge;
  Triangle T;      // owner triangle
  float sx, sy, dx, dy;  // owner's source and destination centres
};

// Evaluate the pair (p, q), q = p + (d_row, d_col); ids and depths already loaded.
__device__ __forceinline__ Pair eval_pair(const DrAntialiasArgs& a, int b, int row, int col,
                                          int d_row, int d_col, int id_p, int id_q,
                                          float depth_p, float depth_q) {
  Pair pr;
  pr.active = false;
  if (id_p == id_q) return pr;
  const bool horizontal = d_col == 1;
  const float px = pixel_centre(col, a.width), py = pixel_centre(row, a.height);
  const float qx = pixel_centre(col + d_col, a.width), qy = pixel_centre(row + d_row, a.height);
  const uint8_t* sil = a.silhouette + (int64_t)b * a.silhouette_batch_stride;
  Crossing from_p{false, 0.f, 0}, from_q{false, 0.f, 0};
  Triangle Tp, Tq;
  if (id_p >= 0 && sil[id_p] != 0) {
    load_triangle(a, b, id_p, Tp);
    from_p = crossing(Tp, sil[id_p], horizontal, a.width, a.height, px, py, qx, qy);
  }
  if (id_q >= 0 && sil[id_q] != 0) {
    load_triangle(a, b, id_q, Tq);
    from_q = crossing(Tq, sil[id_q], horizontal, a.width, a.height, qx, qy, px, py);
  }
  const bool use_p = from_p.found && (!from_q.found || depth_p <= depth_q);
  const bool use_q = from_q.found && !use_p;
  if (!use_p && !use_q) return pr;
  pr.active = true;
  pr.use_p = use_p;
  if (use_p) {
    pr.t = from_p.t;
    pr.edge = from_p.edge;
    pr.T = Tp;
    pr.sx = px; pr.sy = py; pr.dx = qx; pr.dy = qy;
  } else {
    pr.t = 1.0f - from_q.t;
    pr.edge = from_q.edge;
    pr.T = Tq;
    pr.sx = qx; pr.sy = qy; pr.dx = px; pr.dy = py;
  }
  return pr;
}

// The four pairs of a pixel: as first pixel with its right and lower neighbours, and as
// second pixel with its left and upper neighbours.
struct Neighbour {
  int d_row, d_col;
  bool first;
};
__constant__ Neighbour kPairs[4] = {{0, 1, true}, {1, 0, true}, {0, -1, false}, {-1, 0, false}};

__global__ __launch_bounds__(256) void aa_fwd_kernel(DrAntialiasArgs a, float* out) {
  const int64_t pixel = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (pixel >= (int64_t)a.batch * a.height * a.width) return;
  const int C = a.channels;
  const int col = (int)(pixel % a.width);
  const int64_t rest = pixel / a.width;
  const int row = (int)(rest % a.height);
  const int b = (int)(rest / a.height);
  const float* color = a.color + pixel * C;
  float* o = out + pixel * C;
  for (int c = 0; c < C; ++c) o[c] = color[c];
  float depth;
  const int id = pixel_tri(a, pixel, depth);
  for (int n = 0; n < 4; ++n) {
    const Neighbour nb = kPairs[n];
    const int r2 = row + nb.d_row, c2 = col + nb.d_col;
    if (r2 < 0 || r2 >= a.height || c2 < 0 || c2 >= a.width) continue;
    const int64_t other = pixel + (int64_t)nb.d_row * a.width + nb.d_col;
    float depth2;
    const int id2 = pixel_tri(a, other, depth2);
    if (id2 == id) continue;
    Pair pr;
    if (nb.first)
      pr = eval_pair(a, b, row, col, nb.d_row, nb.d_col, id, id2, depth, depth2);
    else
      pr = eval_pair(a, b, r2, c2, -nb.d_row, -nb.d_col, id2, id, depth2, depth);
    if (!pr.active) continue;
    const float* color2 = a.color + other * C;
    if (nb.first && pr.t < 0.5f) {
      for (int c = 0; c < C; ++c) o[c] += (0.5f - pr.t) * (color2[c] - color[c]);
    } else if (!nb.first && pr.t >= 0.5f) {
      for (int c = 0; c < C; ++c) o[c] += (pr.t - 0.5f) * (color2[c] - color[c]);
    }
  }
}

__global__ __launch_bounds__(256) void aa_bwd_kernel(DrAntialiasArgs a, const float* grad_out,
                                                       float* grad_color, float* grad_pos) {
  const int64_t pixel = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (pixel >= (int64_t)a.batch * a.height * a.width) return;
  const int C = a.channels;
  const int col = (int)(pixel % a.width);
  const int64_t rest = pixel / a.width;
  const int row = (int)(rest % a.height);
  const int b = (int)(rest / a.height);
  const float* g = grad_out + pixel * C;
  float* gc = grad_color ? grad_color + pixel * C : nullptr;
  if (gc)
    for (int c = 0; c < C; ++c) gc[c] = g[c];
  float depth;
  const int id = pixel_tri(a, pixel, depth);
  const int pos_b = a.pos_batch_stride != 0 ? b : 0;
  for (int n = 0; n < 4; ++n) {
    const Neighbour nb = kPairs[n];
    const int r2 = row + nb.d_row, c2 = col + nb.d_col;
    if (r2 < 0 || r2 >= a.height || c2 < 0 || c2 >= a.width) continue;
    const int64_t other = pixel + (int64_t)nb.d_row * a.width + nb.d_col;
    float depth2;
    const int id2 = pixel_tri(a, other, depth2);
    if (id2 == id) continue;
    Pair pr;
    if (nb.first)
      pr = eval_pair(a, b, row, col, nb.d_row, nb.d_col, id, id2, depth, depth2);
    else
      pr = eval_pair(a, b, r2, c2, -nb.d_row, -nb.d_col, id2, id, depth2, depth);
    if (!pr.active) continue;
    const float* g2 = grad_out + other * C;
    // Pair (P, Q) with P the first pixel. delta_P = (0.5 - t)(c_Q - c_P) when t < 0.5,
    // delta_Q = (t - 0.5)(c_P - c_Q) otherwise.
    const bool low = pr.t < 0.5f;
    if (gc) {
      if (nb.first) {
        if (low) for (int c = 0; c < C; ++c) gc[c] -= (0.5f - pr.t) * g[c];
        else for (int c = 0; c < C; ++c) gc[c] += (pr.t - 0.5f) * g2[c];
      } else {
        if (low) for (int c = 0; c < C; ++c) gc[c] += (0.5f - pr.t) * g2[c];
        else for (int c = 0; c < C; ++c) gc[c] -= (pr.t - 0.5f) * g[c];
      }
    }
    if (!nb.first || grad_pos == nullptr) continue;
    // Position gradient, once per pair from its first pixel.
    const float* cP = a.color + pixel * C;
    const float* cQ = a.color + other * C;
    float g_t = 0.0f;
    if (low) {
      for (int c = 0; c < C; ++c) g_t -= g[c] * (cQ[c] - cP[c]);
    } else {
      for (int c = 0; c < C; ++c) g_t += g2[c] * (cP[c] - cQ[c]);
    }
    g_t *= a.boost;
    if (!pr.use_p) g_t = -g_t;  // t = 1 - t_q
    if (g_t == 0.0f) continue;
    float d[6];
    crossing_grad(pr.T, pr.edge, pr.sx, pr.sy, pr.dx, pr.dy, d);
    float* base = grad_pos + (int64_t)pos_b * a.pos_batch_stride;
    const int vi = pr.T.v[(pr.edge + 1) % 3], vj = pr.T.v[(pr.edge + 2) % 3];
    float* pi = base + 4 * (int64_t)vi;
    float* pj = base + 4 * (int64_t)vj;
    atomic_add(pi + 0, g_t * d[0]);
    atomic_add(pi + 1, g_t * d[1]);
    atomic_add(pi + 3, g_t * d[2]);
    atomic_add(pj + 0, g_t * d[3]);
    atomic_add(pj + 1, g_t * d[4]);
    atomic_add(pj + 3, g_t * d[5]);
  }
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
                                  uint8_t* mask, void* stream) {
  if (pos_batch < 0 || num_tri < 0) return DR_ERR_ARGUMENT;
  const int64_t n = (int64_t)pos_batch * num_tri;
  if (n == 0) return DR_OK;
  if (!pos || !tri || !neighbours || !mask) return DR_ERR_ARGUMENT;
  aa_silhouette_kernel<<<blocks_for(n, 256), 256, 0, (hipStream_t)stream>>>(
      pos, pos_batch_stride, pos_batch, tri, num_tri, neighbours, mask);
  return launch_status();
}

extern "C" int dr_antialias_forward(const DrAntialiasArgs* a, float* out, void* stream) {
  if (!valid_args(a) || !out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0 || a->channels == 0) return DR_OK;
  aa_fwd_kernel<<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(*a, out);
  return launch_status();
}

extern "C" int dr_antialias_backward(const DrAntialiasArgs* a, const float* grad_out,
                                     float* grad_color, float* grad_pos, void* stream) {
  if (!valid_args(a) || !grad_out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  aa_bwd_kernel<<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(
      *a, grad_out, grad_color, grad_pos);
  return launch_status();
}
