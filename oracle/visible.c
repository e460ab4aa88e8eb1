/*
 * Brute-force visibility at a list of pixels, in plain C: TEST INFRASTRUCTURE (part of the
 * oracle), never part of the product.
 *
 * A restatement of the reference backend's visibility (src/diffrast/backends/reference.py:
 * _coverage :293-335, _inside_edge :338-365, _visible_triangles :368-397, pixel centres
 * :268-271) evaluated at chosen pixels only, like oracle/reference.py: visible_at, but fast
 * enough to test every triangle of a 1.3M-triangle mesh at thousands of pixels. Each float
 * operation is one rounded IEEE float32 operation in the reference's order: build with
 * -ffp-contract=off and without -ffast-math (no fused multiply-add, no reassociation, IEEE
 * division, denormals kept), as oracle/Makefile does. The per-pixel loop is branch-free so that
 * the compiler runs it on vector lanes, which round exactly as scalar float32 operations do.
 *
 * Pinned by tests/test_oracle_native.py: equal, pixel for pixel and bit for bit in depth, to
 * oracle/reference.py (visible_triangles, visible_at) on random, camera-plane-crossing,
 * degenerate, non-finite, sliver and exact-tie meshes over several peel layers, and to the ids
 * of the golden vectors the reference wrote (tests/golden/raster.npz).
 */
#include <math.h>
#include <stdint.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* reference.py:27 -- a pixel is not drawn where the area is within this many epsilons. */
#define AREA_TOLERANCE 2.0f

/* Pixels per work block: every triangle is set up once per block. */
#define BLOCK 256

/* Pixel centre (2i + 1) / size - 1 as the reference computes it in float32
 * (reference.py:268-271). */
static float centre(int i, int size) {
  const float k = (float)(2 * i + 1);
  return k / (float)size - 1.0f;
}

/* _inside_edge (reference.py:338-365): e, or where it is exactly zero the sign of the
 * screen-space gradient (ci wj - cj wi, aj wi - ai wj), x first. */
static inline int inside_edge(float e, float ai, float ci, float wi, float aj, float cj,
                              float wj, int positive) {
  const float gx = ci * wj - cj * wi;
  const float gy = aj * wi - ai * wj;
  const float tie = gx == 0.0f ? gy : gx;
  const float decided = e == 0.0f ? tie : e;
  return (positive & (decided > 0.0f)) | ((positive ^ 1) & (decided < 0.0f));
}

typedef struct {
  float x[3], y[3], z[3], w[3];
  float reach_x, reach_y;
} Corners;

/* The corners of triangle t of image b; 0 when a coordinate is not finite (such a triangle
 * covers nothing, reference.py:330-334). */
static int corners(const float* pos, int64_t pos_batch_stride, const int32_t* tri, int64_t t,
                   int b, Corners* out) {
  const float* image = pos + (int64_t)b * pos_batch_stride;
  for (int k = 0; k < 3; ++k) {
    const float* v = image + 4 * (int64_t)tri[3 * t + k];
    out->x[k] = v[0];
    out->y[k] = v[1];
    out->z[k] = v[2];
    out->w[k] = v[3];
    if (!isfinite(v[0]) || !isfinite(v[1]) || !isfinite(v[2]) || !isfinite(v[3])) return 0;
  }
  /* max(max(|x0| + |w0|, |x1| + |w1|), |x2| + |w2|), likewise for y. */
  out->reach_x = fmaxf(fmaxf(fabsf(out->x[0]) + fabsf(out->w[0]),
                             fabsf(out->x[1]) + fabsf(out->w[1])),
                       fabsf(out->x[2]) + fabsf(out->w[2]));
  out->reach_y = fmaxf(fmaxf(fabsf(out->y[0]) + fabsf(out->w[0]),
                             fabsf(out->y[1]) + fabsf(out->w[1])),
                       fabsf(out->y[2]) + fabsf(out->w[2]));
  return 1;
}

/* _coverage (reference.py:293-335) of one triangle at the pixel centres [start, end) of a
 * block, merged into the block's nearest (depth, index) by the rules of _visible_triangles
 * (reference.py:368-397): only a strictly nearer depth replaces, so equal depths keep the lower
 * index; with a previous layer only (depth, index) pairs after it count. Each line is one
 * rounded float32 operation in the reference's order (left to right within a line). */
/* Compiled twice, for AVX2 (8 lanes, chosen at load time where the host has it; AVX2 has no
 * fused multiply-add, and contraction is off anyway) and for the baseline x86-64. */
__attribute__((target_clones("avx2", "default"))) static void merge_triangle(
    const Corners* c, int32_t t, int start, int end, const float* restrict px,
    const float* restrict py, const float* restrict pd, const int32_t* restrict pid,
    float* restrict best, int32_t* restrict best_id) {
  const float x0 = c->x[0], x1 = c->x[1], x2 = c->x[2];
  const float y0 = c->y[0], y1 = c->y[1], y2 = c->y[2];
  const float z0 = c->z[0], z1 = c->z[1], z2 = c->z[2];
  const float w0 = c->w[0], w1 = c->w[1], w2 = c->w[2];
  const float reach_x = c->reach_x, reach_y = c->reach_y;
  /* AREA_TOLERANCE * float32 epsilon = 2^-22, a power of two: the product is the same whether
   * the scalar is applied in float or in double and rounded. */
  const float scale = AREA_TOLERANCE * 1.1920928955078125e-07f;
  for (int i = start; i < end; ++i) {
    const float a0 = x0 - px[i] * w0;
    const float a1 = x1 - px[i] * w1;
    const float a2 = x2 - px[i] * w2;
    const float c0 = y0 - py[i] * w0;
    const float c1 = y1 - py[i] * w1;
    const float c2 = y2 - py[i] * w2;
    const float e0 = a1 * c2 - a2 * c1;
    const float e1 = a2 * c0 - a0 * c2;
    const float e2 = a0 * c1 - a1 * c0;
    const float area = e0 + e1 + e2;
    const float ew = e0 * w0 + e1 * w1 + e2 * w2;
    const float depth = (e0 * z0 + e1 * z1 + e2 * z2) / ew;
    const int positive = area > 0.0f;
    int ok = inside_edge(e0, a1, c1, w1, a2, c2, w2, positive);
    ok &= inside_edge(e1, a2, c2, w2, a0, c0, w0, positive);
    ok &= inside_edge(e2, a0, c0, w0, a1, c1, w1, positive);
    const float span_x = fabsf(a0) + fabsf(a1) + fabsf(a2);
    const float span_y = fabsf(c0) + fabsf(c1) + fabsf(c2);
    const float tolerance = (reach_x * span_y + span_x * (reach_y + span_y)) * scale;
    ok &= fabsf(area) > tolerance;
    ok &= (positive & (ew > 0.0f)) | ((positive ^ 1) & (ew < 0.0f));
    ok &= (depth >= -1.0f) & (depth <= 1.0f);
    /* Without a previous layer pd is -inf: every depth that passed the range test is after it. */
    ok &= (depth > pd[i]) | ((depth == pd[i]) & (t > pid[i]));
    const int nearer = ok & (depth < best[i]);
    best[i] = nearer ? depth : best[i];
    best_id[i] = nearer ? t : best_id[i];
  }
}

/*
 * _visible_triangles (reference.py:368-397) at n pixels (b[i], row[i], col[i]) of images of
 * height x width: the nearest covering triangle by (depth, index), ties to the lower index;
 * with prev_depth/prev_id (nullable) only triangles ordered after that pair count (a depth
 * layer behind it). pos is [batch, vertices, 4] with pos_batch_stride floats between images (0:
 * one image for all); tri is [num_tri, 3] with valid rows (num_tri < 2^31). Writes depth (+inf
 * where nothing covers) and id (-1 there). Pixels of one image should be listed together (runs
 * of one image share the triangle set-up); the result does not depend on the order.
 * threads <= 0: the OpenMP default. Returns 0, or -1 for an argument out of range.
 */
int oracle_visible_at(const float* pos, int64_t pos_batch_stride, const int32_t* tri,
                      int64_t num_tri, int height, int width, int64_t n, const int32_t* b,
                      const int32_t* row, const int32_t* col, const float* prev_depth,
                      const int64_t* prev_id, float* depth, int64_t* id, int threads) {
  if (n < 0 || num_tri < 0 || num_tri >= INT32_MAX || height <= 0 || width <= 0) return -1;
  for (int64_t i = 0; i < n; ++i)
    if (row[i] < 0 || row[i] >= height || col[i] < 0 || col[i] >= width || b[i] < 0) return -1;
  const int64_t blocks = (n + BLOCK - 1) / BLOCK;
  const int peel = prev_depth != 0 && prev_id != 0;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
  for (int64_t blk = 0; blk < blocks; ++blk) {
    const int64_t first = blk * BLOCK;
    const int count = (int)(n - first < BLOCK ? n - first : BLOCK);
    float px[BLOCK], py[BLOCK], best[BLOCK], pd[BLOCK];
    int32_t best_id[BLOCK], pid[BLOCK];
    int image[BLOCK];
    for (int i = 0; i < count; ++i) {
      px[i] = centre(col[first + i], width);
      py[i] = centre(row[first + i], height);
      best[i] = INFINITY;
      best_id[i] = -1;
      image[i] = b[first + i];
      pd[i] = peel ? prev_depth[first + i] : -INFINITY;
      /* Clamped into int32: below -1 or beyond the last triangle orders alike. */
      const int64_t p = peel ? prev_id[first + i] : 0;
      pid[i] = (int32_t)(p < -1 ? -1 : p > num_tri ? num_tri : p);
    }
    /* Runs of pixels of one image share the triangle set-up. */
    int start = 0;
    while (start < count) {
      int end = start + 1;
      while (end < count && image[end] == image[start]) ++end;
      for (int64_t t = 0; t < num_tri; ++t) {
        Corners c;
        if (!corners(pos, pos_batch_stride, tri, t, image[start], &c)) continue;
        merge_triangle(&c, (int32_t)t, start, end, px, py, pd, pid, best, best_id);
      }
      start = end;
    }
    for (int i = 0; i < count; ++i) {
      depth[first + i] = best[i];
      id[first + i] = best_id[i];
    }
  }
  return 0;
}
