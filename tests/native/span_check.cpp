// Soundness of the row spans: every pixel centre that covers() accepts lies inside the span
// that row_span() gives for its row. Triangles of many shapes (slivers, near-horizontal and
// exactly horizontal edges, vertices on pixel centres, large or tiny w, vertices far off
// screen) are drawn at several image sizes; every centre of a window around each triangle is
// tested. Prints "ok <checks> <accepted> <span pixels>" or the first failing case.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "../../diffrast_amd/csrc/coverage.h"

using namespace dr;

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static uint64_t next_u64() {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return rng_state;
}
static double uniform(double a, double b) { return a + (b - a) * (double)(next_u64() >> 11) * 0x1p-53; }
static int pick(int n) { return (int)(next_u64() % (uint64_t)n); }

static float centre(int i, int size) { return (float)(2 * i + 1) / (float)size - 1.0f; }

// A triangle that gets no spans (a vertex at or behind the camera plane, or too thin for the
// orientation bound) must leave every column of every row to the box: row_span() returns the
// range it was given.
static int check_without_spans() {
  const float cases[3][3][3] = {
      {{-0.2f, 0.1f, 1.0f}, {0.3f, -0.4f, 0.0f}, {0.5f, 0.5f, 2.0f}},     // w = 0 at a vertex
      {{0.1f, 0.2f, 1.0f}, {0.4f, 0.1f, -1.0f}, {-0.3f, -0.2f, 1.5f}},    // w < 0 at a vertex
      {{0.1f, 0.1f, 1.0f}, {0.2f, 0.2f, 1.0f}, {0.3f, 0.3f, 1.0f}},       // collinear: no area
  };
  for (int c = 0; c < 3; ++c) {
    float x[3], y[3], w[3];
    for (int k = 0; k < 3; ++k) {
      x[k] = cases[c][k][0] * cases[c][k][2];
      y[k] = cases[c][k][1] * cases[c][k][2];
      w[k] = cases[c][k][2];
    }
    RowSpans s;
    if (span_setup(x, y, w, reach(x, w), reach(y, w), 64, 16, s)) {
      printf("case %d without spans got spans\n", c);
      return 1;
    }
    for (int r = 0; r < 64; ++r) {
      int lo = 3, hi = 11;
      row_span(s, centre(r, 64), lo, hi);
      if (lo != 3 || hi != 11) {
        printf("case %d row %d without spans: [%d, %d] instead of [3, 11]\n", c, r, lo, hi);
        return 1;
      }
    }
  }
  return 0;
}

int main(int argc, char** argv) {
  if (check_without_spans() != 0) return 1;
  const long triangles = argc > 1 ? atol(argv[1]) : 200000;
  const int sizes[] = {16, 37, 64, 256, 1024, 4096};
  long checks = 0, accepted = 0, span_pixels = 0, with_spans = 0;
  for (long n = 0; n < triangles; ++n) {
    const int width = sizes[pick(6)], height = sizes[pick(6)];
    float X[3], Y[3], W[3];
    const int shape = pick(8);
    const double size = shape == 6 ? uniform(0.0, 4.0 / width) : uniform(0.001, 0.6);
    const double cx = uniform(-1.1, 1.1), cy = uniform(-1.1, 1.1);
    for (int k = 0; k < 3; ++k) {
      X[k] = (float)(cx + uniform(-size, size));
      Y[k] = (float)(cy + uniform(-size, size));
      W[k] = (float)uniform(0.5, 3.0);
    }
    if (shape == 1) {  // sliver: third vertex near the line through the first two
      const double t = uniform(-0.5, 1.5), off = uniform(-1e-3, 1e-3) * size;
      X[2] = (float)(X[0] + t * (X[1] - X[0]) + off);
      Y[2] = (float)(Y[0] + t * (Y[1] - Y[0]) - off);
    } else if (shape == 2) {  // exactly horizontal or vertical edge
      if (pick(2)) Y[1] = Y[0]; else X[1] = X[0];
    } else if (shape == 3) {  // nearly horizontal edge
      Y[1] = (float)(Y[0] + uniform(-1e-6, 1e-6));
    } else if (shape == 4) {  // vertices on pixel centres
      for (int k = 0; k < 3; ++k) {
        X[k] = centre(pick(width), width);
        Y[k] = centre(pick(height), height);
      }
    } else if (shape == 5) {  // vertices far off screen
      for (int k = 0; k < 3; ++k) {
        X[k] = (float)uniform(-40.0, 40.0);
        Y[k] = (float)uniform(-40.0, 40.0);
      }
    } else if (shape == 7) {  // strong perspective
      for (int k = 0; k < 3; ++k) W[k] = (float)(pick(2) ? uniform(0.01, 0.05) : uniform(20.0, 100.0));
    }
    Tri T;
    for (int k = 0; k < 3; ++k) {
      T.x[k] = X[k] * W[k];
      T.y[k] = Y[k] * W[k];
      T.z[k] = (float)uniform(-0.9, 0.9) * W[k];
      T.w[k] = W[k];
    }
    T.reach_x = reach(T.x, T.w);
    T.reach_y = reach(T.y, T.w);
    RowSpans s;
    const int x0 = pick(width);  // column origin, as a tile's
    if (!span_setup(T.x, T.y, T.w, T.reach_x, T.reach_y, width, x0, s)) continue;
    ++with_spans;
    // A window of at most 160 x 160 centres around the projected box.
    double lo_x = 1e9, hi_x = -1e9, lo_y = 1e9, hi_y = -1e9;
    for (int k = 0; k < 3; ++k) {
      const double px = ((double)X[k] + 1.0) * 0.5 * width - 0.5, py = ((double)Y[k] + 1.0) * 0.5 * height - 0.5;
      lo_x = px < lo_x ? px : lo_x; hi_x = px > hi_x ? px : hi_x;
      lo_y = py < lo_y ? py : lo_y; hi_y = py > hi_y ? py : hi_y;
    }
    int c0 = (int)(lo_x - 2), c1 = (int)(hi_x + 3), y0 = (int)(lo_y - 2), y1 = (int)(hi_y + 3);
    c0 = c0 < 0 ? 0 : c0; y0 = y0 < 0 ? 0 : y0;
    c1 = c1 > width - 1 ? width - 1 : c1; y1 = y1 > height - 1 ? height - 1 : y1;
    if (c1 - c0 > 159) { c0 += pick(c1 - c0 - 159); c1 = c0 + 159; }
    if (y1 - y0 > 159) { y0 += pick(y1 - y0 - 159); y1 = y0 + 159; }
    for (int iy = y0; iy <= y1; ++iy) {
      const float py = centre(iy, height);
      int lo = c0 - x0, hi = c1 - x0;
      row_span(s, py, lo, hi);
      lo += x0;
      hi += x0;
      if (lo <= hi) span_pixels += hi - lo + 1;
      for (int ix = c0; ix <= c1; ++ix) {
        float depth;
        ++checks;
        if (!covers(T.x, T.y, T.z, T.w, T.reach_x, T.reach_y, centre(ix, width), py, depth)) continue;
        ++accepted;
        if (ix < lo || ix > hi) {
          printf("miss triangle %ld shape %d size %dx%d pixel (%d, %d) span [%d, %d]\n", n, shape, width, height, ix, iy, lo, hi);
          for (int k = 0; k < 3; ++k) printf("  v%d %.9g %.9g %.9g\n", k, T.x[k], T.y[k], T.w[k]);
          return 1;
        }
      }
    }
  }
  printf("ok %ld %ld %ld %ld\n", checks, accepted, span_pixels, with_spans);
  return 0;
}
