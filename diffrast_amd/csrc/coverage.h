// Coverage of a pixel centre by a triangle, and the row spans that bound it.
//
// covers() is the reference backend's test in its own float32 operation order
// (src/diffrast/backends/reference.py:293-365), so that ids match bit for bit. span_setup() and
// row_span() give, for one row of pixel centres, a column range that contains every centre
// covers() can accept: the tile pass only tests those, instead of the triangle's whole box.
//
// The functions are plain C++ on both sides (host and device) so that the bound can be checked
// on the CPU against covers() itself. Sources must be compiled with -ffp-contract=off.
#pragma once

#include <math.h>

#ifdef __HIPCC__
#define DR_HD __host__ __device__ inline
#else
#define DR_HD inline
#endif

namespace dr {

constexpr float kAreaTolerance = 2.384185791015625e-07f;  // 2 * float32 epsilon

struct Tri {
  float x[3], y[3], z[3], w[3];
  float reach_x, reach_y;  // max_k |x_k| + |w_k| and likewise for y (reference.py:321-326)
};

// max_k |a_k| + |w_k|
DR_HD float reach(const float* a, const float* w) {
  return fmaxf(fmaxf(fabsf(a[0]) + fabsf(w[0]), fabsf(a[1]) + fabsf(w[1])),
               fabsf(a[2]) + fabsf(w[2]));
}

// Fill rule of one edge (reference.py:338-365): the value whose sign decides, e itself unless it
// is 0, then the tie-break gx, or gy when gx is 0 too.
DR_HD float tie_broken(float e, float ai, float ci, float wi, float aj, float cj, float wj) {
  if (e != 0.0f) return e;
  const float gx = ci * wj - cj * wi;
  const float gy = aj * wi - ai * wj;
  return (gx == 0.0f) ? gy : gx;
}

// Coverage of pixel centre (px, py) and depth there: the reference's operations in its order
// (reference.py:301-335), one rounding each. The triangle is known to be finite.
DR_HD bool covers(const float* x, const float* y, const float* z, const float* w, float reach_x,
                  float reach_y, float px, float py, float& depth) {
  const float a0 = x[0] - px * w[0];
  const float a1 = x[1] - px * w[1];
  const float a2 = x[2] - px * w[2];
  const float c0 = y[0] - py * w[0];
  const float c1 = y[1] - py * w[1];
  const float c2 = y[2] - py * w[2];
  const float e0 = a1 * c2 - a2 * c1;
  const float e1 = a2 * c0 - a0 * c2;
  const float e2 = a0 * c1 - a1 * c0;
  const float s = e0 + e1 + e2;
  const bool positive = s > 0.0f;
  // An edge passes when its value has the orientation's sign (q > 0 for a positive one, q < 0
  // otherwise: one comparison of q or -q, negation being exact; a zero or NaN q fails). The
  // tie-breaks of edges through the centre are rare: one branch for all three.
  float q0 = e0, q1 = e1, q2 = e2;
  if (e0 == 0.0f || e1 == 0.0f || e2 == 0.0f) {
    q0 = tie_broken(e0, a1, c1, w[1], a2, c2, w[2]);
    q1 = tie_broken(e1, a2, c2, w[2], a0, c0, w[0]);
    q2 = tie_broken(e2, a0, c0, w[0], a1, c1, w[1]);
  }
  const bool in0 = (positive ? q0 : -q0) > 0.0f;
  const bool in1 = (positive ? q1 : -q1) > 0.0f;
  const bool in2 = (positive ? q2 : -q2) > 0.0f;
  if (!(in0 & in1 & in2)) return false;
  const float span_x = fabsf(a0) + fabsf(a1) + fabsf(a2);
  const float span_y = fabsf(c0) + fabsf(c1) + fabsf(c2);
  if (!(fabsf(s) > (reach_x * span_y + span_x * (reach_y + span_y)) * kAreaTolerance))
    return false;
  const float ew = e0 * w[0] + e1 * w[1] + e2 * w[2];
  if (!((positive ? ew : -ew) > 0.0f)) return false;
  depth = (e0 * z[0] + e1 * z[1] + e2 * z[2]) / ew;
  return depth >= -1.0f && depth <= 1.0f;
}

// ---- row spans ------------------------------------------------------------------------------
//
// With a = x - px w and c = y - py w, covers() computes e_k = a_i c_j - a_j c_i for the edges
// (i, j) = (1, 2), (2, 0), (0, 1). In exact arithmetic the px * py terms cancel:
//
//     e_k(px, py) = K_k - py Xw_k - px Wy_k,
//     K_k = x_i y_j - x_j y_i,  Xw_k = x_i w_j - x_j w_i,  Wy_k = w_i y_j - w_j y_i,
//
// a linear function of the pixel centre. Rounding: |a_k| <= reach_x and |c_k| <= reach_y for
// centres inside [-1, 1]^2; a and c carry two roundings each, the products and the difference
// one each, so the computed e_k is within 12 eps reach_x reach_y (eps = 2^-24) of the exact
// value at the same float centre. B = 2^-20 reach_x reach_y bounds that with room to spare.
//
// Orientation: with every w > 0, e_k = w_i w_j f_k with f_k the 2D edge function of the
// projected triangle, and sum_k f_k = 2A (twice its signed area). det = sum_k w_k K_k =
// w0 w1 w2 2A gives the orientation sign S. A centre is only accepted when every computed e_k
// has the sign covers() picked from s = e0 + e1 + e2 (or is 0 under the fill rule). If that sign
// is S, then S e_k >= -B for the exact values. If it is -S, then S f_k <= B / (w_i w_j) for
// every k, whose sum gives |det| <= B (w0 + w1 + w2); so when |det| exceeds that, only the first
// case happens, and every accepted centre satisfies the three linear inequalities
//
//     S e_k(px, py) >= -B,
//
// which, for a fixed row py, bound px from above (S Wy_k > 0) or below (S Wy_k < 0), or accept
// or reject the whole row (Wy_k = 0). Triangles that fail the |det| test, or have some w <= 0,
// get no spans (their whole box is tested).
//
// The coefficients are formed in double: products of two floats are exact there and each
// further operation rounds by 2^-53 relative, some 2^-27 of B, which the slack of B absorbs.
// A bound is then moved to pixel-index space, ix = (px + 1) size / 2 - 1/2, where the float
// pixel centres (rounded twice, within 2^-22 of (2 ix + 1) / size - 1) add at most 2^-23 size;
// the margin is twice that plus 2^-16. An edge whose index-space coefficients exceed 2^30
// (nearly parallel to the rows) is left out: fewer constraints, a wider span.

// Which side an edge bounds is the sign of S_k = sg Wy_k, and with every w > 0 that is the sign
// of Y_j - Y_i (Y = y / w, the projected row coordinate; the float64 Wy_k is a rounded difference
// of exact products, so it keeps the exact sign). The three differences Y_j - Y_i around the
// triangle sum to 0, so at most two edges bound a row from above and at most two from below.

struct RowSpans {
  // Column bounds relative to the column origin x0 given to span_setup(), for the row centre py:
  // col <= hi_u[k] + hi_v[k] * py and col >= lo_u[k] + lo_v[k] * py for k = 0, 1 (+-inf and 0
  // where fewer edges bound that side), and the row is empty when row_u + row_v * py < 0.
  float hi_u[2], hi_v[2], lo_u[2], lo_v[2];
  float row_u, row_v;
};

// Bounds that constrain nothing: every column of every row.
DR_HD void no_spans(RowSpans& s) {
  s.hi_u[0] = s.hi_u[1] = HUGE_VALF;
  s.lo_u[0] = s.lo_u[1] = -HUGE_VALF;
  s.hi_v[0] = s.hi_v[1] = s.lo_v[0] = s.lo_v[1] = 0.0f;
  s.row_u = 1.0f;
  s.row_v = 0.0f;
}

// 1 / S (S finite and non-zero) for the span bounds. On the GPU: the hardware's approximate
// reciprocal and two Newton steps (a relative error far below 2^-50 from any start better than
// 2^-13; a correctly rounded float64 division is some ten float64 instructions); on the host, the
// division. Either is far inside the 2^-21 (|u| + |v|) slack of the bounds.
DR_HD double span_recip(double S) {
#if defined(__HIP_DEVICE_COMPILE__)
  double r = __builtin_amdgcn_rcp(S);
  r = fma(r, fma(-S, r, 1.0), r);
  return fma(r, fma(-S, r, 1.0), r);
#else
  return 1.0 / S;
#endif
}

// Bounds of the row spans of triangle (x, y, w) in an image `width` pixels across, as column
// offsets from x0; false when the triangle gets no spans (s then constrains nothing: the whole
// box is tested). Formed in double, then rounded to float with a margin of 2^-21 (|u| + |v|)
// that covers the rounding of the float evaluation in row_span() (at most about 2 eps
// (|u| + |v|) for |py| <= 1); an edge whose coefficients reach 2^30 is left out.
DR_HD bool span_setup(const float* x, const float* y, const float* w, float reach_x,
                      float reach_y, int width, int x0, RowSpans& s) {
  no_spans(s);
  if (!(w[0] > 0.0f && w[1] > 0.0f && w[2] > 0.0f)) return false;
  double K[3], Xw[3], Wy[3];
  for (int k = 0; k < 3; ++k) {
    const int i = k == 2 ? 0 : k + 1, j = k == 0 ? 2 : k - 1;
    K[k] = (double)x[i] * (double)y[j] - (double)x[j] * (double)y[i];
    Xw[k] = (double)x[i] * (double)w[j] - (double)x[j] * (double)w[i];
    Wy[k] = (double)w[i] * (double)y[j] - (double)w[j] * (double)y[i];
  }
  const double B = ldexp((double)reach_x * (double)reach_y, -20);
  const double det = (double)w[0] * K[0] + (double)w[1] * K[1] + (double)w[2] * K[2];
  if (!(fabs(det) > 1.25 * B * ((double)w[0] + (double)w[1] + (double)w[2]))) return false;
  const double sg = det > 0.0 ? 1.0 : -1.0;
  const double half = 0.5 * (double)width;
  const double m = ldexp((double)width, -22) + 0x1p-16;
  RowSpans t;
  no_spans(t);
  int highs = 0, lows = 0;
  for (int k = 0; k < 3; ++k) {
    const double S = sg * Wy[k], U = sg * K[k] + B, V = -sg * Xw[k];
    if (S == 0.0) {  // at most one edge: two would make the triangle degenerate
      t.row_u = (float)(U + ldexp(fabs(U) + fabs(V), -21));
      t.row_v = (float)V;
      continue;
    }
    const double inv = span_recip(S);
    const double u = (U * inv + 1.0) * half - 0.5 - (double)x0, v = V * inv * half;
    if (!(fabs(u) < 0x1p30 && fabs(v) < 0x1p30)) continue;
    const double slack = m + ldexp(fabs(u) + fabs(v), -21);
    // A third bound on one side would contradict the sign argument above; were it ever to
    // happen, the triangle would get no spans (its whole box tested), never a wrong one.
    // (Slots by constant index: a run-time index would put t in scratch memory on the GPU.)
    if (S > 0.0) {
      if (highs == 2) return false;
      const float bu = (float)(u + slack), bv = (float)v;
      if (highs++ == 0) {
        t.hi_u[0] = bu;
        t.hi_v[0] = bv;
      } else {
        t.hi_u[1] = bu;
        t.hi_v[1] = bv;
      }
    } else {
      if (lows == 2) return false;
      const float bu = (float)(u - slack), bv = (float)v;
      if (lows++ == 0) {
        t.lo_u[0] = bu;
        t.lo_v[0] = bv;
      } else {
        t.lo_u[1] = bu;
        t.lo_v[1] = bv;
      }
    }
  }
  s = t;
  return true;
}

// Column offsets of row centre py (float, as covers() gets it) that may be covered, clipped to
// [lo, hi] as given (floats holding integers): on return lo = the first, hi = the last, both
// integers within the given range when lo <= hi; lo > hi for none.
DR_HD void row_bounds(const RowSpans& s, float py, float& lo, float& hi) {
  const float h =
      fminf(fminf(fmaf(s.hi_v[0], py, s.hi_u[0]), fmaf(s.hi_v[1], py, s.hi_u[1])), hi);
  const float l =
      fmaxf(fmaxf(fmaf(s.lo_v[0], py, s.lo_u[0]), fmaf(s.lo_v[1], py, s.lo_u[1])), lo);
  const bool row = !(fmaf(s.row_v, py, s.row_u) < 0.0f);
  lo = ceilf(l);
  hi = row ? floorf(h) : -HUGE_VALF;
}

// The same in integers: [lo, hi] clipped to the given range (|lo|, |hi| < 2^24); lo > hi for none.
DR_HD void row_span(const RowSpans& s, float py, int& lo, int& hi) {
  float l = (float)lo, h = (float)hi;
  row_bounds(s, py, l, h);
  if (l <= h) {
    lo = (int)l;
    hi = (int)h;
  } else {
    lo = 1;
    hi = 0;
  }
}

}  // namespace dr
