// Per-pixel arithmetic of a texture lookup, for float32 (the product kernels) and float64 (the
// gradient-check kernels), shared by texture.hip and f64.hip.
//
// It follows the reference backend: texel coordinates and boundaries
// (src/diffrast/backends/reference.py:555-672), level of detail and level blending
// (reference.py:491-501, 522-552), cube-map projection and the integer edge fold
// (src/diffrast/backends/_cube.py:44-143). S is the scalar type; the arrays of DrTextureArgs
// (texels, uv, uv_da, bias) hold S values. With S = float every expression is the single
// float32 operation it was written as (sources are compiled with -ffp-contract=off).
#pragma once

#include <float.h>

#include <type_traits>

#include "common.h"

namespace dr {
namespace tex {
namespace {  // internal linkage: each source that includes this has its own copy

// ---- scalar helpers ---------------------------------------------------------------------------

template <class S>
__device__ __forceinline__ const S* as(const float* p) {
  return reinterpret_cast<const S*>(p);
}
template <class S>
__device__ __forceinline__ S s_floor(S x) {
  if constexpr (std::is_same_v<S, float>) return floorf(x); else return floor(x);
}
template <class S>
__device__ __forceinline__ S s_abs(S x) {
  if constexpr (std::is_same_v<S, float>) return fabsf(x); else return fabs(x);
}
template <class S>
__device__ __forceinline__ S s_min(S a, S b) {
  if constexpr (std::is_same_v<S, float>) return fminf(a, b); else return fmin(a, b);
}
template <class S>
__device__ __forceinline__ S s_max(S a, S b) {
  if constexpr (std::is_same_v<S, float>) return fmaxf(a, b); else return fmax(a, b);
}
template <class S>
__device__ __forceinline__ S s_log2(S x) {
  if constexpr (std::is_same_v<S, float>) return log2f(x); else return log2(x);
}
template <class S>
__device__ __forceinline__ S s_nan() {
  if constexpr (std::is_same_v<S, float>) return __int_as_float(0x7fc00000);
  else return __longlong_as_double(0x7ff8000000000000ll);
}
// Smallest normal value of S (torch.finfo(dtype).tiny, _cube.py:67).
template <class S>
__device__ __forceinline__ S s_tiny() {
  if constexpr (std::is_same_v<S, float>) return 1.17549435e-38f; else return DBL_MIN;
}

template <class S> constexpr S kFootprintLimit = S(1e18);   // reference.py:402
template <class S> constexpr S kDerivativeLimit = S(1e18);  // _cube.py:36
template <class S> constexpr S kMinFootprint = S(1e-30);    // reference.py:501
template <class S> constexpr S kLn2 = S(0.693147180559945309417232121458176568);

// ---- cube geometry (_cube.py) -------------------------------------------------------------------

// Per face: major axis, s axis and t axis as integer 3-vectors (_cube.py:31-33).
__constant__ int kMajor[6][3] = {{1, 0, 0}, {-1, 0, 0}, {0, 1, 0}, {0, -1, 0}, {0, 0, 1}, {0, 0, -1}};
__constant__ int kSAxis[6][3] = {{0, 0, -1}, {0, 0, 1}, {1, 0, 0}, {1, 0, 0}, {1, 0, 0}, {-1, 0, 0}};
__constant__ int kTAxis[6][3] = {{0, -1, 0}, {0, -1, 0}, {0, 0, 1}, {0, 0, -1}, {0, -1, 0}, {0, -1, 0}};

__device__ __forceinline__ int floor_div2(int v) { return v >= 0 ? v / 2 : -((-v + 1) / 2); }

// Fold a texel one step outside its face onto the neighbouring face (_cube.py:105-143).
// Returns false beyond a corner, where no texel exists.
__device__ __forceinline__ bool cube_fold(int& face, int& row, int& col, int size) {
  const bool over_col = col < 0 || col >= size;
  const bool over_row = row < 0 || row >= size;
  const int sc = 2 * col + 1 - size, tc = 2 * row + 1 - size;
  int point[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    int p = size * kMajor[face][k] + sc * kSAxis[face][k] + tc * kTAxis[face][k];
    p = min(max(p, -size), size);
    if (over_col || over_row) p -= kMajor[face][k];
    point[k] = p;
  }
  int axis = 0;
  int best = abs(point[0]);
  if (abs(point[1]) > best) { axis = 1; best = abs(point[1]); }
  if (abs(point[2]) > best) axis = 2;
  face = 2 * axis + (point[axis] < 0 ? 1 : 0);
  int s_dot = 0, t_dot = 0;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    s_dot += point[k] * kSAxis[face][k];
    t_dot += point[k] * kTAxis[face][k];
  }
  col = max(floor_div2(s_dot + size - 1), 0);
  row = max(floor_div2(t_dot + size - 1), 0);
  return !(over_col && over_row);
}

template <class S>
struct CubeProj {
  bool valid, undefined;
  int face;
  S length, ma, rs, rt;
  S dn[3];
  S da[3][2];           // clamped, scaled derivatives
  bool da_pass[3][2];   // inside the clamp
  S d_ma[2], d_sc[2], d_tc[2];
  S st[2];
  S st_da[4];           // ds/dx, ds/dy, dt/dx, dt/dy
};

// Face selection and face coordinates of a direction (_cube.py:44-102).
template <class S>
__device__ __forceinline__ void cube_project(const S* dir, const S* dir_da, CubeProj<S>& P) {
  S d[3] = {dir[0], dir[1], dir[2]};
  const S ax0 = s_abs(d[0]), ay0 = s_abs(d[1]), az0 = s_abs(d[2]);
  P.valid = isfinite(d[0]) && isfinite(d[1]) && isfinite(d[2]) &&
            s_max(s_max(ax0, ay0), az0) >= s_tiny<S>();
  if (!P.valid) {
    d[0] = S(0);
    d[1] = S(0);
    d[2] = S(1);
  }
  const S ax = s_abs(d[0]), ay = s_abs(d[1]), az = s_abs(d[2]);
  const bool x_major = ax >= ay && ax >= az;
  const bool y_major = !x_major && ay >= az;
  const int axis = x_major ? 0 : (y_major ? 1 : 2);
  P.face = 2 * axis + (d[axis] < S(0) ? 1 : 0);
  P.length = s_max(s_max(ax, ay), az);
#pragma unroll
  for (int k = 0; k < 3; ++k) P.dn[k] = d[k] / P.length;
  const int* M = kMajor[P.face];
  const int* A = kSAxis[P.face];
  const int* T = kTAxis[P.face];
  P.ma = P.dn[0] * (S)M[0] + P.dn[1] * (S)M[1] + P.dn[2] * (S)M[2];
  const S sc = P.dn[0] * (S)A[0] + P.dn[1] * (S)A[1] + P.dn[2] * (S)A[2];
  const S tc = P.dn[0] * (S)T[0] + P.dn[1] * (S)T[1] + P.dn[2] * (S)T[2];
  P.rs = sc / P.ma;
  P.rt = tc / P.ma;
  P.st[0] = S(0.5) * (P.rs + S(1));
  P.st[1] = S(0.5) * (P.rt + S(1));
  P.undefined = false;
  if (dir_da == nullptr) return;
  bool any_nan = false;
  for (int i = 0; i < 6; ++i) any_nan = any_nan || isnan(dir_da[i]);
  P.undefined = P.valid && any_nan;
  const bool use = P.valid && !P.undefined;
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const S v = (use ? dir_da[2 * k + j] : S(0)) / P.length;
      P.da_pass[k][j] = v >= -kDerivativeLimit<S> && v <= kDerivativeLimit<S>;
      P.da[k][j] = s_min(s_max(v, -kDerivativeLimit<S>), kDerivativeLimit<S>);
    }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    P.d_ma[j] = P.da[0][j] * (S)M[0] + P.da[1][j] * (S)M[1] + P.da[2][j] * (S)M[2];
    P.d_sc[j] = P.da[0][j] * (S)A[0] + P.da[1][j] * (S)A[1] + P.da[2][j] * (S)A[2];
    P.d_tc[j] = P.da[0][j] * (S)T[0] + P.da[1][j] * (S)T[1] + P.da[2][j] * (S)T[2];
  }
  const S nan = s_nan<S>();
  P.st_da[0] = P.undefined ? nan : S(0.5) * (P.d_sc[0] - P.rs * P.d_ma[0]) / P.ma;
  P.st_da[1] = P.undefined ? nan : S(0.5) * (P.d_sc[1] - P.rs * P.d_ma[1]) / P.ma;
  P.st_da[2] = P.undefined ? nan : S(0.5) * (P.d_tc[0] - P.rt * P.d_ma[0]) / P.ma;
  P.st_da[3] = P.undefined ? nan : S(0.5) * (P.d_tc[1] - P.rt * P.d_ma[1]) / P.ma;
}

// Gradient of cube_project: from d(loss)/d(st) and d(loss)/d(st_da) to the direction and
// its derivatives (3 and 6 values); g_sda is used when use_sda is set.
template <class S>
__device__ __forceinline__ void cube_project_backward(const CubeProj<S>& P, S g_s, S g_t,
                                                      bool use_sda, const S (&g_sda)[4],
                                                      S (&grad_dir)[3], S (&grad_dir_da)[6]) {
  const int* M = kMajor[P.face];
  const int* A = kSAxis[P.face];
  const int* T = kTAxis[P.face];
  // Gradient only: multiplies by the reciprocals (two divisions instead of 25; each product
  // is within two ulp of the quotient).
  const S inv_ma = S(1) / P.ma, inv_length = S(1) / P.length;
  S g_rs = S(0.5) * g_s, g_rt = S(0.5) * g_t, g_ma = S(0);
  S g_dsc[2] = {S(0), S(0)}, g_dtc[2] = {S(0), S(0)}, g_dma[2] = {S(0), S(0)};
  if (use_sda && !P.undefined) {
    const S gds[2] = {g_sda[0], g_sda[1]}, gdt[2] = {g_sda[2], g_sda[3]};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const S ds = P.st_da[j], dt = P.st_da[2 + j];
      g_rs += gds[j] * (S(-0.5) * P.d_ma[j] * inv_ma);
      g_rt += gdt[j] * (S(-0.5) * P.d_ma[j] * inv_ma);
      g_ma -= (gds[j] * ds + gdt[j] * dt) * inv_ma;
      g_dsc[j] = S(0.5) * gds[j] * inv_ma;
      g_dtc[j] = S(0.5) * gdt[j] * inv_ma;
      g_dma[j] = S(-0.5) * (gds[j] * P.rs + gdt[j] * P.rt) * inv_ma;
    }
  }
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      S g = g_dsc[j] * (S)A[k] + g_dtc[j] * (S)T[k] + g_dma[j] * (S)M[k];
      g = (P.valid && !P.undefined && P.da_pass[k][j]) ? g * inv_length : S(0);
      grad_dir_da[2 * k + j] = g;
    }
  g_ma -= (g_rs * P.rs + g_rt * P.rt) * inv_ma;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const S g_dn = (g_rs * (S)A[k] + g_rt * (S)T[k]) * inv_ma + g_ma * (S)M[k];
    grad_dir[k] = P.valid ? g_dn * inv_length : S(0);
  }
}

// ---- 2D coordinates, taps and levels ----------------------------------------------------------

template <class S>
struct Axis {
  S x;         // continuous texel coordinate
  bool bad;    // not finite (then x = 0)
  bool pass;   // gradient reaches the input coordinate
};

// coord * size - shift, wrapped or saturated as for the boundary (reference.py:615-633).
template <class S>
__device__ __forceinline__ Axis<S> texel_axis(S coord, int size, S shift, int boundary) {
  Axis<S> A;
  S c = coord;
  if (boundary == DR_BOUNDARY_WRAP) c = c - s_floor(c);
  A.x = c * (S)size - shift;
  A.pass = true;
  if (boundary == DR_BOUNDARY_CLAMP || boundary == DR_BOUNDARY_ZERO) {
    if (A.x < S(-1)) { A.x = S(-1); A.pass = false; }
    if (A.x > (S)size) { A.x = (S)size; A.pass = false; }
  }
  A.bad = !isfinite(A.x);
  if (A.bad) {
    A.x = S(0);
    A.pass = false;
  }
  return A;
}

// i mod n (non-negative). Tap positions come from coordinates already wrapped into [0, 1], so
// they lie in [-1, n]: one add or subtract; the division is left for anything else.
__device__ __forceinline__ int wrap_index(int i, int n) {
  int r = i < 0 ? i + n : (i >= n ? i - n : i);
  if (r < 0 || r >= n) {
    r = i % n;
    r = r < 0 ? r + n : r;
  }
  return r;
}

// Texel index (in texels from the start of the image's packed buffer, which holds fewer than
// 2^32 texels) of integer tap (row, col) of a level; false when the tap reads zero
// (reference.py:636-672).
__device__ __forceinline__ bool tap(int row, int col, int face, int h, int w, int64_t offset,
                                    int boundary, uint32_t& index) {
  bool valid = true;
  if (boundary == DR_BOUNDARY_CUBE) {
    valid = cube_fold(face, row, col, w);
  } else if (boundary == DR_BOUNDARY_WRAP) {
    row = wrap_index(row, h);
    col = wrap_index(col, w);
  } else {
    if (boundary == DR_BOUNDARY_ZERO) valid = row >= 0 && row < h && col >= 0 && col < w;
    row = min(max(row, 0), h - 1);
    col = min(max(col, 0), w - 1);
  }
  if (face >= 0) row += face * h;
  index = (uint32_t)offset + (uint32_t)row * (uint32_t)w + (uint32_t)col;
  return valid;
}

// Rows (or columns) i and i + 1 of a level n texels long under a 2D boundary: wrapped or
// clamped into [0, n), and whether each reads a texel (as tap() decides for each tap; the
// four taps of a bilinear lookup combine two of each).
struct AxisPair {
  int at[2];
  bool valid[2];
};

__device__ __forceinline__ AxisPair axis_pair(int i, int n, int boundary) {
  AxisPair p;
  if (boundary == DR_BOUNDARY_WRAP) {
    p.at[0] = wrap_index(i, n);
    p.at[1] = p.at[0] + 1 == n ? 0 : p.at[0] + 1;  // (i + 1) mod n
    p.valid[0] = p.valid[1] = true;
  } else {
    const bool zero = boundary == DR_BOUNDARY_ZERO;
    p.valid[0] = !zero || (i >= 0 && i < n);
    p.valid[1] = !zero || (i + 1 >= 0 && i + 1 < n);
    p.at[0] = min(max(i, 0), n - 1);
    p.at[1] = min(max(i + 1, 0), n - 1);
  }
  return p;
}

template <class S>
struct Bilinear {
  uint32_t index[4];  // texels from the start of the image's packed buffer (tap())
  bool valid[4];
  S fx, fy;
  bool bad;
  bool pass_x, pass_y;
  S size_x, size_y;
  // Cube corners: taps beyond two edges count as the mean of the other three.
  bool cube;
  S corner[4];  // 1 where (left|right) & (above|below) for taps 00, 01, 10, 11
};

// CUBE: boundary is DR_BOUNDARY_CUBE, else one of the 2D boundaries (known when compiling, so
// that 2D lookups carry no cube-corner arithmetic).
template <class S, bool CUBE>
__device__ __forceinline__ Bilinear<S> bilinear_setup(S s, S t, int face, int h, int w,
                                                      int64_t offset, int boundary) {
  Bilinear<S> L;
  const Axis<S> X = texel_axis(s, w, S(0.5), boundary);
  const Axis<S> Y = texel_axis(t, h, S(0.5), boundary);
  const S x0 = s_floor(X.x), y0 = s_floor(Y.x);
  L.fx = X.x - x0;
  L.fy = Y.x - y0;
  L.bad = X.bad || Y.bad;
  L.pass_x = X.pass;
  L.pass_y = Y.pass;
  L.size_x = (S)w;
  L.size_y = (S)h;
  const int col = (int)x0, row = (int)y0;
  L.cube = CUBE;
  if constexpr (CUBE) {
    L.valid[0] = tap(row, col, face, h, w, offset, boundary, L.index[0]);
    L.valid[1] = tap(row, col + 1, face, h, w, offset, boundary, L.index[1]);
    L.valid[2] = tap(row + 1, col, face, h, w, offset, boundary, L.index[2]);
    L.valid[3] = tap(row + 1, col + 1, face, h, w, offset, boundary, L.index[3]);
  } else {
    // The two rows and two columns once each, then the four taps from them.
    const AxisPair R = axis_pair(row, h, boundary), K = axis_pair(col, w, boundary);
    const uint32_t above = (uint32_t)offset + (uint32_t)R.at[0] * (uint32_t)w;
    const uint32_t below = (uint32_t)offset + (uint32_t)R.at[1] * (uint32_t)w;
    L.index[0] = above + K.at[0];
    L.index[1] = above + K.at[1];
    L.index[2] = below + K.at[0];
    L.index[3] = below + K.at[1];
    L.valid[0] = R.valid[0] && K.valid[0];
    L.valid[1] = R.valid[0] && K.valid[1];
    L.valid[2] = R.valid[1] && K.valid[0];
    L.valid[3] = R.valid[1] && K.valid[1];
  }
  if (L.cube) {
    const bool left = col < 0, right = col + 1 >= w, above = row < 0, below = row + 1 >= h;
    L.corner[0] = (left && above) ? S(1) : S(0);
    L.corner[1] = (right && above) ? S(1) : S(0);
    L.corner[2] = (left && below) ? S(1) : S(0);
    L.corner[3] = (right && below) ? S(1) : S(0);
  }
  return L;
}

// Value of one channel (reference.py:601-611).
template <class S>
__device__ __forceinline__ S bilinear_value(const Bilinear<S>& L, const S (&t)[4]) {
  const S fx = L.fx, fy = L.fy;
  S out = (S(1) - fy) * ((S(1) - fx) * t[0] + fx * t[1]) + fy * ((S(1) - fx) * t[2] + fx * t[3]);
  if (L.cube) {
    const S missing = (S(1) - fy) * ((S(1) - fx) * L.corner[0] + fx * L.corner[1]) +
                      fy * ((S(1) - fx) * L.corner[2] + fx * L.corner[3]);
    out = out + missing * (t[0] + t[1] + t[2] + t[3]) / S(3);
  }
  return out;
}

// Gradient of one channel's value: texel weights and d/dfx, d/dfy.
template <class S>
__device__ __forceinline__ void bilinear_grad(const Bilinear<S>& L, const S (&t)[4],
                                              S (&wgt)[4], S& dfx, S& dfy) {
  const S fx = L.fx, fy = L.fy;
  wgt[0] = (S(1) - fy) * (S(1) - fx);
  wgt[1] = (S(1) - fy) * fx;
  wgt[2] = fy * (S(1) - fx);
  wgt[3] = fy * fx;
  dfx = (S(1) - fy) * (t[1] - t[0]) + fy * (t[3] - t[2]);
  dfy = ((S(1) - fx) * t[2] + fx * t[3]) - ((S(1) - fx) * t[0] + fx * t[1]);
  if (L.cube) {
    const S missing = (S(1) - fy) * ((S(1) - fx) * L.corner[0] + fx * L.corner[1]) +
                      fy * ((S(1) - fx) * L.corner[2] + fx * L.corner[3]);
    const S share = (t[0] + t[1] + t[2] + t[3]) / S(3);
    const S dm_dfx = (S(1) - fy) * (L.corner[1] - L.corner[0]) + fy * (L.corner[3] - L.corner[2]);
    const S dm_dfy = ((S(1) - fx) * L.corner[2] + fx * L.corner[3]) -
                     ((S(1) - fx) * L.corner[0] + fx * L.corner[1]);
    dfx += dm_dfx * share;
    dfy += dm_dfy * share;
#pragma unroll
    for (int k = 0; k < 4; ++k) wgt[k] += missing / S(3);
  }
}

// bilinear_grad and bilinear_value of one channel in one pass, for the backward kernels: the
// cube-corner mean is the tap sum times 1/3 (within an ulp of the quotient), shared by the
// value and the derivatives.
template <class S>
__device__ __forceinline__ S bilinear_grad_value(const Bilinear<S>& L, const S (&t)[4],
                                                 S& dfx, S& dfy) {
  const S fx = L.fx, fy = L.fy;
  const S top = (S(1) - fx) * t[0] + fx * t[1], bottom = (S(1) - fx) * t[2] + fx * t[3];
  S value = (S(1) - fy) * top + fy * bottom;
  dfx = (S(1) - fy) * (t[1] - t[0]) + fy * (t[3] - t[2]);
  dfy = bottom - top;
  if (L.cube) {
    const S missing = (S(1) - fy) * ((S(1) - fx) * L.corner[0] + fx * L.corner[1]) +
                      fy * ((S(1) - fx) * L.corner[2] + fx * L.corner[3]);
    const S share = (t[0] + t[1] + t[2] + t[3]) * S(1.0 / 3.0);
    const S dm_dfx = (S(1) - fy) * (L.corner[1] - L.corner[0]) + fy * (L.corner[3] - L.corner[2]);
    const S dm_dfy = ((S(1) - fx) * L.corner[2] + fx * L.corner[3]) -
                     ((S(1) - fx) * L.corner[0] + fx * L.corner[1]);
    dfx += dm_dfx * share;
    dfy += dm_dfy * share;
    value = value + missing * share;
  }
  return value;
}

// (du/dx, du/dy, dv/dx, dv/dy) of a pixel.
template <class S>
struct Deriv4 {
  S x, y, z, w;
};

// Level of detail from the footprint (reference.py:491-501); width and height are those of the
// base level.
template <class S>
__device__ __forceinline__ S footprint_lod(const Deriv4<S>& da, int height, int width) {
  const S W = (S)width, H = (S)height, L = kFootprintLimit<S>;
  const S cx0 = s_min(s_max(da.x * W, -L), L), cy0 = s_min(s_max(da.z * H, -L), L);
  const S cx1 = s_min(s_max(da.y * W, -L), L), cy1 = s_min(s_max(da.w * H, -L), L);
  const S len_x = cx0 * cx0 + cy0 * cy0;
  const S len_y = cx1 * cx1 + cy1 * cy1;
  if (isnan(da.x) || isnan(da.y) || isnan(da.z) || isnan(da.w)) return s_nan<S>();
  return S(0.5) * s_log2(s_max(s_max(len_x, len_y), kMinFootprint<S>));
}

template <class S>
__device__ __forceinline__ void footprint_lod_grad(const Deriv4<S>& da, int height, int width,
                                                   S g, S* grad) {
  const S W = (S)width, H = (S)height, L = kFootprintLimit<S>;
  const S v[4] = {da.x * W, da.y * W, da.z * H, da.w * H};  // du/dx, du/dy, dv/dx, dv/dy
  S c[4];
  bool pass[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    pass[i] = v[i] >= -L && v[i] <= L;
    c[i] = s_min(s_max(v[i], -L), L);
  }
  const S len_x = c[0] * c[0] + c[2] * c[2];
  const S len_y = c[1] * c[1] + c[3] * c[3];
  const S m = s_max(len_x, len_y);
  S g_m = m >= kMinFootprint<S> ? g * S(0.5) / (m * kLn2<S>) : S(0);
  // torch.maximum splits the gradient evenly between equal arguments.
  const S share_x = len_x > len_y ? S(1) : (len_x == len_y ? S(0.5) : S(0));
  const S share_y = S(1) - share_x;
  const S g_x = g_m * share_x, g_y = g_m * share_y;
  const S scale[4] = {W, W, H, H};
  const S gl[4] = {g_x, g_y, g_x, g_y};
#pragma unroll
  for (int i = 0; i < 4; ++i) grad[i] = pass[i] ? gl[i] * S(2) * c[i] * scale[i] : S(0);
}

// Everything a pixel's lookup needs, shared by the forward and backward kernels.
template <class S>
struct Lookup {
  bool dir_invalid;  // cube direction that selects nothing: reads zero, no gradient
  bool bad;          // NaN output, no gradient
  int face;
  S s, t;
  int levels;        // 1 or 2 bilinear lookups (0 for nearest)
  int level[2];
  S level_weight[2];
  bool lod_grad;     // the blend factor passes a gradient to the level of detail
  S lod_raw;
  bool mip;
  CubeProj<S> P;
};

template <class S>
__device__ __forceinline__ Deriv4<S> load_deriv4(const S* p) {
  if constexpr (std::is_same_v<S, float>) {
    const float4 v = load4(p);
    return {v.x, v.y, v.z, v.w};
  } else {
    return {p[0], p[1], p[2], p[3]};
  }
}

// A filter or boundary mode given as a template argument: a DR_FILTER_* or DR_BOUNDARY_* value
// fixed when compiling (which drops the other modes' code and registers from the kernel), or
// kAnyMode to read it from the arguments at run time.
constexpr int kAnyMode = -1;

// CUBE: a.boundary is DR_BOUNDARY_CUBE (the kernels are compiled for both cases, so that the
// 2D one carries no cube-map state). FILTER: a.filter, or kAnyMode.
template <class S, bool CUBE, int FILTER = kAnyMode>
__device__ __forceinline__ void lookup_setup(const DrTextureArgs& a, int64_t pixel, Lookup<S>& K) {
  constexpr bool cube = CUBE;
  const int filter = FILTER == kAnyMode ? a.filter : FILTER;
  const bool mip = filter == DR_FILTER_MIP_NEAREST || filter == DR_FILTER_MIP_LINEAR;
  const S* uv = as<S>(a.uv);
  const S* uv_da = as<S>(a.uv_da);
  K.mip = mip;
  K.dir_invalid = false;
  K.face = -1;
  // The derivatives are held by value: a pointer that could address either this thread's
  // registers or global memory would force them into scratch memory.
  bool has_da = false;
  Deriv4<S> da = {S(0), S(0), S(0), S(0)};
  if (cube) {
    cube_project<S>(uv + 3 * pixel, (mip && uv_da) ? uv_da + 6 * pixel : nullptr, K.P);
    K.dir_invalid = !K.P.valid;
    K.face = K.P.face;
    K.s = K.P.st[0];
    K.t = K.P.st[1];
    if (mip && uv_da) {
      da = {K.P.st_da[0], K.P.st_da[1], K.P.st_da[2], K.P.st_da[3]};
      has_da = true;
    }
  } else {
    K.s = uv[2 * pixel];
    K.t = uv[2 * pixel + 1];
    if (mip && uv_da) {
      da = load_deriv4(uv_da + 4 * pixel);
      has_da = true;
    }
  }
  K.bad = false;
  K.lod_grad = false;
  K.level[0] = K.level[1] = 0;
  K.level_weight[0] = S(1);
  K.level_weight[1] = S(0);
  if (!mip) {
    K.levels = filter == DR_FILTER_NEAREST ? 0 : 1;
    return;
  }
  S lod = S(0);
  if (has_da) lod = lod + footprint_lod(da, a.level_height[0], a.level_width[0]);
  if (a.bias) lod = lod + as<S>(a.bias)[pixel];
  K.lod_raw = lod;
  const int top = a.num_levels - 1;
  K.bad = isnan(lod);
  if (K.bad) lod = S(0);
  const bool inside = lod >= S(0) && lod <= (S)top;
  lod = s_min(s_max(lod, S(0)), (S)top);
  const bool blend = filter == DR_FILTER_MIP_LINEAR;
  const int lower = (int)s_floor(lod + (blend ? S(0) : S(0.5)));
  K.level[0] = lower;
  if (blend) {
    K.levels = 2;
    K.level[1] = min(lower + 1, top);
    const S frac = lod - (S)lower;
    K.level_weight[0] = S(1) - frac;
    K.level_weight[1] = frac;
    K.lod_grad = inside && !K.bad;
  } else {
    K.levels = 1;
  }
}

// Sizes and packed offset of the two levels a lookup may use. The level index differs per lane,
// so these are memory reads: both levels' are issued together, before either is used.
struct LevelDims {
  int h[2], w[2];
  int64_t off[2];
};

template <class S>
__device__ __forceinline__ LevelDims lookup_levels(const DrTextureArgs& a, const Lookup<S>& K) {
  LevelDims D;
#pragma unroll
  for (int l = 0; l < 2; ++l) {
    const int k = K.level[l];
    D.h[l] = a.level_height[k];
    D.w[l] = a.level_width[k];
    D.off[l] = a.level_offset[k];
  }
  return D;
}

// BOUNDARY: a.boundary (ignored for cube maps), or kAnyMode.
template <bool CUBE, int BOUNDARY = kAnyMode, class S>
__device__ __forceinline__ Bilinear<S> level_setup(const DrTextureArgs& a, const Lookup<S>& K,
                                                   const LevelDims& D, int l) {
  const int boundary =
      CUBE ? (int)DR_BOUNDARY_CUBE : (BOUNDARY == kAnyMode ? a.boundary : BOUNDARY);
  return bilinear_setup<S, CUBE>(K.s, K.t, K.face, D.h[l], D.w[l], D.off[l], boundary);
}

// Nearest: the texel containing the coordinate (reference.py:555-573). BOUNDARY: a.boundary,
// or kAnyMode.
template <int BOUNDARY = kAnyMode, class S>
__device__ __forceinline__ bool nearest_setup(const DrTextureArgs& a, const Lookup<S>& K,
                                              uint32_t& index, bool& valid) {
  const int h = a.level_height[0], w = a.level_width[0];
  const int mode = BOUNDARY == kAnyMode ? a.boundary : BOUNDARY;
  const Axis<S> X = texel_axis(K.s, w, S(0), mode);
  const Axis<S> Y = texel_axis(K.t, h, S(0), mode);
  const int boundary = mode == DR_BOUNDARY_CUBE ? DR_BOUNDARY_CLAMP : mode;
  valid = tap((int)s_floor(Y.x), (int)s_floor(X.x), K.face, h, w, a.level_offset[0], boundary,
              index);
  return X.bad || Y.bad;
}

}  // namespace
}  // namespace tex
}  // namespace dr
