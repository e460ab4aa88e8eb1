// Texture sampling for gfx950: 2D textures and cube maps, nearest / bilinear / mipmapped
// lookups with wrap, clamp or zero boundaries, their gradients, and the mip chain.
//
// The arithmetic follows the reference backend: texel coordinates and boundaries
// (src/diffrast/backends/reference.py:555-672), level of detail and level blending
// (reference.py:491-501, 522-552), cube-map projection and the integer edge fold
// (src/diffrast/backends/_cube.py:44-143). One thread per pixel computes the tap addresses
// of its one or two levels once and loops over channels. All levels live in one packed
// buffer [tex_batch, texels, channels], so a mipmapped lookup is two bilinear lookups
// wherever the pixel's levels are.
//
// The backward pass writes the coordinate, derivative and bias gradients per pixel; texel
// gradients are summed per workgroup in an LDS table (fixed point, after runs of neighbouring
// pixels on one texel have summed) and reach global memory with one fp32 atomic per row and
// channel. The mip chain uses exact area weights (reference.py:449-488): where sizes halve
// exactly, a workgroup takes a 64 x 64 tile through six levels in LDS; odd sizes go level by
// level. Its adjoint is a gather, so it needs no atomics.
#include <type_traits>

#include "common.h"

namespace dr {
namespace {

constexpr float kFootprintLimit = 1e18f;  // reference.py:402
constexpr float kDerivativeLimit = 1e18f; // _cube.py:36
constexpr float kMinFootprint = 1e-30f;   // reference.py:501
constexpr float kLn2 = 0.693147180559945309f;

// ---- cube geometry (_cube.py) -----------------------------------------------------------

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

struct CubeProj {
  bool valid, undefined;
  int face;
  float length, ma, rs, rt;
  float dn[3];
  float da[3][2];       // clamped, scaled derivatives
  bool da_pass[3][2];   // inside the clamp
  float d_ma[2], d_sc[2], d_tc[2];
  float st[2];
  float st_da[4];       // ds/dx, ds/dy, dt/dx, dt/dy
};

// Face selection and face coordinates of a direction (_cube.py:44-102).
__device__ __forceinline__ void cube_project(const float* dir, const float* dir_da, CubeProj& P) {
  float d[3] = {dir[0], dir[1], dir[2]};
  const float ax0 = fabsf(d[0]), ay0 = fabsf(d[1]), az0 = fabsf(d[2]);
  P.valid = isfinite(d[0]) && isfinite(d[1]) && isfinite(d[2]) &&
            fmaxf(fmaxf(ax0, ay0), az0) >= 1.17549435e-38f;
  if (!P.valid) {
    d[0] = 0.0f;
    d[1] = 0.0f;
    d[2] = 1.0f;
  }
  const float ax = fabsf(d[0]), ay = fabsf(d[1]), az = fabsf(d[2]);
  const bool x_major = ax >= ay && ax >= az;
  const bool y_major = !x_major && ay >= az;
  const int axis = x_major ? 0 : (y_major ? 1 : 2);
  P.face = 2 * axis + (d[axis] < 0.0f ? 1 : 0);
  P.length = fmaxf(fmaxf(ax, ay), az);
#pragma unroll
  for (int k = 0; k < 3; ++k) P.dn[k] = d[k] / P.length;
  const int* M = kMajor[P.face];
  const int* S = kSAxis[P.face];
  const int* T = kTAxis[P.face];
  P.ma = P.dn[0] * (float)M[0] + P.dn[1] * (float)M[1] + P.dn[2] * (float)M[2];
  const float sc = P.dn[0] * (float)S[0] + P.dn[1] * (float)S[1] + P.dn[2] * (float)S[2];
  const float tc = P.dn[0] * (float)T[0] + P.dn[1] * (float)T[1] + P.dn[2] * (float)T[2];
  P.rs = sc / P.ma;
  P.rt = tc / P.ma;
  P.st[0] = 0.5f * (P.rs + 1.0f);
  P.st[1] = 0.5f * (P.rt + 1.0f);
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
      const float v = (use ? dir_da[2 * k + j] : 0.0f) / P.length;
      P.da_pass[k][j] = v >= -kDerivativeLimit && v <= kDerivativeLimit;
      P.da[k][j] = fminf(fmaxf(v, -kDerivativeLimit), kDerivativeLimit);
    }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    P.d_ma[j] = P.da[0][j] * (float)M[0] + P.da[1][j] * (float)M[1] + P.da[2][j] * (float)M[2];
    P.d_sc[j] = P.da[0][j] * (float)S[0] + P.da[1][j] * (float)S[1] + P.da[2][j] * (float)S[2];
    P.d_tc[j] = P.da[0][j] * (float)T[0] + P.da[1][j] * (float)T[1] + P.da[2][j] * (float)T[2];
  }
  const float nan = __int_as_float(0x7fc00000);
  P.st_da[0] = P.undefined ? nan : 0.5f * (P.d_sc[0] - P.rs * P.d_ma[0]) / P.ma;
  P.st_da[1] = P.undefined ? nan : 0.5f * (P.d_sc[1] - P.rs * P.d_ma[1]) / P.ma;
  P.st_da[2] = P.undefined ? nan : 0.5f * (P.d_tc[0] - P.rt * P.d_ma[0]) / P.ma;
  P.st_da[3] = P.undefined ? nan : 0.5f * (P.d_tc[1] - P.rt * P.d_ma[1]) / P.ma;
}

// Gradient of cube_project: from d(loss)/d(st) and d(loss)/d(st_da) to the direction and
// its derivatives (3 and 6 values); g_sda is used when use_sda is set.
__device__ __forceinline__ void cube_project_backward(const CubeProj& P, float g_s, float g_t,
                                                      bool use_sda, const float (&g_sda)[4],
                                                      float (&grad_dir)[3],
                                                      float (&grad_dir_da)[6]) {
  const int* M = kMajor[P.face];
  const int* S = kSAxis[P.face];
  const int* T = kTAxis[P.face];
  float g_rs = 0.5f * g_s, g_rt = 0.5f * g_t, g_ma = 0.0f;
  float g_dsc[2] = {0.f, 0.f}, g_dtc[2] = {0.f, 0.f}, g_dma[2] = {0.f, 0.f};
  if (use_sda && !P.undefined) {
    const float gds[2] = {g_sda[0], g_sda[1]}, gdt[2] = {g_sda[2], g_sda[3]};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float ds = P.st_da[j], dt = P.st_da[2 + j];
      g_rs += gds[j] * (-0.5f * P.d_ma[j] / P.ma);
      g_rt += gdt[j] * (-0.5f * P.d_ma[j] / P.ma);
      g_ma -= (gds[j] * ds + gdt[j] * dt) / P.ma;
      g_dsc[j] = 0.5f * gds[j] / P.ma;
      g_dtc[j] = 0.5f * gdt[j] / P.ma;
      g_dma[j] = -0.5f * (gds[j] * P.rs + gdt[j] * P.rt) / P.ma;
    }
  }
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float g = g_dsc[j] * (float)S[k] + g_dtc[j] * (float)T[k] + g_dma[j] * (float)M[k];
      g = (P.valid && !P.undefined && P.da_pass[k][j]) ? g / P.length : 0.0f;
      grad_dir_da[2 * k + j] = g;
    }
  g_ma -= (g_rs * P.rs + g_rt * P.rt) / P.ma;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float g_dn = (g_rs * (float)S[k] + g_rt * (float)T[k]) / P.ma + g_ma * (float)M[k];
    grad_dir[k] = P.valid ? g_dn / P.length : 0.0f;
  }
}

// ---- 2D coordinates, taps and levels ----------------------------------------------------

struct Axis {
  float x;     // continuous texel coordinate
  bool bad;    // not finite (then x = 0)
  bool pass;   // gradient reaches the input coordinate
};

// coord * size - shift, wrapped or saturated as for the boundary (reference.py:615-633).
__device__ __forceinline__ Axis texel_axis(float coord, int size, float shift, int boundary) {
  Axis A;
  float c = coord;
  if (boundary == DR_BOUNDARY_WRAP) c = c - floorf(c);
  A.x = c * (float)size - shift;
  A.pass = true;
  if (boundary == DR_BOUNDARY_CLAMP || boundary == DR_BOUNDARY_ZERO) {
    if (A.x < -1.0f) { A.x = -1.0f; A.pass = false; }
    if (A.x > (float)size) { A.x = (float)size; A.pass = false; }
  }
  A.bad = !isfinite(A.x);
  if (A.bad) {
    A.x = 0.0f;
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

// Texel index (in texels from the start of the image's packed buffer) of integer tap
// (row, col) of a level; false when the tap reads zero (reference.py:636-672).
__device__ __forceinline__ bool tap(int row, int col, int face, int h, int w, int64_t offset,
                                    int boundary, int64_t& index) {
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
  index = offset + (int64_t)row * w + col;
  return valid;
}

struct Bilinear {
  int64_t index[4];
  bool valid[4];
  float fx, fy;
  bool bad;
  bool pass_x, pass_y;
  float size_x, size_y;
  // Cube corners: taps beyond two edges count as the mean of the other three.
  bool cube;
  float corner[4];  // 1 where (left|right) & (above|below) for taps 00, 01, 10, 11
};

__device__ __forceinline__ Bilinear bilinear_setup(float s, float t, int face, int h, int w,
                                                   int64_t offset, int boundary) {
  Bilinear L;
  const Axis X = texel_axis(s, w, 0.5f, boundary);
  const Axis Y = texel_axis(t, h, 0.5f, boundary);
  const float x0 = floorf(X.x), y0 = floorf(Y.x);
  L.fx = X.x - x0;
  L.fy = Y.x - y0;
  L.bad = X.bad || Y.bad;
  L.pass_x = X.pass;
  L.pass_y = Y.pass;
  L.size_x = (float)w;
  L.size_y = (float)h;
  const int col = (int)x0, row = (int)y0;
  L.valid[0] = tap(row, col, face, h, w, offset, boundary, L.index[0]);
  L.valid[1] = tap(row, col + 1, face, h, w, offset, boundary, L.index[1]);
  L.valid[2] = tap(row + 1, col, face, h, w, offset, boundary, L.index[2]);
  L.valid[3] = tap(row + 1, col + 1, face, h, w, offset, boundary, L.index[3]);
  L.cube = boundary == DR_BOUNDARY_CUBE;
  if (L.cube) {
    const bool left = col < 0, right = col + 1 >= w, above = row < 0, below = row + 1 >= h;
    L.corner[0] = (left && above) ? 1.0f : 0.0f;
    L.corner[1] = (right && above) ? 1.0f : 0.0f;
    L.corner[2] = (left && below) ? 1.0f : 0.0f;
    L.corner[3] = (right && below) ? 1.0f : 0.0f;
  }
  return L;
}

// Channels [c0, c0 + N) of the four taps (0 past C or for an invalid tap), all loads issued
// together.
template <int N>
__device__ __forceinline__ void fetch_taps(const float* __restrict__ texels, const Bilinear& L,
                                           int C, int c0, float (&t)[4][N]) {
  if constexpr (N == 4) {
    // Four-channel texels on a 16-byte aligned buffer: one 16-byte load per tap.
    if (C == 4 && (reinterpret_cast<uintptr_t>(texels) & 15u) == 0) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 v = L.valid[k] ? *reinterpret_cast<const float4*>(texels + L.index[k] * 4)
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        t[k][0] = v.x;
        t[k][1] = v.y;
        t[k][2] = v.z;
        t[k][3] = v.w;
      }
      return;
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float* row = texels + L.index[k] * C + c0;
#pragma unroll
    for (int c = 0; c < N; ++c) t[k][c] = (L.valid[k] && c0 + c < C) ? row[c] : 0.0f;
  }
}

template <int N>
__device__ __forceinline__ void tap_column(const float (&t)[4][N], int c, float (&out)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) out[k] = t[k][c];
}

// Value of one channel (reference.py:601-611).
__device__ __forceinline__ float bilinear_value(const Bilinear& L, const float (&t)[4]) {
  const float fx = L.fx, fy = L.fy;
  float out = (1.0f - fy) * ((1.0f - fx) * t[0] + fx * t[1]) +
              fy * ((1.0f - fx) * t[2] + fx * t[3]);
  if (L.cube) {
    const float missing = (1.0f - fy) * ((1.0f - fx) * L.corner[0] + fx * L.corner[1]) +
                          fy * ((1.0f - fx) * L.corner[2] + fx * L.corner[3]);
    out = out + missing * (t[0] + t[1] + t[2] + t[3]) / 3.0f;
  }
  return out;
}

// Gradient of one channel's value: texel weights and d/dfx, d/dfy.
__device__ __forceinline__ void bilinear_grad(const Bilinear& L, const float (&t)[4],
                                              float (&wgt)[4], float& dfx, float& dfy) {
  const float fx = L.fx, fy = L.fy;
  wgt[0] = (1.0f - fy) * (1.0f - fx);
  wgt[1] = (1.0f - fy) * fx;
  wgt[2] = fy * (1.0f - fx);
  wgt[3] = fy * fx;
  dfx = (1.0f - fy) * (t[1] - t[0]) + fy * (t[3] - t[2]);
  dfy = ((1.0f - fx) * t[2] + fx * t[3]) - ((1.0f - fx) * t[0] + fx * t[1]);
  if (L.cube) {
    const float missing = (1.0f - fy) * ((1.0f - fx) * L.corner[0] + fx * L.corner[1]) +
                          fy * ((1.0f - fx) * L.corner[2] + fx * L.corner[3]);
    const float share = (t[0] + t[1] + t[2] + t[3]) / 3.0f;
    const float dm_dfx = (1.0f - fy) * (L.corner[1] - L.corner[0]) + fy * (L.corner[3] - L.corner[2]);
    const float dm_dfy = ((1.0f - fx) * L.corner[2] + fx * L.corner[3]) -
                         ((1.0f - fx) * L.corner[0] + fx * L.corner[1]);
    dfx += dm_dfx * share;
    dfy += dm_dfy * share;
#pragma unroll
    for (int k = 0; k < 4; ++k) wgt[k] += missing / 3.0f;
  }
}

// Level of detail from the footprint (reference.py:491-501). uv_da = (du/dx, du/dy, dv/dx,
// dv/dy); width and height are those of the base level.
__device__ __forceinline__ float footprint_lod(const float4& da, int height, int width) {
  const float W = (float)width, H = (float)height, L = kFootprintLimit;
  const float cx0 = fminf(fmaxf(da.x * W, -L), L), cy0 = fminf(fmaxf(da.z * H, -L), L);
  const float cx1 = fminf(fmaxf(da.y * W, -L), L), cy1 = fminf(fmaxf(da.w * H, -L), L);
  const float len_x = cx0 * cx0 + cy0 * cy0;
  const float len_y = cx1 * cx1 + cy1 * cy1;
  if (isnan(da.x) || isnan(da.y) || isnan(da.z) || isnan(da.w))
    return __int_as_float(0x7fc00000);
  return 0.5f * log2f(fmaxf(fmaxf(len_x, len_y), kMinFootprint));
}

__device__ __forceinline__ void footprint_lod_grad(const float4& da, int height, int width,
                                                   float g, float* grad) {
  const float W = (float)width, H = (float)height, L = kFootprintLimit;
  const float v[4] = {da.x * W, da.y * W, da.z * H, da.w * H};  // du/dx, du/dy, dv/dx, dv/dy
  float c[4];
  bool pass[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    pass[i] = v[i] >= -L && v[i] <= L;
    c[i] = fminf(fmaxf(v[i], -L), L);
  }
  const float len_x = c[0] * c[0] + c[2] * c[2];
  const float len_y = c[1] * c[1] + c[3] * c[3];
  const float m = fmaxf(len_x, len_y);
  float g_m = m >= kMinFootprint ? g * 0.5f / (m * kLn2) : 0.0f;
  // torch.maximum splits the gradient evenly between equal arguments.
  const float share_x = len_x > len_y ? 1.0f : (len_x == len_y ? 0.5f : 0.0f);
  const float share_y = 1.0f - share_x;
  const float g_x = g_m * share_x, g_y = g_m * share_y;
  const float scale[4] = {W, W, H, H};
  const float gl[4] = {g_x, g_y, g_x, g_y};
#pragma unroll
  for (int i = 0; i < 4; ++i) grad[i] = pass[i] ? gl[i] * 2.0f * c[i] * scale[i] : 0.0f;
}

// Everything a pixel's lookup needs, shared by the forward and backward kernels.
struct Lookup {
  bool dir_invalid;  // cube direction that selects nothing: reads zero, no gradient
  bool bad;          // NaN output, no gradient
  int face;
  float s, t;
  int levels;        // 1 or 2 bilinear lookups (0 for nearest)
  int level[2];
  float level_weight[2];
  bool lod_grad;     // the blend factor passes a gradient to the level of detail
  float lod_raw;
  bool mip;
  CubeProj P;
};

// CUBE: a.boundary is DR_BOUNDARY_CUBE (the kernels are compiled for both cases, so that the
// 2D one carries no cube-map state).
template <bool CUBE>
__device__ __forceinline__ void lookup_setup(const DrTextureArgs& a, int64_t pixel, Lookup& K) {
  constexpr bool cube = CUBE;
  const bool mip = a.filter == DR_FILTER_MIP_NEAREST || a.filter == DR_FILTER_MIP_LINEAR;
  K.mip = mip;
  K.dir_invalid = false;
  K.face = -1;
  // (du/dx, du/dy, dv/dx, dv/dy), held by value: a pointer that could address either this
  // thread's registers or global memory would force them into scratch memory.
  bool has_da = false;
  float4 da = make_float4(0.f, 0.f, 0.f, 0.f);
  if (cube) {
    cube_project(a.uv + 3 * pixel, (mip && a.uv_da) ? a.uv_da + 6 * pixel : nullptr, K.P);
    K.dir_invalid = !K.P.valid;
    K.face = K.P.face;
    K.s = K.P.st[0];
    K.t = K.P.st[1];
    if (mip && a.uv_da) {
      da = make_float4(K.P.st_da[0], K.P.st_da[1], K.P.st_da[2], K.P.st_da[3]);
      has_da = true;
    }
  } else {
    K.s = a.uv[2 * pixel];
    K.t = a.uv[2 * pixel + 1];
    if (mip && a.uv_da) {
      da = load4(a.uv_da + 4 * pixel);
      has_da = true;
    }
  }
  K.bad = false;
  K.lod_grad = false;
  K.level[0] = K.level[1] = 0;
  K.level_weight[0] = 1.0f;
  K.level_weight[1] = 0.0f;
  if (!mip) {
    K.levels = a.filter == DR_FILTER_NEAREST ? 0 : 1;
    return;
  }
  float lod = 0.0f;
  if (has_da) lod = lod + footprint_lod(da, a.level_height[0], a.level_width[0]);
  if (a.bias) lod = lod + a.bias[pixel];
  K.lod_raw = lod;
  const int top = a.num_levels - 1;
  K.bad = isnan(lod);
  if (K.bad) lod = 0.0f;
  const bool inside = lod >= 0.0f && lod <= (float)top;
  lod = fminf(fmaxf(lod, 0.0f), (float)top);
  const bool blend = a.filter == DR_FILTER_MIP_LINEAR;
  const int lower = (int)floorf(lod + (blend ? 0.0f : 0.5f));
  K.level[0] = lower;
  if (blend) {
    K.levels = 2;
    K.level[1] = min(lower + 1, top);
    const float frac = lod - (float)lower;
    K.level_weight[0] = 1.0f - frac;
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

__device__ __forceinline__ LevelDims lookup_levels(const DrTextureArgs& a, const Lookup& K) {
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

__device__ __forceinline__ Bilinear level_setup(const DrTextureArgs& a, const Lookup& K,
                                                const LevelDims& D, int l) {
  return bilinear_setup(K.s, K.t, K.face, D.h[l], D.w[l], D.off[l], a.boundary);
}

// Nearest: the texel containing the coordinate (reference.py:555-573).
__device__ __forceinline__ bool nearest_setup(const DrTextureArgs& a, const Lookup& K,
                                              int64_t& index, bool& valid) {
  const int h = a.level_height[0], w = a.level_width[0];
  const Axis X = texel_axis(K.s, w, 0.0f, a.boundary);
  const Axis Y = texel_axis(K.t, h, 0.0f, a.boundary);
  const int boundary = a.boundary == DR_BOUNDARY_CUBE ? DR_BOUNDARY_CLAMP : a.boundary;
  valid = tap((int)floorf(Y.x), (int)floorf(X.x), K.face, h, w, a.level_offset[0], boundary,
              index);
  return X.bad || Y.bad;
}

// NC channels per pass (the channel count when it is 1-4; 4 with a loop for more). Every tap
// of a pass is loaded before its stores.
template <int NC, bool CUBE>
__global__ __launch_bounds__(256) void tex_fwd_kernel(DrTextureArgs a, float* __restrict__ out) {
  const int64_t pixel = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (pixel >= (int64_t)a.batch * a.height * a.width) return;
  const int C = a.channels;
  float* o = out + pixel * C;
  Lookup K;
  lookup_setup<CUBE>(a, pixel, K);
  if (K.dir_invalid) {
    for (int c = 0; c < C; ++c) o[c] = 0.0f;
    return;
  }
  const int64_t image = pixel / ((int64_t)a.height * a.width);
  const float* __restrict__ texels = a.texels + (a.tex_batch > 1 ? image * a.num_texels * C : 0);
  const float nan = __int_as_float(0x7fc00000);
  if (K.levels == 0) {
    int64_t index;
    bool valid;
    const bool bad = nearest_setup(a, K, index, valid);
    for (int c = 0; c < C; ++c) o[c] = bad ? nan : (valid ? texels[index * C + c] : 0.0f);
    return;
  }
  const LevelDims D = lookup_levels(a, K);
  const Bilinear L0 = level_setup(a, K, D, 0);
  const bool two = K.levels == 2;
  const Bilinear L1 = two ? level_setup(a, K, D, 1) : L0;
  const bool bad = K.bad || L0.bad || (two && L1.bad);
  const float frac = K.level_weight[1];
  for (int c0 = 0; c0 < C; c0 += NC) {
    float t[4][NC], u[4][NC];
    fetch_taps<NC>(texels, L0, C, c0, t);
    if (two) fetch_taps<NC>(texels, L1, C, c0, u);
    float res[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float tc[4], uc[4];
      tap_column(t, c, tc);
      if (two) {
        tap_column(u, c, uc);
        res[c] = bilinear_value(L0, tc) * (1.0f - frac) + bilinear_value(L1, uc) * frac;
      } else {
        res[c] = bilinear_value(L0, tc);
      }
      if (bad) res[c] = nan;
    }
    if constexpr (NC == 4) {
      if (C == 4 && (reinterpret_cast<uintptr_t>(o) & 15u) == 0) {
        *reinterpret_cast<float4*>(o) = make_float4(res[0], res[1], res[2], res[3]);
        continue;
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (c0 + c < C) o[c0 + c] = res[c];
  }
}

// Coordinate-gradient contributions of one level: d/dfx, d/dfy summed over channels with the
// level weight, and the level's value per channel for the blend-factor gradient.
template <int N>
__device__ __forceinline__ void level_coordinate_grads(const Bilinear& L,
                                                       const float* __restrict__ texels,
                                                       const float* __restrict__ g, int C,
                                                       float level_weight, float& g_fx,
                                                       float& g_fy, bool want_value,
                                                       float& g_value) {
  for (int c0 = 0; c0 < C; c0 += N) {
    float t[4][N], gc[N];
    fetch_taps<N>(texels, L, C, c0, t);
    bool loaded = false;
    if constexpr (N == 4) {
      if (C == 4 && (reinterpret_cast<uintptr_t>(g) & 15u) == 0) {
        const float4 v = *reinterpret_cast<const float4*>(g);
        gc[0] = v.x;
        gc[1] = v.y;
        gc[2] = v.z;
        gc[3] = v.w;
        loaded = true;
      }
    }
    if (!loaded)
#pragma unroll
      for (int c = 0; c < N; ++c) gc[c] = c0 + c < C ? g[c0 + c] : 0.0f;
#pragma unroll
    for (int c = 0; c < N; ++c) {
      if (c0 + c >= C) continue;
      float tc[4], wgt[4], dfx, dfy;
      tap_column(t, c, tc);
      bilinear_grad(L, tc, wgt, dfx, dfy);
      const float gl = gc[c] * level_weight;
      g_fx += gl * dfx;
      g_fy += gl * dfy;
      if (want_value) g_value += gc[c] * bilinear_value(L, tc);
    }
  }
}

// Table keys (texel rows of the packed buffer, 0xffffffff for none) and weights of a level's
// taps. A tap of weight 0 (the second level when the blend factor is 0, or an axis with fraction
// 0) adds nothing and gets no key.
__device__ __forceinline__ void level_taps(const Bilinear& L, float level_weight,
                                           int64_t tex_off, uint32_t* key, float* weight) {
  float t0[4] = {0.f, 0.f, 0.f, 0.f}, wgt[4], dfx, dfy;
  bilinear_grad(L, t0, wgt, dfx, dfy);  // the weights do not depend on texel values
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    weight[k] = level_weight * wgt[k];
    key[k] = L.valid[k] && weight[k] != 0.0f ? (uint32_t)(tex_off + L.index[k]) : 0xffffffffu;
  }
}

template <int NC, bool CUBE>
__global__ __launch_bounds__(256) void tex_bwd_kernel(DrTextureArgs a, const float* grad_out,
                                                      float* grad_texels, float* grad_uv,
                                                      float* grad_uv_da, float* grad_bias) {
  using Table = RowTable<512, 4>;
  __shared__ Table table;
  table.init();
  const TilePixel tp = tile_pixel(a.batch, a.height, a.width);
  const int64_t pixel = tp.pixel;
  const int C = a.channels;
  constexpr bool cube = CUBE;
  const float* g = grad_out + (tp.inside ? pixel * C : 0);
  const int64_t tex_off = a.tex_batch > 1 ? (int64_t)tp.b * a.num_texels : 0;
  const float* texels = a.texels + tex_off * C;

  Lookup K;
  // Texel gradient targets: taps 0-3 of the first level, 4-7 of the second.
  uint32_t tap_key[8];
  float tap_weight[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    tap_key[k] = Table::kEmpty;
    tap_weight[k] = 0.0f;
  }
  float g_s = 0.0f, g_t = 0.0f, g_lod = 0.0f;
  bool live = false;
  if (tp.inside) {
    lookup_setup<CUBE>(a, pixel, K);
    live = !K.dir_invalid;
  }
  if (live && K.levels == 0) {
    int64_t index;
    bool valid;
    const bool bad = nearest_setup(a, K, index, valid);
    if (!bad && valid) {
      tap_key[0] = (uint32_t)(tex_off + index);
      tap_weight[0] = 1.0f;
    }
    live = false;  // no coordinate gradient
  } else if (live) {
    const LevelDims D = lookup_levels(a, K);
    const Bilinear L0 = level_setup(a, K, D, 0);
    Bilinear L1 = L0;
    const bool two = K.levels == 2;
    if (two) L1 = level_setup(a, K, D, 1);
    if (K.bad || L0.bad || (two && L1.bad)) {
      live = false;
    } else {
      float fx0 = 0.f, fy0 = 0.f, fx1 = 0.f, fy1 = 0.f, v0 = 0.f, v1 = 0.f;
      level_coordinate_grads<NC>(L0, texels, g, C, K.level_weight[0], fx0, fy0, two, v0);
      level_taps(L0, K.level_weight[0], tex_off, tap_key, tap_weight);
      if (L0.pass_x) g_s += fx0 * L0.size_x;
      if (L0.pass_y) g_t += fy0 * L0.size_y;
      if (two) {
        level_coordinate_grads<NC>(L1, texels, g, C, K.level_weight[1], fx1, fy1, true, v1);
        level_taps(L1, K.level_weight[1], tex_off, tap_key + 4, tap_weight + 4);
        if (L1.pass_x) g_s += fx1 * L1.size_x;
        if (L1.pass_y) g_t += fy1 * L1.size_y;
        g_lod = K.lod_grad ? v1 - v0 : 0.0f;
      }
    }
  }

  if (tp.inside) {
    float g_da[4] = {0.f, 0.f, 0.f, 0.f};
    const bool has_da = K.mip && a.uv_da != nullptr;
    if (live && has_da && g_lod != 0.0f) {
      const float4 da = cube ? make_float4(K.P.st_da[0], K.P.st_da[1], K.P.st_da[2], K.P.st_da[3])
                             : load4(a.uv_da + 4 * pixel);
      footprint_lod_grad(da, a.level_height[0], a.level_width[0], g_lod, g_da);
    }
    if (grad_bias) grad_bias[pixel] = live ? g_lod : 0.0f;
    if (cube) {
      float gdir[3] = {0.f, 0.f, 0.f}, gdir_da[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (live) cube_project_backward(K.P, g_s, g_t, has_da, g_da, gdir, gdir_da);
      if (grad_uv)
        for (int k = 0; k < 3; ++k) grad_uv[3 * pixel + k] = gdir[k];
      if (grad_uv_da)
        for (int k = 0; k < 6; ++k) grad_uv_da[6 * pixel + k] = gdir_da[k];
    } else {
      if (grad_uv) {
        grad_uv[2 * pixel] = live ? g_s : 0.0f;
        grad_uv[2 * pixel + 1] = live ? g_t : 0.0f;
      }
      if (grad_uv_da)
        for (int k = 0; k < 4; ++k) grad_uv_da[4 * pixel + k] = live ? g_da[k] : 0.0f;
    }
  }
  if (grad_texels == nullptr) return;  // uniform over the workgroup

  // Texel gradients, four channels per pass through the workgroup's table: tap k adds
  // g[c] * weight[k] to its texel row.
  float w_max = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (tap_key[k] != Table::kEmpty) w_max = fmaxf(w_max, fabsf(tap_weight[k]));
  for (int c0 = 0; c0 < C; c0 += 4) {
    const int n = min(4, C - c0);
    float gc[4] = {0.f, 0.f, 0.f, 0.f};
    if (!(n == 4 && load_wide<4>(g + c0, gc)))
#pragma unroll
      for (int c = 0; c < 4; ++c) gc[c] = c < n ? g[c0 + c] : 0.0f;
    // The largest |g[c] * weight[k]| of this lane (rounding is monotone, so the product of the
    // two largest factors is the largest product).
    float g_max = 0.0f;
    bool finite = true;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      finite = finite && isfinite(gc[c]);
      g_max = fmaxf(g_max, fabsf(gc[c]));
    }
    if (!finite) g_max = __int_as_float(0x7f800000);
    const float lane_max = w_max > 0.0f ? g_max * w_max : 0.0f;
    const FixedPass f = table.begin(lane_max);
    // One tap at a time (the tap index is uniform): unrolled, the taps' table updates would
    // interleave and hold many more registers. In 2D, neighbouring pixels of a tile row whose
    // tap falls on the same texel sum first, and the last of them adds the sum (cube faces
    // give fewer such runs than the summing costs).
#pragma unroll 1
    for (int k = 0; k < 8; ++k) {
      const uint32_t key = tap_key[k];
      float v[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = gc[c] * tap_weight[k];
      if constexpr (CUBE) {
        table.add_wave(key, v, n, grad_texels + c0, C, f);
      } else {
        if (__ballot(key != Table::kEmpty) == 0) continue;  // uniform
        const bool last = row_run_sums(key, v);
        if (last && key != Table::kEmpty) table.add_or_global(key, v, n, grad_texels + c0, C, f);
      }
    }
    __syncthreads();
    table.flush(grad_texels + c0, C, n, f);
    if (c0 + 4 < C) {
      __syncthreads();
      table.reset();
    }
  }
}

// ---- mip chain --------------------------------------------------------------------------

// Weight of source texel i in destination texel r along an axis of n source texels: the
// overlap of their extents when n texels are split into ceil(n / 2) equal bins, over the bin
// width (reference.py:449-488). Exact integers scaled by 1 / n.
__device__ __forceinline__ float axis_weight(int r, int i, int n) {
  if (n == 1) return (r == 0 && i == 0) ? 1.0f : 0.0f;
  if ((n & 1) == 0) return (i >> 1) == r ? 0.5f : 0.0f;
  const int m = (n + 1) / 2;
  const int overlap = min((r + 1) * n, (i + 1) * m) - max(r * n, i * m);
  return overlap > 0 ? (float)overlap / (float)n : 0.0f;
}

// First source texel and tap count of destination texel r along an axis.
__device__ __forceinline__ void axis_taps(int r, int n, int& first, int& count) {
  if (n == 1) { first = 0; count = 1; return; }
  if ((n & 1) == 0) { first = 2 * r; count = 2; return; }
  const int m = (n + 1) / 2;
  first = (int)((int64_t)r * n / m);
  count = min(3, n - first);
}

struct MipLevels {
  int h[DR_MAX_LEVELS], w[DR_MAX_LEVELS];
  int64_t off[DR_MAX_LEVELS];
};

// Level k + 1 from level k, one thread per destination texel and channel.
__global__ __launch_bounds__(256) void mip_down(float* texels, int C, int64_t num_texels,
                                                       int faces, MipLevels L, int k,
                                                       int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const int h = L.h[k], w = L.w[k], h2 = L.h[k + 1], w2 = L.w[k + 1];
  const int c = (int)(i % C);
  int64_t rest = i / C;
  const int col = (int)(rest % w2);
  rest /= w2;
  const int row = (int)(rest % h2);
  rest /= h2;
  const int face = (int)(rest % faces);
  const int64_t image = rest / faces;
  const float* src = texels + image * num_texels * C + (L.off[k] + (int64_t)face * h * w) * C;
  float* dst = texels + image * num_texels * C + (L.off[k + 1] + (int64_t)face * h2 * w2) * C;
  int r0, nr, c0, nc;
  axis_taps(row, h, r0, nr);
  axis_taps(col, w, c0, nc);
  float sum = 0.0f;
  for (int ri = 0; ri < nr; ++ri) {
    const float wr = axis_weight(row, r0 + ri, h);
    for (int ci = 0; ci < nc; ++ci) {
      const float wc = axis_weight(col, c0 + ci, w);
      sum += (wr * wc) * src[((int64_t)(r0 + ri) * w + (c0 + ci)) * C + c];
    }
  }
  dst[((int64_t)row * w2 + col) * C + c] = sum;
}

// Adjoint of mip_down: source texel (i, j) of level k gathers the gradient of the
// destination texels of level k + 1 whose bins overlap it.
__global__ __launch_bounds__(256) void mip_up(float* grad, int C, int64_t num_texels,
                                                     int faces, MipLevels L, int k,
                                                     int64_t count) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= count) return;
  const int h = L.h[k], w = L.w[k], h2 = L.h[k + 1], w2 = L.w[k + 1];
  const int c = (int)(idx % C);
  int64_t rest = idx / C;
  const int j = (int)(rest % w);
  rest /= w;
  const int i = (int)(rest % h);
  rest /= h;
  const int face = (int)(rest % faces);
  const int64_t image = rest / faces;
  float* src = grad + image * num_texels * C + (L.off[k] + (int64_t)face * h * w) * C;
  const float* dst =
      grad + image * num_texels * C + (L.off[k + 1] + (int64_t)face * h2 * w2) * C;
  // Destination rows (cols) that can overlap source row i (col j).
  const int r_mid = (h & 1) ? (int)((int64_t)i * h2 / h) : i / 2;
  const int c_mid = (w & 1) ? (int)((int64_t)j * w2 / w) : j / 2;
  float sum = 0.0f;
  for (int r = max(r_mid - 1, 0); r <= min(r_mid + 1, h2 - 1); ++r) {
    const float wr = axis_weight(r, i, h);
    if (wr == 0.0f) continue;
    for (int cc = max(c_mid - 1, 0); cc <= min(c_mid + 1, w2 - 1); ++cc) {
      const float wc = axis_weight(cc, j, w);
      if (wc == 0.0f) continue;
      sum += (wr * wc) * dst[((int64_t)r * w2 + cc) * C + c];
    }
  }
  src[((int64_t)i * w + j) * C + c] += sum;
}

// ---- mip chain in tile stages ------------------------------------------------------------
//
// Where a level's sizes are divisible by 2^G (G >= 2), the next G levels halve exactly and each
// texel has exactly one parent: a workgroup then takes a tile of 2^G x 2^G texels of the bottom
// level through all G levels, keeping the levels in between in LDS, instead of one launch (and
// one pass over memory) per level. The arithmetic is mip_down's and mip_up's for even sizes:
// a texel is ((a / 4 + b / 4) + c / 4) + d / 4 of its children in row-major order, and in the
// adjoint a child adds a quarter of its parent's total.

constexpr int kMipStageLevels = 6;  // at most 64 x 64 bottom texels per tile: 32 x 32 above

// Up to four channels of texel p (n valid; vec: four channels on a 16-byte aligned buffer).
__device__ __forceinline__ float4 load_texel(const float* p, int n, bool vec) {
  if (vec) return *reinterpret_cast<const float4*>(p);
  return make_float4(p[0], n > 1 ? p[1] : 0.f, n > 2 ? p[2] : 0.f, n > 3 ? p[3] : 0.f);
}

__device__ __forceinline__ void store_texel(float* p, float4 v, int n, bool vec) {
  if (vec) {
    *reinterpret_cast<float4*>(p) = v;
    return;
  }
  p[0] = v.x;
  if (n > 1) p[1] = v.y;
  if (n > 2) p[2] = v.z;
  if (n > 3) p[3] = v.w;
}

__device__ __forceinline__ float4 quad_mean(float4 a, float4 b, float4 c, float4 d) {
  auto mean = [](float a, float b, float c, float d) {
    return ((0.25f * a + 0.25f * b) + 0.25f * c) + 0.25f * d;
  };
  return make_float4(mean(a.x, b.x, c.x, d.x), mean(a.y, b.y, c.y, d.y),
                     mean(a.z, b.z, c.z, d.z), mean(a.w, b.w, c.w, d.w));
}

__device__ __forceinline__ float4 add_quarter(float4 own, float4 parent) {
  return make_float4(own.x + 0.25f * parent.x, own.y + 0.25f * parent.y,
                     own.z + 0.25f * parent.z, own.w + 0.25f * parent.w);
}

// The tile of this workgroup: (image, face) and tile coordinates in units of 2^G bottom texels.
struct MipTile {
  int64_t image;
  int face, tx, ty;
};

__device__ __forceinline__ MipTile mip_tile(const MipLevels& L, int k, int G, int faces) {
  const int tiles_x = L.w[k] >> G, tiles_y = L.h[k] >> G;
  int64_t b = blockIdx.x;
  MipTile T;
  T.tx = (int)(b % tiles_x);
  b /= tiles_x;
  T.ty = (int)(b % tiles_y);
  b /= tiles_y;
  T.face = (int)(b % faces);
  T.image = b / faces;
  return T;
}

__device__ __forceinline__ float* mip_level(float* texels, int64_t num_texels, int C,
                                            const MipLevels& L, const MipTile& T, int lvl) {
  return texels + T.image * num_texels * C + (L.off[lvl] + (int64_t)T.face * L.h[lvl] * L.w[lvl]) * C;
}

// Levels k + 1 .. k + G from level k, one tile per workgroup. With `base` (k == 0 only), level
// 0 is read from there -- [images, faces * h * w, C], the layout of level 0 on its own -- and
// copied into the packed buffer on the way (each of its texels is read once).
__global__ __launch_bounds__(256) void mip_down_stage(float* texels, const float* base, int C,
                                                      int64_t num_texels, int faces,
                                                      MipLevels L, int k, int G) {
  __shared__ float4 s_buf[2][1 << (2 * kMipStageLevels - 2)];
  const MipTile T = mip_tile(L, k, G, faces);
  const bool vec = C == 4 && (reinterpret_cast<uintptr_t>(texels) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(base) & 15u) == 0;
  for (int c0 = 0; c0 < C; c0 += 4) {
    const int n = min(4, C - c0);
    int side = 1 << (G - 1);  // the tile's side at level k + 1
    {
      float* level = mip_level(texels, num_texels, C, L, T, k) + c0;
      const float* src =
          base ? base + (T.image * faces + T.face) * (int64_t)L.h[0] * L.w[0] * C + c0 : level;
      float* dst = mip_level(texels, num_texels, C, L, T, k + 1) + c0;
      const int64_t w = L.w[k], w1 = L.w[k + 1];
      for (int i = threadIdx.x; i < side * side; i += blockDim.x) {
        const int r = T.ty * side + i / side, c = T.tx * side + i % side;
        const int64_t at = ((int64_t)(2 * r) * w + 2 * c) * C;
        const float* p = src + at;
        const float4 a = load_texel(p, n, vec), b = load_texel(p + C, n, vec);
        const float4 cc = load_texel(p + w * C, n, vec), d = load_texel(p + w * C + C, n, vec);
        if (base) {
          float* q = level + at;
          store_texel(q, a, n, vec);
          store_texel(q + C, b, n, vec);
          store_texel(q + w * C, cc, n, vec);
          store_texel(q + w * C + C, d, n, vec);
        }
        const float4 o = quad_mean(a, b, cc, d);
        store_texel(dst + ((int64_t)r * w1 + c) * C, o, n, vec);
        s_buf[0][i] = o;
      }
    }
    int cur = 0;
    for (int lvl = k + 2; lvl <= k + G; ++lvl) {
      __syncthreads();
      const int below = side;
      side >>= 1;
      float* dst = mip_level(texels, num_texels, C, L, T, lvl) + c0;
      const int64_t wl = L.w[lvl];
      const float4* s = s_buf[cur];
      for (int i = threadIdx.x; i < side * side; i += blockDim.x) {
        const int r = i / side, c = i % side;
        const float4* q = s + 2 * r * below + 2 * c;
        const float4 o = quad_mean(q[0], q[1], q[below], q[below + 1]);
        store_texel(dst + ((int64_t)(T.ty * side + r) * wl + T.tx * side + c) * C, o, n, vec);
        s_buf[cur ^ 1][i] = o;
      }
      cur ^= 1;
    }
    __syncthreads();  // the next channel group reuses the LDS
  }
}

// Adjoint of mip_down_stage: the totals of level k + G (final: the stages above ran first) fold
// down through levels k + G - 1 .. k of the tile, each texel adding a quarter of its parent's
// total to its own gradient, which becomes its total.
__global__ __launch_bounds__(256) void mip_up_stage(float* grad, int C, int64_t num_texels,
                                                    int faces, MipLevels L, int k, int G) {
  __shared__ float4 s_buf[2][1 << (2 * kMipStageLevels - 2)];
  const MipTile T = mip_tile(L, k, G, faces);
  const bool vec = C == 4 && (reinterpret_cast<uintptr_t>(grad) & 15u) == 0;
  for (int c0 = 0; c0 < C; c0 += 4) {
    const int n = min(4, C - c0);
    int cur = 0;
    if (threadIdx.x == 0) {
      const float* top = mip_level(grad, num_texels, C, L, T, k + G) + c0;
      s_buf[0][0] = load_texel(top + ((int64_t)T.ty * L.w[k + G] + T.tx) * C, n, vec);
    }
    int side = 1;  // the tile's side at the level in s_buf[cur]
    for (int lvl = k + G - 1; lvl >= k; --lvl) {
      __syncthreads();
      const int above = side;
      side <<= 1;
      float* g = mip_level(grad, num_texels, C, L, T, lvl) + c0;
      const int64_t wl = L.w[lvl];
      const float4* s = s_buf[cur];
      for (int i = threadIdx.x; i < side * side; i += blockDim.x) {
        const int r = i / side, c = i % side;
        float* p = g + ((int64_t)(T.ty * side + r) * wl + T.tx * side + c) * C;
        const float4 o = add_quarter(load_texel(p, n, vec), s[(r >> 1) * above + (c >> 1)]);
        store_texel(p, o, n, vec);
        if (lvl > k) s_buf[cur ^ 1][i] = o;
      }
      cur ^= 1;
    }
    __syncthreads();  // the next channel group reuses the LDS
  }
}

// Tile stages and single levels of a chain: stage (k, G) builds levels k + 1 .. k + G, in one
// tile-stage launch when G >= 2, else (G == 1) with mip_down.
struct MipPlan {
  int count;
  int k[DR_MAX_LEVELS], G[DR_MAX_LEVELS];
};

MipPlan mip_plan(const MipLevels& L, int num_levels) {
  MipPlan P{};
  for (int k = 0; k + 1 < num_levels;) {
    int G = 0;
    while (G < kMipStageLevels && k + G + 1 < num_levels && L.h[k] % (2 << G) == 0 &&
           L.w[k] % (2 << G) == 0)
      ++G;
    if (G < 2) G = 1;
    P.k[P.count] = k;
    P.G[P.count] = G;
    ++P.count;
    k += G;
  }
  return P;
}

int64_t stage_tiles(const MipLevels& L, int k, int G, int64_t images) {
  return images * (int64_t)(L.h[k] >> G) * (L.w[k] >> G);
}

bool valid_levels(int num_levels, const int32_t* h, const int32_t* w, const int64_t* off) {
  if (num_levels < 1 || num_levels > DR_MAX_LEVELS || !h || !w || !off) return false;
  for (int k = 0; k < num_levels; ++k)
    if (h[k] <= 0 || w[k] <= 0 || off[k] < 0) return false;
  for (int k = 0; k + 1 < num_levels; ++k)
    if (h[k + 1] != (h[k] + 1) / 2 || w[k + 1] != (w[k] + 1) / 2) return false;
  return true;
}

MipLevels copy_levels(int n, const int32_t* h, const int32_t* w, const int64_t* off) {
  MipLevels L{};
  for (int k = 0; k < n; ++k) {
    L.h[k] = h[k];
    L.w[k] = w[k];
    L.off[k] = off[k];
  }
  return L;
}

bool valid_args(const DrTextureArgs* a) {
  if (!a || !a->texels || !a->uv || a->batch < 0 || a->height <= 0 || a->width <= 0) return false;
  if (a->channels <= 0 || a->tex_batch < 1 || a->num_levels < 1 || a->num_levels > DR_MAX_LEVELS)
    return false;
  if (a->filter < 0 || a->filter > 3 || a->boundary < 0 || a->boundary > 3) return false;
  if ((a->boundary == DR_BOUNDARY_CUBE) != (a->faces == 6)) return false;
  if (a->faces != 1 && a->faces != 6) return false;
  for (int k = 0; k < a->num_levels; ++k)
    if (a->level_height[k] <= 0 || a->level_width[k] <= 0) return false;
  return true;
}

// Kernels templated on NC channels per pass: 1-4 as they are, more in passes of 4.
template <typename F>
int dispatch_channels(int channels, F f) {
  switch (channels) {
    case 1: return f(std::integral_constant<int, 1>());
    case 2: return f(std::integral_constant<int, 2>());
    case 3: return f(std::integral_constant<int, 3>());
    default: return f(std::integral_constant<int, 4>());
  }
}

}  // namespace
}  // namespace dr

using namespace dr;

extern "C" int dr_texture_forward(const DrTextureArgs* a, float* out, void* stream) {
  if (!valid_args(a) || !out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  const DrTextureArgs args = *a;
  const bool cube = args.boundary == DR_BOUNDARY_CUBE;
  return dispatch_channels(args.channels, [&](auto nc) {
    constexpr int NC = decltype(nc)::value;
    if (cube)
      tex_fwd_kernel<NC, true><<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(args, out);
    else
      tex_fwd_kernel<NC, false><<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(args, out);
    return launch_status();
  });
}

extern "C" int dr_texture_backward(const DrTextureArgs* a, const float* grad_out,
                                   float* grad_texels, float* grad_uv, float* grad_uv_da,
                                   float* grad_bias, void* stream) {
  if (!valid_args(a) || !grad_out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  if ((int64_t)a->tex_batch * a->num_texels >= 0xffffffffLL) return DR_ERR_ARGUMENT;
  const DrTextureArgs args = *a;
  const bool cube = args.boundary == DR_BOUNDARY_CUBE;
  const int64_t blocks = tile_blocks(args.batch, args.height, args.width);
  float* g_da = args.uv_da ? grad_uv_da : nullptr;
  float* g_bias = args.bias ? grad_bias : nullptr;
  return dispatch_channels(args.channels, [&](auto nc) {
    constexpr int NC = decltype(nc)::value;
    if (cube)
      tex_bwd_kernel<NC, true><<<blocks, 256, 0, (hipStream_t)stream>>>(
          args, grad_out, grad_texels, grad_uv, g_da, g_bias);
    else
      tex_bwd_kernel<NC, false><<<blocks, 256, 0, (hipStream_t)stream>>>(
          args, grad_out, grad_texels, grad_uv, g_da, g_bias);
    return launch_status();
  });
}

// Copies level 0 from its own array into the packed buffer (when no tile stage does it):
// `count` values, base_values per batch entry of `base`, packed_values per entry of `texels`.
__global__ __launch_bounds__(256) void mip_copy_base(float* texels, const float* base,
                                                     int64_t packed_values, int64_t base_values,
                                                     int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const int64_t image = i / base_values, v = i - image * base_values;
  texels[image * packed_values + v] = base[i];
}

extern "C" int dr_mip_build(float* texels, const float* base, int32_t tex_batch,
                            int32_t channels, int64_t num_texels, int32_t faces,
                            int32_t num_levels, const int32_t* level_height,
                            const int32_t* level_width, const int64_t* level_offset,
                            void* stream) {
  if (!texels || tex_batch < 1 || channels < 1 || (faces != 1 && faces != 6) ||
      !valid_levels(num_levels, level_height, level_width, level_offset))
    return DR_ERR_ARGUMENT;
  const MipLevels L = copy_levels(num_levels, level_height, level_width, level_offset);
  const MipPlan P = mip_plan(L, num_levels);
  const int64_t images = (int64_t)tex_batch * faces;
  const int64_t base_texels = (int64_t)faces * L.h[0] * L.w[0];
  if (base != nullptr && base_texels > num_texels) return DR_ERR_ARGUMENT;
  // Level 0 from `base`: the first tile stage copies it as it reads it; otherwise a copy first.
  const bool staged_copy = base != nullptr && P.count > 0 && P.G[0] >= 2;
  if (base != nullptr && !staged_copy) {
    const int64_t count = (int64_t)tex_batch * base_texels * channels;
    mip_copy_base<<<blocks_for(count, 256), 256, 0, (hipStream_t)stream>>>(
        texels, base, num_texels * channels, base_texels * channels, count);
  }
  for (int s = 0; s < P.count; ++s) {
    const int k = P.k[s], G = P.G[s];
    if (G >= 2) {
      mip_down_stage<<<(unsigned)stage_tiles(L, k, G, images), 256, 0, (hipStream_t)stream>>>(
          texels, s == 0 && staged_copy ? base : nullptr, channels, num_texels, faces, L, k, G);
      continue;
    }
    const int64_t count = images * L.h[k + 1] * L.w[k + 1] * channels;
    mip_down<<<blocks_for(count, 256), 256, 0, (hipStream_t)stream>>>(
        texels, channels, num_texels, faces, L, k, count);
  }
  return launch_status();
}

extern "C" int dr_mip_build_backward(float* grad_texels, int32_t tex_batch, int32_t channels,
                                     int64_t num_texels, int32_t faces, int32_t num_levels,
                                     const int32_t* level_height, const int32_t* level_width,
                                     const int64_t* level_offset, void* stream) {
  if (!grad_texels || tex_batch < 1 || channels < 1 || (faces != 1 && faces != 6) ||
      !valid_levels(num_levels, level_height, level_width, level_offset))
    return DR_ERR_ARGUMENT;
  const MipLevels L = copy_levels(num_levels, level_height, level_width, level_offset);
  const MipPlan P = mip_plan(L, num_levels);
  const int64_t images = (int64_t)tex_batch * faces;
  for (int s = P.count - 1; s >= 0; --s) {
    const int k = P.k[s], G = P.G[s];
    if (G >= 2) {
      mip_up_stage<<<(unsigned)stage_tiles(L, k, G, images), 256, 0, (hipStream_t)stream>>>(
          grad_texels, channels, num_texels, faces, L, k, G);
      continue;
    }
    const int64_t count = images * L.h[k] * L.w[k] * channels;
    mip_up<<<blocks_for(count, 256), 256, 0, (hipStream_t)stream>>>(
        grad_texels, channels, num_texels, faces, L, k, count);
  }
  return launch_status();
}
