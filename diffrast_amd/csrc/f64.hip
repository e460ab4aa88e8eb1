// float64 variants of resolve, interpolate, texture and antialias, for gradient-check-grade
// work: the reference's GPU backend accepts float64 tensors at the backend level and computes
// in double (its tests: resolve to 1e-12, tests/test_coverage.py:792-808; interpolate and texture
// gradcheck, tests/test_triton.py:234-240, :303-319; antialias to 1e-9, :408-415).
//
// These kernels favour plain structure over speed: one thread per pixel, gradient scatters with
// float64 atomics. The arithmetic is the reference backend's (src/diffrast/backends/reference.py)
// evaluated in double. Visibility is not here: as in the reference's GPU backend, it runs on a
// float32 copy of the positions (raster.hip) and only the resolve is float64.
#include <float.h>

#include "common.h"
#include "texture_math.h"

namespace dr {
namespace f64 {
namespace {

using tex::as;

__device__ __forceinline__ double centre(int i, int size) {
  return (double)(2 * i + 1) / (double)size - 1.0;  // reference.py:268-271, in float64
}

__device__ __forceinline__ void add64(double* p, double v) { unsafeAtomicAdd(p, v); }

// ---- resolve (reference.py:69-114, 274-290) --------------------------------------------------

struct Tri64 {
  double x[3], y[3], z[3], w[3];
  int64_t row[3];  // vertex rows of pos (image offset included)
};

__device__ __forceinline__ void load_tri64(const DrRasterGeometry& g, int b, int t, Tri64& T) {
  const double* P = as<double>(g.pos);
  const int64_t base = (int64_t)b * (g.pos_batch_stride / 4);
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    T.row[k] = base + g.tri[3 * (int64_t)t + k];
    const double* p = P + 4 * T.row[k];
    T.x[k] = p[0];
    T.y[k] = p[1];
    T.z[k] = p[2];
    T.w[k] = p[3];
  }
}

struct Res64 {
  double a[3], c[3], e[3], area, b[3], depth, num, den, dex[3], dey[3], sdx, sdy;
  double db_dx[3], db_dy[3];
};

__device__ __forceinline__ void resolve64(const Tri64& T, double px, double py, Res64& R) {
  for (int k = 0; k < 3; ++k) {
    R.a[k] = T.x[k] - px * T.w[k];
    R.c[k] = T.y[k] - py * T.w[k];
  }
  R.e[0] = R.a[1] * R.c[2] - R.a[2] * R.c[1];
  R.e[1] = R.a[2] * R.c[0] - R.a[0] * R.c[2];
  R.e[2] = R.a[0] * R.c[1] - R.a[1] * R.c[0];
  R.area = R.e[0] + R.e[1] + R.e[2];
  for (int k = 0; k < 3; ++k) R.b[k] = R.e[k] / R.area;
  R.num = R.b[0] * T.z[0] + R.b[1] * T.z[1] + R.b[2] * T.z[2];
  R.den = R.b[0] * T.w[0] + R.b[1] * T.w[1] + R.b[2] * T.w[2];
  R.depth = R.num / R.den;
  R.dex[0] = T.w[2] * R.c[1] - T.w[1] * R.c[2];
  R.dex[1] = T.w[0] * R.c[2] - T.w[2] * R.c[0];
  R.dex[2] = T.w[1] * R.c[0] - T.w[0] * R.c[1];
  R.dey[0] = R.a[2] * T.w[1] - R.a[1] * T.w[2];
  R.dey[1] = R.a[0] * T.w[2] - R.a[2] * T.w[0];
  R.dey[2] = R.a[1] * T.w[0] - R.a[0] * T.w[1];
  R.sdx = R.dex[0] + R.dex[1] + R.dex[2];
  R.sdy = R.dey[0] + R.dey[1] + R.dey[2];
  for (int k = 0; k < 3; ++k) {
    R.db_dx[k] = (R.dex[k] - R.b[k] * R.sdx) / R.area;
    R.db_dy[k] = (R.dey[k] - R.b[k] * R.sdy) / R.area;
  }
}

struct Pix {
  int b, x, y;
};

__device__ __forceinline__ Pix split(int64_t i, int height, int width) {
  Pix p;
  p.x = (int)(i % width);
  const int64_t r = i / width;
  p.y = (int)(r % height);
  p.b = (int)(r / height);
  return p;
}

__global__ __launch_bounds__(256) void resolve_fwd(DrRasterGeometry g, const uint64_t* keys,
                                                   double* rast, double* rast_db, double sx,
                                                   double sy) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)g.batch * g.height * g.width) return;
  double* r = rast + 4 * i;
  double* d = rast_db ? rast_db + 4 * i : nullptr;
  if (keys[i] == kEmptyKey) {
    for (int k = 0; k < 4; ++k) {
      r[k] = 0.0;
      if (d) d[k] = 0.0;
    }
    return;
  }
  const int t = (int)(uint32_t)keys[i];
  const Pix p = split(i, g.height, g.width);
  Tri64 T;
  load_tri64(g, p.b, t, T);
  Res64 R;
  resolve64(T, centre(p.x, g.width), centre(p.y, g.height), R);
  r[0] = R.b[0];
  r[1] = R.b[1];
  r[2] = R.depth;
  r[3] = (double)(t + 1);
  if (d) {
    d[0] = R.db_dx[0] * sx;
    d[1] = R.db_dy[0] * sy;
    d[2] = R.db_dx[1] * sx;
    d[3] = R.db_dy[1] * sy;
  }
}

// Reverse mode of resolve64 (the same steps as resolve_bwd_kernel's float32 ones).
__global__ __launch_bounds__(256) void resolve_bwd(DrRasterGeometry g, const uint64_t* keys,
                                                   const double* grad_rast,
                                                   const double* grad_db, double* grad_pos,
                                                   double sx, double sy) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)g.batch * g.height * g.width || keys[i] == kEmptyKey) return;
  const int t = (int)(uint32_t)keys[i];
  const Pix p = split(i, g.height, g.width);
  Tri64 T;
  load_tri64(g, p.b, t, T);
  const double px = centre(p.x, g.width), py = centre(p.y, g.height);
  Res64 R;
  resolve64(T, px, py, R);
  const double* gr = grad_rast + 4 * i;
  double gb[3] = {gr[0], gr[1], 0.0}, gz[3], gw[3];
  const double g_num = gr[2] / R.den, g_den = -gr[2] * R.depth / R.den;
  for (int k = 0; k < 3; ++k) {
    gb[k] += g_num * T.z[k] + g_den * T.w[k];
    gz[k] = g_num * R.b[k];
    gw[k] = g_den * R.b[k];
  }
  double g_area = 0.0, g_dex[3] = {0, 0, 0}, g_dey[3] = {0, 0, 0};
  if (grad_db) {
    const double* gd = grad_db + 4 * i;
    const double gx[3] = {gd[0] * sx, gd[2] * sx, 0.0}, gy[3] = {gd[1] * sy, gd[3] * sy, 0.0};
    double dot_x = 0.0, dot_y = 0.0;
    for (int k = 0; k < 3; ++k) {
      dot_x += gx[k] * R.b[k];
      dot_y += gy[k] * R.b[k];
      gb[k] -= (gx[k] * R.sdx + gy[k] * R.sdy) / R.area;
      g_area -= (gx[k] * R.db_dx[k] + gy[k] * R.db_dy[k]) / R.area;
    }
    for (int k = 0; k < 3; ++k) {
      g_dex[k] = (gx[k] - dot_x) / R.area;
      g_dey[k] = (gy[k] - dot_y) / R.area;
    }
  }
  double dot_b = 0.0;
  for (int k = 0; k < 3; ++k) dot_b += gb[k] * R.b[k];
  g_area -= dot_b / R.area;
  double ge[3];
  for (int k = 0; k < 3; ++k) ge[k] = gb[k] / R.area + g_area;
  // e = a x c, dex = c x w, dey = w x a: for u x v with upstream G, grad u = v x G and
  // grad v = G x u.
  auto cross = [](const double* u, const double* v, double* o) {
    o[0] = u[1] * v[2] - u[2] * v[1];
    o[1] = u[2] * v[0] - u[0] * v[2];
    o[2] = u[0] * v[1] - u[1] * v[0];
  };
  double ga[3], gc[3], tmp[3];
  cross(R.c, ge, ga);
  cross(ge, R.a, gc);
  cross(T.w, g_dex, tmp);
  for (int k = 0; k < 3; ++k) gc[k] += tmp[k];
  cross(g_dex, R.c, tmp);
  for (int k = 0; k < 3; ++k) gw[k] += tmp[k];
  cross(R.a, g_dey, tmp);
  for (int k = 0; k < 3; ++k) gw[k] += tmp[k];
  cross(g_dey, T.w, tmp);
  for (int k = 0; k < 3; ++k) ga[k] += tmp[k];
  for (int k = 0; k < 3; ++k) {
    double* q = grad_pos + 4 * T.row[k];
    add64(q + 0, ga[k]);
    add64(q + 1, gc[k]);
    add64(q + 2, gz[k]);
    add64(q + 3, gw[k] - px * ga[k] - py * gc[k]);
  }
}

// ---- interpolate (reference.py:117-146) -------------------------------------------------------

__device__ __forceinline__ int rast_tri(const double* r, int num_tri) {
  const double id = rint(r[3]);
  return (id >= 1.0 && id <= (double)num_tri) ? (int)id - 1 : -1;
}

__global__ __launch_bounds__(256) void interp_fwd(DrInterpolateArgs a, double* out,
                                                  double* out_da) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.batch * a.height * a.width) return;
  const int C = a.channels, D = a.num_diff;
  const double* r = as<double>(a.rast) + 4 * i;
  const int t = rast_tri(r, a.num_tri);
  double* o = out + i * C;
  double* od = out_da ? out_da + i * 2 * D : nullptr;
  if (t < 0) {
    for (int c = 0; c < C; ++c) o[c] = 0.0;
    for (int k = 0; k < 2 * D && od; ++k) od[k] = 0.0;
    return;
  }
  const int b = (int)(i / ((int64_t)a.height * a.width));
  const double* A = as<double>(a.attr) + (int64_t)b * a.attr_batch_stride;
  const double* a0 = A + (int64_t)a.tri[3 * (int64_t)t] * C;
  const double* a1 = A + (int64_t)a.tri[3 * (int64_t)t + 1] * C;
  const double* a2 = A + (int64_t)a.tri[3 * (int64_t)t + 2] * C;
  const double u = r[0], v = r[1];
  for (int c = 0; c < C; ++c) o[c] = u * a0[c] + v * a1[c] + (1.0 - u - v) * a2[c];
  if (!od) return;
  const double* db = as<double>(a.rast_db) + 4 * i;
  for (int k = 0; k < D; ++k) {
    const int c = a.diff[k];
    const double du = a0[c] - a2[c], dv = a1[c] - a2[c];
    od[2 * k] = db[0] * du + db[2] * dv;
    od[2 * k + 1] = db[1] * du + db[3] * dv;
  }
}

__global__ __launch_bounds__(256) void interp_bwd(DrInterpolateArgs a, const double* grad_out,
                                                  const double* grad_da, double* grad_attr,
                                                  double* grad_rast, double* grad_db) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.batch * a.height * a.width) return;
  const int C = a.channels, D = a.num_diff;
  const double* r = as<double>(a.rast) + 4 * i;
  const int t = rast_tri(r, a.num_tri);
  double gu = 0.0, gv = 0.0, gd[4] = {0.0, 0.0, 0.0, 0.0};
  if (t >= 0) {
    const int b = (int)(i / ((int64_t)a.height * a.width));
    const int64_t offset = (int64_t)b * a.attr_batch_stride;
    const double* A = as<double>(a.attr) + offset;
    const int64_t rows[3] = {a.tri[3 * (int64_t)t], a.tri[3 * (int64_t)t + 1],
                             a.tri[3 * (int64_t)t + 2]};
    const double u = r[0], v = r[1], wgt[3] = {u, v, 1.0 - u - v};
    const double* g = grad_out + i * C;
    for (int c = 0; c < C; ++c) {
      gu += g[c] * (A[rows[0] * C + c] - A[rows[2] * C + c]);
      gv += g[c] * (A[rows[1] * C + c] - A[rows[2] * C + c]);
      if (grad_attr)
        for (int k = 0; k < 3; ++k) add64(grad_attr + offset + rows[k] * C + c, g[c] * wgt[k]);
    }
    if (D > 0 && grad_da != nullptr) {
      const double* db = as<double>(a.rast_db) + 4 * i;
      const double* gda = grad_da + i * 2 * D;
      for (int k = 0; k < D; ++k) {
        const int c = a.diff[k];
        const double gx = gda[2 * k], gy = gda[2 * k + 1];
        const double du = A[rows[0] * C + c] - A[rows[2] * C + c];
        const double dv = A[rows[1] * C + c] - A[rows[2] * C + c];
        gd[0] += gx * du;
        gd[1] += gy * du;
        gd[2] += gx * dv;
        gd[3] += gy * dv;
        if (grad_attr) {
          const double g0 = gx * db[0] + gy * db[1], g1 = gx * db[2] + gy * db[3];
          add64(grad_attr + offset + rows[0] * C + c, g0);
          add64(grad_attr + offset + rows[1] * C + c, g1);
          add64(grad_attr + offset + rows[2] * C + c, -g0 - g1);
        }
      }
    }
  }
  if (grad_rast) {
    double* q = grad_rast + 4 * i;
    q[0] = gu;
    q[1] = gv;
    q[2] = 0.0;
    q[3] = 0.0;
  }
  if (grad_db)
    for (int k = 0; k < 4; ++k) grad_db[4 * i + k] = gd[k];
}

// ---- texture -----------------------------------------------------------------------------------

using tex::Bilinear;
using tex::Lookup;

template <bool CUBE>
__global__ __launch_bounds__(256) void tex_fwd(DrTextureArgs a, double* out) {
  const int64_t pixel = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (pixel >= (int64_t)a.batch * a.height * a.width) return;
  const int C = a.channels;
  double* o = out + pixel * C;
  Lookup<double> K;
  tex::lookup_setup<double, CUBE>(a, pixel, K);
  if (K.dir_invalid) {
    for (int c = 0; c < C; ++c) o[c] = 0.0;
    return;
  }
  const int64_t image = pixel / ((int64_t)a.height * a.width);
  const double* texels = as<double>(a.texels) + (a.tex_batch > 1 ? image * a.num_texels * C : 0);
  const double nan = tex::s_nan<double>();
  if (K.levels == 0) {
    uint32_t index;
    bool valid;
    const bool bad = tex::nearest_setup(a, K, index, valid);
    for (int c = 0; c < C; ++c) o[c] = bad ? nan : (valid ? texels[(int64_t)index * C + c] : 0.0);
    return;
  }
  const tex::LevelDims D = tex::lookup_levels(a, K);
  const Bilinear<double> L0 = tex::level_setup<CUBE>(a, K, D, 0);
  const bool two = K.levels == 2;
  const Bilinear<double> L1 = two ? tex::level_setup<CUBE>(a, K, D, 1) : L0;
  const bool bad = K.bad || L0.bad || (two && L1.bad);
  const double frac = K.level_weight[1];
  for (int c = 0; c < C; ++c) {
    double t0[4], t1[4];
    for (int k = 0; k < 4; ++k) {
      t0[k] = L0.valid[k] ? texels[(int64_t)L0.index[k] * C + c] : 0.0;
      t1[k] = two && L1.valid[k] ? texels[(int64_t)L1.index[k] * C + c] : 0.0;
    }
    double v = tex::bilinear_value(L0, t0);
    if (two) v = v * (1.0 - frac) + tex::bilinear_value(L1, t1) * frac;
    o[c] = bad ? nan : v;
  }
}

template <bool CUBE>
__global__ __launch_bounds__(256) void tex_bwd(DrTextureArgs a, const double* grad_out,
                                               double* grad_texels, double* grad_uv,
                                               double* grad_uv_da, double* grad_bias) {
  const int64_t pixel = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (pixel >= (int64_t)a.batch * a.height * a.width) return;
  const int C = a.channels;
  const double* g = grad_out + pixel * C;
  const int64_t image = pixel / ((int64_t)a.height * a.width);
  const int64_t tex_off = a.tex_batch > 1 ? image * a.num_texels : 0;
  const double* texels = as<double>(a.texels) + tex_off * C;
  double* gt = grad_texels ? grad_texels + tex_off * C : nullptr;
  Lookup<double> K;
  tex::lookup_setup<double, CUBE>(a, pixel, K);
  bool live = !K.dir_invalid;
  double g_s = 0.0, g_t = 0.0, g_lod = 0.0;
  if (live && K.levels == 0) {
    uint32_t index;
    bool valid;
    const bool bad = tex::nearest_setup(a, K, index, valid);
    if (!bad && valid && gt)
      for (int c = 0; c < C; ++c) add64(gt + (int64_t)index * C + c, g[c]);
    live = false;  // nearest passes no coordinate gradient
  } else if (live) {
    const tex::LevelDims D = tex::lookup_levels(a, K);
    const Bilinear<double> L[2] = {tex::level_setup<CUBE>(a, K, D, 0),
                                   K.levels == 2 ? tex::level_setup<CUBE>(a, K, D, 1)
                                                 : tex::level_setup<CUBE>(a, K, D, 0)};
    const int levels = K.levels;
    if (K.bad || L[0].bad || (levels == 2 && L[1].bad)) {
      live = false;
    } else {
      double value[2] = {0.0, 0.0};
      for (int l = 0; l < levels; ++l) {
        double g_fx = 0.0, g_fy = 0.0;
        for (int c = 0; c < C; ++c) {
          double t[4], wgt[4], dfx, dfy;
          for (int k = 0; k < 4; ++k) t[k] = L[l].valid[k] ? texels[(int64_t)L[l].index[k] * C + c] : 0.0;
          tex::bilinear_grad(L[l], t, wgt, dfx, dfy);
          const double gl = g[c] * K.level_weight[l];
          g_fx += gl * dfx;
          g_fy += gl * dfy;
          value[l] += g[c] * tex::bilinear_value(L[l], t);
          if (gt)
            for (int k = 0; k < 4; ++k)
              if (L[l].valid[k] && wgt[k] * K.level_weight[l] != 0.0)
                add64(gt + (int64_t)L[l].index[k] * C + c, gl * wgt[k]);
        }
        if (L[l].pass_x) g_s += g_fx * L[l].size_x;
        if (L[l].pass_y) g_t += g_fy * L[l].size_y;
      }
      if (levels == 2 && K.lod_grad) g_lod = value[1] - value[0];
    }
  }
  double g_da[4] = {0.0, 0.0, 0.0, 0.0};
  const bool has_da = K.mip && a.uv_da != nullptr;
  if (live && has_da && g_lod != 0.0) {
    const tex::Deriv4<double> da =
        CUBE ? tex::Deriv4<double>{K.P.st_da[0], K.P.st_da[1], K.P.st_da[2], K.P.st_da[3]}
             : tex::load_deriv4(as<double>(a.uv_da) + 4 * pixel);
    tex::footprint_lod_grad(da, a.level_height[0], a.level_width[0], g_lod, g_da);
  }
  if (grad_bias) grad_bias[pixel] = live ? g_lod : 0.0;
  if (CUBE) {
    double gdir[3] = {0, 0, 0}, gdir_da[6] = {0, 0, 0, 0, 0, 0};
    if (live) tex::cube_project_backward(K.P, g_s, g_t, has_da, g_da, gdir, gdir_da);
    if (grad_uv)
      for (int k = 0; k < 3; ++k) grad_uv[3 * pixel + k] = gdir[k];
    if (grad_uv_da)
      for (int k = 0; k < 6; ++k) grad_uv_da[6 * pixel + k] = gdir_da[k];
  } else {
    if (grad_uv) {
      grad_uv[2 * pixel] = live ? g_s : 0.0;
      grad_uv[2 * pixel + 1] = live ? g_t : 0.0;
    }
    if (grad_uv_da)
      for (int k = 0; k < 4; ++k) grad_uv_da[4 * pixel + k] = live ? g_da[k] : 0.0;
  }
}

// ---- mip chain (reference.py:433-488) ------------------------------------------------------

// Weight of source texel i in destination texel r along an axis of n source texels: the overlap
// of their extents when n texels are split into ceil(n / 2) equal bins, over the bin width.
__device__ __forceinline__ double axis_weight(int r, int i, int n) {
  if (n == 1) return (r == 0 && i == 0) ? 1.0 : 0.0;
  if ((n & 1) == 0) return (i >> 1) == r ? 0.5 : 0.0;
  const int m = (n + 1) / 2;
  const int overlap = min((r + 1) * n, (i + 1) * m) - max(r * n, i * m);
  return overlap > 0 ? (double)overlap / (double)n : 0.0;
}

__device__ __forceinline__ void axis_taps(int r, int n, int& first, int& count) {
  if (n == 1) { first = 0; count = 1; return; }
  if ((n & 1) == 0) { first = 2 * r; count = 2; return; }
  const int m = (n + 1) / 2;
  first = (int)((int64_t)r * n / m);
  count = min(3, n - first);
}

struct Levels {
  int h[DR_MAX_LEVELS], w[DR_MAX_LEVELS];
  int64_t off[DR_MAX_LEVELS];
};

// Level k + 1 from level k, one thread per destination texel and channel. With `base`, level k
// (k = 0) is read from there and copied into the packed buffer by the thread of its first tap.
__global__ __launch_bounds__(256) void mip_down(double* texels, const double* base, int C,
                                                int64_t num_texels, int faces, Levels L, int k,
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
  const double* src = base ? base + (image * faces + face) * (int64_t)h * w * C
                           : texels + image * num_texels * C + (L.off[k] + (int64_t)face * h * w) * C;
  double* dst = texels + image * num_texels * C + (L.off[k + 1] + (int64_t)face * h2 * w2) * C;
  int r0, nr, c0, nc;
  axis_taps(row, h, r0, nr);
  axis_taps(col, w, c0, nc);
  double sum = 0.0;
  for (int ri = 0; ri < nr; ++ri) {
    const double wr = axis_weight(row, r0 + ri, h);
    for (int ci = 0; ci < nc; ++ci) {
      const double wc = axis_weight(col, c0 + ci, w);
      sum += (wr * wc) * src[((int64_t)(r0 + ri) * w + (c0 + ci)) * C + c];
    }
  }
  dst[((int64_t)row * w2 + col) * C + c] = sum;
}

__global__ __launch_bounds__(256) void copy_base(double* texels, const double* base,
                                                 int64_t packed_values, int64_t base_values,
                                                 int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const int64_t image = i / base_values;
  texels[image * packed_values + (i - image * base_values)] = base[i];
}

// Adjoint of mip_down: texel (i, j) of level k gathers the gradient of the texels of level k + 1
// whose bins overlap it.
__global__ __launch_bounds__(256) void mip_up(double* grad, int C, int64_t num_texels, int faces,
                                              Levels L, int k, int64_t count) {
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
  double* src = grad + image * num_texels * C + (L.off[k] + (int64_t)face * h * w) * C;
  const double* dst = grad + image * num_texels * C + (L.off[k + 1] + (int64_t)face * h2 * w2) * C;
  const int r_mid = (h & 1) ? (int)((int64_t)i * h2 / h) : i / 2;
  const int c_mid = (w & 1) ? (int)((int64_t)j * w2 / w) : j / 2;
  double sum = 0.0;
  for (int r = max(r_mid - 1, 0); r <= min(r_mid + 1, h2 - 1); ++r) {
    const double wr = axis_weight(r, i, h);
    if (wr == 0.0) continue;
    for (int cc = max(c_mid - 1, 0); cc <= min(c_mid + 1, w2 - 1); ++cc) {
      const double wc = axis_weight(cc, j, w);
      if (wc == 0.0) continue;
      sum += (wr * wc) * dst[((int64_t)r * w2 + cc) * C + c];
    }
  }
  src[((int64_t)i * w + j) * C + c] += sum;
}

// ---- antialias (reference.py:202-265, 675-814) --------------------------------------------------

constexpr double kEdgeTie64 = 4.0 * DBL_EPSILON;  // EDGE_TIE * finfo(float64).eps
constexpr double kAxisTie64 = 1.0 + 1e-4;
constexpr uint8_t kActive = 0x8, kOwnerFirst = 0x4;

struct Tri2 {
  double x[3], y[3], w[3];
  int64_t row[3];
};

__device__ __forceinline__ void load_tri2(const DrAntialiasArgs& a, int b, int t, Tri2& T) {
  const double* P = as<double>(a.pos) + (int64_t)b * a.pos_batch_stride;
  const int64_t base = (int64_t)b * (a.pos_batch_stride / 4);
  for (int k = 0; k < 3; ++k) {
    const int v = a.tri[3 * (int64_t)t + k];
    T.row[k] = base + v;
    T.x[k] = P[4 * (int64_t)v];
    T.y[k] = P[4 * (int64_t)v + 1];
    T.w[k] = P[4 * (int64_t)v + 3];
  }
}

// Silhouette bits of (pos batch, triangle) i (reference.py:790-814): the edge's line as the
// cross product of its vertices' (x, y, w), rounded as torch.linalg.cross rounds it on the CPU
// (the first product exact inside a fused multiply-add, float64 as for float32).
__global__ __launch_bounds__(256) void silhouettes(const double* pos, int64_t stride, int pos_batch,
                                                   const int32_t* tri, int num_tri,
                                                   const int32_t* nbr, uint8_t* mask) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)pos_batch * num_tri) return;
  const int b = (int)(i / num_tri), t = (int)(i - (int64_t)b * num_tri);
  const double* P = pos + (int64_t)b * stride;
  auto xyw = [&](int v, double* o) {
    o[0] = P[4 * (int64_t)v];
    o[1] = P[4 * (int64_t)v + 1];
    o[2] = P[4 * (int64_t)v + 3];
  };
  double p[3][3];
  for (int k = 0; k < 3; ++k) xyw(tri[3 * (int64_t)t + k], p[k]);
  uint8_t bits = 0;
  for (int k = 0; k < 3; ++k) {
    const int partner = nbr[3 * (int64_t)t + k];
    if (partner < 0) {
      bits |= (uint8_t)(1u << k);
      continue;
    }
    const double* s = p[(k + 1) % 3];
    const double* e = p[(k + 2) % 3];
    const double line[3] = {fma(s[1], e[2], -(s[2] * e[1])), fma(s[2], e[0], -(s[0] * e[2])),
                            fma(s[0], e[1], -(s[1] * e[0]))};
    double q[3];
    xyw(tri[partner], q);  // the vertex opposite the partner edge
    auto side = [&](const double* v) {
      const double d = (line[0] * v[0] + line[1] * v[1]) + line[2] * v[2];
      const double x = d * v[2];
      return x > 0.0 ? 1.0 : (x < 0.0 ? -1.0 : 0.0);
    };
    if (side(p[k]) * side(q) > 0.0) bits |= (uint8_t)(1u << k);
  }
  mask[i] = bits;
}

struct Cross64 {
  bool found;
  double t;
  int edge;
};

// Exit of triangle T (shown at the source centre) along the segment to the destination centre.
__device__ __forceinline__ Cross64 crossing64(const Tri2& T, uint8_t sil, bool horizontal,
                                              int width, int height, double sx, double sy,
                                              double dx, double dy) {
  Cross64 out{false, 0.0, 0};
  double es[3], ed[3], slack[3], as_[3], cs[3], ad[3], cd[3];
  for (int k = 0; k < 3; ++k) {
    as_[k] = T.x[k] - sx * T.w[k];
    cs[k] = T.y[k] - sy * T.w[k];
    ad[k] = T.x[k] - dx * T.w[k];
    cd[k] = T.y[k] - dy * T.w[k];
  }
  for (int k = 0; k < 3; ++k) {
    const int i = (k + 1) % 3, j = (k + 2) % 3;
    es[k] = as_[i] * cs[j] - as_[j] * cs[i];
    ed[k] = ad[i] * cd[j] - ad[j] * cd[i];
    const double rxi = fabs(T.x[i]) + fabs(T.w[i]), rxj = fabs(T.x[j]) + fabs(T.w[j]);
    const double ryi = fabs(T.y[i]) + fabs(T.w[i]), ryj = fabs(T.y[j]) + fabs(T.w[j]);
    slack[k] = ((rxi + fabs(ad[i])) * fabs(cd[j]) + (rxj + fabs(ad[j])) * fabs(cd[i]) +
                ryj * fabs(ad[i]) + ryi * fabs(ad[j])) * kEdgeTie64;
  }
  const double sign = (es[0] + es[1] + es[2]) < 0.0 ? -1.0 : 1.0;
  bool any = false;
  double best = HUGE_VAL;
  int edge = 0;
  for (int k = 0; k < 3; ++k) {
    const double span = es[k] - ed[k];
    if ((ed[k] * sign <= slack[k]) && (span * sign > 2.0 * slack[k])) {
      any = true;
      const double t = es[k] / span;
      if (t < best) {
        best = t;
        edge = k;
      }
    }
  }
  if (!any || !((sil >> edge) & 1u)) return out;
  const int i = (edge + 1) % 3, j = (edge + 2) % 3;
  const double steep = fabs(T.w[j] * T.y[i] - T.w[i] * T.y[j]) * (double)height * kAxisTie64;
  const double flat = fabs(T.x[j] * T.w[i] - T.x[i] * T.w[j]) * (double)width;
  if (!(horizontal ? steep >= flat : flat > steep)) return out;
  out.found = true;
  out.t = best;
  out.edge = edge;
  return out;
}

__device__ __forceinline__ int aa_tri(const DrAntialiasArgs& a, int64_t pixel, double& depth) {
  const double* r = as<double>(a.rast) + 4 * pixel;
  depth = r[2];
  const double id = rint(r[3]);
  return (id >= 1.0 && id <= (double)a.num_tri) ? (int)id - 1 : -1;
}

// Per pixel, the pairs with its right and lower neighbours: t and (active, owner, edge) bits.
__global__ __launch_bounds__(256) void aa_pairs(DrAntialiasArgs a, double2* pair_t,
                                                uchar2* pair_bits) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.batch * a.height * a.width) return;
  const Pix p = split(i, a.height, a.width);
  const uint8_t* sil = a.silhouette + (int64_t)p.b * a.silhouette_batch_stride;
  double depth;
  const int id = aa_tri(a, i, depth);
  double t_pair[2] = {0.0, 0.0};
  uint8_t bits[2] = {0, 0};
  for (int dir = 0; dir < 2; ++dir) {
    const bool horizontal = dir == 0;
    if (horizontal ? p.x + 1 >= a.width : p.y + 1 >= a.height) continue;
    const int64_t q = horizontal ? i + 1 : i + a.width;
    double depth_q;
    const int id_q = aa_tri(a, q, depth_q);
    if (id == id_q) continue;
    const double sx = centre(p.x, a.width), sy = centre(p.y, a.height);
    const double qx = horizontal ? centre(p.x + 1, a.width) : sx;
    const double qy = horizontal ? sy : centre(p.y + 1, a.height);
    Cross64 from_p{false, 0.0, 0}, from_q{false, 0.0, 0};
    if (id >= 0) {
      Tri2 T;
      load_tri2(a, a.pos_batch_stride ? p.b : 0, id, T);
      from_p = crossing64(T, sil[id], horizontal, a.width, a.height, sx, sy, qx, qy);
    }
    if (id_q >= 0) {
      Tri2 T;
      load_tri2(a, a.pos_batch_stride ? p.b : 0, id_q, T);
      from_q = crossing64(T, sil[id_q], horizontal, a.width, a.height, qx, qy, sx, sy);
    }
    const bool use_p = from_p.found && (!from_q.found || depth <= depth_q);
    const bool use_q = from_q.found && !use_p;
    if (!use_p && !use_q) continue;
    t_pair[dir] = use_p ? from_p.t : 1.0 - from_q.t;
    bits[dir] = (uint8_t)(kActive | (use_p ? kOwnerFirst : 0) | (use_p ? from_p.edge : from_q.edge));
  }
  pair_t[i] = make_double2(t_pair[0], t_pair[1]);
  pair_bits[i] = make_uchar2(bits[0], bits[1]);
}

// The pixel's (up to) four pairs: right, down (it is the first pixel), left, up (the second).
struct Pairs64 {
  bool active[4], first[4];
  double t[4];
  int64_t other[4];
};

__device__ __forceinline__ Pairs64 pairs_of(const DrAntialiasArgs& a, int64_t i, const Pix& p,
                                            const double2* pair_t, const uchar2* pair_bits) {
  Pairs64 P;
  const int64_t left = i - 1, up = i - a.width;
  P.active[0] = pair_bits[i].x & kActive;
  P.t[0] = pair_t[i].x;
  P.other[0] = i + 1;
  P.active[1] = pair_bits[i].y & kActive;
  P.t[1] = pair_t[i].y;
  P.other[1] = i + a.width;
  P.active[2] = p.x > 0 && (pair_bits[left].x & kActive);
  P.t[2] = p.x > 0 ? pair_t[left].x : 0.0;
  P.other[2] = left;
  P.active[3] = p.y > 0 && (pair_bits[up].y & kActive);
  P.t[3] = p.y > 0 ? pair_t[up].y : 0.0;
  P.other[3] = up;
  for (int n = 0; n < 4; ++n) P.first[n] = n < 2;
  return P;
}

// Weight of the partner's colour difference that pair n gives this pixel (reference.py:253-264).
__device__ __forceinline__ double take(const Pairs64& P, int n) {
  if (!P.active[n]) return 0.0;
  const double t = P.t[n];
  if (P.first[n]) return t < 0.5 ? 0.5 - t : 0.0;
  return t >= 0.5 ? t - 0.5 : 0.0;
}

__global__ __launch_bounds__(256) void aa_blend(DrAntialiasArgs a, const double2* pair_t,
                                                const uchar2* pair_bits, double* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.batch * a.height * a.width) return;
  const Pix p = split(i, a.height, a.width);
  const Pairs64 P = pairs_of(a, i, p, pair_t, pair_bits);
  const int C = a.channels;
  const double* color = as<double>(a.color);
  for (int c = 0; c < C; ++c) {
    const double own = color[i * C + c];
    double v = own;
    for (int n = 0; n < 4; ++n) {
      const double w = take(P, n);
      if (w != 0.0) v += w * (color[P.other[n] * C + c] - own);
    }
    out[i * C + c] = v;
  }
}

// Colour gradient as a gather over the pixel's pairs; the position gradient of each active pair
// (written by its first pixel) through float64 atomics on the two vertices of the owner's edge.
__global__ __launch_bounds__(256) void aa_bwd(DrAntialiasArgs a, const double2* pair_t,
                                              const uchar2* pair_bits, const double* grad_out,
                                              double* grad_color, double* grad_pos) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.batch * a.height * a.width) return;
  const Pix p = split(i, a.height, a.width);
  const Pairs64 P = pairs_of(a, i, p, pair_t, pair_bits);
  const int C = a.channels;
  const double* color = as<double>(a.color);
  if (grad_color) {
    // out_i = c_i + sum_n w_n (c_other - c_i), and each partner j that takes from i adds
    // w_j (c_i - c_j) to its own output.
    for (int c = 0; c < C; ++c) {
      double gsum = grad_out[i * C + c];
      for (int n = 0; n < 4; ++n) {
        const double w = take(P, n);
        if (w != 0.0) gsum -= w * grad_out[i * C + c];
        if (!P.active[n]) continue;
        // The partner's weight on this pixel: the same pair seen from the other side.
        const double t = P.t[n];
        const double wo = P.first[n] ? (t >= 0.5 ? t - 0.5 : 0.0) : (t < 0.5 ? 0.5 - t : 0.0);
        if (wo != 0.0) gsum += wo * grad_out[P.other[n] * C + c];
      }
      grad_color[i * C + c] = gsum;
    }
  }
  if (grad_pos == nullptr) return;
  for (int dir = 0; dir < 2; ++dir) {
    if (!P.active[dir]) continue;
    const uint8_t bits = dir == 0 ? pair_bits[i].x : pair_bits[i].y;
    const bool owner_first = bits & kOwnerFirst;
    const int edge = bits & 3;
    const int64_t q = P.other[dir];
    const double t = P.t[dir];
    // d loss / d t: the pixel taking colour gets (0.5 - t) (c_q - c_p) or (t - 0.5) (c_p - c_q).
    double g_t = 0.0;
    for (int c = 0; c < C; ++c) {
      const double cp = color[i * C + c], cq = color[q * C + c];
      g_t += t < 0.5 ? -grad_out[i * C + c] * (cq - cp) : grad_out[q * C + c] * (cp - cq);
    }
    g_t *= (double)a.boost;
    // t = t_src (owner is the first pixel) or 1 - t_src (owner is the second).
    if (!owner_first) g_t = -g_t;
    const Pix pq = split(q, a.height, a.width);
    const Pix src = owner_first ? p : pq, dst = owner_first ? pq : p;
    double d;
    const int id = aa_tri(a, owner_first ? i : q, d);
    Tri2 T;
    const int img = a.pos_batch_stride ? p.b : 0;
    load_tri2(a, img, id, T);
    const double sx = centre(src.x, a.width), sy = centre(src.y, a.height);
    const double dx = centre(dst.x, a.width), dy = centre(dst.y, a.height);
    const int vi = (edge + 1) % 3, vj = (edge + 2) % 3;
    const double asi = T.x[vi] - sx * T.w[vi], csi = T.y[vi] - sy * T.w[vi];
    const double asj = T.x[vj] - sx * T.w[vj], csj = T.y[vj] - sy * T.w[vj];
    const double adi = T.x[vi] - dx * T.w[vi], cdi = T.y[vi] - dy * T.w[vi];
    const double adj = T.x[vj] - dx * T.w[vj], cdj = T.y[vj] - dy * T.w[vj];
    const double es = asi * csj - asj * csi, ed = adi * cdj - adj * cdi;
    const double span = es - ed;
    const double k_s = g_t * (-ed / (span * span)), k_d = g_t * (es / (span * span));
    // d e / d (x_i, y_i, w_i, x_j, y_j, w_j) at a centre (px, py).
    const double gi[3] = {k_s * csj + k_d * cdj, -k_s * asj - k_d * adj,
                          k_s * (-sx * csj + sy * asj) + k_d * (-dx * cdj + dy * adj)};
    const double gj[3] = {-k_s * csi - k_d * cdi, k_s * asi + k_d * adi,
                          k_s * (sx * csi - sy * asi) + k_d * (dx * cdi - dy * adi)};
    double* qi = grad_pos + 4 * T.row[vi];
    double* qj = grad_pos + 4 * T.row[vj];
    add64(qi + 0, gi[0]);
    add64(qi + 1, gi[1]);
    add64(qi + 3, gi[2]);
    add64(qj + 0, gj[0]);
    add64(qj + 1, gj[1]);
    add64(qj + 3, gj[2]);
  }
}

Levels copy_levels(int n, const int32_t* h, const int32_t* w, const int64_t* off) {
  Levels L{};
  for (int k = 0; k < n; ++k) {
    L.h[k] = h[k];
    L.w[k] = w[k];
    L.off[k] = off[k];
  }
  return L;
}

bool valid_levels(int n, const int32_t* h, const int32_t* w, const int64_t* off) {
  if (n < 1 || n > DR_MAX_LEVELS || !h || !w || !off) return false;
  for (int k = 0; k < n; ++k)
    if (h[k] <= 0 || w[k] <= 0 || off[k] < 0) return false;
  for (int k = 0; k + 1 < n; ++k)
    if (h[k + 1] != (h[k] + 1) / 2 || w[k + 1] != (w[k] + 1) / 2) return false;
  return true;
}

}  // namespace
}  // namespace f64
}  // namespace dr

using namespace dr;

static bool geometry_ok(const DrRasterGeometry* g) {
  return g && g->batch >= 0 && g->height > 0 && g->width > 0 && g->num_tri >= 0 &&
         (g->batch == 0 || g->num_tri == 0 || (g->pos && g->tri));
}

extern "C" int dr_resolve_forward_f64(const DrRasterGeometry* g, const uint64_t* keys,
                                      double* rast, double* rast_db, void* stream) {
  if (!geometry_ok(g) || !rast || (g->batch > 0 && !keys)) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)g->batch * g->height * g->width;
  if (pixels == 0) return DR_OK;
  f64::resolve_fwd<<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(
      *g, keys, rast, rast_db, 2.0 / g->width, 2.0 / g->height);
  return launch_status();
}

extern "C" int dr_resolve_backward_f64(const DrRasterGeometry* g, const uint64_t* keys,
                                       const double* grad_rast, const double* grad_rast_db,
                                       double* grad_pos, void* stream) {
  if (!geometry_ok(g) || !grad_rast || !grad_pos) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)g->batch * g->height * g->width;
  if (pixels == 0) return DR_OK;
  f64::resolve_bwd<<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(
      *g, keys, grad_rast, grad_rast_db, grad_pos, 2.0 / g->width, 2.0 / g->height);
  return launch_status();
}

static bool interp_ok(const DrInterpolateArgs* a) {
  return a && a->batch >= 0 && a->height > 0 && a->width > 0 && a->channels > 0 &&
         a->num_diff >= 0 && (a->num_diff == 0 || (a->rast_db && a->diff)) &&
         (a->batch == 0 || (a->attr && a->rast && (a->num_tri == 0 || a->tri)));
}

extern "C" int dr_interpolate_forward_f64(const DrInterpolateArgs* a, double* out,
                                          double* out_da, void* stream) {
  if (!interp_ok(a) || !out || (a->num_diff > 0 && !out_da)) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  f64::interp_fwd<<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(
      *a, out, a->num_diff > 0 ? out_da : nullptr);
  return launch_status();
}

extern "C" int dr_interpolate_backward_f64(const DrInterpolateArgs* a, const double* grad_out,
                                           const double* grad_out_da, double* grad_attr,
                                           double* grad_rast, double* grad_rast_db,
                                           void* stream) {
  if (!interp_ok(a) || !grad_out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  f64::interp_bwd<<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(
      *a, grad_out, a->num_diff > 0 ? grad_out_da : nullptr, grad_attr, grad_rast,
      a->num_diff > 0 ? grad_rast_db : nullptr);
  return launch_status();
}

static bool texture_ok(const DrTextureArgs* a) {
  if (!a || !a->texels || !a->uv || a->batch < 0 || a->height <= 0 || a->width <= 0) return false;
  // Texel indices within an image's packed buffer are 32-bit.
  if (a->num_texels < 1 || a->num_texels >= 0xffffffffLL) return false;
  if (a->channels <= 0 || a->tex_batch < 1 || a->num_levels < 1 || a->num_levels > DR_MAX_LEVELS)
    return false;
  if (a->filter < 0 || a->filter > 3 || a->boundary < 0 || a->boundary > 3) return false;
  if ((a->boundary == DR_BOUNDARY_CUBE) != (a->faces == 6) || (a->faces != 1 && a->faces != 6))
    return false;
  for (int k = 0; k < a->num_levels; ++k)
    if (a->level_height[k] <= 0 || a->level_width[k] <= 0) return false;
  return true;
}

extern "C" int dr_texture_forward_f64(const DrTextureArgs* a, double* out, void* stream) {
  if (!texture_ok(a) || !out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  const hipStream_t s = (hipStream_t)stream;
  if (a->boundary == DR_BOUNDARY_CUBE)
    f64::tex_fwd<true><<<blocks_for(pixels, 256), 256, 0, s>>>(*a, out);
  else
    f64::tex_fwd<false><<<blocks_for(pixels, 256), 256, 0, s>>>(*a, out);
  return launch_status();
}

extern "C" int dr_texture_backward_f64(const DrTextureArgs* a, const double* grad_out,
                                       double* grad_texels, double* grad_uv,
                                       double* grad_uv_da, double* grad_bias, void* stream) {
  if (!texture_ok(a) || !grad_out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  const hipStream_t s = (hipStream_t)stream;
  double* g_da = a->uv_da ? grad_uv_da : nullptr;
  double* g_bias = a->bias ? grad_bias : nullptr;
  if (a->boundary == DR_BOUNDARY_CUBE)
    f64::tex_bwd<true><<<blocks_for(pixels, 256), 256, 0, s>>>(*a, grad_out, grad_texels,
                                                              grad_uv, g_da, g_bias);
  else
    f64::tex_bwd<false><<<blocks_for(pixels, 256), 256, 0, s>>>(*a, grad_out, grad_texels,
                                                               grad_uv, g_da, g_bias);
  return launch_status();
}

extern "C" int dr_mip_build_f64(double* texels, const double* base, int32_t tex_batch,
                                int32_t channels, int64_t num_texels, int32_t faces,
                                int32_t num_levels, const int32_t* level_height,
                                const int32_t* level_width, const int64_t* level_offset,
                                void* stream) {
  if (!texels || tex_batch < 1 || channels < 1 || (faces != 1 && faces != 6) ||
      !f64::valid_levels(num_levels, level_height, level_width, level_offset))
    return DR_ERR_ARGUMENT;
  const f64::Levels L = f64::copy_levels(num_levels, level_height, level_width, level_offset);
  const hipStream_t s = (hipStream_t)stream;
  const int64_t images = (int64_t)tex_batch * faces;
  const int64_t base_texels = (int64_t)faces * L.h[0] * L.w[0];
  if (base != nullptr) {
    if (base_texels > num_texels) return DR_ERR_ARGUMENT;
    const int64_t count = (int64_t)tex_batch * base_texels * channels;
    f64::copy_base<<<blocks_for(count, 256), 256, 0, s>>>(texels, base, num_texels * channels,
                                                         base_texels * channels, count);
  }
  for (int k = 0; k + 1 < num_levels; ++k) {
    const int64_t count = images * L.h[k + 1] * L.w[k + 1] * channels;
    f64::mip_down<<<blocks_for(count, 256), 256, 0, s>>>(texels, nullptr, channels, num_texels,
                                                        faces, L, k, count);
  }
  return launch_status();
}

extern "C" int dr_mip_build_backward_f64(double* grad_texels, int32_t tex_batch,
                                         int32_t channels, int64_t num_texels, int32_t faces,
                                         int32_t num_levels, const int32_t* level_height,
                                         const int32_t* level_width,
                                         const int64_t* level_offset, void* stream) {
  if (!grad_texels || tex_batch < 1 || channels < 1 || (faces != 1 && faces != 6) ||
      !f64::valid_levels(num_levels, level_height, level_width, level_offset))
    return DR_ERR_ARGUMENT;
  const f64::Levels L = f64::copy_levels(num_levels, level_height, level_width, level_offset);
  const int64_t images = (int64_t)tex_batch * faces;
  for (int k = num_levels - 2; k >= 0; --k) {
    const int64_t count = images * L.h[k] * L.w[k] * channels;
    f64::mip_up<<<blocks_for(count, 256), 256, 0, (hipStream_t)stream>>>(
        grad_texels, channels, num_texels, faces, L, k, count);
  }
  return launch_status();
}

extern "C" int dr_silhouette_mask_f64(const double* pos, int64_t pos_batch_stride,
                                      int32_t pos_batch, const int32_t* tri, int32_t num_tri,
                                      const int32_t* neighbours, uint8_t* mask, void* stream) {
  if (pos_batch < 1 || num_tri < 0 || !mask || (num_tri > 0 && (!pos || !tri || !neighbours)))
    return DR_ERR_ARGUMENT;
  const int64_t n = (int64_t)pos_batch * num_tri;
  if (n == 0) return DR_OK;
  f64::silhouettes<<<blocks_for(n, 256), 256, 0, (hipStream_t)stream>>>(
      pos, pos_batch_stride, pos_batch, tri, num_tri, neighbours, mask);
  return launch_status();
}

static bool aa_ok(const DrAntialiasArgs* a) {
  return a && a->batch >= 0 && a->height > 0 && a->width > 0 && a->channels > 0 &&
         (a->batch == 0 || (a->color && a->rast && a->pos && a->silhouette &&
                            (a->num_tri == 0 || a->tri)));
}

extern "C" int dr_antialias_workspace_size_f64(const DrAntialiasArgs* a, size_t* bytes) {
  if (!aa_ok(a) || !bytes) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  *bytes = (size_t)pixels * (sizeof(double2) + sizeof(uchar2));
  return DR_OK;
}

extern "C" int dr_antialias_forward_f64(const DrAntialiasArgs* a, void* pairs,
                                        size_t pairs_bytes, double* out, void* stream) {
  if (!aa_ok(a) || !out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  if (!pairs || pairs_bytes < (size_t)pixels * (sizeof(double2) + sizeof(uchar2)))
    return DR_ERR_CAPACITY;
  double2* t = (double2*)pairs;
  uchar2* bits = (uchar2*)((char*)pairs + pixels * sizeof(double2));
  const hipStream_t s = (hipStream_t)stream;
  f64::aa_pairs<<<blocks_for(pixels, 256), 256, 0, s>>>(*a, t, bits);
  f64::aa_blend<<<blocks_for(pixels, 256), 256, 0, s>>>(*a, t, bits, out);
  return launch_status();
}

extern "C" int dr_antialias_backward_f64(const DrAntialiasArgs* a, const void* pairs,
                                         size_t pairs_bytes, const double* grad_out,
                                         double* grad_color, double* grad_pos, void* stream) {
  if (!aa_ok(a) || !grad_out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  if (!pairs || pairs_bytes < (size_t)pixels * (sizeof(double2) + sizeof(uchar2)))
    return DR_ERR_CAPACITY;
  const double2* t = (const double2*)pairs;
  const uchar2* bits = (const uchar2*)((const char*)pairs + pixels * sizeof(double2));
  f64::aa_bwd<<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(
      *a, t, bits, grad_out, grad_color, grad_pos);
  return launch_status();
}
