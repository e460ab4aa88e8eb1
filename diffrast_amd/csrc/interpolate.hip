// Interpolate for gfx950: per-pixel barycentric blend of vertex attributes and its gradient.
//
// out = u a0 + v a1 + (1 - u - v) a2 per channel, and for each channel listed in `diff` the
// screen-space derivatives (du/dx (a0 - a2) + dv/dx (a1 - a2), du/dy (...) + dv/dy (...)),
// as in the reference backend (src/diffrast/backends/reference.py:117-146), in its operation
// order. One thread per pixel: the rast / rast_db / out streams are read and written in pixel
// order (coalesced), while the three attribute rows are gathered through the index buffer,
// served mostly by the L2 and the Infinity Cache. Shared attributes have batch stride 0.
//
// The backward pass writes grad_rast and grad_rast_db per pixel (channel sums held in
// registers) and accumulates grad_attr with fp32 atomics; pixels of a wave that show the same
// triangle are summed in the wave first.
#include "common.h"

namespace dr {
namespace {

struct Pixel {
  bool valid;
  int t;
  int64_t rows[3];  // attribute row offsets (floats) of the three vertices
  float u, v;
};

__device__ __forceinline__ Pixel load_pixel(const DrInterpolateArgs& a, int64_t pixel,
                                            float4& r) {
  Pixel p;
  r = load4(a.rast + 4 * pixel);
  // rast stores id + 1 as a float; ids past the end of tri are background (reference.py:128).
  const float id = rintf(r.w);
  p.valid = id >= 1.0f && id <= (float)a.num_tri;
  p.t = p.valid ? (int)id - 1 : 0;
  p.u = r.x;
  p.v = r.y;
  if (p.valid) {
    const int64_t image = pixel / ((int64_t)a.height * a.width);
    const int64_t base = image * a.attr_batch_stride;
    const int32_t* row = a.tri + 3 * (int64_t)p.t;
#pragma unroll
    for (int k = 0; k < 3; ++k) p.rows[k] = base + (int64_t)row[k] * a.channels;
  }
  return p;
}

template <int NC>
__global__ __launch_bounds__(256) void interp_fwd_kernel(DrInterpolateArgs a, float* out,
                                                      float* out_da) {
  const int64_t pixel = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (pixel >= (int64_t)a.batch * a.height * a.width) return;
  const int C = NC > 0 ? NC : a.channels;
  float4 r;
  const Pixel p = load_pixel(a, pixel, r);
  float* o = out + pixel * C;
  float* od = out_da ? out_da + pixel * 2 * a.num_diff : nullptr;
  if (!p.valid) {
    for (int c = 0; c < C; ++c) o[c] = 0.0f;
    if (od)
      for (int k = 0; k < 2 * a.num_diff; ++k) od[k] = 0.0f;
    return;
  }
  const float* a0 = a.attr + p.rows[0];
  const float* a1 = a.attr + p.rows[1];
  const float* a2 = a.attr + p.rows[2];
  const float w = 1.0f - p.u - p.v;
#pragma unroll
  for (int c = 0; c < C; ++c) o[c] = p.u * a0[c] + p.v * a1[c] + w * a2[c];
  if (od) {
    const float4 db = load4(a.rast_db + 4 * pixel);  // du/dx, du/dy, dv/dx, dv/dy
    for (int k = 0; k < a.num_diff; ++k) {
      const int c = a.diff[k];
      const float da_du = a0[c] - a2[c];
      const float da_dv = a1[c] - a2[c];
      od[2 * k] = db.x * da_du + db.z * da_dv;
      od[2 * k + 1] = db.y * da_du + db.w * da_dv;
    }
  }
}

template <int NC>
__global__ __launch_bounds__(256) void interp_bwd_kernel(DrInterpolateArgs a,
                                                         const float* grad_out,
                                                         const float* grad_da, float* grad_attr,
                                                         float* grad_rast, float* grad_db) {
  __shared__ RowTable<512, 8> table;
  table.init();  // the first pass's barriers order it before any add
  const TilePixel tp = tile_pixel(a.batch, a.height, a.width);
  const int64_t pixel = tp.pixel;
  const int C = NC > 0 ? NC : a.channels;
  Pixel p;
  p.valid = false;
  p.u = p.v = 0.0f;
  float4 db = make_float4(0.f, 0.f, 0.f, 0.f);
  if (tp.inside) {
    float4 r;
    p = load_pixel(a, pixel, r);
    if (p.valid && a.num_diff > 0) db = load4(a.rast_db + 4 * pixel);
  }
  const float* g = grad_out + (tp.inside ? pixel * C : 0);
  const float* gd = (grad_da && tp.inside) ? grad_da + pixel * 2 * a.num_diff : nullptr;

  if (tp.inside && (grad_rast || grad_db)) {
    float gu = 0.f, gv = 0.f, g_dudx = 0.f, g_dudy = 0.f, g_dvdx = 0.f, g_dvdy = 0.f;
    if (p.valid) {
      const float* a0 = a.attr + p.rows[0];
      const float* a1 = a.attr + p.rows[1];
      const float* a2 = a.attr + p.rows[2];
#pragma unroll
      for (int c = 0; c < C; ++c) {
        gu += g[c] * (a0[c] - a2[c]);
        gv += g[c] * (a1[c] - a2[c]);
      }
      if (gd) {
        for (int k = 0; k < a.num_diff; ++k) {
          const int c = a.diff[k];
          const float da_du = a0[c] - a2[c], da_dv = a1[c] - a2[c];
          g_dudx += gd[2 * k] * da_du;
          g_dudy += gd[2 * k + 1] * da_du;
          g_dvdx += gd[2 * k] * da_dv;
          g_dvdy += gd[2 * k + 1] * da_dv;
        }
      }
    }
    if (grad_rast) store4(grad_rast + 4 * pixel, make_float4(gu, gv, 0.f, 0.f));
    if (grad_db) store4(grad_db + 4 * pixel, make_float4(g_dudx, g_dudy, g_dvdx, g_dvdy));
  }
  if (!grad_attr || C == 0) return;  // uniform over the workgroup

  // Rows of the attribute table are the keys (p.rows holds their float offsets), C floats per
  // row, 8 per pass. Pixels of a tile row that show one triangle are summed first, so each
  // run of them makes one table update per vertex.
  uint32_t keys[3];
#pragma unroll
  for (int k = 0; k < 3; ++k)
    keys[k] = p.valid ? (uint32_t)(p.rows[k] / C) : RowTable<512, 8>::kEmpty;
  const uint32_t run_key = p.valid ? (uint32_t)p.t : 0xffffffffu;
  const float w = 1.0f - p.u - p.v;
  for (int c0 = 0; c0 < C; c0 += 8) {
    const int n = min(8, C - c0);
    float v[24];  // vertex k, channel c at v[8 k + c]
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      v[c] = v[8 + c] = v[16 + c] = 0.0f;
      if (c >= n || !p.valid) continue;
      const float gc = g[c0 + c];
      v[c] = gc * p.u;
      v[8 + c] = gc * p.v;
      v[16 + c] = gc * w;
      if (gd) {
        for (int k = 0; k < a.num_diff; ++k) {
          if (a.diff[k] != c0 + c) continue;
          const float t0 = gd[2 * k] * db.x + gd[2 * k + 1] * db.y;
          const float t1 = gd[2 * k] * db.z + gd[2 * k + 1] * db.w;
          v[c] += t0;
          v[8 + c] += t1;
          v[16 + c] -= t0 + t1;
        }
      }
    }
    const bool last = row_run_sums(run_key, v);
    __syncthreads();
    if (last && p.valid) {
#pragma unroll
      for (int k = 0; k < 3; ++k) table.add_or_global(keys[k], v + 8 * k, n, grad_attr + c0, C);
    }
    __syncthreads();
    table.flush(grad_attr + c0, C, n);
    if (c0 + 8 < C) {
      __syncthreads();
      table.reset();
    }
  }
}

template <typename F>
int dispatch_channels(int channels, F f) {
  switch (channels) {
    case 1: return f(std::integral_constant<int, 1>());
    case 2: return f(std::integral_constant<int, 2>());
    case 3: return f(std::integral_constant<int, 3>());
    case 4: return f(std::integral_constant<int, 4>());
    case 8: return f(std::integral_constant<int, 8>());
    default: return f(std::integral_constant<int, 0>());
  }
}

bool valid_args(const DrInterpolateArgs* a) {
  if (!a || a->batch < 0 || a->height <= 0 || a->width <= 0 || a->channels < 0) return false;
  if (a->num_tri < 0 || a->num_diff < 0) return false;
  if (a->num_diff > 0 && (!a->rast_db || !a->diff)) return false;
  return true;
}

}  // namespace
}  // namespace dr

using namespace dr;

extern "C" int dr_interpolate_forward(const DrInterpolateArgs* a, float* out, float* out_da,
                                      void* stream) {
  if (!valid_args(a) || !out || (a->num_diff > 0 && !out_da)) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0 || (a->channels == 0 && a->num_diff == 0)) return DR_OK;
  const DrInterpolateArgs args = *a;
  return dispatch_channels(args.channels, [&](auto nc) {
    interp_fwd_kernel<decltype(nc)::value><<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(
        args, out, args.num_diff > 0 ? out_da : nullptr);
    return launch_status();
  });
}

extern "C" int dr_interpolate_backward(const DrInterpolateArgs* a, const float* grad_out,
                                       const float* grad_out_da, float* grad_attr,
                                       float* grad_rast, float* grad_rast_db, void* stream) {
  if (!valid_args(a) || !grad_out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  // Rows of the attribute table are 32-bit keys of the workgroup scatter table.
  const int64_t rows = (a->attr_batch_stride != 0 ? (int64_t)a->batch : 1) * a->num_vertices;
  if (grad_attr && rows >= 0xffffffffLL) return DR_ERR_ARGUMENT;
  const float* gda = a->num_diff > 0 ? grad_out_da : nullptr;
  return dispatch_channels(a->channels, [&](auto nc) {
    interp_bwd_kernel<decltype(nc)::value>
        <<<tile_blocks(a->batch, a->height, a->width), 256, 0, (hipStream_t)stream>>>(
            *a, grad_out, gda, grad_attr, grad_rast, a->num_diff > 0 ? grad_rast_db : nullptr);
    return launch_status();
  });
}
