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
// registers) and accumulates grad_attr through the workgroup's row table; pixels of a tile row
// that show the same triangle are summed first. Without grad_attr it is a gather kernel like
// the forward pass.
#include "common.h"

namespace dr {
namespace {

struct Pixel {
  bool valid;
  int t;
  uint32_t row[3];  // attribute rows (image * rows per image + vertex) of the three vertices
  float u, v;
};

// The pixel of `image` whose rast value is r and, for a covered pixel, its triangle's index row.
// rows_per_image is 0 for attributes shared by all images.
__device__ __forceinline__ Pixel pixel_of(const DrInterpolateArgs& a, const float4& r, int image,
                                          uint32_t rows_per_image) {
  Pixel p;
  // rast stores id + 1 as a float; ids past the end of tri are background (reference.py:128).
  const float id = rintf(r.w);
  p.valid = id >= 1.0f && id <= (float)a.num_tri;
  p.t = p.valid ? (int)id - 1 : 0;
  p.u = r.x;
  p.v = r.y;
  p.row[0] = p.row[1] = p.row[2] = 0u;
  if (p.valid) {
    const int32_t* tri = a.tri + 3 * (int64_t)p.t;
    const uint32_t base = (uint32_t)image * rows_per_image;
#pragma unroll
    for (int k = 0; k < 3; ++k) p.row[k] = base + (uint32_t)tri[k];
  }
  return p;
}

__device__ __forceinline__ Pixel load_pixel(const DrInterpolateArgs& a, int64_t pixel, int image,
                                            uint32_t rows_per_image) {
  return pixel_of(a, load4(a.rast + 4 * pixel), image, rows_per_image);
}

// The three attribute rows of a pixel, channels [c0, c0 + N), in registers (0 past C).
template <int N>
__device__ __forceinline__ void load_rows(const float* attr, const Pixel& p, int C, int c0,
                                          float (&A)[3][N]) {
  // Whole-row loads when every row of the pass is 16-byte aligned: a condition on the buffer
  // and the channel count alone, the same for every lane.
  if constexpr (N % 4 == 0) {
    if (C % 4 == 0 && c0 + N <= C && (reinterpret_cast<uintptr_t>(attr) & 15u) == 0) {
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const float4* row = reinterpret_cast<const float4*>(attr + (int64_t)p.row[k] * C + c0);
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
          const float4 q = row[i];
          A[k][4 * i] = q.x;
          A[k][4 * i + 1] = q.y;
          A[k][4 * i + 2] = q.z;
          A[k][4 * i + 3] = q.w;
        }
      }
      return;
    }
  }
  if constexpr (N == 2) {
    if (C == 2 && (reinterpret_cast<uintptr_t>(attr) & 7u) == 0) {
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const float2 q = reinterpret_cast<const float2*>(attr)[p.row[k]];
        A[k][0] = q.x;
        A[k][1] = q.y;
      }
      return;
    }
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float* row = attr + (int64_t)p.row[k] * C + c0;
#pragma unroll
    for (int c = 0; c < N; ++c) A[k][c] = (c0 + c < C) ? row[c] : 0.0f;
  }
}

// A[k][c] for a channel index c < N known only at run time, without indexing registers.
template <int N>
__device__ __forceinline__ float pick(const float (&row)[N], int c) {
  float v = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) v = (i == c) ? row[i] : v;
  return v;
}

// Channels per pass of the generic kernel (any channel count).
constexpr int kGenericChannels = 4;

// Width of the gather kernels' tiles (pixel_slots): 32 x 8 per pixel slot. At 8 x 1024^2 with
// 1.3 M triangles, against 16 x 16: forward -3 us, backward without an attribute gradient -8 us
// (64 x 4: forward +25 us); the resolve keeps 16 x 16 (+2 us at 32).
constexpr int kGatherTileWidth = 32;

// PPT pixels per thread, in rows or tiles (pixel_slots). The pixels' loads go out level by
// level -- rast, then the triangles' index rows, then the attribute rows -- so that a thread
// waits once per level for all its pixels, not once per pixel: the gathers are latency-bound.
// DIFF: out_da is written (num_diff > 0); without it the kernel holds no derivative state.
template <int NC, int PPT, bool TILES, bool DIFF>
__global__ __launch_bounds__(256) void interp_fwd_kernel(DrInterpolateArgs a,
                                                         float* __restrict__ out,
                                                         float* __restrict__ out_da,
                                                         uint32_t rows_per_image) {
  const PixelSlots<PPT> s =
      pixel_slots<PPT, TILES, kGatherTileWidth>(a.batch, a.height, a.width);
  const int C = NC > 0 ? NC : a.channels;
  constexpr int N = NC > 0 ? NC : kGenericChannels;
  const int64_t* pixel = s.pixel;
  float4 r[PPT];
#pragma unroll
  for (int j = 0; j < PPT; ++j)
    r[j] = s.inside[j] ? load4(a.rast + 4 * pixel[j]) : make_float4(0.f, 0.f, 0.f, 0.f);
  Pixel p[PPT];
  float4 db[PPT];
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    p[j] = pixel_of(a, r[j], s.b[j], rows_per_image);
    db[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (DIFF && p[j].valid) db[j] = load4(a.rast_db + 4 * pixel[j]);  // du/dx, du/dy, dv/dx, dv/dy
  }
  for (int c0 = 0; c0 < C; c0 += N) {
    float A[PPT][3][N];
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      if (p[j].valid) {
        load_rows<N>(a.attr, p[j], C, c0, A[j]);
      } else {
#pragma unroll
        for (int c = 0; c < N; ++c) A[j][0][c] = A[j][1][c] = A[j][2][c] = 0.0f;
      }
    }
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      if (!s.inside[j]) continue;
      const float u = p[j].u, v = p[j].v, w = 1.0f - u - v;
      float res[N];
#pragma unroll
      for (int c = 0; c < N; ++c)
        res[c] = p[j].valid ? u * A[j][0][c] + v * A[j][1][c] + w * A[j][2][c] : 0.0f;
      if constexpr (DIFF) {
        float* od = out_da + pixel[j] * 2 * a.num_diff;
        for (int k = 0; k < a.num_diff; ++k) {
          const int c = a.diff[k] - c0;
          if (c < 0 || c >= N) continue;
          const float da_du = pick(A[j][0], c) - pick(A[j][2], c);
          const float da_dv = pick(A[j][1], c) - pick(A[j][2], c);
          od[2 * k] = p[j].valid ? db[j].x * da_du + db[j].z * da_dv : 0.0f;
          od[2 * k + 1] = p[j].valid ? db[j].y * da_du + db[j].w * da_dv : 0.0f;
        }
      }
      float* o = out + pixel[j] * C;
#pragma unroll
      for (int c = 0; c < N; ++c)
        if (c0 + c < C) o[c0 + c] = res[c];
    }
  }
}

// DIFF: num_diff > 0 (grad_db is written, grad_da read if given); without it the kernel holds
// no derivative state.
template <int NC, bool DIFF>
__global__ __launch_bounds__(256) void interp_bwd_kernel(DrInterpolateArgs a,
                                                         const float* __restrict__ grad_out,
                                                         const float* __restrict__ grad_da,
                                                         float* __restrict__ grad_attr,
                                                         float* __restrict__ grad_rast,
                                                         float* __restrict__ grad_db,
                                                         uint32_t rows_per_image) {
  using Table = RowTable<256, 8>;
  __shared__ Table table;
  const bool scatter = grad_attr != nullptr && a.channels > 0;  // uniform over the workgroup
  if (scatter) table.init();  // the first pass's barriers order it before any add
  const TilePixel tp = tile_pixel(a.batch, a.height, a.width);
  const int64_t pixel = tp.pixel;
  const int C = NC > 0 ? NC : a.channels;
  const int D = DIFF && grad_da != nullptr ? a.num_diff : 0;
  Pixel p;
  p.valid = false;
  p.t = 0;
  p.u = p.v = 0.0f;
  p.row[0] = p.row[1] = p.row[2] = 0u;
  float4 db = make_float4(0.f, 0.f, 0.f, 0.f);
  if (tp.inside) {
    p = load_pixel(a, pixel, tp.b, rows_per_image);
    if (DIFF && p.valid) db = load4(a.rast_db + 4 * pixel);
  }
  const float w = 1.0f - p.u - p.v;
  const float* g = grad_out + (tp.inside ? pixel * C : 0);
  const float* gd = (D > 0 && tp.inside) ? grad_da + pixel * 2 * D : nullptr;
  const uint32_t run_key = p.valid ? (uint32_t)p.t : 0xffffffffu;
  float gu = 0.f, gv = 0.f, g_dudx = 0.f, g_dudy = 0.f, g_dvdx = 0.f, g_dvdy = 0.f;

  constexpr int N = NC > 0 && NC < 8 ? NC : 8;  // channels per pass through the table
  for (int c0 = 0; c0 < C; c0 += N) {
    float A[3][N], G[N];
    const bool live = p.valid;
    if (live) load_rows<N>(a.attr, p, C, c0, A);
    const bool wide = live && c0 + N <= C && load_wide<N>(g + c0, G);
#pragma unroll
    for (int c = 0; c < N; ++c) {
      if (!live) A[0][c] = A[1][c] = A[2][c] = 0.0f;
      if (!wide) G[c] = (live && c0 + c < C) ? g[c0 + c] : 0.0f;
    }
    // Vertex k, channel c at v[N k + c].
    float v[3 * N];
#pragma unroll
    for (int c = 0; c < N; ++c) {
      gu += G[c] * (A[0][c] - A[2][c]);
      gv += G[c] * (A[1][c] - A[2][c]);
      v[c] = G[c] * p.u;
      v[N + c] = G[c] * p.v;
      v[2 * N + c] = G[c] * w;
    }
    if (DIFF && gd != nullptr && live) {
      for (int k = 0; k < D; ++k) {
        const int c = a.diff[k] - c0;
        if (c < 0 || c >= N) continue;
        const float gx = gd[2 * k], gy = gd[2 * k + 1];
        const float da_du = pick(A[0], c) - pick(A[2], c);
        const float da_dv = pick(A[1], c) - pick(A[2], c);
        g_dudx += gx * da_du;
        g_dudy += gy * da_du;
        g_dvdx += gx * da_dv;
        g_dvdy += gy * da_dv;
        const float t0 = gx * db.x + gy * db.y;
        const float t1 = gx * db.z + gy * db.w;
#pragma unroll
        for (int i = 0; i < N; ++i) {
          if (i != c) continue;
          v[i] += t0;
          v[N + i] += t1;
          v[2 * N + i] -= t0 + t1;
        }
      }
    }
    if (!scatter) continue;
    // Pixels of a tile row that show one triangle are summed first, so each run of them makes
    // one table update per vertex.
    const int n = min(N, C - c0);
    if constexpr (!DIFF) {
      // One vertex at a time (fewer registers than all three at once), the table's scale set
      // beforehand from a bound of every value added: a run sum of at most 16 products
      // G[c] * b_k, each at most max |G| * max |b| (rounding is monotone).
      float g_max = 0.0f;
      bool bad = !(isfinite(p.u) && isfinite(p.v) && isfinite(w));
#pragma unroll
      for (int c = 0; c < N; ++c) {
        bad = bad || !isfinite(G[c]);
        g_max = fmaxf(g_max, fabsf(G[c]));
      }
      const float b_max = fmaxf(fmaxf(fabsf(p.u), fabsf(p.v)), fabsf(w));
      const float bound = bad ? __int_as_float(0x7f800000) : 16.0f * (g_max * b_max);
      const FixedPass f = table.begin(live ? bound : 0.0f);
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const float b = k == 0 ? p.u : (k == 1 ? p.v : w);
        float vk[N];
#pragma unroll
        for (int c = 0; c < N; ++c) vk[c] = G[c] * b;
        const bool last = row_run_sums(run_key, vk);
        if (last && live) table.add_or_global(p.row[k], vk, n, grad_attr + c0, C, f);
      }
      __syncthreads();
      table.flush(grad_attr + c0, C, n, f);
      if (c0 + N < C) {
        __syncthreads();
        table.reset();
      }
      continue;
    }
    const bool last = row_run_sums(run_key, v);
    const bool adds = last && live;
    const FixedPass f = table.begin(adds ? max_magnitude(v, 3 * N) : 0.0f);
    if (adds) {
#pragma unroll
      for (int k = 0; k < 3; ++k)
        table.add_or_global(p.row[k], v + N * k, n, grad_attr + c0, C, f);
    }
    __syncthreads();
    table.flush(grad_attr + c0, C, n, f);
    if (c0 + N < C) {
      __syncthreads();
      table.reset();
    }
  }
  if (tp.inside) {
    if (grad_rast) store4(grad_rast + 4 * pixel, make_float4(gu, gv, 0.f, 0.f));
    if (DIFF && grad_db) store4(grad_db + 4 * pixel, make_float4(g_dudx, g_dudy, g_dvdx, g_dvdy));
  }
}

// The backward pass without an attribute gradient (constant attributes): grad_rast and, with
// DIFF, grad_rast_db only, in the forward pass's gather layout and without the scatter table --
// PPT pixels per thread, their rast, then the index rows, then the upstream gradients and the
// attribute rows, each level's loads issued together (rast_db itself takes no part: only the
// attribute gradient depends on it). The sums run in the order of interp_bwd_kernel (channels
// in passes of N, derivatives in list order in a pass).
template <int NC, int PPT, bool TILES, bool DIFF>
__global__ __launch_bounds__(256) void interp_bwd_rast_kernel(DrInterpolateArgs a,
                                                              const float* __restrict__ grad_out,
                                                              const float* __restrict__ grad_da,
                                                              float* __restrict__ grad_rast,
                                                              float* __restrict__ grad_db,
                                                              uint32_t rows_per_image) {
  const PixelSlots<PPT> s =
      pixel_slots<PPT, TILES, kGatherTileWidth>(a.batch, a.height, a.width);
  const int C = NC > 0 ? NC : a.channels;
  constexpr int N = NC > 0 && NC < 8 ? NC : 8;
  const int D = DIFF && grad_da != nullptr ? a.num_diff : 0;
  const int64_t* pixel = s.pixel;
  float4 r[PPT];
#pragma unroll
  for (int j = 0; j < PPT; ++j)
    r[j] = s.inside[j] ? load4(a.rast + 4 * pixel[j]) : make_float4(0.f, 0.f, 0.f, 0.f);
  Pixel p[PPT];
#pragma unroll
  for (int j = 0; j < PPT; ++j) p[j] = pixel_of(a, r[j], s.b[j], rows_per_image);
  float gu[PPT], gv[PPT], g_dudx[PPT], g_dudy[PPT], g_dvdx[PPT], g_dvdy[PPT];
#pragma unroll
  for (int j = 0; j < PPT; ++j) gu[j] = gv[j] = g_dudx[j] = g_dudy[j] = g_dvdx[j] = g_dvdy[j] = 0.f;
  for (int c0 = 0; c0 < C; c0 += N) {
    float A[PPT][3][N], G[PPT][N];
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const bool live = p[j].valid;
      const float* g = grad_out + (live ? pixel[j] * C : 0);
      const bool wide = live && c0 + N <= C && load_wide<N>(g + c0, G[j]);
      if (!wide)
#pragma unroll
        for (int c = 0; c < N; ++c) G[j][c] = (live && c0 + c < C) ? g[c0 + c] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      if (p[j].valid) {
        load_rows<N>(a.attr, p[j], C, c0, A[j]);
      } else {
#pragma unroll
        for (int c = 0; c < N; ++c) A[j][0][c] = A[j][1][c] = A[j][2][c] = 0.0f;
      }
    }
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
#pragma unroll
      for (int c = 0; c < N; ++c) {
        gu[j] += G[j][c] * (A[j][0][c] - A[j][2][c]);
        gv[j] += G[j][c] * (A[j][1][c] - A[j][2][c]);
      }
      if (DIFF && D > 0 && p[j].valid) {
        const float* gd = grad_da + pixel[j] * 2 * D;
        for (int k = 0; k < D; ++k) {
          const int c = a.diff[k] - c0;
          if (c < 0 || c >= N) continue;
          const float gx = gd[2 * k], gy = gd[2 * k + 1];
          const float da_du = pick(A[j][0], c) - pick(A[j][2], c);
          const float da_dv = pick(A[j][1], c) - pick(A[j][2], c);
          g_dudx[j] += gx * da_du;
          g_dudy[j] += gy * da_du;
          g_dvdx[j] += gx * da_dv;
          g_dvdy[j] += gy * da_dv;
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < PPT; ++j) {
    if (!s.inside[j]) continue;
    if (grad_rast) store4(grad_rast + 4 * pixel[j], make_float4(gu[j], gv[j], 0.f, 0.f));
    if (DIFF && grad_db)
      store4(grad_db + 4 * pixel[j], make_float4(g_dudx[j], g_dudy[j], g_dvdx[j], g_dvdy[j]));
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

// f(std::true_type) when the call has derivatives, else f(std::false_type).
template <typename F>
int with_derivatives(bool diff, F f) {
  return diff ? f(std::true_type()) : f(std::false_type());
}

// Attribute rows per image: 0 when shared, else attr_batch_stride / channels.
uint32_t image_rows(const DrInterpolateArgs& a) {
  return a.attr_batch_stride == 0 || a.channels == 0
             ? 0u
             : (uint32_t)(a.attr_batch_stride / a.channels);
}

bool valid_args(const DrInterpolateArgs* a) {
  if (!a || a->batch < 0 || a->height <= 0 || a->width <= 0 || a->channels < 0) return false;
  if (a->num_tri < 0 || a->num_diff < 0 || a->num_vertices < 0) return false;
  if (a->num_diff > 0 && (!a->rast_db || !a->diff)) return false;
  // Attribute rows (and the gradient table's keys) are 32-bit: whole rows per image, fewer
  // than 2^32 - 1 rows in all.
  if (a->attr_batch_stride < 0) return false;
  if (a->channels > 0 && a->attr_batch_stride % a->channels != 0) return false;
  const int64_t per_image = a->channels > 0 ? a->attr_batch_stride / a->channels : 0;
  const int64_t rows = per_image != 0 ? per_image * a->batch : (int64_t)a->num_vertices;
  if (rows >= 0xffffffffLL || per_image >= 0xffffffffLL) return false;
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
  const uint32_t rows_per_image = image_rows(args);
  float* da = args.num_diff > 0 ? out_da : nullptr;
  // The index rows and attribute rows one image's pixels may gather.
  const int64_t rows = rows_per_image != 0 ? rows_per_image : args.num_vertices;
  const bool tiles = gather_tiles(12 * (int64_t)args.num_tri + 4 * rows * args.channels);
  return dispatch_channels(args.channels, [&](auto nc) {
    return with_derivatives(args.num_diff > 0, [&](auto diff) {
      constexpr int NC = decltype(nc)::value;
      constexpr bool DIFF = decltype(diff)::value;
      constexpr int PPT = NC > 0 ? 2 : 1;  // pixels per thread
      constexpr int TW = kGatherTileWidth;
      const hipStream_t st = (hipStream_t)stream;
      if (tiles)
        interp_fwd_kernel<NC, PPT, true, DIFF>
            <<<pixel_slot_blocks<PPT, true, TW>(args.batch, args.height, args.width), 256, 0,
               st>>>(args, out, da, rows_per_image);
      else
        interp_fwd_kernel<NC, PPT, false, DIFF>
            <<<pixel_slot_blocks<PPT, false, TW>(args.batch, args.height, args.width), 256, 0,
               st>>>(args, out, da, rows_per_image);
      return launch_status();
    });
  });
}

extern "C" int dr_interpolate_backward(const DrInterpolateArgs* a, const float* grad_out,
                                       const float* grad_out_da, float* grad_attr,
                                       float* grad_rast, float* grad_rast_db, void* stream) {
  if (!valid_args(a) || !grad_out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  const uint32_t rows_per_image = image_rows(*a);
  const float* gda = a->num_diff > 0 ? grad_out_da : nullptr;
  if (grad_attr == nullptr || a->channels == 0) {
    const DrInterpolateArgs args = *a;
    const int64_t rows = rows_per_image != 0 ? rows_per_image : args.num_vertices;
    const bool tiles = gather_tiles(12 * (int64_t)args.num_tri + 4 * rows * args.channels);
    return dispatch_channels(args.channels, [&](auto nc) {
      return with_derivatives(args.num_diff > 0, [&](auto diff) {
        constexpr int NC = decltype(nc)::value;
        constexpr bool DIFF = decltype(diff)::value;
        // One pixel per thread: at 8 x 1024^2 with 1.3 M triangles (uv, 'all' derivatives)
        // 165 us in 16 x 16 tiles, two per thread the same, four +15 us; rows +13 us.
        constexpr int PPT = 1;
        constexpr int TW = kGatherTileWidth;
        const hipStream_t st = (hipStream_t)stream;
        float* gdb = args.num_diff > 0 ? grad_rast_db : nullptr;
        if (tiles)
          interp_bwd_rast_kernel<NC, PPT, true, DIFF>
              <<<pixel_slot_blocks<PPT, true, TW>(args.batch, args.height, args.width), 256, 0,
                 st>>>(args, grad_out, gda, grad_rast, gdb, rows_per_image);
        else
          interp_bwd_rast_kernel<NC, PPT, false, DIFF>
              <<<pixel_slot_blocks<PPT, false, TW>(args.batch, args.height, args.width), 256, 0,
                 st>>>(args, grad_out, gda, grad_rast, gdb, rows_per_image);
        return launch_status();
      });
    });
  }
  return dispatch_channels(a->channels, [&](auto nc) {
    return with_derivatives(a->num_diff > 0, [&](auto diff) {
      interp_bwd_kernel<decltype(nc)::value, decltype(diff)::value>
          <<<tile_blocks(a->batch, a->height, a->width), 256, 0, (hipStream_t)stream>>>(
              *a, grad_out, gda, grad_attr, grad_rast, a->num_diff > 0 ? grad_rast_db : nullptr,
              rows_per_image);
      return launch_status();
    });
  });
}
