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
#include "texture_math.h"

namespace dr {
namespace {

using namespace tex;

// Channels [c0, c0 + N) of the four taps (0 past C or for an invalid tap), all loads issued
// together.
template <int N>
__device__ __forceinline__ void fetch_taps(const float* __restrict__ texels, const Bilinear<float>& L,
                                           int C, int c0, float (&t)[4][N]) {
  if constexpr (N == 4) {
    // Four-channel texels on a 16-byte aligned buffer: one 16-byte load per tap.
    if (C == 4 && (reinterpret_cast<uintptr_t>(texels) & 15u) == 0) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float4 v = L.valid[k] ? *reinterpret_cast<const float4*>(texels + (size_t)L.index[k] * 4)
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
    const float* row = texels + (size_t)L.index[k] * C + c0;
#pragma unroll
    for (int c = 0; c < N; ++c) t[k][c] = (L.valid[k] && c0 + c < C) ? row[c] : 0.0f;
  }
}

template <int N>
__device__ __forceinline__ void tap_column(const float (&t)[4][N], int c, float (&out)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) out[k] = t[k][c];
}

// NC channels per pass (the channel count when it is 1-4; 4 with a loop for more). Every tap
// of a pass is loaded before its stores. FILTER and BOUNDARY: a.filter and a.boundary, fixed
// when compiling (DR_BOUNDARY_CUBE for cube maps; FILTER may be kAnyMode: read at run time).
template <int NC, bool CUBE, int FILTER, int BOUNDARY>
__global__ __launch_bounds__(256) void tex_fwd_kernel(DrTextureArgs a, float* __restrict__ out) {
  const int64_t pixel = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (pixel >= (int64_t)a.batch * a.height * a.width) return;
  const int C = a.channels;
  float* o = out + pixel * C;
  Lookup<float> K;
  lookup_setup<float, CUBE, FILTER>(a, pixel, K);
  if (K.dir_invalid) {
    for (int c = 0; c < C; ++c) o[c] = 0.0f;
    return;
  }
  // The image's texture (the division only for per-image textures: it is some 40 VALU
  // instructions in 64 bits).
  const int64_t image = a.tex_batch > 1 ? pixel / ((int64_t)a.height * a.width) : 0;
  const float* __restrict__ texels = a.texels + image * a.num_texels * C;
  const float nan = __int_as_float(0x7fc00000);
  if (K.levels == 0) {
    uint32_t index;
    bool valid;
    const bool bad = nearest_setup<BOUNDARY>(a, K, index, valid);
    for (int c = 0; c < C; ++c) o[c] = bad ? nan : (valid ? texels[(size_t)index * C + c] : 0.0f);
    return;
  }
  const LevelDims D = lookup_levels(a, K);
  const Bilinear<float> L0 = level_setup<CUBE, BOUNDARY>(a, K, D, 0);
  const bool two = K.levels == 2;
  const Bilinear<float> L1 = two ? level_setup<CUBE, BOUNDARY>(a, K, D, 1) : L0;
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
__device__ __forceinline__ void level_coordinate_grads(const Bilinear<float>& L,
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
      float tc[4], dfx, dfy;
      tap_column(t, c, tc);
      const float value = bilinear_grad_value(L, tc, dfx, dfy);
      const float gl = gc[c] * level_weight;
      g_fx += gl * dfx;
      g_fy += gl * dfy;
      if (want_value) g_value += gc[c] * value;
    }
  }
}

// Table keys (texel rows of the packed buffer, 0xffffffff for none) and weights of a level's
// taps. A tap of weight 0 (the second level when the blend factor is 0, or an axis with fraction
// 0) adds nothing and gets no key.
__device__ __forceinline__ void level_taps(const Bilinear<float>& L, float level_weight,
                                           int64_t tex_off, uint32_t* key, float* weight) {
  float t0[4] = {0.f, 0.f, 0.f, 0.f}, wgt[4], dfx, dfy;
  bilinear_grad(L, t0, wgt, dfx, dfy);  // the weights do not depend on texel values
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    weight[k] = level_weight * wgt[k];
    key[k] = L.valid[k] && weight[k] != 0.0f ? (uint32_t)(tex_off + L.index[k]) : 0xffffffffu;
  }
}

// The 2D kernels are held to 72 VGPRs: seven waves per SIMD, as many as the table's LDS allows
// (measured: 393 -> 388 us at 8 x 1024^2 with a 1024^2 texture, against six waves at 74 VGPRs;
// the cube-map kernels spill at such budgets and keep their own).
template <int NC, bool CUBE, int FILTER, int BOUNDARY>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(CUBE ? 1 : 7))) void
tex_bwd_kernel(DrTextureArgs a, const float* grad_out, float* grad_texels, float* grad_uv,
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

  Lookup<float> K;
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
    lookup_setup<float, CUBE, FILTER>(a, pixel, K);
    live = !K.dir_invalid;
  }
  if (live && K.levels == 0) {
    uint32_t index;
    bool valid;
    const bool bad = nearest_setup<BOUNDARY>(a, K, index, valid);
    if (!bad && valid) {
      tap_key[0] = (uint32_t)(tex_off + index);
      tap_weight[0] = 1.0f;
    }
    live = false;  // no coordinate gradient
  } else if (live) {
    const LevelDims D = lookup_levels(a, K);
    const Bilinear<float> L0 = level_setup<CUBE, BOUNDARY>(a, K, D, 0);
    Bilinear<float> L1 = L0;
    const bool two = K.levels == 2;
    if (two) L1 = level_setup<CUBE, BOUNDARY>(a, K, D, 1);
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
      const Deriv4<float> da = cube ? Deriv4<float>{K.P.st_da[0], K.P.st_da[1], K.P.st_da[2],
                                                    K.P.st_da[3]}
                                    : load_deriv4(a.uv_da + 4 * pixel);
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
    // tap on the finer level falls on the same texel sum first, and the last of them adds the
    // sum; the coarser level's taps (4-7) and cube faces go to the table directly, where the
    // summing costs more than the table updates it saves (measured: texture backward at
    // 8 x 1024^2 with a 1024^2 texture 491 -> 481 us without the coarser level's sums).
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
        const bool last = k >= 4 || row_run_sums(key, v);
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

// At most 32 x 32 bottom texels per tile (16 x 16 above it in LDS): a 1024^2 level gives 1024
// workgroups, and the chain above 32^2 is one more single-workgroup stage. (Tiles of 64 x 64
// gave a quarter as many workgroups and 32 KB of LDS each: mip chain 1024^2 x 4, built and
// folded back, 63 -> 53 us; tiles of 16 x 16 need a third stage, 66 us.)
constexpr int kMipStageLevels = 5;

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

// Calls f(channel group, cube, filter, boundary) with each as a compile-time constant
// (std::integral_constant), from a's channel count and modes (checked by valid_args): the
// kernels are compiled for every combination, each without the other modes' code.
template <typename F>
int texture_modes(const DrTextureArgs& a, F f) {
  auto with_boundary = [&](auto nc, auto filter) {
    using std::integral_constant;
    switch (a.boundary) {
      case DR_BOUNDARY_CUBE:
        return f(nc, std::true_type(), filter, integral_constant<int, DR_BOUNDARY_CUBE>());
      case DR_BOUNDARY_WRAP:
        return f(nc, std::false_type(), filter, integral_constant<int, DR_BOUNDARY_WRAP>());
      case DR_BOUNDARY_CLAMP:
        return f(nc, std::false_type(), filter, integral_constant<int, DR_BOUNDARY_CLAMP>());
      default:
        return f(nc, std::false_type(), filter, integral_constant<int, DR_BOUNDARY_ZERO>());
    }
  };
  return channel_groups(a.channels, [&](auto nc) {
    using std::integral_constant;
    switch (a.filter) {
      case DR_FILTER_NEAREST:
        return with_boundary(nc, integral_constant<int, DR_FILTER_NEAREST>());
      case DR_FILTER_LINEAR:
        return with_boundary(nc, integral_constant<int, DR_FILTER_LINEAR>());
      case DR_FILTER_MIP_NEAREST:
        return with_boundary(nc, integral_constant<int, DR_FILTER_MIP_NEAREST>());
      default:
        return with_boundary(nc, integral_constant<int, DR_FILTER_MIP_LINEAR>());
    }
  });
}

bool valid_args(const DrTextureArgs* a) {
  if (!a || !a->texels || !a->uv || a->batch < 0 || a->height <= 0 || a->width <= 0) return false;
  // Texel indices within an image's packed buffer are 32-bit.
  if (a->num_texels < 1 || a->num_texels >= 0xffffffffLL) return false;
  if (a->channels <= 0 || a->tex_batch < 1 || a->num_levels < 1 || a->num_levels > DR_MAX_LEVELS)
    return false;
  if (a->filter < 0 || a->filter > 3 || a->boundary < 0 || a->boundary > 3) return false;
  if ((a->boundary == DR_BOUNDARY_CUBE) != (a->faces == 6)) return false;
  if (a->faces != 1 && a->faces != 6) return false;
  for (int k = 0; k < a->num_levels; ++k)
    if (a->level_height[k] <= 0 || a->level_width[k] <= 0) return false;
  return true;
}

}  // namespace
}  // namespace dr

using namespace dr;

extern "C" int dr_texture_forward(const DrTextureArgs* a, float* out, void* stream) {
  if (!valid_args(a) || !out) return DR_ERR_ARGUMENT;
  const int64_t pixels = (int64_t)a->batch * a->height * a->width;
  if (pixels == 0) return DR_OK;
  const DrTextureArgs args = *a;
  return texture_modes(args, [&](auto nc, auto cube, auto filter, auto boundary) {
    tex_fwd_kernel<decltype(nc)::value, decltype(cube)::value, decltype(filter)::value,
                   decltype(boundary)::value>
        <<<blocks_for(pixels, 256), 256, 0, (hipStream_t)stream>>>(args, out);
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
  const int64_t blocks = tile_blocks(args.batch, args.height, args.width);
  float* g_da = args.uv_da ? grad_uv_da : nullptr;
  float* g_bias = args.bias ? grad_bias : nullptr;
  return texture_modes(args, [&](auto nc, auto cube, auto filter, auto boundary) {
    // Cube maps read the filter at run time: fixed, the trilinear cube-map kernel holds more
    // registers (123 against 94 VGPRs) and runs slower.
    constexpr bool kCube = decltype(cube)::value;
    constexpr int kFilter = kCube ? kAnyMode : decltype(filter)::value;
    tex_bwd_kernel<decltype(nc)::value, kCube, kFilter, decltype(boundary)::value>
        <<<blocks, 256, 0, (hipStream_t)stream>>>(args, grad_out, grad_texels, grad_uv, g_da,
                                                  g_bias);
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
