/*
 * diffrast_hip.h -- C ABI of libdiffrast_hip.so, the MI355X (gfx950) kernels behind the
 * diffrast render pipeline: rasterize, interpolate, texture and antialias, forward and
 * backward.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t (passed as void*),
 * enqueues its kernels on that stream and returns 0 or an error code (dr_error_string).
 * Apart from dr_raster_visibility_static, the library allocates no device memory: the caller
 * allocates every output, gradient and workspace buffer (the *_workspace_size queries give
 * sizes) and zeroes the targets of gradient accumulation. Its mutable global state is small
 * and named where it lives: the static 64 MiB device buffer of dr_raster_visibility_static
 * (one per device, created when the library's code is loaded on it) with that buffer's
 * device addresses, and the per-host-thread pinned buffer of dr_raster_visibility_begin.
 * Calls are re-entrant and ordered by their stream (dr_raster_visibility_static: see there). All float data is float32; every array is dense (C-contiguous).
 *
 * Each entry point cites the interface of the reference diffrast (github.com/sennecools/
 * diffrast) that it replaces. The reference's GPU path is Python: its backend modules
 * (src/diffrast/backends/triton.py) are called by src/diffrast/ops.py; the functions below
 * are what that backend module binds, through ctypes, in diffrast_amd/backends/_lib.py.
 */
#ifndef DIFFRAST_HIP_H
#define DIFFRAST_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  DR_OK = 0,
  DR_ERR_ARGUMENT = 1001,  /* a size, pointer or mode is out of range */
  DR_ERR_CAPACITY = 1002,  /* a workspace or buffer is smaller than required */
  DR_ERR_HIP = 1003,       /* the HIP runtime reported an error (see dr_error_string) */
  DR_ERR_SCRATCH = 1004,   /* more than the allocation-free entry point's static buffer holds */
};

/* Message for a code returned by any entry point (static storage). */
const char* dr_error_string(int code);
/* ABI version; bumped whenever a struct or an entry point below changes. */
int dr_abi_version(void);
/* sizeof of the argument structs, in the order DrRasterGeometry, DrInterpolateArgs,
 * DrTextureArgs, DrAntialiasArgs (which = 0..3); -1 otherwise. Lets bindings check layout. */
int dr_struct_size(int which);

/* ---------------------------------------------------------------------------------------
 * Rasterize: visibility (nearest triangle per pixel, as a 64-bit key) and resolve
 * (rast, rast_db and their gradient).
 *
 * Replaces the reference backend entry rasterize_layer(pos, tri, resolution, grad_db,
 * previous) (src/diffrast/backends/triton.py:21-40, reference.py:45-66) and the range-mode
 * loop of src/diffrast/ops.py:69-74 / peeling.py:80-92, which become one launch here.
 *
 * A key packs the depth z/w (order-preserving, -0 folded into +0) in the high 32 bits and
 * the triangle row in the low 32 bits; UINT64_MAX means empty. Layers of a depth peel are
 * keys strictly greater than the previous layer's key at the same pixel.
 * ------------------------------------------------------------------------------------- */
typedef struct DrRasterGeometry {
  const float* pos;            /* float4 (x, y, z, w) per vertex */
  int64_t pos_batch_stride;    /* floats between the vertex arrays of two images; 0: shared */
  const int32_t* tri;          /* [num_tri, 3] vertex indices, already range-checked */
  int32_t num_tri;
  int32_t batch;               /* number of images */
  int32_t height;
  int32_t width;
  const int32_t* ranges;       /* NULL (every image draws all of tri), or [batch, 2] of
                                  (start, count) per image, on the device (range mode) */
  const int64_t* range_prefix; /* with ranges: [batch + 1] exclusive prefix sum of counts */
  int64_t num_instances;       /* batch * num_tri, or range_prefix[batch] */
  int32_t num_vertices;        /* vertices per image in pos */
  int32_t reserved;            /* 0 */
  const void* order;           /* NULL, or the processing order dr_raster_order wrote for this
                                  tri (and num_vertices), reused instead of computed again */
} DrRasterGeometry;

/* Bytes of the visibility workspace for this geometry. */
int dr_raster_workspace_size(const DrRasterGeometry* g, size_t* bytes);

/* The processing order of a large mesh, for reuse: its triangles sorted by the Morton code of
 * their centroid in the first image's clip space (an affine image of world space, so the order
 * keeps its locality for any camera), each with its three vertex rows. The visibility passes
 * compute it in every call that gets geometry.order == NULL; a caller that draws one tri many
 * times computes it once with dr_raster_order and passes it in. The keys do not depend on the
 * order (only the speed does), so an order computed from other positions of the same tri is
 * valid; one computed from another tri (or num_vertices) is not. *bytes = 0 when the geometry
 * keeps the mesh's own order (range mode, or fewer than 8192 triangles). workspace is a
 * visibility workspace (dr_raster_workspace_size). No counterpart in the reference: its Triton
 * rasterizer bins triangles in index order (_triton_rasterize.py:371-424). */
int dr_raster_order_size(const DrRasterGeometry* g, size_t* bytes);
int dr_raster_order(const DrRasterGeometry* g, void* order, size_t order_bytes, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Visibility, first part: clears keys, orders the triangles of a large mesh spatially,
 * rasterizes triangles with a small bounding box directly, bins the others into 16x16 tiles
 * (counts and scan) and orders the tiles for the tile pass. Waits for the stream and returns
 * in counts[0..3] the number of setup workgroups (each with up to 256 binned triangles), tile
 * entries, workgroups of the tile pass (8 x the busy tiles of the XCD share with the most), and
 * tiles with at least one entry.
 * prev_keys (nullable) is the previous depth layer. */
int dr_raster_visibility_begin(const DrRasterGeometry* g, const uint64_t* prev_keys,
                               uint64_t* keys, void* workspace, size_t workspace_bytes,
                               uint32_t counts[4], void* stream);

/* dr_raster_visibility_begin without the wait: queues the same work and a copy of the four
 * counts into host_counts (pinned host memory, e.g. from hipHostMalloc), and returns. The
 * counts are there once the stream has passed this point (an event recorded after the call).
 * Meanwhile the caller may queue dr_raster_visibility_bin and dr_raster_visibility_tiles with
 * counts {0, capacity of its entry buffer, 0, 0}: if the lists fit, they complete the
 * visibility; if not (host_counts[1] > capacity), both returned at once and the caller either
 * calls them again with the counts and a buffer of host_counts[1] entries, or queues
 * dr_raster_visibility_overflow right after them (no wait). host_counts may be NULL (no copy).
 * (Same reference interfaces as dr_raster_visibility_begin.) */
int dr_raster_visibility_start(const DrRasterGeometry* g, const uint64_t* prev_keys,
                               uint64_t* keys, void* workspace, size_t workspace_bytes,
                               uint32_t* host_counts, void* stream);

/* Visibility, second part: fills the per-tile lists. entries holds counts[1] entries of 8
 * bytes (8-byte aligned): the lists of all tiles, tile by tile, near to far; an entry is a
 * binned triangle's record number (uint32) and a lower bound of its depth (float32), by which
 * the tile pass skips triangles behind every key of a tile without reading their records. Nothing to do when counts[1] == 0. counts[1]
 * may also be a capacity larger than the lists: the kernel returns at once if they exceed it.
 * (The reference's pure-PyTorch visibility tests every triangle at every pixel,
 * reference.py:368-397; its Triton path bins triangles into tile chunks,
 * _triton_rasterize.py:371-424, and keeps the nearest per pixel in _tile_kernel,
 * _triton_rasterize.py:219-269.) */
int dr_raster_visibility_bin(const DrRasterGeometry* g, void* workspace, size_t workspace_bytes,
                             void* entries, const uint32_t counts[4], void* stream);

/* Visibility, third part: rasterizes the binned triangles tile by tile into keys, after
 * dr_raster_visibility_bin with the same entries and counts. Nothing to do when
 * counts[1] == 0. counts[2] is the pass's grid: 0, or at least one workgroup per 16x16 tile,
 * runs one workgroup per tile when that is at most 65536 workgroups; any smaller grid (rounded
 * up to a multiple of 8) runs a looping kernel in which each workgroup takes every
 * (grid / 8)-th busy tile of its XCD share. Either way every tile is covered, whatever
 * counts[2] and counts[3] hold; counts[2] as dr_raster_visibility_begin returns it is the
 * smallest grid that gives each busy tile its own workgroup. counts[3] is not read. */
int dr_raster_visibility_tiles(const DrRasterGeometry* g, const uint64_t* prev_keys,
                               uint64_t* keys, void* workspace, size_t workspace_bytes,
                               const void* entries, const uint32_t counts[4], void* stream);

/* The overflow pass on its own, after dr_raster_visibility_bin and _tiles were queued with a
 * buffer of entry_capacity entries: when the lists turned out longer (the device knows; the
 * host need not), it rasterizes the binned triangles straight into keys; otherwise it returns
 * at once. dr_raster_visibility_start (host_counts may be NULL), _bin, _tiles and this pass,
 * queued in turn, are dr_raster_visibility below in four calls. */
int dr_raster_visibility_overflow(const DrRasterGeometry* g, const uint64_t* prev_keys,
                                  uint64_t* keys, void* workspace, size_t workspace_bytes,
                                  uint32_t entry_capacity, void* stream);

/* The whole visibility in one call that never waits for the host: the work of
 * dr_raster_visibility_start, then the bin and tile passes with an entry buffer of
 * entry_capacity 8-byte entries (entries may be NULL when it is 0) and a tile pass of tile_groups
 * workgroups (as counts[2] above; 0: one per tile), then an overflow pass. If the tile lists
 * turn out longer than the buffer, the bin and tile passes return without work and the overflow
 * pass rasterizes the binned triangles straight into keys (64-bit atomic min per covered pixel:
 * the same keys, more work), so the result never depends on the capacity. host_counts
 * (nullable; pinned host memory) receives the four counts of dr_raster_visibility_begin once
 * the stream passes this call, for sizing the next call of the same shape. Nothing here
 * allocates or synchronises, so the call can be captured in a HIP graph (host_counts NULL).
 * (Same reference interfaces as dr_raster_visibility_begin: rasterize_layer,
 * src/diffrast/backends/triton.py:21-40, whose binning sizes its buffers on the host,
 * _triton_rasterize.py:387-424.) */
int dr_raster_visibility(const DrRasterGeometry* g, const uint64_t* prev_keys, uint64_t* keys,
                         void* workspace, size_t workspace_bytes, void* entries,
                         uint32_t entry_capacity, uint32_t tile_groups, uint32_t* host_counts,
                         void* stream);

/* dr_raster_visibility without a workspace or an entry buffer from the caller: both live in
 * one static device buffer of 64 MiB, `scratch`, so the call allocates nothing (no hipMalloc,
 * no allocating library routine) and waits for nothing. No counterpart in the reference: it is
 * for callers that cannot allocate -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation. Limit: the visibility workspace of the geometry
 * (dr_raster_workspace_size) must leave room for 4096 tile entries, i.e. be at most
 * 64 MiB - 32 KiB (DR_ERR_SCRATCH otherwise: about 590K triangle instances at 512x512, 710K
 * at 4 x 1024^2); tile lists beyond the rest of the buffer go through the overflow pass.
 * The buffer is part of the library's device code: each GPU on which the library's code is
 * loaded (the first launch of any of its kernels there, whichever entry point) holds its own
 * 64 MiB copy until the process ends, also in processes that never call this entry point.
 * Every call on a GPU shares that GPU's buffer: calls that overlap on one GPU (other streams,
 * other threads) race and must be serialised by the caller.
 * Each call prepares what it reads, so what an earlier call left there does not matter. */
int dr_raster_visibility_static(const DrRasterGeometry* g, const uint64_t* prev_keys,
                                uint64_t* keys, void* stream);

/* rast [batch, h, w, 4] = (u, v, z/w, id + 1) and rast_db [batch, h, w, 4] = (du/dx, du/dy,
 * dv/dx, dv/dy) from keys; zeros where a key is empty. rast_db may be NULL.
 * (reference.py:69-114; Triton resolve _triton_resolve.py:84-116) */
int dr_resolve_forward(const DrRasterGeometry* g, const uint64_t* keys, float* rast,
                       float* rast_db, void* stream);

/* Accumulates into grad_pos (same layout as pos; batch 1 when pos is shared) the gradient
 * of rast[..., 0:3] (grad_rast) and, if grad_rast_db is not NULL, of rast_db.
 * (_triton_resolve.py:156-244) */
int dr_resolve_backward(const DrRasterGeometry* g, const uint64_t* keys, const float* grad_rast,
                        const float* grad_rast_db, float* grad_pos, void* stream);

/* ---------------------------------------------------------------------------------------
 * Interpolate. Replaces interpolate(attr, rast, tri, rast_db, diff_attrs)
 * (src/diffrast/backends/triton.py:50-56, reference.py:117-146).
 * ------------------------------------------------------------------------------------- */
typedef struct DrInterpolateArgs {
  const float* attr;           /* [attr_batch, num_vertices, channels] */
  int64_t attr_batch_stride;   /* floats; 0 when shared by all images */
  int32_t num_vertices;
  int32_t channels;
  const float* rast;           /* [batch, h, w, 4] */
  const float* rast_db;        /* [batch, h, w, 4]; may be NULL when num_diff == 0 */
  const int32_t* tri;          /* [num_tri, 3] */
  int32_t num_tri;
  int32_t batch;
  int32_t height;
  int32_t width;
  int32_t num_diff;            /* channels with screen-space derivatives */
  const int32_t* diff;         /* [num_diff] channel indices, on the device */
} DrInterpolateArgs;

/* out [batch, h, w, channels], out_da [batch, h, w, 2 * num_diff] (NULL if num_diff == 0). */
int dr_interpolate_forward(const DrInterpolateArgs* a, float* out, float* out_da, void* stream);

/* Gradients: grad_attr is accumulated (zeroed by the caller; layout of attr); grad_rast
 * [batch, h, w, 4] and grad_rast_db [batch, h, w, 4] are written. Any output may be NULL;
 * grad_out_da may be NULL (no gradient reaches out_da). */
int dr_interpolate_backward(const DrInterpolateArgs* a, const float* grad_out,
                            const float* grad_out_da, float* grad_attr, float* grad_rast,
                            float* grad_rast_db, void* stream);

/* ---------------------------------------------------------------------------------------
 * Texture. Replaces texture(tex, uv, uv_da, filter_mode, boundary_mode, max_mip_level,
 * mip_level_bias, mip, packed) (src/diffrast/backends/triton.py:59-79, reference.py:149-194,
 * cube maps _cube.py:44-143) and the mip chain / packing of reference.py:405-519.
 *
 * Texels of every level live in one packed buffer [tex_batch, num_texels, channels]; level k
 * starts at texel level_offset[k] and holds faces * level_height[k] * level_width[k] texels
 * (faces = 6 for a cube map, face f at rows [f h, (f + 1) h)).
 * ------------------------------------------------------------------------------------- */
#define DR_MAX_LEVELS 32
enum { DR_FILTER_NEAREST = 0, DR_FILTER_LINEAR = 1, DR_FILTER_MIP_NEAREST = 2,
       DR_FILTER_MIP_LINEAR = 3 };
enum { DR_BOUNDARY_WRAP = 0, DR_BOUNDARY_CLAMP = 1, DR_BOUNDARY_ZERO = 2, DR_BOUNDARY_CUBE = 3 };

typedef struct DrTextureArgs {
  const float* texels;         /* packed levels */
  int32_t tex_batch;           /* 1 (shared) or batch */
  int32_t channels;
  int64_t num_texels;          /* texels per batch entry of the packed buffer (< 2^32 - 1) */
  int32_t num_levels;          /* levels a lookup may use (<= DR_MAX_LEVELS) */
  int32_t faces;               /* 1, or 6 for a cube map */
  int32_t level_height[DR_MAX_LEVELS];
  int32_t level_width[DR_MAX_LEVELS];
  int64_t level_offset[DR_MAX_LEVELS];
  const float* uv;             /* [batch, h, w, 2], or 3 direction components for a cube */
  const float* uv_da;          /* [batch, h, w, 4] (6 for a cube) or NULL */
  const float* bias;           /* [batch, h, w] mip level bias or NULL */
  int32_t batch;
  int32_t height;
  int32_t width;
  int32_t filter;              /* DR_FILTER_* */
  int32_t boundary;            /* DR_BOUNDARY_* */
} DrTextureArgs;

/* out [batch, h, w, channels]. */
int dr_texture_forward(const DrTextureArgs* a, float* out, void* stream);

/* grad_texels (packed layout, zeroed by the caller) is accumulated; grad_uv, grad_uv_da and
 * grad_bias (each nullable) are written. */
int dr_texture_backward(const DrTextureArgs* a, const float* grad_out, float* grad_texels,
                        float* grad_uv, float* grad_uv_da, float* grad_bias, void* stream);

/* Builds levels 1 .. num_levels-1 of the packed buffer from level 0, halving each size
 * (rounding up) with exact area weights (reference.py:433-488). base (nullable) holds level 0
 * on its own, [tex_batch, faces * level_height[0] * level_width[0], channels]: it is copied
 * into the packed buffer by the same pass that reads it; NULL: level 0 is there already. */
int dr_mip_build(float* texels, const float* base, int32_t tex_batch, int32_t channels,
                 int64_t num_texels, int32_t faces, int32_t num_levels,
                 const int32_t* level_height, const int32_t* level_width,
                 const int64_t* level_offset, void* stream);

/* Adjoint of dr_mip_build: adds the gradient held in levels num_levels-1 .. 1 of the packed
 * gradient buffer down into level 0, in place. */
int dr_mip_build_backward(float* grad_texels, int32_t tex_batch, int32_t channels,
                          int64_t num_texels, int32_t faces, int32_t num_levels,
                          const int32_t* level_height, const int32_t* level_width,
                          const int64_t* level_offset, void* stream);

/* ---------------------------------------------------------------------------------------
 * Antialias. Replaces antialias(color, rast, pos, tri, pos_gradient_boost, neighbours)
 * (src/diffrast/backends/triton.py:82-92, reference.py:202-265, 675-765) and the edge
 * adjacency and silhouette classification (reference.py:768-814, topology.py:19-72).
 * ------------------------------------------------------------------------------------- */

/* Bytes of workspace for dr_edge_neighbours. */
int dr_edge_hash_workspace_size(int32_t num_tri, size_t* bytes);

/* neighbours [num_tri, 3] int32: for edge k (opposite vertex k) of each triangle, the number
 * 3 t' + k' of the same edge in the only other triangle that uses it, or -1 when no other
 * triangle or more than one does. Built with a GPU hash table (reference.py:768-787). */
int dr_edge_neighbours(const int32_t* tri, int32_t num_tri, void* workspace,
                       size_t workspace_bytes, int32_t* neighbours, void* stream);

/* mask [pos_batch, num_tri] uint8, bit k set when edge k is a silhouette: unshared,
 * non-manifold, or folded in this projection (reference.py:790-814). With rast
 * ([batch, height, width, 4], not NULL) only the triangles that rast shows get their bits and
 * every other entry is 0: antialiasing reads the bits of shown triangles only
 * (reference.py:228-258). pos_batch is 1 or batch. */
int dr_silhouette_mask(const float* pos, int64_t pos_batch_stride, int32_t pos_batch,
                       const int32_t* tri, int32_t num_tri, const int32_t* neighbours,
                       const float* rast, int32_t batch, int32_t height, int32_t width,
                       uint8_t* mask, void* stream);

typedef struct DrAntialiasArgs {
  const float* color;          /* [batch, h, w, channels] */
  int32_t channels;
  int32_t batch;
  int32_t height;
  int32_t width;
  const float* rast;           /* [batch, h, w, 4] */
  const float* pos;            /* float4 per vertex */
  int64_t pos_batch_stride;    /* floats; 0 when shared */
  const int32_t* tri;
  int32_t num_tri;
  const uint8_t* silhouette;   /* dr_silhouette_mask output */
  int64_t silhouette_batch_stride; /* num_tri, or 0 when pos is shared */
  float boost;                 /* pos_gradient_boost */
} DrAntialiasArgs;

/* Bytes of the pair records that dr_antialias_forward writes and dr_antialias_backward
 * reads (10 per pixel and one per 16x16 tile). */
int dr_antialias_workspace_size(const DrAntialiasArgs* a, size_t* bytes);

/* out [batch, h, w, channels] = color blended across silhouette edges; also fills the pair
 * records (crossing t and owner/edge bits of each pixel's right and lower pair). */
int dr_antialias_forward(const DrAntialiasArgs* a, void* pairs, size_t pairs_bytes, float* out,
                         void* stream);

/* grad_color (written, nullable) and grad_pos (accumulated, nullable; layout of pos) from the
 * pair records of the forward pass. */
int dr_antialias_backward(const DrAntialiasArgs* a, const void* pairs, size_t pairs_bytes,
                          const float* grad_out, float* grad_color, float* grad_pos,
                          void* stream);

/* ---------------------------------------------------------------------------------------
 * float64 variants, for gradient-check-grade work. The reference's GPU backend accepts float64
 * tensors at the backend level (its resolve is checked to 1e-12, tests/test_coverage.py:792-808;
 * interpolate and texture by gradcheck, tests/test_triton.py:234-240, :303-319; antialias to
 * 1e-9, :408-415) and runs the same entry points: rasterize, interpolate, texture and
 * antialias of src/diffrast/backends/triton.py:14-92. Here each has a _f64 twin taking the same
 * argument structs, whose float arrays (pos, attr, rast, rast_db, texels, uv, uv_da, bias, color)
 * then hold doubles, with strides counted in doubles; outputs and gradients are double. These
 * kernels are plain (one thread per pixel, float64 atomics). Visibility has no twin: as in the
 * reference's GPU backend, the keys come from float32 positions, and only the resolve is
 * float64.
 * ------------------------------------------------------------------------------------- */

/* dr_resolve_forward / _backward in double (grad_pos accumulated, zeroed by the caller). */
int dr_resolve_forward_f64(const DrRasterGeometry* g, const uint64_t* keys, double* rast,
                           double* rast_db, void* stream);
int dr_resolve_backward_f64(const DrRasterGeometry* g, const uint64_t* keys,
                            const double* grad_rast, const double* grad_rast_db,
                            double* grad_pos, void* stream);

/* dr_interpolate_forward / _backward in double (grad_attr accumulated, zeroed by the caller). */
int dr_interpolate_forward_f64(const DrInterpolateArgs* a, double* out, double* out_da,
                               void* stream);
int dr_interpolate_backward_f64(const DrInterpolateArgs* a, const double* grad_out,
                                const double* grad_out_da, double* grad_attr, double* grad_rast,
                                double* grad_rast_db, void* stream);

/* dr_texture_forward / _backward and the mip chain in double (grad_texels accumulated, zeroed by
 * the caller). */
int dr_texture_forward_f64(const DrTextureArgs* a, double* out, void* stream);
int dr_texture_backward_f64(const DrTextureArgs* a, const double* grad_out, double* grad_texels,
                            double* grad_uv, double* grad_uv_da, double* grad_bias,
                            void* stream);
int dr_mip_build_f64(double* texels, const double* base, int32_t tex_batch, int32_t channels,
                     int64_t num_texels, int32_t faces, int32_t num_levels,
                     const int32_t* level_height, const int32_t* level_width,
                     const int64_t* level_offset, void* stream);
int dr_mip_build_backward_f64(double* grad_texels, int32_t tex_batch, int32_t channels,
                              int64_t num_texels, int32_t faces, int32_t num_levels,
                              const int32_t* level_height, const int32_t* level_width,
                              const int64_t* level_offset, void* stream);

/* Silhouette bits of every (pos batch, triangle) from float64 positions (as dr_silhouette_mask
 * without rast). */
int dr_silhouette_mask_f64(const double* pos, int64_t pos_batch_stride, int32_t pos_batch,
                           const int32_t* tri, int32_t num_tri, const int32_t* neighbours,
                           uint8_t* mask, void* stream);

/* Antialias in double: pair records of 18 bytes per pixel (dr_antialias_workspace_size_f64);
 * grad_pos accumulated, zeroed by the caller. */
int dr_antialias_workspace_size_f64(const DrAntialiasArgs* a, size_t* bytes);
int dr_antialias_forward_f64(const DrAntialiasArgs* a, void* pairs, size_t pairs_bytes,
                             double* out, void* stream);
int dr_antialias_backward_f64(const DrAntialiasArgs* a, const void* pairs, size_t pairs_bytes,
                              const double* grad_out, double* grad_color, double* grad_pos,
                              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DIFFRAST_HIP_H */
