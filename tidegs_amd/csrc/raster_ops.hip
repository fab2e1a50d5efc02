// gsplat-compatible rasterize_to_pixels forward/backward entry points.
//
// Reference: gsplat/cuda/csrc/rasterize_to_pixels_fwd.cu:162-284 and
// rasterize_to_pixels_bwd.cu:251-402.  means2d/conics/colors/opacities are
// either [C,N,*] or packed [nnz,*]; flatten_ids index the flattened leading
// dimension in both cases, so one code path serves both.  Gradient buffers
// must be zero-initialised by the caller (the reference allocates them with
// zeros_like).  Channel counts are instantiated for {1,2,3,4,8,16,32};
// tile_size for {8,16}.
#include "raster.cuh"

template <int CDIM, int TILE>
static void launch_fwd(const RasterGeom& G, const SoASplats<CDIM>& src, const float* bg,
                       const int32_t* offsets, const int32_t* flat, float* colors, float* alphas,
                       int32_t* last, hipStream_t s) {
  hipLaunchKernelGGL((raster_fwd_kernel<CDIM, TILE, SoASplats<CDIM>>), raster_fwd_grid(G),
                     dim3(TILE * TILE), 0, s, G, src, bg, offsets, flat, colors, alphas, last);
}

template <int CDIM, int TILE>
static void launch_bwd(const RasterGeom& G, const SoASplats<CDIM>& src, const SoAGrads<CDIM>& dst,
                       const float* bg, const int32_t* offsets, const int32_t* flat,
                       const float* alphas, const int32_t* last, const float* v_colors,
                       const float* v_alphas, hipStream_t s) {
  hipLaunchKernelGGL((raster_bwd_kernel<CDIM, TILE, SoASplats<CDIM>, SoAGrads<CDIM>>),
                     raster_bwd_grid(G), dim3(TILE * TILE), 0, s, G, src, dst, bg, offsets, flat,
                     alphas, last, v_colors, v_alphas);
}

template <int CDIM>
static int dispatch_fwd(uint32_t tile_size, const RasterGeom& G, const float* means2d,
                        const float* conics, const float* colors, const float* opacities,
                        const float* bg, const int32_t* offsets, const int32_t* flat,
                        float* out_colors, float* out_alphas, int32_t* last, hipStream_t s) {
  SoASplats<CDIM> src{means2d, conics, colors, opacities};
  if (tile_size == 16)
    launch_fwd<CDIM, 16>(G, src, bg, offsets, flat, out_colors, out_alphas, last, s);
  else if (tile_size == 8)
    launch_fwd<CDIM, 8>(G, src, bg, offsets, flat, out_colors, out_alphas, last, s);
  else {
    tgs_set_error("rasterize_to_pixels: tile_size %u not supported (8 or 16)", tile_size);
    return TGS_ERR_UNSUPPORTED;
  }
  TGS_RETURN_LAUNCH("tgs_rasterize_to_pixels_fwd");
}

template <int CDIM>
static int dispatch_bwd(uint32_t tile_size, const RasterGeom& G, const float* means2d,
                        const float* conics, const float* colors, const float* opacities,
                        const float* bg, const int32_t* offsets, const int32_t* flat,
                        const float* alphas, const int32_t* last, const float* v_colors,
                        const float* v_alphas, float* v_means2d_abs, float* v_means2d,
                        float* v_conics, float* v_colors_out, float* v_opacities, hipStream_t s) {
  SoASplats<CDIM> src{means2d, conics, colors, opacities};
  SoAGrads<CDIM> dst{v_means2d, v_conics, v_colors_out, v_opacities, v_means2d_abs};
  if (tile_size == 16)
    launch_bwd<CDIM, 16>(G, src, dst, bg, offsets, flat, alphas, last, v_colors, v_alphas, s);
  else if (tile_size == 8)
    launch_bwd<CDIM, 8>(G, src, dst, bg, offsets, flat, alphas, last, v_colors, v_alphas, s);
  else {
    tgs_set_error("rasterize_to_pixels: tile_size %u not supported (8 or 16)", tile_size);
    return TGS_ERR_UNSUPPORTED;
  }
  TGS_RETURN_LAUNCH("tgs_rasterize_to_pixels_bwd");
}

#define TGS_CHANNEL_CASES(X) X(1) X(2) X(3) X(4) X(8) X(16) X(32)

extern "C" int tgs_rasterize_supported_channels(int32_t* out, int32_t cap) {
  const int32_t list[] = {1, 2, 3, 4, 8, 16, 32};
  const int32_t n = (int32_t)(sizeof(list) / sizeof(list[0]));
  for (int32_t k = 0; k < n && k < cap; ++k) out[k] = list[k];
  return n;
}

extern "C" int tgs_rasterize_to_pixels_fwd(
    uint32_t C, uint32_t channels, const float* means2d, const float* conics, const float* colors,
    const float* opacities, const float* backgrounds, uint32_t image_width, uint32_t image_height,
    uint32_t tile_size, uint32_t tile_width, uint32_t tile_height, const int32_t* tile_offsets,
    const int32_t* flatten_ids, uint32_t n_isects, float* render_colors, float* render_alphas,
    int32_t* last_ids, hipStream_t stream) {
  if (C == 0 || image_width == 0 || image_height == 0) return TGS_OK;
  TGS_CHECK_ARG(tile_offsets && render_colors && render_alphas && last_ids,
                "rasterize_to_pixels_fwd: null pointer");
  TGS_CHECK_ARG(n_isects == 0 || (means2d && conics && colors && opacities && flatten_ids),
                "rasterize_to_pixels_fwd: null splat pointer");
  TGS_CHECK_ARG(tile_width * tile_size >= image_width && tile_height * tile_size >= image_height,
                "rasterize_to_pixels_fwd: tile grid does not cover the image");
  TGS_CHECK_ARG(C <= 65535 && tile_width <= 65535 && tile_height <= 65535,
                "rasterize_to_pixels_fwd: at most 65535 cameras and tiles per image side");
  const RasterGeom G{C, image_width, image_height, tile_width, tile_height, n_isects};
#define TGS_FWD_CASE(D)                                                                      \
  case D:                                                                                    \
    return dispatch_fwd<D>(tile_size, G, means2d, conics, colors, opacities, backgrounds,     \
                           tile_offsets, flatten_ids, render_colors, render_alphas, last_ids, \
                           stream);
  switch (channels) {
    TGS_CHANNEL_CASES(TGS_FWD_CASE)
    default:
      tgs_set_error("rasterize_to_pixels: unsupported number of channels %u", channels);
      return TGS_ERR_UNSUPPORTED;
  }
#undef TGS_FWD_CASE
}

extern "C" int tgs_rasterize_to_pixels_bwd(
    uint32_t C, uint32_t channels, const float* means2d, const float* conics, const float* colors,
    const float* opacities, const float* backgrounds, uint32_t image_width, uint32_t image_height,
    uint32_t tile_size, uint32_t tile_width, uint32_t tile_height, const int32_t* tile_offsets,
    const int32_t* flatten_ids, uint32_t n_isects, const float* render_alphas,
    const int32_t* last_ids, const float* v_render_colors, const float* v_render_alphas,
    float* v_means2d_abs, float* v_means2d, float* v_conics, float* v_colors, float* v_opacities,
    hipStream_t stream) {
  if (C == 0 || n_isects == 0 || image_width == 0 || image_height == 0) return TGS_OK;
  TGS_CHECK_ARG(means2d && conics && colors && opacities && tile_offsets && flatten_ids &&
                    render_alphas && last_ids && v_render_colors && v_means2d && v_conics &&
                    v_colors && v_opacities,
                "rasterize_to_pixels_bwd: null pointer");
  TGS_CHECK_ARG(tile_width * tile_size >= image_width && tile_height * tile_size >= image_height,
                "rasterize_to_pixels_bwd: tile grid does not cover the image");
  TGS_CHECK_ARG(C <= 65535 && tile_width <= 65535 && tile_height <= 65535,
                "rasterize_to_pixels_bwd: at most 65535 cameras and tiles per image side");
  const RasterGeom G{C, image_width, image_height, tile_width, tile_height, n_isects};
#define TGS_BWD_CASE(D)                                                                         \
  case D:                                                                                       \
    return dispatch_bwd<D>(tile_size, G, means2d, conics, colors, opacities, backgrounds,        \
                           tile_offsets, flatten_ids, render_alphas, last_ids, v_render_colors,  \
                           v_render_alphas, v_means2d_abs, v_means2d, v_conics, v_colors,        \
                           v_opacities, stream);
  switch (channels) {
    TGS_CHANNEL_CASES(TGS_BWD_CASE)
    default:
      tgs_set_error("rasterize_to_pixels: unsupported number of channels %u", channels);
      return TGS_ERR_UNSUPPORTED;
  }
#undef TGS_BWD_CASE
}

// ---------------------------------------------------------------------------
// Packed records for the 3-channel case: the drop-in op packs gsplat's SoA
// tensors into the fused step's 48-byte splat records (one gather per
// staged Gaussian instead of four) and runs tgs_tide_rasterize_fwd/bwd on
// them; the backward's 9-float gradient records are unpacked into the SoA
// gradient tensors.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) pack_splats_kernel(uint64_t n, const float* __restrict__ m2d,
                                                          const float* __restrict__ con,
                                                          const float* __restrict__ col,
                                                          const float* __restrict__ op,
                                                          float4* __restrict__ rec) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= n) return;
  rec[3 * i + 0] = make_float4(m2d[2 * i], m2d[2 * i + 1], op[i], 0.f);
  rec[3 * i + 1] = make_float4(con[3 * i], con[3 * i + 1], con[3 * i + 2], 0.f);
  // a colour of -0.0 marks a channel clamped by the projection (the packed
  // rasterizer then drops its gradient); caller colours carry no such mark
  auto unmark = [](float c) { return __float_as_uint(c) == 0x80000000u ? 0.f : c; };
  rec[3 * i + 2] =
      make_float4(unmark(col[3 * i]), unmark(col[3 * i + 1]), unmark(col[3 * i + 2]), 0.f);
}

__global__ void __launch_bounds__(256) unpack_splat_grads_kernel(
    uint64_t n, const float* __restrict__ g, float* __restrict__ v_m2d,
    float* __restrict__ v_con, float* __restrict__ v_col, float* __restrict__ v_op) {
  const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if (i >= n) return;
  const float* r = g + 9 * i;
  v_m2d[2 * i] = r[0];
  v_m2d[2 * i + 1] = r[1];
  v_con[3 * i] = r[2];
  v_con[3 * i + 1] = r[3];
  v_con[3 * i + 2] = r[4];
  v_col[3 * i] = r[5];
  v_col[3 * i + 1] = r[6];
  v_col[3 * i + 2] = r[7];
  v_op[i] = r[8];
}

extern "C" int tgs_pack_splats(uint64_t n, const float* means2d, const float* conics,
                               const float* colors, const float* opacities, float* splats,
                               hipStream_t stream) {
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(means2d && conics && colors && opacities && splats, "pack_splats: null pointer");
  TGS_CHECK_ARG(((uintptr_t)splats & 15u) == 0, "pack_splats: splats must be 16-byte aligned");
  hipLaunchKernelGGL(pack_splats_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     n, means2d, conics, colors, opacities, (float4*)splats);
  TGS_RETURN_LAUNCH("tgs_pack_splats");
}

extern "C" int tgs_unpack_splat_grads(uint64_t n, const float* splat_grads, float* v_means2d,
                                      float* v_conics, float* v_colors, float* v_opacities,
                                      hipStream_t stream) {
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(splat_grads && v_means2d && v_conics && v_colors && v_opacities,
                "unpack_splat_grads: null pointer");
  hipLaunchKernelGGL(unpack_splat_grads_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     stream, n, splat_grads, v_means2d, v_conics, v_colors, v_opacities);
  TGS_RETURN_LAUNCH("tgs_unpack_splat_grads");
}

