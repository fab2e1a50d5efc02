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
  hipLaunchKernelGGL((raster_fwd_kernel<CDIM, TILE, SoASplats<CDIM>>),
                     dim3(G.C, G.tile_h, G.tile_w), dim3(TILE * TILE), 0, s, G, src, bg, offsets,
                     flat, colors, alphas, last);
}

template <int CDIM, int TILE>
static void launch_bwd(const RasterGeom& G, const SoASplats<CDIM>& src, const SoAGrads<CDIM>& dst,
                       const float* bg, const int32_t* offsets, const int32_t* flat,
                       const float* alphas, const int32_t* last, const float* v_colors,
                       const float* v_alphas, hipStream_t s) {
  hipLaunchKernelGGL((raster_bwd_kernel<CDIM, TILE, SoASplats<CDIM>, SoAGrads<CDIM>>),
                     dim3(G.C, G.tile_h, G.tile_w), dim3(TILE * TILE), 0, s, G, src, dst, bg,
                     offsets, flat, alphas, last, v_colors, v_alphas);
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
