// Gaussian-tile intersection: per-Gaussian tile counts, key/id emission and
// per-(camera, tile) offset encoding.
//
// Reference: gsplat/cuda/csrc/isect_tiles.cu:14-98 (kernel), :100-232 (host),
// :234-301 (offset encode).
//   tile rect  [floor(x/ts - r/ts), ceil(x/ts + r/ts)) clamped to the grid
//   key        cam << (32 + tile_bits) | tile << 32 | int32 bits of depth
//              (sign-extended to 64 bits, as the reference does)
//   flatten id index into [C*N] (non-packed) or [nnz] (packed)
//   offsets    offsets[c, tile] = first isect index of that (camera, tile) run;
//              empty tiles take the next run's start; trailing tiles take n.
#include "tgs_common.cuh"

struct TileRect {
  uint32_t x0, y0, x1, y1;
};

// Clamp a floor/ceil value into [0, limit] the way the reference's unsigned
// conversion followed by min/max does for finite inputs.
__device__ __forceinline__ uint32_t clamp_tile(float v, uint32_t limit) {
  if (!(v > 0.f)) return 0u;  // negatives (and NaN) saturate to 0
  if (v >= (float)limit) return limit;
  return (uint32_t)v;
}

__device__ __forceinline__ TileRect tile_rect(float mx, float my, int32_t radius, uint32_t tile_size,
                                              uint32_t tw, uint32_t th) {
  const float ts = (float)tile_size;
  const float tr = (float)radius / ts;
  const float tx = mx / ts;
  const float ty = my / ts;
  TileRect r;
  r.x0 = clamp_tile(floorf(tx - tr), tw);
  r.y0 = clamp_tile(floorf(ty - tr), th);
  r.x1 = clamp_tile(ceilf(tx + tr), tw);
  r.y1 = clamp_tile(ceilf(ty + tr), th);
  return r;
}

__global__ void __launch_bounds__(256) isect_count_kernel(
    uint64_t total, const float* __restrict__ means2d, const int32_t* __restrict__ radii,
    uint32_t tile_size, uint32_t tw, uint32_t th, int32_t* __restrict__ tiles_per_gauss) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int32_t radius = radii[idx];
  if (radius <= 0) {
    tiles_per_gauss[idx] = 0;
    return;
  }
  const TileRect r = tile_rect(means2d[idx * 2], means2d[idx * 2 + 1], radius, tile_size, tw, th);
  const uint32_t nx = r.x1 > r.x0 ? r.x1 - r.x0 : 0u;
  const uint32_t ny = r.y1 > r.y0 ? r.y1 - r.y0 : 0u;
  tiles_per_gauss[idx] = (int32_t)(nx * ny);
}

__global__ void __launch_bounds__(256) isect_emit_kernel(
    uint64_t total, uint32_t N, const int64_t* __restrict__ camera_ids,
    const float* __restrict__ means2d, const int32_t* __restrict__ radii,
    const float* __restrict__ depths, const int64_t* __restrict__ cum_tiles, uint32_t tile_size,
    uint32_t tw, uint32_t th, uint32_t tile_n_bits, int64_t* __restrict__ isect_ids,
    int32_t* __restrict__ flatten_ids) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int32_t radius = radii[idx];
  if (radius <= 0) return;
  const TileRect r = tile_rect(means2d[idx * 2], means2d[idx * 2 + 1], radius, tile_size, tw, th);
  const int64_t cid = camera_ids ? camera_ids[idx] : (int64_t)(idx / N);
  const int64_t cam_enc = cid << (32 + tile_n_bits);
  const int64_t depth_enc = (int64_t)__float_as_int(depths[idx]);  // sign-extended
  int64_t cur = idx == 0 ? 0 : cum_tiles[idx - 1];
  for (uint32_t y = r.y0; y < r.y1; ++y) {
    for (uint32_t x = r.x0; x < r.x1; ++x) {
      const int64_t tile = (int64_t)y * tw + x;
      isect_ids[cur] = cam_enc | (tile << 32) | depth_enc;
      flatten_ids[cur] = (int32_t)idx;
      ++cur;
    }
  }
}

__global__ void __launch_bounds__(256) isect_offset_encode_kernel(
    uint64_t n_isects, const int64_t* __restrict__ isect_ids, uint32_t C, uint32_t n_tiles,
    uint32_t tile_n_bits, int32_t* __restrict__ offsets) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n_isects) return;
  const int64_t total = (int64_t)C * n_tiles;
  const int64_t tmask = ((int64_t)1 << tile_n_bits) - 1;
  auto bucket = [&](int64_t key) {
    const int64_t hi = key >> 32;
    int64_t id = (hi >> tile_n_bits) * n_tiles + (hi & tmask);
    // Keys built from non-negative depths always land in [0, total); clamp so
    // malformed keys can never write outside offsets.
    if (id < 0) id = -1;
    if (id >= total) id = total - 1;
    return id;
  };
  const int64_t cur = bucket(isect_ids[idx]);
  if (idx == 0) {
    for (int64_t i = 0; i <= cur; ++i) offsets[i] = 0;
  }
  if (idx == n_isects - 1) {
    for (int64_t i = cur + 1; i < total; ++i) offsets[i] = (int32_t)n_isects;
  }
  if (idx > 0) {
    const int64_t prev = bucket(isect_ids[idx - 1]);
    if (prev == cur) return;
    for (int64_t i = prev + 1; i <= cur; ++i) offsets[i] = (int32_t)idx;
  }
}

extern "C" uint32_t tgs_bit_width(uint32_t v) {
  uint32_t b = 0;
  while (v) {
    ++b;
    v >>= 1;
  }
  return b;
}

extern "C" int tgs_isect_tiles_count(uint64_t total, const float* means2d, const int32_t* radii,
                                     uint32_t tile_size, uint32_t tile_width,
                                     uint32_t tile_height, int32_t* tiles_per_gauss,
                                     hipStream_t stream) {
  if (total == 0) return TGS_OK;
  TGS_CHECK_ARG(means2d && radii && tiles_per_gauss, "isect_tiles_count: null pointer");
  TGS_CHECK_ARG(tile_size > 0, "tile_size must be > 0");
  TGS_CHECK_ARG(total < (1ull << 31), "isect_tiles: C*N (or nnz) must fit int32 flatten ids");
  hipLaunchKernelGGL(isect_count_kernel, dim3(tgs_blocks(total, 256)), dim3(256), 0, stream,
                     total, means2d, radii, tile_size, tile_width, tile_height, tiles_per_gauss);
  TGS_RETURN_LAUNCH("tgs_isect_tiles_count");
}

// camera_ids: [total] int64 for packed inputs, or null with N = Gaussians per
// camera for [C, N] inputs.
extern "C" int tgs_isect_tiles_emit(uint64_t total, uint32_t N, const int64_t* camera_ids,
                                    const float* means2d, const int32_t* radii,
                                    const float* depths, const int64_t* cum_tiles_per_gauss,
                                    uint32_t tile_size, uint32_t tile_width, uint32_t tile_height,
                                    uint32_t tile_n_bits, int64_t* isect_ids,
                                    int32_t* flatten_ids, hipStream_t stream) {
  if (total == 0) return TGS_OK;
  TGS_CHECK_ARG(means2d && radii && depths && cum_tiles_per_gauss && isect_ids && flatten_ids,
                "isect_tiles_emit: null pointer");
  TGS_CHECK_ARG(camera_ids || N > 0, "isect_tiles_emit: need camera_ids or N");
  hipLaunchKernelGGL(isect_emit_kernel, dim3(tgs_blocks(total, 256)), dim3(256), 0, stream, total,
                     N, camera_ids, means2d, radii, depths, cum_tiles_per_gauss, tile_size,
                     tile_width, tile_height, tile_n_bits, isect_ids, flatten_ids);
  TGS_RETURN_LAUNCH("tgs_isect_tiles_emit");
}

extern "C" int tgs_isect_offset_encode(uint64_t n_isects, const int64_t* isect_ids, uint32_t C,
                                       uint32_t tile_width, uint32_t tile_height,
                                       int32_t* offsets, hipStream_t stream) {
  const uint64_t total = (uint64_t)C * tile_width * tile_height;
  if (total == 0) return TGS_OK;
  TGS_CHECK_ARG(offsets != nullptr, "isect_offset_encode: null offsets");
  if (n_isects == 0) {
    // reference: offsets.fill_(0) (isect_tiles.cu:298)
    return tgs_fill_u32(offsets, total, 0u, stream);
  }
  TGS_CHECK_ARG(isect_ids != nullptr, "isect_offset_encode: null isect_ids");
  const uint32_t n_tiles = tile_width * tile_height;
  const uint32_t tile_n_bits = tgs_bit_width(n_tiles);
  hipLaunchKernelGGL(isect_offset_encode_kernel, dim3(tgs_blocks(n_isects, 256)), dim3(256), 0,
                     stream, n_isects, isect_ids, C, n_tiles, tile_n_bits, offsets);
  TGS_RETURN_LAUNCH("tgs_isect_offset_encode");
}
