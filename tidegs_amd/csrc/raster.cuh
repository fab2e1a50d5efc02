// Tile-based alpha compositing, forward and backward, for wave64 / gfx950.
//
// Reference: gsplat/cuda/csrc/rasterize_to_pixels_fwd.cu:14-160 and
// rasterize_to_pixels_bwd.cu:14-249.  Per pixel (px = j + 0.5, py = i + 0.5):
//   sigma = 0.5 (a dx^2 + c dy^2) + b dx dy,  (dx, dy) = mean2d - pixel
//   alpha = min(0.999, opacity * exp(-sigma)); skip if sigma < 0 or alpha < 1/255
//   stop (exclusive) once T (1 - alpha) <= 1e-4
//   color += c alpha T; T *= 1 - alpha; last_id = index of the last contributor
// Backward replays the tile back to front from last_id, recovering T by
// division, and accumulates dL/d(mean2d, conic, color, opacity).
//
// One workgroup = one TILE x TILE tile (256 threads = 4 wavefronts for
// TILE=16).  The tile's Gaussians are staged through LDS in batches of one per
// thread.  In the backward, each wavefront reduces a Gaussian's gradient
// across its 64 pixels with DPP (tgs_wave_sum) and then issues one atomic
// instruction whose lane k adds value k, i.e. one atomic per Gaussian per
// wave rather than one per value from a single lane.
//
// The splat source/gradient sink are policies so the same kernels serve
// gsplat's SoA tensors (drop-in op) and the packed 48-byte splat records of the
// fused resident step.
#pragma once

#include "tgs_common.cuh"

template <int CDIM>
struct SplatData {
  float x, y, op;
  float a, b, c;
  float col[CDIM];
};

// gsplat tensor layout: means2d [*,2], conics [*,3], colors [*,CDIM], opacities [*].
template <int CDIM>
struct SoASplats {
  const float* means2d;
  const float* conics;
  const float* colors;
  const float* opacities;
  __device__ __forceinline__ void load(int32_t g, SplatData<CDIM>& s) const {
    s.x = means2d[(int64_t)g * 2 + 0];
    s.y = means2d[(int64_t)g * 2 + 1];
    s.op = opacities[g];
    s.a = conics[(int64_t)g * 3 + 0];
    s.b = conics[(int64_t)g * 3 + 1];
    s.c = conics[(int64_t)g * 3 + 2];
#pragma unroll
    for (int k = 0; k < CDIM; ++k) s.col[k] = colors[(int64_t)g * CDIM + k];
  }
};

// Gradient value order k: 0..1 mean2d, 2..4 conic, 5..5+CDIM-1 color,
// 5+CDIM opacity, 6+CDIM..7+CDIM |mean2d| (absgrad only).
template <int CDIM>
struct SoAGrads {
  float* v_means2d;
  float* v_conics;
  float* v_colors;
  float* v_opacities;
  float* v_means2d_abs;  // may be null
  static constexpr int NV = 6 + CDIM;
  __device__ __forceinline__ int n_values() const { return v_means2d_abs ? NV + 2 : NV; }
  __device__ __forceinline__ float* ptr(int32_t g, int k) const {
    const int64_t gg = g;
    if (k < 2) return v_means2d + gg * 2 + k;
    if (k < 5) return v_conics + gg * 3 + (k - 2);
    if (k < 5 + CDIM) return v_colors + gg * CDIM + (k - 5);
    if (k == 5 + CDIM) return v_opacities + gg;
    return v_means2d_abs + gg * 2 + (k - 6 - CDIM);
  }
};

// Packed per-splat records of the fused step (CDIM = 3):
//   rec[3g+0] = {x, y, opacity, depth}, rec[3g+1] = {a, b, c, radius},
//   rec[3g+2] = {r, g, b, 0};  gradients grads[9g + k] in SoAGrads' k order.
struct PackedSplats {
  const float4* rec;
  __device__ __forceinline__ void load(int32_t g, SplatData<3>& s) const {
    const float4 r0 = rec[(int64_t)g * 3 + 0];
    const float4 r1 = rec[(int64_t)g * 3 + 1];
    const float4 r2 = rec[(int64_t)g * 3 + 2];
    s.x = r0.x;
    s.y = r0.y;
    s.op = r0.z;
    s.a = r1.x;
    s.b = r1.y;
    s.c = r1.z;
    s.col[0] = r2.x;
    s.col[1] = r2.y;
    s.col[2] = r2.z;
  }
};

struct PackedGrads {
  float* grads;  // [V, 9]
  static constexpr int NV = 9;
  __device__ __forceinline__ int n_values() const { return NV; }
  __device__ __forceinline__ float* ptr(int32_t g, int k) const { return grads + (int64_t)g * 9 + k; }
};

struct RasterGeom {
  uint32_t C;
  uint32_t W, H;
  uint32_t tile_w, tile_h;
  uint32_t n_isects;
};

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <int CDIM, int TILE, class Src>
__global__ void __launch_bounds__(TILE* TILE) raster_fwd_kernel(
    RasterGeom G, Src src, const float* __restrict__ backgrounds,
    const int32_t* __restrict__ tile_offsets, const int32_t* __restrict__ flatten_ids,
    float* __restrict__ render_colors, float* __restrict__ render_alphas,
    int32_t* __restrict__ last_ids) {
  constexpr int BLOCK = TILE * TILE;
  __shared__ int32_t s_id[BLOCK];
  __shared__ float s_xyo[BLOCK][3];
  __shared__ float s_con[BLOCK][3];
  __shared__ float s_col[BLOCK][CDIM];

  const uint32_t cam = blockIdx.x;
  const uint32_t ty = blockIdx.y, tx = blockIdx.z;
  const uint32_t tile_id = ty * G.tile_w + tx;
  const uint32_t tr = threadIdx.x;
  const uint32_t i = ty * TILE + tr / TILE;
  const uint32_t j = tx * TILE + tr % TILE;
  const uint64_t img = (uint64_t)cam * G.H * G.W;
  const bool inside = i < G.H && j < G.W;
  const float px = (float)j + 0.5f, py = (float)i + 0.5f;

  const int32_t* offs = tile_offsets + (uint64_t)cam * G.tile_h * G.tile_w;
  const int32_t range_start = offs[tile_id];
  const int32_t range_end = (cam == G.C - 1 && tile_id == G.tile_w * G.tile_h - 1)
                                ? (int32_t)G.n_isects
                                : offs[tile_id + 1];
  const int32_t n_batches = (range_end - range_start + BLOCK - 1) / BLOCK;

  float T = 1.f;
  uint32_t cur_idx = 0;
  bool done = !inside;
  float pix[CDIM];
#pragma unroll
  for (int k = 0; k < CDIM; ++k) pix[k] = 0.f;

  for (int32_t b = 0; b < n_batches; ++b) {
    if (__syncthreads_count(done) >= BLOCK) break;
    const int32_t batch_start = range_start + BLOCK * b;
    const int32_t idx = batch_start + (int32_t)tr;
    if (idx < range_end) {
      const int32_t g = flatten_ids[idx];
      SplatData<CDIM> s;
      src.load(g, s);
      s_id[tr] = g;
      s_xyo[tr][0] = s.x;
      s_xyo[tr][1] = s.y;
      s_xyo[tr][2] = s.op;
      s_con[tr][0] = s.a;
      s_con[tr][1] = s.b;
      s_con[tr][2] = s.c;
#pragma unroll
      for (int k = 0; k < CDIM; ++k) s_col[tr][k] = s.col[k];
    }
    __syncthreads();
    const int32_t batch_size = min(BLOCK, range_end - batch_start);
    for (int32_t t = 0; t < batch_size && !done; ++t) {
      const float dx = s_xyo[t][0] - px;
      const float dy = s_xyo[t][1] - py;
      const float sigma =
          0.5f * (s_con[t][0] * dx * dx + s_con[t][2] * dy * dy) + s_con[t][1] * dx * dy;
      const float alpha = fminf(0.999f, s_xyo[t][2] * tgs_fast_exp(-sigma));
      if (sigma < 0.f || alpha < 1.f / 255.f) continue;
      const float next_T = T * (1.f - alpha);
      if (next_T <= 1e-4f) {
        done = true;
        break;
      }
      const float vis = alpha * T;
#pragma unroll
      for (int k = 0; k < CDIM; ++k) pix[k] += s_col[t][k] * vis;
      cur_idx = (uint32_t)(batch_start + t);
      T = next_T;
    }
  }
  if (inside) {
    const uint64_t pid = img + (uint64_t)i * G.W + j;
    render_alphas[pid] = 1.f - T;
#pragma unroll
    for (int k = 0; k < CDIM; ++k)
      render_colors[pid * CDIM + k] =
          backgrounds ? pix[k] + T * backgrounds[cam * CDIM + k] : pix[k];
    last_ids[pid] = (int32_t)cur_idx;
  }
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
template <int CDIM, int TILE, class Src, class Sink>
__global__ void __launch_bounds__(TILE* TILE) raster_bwd_kernel(
    RasterGeom G, Src src, Sink sink, const float* __restrict__ backgrounds,
    const int32_t* __restrict__ tile_offsets, const int32_t* __restrict__ flatten_ids,
    const float* __restrict__ render_alphas, const int32_t* __restrict__ last_ids,
    const float* __restrict__ v_render_colors, const float* __restrict__ v_render_alphas) {
  constexpr int BLOCK = TILE * TILE;
  __shared__ int32_t s_id[BLOCK];
  __shared__ float s_xyo[BLOCK][3];
  __shared__ float s_con[BLOCK][3];
  __shared__ float s_col[BLOCK][CDIM];

  const uint32_t cam = blockIdx.x;
  const uint32_t ty = blockIdx.y, tx = blockIdx.z;
  const uint32_t tile_id = ty * G.tile_w + tx;
  const uint32_t tr = threadIdx.x;
  const int lane = tr & 63;
  const uint32_t i = ty * TILE + tr / TILE;
  const uint32_t j = tx * TILE + tr % TILE;
  const bool inside = i < G.H && j < G.W;
  const float px = (float)j + 0.5f, py = (float)i + 0.5f;
  const uint64_t img = (uint64_t)cam * G.H * G.W;
  const uint64_t pid = img + min((uint64_t)i * G.W + j, (uint64_t)G.W * G.H - 1);

  const int32_t* offs = tile_offsets + (uint64_t)cam * G.tile_h * G.tile_w;
  const int32_t range_start = offs[tile_id];
  const int32_t range_end = (cam == G.C - 1 && tile_id == G.tile_w * G.tile_h - 1)
                                ? (int32_t)G.n_isects
                                : offs[tile_id + 1];
  const int32_t n_batches = (range_end - range_start + BLOCK - 1) / BLOCK;

  const float T_final = 1.f - render_alphas[pid];
  float T = T_final;
  float buffer[CDIM];
  float v_rc[CDIM];
#pragma unroll
  for (int k = 0; k < CDIM; ++k) {
    buffer[k] = 0.f;
    v_rc[k] = v_render_colors[pid * CDIM + k];
  }
  const float v_ra = v_render_alphas ? v_render_alphas[pid] : 0.f;
  float bg_dot = 0.f;
  if (backgrounds) {
#pragma unroll
    for (int k = 0; k < CDIM; ++k) bg_dot += backgrounds[cam * CDIM + k] * v_rc[k];
  }
  const int32_t bin_final = inside ? last_ids[pid] : 0;
  const int32_t wave_bin_final = tgs_wave_max_i32(bin_final);
  const int n_vals = sink.n_values();

  for (int32_t b = 0; b < n_batches; ++b) {
    __syncthreads();
    const int32_t batch_end = range_end - 1 - BLOCK * b;
    const int32_t batch_size = min(BLOCK, batch_end + 1 - range_start);
    const int32_t idx = batch_end - (int32_t)tr;
    if (idx >= range_start) {
      const int32_t g = flatten_ids[idx];
      SplatData<CDIM> s;
      src.load(g, s);
      s_id[tr] = g;
      s_xyo[tr][0] = s.x;
      s_xyo[tr][1] = s.y;
      s_xyo[tr][2] = s.op;
      s_con[tr][0] = s.a;
      s_con[tr][1] = s.b;
      s_con[tr][2] = s.c;
#pragma unroll
      for (int k = 0; k < CDIM; ++k) s_col[tr][k] = s.col[k];
    }
    __syncthreads();
    for (int32_t t = max(0, batch_end - wave_bin_final); t < batch_size; ++t) {
      bool valid = inside && (batch_end - t <= bin_final);
      float alpha = 0.f, vis = 0.f, dx = 0.f, dy = 0.f;
      const float op = s_xyo[t][2];
      const float ca = s_con[t][0], cb = s_con[t][1], cc = s_con[t][2];
      if (valid) {
        dx = s_xyo[t][0] - px;
        dy = s_xyo[t][1] - py;
        const float sigma = 0.5f * (ca * dx * dx + cc * dy * dy) + cb * dx * dy;
        vis = tgs_fast_exp(-sigma);
        alpha = fminf(0.999f, op * vis);
        if (sigma < 0.f || alpha < 1.f / 255.f) valid = false;
      }
      if (!tgs_ballot(valid)) continue;

      // vals: v_xy(2), v_conic(3), v_rgb(CDIM), v_opacity, |v_xy|(2)
      float vals[8 + CDIM];
#pragma unroll
      for (int k = 0; k < 8 + CDIM; ++k) vals[k] = 0.f;
      if (valid) {
        const float ra = 1.f / (1.f - alpha);
        T *= ra;
        const float fac = alpha * T;
        float v_alpha = 0.f;
#pragma unroll
        for (int k = 0; k < CDIM; ++k) {
          vals[5 + k] = fac * v_rc[k];
          v_alpha += (s_col[t][k] * T - buffer[k] * ra) * v_rc[k];
        }
        v_alpha += T_final * ra * v_ra;
        if (backgrounds) v_alpha += -T_final * ra * bg_dot;
        if (op * vis <= 0.999f) {
          const float v_sigma = -op * vis * v_alpha;
          vals[2] = 0.5f * v_sigma * dx * dx;
          vals[3] = v_sigma * dx * dy;
          vals[4] = 0.5f * v_sigma * dy * dy;
          vals[0] = v_sigma * (ca * dx + cb * dy);
          vals[1] = v_sigma * (cb * dx + cc * dy);
          vals[6 + CDIM] = fabsf(vals[0]);
          vals[7 + CDIM] = fabsf(vals[1]);
          vals[5 + CDIM] = vis * v_alpha;
        }
#pragma unroll
        for (int k = 0; k < CDIM; ++k) buffer[k] += s_col[t][k] * fac;
      }
      float mine = 0.f;
#pragma unroll
      for (int k = 0; k < 8 + CDIM; ++k) {
        if (k < n_vals) {
          const float s = tgs_wave_sum(vals[k]);
          if (lane == k) mine = s;
        }
      }
      if (lane < n_vals) tgs_atomic_add(sink.ptr(s_id[t], lane), mine);
    }
  }
}
