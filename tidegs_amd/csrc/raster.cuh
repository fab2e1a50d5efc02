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
// MI355X layout.  One workgroup = one TILE x TILE tile; for TILE = 16 that is
// four wavefronts, wave w owning pixel rows [4w, 4w+4).  Each batch of the
// tile's Gaussians is staged through LDS (one per thread) together with:
//   * the log2-domain exponent coefficients, so that
//       power = log2(opacity) - sigma * log2(e)
//     costs five FMAs per pixel and alpha = exp2(power) (v_exp_f32);
//   * the bounding box of the Gaussian's alpha >= 1/255 ellipse
//     (0.5 d^T Q d <= ln(255 opacity)), which is exact: pixels outside it
//     are skipped by the reference too.
// Every wavefront then compacts the batch to the Gaussians whose box meets its
// own 16x4 pixel strip and loops only over those.
// In the backward each wavefront reduces a Gaussian's nine gradient values
// with a reduce-scatter (v_permlane32_swap / v_permlane16_swap / DPP) that
// leaves each value's total in one quad, then one atomic instruction adds all
// nine (lane 4q handles value of quad q).  The pixel-side products are
// accumulated as moments (sum v_sigma dx, dx^2, ...) and turned into mean2d /
// conic / opacity gradients once per Gaussian after the reduction.
//
// The splat source/gradient sink are policies so the same kernels serve
// gsplat's SoA tensors (drop-in op) and the packed 48-byte splat records of the
// fused resident step.
#pragma once

#include "tgs_common.cuh"

#define RS_LOG2E 1.4426950408889634f
#define RS_LOG2_MIN_ALPHA (-7.9943534f)  // log2(1/255), rounded down

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
  __device__ __forceinline__ bool absgrad() const { return v_means2d_abs != nullptr; }
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
  __device__ __forceinline__ bool absgrad() const { return false; }
  __device__ __forceinline__ float* ptr(int32_t g, int k) const { return grads + (int64_t)g * 9 + k; }
};

struct RasterGeom {
  uint32_t C;
  uint32_t W, H;
  uint32_t tile_w, tile_h;
  uint32_t n_isects;
};

// ---------------------------------------------------------------------------
// Staged Gaussian: exponent coefficients and the alpha >= 1/255 box.
// ---------------------------------------------------------------------------
struct StagedGeo {
  float4 g0;   // x, y, A = -0.5 log2e a, B = -log2e b
  float4 g1;   // C = -0.5 log2e c, L = log2(opacity), 0, 0
  float4 box;  // x_lo, x_hi, y_lo, y_hi of the alpha >= 1/255 ellipse
};

template <int CDIM>
__device__ __forceinline__ StagedGeo stage_geo(const SplatData<CDIM>& s) {
  StagedGeo o;
  o.g0 = make_float4(s.x, s.y, -0.5f * RS_LOG2E * s.a, -RS_LOG2E * s.b);
  const float L = __builtin_amdgcn_logf(s.op);  // log2; -inf for 0, NaN for < 0
  o.g1 = make_float4(-0.5f * RS_LOG2E * s.c, s.op > 0.f ? L : -INFINITY, 0.f, 0.f);
  // alpha >= 1/255 needs sigma <= t = ln(255 op).  On {0.5 d^T Q d <= t} the
  // extents are |dx| <= sqrt(2 t c / det), |dy| <= sqrt(2 t a / det).
  const float t = logf(255.f * s.op);
  const float det = s.a * s.c - s.b * s.b;
  if (!(s.op > 0.f) || t <= 0.f) {
    o.box = make_float4(INFINITY, -INFINITY, INFINITY, -INFINITY);  // never visible
  } else if (!(det > 0.f) || !(s.a > 0.f) || !(s.c > 0.f)) {
    o.box = make_float4(-INFINITY, INFINITY, -INFINITY, INFINITY);  // no bound: never cull
  } else {
    const float tt = t * 1.001f + 1e-3f;  // conservative margin over rounding
    const float ex = sqrtf(2.f * tt * s.c / det) * 1.001f + 1e-3f;
    const float ey = sqrtf(2.f * tt * s.a / det) * 1.001f + 1e-3f;
    o.box = make_float4(s.x - ex, s.x + ex, s.y - ey, s.y + ey);
  }
  return o;
}

// power = log2(op) - sigma log2(e) at offset (dx, dy) = mean - pixel.
__device__ __forceinline__ float raster_power(const float4& g0, const float4& g1, float dx,
                                              float dy) {
  const float t2 = fmaf(g0.z, dx, g0.w * dy);
  const float s = fmaf(g1.x * dy, dy, g1.y);
  return fmaf(t2, dx, s);
}

// Compact batch entries [j_lo, batch_size) whose box meets the wave's pixel
// strip into s_list (ascending j).  Returns the count (wave-uniform).
template <int BLOCK>
__device__ __forceinline__ int build_wave_list(const float4* s_box, uint8_t* s_list, int j_lo,
                                               int batch_size, float x0, float x1, float y0,
                                               float y1) {
  const int lane = threadIdx.x & 63;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int count = 0;
#pragma unroll
  for (int k = 0; k < BLOCK; k += 64) {
    const int j = k + lane;
    bool hit = false;
    if (j >= j_lo && j < batch_size) {
      const float4 b = s_box[j];
      hit = !(b.y < x0 || b.x > x1 || b.w < y0 || b.z > y1);
    }
    const uint64_t m = tgs_ballot(hit);
    if (hit) s_list[count + __popcll(m & lt)] = (uint8_t)j;
    count += __popcll(m);
  }
  __builtin_amdgcn_wave_barrier();
  return count;
}

// ---------------------------------------------------------------------------
// Reduce-scatter of up to 10 wave values (gfx950).  Afterwards every lane of
// quad q (lanes 4q..4q+3) holds the wave total of value rs_value_of_quad(q);
// values >= the caller's count are zero padding.
//   step A  v_permlane32_swap: value 2j in lanes 0-31, 2j+1 in lanes 32-63
//   step B  v_permlane16_swap: each 16-lane row holds one value
//   step C  select + DPP row_ror:8: each 8-lane half row holds one value
//   step D  select + DPP row_half_mirror: each quad holds one value
//   step E  DPP quad_perm adds
// ---------------------------------------------------------------------------
__device__ __forceinline__ int rs_value_of_quad(int q) {
  const int rmap = (0x3120 >> (4 * (q >> 2))) & 0xF;  // [0,2,1,3][q>>2]
  return 8 * (q & 1) + 4 * ((q >> 1) & 1) + rmap;
}

__device__ __forceinline__ void rs_swap32(float a, float b, float& x, float& y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                  false);
  x = __uint_as_float(r[0]);
  y = __uint_as_float(r[1]);
}

__device__ __forceinline__ void rs_swap16(float a, float b, float& x, float& y) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                  false);
  x = __uint_as_float(r[0]);
  y = __uint_as_float(r[1]);
}

__device__ __forceinline__ float rs_reduce10(const float v[10]) {
  const int lane = threadIdx.x & 63;
  float R[5];
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    float x, y;
    rs_swap32(v[2 * j], v[2 * j + 1], x, y);
    R[j] = x + y;
  }
  float S[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    float x, y;
    rs_swap16(R[2 * j], (2 * j + 1 < 5) ? R[2 * j + 1] : 0.f, x, y);
    S[j] = x + y;
  }
  const int l16 = lane & 15;
  auto split8 = [&](float x, float y) {
    const float keep = l16 < 8 ? x : y;
    const float send = l16 < 8 ? y : x;
    return keep + tgs_dpp<0x128>(send);  // row_ror:8
  };
  const float U0 = split8(S[0], S[1]);
  const float U1 = split8(S[2], 0.f);
  const int l8 = lane & 7;
  const float keep = l8 < 4 ? U0 : U1;
  const float send = l8 < 4 ? U1 : U0;
  float V = keep + tgs_dpp<0x141>(send);  // row_half_mirror
  V += tgs_dpp<0xB1>(V);                  // quad_perm [1,0,3,2]
  V += tgs_dpp<0x4E>(V);                  // quad_perm [2,3,0,1]
  return V;
}

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
  constexpr int WAVES = BLOCK / 64;
  constexpr int ROWS = 64 / TILE;  // pixel rows per wavefront
  __shared__ float4 s_g0[BLOCK];
  __shared__ float4 s_g1[BLOCK];
  __shared__ float4 s_box[BLOCK];
  __shared__ float s_col[BLOCK][CDIM];
  __shared__ uint8_t s_list[WAVES][BLOCK];

  const uint32_t cam = blockIdx.x;
  const uint32_t ty = blockIdx.y, tx = blockIdx.z;
  const uint32_t tile_id = ty * G.tile_w + tx;
  const uint32_t tr = threadIdx.x;
  const int wave = tr >> 6;
  const uint32_t i = ty * TILE + tr / TILE;
  const uint32_t j = tx * TILE + tr % TILE;
  const uint64_t img = (uint64_t)cam * G.H * G.W;
  const bool inside = i < G.H && j < G.W;
  const float px = (float)j + 0.5f, py = (float)i + 0.5f;
  // pixel-centre extent of this wavefront's strip
  const float wx0 = (float)(tx * TILE) + 0.5f, wx1 = wx0 + (float)(TILE - 1);
  const float wy0 = (float)(ty * TILE + wave * ROWS) + 0.5f, wy1 = wy0 + (float)(ROWS - 1);

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
      SplatData<CDIM> s;
      src.load(flatten_ids[idx], s);
      const StagedGeo sg = stage_geo<CDIM>(s);
      s_g0[tr] = sg.g0;
      s_g1[tr] = sg.g1;
      s_box[tr] = sg.box;
#pragma unroll
      for (int k = 0; k < CDIM; ++k) s_col[tr][k] = s.col[k];
    }
    __syncthreads();
    const int32_t batch_size = min(BLOCK, range_end - batch_start);
    int n_list = 0;
    if (tgs_ballot(!done))
      n_list = build_wave_list<BLOCK>(s_box, s_list[wave], 0, batch_size, wx0, wx1, wy0, wy1);
    for (int li = 0; li < n_list; ++li) {
      if (!tgs_ballot(!done)) break;
      const int t = s_list[wave][li];
      if (done) continue;
      const float4 g0 = s_g0[t];
      const float4 g1 = s_g1[t];
      const float dx = g0.x - px, dy = g0.y - py;
      const float power = raster_power(g0, g1, dx, dy);
      // sigma < 0  <=>  power > log2(op);  alpha < 1/255  <=>  power < log2(1/255)
      if (power > g1.y || power < RS_LOG2_MIN_ALPHA) continue;
      const float alpha = fminf(0.999f, __builtin_amdgcn_exp2f(power));
      const float next_T = T * (1.f - alpha);
      if (next_T <= 1e-4f) {
        done = true;
        continue;
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
  constexpr int WAVES = BLOCK / 64;
  constexpr int ROWS = 64 / TILE;
  // value slots: 0,1 mean2d; 2..4 conic; 5.. color; 5+CDIM opacity; then |mean2d|
  constexpr int NV = 6 + CDIM;
  constexpr bool FAST = NV <= 10;  // reduce-scatter path
  __shared__ float4 s_g0[BLOCK];
  __shared__ float4 s_g1[BLOCK];
  __shared__ float4 s_box[BLOCK];
  __shared__ float4 s_abc[BLOCK];  // a, b, c, 1/op
  __shared__ float s_col[BLOCK][CDIM];
  __shared__ int32_t s_id[BLOCK];
  __shared__ uint8_t s_list[WAVES][BLOCK];

  const uint32_t cam = blockIdx.x;
  const uint32_t ty = blockIdx.y, tx = blockIdx.z;
  const uint32_t tile_id = ty * G.tile_w + tx;
  const uint32_t tr = threadIdx.x;
  const int lane = tr & 63;
  const int wave = tr >> 6;
  const uint32_t i = ty * TILE + tr / TILE;
  const uint32_t j = tx * TILE + tr % TILE;
  const bool inside = i < G.H && j < G.W;
  const float px = (float)j + 0.5f, py = (float)i + 0.5f;
  const float wx0 = (float)(tx * TILE) + 0.5f, wx1 = wx0 + (float)(TILE - 1);
  const float wy0 = (float)(ty * TILE + wave * ROWS) + 0.5f, wy1 = wy0 + (float)(ROWS - 1);
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
  // T_final * ra * v_ra - T_final * ra * bg_dot = ra * tf_term
  const float tf_term = T_final * v_ra - T_final * bg_dot;
  const int32_t bin_final = inside ? last_ids[pid] : 0;
  const int32_t wave_bin_final = tgs_wave_max_i32(bin_final);
  const bool absg = sink.absgrad();

  for (int32_t b = 0; b < n_batches; ++b) {
    __syncthreads();
    const int32_t batch_end = range_end - 1 - BLOCK * b;
    const int32_t batch_size = min(BLOCK, batch_end + 1 - range_start);
    const int32_t idx = batch_end - (int32_t)tr;
    if (idx >= range_start) {
      const int32_t g = flatten_ids[idx];
      SplatData<CDIM> s;
      src.load(g, s);
      const StagedGeo sg = stage_geo<CDIM>(s);
      s_g0[tr] = sg.g0;
      s_g1[tr] = sg.g1;
      s_box[tr] = sg.box;
      s_abc[tr] = make_float4(s.a, s.b, s.c, 1.f / s.op);
      s_id[tr] = g;
#pragma unroll
      for (int k = 0; k < CDIM; ++k) s_col[tr][k] = s.col[k];
    }
    __syncthreads();
    // entries with global index > wave_bin_final contribute to no pixel of this wave
    const int j_lo = max(0, batch_end - wave_bin_final);
    const int n_list =
        build_wave_list<BLOCK>(s_box, s_list[wave], j_lo, batch_size, wx0, wx1, wy0, wy1);
    for (int li = 0; li < n_list; ++li) {
      const int t = s_list[wave][li];
      bool valid = inside && (batch_end - t <= bin_final);
      const float4 g0 = s_g0[t];
      const float4 g1 = s_g1[t];
      const float dx = g0.x - px, dy = g0.y - py;
      const float power = raster_power(g0, g1, dx, dy);
      if (power > g1.y || power < RS_LOG2_MIN_ALPHA) valid = false;
      if (!tgs_ballot(valid)) continue;

      // per-pixel values: 0 sum v_sigma dx, 1 sum v_sigma dy, 2 v_sigma dx^2,
      // 3 v_sigma dx dy, 4 v_sigma dy^2, 5.. color, 5+CDIM v_sigma, then |v_xy|
      float vals[NV + 2];
#pragma unroll
      for (int k = 0; k < NV + 2; ++k) vals[k] = 0.f;
      if (valid) {
        const float raw = __builtin_amdgcn_exp2f(power);  // opacity * exp(-sigma)
        const float alpha = fminf(0.999f, raw);
        const float ra = __builtin_amdgcn_rcpf(1.f - alpha);
        T *= ra;
        const float fac = alpha * T;
        float v_alpha = ra * tf_term;
#pragma unroll
        for (int k = 0; k < CDIM; ++k) {
          const float ck = s_col[t][k];
          vals[5 + k] = fac * v_rc[k];
          v_alpha += (ck * T - buffer[k] * ra) * v_rc[k];
          buffer[k] += ck * fac;
        }
        if (raw <= 0.999f) {
          const float v_sigma = -raw * v_alpha;
          const float mx = v_sigma * dx, my = v_sigma * dy;
          vals[0] = mx;
          vals[1] = my;
          vals[2] = mx * dx;
          vals[3] = mx * dy;
          vals[4] = my * dy;
          vals[5 + CDIM] = v_sigma;
          if (absg) {
            const float4 q = s_abc[t];
            vals[NV] = fabsf(v_sigma * (q.x * dx + q.y * dy));
            vals[NV + 1] = fabsf(v_sigma * (q.y * dx + q.z * dy));
          }
        }
      }
      // wave totals -> final gradient values of this Gaussian
      const float4 q = s_abc[t];
      const int32_t gid = s_id[t];
      if (FAST && !absg) {
        float v10[10];
#pragma unroll
        for (int k = 0; k < 10; ++k) v10[k] = k < NV ? vals[k] : 0.f;
        const float tot = rs_reduce10(v10);
        // lane 4q owns value k = rs_value_of_quad(q); the moments are turned into
        // gradients with the Gaussian's constants (mean2d: Q m; conic: halves).
        const int quad = lane >> 2;
        const int k = rs_value_of_quad(quad);
        // neighbour totals needed for mean2d: fetch via readlane of the quads
        // holding values 0 and 1 (quads 0 and 8).
        const float m0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot), 0));
        const float m1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot), 32));
        float out = tot;
        if (k == 0) out = q.x * m0 + q.y * m1;
        else if (k == 1) out = q.y * m0 + q.z * m1;
        else if (k == 2 || k == 4) out = 0.5f * tot;
        else if (k == 5 + CDIM) out = -tot * q.w;
        if ((lane & 3) == 0 && k < NV) tgs_atomic_add(sink.ptr(gid, k), out);
      } else {
        float mine = 0.f;
        float tot[NV + 2];
#pragma unroll
        for (int k = 0; k < NV + 2; ++k) tot[k] = 0.f;
#pragma unroll
        for (int k = 0; k < NV + 2; ++k)
          if (k < NV || absg) tot[k] = tgs_wave_sum(vals[k]);
        const int nv = absg ? NV + 2 : NV;
#pragma unroll
        for (int k = 0; k < NV + 2; ++k) {
          float o = tot[k];
          if (k == 0) o = q.x * tot[0] + q.y * tot[1];
          else if (k == 1) o = q.y * tot[0] + q.z * tot[1];
          else if (k == 2 || k == 4) o = 0.5f * tot[k];
          else if (k == 5 + CDIM) o = -tot[k] * q.w;
          if (lane == k) mine = o;
        }
        if (lane < nv) tgs_atomic_add(sink.ptr(gid, lane), mine);
      }
    }
  }
}
