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
// own 16x4 pixel strip; each lane marks which of those reach its pixel and
// walks only its own marks (lane-compacted iteration, below).
// In the backward each lane leaves its per-(Gaussian, pixel) terms in a
// compact LDS pair buffer and owner lanes sum them per Gaussian as moments
// (sum v_sigma dx, dx^2, ...), turned into mean2d / conic / opacity gradients
// once per Gaussian and wavefront.
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
  float2 g1;   // C = -0.5 log2e c, L = log2(opacity)
  float4 box;  // x_lo, x_hi, y_lo, y_hi of the alpha >= 1/255 ellipse
};

template <int CDIM>
__device__ __forceinline__ StagedGeo stage_geo(const SplatData<CDIM>& s) {
  StagedGeo o;
  o.g0 = make_float4(s.x, s.y, -0.5f * RS_LOG2E * s.a, -RS_LOG2E * s.b);
  const float L = __builtin_amdgcn_logf(s.op);  // log2; -inf for 0, NaN for < 0
  o.g1 = make_float2(-0.5f * RS_LOG2E * s.c, s.op > 0.f ? L : -INFINITY);
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

// Conic (a, b, c) and 1/opacity recovered from the staged coefficients.
__device__ __forceinline__ float4 staged_conic_rop(const float4& g0, const float2& g1) {
  constexpr float k = 1.f / RS_LOG2E;
  return make_float4(-2.f * k * g0.z, -k * g0.w, -2.f * k * g1.x, __builtin_amdgcn_exp2f(-g1.y));
}

// power = log2(op) - sigma log2(e) at offset (dx, dy) = mean - pixel.
__device__ __forceinline__ float raster_power(const float4& g0, const float2& g1, float dx,
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
// Lane-compacted iteration.  A wavefront's list holds every Gaussian whose box
// meets its strip, but a small Gaussian covers only a few of its 64 pixels,
// so looping over the list with one pixel per lane leaves most lanes idle.
// Instead every lane first records, in a bitmask over list positions, which
// Gaussians actually reach its pixel (the cheap alpha test), and then walks
// only its own set bits in list order: the wavefront iterates
// max_lane(|own set|) times instead of |list| times.
// ---------------------------------------------------------------------------
template <int BLOCK>
struct LaneMask {
  static constexpr int WORDS = BLOCK / 32;
  uint32_t w[WORDS];
};

// Bit li of the mask is set iff list entry li passes the pixel test of
// rasterize_to_pixels_{fwd,bwd}.cu (sigma >= 0 and alpha >= 1/255) and, in
// the backward, its batch index is not behind the pixel's last contributor.
template <int BLOCK>
__device__ __forceinline__ void lane_masks(LaneMask<BLOCK>& m, const uint8_t* list, int n_list,
                                           const float4* s_g0, const float2* s_g1, float px,
                                           float py, bool active, int t_min) {
#pragma unroll
  for (int W = 0; W < LaneMask<BLOCK>::WORDS; ++W) {
    uint32_t mw = 0;
    if (W * 32 < n_list) {
      const int lim = min(32, n_list - W * 32);
      for (int bb = 0; bb < lim; ++bb) {
        const int t = list[W * 32 + bb];
        const float4 g0 = s_g0[t];
        const float2 g1 = s_g1[t];
        const float power = raster_power(g0, g1, g0.x - px, g0.y - py);
        const bool ok = t >= t_min && !(power > g1.y || power < RS_LOG2_MIN_ALPHA);
        mw |= (ok ? 1u : 0u) << bb;
      }
    }
    m.w[W] = active ? mw : 0u;
  }
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
#define RF_BATCH 128  // Gaussians staged per batch

template <int CDIM, int TILE, class Src>
__global__ void __launch_bounds__(TILE* TILE) raster_fwd_kernel(
    RasterGeom G, Src src, const float* __restrict__ backgrounds,
    const int32_t* __restrict__ tile_offsets, const int32_t* __restrict__ flatten_ids,
    float* __restrict__ render_colors, float* __restrict__ render_alphas,
    int32_t* __restrict__ last_ids) {
  constexpr int BLOCK = TILE * TILE;
  constexpr int WAVES = BLOCK / 64;
  constexpr int ROWS = 64 / TILE;  // pixel rows per wavefront
  constexpr int BATCH = RF_BATCH < BLOCK ? RF_BATCH : BLOCK;
  __shared__ float4 s_g0[BATCH];
  __shared__ float2 s_g1[BATCH];
  __shared__ float4 s_box[BATCH];
  __shared__ float s_col[BATCH][CDIM];
  __shared__ uint8_t s_list[WAVES][BATCH];

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
  const int32_t n_batches = (range_end - range_start + BATCH - 1) / BATCH;

  float T = 1.f;
  uint32_t cur_idx = 0;
  bool done = !inside;
  float pix[CDIM];
#pragma unroll
  for (int k = 0; k < CDIM; ++k) pix[k] = 0.f;

  for (int32_t b = 0; b < n_batches; ++b) {
    if (__syncthreads_count(done) >= BLOCK) break;
    const int32_t batch_start = range_start + BATCH * b;
    const int32_t idx = batch_start + (int32_t)tr;
    if ((int)tr < BATCH && idx < range_end) {
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
    const int32_t batch_size = min(BATCH, range_end - batch_start);
    int n_list = 0;
    if (tgs_ballot(!done))
      n_list = build_wave_list<BATCH>(s_box, s_list[wave], 0, batch_size, wx0, wx1, wy0, wy1);
    LaneMask<BATCH> m;
    lane_masks<BATCH>(m, s_list[wave], n_list, s_g0, s_g1, px, py, !done, 0);
#pragma unroll
    for (int W = 0; W < LaneMask<BATCH>::WORDS; ++W) {
      if (W * 32 >= n_list) break;
      uint32_t mw = m.w[W];
      while (true) {
        const bool act = mw != 0u && !done;
        if (!tgs_ballot(act)) break;
        if (act) {
          const int bit = __builtin_ctz(mw);
          mw &= mw - 1u;
          const int t = s_list[wave][W * 32 + bit];
          const float4 g0 = s_g0[t];
          const float2 g1 = s_g1[t];
          const float power = raster_power(g0, g1, g0.x - px, g0.y - py);
          const float alpha = fminf(0.999f, __builtin_amdgcn_exp2f(power));
          const float next_T = T * (1.f - alpha);
          if (next_T <= 1e-4f) {
            done = true;
          } else {
            const float vis = alpha * T;
#pragma unroll
            for (int k = 0; k < CDIM; ++k) pix[k] += s_col[t][k] * vis;
            cur_idx = (uint32_t)(batch_start + t);
            T = next_T;
          }
        }
      }
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
// Backward.  Per batch and wavefront:
//   1. test     as in the forward: each lane's bitmask over the list (alpha
//               test and last-contributor bound); the wavefront's ballot of
//               each entry is that Gaussian's pixel mask, and a running sum of
//               their popcounts gives each entry's slot range in a compact
//               (Gaussian, pixel) pair buffer;
//   2. walk     each lane walks its own entries back to front (T, colour
//               buffer) and leaves (alpha T, v_sigma) in the entry's slot
//               range at its rank among the entry's pixels;
//   3. owners   lanes 4e..4e+3 own entry e of a group of 16, each summing the
//               moments (v_sigma dx, dy, dx^2, dx dy, dy^2, v_sigma, colour
//               terms, |v_mean2d|) over the pairs of its 16 pixel lanes; a quad
//               DPP sum gives the entry's totals, turned into mean2d / conic /
//               opacity gradients with its constants;
//   4. flush    (entry, value) pairs in value-fastest order, so each atomic
//               instruction covers a few Gaussians' contiguous records.
// No lane ever adds to a shared location: no LDS atomics and no per-entry
// wave reduction.  When a batch has more pairs than the buffer holds, the list
// is processed in consecutive segments (each Gaussian's pairs fit: <= 64).
// ---------------------------------------------------------------------------
#define RB_PAIRS 384  // pair-buffer slots per wavefront
#define RB_BATCH 64  // Gaussians staged per batch

template <int CDIM, int TILE, class Src, class Sink>
__global__ void __launch_bounds__(TILE* TILE) raster_bwd_kernel(
    RasterGeom G, Src src, Sink sink, const float* __restrict__ backgrounds,
    const int32_t* __restrict__ tile_offsets, const int32_t* __restrict__ flatten_ids,
    const float* __restrict__ render_alphas, const int32_t* __restrict__ last_ids,
    const float* __restrict__ v_render_colors, const float* __restrict__ v_render_alphas) {
  constexpr int BLOCK = TILE * TILE;
  constexpr int WAVES = BLOCK / 64;
  constexpr int ROWS = 64 / TILE;
  constexpr int BATCH = RB_BATCH < BLOCK ? RB_BATCH : BLOCK;
  constexpr int WORDS = BATCH / 32;
  // value slots: 0,1 mean2d; 2..4 conic; 5.. color; 5+CDIM opacity; then |mean2d|
  constexpr int NV = 6 + CDIM;
  constexpr int NA = NV + 2;
  __shared__ float4 s_g0[BATCH];
  __shared__ float2 s_g1[BATCH];
  __shared__ float s_col[BATCH][CDIM];
  __shared__ float s_vrc[BLOCK][CDIM];  // dL/dcolor of each pixel
  __shared__ int32_t s_id[BATCH];
  __shared__ uint8_t s_list[WAVES][BATCH];
  // boxes are dead once the lists are built (barrier), then the pair buffer
  // (alpha T, v_sigma) takes their place
  __shared__ union {
    float4 box[BATCH];
    float2 pair[WAVES][RB_PAIRS];
  } s_u;
  __shared__ uint64_t s_em[WAVES][BATCH];         // pixel mask of each list entry
  __shared__ uint16_t s_po[WAVES][BATCH + 1];     // first pair slot of each list entry
  __shared__ float s_stage[WAVES][16 * NA];

  const uint32_t cam = blockIdx.x;
  const uint32_t ty = blockIdx.y, tx = blockIdx.z;
  const uint32_t tile_id = ty * G.tile_w + tx;
  const uint32_t tr = threadIdx.x;
  const int lane = tr & 63;
  const int wave = tr >> 6;
  const uint64_t lt_mask = (1ull << lane) - 1ull;
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
  const int32_t n_batches = (range_end - range_start + BATCH - 1) / BATCH;

  const float T_final = 1.f - render_alphas[pid];
  float T = T_final;
  float buffer[CDIM];
  float v_rc[CDIM];
#pragma unroll
  for (int k = 0; k < CDIM; ++k) {
    buffer[k] = 0.f;
    v_rc[k] = v_render_colors[pid * CDIM + k];
    s_vrc[tr][k] = v_rc[k];
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
  const int nval = absg ? NA : NV;
  // owner role within a group of 16 entries: entry oe, pixel lanes [16 oq, 16 oq + 16)
  const int oe = lane >> 2, oq = lane & 3;

  for (int32_t b = 0; b < n_batches; ++b) {
    __syncthreads();
    const int32_t batch_end = range_end - 1 - BATCH * b;
    const int32_t batch_size = min(BATCH, batch_end + 1 - range_start);
    const int32_t idx = batch_end - (int32_t)tr;
    if ((int)tr < BATCH && idx >= range_start) {
      const int32_t g = flatten_ids[idx];
      SplatData<CDIM> s;
      src.load(g, s);
      const StagedGeo sg = stage_geo<CDIM>(s);
      s_g0[tr] = sg.g0;
      s_g1[tr] = sg.g1;
      s_u.box[tr] = sg.box;
      s_id[tr] = g;
#pragma unroll
      for (int k = 0; k < CDIM; ++k) s_col[tr][k] = s.col[k];
    }
    __syncthreads();
    // entries with global index > wave_bin_final contribute to no pixel of this wave
    const int j_lo = max(0, batch_end - wave_bin_final);
    const int n_list =
        build_wave_list<BATCH>(s_u.box, s_list[wave], j_lo, batch_size, wx0, wx1, wy0, wy1);
    // 1. test; batch entry t is global index batch_end - t: at or before bin_final
    const int t_min = batch_end - bin_final;
    uint32_t m[WORDS];
    uint32_t n_pairs = 0;  // wave-uniform
#pragma unroll
    for (int W = 0; W < WORDS; ++W) {
      uint32_t mw = 0;
      for (int bb = 0; bb < 32 && W * 32 + bb < n_list; ++bb) {
        const int li = W * 32 + bb;
        const int t = s_list[wave][li];
        const float4 g0 = s_g0[t];
        const float2 g1 = s_g1[t];
        const float power = raster_power(g0, g1, g0.x - px, g0.y - py);
        const bool ok =
            inside && t >= t_min && !(power > g1.y || power < RS_LOG2_MIN_ALPHA);
        mw |= (ok ? 1u : 0u) << bb;
        const uint64_t em = tgs_ballot(ok);
        if (lane == 0) {
          s_em[wave][li] = em;
          s_po[wave][li] = (uint16_t)n_pairs;
        }
        n_pairs += (uint32_t)__popcll(em);
      }
      m[W] = mw;
    }
    if (lane == 0) s_po[wave][n_list] = (uint16_t)n_pairs;
    __syncthreads();  // every wavefront is past its list build: boxes are dead
    int a = 0;        // first list entry of the current segment
    while (a < n_list) {
      const uint32_t base = s_po[wave][a];
      // largest end with at most RB_PAIRS pairs (an entry has <= 64)
      int e_end = n_list;
      if (n_pairs - base > RB_PAIRS) {
        int lo = a + 1, hi = n_list;  // s_po[lo] - base <= RB_PAIRS < s_po[hi] - base
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if ((uint32_t)s_po[wave][mid] - base <= RB_PAIRS) lo = mid;
          else hi = mid;
        }
        e_end = lo;
      }
      // 2. per-pixel walk over entries [a, e_end), back to front
#pragma unroll
      for (int W = 0; W < WORDS; ++W) {
        if (W * 32 >= e_end || W * 32 + 32 <= a) continue;
        const int lo_b = max(a - W * 32, 0), hi_b = min(e_end - W * 32, 32);
        const uint32_t range = (hi_b >= 32 ? 0xffffffffu : ((1u << hi_b) - 1u)) &
                               ~((1u << lo_b) - 1u);
        uint32_t mw = m[W] & range;
        while (tgs_ballot(mw != 0u)) {
          if (mw != 0u) {
            const int li = W * 32 + __builtin_ctz(mw);
            mw &= mw - 1u;
            const int t = s_list[wave][li];
            const float4 g0 = s_g0[t];
            const float2 g1 = s_g1[t];
            const float power = raster_power(g0, g1, g0.x - px, g0.y - py);
            const float raw = __builtin_amdgcn_exp2f(power);  // opacity * exp(-sigma)
            const float alpha = fminf(0.999f, raw);
            const float ra = __builtin_amdgcn_rcpf(1.f - alpha);
            T *= ra;
            const float fac = alpha * T;
            float v_alpha = ra * tf_term;
#pragma unroll
            for (int k = 0; k < CDIM; ++k) {
              const float ck = s_col[t][k];
              v_alpha += (ck * T - buffer[k] * ra) * v_rc[k];
              buffer[k] += ck * fac;
            }
            // reference: the sigma terms only where alpha was not clamped
            const float v_sigma = raw <= 0.999f ? -raw * v_alpha : 0.f;
            const uint32_t slot = (uint32_t)s_po[wave][li] - base +
                                  (uint32_t)__popcll(s_em[wave][li] & lt_mask);
            s_u.pair[wave][slot] = make_float2(fac, v_sigma);
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // 3. owners, groups of 16 entries
      for (int e0 = a; e0 < e_end; e0 += 16) {
        const int gn = min(16, e_end - e0);
        float acc[NA];
#pragma unroll
        for (int k = 0; k < NA; ++k) acc[k] = 0.f;
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (oe < gn) {
          const int li = e0 + oe;
          const int t = s_list[wave][li];
          const float4 g0 = s_g0[t];
          q = staged_conic_rop(g0, s_g1[t]);
          const uint64_t em = s_em[wave][li];
          const uint64_t below = oq == 0 ? 0ull : (em & (~0ull >> (64 - 16 * oq)));
          uint32_t slot = (uint32_t)s_po[wave][li] - base + (uint32_t)__popcll(below);
          uint32_t rb = (uint32_t)(em >> (16 * oq)) & 0xffffu;
          while (rb != 0u) {
            const int pl = 16 * oq + __builtin_ctz(rb);
            rb &= rb - 1u;
            const float2 pr = s_u.pair[wave][slot++];
            const int pix = wave * 64 + pl;
            const float dx = g0.x - ((float)(tx * TILE + pix % TILE) + 0.5f);
            const float dy = g0.y - ((float)(ty * TILE + pix / TILE) + 0.5f);
            const float vs = pr.y;
            const float mx = vs * dx, my = vs * dy;
            acc[0] += mx;
            acc[1] += my;
            acc[2] += mx * dx;
            acc[3] += mx * dy;
            acc[4] += my * dy;
#pragma unroll
            for (int k = 0; k < CDIM; ++k) acc[5 + k] += pr.x * s_vrc[pix][k];
            acc[5 + CDIM] += vs;
            if (absg) {
              acc[NV] += fabsf(q.x * mx + q.y * my);
              acc[NV + 1] += fabsf(q.y * mx + q.z * my);
            }
          }
        }
#pragma unroll
        for (int k = 0; k < NA; ++k) {
          if (k < NV || absg) {
            acc[k] += tgs_dpp<0xB1>(acc[k]);  // quad_perm [1,0,3,2]
            acc[k] += tgs_dpp<0x4E>(acc[k]);  // quad_perm [2,3,0,1]
          }
        }
        if (oq == 0 && oe < gn) {
          float* st = s_stage[wave] + oe * nval;
          st[0] = q.x * acc[0] + q.y * acc[1];
          st[1] = q.y * acc[0] + q.z * acc[1];
          st[2] = 0.5f * acc[2];
          st[3] = acc[3];
          st[4] = 0.5f * acc[4];
#pragma unroll
          for (int k = 0; k < CDIM; ++k) st[5 + k] = acc[5 + k];
          st[5 + CDIM] = -acc[5 + CDIM] * q.w;
          if (absg) {
            st[NV] = acc[NV];
            st[NV + 1] = acc[NV + 1];
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // 4. flush
        const int total = gn * nval;
        for (int L = lane; L < total; L += 64) {
          const int e = absg ? L / NA : L / NV;
          const int k = L - e * nval;
          const float v = s_stage[wave][L];
          if (v != 0.f) tgs_atomic_add(sink.ptr(s_id[s_list[wave][e0 + e]], k), v);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      a = e_end;
    }
  }
}
