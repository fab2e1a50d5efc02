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
//     (0.5 d^T Q d <= ln(255 opacity)): pixels outside it are skipped by the
//     reference too.
// Every wavefront compacts the batch to the Gaussians whose box meets its own
// pixel strip, and computes for each of them, one lane per (Gaussian, pixel
// row), the row's interval of pixels that can reach alpha >= 1/255: a
// conservative superset of the pixels that pass the reference's test (the
// quadratic's roots with a bound on the rounding of the per-pixel
// evaluation).  The intervals, as a 64-bit pixel mask per Gaussian, give each
// lane the list positions its pixel may use; the lane walks only those, and
// the exact per-pixel test decides inside the walk (lane-compacted
// iteration).
// In the backward each lane leaves its per-(Gaussian, pixel) terms in a
// compact LDS pair buffer and owner lanes sum them per Gaussian as moments
// (sum v_sigma dx, dx^2, ...), turned into mean2d / conic / opacity gradients
// once per Gaussian and wavefront.
//
// The splat source/gradient sink are policies so the same kernels serve
// gsplat's SoA tensors (drop-in op) and the packed 48-byte splat records of the
// fused resident step.
#pragma once

#include <type_traits>

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
  static constexpr bool CLAMP_MARKS = false;
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
  static constexpr bool MAY_ABS = true;  // |mean2d| gradients when v_means2d_abs is set
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
// A colour channel stored as -0.0 was clamped by the projection
// (clamp_min(SH + 0.5, 0), whose gradient is zero there): the backward
// writes a zero colour gradient for it.
struct PackedSplats {
  static constexpr bool CLAMP_MARKS = true;
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
  static constexpr bool MAY_ABS = false;
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
  float4 cov;  // row-coverage constants (cover_row): 2n, 1/n, k0, mode
};

#define RS_COVER_QUAD 0.f  // bounded: the row intervals come from the quadratic
#define RS_COVER_ALL 1.f   // no bound (degenerate conic, non-finite values): every pixel
#define RS_COVER_NONE 2.f  // never visible (log2 opacity below the alpha threshold)

template <int CDIM>
__device__ __forceinline__ StagedGeo stage_geo(const SplatData<CDIM>& s) {
  StagedGeo o;
  o.g0 = make_float4(s.x, s.y, -0.5f * RS_LOG2E * s.a, -RS_LOG2E * s.b);
  const float L = __builtin_amdgcn_logf(s.op);  // log2; -inf for 0, NaN for < 0
  o.g1 = make_float2(-0.5f * RS_LOG2E * s.c, s.op > 0.f ? L : -INFINITY);
  // alpha >= 1/255 needs sigma <= t = ln(255 op) = (L - log2(1/255)) ln 2,
  // from the same L as the per-pixel test: t < 0 exactly when no pixel can
  // pass it.  On {0.5 d^T Q d <= t} the extents are |dx| <= sqrt(2 t c / det),
  // |dy| <= sqrt(2 t a / det); the hardware reciprocal and square root
  // (1 ulp) sit far inside the 0.1 % + 1e-3 margins.
  const float t = (L - RS_LOG2_MIN_ALPHA) * 0.6931471805599453f;
  const float det = s.a * s.c - s.b * s.b;
  o.cov = make_float4(0.f, 0.f, 0.f, RS_COVER_ALL);
  if (!(s.op > 0.f) || !(t >= 0.f)) {
    o.box = make_float4(INFINITY, -INFINITY, INFINITY, -INFINITY);  // never visible
    o.cov.w = RS_COVER_NONE;
  } else if (!(det > 0.f) || !(s.a > 0.f) || !(s.c > 0.f)) {
    o.box = make_float4(-INFINITY, INFINITY, -INFINITY, INFINITY);  // no bound: never cull
  } else {
    const float tt = t * 1.001f + 1e-3f;  // conservative margin over rounding
    const float rdet = __builtin_amdgcn_rcpf(det);
    const float ex = __builtin_amdgcn_sqrtf(2.f * tt * s.c * rdet) * 1.001f + 1e-3f;
    const float ey = __builtin_amdgcn_sqrtf(2.f * tt * s.a * rdet) * 1.001f + 1e-3f;
    o.box = make_float4(s.x - ex, s.x + ex, s.y - ey, s.y + ey);
    // cover_row: n = -2A > 0; delta bounds the rounding of the per-pixel
    // evaluation (three FMAs: < 3 ulp of the largest term, itself <= M on
    // the box) with a wide margin, 2^-17 M
    const float A = o.g0.z, B = o.g0.w, C = o.g1.x;
    const float M = fabsf(A) * ex * ex + fabsf(B) * ex * ey + fabsf(C) * ey * ey + fabsf(L) + 8.f;
    const float delta = M * 0x1p-17f + 1e-6f;
    const float n = -2.f * A;
    if (__builtin_isfinite(o.box.x) && __builtin_isfinite(o.box.y) &&
        __builtin_isfinite(o.box.z) && __builtin_isfinite(o.box.w) && __builtin_isfinite(L) &&
        __builtin_isfinite(M) && n > 0.f)
      o.cov = make_float4(2.f * n, __builtin_amdgcn_rcpf(n), (L - RS_LOG2_MIN_ALPHA) + delta,
                          RS_COVER_QUAD);
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
// strip into s_list (ascending j, stored as j * SCALE).  Returns the count
// (wave-uniform); `hits` receives the membership bits of entries 0..63 (bit j
// set iff j is listed).
template <int BLOCK, typename LT = uint8_t, int SCALE = 1>
__device__ __forceinline__ int build_wave_list(const float4* s_box, LT* s_list, int j_lo,
                                               int batch_size, float x0, float x1, float y0,
                                               float y1, uint64_t& hits) {
  int count = 0;
#pragma unroll
  for (int k = 0; k < BLOCK; k += 64) {
    const int j = k + (int)(threadIdx.x & 63);
    bool hit = false;
    if (j >= j_lo && j < batch_size) {
      const float4 b = s_box[j];
      hit = !(b.y < x0 || b.x > x1 || b.w < y0 || b.z > y1);
    }
    const uint64_t m = tgs_ballot(hit);
    if (k == 0) hits = m;
    // rank among the hits below this lane: mbcnt counts the mask bits of lower lanes
    const int rank = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    if (hit) s_list[count + rank] = (LT)(j * SCALE);
    count += __popcll(m);
  }
  __builtin_amdgcn_wave_barrier();
  return count;
}

// ---------------------------------------------------------------------------
// Coverage of one pixel row by a staged Gaussian: the TILE-bit mask of pixel
// centres px = px0 + j (j < TILE) on row py that can pass the alpha test.
//
// With dx = gx - px and dy = gy - py, power = A dx^2 + B dx dy + C dy^2 + L
// (A < 0 for a bounded Gaussian).  On the row it is a quadratic in dx, and
// power >= thr - delta holds between its roots:
//   A dx^2 + h dx + k >= 0,  h = B dy,  k = C dy^2 + k0,  k0 = L - thr + delta,
//   dx in [(h - sqrt(D)) / n, (h + sqrt(D)) / n],  n = -2A,  D = h^2 + 2 n k.
// delta (stage_geo) covers the rounding of the per-pixel evaluation, and the
// pixel interval is widened by far more than the rounding of the roots (the
// hardware sqrt and reciprocal are within 1 ulp; the margin is 2^-10 of the
// interval's extent plus 1e-3 px), so the mask contains every pixel whose
// evaluated power passes.  A row with D < 0 misses the (threshold - delta)
// ellipse, which contains the alpha >= 1/255 one, so no box test is needed.
// The interval's ends are clamped into the tile before rounding (first pixel
// in [0, TILE], last in [-1, TILE - 1]), so an empty or off-tile interval
// gives an empty mask without a separate test.  Degenerate or non-finite
// Gaussians (mode RS_COVER_ALL) cover every pixel (the exact test decides);
// invisible ones (RS_COVER_NONE) are never listed.
// ---------------------------------------------------------------------------
template <int TILE>
__device__ __forceinline__ uint32_t cover_row(const float4& g0, const float2& g1,
                                              const float4& cov, float px0, float py) {
  constexpr uint32_t FULL = (1u << TILE) - 1u;
  const float dy = g0.y - py;
  const float h = g0.w * dy;
  const float k = fmaf(g1.x * dy, dy, cov.z);
  const float D = fmaf(h, h, cov.x * k);
  const float half = __builtin_amdgcn_sqrtf(fmaxf(D, 0.f)) * cov.y;
  const float cen = h * cov.y;
  const float base = g0.x - px0;
  const float m = 1e-3f + 0x1p-10f * (fabsf(cen) + half) + 0x1p-20f * fabsf(base);
  // px = gx - dx  =>  j = px - px0 in [base - cen - half, base - cen + half]
  const float lo = __builtin_amdgcn_fmed3f(base - cen - half - m, 0.f, (float)TILE);
  const float hi = __builtin_amdgcn_fmed3f(base - cen + half + m, -1.f, (float)(TILE - 1));
  const int jlo = (int)ceilf(lo);   // 0 .. TILE
  const int jhi = (int)floorf(hi);  // -1 .. TILE - 1
  const uint32_t quad = (FULL >> (TILE - 1 - jhi)) & (FULL << jlo);
  return cov.w == RS_COVER_QUAD ? (D >= 0.f ? quad : 0u) : FULL;
}

// A staged Gaussian as one LDS record, so that a lane reading the entry it
// walks needs one address computation (the record's base) and immediate
// offsets for the rest.  Size 48 bytes at 3 channels.
template <int CDIM>
struct alignas(16) StagedRec {
  float4 g0;  // x, y, A, B
  float4 g1;  // C, L, -, -
  float col[CDIM];
};

// Exponent coefficients of list entry t, from separate arrays or from records.
struct GeoArrays {
  const float4* g0;
  const float2* g1;
  __device__ __forceinline__ float4 G0(int t) const { return g0[t]; }
  __device__ __forceinline__ float2 G1(int t) const { return g1[t]; }
};
template <int CDIM>
struct GeoRecs {
  const StagedRec<CDIM>* r;
  __device__ __forceinline__ float4 G0(int t) const { return r[t].g0; }
  __device__ __forceinline__ float2 G1(int t) const { return make_float2(r[t].g1.x, r[t].g1.y); }
};

// Pixel-row masks of the first n_list entries of a wavefront's list: lane
// (e, r) computes entry li0 + e, row r.  The ROWS masks of an entry form its
// 64-bit pixel mask (bit r * TILE + j = pixel (r, j) of the strip = lane
// r * TILE + j), stored as two 32-bit halves: s_emh[0][li] holds lanes 0..31,
// s_emh[1][li] lanes 32..63, so that a lane reads only its own half.
template <int TILE, int BATCH, class Geo, typename LT = uint8_t, int SCALE = 1>
__device__ __forceinline__ void strip_masks(const LT* s_list, int n_list, const Geo geo,
                                            const float4* s_cov, uint32_t (*s_emh)[BATCH],
                                            float px0, float py0, uint64_t alive) {
  using RM = typename std::conditional<TILE == 16, uint16_t, uint8_t>::type;
  constexpr int ROWS = 64 / TILE;
  constexpr int PER = 64 / ROWS;  // entries per pass
  const int lane = threadIdx.x & 63;
  const int e = lane / ROWS, r = lane % ROWS;
  const uint32_t alive_row = (uint32_t)(alive >> (r * TILE)) & ((1u << TILE) - 1u);
  for (int li0 = 0; li0 < n_list; li0 += PER) {
    const int li = li0 + e;
    if (li < n_list) {
      const int t = (int)s_list[li] / SCALE;
      const uint32_t m =
          cover_row<TILE>(geo.G0(t), geo.G1(t), s_cov[t], px0, py0 + (float)r);
      reinterpret_cast<RM*>(&s_emh[(r * TILE) >> 5][li])[((r * TILE) & 31) / TILE] =
          (RM)(m & alive_row);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// This lane's bits of the list masks: bit li of word li / 32 is this lane's
// bit of entry li's mask, for li in [li_min, n_list).  `half` is the lane's
// half row s_emh[lane / 32] (16-byte aligned): one LDS read serves four
// entries.  UNROLL picks a fully unrolled read sequence (faster where the
// kernel has registers to spare) over a compact loop per word.
template <int WORDS, bool UNROLL>
__device__ __forceinline__ void lane_bits(const uint32_t* half, int n_list, int li_min,
                                          uint32_t (&mw)[WORDS]) {
  const uint32_t sh = threadIdx.x & 31;
  const uint4* q4 = reinterpret_cast<const uint4*>(half);
  if (UNROLL) {
#pragma unroll
    for (int W = 0; W < WORDS; ++W) mw[W] = 0u;
#pragma unroll
    for (int q = 0; q < WORDS * 8; ++q) {
      if (4 * q >= n_list) break;
      const uint4 x = q4[q];
      const uint32_t b = ((x.x >> sh) & 1u) | (((x.y >> sh) & 1u) << 1) |
                         (((x.z >> sh) & 1u) << 2) | (((x.w >> sh) & 1u) << 3);
      mw[q >> 3] |= b << (4 * (q & 7));
    }
  } else {
#pragma unroll
    for (int W = 0; W < WORDS; ++W) {
      uint32_t w = 0u;
      const int qn = min(8, (n_list - 32 * W + 3) >> 2);  // wave-uniform
#pragma unroll 1
      for (int q = 0; q < qn; ++q) {
        const uint4 x = q4[8 * W + q];
        const uint32_t b = ((x.x >> sh) & 1u) | (((x.y >> sh) & 1u) << 1) |
                           (((x.z >> sh) & 1u) << 2) | (((x.w >> sh) & 1u) << 3);
        w |= b << (4 * q);
      }
      mw[W] = w;
    }
  }
  // keep positions [li_min, n_list): the words past n_list hold stale masks
#pragma unroll
  for (int W = 0; W < WORDS; ++W) {
    const int lo = min(max(li_min - 32 * W, 0), 32), hi = min(max(n_list - 32 * W, 0), 32);
    const uint32_t below_hi = hi >= 32 ? 0xffffffffu : ((1u << hi) - 1u);
    const uint32_t below_lo = lo >= 32 ? 0xffffffffu : ((1u << lo) - 1u);
    mw[W] &= below_hi & ~below_lo;
  }
}

// Two 16 x 16 bit transposes at once within each 16-lane row of the
// wavefront, one per 16-bit half of a word: lane e of a row holds
// x = M[e] | N[e] << 16 (bit c of M[e] = M[e][c]); afterwards lane c holds
// bit e = M[e][c] and bit 16 + e = N[e][c].  Four exchange stages j = 8, 4,
// 2, 1: a lane whose index has bit j clear keeps its bits b with b & j == 0
// and takes the bits of lane + j shifted up by j into the others; a lane with
// bit j set keeps the bits with b & j set and takes the bits of lane - j
// shifted down by j.  The masks repeat per half, and a bit that a shift
// carries across the halves' boundary always lands in a position the mask
// drops.  The partner's word comes by DPP (row_shl / row_shr).
__device__ __forceinline__ uint32_t row_transpose16x2(uint32_t x) {
  const uint32_t l = threadIdx.x & 15u;
#define RT_STAGE(J, M0, SHL, SHR)                                         \
  {                                                                       \
    const uint32_t up = tgs_dpp_u32<SHL, 0xf, 0xf, true>(x << J) & ~(M0); \
    const uint32_t dn = tgs_dpp_u32<SHR, 0xf, 0xf, true>(x >> J) & (M0);  \
    x = (l & J) ? ((x & ~(M0)) | dn) : ((x & (M0)) | up);                 \
  }
  RT_STAGE(8, 0x00ff00ffu, 0x108, 0x118)  // row_shl:8 / row_shr:8
  RT_STAGE(4, 0x0f0f0f0fu, 0x104, 0x114)
  RT_STAGE(2, 0x33333333u, 0x102, 0x112)
  RT_STAGE(1, 0x55555555u, 0x101, 0x111)
#undef RT_STAGE
  return x;
}

// This lane's coverage bits over list entries [0, n_list) (TILE == 16): bit
// li of mw[li / 32] is set when entry li's row interval (cover_row) holds the
// lane's own pixel (strip row lane / 16, column lane % 16) and the pixel is
// alive.  Per word of 32 entries lane 16 r + e computes entries 32 w + e and
// 32 w + 16 + e on strip row r, and row_transpose16x2 hands lane 16 r + c the
// word's bits of pixel (r, c): no round trip of the masks through LDS and no
// per-entry bit extraction.  With STORE the row masks also go to s_emh as two
// 32-bit halves per entry (s_emh[0][li]: rows 0-1, s_emh[1][li]: rows 2-3), as
// strip_masks stores them.
template <int BATCH, int WORDS, bool STORE, class Geo, typename LT, int SCALE>
__device__ __forceinline__ void strip_bits(const LT* s_list, int n_list, const Geo geo,
                                           const float4* s_cov, uint32_t (*s_emh)[BATCH],
                                           float px0, float py0, uint64_t alive,
                                           uint32_t (&mw)[WORDS]) {
  static_assert(WORDS * 32 == BATCH, "one word per 32 entries");
  const int lane = threadIdx.x & 63;
  const int r = lane >> 4, e = lane & 15;
  const uint32_t alive_row = (uint32_t)(alive >> (r * 16)) & 0xffffu;
  const float py = py0 + (float)r;
  auto cover = [&](int li) {
    const int t = (int)s_list[li] / SCALE;
    const uint32_t x =
        cover_row<16>(geo.G0(t), geo.G1(t), s_cov[t], px0, py) & alive_row;
    if (STORE) reinterpret_cast<uint16_t*>(&s_emh[r >> 1][li])[r & 1] = (uint16_t)x;
    return x;
  };
#pragma unroll
  for (int w = 0; w < WORDS; ++w) {
    mw[w] = 0u;
    if (32 * w >= n_list) continue;  // wave-uniform
    uint32_t x = 0u;
    if (32 * w + e < n_list) x = cover(32 * w + e);
    if (32 * w + 16 < n_list && 32 * w + 16 + e < n_list) x |= cover(32 * w + 16 + e) << 16;
    mw[w] = row_transpose16x2(x);
  }
  if (STORE) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// ---------------------------------------------------------------------------
// Workgroup order.  Workgroups start in linear-id order (x fastest) and go to
// the 8 XCDs round-robin.  Both kernels take one camera at a time, so the
// concurrent workgroups read one camera's splat records (which fit the
// last-level cache); within the camera the forward walks tiles row-major and
// the backward column-major, the faster order of each measured on the cfg3
// and cfg4 scenes (forward 4.64 -> 4.28 ms, backward 10.66 -> 10.18 ms at
// cfg3 against camera-fastest).  The backward's columns are also dealt out
// by XCD (xcd_line_order): each XCD walks whole tile columns, its own one of
// every 8 neighbouring columns, so tiles that share Gaussians vertically
// share an L2 (11.32 -> 11.22 ms at cfg3; the same by rows in the forward:
// 4.50 -> 4.57 ms, not used).
//   forward grid  (tile_w, tile_h, C)
//   backward grid (tile_h, tile_w, C)
// ---------------------------------------------------------------------------
inline dim3 raster_fwd_grid(const RasterGeom& G) { return dim3(G.tile_w, G.tile_h, G.C); }
inline dim3 raster_bwd_grid(const RasterGeom& G) { return dim3(G.tile_h, G.tile_w, G.C); }

// Workgroup lin (camera-local; consecutive workgroups go to the 8 XCDs in
// turn) -> (line, pos): line 8 * ((lin / 8) / len) + lin % 8, position
// (lin / 8) % len, so XCD x takes line x of each block of 8 lines whole.
// Lines past the last whole block of 8 keep the plain order.  A bijection of
// [0, n_lines * len).
__device__ __forceinline__ void xcd_line_order(uint32_t lin, uint32_t n_lines, uint32_t len,
                                               uint32_t& line, uint32_t& pos) {
  const uint32_t whole = (n_lines / 8u) * 8u * len;
  if (lin < whole) {
    const uint32_t j = lin >> 3;
    line = (j / len) * 8u + (lin & 7u);
    pos = j % len;
  } else {
    const uint32_t r = lin - whole;
    line = (n_lines / 8u) * 8u + r / len;
    pos = r % len;
  }
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
#define RF_BATCH 128  // Gaussians staged per batch

// (up to 4 channels the forward fits 64 VGPRs: 8 wavefronts per SIMD)
// COUNT: also count each pixel's composited Gaussians into n_contrib (a
// measurement aid; the plain variant leaves that counter out of the walk)
template <int CDIM, int TILE, class Src, bool COUNT = false>
__global__ void __launch_bounds__(TILE* TILE, CDIM <= 4 ? 8 : 1) raster_fwd_kernel(
    RasterGeom G, Src src, const float* __restrict__ backgrounds,
    const int32_t* __restrict__ tile_offsets, const int32_t* __restrict__ flatten_ids,
    float* __restrict__ render_colors, float* __restrict__ render_alphas,
    int32_t* __restrict__ last_ids, float4* __restrict__ clear = nullptr, uint64_t clear_n4 = 0,
    int32_t* __restrict__ n_contrib = nullptr) {
  constexpr int BLOCK = TILE * TILE;
  constexpr int WAVES = BLOCK / 64;
  constexpr int ROWS = 64 / TILE;  // pixel rows per wavefront
  constexpr int BATCH = RF_BATCH < BLOCK ? RF_BATCH : BLOCK;
  if (clear_n4) {
    // Side job: zero a buffer (the backward's gradient records) while the
    // compositing keeps the vector units busy; each workgroup stores its own
    // slice of clear_n4 16-byte words.
    const uint64_t groups = (uint64_t)gridDim.x * gridDim.y * gridDim.z;
    const uint64_t g = ((uint64_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    const uint64_t per = (clear_n4 + groups - 1) / groups;
    const uint64_t end = min(clear_n4, (g + 1) * per);
    for (uint64_t w = g * per + threadIdx.x; w < end; w += BLOCK)
      clear[w] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  constexpr int WORDS = BATCH / 32;
  __shared__ StagedRec<CDIM> s_rec[BATCH];
  __shared__ float4 s_box[BATCH];
  __shared__ float4 s_cov[BATCH];
  // each wavefront's list of staged entries as byte offsets of their records
  constexpr int RSZ = (int)sizeof(StagedRec<CDIM>);
  static_assert(BATCH * RSZ < 65536, "record offsets fit 16 bits");
  __shared__ uint16_t s_list[WAVES][BATCH];
  // the entries' row masks pass through LDS only for 8-pixel tiles (16-pixel
  // tiles transpose them in registers: strip_bits)
  constexpr int EMH = TILE == 16 ? 1 : BATCH;
  __shared__ __align__(16) uint32_t s_emh[WAVES][2][EMH];

  const uint32_t cam = blockIdx.z;
  const uint32_t ty = blockIdx.y, tx = blockIdx.x;
  const uint32_t tile_id = ty * G.tile_w + tx;
  const uint32_t tr = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane((int)(tr >> 6));  // wave-uniform
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

  // T > 0 while the pixel composites; a stopped pixel (or one outside the
  // image) holds -T, so the sign is its done flag and |T| its transmittance
  float T = inside ? 1.f : -1.f;
  uint32_t cur_idx = 0;
  int32_t n_comp = 0;  // Gaussians composited into this pixel
  float pix[CDIM];
#pragma unroll
  for (int k = 0; k < CDIM; ++k) pix[k] = 0.f;

  for (int32_t b = 0; b < n_batches; ++b) {
    if (__syncthreads_count(T < 0.f) >= BLOCK) break;
    const int32_t batch_start = range_start + BATCH * b;
    const int32_t idx = batch_start + (int32_t)tr;
    const bool have = (int)tr < BATCH && idx < range_end;
    SplatData<CDIM> s;
    if (have) src.load(flatten_ids[idx], s);
    bool odd_colour = false;
    if (have) {
      const StagedGeo sg = stage_geo<CDIM>(s);
      s_rec[tr].g0 = sg.g0;
      s_rec[tr].g1 = make_float4(sg.g1.x, sg.g1.y, 0.f, 0.f);
      s_box[tr] = sg.box;
      s_cov[tr] = sg.cov;
#pragma unroll
      for (int k = 0; k < CDIM; ++k) {
        s_rec[tr].col[k] = s.col[k];
        odd_colour |= !__builtin_isfinite(s.col[k]);
      }
    }
    // a batch with a non-finite colour walks with selects instead of
    // multiplying colours by zero (inf * 0 would reach pixels the Gaussian
    // does not composite)
    const bool safe_walk = __syncthreads_or(odd_colour) != 0;
    const int32_t batch_size = min(BATCH, range_end - batch_start);
    const uint64_t alive = tgs_ballot(T > 0.f);
    if (!alive) continue;
    uint64_t hits;
    const int n_list = build_wave_list<BATCH, uint16_t, RSZ>(s_box, s_list[wave], 0, batch_size,
                                                            wx0, wx1, wy0, wy1, hits);
    // list positions past the list name staged record 0, so a lane with no
    // entry left reads a staged record without a select
#pragma unroll
    for (int k = 0; k < BATCH; k += 64)
      if (n_list <= k + (int)(tr & 63)) s_list[wave][k + (tr & 63)] = 0;
    __builtin_amdgcn_wave_barrier();
    uint32_t mw[WORDS];
    if constexpr (TILE == 16) {
      strip_bits<BATCH, WORDS, false, GeoRecs<CDIM>, uint16_t, RSZ>(
          s_list[wave], n_list, GeoRecs<CDIM>{s_rec}, s_cov, nullptr, wx0, wy0, alive, mw);
    } else {
      strip_masks<TILE, BATCH, GeoRecs<CDIM>, uint16_t, RSZ>(
          s_list[wave], n_list, GeoRecs<CDIM>{s_rec}, s_cov, s_emh[wave], wx0, wy0, alive);
      lane_bits<WORDS, false>(s_emh[wave][(tr & 63) >> 5], n_list, 0, mw);
    }
    // the wavefront's list addressed from the lane index (a VGPR base, so the
    // walk's address add pairs with other VALU work)
    const uint16_t* my_list = &s_list[0][0] + (tr & ~63u) * (BATCH / 64);
    const char* rec_base = reinterpret_cast<const char*>(s_rec);
    // record offset of this batch's last composited Gaussian (0xffff: none);
    // the contributor index is derived from it once per batch, not per step
    uint32_t cur_off = 0xffffu;
    auto walk = [&](auto safe_tag) {
      constexpr bool SAFE = decltype(safe_tag)::value;
#pragma unroll
      for (int W = 0; W < WORDS; ++W) {
        if (W * 32 >= n_list) break;
        uint32_t m = T < 0.f ? 0u : mw[W];
        // every lane runs the body (no exec-mask branches): a lane with no
        // entry left reads staged record 0 and changes nothing; a Gaussian
        // failing the alpha test, or the one that would take T to the
        // threshold, adds exactly zero; a lane reaching the threshold clears m
        if (tgs_ballot(m != 0u)) do {
          const bool act = m != 0u;
          const int bit = __builtin_ctz(m | 0x80000000u);  // 31 where m is empty
          m &= m - 1u;
          const uint32_t off = my_list[W * 32 + bit];
          const StagedRec<CDIM>& rec = *reinterpret_cast<const StagedRec<CDIM>*>(rec_base + off);
          const float4 g0 = rec.g0;
          const float4 g1 = rec.g1;
          const float power = raster_power(g0, make_float2(g1.x, g1.y), g0.x - px, g0.y - py);
          const bool pass = act && !(power > g1.y || power < RS_LOG2_MIN_ALPHA);
          const float alpha = fminf(0.999f, __builtin_amdgcn_exp2f(power));
          const float next_T = T * (1.f - alpha);
          // alpha is never NaN (fminf keeps 0.999) and T is finite, so
          // next_T > 1e-4 is the reference's !(next_T <= 1e-4): one compare
          const bool big = next_T > 1e-4f;
          const bool comp = pass && big;
          const bool stop = pass != comp;  // pass && !big, from the lane masks
          m = stop ? 0u : m;
          const float vis = comp ? alpha * T : 0.f;
#pragma unroll
          for (int k = 0; k < CDIM; ++k)
            pix[k] = SAFE ? (comp ? fmaf(rec.col[k], vis, pix[k]) : pix[k])
                          : fmaf(rec.col[k], vis, pix[k]);
          cur_off = comp ? off : cur_off;
          if (COUNT) n_comp += comp ? 1 : 0;
          T = comp ? next_T : (stop ? -T : T);
        } while (tgs_ballot(m != 0u));
      }
    };
    if (safe_walk) walk(std::true_type{});
    else walk(std::false_type{});
    if (cur_off != 0xffffu) cur_idx = (uint32_t)batch_start + cur_off / (uint32_t)RSZ;
  }
  T = fabsf(T);
  if (inside) {
    const uint64_t pid = img + (uint64_t)i * G.W + j;
    render_alphas[pid] = 1.f - T;
#pragma unroll
    for (int k = 0; k < CDIM; ++k)
      render_colors[pid * CDIM + k] =
          backgrounds ? pix[k] + T * backgrounds[cam * CDIM + k] : pix[k];
    last_ids[pid] = (int32_t)cur_idx;
    if (COUNT) n_contrib[pid] = n_comp;
  }
}

// Inclusive prefix sum over the 64 lanes, in DPP: shifts by 1, 2, 4, 8 within
// each 16-lane row (lanes shifted in from outside the row add 0), then row 0's
// total into row 1 and row 2's into row 3 (row_bcast:15), then the total of
// rows 0-1 into rows 2 and 3 (row_bcast:31).  No lane-address registers.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  v += tgs_dpp_u32<0x111, 0xf, 0xf, true>(v);  // row_shr:1
  v += tgs_dpp_u32<0x112, 0xf, 0xf, true>(v);  // row_shr:2
  v += tgs_dpp_u32<0x114, 0xf, 0xf, true>(v);  // row_shr:4
  v += tgs_dpp_u32<0x118, 0xf, 0xf, true>(v);  // row_shr:8
  v += tgs_dpp_u32<0x142, 0xa>(v);             // row_bcast:15 into rows 1 and 3
  v += tgs_dpp_u32<0x143, 0xc>(v);             // row_bcast:31 into rows 2 and 3
  return v;
}

// ---------------------------------------------------------------------------
// Backward.  Per batch and wavefront:
//   1. masks    as in the forward: the list of entries whose box meets the
//               strip, each entry's 64-bit pixel mask (rows' coverage, lanes
//               that still composite part of the batch), a prefix sum of the
//               masks' popcounts giving each entry's slot range in a
//               (Gaussian, pixel) pair buffer, and each lane's bits over the
//               list (positions behind its own last contributor cleared);
//   2. walk     each lane walks its own entries back to front, applies the
//               exact test, carries T and the colour buffer, and leaves
//               (alpha T, v_sigma) in the entry's slot range at its rank among
//               the entry's pixels (slots of pixels that fail the test or
//               never composite the entry stay zero);
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
// Pair-buffer slots per wavefront.  The workgroup's LDS decides how many
// workgroups share a CU: measured on MI355X, 26656 bytes of static LDS still
// run 6 per CU and 26912 bytes only 5 (12.45 against 11.2 ms at cfg3), a limit
// the compiler's occupancy remark does not show.  At 3 channels the kernel
// uses 26400 bytes with 304 slots; 192 / 256 / 288 / 304 slots measured
// 12.25 / 11.5 / 11.3 / 11.2 ms (fewer segments per unit).
#define RB_PAIRS 304
#define RB_BATCH 64  // Gaussians staged per batch

template <int CDIM, int TILE, class Src, class Sink>
__global__ void __launch_bounds__(TILE* TILE, CDIM <= 4 ? 6 : 1) raster_bwd_kernel(
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
  // three colours padded to four (the fourth holds the Gaussian id): the walk
  // reads the colours with one 16-byte read
  // at the same t * 16 address as s_g0
  constexpr int CPAD = CDIM == 3 ? 4 : CDIM;
  __shared__ __align__(16) float s_col[BATCH][CPAD];
  __shared__ float s_vrc[BLOCK][CDIM];  // dL/dcolor of each pixel
  // the staged Gaussians' ids; at 3 channels they sit in the padding float of
  // s_col (256 bytes of LDS that keep the workgroup within 6 per CU)
  __shared__ int32_t s_id[CDIM == 3 ? 1 : BATCH];
  // each wavefront's list of staged entries as byte offsets t * 16 (the
  // stride of s_g0 and s_col; s_g1's is half of it)
  __shared__ uint16_t s_list[WAVES][BATCH];
  __shared__ float4 s_box[BATCH];
  __shared__ float4 s_cov[BATCH];
  __shared__ int32_t s_bin_max[WAVES];
  __shared__ float2 s_pair[WAVES][RB_PAIRS];  // (alpha T, v_sigma)
  __shared__ __align__(16) uint32_t s_emh[WAVES][2][BATCH];  // pixel mask halves of each list entry
  // first pair slot of each list entry's half: [0][li] that of lanes 0..31
  // (and [0][n_list] the list's total), [1][li] that of lanes 32..63
  __shared__ uint16_t s_poh[WAVES][2][BATCH + 1];
  __shared__ float s_stage[WAVES][32 * (Sink::MAY_ABS ? NA : NV)];  // one owner group's values
  __shared__ int32_t s_gid[WAVES][32];            // and their Gaussian ids

  const uint32_t cam = blockIdx.z;
  uint32_t ty, tx;
  xcd_line_order(blockIdx.y * G.tile_h + blockIdx.x, G.tile_w, G.tile_h, tx, ty);
  const uint32_t tile_id = ty * G.tile_w + tx;
  const uint32_t tr = threadIdx.x;
  static_assert(BATCH == 64, "one list entry per lane");
  const int lane = tr & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(tr >> 6));  // wave-uniform
  const int half = lane >> 5;
  const uint32_t lt_half = (1u << (lane & 31)) - 1u;  // lanes below this one in its half
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

  const float T_final = 1.f - render_alphas[pid];
  float T = T_final;
  float v_rc[CDIM];
#pragma unroll
  for (int k = 0; k < CDIM; ++k) {
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
  // the colour sum behind the current Gaussian enters v_alpha only through its
  // dot product with dL/dcolor, buffer_dot = sum_k buffer_k v_rc_k, and only as
  // tf_term - buffer_dot: the walk carries that difference
  float tf_dot = tf_term;
  const int32_t bin_final = inside ? last_ids[pid] : -1;
  const int32_t wave_bin_final = tgs_wave_max_i32(bin_final);
  // entries behind the tile's last contributor (any pixel's last_id) touch no
  // pixel: the back-to-front walk starts at the last one
  if (lane == 0) s_bin_max[wave] = wave_bin_final;
  __syncthreads();
  int32_t tile_bin_final = s_bin_max[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) tile_bin_final = max(tile_bin_final, s_bin_max[w]);
  const int32_t live_end = min(range_end, tile_bin_final + 1);
  const int32_t n_batches =
      live_end > range_start ? (live_end - range_start + BATCH - 1) / BATCH : 0;
  const bool absg = sink.absgrad();
  const int nval = absg ? NA : NV;
  // owner role within a group of 32 entries: entry oe, pixel bits [32 oh, 32 oh + 32)
  const int oe = lane >> 1, oh = lane & 1;

  for (int32_t b = 0; b < n_batches; ++b) {
    __syncthreads();
    const int32_t batch_end = live_end - 1 - BATCH * b;
    const int32_t batch_size = min(BATCH, batch_end + 1 - range_start);
    const int32_t idx = batch_end - (int32_t)tr;
    const bool have = (int)tr < BATCH && idx >= range_start;
    const int32_t g = have ? flatten_ids[idx] : 0;
    SplatData<CDIM> s;
    if (have) src.load(g, s);
    bool odd_colour = false;
    if (have) {
      const StagedGeo sg = stage_geo<CDIM>(s);
      s_g0[tr] = sg.g0;
      s_g1[tr] = sg.g1;
      s_box[tr] = sg.box;
      s_cov[tr] = sg.cov;
      if constexpr (CDIM == 3) s_col[tr][3] = __int_as_float(g);
      else s_id[tr] = g;
#pragma unroll
      for (int k = 0; k < CDIM; ++k) {
        s_col[tr][k] = s.col[k];
        odd_colour |= !__builtin_isfinite(s.col[k]);
      }
    }
    // a batch with a non-finite colour keeps the colour sum behind a pixel
    // with a select (a Gaussian failing the exact test must not add 0 * inf)
    const bool safe_walk = __syncthreads_or(odd_colour) != 0;
    // batch entry t is global index batch_end - t; a pixel composites the
    // entries at or before its last contributor: t >= t_min
    const int t_min = batch_end - bin_final;
    const uint64_t alive = tgs_ballot(inside && t_min < batch_size);
    // entries with global index > wave_bin_final contribute to no pixel of this wave
    const int j_lo = max(0, batch_end - wave_bin_final);
    int n_list = 0;
    uint64_t hits = 0;
    if (alive)
      n_list = build_wave_list<BATCH, uint16_t, 16>(s_box, s_list[wave], j_lo, batch_size, wx0,
                                                    wx1, wy0, wy1, hits);
    // 1. pixel masks, slot ranges and this lane's bits over the list
    uint32_t m[WORDS];
#pragma unroll
    for (int W = 0; W < WORDS; ++W) m[W] = 0u;
    uint32_t n_pairs = 0;  // wave-uniform
    if (n_list) {
      // the row masks go to s_emh (pair slots, owners); at 16-pixel tiles the
      // lane's bits come from a register transpose of the same masks
      if constexpr (TILE == 16)
        strip_bits<BATCH, WORDS, true, GeoArrays, uint16_t, 16>(
            s_list[wave], n_list, GeoArrays{s_g0, s_g1}, s_cov, s_emh[wave], wx0, wy0,
            alive, m);
      else
        strip_masks<TILE, BATCH, GeoArrays, uint16_t, 16>(s_list[wave], n_list,
                                                           GeoArrays{s_g0, s_g1}, s_cov,
                                                           s_emh[wave], wx0, wy0, alive);
      uint32_t c_lo = 0u, c_hi = 0u;
      if (lane < n_list) {
        c_lo = (uint32_t)__popc(s_emh[wave][0][lane]);
        c_hi = (uint32_t)__popc(s_emh[wave][1][lane]);
      }
      const uint32_t cnt = c_lo + c_hi;
      const uint32_t inc = wave_incl_scan(cnt);
      if (lane < n_list) {
        s_poh[wave][0][lane] = (uint16_t)(inc - cnt);
        s_poh[wave][1][lane] = (uint16_t)(inc - cnt + c_lo);
      }
      n_pairs = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
      if (lane == 63) s_poh[wave][0][n_list] = (uint16_t)inc;
      // list positions before li_min hold entries behind this lane's last
      // contributor: the listed entries t < t_min (the list is ascending in t)
      const int li_min =
          t_min <= 0 ? 0
                     : __popcll(hits & (t_min >= 64 ? ~0ull : ((1ull << t_min) - 1ull)));
      if constexpr (TILE == 16) {
        // strip_bits left bits [0, n_list) of alive lanes; drop those before li_min
#pragma unroll
        for (int W = 0; W < WORDS; ++W) {
          const int lo = min(max(li_min - 32 * W, 0), 32);
          m[W] &= lo >= 32 ? 0u : ~((1u << lo) - 1u);
        }
      } else {
        lane_bits<WORDS, true>(s_emh[wave][half], n_list, li_min, m);
        if (!((alive >> lane) & 1ull)) {
#pragma unroll
          for (int W = 0; W < WORDS; ++W) m[W] = 0u;
        }
      }
    }
    int a = 0;        // first list entry of the current segment
    while (a < n_list) {
      const uint32_t base = s_poh[wave][0][a];
      // largest end with at most RB_PAIRS pairs (an entry has <= 64)
      int e_end = n_list;
      if (n_pairs - base > RB_PAIRS) {
        int lo = a + 1, hi = n_list;  // s_poh[0][lo] - base <= RB_PAIRS < s_poh[0][hi] - base
        while (hi - lo > 1) {
          const int mid = (lo + hi) >> 1;
          if ((uint32_t)s_poh[wave][0][mid] - base <= RB_PAIRS) lo = mid;
          else hi = mid;
        }
        e_end = lo;
      }
      // zero the segment's slots: pixels that fail the exact test or do not
      // composite an entry leave theirs untouched
      const uint32_t seg_pairs = (uint32_t)s_poh[wave][0][e_end] - base;
      for (uint32_t s = lane; s < seg_pairs; s += 64) s_pair[wave][s] = make_float2(0.f, 0.f);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // 2. per-pixel walk over entries [a, e_end), back to front.  Addresses
      //    come from VGPR bases (the lane index, not the wave-uniform SGPR
      //    index): the list, the staged records, and the pair buffer moved
      //    back by the segment's first slot, so a pair's slot address is
      //    pair_v + 8 (first slot of its half + rank among the half's pixels)
      const uint16_t* my_list = &s_list[0][0] + (tr & ~63u);
      const char* g0_base = reinterpret_cast<const char*>(s_g0);
      const char* g1_base = reinterpret_cast<const char*>(s_g1);
      const char* col_base = reinterpret_cast<const char*>(&s_col[0][0]);
      char* pair_v = reinterpret_cast<char*>(&s_pair[0][0]) + (tr >> 6) * (RB_PAIRS * 8) -
                     8 * (int)base;
      auto walk = [&](auto safe_tag) {
        constexpr bool SAFE = decltype(safe_tag)::value;
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
              const uint32_t t16 = my_list[li];
              const float4 g0 = *reinterpret_cast<const float4*>(g0_base + t16);
              const float2 g1 = *reinterpret_cast<const float2*>(g1_base + (t16 >> 1));
              float4 col = make_float4(0.f, 0.f, 0.f, 0.f);
              if constexpr (CPAD == 4) col = *reinterpret_cast<const float4*>(col_base + t16);
              const float power = raster_power(g0, g1, g0.x - px, g0.y - py);
              // predicated rather than branched: a pixel failing the exact
              // test keeps T and the colour buffer and writes (0, 0), the
              // value its zeroed slot already holds
              const bool pass = !(power > g1.y || power < RS_LOG2_MIN_ALPHA);
              const float raw = __builtin_amdgcn_exp2f(power);  // opacity * exp(-sigma)
              const float alpha = fminf(0.999f, raw);
              const float ra = __builtin_amdgcn_rcpf(1.f - alpha);
              const float Tn = T * ra;
              T = pass ? Tn : T;
              // v_alpha = sum_k (c_k T - buffer_k ra) v_rc_k + ra tf_term
              const float ck[4] = {col.x, col.y, col.z, col.w};
              float cv = (CPAD == 4 ? ck[0] : s_col[t16 >> 4][0]) * v_rc[0];
#pragma unroll
              for (int k = 1; k < CDIM; ++k)
                cv = fmaf(CPAD == 4 ? ck[k] : s_col[t16 >> 4][k], v_rc[k], cv);
              const float v_alpha = fmaf(Tn, cv, ra * tf_dot);
              const float fac = pass ? alpha * Tn : 0.f;
              tf_dot = SAFE ? (pass ? fmaf(-fac, cv, tf_dot) : tf_dot) : fmaf(-fac, cv, tf_dot);
              // reference: the sigma terms only where alpha was not clamped
              const float v_sigma = pass && raw <= 0.999f ? -raw * v_alpha : 0.f;
              const uint32_t slot = (uint32_t)s_poh[wave][half][li] +
                                    (uint32_t)__popc(s_emh[wave][half][li] & lt_half);
              *reinterpret_cast<float2*>(pair_v + 8 * slot) = make_float2(fac, v_sigma);
            }
          }
        }
      };
      if (safe_walk) walk(std::true_type{});
      else walk(std::false_type{});
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // 3. owners, groups of 32 entries: lanes 2e, 2e+1 own entry e, each
      //    summing the moments over one half of the strip (pixel bits
      //    [32h, 32h+32)); one DPP step adds the halves and lane 2e stages
      //    the entry's gradient values
      for (int e0 = a; e0 < e_end; e0 += 32) {
        const int gn = min(32, e_end - e0);
        float acc[NA];
#pragma unroll
        for (int k = 0; k < NA; ++k) acc[k] = 0.f;
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        int t = 0;
        if (oe < gn) {
          const int li = e0 + oe;
          t = s_list[wave][li] >> 4;
          const float4 g0 = s_g0[t];
          q = staged_conic_rop(g0, s_g1[t]);
          uint32_t slot = (uint32_t)s_poh[wave][oh][li] - base;
          const uint32_t hb = s_emh[wave][oh][li];
          if (TILE == 16) {
            // the half is two pixel rows; within a row dy is constant, so
            // each row's dy moments follow from its sum(v_sigma) and
            // sum(v_sigma dx)
            const float gxr = g0.x - ((float)(tx * TILE) + 0.5f);
            const float dy0 = g0.y - ((float)(ty * TILE + wave * ROWS + 2 * oh) + 0.5f);
            const float dy1 = g0.y - ((float)(ty * TILE + wave * ROWS + 2 * oh + 1) + 0.5f);
            float s0[2], s1[2], s2[2];
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
              uint32_t rb = (hb >> (16 * rr)) & 0xffffu;
              const float* vrc = &s_vrc[wave * 64 + 32 * oh + 16 * rr][0];
              const float dy = rr == 0 ? dy0 : dy1;
              // the second row's pairs follow the first row's popcount ones,
              // so the loop advances only its pointer
              const float2* pp =
                  &s_pair[wave][slot + (rr == 0 ? 0u : (uint32_t)__popc(hb & 0xffffu))];
              float a0 = 0.f, a1 = 0.f, a2 = 0.f;
              while (rb != 0u) {
                const int jc = __builtin_ctz(rb);
                rb &= rb - 1u;
                const float2 pr = *pp++;
                const float dx = gxr - (float)jc;
                const float vs = pr.y;
                const float mx = vs * dx;
                a0 += vs;
                a1 += mx;
                a2 = fmaf(mx, dx, a2);
#pragma unroll
                for (int k = 0; k < CDIM; ++k)
                  acc[5 + k] = fmaf(pr.x, vrc[jc * CDIM + k], acc[5 + k]);
                if (absg) {
                  const float my = vs * dy;
                  acc[NV] += fabsf(q.x * mx + q.y * my);
                  acc[NV + 1] += fabsf(q.y * mx + q.z * my);
                }
              }
              s0[rr] = a0;
              s1[rr] = a1;
              s2[rr] = a2;
            }
            acc[0] = s1[0] + s1[1];
            acc[1] = dy0 * s0[0] + dy1 * s0[1];
            acc[2] = s2[0] + s2[1];
            acc[3] = dy0 * s1[0] + dy1 * s1[1];
            acc[4] = dy0 * dy0 * s0[0] + dy1 * dy1 * s0[1];
            acc[5 + CDIM] = s0[0] + s0[1];
          } else {
            uint32_t rb = hb;
            while (rb != 0u) {
              const int pl = 32 * oh + __builtin_ctz(rb);
              rb &= rb - 1u;
              const float2 pr = s_pair[wave][slot++];
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
        }
#pragma unroll
        for (int k = 0; k < NA; ++k) {
          if (k < NV || absg) {
            // full quad permute: every source lane exists, so bound_ctrl only
            // lets the compiler fold the move into the add
            acc[k] += tgs_dpp<0xB1, 0xf, 0xf, true>(acc[k]);  // quad_perm [1,0,3,2]
          }
        }
        if (oh == 0 && oe < gn) {
          if constexpr (CDIM == 3) s_gid[wave][oe] = __float_as_int(s_col[t][3]);
          else s_gid[wave][oe] = s_id[t];
          float* st = s_stage[wave] + oe * nval;
          st[0] = q.x * acc[0] + q.y * acc[1];
          st[1] = q.y * acc[0] + q.z * acc[1];
          st[2] = 0.5f * acc[2];
          st[3] = acc[3];
          st[4] = 0.5f * acc[4];
#pragma unroll
          for (int k = 0; k < CDIM; ++k)
            st[5 + k] = Src::CLAMP_MARKS && __float_as_uint(s_col[t][k]) == 0x80000000u
                            ? 0.f
                            : acc[5 + k];
          st[5 + CDIM] = -acc[5 + CDIM] * q.w;
          if (absg) {
            st[NV] = acc[NV];
            st[NV + 1] = acc[NV + 1];
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // 4. flush: (entry, value) pairs in value-fastest order, so that each
        //    atomic instruction covers a few Gaussians' contiguous records
        //    (the memory system merges the lanes that hit one line)
        const int total = gn * nval;
        for (int L = lane; L < total; L += 64) {
          const int e = absg ? L / NA : L / NV;
          const int k = L - e * nval;
          const float v = s_stage[wave][L];
          if (v != 0.f) tgs_atomic_add(sink.ptr(s_gid[wave][e], k), v);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      // every lane has read its pairs before the next segment clears them
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      a = e_end;
    }
  }
}
