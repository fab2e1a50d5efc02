/*
 * CPU restatement of gsplat's tile rasterizer (test oracle, not product code).
 *
 * Forward follows gsplat/cuda/csrc/rasterize_to_pixels_fwd.cu:14-160, backward
 * rasterize_to_pixels_bwd.cu:14-249, pixel by pixel and Gaussian by Gaussian in
 * the same order.  REAL is float (oracle_raster_f32) or double
 * (oracle_raster_f64); gradients are accumulated in double.  exp() is libm's.
 * The 32-lane "warp.any" skip of the reference only skips work whose
 * contributions are zero, so it has no counterpart here.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifndef REAL
#define REAL float
#endif
#ifndef SUFFIX
#define SUFFIX f32
#endif
#define CAT2(a, b) a##_##b
#define CAT(a, b) CAT2(a, b)
#define FN(name) CAT(name, SUFFIX)

static REAL rmin(REAL a, REAL b) { return a < b ? a : b; }

static REAL rexp(REAL x) { return (REAL)exp((double)x); }

/* the largest channel count the reference instantiates
 * (rasterize_to_pixels_fwd.cu:261-283) */
#define ORACLE_MAX_D 513

/* means2d [*,2], conics [*,3], colors [*,D], opac [*]; offsets [C,th,tw];
 * outputs colors [C,H,W,D], alphas [C,H,W], last_ids [C,H,W]. */
void FN(oracle_raster_fwd)(int C, int D, const REAL* means2d, const REAL* conics,
                           const REAL* colors, const REAL* opac, const REAL* backgrounds, int W,
                           int H, int tile, int tw, int th, const int32_t* offsets,
                           const int32_t* flat, int n_isects, REAL* out_colors, REAL* out_alphas,
                           int32_t* last_ids) {
  REAL pix[ORACLE_MAX_D];
  for (int c = 0; c < C; ++c) {
    for (int i = 0; i < H; ++i) {
      for (int j = 0; j < W; ++j) {
        const int tid = (i / tile) * tw + (j / tile);
        const int64_t toff = (int64_t)c * th * tw + tid;
        const int start = offsets[toff];
        const int end = (c == C - 1 && tid == tw * th - 1) ? n_isects : offsets[toff + 1];
        const REAL px = (REAL)j + (REAL)0.5, py = (REAL)i + (REAL)0.5;
        REAL T = 1;
        int cur = 0;
        for (int k = 0; k < D; ++k) pix[k] = 0;
        for (int idx = start; idx < end; ++idx) {
          const int g = flat[idx];
          const REAL dx = means2d[2 * (int64_t)g] - px, dy = means2d[2 * (int64_t)g + 1] - py;
          const REAL a = conics[3 * (int64_t)g], b = conics[3 * (int64_t)g + 1],
                     cc = conics[3 * (int64_t)g + 2];
          const REAL sigma = (REAL)0.5 * (a * dx * dx + cc * dy * dy) + b * dx * dy;
          const REAL alpha = rmin((REAL)0.999, opac[g] * rexp(-sigma));
          if (sigma < 0 || alpha < (REAL)1 / (REAL)255) continue;
          const REAL next_T = T * (1 - alpha);
          if (next_T <= (REAL)1e-4) break;
          const REAL vis = alpha * T;
          for (int k = 0; k < D; ++k) pix[k] += colors[(int64_t)g * D + k] * vis;
          cur = idx;
          T = next_T;
        }
        const int64_t pid = ((int64_t)c * H + i) * W + j;
        out_alphas[pid] = 1 - T;
        for (int k = 0; k < D; ++k)
          out_colors[pid * D + k] = backgrounds ? pix[k] + T * backgrounds[c * D + k] : pix[k];
        last_ids[pid] = cur;
      }
    }
  }
}

/* Gradients (double, zero-initialised by the caller): v_means2d [*,2],
 * v_conics [*,3], v_colors [*,D], v_opac [*], v_abs [*,2] (nullable). */
void FN(oracle_raster_bwd)(int C, int D, const REAL* means2d, const REAL* conics,
                           const REAL* colors, const REAL* opac, const REAL* backgrounds, int W,
                           int H, int tile, int tw, int th, const int32_t* offsets,
                           const int32_t* flat, int n_isects, const REAL* alphas,
                           const int32_t* last_ids, const REAL* v_out, const REAL* v_alpha_out,
                           double* v_means2d, double* v_conics, double* v_colors, double* v_opac,
                           double* v_abs) {
  REAL buffer[ORACLE_MAX_D], v_rc[ORACLE_MAX_D];
  for (int c = 0; c < C; ++c) {
    for (int i = 0; i < H; ++i) {
      for (int j = 0; j < W; ++j) {
        const int tid = (i / tile) * tw + (j / tile);
        const int64_t toff = (int64_t)c * th * tw + tid;
        const int start = offsets[toff];
        const int end = (c == C - 1 && tid == tw * th - 1) ? n_isects : offsets[toff + 1];
        const REAL px = (REAL)j + (REAL)0.5, py = (REAL)i + (REAL)0.5;
        const int64_t pid = ((int64_t)c * H + i) * W + j;
        const REAL T_final = 1 - alphas[pid];
        REAL T = T_final;
        const int bin_final = last_ids[pid];
        REAL bg_dot = 0;
        for (int k = 0; k < D; ++k) {
          buffer[k] = 0;
          v_rc[k] = v_out[pid * D + k];
          if (backgrounds) bg_dot += backgrounds[c * D + k] * v_rc[k];
        }
        const REAL v_ra = v_alpha_out ? v_alpha_out[pid] : 0;
        for (int idx = end - 1; idx >= start; --idx) {
          if (idx > bin_final) continue;
          const int g = flat[idx];
          const REAL dx = means2d[2 * (int64_t)g] - px, dy = means2d[2 * (int64_t)g + 1] - py;
          const REAL a = conics[3 * (int64_t)g], b = conics[3 * (int64_t)g + 1],
                     cc = conics[3 * (int64_t)g + 2];
          const REAL op = opac[g];
          const REAL sigma = (REAL)0.5 * (a * dx * dx + cc * dy * dy) + b * dx * dy;
          const REAL vis = rexp(-sigma);
          const REAL alpha = rmin((REAL)0.999, op * vis);
          if (sigma < 0 || alpha < (REAL)1 / (REAL)255) continue;
          const REAL ra = 1 / (1 - alpha);
          T *= ra;
          const REAL fac = alpha * T;
          REAL v_alpha = 0;
          for (int k = 0; k < D; ++k) {
            v_colors[(int64_t)g * D + k] += (double)(fac * v_rc[k]);
            v_alpha += (colors[(int64_t)g * D + k] * T - buffer[k] * ra) * v_rc[k];
          }
          v_alpha += T_final * ra * v_ra;
          if (backgrounds) v_alpha += -T_final * ra * bg_dot;
          if (op * vis <= (REAL)0.999) {
            const REAL v_sigma = -op * vis * v_alpha;
            v_conics[3 * (int64_t)g + 0] += (double)((REAL)0.5 * v_sigma * dx * dx);
            v_conics[3 * (int64_t)g + 1] += (double)(v_sigma * dx * dy);
            v_conics[3 * (int64_t)g + 2] += (double)((REAL)0.5 * v_sigma * dy * dy);
            const REAL vx = v_sigma * (a * dx + b * dy);
            const REAL vy = v_sigma * (b * dx + cc * dy);
            v_means2d[2 * (int64_t)g + 0] += (double)vx;
            v_means2d[2 * (int64_t)g + 1] += (double)vy;
            if (v_abs) {
              v_abs[2 * (int64_t)g + 0] += fabs((double)vx);
              v_abs[2 * (int64_t)g + 1] += fabs((double)vy);
            }
            v_opac[g] += (double)(vis * v_alpha);
          }
          for (int k = 0; k < D; ++k) buffer[k] += colors[(int64_t)g * D + k] * fac;
        }
      }
    }
  }
}

/* Which compositing decisions of the forward (the alpha >= 1/255 test and
 * the T <= 1e-4 stop of rasterize_to_pixels_fwd.cu:110-131) differ between
 * two sets of splat parameters over the same intersection lists: set A
 * (means2d_a, conics_a, opac_a) and set B, e.g. the same Gaussians projected
 * by two float32 evaluations.  A pixel whose sequence of decisions differs
 * is flagged in flip_pix [C,H,W] (uint8), and every entry that composites
 * into such a pixel under either set is flagged in entry_flag [*] (uint8):
 * those are the entries whose gradients a float32 rounding of the
 * projection can move by a whole pixel's contribution.  mark_pix [C,H,W]
 * (nullable) names more pixels whose composited entries are flagged too
 * (e.g. the neighbourhood through which a loss couples pixels). */
static int FN(decide)(const REAL* means2d, const REAL* conics, const REAL* opac, int g, REAL px,
                      REAL py, REAL* T) {
  /* 0: skipped, 1: composited, 2: stop (T would reach the threshold) */
  const REAL dx = means2d[2 * (int64_t)g] - px, dy = means2d[2 * (int64_t)g + 1] - py;
  const REAL a = conics[3 * (int64_t)g], b = conics[3 * (int64_t)g + 1],
             cc = conics[3 * (int64_t)g + 2];
  const REAL sigma = (REAL)0.5 * (a * dx * dx + cc * dy * dy) + b * dx * dy;
  const REAL alpha = rmin((REAL)0.999, opac[g] * rexp(-sigma));
  if (sigma < 0 || alpha < (REAL)1 / (REAL)255) return 0;
  const REAL next_T = *T * (1 - alpha);
  if (next_T <= (REAL)1e-4) return 2;
  *T = next_T;
  return 1;
}

void FN(oracle_raster_decision_flips)(int C, const REAL* means2d_a, const REAL* conics_a,
                                      const REAL* opac_a, const REAL* means2d_b,
                                      const REAL* conics_b, const REAL* opac_b, int W, int H,
                                      int tile, int tw, int th, const int32_t* offsets,
                                      const int32_t* flat, int n_isects, const uint8_t* mark_pix,
                                      uint8_t* flip_pix, uint8_t* entry_flag) {
  for (int c = 0; c < C; ++c) {
    for (int i = 0; i < H; ++i) {
      for (int j = 0; j < W; ++j) {
        const int tid = (i / tile) * tw + (j / tile);
        const int64_t toff = (int64_t)c * th * tw + tid;
        const int start = offsets[toff];
        const int end = (c == C - 1 && tid == tw * th - 1) ? n_isects : offsets[toff + 1];
        const REAL px = (REAL)j + (REAL)0.5, py = (REAL)i + (REAL)0.5;
        const int64_t pid = ((int64_t)c * H + i) * W + j;
        REAL Ta = 1, Tb = 1;
        int differ = 0, done_a = 0, done_b = 0;
        for (int idx = start; idx < end && !(done_a && done_b); ++idx) {
          const int g = flat[idx];
          const int da = done_a ? -1 : FN(decide)(means2d_a, conics_a, opac_a, g, px, py, &Ta);
          const int db = done_b ? -1 : FN(decide)(means2d_b, conics_b, opac_b, g, px, py, &Tb);
          if (da != db) differ = 1;
          if (da == 2) done_a = 1;
          if (db == 2) done_b = 1;
        }
        flip_pix[pid] = (uint8_t)differ;
        if (!(differ || (mark_pix && mark_pix[pid]))) continue;
        /* second walk: flag the entries composited under either set */
        Ta = 1;
        Tb = 1;
        done_a = done_b = 0;
        for (int idx = start; idx < end && !(done_a && done_b); ++idx) {
          const int g = flat[idx];
          const int da = done_a ? -1 : FN(decide)(means2d_a, conics_a, opac_a, g, px, py, &Ta);
          const int db = done_b ? -1 : FN(decide)(means2d_b, conics_b, opac_b, g, px, py, &Tb);
          if (da == 1 || db == 1) entry_flag[g] = 1;
          if (da == 2) done_a = 1;
          if (db == 2) done_b = 1;
        }
      }
    }
  }
}
