// Fused per-batch TideGS step over the resident [N,59] Gaussian table.
//
// What TideGS does per batch (strategies/tide_engine/engine.py:1435-2737):
//   filters  = packed projection per camera (base_engine.py:222-461,
//              gsplat fully_fused_projection_packed_fwd.cu:19-183)
//   touched  = union of the filters (engine.py:1801-1827)
//   per camera: gather rows + activations (engine.py:2255-2268), projection,
//              SH colors, isect + sort, rasterize, loss, backward, scatter_add
//              of the row gradients into the compact [T, .] buffers
//              (engine.py:2434-2469)
//   resident Adam over the touched rows (runtime.py:1741-1791)
// Here the same computation is reorganised for one GPU launch per stage over
// the whole batch:
//   tide_visibility  one pass over rows: per-camera visibility bits with the
//                    packed-projection rule, per-block counts
//   tide_compact     per-camera visible lists ("entries", ascending rows as the
//                    reference filters), the touched-row list and, per touched
//                    row, the list of its entries in camera order ("visits")
//   tide_project_fwd projection + SH colour + activations for every entry,
//                    written as one 48-byte splat record
//   tide_isect_emit  batched keys camera|tile|depth for one sort of the batch
//   (rasterize fwd / bwd with the packed splat policy, see raster.cuh)
//   tide_project_bwd one thread per touched row walks its visits in camera
//                    order, accumulates the projection/SH/activation VJPs and
//                    writes the row's 59 gradients once (no atomics and no
//                    read-modify-write of the compact gradient); the fused
//                    variant applies the resident optimizer update to the
//                    row in the same launch instead of writing the gradients.
// Resident table columns (TideGS CACHE order, storage/block_reader.py:35-44):
//   xyz 0..2 | log-scale 3..5 | quat 6..9 (w,x,y,z) | opacity logit 10 | SH 11..58
// with SH coefficient k, channel c at column 11 + 3k + c.
#include <cmath>

#include "projection.cuh"
#include "raster.cuh"
#include "resident_optim.cuh"
#include "sh.cuh"

#define TIDE_ROW 59
#define TIDE_MAX_CAMS 32
#define VIS_THREADS 256

struct TideCams {
  const float* viewmats;  // [C,16]
  const float* Ks;        // [C,9]
  const float* campos;    // [C,3] camera centres in world space
  uint32_t C;
};

struct CamLDS {
  Cam cam[TIDE_MAX_CAMS];
  float campos[TIDE_MAX_CAMS][3];
  float lim[TIDE_MAX_CAMS][2];  // projection clamp 1.3 * (0.5 W / fx), 1.3 * (0.5 H / fy)
};

__device__ __forceinline__ void load_cams_lds(const TideCams& tc, CamLDS& s, int W = 0,
                                              int H = 0) {
  for (uint32_t c = threadIdx.x; c < tc.C; c += blockDim.x) {
    s.cam[c] = load_cam(tc.viewmats + c * 16, tc.Ks + c * 9);
    s.campos[c][0] = tc.campos[c * 3 + 0];
    s.campos[c][1] = tc.campos[c * 3 + 1];
    s.campos[c][2] = tc.campos[c * 3 + 2];
    s.lim[c][0] = 1.3f * (0.5f * (float)W / s.cam[c].fx);
    s.lim[c][1] = 1.3f * (0.5f * (float)H / s.cam[c].fy);
  }
  __syncthreads();
}

// torch.nn.functional.normalize: q / max(|q|, 1e-12)
__device__ __forceinline__ void normalize4(const float* q, float out[4], float& inv_norm) {
  const float n = sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
  const float d = fmaxf(n, 1e-12f);
  inv_norm = 1.f / d;
#pragma unroll
  for (int k = 0; k < 4; ++k) out[k] = q[k] / d;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + expf(-x)); }

// Packed-projection visibility (fully_fused_projection_packed_fwd.cu:50-131):
// same culls as the render projection but radius = ceil(3 sqrt(max(v1, v2)))
// with the 0.1 floor.
__device__ __forceinline__ bool packed_visible(const float p[3], const m3& Sigma, const Cam& cam,
                                               int W, int H, float eps2d, float near_plane,
                                               float far_plane, float radius_clip, float& depth) {
  float pc[3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
    pc[i] = cam.R[i][0] * p[0] + cam.R[i][1] * p[1] + cam.R[i][2] * p[2] + cam.t[i];
  depth = pc[2];
  if (pc[2] < near_plane || pc[2] > far_plane) return false;
  m3 Rc;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) Rc.m[i][j] = cam.R[i][j];
  const m3 Sc = m3_mul_bt(m3_mul(Rc, Sigma), Rc);
  const float x = pc[0], y = pc[1], z = pc[2];
  const float lim_x = 1.3f * (0.5f * (float)W / cam.fx);
  const float lim_y = 1.3f * (0.5f * (float)H / cam.fy);
  const float rz = 1.f / z, rz2 = rz * rz;
  const float tx = z * fminf(lim_x, fmaxf(-lim_x, x * rz));
  const float ty = z * fminf(lim_y, fmaxf(-lim_y, y * rz));
  const float J00 = cam.fx * rz, J02 = -cam.fx * tx * rz2;
  const float J11 = cam.fy * rz, J12 = -cam.fy * ty * rz2;
  float JS0[3], JS1[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    JS0[k] = J00 * Sc.m[0][k] + J02 * Sc.m[2][k];
    JS1[k] = J11 * Sc.m[1][k] + J12 * Sc.m[2][k];
  }
  const float a = JS0[0] * J00 + JS0[2] * J02 + eps2d;
  const float b = JS0[1] * J11 + JS0[2] * J12;
  const float d = JS1[1] * J11 + JS1[2] * J12 + eps2d;
  const float det = a * d - b * b;
  if (det <= 0.f) return false;
  const float bb = 0.5f * (a + d);
  const float s = sqrtf(fmaxf(0.1f, bb * bb - det));
  const float radius = ceilf(3.f * sqrtf(fmaxf(bb + s, bb - s)));
  if (radius <= radius_clip) return false;
  const float mx = cam.fx * x * rz + cam.cx;
  const float my = cam.fy * y * rz + cam.cy;
  if (mx + radius <= 0.f || mx - radius >= (float)W || my + radius <= 0.f ||
      my - radius >= (float)H)
    return false;
  return true;
}

__device__ __forceinline__ m3 row_covariance(const float* __restrict__ row) {
  const float s[3] = {expf(row[3]), expf(row[4]), expf(row[5])};
  float qn[4], inv;
  normalize4(row + 6, qn, inv);
  return covar_from_quat_scale(qn, s);
}

#define TIDE_RANGE_SLOTS 64  // {min, max} pairs of the depth-key range

// ---------------------------------------------------------------------------
// Visibility + per-block counts.  counts layout (uint32, block-minor):
//   [c * nb + b]        visible rows of camera c in block b   (c < C)
//   [C * nb + b]        touched rows in block b
//   [(C+1) * nb + b]    visits (sum of popcount(mask)) in block b
// With depth_range (TIDE_RANGE_SLOTS {min, max} pairs set to {~0, 0} by the
// launch), the smallest and largest float bits of the visible entries' depths
// (positive, so ordered like the depths) are folded in, workgroup b into
// pair b mod TIDE_RANGE_SLOTS (atomics on one pair from every workgroup would
// serialize): the depth sort's key range is the min / max over the pairs.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(VIS_THREADS) tide_visibility_kernel(
    uint64_t n_rows, const float* __restrict__ params, uint32_t row_stride, TideCams tc, int W,
    int H, float eps2d, float near_plane, float far_plane, float radius_clip,
    uint32_t* __restrict__ masks, uint32_t* __restrict__ counts,
    uint32_t* __restrict__ depth_range) {
  __shared__ CamLDS s_cam;
  __shared__ uint32_t s_cnt[TIDE_MAX_CAMS + 2];
  __shared__ uint32_t s_rng[2];
  load_cams_lds(tc, s_cam);
  if (threadIdx.x < TIDE_MAX_CAMS + 2) s_cnt[threadIdx.x] = 0;
  if (threadIdx.x < 2) s_rng[threadIdx.x] = threadIdx.x == 0 ? 0xffffffffu : 0u;
  __syncthreads();
  const uint64_t n = (uint64_t)blockIdx.x * VIS_THREADS + threadIdx.x;
  const uint32_t nb = gridDim.x;
  uint32_t mask = 0;
  uint32_t kmin = 0xffffffffu, kmax = 0u;
  if (n < n_rows) {
    const float* row = params + n * row_stride;
    const float p[3] = {row[0], row[1], row[2]};
    const m3 Sigma = row_covariance(row);
    for (uint32_t c = 0; c < tc.C; ++c) {
      float depth;
      if (packed_visible(p, Sigma, s_cam.cam[c], W, H, eps2d, near_plane, far_plane, radius_clip,
                         depth)) {
        mask |= 1u << c;
        kmin = min(kmin, __float_as_uint(depth));
        kmax = max(kmax, __float_as_uint(depth));
      }
    }
    masks[n] = mask;
  }
  if (depth_range) {  // wave min / max first: one LDS update per wavefront
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, off, 64));
      kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, off, 64));
    }
    if ((threadIdx.x & 63) == 0 && kmax >= kmin) {
      atomicMin(&s_rng[0], kmin);
      atomicMax(&s_rng[1], kmax);
    }
  }
  const int lane = threadIdx.x & 63;
  for (uint32_t c = 0; c < tc.C; ++c) {
    const uint32_t cnt = (uint32_t)__popcll(tgs_ballot((mask >> c) & 1u));
    if (lane == 0 && cnt) atomicAdd(&s_cnt[c], cnt);
  }
  const uint32_t tcnt = (uint32_t)__popcll(tgs_ballot(mask != 0));
  if (lane == 0 && tcnt) atomicAdd(&s_cnt[tc.C], tcnt);
  atomicAdd(&s_cnt[tc.C + 1], (uint32_t)__popc(mask));
  __syncthreads();
  if (threadIdx.x < tc.C + 2) counts[(uint64_t)threadIdx.x * nb + blockIdx.x] = s_cnt[threadIdx.x];
  if (depth_range && threadIdx.x == 0 && s_rng[1] >= s_rng[0]) {
    uint32_t* slot = depth_range + 2 * (blockIdx.x % TIDE_RANGE_SLOTS);
    atomicMin(&slot[0], s_rng[0]);
    atomicMax(&slot[1], s_rng[1]);
  }
}

__global__ void tide_range_init_kernel(uint32_t* __restrict__ r) {
  if (threadIdx.x < 2 * TIDE_RANGE_SLOTS) r[threadIdx.x] = (threadIdx.x & 1u) ? 0u : 0xffffffffu;
}

// offs = exclusive scan of counts (same layout).  Writes:
//   entries[base_c + rank] = row          (camera lists, concatenated, ascending rows)
//   touched[t] = row, visit_base[t] = first visit of row t (visit_base[T] = total)
//   visits[visit_base[t] + j] = entry of the j-th camera (ascending) seeing row t
//   totals[0..C-1] = V_c, totals[C] = T, totals[C+1] = sum_c V_c
__global__ void __launch_bounds__(VIS_THREADS) tide_compact_kernel(
    uint64_t n_rows, uint32_t C, const uint32_t* __restrict__ masks,
    const uint32_t* __restrict__ offs, int32_t* __restrict__ entries,
    int32_t* __restrict__ touched, int32_t* __restrict__ visit_base,
    int32_t* __restrict__ visits, uint32_t* __restrict__ totals) {
  __shared__ uint32_t s_wave[VIS_THREADS / 64][TIDE_MAX_CAMS + 2];
  extern __shared__ uint32_t s_vis[];  // [waves][64 * C] visit staging
  const uint32_t nb = gridDim.x;
  const uint64_t n = (uint64_t)blockIdx.x * VIS_THREADS + threadIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const uint32_t mask = n < n_rows ? masks[n] : 0u;
  const uint32_t total_entries = offs[(uint64_t)C * nb];  // sum of V_c
  const uint32_t total_touched = offs[(uint64_t)(C + 1) * nb] - total_entries;

  // per-wave ranks and counts: cameras, touched, visits
  uint32_t rank[TIDE_MAX_CAMS];
#pragma unroll
  for (uint32_t c = 0; c < TIDE_MAX_CAMS; ++c) {
    if (c < C) {
      const uint64_t b = tgs_ballot((mask >> c) & 1u);
      rank[c] = (uint32_t)__popcll(b & lt);
      if (lane == 0) s_wave[wave][c] = (uint32_t)__popcll(b);
    }
  }
  const uint64_t tb = tgs_ballot(mask != 0);
  const uint32_t trank = (uint32_t)__popcll(tb & lt);
  if (lane == 0) s_wave[wave][C] = (uint32_t)__popcll(tb);
  // inclusive wave scan of popcount(mask)
  const uint32_t pc = (uint32_t)__popc(mask);
  uint32_t inc = pc;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = __shfl_up(inc, off, 64);
    if (lane >= off) inc += o;
  }
  if (lane == 63) s_wave[wave][C + 1] = inc;
  __syncthreads();
  if (__builtin_amdgcn_readfirstlane((int)(tb == 0ull))) return;  // no touched row in the wave

  auto wave_prefix = [&](uint32_t k) {
    uint32_t s = 0;
    for (int w = 0; w < wave; ++w) s += s_wave[w][k];
    return s;
  };
  const bool act = n < n_rows && mask != 0u;
  // the wave's visits are one contiguous range [wv0, wv0 + s_wave[wave][C+1]):
  // each lane puts its visits into the wave's LDS slice, and the wave stores
  // the slice with consecutive lanes (whole lines instead of one scattered
  // word per lane and camera)
  const uint32_t wv0 = offs[(uint64_t)(C + 1) * nb + blockIdx.x] - total_entries - total_touched +
                       wave_prefix(C + 1);
  uint32_t* sv = s_vis + (uint64_t)wave * 64u * C;
  if (act) {
    const uint32_t t =
        offs[(uint64_t)C * nb + blockIdx.x] - total_entries + wave_prefix(C) + trank;
    touched[t] = (int32_t)n;
    visit_base[t] = (int32_t)(wv0 + (inc - pc));
  }
  uint32_t j = inc - pc;
  for (uint32_t c = 0; c < C; ++c) {
    if (act && ((mask >> c) & 1u)) {
      const uint32_t e = offs[(uint64_t)c * nb + blockIdx.x] + wave_prefix(c) + rank[c];
      entries[e] = (int32_t)n;
      sv[j++] = e;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint32_t wtot = s_wave[wave][C + 1];
  for (uint32_t k = (uint32_t)lane; k < wtot; k += 64u) visits[wv0 + k] = (int32_t)sv[k];
  (void)totals;
}

__global__ void tide_totals_kernel(uint32_t C, uint32_t nb, const uint32_t* __restrict__ counts,
                                   const uint32_t* __restrict__ offs,
                                   uint32_t* __restrict__ totals,
                                   int32_t* __restrict__ cam_offsets,
                                   int32_t* __restrict__ visit_base) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  const uint64_t last = (uint64_t)(C + 2) * nb - 1;
  const uint32_t grand = offs[last] + counts[last];
  const uint32_t ents = offs[(uint64_t)C * nb];
  const uint32_t tch = offs[(uint64_t)(C + 1) * nb] - ents;
  for (uint32_t c = 0; c < C; ++c) {
    const uint32_t lo = offs[(uint64_t)c * nb];
    const uint32_t hi = offs[(uint64_t)(c + 1) * nb];
    totals[c] = hi - lo;
    cam_offsets[c] = (int32_t)lo;
  }
  cam_offsets[C] = (int32_t)ents;
  totals[C] = tch;
  totals[C + 1] = ents;
  totals[C + 2] = grand - ents - tch;  // visits (== ents)
  visit_base[tch] = (int32_t)ents;
}

// ---------------------------------------------------------------------------
// Forward projection + SH for every entry -> packed splat records.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t entry_camera(const int32_t* s_off, uint32_t C, uint32_t e) {
  uint32_t c = 0;
  while (c + 1 < C && (uint32_t)s_off[c + 1] <= e) ++c;
  return c;
}

// Tile rectangle [x0,x1) x [y0,y1) of one entry, 8 bits per bound (grids up
// to 255 x 255 tiles), carried through the depth sort beside the entry index.
__device__ __forceinline__ uint32_t pack_rect(uint32_t x0, uint32_t x1, uint32_t y0, uint32_t y1) {
  return x0 | (x1 << 8) | (y0 << 16) | (y1 << 24);
}
__device__ __forceinline__ uint32_t rect_tiles(uint32_t rc) {
  const uint32_t x0 = rc & 255u, x1 = (rc >> 8) & 255u, y0 = (rc >> 16) & 255u, y1 = rc >> 24;
  return (x1 > x0 ? x1 - x0 : 0u) * (y1 > y0 ? y1 - y0 : 0u);
}

// Projection + SH colour of one (camera, row) entry e into the packed splat
// record, its depth key and its tile rectangle; returns the rectangle's area
// (the entry's intersection count).
__device__ __forceinline__ uint32_t project_entry(
    const float p[3], const m3& Sigma, float opac, const float* sh, const Cam& cam,
    const float* campos, int W, int H, float eps2d, float near_plane, float far_plane,
    float radius_clip, int sh_degree, uint32_t tile_size, uint32_t tw, uint32_t th, uint32_t e,
    float4* __restrict__ splats, uint32_t* __restrict__ depth_keys,
    uint64_t* __restrict__ entry_rects, uint32_t& key) {
  const ProjResult r =
      project_forward(p, Sigma, cam, W, H, eps2d, near_plane, far_plane, radius_clip);
  float4* out = splats + (uint64_t)e * 3;
  if (r.radius <= 0) {
    out[0] = make_float4(0.f, 0.f, 0.f, 0.f);
    out[1] = make_float4(0.f, 0.f, 0.f, 0.f);
    out[2] = make_float4(0.f, 0.f, 0.f, 0.f);
    key = 0xffffffffu;
    depth_keys[e] = 0xffffffffu;
    entry_rects[e] = (uint64_t)e;  // empty rectangle
    return 0u;
  }
  float col[3];
  sh_eval3(sh_degree, p[0] - campos[0], p[1] - campos[1], p[2] - campos[2], sh, col);
  out[0] = make_float4(r.mean2d[0], r.mean2d[1], opac, r.depth);
  out[1] = make_float4(r.conic[0], r.conic[1], r.conic[2], (float)r.radius);
  // colour = clamp_min(SH + 0.5, 0); a clamped channel is stored as -0.0, so
  // that the rasterizer backward gives it a zero gradient (the clamp's VJP)
  auto clamp_mark = [](float v) { return v >= 0.f ? v : -0.f; };
  out[2] = make_float4(clamp_mark(col[0] + 0.5f), clamp_mark(col[1] + 0.5f),
                       clamp_mark(col[2] + 0.5f), 0.f);
  // tile count (isect_tiles.cu:55-70)
  const float ts = (float)tile_size;
  const float trd = (float)r.radius / ts;
  const float txx = r.mean2d[0] / ts, tyy = r.mean2d[1] / ts;
  auto clampu = [](float v, uint32_t lim) -> uint32_t {
    if (!(v > 0.f)) return 0u;
    if (v >= (float)lim) return lim;
    return (uint32_t)v;
  };
  const uint32_t x0 = clampu(floorf(txx - trd), tw), x1 = clampu(ceilf(txx + trd), tw);
  const uint32_t y0 = clampu(floorf(tyy - trd), th), y1 = clampu(ceilf(tyy + trd), th);
  // depth > near_plane > 0, so the float bits order like the depths
  key = __float_as_uint(r.depth);
  depth_keys[e] = key;
  entry_rects[e] = ((uint64_t)pack_rect(x0, x1, y0, y1) << 32) | e;
  return (x1 - x0) * (y1 - y0);  // x1 >= x0 and y1 >= y0 (clamped floor / ceil)
}

// One thread per touched row: the row (59 floats) is read once and projected
// into every camera it is visible in (its visits, in camera order, are the
// set bits of its visibility mask); SH coefficients stay in registers.  With
// isect_totals (zeroed by the launch) the per-camera intersection counts are
// summed too: a wave sum per camera step, LDS counters per workgroup, one
// 64-bit atomic per camera and workgroup.  With depth_range (TIDE_RANGE_SLOTS
// {min, max} pairs, initialised by the launch) the smallest and largest depth
// key written (culled entries' sentinels excluded) are folded in as the
// visibility pass does, so the host can check that the depth sort's key
// range, taken from the visibility pass, holds every key.
__global__ void __launch_bounds__(256) tide_project_fwd_kernel(
    uint32_t n_touched, const uint32_t* __restrict__ n_touched_dev,
    const int32_t* __restrict__ touched,
    const int32_t* __restrict__ visit_base, const int32_t* __restrict__ visits,
    const uint32_t* __restrict__ masks, TideCams tc, const float* __restrict__ params,
    uint32_t row_stride, int W, int H, float eps2d, float near_plane, float far_plane,
    float radius_clip, int sh_degree, uint32_t tile_size, uint32_t tw, uint32_t th,
    float4* __restrict__ splats,
    uint32_t* __restrict__ depth_keys, uint64_t* __restrict__ entry_rects,
    int64_t* __restrict__ isect_totals, uint32_t* __restrict__ depth_range) {
  __shared__ CamLDS s_cam;
  __shared__ uint32_t s_area[TIDE_MAX_CAMS];
  __shared__ uint32_t s_rng[2];
  load_cams_lds(tc, s_cam);
  if (threadIdx.x < TIDE_MAX_CAMS) s_area[threadIdx.x] = 0u;
  if (threadIdx.x < 2) s_rng[threadIdx.x] = threadIdx.x == 0 ? 0xffffffffu : 0u;
  __syncthreads();
  const uint32_t limit = n_touched_dev ? min(*n_touched_dev, n_touched) : n_touched;
  if (blockIdx.x * blockDim.x >= limit) return;  // the whole workgroup
  // rows past the touched count stay in the loop (empty visibility mask) so
  // the wave sums run on full wavefronts
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  const bool active = t < limit;
  const uint32_t n = active ? (uint32_t)touched[t] : 0u;
  const float* row = params + (uint64_t)n * row_stride;
  const float p[3] = {row[0], row[1], row[2]};
  const m3 Sigma = row_covariance(row);
  const float opac = sigmoidf_(row[10]);
  float sh[48];
#pragma unroll
  for (int k = 0; k < 48; ++k) sh[k] = row[11 + k];
  const uint32_t mask = active ? masks[n] : 0u;
  const int32_t* vis = visits + (active ? visit_base[t] : 0);
  // cameras in lockstep across the wavefront: the camera's constants are an
  // LDS broadcast, and the lanes seeing camera c write consecutive entries of
  // its list (coalesced records)
  int j = 0;
  uint32_t kmin = 0xffffffffu, kmax = 0u;
  for (uint32_t c = 0; c < tc.C; ++c) {
    uint32_t area = 0u;
    if ((mask >> c) & 1u) {
      const uint32_t e = (uint32_t)vis[j++];
      uint32_t key;
      area = project_entry(p, Sigma, opac, sh, s_cam.cam[c], s_cam.campos[c], W, H, eps2d,
                           near_plane, far_plane, radius_clip, sh_degree, tile_size, tw, th, e,
                           splats, depth_keys, entry_rects, key);
      if (key != 0xffffffffu) {
        kmin = min(kmin, key);
        kmax = max(kmax, key);
      }
    }
    if (isect_totals) {
      const uint32_t wsum = (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_scan(area), 63);
      if ((threadIdx.x & 63u) == 0u && wsum) atomicAdd(&s_area[c], wsum);
    }
  }
  if (depth_range) {  // wave min / max, then one LDS update per wavefront
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, off, 64));
      kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, off, 64));
    }
    if ((threadIdx.x & 63) == 0 && kmax >= kmin) {
      atomicMin(&s_rng[0], kmin);
      atomicMax(&s_rng[1], kmax);
    }
  }
  if (isect_totals || depth_range) __syncthreads();
  if (isect_totals && threadIdx.x < tc.C && s_area[threadIdx.x])
    atomicAdd((unsigned long long*)&isect_totals[threadIdx.x],
              (unsigned long long)s_area[threadIdx.x]);
  if (depth_range && threadIdx.x == 0 && s_rng[1] >= s_rng[0]) {
    uint32_t* slot = depth_range + 2 * (blockIdx.x % TIDE_RANGE_SLOTS);
    atomicMin(&slot[0], s_rng[0]);
    atomicMax(&slot[1], s_rng[1]);
  }
}


// ---------------------------------------------------------------------------
// Intersections in the reference's order (isect_tiles.cu:73-98,189-227).
// The reference emits camera|tile|depth keys in (camera, entry) order and
// stable-sorts them, i.e. orders intersections by (camera, tile, depth bits,
// entry).  Here entries are first stable-sorted by depth bits within each
// camera (carrying their tile rectangles), intersections are emitted in that
// order with camera|tile keys, and a stable sort of the tile bits within each
// camera gives the same total order.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) tide_isect_count_kernel(
    uint32_t n_entries, const uint64_t* __restrict__ rects, int32_t* __restrict__ tiles) {
  const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n_entries) return;
  tiles[j] = (int32_t)rect_tiles((uint32_t)(rects[j] >> 32));
}

// Per-camera intersection counts from the (unsorted) tile rectangles: the
// sum of the rectangles' areas over each camera's entries.  Each workgroup
// sums ISECT_TOTAL_PER_BLOCK consecutive entries into LDS counters and adds
// them to the camera totals with one 64-bit atomic per camera it met.
#define ISECT_TOTAL_ITEMS 32
#define ISECT_TOTAL_PER_BLOCK (256 * ISECT_TOTAL_ITEMS)

__global__ void tide_zero_i64_kernel(int64_t* __restrict__ p, uint32_t n) {
  if (threadIdx.x < n) p[threadIdx.x] = 0;
}

__global__ void __launch_bounds__(256) tide_isect_totals_kernel(
    uint32_t n_cap, const uint32_t* __restrict__ n_dev, const uint64_t* __restrict__ rects,
    const int32_t* __restrict__ cam_offsets, uint32_t C, int64_t* __restrict__ totals) {
  __shared__ int32_t s_off[TIDE_MAX_CAMS + 1];
  __shared__ uint32_t s_sum[TIDE_MAX_CAMS];
  if (threadIdx.x <= C) s_off[threadIdx.x] = cam_offsets[threadIdx.x];
  if (threadIdx.x < TIDE_MAX_CAMS) s_sum[threadIdx.x] = 0u;
  __syncthreads();
  const uint32_t n = n_dev ? min(*n_dev, n_cap) : n_cap;
  const uint32_t base = blockIdx.x * ISECT_TOTAL_PER_BLOCK;
  if (base >= n) return;
  // entries are grouped by camera: a thread's entries ascend, so its camera
  // only moves forward; the running sum goes to LDS when it does
  // all of the thread's rectangles (high words) are loaded before any is used
  const uint32_t* hi = reinterpret_cast<const uint32_t*>(rects) + 1;
  uint32_t rc[ISECT_TOTAL_ITEMS];
#pragma unroll
  for (int k = 0; k < ISECT_TOTAL_ITEMS; ++k) {
    const uint32_t e = base + (uint32_t)k * 256u + threadIdx.x;
    rc[k] = e < n ? hi[2ull * e] : 0u;
  }
  uint32_t e = base + threadIdx.x;
  uint32_t c = entry_camera(s_off, C, min(e, n - 1));
  uint32_t acc = 0u;
#pragma unroll
  for (int k = 0; k < ISECT_TOTAL_ITEMS; ++k, e += 256u) {
    while (c + 1 < C && e >= (uint32_t)s_off[c + 1]) {
      if (acc) atomicAdd(&s_sum[c], acc);
      acc = 0u;
      ++c;
    }
    acc += rect_tiles(rc[k]);
  }
  if (acc) atomicAdd(&s_sum[c], acc);
  __syncthreads();
  if (threadIdx.x < C && s_sum[threadIdx.x])
    atomicAdd((unsigned long long*)&totals[threadIdx.x], (unsigned long long)s_sum[threadIdx.x]);
}

__global__ void tide_isect_segments_kernel(uint32_t C, const int32_t* __restrict__ cam_offsets,
                                           const int64_t* __restrict__ cum_tiles,
                                           int64_t* __restrict__ seg) {
  const uint32_t c = threadIdx.x;
  if (c > C) return;
  const int32_t o = cam_offsets[c];
  seg[c] = o > 0 ? cum_tiles[o - 1] : 0;
}

__global__ void __launch_bounds__(256) tide_isect_emit_kernel(
    uint32_t n_entries, const int32_t* __restrict__ cam_offsets, uint32_t C,
    const uint64_t* __restrict__ rects, const int64_t* __restrict__ cum_tiles, uint32_t tw,
    uint32_t tile_n_bits, uint32_t* __restrict__ keys, int32_t* __restrict__ flatten_ids) {
  __shared__ int32_t s_off[TIDE_MAX_CAMS + 1];
  if (threadIdx.x <= C) s_off[threadIdx.x] = cam_offsets[threadIdx.x];
  __syncthreads();
  const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= n_entries) return;
  const uint64_t v = rects[j];
  const uint32_t rc = (uint32_t)(v >> 32);
  const uint32_t x0 = rc & 255u, x1 = (rc >> 8) & 255u, y0 = (rc >> 16) & 255u, y1 = rc >> 24;
  const uint32_t cam_enc = entry_camera(s_off, C, j) << tile_n_bits;
  const int32_t e = (int32_t)(uint32_t)v;
  uint32_t cur = j == 0 ? 0u : (uint32_t)cum_tiles[j - 1];
  for (uint32_t y = y0; y < y1; ++y)
    for (uint32_t x = x0; x < x1; ++x) {
      keys[cur] = cam_enc | (y * tw + x);
      flatten_ids[cur] = e;
      ++cur;
    }
}

// Emission with block-local offsets: the depth-ordered entries are taken in
// blocks of EMIT_ENTRIES; tide_isect_block_sums_kernel sums each block's
// rectangle areas, the host-side launch scans those sums (exclusive), and
// the emission kernel turns a block's base into its entries' first
// intersection slots with wave prefix sums.  Entry k * 256 + t of a block is
// item k of thread t, so each round of stores covers 256 consecutive entries
// (the per-entry int64 offsets of the count + scan form are never written).
#define EMIT_ITEMS 8
#define EMIT_ENTRIES (256 * EMIT_ITEMS)

__global__ void __launch_bounds__(256) tide_isect_block_sums_kernel(
    uint32_t n_entries, const uint64_t* __restrict__ rects, uint32_t* __restrict__ block_sums) {
  __shared__ uint32_t s_w[4];
  const uint32_t base = blockIdx.x * EMIT_ENTRIES;
  const uint32_t* hi = reinterpret_cast<const uint32_t*>(rects) + 1;
  uint32_t rc[EMIT_ITEMS];
#pragma unroll
  for (int k = 0; k < EMIT_ITEMS; ++k) {
    const uint32_t e = base + (uint32_t)k * 256u + threadIdx.x;
    rc[k] = e < n_entries ? hi[2ull * e] : 0u;
  }
  uint32_t acc = 0u;
#pragma unroll
  for (int k = 0; k < EMIT_ITEMS; ++k) acc += rect_tiles(rc[k]);
  const uint32_t inc = wave_incl_scan(acc);
  if ((threadIdx.x & 63u) == 63u) s_w[threadIdx.x >> 6] = inc;
  __syncthreads();
  if (threadIdx.x == 0) block_sums[blockIdx.x] = s_w[0] + s_w[1] + s_w[2] + s_w[3];
}

// The tile-bit sort's first-pass digit counts, counted while emitting (the
// layout of tgs_segmented_sort_pairs_u32_hist0: segments = cameras, sort
// tiles of EMIT_SORT_TILE intersections).  A block's outputs are consecutive
// slots: their first EMIT_HWIN sort tiles are counted in LDS and added once
// per (tile, digit); slots past them add to the global counts directly.
#define EMIT_SORT_TILE 4096  // the sort's tile for 4-byte keys and values
#define EMIT_HWIN 4
struct EmitHist {
  uint32_t* hist;      // tile_base[C] * 256 words
  uint64_t words;      // bound of every index written
  uint32_t mask;       // first-pass digit mask
  uint32_t seg_start[TIDE_MAX_CAMS + 1];  // first intersection slot of each camera
  uint32_t tile_base[TIDE_MAX_CAMS + 1];  // first sort tile of each camera
};

__device__ __forceinline__ void emit_hist_add(const EmitHist& eh, uint32_t c, uint32_t g,
                                              uint32_t d, uint32_t n) {
  const uint32_t tb = eh.tile_base[c];
  const uint64_t idx = (uint64_t)tb * 256u + (uint64_t)d * (eh.tile_base[c + 1] - tb) + (g - tb);
  if (idx < eh.words) atomicAdd(&eh.hist[idx], n);
}

template <bool HIST>
__global__ void __launch_bounds__(256) tide_isect_emit_blocked_kernel(
    uint32_t n_entries, const int32_t* __restrict__ cam_offsets, uint32_t C,
    const uint64_t* __restrict__ rects, const uint32_t* __restrict__ block_base, uint32_t tw,
    uint32_t tile_n_bits, uint32_t* __restrict__ keys, int32_t* __restrict__ flatten_ids,
    EmitHist eh) {
  __shared__ int32_t s_off[TIDE_MAX_CAMS + 1];
  __shared__ uint32_t s_tot[EMIT_ITEMS][4];  // per round, each wavefront's area sum
  __shared__ uint32_t s_h[HIST ? EMIT_HWIN : 1][256];
  if (threadIdx.x <= C) s_off[threadIdx.x] = cam_offsets[threadIdx.x];
  uint32_t g_lo = 0;  // sort tile of the block's first slot
  if (HIST) {
#pragma unroll
    for (int j = 0; j < EMIT_HWIN; ++j) s_h[j][threadIdx.x] = 0u;
    const uint32_t r0 = block_base[blockIdx.x];
    uint32_t cl = 0;
    while (cl + 1 < C && eh.seg_start[cl + 1] <= r0) ++cl;
    g_lo = eh.tile_base[cl] + (r0 - eh.seg_start[cl]) / EMIT_SORT_TILE;
  }
  const uint32_t base = blockIdx.x * EMIT_ENTRIES;
  const uint32_t wave = threadIdx.x >> 6;
  uint64_t v[EMIT_ITEMS];
#pragma unroll
  for (int k = 0; k < EMIT_ITEMS; ++k) {
    const uint32_t e = base + (uint32_t)k * 256u + threadIdx.x;
    v[k] = e < n_entries ? rects[e] : 0ull;  // an empty rectangle past the end
  }
  uint32_t excl[EMIT_ITEMS];  // area prefix within the round's wavefront
#pragma unroll
  for (int k = 0; k < EMIT_ITEMS; ++k) {
    const uint32_t a = rect_tiles((uint32_t)(v[k] >> 32));
    const uint32_t inc = wave_incl_scan(a);
    excl[k] = inc - a;
    if ((threadIdx.x & 63u) == 63u) s_tot[k][wave] = inc;
  }
  __syncthreads();
  uint32_t run = block_base[blockIdx.x];  // first slot of the round
  uint32_t c = 0;                         // camera of the thread's entries (ascending)
#pragma unroll
  for (int k = 0; k < EMIT_ITEMS; ++k) {
    uint32_t before = 0u, round = 0u;
#pragma unroll
    for (uint32_t w = 0; w < 4; ++w) {
      const uint32_t t = s_tot[k][w];
      before += w < wave ? t : 0u;
      round += t;
    }
    const uint32_t e = base + (uint32_t)k * 256u + threadIdx.x;
    if (e < n_entries) {
      while (c + 1 < C && (uint32_t)s_off[c + 1] <= e) ++c;
      const uint32_t rc = (uint32_t)(v[k] >> 32);
      const uint32_t x0 = rc & 255u, x1 = (rc >> 8) & 255u, y0 = (rc >> 16) & 255u,
                     y1 = rc >> 24;
      const uint32_t cam_enc = c << tile_n_bits;
      const int32_t id = (int32_t)(uint32_t)v[k];
      uint32_t cur = run + before + excl[k];
      for (uint32_t y = y0; y < y1; ++y)
        for (uint32_t x = x0; x < x1; ++x) {
          keys[cur] = cam_enc | (y * tw + x);
          flatten_ids[cur] = id;
          if (HIST) {
            const uint32_t g = eh.tile_base[c] + (cur - eh.seg_start[c]) / EMIT_SORT_TILE;
            const uint32_t d = (y * tw + x) & eh.mask;
            if (g - g_lo < EMIT_HWIN) atomicAdd(&s_h[g - g_lo][d], 1u);
            else emit_hist_add(eh, c, g, d, 1u);
          }
          ++cur;
        }
    }
    run += round;
  }
  if (HIST) {
    __syncthreads();
#pragma unroll
    for (int j = 0; j < EMIT_HWIN; ++j) {
      const uint32_t n = s_h[j][threadIdx.x];
      const uint32_t g = g_lo + (uint32_t)j;
      if (n != 0u && g < eh.tile_base[C]) {
        uint32_t cg = 0;
        while (cg + 1 < C && eh.tile_base[cg + 1] <= g) ++cg;
        emit_hist_add(eh, cg, g, threadIdx.x, n);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Emission fused with the tile-bit sort's first pass.  The depth-ordered
// entries of each camera are taken in blocks of FE_ENTRIES (a block never
// spans two cameras).  tide_isect_fused_count_kernel counts every block's
// intersections by first-pass digit (tile & mask) into hist, laid out
// [camera][digit][block of the camera], so that its exclusive scan is the
// first output slot of every (camera, digit, block).  tide_isect_fused_
// scatter_kernel then generates each block's intersections in emission order
// (entries in depth order, each entry's tiles row by row) in LDS chunks of
// FE_CHUNK, ranks each chunk stably by the digit (ballot matching and per-wave
// digit counters, as the radix passes do), and writes every digit's run of the
// chunk contiguously at its slot: the emission's keys and flatten ids never
// reach memory in emission order.  Stable in the emission order, so the
// remaining tile-bit passes give the reference's order unchanged.
// ---------------------------------------------------------------------------
#define FE_ENTRIES 1024
#define FE_ITEMS (FE_ENTRIES / 256)
#define FE_CHUNK 2048
#define FE_KEYS (FE_CHUNK / 256)

struct FusedEmit {
  uint32_t C;
  uint32_t tw, tile_n_bits;
  uint32_t mask;                          // first-pass digit of a tile: tile & mask
  uint32_t ent_off[TIDE_MAX_CAMS + 1];    // first depth-ordered entry of each camera
  uint32_t blk_first[TIDE_MAX_CAMS + 1];  // first block of each camera
};

__device__ __forceinline__ void fe_block(const FusedEmit& fe, uint32_t b, uint32_t& c,
                                         uint32_t& bl, uint32_t& e0, uint32_t& e1) {
  c = 0;
  while (c + 1 < fe.C && fe.blk_first[c + 1] <= b) ++c;
  bl = b - fe.blk_first[c];
  e0 = fe.ent_off[c] + bl * FE_ENTRIES;
  e1 = min(e0 + FE_ENTRIES, fe.ent_off[c + 1]);
}

// hist word of (camera c, digit d, block bl of c)
__device__ __forceinline__ uint64_t fe_hist_index(const FusedEmit& fe, uint32_t c, uint32_t d,
                                                  uint32_t bl) {
  const uint32_t nb = fe.blk_first[c + 1] - fe.blk_first[c];
  return (uint64_t)fe.blk_first[c] * (fe.mask + 1u) + (uint64_t)d * nb + bl;
}

__global__ void __launch_bounds__(256) tide_isect_fused_count_kernel(
    FusedEmit fe, const uint64_t* __restrict__ rects, uint32_t* __restrict__ hist) {
  __shared__ uint32_t s_cnt[256];
  uint32_t c, bl, e0, e1;
  fe_block(fe, blockIdx.x, c, bl, e0, e1);
  s_cnt[threadIdx.x] = 0u;
  __syncthreads();
  const uint32_t* hi = reinterpret_cast<const uint32_t*>(rects) + 1;
  uint32_t rc[FE_ITEMS];
#pragma unroll
  for (int k = 0; k < FE_ITEMS; ++k) {
    const uint32_t e = e0 + (uint32_t)k * 256u + threadIdx.x;
    rc[k] = e < e1 ? hi[2ull * e] : 0u;  // 0: an empty rectangle
  }
#pragma unroll
  for (int k = 0; k < FE_ITEMS; ++k) {
    const uint32_t x0 = rc[k] & 255u, x1 = (rc[k] >> 8) & 255u, y0 = (rc[k] >> 16) & 255u,
                   y1 = rc[k] >> 24;
    for (uint32_t y = y0; y < y1; ++y)
      for (uint32_t x = x0; x < x1; ++x) atomicAdd(&s_cnt[(y * fe.tw + x) & fe.mask], 1u);
  }
  __syncthreads();
  if (threadIdx.x <= fe.mask) hist[fe_hist_index(fe, c, threadIdx.x, bl)] = s_cnt[threadIdx.x];
}

__global__ void __launch_bounds__(256) tide_isect_fused_scatter_kernel(
    FusedEmit fe, const uint64_t* __restrict__ rects, const uint32_t* __restrict__ hist_scan,
    uint32_t n_isects, uint32_t* __restrict__ keys, int32_t* __restrict__ flatten_ids) {
  constexpr int WAVES = 4;
  __shared__ uint32_t s_k[FE_CHUNK];
  __shared__ int32_t s_v[FE_CHUNK];
  __shared__ uint32_t s_wh[WAVES][256];
  __shared__ uint32_t s_start[256];
  __shared__ uint32_t s_gofs[256];
  __shared__ uint32_t s_run[256];  // the block's slots of each digit so far
  __shared__ uint32_t s_tot[FE_ITEMS][WAVES];
  __shared__ uint32_t s_wsum[WAVES];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t lt = (1ull << lane) - 1ull;
  uint32_t c, bl, e0, e1;
  fe_block(fe, blockIdx.x, c, bl, e0, e1);
  const uint32_t cam_enc = c << fe.tile_n_bits;
  // the block's entries: item k of thread t is entry e0 + k * 256 + t; each
  // entry's first intersection of the block from a scan in entry order
  uint32_t rc[FE_ITEMS], p[FE_ITEMS];
  int32_t id[FE_ITEMS];
#pragma unroll
  for (int k = 0; k < FE_ITEMS; ++k) {
    const uint32_t e = e0 + (uint32_t)k * 256u + threadIdx.x;
    const uint64_t v = e < e1 ? rects[e] : 0ull;  // an empty rectangle past the end
    rc[k] = (uint32_t)(v >> 32);
    id[k] = (int32_t)(uint32_t)v;
    const uint32_t a = rect_tiles(rc[k]);
    const uint32_t inc = wave_incl_scan(a);
    p[k] = inc - a;
    if (lane == 63) s_tot[k][wave] = inc;
  }
  s_run[threadIdx.x] = 0u;
  s_gofs[threadIdx.x] = threadIdx.x <= fe.mask ? hist_scan[fe_hist_index(fe, c, threadIdx.x, bl)]
                                               : 0u;
  __syncthreads();
  uint32_t n_b = 0;  // the block's intersections
#pragma unroll
  for (int k = 0; k < FE_ITEMS; ++k) {
    uint32_t before = 0u, round = 0u;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const uint32_t t = s_tot[k][w];
      before += w < wave ? t : 0u;
      round += t;
    }
    p[k] += n_b + before;
    n_b += round;
  }
  // s_gofs holds each digit's first slot for the block until the chunk loop
  // turns it into per-chunk bases; keep the block bases in s_start's place
  uint32_t gbase = s_gofs[threadIdx.x];
  for (uint32_t q0 = 0; q0 < n_b; q0 += FE_CHUNK) {
    const uint32_t m = min((uint32_t)FE_CHUNK, n_b - q0);
    // 1. the chunk's intersections in emission order
#pragma unroll
    for (int k = 0; k < FE_ITEMS; ++k) {
      const uint32_t a = rect_tiles(rc[k]);
      const uint32_t lo = max(p[k], q0), hi = min(p[k] + a, q0 + FE_CHUNK);
      if (lo < hi) {
        const uint32_t x0 = rc[k] & 255u, x1 = (rc[k] >> 8) & 255u, y0 = (rc[k] >> 16) & 255u;
        const uint32_t w = x1 - x0;
        const uint32_t o = lo - p[k];  // nonzero only for an entry spanning chunks
        uint32_t y = y0 + (o ? o / w : 0u);
        uint32_t x = x0 + (o ? o % w : 0u);
        for (uint32_t i = lo - q0; i < hi - q0; ++i) {
          s_k[i] = cam_enc | (y * fe.tw + x);
          s_v[i] = id[k];
          if (++x == x1) {
            x = x0;
            ++y;
          }
        }
      }
    }
    if (threadIdx.x < 256) {
#pragma unroll
      for (int w = 0; w < WAVES; ++w) s_wh[w][threadIdx.x] = 0u;
    }
    __syncthreads();
    // 2. stable rank by digit: wave w owns chunk positions [w * 1024, (w + 1) * 1024)
    //    in rounds of 64
    uint32_t kk[FE_KEYS];
    int32_t vv[FE_KEYS];
    uint32_t rk[FE_KEYS];
#pragma unroll
    for (int r = 0; r < FE_KEYS; ++r) {
      const uint32_t li = (uint32_t)(wave * 64 * FE_KEYS + r * 64 + lane);
      const bool valid = li < m;
      kk[r] = valid ? s_k[li] : 0u;
      vv[r] = valid ? s_v[li] : 0;
      const uint32_t d = kk[r] & fe.mask;
      uint64_t peers = tgs_ballot(valid);
      rk[r] = 0u;
      if (peers) {
        const uint32_t d0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)d);
        if (tgs_ballot(valid && d == d0) != peers) {
#pragma unroll
          for (int bb = 0; bb < 8; ++bb) {
            if ((fe.mask >> bb) == 0u) break;
            const bool bit = (d >> bb) & 1u;
            const uint64_t mm = tgs_ballot(bit);
            peers &= bit ? mm : ~mm;
          }
        }
        const uint32_t before = s_wh[wave][d];
        __builtin_amdgcn_wave_barrier();
        if (valid && (peers >> lane) == 1ull) s_wh[wave][d] = before + (uint32_t)__popcll(peers);
        __builtin_amdgcn_wave_barrier();
        rk[r] = before + (uint32_t)__popcll(peers & lt);
      }
    }
    __syncthreads();
    // 3. digit t: per-wave offsets, chunk start, output base
    uint32_t tot = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const uint32_t cnt = s_wh[w][threadIdx.x];
      s_wh[w][threadIdx.x] = tot;
      tot += cnt;
    }
    uint32_t inc = wave_incl_scan(tot);
    if (lane == 63) s_wsum[wave] = inc;
    __syncthreads();
    uint32_t st = inc - tot;
    for (int w = 0; w < wave; ++w) st += s_wsum[w];
    s_start[threadIdx.x] = st;
    s_gofs[threadIdx.x] = gbase + s_run[threadIdx.x] - st;
    __syncthreads();
    // 4. the chunk in (digit, emission) order into LDS, then each digit's run
    //    written contiguously
#pragma unroll
    for (int r = 0; r < FE_KEYS; ++r) {
      const uint32_t li = (uint32_t)(wave * 64 * FE_KEYS + r * 64 + lane);
      if (li < m) {
        const uint32_t d = kk[r] & fe.mask;
        const uint32_t pos = s_start[d] + s_wh[wave][d] + rk[r];
        s_k[pos] = kk[r];
        s_v[pos] = vv[r];
      }
    }
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < m; j += 256) {
      const uint32_t key = s_k[j];
      const uint32_t o = s_gofs[key & fe.mask] + j;
      if (o < n_isects) {
        keys[o] = key;
        flatten_ids[o] = s_v[j];
      }
    }
    s_run[threadIdx.x] += tot;
    __syncthreads();
  }
}

__global__ void tide_zero_u32_kernel(uint32_t* __restrict__ p, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// isect_offset_encode (isect_tiles.cu:234-301) over camera|tile keys.
// Tile offsets by search: bucket b = (camera, tile) gets the index of the
// first sorted key >= its own key (camera << tile_n_bits | tile), which is the
// reference's encoding (isect_tiles.cu:234-301: a bucket with no
// intersections takes the next occupied bucket's start, buckets after the
// last key take n_isects).  One thread per bucket, a branch-free binary
// search with a uniform trip count (log2 of top + 1 probes, top = the largest
// power of two <= n_isects): the 130k buckets of a 16-camera 1080p batch
// probe about 27 keys each instead of one pass over every sorted key.
__global__ void __launch_bounds__(256) tide_offset_search_kernel(
    uint32_t n_isects, const uint32_t* __restrict__ keys, uint32_t n_buckets, uint32_t n_tiles,
    uint32_t tile_n_bits, uint32_t top, int32_t* __restrict__ offsets) {
  const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_buckets) return;
  const uint32_t cam = b / n_tiles;
  const uint32_t kb = (cam << tile_n_bits) | (b - cam * n_tiles);
  uint32_t pos = 0;  // keys[0, pos) are all < kb
  for (uint32_t step = top; step != 0u; step >>= 1) {
    const uint32_t p = pos + step;
    if (p <= n_isects && keys[p - 1] < kb) pos = p;
  }
  offsets[b] = (int32_t)pos;
}

// The reference's int64 intersection ids (camera|tile << 32 | depth bits,
// isect_tiles.cu:89-94), rebuilt from the sorted keys for inspection.
__global__ void __launch_bounds__(256) tide_isect_ids_kernel(
    uint32_t n_isects, const uint32_t* __restrict__ keys, const int32_t* __restrict__ fids,
    const float4* __restrict__ splats, int64_t* __restrict__ isect_ids) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_isects) return;
  const float depth = splats[(uint64_t)fids[i] * 3].w;
  isect_ids[i] = ((int64_t)keys[i] << 32) | (int64_t)__float_as_int(depth);
}

// ---------------------------------------------------------------------------
// Backward: one thread per touched row.
// ---------------------------------------------------------------------------
// VJP of the render projection of one (row, camera) visit
// (fully_fused_projection_bwd.cu:199-366 composed with the forward of
// fully_fused_projection_fwd.cu:18-129), restated for the resident step.
// Entries the forward culled carry zero splat gradients, so the backward
// skips only the visits where its own arithmetic would not be finite: depth
// outside [near, far] or a non-positive 2D determinant.  Reciprocals use the
// hardware rcp (1 ulp); the camera-space covariance, its gradient and the
// world-space covariance gradient are symmetric and formed from their six
// unique entries (order 00, 01, 02, 11, 12, 22).  Adds d/dmean to v_p and
// d/dSigma to vS; returns false for a skipped visit.
__device__ __forceinline__ bool tide_visit_backward(const float p[3], const float S[6],
                                                    const Cam& cam, float lim_x, float lim_y,
                                                    float eps2d, float near_plane,
                                                    float far_plane, const float vm[2],
                                                    const float vc[3], float v_p[3],
                                                    float vS[6]) {
  const auto& R = cam.R;
  float pc[3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
    pc[i] = cam.R[i][0] * p[0] + cam.R[i][1] * p[1] + cam.R[i][2] * p[2] + cam.t[i];
  const float x = pc[0], y = pc[1], z = pc[2];
  if (!(z >= near_plane && z <= far_plane)) return false;
  // Sc = R Sigma R^T
  float RS[3][3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    RS[i][0] = R[i][0] * S[0] + R[i][1] * S[1] + R[i][2] * S[2];
    RS[i][1] = R[i][0] * S[1] + R[i][1] * S[3] + R[i][2] * S[4];
    RS[i][2] = R[i][0] * S[2] + R[i][1] * S[4] + R[i][2] * S[5];
  }
  auto dot3 = [](const float* a, const float* b) { return a[0] * b[0] + a[1] * b[1] + a[2] * b[2]; };
  const float c00 = dot3(RS[0], R[0]), c01 = dot3(RS[0], R[1]), c02 = dot3(RS[0], R[2]);
  const float c11 = dot3(RS[1], R[1]), c12 = dot3(RS[1], R[2]), c22 = dot3(RS[2], R[2]);
  const float fx = cam.fx, fy = cam.fy;
  const float rz = __builtin_amdgcn_rcpf(z);
  const float rz2 = rz * rz, rz3 = rz2 * rz;
  const float xr = x * rz, yr = y * rz;
  const float tx = z * fminf(lim_x, fmaxf(-lim_x, xr));
  const float ty = z * fminf(lim_y, fmaxf(-lim_y, yr));
  const float J00 = fx * rz, J02 = -fx * tx * rz2;
  const float J11 = fy * rz, J12 = -fy * ty * rz2;
  // J Sc (2x3) and cov2d = J Sc J^T + eps2d I
  const float JS0[3] = {J00 * c00 + J02 * c02, J00 * c01 + J02 * c12, J00 * c02 + J02 * c22};
  const float JS1[3] = {J11 * c01 + J12 * c02, J11 * c11 + J12 * c12, J11 * c12 + J12 * c22};
  const float a = JS0[0] * J00 + JS0[2] * J02 + eps2d;
  const float b = JS0[1] * J11 + JS0[2] * J12;
  const float d = JS1[1] * J11 + JS1[2] * J12 + eps2d;
  const float det = a * d - b * b;
  if (!(det > 0.f)) return false;
  const float inv = __builtin_amdgcn_rcpf(det);
  const float P00 = d * inv, P01 = -b * inv, P11 = a * inv;
  // conic = cov2d^-1: dL/dcov2d = -P G P (symmetric; G's off-diagonal split
  // evenly over the two entries)
  const float G00 = vc[0], G01 = 0.5f * vc[1], G11 = vc[2];
  const float T00 = G00 * P00 + G01 * P01, T01 = G00 * P01 + G01 * P11;
  const float T10 = G01 * P00 + G11 * P01, T11 = G01 * P01 + G11 * P11;
  const float C00 = -(P00 * T00 + P01 * T10);
  const float C01 = -(P00 * T01 + P01 * T11);
  const float C11 = -(P01 * T01 + P11 * T11);
  // dL/dSc = J^T C J
  const float GJ0[3] = {C00 * J00, C01 * J11, C00 * J02 + C01 * J12};
  const float GJ1[3] = {C01 * J00, C11 * J11, C01 * J02 + C11 * J12};
  const float g[6] = {J00 * GJ0[0], J00 * GJ0[1], J00 * GJ0[2],
                      J11 * GJ1[1], J11 * GJ1[2], J02 * GJ0[2] + J12 * GJ1[2]};
  // dL/dJ = 2 C J Sc (entries 00, 02, 11, 12 are the ones J depends on)
  const float GJm00 = 2.f * (C00 * JS0[0] + C01 * JS1[0]);
  const float GJm02 = 2.f * (C00 * JS0[2] + C01 * JS1[2]);
  const float GJm11 = 2.f * (C01 * JS0[1] + C11 * JS1[1]);
  const float GJm12 = 2.f * (C01 * JS0[2] + C11 * JS1[2]);
  float gpc0 = fx * rz * vm[0];
  float gpc1 = fy * rz * vm[1];
  float gpc2 = -(fx * x * vm[0] + fy * y * vm[1]) * rz2;
  if (xr <= lim_x && xr >= -lim_x)
    gpc0 += -fx * rz2 * GJm02;
  else
    gpc2 += -fx * rz3 * GJm02 * tx;
  if (yr <= lim_y && yr >= -lim_y)
    gpc1 += -fy * rz2 * GJm12;
  else
    gpc2 += -fy * rz3 * GJm12 * ty;
  gpc2 += -fx * rz2 * GJm00 - fy * rz2 * GJm11 + 2.f * fx * tx * rz3 * GJm02 +
          2.f * fy * ty * rz3 * GJm12;
#pragma unroll
  for (int j = 0; j < 3; ++j) v_p[j] += R[0][j] * gpc0 + R[1][j] * gpc1 + R[2][j] * gpc2;
  // dL/dSigma = R^T (dL/dSc) R
  float U[3][3];  // (dL/dSc) R
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    U[0][j] = g[0] * R[0][j] + g[1] * R[1][j] + g[2] * R[2][j];
    U[1][j] = g[1] * R[0][j] + g[3] * R[1][j] + g[4] * R[2][j];
    U[2][j] = g[2] * R[0][j] + g[4] * R[1][j] + g[5] * R[2][j];
  }
  auto col = [&](int i, int j) { return R[0][i] * U[0][j] + R[1][i] * U[1][j] + R[2][i] * U[2][j]; };
  vS[0] += col(0, 0);
  vS[1] += col(0, 1);
  vS[2] += col(0, 2);
  vS[3] += col(1, 1);
  vS[4] += col(1, 2);
  vS[5] += col(2, 2);
  return true;
}
// The 59 gradients (CACHE order) of touched row t, whose table row is `r`,
// into out[0..58], the lane's own LDS row.  The row's SH coefficients are
// staged in out[11..58] and read from there by the visit loop (48 fewer
// registers), then overwritten by their gradients.
__device__ __forceinline__ void tide_row_grads(
    uint32_t t, int32_t r, const int32_t* __restrict__ visit_base,
    const int32_t* __restrict__ visits, const uint32_t* __restrict__ masks, const CamLDS& s_cam,
    uint32_t n_cams, const float* params, uint32_t row_stride, int W, int H, float eps2d,
    float near_plane, float far_plane, float radius_clip, int sh_degree,
    const float* __restrict__ splat_grads, float* out) {
  const float* row = params + (uint64_t)r * row_stride;
  const float p[3] = {row[0], row[1], row[2]};
  const float s[3] = {expf(row[3]), expf(row[4]), expf(row[5])};
  float qn[4], qinv;
  normalize4(row + 6, qn, qinv);
  const m3 Sigma = covar_from_quat_scale(qn, s);
  const float opac = sigmoidf_(row[10]);
  const float* sh = out + 11;
#pragma unroll
  for (int k = 0; k < 48; ++k) out[11 + k] = row[11 + k];

  float v_sh[48];
#pragma unroll
  for (int k = 0; k < 48; ++k) v_sh[k] = 0.f;
  float v_p[3] = {0.f, 0.f, 0.f};
  const float S6[6] = {Sigma.m[0][0], Sigma.m[0][1], Sigma.m[0][2],
                       Sigma.m[1][1], Sigma.m[1][2], Sigma.m[2][2]};
  float vS[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float v_op = 0.f;

  // visits in camera order = the set bits of the row's visibility mask
  // (cameras in lockstep across the wavefront: LDS broadcasts of the camera,
  // and the lanes seeing camera c read consecutive splat-gradient records).
  // The splat records' colour gradients are already zero where the forward
  // clamped the colour (clamp_min(SH + 0.5, 0)), so the SH colour itself is
  // not re-evaluated.
  const uint32_t mask = masks[r];
  const int32_t* vis = visits + visit_base[t];
  int j = 0;
  for (uint32_t c = 0; c < n_cams; ++c) {
    if (!((mask >> c) & 1u)) continue;
    const uint32_t e = (uint32_t)vis[j++];
    const float* g = splat_grads + (uint64_t)e * 9;
    const float vm[2] = {g[0], g[1]};
    const float vc[3] = {g[2], g[3], g[4]};
    const float vcol[3] = {g[5], g[6], g[7]};
    v_op += g[8];
    if (!tide_visit_backward(p, S6, s_cam.cam[c], s_cam.lim[c][0], s_cam.lim[c][1], eps2d,
                             near_plane, far_plane, vm, vc, v_p, vS))
      continue;
    const float dx = p[0] - s_cam.campos[c][0], dy = p[1] - s_cam.campos[c][1],
                dz = p[2] - s_cam.campos[c][2];
    // the parked coefficients are read per visit, not hoisted into registers
    asm volatile("" ::: "memory");
    float vdir[3];
    sh_vjp3<true, true>(sh_degree, dx, dy, dz, sh, vcol, v_sh, true, vdir);
#pragma unroll
    for (int k = 0; k < 3; ++k) v_p[k] += vdir[k];
  }
  m3 v_S;
  v_S.m[0][0] = vS[0];
  v_S.m[0][1] = v_S.m[1][0] = vS[1];
  v_S.m[0][2] = v_S.m[2][0] = vS[2];
  v_S.m[1][1] = vS[3];
  v_S.m[1][2] = v_S.m[2][1] = vS[4];
  v_S.m[2][2] = vS[5];
  // Sigma(q_n, s) -> (v_qn, v_s); then the activation VJPs:
  // exp: v_logscale = v_s * s; normalize: v_q = (v_qn - (v_qn.qn) qn) / max(|q|, eps);
  // sigmoid: v_logit = v_op * o * (1 - o).
  float vq[4], vs[3];
  covar_vjp_quat_scale(qn, s, v_S, vq, vs);
  const float dot = vq[0] * qn[0] + vq[1] * qn[1] + vq[2] * qn[2] + vq[3] * qn[3];
  out[0] = v_p[0];
  out[1] = v_p[1];
  out[2] = v_p[2];
  out[3] = vs[0] * s[0];
  out[4] = vs[1] * s[1];
  out[5] = vs[2] * s[2];
#pragma unroll
  for (int k = 0; k < 4; ++k) out[6 + k] = (vq[k] - dot * qn[k]) * qinv;
  out[10] = v_op * (1.f - opac) * opac;
#pragma unroll
  for (int k = 0; k < 48; ++k) out[11 + k] = v_sh[k];
}

// Odd LDS pitch of a parked row: accesses with lane = row and with lane =
// column are both free of bank conflicts.
#define ROW_PITCH 59

__global__ void __launch_bounds__(256) tide_project_bwd_kernel(
    uint32_t n_touched, const int32_t* __restrict__ touched,
    const int32_t* __restrict__ visit_base, const int32_t* __restrict__ visits,
    const uint32_t* __restrict__ masks, TideCams tc, const float* __restrict__ params,
    uint32_t row_stride, int W, int H, float eps2d, float near_plane, float far_plane,
    float radius_clip, int sh_degree, const float* __restrict__ splat_grads,
    float* __restrict__ grads, uint32_t grad_stride) {
  __shared__ CamLDS s_cam;
  __shared__ float s_g[4][64 * ROW_PITCH];
  load_cams_lds(tc, s_cam, W, H);
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t t0 = blockIdx.x * blockDim.x + (uint32_t)wv * 64u;  // the wavefront's first row
  const uint32_t t = t0 + (uint32_t)lane;
  float* sg = s_g[wv];
  if (t < n_touched)
    tide_row_grads(t, touched[t], visit_base, visits, masks, s_cam, tc.C, params, row_stride, W,
                   H, eps2d, near_plane, far_plane, radius_clip, sh_degree, splat_grads,
                   sg + lane * ROW_PITCH);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (t0 >= n_touched) return;
  const int n_w = n_touched - t0 < 64u ? (int)(n_touched - t0) : 64;
  // row by row with lane = column; the padding of a padded row is zeroed so
  // that the whole row is written
  for (int u = 0; u < n_w; ++u) {
    float* out = grads + (uint64_t)(t0 + u) * grad_stride;
    for (uint32_t k = lane; k < grad_stride; k += 64)
      out[k] = k < TIDE_ROW ? sg[u * ROW_PITCH + k] : 0.f;
  }
}

// Projection backward fused with the resident optimizer update of the same
// rows (the step's last two stages in one launch; the compact gradient rows
// never reach memory).  Phase 1 is tide_project_bwd per thread, with the
// row's 59 gradients parked in LDS (lane = row).  Phase 2 walks the
// wavefront's 64 touched rows (sorted) with lane = column: runs of up to
// FUSED_ROWS rows inside one resident block share one buffer descriptor per
// table, every row a scalar byte offset from it, and each element gets the
// resident optimizer's update (optim_update, the same as
// tgs_resident_adam_step / tgs_resident_sophia_step).  Rows are unique, so a
// row's parameters are read (phase 1) and written (phase 2) by one
// wavefront only.
#define FUSED_ROWS 32   // rows in flight per wavefront in phase 2
#define FUSED_THREADS 64  // one wavefront per workgroup: 17.8 KB of LDS, 9 per CU

struct TideOptim {
  OptimLayout L;
  const float* bias1;        // [slots] (Adam)
  const float* denom_scale;  // [slots] (Adam)
  float* m;                  // [slots * block_size, state_pitch]
  float* v;
  float lr[6];  // xyz, log-scale, quat, opacity, SH dc, SH rest (CACHE column order)
  float beta1, beta2, eps, batch_size, rho;
  int update_h;
  int state_pitch;
  int* error_flag;
};

template <bool SOPHIA, bool POW2_BS>
__global__ void __launch_bounds__(FUSED_THREADS) tide_project_bwd_optim_kernel(
    uint32_t n_touched, const int32_t* __restrict__ touched,
    const int32_t* __restrict__ visit_base, const int32_t* __restrict__ visits,
    const uint32_t* __restrict__ masks, TideCams tc, float* __restrict__ params,
    uint32_t row_stride, int W, int H, float eps2d, float near_plane, float far_plane,
    float radius_clip, int sh_degree, const float* __restrict__ splat_grads, TideOptim O) {
  __shared__ CamLDS s_cam;
  __shared__ float s_g[FUSED_THREADS / 64][64 * ROW_PITCH];
  load_cams_lds(tc, s_cam, W, H);
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t t0 = blockIdx.x * blockDim.x + (uint32_t)wv * 64u;  // the wavefront's first row
  const uint32_t t = t0 + (uint32_t)lane;
  float* sg = s_g[wv];
  int32_t my_row = 0;
  if (t < n_touched) {
    my_row = touched[t];
    tide_row_grads(t, my_row, visit_base, visits, masks, s_cam, tc.C, params, row_stride, W, H,
                   eps2d, near_plane, far_plane, radius_clip, sh_degree, splat_grads,
                   sg + lane * ROW_PITCH);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (t0 >= n_touched) return;
  const int n_w = n_touched - t0 < 64u ? (int)(n_touched - t0) : 64;

  const bool act = lane < TIDE_ROW;
  const int PW = (int)row_stride, SW = O.state_pitch;
  const int64_t PB = (int64_t)PW * 4, SB = (int64_t)SW * 4;
  const uint32_t voff_p = lane < PW ? (uint32_t)lane * 4u : TGS_OFF_NONE;
  const uint32_t voff_s = lane < SW ? (uint32_t)lane * 4u : TGS_OFF_NONE;
  const int comp = lane < 3 ? 0 : lane < 6 ? 1 : lane < 10 ? 2 : lane < 11 ? 3 : lane < 14 ? 4 : 5;
  const float lr_lane = act ? O.lr[comp] : 0.f;
  const float one_m_b1 = 1.0f - O.beta1;
  const float one_m_b2 = 1.0f - O.beta2;
  // a run is a prefix of strictly increasing rows inside one resident block
  const int32_t prev_row = __shfl_up(my_row, 1);
  const bool rising = lane == 0 || my_row > prev_row;
  BlockCache bc;
  for (int u0 = 0; u0 < n_w;) {
    const int n = n_w - u0 < FUSED_ROWS ? n_w - u0 : FUSED_ROWS;
    const int64_t r_first = (int64_t)__builtin_amdgcn_readlane(my_row, u0);
    if (!bc.lookup(O.L, r_first)) {
      // a touched row outside every resident block: the host checks this flag
      // and raises (the reference raises on a missing slot,
      // gpu_resident_optimizer.py:275-279); the row keeps its values
      if (lane == 0) atomicOr(O.error_flag, 1);
      ++u0;
      continue;
    }
    // the leading rows from u0 that rise and lie in this block
    const bool in_run = lane >= u0 && lane < u0 + n && (int64_t)my_row < bc.end &&
                        (lane == u0 || rising);
    const int k = __builtin_ctzll(~(__ballot(in_run) >> u0));  // >= 1: lane u0 is in
    const int64_t r_last = (int64_t)__builtin_amdgcn_readlane(my_row, u0 + k - 1);
    const int64_t span = r_last - r_first + 1;
    const int64_t srow = bc.slot * O.L.block_size + (r_first - bc.start);
    const auto rp = tgs_rsrc(params + r_first * PW, span * PB);
    const auto rm = tgs_rsrc(O.m + srow * SW, span * SB);
    const auto rv = tgs_rsrc(O.v + srow * SW, span * SB);
    const float sc = SOPHIA ? lr_lane : lr_lane / tgs_readlane_f32(O.bias1[bc.slot], 0);
    const float dsc = SOPHIA ? 1.f : tgs_readlane_f32(O.denom_scale[bc.slot], 0);
    float gv[FUSED_ROWS], mv[FUSED_ROWS], vv[FUSED_ROWS], pv[FUSED_ROWS];
#pragma unroll
    for (int u = 0; u < FUSED_ROWS; ++u) {
      if (u < k) {
        const uint32_t d = (uint32_t)(__builtin_amdgcn_readlane(my_row, u0 + u) - (int32_t)r_first);
        gv[u] = act ? sg[(u0 + u) * ROW_PITCH + lane] : 0.f;
        mv[u] = tgs_bload_nt(rm, voff_s, d * (uint32_t)SB);
        vv[u] = tgs_bload_nt(rv, voff_s, d * (uint32_t)SB);
        pv[u] = tgs_bload(rp, voff_p, d * (uint32_t)PB);
      }
    }
#pragma unroll
    for (int u = 0; u < FUSED_ROWS; ++u) {
      if (u < k) {
        const uint32_t d = (uint32_t)(__builtin_amdgcn_readlane(my_row, u0 + u) - (int32_t)r_first);
        float m1 = mv[u], v1 = vv[u], p1 = pv[u];
        optim_update<SOPHIA, POW2_BS>(gv[u], m1, v1, p1, sc, dsc, O.beta1, O.beta2, one_m_b1, one_m_b2,
                             O.eps, O.batch_size, O.rho, O.update_h);
        tgs_bstore_nt(act ? m1 : mv[u], rm, voff_s, d * (uint32_t)SB);
        tgs_bstore_nt(act ? v1 : vv[u], rv, voff_s, d * (uint32_t)SB);
        tgs_bstore_nt(act ? p1 : pv[u], rp, voff_p, d * (uint32_t)PB);
      }
    }
    u0 += k;
  }
}

// Camera centres: the translation of inverse(viewmat) for an affine world->camera
// matrix [A | t; 0 0 0 1], i.e. -A^{-1} t (engine.py:459 via the SH
// directions), evaluated in double from the adjugate.
__global__ void tide_camera_centers_kernel(uint32_t C, const float* __restrict__ viewmats,
                                           float* __restrict__ campos) {
  const uint32_t c = threadIdx.x;
  if (c >= C) return;
  const float* M = viewmats + (uint64_t)c * 16;
  double a[3][3], t[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
#pragma unroll
    for (int j = 0; j < 3; ++j) a[i][j] = M[i * 4 + j];
    t[i] = M[i * 4 + 3];
  }
  double adj[3][3];
  adj[0][0] = a[1][1] * a[2][2] - a[1][2] * a[2][1];
  adj[0][1] = a[0][2] * a[2][1] - a[0][1] * a[2][2];
  adj[0][2] = a[0][1] * a[1][2] - a[0][2] * a[1][1];
  adj[1][0] = a[1][2] * a[2][0] - a[1][0] * a[2][2];
  adj[1][1] = a[0][0] * a[2][2] - a[0][2] * a[2][0];
  adj[1][2] = a[0][2] * a[1][0] - a[0][0] * a[1][2];
  adj[2][0] = a[1][0] * a[2][1] - a[1][1] * a[2][0];
  adj[2][1] = a[0][1] * a[2][0] - a[0][0] * a[2][1];
  adj[2][2] = a[0][0] * a[1][1] - a[0][1] * a[1][0];
  const double det = a[0][0] * adj[0][0] + a[0][1] * adj[1][0] + a[0][2] * adj[2][0];
#pragma unroll
  for (int i = 0; i < 3; ++i)
    campos[c * 3 + i] = (float)(-(adj[i][0] * t[0] + adj[i][1] * t[1] + adj[i][2] * t[2]) / det);
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
static int check_cams(uint32_t C) {
  TGS_CHECK_ARG(C >= 1 && C <= TIDE_MAX_CAMS, "tide step: 1..%d cameras per batch (got %u)",
                TIDE_MAX_CAMS, C);
  return TGS_OK;
}

extern "C" int tgs_tide_camera_centers(uint32_t C, const float* viewmats, float* campos,
                                       hipStream_t stream) {
  int rc = check_cams(C);
  if (rc) return rc;
  TGS_CHECK_ARG(viewmats && campos, "tide_camera_centers: null");
  hipLaunchKernelGGL(tide_camera_centers_kernel, dim3(1), dim3(64), 0, stream, C, viewmats, campos);
  TGS_RETURN_LAUNCH("tgs_tide_camera_centers");
}

extern "C" uint32_t tgs_tide_row_blocks(uint64_t n_rows) {
  return (uint32_t)((n_rows + VIS_THREADS - 1) / VIS_THREADS);
}

extern "C" int tgs_tide_visibility(uint64_t n_rows, const float* params, uint32_t row_stride,
                                   uint32_t C,
                                   const float* viewmats, const float* Ks, const float* campos,
                                   int32_t W, int32_t H, float eps2d, float near_plane,
                                   float far_plane, float radius_clip, uint32_t* masks,
                                   uint32_t* counts, uint32_t* depth_range, hipStream_t stream) {
  int rc = check_cams(C);
  if (rc) return rc;
  if (depth_range)
    hipLaunchKernelGGL(tide_range_init_kernel, dim3(1), dim3(2 * TIDE_RANGE_SLOTS), 0, stream,
                       depth_range);
  if (n_rows == 0) TGS_RETURN_LAUNCH("tgs_tide_visibility");
  TGS_CHECK_ARG(params && viewmats && Ks && campos && masks && counts, "tide_visibility: null");
  TGS_CHECK_ARG(n_rows < (1ull << 31), "tide_visibility: at most 2^31-1 rows");
  TGS_CHECK_ARG(row_stride >= TIDE_ROW, "tide step: row_stride must be >= %d", TIDE_ROW);
  TideCams tc{viewmats, Ks, campos, C};
  hipLaunchKernelGGL(tide_visibility_kernel, dim3(tgs_tide_row_blocks(n_rows)), dim3(VIS_THREADS),
                     0, stream, n_rows, params, row_stride, tc, W, H, eps2d, near_plane, far_plane,
                     radius_clip, masks, counts, depth_range);
  TGS_RETURN_LAUNCH("tgs_tide_visibility");
}

extern "C" int tgs_tide_compact(uint64_t n_rows, uint32_t C, const uint32_t* masks,
                                const uint32_t* counts, const uint32_t* offs, int32_t* entries,
                                int32_t* touched, int32_t* visit_base, int32_t* visits,
                                uint32_t* totals, int32_t* cam_offsets, hipStream_t stream) {
  int rc = check_cams(C);
  if (rc) return rc;
  if (n_rows == 0) return TGS_OK;
  TGS_CHECK_ARG(masks && counts && offs && entries && touched && visit_base && visits && totals &&
                    cam_offsets,
                "tide_compact: null");
  const uint32_t nb = tgs_tide_row_blocks(n_rows);
  hipLaunchKernelGGL(tide_compact_kernel, dim3(nb), dim3(VIS_THREADS),
                     (size_t)VIS_THREADS * C * sizeof(uint32_t), stream, n_rows, C, masks, offs,
                     entries, touched, visit_base, visits, totals);
  TGS_LAUNCH_CHECK("tgs_tide_compact");
  hipLaunchKernelGGL(tide_totals_kernel, dim3(1), dim3(64), 0, stream, C, nb, counts, offs,
                     totals, cam_offsets, visit_base);
  TGS_RETURN_LAUNCH("tgs_tide_compact");
}

extern "C" int tgs_tide_project_fwd(uint32_t n_touched, const uint32_t* n_touched_dev,
                                    const int32_t* touched,
                                    const int32_t* visit_base, const int32_t* visits,
                                    const uint32_t* masks, uint32_t C, const float* params,
                                    uint32_t row_stride, const float* viewmats, const float* Ks,
                                    const float* campos, int32_t W, int32_t H, float eps2d,
                                    float near_plane, float far_plane, float radius_clip,
                                    int32_t sh_degree, uint32_t tile_size, uint32_t tile_width,
                                    uint32_t tile_height,
                                    float* splats, uint32_t* depth_keys, uint64_t* entry_rects,
                                    int64_t* isect_totals, uint32_t* depth_range,
                                    hipStream_t stream) {
  int rc = check_cams(C);
  if (rc) return rc;
  if (isect_totals)
    hipLaunchKernelGGL(tide_zero_i64_kernel, dim3(1), dim3(64), 0, stream, isect_totals, C);
  if (depth_range)
    hipLaunchKernelGGL(tide_range_init_kernel, dim3(1), dim3(2 * TIDE_RANGE_SLOTS), 0, stream,
                       depth_range);
  if (n_touched == 0) TGS_RETURN_LAUNCH("tgs_tide_project_fwd");
  TGS_CHECK_ARG(touched && visit_base && visits && masks && params && viewmats && Ks && campos &&
                    splats && depth_keys && entry_rects,
                "tide_project_fwd: null");
  TGS_CHECK_ARG(tile_width >= 1 && tile_width <= 255 && tile_height >= 1 && tile_height <= 255,
                "tide step: tile grid must be at most 255 x 255 tiles (got %u x %u)", tile_width,
                tile_height);
  TGS_CHECK_ARG(sh_degree >= 0 && sh_degree <= 3, "tide step: sh_degree must be in [0,3]");
  TGS_CHECK_ARG(((uintptr_t)splats & 15) == 0, "tide_project_fwd: splats must be 16-byte aligned");
  TGS_CHECK_ARG(row_stride >= TIDE_ROW, "tide step: row_stride must be >= %d", TIDE_ROW);
  TideCams tc{viewmats, Ks, campos, C};
  hipLaunchKernelGGL(tide_project_fwd_kernel, dim3(tgs_blocks(n_touched, 256)), dim3(256), 0,
                     stream, n_touched, n_touched_dev, touched, visit_base, visits, masks, tc,
                     params, row_stride,
                     W, H,
                     eps2d, near_plane, far_plane, radius_clip, sh_degree, tile_size, tile_width,
                     tile_height, (float4*)splats, depth_keys, entry_rects, isect_totals,
                     depth_range);
  TGS_RETURN_LAUNCH("tgs_tide_project_fwd");
}


extern "C" int tgs_tide_isect_count(uint32_t n_entries, const uint64_t* entry_rects,
                                    int32_t* tiles, hipStream_t stream) {
  if (n_entries == 0) return TGS_OK;
  TGS_CHECK_ARG(entry_rects && tiles, "tide_isect_count: null");
  hipLaunchKernelGGL(tide_isect_count_kernel, dim3(tgs_blocks(n_entries, 256)), dim3(256), 0,
                     stream, n_entries, entry_rects, tiles);
  TGS_RETURN_LAUNCH("tgs_tide_isect_count");
}

extern "C" int tgs_tide_isect_totals(uint32_t n_entries, const uint32_t* n_entries_dev,
                                     const uint64_t* entry_rects, const int32_t* cam_offsets,
                                     uint32_t C, int64_t* isect_totals, hipStream_t stream) {
  int rc = check_cams(C);
  if (rc) return rc;
  TGS_CHECK_ARG(isect_totals && cam_offsets, "tide_isect_totals: null");
  hipLaunchKernelGGL(tide_zero_i64_kernel, dim3(1), dim3(64), 0, stream, isect_totals, C);
  if (n_entries == 0) TGS_RETURN_LAUNCH("tgs_tide_isect_totals");
  TGS_CHECK_ARG(entry_rects != nullptr, "tide_isect_totals: null rects");
  const uint64_t blocks = ((uint64_t)n_entries + ISECT_TOTAL_PER_BLOCK - 1) / ISECT_TOTAL_PER_BLOCK;
  hipLaunchKernelGGL(tide_isect_totals_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     n_entries, n_entries_dev, entry_rects, cam_offsets, C, isect_totals);
  TGS_RETURN_LAUNCH("tgs_tide_isect_totals");
}

extern "C" int tgs_tide_isect_segments(uint32_t C, const int32_t* cam_offsets,
                                       const int64_t* cum_tiles, int64_t* seg,
                                       hipStream_t stream) {
  int rc = check_cams(C);
  if (rc) return rc;
  TGS_CHECK_ARG(cam_offsets && cum_tiles && seg, "tide_isect_segments: null");
  hipLaunchKernelGGL(tide_isect_segments_kernel, dim3(1), dim3(64), 0, stream, C, cam_offsets,
                     cum_tiles, seg);
  TGS_RETURN_LAUNCH("tgs_tide_isect_segments");
}

extern "C" int tgs_tide_isect_emit(uint32_t n_entries, const int32_t* cam_offsets, uint32_t C,
                                   const uint64_t* entry_rects, const int64_t* cum_tiles,
                                   uint32_t tile_width, uint32_t tile_n_bits, uint32_t* keys,
                                   int32_t* flatten_ids, hipStream_t stream) {
  int rc = check_cams(C);
  if (rc) return rc;
  if (n_entries == 0) return TGS_OK;
  TGS_CHECK_ARG(cam_offsets && entry_rects && cum_tiles && keys && flatten_ids,
                "tide_isect_emit: null");
  TGS_CHECK_ARG(tile_n_bits <= 16, "tide_isect_emit: tile_n_bits must be <= 16");
  hipLaunchKernelGGL(tide_isect_emit_kernel, dim3(tgs_blocks(n_entries, 256)), dim3(256), 0,
                     stream, n_entries, cam_offsets, C, entry_rects, cum_tiles, tile_width,
                     tile_n_bits, keys, flatten_ids);
  TGS_RETURN_LAUNCH("tgs_tide_isect_emit");
}

extern "C" uint32_t tgs_tide_isect_emit_blocks(uint32_t n_entries) {
  return (uint32_t)(((uint64_t)n_entries + EMIT_ENTRIES - 1) / EMIT_ENTRIES);
}

extern "C" int tgs_tide_isect_block_sums(uint32_t n_entries, const uint64_t* entry_rects,
                                         uint32_t* block_sums, hipStream_t stream) {
  if (n_entries == 0) return TGS_OK;
  TGS_CHECK_ARG(entry_rects && block_sums, "tide_isect_block_sums: null");
  hipLaunchKernelGGL(tide_isect_block_sums_kernel, dim3(tgs_tide_isect_emit_blocks(n_entries)),
                     dim3(256), 0, stream, n_entries, entry_rects, block_sums);
  TGS_RETURN_LAUNCH("tgs_tide_isect_block_sums");
}

extern "C" int tgs_tide_isect_emit_blocked(uint32_t n_entries, const int32_t* cam_offsets,
                                           uint32_t C, const uint64_t* entry_rects,
                                           const uint32_t* block_base, uint32_t tile_width,
                                           uint32_t tile_n_bits, uint32_t* keys,
                                           int32_t* flatten_ids, hipStream_t stream) {
  int rc = check_cams(C);
  if (rc) return rc;
  if (n_entries == 0) return TGS_OK;
  TGS_CHECK_ARG(cam_offsets && entry_rects && block_base && keys && flatten_ids,
                "tide_isect_emit_blocked: null");
  TGS_CHECK_ARG(tile_n_bits <= 16, "tide_isect_emit_blocked: tile_n_bits must be <= 16");
  hipLaunchKernelGGL(tide_isect_emit_blocked_kernel<false>,
                     dim3(tgs_tide_isect_emit_blocks(n_entries)), dim3(256), 0, stream, n_entries,
                     cam_offsets, C, entry_rects, block_base, tile_width, tile_n_bits, keys,
                     flatten_ids, EmitHist{});
  TGS_RETURN_LAUNCH("tgs_tide_isect_emit_blocked");
}

extern "C" int tgs_tide_isect_emit_blocked_hist(
    uint32_t n_entries, const int32_t* cam_offsets, uint32_t C, const uint64_t* entry_rects,
    const uint32_t* block_base, uint32_t tile_width, uint32_t tile_n_bits, uint32_t* keys,
    int32_t* flatten_ids, const uint32_t* isect_cam_offsets, uint32_t* hist,
    uint64_t hist_words, hipStream_t stream) {
  int rc = check_cams(C);
  if (rc) return rc;
  TGS_CHECK_ARG(cam_offsets && entry_rects && block_base && keys && flatten_ids &&
                    isect_cam_offsets && hist,
                "tide_isect_emit_blocked_hist: null");
  TGS_CHECK_ARG(tile_n_bits >= 1 && tile_n_bits <= 16,
                "tide_isect_emit_blocked_hist: tile_n_bits must be in [1, 16]");
  EmitHist eh{};
  eh.hist = hist;
  // the sort's first pass over bits [0, tile_n_bits): ceil(bits / 8) passes
  // of ceil(bits / passes) bits (the split tgs_segmented_sort_pairs_u32_hist0
  // makes)
  const uint32_t passes = (tile_n_bits + 7) / 8;
  eh.mask = (1u << ((tile_n_bits + passes - 1) / passes)) - 1u;
  uint32_t tiles = 0;
  for (uint32_t c = 0; c <= C; ++c) {
    TGS_CHECK_ARG(c == 0 || isect_cam_offsets[c] >= isect_cam_offsets[c - 1],
                  "tide_isect_emit_blocked_hist: offsets decrease");
    eh.seg_start[c] = isect_cam_offsets[c];
    eh.tile_base[c] = tiles;
    if (c < C)
      tiles += (isect_cam_offsets[c + 1] - isect_cam_offsets[c] + EMIT_SORT_TILE - 1) /
               EMIT_SORT_TILE;
  }
  const uint64_t words = (uint64_t)tiles * 256u;
  TGS_CHECK_ARG(words <= hist_words, "tide_isect_emit_blocked_hist: histogram buffer too small");
  eh.words = words;
  if (words) {
    hipLaunchKernelGGL(tide_zero_u32_kernel, dim3((unsigned)((words + 255) / 256 < 4096 ? (words + 255) / 256 : 4096)),
                       dim3(256), 0, stream, hist, words);
    TGS_LAUNCH_CHECK("tide_zero_u32");
  }
  if (n_entries == 0) return TGS_OK;
  hipLaunchKernelGGL(tide_isect_emit_blocked_kernel<true>,
                     dim3(tgs_tide_isect_emit_blocks(n_entries)), dim3(256), 0, stream, n_entries,
                     cam_offsets, C, entry_rects, block_base, tile_width, tile_n_bits, keys,
                     flatten_ids, eh);
  TGS_RETURN_LAUNCH("tgs_tide_isect_emit_blocked_hist");
}

// First-pass digit width of the tile-bit sort over tile_n_bits bits: the bits
// split into ceil(bits / 8) passes of ceil(bits / passes) bits.
extern "C" uint32_t tgs_tide_isect_fused_digit_bits(uint32_t tile_n_bits) {
  if (tile_n_bits == 0) return 0;
  const uint32_t passes = (tile_n_bits + 7) / 8;
  return (tile_n_bits + passes - 1) / passes;
}

static int fused_emit_setup(uint32_t C, const uint32_t* cam_offsets, uint32_t tile_width,
                            uint32_t tile_n_bits, FusedEmit& fe, uint32_t& n_blocks,
                            const char* who) {
  int rc = check_cams(C);
  if (rc) return rc;
  TGS_CHECK_ARG(cam_offsets, "%s: null camera offsets", who);
  TGS_CHECK_ARG(tile_n_bits >= 1 && tile_n_bits <= 16, "%s: tile_n_bits must be in [1, 16]", who);
  TGS_CHECK_ARG(tile_width >= 1 && tile_width <= 255, "%s: tile_width must be in [1, 255]", who);
  fe = FusedEmit{};
  fe.C = C;
  fe.tw = tile_width;
  fe.tile_n_bits = tile_n_bits;
  fe.mask = (1u << tgs_tide_isect_fused_digit_bits(tile_n_bits)) - 1u;
  uint64_t blocks = 0;
  for (uint32_t c = 0; c <= C; ++c) {
    TGS_CHECK_ARG(c == 0 || cam_offsets[c] >= cam_offsets[c - 1], "%s: camera offsets decrease",
                  who);
    fe.ent_off[c] = cam_offsets[c];
    fe.blk_first[c] = (uint32_t)blocks;
    if (c < C) blocks += (cam_offsets[c + 1] - cam_offsets[c] + FE_ENTRIES - 1) / FE_ENTRIES;
  }
  TGS_CHECK_ARG(blocks < (1ull << 31), "%s: too many entry blocks", who);
  n_blocks = (uint32_t)blocks;
  return TGS_OK;
}

extern "C" uint64_t tgs_tide_isect_fused_hist_words(uint32_t C, const uint32_t* cam_offsets,
                                                    uint32_t tile_n_bits) {
  FusedEmit fe;
  uint32_t nb = 0;
  if (fused_emit_setup(C, cam_offsets, 1, tile_n_bits, fe, nb, "tide_isect_fused_hist_words"))
    return 0;
  return (uint64_t)nb * (fe.mask + 1u);
}

extern "C" int tgs_tide_isect_fused_count(uint32_t C, const uint32_t* cam_offsets,
                                          const uint64_t* entry_rects, uint32_t tile_width,
                                          uint32_t tile_n_bits, uint32_t* hist,
                                          uint64_t hist_words, hipStream_t stream) {
  FusedEmit fe;
  uint32_t nb = 0;
  int rc = fused_emit_setup(C, cam_offsets, tile_width, tile_n_bits, fe, nb,
                            "tide_isect_fused_count");
  if (rc) return rc;
  if (nb == 0) return TGS_OK;
  TGS_CHECK_ARG(entry_rects && hist, "tide_isect_fused_count: null");
  TGS_CHECK_ARG((uint64_t)nb * (fe.mask + 1u) <= hist_words,
                "tide_isect_fused_count: histogram buffer too small");
  hipLaunchKernelGGL(tide_isect_fused_count_kernel, dim3(nb), dim3(256), 0, stream, fe, entry_rects,
                     hist);
  TGS_RETURN_LAUNCH("tgs_tide_isect_fused_count");
}

extern "C" int tgs_tide_isect_fused_scatter(uint32_t C, const uint32_t* cam_offsets,
                                            const uint64_t* entry_rects, uint32_t tile_width,
                                            uint32_t tile_n_bits, const uint32_t* hist_scan,
                                            uint64_t hist_words, uint32_t n_isects,
                                            uint32_t* keys, int32_t* flatten_ids,
                                            hipStream_t stream) {
  FusedEmit fe;
  uint32_t nb = 0;
  int rc = fused_emit_setup(C, cam_offsets, tile_width, tile_n_bits, fe, nb,
                            "tide_isect_fused_scatter");
  if (rc) return rc;
  if (nb == 0 || n_isects == 0) return TGS_OK;
  TGS_CHECK_ARG(entry_rects && hist_scan && keys && flatten_ids, "tide_isect_fused_scatter: null");
  TGS_CHECK_ARG((uint64_t)nb * (fe.mask + 1u) <= hist_words,
                "tide_isect_fused_scatter: histogram buffer too small");
  TGS_CHECK_ARG(C - 1 < (1u << (32 - tile_n_bits)),
                "tide_isect_fused_scatter: camera | tile keys do not fit 32 bits");
  hipLaunchKernelGGL(tide_isect_fused_scatter_kernel, dim3(nb), dim3(256), 0, stream, fe,
                     entry_rects, hist_scan, n_isects, keys, flatten_ids);
  TGS_RETURN_LAUNCH("tgs_tide_isect_fused_scatter");
}

extern "C" int tgs_tide_offset_encode(uint32_t n_isects, const uint32_t* keys, uint32_t C,
                                      uint32_t tile_width, uint32_t tile_height,
                                      uint32_t tile_n_bits, int32_t* offsets,
                                      hipStream_t stream) {
  const uint64_t total = (uint64_t)C * tile_width * tile_height;
  if (total == 0) return TGS_OK;
  TGS_CHECK_ARG(offsets && (n_isects == 0 || keys), "tide_offset_encode: null");
  TGS_CHECK_ARG(total < (1ull << 31), "tide_offset_encode: too many buckets");
  if (n_isects == 0) return tgs_fill_u32(offsets, total, 0u, stream);
  TGS_CHECK_ARG(tile_n_bits < 32 && (uint64_t)tile_width * tile_height <= (1ull << tile_n_bits) &&
                    ((uint64_t)(C - 1) << tile_n_bits) < (1ull << 32),
                "tide_offset_encode: camera | tile keys do not fit 32 bits");
  uint32_t top = 1u;
  while (top <= n_isects / 2u) top <<= 1;
  hipLaunchKernelGGL(tide_offset_search_kernel, dim3(tgs_blocks(total, 256)), dim3(256), 0, stream,
                     n_isects, keys, (uint32_t)total, tile_width * tile_height, tile_n_bits, top,
                     offsets);
  TGS_RETURN_LAUNCH("tgs_tide_offset_encode");
}

extern "C" int tgs_tide_isect_ids(uint32_t n_isects, const uint32_t* keys,
                                  const int32_t* flatten_ids, const float* splats,
                                  int64_t* isect_ids, hipStream_t stream) {
  if (n_isects == 0) return TGS_OK;
  TGS_CHECK_ARG(keys && flatten_ids && splats && isect_ids, "tide_isect_ids: null");
  hipLaunchKernelGGL(tide_isect_ids_kernel, dim3(tgs_blocks(n_isects, 256)), dim3(256), 0, stream,
                     n_isects, keys, flatten_ids, (const float4*)splats, isect_ids);
  TGS_RETURN_LAUNCH("tgs_tide_isect_ids");
}

extern "C" int tgs_tide_rasterize_fwd(uint32_t C, const float* splats, const float* backgrounds,
                                      uint32_t W, uint32_t H, uint32_t tile_width,
                                      uint32_t tile_height, const int32_t* tile_offsets,
                                      const int32_t* flatten_ids, uint32_t n_isects,
                                      float* images, float* alphas, int32_t* last_ids,
                                      int32_t* n_contrib, float* clear, uint64_t clear_words,
                                      hipStream_t stream) {
  TGS_CHECK_ARG(clear_words % 4 == 0 && (clear_words == 0 || clear) &&
                    ((uintptr_t)clear & 15u) == 0,
                "tide_rasterize_fwd: clear needs a 16-byte aligned buffer of 4k words");
  if (C == 0 || W == 0 || H == 0) return clear_words ? tgs_fill_u32(clear, clear_words, 0u, stream)
                                                     : TGS_OK;
  TGS_CHECK_ARG(tile_offsets && images && alphas && last_ids, "tide_rasterize_fwd: null");
  TGS_CHECK_ARG(n_isects == 0 || (splats && flatten_ids), "tide_rasterize_fwd: null splats");
  TGS_CHECK_ARG(tile_width * 16 >= W && tile_height * 16 >= H, "tide_rasterize_fwd: tile grid");
  TGS_CHECK_ARG(C <= 65535 && tile_width <= 65535 && tile_height <= 65535,
                "tide_rasterize_fwd: at most 65535 cameras and tiles per image side");
  const RasterGeom G{C, W, H, tile_width, tile_height, n_isects};
  if (n_contrib)
    hipLaunchKernelGGL((raster_fwd_kernel<3, 16, PackedSplats, true>), raster_fwd_grid(G),
                       dim3(256), 0, stream, G, PackedSplats{(const float4*)splats}, backgrounds,
                       tile_offsets, flatten_ids, images, alphas, last_ids, (float4*)clear,
                       (uint64_t)clear_words / 4, n_contrib);
  else
    hipLaunchKernelGGL((raster_fwd_kernel<3, 16, PackedSplats>), raster_fwd_grid(G), dim3(256), 0,
                       stream, G, PackedSplats{(const float4*)splats}, backgrounds,
                       tile_offsets, flatten_ids, images, alphas, last_ids, (float4*)clear,
                       (uint64_t)clear_words / 4, nullptr);
  TGS_RETURN_LAUNCH("tgs_tide_rasterize_fwd");
}

extern "C" int tgs_tide_rasterize_bwd(uint32_t C, const float* splats, const float* backgrounds,
                                      uint32_t W, uint32_t H, uint32_t tile_width,
                                      uint32_t tile_height, const int32_t* tile_offsets,
                                      const int32_t* flatten_ids, uint32_t n_isects,
                                      const float* alphas, const int32_t* last_ids,
                                      const float* v_images, const float* v_alphas,
                                      float* splat_grads, hipStream_t stream) {
  if (C == 0 || W == 0 || H == 0 || n_isects == 0) return TGS_OK;
  TGS_CHECK_ARG(splats && tile_offsets && flatten_ids && alphas && last_ids && v_images &&
                    splat_grads,
                "tide_rasterize_bwd: null");
  TGS_CHECK_ARG(tile_width * 16 >= W && tile_height * 16 >= H, "tide_rasterize_bwd: tile grid");
  TGS_CHECK_ARG(C <= 65535 && tile_width <= 65535 && tile_height <= 65535,
                "tide_rasterize_bwd: at most 65535 cameras and tiles per image side");
  const RasterGeom G{C, W, H, tile_width, tile_height, n_isects};
  hipLaunchKernelGGL((raster_bwd_kernel<3, 16, PackedSplats, PackedGrads>), raster_bwd_grid(G),
                     dim3(256), 0, stream, G,
                     PackedSplats{(const float4*)splats}, PackedGrads{splat_grads}, backgrounds,
                     tile_offsets, flatten_ids, alphas, last_ids, v_images, v_alphas);
  TGS_RETURN_LAUNCH("tgs_tide_rasterize_bwd");
}

extern "C" int tgs_tide_project_bwd_update(
    uint32_t n_touched, const int32_t* touched, const int32_t* visit_base, const int32_t* visits,
    const uint32_t* masks, uint32_t C, float* params, uint32_t row_stride, const float* viewmats,
    const float* Ks, const float* campos, int32_t W, int32_t H, float eps2d, float near_plane,
    float far_plane, float radius_clip, int32_t sh_degree, const float* splat_grads,
    const int64_t* block_starts, const int64_t* block_ends, const int64_t* block_slots,
    int64_t n_layout, int64_t block_size, const float* bias_correction1, const float* denom_scale,
    float* exp_avg, float* exp_avg_sq, uint32_t state_pitch, const float* lrs, int32_t optimizer,
    float beta1, float beta2, float eps, float batch_size, float rho, int32_t update_hessian,
    int32_t* error_flag, hipStream_t stream) {
  const char* name = "tgs_tide_project_bwd_update";
  int rc = check_cams(C);
  if (rc) return rc;
  TGS_CHECK_ARG(optimizer == 0 || optimizer == 1, "%s: optimizer must be 0 (Adam) or 1 (Sophia)",
                name);
  if (n_touched == 0) return TGS_OK;
  TGS_CHECK_ARG(touched && visit_base && visits && masks && params && viewmats && Ks && campos &&
                    splat_grads && block_starts && block_ends && block_slots && exp_avg &&
                    exp_avg_sq && lrs && error_flag,
                "%s: null", name);
  TGS_CHECK_ARG(optimizer == 1 || (bias_correction1 && denom_scale), "%s: null bias table", name);
  TGS_CHECK_ARG(sh_degree >= 0 && sh_degree <= 3, "tide step: sh_degree must be in [0,3]");
  TGS_CHECK_ARG(row_stride >= TIDE_ROW && row_stride <= 64 && state_pitch >= TIDE_ROW &&
                    state_pitch <= 64,
                "%s: row_stride and state_pitch must be in [%d, 64]", name, TIDE_ROW);
  // a run of rows inside one block is addressed by 32-bit byte offsets
  TGS_CHECK_ARG(n_layout >= 1 && block_size >= 1 && block_size <= (1 << 22),
                "%s: need a non-empty layout and 1 <= block_size <= 2^22", name);
  int shift = -1;
  if ((block_size & (block_size - 1)) == 0)
    for (shift = 0; ((int64_t)1 << shift) < block_size; ++shift) {
    }
  TideCams tc{viewmats, Ks, campos, C};
  TideOptim O;
  O.L = OptimLayout{block_starts, block_ends, block_slots, n_layout, block_size, shift};
  O.bias1 = bias_correction1;
  O.denom_scale = denom_scale;
  O.m = exp_avg;
  O.v = exp_avg_sq;
  for (int k = 0; k < 6; ++k) O.lr[k] = lrs[k];
  O.beta1 = beta1;
  O.beta2 = beta2;
  O.eps = eps;
  O.batch_size = batch_size;
  O.rho = rho;
  O.update_h = update_hessian;
  O.state_pitch = (int)state_pitch;
  O.error_flag = error_flag;
#define TIDE_FUSED_LAUNCH(SOPHIA, POW2)                                                          \
  hipLaunchKernelGGL((tide_project_bwd_optim_kernel<SOPHIA, POW2>),                              \
                     dim3(tgs_blocks(n_touched, FUSED_THREADS)), dim3(FUSED_THREADS), 0, stream, \
                     n_touched, touched, visit_base, visits, masks, tc, params, row_stride, W, H, \
                     eps2d, near_plane, far_plane, radius_clip, sh_degree, splat_grads, O)
  int bs_exp = 0;
  const bool pow2 = batch_size > 0.f && std::frexp(batch_size, &bs_exp) == 0.5f;
  if (optimizer == 1) {
    if (pow2) TIDE_FUSED_LAUNCH(true, true);
    else TIDE_FUSED_LAUNCH(true, false);
  } else {
    if (pow2) TIDE_FUSED_LAUNCH(false, true);
    else TIDE_FUSED_LAUNCH(false, false);
  }
#undef TIDE_FUSED_LAUNCH
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_tide_project_bwd(uint32_t n_touched, const int32_t* touched,
                                    const int32_t* visit_base, const int32_t* visits,
                                    const uint32_t* masks, uint32_t C, const float* params,
                                    uint32_t row_stride, const float* viewmats, const float* Ks,
                                    const float* campos, int32_t W, int32_t H, float eps2d,
                                    float near_plane, float far_plane, float radius_clip,
                                    int32_t sh_degree, const float* splat_grads, float* grads,
                                    uint32_t grad_stride, hipStream_t stream) {
  int rc = check_cams(C);
  if (rc) return rc;
  if (n_touched == 0) return TGS_OK;
  TGS_CHECK_ARG(touched && visit_base && visits && masks && params && viewmats && Ks && campos &&
                    splat_grads && grads,
                "tide_project_bwd: null");
  TGS_CHECK_ARG(sh_degree >= 0 && sh_degree <= 3, "tide step: sh_degree must be in [0,3]");
  TGS_CHECK_ARG(row_stride >= TIDE_ROW && grad_stride >= TIDE_ROW,
                "tide step: row_stride and grad_stride must be >= %d", TIDE_ROW);
  TideCams tc{viewmats, Ks, campos, C};
  hipLaunchKernelGGL(tide_project_bwd_kernel, dim3(tgs_blocks(n_touched, 256)), dim3(256), 0,
                     stream, n_touched, touched, visit_base, visits, masks, tc, params, row_stride,
                     W, H, eps2d, near_plane, far_plane, radius_clip, sh_degree, splat_grads, grads,
                     grad_stride);
  TGS_RETURN_LAUNCH("tgs_tide_project_bwd");
}
