// Fused resident-slot optimizer steps (Adam and Sophia) over touched rows.
//
// Semantics follow TideGS's GPUResidentAdam
// (strategies/tide_engine/gpu_resident_optimizer.py:16-70 kernel, :266-300 slot
// mapping, :302-337 per-slot bias tables):
//   g  = grad / batch_size
//   m  = b1*m + (1-b1)*g
//   v  = b2*v + (1-b2)*g*g
//   p -= (lr_col / bias1[slot]) * m / (sqrt(v)/denom_scale[slot] + eps)
// where a touched working-set row maps to its resident state row through the
// block layout (sorted [start,end) slices, one state slot per block):
//   pos = #ends <= row, state_row = slot[pos]*block_size + (row - start[pos]).
//
// The reference issues one Triton launch per component (6 per step) plus host
// searchsorted/index_select.  Here a single launch covers all 59 columns: one
// wavefront walks a contiguous range of touched rows, four rows in flight,
// lane l handles column l (59 of 64 lanes busy), and the row -> (slot, state
// row) lookup is a wave-uniform binary search on the scalar unit that runs
// only when the (sorted) rows cross into another resident block.  The column -> (component tensor,
// column) map is fixed per lane, so the same kernel serves six split component
// tensors or one unified [N,59] table.
//
// Sophia (no reference; Liu et al. 2023, arXiv 2305.14342, Alg. 3 with the
// per-coordinate clip of SURVEY row A14):
//   m  = b1*m + (1-b1)*g
//   h  = b2*h + (1-b2)*g*g        (only on Hessian-refresh steps)
//   p -= lr_col * clamp(m / max(h, eps), -rho, rho)

#include "tgs_common.cuh"

#define TGS_MAX_COMP 8

struct OptimComponents {
  float* param[TGS_MAX_COMP];
  const float* grad[TGS_MAX_COMP];
  float* m[TGS_MAX_COMP];
  float* v[TGS_MAX_COMP];
  int width[TGS_MAX_COMP];
  int64_t pstride[TGS_MAX_COMP];  // row strides (elements) of param, grad, state
  int64_t gstride[TGS_MAX_COMP];
  int64_t sstride[TGS_MAX_COMP];
  float lr[TGS_MAX_COMP];
  int n;
  int total;    // sum of widths
  int unified;  // components are adjacent columns of one table for param,
                // grad and both states, every row stride == total
};

struct OptimLayout {
  const int64_t* starts;  // [L] sorted ascending
  const int64_t* ends;    // [L]
  const int64_t* slots;   // [L]
  int64_t n;              // L
  int64_t block_size;
};

// Resolve lane -> (component, column); lanes beyond the total width get comp=-1.
__device__ __forceinline__ void lane_column(const OptimComponents& c, int lane, int& comp,
                                            int& col) {
  comp = -1;
  col = 0;
  int base = 0;
#pragma unroll
  for (int k = 0; k < TGS_MAX_COMP; ++k) {
    if (k < c.n) {
      if (lane >= base && lane < base + c.width[k]) {
        comp = k;
        col = lane - base;
      }
      base += c.width[k];
    }
  }
}

// Number of ends <= row (searchsorted right=True), wave-uniform.
__device__ __forceinline__ int64_t layout_search(const OptimLayout& L, int64_t row) {
  int64_t lo = 0, hi = L.n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (L.ends[mid] <= row)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// The resident block holding the current rows: [start, end) -> slot.  Touched
// rows arrive sorted, so a wavefront walking a contiguous range of them
// searches the layout only when it crosses into another block.
struct BlockCache {
  int64_t start = 0, end = 0, slot = 0;  // empty until the first lookup
  bool ok = false;
  __device__ __forceinline__ bool lookup(const OptimLayout& L, int64_t row) {
    if (row >= start && row < end) return true;
    const int64_t pos = layout_search(L, row);
    ok = false;
    start = end = 0;
    if (pos < L.n) {
      const int64_t s = L.starts[pos], e = L.ends[pos];
      if (row >= s && row < e && row - s < L.block_size) {
        start = s;
        end = e;
        slot = L.slots[pos];
        ok = true;
      }
    }
    return ok;
  }
};

#define OPT_UNROLL 4
#define OPT_RUN 64  // rows per flat-path run

template <typename IdxT, bool SOPHIA>
__global__ void __launch_bounds__(256) resident_optim_kernel(
    int64_t n_rows, const IdxT* __restrict__ local_rows, OptimLayout L,
    const float* __restrict__ bias1, const float* __restrict__ denom_scale, OptimComponents C,
    float beta1, float beta2, float eps, float batch_size, float rho, int update_h,
    int* __restrict__ error_flag) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t n_waves = (int64_t)gridDim.x * (blockDim.x >> 6);

  int comp, col;
  lane_column(C, lane, comp, col);
  const bool active = comp >= 0;
  float* param = nullptr;
  const float* grad = nullptr;
  float* m = nullptr;
  float* v = nullptr;
  int64_t pstride = 0, gstride = 0, sstride = 0;
  float lr = 0.f;
  if (active) {
    param = C.param[comp];
    grad = C.grad[comp];
    m = C.m[comp];
    v = C.v[comp];
    pstride = C.pstride[comp];
    gstride = C.gstride[comp];
    sstride = C.sstride[comp];
    lr = C.lr[comp];
  }
  const float one_m_b1 = 1.0f - beta1;
  const float one_m_b2 = 1.0f - beta2;

  // per-column learning rate (for the flat path: column -> lr)
  __shared__ float s_lr[64];
  __shared__ float s_scale[4][64];  // per wavefront: step size per column of the current run
  if (threadIdx.x < 64) s_lr[threadIdx.x] = active ? lr : 0.f;
  __syncthreads();

  // a contiguous range of touched rows per wavefront
  const int64_t per = (n_rows + n_waves - 1) / n_waves;
  const int64_t t0 = wave * per;
  const int64_t t1 = t0 + per < n_rows ? t0 + per : n_rows;
  BlockCache bc;
  int64_t t = t0;
  while (t < t1) {
    // Flat path: when the next rows are consecutive and inside one resident
    // block, param, grad and state rows of the run are each one contiguous span
    // (unified table), streamed 64 floats per instruction across row bounds.
    if (C.unified) {
      const int64_t te = t + OPT_RUN < t1 ? t + OPT_RUN : t1;
      const int64_t r0 = (int64_t)local_rows[t], rl = (int64_t)local_rows[te - 1];
      if (rl - r0 == te - 1 - t && bc.lookup(L, r0) && rl < bc.end &&
          rl - bc.start < L.block_size) {
        const int W = C.total;
        const int64_t F = (te - t) * W;
        const float* __restrict__ g = C.grad[0] + t * W;
        float* __restrict__ p = C.param[0] + r0 * W;
        const int64_t srow = bc.slot * L.block_size + (r0 - bc.start);
        float* __restrict__ mp = C.m[0] + srow * W;
        float* __restrict__ vp = C.v[0] + srow * W;
        float dsc = 1.f;
        // per-column step size lr (Adam: lr / bias1 of this slot, the
        // reference's rounding of (lr / bias1) * m)
        float* s_sc = s_scale[threadIdx.x >> 6];
        if (lane < W) s_sc[lane] = SOPHIA ? s_lr[lane] : s_lr[lane] / bias1[bc.slot];
        if (!SOPHIA) dsc = denom_scale[bc.slot];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int step = 64 % W;
        int c = lane % W;  // column of element lane + 64 k
        for (int64_t i0 = lane; i0 < F; i0 += 64 * OPT_UNROLL) {
          float gv[OPT_UNROLL], mv[OPT_UNROLL], vv[OPT_UNROLL], pv[OPT_UNROLL];
#pragma unroll
          for (int u = 0; u < OPT_UNROLL; ++u) {
            const int64_t i = i0 + 64 * u;
            if (i < F) {
              gv[u] = g[i];
              mv[u] = mp[i];
              vv[u] = vp[i];
              pv[u] = p[i];
            }
          }
#pragma unroll
          for (int u = 0; u < OPT_UNROLL; ++u) {
            const int64_t i = i0 + 64 * u;
            if (i < F) {
              const float gg = gv[u] / batch_size;
              const float m1 = beta1 * mv[u] + one_m_b1 * gg;
              float v1 = vv[u];
              float p1 = pv[u];
              const float sc = s_sc[c];
              if (SOPHIA) {
                if (update_h) v1 = beta2 * v1 + one_m_b2 * gg * gg;
                float r = m1 / fmaxf(v1, eps);
                r = fminf(fmaxf(r, -rho), rho);
                p1 -= sc * r;
              } else {
                v1 = beta2 * v1 + one_m_b2 * gg * gg;
                const float denom = sqrtf(v1) / dsc + eps;
                p1 -= sc * m1 / denom;
              }
              mp[i] = m1;
              vp[i] = v1;
              p[i] = p1;
            }
            c += step;
            if (c >= W) c -= W;
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        t = te;
        continue;
      }
    }
    // Per-row path: OPT_UNROLL rows in flight, lane = column.
    const int64_t tb = t;
    const int64_t te = tb + OPT_UNROLL < t1 ? tb + OPT_UNROLL : t1;
    int64_t poff[OPT_UNROLL], soff[OPT_UNROLL];
    float scale[OPT_UNROLL], dscale[OPT_UNROLL];
    bool live[OPT_UNROLL];
#pragma unroll
    for (int u = 0; u < OPT_UNROLL; ++u) {
      live[u] = false;
      poff[u] = soff[u] = 0;
      scale[u] = dscale[u] = 1.f;
      if (tb + u < te) {
        const int64_t row = (int64_t)local_rows[tb + u];
        if (bc.lookup(L, row)) {
          live[u] = active;
          poff[u] = row * pstride + col;
          soff[u] = (bc.slot * L.block_size + (row - bc.start)) * sstride + col;
          if (!SOPHIA) {
            scale[u] = lr / bias1[bc.slot];  // same rounding as (lr / bias1) * m
            dscale[u] = denom_scale[bc.slot];
          }
        } else if (lane == 0) {
          // A touched row outside every resident block: the host checks this
          // flag and raises (the reference raises on a missing slot, :275-279).
          atomicOr(error_flag, 1);
        }
      }
    }
    float g[OPT_UNROLL], mm[OPT_UNROLL], vv[OPT_UNROLL], p[OPT_UNROLL];
#pragma unroll
    for (int u = 0; u < OPT_UNROLL; ++u) {
      if (live[u]) {
        g[u] = grad[(tb + u) * gstride + col];
        mm[u] = m[soff[u]];
        vv[u] = v[soff[u]];
        p[u] = param[poff[u]];
      }
    }
#pragma unroll
    for (int u = 0; u < OPT_UNROLL; ++u) {
      if (!live[u]) continue;
      const float gg = g[u] / batch_size;
      float m1 = beta1 * mm[u] + one_m_b1 * gg;
      float v1 = vv[u];
      float p1 = p[u];
      if (SOPHIA) {
        if (update_h) v1 = beta2 * v1 + one_m_b2 * gg * gg;
        float r = m1 / fmaxf(v1, eps);
        r = fminf(fmaxf(r, -rho), rho);
        p1 -= lr * r;
      } else {
        v1 = beta2 * v1 + one_m_b2 * gg * gg;
        const float denom = sqrtf(v1) / dscale[u] + eps;
        p1 -= scale[u] * m1 / denom;
      }
      m[soff[u]] = m1;
      v[soff[u]] = v1;
      param[poff[u]] = p1;
    }
    t = te;
  }
}

// Per layout entry: number of touched rows inside [start,end) of the sorted
// touched-row list (replaces unique_consecutive + D2H at :293-297 with one
// tiny kernel; the host still reads the counts back to advance slot steps).
template <typename IdxT>
__global__ void block_touch_counts_kernel(int64_t n_rows, const IdxT* __restrict__ rows,
                                          OptimLayout L, int64_t* __restrict__ counts) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= L.n) return;
  auto lower = [&](int64_t key) {
    int64_t lo = 0, hi = n_rows;
    while (lo < hi) {
      int64_t mid = (lo + hi) >> 1;
      if ((int64_t)rows[mid] < key)
        lo = mid + 1;
      else
        hi = mid;
    }
    return lo;
  };
  counts[i] = lower(L.ends[i]) - lower(L.starts[i]);
}

static int fill_components(OptimComponents& C, int n_comp, float* const* params,
                           const float* const* grads, float* const* m, float* const* v,
                           const int32_t* widths, const int64_t* strides, const float* lrs) {
  TGS_CHECK_ARG(n_comp >= 1 && n_comp <= TGS_MAX_COMP, "n_components must be in [1,%d]",
                TGS_MAX_COMP);
  int total = 0;
  C.n = n_comp;
  for (int k = 0; k < TGS_MAX_COMP; ++k) {
    if (k < n_comp) {
      TGS_CHECK_ARG(params[k] && grads[k] && m[k] && v[k], "component %d has a null pointer", k);
      TGS_CHECK_ARG(widths[k] >= 1, "component %d width must be >= 1", k);
      C.param[k] = params[k];
      C.grad[k] = grads[k];
      C.m[k] = m[k];
      C.v[k] = v[k];
      C.width[k] = widths[k];
      C.pstride[k] = strides ? strides[3 * k + 0] : widths[k];
      C.gstride[k] = strides ? strides[3 * k + 1] : widths[k];
      C.sstride[k] = strides ? strides[3 * k + 2] : widths[k];
      TGS_CHECK_ARG(C.pstride[k] >= widths[k] && C.gstride[k] >= widths[k] &&
                        C.sstride[k] >= widths[k],
                    "component %d: row stride smaller than its width", k);
      C.lr[k] = lrs[k];
      total += widths[k];
    } else {
      C.param[k] = nullptr;
      C.grad[k] = nullptr;
      C.m[k] = nullptr;
      C.v[k] = nullptr;
      C.width[k] = 0;
      C.pstride[k] = C.gstride[k] = C.sstride[k] = 0;
      C.lr[k] = 0.f;
    }
  }
  TGS_CHECK_ARG(total <= 64, "total row width %d exceeds one wavefront (64)", total);
  C.total = total;
  int unified = 1, col = 0;
  for (int k = 0; k < n_comp; ++k) {
    unified &= C.pstride[k] == total && C.gstride[k] == total && C.sstride[k] == total;
    unified &= C.param[k] == C.param[0] + col && C.grad[k] == C.grad[0] + col &&
               C.m[k] == C.m[0] + col && C.v[k] == C.v[0] + col;
    col += widths[k];
  }
  C.unified = unified;
  return TGS_OK;
}

template <bool SOPHIA>
static int launch_optim(int64_t n_rows, const void* local_rows, int index_is_i64,
                        const int64_t* starts, const int64_t* ends, const int64_t* slots,
                        int64_t n_layout, int64_t block_size, const float* bias1,
                        const float* denom_scale, int n_comp, float* const* params,
                        const float* const* grads, float* const* m, float* const* v,
                        const int32_t* widths, const int64_t* strides, const float* lrs,
                        float beta1, float beta2, float eps, float batch_size, float rho,
                        int update_h, int* error_flag, hipStream_t stream) {
  TGS_CHECK_ARG(n_rows >= 0, "n_rows must be >= 0");
  if (n_rows == 0) return TGS_OK;
  TGS_CHECK_ARG(local_rows && starts && ends && slots && error_flag, "null index pointer");
  TGS_CHECK_ARG(n_layout >= 1 && block_size >= 1, "empty block layout");
  if (!SOPHIA) TGS_CHECK_ARG(bias1 && denom_scale, "null bias table");
  OptimComponents C;
  int rc = fill_components(C, n_comp, params, grads, m, v, widths, strides, lrs);
  if (rc) return rc;
  OptimLayout L{starts, ends, slots, n_layout, block_size};
  const int threads = 256;
  // each wavefront takes a contiguous range of >= 16 rows; at most ~8 waves
  // per SIMD over 256 CUs
  int64_t waves_needed = (n_rows + 15) / 16;
  int64_t blocks = (waves_needed + 3) / 4;
  if (blocks > 256 * 32) blocks = 256 * 32;
  if (blocks < 1) blocks = 1;
  if (index_is_i64)
    hipLaunchKernelGGL((resident_optim_kernel<int64_t, SOPHIA>), dim3((unsigned)blocks),
                       dim3(threads), 0, stream, n_rows, (const int64_t*)local_rows, L, bias1,
                       denom_scale, C, beta1, beta2, eps, batch_size, rho, update_h, error_flag);
  else
    hipLaunchKernelGGL((resident_optim_kernel<int32_t, SOPHIA>), dim3((unsigned)blocks),
                       dim3(threads), 0, stream, n_rows, (const int32_t*)local_rows, L, bias1,
                       denom_scale, C, beta1, beta2, eps, batch_size, rho, update_h, error_flag);
  TGS_RETURN_LAUNCH(SOPHIA ? "tgs_resident_sophia_step" : "tgs_resident_adam_step");
}

extern "C" int tgs_resident_adam_step(
    int64_t n_rows, const void* local_rows, int index_is_i64, const int64_t* block_starts,
    const int64_t* block_ends, const int64_t* block_slots, int64_t n_layout, int64_t block_size,
    const float* bias_correction1, const float* denom_scale, int n_components,
    float* const* params, const float* const* grads, float* const* exp_avg,
    float* const* exp_avg_sq, const int32_t* widths, const int64_t* row_strides, const float* lrs,
    float beta1, float beta2, float eps, float batch_size, int* error_flag, hipStream_t stream) {
  return launch_optim<false>(n_rows, local_rows, index_is_i64, block_starts, block_ends,
                             block_slots, n_layout, block_size, bias_correction1, denom_scale,
                             n_components, params, grads, exp_avg, exp_avg_sq, widths, row_strides,
                             lrs, beta1, beta2, eps, batch_size, 0.f, 1, error_flag, stream);
}

extern "C" int tgs_resident_sophia_step(
    int64_t n_rows, const void* local_rows, int index_is_i64, const int64_t* block_starts,
    const int64_t* block_ends, const int64_t* block_slots, int64_t n_layout, int64_t block_size,
    int n_components, float* const* params, const float* const* grads, float* const* exp_avg,
    float* const* hessian, const int32_t* widths, const int64_t* row_strides, const float* lrs,
    float beta1, float beta2, float eps, float rho, float batch_size, int update_hessian,
    int* error_flag, hipStream_t stream) {
  return launch_optim<true>(n_rows, local_rows, index_is_i64, block_starts, block_ends,
                            block_slots, n_layout, block_size, nullptr, nullptr, n_components,
                            params, grads, exp_avg, hessian, widths, row_strides, lrs, beta1,
                            beta2, eps, batch_size, rho, update_hessian, error_flag, stream);
}

extern "C" int tgs_block_touch_counts(int64_t n_rows, const void* rows, int index_is_i64,
                                      const int64_t* block_starts, const int64_t* block_ends,
                                      int64_t n_layout, int64_t* counts, hipStream_t stream) {
  TGS_CHECK_ARG(n_layout >= 0 && n_rows >= 0, "negative size");
  if (n_layout == 0) return TGS_OK;
  TGS_CHECK_ARG(block_starts && block_ends && counts && (rows || n_rows == 0), "null pointer");
  OptimLayout L{block_starts, block_ends, nullptr, n_layout, 0};
  if (index_is_i64)
    hipLaunchKernelGGL(block_touch_counts_kernel<int64_t>, dim3(tgs_blocks(n_layout, 256)),
                       dim3(256), 0, stream, n_rows, (const int64_t*)rows, L, counts);
  else
    hipLaunchKernelGGL(block_touch_counts_kernel<int32_t>, dim3(tgs_blocks(n_layout, 256)),
                       dim3(256), 0, stream, n_rows, (const int32_t*)rows, L, counts);
  TGS_RETURN_LAUNCH("tgs_block_touch_counts");
}
