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
// searchsorted/index_select.  Here a single launch covers all 59 columns: a
// wavefront takes groups of touched rows (several rows in flight), lane l
// handles column l (59 of 64 lanes busy), and the row -> (slot, state row)
// lookup is wave-uniform and runs only when the (sorted) rows cross into
// another resident block (see BlockCache).  The column -> (component tensor,
// column) map is fixed per lane, so one kernel family serves six split
// component tensors or one unified [N,59] table.  The building blocks are
// shared with the projection backward's fused update (resident_optim.cuh).
//
// Sophia (no reference; Liu et al. 2023, arXiv 2305.14342, Alg. 3, with a
// per-coordinate clip of the update ratio):
//   m  = b1*m + (1-b1)*g
//   h  = b2*h + (1-b2)*g*g        (only on Hessian-refresh steps)
//   p -= lr_col * clamp(m / max(h, eps), -rho, rho)

#include "resident_optim.cuh"

#define OPT_ROWS 8  // rows in flight per wavefront (row path)
#define OPT_UNROLL 4
#define OPT_RUN 64  // rows per flat-path run

// Unified layout: param, grad and both state tables each hold all W columns
// of a row contiguously, at row strides PW, GW and SW (each <= 64 floats: 59
// for dense tables, 64 for the padded layout whose rows are whole 256-byte
// lines).  Groups of OPT_RUN sorted touched rows are dealt to the wavefronts
// round-robin.
//   * flat path (dense tables only): when the group's rows are consecutive and
//     inside one resident block, every table's part is one contiguous span,
//     streamed 64 floats per instruction across row bounds;
//   * row path: OPT_ROWS rows at a time, lane = column.  The row ids arrive
//     with one vector load and are read back as scalars.  For rows inside one
//     resident block each table gets one buffer descriptor at the first row
//     and every row is a scalar byte offset from it, so a load is (descriptor,
//     the lane's column offset, the row's scalar offset): one data VGPR per
//     load and 4 * OPT_ROWS loads in flight per wavefront.  Padding lanes
//     (W <= lane < stride) write back what they read, so a padded row is
//     stored as a whole line and its padding keeps its bits.
template <typename IdxT, bool SOPHIA>
__global__ void __launch_bounds__(256) resident_optim_unified_kernel(
    int64_t n_rows, const IdxT* __restrict__ local_rows, OptimLayout L,
    const float* __restrict__ bias1, const float* __restrict__ denom_scale, OptimComponents C,
    float beta1, float beta2, float eps, float batch_size, float rho, int update_h,
    int* __restrict__ error_flag) {
  const int lane = threadIdx.x & 63;
  // threadIdx.x >> 6 is the same in every lane of a wavefront; readfirstlane
  // tells the compiler so, which keeps the row range and every address derived
  // from it in scalar registers
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) +
                       __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n_waves = (int64_t)gridDim.x * (blockDim.x >> 6);
  const int W = C.total;
  const int PW = C.pw, GW = C.gw, SW = C.sw;
  const int64_t PB = (int64_t)PW * 4, GB = (int64_t)GW * 4, SB = (int64_t)SW * 4;  // row bytes
  const bool act = lane < W;
  const uint32_t voff_g = act ? (uint32_t)lane * 4u : TGS_OFF_NONE;
  const uint32_t voff_p = lane < PW ? (uint32_t)lane * 4u : TGS_OFF_NONE;
  const uint32_t voff_s = lane < SW ? (uint32_t)lane * 4u : TGS_OFF_NONE;
  const bool dense = PW == W && GW == W && SW == W;
  const float one_m_b1 = 1.0f - beta1;
  const float one_m_b2 = 1.0f - beta2;
  const float* P = C.param[0];
  const float* G = C.grad[0];
  const float* M = C.m[0];
  const float* V = C.v[0];

  // per-column learning rate
  __shared__ float s_lr[64];
  __shared__ float s_scale[4][64];  // per wavefront: step size per column of the current run
  if (threadIdx.x < 64) {
    float lr = 0.f;
    int base = 0;
#pragma unroll
    for (int k = 0; k < TGS_MAX_COMP; ++k) {
      if (k < C.n) {
        if ((int)threadIdx.x >= base && (int)threadIdx.x < base + C.width[k]) lr = C.lr[k];
        base += C.width[k];
      }
    }
    s_lr[threadIdx.x] = lr;
  }
  __syncthreads();
  const float lr_lane = s_lr[lane];

  // Groups of OPT_RUN touched rows, dealt to the wavefronts round-robin: the
  // rows in flight across the whole GPU at any moment then lie in one narrow
  // window of each table, instead of one region per wavefront spread over
  // the whole table.
  BlockCache bc;
  const int64_t n_groups = (n_rows + OPT_RUN - 1) / OPT_RUN;
  for (int64_t grp = wave; grp < n_groups; grp += n_waves) {
    int64_t t = grp * OPT_RUN;
    const int64_t t1 = t + OPT_RUN < n_rows ? t + OPT_RUN : n_rows;
    if (dense) {
      const int64_t r0 = tgs_uniform_i64((int64_t)local_rows[t]);
      const int64_t rl = tgs_uniform_i64((int64_t)local_rows[t1 - 1]);
      if (t1 - t >= 16 && rl - r0 == t1 - 1 - t && bc.lookup(L, r0) && rl < bc.end &&
          rl - bc.start < L.block_size) {
        const int64_t F = (t1 - t) * W;  // <= OPT_RUN * 64 floats
        const int64_t srow = bc.slot * L.block_size + (r0 - bc.start);
        const auto rg = tgs_rsrc(G + t * W, F * 4);
        const auto rp = tgs_rsrc(P + r0 * W, F * 4);
        const auto rm = tgs_rsrc(M + srow * W, F * 4);
        const auto rv = tgs_rsrc(V + srow * W, F * 4);
        float* s_sc = s_scale[threadIdx.x >> 6];
        s_sc[lane] = SOPHIA ? lr_lane : lr_lane / tgs_readlane_f32(bias1[bc.slot], 0);
        const float dsc = SOPHIA ? 1.f : tgs_readlane_f32(denom_scale[bc.slot], 0);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int step = 64 % W;
        int c = lane % W;  // column of element lane + 64 k
        // elements past F read as 0 and their stores are dropped (range check)
        for (uint32_t i0 = (uint32_t)lane; i0 < (uint32_t)F; i0 += 64 * OPT_UNROLL) {
          float gv[OPT_UNROLL], mv[OPT_UNROLL], vv[OPT_UNROLL], pv[OPT_UNROLL];
#pragma unroll
          for (int u = 0; u < OPT_UNROLL; ++u) {
            const uint32_t o = (i0 + 64u * u) * 4u;
            gv[u] = tgs_bload(rg, o, 0);
            mv[u] = tgs_bload_nt(rm, o, 0);
            vv[u] = tgs_bload_nt(rv, o, 0);
            pv[u] = tgs_bload(rp, o, 0);
          }
#pragma unroll
          for (int u = 0; u < OPT_UNROLL; ++u) {
            const uint32_t o = (i0 + 64u * u) * 4u;
            optim_update<SOPHIA>(gv[u], mv[u], vv[u], pv[u], s_sc[c], dsc, beta1, beta2,
                                 one_m_b1, one_m_b2, eps, batch_size, rho, update_h);
            tgs_bstore_nt(mv[u], rm, o, 0);
            tgs_bstore_nt(vv[u], rv, o, 0);
            tgs_bstore_nt(pv[u], rp, o, 0);
            c += step;
            if (c >= W) c -= W;
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        continue;
      }
    }
    // row path: OPT_ROWS rows (sorted) at a time
    for (; t < t1;) {
      const int n = (int)(t1 - t < OPT_ROWS ? t1 - t : OPT_ROWS);
      const int64_t my_row = lane < n ? (int64_t)local_rows[t + lane] : 0;
      const int64_t r_first = tgs_readlane_i64(my_row, 0);
      const int64_t r_last = tgs_readlane_i64(my_row, n - 1);
      const int64_t rows_span = r_last - r_first + 1;
      const auto rg = tgs_rsrc(G + t * GW, n * GB);
      if (bc.lookup(L, r_first) && r_last < bc.end && r_last - bc.start < L.block_size &&
          rows_span * 256 < 0x7fffffff) {
        // every row of the group is in this block: one descriptor per table
        const int64_t srow = bc.slot * L.block_size + (r_first - bc.start);
        const auto rp = tgs_rsrc(P + r_first * PW, rows_span * PB);
        const auto rm = tgs_rsrc(M + srow * SW, rows_span * SB);
        const auto rv = tgs_rsrc(V + srow * SW, rows_span * SB);
        const float sc = SOPHIA ? lr_lane : lr_lane / tgs_readlane_f32(bias1[bc.slot], 0);
        const float dsc = SOPHIA ? 1.f : tgs_readlane_f32(denom_scale[bc.slot], 0);
        float gv[OPT_ROWS], mv[OPT_ROWS], vv[OPT_ROWS], pv[OPT_ROWS];
#pragma unroll
        for (int u = 0; u < OPT_ROWS; ++u) {
          if (u < n) {
            const int64_t d = tgs_readlane_i64(my_row, u) - r_first;
            gv[u] = tgs_bload(rg, voff_g, (uint32_t)(u * GB));
            mv[u] = tgs_bload_nt(rm, voff_s, (uint32_t)(d * SB));
            vv[u] = tgs_bload_nt(rv, voff_s, (uint32_t)(d * SB));
            pv[u] = tgs_bload(rp, voff_p, (uint32_t)(d * PB));
          }
        }
#pragma unroll
        for (int u = 0; u < OPT_ROWS; ++u) {
          if (u < n) {
            const int64_t d = tgs_readlane_i64(my_row, u) - r_first;
            float m1 = mv[u], v1 = vv[u], p1 = pv[u];
            optim_update<SOPHIA>(gv[u], m1, v1, p1, sc, dsc, beta1, beta2, one_m_b1, one_m_b2,
                                 eps, batch_size, rho, update_h);
            tgs_bstore_nt(act ? m1 : mv[u], rm, voff_s, (uint32_t)(d * SB));
            tgs_bstore_nt(act ? v1 : vv[u], rv, voff_s, (uint32_t)(d * SB));
            tgs_bstore_nt(act ? p1 : pv[u], rp, voff_p, (uint32_t)(d * PB));
          }
        }
      } else {
        // the rows straddle resident blocks (or span 2 GB): one row at a time
        for (int u = 0; u < n; ++u) {
          const int64_t row = tgs_readlane_i64(my_row, u);
          if (!bc.lookup(L, row)) {
            // a touched row outside every resident block: the host checks this
            // flag and raises (the reference raises on a missing slot, :275-279)
            if (lane == 0) atomicOr(error_flag, 1);
            continue;
          }
          const int64_t srow = bc.slot * L.block_size + (row - bc.start);
          const auto rp = tgs_rsrc(P + row * PW, PB);
          const auto rm = tgs_rsrc(M + srow * SW, SB);
          const auto rv = tgs_rsrc(V + srow * SW, SB);
          const float sc = SOPHIA ? lr_lane : lr_lane / tgs_readlane_f32(bias1[bc.slot], 0);
          const float dsc = SOPHIA ? 1.f : tgs_readlane_f32(denom_scale[bc.slot], 0);
          const float gv = tgs_bload(rg, voff_g, (uint32_t)(u * GB));
          const float mv = tgs_bload_nt(rm, voff_s, 0), vv = tgs_bload_nt(rv, voff_s, 0);
          const float pv = tgs_bload(rp, voff_p, 0);
          float m1 = mv, v1 = vv, p1 = pv;
          optim_update<SOPHIA>(gv, m1, v1, p1, sc, dsc, beta1, beta2, one_m_b1, one_m_b2, eps,
                               batch_size, rho, update_h);
          tgs_bstore_nt(act ? m1 : mv, rm, voff_s, 0);
          tgs_bstore_nt(act ? v1 : vv, rv, voff_s, 0);
          tgs_bstore_nt(act ? p1 : pv, rp, voff_p, 0);
        }
      }
      t += n;
    }
  }
}

// Any layout: per-component pointers and row strides, one row per step with
// lane = column (the reference's six separate component tensors, or a table
// whose column order differs from the state's).
template <typename IdxT, bool SOPHIA>
__global__ void __launch_bounds__(256) resident_optim_kernel(
    int64_t n_rows, const IdxT* __restrict__ local_rows, OptimLayout L,
    const float* __restrict__ bias1, const float* __restrict__ denom_scale, OptimComponents C,
    float beta1, float beta2, float eps, float batch_size, float rho, int update_h,
    int* __restrict__ error_flag) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) +
                       __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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

  const int64_t per = (n_rows + n_waves - 1) / n_waves;
  const int64_t t0 = wave * per;
  const int64_t t1 = t0 + per < n_rows ? t0 + per : n_rows;
  BlockCache bc;
  for (int64_t tb = t0; tb < t1; tb += OPT_UNROLL) {
    const int64_t te = tb + OPT_UNROLL < t1 ? tb + OPT_UNROLL : t1;
    int64_t poff[OPT_UNROLL], soff[OPT_UNROLL];
    float scale[OPT_UNROLL], dscale[OPT_UNROLL];
    bool live[OPT_UNROLL];
#pragma unroll
    for (int u = 0; u < OPT_UNROLL; ++u) {
      live[u] = false;
      poff[u] = soff[u] = 0;
      scale[u] = lr;
      dscale[u] = 1.f;
      if (tb + u < te) {
        const int64_t row = (int64_t)local_rows[tb + u];
        if (bc.lookup(L, row)) {
          live[u] = active;
          poff[u] = row * pstride + col;
          soff[u] = (bc.slot * L.block_size + (row - bc.start)) * sstride + col;
          if (!SOPHIA) {
            scale[u] = lr / bias1[bc.slot];
            dscale[u] = denom_scale[bc.slot];
          }
        } else if (lane == 0) {
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
      optim_update<SOPHIA>(g[u], mm[u], vv[u], p[u], scale[u], dscale[u], beta1, beta2,
                           one_m_b1, one_m_b2, eps, batch_size, rho, update_h);
      m[soff[u]] = mm[u];
      v[soff[u]] = vv[u];
      param[poff[u]] = p[u];
    }
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
    unified &= C.pstride[k] == C.pstride[0] && C.gstride[k] == C.gstride[0] &&
               C.sstride[k] == C.sstride[0];
    unified &= C.param[k] == C.param[0] + col && C.grad[k] == C.grad[0] + col &&
               C.m[k] == C.m[0] + col && C.v[k] == C.v[0] + col;
    col += widths[k];
  }
  unified &= C.pstride[0] <= 64 && C.gstride[0] <= 64 && C.sstride[0] <= 64;
  C.unified = unified;
  C.pw = (int)C.pstride[0];
  C.gw = (int)C.gstride[0];
  C.sw = (int)C.sstride[0];
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
  int shift = -1;
  if ((block_size & (block_size - 1)) == 0)
    for (shift = 0; ((int64_t)1 << shift) < block_size; ++shift) {
    }
  OptimLayout L{starts, ends, slots, n_layout, block_size, shift};
  const int threads = 256;
  int64_t blocks;
  if (C.unified) {
    // round-robin groups of OPT_RUN rows; 8 wavefronts per SIMD at most
    blocks = ((n_rows + OPT_RUN - 1) / OPT_RUN + 3) / 4;
    if (blocks > 256 * 8) blocks = 256 * 8;
  } else {
    // each wavefront takes a contiguous range of >= 16 rows
    int64_t waves_needed = (n_rows + 15) / 16;
    blocks = (waves_needed + 3) / 4;
    if (blocks > 256 * 32) blocks = 256 * 32;
  }
  if (blocks < 1) blocks = 1;
#define TGS_OPTIM_LAUNCH(KERNEL, IDX)                                                     \
  hipLaunchKernelGGL((KERNEL<IDX, SOPHIA>), dim3((unsigned)blocks), dim3(threads), 0, stream,  \
                     n_rows, (const IDX*)local_rows, L, bias1, denom_scale, C, beta1, beta2, eps, \
                     batch_size, rho, update_h, error_flag)
  if (C.unified) {
    if (index_is_i64)
      TGS_OPTIM_LAUNCH(resident_optim_unified_kernel, int64_t);
    else
      TGS_OPTIM_LAUNCH(resident_optim_unified_kernel, int32_t);
  } else {
    if (index_is_i64)
      TGS_OPTIM_LAUNCH(resident_optim_kernel, int64_t);
    else
      TGS_OPTIM_LAUNCH(resident_optim_kernel, int32_t);
  }
#undef TGS_OPTIM_LAUNCH
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
  OptimLayout L{block_starts, block_ends, nullptr, n_layout, 0, -1};
  if (index_is_i64)
    hipLaunchKernelGGL(block_touch_counts_kernel<int64_t>, dim3(tgs_blocks(n_layout, 256)),
                       dim3(256), 0, stream, n_rows, (const int64_t*)rows, L, counts);
  else
    hipLaunchKernelGGL(block_touch_counts_kernel<int32_t>, dim3(tgs_blocks(n_layout, 256)),
                       dim3(256), 0, stream, n_rows, (const int32_t*)rows, L, counts);
  TGS_RETURN_LAUNCH("tgs_block_touch_counts");
}
