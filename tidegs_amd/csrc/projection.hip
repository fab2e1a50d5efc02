// gsplat-compatible fully_fused_projection forward/backward (non-packed).
//
// Reference: gsplat/cuda/csrc/fully_fused_projection_fwd.cu:18-181 and
// fully_fused_projection_bwd.cu:18-268.  Layouts match the reference tensors:
// means [N,3], quats [N,4] (w,x,y,z), scales [N,3], covars [N,6] (upper tri),
// viewmats [C,4,4] row-major world-to-camera, Ks [C,3,3];
// radii [C,N] i32, means2d [C,N,2], depths [C,N], conics [C,N,3],
// compensations [C,N].
//
// Forward: one thread per (camera, Gaussian).  Culled entries get radius 0 and
// zeros elsewhere (the reference leaves them uninitialised).
// Backward: one thread per Gaussian looping over cameras, so the per-Gaussian
// gradients are written once, without atomics and in a fixed order; only the
// optional viewmat gradient needs a cross-Gaussian reduction (DPP wave sum,
// then one atomic per wave per entry).
#include "projection.cuh"

__global__ void __launch_bounds__(256) proj_fwd_kernel(
    uint32_t C, uint32_t N, const float* __restrict__ means, const float* __restrict__ covars,
    const float* __restrict__ quats, const float* __restrict__ scales,
    const float* __restrict__ viewmats, const float* __restrict__ Ks, int W, int H, float eps2d,
    float near_plane, float far_plane, float radius_clip, int32_t* __restrict__ radii,
    float* __restrict__ means2d, float* __restrict__ depths, float* __restrict__ conics,
    float* __restrict__ compensations) {
  const uint64_t idx = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (uint64_t)C * N) return;
  const uint32_t cid = (uint32_t)(idx / N);
  const uint32_t gid = (uint32_t)(idx % N);
  const Cam cam = load_cam(viewmats + cid * 16, Ks + cid * 9);
  const float p[3] = {means[gid * 3 + 0], means[gid * 3 + 1], means[gid * 3 + 2]};
  m3 Sigma;
  if (covars) {
    Sigma = covar_from_6(covars + (uint64_t)gid * 6);
  } else {
    const float q[4] = {quats[gid * 4 + 0], quats[gid * 4 + 1], quats[gid * 4 + 2],
                        quats[gid * 4 + 3]};
    const float s[3] = {scales[gid * 3 + 0], scales[gid * 3 + 1], scales[gid * 3 + 2]};
    Sigma = covar_from_quat_scale(q, s);
  }
  const ProjResult r =
      project_forward(p, Sigma, cam, W, H, eps2d, near_plane, far_plane, radius_clip);
  radii[idx] = r.radius;
  const bool ok = r.radius > 0;
  means2d[idx * 2 + 0] = ok ? r.mean2d[0] : 0.f;
  means2d[idx * 2 + 1] = ok ? r.mean2d[1] : 0.f;
  depths[idx] = ok ? r.depth : 0.f;
  conics[idx * 3 + 0] = ok ? r.conic[0] : 0.f;
  conics[idx * 3 + 1] = ok ? r.conic[1] : 0.f;
  conics[idx * 3 + 2] = ok ? r.conic[2] : 0.f;
  if (compensations) compensations[idx] = ok ? r.comp : 0.f;
}

__global__ void __launch_bounds__(256) proj_bwd_kernel(
    uint32_t C, uint32_t N, const float* __restrict__ means, const float* __restrict__ covars,
    const float* __restrict__ quats, const float* __restrict__ scales,
    const float* __restrict__ viewmats, const float* __restrict__ Ks, int W, int H, float eps2d,
    const int32_t* __restrict__ radii, const float* __restrict__ conics,
    const float* __restrict__ compensations, const float* __restrict__ v_means2d,
    const float* __restrict__ v_depths, const float* __restrict__ v_conics,
    const float* __restrict__ v_compensations, float* __restrict__ v_means,
    float* __restrict__ v_covars, float* __restrict__ v_quats, float* __restrict__ v_scales,
    float* __restrict__ v_viewmats) {
  const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
  const bool in_range = gid < N;
  const uint32_t g = in_range ? gid : 0;
  const float p[3] = {means[g * 3 + 0], means[g * 3 + 1], means[g * 3 + 2]};
  float q[4] = {1.f, 0.f, 0.f, 0.f}, s[3] = {1.f, 1.f, 1.f};
  m3 Sigma;
  if (covars) {
    Sigma = covar_from_6(covars + (uint64_t)g * 6);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) q[k] = quats[g * 4 + k];
#pragma unroll
    for (int k = 0; k < 3; ++k) s[k] = scales[g * 3 + k];
    Sigma = covar_from_quat_scale(q, s);
  }
  float acc_p[3] = {0.f, 0.f, 0.f};
  m3 acc_S;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) acc_S.m[i][j] = 0.f;
  const bool want_cam = v_viewmats != nullptr;

  for (uint32_t c = 0; c < C; ++c) {
    const uint64_t idx = (uint64_t)c * N + g;
    const bool live = in_range && radii[idx] > 0;
    ProjGrad pg;
    bool have = false;
    if (live) {
      const Cam cam = load_cam(viewmats + c * 16, Ks + c * 9);
      const float conic[3] = {conics[idx * 3 + 0], conics[idx * 3 + 1], conics[idx * 3 + 2]};
      const float vm[2] = {v_means2d[idx * 2 + 0], v_means2d[idx * 2 + 1]};
      const float vc[3] = {v_conics[idx * 3 + 0], v_conics[idx * 3 + 1], v_conics[idx * 3 + 2]};
      const bool has_vc = v_compensations != nullptr;
      project_backward(p, Sigma, cam, W, H, eps2d, conic, has_vc ? compensations[idx] : 0.f, vm,
                       v_depths ? v_depths[idx] : 0.f, vc, has_vc,
                       has_vc ? v_compensations[idx] : 0.f, want_cam, pg);
      have = true;
#pragma unroll
      for (int k = 0; k < 3; ++k) acc_p[k] += pg.v_p[k];
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc_S.m[i][j] += pg.v_Sigma.m[i][j];
    }
    if (want_cam) {
      // Wave-uniform: every lane takes part in the 12 reductions.
      float vals[12];
#pragma unroll
      for (int i = 0; i < 3; ++i) {
#pragma unroll
        for (int j = 0; j < 3; ++j) vals[i * 4 + j] = have ? pg.v_R.m[i][j] : 0.f;
        vals[i * 4 + 3] = have ? pg.v_t[i] : 0.f;
      }
      const uint64_t any = tgs_ballot(have);
      if (any) {
        float mine = 0.f;
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int k = 0; k < 12; ++k) {
          const float sum = tgs_wave_sum(vals[k]);
          if (lane == k) mine = sum;
        }
        if (lane < 12) tgs_atomic_add(v_viewmats + c * 16 + lane, mine);
      }
    }
  }
  if (!in_range) return;
#pragma unroll
  for (int k = 0; k < 3; ++k) v_means[g * 3 + k] = acc_p[k];
  if (covars) {
    float* o = v_covars + (uint64_t)g * 6;
    o[0] = acc_S.m[0][0];
    o[1] = acc_S.m[0][1] + acc_S.m[1][0];
    o[2] = acc_S.m[0][2] + acc_S.m[2][0];
    o[3] = acc_S.m[1][1];
    o[4] = acc_S.m[1][2] + acc_S.m[2][1];
    o[5] = acc_S.m[2][2];
  } else {
    float vq[4], vs[3];
    covar_vjp_quat_scale(q, s, acc_S, vq, vs);
#pragma unroll
    for (int k = 0; k < 4; ++k) v_quats[g * 4 + k] = vq[k];
#pragma unroll
    for (int k = 0; k < 3; ++k) v_scales[g * 3 + k] = vs[k];
  }
}

extern "C" int tgs_fully_fused_projection_fwd(
    uint32_t C, uint32_t N, const float* means, const float* covars, const float* quats,
    const float* scales, const float* viewmats, const float* Ks, int32_t image_width,
    int32_t image_height, float eps2d, float near_plane, float far_plane, float radius_clip,
    int32_t* radii, float* means2d, float* depths, float* conics, float* compensations,
    hipStream_t stream) {
  if ((uint64_t)C * N == 0) return TGS_OK;
  TGS_CHECK_ARG(means && viewmats && Ks && radii && means2d && depths && conics,
                "fully_fused_projection_fwd: null pointer");
  TGS_CHECK_ARG(covars || (quats && scales),
                "fully_fused_projection_fwd: need covars or quats+scales");
  TGS_CHECK_ARG((uint64_t)C * N < (1ull << 32), "C*N must be < 2^32");
  hipLaunchKernelGGL(proj_fwd_kernel, dim3(tgs_blocks((uint64_t)C * N, 256)), dim3(256), 0,
                     stream, C, N, means, covars, quats, scales, viewmats, Ks, image_width,
                     image_height, eps2d, near_plane, far_plane, radius_clip, radii, means2d,
                     depths, conics, compensations);
  TGS_RETURN_LAUNCH("tgs_fully_fused_projection_fwd");
}

extern "C" int tgs_fully_fused_projection_bwd(
    uint32_t C, uint32_t N, const float* means, const float* covars, const float* quats,
    const float* scales, const float* viewmats, const float* Ks, int32_t image_width,
    int32_t image_height, float eps2d, const int32_t* radii, const float* conics,
    const float* compensations, const float* v_means2d, const float* v_depths,
    const float* v_conics, const float* v_compensations, float* v_means, float* v_covars,
    float* v_quats, float* v_scales, float* v_viewmats, hipStream_t stream) {
  if (N == 0) return TGS_OK;
  TGS_CHECK_ARG(means && viewmats && Ks && radii && conics && v_means2d && v_conics && v_means,
                "fully_fused_projection_bwd: null pointer");
  TGS_CHECK_ARG(covars ? (v_covars != nullptr) : (quats && scales && v_quats && v_scales),
                "fully_fused_projection_bwd: need covars/v_covars or quats/scales/v_quats/v_scales");
  TGS_CHECK_ARG(!v_compensations || compensations,
                "fully_fused_projection_bwd: v_compensations needs compensations");
  TGS_CHECK_ARG((uint64_t)C * N < (1ull << 32), "C*N must be < 2^32");
  hipLaunchKernelGGL(proj_bwd_kernel, dim3(tgs_blocks(N, 256)), dim3(256), 0, stream, C, N,
                     means, covars, quats, scales, viewmats, Ks, image_width, image_height, eps2d,
                     radii, conics, compensations, v_means2d, v_depths, v_conics, v_compensations,
                     v_means, v_covars, v_quats, v_scales, v_viewmats);
  TGS_RETURN_LAUNCH("tgs_fully_fused_projection_bwd");
}

// ---------------------------------------------------------------------------
// Packed projection (fully_fused_projection_packed_fwd.cu:19-275,
// fully_fused_projection_packed_bwd.cu:18-260).  Two passes as the reference:
// per block of PACKED_THREADS Gaussians of one camera, (1) count the entries
// that survive the culls with the packed radius rule, (2) after a scan of the
// counts, write each survivor at its block offset plus its rank in the block.
// Output order: camera-major, Gaussian ascending.
// ---------------------------------------------------------------------------
#define PACKED_THREADS 256

__device__ __forceinline__ m3 packed_sigma(uint32_t gid, const float* __restrict__ covars,
                                           const float* __restrict__ quats,
                                           const float* __restrict__ scales) {
  if (covars) return covar_from_6(covars + (uint64_t)gid * 6);
  const float q[4] = {quats[gid * 4 + 0], quats[gid * 4 + 1], quats[gid * 4 + 2],
                      quats[gid * 4 + 3]};
  const float s[3] = {scales[gid * 3 + 0], scales[gid * 3 + 1], scales[gid * 3 + 2]};
  return covar_from_quat_scale(q, s);
}

// grid (blocks_per_row, C): block (b, c) covers Gaussians [b*256, b*256+256) of camera c.
template <bool WRITE>
__global__ void __launch_bounds__(PACKED_THREADS) proj_packed_kernel(
    uint32_t C, uint32_t N, const float* __restrict__ means, const float* __restrict__ covars,
    const float* __restrict__ quats, const float* __restrict__ scales,
    const float* __restrict__ viewmats, const float* __restrict__ Ks, int W, int H, float eps2d,
    float near_plane, float far_plane, float radius_clip, int32_t* __restrict__ block_counts,
    const int32_t* __restrict__ block_offsets, int32_t* __restrict__ indptr,
    int64_t* __restrict__ camera_ids, int64_t* __restrict__ gaussian_ids,
    int32_t* __restrict__ radii, float* __restrict__ means2d, float* __restrict__ depths,
    float* __restrict__ conics, float* __restrict__ compensations) {
  __shared__ uint32_t s_wave[PACKED_THREADS / 64];
  const uint32_t cid = blockIdx.y;
  const uint32_t gid = blockIdx.x * PACKED_THREADS + threadIdx.x;
  const uint32_t block = cid * gridDim.x + blockIdx.x;
  ProjResult r;
  r.radius = 0;
  if (gid < N) {
    const Cam cam = load_cam(viewmats + cid * 16, Ks + cid * 9);
    const float p[3] = {means[gid * 3 + 0], means[gid * 3 + 1], means[gid * 3 + 2]};
    r = project_forward<true>(p, packed_sigma(gid, covars, quats, scales), cam, W, H, eps2d,
                              near_plane, far_plane, radius_clip);
  }
  const bool valid = r.radius > 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t m = tgs_ballot(valid);
  if (lane == 0) s_wave[wave] = (uint32_t)__popcll(m);
  __syncthreads();
  if (!WRITE) {
    if (threadIdx.x == 0) {
      uint32_t total = 0;
#pragma unroll
      for (int w = 0; w < PACKED_THREADS / 64; ++w) total += s_wave[w];
      block_counts[block] = (int32_t)total;
    }
    return;
  }
  uint32_t rank = (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
  for (int w = 0; w < wave; ++w) rank += s_wave[w];
  if (valid) {
    const uint32_t o = (uint32_t)block_offsets[block] + rank;
    camera_ids[o] = cid;
    gaussian_ids[o] = gid;
    radii[o] = r.radius;
    means2d[o * 2 + 0] = r.mean2d[0];
    means2d[o * 2 + 1] = r.mean2d[1];
    depths[o] = r.depth;
    conics[o * 3 + 0] = r.conic[0];
    conics[o * 3 + 1] = r.conic[1];
    conics[o * 3 + 2] = r.conic[2];
    if (compensations) compensations[o] = r.comp;
  }
  // indptr[c] = first entry of camera c (its first block's offset)
  if (threadIdx.x == 0 && blockIdx.x == 0) indptr[cid] = block_offsets[block];
}

// One thread per packed entry.  sparse_grad: the VJPs stay per entry ([nnz, .]);
// otherwise they are summed into the [N, .] gradients (atomics: the entries of
// one Gaussian sit in different cameras).
__global__ void __launch_bounds__(256) proj_packed_bwd_kernel(
    uint32_t nnz, const float* __restrict__ means, const float* __restrict__ covars,
    const float* __restrict__ quats, const float* __restrict__ scales,
    const float* __restrict__ viewmats, const float* __restrict__ Ks, int W, int H, float eps2d,
    const int64_t* __restrict__ camera_ids, const int64_t* __restrict__ gaussian_ids,
    const float* __restrict__ conics, const float* __restrict__ compensations,
    const float* __restrict__ v_means2d, const float* __restrict__ v_depths,
    const float* __restrict__ v_conics, const float* __restrict__ v_compensations,
    int sparse_grad, float* __restrict__ v_means, float* __restrict__ v_covars,
    float* __restrict__ v_quats, float* __restrict__ v_scales, float* __restrict__ v_viewmats) {
  const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= nnz) return;
  const uint32_t cid = (uint32_t)camera_ids[idx];
  const uint32_t gid = (uint32_t)gaussian_ids[idx];
  const Cam cam = load_cam(viewmats + cid * 16, Ks + cid * 9);
  const float p[3] = {means[gid * 3 + 0], means[gid * 3 + 1], means[gid * 3 + 2]};
  float q[4] = {1.f, 0.f, 0.f, 0.f}, s[3] = {1.f, 1.f, 1.f};
  m3 Sigma;
  if (covars) {
    Sigma = covar_from_6(covars + (uint64_t)gid * 6);
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) q[k] = quats[gid * 4 + k];
#pragma unroll
    for (int k = 0; k < 3; ++k) s[k] = scales[gid * 3 + k];
    Sigma = covar_from_quat_scale(q, s);
  }
  const float conic[3] = {conics[idx * 3 + 0], conics[idx * 3 + 1], conics[idx * 3 + 2]};
  const float vm[2] = {v_means2d[idx * 2 + 0], v_means2d[idx * 2 + 1]};
  const float vc[3] = {v_conics[idx * 3 + 0], v_conics[idx * 3 + 1], v_conics[idx * 3 + 2]};
  const bool has_vc = v_compensations != nullptr;
  const bool want_cam = v_viewmats != nullptr;
  ProjGrad pg;
  project_backward(p, Sigma, cam, W, H, eps2d, conic, has_vc ? compensations[idx] : 0.f, vm,
                   v_depths ? v_depths[idx] : 0.f, vc, has_vc, has_vc ? v_compensations[idx] : 0.f,
                   want_cam, pg);
  const uint64_t o = sparse_grad ? idx : gid;
  auto put = [&](float* base, uint64_t k, float v) {
    if (sparse_grad) base[k] = v;
    else tgs_atomic_add(base + k, v);
  };
#pragma unroll
  for (int k = 0; k < 3; ++k) put(v_means, o * 3 + k, pg.v_p[k]);
  if (covars) {
    const m3& S = pg.v_Sigma;
    put(v_covars, o * 6 + 0, S.m[0][0]);
    put(v_covars, o * 6 + 1, S.m[0][1] + S.m[1][0]);
    put(v_covars, o * 6 + 2, S.m[0][2] + S.m[2][0]);
    put(v_covars, o * 6 + 3, S.m[1][1]);
    put(v_covars, o * 6 + 4, S.m[1][2] + S.m[2][1]);
    put(v_covars, o * 6 + 5, S.m[2][2]);
  } else {
    float vq[4], vs[3];
    covar_vjp_quat_scale(q, s, pg.v_Sigma, vq, vs);
#pragma unroll
    for (int k = 0; k < 4; ++k) put(v_quats, o * 4 + k, vq[k]);
#pragma unroll
    for (int k = 0; k < 3; ++k) put(v_scales, o * 3 + k, vs[k]);
  }
  if (want_cam) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
      for (int j = 0; j < 3; ++j) tgs_atomic_add(v_viewmats + cid * 16 + i * 4 + j, pg.v_R.m[i][j]);
      tgs_atomic_add(v_viewmats + cid * 16 + i * 4 + 3, pg.v_t[i]);
    }
  }
}

extern "C" uint32_t tgs_fully_fused_projection_packed_blocks(uint32_t N) {
  return (N + PACKED_THREADS - 1) / PACKED_THREADS;
}

extern "C" int tgs_fully_fused_projection_packed_count(
    uint32_t C, uint32_t N, const float* means, const float* covars, const float* quats,
    const float* scales, const float* viewmats, const float* Ks, int32_t image_width,
    int32_t image_height, float eps2d, float near_plane, float far_plane, float radius_clip,
    int32_t* block_counts, hipStream_t stream) {
  if ((uint64_t)C * N == 0) return TGS_OK;
  TGS_CHECK_ARG(means && viewmats && Ks && block_counts,
                "fully_fused_projection_packed_count: null pointer");
  TGS_CHECK_ARG(covars || (quats && scales),
                "fully_fused_projection_packed_count: need covars or quats+scales");
  TGS_CHECK_ARG(C <= 65535 && (uint64_t)C * N < (1ull << 31), "packed projection: C*N too large");
  const uint32_t nb = tgs_fully_fused_projection_packed_blocks(N);
  hipLaunchKernelGGL((proj_packed_kernel<false>), dim3(nb, C), dim3(PACKED_THREADS), 0, stream, C,
                     N, means, covars, quats, scales, viewmats, Ks, image_width, image_height,
                     eps2d, near_plane, far_plane, radius_clip, block_counts, nullptr, nullptr,
                     nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
  TGS_RETURN_LAUNCH("tgs_fully_fused_projection_packed_count");
}

extern "C" int tgs_fully_fused_projection_packed_fwd(
    uint32_t C, uint32_t N, const float* means, const float* covars, const float* quats,
    const float* scales, const float* viewmats, const float* Ks, int32_t image_width,
    int32_t image_height, float eps2d, float near_plane, float far_plane, float radius_clip,
    const int32_t* block_offsets, uint32_t nnz, int32_t* indptr, int64_t* camera_ids,
    int64_t* gaussian_ids, int32_t* radii, float* means2d, float* depths, float* conics,
    float* compensations, hipStream_t stream) {
  TGS_CHECK_ARG(indptr, "fully_fused_projection_packed_fwd: null indptr");
  if ((uint64_t)C * N == 0 || nnz == 0) {
    if (C + 1 > 0) return tgs_fill_u32(indptr, C + 1, 0u, stream);
    return TGS_OK;
  }
  TGS_CHECK_ARG(means && viewmats && Ks && block_offsets && camera_ids && gaussian_ids && radii &&
                    means2d && depths && conics,
                "fully_fused_projection_packed_fwd: null pointer");
  TGS_CHECK_ARG(covars || (quats && scales),
                "fully_fused_projection_packed_fwd: need covars or quats+scales");
  TGS_CHECK_ARG(C <= 65535 && (uint64_t)C * N < (1ull << 31), "packed projection: C*N too large");
  const uint32_t nb = tgs_fully_fused_projection_packed_blocks(N);
  hipLaunchKernelGGL((proj_packed_kernel<true>), dim3(nb, C), dim3(PACKED_THREADS), 0, stream, C,
                     N, means, covars, quats, scales, viewmats, Ks, image_width, image_height,
                     eps2d, near_plane, far_plane, radius_clip, nullptr, block_offsets, indptr,
                     camera_ids, gaussian_ids, radii, means2d, depths, conics, compensations);
  TGS_LAUNCH_CHECK("tgs_fully_fused_projection_packed_fwd");
  // indptr[C] = nnz
  return tgs_fill_u32(indptr + C, 1, nnz, stream);
}

extern "C" int tgs_fully_fused_projection_packed_bwd(
    uint32_t C, uint32_t N, uint32_t nnz, const float* means, const float* covars,
    const float* quats, const float* scales, const float* viewmats, const float* Ks,
    int32_t image_width, int32_t image_height, float eps2d, const int64_t* camera_ids,
    const int64_t* gaussian_ids, const float* conics, const float* compensations,
    const float* v_means2d, const float* v_depths, const float* v_conics,
    const float* v_compensations, int sparse_grad, float* v_means, float* v_covars,
    float* v_quats, float* v_scales, float* v_viewmats, hipStream_t stream) {
  if (nnz == 0) return TGS_OK;
  TGS_CHECK_ARG(means && viewmats && Ks && camera_ids && gaussian_ids && conics && v_means2d &&
                    v_conics && v_means,
                "fully_fused_projection_packed_bwd: null pointer");
  TGS_CHECK_ARG(covars ? (v_covars != nullptr) : (quats && scales && v_quats && v_scales),
                "fully_fused_projection_packed_bwd: need covars/v_covars or "
                "quats/scales/v_quats/v_scales");
  TGS_CHECK_ARG(!v_compensations || compensations,
                "fully_fused_projection_packed_bwd: v_compensations needs compensations");
  (void)C;
  (void)N;
  hipLaunchKernelGGL(proj_packed_bwd_kernel, dim3(tgs_blocks(nnz, 256)), dim3(256), 0, stream, nnz,
                     means, covars, quats, scales, viewmats, Ks, image_width, image_height, eps2d,
                     camera_ids, gaussian_ids, conics, compensations, v_means2d, v_depths,
                     v_conics, v_compensations, sparse_grad, v_means, v_covars, v_quats, v_scales,
                     v_viewmats);
  TGS_RETURN_LAUNCH("tgs_fully_fused_projection_packed_bwd");
}
