// Block frustum culling for a batch of cameras.
//
// TideGS culls blocks on the CPU, one camera at a time
// (storage/gaussian_block.py:264-532, FrustumCuller): every block is a
// bounding sphere (centre = bounds midpoint, radius = half the bounds
// diagonal x 1.15), and a block is visible when its centre's signed distance
// to each of the camera's six normalized frustum planes is >= -radius.  At
// 4096 Gaussians per block a billion-Gaussian scene has ~250k blocks, so a
// batch of 16 cameras is ~16 numpy passes over (blocks x 6 x 4) temporaries.
// Here one launch tests every block (or a subset) against all cameras of the
// batch and sets bit c of masks[block] for camera c, with the same float32
// operation order as the numpy expressions (products, then left-to-right
// sums; contraction into fused multiply-adds is switched off in these
// kernels, and the square root is correctly rounded), so the masks equal the
// reference's lists.
#include "tgs_common.cuh"

#define CULL_THREADS 256
#define CULL_MAX_CAMERAS 32

namespace {

// Correctly rounded float sqrt: the hardware estimate (within 1 ulp) moved
// to a neighbour when the fma residuals against the neighbours show the
// square root lies past the midpoint (the correction LLVM uses for
// correctly rounded f32 sqrt); tiny inputs are scaled by 2^32 first.
__device__ __forceinline__ float sqrt_rn(float x) {
  const bool tiny = x < 0x1.0p-96f;
  const float xs = tiny ? x * 0x1.0p+32f : x;
  float s = __builtin_amdgcn_sqrtf(xs);
  if (xs > 0.0f && xs < __builtin_inff()) {
    const float s_dn = __int_as_float(__float_as_int(s) - 1);
    const float s_up = __int_as_float(__float_as_int(s) + 1);
    const float r_dn = __builtin_fmaf(-s_dn, s, xs);
    const float r_up = __builtin_fmaf(-s_up, s, xs);
    if (r_dn <= 0.0f) s = s_dn;
    if (r_up > 0.0f) s = s_up;
  }
  return tiny ? s * 0x1.0p-16f : s;
}

// centre = (min + max) / 2; radius = (sqrt(dx^2 + dy^2 + dz^2) / 2) * 1.15
// (gaussian_block.py:285-296 and :322-325).
__global__ __launch_bounds__(CULL_THREADS) void cull_spheres_kernel(const float* __restrict__ bounds,
                                                                    uint32_t nb,
                                                                    float* __restrict__ centers,
                                                                    float* __restrict__ radii) {
#pragma clang fp contract(off)
  const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nb) return;
  const float* bb = bounds + (uint64_t)b * 6;
  float ss = 0.0f;
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    centers[(uint64_t)b * 3 + d] = (bb[d] + bb[3 + d]) * 0.5f;
    const float e = bb[3 + d] - bb[d];
    const float e2 = e * e;
    ss = d == 0 ? e2 : ss + e2;
  }
  radii[b] = (sqrt_rn(ss) * 0.5f) * 1.15f;
}

// planes: [C][6][4] normalized (A, B, C, D); masks[b] gets bit c.
__global__ __launch_bounds__(CULL_THREADS) void cull_blocks_kernel(
    const float* __restrict__ centers, const float* __restrict__ radii,
    const int64_t* __restrict__ block_ids, uint32_t n, const float* __restrict__ planes,
    uint32_t C, uint32_t* __restrict__ masks) {
#pragma clang fp contract(off)
  __shared__ float s_planes[CULL_MAX_CAMERAS * 24];
  for (uint32_t j = threadIdx.x; j < C * 24; j += blockDim.x) s_planes[j] = planes[j];
  __syncthreads();
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t b = block_ids ? (uint64_t)block_ids[i] : i;
  const float cx = centers[b * 3 + 0], cy = centers[b * 3 + 1], cz = centers[b * 3 + 2];
  const float neg_r = -radii[b];
  uint32_t bits = 0;
  for (uint32_t c = 0; c < C; ++c) {
    bool inside = true;
#pragma unroll
    for (int p = 0; p < 6; ++p) {
      const float* pl = s_planes + c * 24 + p * 4;
      const float px = pl[0] * cx, py = pl[1] * cy, pz = pl[2] * cz;
      float sd = px + py;
      sd = sd + pz;
      sd = sd + pl[3];  // the homogeneous coordinate is 1
      inside = inside && (sd >= neg_r);
    }
    bits |= inside ? (1u << c) : 0u;
  }
  masks[i] = bits;
}

// Legacy cone + distance test (gaussian_block.py:465-510): block i is
// visible when |c_i - cam| <= threshold and either the direction to it has
// cosine > -0.3 with the camera's forward axis or it sits at the camera
// (distance < 1e-6).  Evaluated in float64, so its decisions equal the
// reference's numpy evaluation except within rounding of the two thresholds.
__global__ __launch_bounds__(CULL_THREADS) void cull_cone_kernel(
    const float* __restrict__ centers, uint32_t nb, double cx, double cy, double cz, double fx,
    double fy, double fz, double threshold, uint8_t* __restrict__ visible) {
  const uint32_t i = blockIdx.x * CULL_THREADS + threadIdx.x;
  if (i >= nb) return;
  const double tx = (double)centers[3 * (uint64_t)i] - cx;
  const double ty = (double)centers[3 * (uint64_t)i + 1] - cy;
  const double tz = (double)centers[3 * (uint64_t)i + 2] - cz;
  const double dist = sqrt(tx * tx + ty * ty + tz * tz);
  const double rn = 1.0 / (dist + 1e-8);
  const double dot = tx * rn * fx + ty * rn * fy + tz * rn * fz;
  visible[i] = (uint8_t)(dist <= threshold && (dot > -0.3 || dist < 1e-6));
}

}  // namespace

extern "C" int tgs_cull_blocks_cone(const float* centers, uint32_t nb, double cam_x, double cam_y,
                                    double cam_z, double fwd_x, double fwd_y, double fwd_z,
                                    double threshold, uint8_t* visible, hipStream_t stream) {
  const char* name = "tgs_cull_blocks_cone";
  if (nb == 0) return TGS_OK;
  TGS_CHECK_ARG(centers && visible, "%s: null pointer", name);
  hipLaunchKernelGGL(cull_cone_kernel, dim3(tgs_blocks(nb, CULL_THREADS)), dim3(CULL_THREADS), 0,
                     stream, centers, nb, cam_x, cam_y, cam_z, fwd_x, fwd_y, fwd_z, threshold,
                     visible);
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_cull_block_spheres(const float* bounds, uint32_t nb, float* centers,
                                      float* radii, hipStream_t stream) {
  const char* name = "tgs_cull_block_spheres";
  if (nb == 0) return TGS_OK;
  TGS_CHECK_ARG(bounds && centers && radii, "%s: null pointer", name);
  hipLaunchKernelGGL(cull_spheres_kernel, dim3(tgs_blocks(nb, CULL_THREADS)), dim3(CULL_THREADS), 0,
                     stream, bounds, nb, centers, radii);
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_cull_blocks(const float* centers, const float* radii, const int64_t* block_ids,
                               uint32_t n, const float* planes, uint32_t C, uint32_t* masks,
                               hipStream_t stream) {
  const char* name = "tgs_cull_blocks";
  TGS_CHECK_ARG(C >= 1 && C <= CULL_MAX_CAMERAS, "%s: 1..%d cameras per launch, got %u", name,
                CULL_MAX_CAMERAS, C);
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(centers && radii && planes && masks, "%s: null pointer", name);
  hipLaunchKernelGGL(cull_blocks_kernel, dim3(tgs_blocks(n, CULL_THREADS)), dim3(CULL_THREADS), 0,
                     stream, centers, radii, block_ids, n, planes, C, masks);
  TGS_RETURN_LAUNCH(name);
}
