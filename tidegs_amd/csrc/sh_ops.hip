// gsplat-compatible spherical_harmonics forward/backward.
//
// Reference: gsplat/cuda/csrc/compute_sh_fwd.cu:9-58, compute_sh_bwd.cu:68-136.
// dirs [n,3], coeffs [n,K,3], masks [n] (bool, optional), colors [n,3].
// One thread per element evaluates all three channels from one basis pass
// (the reference runs one thread per (element, channel)).  The backward
// writes every v_coeffs entry (zeros above the active degree and for masked
// elements) and writes v_dirs directly, so no zero-fill or atomics are needed.
#include "sh.cuh"

__global__ void __launch_bounds__(256) sh_fwd_kernel(uint32_t n, uint32_t K, int degree,
                                                     const float* __restrict__ dirs,
                                                     const float* __restrict__ coeffs,
                                                     const uint8_t* __restrict__ masks,
                                                     float* __restrict__ colors) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float out[3] = {0.f, 0.f, 0.f};
  if (!masks || masks[i]) {
    sh_eval3(degree, dirs[i * 3 + 0], dirs[i * 3 + 1], dirs[i * 3 + 2],
             coeffs + (uint64_t)i * K * 3, out);
  }
  colors[i * 3 + 0] = out[0];
  colors[i * 3 + 1] = out[1];
  colors[i * 3 + 2] = out[2];
}

__global__ void __launch_bounds__(256) sh_bwd_kernel(uint32_t n, uint32_t K, int degree,
                                                     const float* __restrict__ dirs,
                                                     const float* __restrict__ coeffs,
                                                     const uint8_t* __restrict__ masks,
                                                     const float* __restrict__ v_colors,
                                                     float* __restrict__ v_coeffs,
                                                     float* __restrict__ v_dirs) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float* vc = v_coeffs + (uint64_t)i * K * 3;
  const int used = (degree + 1) * (degree + 1);
  float vd[3] = {0.f, 0.f, 0.f};
  int first_zero = 0;
  if (!masks || masks[i]) {
    const float vcol[3] = {v_colors[i * 3 + 0], v_colors[i * 3 + 1], v_colors[i * 3 + 2]};
    sh_vjp3(degree, dirs[i * 3 + 0], dirs[i * 3 + 1], dirs[i * 3 + 2],
            coeffs + (uint64_t)i * K * 3, vcol, vc, v_dirs != nullptr, vd);
    first_zero = used;
  }
  for (uint32_t k = (uint32_t)first_zero * 3; k < K * 3; ++k) vc[k] = 0.f;
  if (v_dirs) {
    v_dirs[i * 3 + 0] = vd[0];
    v_dirs[i * 3 + 1] = vd[1];
    v_dirs[i * 3 + 2] = vd[2];
  }
}

extern "C" int tgs_compute_sh_fwd(uint32_t n, uint32_t K, int32_t degrees_to_use,
                                  const float* dirs, const float* coeffs, const uint8_t* masks,
                                  float* colors, hipStream_t stream) {
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(dirs && coeffs && colors, "compute_sh_fwd: null pointer");
  TGS_CHECK_ARG(degrees_to_use >= 0 && degrees_to_use <= 4, "degrees_to_use must be in [0,4]");
  TGS_CHECK_ARG((uint32_t)((degrees_to_use + 1) * (degrees_to_use + 1)) <= K,
                "coeffs has K=%u bases, degree %d needs %d", K, degrees_to_use,
                (degrees_to_use + 1) * (degrees_to_use + 1));
  hipLaunchKernelGGL(sh_fwd_kernel, dim3(tgs_blocks(n, 256)), dim3(256), 0, stream, n, K,
                     degrees_to_use, dirs, coeffs, masks, colors);
  TGS_RETURN_LAUNCH("tgs_compute_sh_fwd");
}

extern "C" int tgs_compute_sh_bwd(uint32_t n, uint32_t K, int32_t degrees_to_use,
                                  const float* dirs, const float* coeffs, const uint8_t* masks,
                                  const float* v_colors, float* v_coeffs, float* v_dirs,
                                  hipStream_t stream) {
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(dirs && coeffs && v_colors && v_coeffs, "compute_sh_bwd: null pointer");
  TGS_CHECK_ARG(degrees_to_use >= 0 && degrees_to_use <= 4, "degrees_to_use must be in [0,4]");
  TGS_CHECK_ARG((uint32_t)((degrees_to_use + 1) * (degrees_to_use + 1)) <= K,
                "coeffs has K=%u bases, degree %d needs %d", K, degrees_to_use,
                (degrees_to_use + 1) * (degrees_to_use + 1));
  hipLaunchKernelGGL(sh_bwd_kernel, dim3(tgs_blocks(n, 256)), dim3(256), 0, stream, n, K,
                     degrees_to_use, dirs, coeffs, masks, v_colors, v_coeffs, v_dirs);
  TGS_RETURN_LAUNCH("tgs_compute_sh_bwd");
}
