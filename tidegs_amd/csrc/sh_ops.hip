// gsplat-compatible spherical_harmonics forward/backward.
//
// Reference: gsplat/cuda/csrc/compute_sh_fwd.cu:9-58, compute_sh_bwd.cu:68-136.
// dirs [n,3], coeffs [n,K,3], masks [n] (bool, optional), colors [n,3].
// One lane per element evaluates all three channels from one basis pass
// (the reference runs one thread per (element, channel)).  The backward
// writes every v_coeffs entry (zeros above the active degree and for masked
// elements) and writes v_dirs directly, so no zero-fill or atomics are needed.
#include "sh.cuh"

// One thread per element; the basis count K is a template parameter, so an
// element's coefficient row (3K floats) lives in registers and, for K = 4 and
// 16 (rows of 48 and 192 bytes, 16-byte aligned), moves as 16-byte loads and
// stores: 12 vector stores per row instead of 48 scalar ones, which is what
// keeps the backward's row writes from fragmenting into partial lines.
template <int K, bool VEC>
__device__ __forceinline__ void sh_row_load(const float* __restrict__ src, float (&r)[3 * K]) {
  if constexpr (VEC && (3 * K) % 4 == 0) {
    const float4* s4 = reinterpret_cast<const float4*>(src);
#pragma unroll
    for (int j = 0; j < 3 * K / 4; ++j) {
      const float4 v = s4[j];
      r[4 * j] = v.x;
      r[4 * j + 1] = v.y;
      r[4 * j + 2] = v.z;
      r[4 * j + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 3 * K; ++j) r[j] = src[j];
  }
}

template <int K, bool VEC>
__device__ __forceinline__ void sh_row_store(float* __restrict__ dst, const float (&r)[3 * K]) {
  if constexpr (VEC && (3 * K) % 4 == 0) {
    float4* d4 = reinterpret_cast<float4*>(dst);
#pragma unroll
    for (int j = 0; j < 3 * K / 4; ++j)
      d4[j] = make_float4(r[4 * j], r[4 * j + 1], r[4 * j + 2], r[4 * j + 3]);
  } else {
#pragma unroll
    for (int j = 0; j < 3 * K; ++j) dst[j] = r[j];
  }
}

template <int K, bool VEC>
__global__ void __launch_bounds__(256) sh_fwd_kernel(uint32_t n, int degree,
                                                     const float* __restrict__ dirs,
                                                     const float* __restrict__ coeffs,
                                                     const uint8_t* __restrict__ masks,
                                                     float* __restrict__ colors) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float out[3] = {0.f, 0.f, 0.f};
  if (!masks || masks[i]) {
    float c[3 * K];
    sh_row_load<K, VEC>(coeffs + (uint64_t)i * 3 * K, c);
    sh_eval3(degree, dirs[i * 3 + 0], dirs[i * 3 + 1], dirs[i * 3 + 2], c, out);
  }
  colors[i * 3 + 0] = out[0];
  colors[i * 3 + 1] = out[1];
  colors[i * 3 + 2] = out[2];
}

template <int K, bool VEC>
__global__ void __launch_bounds__(256) sh_bwd_kernel(uint32_t n, int degree,
                                                     const float* __restrict__ dirs,
                                                     const float* __restrict__ coeffs,
                                                     const uint8_t* __restrict__ masks,
                                                     const float* __restrict__ v_colors,
                                                     float* __restrict__ v_coeffs,
                                                     float* __restrict__ v_dirs) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float vc[3 * K];
#pragma unroll
  for (int k = 0; k < 3 * K; ++k) vc[k] = 0.f;
  float vd[3] = {0.f, 0.f, 0.f};
  if (!masks || masks[i]) {
    const float vcol[3] = {v_colors[i * 3 + 0], v_colors[i * 3 + 1], v_colors[i * 3 + 2]};
    float c[3 * K];
    if (v_dirs) sh_row_load<K, VEC>(coeffs + (uint64_t)i * 3 * K, c);
    sh_vjp3(degree, dirs[i * 3 + 0], dirs[i * 3 + 1], dirs[i * 3 + 2], c, vcol, vc,
            v_dirs != nullptr, vd);
  }
  sh_row_store<K, VEC>(v_coeffs + (uint64_t)i * 3 * K, vc);
  if (v_dirs) {
    v_dirs[i * 3 + 0] = vd[0];
    v_dirs[i * 3 + 1] = vd[1];
    v_dirs[i * 3 + 2] = vd[2];
  }
}

// Any other basis count (K >= (degree + 1)^2): rows addressed in memory.
__global__ void __launch_bounds__(256) sh_fwd_any_kernel(uint32_t n, uint32_t K, int degree,
                                                         const float* __restrict__ dirs,
                                                         const float* __restrict__ coeffs,
                                                         const uint8_t* __restrict__ masks,
                                                         float* __restrict__ colors) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float out[3] = {0.f, 0.f, 0.f};
  if (!masks || masks[i])
    sh_eval3(degree, dirs[i * 3 + 0], dirs[i * 3 + 1], dirs[i * 3 + 2],
             coeffs + (uint64_t)i * K * 3, out);
  colors[i * 3 + 0] = out[0];
  colors[i * 3 + 1] = out[1];
  colors[i * 3 + 2] = out[2];
}

__global__ void __launch_bounds__(256) sh_bwd_any_kernel(uint32_t n, uint32_t K, int degree,
                                                         const float* __restrict__ dirs,
                                                         const float* __restrict__ coeffs,
                                                         const uint8_t* __restrict__ masks,
                                                         const float* __restrict__ v_colors,
                                                         float* __restrict__ v_coeffs,
                                                         float* __restrict__ v_dirs) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float* vc = v_coeffs + (uint64_t)i * K * 3;
  float vd[3] = {0.f, 0.f, 0.f};
  uint32_t first_zero = 0;
  if (!masks || masks[i]) {
    const float vcol[3] = {v_colors[i * 3 + 0], v_colors[i * 3 + 1], v_colors[i * 3 + 2]};
    sh_vjp3(degree, dirs[i * 3 + 0], dirs[i * 3 + 1], dirs[i * 3 + 2],
            coeffs + (uint64_t)i * K * 3, vcol, vc, v_dirs != nullptr, vd);
    first_zero = (uint32_t)((degree + 1) * (degree + 1));
  }
  for (uint32_t k = first_zero * 3; k < K * 3; ++k) vc[k] = 0.f;
  if (v_dirs) {
    v_dirs[i * 3 + 0] = vd[0];
    v_dirs[i * 3 + 1] = vd[1];
    v_dirs[i * 3 + 2] = vd[2];
  }
}

#define TGS_SH_BASES(X) X(1) X(4) X(9) X(16) X(25)

extern "C" int tgs_compute_sh_fwd(uint32_t n, uint32_t K, int32_t degrees_to_use,
                                  const float* dirs, const float* coeffs, const uint8_t* masks,
                                  float* colors, hipStream_t stream) {
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(dirs && coeffs && colors, "compute_sh_fwd: null pointer");
  TGS_CHECK_ARG(degrees_to_use >= 0 && degrees_to_use <= 4, "degrees_to_use must be in [0,4]");
  TGS_CHECK_ARG((uint32_t)((degrees_to_use + 1) * (degrees_to_use + 1)) <= K,
                "coeffs has K=%u bases, degree %d needs %d", K, degrees_to_use,
                (degrees_to_use + 1) * (degrees_to_use + 1));
  const bool vec = ((uintptr_t)coeffs & 15u) == 0;
#define TGS_SH_FWD_CASE(B)                                                                    \
  case B:                                                                                      \
    if (vec)                                                                                   \
      hipLaunchKernelGGL((sh_fwd_kernel<B, true>), dim3(tgs_blocks(n, 256)), dim3(256), 0,      \
                         stream, n, degrees_to_use, dirs, coeffs, masks, colors);              \
    else                                                                                       \
      hipLaunchKernelGGL((sh_fwd_kernel<B, false>), dim3(tgs_blocks(n, 256)), dim3(256), 0,     \
                         stream, n, degrees_to_use, dirs, coeffs, masks, colors);              \
    break;
  switch (K) {
    TGS_SH_BASES(TGS_SH_FWD_CASE)
    default:
      hipLaunchKernelGGL(sh_fwd_any_kernel, dim3(tgs_blocks(n, 256)), dim3(256), 0, stream, n,
                         K, degrees_to_use, dirs, coeffs, masks, colors);
  }
#undef TGS_SH_FWD_CASE
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
  const bool vec = ((uintptr_t)coeffs & 15u) == 0 && ((uintptr_t)v_coeffs & 15u) == 0;
#define TGS_SH_BWD_CASE(B)                                                                    \
  case B:                                                                                      \
    if (vec)                                                                                   \
      hipLaunchKernelGGL((sh_bwd_kernel<B, true>), dim3(tgs_blocks(n, 256)), dim3(256), 0,      \
                         stream, n, degrees_to_use, dirs, coeffs, masks, v_colors, v_coeffs,    \
                         v_dirs);                                                              \
    else                                                                                       \
      hipLaunchKernelGGL((sh_bwd_kernel<B, false>), dim3(tgs_blocks(n, 256)), dim3(256), 0,     \
                         stream, n, degrees_to_use, dirs, coeffs, masks, v_colors, v_coeffs,    \
                         v_dirs);                                                              \
    break;
  switch (K) {
    TGS_SH_BASES(TGS_SH_BWD_CASE)
    default:
      hipLaunchKernelGGL(sh_bwd_any_kernel, dim3(tgs_blocks(n, 256)), dim3(256), 0, stream, n,
                         K, degrees_to_use, dirs, coeffs, masks, v_colors, v_coeffs, v_dirs);
  }
#undef TGS_SH_BWD_CASE
  TGS_RETURN_LAUNCH("tgs_compute_sh_bwd");
}
