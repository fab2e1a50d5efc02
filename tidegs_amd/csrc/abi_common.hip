// Library-wide C-ABI helpers: version, last-error text, zero fill.
#include <stdarg.h>
#include <stdio.h>

#include "tgs_common.cuh"

static thread_local char g_last_error[512] = {0};

void tgs_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

extern "C" const char* tgs_last_error(void) { return g_last_error; }

extern "C" int tgs_abi_version(void) { return 1; }

// Grid-stride zero fill.  Used instead of hipMemsetAsync so every clear is a
// plain kernel node if a caller captures the stream into a HIP graph.
__global__ void fill_u32_kernel(uint32_t* __restrict__ p, uint64_t n, uint32_t value) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = value;
}

extern "C" int tgs_fill_u32(void* ptr, uint64_t n_words, uint32_t value, hipStream_t stream) {
  if (n_words == 0) return TGS_OK;
  TGS_CHECK_ARG(ptr != nullptr, "tgs_fill_u32: null pointer");
  uint64_t blocks = (n_words + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     (uint32_t*)ptr, n_words, value);
  TGS_RETURN_LAUNCH("tgs_fill_u32");
}

// VALU issue-rate probe (a measurement aid, like a plain copy for HBM): every
// thread runs `iters` rounds of 8 independent operations of one instruction
// form, i.e. 8 * iters wave64 VALU instructions per wavefront, and stores its
// results so that nothing is dropped.  Forms:
//   0  v_mul_f32, both operands in VGPRs (a per-lane factor just below 1)
//   1  v_mul_f32 with a scalar (SGPR) operand
//   2  v_add_u32 with both operands in VGPRs
//   3  v_xor_b32 with a scalar operand
//   4  v_fma_f32, three VGPR operands
//   5  v_exp_f32 (transcendental)
// On gfx950 form 0 issues fastest, so timing it gives the VALU roofline's
// peak rate on the machine at hand; the others show what the instruction form
// costs.
template <int FORM>
__global__ void __launch_bounds__(256) valu_probe_kernel(float* __restrict__ out, uint32_t iters,
                                                         float x) {
  float a[8];
  uint32_t u[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    a[k] = FORM == 5 ? (float)k * 0.1f : (float)(threadIdx.x + k);
    u[k] = threadIdx.x * 7u + (uint32_t)k;
  }
  const float z = x - (float)(threadIdx.x & 63) * 1e-9f;  // per lane: a VGPR operand
  const float y = (float)(threadIdx.x & 63) * 1e-9f;
  const uint32_t w = threadIdx.x * 3u + 1u;
  const uint32_t c = __float_as_uint(x);                  // uniform: an SGPR operand
  for (uint32_t i = 0; i < iters; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (FORM == 0) a[k] = a[k] * z;
      if (FORM == 1) a[k] = a[k] * x;
      if (FORM == 2) u[k] = u[k] + w;
      if (FORM == 3) u[k] = u[k] ^ c;
      if (FORM == 4) a[k] = fmaf(a[k], z, y);
      if (FORM == 5) a[k] = __builtin_amdgcn_exp2f(-a[k]);  // stays in [0.5, 1]
    }
    if (FORM == 4 || FORM == 5) asm volatile("" ::: "memory");
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += FORM == 2 || FORM == 3 ? (float)(u[k] & 0xffffu) : a[k];
  out[(uint64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

extern "C" int tgs_valu_probe(float* out, uint32_t blocks, uint32_t iters, int32_t form,
                              hipStream_t stream) {
  if (blocks == 0) return TGS_OK;
  TGS_CHECK_ARG(out != nullptr, "tgs_valu_probe: null pointer");
  TGS_CHECK_ARG(form >= 0 && form <= 5, "tgs_valu_probe: form must be 0..5");
  const dim3 g(blocks), b(256);
  const float x = 0.999999f;
  switch (form) {
    case 0: hipLaunchKernelGGL(valu_probe_kernel<0>, g, b, 0, stream, out, iters, x); break;
    case 1: hipLaunchKernelGGL(valu_probe_kernel<1>, g, b, 0, stream, out, iters, x); break;
    case 2: hipLaunchKernelGGL(valu_probe_kernel<2>, g, b, 0, stream, out, iters, x); break;
    case 3: hipLaunchKernelGGL(valu_probe_kernel<3>, g, b, 0, stream, out, iters, x); break;
    case 4: hipLaunchKernelGGL(valu_probe_kernel<4>, g, b, 0, stream, out, iters, x); break;
    default: hipLaunchKernelGGL(valu_probe_kernel<5>, g, b, 0, stream, out, iters, x); break;
  }
  TGS_RETURN_LAUNCH("tgs_valu_probe");
}
