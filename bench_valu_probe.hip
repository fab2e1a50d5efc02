// VALU issue-rate probe for bench.py's compositing-kernel roofline: a
// measurement aid with no counterpart in the reference, built into its own
// library (bench_valu_probe.so) beside bench.py and never part of
// libtidegs_amd.so.
//
#include <hip/hip_runtime.h>
#include <stdint.h>

// Like a plain copy for HBM, a synthetic stream for the VALU: every
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
  if (blocks == 0) return 0;
  if (out == nullptr || form < 0 || form > 5) return -1;
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
  return (int)hipGetLastError();
}
