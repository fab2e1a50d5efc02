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
// thread runs `iters` rounds of 8 independent fused multiply-adds, i.e.
// 8 * iters wave64 v_fma_f32 instructions per wavefront, and stores its sums so
// that nothing is dropped.  Timing it gives the VALU roofline's peak rate on
// the machine at hand (wave64 FMA instructions per second).
__global__ void __launch_bounds__(256) valu_probe_kernel(float* __restrict__ out, uint32_t iters,
                                                         float x) {
  float a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) a[k] = (float)(threadIdx.x + k);
  const float y = x * 0.5f;
  for (uint32_t i = 0; i < iters; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k) a[k] = fmaf(a[k], x, y);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += a[k];
  out[(uint64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

extern "C" int tgs_valu_probe(float* out, uint32_t blocks, uint32_t iters, hipStream_t stream) {
  if (blocks == 0) return TGS_OK;
  TGS_CHECK_ARG(out != nullptr, "tgs_valu_probe: null pointer");
  hipLaunchKernelGGL(valu_probe_kernel, dim3(blocks), dim3(256), 0, stream, out, iters,
                     0.999999f);
  TGS_RETURN_LAUNCH("tgs_valu_probe");
}
