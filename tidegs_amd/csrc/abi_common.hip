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
