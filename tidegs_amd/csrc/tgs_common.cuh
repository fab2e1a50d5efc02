// Shared device helpers for the TideGS MI355X (gfx950, CDNA4) kernels.
//
// Everything here is written for 64-lane wavefronts.  Matrices are plain
// row-major float arrays (M[r][c]); there is no glm and no CUDA shim.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define TGS_WAVE 64

// Status codes returned by every extern "C" entry point (0 = success,
// positive = hipError_t, negative = argument errors detected on the host).
enum {
  TGS_OK = 0,
  TGS_ERR_ARG = -1,        // invalid size / null pointer
  TGS_ERR_UNSUPPORTED = -2, // e.g. channel count not instantiated
  TGS_ERR_WORKSPACE = -3,  // workspace smaller than the queried size
};

// Per-thread last-error text for the host wrapper (reentrant across threads).
void tgs_set_error(const char* fmt, ...);

// Word fill kernel launch (abi_common.hip), used instead of hipMemsetAsync.
extern "C" int tgs_fill_u32(void* ptr, uint64_t n_words, uint32_t value, hipStream_t stream);

#define TGS_CHECK_ARG(cond, ...)          \
  do {                                    \
    if (!(cond)) {                        \
      tgs_set_error(__VA_ARGS__);         \
      return TGS_ERR_ARG;                 \
    }                                     \
  } while (0)

#define TGS_RETURN_LAUNCH(name)                                     \
  do {                                                              \
    hipError_t _e = hipGetLastError();                              \
    if (_e != hipSuccess) {                                         \
      tgs_set_error("%s: launch failed: %s", name, hipGetErrorString(_e)); \
      return (int)_e;                                               \
    }                                                               \
    return TGS_OK;                                                  \
  } while (0)

#define TGS_LAUNCH_CHECK(name)                                      \
  do {                                                              \
    hipError_t _e = hipGetLastError();                              \
    if (_e != hipSuccess) {                                         \
      tgs_set_error("%s: launch failed: %s", name, hipGetErrorString(_e)); \
      return (int)_e;                                               \
    }                                                               \
  } while (0)

static inline unsigned tgs_blocks(uint64_t n, unsigned threads) {
  return (unsigned)((n + threads - 1) / threads);
}

// ---------------------------------------------------------------------------
// Small float math
// ---------------------------------------------------------------------------

// exp(x) = 2^(x * log2(e)) on the hardware exp2 unit (v_exp_f32, ~1 ulp on
// the exp2 result; total relative error <= ~(1 + |x|) * 2^-23 for the
// |x| <= 20 range the compositing kernels use).  Inputs below -126/log2(e)
// flush to zero like the hardware instruction does.
__device__ __forceinline__ float tgs_fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

struct m3 {
  float m[3][3];
};

__device__ __forceinline__ m3 m3_mul(const m3& a, const m3& b) {
  m3 r;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      r.m[i][j] = a.m[i][0] * b.m[0][j] + a.m[i][1] * b.m[1][j] + a.m[i][2] * b.m[2][j];
  return r;
}

// a * b^T
__device__ __forceinline__ m3 m3_mul_bt(const m3& a, const m3& b) {
  m3 r;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      r.m[i][j] = a.m[i][0] * b.m[j][0] + a.m[i][1] * b.m[j][1] + a.m[i][2] * b.m[j][2];
  return r;
}

// a^T * b
__device__ __forceinline__ m3 m3_mul_at(const m3& a, const m3& b) {
  m3 r;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      r.m[i][j] = a.m[0][i] * b.m[0][j] + a.m[1][i] * b.m[1][j] + a.m[2][i] * b.m[2][j];
  return r;
}

// ---------------------------------------------------------------------------
// Wavefront (64-lane) reductions built on DPP.  After the row steps every lane
// of a 16-lane row holds its row sum; row_bcast:15 / row_bcast:31 then carry
// the row sums upward so that lane 63 holds the wave total, which readlane
// returns as a wave-uniform value.
// ---------------------------------------------------------------------------

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf, bool BOUND_CTRL = false>
__device__ __forceinline__ float tgs_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK,
                                                    BANK_MASK, BOUND_CTRL));
}

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf, bool BOUND_CTRL = false>
__device__ __forceinline__ uint32_t tgs_dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, BANK_MASK, BOUND_CTRL);
}

__device__ __forceinline__ float tgs_wave_sum(float v) {
  v += tgs_dpp<0xB1>(v);           // quad_perm [1,0,3,2]
  v += tgs_dpp<0x4E>(v);           // quad_perm [2,3,0,1]
  v += tgs_dpp<0x141>(v);          // row_half_mirror
  v += tgs_dpp<0x140>(v);          // row_mirror
  v += tgs_dpp<0x142, 0xa>(v);     // row_bcast:15 into rows 1 and 3
  v += tgs_dpp<0x143, 0xc>(v);     // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ int tgs_wave_max_i32(int v) {
  // Butterfly over ds_swizzle-free xor shuffles; only used once per tile.
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    int o = __shfl_xor(v, off, 64);
    v = v > o ? v : o;
  }
  return v;
}

__device__ __forceinline__ uint64_t tgs_ballot(bool p) {
  return __ballot(p);
}

__device__ __forceinline__ void tgs_atomic_add(float* p, float v) {
  unsafeAtomicAdd(p, v);
}
