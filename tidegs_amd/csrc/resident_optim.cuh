// Resident-slot optimizer building blocks shared by the standalone update
// (resident_optim.hip) and the fused projection-backward + update
// (tide_step.hip): the block layout lookup, the per-element Adam / Sophia
// update and raw buffer accesses.
#pragma once
#include "tgs_common.cuh"

#define TGS_MAX_COMP 8

__device__ __forceinline__ int64_t tgs_readlane_i64(int64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ float tgs_readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

struct OptimComponents {
  float* param[TGS_MAX_COMP];
  const float* grad[TGS_MAX_COMP];
  float* m[TGS_MAX_COMP];
  float* v[TGS_MAX_COMP];
  int width[TGS_MAX_COMP];
  int64_t pstride[TGS_MAX_COMP];  // row strides (elements) of param, grad, state
  int64_t gstride[TGS_MAX_COMP];
  int64_t sstride[TGS_MAX_COMP];
  float lr[TGS_MAX_COMP];
  int n;
  int total;    // sum of widths
  int unified;  // components are adjacent columns of one table for param,
                // grad and both states, each table with one row stride <= 64
  int pw, gw, sw;  // unified: the param, grad and state row strides
};

struct OptimLayout {
  const int64_t* starts;  // [L] sorted ascending
  const int64_t* ends;    // [L]
  const int64_t* slots;   // [L]
  int64_t n;              // L
  int64_t block_size;
  int block_shift;        // log2(block_size) when it is a power of two, else -1
};

// Resolve lane -> (component, column); lanes beyond the total width get comp=-1.
__device__ __forceinline__ void lane_column(const OptimComponents& c, int lane, int& comp,
                                            int& col) {
  comp = -1;
  col = 0;
  int base = 0;
#pragma unroll
  for (int k = 0; k < TGS_MAX_COMP; ++k) {
    if (k < c.n) {
      if (lane >= base && lane < base + c.width[k]) {
        comp = k;
        col = lane - base;
      }
      base += c.width[k];
    }
  }
}

// A wave-uniform 64-bit value loaded from memory, moved to scalar registers
// (the compiler cannot prove the layout tables read-only, so the loads are
// vector loads; the readfirstlane keeps everything derived from them scalar).
__device__ __forceinline__ int64_t tgs_uniform_i64(int64_t v) {
  return tgs_readlane_i64(v, 0);
}

// Number of ends <= row (searchsorted right=True), wave-uniform.
__device__ __forceinline__ int64_t layout_search(const OptimLayout& L, int64_t row) {
  int64_t lo = 0, hi = L.n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (tgs_uniform_i64(L.ends[mid]) <= row)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// The resident block holding the current rows: [start, end) -> slot.  Touched
// rows arrive sorted, so a wavefront walking a contiguous range of them
// searches the layout only when it crosses into another block.
struct BlockCache {
  int64_t start = 0, end = 0, slot = 0;  // empty until the first lookup
  int64_t s0 = -1;                       // starts[0], loaded on first use
  bool ok = false;
  __device__ __forceinline__ bool lookup(const OptimLayout& L, int64_t row) {
    if (row >= start && row < end) return true;
    // Blocks of a working set usually sit back to back from starts[0]: guess
    // the position from the row, check it with one pair of loads, and fall
    // back to the binary search when the guess misses.
    int64_t pos = -1;
    if (L.block_shift >= 0) {
      if (s0 < 0) s0 = tgs_uniform_i64(L.starts[0]);
      const int64_t g = row >= s0 ? (row - s0) >> L.block_shift : -1;
      if (g >= 0 && g < L.n) {
        const int64_t gs = tgs_uniform_i64(L.starts[g]), ge = tgs_uniform_i64(L.ends[g]);
        if (row >= gs && row < ge) pos = g;
      }
    }
    if (pos < 0) pos = layout_search(L, row);
    ok = false;
    start = end = 0;
    if (pos < L.n) {
      const int64_t s = tgs_uniform_i64(L.starts[pos]), e = tgs_uniform_i64(L.ends[pos]);
      if (row >= s && row < e && row - s < L.block_size) {
        start = s;
        // a slice longer than a block keeps only its first block_size rows:
        // later rows miss the cache, and the search rejects them
        end = e - s < L.block_size ? e : s + L.block_size;
        slot = tgs_uniform_i64(L.slots[pos]);
        ok = true;
      }
    }
    return ok;
  }
};

// Adam / Sophia update of one element; `sc` is lr / bias1 (Adam: the
// reference's rounding of (lr / bias1) * m) or lr (Sophia), `dsc` the slot's
// sqrt(1 - b2^t).  The moment EMAs are written as explicit fused
// multiply-adds (b * m + (1 - b) * g with one rounding of the sum), and
// contraction is otherwise off, so that every kernel that inlines this
// update rounds identically.
// POW2_BS: batch_size is a power of two, so g / batch_size is exactly
// g * (1 / batch_size) (both round the same exact value once).
template <bool SOPHIA, bool POW2_BS = false>
__device__ __forceinline__ void optim_update(float gv, float& mv, float& vv, float& pv, float sc,
                                             float dsc, float beta1, float beta2, float one_m_b1,
                                             float one_m_b2, float eps, float batch_size,
                                             float rho, int update_h) {
#pragma clang fp contract(off)
  const float gg = POW2_BS ? gv * (1.0f / batch_size) : gv / batch_size;
  mv = __builtin_fmaf(beta1, mv, one_m_b1 * gg);
  if (SOPHIA) {
    if (update_h) vv = __builtin_fmaf(beta2, vv, (one_m_b2 * gg) * gg);
    float r = mv / fmaxf(vv, eps);
    r = fminf(fmaxf(r, -rho), rho);
    pv -= sc * r;
  } else {
    vv = __builtin_fmaf(beta2, vv, (one_m_b2 * gg) * gg);
    const float denom = sqrtf(vv) / dsc + eps;
    pv -= sc * mv / denom;
  }
}


// Raw dword buffer over [base, base + bytes): an access whose byte offset
// (lane offset + scalar offset) falls outside the range reads 0 or is dropped
// by the address unit.  The third-dword value
// is the gfx9-family raw-buffer format (32-bit data, no swizzle).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tgs_rsrc(const float* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, (int)bytes, 0x00020000);
}
// The b32 builtins move raw 32-bit words: reinterpret, never convert.
__device__ __forceinline__ float tgs_bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ void tgs_bstore(float v, __amdgpu_buffer_rsrc_t r, uint32_t voff,
                                           uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voff, soff, 0);
}
// Non-temporal forms (cache policy nt) for the optimizer state: each touched
// row's moments are read once and each row's p, m, v written once per step,
// and nothing reads them again before the next step, so they stream past the
// caches instead of displacing the step's reused data (fused update at cfg3:
// 1.90 -> 1.83 ms with the moments' loads and all three stores so marked).
__device__ __forceinline__ float tgs_bload_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                              uint32_t soff) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 2));
}
__device__ __forceinline__ void tgs_bstore_nt(float v, __amdgpu_buffer_rsrc_t r, uint32_t voff,
                                              uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voff, soff, 2);
}
// A lane offset that every range check rejects (with any scalar offset below
// 2^31 added it stays at or above 2^31, beyond every descriptor's range).
#define TGS_OFF_NONE 0x80000000u
