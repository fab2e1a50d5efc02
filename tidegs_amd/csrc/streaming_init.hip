// GPU build of the Morton-sorted base file (the streaming PLY initializer).
//
// TideGS's streaming_ply_to_ssd_base (storage/streaming_ply_init.py:541-696)
// turns a PLY into base_file.bin on the CPU: Morton codes of the positions,
// records bucketed by the top 10 code bits into temporary files, each bucket
// sorted in memory (or split again by the next 10 bits when it exceeds the
// sort-memory limit, down to whole codes), a log-scale per sorted bucket, and
// per-block xyz bounds.  The order it produces is the stable sort of the
// vertices by Morton code; the buckets only decide which rows share a scale.
// With the scene in HBM (288 GB holds ~1.2 billion 236-byte rows) the same
// result comes from one sort and a few passes:
//   tgs_init_scene_bounds  - xyz min/max (pass 1 of the reference)
//   tgs_init_morton_codes  - 30-bit codes (streaming_ply_init.py:154-168)
//   (stable radix sort of (code, vertex) pairs: tgs_segmented_sort_pairs_u32)
//   tgs_init_prefix_counts - sizes of the 10-bit and 20-bit code buckets
//   tgs_init_leaf_flags    - first row of every sorted bucket ("leaf"): the
//                            bucket level is chosen from those sizes exactly
//                            as the recursion of :319-538 chooses it
//   tgs_init_leaf_stats    - per-leaf xyz min/max and row count
//   tgs_init_pack_rows     - the 59-float rows of :234-248 in sorted order
//                            with their leaf's log-scale
// and the per-block bounds come from tgs_ws_block_bounds.
#include "tgs_common.cuh"

#define INIT_THREADS 256

namespace {

// Order-preserving map of a float to uint32 (for atomic min/max).
__device__ __forceinline__ uint32_t ord_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float ord_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o));
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o));
  return v;
}

__global__ void init_bounds_reset_kernel(uint32_t* keys) {
  if (threadIdx.x < 6) keys[threadIdx.x] = threadIdx.x < 3 ? 0xffffffffu : 0u;
}

__global__ __launch_bounds__(INIT_THREADS) void init_scene_bounds_kernel(
    const float* __restrict__ xyz, uint64_t n, uint32_t* __restrict__ keys) {
  uint32_t lo[3] = {0xffffffffu, 0xffffffffu, 0xffffffffu}, hi[3] = {0u, 0u, 0u};
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const uint32_t k = ord_key(xyz[i * 3 + d]);
      lo[d] = min(lo[d], k);
      hi[d] = max(hi[d], k);
    }
  }
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    lo[d] = wave_min_u32(lo[d]);
    hi[d] = wave_max_u32(hi[d]);
  }
  if ((threadIdx.x & (TGS_WAVE - 1)) == 0) {
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      atomicMin(&keys[d], lo[d]);
      atomicMax(&keys[3 + d], hi[d]);
    }
  }
}

__global__ void init_bounds_finish_kernel(const uint32_t* keys, float* bounds) {
  if (threadIdx.x < 6) bounds[threadIdx.x] = ord_float(keys[threadIdx.x]);
}

// 10-bit spread of one axis (streaming_ply_init.py:158-163).
__device__ __forceinline__ uint32_t spread_bits(uint32_t v) {
  v = (v | (v << 16)) & 0x030000FFu;
  v = (v | (v << 8)) & 0x0300F00Fu;
  v = (v | (v << 4)) & 0x030C30C3u;
  v = (v | (v << 2)) & 0x09249249u;
  return v;
}

__global__ __launch_bounds__(INIT_THREADS) void init_morton_kernel(
    const float* __restrict__ xyz, uint64_t n, const float* __restrict__ bounds,
    uint32_t* __restrict__ codes) {
  float mn[3], den[3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    mn[d] = bounds[d];
    // (max - min) + 1e-8 in float32, as numpy evaluates it
    den[d] = __fadd_rn(__fsub_rn(bounds[3 + d], bounds[d]), 1e-8f);
  }
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    uint32_t q[3];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const float norm = __fdiv_rn(__fsub_rn(xyz[i * 3 + d], mn[d]), den[d]);
      const float s = __fmul_rn(norm, 1023.0f);
      // astype(uint32) truncates; the value is >= 0 for points inside the bounds
      uint32_t v = s >= 4294967040.0f ? 0xffffffffu : (s > 0.0f ? (uint32_t)s : 0u);
      q[d] = v > 1023u ? 1023u : v;
    }
    codes[i] = spread_bits(q[0]) | (spread_bits(q[1]) << 1) | (spread_bits(q[2]) << 2);
  }
}

__global__ __launch_bounds__(INIT_THREADS) void init_prefix_counts_kernel(
    const uint32_t* __restrict__ codes, uint64_t n, uint32_t* __restrict__ counts0,
    uint32_t* __restrict__ counts1) {
  __shared__ uint32_t h0[1024];
  for (int j = threadIdx.x; j < 1024; j += INIT_THREADS) h0[j] = 0;
  __syncthreads();
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    const uint32_t c = codes[i];
    atomicAdd(&h0[(c >> 20) & 1023u], 1u);
    atomicAdd(&counts1[(c >> 10) & 0xFFFFFu], 1u);
  }
  __syncthreads();
  for (int j = threadIdx.x; j < 1024; j += INIT_THREADS)
    if (h0[j]) atomicAdd(&counts0[j], h0[j]);
}

// Leaf key of a code: its 10-bit bucket when that bucket fits the sort
// memory, else its 20-bit child when that fits, else the whole code.
__device__ __forceinline__ uint64_t leaf_key(uint32_t c, const uint8_t* big0, const uint8_t* big1) {
  const uint32_t p0 = (c >> 20) & 1023u, p1 = (c >> 10) & 0xFFFFFu;
  if (!big0[p0]) return ((uint64_t)0 << 32) | p0;
  if (!big1[p1]) return ((uint64_t)1 << 32) | p1;
  return ((uint64_t)2 << 32) | c;
}

__global__ __launch_bounds__(INIT_THREADS) void init_leaf_flags_kernel(
    const uint32_t* __restrict__ codes, uint64_t n, const uint8_t* __restrict__ big0,
    const uint8_t* __restrict__ big1, int32_t* __restrict__ flags) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    const uint64_t k = leaf_key(codes[i], big0, big1);
    flags[i] = (i == 0 || leaf_key(codes[i - 1], big0, big1) != k) ? 1 : 0;
  }
}

// stats[leaf * 8 + {0..2}] = ord_key(min xyz), {3..5} = ord_key(max xyz),
// {6} = rows, {7} = the code of the leaf's first row.  Sorted rows make most
// waves fall in one leaf: those reduce in registers and add once.
__global__ __launch_bounds__(INIT_THREADS) void init_leaf_stats_kernel(
    const int64_t* __restrict__ leaf_incl, const uint32_t* __restrict__ sorted_codes,
    const uint32_t* __restrict__ perm, const float* __restrict__ xyz, uint64_t n,
    uint32_t* __restrict__ stats) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  // every lane of a wave runs the same trip count (uniform loop bound)
  const uint64_t base0 = (uint64_t)blockIdx.x * blockDim.x + (threadIdx.x & ~(uint64_t)(TGS_WAVE - 1));
  for (uint64_t w0 = base0; w0 < n; w0 += stride) {
    const uint64_t i = w0 + (threadIdx.x & (TGS_WAVE - 1));
    const bool live = i < n;
    int64_t leaf = -1;
    uint32_t k[3] = {0xffffffffu, 0xffffffffu, 0xffffffffu};
    uint32_t km[3] = {0u, 0u, 0u};
    if (live) {
      leaf = leaf_incl[i] - 1;
      const uint32_t v = perm[i];
#pragma unroll
      for (int d = 0; d < 3; ++d) k[d] = km[d] = ord_key(xyz[(uint64_t)v * 3 + d]);
      if (i == 0 || leaf_incl[i - 1] != leaf_incl[i]) stats[(uint64_t)leaf * 8 + 7] = sorted_codes[i];
    }
    const int64_t first = __shfl(leaf, 0);
    const bool uniform = __all(!live || leaf == first);
    if (uniform) {
      const uint32_t cnt = (uint32_t)__popcll(__ballot(live));
#pragma unroll
      for (int d = 0; d < 3; ++d) {
        k[d] = wave_min_u32(k[d]);
        km[d] = wave_max_u32(km[d]);
      }
      if ((threadIdx.x & (TGS_WAVE - 1)) == 0) {
        uint32_t* s = stats + (uint64_t)first * 8;
#pragma unroll
        for (int d = 0; d < 3; ++d) {
          atomicMin(&s[d], k[d]);
          atomicMax(&s[3 + d], km[d]);
        }
        atomicAdd(&s[6], cnt);
      }
    } else if (live) {
      uint32_t* s = stats + (uint64_t)leaf * 8;
#pragma unroll
      for (int d = 0; d < 3; ++d) {
        atomicMin(&s[d], k[d]);
        atomicMax(&s[3 + d], km[d]);
      }
      atomicAdd(&s[6], 1u);
    }
  }
}

__global__ void init_stats_reset_kernel(uint32_t* stats, uint64_t n_leaves) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n_leaves * 8; i += stride) {
    const uint32_t f = (uint32_t)(i & 7);
    stats[i] = f < 3 ? 0xffffffffu : 0u;
  }
}

__global__ void init_stats_finish_kernel(uint32_t* stats, uint64_t n_leaves) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n_leaves * 8; i += stride) {
    const uint32_t f = (uint32_t)(i & 7);
    if (f < 6) stats[i] = __float_as_uint(ord_float(stats[i]));
  }
}

// Row r of the base file (streaming_ply_init.py:234-248, scale from :361-367):
// xyz | leaf log-scale x3 | (1,0,0,0) | opacity logit | dc | 45 zeros.
// A workgroup writes 64 consecutive rows (64*59 floats) with stores
// contiguous across the wave; units are dealt grid-stride.
__global__ __launch_bounds__(INIT_THREADS) void init_pack_rows_kernel(
    const uint32_t* __restrict__ perm, const int64_t* __restrict__ leaf_incl,
    const float* __restrict__ xyz, const float* __restrict__ dc,
    const float* __restrict__ leaf_scales, float opacity_logit, uint64_t n,
    float* __restrict__ table) {
  constexpr int K = (64 * 59 + INIT_THREADS - 1) / INIT_THREADS;
  const uint64_t units = (n + 63) / 64;
  for (uint64_t u = blockIdx.x; u < units; u += gridDim.x) {
    const uint64_t r0 = u * 64;
    const int nrows = (int)((n - r0) < 64 ? (n - r0) : 64);
    const int nel = nrows * 59;
    float* __restrict__ out = table + r0 * 59;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int e = threadIdx.x + k * INIT_THREADS;
      if (e >= nel) continue;
      const int rl = e / 59;
      const int c = e - rl * 59;
      const uint64_t r = r0 + rl;
      float v = 0.0f;
      if (c < 3) {
        v = xyz[(uint64_t)perm[r] * 3 + c];
      } else if (c < 6) {
        v = leaf_scales[leaf_incl[r] - 1];
      } else if (c == 6) {
        v = 1.0f;
      } else if (c == 10) {
        v = opacity_logit;
      } else if (c >= 11 && c < 14) {
        v = dc[(uint64_t)perm[r] * 3 + (c - 11)];
      }
      out[e] = v;
    }
  }
}

unsigned grid_for(uint64_t n, unsigned cap = 8192) {
  uint64_t g = (n + INIT_THREADS - 1) / INIT_THREADS;
  if (g > cap) g = cap;
  if (g == 0) g = 1;
  return (unsigned)g;
}

}  // namespace

extern "C" int tgs_init_scene_bounds(const float* xyz, uint64_t n, uint32_t* scratch,
                                     float* bounds, hipStream_t stream) {
  const char* name = "tgs_init_scene_bounds";
  TGS_CHECK_ARG(n > 0, "%s: no points", name);
  TGS_CHECK_ARG(xyz && scratch && bounds, "%s: null pointer", name);
  hipLaunchKernelGGL(init_bounds_reset_kernel, dim3(1), dim3(64), 0, stream, scratch);
  TGS_LAUNCH_CHECK(name);
  hipLaunchKernelGGL(init_scene_bounds_kernel, dim3(grid_for(n, 2048)), dim3(INIT_THREADS), 0,
                     stream, xyz, n, scratch);
  TGS_LAUNCH_CHECK(name);
  hipLaunchKernelGGL(init_bounds_finish_kernel, dim3(1), dim3(64), 0, stream, scratch, bounds);
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_init_morton_codes(const float* xyz, uint64_t n, const float* bounds,
                                     uint32_t* codes, hipStream_t stream) {
  const char* name = "tgs_init_morton_codes";
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(xyz && bounds && codes, "%s: null pointer", name);
  hipLaunchKernelGGL(init_morton_kernel, dim3(grid_for(n)), dim3(INIT_THREADS), 0, stream, xyz, n,
                     bounds, codes);
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_init_prefix_counts(const uint32_t* codes, uint64_t n, uint32_t* counts0,
                                      uint32_t* counts1, hipStream_t stream) {
  const char* name = "tgs_init_prefix_counts";
  TGS_CHECK_ARG(counts0 && counts1, "%s: null pointer", name);
  int rc = tgs_fill_u32(counts0, 1024, 0u, stream);
  if (rc) return rc;
  rc = tgs_fill_u32(counts1, 1u << 20, 0u, stream);
  if (rc) return rc;
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(codes, "%s: null pointer", name);
  hipLaunchKernelGGL(init_prefix_counts_kernel, dim3(grid_for(n, 2048)), dim3(INIT_THREADS), 0,
                     stream, codes, n, counts0, counts1);
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_init_leaf_flags(const uint32_t* sorted_codes, uint64_t n, const uint8_t* big0,
                                   const uint8_t* big1, int32_t* flags, hipStream_t stream) {
  const char* name = "tgs_init_leaf_flags";
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(sorted_codes && big0 && big1 && flags, "%s: null pointer", name);
  hipLaunchKernelGGL(init_leaf_flags_kernel, dim3(grid_for(n)), dim3(INIT_THREADS), 0, stream,
                     sorted_codes, n, big0, big1, flags);
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_init_leaf_stats(const int64_t* leaf_incl, const uint32_t* sorted_codes,
                                   const uint32_t* perm, const float* xyz, uint64_t n,
                                   uint64_t n_leaves, uint32_t* stats, hipStream_t stream) {
  const char* name = "tgs_init_leaf_stats";
  if (n == 0 || n_leaves == 0) return TGS_OK;
  TGS_CHECK_ARG(leaf_incl && sorted_codes && perm && xyz && stats, "%s: null pointer", name);
  hipLaunchKernelGGL(init_stats_reset_kernel, dim3(grid_for(n_leaves * 8)), dim3(INIT_THREADS), 0,
                     stream, stats, n_leaves);
  TGS_LAUNCH_CHECK(name);
  hipLaunchKernelGGL(init_leaf_stats_kernel, dim3(grid_for(n)), dim3(INIT_THREADS), 0, stream,
                     leaf_incl, sorted_codes, perm, xyz, n, stats);
  TGS_LAUNCH_CHECK(name);
  hipLaunchKernelGGL(init_stats_finish_kernel, dim3(grid_for(n_leaves * 8)), dim3(INIT_THREADS), 0,
                     stream, stats, n_leaves);
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_init_pack_rows(const uint32_t* perm, const int64_t* leaf_incl, const float* xyz,
                                  const float* dc, const float* leaf_scales, float opacity_logit,
                                  uint64_t n, float* table, hipStream_t stream) {
  const char* name = "tgs_init_pack_rows";
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(perm && leaf_incl && xyz && dc && leaf_scales && table, "%s: null pointer", name);
  uint64_t units = (n + 63) / 64;
  hipLaunchKernelGGL(init_pack_rows_kernel, dim3((unsigned)(units < 8192 ? units : 8192)),
                     dim3(INIT_THREADS), 0,
                     stream, perm, leaf_incl, xyz, dc, leaf_scales, opacity_logit, n, table);
  TGS_RETURN_LAUNCH(name);
}
