// Resident-set materialization and writeback over the resident fp32 table.
//
// The resident working set is ONE row-major table of Gaussians in CACHE
// column order (xyz 0:3 | scaling 3:6 | rotation 6:10 | opacity 10 |
// features_dc 11:14 | features_rest 14:59), with a row pitch of 59 floats
// (dense) or 64 floats (padded: every row one 256-byte line, padding zero),
// plus an int64 local->global id per row.  TideGS keeps six component tensors
// per buffer and moves them with Triton kernels
// (strategies/tide_engine/double_buffer_gpu.py:38-210,
// strategies/tide_engine/gpu_working_set.py:33-116); with one table every one
// of those moves is a segmented row copy, so one templated mover serves them
// all:
//   copy kept blocks   (double_buffer_gpu.py:41-128, :811-872)
//   unpack streamed    (double_buffer_gpu.py:151-210, :1060-1082), CACHE or
//                      UNIFIED packed rows, with the cold-id fill (:130-149,
//                      :928-963) fused in
//   pack dirty rows    (gpu_working_set.py:33-87, :895-988)
// and two more kernels do the per-block xyz bounds
// (gpu_working_set.py:89-116, :990-1062) and the compact block-start
// table and global->local map (double_buffer_gpu.py:212-255).
//
// Work unit of the mover: 64 consecutive rows of one block segment.  A
// workgroup of 256 threads moves the unit's 64*DP destination floats with
// dword accesses that are contiguous across the wave (each wave instruction
// touches 256 consecutive bytes), every thread holding its ceil(64*DP/256)
// loads in flight before its stores.  Padding columns of a 64-pitch
// destination are written as zeros, so a padded table keeps whole-line rows
// and zero padding.  Units are dealt to a bounded grid in a grid-stride loop,
// so a billion-row set launches as easily as a small one.
#include "tgs_common.cuh"

#define WS_THREADS 256
#define WS_UNIT_ROWS 64
#define WS_COLS 59
#define WS_MAX_GRID 8192

namespace {

struct MoveArgs {
  const float* src;
  float* dst;
  const int64_t* src_starts;      // [n_seg] first source row per segment, or null
  const int64_t* dst_starts;      // [n_seg] first destination row per segment, or null
  const int64_t* counts;          // [n_seg] rows per segment, or null (implicit rule)
  const int64_t* src_gids;        // copy ids from the source rows, or null
  const int64_t* fill_block_ids;  // write block_id*block_rows + row_in_block, or null
  int64_t* dst_gids;              // destination ids (null: no id work)
  int64_t src_base;               // implicit segment s starts at src_base + s*block_rows
  int64_t dst_base;
  int64_t num_rows;               // implicit rule: rows of segment s = min(block_rows, num_rows - s*block_rows)
  uint32_t block_rows;
  uint32_t units_per_seg;
  uint64_t n_work;
};

// Source column of CACHE column c for a packed row in UNIFIED order
// (xyz 0:3 | opacity 3 | scaling 4:7 | rotation 7:11 | dc 11:14 | rest 14:59),
// the column tables of double_buffer_gpu.py:714-735.
template <bool UNIFIED>
__device__ __forceinline__ int source_column(int c) {
  if constexpr (!UNIFIED) {
    return c;
  } else {
    return c == 10 ? 3 : ((c >= 3 && c < 10) ? c + 1 : c);
  }
}

template <int SP, int DP, bool UNIFIED>
__global__ __launch_bounds__(WS_THREADS) void ws_move_rows_kernel(MoveArgs a) {
  constexpr int K = (WS_UNIT_ROWS * DP + WS_THREADS - 1) / WS_THREADS;
  const int tid = threadIdx.x;
  for (uint64_t w = blockIdx.x; w < a.n_work; w += gridDim.x) {
    const uint32_t s = (uint32_t)(w / a.units_per_seg);
    const uint32_t unit = (uint32_t)(w - (uint64_t)s * a.units_per_seg);
    int64_t len;
    if (a.counts) {
      len = a.counts[s];
      if (len > (int64_t)a.block_rows) len = a.block_rows;
    } else {
      len = a.num_rows - (int64_t)s * a.block_rows;
      if (len > (int64_t)a.block_rows) len = a.block_rows;
    }
    const int64_t r0 = (int64_t)unit * WS_UNIT_ROWS;
    if (r0 >= len) continue;  // uniform over the workgroup
    const int nrows = (int)((len - r0) < WS_UNIT_ROWS ? (len - r0) : WS_UNIT_ROWS);
    const int64_t srow = (a.src_starts ? a.src_starts[s] : a.src_base + (int64_t)s * a.block_rows) + r0;
    const int64_t drow = (a.dst_starts ? a.dst_starts[s] : a.dst_base + (int64_t)s * a.block_rows) + r0;
    const float* __restrict__ sp = a.src + srow * SP;
    float* __restrict__ dp = a.dst + drow * DP;
    const int nel = nrows * DP;
    // rows are streamed: non-temporal loads and stores (each byte moves once;
    // kept-block copy 4.58 -> 5.00 TB/s, pack 4.7 -> 5.1 TB/s)
    float v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int e = tid + k * WS_THREADS;
      v[k] = 0.0f;
      if (e < nel) {
        if constexpr (SP == DP && !UNIFIED) {
          v[k] = __builtin_nontemporal_load(&sp[e]);
        } else {
          const int r = e / DP;
          const int c = e - r * DP;
          if (DP == WS_COLS || c < WS_COLS)
            v[k] = __builtin_nontemporal_load(&sp[r * SP + source_column<UNIFIED>(c)]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int e = tid + k * WS_THREADS;
      if (e < nel) __builtin_nontemporal_store(v[k], &dp[e]);
    }
    if (a.dst_gids && tid < nrows) {
      int64_t gid;
      if (a.src_gids) {
        gid = a.src_gids[srow + tid];
      } else {
        gid = a.fill_block_ids[s] * (int64_t)a.block_rows + r0 + tid;
      }
      a.dst_gids[drow + tid] = gid;
    }
  }
}

template <int SP, int DP, bool UNIFIED>
int launch_move(const MoveArgs& a, hipStream_t stream, const char* name) {
  if (a.n_work == 0) return TGS_OK;
  const uint64_t grid = a.n_work < WS_MAX_GRID ? a.n_work : WS_MAX_GRID;
  hipLaunchKernelGGL((ws_move_rows_kernel<SP, DP, UNIFIED>), dim3((unsigned)grid),
                     dim3(WS_THREADS), 0, stream, a);
  TGS_RETURN_LAUNCH(name);
}

bool pitch_ok(uint32_t p) { return p == 59 || p == 64; }

int dispatch_move(uint32_t sp, uint32_t dp, bool unified, const MoveArgs& a, hipStream_t stream,
                  const char* name) {
  if (unified) {
    if (sp != 59) {
      tgs_set_error("%s: UNIFIED packed rows are 59 floats wide", name);
      return TGS_ERR_UNSUPPORTED;
    }
    return dp == 59 ? launch_move<59, 59, true>(a, stream, name)
                    : launch_move<59, 64, true>(a, stream, name);
  }
  if (sp == 59 && dp == 59) return launch_move<59, 59, false>(a, stream, name);
  if (sp == 59 && dp == 64) return launch_move<59, 64, false>(a, stream, name);
  if (sp == 64 && dp == 59) return launch_move<64, 59, false>(a, stream, name);
  return launch_move<64, 64, false>(a, stream, name);
}

uint32_t units_per_segment(uint32_t block_rows) {
  return (block_rows + WS_UNIT_ROWS - 1) / WS_UNIT_ROWS;
}

// ---------------------------------------------------------------------------
// Per-block xyz bounds: one workgroup per block segment (grid-stride), each
// thread folding rows tid, tid+256, ... < length; wave reductions by
// cross-lane shuffles, then 4 wave partials through LDS.  Empty segments keep
// the initial values (1e20 / -1e20), as gpu_working_set.py:102-115 does for
// masked rows.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

template <int P>
__global__ __launch_bounds__(WS_THREADS) void ws_block_bounds_kernel(
    const float* __restrict__ table, const int64_t* __restrict__ starts,
    const int64_t* __restrict__ lengths, uint32_t n_blocks, uint32_t block_rows,
    float* __restrict__ bounds) {
  __shared__ float red[WS_THREADS / TGS_WAVE][6];
  const int tid = threadIdx.x;
  const int wave = tid / TGS_WAVE, lane = tid % TGS_WAVE;
  for (uint32_t b = blockIdx.x; b < n_blocks; b += gridDim.x) {
    int64_t len = lengths[b];
    if (len > (int64_t)block_rows) len = block_rows;
    const float* __restrict__ base = table + starts[b] * P;
    float lo[3] = {1.0e20f, 1.0e20f, 1.0e20f};
    float hi[3] = {-1.0e20f, -1.0e20f, -1.0e20f};
    int64_t r = tid;
    for (; r + 3 * WS_THREADS < len; r += 4 * WS_THREADS) {
      float x[4][3];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int d = 0; d < 3; ++d) x[u][d] = base[(r + u * WS_THREADS) * P + d];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int d = 0; d < 3; ++d) {
          lo[d] = fminf(lo[d], x[u][d]);
          hi[d] = fmaxf(hi[d], x[u][d]);
        }
    }
    for (; r < len; r += WS_THREADS) {
#pragma unroll
      for (int d = 0; d < 3; ++d) {
        const float x = base[r * P + d];
        lo[d] = fminf(lo[d], x);
        hi[d] = fmaxf(hi[d], x);
      }
    }
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      lo[d] = wave_min(lo[d]);
      hi[d] = wave_max(hi[d]);
    }
    if (lane == 0) {
#pragma unroll
      for (int d = 0; d < 3; ++d) {
        red[wave][d] = lo[d];
        red[wave][3 + d] = hi[d];
      }
    }
    __syncthreads();
    if (tid < 6) {
      float acc = red[0][tid];
#pragma unroll
      for (int w = 1; w < WS_THREADS / TGS_WAVE; ++w)
        acc = tid < 3 ? fminf(acc, red[w][tid]) : fmaxf(acc, red[w][tid]);
      bounds[(uint64_t)b * 6 + tid] = acc;
    }
    __syncthreads();  // red is reused by the next segment
  }
}

// ---------------------------------------------------------------------------
// Compact block-start table (double_buffer_gpu.py:212-233): fill with -1,
// then scatter the start of every loaded block whose id is in range.
// ---------------------------------------------------------------------------
__global__ void ws_fill_i64_kernel(int64_t* __restrict__ p, uint64_t n, int64_t value) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = value;
}

__global__ void ws_scatter_block_starts_kernel(const int64_t* __restrict__ block_ids,
                                               const int64_t* __restrict__ local_starts,
                                               uint32_t n_loaded, int64_t* __restrict__ block_starts,
                                               uint32_t num_blocks) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_loaded) return;
  const int64_t id = block_ids[i];
  if (id >= 0 && id < (int64_t)num_blocks) block_starts[id] = local_starts[i];
}

// Cold-block ids (double_buffer_gpu.py:130-149): row r of the streamed range
// belongs to block_ids[r / block_rows] at offset r % block_rows.
__global__ void ws_fill_ids_kernel(const int64_t* __restrict__ block_ids,
                                   int64_t* __restrict__ dst_gids, uint64_t num_rows,
                                   uint32_t block_rows) {
  uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; r < num_rows; r += stride) {
    const uint64_t b = r / block_rows;
    dst_gids[r] = block_ids[b] * (int64_t)block_rows + (int64_t)(r - b * block_rows);
  }
}

// Global -> working-set-local ids (double_buffer_gpu.py:236-255): floor
// division by the block size, ids whose block is out of range or not loaded
// map to -1.
__global__ void ws_global_to_local_kernel(const int64_t* __restrict__ global_ids, uint64_t n,
                                          const int64_t* __restrict__ block_starts,
                                          uint32_t num_blocks, uint32_t block_size,
                                          int64_t* __restrict__ local_ids) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  const int64_t bs = block_size;
  for (; i < n; i += stride) {
    const int64_t g = global_ids[i];
    const int64_t q = g >= 0 ? g / bs : -((-g + bs - 1) / bs);
    const int64_t safe = q < 0 ? 0 : (q > (int64_t)num_blocks - 1 ? (int64_t)num_blocks - 1 : q);
    const int64_t start = block_starts[safe];
    local_ids[i] = (q != safe || start < 0) ? -1 : start + (g - q * bs);
  }
}

}  // namespace

extern "C" int tgs_ws_copy_rows(const float* src, uint32_t src_pitch, const int64_t* src_gids,
                                const int64_t* src_starts, const int64_t* dst_starts,
                                uint32_t n_blocks, int64_t num_rows, uint32_t block_rows,
                                float* dst, uint32_t dst_pitch, int64_t* dst_gids,
                                hipStream_t stream) {
  const char* name = "tgs_ws_copy_rows";
  TGS_CHECK_ARG(num_rows >= 0 && block_rows > 0, "%s: num_rows must be >= 0, block_rows > 0", name);
  if (num_rows == 0) return TGS_OK;
  TGS_CHECK_ARG(src && dst && src_starts && dst_starts, "%s: null pointer", name);
  TGS_CHECK_ARG(pitch_ok(src_pitch) && pitch_ok(dst_pitch), "%s: row pitch must be 59 or 64", name);
  TGS_CHECK_ARG((src_gids == nullptr) == (dst_gids == nullptr),
                "%s: pass both id arrays or neither", name);
  const uint64_t n_seg = ((uint64_t)num_rows + block_rows - 1) / block_rows;
  TGS_CHECK_ARG(n_seg <= n_blocks, "%s: %llu rows span %llu blocks of %u rows but %u starts given",
                name, (unsigned long long)num_rows, (unsigned long long)n_seg, block_rows, n_blocks);
  MoveArgs a{};
  a.src = src;
  a.dst = dst;
  a.src_starts = src_starts;
  a.dst_starts = dst_starts;
  a.src_gids = src_gids;
  a.dst_gids = dst_gids;
  a.num_rows = num_rows;
  a.block_rows = block_rows;
  a.units_per_seg = units_per_segment(block_rows);
  a.n_work = n_seg * a.units_per_seg;
  return dispatch_move(src_pitch, dst_pitch, false, a, stream, name);
}

extern "C" int tgs_ws_fill_global_ids(const int64_t* block_ids, uint32_t n_blocks,
                                      int64_t* dst_gids, int64_t target_offset, int64_t num_rows,
                                      uint32_t block_rows, hipStream_t stream) {
  const char* name = "tgs_ws_fill_global_ids";
  TGS_CHECK_ARG(num_rows >= 0 && block_rows > 0 && target_offset >= 0,
                "%s: num_rows and target_offset must be >= 0, block_rows > 0", name);
  if (num_rows == 0) return TGS_OK;
  TGS_CHECK_ARG(block_ids && dst_gids, "%s: null pointer", name);
  const uint64_t n_seg = ((uint64_t)num_rows + block_rows - 1) / block_rows;
  TGS_CHECK_ARG(n_seg <= n_blocks, "%s: %llu rows span %llu blocks but %u block ids given", name,
                (unsigned long long)num_rows, (unsigned long long)n_seg, n_blocks);
  uint64_t grid = ((uint64_t)num_rows + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(ws_fill_ids_kernel, dim3((unsigned)grid), dim3(256), 0, stream, block_ids,
                     dst_gids + target_offset, (uint64_t)num_rows, block_rows);
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_ws_unpack_rows(const float* packed, int source_layout, int64_t num_rows,
                                  float* dst, uint32_t dst_pitch, int64_t target_offset,
                                  const int64_t* block_ids, uint32_t n_blocks, uint32_t block_rows,
                                  int64_t* dst_gids, hipStream_t stream) {
  const char* name = "tgs_ws_unpack_rows";
  TGS_CHECK_ARG(num_rows >= 0 && block_rows > 0 && target_offset >= 0,
                "%s: num_rows and target_offset must be >= 0, block_rows > 0", name);
  TGS_CHECK_ARG(source_layout == 0 || source_layout == 1,
                "%s: source_layout must be 0 (CACHE) or 1 (UNIFIED)", name);
  if (num_rows == 0) return TGS_OK;
  TGS_CHECK_ARG(packed && dst, "%s: null pointer", name);
  TGS_CHECK_ARG(pitch_ok(dst_pitch), "%s: row pitch must be 59 or 64", name);
  TGS_CHECK_ARG((block_ids == nullptr) == (dst_gids == nullptr),
                "%s: pass block_ids and dst_gids together or neither", name);
  const uint64_t n_seg = ((uint64_t)num_rows + block_rows - 1) / block_rows;
  TGS_CHECK_ARG(!block_ids || n_seg <= n_blocks,
                "%s: %llu rows span %llu blocks but %u block ids given", name,
                (unsigned long long)num_rows, (unsigned long long)n_seg, n_blocks);
  MoveArgs a{};
  a.src = packed;
  a.dst = dst;
  a.fill_block_ids = block_ids;
  a.dst_gids = dst_gids;
  a.src_base = 0;
  a.dst_base = target_offset;
  a.num_rows = num_rows;
  a.block_rows = block_rows;
  a.units_per_seg = units_per_segment(block_rows);
  a.n_work = n_seg * a.units_per_seg;
  return dispatch_move(59, dst_pitch, source_layout == 1, a, stream, name);
}

extern "C" int tgs_ws_pack_rows(const float* src, uint32_t src_pitch, const int64_t* src_starts,
                                const int64_t* row_counts, const int64_t* out_starts,
                                uint32_t n_blocks, uint32_t block_rows, float* out,
                                hipStream_t stream) {
  const char* name = "tgs_ws_pack_rows";
  TGS_CHECK_ARG(block_rows > 0, "%s: block_rows must be > 0", name);
  if (n_blocks == 0) return TGS_OK;
  TGS_CHECK_ARG(src && src_starts && row_counts && out_starts && out, "%s: null pointer", name);
  TGS_CHECK_ARG(pitch_ok(src_pitch), "%s: row pitch must be 59 or 64", name);
  MoveArgs a{};
  a.src = src;
  a.dst = out;
  a.src_starts = src_starts;
  a.dst_starts = out_starts;
  a.counts = row_counts;
  a.block_rows = block_rows;
  a.units_per_seg = units_per_segment(block_rows);
  a.n_work = (uint64_t)n_blocks * a.units_per_seg;
  return dispatch_move(src_pitch, 59, false, a, stream, name);
}

extern "C" int tgs_ws_block_bounds(const float* table, uint32_t pitch, const int64_t* starts,
                                   const int64_t* lengths, uint32_t n_blocks, uint32_t block_rows,
                                   float* bounds, hipStream_t stream) {
  const char* name = "tgs_ws_block_bounds";
  TGS_CHECK_ARG(block_rows > 0, "%s: block_rows must be > 0", name);
  if (n_blocks == 0) return TGS_OK;
  TGS_CHECK_ARG(table && starts && lengths && bounds, "%s: null pointer", name);
  TGS_CHECK_ARG(pitch_ok(pitch) || pitch == 3, "%s: row pitch must be 3, 59 or 64", name);
  const unsigned grid = n_blocks < WS_MAX_GRID ? n_blocks : WS_MAX_GRID;
  if (pitch == 3)
    hipLaunchKernelGGL(ws_block_bounds_kernel<3>, dim3(grid), dim3(WS_THREADS), 0, stream, table,
                       starts, lengths, n_blocks, block_rows, bounds);
  else if (pitch == 59)
    hipLaunchKernelGGL(ws_block_bounds_kernel<59>, dim3(grid), dim3(WS_THREADS), 0, stream, table,
                       starts, lengths, n_blocks, block_rows, bounds);
  else
    hipLaunchKernelGGL(ws_block_bounds_kernel<64>, dim3(grid), dim3(WS_THREADS), 0, stream, table,
                       starts, lengths, n_blocks, block_rows, bounds);
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_ws_build_block_starts(const int64_t* block_ids, const int64_t* local_starts,
                                         uint32_t n_loaded, int64_t* block_starts,
                                         uint32_t num_blocks, hipStream_t stream) {
  const char* name = "tgs_ws_build_block_starts";
  if (num_blocks == 0) return TGS_OK;
  TGS_CHECK_ARG(block_starts, "%s: null pointer", name);
  TGS_CHECK_ARG(n_loaded == 0 || (block_ids && local_starts), "%s: null pointer", name);
  unsigned grid = tgs_blocks(num_blocks, 256);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(ws_fill_i64_kernel, dim3(grid), dim3(256), 0, stream, block_starts,
                     (uint64_t)num_blocks, (int64_t)-1);
  TGS_LAUNCH_CHECK(name);
  if (n_loaded == 0) return TGS_OK;
  hipLaunchKernelGGL(ws_scatter_block_starts_kernel, dim3(tgs_blocks(n_loaded, 256)), dim3(256), 0,
                     stream, block_ids, local_starts, n_loaded, block_starts, num_blocks);
  TGS_RETURN_LAUNCH(name);
}

extern "C" int tgs_ws_global_to_local(const int64_t* global_ids, uint64_t n,
                                      const int64_t* block_starts, uint32_t num_blocks,
                                      uint32_t block_size, int64_t* local_ids,
                                      hipStream_t stream) {
  const char* name = "tgs_ws_global_to_local";
  TGS_CHECK_ARG(block_size > 0 && num_blocks > 0, "%s: block_size and num_blocks must be > 0", name);
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(global_ids && block_starts && local_ids, "%s: null pointer", name);
  uint64_t grid = (n + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(ws_global_to_local_kernel, dim3((unsigned)grid), dim3(256), 0, stream,
                     global_ids, n, block_starts, num_blocks, block_size, local_ids);
  TGS_RETURN_LAUNCH(name);
}
