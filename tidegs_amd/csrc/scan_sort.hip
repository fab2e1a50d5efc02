// Device-wide scan and stable LSD radix sort of (uint64 key, uint32 value)
// pairs, written for wave64.
//
// The tile-intersection sort (gsplat isect_tiles.cu:189-227 calls
// cub::DeviceRadixSort::SortPairs on bits [0, 32+tile_bits+cam_bits)) needs a
// stable ascending sort on a bit range of the key.  Because every flatten id
// appears at most once per (camera, tile) key prefix, "stable on the key bits"
// equals "ascending in (key bits, input position)", a total order, so any
// correct stable sort reproduces the reference output bit for bit.
//
// Scan: reduce-then-scan in three kernels (block sums, one-block scan of the
// sums, per-block rescan), no inter-block spin-waits.
// Radix pass (8-bit digit, 4096-key tiles of 256 threads x 16 keys):
//   upsweep   per-tile digit histogram -> hist[digit * n_tiles + tile]
//   scan      exclusive scan of hist (digit-major => global digit offsets)
//   downsweep per-tile stable ranking: 8 ballots give each lane the set of
//             lanes in its wave holding the same digit; per-wave counts in LDS
//             give the offsets of earlier waves and rounds.
#include "tgs_common.cuh"

#define SCAN_THREADS 256
#define SCAN_ITEMS 8
#define SCAN_CHUNK (SCAN_THREADS * SCAN_ITEMS)

#define SORT_THREADS 256
#define SORT_ITEMS 16
#define SORT_TILE (SORT_THREADS * SORT_ITEMS)
#define SORT_BINS 256

// ---------------------------------------------------------------------------
// Block-level exclusive scan of one value per thread (256 threads, 4 waves).
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* s_wave, T& total) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  T inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    T o = __shfl_up(inc, off, 64);
    if (lane >= off) inc += o;
  }
  if (lane == 63) s_wave[wave] = inc;
  __syncthreads();
  T wave_base = 0;
  T tot = 0;
#pragma unroll
  for (int w = 0; w < SCAN_THREADS / 64; ++w) {
    const T s = s_wave[w];
    if (w < wave) wave_base += s;
    tot += s;
  }
  __syncthreads();
  total = tot;
  return wave_base + inc - v;
}

template <typename InT, typename OutT>
__global__ void __launch_bounds__(SCAN_THREADS) scan_reduce_kernel(const InT* __restrict__ in,
                                                                   uint64_t n,
                                                                   OutT* __restrict__ sums) {
  __shared__ OutT s_wave[SCAN_THREADS / 64];
  const uint64_t base = (uint64_t)blockIdx.x * SCAN_CHUNK;
  OutT acc = 0;
#pragma unroll
  for (int k = 0; k < SCAN_ITEMS; ++k) {
    const uint64_t i = base + (uint64_t)k * SCAN_THREADS + threadIdx.x;
    if (i < n) acc += (OutT)in[i];
  }
  OutT total;
  (void)block_exclusive_scan<OutT>(acc, s_wave, total);
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// In-place exclusive scan of `n` block sums by one block.
template <typename OutT>
__global__ void __launch_bounds__(SCAN_THREADS) scan_sums_kernel(OutT* __restrict__ sums,
                                                                 uint64_t n) {
  __shared__ OutT s_wave[SCAN_THREADS / 64];
  OutT carry = 0;
  for (uint64_t base = 0; base < n; base += SCAN_THREADS) {
    const uint64_t i = base + threadIdx.x;
    const OutT v = i < n ? sums[i] : (OutT)0;
    OutT total;
    const OutT ex = block_exclusive_scan<OutT>(v, s_wave, total);
    if (i < n) sums[i] = carry + ex;
    carry += total;
  }
}

template <typename InT, typename OutT, bool INCLUSIVE>
__global__ void __launch_bounds__(SCAN_THREADS) scan_apply_kernel(const InT* __restrict__ in,
                                                                  uint64_t n,
                                                                  const OutT* __restrict__ sums,
                                                                  OutT* __restrict__ out) {
  __shared__ OutT s_wave[SCAN_THREADS / 64];
  // Blocked arrangement: thread t owns items [t*ITEMS, (t+1)*ITEMS).
  const uint64_t base = (uint64_t)blockIdx.x * SCAN_CHUNK + (uint64_t)threadIdx.x * SCAN_ITEMS;
  OutT vals[SCAN_ITEMS];
  OutT acc = 0;
#pragma unroll
  for (int k = 0; k < SCAN_ITEMS; ++k) {
    const uint64_t i = base + k;
    vals[k] = i < n ? (OutT)in[i] : (OutT)0;
    acc += vals[k];
  }
  OutT total;
  OutT run = block_exclusive_scan<OutT>(acc, s_wave, total) + sums[blockIdx.x];
#pragma unroll
  for (int k = 0; k < SCAN_ITEMS; ++k) {
    const uint64_t i = base + k;
    if (INCLUSIVE) run += vals[k];
    if (i < n) out[i] = run;
    if (!INCLUSIVE) run += vals[k];
  }
}

static uint64_t scan_blocks(uint64_t n) { return (n + SCAN_CHUNK - 1) / SCAN_CHUNK; }

template <typename InT, typename OutT, bool INCLUSIVE>
static int launch_scan(const InT* in, OutT* out, uint64_t n, OutT* sums, hipStream_t stream) {
  if (n == 0) return TGS_OK;
  const uint64_t nb = scan_blocks(n);
  hipLaunchKernelGGL((scan_reduce_kernel<InT, OutT>), dim3((unsigned)nb), dim3(SCAN_THREADS), 0,
                     stream, in, n, sums);
  hipLaunchKernelGGL((scan_sums_kernel<OutT>), dim3(1), dim3(SCAN_THREADS), 0, stream, sums, nb);
  hipLaunchKernelGGL((scan_apply_kernel<InT, OutT, INCLUSIVE>), dim3((unsigned)nb),
                     dim3(SCAN_THREADS), 0, stream, in, n, sums, out);
  TGS_RETURN_LAUNCH("scan");
}

extern "C" size_t tgs_scan_workspace_size(uint64_t n) {
  return (size_t)(scan_blocks(n) + 1) * sizeof(int64_t);
}

// out[i] = sum(in[0..i]) (int32 in, int64 out), as torch.cumsum does in
// isect_tiles.cu:165.
extern "C" int tgs_inclusive_scan_i32_i64(const int32_t* in, int64_t* out, uint64_t n,
                                          void* workspace, size_t workspace_bytes,
                                          hipStream_t stream) {
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(in && out && workspace, "inclusive_scan: null pointer");
  if (workspace_bytes < tgs_scan_workspace_size(n)) {
    tgs_set_error("inclusive_scan: workspace %zu < %zu bytes", workspace_bytes,
                  tgs_scan_workspace_size(n));
    return TGS_ERR_WORKSPACE;
  }
  return launch_scan<int32_t, int64_t, true>(in, out, n, (int64_t*)workspace, stream);
}

// Exclusive scan of uint32 -> uint32 (radix histograms, compaction).
static int exclusive_scan_u32(const uint32_t* in, uint32_t* out, uint64_t n, void* ws,
                              hipStream_t stream) {
  return launch_scan<uint32_t, uint32_t, false>(in, out, n, (uint32_t*)ws, stream);
}

extern "C" int tgs_exclusive_scan_u32(const uint32_t* in, uint32_t* out, uint64_t n,
                                      void* workspace, size_t workspace_bytes,
                                      hipStream_t stream) {
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(in && out && workspace, "exclusive_scan_u32: null pointer");
  if (workspace_bytes < tgs_scan_workspace_size(n)) {
    tgs_set_error("exclusive_scan_u32: workspace too small");
    return TGS_ERR_WORKSPACE;
  }
  return exclusive_scan_u32(in, out, n, workspace, stream);
}

// ---------------------------------------------------------------------------
// Radix sort
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t digit_of(uint64_t key, int shift, uint32_t mask) {
  return (uint32_t)(key >> shift) & mask;
}

__global__ void __launch_bounds__(SORT_THREADS) radix_upsweep_kernel(
    const uint64_t* __restrict__ keys, uint64_t n, int shift, uint32_t mask, uint32_t n_tiles,
    uint32_t* __restrict__ hist) {
  __shared__ uint32_t s_hist[SORT_BINS];
  s_hist[threadIdx.x] = 0;
  __syncthreads();
  const uint64_t base = (uint64_t)blockIdx.x * SORT_TILE;
#pragma unroll 4
  for (int r = 0; r < SORT_ITEMS; ++r) {
    const uint64_t i = base + (uint64_t)r * SORT_THREADS + threadIdx.x;
    if (i < n) atomicAdd(&s_hist[digit_of(keys[i], shift, mask)], 1u);
  }
  __syncthreads();
  hist[(uint64_t)threadIdx.x * n_tiles + blockIdx.x] = s_hist[threadIdx.x];
}

__global__ void __launch_bounds__(SORT_THREADS) radix_downsweep_kernel(
    const uint64_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, uint64_t n,
    int shift, uint32_t mask, uint32_t n_tiles, const uint32_t* __restrict__ hist_scan,
    uint64_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out) {
  __shared__ uint32_t s_base[SORT_BINS];                       // global offset of digit
  __shared__ uint32_t s_wave[SORT_THREADS / 64][SORT_BINS];    // per-wave counts this round
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  s_base[threadIdx.x] = hist_scan[(uint64_t)threadIdx.x * n_tiles + blockIdx.x];
#pragma unroll
  for (int w = 0; w < SORT_THREADS / 64; ++w) s_wave[w][threadIdx.x] = 0;
  __syncthreads();

  const uint64_t base = (uint64_t)blockIdx.x * SORT_TILE;
  for (int r = 0; r < SORT_ITEMS; ++r) {
    const uint64_t i = base + (uint64_t)r * SORT_THREADS + threadIdx.x;
    const bool valid = i < n;
    uint64_t key = 0;
    uint32_t val = 0;
    if (valid) {
      key = keys_in[i];
      val = vals_in[i];
    }
    const uint32_t d = digit_of(key, shift, mask);
    uint64_t peers = tgs_ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool bit = (d >> b) & 1u;
      const uint64_t m = tgs_ballot(bit);
      peers &= bit ? m : ~m;
    }
    const uint32_t rank = (uint32_t)__popcll(peers & lt_mask);
    const uint32_t cnt = (uint32_t)__popcll(peers);
    // The highest peer lane publishes the wave's count for this digit.
    const bool leader = valid && ((peers >> lane) == 1ull);
    if (leader) s_wave[wave][d] = cnt;
    __syncthreads();
    if (valid) {
      uint32_t off = s_base[d] + rank;
      for (int w = 0; w < wave; ++w) off += s_wave[w][d];
      keys_out[off] = key;
      vals_out[off] = val;
    }
    __syncthreads();
    // Thread t owns digit t: fold this round's counts into the base and clear.
    uint32_t add = 0;
#pragma unroll
    for (int w = 0; w < SORT_THREADS / 64; ++w) {
      add += s_wave[w][threadIdx.x];
      s_wave[w][threadIdx.x] = 0;
    }
    s_base[threadIdx.x] += add;
    __syncthreads();
  }
}

static uint64_t sort_tiles(uint64_t n) { return (n + SORT_TILE - 1) / SORT_TILE; }

extern "C" size_t tgs_radix_sort_workspace_size(uint64_t n) {
  const uint64_t tiles = sort_tiles(n);
  const uint64_t hist = tiles * SORT_BINS;
  // hist + scanned hist + scan block sums, each 256-byte aligned.
  auto al = [](uint64_t b) { return (b + 255) & ~255ull; };
  return (size_t)(al(hist * 4) * 2 + al(tgs_scan_workspace_size(hist)));
}

// Stable ascending sort of (keys, vals) on key bits [begin_bit, end_bit).
// Data ping-pongs between (keys, vals) and (keys_alt, vals_alt); *selector is
// set to 0 if the result is in keys/vals and 1 if in keys_alt/vals_alt
// (the cub::DoubleBuffer convention used at isect_tiles.cu:196-217).
extern "C" int tgs_radix_sort_pairs(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt,
                                    uint32_t* vals_alt, uint64_t n, int begin_bit, int end_bit,
                                    void* workspace, size_t workspace_bytes, int* selector,
                                    hipStream_t stream) {
  TGS_CHECK_ARG(selector != nullptr, "radix_sort: null selector");
  *selector = 0;
  if (n <= 1 || end_bit <= begin_bit) return TGS_OK;
  TGS_CHECK_ARG(keys && vals && keys_alt && vals_alt && workspace, "radix_sort: null pointer");
  TGS_CHECK_ARG(begin_bit >= 0 && end_bit <= 64, "radix_sort: bit range out of [0,64]");
  TGS_CHECK_ARG(n < (1ull << 32), "radix_sort: n must be < 2^32");
  if (workspace_bytes < tgs_radix_sort_workspace_size(n)) {
    tgs_set_error("radix_sort: workspace %zu < %zu", workspace_bytes,
                  tgs_radix_sort_workspace_size(n));
    return TGS_ERR_WORKSPACE;
  }
  const uint64_t tiles = sort_tiles(n);
  const uint64_t hist_n = tiles * SORT_BINS;
  auto al = [](uint64_t b) { return (b + 255) & ~255ull; };
  uint8_t* ws = (uint8_t*)workspace;
  uint32_t* hist = (uint32_t*)ws;
  uint32_t* hist_scan = (uint32_t*)(ws + al(hist_n * 4));
  void* scan_ws = ws + 2 * al(hist_n * 4);

  uint64_t* kin = keys;
  uint32_t* vin = vals;
  uint64_t* kout = keys_alt;
  uint32_t* vout = vals_alt;
  int sel = 0;
  for (int shift = begin_bit; shift < end_bit; shift += 8) {
    const int bits = (end_bit - shift) < 8 ? (end_bit - shift) : 8;
    const uint32_t mask = (1u << bits) - 1u;
    hipLaunchKernelGGL(radix_upsweep_kernel, dim3((unsigned)tiles), dim3(SORT_THREADS), 0, stream,
                       kin, n, shift, mask, (uint32_t)tiles, hist);
    TGS_LAUNCH_CHECK("radix_upsweep");
    int rc = exclusive_scan_u32(hist, hist_scan, hist_n, scan_ws, stream);
    if (rc) return rc;
    hipLaunchKernelGGL(radix_downsweep_kernel, dim3((unsigned)tiles), dim3(SORT_THREADS), 0,
                       stream, kin, vin, n, shift, mask, (uint32_t)tiles, hist_scan, kout, vout);
    TGS_LAUNCH_CHECK("radix_downsweep");
    uint64_t* tk = kin;
    kin = kout;
    kout = tk;
    uint32_t* tv = vin;
    vin = vout;
    vout = tv;
    sel ^= 1;
  }
  *selector = sel;
  return TGS_OK;
}
