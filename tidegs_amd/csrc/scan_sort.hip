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
// Radix pass (<= 8-bit digit, 4096-key tiles of 256 threads x 16 keys):
//   hist      per-tile digit histogram -> hist[segment][digit][tile]
//   scan      exclusive scan of hist (digit-major => global digit offsets)
//   scatter   per-tile stable ranking (ballot matching + per-wave counters),
//             LDS reorder, coalesced write of each digit run.
#include <mutex>

#include "tgs_common.cuh"

#define SCAN_THREADS 256
#define SCAN_ITEMS 16
#define SCAN_CHUNK (SCAN_THREADS * SCAN_ITEMS)

#define SORT_THREADS 256
#define SORT_ITEMS 16
#define SORT_TILE (SORT_THREADS * SORT_ITEMS)
#define SORT_BINS 256
#define RADIX_MAX_SEGS 64

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

// In-place exclusive scan of `n` block sums by one block: each thread scans a
// contiguous run of the sums, one block-wide scan joins the runs.
template <typename OutT>
__global__ void __launch_bounds__(SCAN_THREADS) scan_sums_kernel(OutT* __restrict__ sums,
                                                                 uint64_t n) {
  __shared__ OutT s_wave[SCAN_THREADS / 64];
  const uint64_t per = (n + SCAN_THREADS - 1) / SCAN_THREADS;
  const uint64_t b0 = (uint64_t)threadIdx.x * per;
  const uint64_t b1 = b0 + per < n ? b0 + per : n;
  OutT run = 0;
  for (uint64_t i = b0; i < b1; ++i) run += sums[i];
  OutT total;
  OutT carry = block_exclusive_scan<OutT>(run, s_wave, total);
  for (uint64_t i = b0; i < b1; ++i) {
    const OutT v = sums[i];
    sums[i] = carry;
    carry += v;
  }
}

// Wave-level inclusive scan (wave64, shuffles).
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const T o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  return v;
}

// Striped arrangement: wave w of the block owns items [w*64*ITEMS, (w+1)*64*ITEMS)
// of the chunk in rounds of 64 consecutive items, so every load and store of
// a round is one contiguous span.
template <typename InT, typename OutT, bool INCLUSIVE>
__global__ void __launch_bounds__(SCAN_THREADS) scan_apply_kernel(const InT* __restrict__ in,
                                                                  uint64_t n,
                                                                  const OutT* __restrict__ sums,
                                                                  OutT* __restrict__ out) {
  __shared__ OutT s_wtot[SCAN_THREADS / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t wbase = (uint64_t)blockIdx.x * SCAN_CHUNK + (uint64_t)wave * 64 * SCAN_ITEMS;
  OutT vals[SCAN_ITEMS];
  OutT acc = 0;
#pragma unroll
  for (int k = 0; k < SCAN_ITEMS; ++k) {
    const uint64_t i = wbase + (uint64_t)k * 64 + lane;
    vals[k] = i < n ? (OutT)in[i] : (OutT)0;
    acc += vals[k];
  }
  // wave total -> exclusive prefix of the waves before this one
  OutT wt = acc;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) wt += __shfl_xor(wt, off, 64);
  if (lane == 0) s_wtot[wave] = wt;
  __syncthreads();
  OutT carry = sums[blockIdx.x];
  for (int w = 0; w < wave; ++w) carry += s_wtot[w];
#pragma unroll
  for (int k = 0; k < SCAN_ITEMS; ++k) {
    const OutT inc = wave_inclusive_scan<OutT>(vals[k]);
    const uint64_t i = wbase + (uint64_t)k * 64 + lane;
    if (i < n) out[i] = carry + (INCLUSIVE ? inc : inc - vals[k]);
    carry += __shfl(inc, 63, 64);
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
//
// Segmented LSD passes: the key range [0, n) is split into segments (one for
// a plain sort; one per camera for the fused step, where entries and
// intersections are already grouped by camera) and tiles never straddle a
// segment, so one pass sorts every segment independently.  The histogram is
// laid out [segment][digit][tile of segment]; its exclusive scan is then the
// absolute output offset of (segment, digit, tile).
// ---------------------------------------------------------------------------

struct RadixSegs {
  uint32_t n;                             // number of segments (>= 1)
  uint32_t key_off[RADIX_MAX_SEGS + 1];   // key_off[0] = 0, key_off[n] = n_keys
  uint32_t tile_base[RADIX_MAX_SEGS + 1]; // first tile of each segment
  // 32-bit keys are ranked as min(key - key_base, key_cap) (keys below the
  // base as 0): an order-preserving map of a key range onto its low bits, with
  // every key past the range tied at key_cap.  (0, ~0) ranks the keys as they are.
  uint32_t key_base = 0, key_cap = 0xffffffffu;
};

struct TileRange {
  uint32_t start, count;  // keys [start, start + count)
  uint32_t hbase, stride; // hist index of digit d: hbase + d * stride
};

// nbins: the pass's digit count (1 << bits); the histogram holds nbins counts
// per tile, [segment][digit][tile of segment]
__device__ __forceinline__ TileRange radix_tile(const RadixSegs& sg, uint32_t b, uint32_t nbins) {
  uint32_t lo = 0, hi = sg.n;  // largest s with tile_base[s] <= b
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (sg.tile_base[mid] <= b) lo = mid;
    else hi = mid;
  }
  const uint32_t t = b - sg.tile_base[lo];
  const uint32_t nts = sg.tile_base[lo + 1] - sg.tile_base[lo];
  TileRange r;
  r.start = sg.key_off[lo] + t * SORT_TILE;
  const uint32_t end = sg.key_off[lo + 1];
  r.count = end > r.start ? min((uint32_t)SORT_TILE, end - r.start) : 0u;
  r.hbase = sg.tile_base[lo] * nbins + t;
  r.stride = nts;
  return r;
}

template <typename K>
__device__ __forceinline__ uint32_t digit_of(K key, const RadixSegs& sg, int shift,
                                            uint32_t mask) {
  if constexpr (sizeof(K) == 4) {
    // max-then-subtract is a clamped (saturating) subtract; the same select
    // written as (k < base ? 0 : min(k - base, cap)) compiles for gfx950 to an
    // unclamped subtract, so keys below the base would wrap
    const uint32_t r = min(max((uint32_t)key, sg.key_base) - sg.key_base, sg.key_cap);
    return (r >> shift) & mask;
  } else {
    return (uint32_t)(key >> shift) & mask;
  }
}

template <typename K>
__global__ void __launch_bounds__(SORT_THREADS) radix_hist_kernel(const K* __restrict__ keys,
                                                                  RadixSegs sg, int shift,
                                                                  uint32_t mask, uint32_t nbins,
                                                                  uint32_t* __restrict__ hist) {
  __shared__ uint32_t s_h[SORT_THREADS / 64][SORT_BINS];
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int w = 0; w < SORT_THREADS / 64; ++w) s_h[w][threadIdx.x] = 0;
  __syncthreads();
  const TileRange tr = radix_tile(sg, blockIdx.x, nbins);
  // A wavefront whose keys share one digit (common for the high digits of
  // sorted-ish keys) adds its count once instead of 64 conflicting atomics.
  // all of the thread's keys are loaded before any is counted, so the tile's
  // loads are in flight together
  K kr[SORT_ITEMS];
#pragma unroll
  for (int r = 0; r < SORT_ITEMS; ++r) {
    const uint32_t i = (uint32_t)r * SORT_THREADS + threadIdx.x;
    kr[r] = i < tr.count ? keys[tr.start + i] : (K)0;
  }
#pragma unroll
  for (int r = 0; r < SORT_ITEMS; ++r) {
    const uint32_t i = (uint32_t)r * SORT_THREADS + threadIdx.x;
    const bool valid = i < tr.count;
    const uint32_t d = valid ? digit_of(kr[r], sg, shift, mask) : 0u;
    const uint32_t d0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)d);
    const uint64_t vm = tgs_ballot(valid);
    const uint64_t same = tgs_ballot(valid && d == d0);
    if (same == vm) {
      if ((threadIdx.x & 63) == 0 && vm) atomicAdd(&s_h[wave][d0], (uint32_t)__popcll(vm));
    } else if (valid) {
      atomicAdd(&s_h[wave][d], 1u);
    }
  }
  __syncthreads();
  uint32_t c = 0;
#pragma unroll
  for (int w = 0; w < SORT_THREADS / 64; ++w) c += s_h[w][threadIdx.x];
  // only the pass's digits: a narrower pass stores (and scans) fewer counts,
  // each a line of its own in this layout
  if (threadIdx.x < nbins) hist[tr.hbase + threadIdx.x * tr.stride] = c;
}

// One tile of 4096 keys per block.  Wave w owns keys [w*1024, (w+1)*1024) of
// the tile in rounds of 64; for each round 8 ballots give a lane the lanes of
// its wave with the same digit, and a per-wave digit counter in LDS carries
// the count of earlier rounds.  The tile is then scattered into LDS in
// (digit, position) order and written out by consecutive threads, so each
// digit's run of the tile is one contiguous store.
template <typename K, typename V>
__global__ void __launch_bounds__(SORT_THREADS) __attribute__((amdgpu_waves_per_eu(4))) radix_scatter_kernel(
    const K* __restrict__ keys_in, const V* __restrict__ vals_in, RadixSegs sg, int shift,
    uint32_t mask, uint32_t nbins, const uint32_t* __restrict__ hist_scan,
    K* __restrict__ keys_out, V* __restrict__ vals_out) {
  constexpr int WAVES = SORT_THREADS / 64;
  __shared__ K s_k[SORT_TILE];
  __shared__ V s_v[SORT_TILE];
  // per-wave digit counters, then each (wave, digit)'s first position in the
  // tile (counts and positions stay below SORT_TILE: 16 bits, so the 8-byte
  // value form's LDS lets 3 workgroups share a CU)
  __shared__ uint16_t s_wh[WAVES][SORT_BINS];
  __shared__ uint32_t s_gofs[SORT_BINS];
  __shared__ uint32_t s_scan[WAVES];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint64_t lt_mask = (1ull << lane) - 1ull;
  const TileRange tr = radix_tile(sg, blockIdx.x, nbins);
#pragma unroll
  for (int w = 0; w < WAVES; ++w) s_wh[w][threadIdx.x] = 0;
  __syncthreads();

  K k[SORT_ITEMS];
  V v[SORT_ITEMS];
  uint32_t rk[SORT_ITEMS];
  const uint32_t wbase = (uint32_t)wave * 64u * SORT_ITEMS;
#pragma unroll
  for (int r = 0; r < SORT_ITEMS; ++r) {
    const uint32_t li = wbase + (uint32_t)r * 64u + lane;
    if (li < tr.count) {
      k[r] = keys_in[tr.start + li];
      v[r] = vals_in[tr.start + li];
    } else {
      k[r] = 0;
      v[r] = 0;
    }
  }
#pragma unroll
  for (int r = 0; r < SORT_ITEMS; ++r) {
    const uint32_t li = wbase + (uint32_t)r * 64u + lane;
    const bool valid = li < tr.count;
    const uint32_t d = digit_of(k[r], sg, shift, mask);
    uint64_t peers = tgs_ballot(valid);
    const uint32_t d0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)d);
    if (tgs_ballot(valid && d == d0) != peers) {  // else every valid lane shares d0
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t m = tgs_ballot(bit);
        peers &= bit ? m : ~m;
      }
    }
    const uint32_t before = s_wh[wave][d];
    __builtin_amdgcn_wave_barrier();
    // the highest lane of each digit group advances the wave's counter
    if (valid && (peers >> lane) == 1ull) s_wh[wave][d] = (uint16_t)(before + (uint32_t)__popcll(peers));
    __builtin_amdgcn_wave_barrier();
    rk[r] = before + (uint32_t)__popcll(peers & lt_mask);
  }
  __syncthreads();
  // thread t owns digit t: per-wave counts, tile total, tile start, then each
  // wave's first position of the digit in the tile
  uint32_t cw[WAVES];
  uint32_t tot = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    cw[w] = s_wh[w][threadIdx.x];
    tot += cw[w];
  }
  uint32_t all;
  const uint32_t st = block_exclusive_scan<uint32_t>(tot, s_scan, all);
  uint32_t run = st;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    s_wh[w][threadIdx.x] = (uint16_t)run;
    run += cw[w];
  }
  // digits past nbins never occur in this pass
  s_gofs[threadIdx.x] =
      threadIdx.x < nbins ? hist_scan[tr.hbase + threadIdx.x * tr.stride] - st : 0u;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < SORT_ITEMS; ++r) {
    const uint32_t li = wbase + (uint32_t)r * 64u + lane;
    if (li < tr.count) {
      const uint32_t d = digit_of(k[r], sg, shift, mask);
      const uint32_t pos = (uint32_t)s_wh[wave][d] + rk[r];
      s_k[pos] = k[r];
      s_v[pos] = v[r];
    }
  }
  __syncthreads();
  for (uint32_t j = threadIdx.x; j < tr.count; j += SORT_THREADS) {
    const K kk = s_k[j];
    const uint32_t o = s_gofs[digit_of(kk, sg, shift, mask)] + j;
    keys_out[o] = kk;
    vals_out[o] = s_v[j];
  }
}

static uint64_t sort_tiles(uint64_t n) { return (n + SORT_TILE - 1) / SORT_TILE; }

static size_t radix_workspace(uint64_t tiles) {
  const uint64_t hist = tiles * SORT_BINS;
  // hist + scanned hist + scan block sums, each 256-byte aligned.
  auto al = [](uint64_t b) { return (b + 255) & ~255ull; };
  return (size_t)(al(hist * 4) * 2 + al(tgs_scan_workspace_size(hist)));
}

extern "C" size_t tgs_radix_sort_workspace_size(uint64_t n) { return radix_workspace(sort_tiles(n)); }

extern "C" size_t tgs_segmented_sort_workspace_size(uint64_t n, uint32_t n_segments) {
  return radix_workspace(sort_tiles(n) + n_segments);
}

// Runs the passes over key bits [begin_bit, end_bit), splitting the range
// into the fewest passes of at most 8 bits with widths as even as possible.
template <typename K, typename V>
static int radix_passes(K* keys, V* vals, K* keys_alt, V* vals_alt, const RadixSegs& sg,
                        int begin_bit, int end_bit, void* workspace, int* selector,
                        hipStream_t stream, bool first_hist_ready = false) {
  const uint64_t tiles = sg.tile_base[sg.n];
  const uint64_t hist_max = tiles * SORT_BINS;  // the workspace's layout
  auto al = [](uint64_t b) { return (b + 255) & ~255ull; };
  uint8_t* ws = (uint8_t*)workspace;
  uint32_t* hist = (uint32_t*)ws;
  uint32_t* hist_scan = (uint32_t*)(ws + al(hist_max * 4));
  void* scan_ws = ws + 2 * al(hist_max * 4);
  K* kin = keys;
  V* vin = vals;
  K* kout = keys_alt;
  V* vout = vals_alt;
  int sel = 0;
  int shift = begin_bit;
  int passes = (end_bit - begin_bit + 7) / 8;
  while (shift < end_bit) {
    const int bits = (end_bit - shift + passes - 1) / passes;
    const uint32_t mask = (1u << bits) - 1u;
    const bool given = first_hist_ready && shift == begin_bit;
    // a histogram the caller counted keeps the 256-digit layout
    const uint32_t nbins = given ? (uint32_t)SORT_BINS : mask + 1u;
    if (!given) {
      hipLaunchKernelGGL((radix_hist_kernel<K>), dim3((unsigned)tiles), dim3(SORT_THREADS), 0,
                         stream, kin, sg, shift, mask, nbins, hist);
      TGS_LAUNCH_CHECK("radix_hist");
    }
    int rc = exclusive_scan_u32(hist, hist_scan, tiles * nbins, scan_ws, stream);
    if (rc) return rc;
    hipLaunchKernelGGL((radix_scatter_kernel<K, V>), dim3((unsigned)tiles), dim3(SORT_THREADS), 0,
                       stream, kin, vin, sg, shift, mask, nbins, hist_scan, kout, vout);
    TGS_LAUNCH_CHECK("radix_scatter");
    K* tk = kin;
    kin = kout;
    kout = tk;
    V* tv = vin;
    vin = vout;
    vout = tv;
    sel ^= 1;
    shift += bits;
    --passes;
  }
  *selector = sel;
  return TGS_OK;
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
  TGS_CHECK_ARG(n < (1ull << 32) - SORT_TILE, "radix_sort: n too large");
  if (workspace_bytes < tgs_radix_sort_workspace_size(n)) {
    tgs_set_error("radix_sort: workspace %zu < %zu", workspace_bytes,
                  tgs_radix_sort_workspace_size(n));
    return TGS_ERR_WORKSPACE;
  }
  RadixSegs sg{};
  sg.n = 1;
  sg.key_off[0] = 0;
  sg.key_off[1] = (uint32_t)n;
  sg.tile_base[0] = 0;
  sg.tile_base[1] = (uint32_t)sort_tiles(n);
  return radix_passes<uint64_t, uint32_t>(keys, vals, keys_alt, vals_alt, sg, begin_bit, end_bit,
                                          workspace, selector, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of tgs_radix_sort_pairs for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops that
// forbid hipMalloc).  Its histograms, their scan and the scan's block sums
// live in a file-scope device array sized for TGS_NOALLOC_SORT_MAX_KEYS keys
// (16.0 MiB held by every GPU the library runs on until the process ends).
// Every pass writes each histogram entry before any is read, so the array
// needs no clearing between calls; calls that overlap on one GPU share it and
// race.  Host code reaches the array only through the address that
// hipGetSymbolAddress returns per device (the symbol's name is a host-side
// stand-in, not a device address).
// ---------------------------------------------------------------------------
#define TGS_NOALLOC_SORT_MAX_KEYS (1ull << 25)
#define TGS_NOALLOC_SORT_TILES ((TGS_NOALLOC_SORT_MAX_KEYS + SORT_TILE - 1) / SORT_TILE)
#define TGS_ALIGN256(b) ((((uint64_t)(b)) + 255ull) & ~255ull)
#define TGS_NOALLOC_SORT_HIST (TGS_NOALLOC_SORT_TILES * SORT_BINS)
#define TGS_NOALLOC_SORT_BYTES                          \
  (TGS_ALIGN256(TGS_NOALLOC_SORT_HIST * 4ull) * 2ull + \
   TGS_ALIGN256((TGS_NOALLOC_SORT_HIST + SCAN_CHUNK - 1) / SCAN_CHUNK * 8ull + 8ull))
#define TGS_MAX_DEVICES 64

static __device__ __align__(256) uint8_t scratch[TGS_NOALLOC_SORT_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[TGS_MAX_DEVICES] = {};

// Device address of `scratch` on the current device, looked up once per device.
static int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    tgs_set_error("radix_sort_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  if (dev < 0 || dev >= TGS_MAX_DEVICES) {
    tgs_set_error("radix_sort_noalloc: device %d out of range", dev);
    return TGS_ERR_ARG;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      tgs_set_error("radix_sort_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return e != hipSuccess ? (int)e : TGS_ERR_ARG;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TGS_OK;
}

extern "C" int tgs_radix_sort_pairs_noalloc(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt,
                                            uint32_t* vals_alt, uint64_t n, int begin_bit,
                                            int end_bit, int* selector, hipStream_t stream) {
  TGS_CHECK_ARG(selector != nullptr, "radix_sort_noalloc: null selector");
  *selector = 0;
  if (n > TGS_NOALLOC_SORT_MAX_KEYS) {
    tgs_set_error("radix_sort_noalloc: %llu keys exceed the allocation-free maximum of %llu; "
                  "use tgs_radix_sort_pairs with a workspace",
                  (unsigned long long)n, (unsigned long long)TGS_NOALLOC_SORT_MAX_KEYS);
    return TGS_ERR_ARG;
  }
  if (n <= 1 || end_bit <= begin_bit) return TGS_OK;
  TGS_CHECK_ARG(keys && vals && keys_alt && vals_alt, "radix_sort_noalloc: null pointer");
  TGS_CHECK_ARG(begin_bit >= 0 && end_bit <= 64, "radix_sort_noalloc: bit range out of [0,64]");
  static_assert(TGS_NOALLOC_SORT_BYTES >=
                    TGS_ALIGN256(TGS_NOALLOC_SORT_HIST * 4ull) * 2ull +
                        TGS_ALIGN256((TGS_NOALLOC_SORT_HIST + SCAN_CHUNK - 1) / SCAN_CHUNK * 8ull +
                                     8ull),
                "scratch smaller than the sort workspace");
  if (radix_workspace(sort_tiles(n)) > TGS_NOALLOC_SORT_BYTES) {
    tgs_set_error("radix_sort_noalloc: workspace %zu exceeds the scratch array",
                  radix_workspace(sort_tiles(n)));
    return TGS_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  const int rc = noalloc_scratch(&ws);
  if (rc) return rc;
  RadixSegs sg{};
  sg.n = 1;
  sg.key_off[0] = 0;
  sg.key_off[1] = (uint32_t)n;
  sg.tile_base[0] = 0;
  sg.tile_base[1] = (uint32_t)sort_tiles(n);
  return radix_passes<uint64_t, uint32_t>(keys, vals, keys_alt, vals_alt, sg, begin_bit, end_bit,
                                          ws, selector, stream);
}

// Segmented stable sort of uint32 keys with 4- or 8-byte values: each segment
// [seg_offsets[s], seg_offsets[s+1]) is sorted on its own.  seg_offsets is a
// HOST array of n_segments+1 non-decreasing offsets from 0 to n.
static int segmented_sort_u32(uint32_t* keys, void* vals, uint32_t* keys_alt, void* vals_alt,
                              uint32_t value_bytes, uint64_t n, uint32_t n_segments,
                              const uint32_t* seg_offsets, uint32_t key_base, uint32_t key_cap,
                              int begin_bit, int end_bit, void* workspace, size_t workspace_bytes,
                              int* selector, hipStream_t stream, bool first_hist_ready);

extern "C" int tgs_segmented_sort_pairs_u32(uint32_t* keys, void* vals, uint32_t* keys_alt,
                                            void* vals_alt, uint32_t value_bytes, uint64_t n,
                                            uint32_t n_segments, const uint32_t* seg_offsets,
                                            int begin_bit, int end_bit, void* workspace,
                                            size_t workspace_bytes, int* selector,
                                            hipStream_t stream) {
  return segmented_sort_u32(keys, vals, keys_alt, vals_alt, value_bytes, n, n_segments,
                            seg_offsets, 0u, 0xffffffffu, begin_bit, end_bit, workspace,
                            workspace_bytes, selector, stream, false);
}

// The same sort (4-byte values) with the first pass's per-tile digit counts
// already in the workspace, counted by the producer of the keys: uint32 word
// tile_base[s] * 256 + d * (tile_base[s + 1] - tile_base[s]) + t holds the
// count of digit d ((key >> begin_bit) & (2^w - 1), w the first pass's width:
// the key bits split into ceil(bits / 8) passes of ceil(bits / passes) bits)
// among keys [t * 4096, t * 4096 + 4096) of segment s, where tile_base[s] sums
// ceil(segment size / 4096) over the segments before s.
extern "C" int tgs_segmented_sort_pairs_u32_hist0(uint32_t* keys, uint32_t* vals,
                                                  uint32_t* keys_alt, uint32_t* vals_alt,
                                                  uint64_t n, uint32_t n_segments,
                                                  const uint32_t* seg_offsets, int begin_bit,
                                                  int end_bit, void* workspace,
                                                  size_t workspace_bytes, int* selector,
                                                  hipStream_t stream) {
  TGS_CHECK_ARG(begin_bit == 0, "segmented_sort_hist0: the precounted first pass starts at bit 0");
  return segmented_sort_u32(keys, vals, keys_alt, vals_alt, 4, n, n_segments, seg_offsets, 0u,
                            0xffffffffu, begin_bit, end_bit, workspace, workspace_bytes, selector,
                            stream, true);
}

// The same sort on key_bits bits of min(key - key_base, 2^key_bits - 1) (keys
// below key_base as 0): a key range known to lie in [key_base, key_base +
// 2^key_bits - 1) is sorted in fewer or narrower passes, and keys past it
// (a sentinel such as 0xffffffff) tie at the top, in their input order.
extern "C" int tgs_segmented_sort_pairs_u32_range(uint32_t* keys, void* vals, uint32_t* keys_alt,
                                                  void* vals_alt, uint32_t value_bytes, uint64_t n,
                                                  uint32_t n_segments,
                                                  const uint32_t* seg_offsets, uint32_t key_base,
                                                  int key_bits, void* workspace,
                                                  size_t workspace_bytes, int* selector,
                                                  hipStream_t stream) {
  TGS_CHECK_ARG(key_bits >= 1 && key_bits <= 32, "segmented_sort_range: key_bits in [1, 32]");
  const uint32_t cap = key_bits == 32 ? 0xffffffffu : (1u << key_bits) - 1u;
  return segmented_sort_u32(keys, vals, keys_alt, vals_alt, value_bytes, n, n_segments,
                            seg_offsets, key_base, cap, 0, key_bits, workspace, workspace_bytes,
                            selector, stream, false);
}

static int segmented_sort_u32(uint32_t* keys, void* vals, uint32_t* keys_alt, void* vals_alt,
                              uint32_t value_bytes, uint64_t n, uint32_t n_segments,
                              const uint32_t* seg_offsets, uint32_t key_base, uint32_t key_cap,
                              int begin_bit, int end_bit, void* workspace, size_t workspace_bytes,
                              int* selector, hipStream_t stream, bool first_hist_ready) {
  TGS_CHECK_ARG(selector != nullptr, "segmented_sort: null selector");
  *selector = 0;
  if (n <= 1 || end_bit <= begin_bit) return TGS_OK;
  TGS_CHECK_ARG(keys && vals && keys_alt && vals_alt && workspace && seg_offsets,
                "segmented_sort: null pointer");
  TGS_CHECK_ARG(value_bytes == 4 || value_bytes == 8, "segmented_sort: value_bytes must be 4 or 8");
  TGS_CHECK_ARG(begin_bit >= 0 && end_bit <= 32, "segmented_sort: bit range out of [0,32]");
  TGS_CHECK_ARG(n < (1ull << 32) - (uint64_t)SORT_TILE * (RADIX_MAX_SEGS + 1),
                "segmented_sort: n too large");
  TGS_CHECK_ARG(n_segments >= 1 && n_segments <= RADIX_MAX_SEGS,
                "segmented_sort: n_segments must be in [1, 64]");
  TGS_CHECK_ARG(seg_offsets[0] == 0 && seg_offsets[n_segments] == n,
                "segmented_sort: segments must cover [0, n)");
  RadixSegs sg{};
  sg.n = n_segments;
  sg.key_base = key_base;
  sg.key_cap = key_cap;
  uint32_t tiles = 0;
  for (uint32_t s = 0; s < n_segments; ++s) {
    TGS_CHECK_ARG(seg_offsets[s + 1] >= seg_offsets[s], "segmented_sort: offsets decrease");
    sg.key_off[s] = seg_offsets[s];
    sg.tile_base[s] = tiles;
    tiles += (uint32_t)sort_tiles(seg_offsets[s + 1] - seg_offsets[s]);
  }
  sg.key_off[n_segments] = (uint32_t)n;
  sg.tile_base[n_segments] = tiles;
  if (workspace_bytes < tgs_segmented_sort_workspace_size(n, n_segments)) {
    tgs_set_error("segmented_sort: workspace %zu < %zu", workspace_bytes,
                  tgs_segmented_sort_workspace_size(n, n_segments));
    return TGS_ERR_WORKSPACE;
  }
  if (tiles == 0) return TGS_OK;
  if (value_bytes == 4)
    return radix_passes<uint32_t, uint32_t>(keys, (uint32_t*)vals, keys_alt, (uint32_t*)vals_alt,
                                            sg, begin_bit, end_bit, workspace, selector, stream,
                                            first_hist_ready);
  TGS_CHECK_ARG(!first_hist_ready, "segmented_sort: a precounted first pass needs 4-byte values");
  return radix_passes<uint32_t, uint64_t>(keys, (uint64_t*)vals, keys_alt, (uint64_t*)vals_alt, sg,
                                          begin_bit, end_bit, workspace, selector, stream);
}
