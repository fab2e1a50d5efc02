/*
 * tidegs_amd.h — C ABI of the MI355X (gfx950) TideGS hot-path kernels.
 *
 * Conventions
 *   - Every pointer is a device pointer (hipMalloc'd / PyTorch caching
 *     allocator) unless stated otherwise; the library never allocates or frees
 *     device memory.  Temporary storage is passed in as `workspace` after a
 *     `*_workspace_size` query, like the reference's CUB_WRAPPER
 *     (gsplat/cuda/csrc/bindings.h:16-23).
 *   - All work is enqueued on the given `stream`; calls are reentrant (no
 *     mutable globals apart from a thread-local error string).
 *   - Return 0 on success, a positive hipError_t on a HIP failure, or a
 *     negative TGS_ERR_* code for an argument error; tgs_last_error() then
 *     describes it (the reference raises through TORCH_CHECK / AT_ERROR,
 *     bindings.h:7-13).
 *   - Floating point is fp32 throughout.
 */
#ifndef TIDEGS_AMD_H
#define TIDEGS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* tgs_stream_t; /* == hipStream_t */

#define TGS_OK 0
#define TGS_ERR_ARG (-1)
#define TGS_ERR_UNSUPPORTED (-2)
#define TGS_ERR_WORKSPACE (-3)

/* ---- library ---------------------------------------------------------- */
int tgs_abi_version(void);
const char* tgs_last_error(void);
/* Zero/constant fill used instead of hipMemsetAsync (kernel node under capture). */
int tgs_fill_u32(void* ptr, uint64_t n_words, uint32_t value, tgs_stream_t stream);

/* ---- projection ------------------------------------------------------- */
/* Replaces fully_fused_projection_fwd_tensor
 * (gsplat/cuda/csrc/fully_fused_projection_fwd.cu:132-181; pybind ext.cpp).
 * means [N,3]; covars [N,6] or null; quats [N,4] (w,x,y,z) + scales [N,3]
 * when covars is null; viewmats [C,4,4] row-major w2c; Ks [C,3,3].
 * Outputs radii [C,N] i32, means2d [C,N,2], depths [C,N], conics [C,N,3],
 * compensations [C,N] or null.  Culled entries: radius 0 and zeros. */
int tgs_fully_fused_projection_fwd(uint32_t C, uint32_t N, const float* means,
                                   const float* covars, const float* quats, const float* scales,
                                   const float* viewmats, const float* Ks, int32_t image_width,
                                   int32_t image_height, float eps2d, float near_plane,
                                   float far_plane, float radius_clip, int32_t* radii,
                                   float* means2d, float* depths, float* conics,
                                   float* compensations, tgs_stream_t stream);

/* Replaces fully_fused_projection_bwd_tensor
 * (gsplat/cuda/csrc/fully_fused_projection_bwd.cu:187-268).  Writes v_means
 * and v_quats/v_scales (or v_covars) for every Gaussian (no zero-fill needed);
 * v_viewmats (nullable) is accumulated and must be zeroed by the caller.
 * v_depths and v_compensations may be null (treated as zero / absent). */
int tgs_fully_fused_projection_bwd(uint32_t C, uint32_t N, const float* means,
                                   const float* covars, const float* quats, const float* scales,
                                   const float* viewmats, const float* Ks, int32_t image_width,
                                   int32_t image_height, float eps2d, const int32_t* radii,
                                   const float* conics, const float* compensations,
                                   const float* v_means2d, const float* v_depths,
                                   const float* v_conics, const float* v_compensations,
                                   float* v_means, float* v_covars, float* v_quats,
                                   float* v_scales, float* v_viewmats, tgs_stream_t stream);

/* Packed projection: replaces fully_fused_projection_packed_fwd_tensor
 * (gsplat/cuda/csrc/fully_fused_projection_packed_fwd.cu:184-275), the
 * projection with the packed radius rule (sqrt(max(0.1, b^2 - det)), :111-119)
 * whose survivors are written as COO entries in camera-major, Gaussian-ascending
 * order.  Same two passes as the reference:
 *   1. tgs_fully_fused_projection_packed_count: per block of 256 Gaussians of
 *      one camera, block_counts[c * blocks + b] = survivors
 *      (blocks = tgs_fully_fused_projection_packed_blocks(N));
 *   2. after an exclusive scan of block_counts into block_offsets (nnz = last
 *      offset + last count), tgs_fully_fused_projection_packed_fwd writes
 *      indptr [C+1], camera_ids/gaussian_ids [nnz] (int64), radii [nnz] (int32),
 *      means2d [nnz,2], depths [nnz], conics [nnz,3], compensations [nnz]
 *      (nullable). */
uint32_t tgs_fully_fused_projection_packed_blocks(uint32_t N);
int tgs_fully_fused_projection_packed_count(uint32_t C, uint32_t N, const float* means,
                                            const float* covars, const float* quats,
                                            const float* scales, const float* viewmats,
                                            const float* Ks, int32_t image_width,
                                            int32_t image_height, float eps2d, float near_plane,
                                            float far_plane, float radius_clip,
                                            int32_t* block_counts, tgs_stream_t stream);
int tgs_fully_fused_projection_packed_fwd(uint32_t C, uint32_t N, const float* means,
                                          const float* covars, const float* quats,
                                          const float* scales, const float* viewmats,
                                          const float* Ks, int32_t image_width,
                                          int32_t image_height, float eps2d, float near_plane,
                                          float far_plane, float radius_clip,
                                          const int32_t* block_offsets, uint32_t nnz,
                                          int32_t* indptr, int64_t* camera_ids,
                                          int64_t* gaussian_ids, int32_t* radii, float* means2d,
                                          float* depths, float* conics, float* compensations,
                                          tgs_stream_t stream);
/* Replaces fully_fused_projection_packed_bwd_tensor
 * (gsplat/cuda/csrc/fully_fused_projection_packed_bwd.cu:18-260).  With
 * sparse_grad the VJPs are written per entry ([nnz, .]); otherwise they are
 * added into [N, .] gradients, which the caller zeroes.  v_viewmats (nullable)
 * is accumulated. */
int tgs_fully_fused_projection_packed_bwd(uint32_t C, uint32_t N, uint32_t nnz, const float* means,
                                          const float* covars, const float* quats,
                                          const float* scales, const float* viewmats,
                                          const float* Ks, int32_t image_width,
                                          int32_t image_height, float eps2d,
                                          const int64_t* camera_ids, const int64_t* gaussian_ids,
                                          const float* conics, const float* compensations,
                                          const float* v_means2d, const float* v_depths,
                                          const float* v_conics, const float* v_compensations,
                                          int sparse_grad, float* v_means, float* v_covars,
                                          float* v_quats, float* v_scales, float* v_viewmats,
                                          tgs_stream_t stream);

/* ---- spherical harmonics ---------------------------------------------- */
/* Replaces compute_sh_fwd_tensor (gsplat/cuda/csrc/compute_sh_fwd.cu:31-58).
 * dirs [n,3], coeffs [n,K,3], masks [n] u8/bool or null -> colors [n,3]. */
int tgs_compute_sh_fwd(uint32_t n, uint32_t K, int32_t degrees_to_use, const float* dirs,
                       const float* coeffs, const uint8_t* masks, float* colors,
                       tgs_stream_t stream);
/* Replaces compute_sh_bwd_tensor (gsplat/cuda/csrc/compute_sh_bwd.cu:101-136).
 * Writes all of v_coeffs [n,K,3]; v_dirs [n,3] nullable. */
int tgs_compute_sh_bwd(uint32_t n, uint32_t K, int32_t degrees_to_use, const float* dirs,
                       const float* coeffs, const uint8_t* masks, const float* v_colors,
                       float* v_coeffs, float* v_dirs, tgs_stream_t stream);

/* ---- tile intersection ------------------------------------------------- */
/* bit_width(v): floor(log2 v) + 1 (isect_tiles.cu:143-144). */
uint32_t tgs_bit_width(uint32_t v);
/* First pass of isect_tiles (isect_tiles.cu:14-71,155-164): tiles_per_gauss. */
int tgs_isect_tiles_count(uint64_t total, const float* means2d, const int32_t* radii,
                          uint32_t tile_size, uint32_t tile_width, uint32_t tile_height,
                          int32_t* tiles_per_gauss, tgs_stream_t stream);
/* torch.cumsum replacement (isect_tiles.cu:165): int32 in, int64 inclusive out. */
size_t tgs_scan_workspace_size(uint64_t n);
int tgs_inclusive_scan_i32_i64(const int32_t* in, int64_t* out, uint64_t n, void* workspace,
                               size_t workspace_bytes, tgs_stream_t stream);
int tgs_exclusive_scan_u32(const uint32_t* in, uint32_t* out, uint64_t n, void* workspace,
                           size_t workspace_bytes, tgs_stream_t stream);
/* Second pass of isect_tiles (isect_tiles.cu:73-98,171-187).  camera_ids
 * [total] i64 for packed inputs, else null with N Gaussians per camera. */
int tgs_isect_tiles_emit(uint64_t total, uint32_t N, const int64_t* camera_ids,
                         const float* means2d, const int32_t* radii, const float* depths,
                         const int64_t* cum_tiles_per_gauss, uint32_t tile_size,
                         uint32_t tile_width, uint32_t tile_height, uint32_t tile_n_bits,
                         int64_t* isect_ids, int32_t* flatten_ids, tgs_stream_t stream);
/* cub::DeviceRadixSort::SortPairs replacement (isect_tiles.cu:189-227): stable
 * ascending sort on key bits [begin_bit, end_bit); double-buffered, *selector
 * (host int) = 0 if the result is in keys/vals, 1 if in keys_alt/vals_alt. */
size_t tgs_radix_sort_workspace_size(uint64_t n);
int tgs_radix_sort_pairs(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt, uint32_t* vals_alt,
                         uint64_t n, int begin_bit, int end_bit, void* workspace,
                         size_t workspace_bytes, int* selector, tgs_stream_t stream);
/* No counterpart in the reference: tgs_radix_sort_pairs without a workspace
 * argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops that forbid hipMalloc).  Its temporary storage
 * is a file-scope device array of 16.0 MiB per GPU, held until the process
 * ends; n may be at most 2^25 (33,554,432) keys, larger n returns
 * TGS_ERR_ARG with an error text.  Calls no allocator.  Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (concurrent streams
 * or threads) race. */
int tgs_radix_sort_pairs_noalloc(uint64_t* keys, uint32_t* vals, uint64_t* keys_alt,
                                 uint32_t* vals_alt, uint64_t n, int begin_bit, int end_bit,
                                 int* selector, tgs_stream_t stream);
/* Segmented stable sort of uint32 keys with 4- or 8-byte values (the
 * camera-grouped sorts of the fused step; a plain sort is one segment): each
 * segment [seg_offsets[s], seg_offsets[s+1]) is sorted on key bits
 * [begin_bit, end_bit) on its own.  seg_offsets is a HOST array of
 * n_segments+1 (<= 65) non-decreasing offsets from 0 to n.  Double-buffered
 * like tgs_radix_sort_pairs. */
size_t tgs_segmented_sort_workspace_size(uint64_t n, uint32_t n_segments);
/* Beside the reference's interface: tgs_segmented_sort_pairs_u32 with 4-byte
 * values whose first pass's per-tile digit counts are already at the start of
 * the workspace (word tile_base[s] * 256 + d * (tile_base[s + 1] -
 * tile_base[s]) + t: digit d among keys [4096 t, 4096 t + 4096) of segment s;
 * tile_base sums ceil(size / 4096) over the earlier segments; the first pass
 * takes ceil(bits / passes) bits, passes = ceil(bits / 8)). */
int tgs_segmented_sort_pairs_u32_hist0(uint32_t* keys, uint32_t* vals, uint32_t* keys_alt,
                                       uint32_t* vals_alt, uint64_t n, uint32_t n_segments,
                                       const uint32_t* seg_offsets, int begin_bit, int end_bit,
                                       void* workspace, size_t workspace_bytes, int* selector,
                                       tgs_stream_t stream);
int tgs_segmented_sort_pairs_u32(uint32_t* keys, void* vals, uint32_t* keys_alt, void* vals_alt,
                                 uint32_t value_bytes, uint64_t n, uint32_t n_segments,
                                 const uint32_t* seg_offsets, int begin_bit, int end_bit,
                                 void* workspace, size_t workspace_bytes, int* selector,
                                 tgs_stream_t stream);
/* The same sort on key_bits bits of min(key - key_base, 2^key_bits - 1), keys
 * below key_base counting as key_base: when the keys lie in [key_base,
 * key_base + 2^key_bits - 1) this is their full order in fewer or narrower
 * passes, and keys above the range (a sentinel such as 0xffffffff) all tie
 * after it in input order.  No counterpart in the reference (its sort takes
 * a bit range only); used by the fused step's depth sort. */
int tgs_segmented_sort_pairs_u32_range(uint32_t* keys, void* vals, uint32_t* keys_alt,
                                       void* vals_alt, uint32_t value_bytes, uint64_t n,
                                       uint32_t n_segments, const uint32_t* seg_offsets,
                                       uint32_t key_base, int key_bits, void* workspace,
                                       size_t workspace_bytes, int* selector,
                                       tgs_stream_t stream);
/* Replaces isect_offset_encode_tensor (isect_tiles.cu:234-301); offsets [C,th,tw]. */
int tgs_isect_offset_encode(uint64_t n_isects, const int64_t* isect_ids, uint32_t C,
                            uint32_t tile_width, uint32_t tile_height, int32_t* offsets,
                            tgs_stream_t stream);

/* ---- rasterization ---------------------------------------------------- */
/* Channel counts with an instantiated kernel; returns their number. */
int tgs_rasterize_supported_channels(int32_t* out, int32_t cap);
/* Replaces rasterize_to_pixels_fwd_tensor (rasterize_to_pixels_fwd.cu:236-284).
 * means2d/conics/colors/opacities [C,N,*] or packed [nnz,*]; backgrounds
 * [C,channels] or null; render_colors [C,H,W,ch], render_alphas [C,H,W,1],
 * last_ids [C,H,W] i32. tile_size 8 or 16. */
int tgs_rasterize_to_pixels_fwd(uint32_t C, uint32_t channels, const float* means2d,
                                const float* conics, const float* colors, const float* opacities,
                                const float* backgrounds, uint32_t image_width,
                                uint32_t image_height, uint32_t tile_size, uint32_t tile_width,
                                uint32_t tile_height, const int32_t* tile_offsets,
                                const int32_t* flatten_ids, uint32_t n_isects,
                                float* render_colors, float* render_alphas, int32_t* last_ids,
                                tgs_stream_t stream);
/* Replaces rasterize_to_pixels_bwd_tensor (rasterize_to_pixels_bwd.cu:347-402).
 * Gradient outputs are accumulated: zero them first.  v_render_alphas and
 * v_means2d_abs (absgrad) may be null. */
int tgs_rasterize_to_pixels_bwd(uint32_t C, uint32_t channels, const float* means2d,
                                const float* conics, const float* colors, const float* opacities,
                                const float* backgrounds, uint32_t image_width,
                                uint32_t image_height, uint32_t tile_size, uint32_t tile_width,
                                uint32_t tile_height, const int32_t* tile_offsets,
                                const int32_t* flatten_ids, uint32_t n_isects,
                                const float* render_alphas, const int32_t* last_ids,
                                const float* v_render_colors, const float* v_render_alphas,
                                float* v_means2d_abs, float* v_means2d, float* v_conics,
                                float* v_colors, float* v_opacities, tgs_stream_t stream);

/* ---- fused SSIM -------------------------------------------------------- */
/* Replaces fusedssim (clm_kernels/ssim.cu:368-408): NCHW img1/img2 ->
 * ssim_map and (all or none) of the three partial maps. */
int tgs_fused_ssim_fwd(int32_t B, int32_t CH, int32_t H, int32_t W, float C1, float C2,
                       const float* img1, const float* img2, float* ssim_map, float* dm_dmu1,
                       float* dm_dsigma1_sq, float* dm_dsigma12, tgs_stream_t stream);
/* Replaces fusedssim_backward (clm_kernels/ssim.cu:410-444). */
int tgs_fused_ssim_bwd(int32_t B, int32_t CH, int32_t H, int32_t W, float C1, float C2,
                       const float* img1, const float* img2, const float* dL_dmap,
                       const float* dm_dmu1, const float* dm_dsigma1_sq, const float* dm_dsigma12,
                       float* dL_dimg1, tgs_stream_t stream);
/* Fused L1 + SSIM training loss of strategies/base_engine.py:464-488 for B
 * rendered images [B,H,W,3] (HWC) against gt [B,3,H,W]: forward and
 * backward in one pass.  sums[2b] += sum|I_b - gt'_b|, sums[2b+1] += sum SSIM
 * (double[2B], caller-zeroed), gt' = clamp(gt / gt_div, 0, 1);
 * v_images = dL_b/dI_b (HWC) of
 * L_b = (1-lambda) mean|I_b-gt'_b| + lambda (1 - mean SSIM_b). */
int tgs_tide_loss(int32_t B, int32_t H, int32_t W, const float* images_hwc, const float* gt_chw,
                  float gt_div, float lambda_dssim, double* sums, float* v_images_hwc,
                  tgs_stream_t stream);

/* ---- resident optimizer ------------------------------------------------ */
/* Replaces the six _fused_resident_adam_kernel launches of GPUResidentAdam.step
 * (strategies/tide_engine/gpu_resident_optimizer.py:16-70, :397-418, :474-499)
 * and its searchsorted slot mapping (:266-300) with one launch.
 * local_rows [n_rows] (i64 if index_is_i64 else i32) index the working-set
 * params; block layout = sorted [start,end) slices with their state slots
 * (device i64 arrays of n_layout); bias tables per slot (:302-337).
 * Host arrays (length n_components <= 8, total width <= 64): params, grads
 * ([n_rows, w] rows), exp_avg, exp_avg_sq ([slots*block_size, w] rows) device
 * pointers, widths, lrs, and row_strides [3*n_components] (param, grad,
 * state row strides in elements; null = dense rows of `width`), so split
 * component tensors and column views of one [N,59] table both work.  error_flag (device int, caller-zeroed) becomes
 * nonzero if a row lies outside every block. */
int tgs_resident_adam_step(int64_t n_rows, const void* local_rows, int index_is_i64,
                           const int64_t* block_starts, const int64_t* block_ends,
                           const int64_t* block_slots, int64_t n_layout, int64_t block_size,
                           const float* bias_correction1, const float* denom_scale,
                           int n_components, float* const* params, const float* const* grads,
                           float* const* exp_avg, float* const* exp_avg_sq,
                           const int32_t* widths, const int64_t* row_strides, const float* lrs,
                           float beta1, float beta2, float eps, float batch_size,
                           int* error_flag, tgs_stream_t stream);
/* Sophia-style step (no reference implementation; defined from Liu et al.
 * 2023): m = b1 m + (1-b1) g; h = b2 h + (1-b2) g*g when update_hessian;
 * p -= lr clamp(m / max(h, eps), -rho, rho).  Same layout as Adam. */
int tgs_resident_sophia_step(int64_t n_rows, const void* local_rows, int index_is_i64,
                             const int64_t* block_starts, const int64_t* block_ends,
                             const int64_t* block_slots, int64_t n_layout, int64_t block_size,
                             int n_components, float* const* params, const float* const* grads,
                             float* const* exp_avg, float* const* hessian, const int32_t* widths,
                             const int64_t* row_strides, const float* lrs, float beta1,
                             float beta2, float eps, float rho, float batch_size,
                             int update_hessian, int* error_flag, tgs_stream_t stream);
/* Touched rows per layout entry (replaces unique_consecutive at
 * gpu_resident_optimizer.py:293-297): counts [n_layout] i64. */
int tgs_block_touch_counts(int64_t n_rows, const void* rows, int index_is_i64,
                           const int64_t* block_starts, const int64_t* block_ends,
                           int64_t n_layout, int64_t* counts, tgs_stream_t stream);

/* ---- fused resident step (one launch per stage for a batch of cameras) ---- */
/* These replace TideGS's per-camera loop (strategies/tide_engine/engine.py:
 * 1435-1827 filters + touched rows, 1874-2695 per-camera render/backward,
 * 2434-2469 scatter_add) over a resident [N,59] fp32 table in CACHE column
 * order (storage/block_reader.py:35-44).  Cameras per batch: 1..32.
 * row_stride (>= 59 floats) is the table's row pitch: 59 for a dense table,
 * 64 for the padded layout whose rows are whole 256-byte lines. */
/* Camera centres campos [C,3] = translation of inverse(viewmats[c]) for affine
 * world->camera matrices (the SH view directions of engine.py:458-512). */
int tgs_tide_camera_centers(uint32_t C, const float* viewmats, float* campos, tgs_stream_t stream);
/* Row blocks of the visibility/compaction passes for n_rows rows. */
uint32_t tgs_tide_row_blocks(uint64_t n_rows);
/* Packed-projection visibility (gsplat fully_fused_projection_packed_fwd.cu:
 * 50-131) of every row in every camera: masks [N] (bit c = camera c), and
 * per-block counts [(C+2)*nb] (per camera, touched rows, visits).  With
 * depth_range (device, may be null; 128 uint32), 64 {min, max} pairs whose
 * min over the mins and max over the maxes are the smallest and largest float
 * bits of the visible entries' depths (pairs that saw none hold {~0, 0}). */
int tgs_tide_visibility(uint64_t n_rows, const float* params, uint32_t row_stride, uint32_t C,
                        const float* viewmats, const float* Ks, const float* campos, int32_t W,
                        int32_t H, float eps2d,
                        float near_plane, float far_plane, float radius_clip, uint32_t* masks,
                        uint32_t* counts, uint32_t* depth_range, tgs_stream_t stream);
/* Compaction from offs = exclusive scan of counts: entries (concatenated
 * per-camera filters, ascending rows, base_engine.py:388-425), touched rows,
 * visit lists per touched row (entries in camera order), totals [C+3]
 * (V_c..., T, sum V, visits) and cam_offsets [C+1]. Buffers sized C*N / N. */
int tgs_tide_compact(uint64_t n_rows, uint32_t C, const uint32_t* masks, const uint32_t* counts,
                     const uint32_t* offs, int32_t* entries, int32_t* touched,
                     int32_t* visit_base, int32_t* visits, uint32_t* totals,
                     int32_t* cam_offsets, tgs_stream_t stream);
/* Projection + SH colour + activations per entry (engine.py:458-512 with
 * base_gaussian_model.py:35-50), one thread per touched row over its visits
 * (entries of the cameras in its visibility mask, camera order) ->
 * splats [V,12] (3 x float4: {x,y,opacity,depth},{a,b,c,radius},{r,g,b,0}),
 * depth_keys [V] (float bits of the depth; 0xffffffff when culled) and
 * entry_rects [V] (tile rectangle x0|x1<<8|y0<<16|y1<<24 in the high word,
 * entry index in the low word; isect_tiles.cu:55-70).  Tile grid at most
 * 255 x 255.  n_touched_dev (device, may be null) holds the touched-row
 * count when the host does not know it yet; n_touched is then the launch's
 * capacity (rows beyond the device count do nothing).  isect_totals (device,
 * may be null) receives the per-camera intersection counts [C] (int64, the
 * sums of the rectangles' areas; the call zeroes it first), so the host can
 * size the intersection buffers while the depth sort runs.  depth_range
 * (device, may be null) receives 64 {min, max} uint32 pairs (the call
 * initialises them) whose min / max are the smallest and largest depth key
 * written, culled entries' 0xffffffff excluded: the host checks with them
 * that the depth sort's key range, taken from tgs_tide_visibility's
 * depth_range, holds every key. */
int tgs_tide_project_fwd(uint32_t n_touched, const uint32_t* n_touched_dev,
                         const int32_t* touched, const int32_t* visit_base,
                         const int32_t* visits, const uint32_t* masks, uint32_t C,
                         const float* params, uint32_t row_stride, const float* viewmats,
                         const float* Ks,
                         const float* campos, int32_t W, int32_t H, float eps2d, float near_plane,
                         float far_plane, float radius_clip, int32_t sh_degree,
                         uint32_t tile_size, uint32_t tile_width, uint32_t tile_height,
                         float* splats, uint32_t* depth_keys, uint64_t* entry_rects,
                         int64_t* isect_totals, uint32_t* depth_range, tgs_stream_t stream);
/* Intersections of the batch in the order of the reference's sort
 * (isect_tiles.cu:73-98,189-227: camera, tile, depth bits, entry).  After
 * tgs_segmented_sort_pairs_u32 of (depth_keys, entry_rects) per camera:
 *   tgs_tide_isect_count     tiles [V] of the depth-ordered entries;
 *   (tgs_inclusive_scan_i32_i64 -> cum_tiles)
 *   tgs_tide_isect_segments  seg [C+1] (int64): first intersection of each
 *                            camera (seg[C] = n_isects; the caller must refuse
 *                            n_isects >= 2^31 before emitting: keys, flatten
 *                            ids and the bucket offsets are 32-bit);
 *   tgs_tide_isect_emit      keys [n_isects] = camera << tile_n_bits | tile,
 *                            flatten_ids = entry index, in depth order;
 *   (tgs_segmented_sort_pairs_u32 of the tile bits per camera)
 *   tgs_tide_offset_encode   offsets [C,th,tw] as tgs_isect_offset_encode;
 *   tgs_tide_isect_ids       the reference's int64 ids (inspection only). */
int tgs_tide_isect_count(uint32_t n_entries, const uint64_t* entry_rects, int32_t* tiles,
                         tgs_stream_t stream);
/* Per-camera intersection counts isect_totals [C] (int64) as the sums of the
 * entries' tile-rectangle areas (the counts isect_tiles.cu:55-70 produces),
 * straight from tgs_tide_project_fwd's entry_rects, so the host can size the
 * intersection buffers while the depth sort runs.  n_entries_dev (device, may
 * be null) holds the entry count; n_entries is then the launch's capacity. */
int tgs_tide_isect_totals(uint32_t n_entries, const uint32_t* n_entries_dev,
                          const uint64_t* entry_rects, const int32_t* cam_offsets, uint32_t C,
                          int64_t* isect_totals, tgs_stream_t stream);
int tgs_tide_isect_segments(uint32_t C, const int32_t* cam_offsets, const int64_t* cum_tiles,
                            int64_t* seg, tgs_stream_t stream);
int tgs_tide_isect_emit(uint32_t n_entries, const int32_t* cam_offsets, uint32_t C,
                        const uint64_t* entry_rects, const int64_t* cum_tiles,
                        uint32_t tile_width, uint32_t tile_n_bits, uint32_t* keys,
                        int32_t* flatten_ids, tgs_stream_t stream);
/* The same emission without per-entry offsets (the form TideStep uses): the
 * depth-ordered entries in blocks of 2048 (tgs_tide_isect_emit_blocks of
 * them); tgs_tide_isect_block_sums writes each block's rectangle-area sum
 * (uint32), the caller scans those sums (tgs_exclusive_scan_u32 -> block_base)
 * and tgs_tide_isect_emit_blocked writes keys and flatten ids exactly as
 * tgs_tide_isect_emit does.  Same 2^31 intersection limit. */
uint32_t tgs_tide_isect_emit_blocks(uint32_t n_entries);
int tgs_tide_isect_block_sums(uint32_t n_entries, const uint64_t* entry_rects,
                              uint32_t* block_sums, tgs_stream_t stream);
int tgs_tide_isect_emit_blocked(uint32_t n_entries, const int32_t* cam_offsets, uint32_t C,
                                const uint64_t* entry_rects, const uint32_t* block_base,
                                uint32_t tile_width, uint32_t tile_n_bits, uint32_t* keys,
                                int32_t* flatten_ids, tgs_stream_t stream);
/* Beside the reference's interface: tgs_tide_isect_emit_blocked that also
 * counts the digits of the first pass of tgs_segmented_sort_pairs_u32_hist0
 * over bits [0, tile_n_bits) (tile & (2^w - 1), w = ceil(tile_n_bits / p),
 * p = ceil(tile_n_bits / 8)) into hist, in the layout that sort reads
 * (segments = cameras, isect_cam_offsets = the C + 1 host-side first
 * intersections per camera); hist (hist_words uint32 words, e.g. the sort's
 * workspace) is cleared first. */
int tgs_tide_isect_emit_blocked_hist(uint32_t n_entries, const int32_t* cam_offsets, uint32_t C,
                                     const uint64_t* entry_rects, const uint32_t* block_base,
                                     uint32_t tile_width, uint32_t tile_n_bits, uint32_t* keys,
                                     int32_t* flatten_ids, const uint32_t* isect_cam_offsets,
                                     uint32_t* hist, uint64_t hist_words, tgs_stream_t stream);
/* Beside the reference's interface: the emission fused with the first pass of
 * the tile-bit sort (the form TideStep uses).  The depth-ordered entries of
 * each camera (cam_offsets: the C + 1 host-side first entries per camera) are
 * taken in blocks of 1024 that never span two cameras.
 *   tgs_tide_isect_fused_digit_bits  the first pass's width w over tile_n_bits
 *                                    bits (ceil(bits / 8) passes of
 *                                    ceil(bits / passes) bits);
 *   tgs_tide_isect_fused_hist_words  hist words: blocks * 2^w;
 *   tgs_tide_isect_fused_count       hist [camera][digit][block of the camera]
 *                                    = the block's intersections with tile &
 *                                    (2^w - 1) == digit;
 *   (tgs_exclusive_scan_u32 of hist -> hist_scan)
 *   tgs_tide_isect_fused_scatter     keys [n_isects] = camera << tile_n_bits |
 *                                    tile and flatten ids in the order of a
 *                                    stable sort of the emission (isect_tiles.cu
 *                                    :73-98 over the depth-ordered entries) on
 *                                    bits [0, w) within each camera;
 *   (tgs_segmented_sort_pairs_u32 on bits [w, tile_n_bits) per camera, when
 *    tile_n_bits > w, completes the tile-bit sort). */
uint32_t tgs_tide_isect_fused_digit_bits(uint32_t tile_n_bits);
uint64_t tgs_tide_isect_fused_hist_words(uint32_t C, const uint32_t* cam_offsets,
                                         uint32_t tile_n_bits);
int tgs_tide_isect_fused_count(uint32_t C, const uint32_t* cam_offsets,
                               const uint64_t* entry_rects, uint32_t tile_width,
                               uint32_t tile_n_bits, uint32_t* hist, uint64_t hist_words,
                               tgs_stream_t stream);
int tgs_tide_isect_fused_scatter(uint32_t C, const uint32_t* cam_offsets,
                                 const uint64_t* entry_rects, uint32_t tile_width,
                                 uint32_t tile_n_bits, const uint32_t* hist_scan,
                                 uint64_t hist_words, uint32_t n_isects, uint32_t* keys,
                                 int32_t* flatten_ids, tgs_stream_t stream);
int tgs_tide_offset_encode(uint32_t n_isects, const uint32_t* keys, uint32_t C,
                           uint32_t tile_width, uint32_t tile_height, uint32_t tile_n_bits,
                           int32_t* offsets, tgs_stream_t stream);
int tgs_tide_isect_ids(uint32_t n_isects, const uint32_t* keys, const int32_t* flatten_ids,
                       const float* splats, int64_t* isect_ids, tgs_stream_t stream);
/* Rasterize forward/backward over packed splats (tile 16, 3 channels);
 * images / v_images [C,H,W,3], alphas [C,H,W], last_ids [C,H,W];
 * splat_grads [V,9] accumulated (zero first): {mean2d 2, conic 3, color 3, opacity};
 * v_alphas [C,H,W] (dL/dalpha, nullable: zero).
 * The forward also zeroes clear[0..clear_words) (nullable; 16-byte aligned,
 * clear_words a multiple of 4), normally the backward's splat_grads: the
 * stores overlap the compositing instead of taking a pass of their own.
 * n_contrib [C,H,W] (nullable) receives each pixel's number of composited
 * Gaussians, the (Gaussian, pixel) pairs the backward replays; gsplat has no
 * such output (a measurement aid). */
int tgs_tide_rasterize_fwd(uint32_t C, const float* splats, const float* backgrounds, uint32_t W,
                           uint32_t H, uint32_t tile_width, uint32_t tile_height,
                           const int32_t* tile_offsets, const int32_t* flatten_ids,
                           uint32_t n_isects, float* images, float* alphas, int32_t* last_ids,
                           int32_t* n_contrib, float* clear, uint64_t clear_words,
                           tgs_stream_t stream);
int tgs_tide_rasterize_bwd(uint32_t C, const float* splats, const float* backgrounds, uint32_t W,
                           uint32_t H, uint32_t tile_width, uint32_t tile_height,
                           const int32_t* tile_offsets, const int32_t* flatten_ids,
                           uint32_t n_isects, const float* alphas, const int32_t* last_ids,
                           const float* v_images, const float* v_alphas, float* splat_grads,
                           tgs_stream_t stream);
/* The drop-in rasterizer's 3-channel path (rasterize_to_pixels_fwd.cu:162-284,
 * rasterize_to_pixels_bwd.cu:251-402 with 3 channels): gsplat's SoA tensors
 * means2d [n,2], conics [n,3], colors [n,3], opacities [n] packed into the
 * splat records above (16-byte aligned [n,12]; radius and depth slots 0), and
 * the [n,9] gradient records unpacked into the SoA gradient tensors. */
int tgs_pack_splats(uint64_t n, const float* means2d, const float* conics, const float* colors,
                    const float* opacities, float* splats, tgs_stream_t stream);
int tgs_unpack_splat_grads(uint64_t n, const float* splat_grads, float* v_means2d,
                           float* v_conics, float* v_colors, float* v_opacities,
                           tgs_stream_t stream);
/* Per touched row: projection + SH + activation backward over its visits in
 * camera order (the set bits of masks[row]); the render projection (near, far,
 * radius_clip as in tgs_tide_project_fwd) is recomputed per visit.  Writes the
 * compact gradient row grads[t * grad_stride + 0..58] once, and zeros in the
 * padding columns 59..grad_stride-1. */
int tgs_tide_project_bwd(uint32_t n_touched, const int32_t* touched, const int32_t* visit_base,
                         const int32_t* visits, const uint32_t* masks, uint32_t C,
                         const float* params, uint32_t row_stride, const float* viewmats,
                         const float* Ks, const float* campos, int32_t W, int32_t H, float eps2d,
                         float near_plane, float far_plane, float radius_clip, int32_t sh_degree,
                         const float* splat_grads, float* grads, uint32_t grad_stride,
                         tgs_stream_t stream);
/* tgs_tide_project_bwd and the resident optimizer update of the same rows in
 * one launch (TideGS runs them as two stages: engine.py:2434-2469 gradient
 * scatter, then gpu_resident_optimizer.py:16-70 / runtime.py:1741-1791 the
 * update): the gradient rows never reach memory.  Each row's 59 gradients
 * get tgs_resident_adam_step's update (optimizer 0; bias_correction1 and
 * denom_scale per slot) or tgs_resident_sophia_step's (optimizer 1, with rho
 * and update_hessian) against the moment tables exp_avg / exp_avg_sq
 * [slots * block_size, state_pitch], slot lookup through the block layout
 * (block_starts/ends/slots, n_layout) as in those entry points.  lrs[6] are
 * the learning rates of the CACHE column groups (xyz, log-scale, quat,
 * opacity, SH dc, SH rest).  params (row pitch row_stride <= 64) is read and
 * updated in place.  The touched rows must be unique and ascending (as
 * tgs_tide_compact writes them); a row outside every resident block keeps
 * its values and sets *error_flag.  block_size <= 2^22. */
int tgs_tide_project_bwd_update(
    uint32_t n_touched, const int32_t* touched, const int32_t* visit_base, const int32_t* visits,
    const uint32_t* masks, uint32_t C, float* params, uint32_t row_stride, const float* viewmats,
    const float* Ks, const float* campos, int32_t W, int32_t H, float eps2d, float near_plane,
    float far_plane, float radius_clip, int32_t sh_degree, const float* splat_grads,
    const int64_t* block_starts, const int64_t* block_ends, const int64_t* block_slots,
    int64_t n_layout, int64_t block_size, const float* bias_correction1, const float* denom_scale,
    float* exp_avg, float* exp_avg_sq, uint32_t state_pitch, const float* lrs, int32_t optimizer,
    float beta1, float beta2, float eps, float batch_size, float rho, int32_t update_hessian,
    int32_t* error_flag, tgs_stream_t stream);

/* ---- resident-set materialization and writeback ------------------------- */
/* The working set is one fp32 table in CACHE column order with row pitch 59
 * (dense) or 64 (padded; padding columns are written as zeros) plus an int64
 * global id per row, instead of the six component tensors of TideGS's
 * GPUBuffer (strategies/tide_engine/double_buffer_gpu.py:258-311).  Source
 * and destination ranges must not overlap.  Block segments follow the
 * reference's row rule: row r of a num_rows range lies in segment
 * r / block_rows at offset r % block_rows (only the last segment may be
 * partial). */
/* Copy kept blocks between two tables, ids included (replaces
 * _copy_resident_rows_kernel, double_buffer_gpu.py:41-128, launched by
 * _copy_resident_blocks :811-872): dst[dst_starts[s] + i] =
 * src[src_starts[s] + i] for segment s; src_gids/dst_gids both null or both
 * set.  n_blocks = length of the starts arrays. */
int tgs_ws_copy_rows(const float* src, uint32_t src_pitch, const int64_t* src_gids,
                     const int64_t* src_starts, const int64_t* dst_starts, uint32_t n_blocks,
                     int64_t num_rows, uint32_t block_rows, float* dst, uint32_t dst_pitch,
                     int64_t* dst_gids, tgs_stream_t stream);
/* Cold-block ids (replaces _fill_cold_global_ids_kernel,
 * double_buffer_gpu.py:130-149, :928-963): dst_gids[target_offset + r] =
 * block_ids[r / block_rows] * block_rows + r % block_rows. */
int tgs_ws_fill_global_ids(const int64_t* block_ids, uint32_t n_blocks, int64_t* dst_gids,
                           int64_t target_offset, int64_t num_rows, uint32_t block_rows,
                           tgs_stream_t stream);
/* Unpack streamed rows (replaces _unpack_streamed_rows_kernel,
 * double_buffer_gpu.py:151-210, launched at :1060-1082): packed [num_rows,59]
 * in CACHE (source_layout 0) or UNIFIED (1: xyz|opacity|scaling|rotation|dc|
 * rest, :714-735) order -> dst rows target_offset.. in CACHE order.  With
 * block_ids and dst_gids set, the cold-id fill above is done in the same pass. */
int tgs_ws_unpack_rows(const float* packed, int source_layout, int64_t num_rows, float* dst,
                       uint32_t dst_pitch, int64_t target_offset, const int64_t* block_ids,
                       uint32_t n_blocks, uint32_t block_rows, int64_t* dst_gids,
                       tgs_stream_t stream);
/* Pack dirty rows for writeback (replaces _pack_resident_rows_kernel,
 * strategies/tide_engine/gpu_working_set.py:33-87, launched by
 * stage_updated_blocks :895-988): out[(out_starts[b] + i) * 59 + c] =
 * src[src_starts[b] + i][c] for i < min(row_counts[b], block_rows). */
int tgs_ws_pack_rows(const float* src, uint32_t src_pitch, const int64_t* src_starts,
                     const int64_t* row_counts, const int64_t* out_starts, uint32_t n_blocks,
                     uint32_t block_rows, float* out, tgs_stream_t stream);
/* Per-block xyz bounds (replaces _resident_block_bounds_kernel,
 * gpu_working_set.py:89-116, launched by stage_block_bounds :990-1062):
 * bounds[b] = {min x,y,z, max x,y,z} over rows starts[b] ..
 * starts[b] + min(lengths[b], block_rows) of a table whose xyz are columns
 * 0..2 (pitch 3 = a bare xyz array, 59 or 64); an empty block gives
 * {1e20 x3, -1e20 x3}. */
int tgs_ws_block_bounds(const float* table, uint32_t pitch, const int64_t* starts,
                        const int64_t* lengths, uint32_t n_blocks, uint32_t block_rows,
                        float* bounds, tgs_stream_t stream);
/* Compact block-start table (replaces _build_block_starts,
 * double_buffer_gpu.py:212-233): block_starts[num_blocks] = -1, then
 * block_starts[block_ids[i]] = local_starts[i] for ids in range. */
int tgs_ws_build_block_starts(const int64_t* block_ids, const int64_t* local_starts,
                              uint32_t n_loaded, int64_t* block_starts, uint32_t num_blocks,
                              tgs_stream_t stream);
/* Global -> working-set-local ids (replaces _global_ids_to_local,
 * double_buffer_gpu.py:236-255): floor(g / block_size) selects the block;
 * ids whose block is out of range or not loaded give -1. */
int tgs_ws_global_to_local(const int64_t* global_ids, uint64_t n, const int64_t* block_starts,
                           uint32_t num_blocks, uint32_t block_size, int64_t* local_ids,
                           tgs_stream_t stream);

/* ---- Morton-sorted base file (streaming initializer) ---------------------- */
/* Replace the CPU passes of streaming_ply_to_ssd_base
 * (storage/streaming_ply_init.py:541-696) for a scene held in HBM; the
 * rows come out in the stable Morton order the reference's bucketed
 * external sort produces (:257-538), with the same per-bucket log-scales.
 * xyz [n,3] fp32.  scene bounds -> bounds[6] = {min x,y,z, max x,y,z}
 * (scratch: 6 u32). */
int tgs_init_scene_bounds(const float* xyz, uint64_t n, uint32_t* scratch, float* bounds,
                          tgs_stream_t stream);
/* 30-bit Morton codes (streaming_ply_init.py:154-168) against bounds[6]. */
int tgs_init_morton_codes(const float* xyz, uint64_t n, const float* bounds, uint32_t* codes,
                          tgs_stream_t stream);
/* Bucket sizes of the top 10 (counts0 [1024]) and top 20 (counts1 [1<<20])
 * code bits; both are zeroed first. */
int tgs_init_prefix_counts(const uint32_t* codes, uint64_t n, uint32_t* counts0,
                           uint32_t* counts1, tgs_stream_t stream);
/* flags[i] = 1 where sorted row i starts a new sorted bucket ("leaf"): the
 * 10-bit bucket unless big0[bucket] (it exceeds the sort memory, :332-350),
 * then the 20-bit child unless big1[child], else the whole code (:469-538). */
int tgs_init_leaf_flags(const uint32_t* sorted_codes, uint64_t n, const uint8_t* big0,
                        const uint8_t* big1, int32_t* flags, tgs_stream_t stream);
/* Per leaf (leaf_incl = inclusive scan of the flags, perm = sorted vertex
 * ids): stats[leaf*8 + 0..2] = min xyz, 3..5 = max xyz (fp32 bits), 6 = rows,
 * 7 = the leaf's first code. */
int tgs_init_leaf_stats(const int64_t* leaf_incl, const uint32_t* sorted_codes,
                        const uint32_t* perm, const float* xyz, uint64_t n, uint64_t n_leaves,
                        uint32_t* stats, tgs_stream_t stream);
/* Base-file rows [n,59] in sorted order (:234-248 with the leaf log-scale of
 * :361-367): xyz | leaf_scales[leaf] x3 | 1,0,0,0 | opacity_logit | dc | 0 x45. */
int tgs_init_pack_rows(const uint32_t* perm, const int64_t* leaf_incl, const float* xyz,
                       const float* dc, const float* leaf_scales, float opacity_logit, uint64_t n,
                       float* table, tgs_stream_t stream);

/* ---- block frustum culling --------------------------------------------- */
/* Bounding spheres of blocks (storage/gaussian_block.py:285-296, :322-325):
 * bounds [nb,6] (min xyz, max xyz) -> centers [nb,3] = (min+max)/2,
 * radii [nb] = (|max-min| / 2) * 1.15, in the reference's float32 order. */
int tgs_cull_block_spheres(const float* bounds, uint32_t nb, float* centers, float* radii,
                           tgs_stream_t stream);
/* 6-plane test of FrustumCuller.cull / cull_subset (gaussian_block.py:356-449)
 * for C <= 32 cameras at once: planes [C,6,4] normalized (A,B,C,D);
 * masks[i] bit c = every signed distance of block (block_ids ? block_ids[i] :
 * i) to camera c's planes is >= -radius; n entries. */
int tgs_cull_blocks(const float* centers, const float* radii, const int64_t* block_ids,
                    uint32_t n, const float* planes, uint32_t C, uint32_t* masks,
                    tgs_stream_t stream);
/* Legacy cone + distance test of FrustumCuller.cull(use_6plane=False)
 * (gaussian_block.py:465-510): visible[i] = |centers[i] - cam| <= threshold
 * and (cosine between (centers[i] - cam) and the unit forward axis > -0.3 or
 * distance < 1e-6); float64 arithmetic.  The caller passes the normalized
 * forward axis (view row 2) and threshold = min(scene_radius / 2, 100) *
 * margin (50 * margin without a scene radius), as the reference computes
 * them. */
int tgs_cull_blocks_cone(const float* centers, uint32_t nb, double cam_x, double cam_y,
                         double cam_z, double fwd_x, double fwd_y, double fwd_z,
                         double threshold, uint8_t* visible, tgs_stream_t stream);

/* ---- on-disk block store (host code, no GPU) ------------------------------ */
/* Parallel reads of n blocks of the base/patch files (replaces the per-block
 * f.seek + f.read + torch.cat of storage/log_storage_manager.py:208-291 and
 * storage/block_reader.py:55-87): block i is nbytes[i] bytes at
 * file_offsets[i] of the open descriptor fds[i], read into HOST memory at
 * (char*)dst + dst_offsets[i] (normally pinned staging) by up to n_threads
 * threads.  A block that ends
 * past its file's end is an error (TGS_ERR_ARG); a failed pread returns its
 * errno. */
int tgs_io_read_blocks(uint32_t n, const int32_t* fds, const int64_t* file_offsets,
                       const int64_t* nbytes, void* dst, const int64_t* dst_offsets,
                       uint32_t n_threads);

#ifdef __cplusplus
}
#endif

#endif /* TIDEGS_AMD_H */
