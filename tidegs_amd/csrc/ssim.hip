// Fused 11x11 Gaussian-window SSIM (sigma 1.5, zero padding, "same" output)
// forward with the three partial-derivative maps, and its backward.
//
// Reference: clm_kernels/ssim.cu:187-286 (fusedssimCUDA), :288-366
// (fusedssim_backwardCUDA), clm_kernels/__init__.py:23-61 (autograd wrapper;
// C1 = 0.01^2, C2 = 0.03^2).  Per pixel and channel:
//   mu = G*x, sigma_xx = G*(x^2) - mu^2, sigma_xy = G*(xy) - mu1 mu2
//   C = 2 mu1 mu2 + C1, D = 2 sigma12 + C2, A = mu1^2 + mu2^2 + C1,
//   B = sigma1^2 + sigma2^2 + C2, m = C D / (A B)
//   dm/dmu1, dm/dsigma1^2 (= -C D / (A B^2)), dm/dsigma12 (= 2 C / (A B))
// Backward: dL/dx = G*(g dm/dmu1) + 2 x G*(g dm/dsigma1^2) + y G*(g dm/dsigma12).
//
// Layout is given by strides (channel, row, column) so one kernel serves NCHW
// tensors (drop-in fused_ssim) and the HWC rendered image of the fused step.
// A 16x16 output tile per 256-thread workgroup with a 26x26 halo in LDS;
// separable passes in the same order as the reference (x first, then y).
// The fused-step mode also folds in the L1 term and the clamp(gt/255, 0, 1)
// target normalisation of strategies/base_engine.py:472-488.
#include "tgs_common.cuh"

#define SS_T 16
#define SS_R 5
#define SS_H (SS_T + 2 * SS_R)  // 26

// Normalised Gaussian window, w_i = exp(-(i-5)^2 / 4.5) / sum_j exp(-(j-5)^2 / 4.5).
__constant__ float c_gauss[11] = {
    0.001028380123898387f, 0.0075987582094967365f, 0.036000773310661316f,
    0.10936068743467331f,  0.21300552785396576f,   0.26601171493530273f,
    0.21300552785396576f,  0.10936068743467331f,   0.036000773310661316f,
    0.0075987582094967365f, 0.001028380123898387f};

struct Img {
  const float* p;
  int64_t bs, cs, ys, xs;  // batch, channel, row, column strides (elements)
  float div;               // value = clamp?(p / div)
  int clamp01;
  __device__ __forceinline__ float at(int b, int c, int y, int x, int H, int W) const {
    if (x < 0 || y < 0 || x >= W || y >= H) return 0.f;
    float v = p[b * bs + c * cs + (int64_t)y * ys + (int64_t)x * xs] / div;
    if (clamp01) v = fminf(fmaxf(v, 0.f), 1.f);
    return v;
  }
};

struct OutImg {
  float* p;
  int64_t bs, cs, ys, xs;
  __device__ __forceinline__ float& at(int b, int c, int y, int x) const {
    return p[b * bs + c * cs + (int64_t)y * ys + (int64_t)x * xs];
  }
};

// Horizontal pass over the 26 halo rows for the 16 output columns, then the
// vertical pass for this thread's output pixel.  `q` computes the quantity to
// filter from the two halo tiles.
template <int NQ, class Q>
__device__ __forceinline__ void sep_conv(float (*h)[SS_H][SS_T], Q q, float out[NQ]) {
  const int tid = threadIdx.x;
  for (int e = tid; e < SS_H * SS_T; e += 256) {
    const int r = e / SS_T, c = e % SS_T;
    float acc[NQ];
#pragma unroll
    for (int k = 0; k < NQ; ++k) acc[k] = 0.f;
#pragma unroll
    for (int t = 0; t < 11; ++t) {
      float v[NQ];
      q(r, c + t, v);
#pragma unroll
      for (int k = 0; k < NQ; ++k) acc[k] += c_gauss[t] * v[k];
    }
#pragma unroll
    for (int k = 0; k < NQ; ++k) h[k][r][c] = acc[k];
  }
  __syncthreads();
  const int ty = tid / SS_T, tx = tid % SS_T;
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < 11; ++t) acc += c_gauss[t] * h[k][ty + t][tx];
    out[k] = acc;
  }
}

__global__ void __launch_bounds__(256) ssim_fwd_kernel(int B, int CH, int H, int W, float C1,
                                                       float C2, Img a, Img b, OutImg map,
                                                       OutImg d_mu1, OutImg d_s11, OutImg d_s12,
                                                       double* __restrict__ sums) {
  __shared__ float s1[SS_H][SS_H];
  __shared__ float s2[SS_H][SS_H];
  __shared__ float h[5][SS_H][SS_T];
  __shared__ float red[2][4];
  const int bidx = blockIdx.z;
  const int x0 = blockIdx.x * SS_T, y0 = blockIdx.y * SS_T;
  const int tid = threadIdx.x;
  const int ty = tid / SS_T, tx = tid % SS_T;
  const int px = x0 + tx, py = y0 + ty;
  const bool inside = px < W && py < H;
  float l1_acc = 0.f, m_acc = 0.f;

  for (int c = 0; c < CH; ++c) {
    __syncthreads();
    for (int e = tid; e < SS_H * SS_H; e += 256) {
      const int r = e / SS_H, col = e % SS_H;
      s1[r][col] = a.at(bidx, c, y0 + r - SS_R, x0 + col - SS_R, H, W);
      s2[r][col] = b.at(bidx, c, y0 + r - SS_R, x0 + col - SS_R, H, W);
    }
    __syncthreads();
    float f[5];
    sep_conv<5>(h, [&](int r, int col, float v[5]) {
      const float u = s1[r][col], w = s2[r][col];
      v[0] = u;
      v[1] = w;
      v[2] = u * u;
      v[3] = w * w;
      v[4] = u * w;
    }, f);
    const float mu1 = f[0], mu2 = f[1];
    const float sigma1_sq = f[2] - mu1 * mu1;
    const float sigma2_sq = f[3] - mu2 * mu2;
    const float sigma12 = f[4] - mu1 * mu2;
    const float Cc = 2.f * mu1 * mu2 + C1;
    const float D = 2.f * sigma12 + C2;
    const float A = mu1 * mu1 + mu2 * mu2 + C1;
    const float Bb = sigma1_sq + sigma2_sq + C2;
    const float m = (Cc * D) / (A * Bb);
    if (inside) {
      if (map.p) map.at(bidx, c, py, px) = m;
      if (d_mu1.p) {
        d_mu1.at(bidx, c, py, px) = (mu2 * 2.f * D) / (A * Bb) - (mu2 * 2.f * Cc) / (A * Bb) -
                                    (mu1 * 2.f * Cc * D) / (A * A * Bb) +
                                    (mu1 * 2.f * Cc * D) / (A * Bb * Bb);
        d_s11.at(bidx, c, py, px) = (-Cc * D) / (A * Bb * Bb);
        d_s12.at(bidx, c, py, px) = (2.f * Cc) / (A * Bb);
      }
      if (sums) {
        l1_acc += fabsf(s1[ty + SS_R][tx + SS_R] - s2[ty + SS_R][tx + SS_R]);
        m_acc += m;
      }
    }
  }
  if (sums) {
    const float l1 = tgs_wave_sum(l1_acc);
    const float ms = tgs_wave_sum(m_acc);
    const int lane = tid & 63, wave = tid >> 6;
    if (lane == 0) {
      red[0][wave] = l1;
      red[1][wave] = ms;
    }
    __syncthreads();
    if (tid == 0) {
      atomicAdd(&sums[2 * bidx + 0], (double)(red[0][0] + red[0][1] + red[0][2] + red[0][3]));
      atomicAdd(&sums[2 * bidx + 1], (double)(red[1][0] + red[1][1] + red[1][2] + red[1][3]));
    }
  }
}

// dL/dimg1.  dmap == null means dL/dmap is the constant `dmap_const` (the
// fused step's mean-SSIM loss).  When l1_weight != 0 the L1 term
// l1_weight * sign(x - y) is added (sign(0) = 0, as torch's abs backward).
__global__ void __launch_bounds__(256) ssim_bwd_kernel(int B, int CH, int H, int W, Img a, Img b,
                                                       Img dmap, float dmap_const, Img d_mu1,
                                                       Img d_s11, Img d_s12, float l1_weight,
                                                       OutImg out) {
  __shared__ float s[3][SS_H][SS_H];
  __shared__ float h[3][SS_H][SS_T];
  const int bidx = blockIdx.z;
  const int x0 = blockIdx.x * SS_T, y0 = blockIdx.y * SS_T;
  const int tid = threadIdx.x;
  const int ty = tid / SS_T, tx = tid % SS_T;
  const int px = x0 + tx, py = y0 + ty;
  const bool inside = px < W && py < H;
  for (int c = 0; c < CH; ++c) {
    __syncthreads();
    for (int e = tid; e < SS_H * SS_H; e += 256) {
      const int r = e / SS_H, col = e % SS_H;
      const int yy = y0 + r - SS_R, xx = x0 + col - SS_R;
      const bool in_img = xx >= 0 && yy >= 0 && xx < W && yy < H;
      const float g = dmap.p ? dmap.at(bidx, c, yy, xx, H, W) : (in_img ? dmap_const : 0.f);
      s[0][r][col] = g * d_mu1.at(bidx, c, yy, xx, H, W);
      s[1][r][col] = g * d_s11.at(bidx, c, yy, xx, H, W);
      s[2][r][col] = g * d_s12.at(bidx, c, yy, xx, H, W);
    }
    __syncthreads();
    float f[3];
    sep_conv<3>(h, [&](int r, int col, float v[3]) {
      v[0] = s[0][r][col];
      v[1] = s[1][r][col];
      v[2] = s[2][r][col];
    }, f);
    if (inside) {
      const float x = a.at(bidx, c, py, px, H, W);
      const float y = b.at(bidx, c, py, px, H, W);
      float gr = f[0] + 2.f * x * f[1] + y * f[2];
      if (l1_weight != 0.f) {
        const float d = x - y;
        gr += d > 0.f ? l1_weight : (d < 0.f ? -l1_weight : 0.f);
      }
      out.at(bidx, c, py, px) = gr;
    }
  }
}

static Img nchw(const float* p, int CH, int H, int W) {
  return Img{p, (int64_t)CH * H * W, (int64_t)H * W, W, 1, 1.f, 0};
}
static OutImg nchw_out(float* p, int CH, int H, int W) {
  return OutImg{p, (int64_t)CH * H * W, (int64_t)H * W, W, 1};
}

extern "C" int tgs_fused_ssim_fwd(int32_t B, int32_t CH, int32_t H, int32_t W, float C1, float C2,
                                  const float* img1, const float* img2, float* ssim_map,
                                  float* dm_dmu1, float* dm_dsigma1_sq, float* dm_dsigma12,
                                  hipStream_t stream) {
  if ((int64_t)B * CH * H * W == 0) return TGS_OK;
  TGS_CHECK_ARG(img1 && img2 && ssim_map, "fused_ssim_fwd: null pointer");
  TGS_CHECK_ARG((dm_dmu1 && dm_dsigma1_sq && dm_dsigma12) ||
                    (!dm_dmu1 && !dm_dsigma1_sq && !dm_dsigma12),
                "fused_ssim_fwd: partial maps must be all set or all null");
  dim3 grid((W + SS_T - 1) / SS_T, (H + SS_T - 1) / SS_T, B);
  hipLaunchKernelGGL(ssim_fwd_kernel, grid, dim3(256), 0, stream, B, CH, H, W, C1, C2,
                     nchw(img1, CH, H, W), nchw(img2, CH, H, W), nchw_out(ssim_map, CH, H, W),
                     nchw_out(dm_dmu1, CH, H, W), nchw_out(dm_dsigma1_sq, CH, H, W),
                     nchw_out(dm_dsigma12, CH, H, W), (double*)nullptr);
  TGS_RETURN_LAUNCH("tgs_fused_ssim_fwd");
}

extern "C" int tgs_fused_ssim_bwd(int32_t B, int32_t CH, int32_t H, int32_t W, float C1, float C2,
                                  const float* img1, const float* img2, const float* dL_dmap,
                                  const float* dm_dmu1, const float* dm_dsigma1_sq,
                                  const float* dm_dsigma12, float* dL_dimg1, hipStream_t stream) {
  (void)C1;
  (void)C2;
  if ((int64_t)B * CH * H * W == 0) return TGS_OK;
  TGS_CHECK_ARG(img1 && img2 && dL_dmap && dm_dmu1 && dm_dsigma1_sq && dm_dsigma12 && dL_dimg1,
                "fused_ssim_bwd: null pointer");
  dim3 grid((W + SS_T - 1) / SS_T, (H + SS_T - 1) / SS_T, B);
  hipLaunchKernelGGL(ssim_bwd_kernel, grid, dim3(256), 0, stream, B, CH, H, W,
                     nchw(img1, CH, H, W), nchw(img2, CH, H, W), nchw(dL_dmap, CH, H, W), 0.f,
                     nchw(dm_dmu1, CH, H, W), nchw(dm_dsigma1_sq, CH, H, W),
                     nchw(dm_dsigma12, CH, H, W), 0.f, nchw_out(dL_dimg1, CH, H, W));
  TGS_RETURN_LAUNCH("tgs_fused_ssim_bwd");
}

// Fused-step loss of strategies/base_engine.py:464-488 for a batch of B
// rendered images: per image b, L_b = (1-lambda) mean|I_b - gt'_b| +
// lambda (1 - mean SSIM(I_b, gt'_b)), gt' = clamp(gt / gt_div, 0, 1), with
// I [B,H,W,3] (HWC, as rendered) and gt [B,3,H,W] (CHW).  The loss is fixed,
// so dL/dSSIM-map is the constant -lambda/N and the whole forward + backward
// runs in one pass per 32x32 output tile and channel, keeping every
// intermediate in LDS:
//   inputs   x, y on the 52x52 region (tile + 2 x 5 halo each side);
//   stats    mu, sigma over the 42x42 region (separable 11-tap window),
//            giving SSIM (summed over the tile's own pixels) and
//            g dm/dmu1, g dm/dsigma1^2, g dm/dsigma12 (zero off the image);
//   gradient G * (g dm) on the tile: f0 + 2 x f1 + y f2, plus the L1 term.
// sums[2b] += sum|I-gt'|, sums[2b+1] += sum SSIM (double, caller-zeroed).
#define TL_T 32                   // output tile edge
#define TL_D1 (TL_T + 2 * SS_R)   // 42: dm region
#define TL_D2 (TL_T + 4 * SS_R)   // 52: input region
#define TL_THREADS (TL_T * TL_T)  // 1024
#define TL_IN_PITCH 53            // >= TL_D2, odd
#define TL_HQ_PITCH 53            // >= TL_D1, odd, 2 x 53 = 42 (mod 64)
#define TL_DM_PITCH 43            // >= TL_D1, odd
#define TL_H2_PITCH 49            // >= TL_T, odd

__global__ void __launch_bounds__(TL_THREADS, 8) tide_loss_kernel(int H, int W,
                                                               const float* __restrict__ images_hwc,
                                                               const float* __restrict__ gt_chw,
                                                               float gt_div, float C1, float C2,
                                                               float g_ssim, float g_l1,
                                                               float* __restrict__ v_images_hwc,
                                                               double* __restrict__ sums) {
  // phase-aliased LDS: inputs -> dm maps, horizontal sums -> backward sums.
  // The horizontal passes give consecutive lanes consecutive rows (odd row
  // pitches: distinct banks); the vertical passes give them consecutive
  // columns, and 2 x 53 = 42 (mod 64 banks) puts the forward vertical pass's
  // second group of lanes (two rows down) on the banks the first leaves free.
  __shared__ union {
    struct {
      float sx[TL_D2][TL_IN_PITCH];
      float sy[TL_D2][TL_IN_PITCH];
    } in;
    float sdm[3][TL_D1][TL_DM_PITCH];
  } su;
  __shared__ union {
    float hq[5][TL_D2][TL_HQ_PITCH];
    float h2[3][TL_D1][TL_H2_PITCH];
  } sv;
  __shared__ float red[2][TL_THREADS / 64];
  auto& sx = su.in.sx;
  auto& sy = su.in.sy;
  auto& sdm = su.sdm;
  auto& hq = sv.hq;
  auto& h2 = sv.h2;
  const int bidx = blockIdx.z;
  const int x0 = blockIdx.x * TL_T, y0 = blockIdx.y * TL_T;
  const int tid = threadIdx.x;
  // output pixels of thread tid < 512: rows 2 rb2 + {0, 1} of column tx2
  const int rb2 = (tid % (TL_T * TL_T / 2)) / TL_T, tx2 = tid % TL_T;
  const int px2 = x0 + tx2, py2 = y0 + 2 * rb2;
  const bool in2[2] = {px2 < W && py2 < H, px2 < W && py2 + 1 < H};
  const int HW = H * W;
  const float* img = images_hwc + (int64_t)bidx * HW * 3;
  const float* gtb = gt_chw + (int64_t)bidx * HW * 3;
  float* vimg = v_images_hwc + (int64_t)bidx * HW * 3;
  const float rdiv = 1.f / gt_div;
  float l1_acc = 0.f, m_acc = 0.f;

  for (int c = 0; c < 3; ++c) {
    const float* gtc = gtb + c * HW;
    __syncthreads();
    // inputs on the 52x52 region, consecutive threads on consecutive columns
    for (int o = tid; o < TL_D2 * TL_D2; o += TL_THREADS) {
      const int r = o / TL_D2, col = o - r * TL_D2;
      const int yy = y0 + r - 2 * SS_R;
      const int xx = x0 + col - 2 * SS_R;
      float u = 0.f, w = 0.f;
      if (xx >= 0 && yy >= 0 && xx < W && yy < H) {
        const int pix = yy * W + xx;
        u = img[pix * 3 + c];
        // gt / gt_div, rounded like the division: product plus one
        // residual correction
        const float g = gtc[pix];
        float q = g * rdiv;
        q = fmaf(fmaf(-q, gt_div, g), rdiv, q);
        w = fminf(fmaxf(q, 0.f), 1.f);
      }
      sx[r][col] = u;
      sy[r][col] = w;
    }
    __syncthreads();
    // threads below 512 keep the inputs of their two output pixels (rows
    // 2 rb2 and 2 rb2 + 1 of column tx2) for the gradient at the end
    float x_own[2] = {0.f, 0.f}, y_own[2] = {0.f, 0.f};
    if (tid < TL_T * TL_T / 2) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        x_own[j] = sx[2 * rb2 + j + 2 * SS_R][tx2 + 2 * SS_R];
        y_own[j] = sy[2 * rb2 + j + 2 * SS_R][tx2 + 2 * SS_R];
        if (in2[j]) l1_acc += fabsf(x_own[j] - y_own[j]);
      }
    }
    // horizontal pass of x, y, x^2, y^2, xy: 52 rows x 42 columns, three
    // consecutive columns per work item (13 inputs; each product formed once),
    // consecutive items on consecutive rows
    for (int o = tid; o < TL_D2 * (TL_D1 / 3); o += TL_THREADS) {
      const int cb = (o / TL_D2) * 3, r = o - (o / TL_D2) * TL_D2;
      float u[13], w[13];
#pragma unroll
      for (int t = 0; t < 13; ++t) {
        u[t] = sx[r][cb + t];
        w[t] = sy[r][cb + t];
      }
#pragma unroll
      for (int k = 0; k < 5; ++k) {
        float v[13];
#pragma unroll
        for (int t = 0; t < 13; ++t)
          v[t] = k == 0 ? u[t] : k == 1 ? w[t] : k == 2 ? u[t] * u[t] : k == 3 ? w[t] * w[t]
                                                                               : u[t] * w[t];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          float q = 0.f;
#pragma unroll
          for (int t = 0; t < 11; ++t) q += c_gauss[t] * v[j + t];
          hq[k][r][cb + j] = q;
        }
      }
    }
    __syncthreads();
    // vertical pass on the 42x42 region, two consecutive rows per work item:
    // SSIM and the scaled partial maps (the inputs are dead: the dm maps take
    // their place)
#pragma unroll 1
    for (int o = tid; o < (TL_D1 / 2) * TL_D1; o += TL_THREADS) {
      const int rq = o / TL_D1, col = o - rq * TL_D1;
      const int rb = 2 * rq;
      float f[2][5];
#pragma unroll
      for (int k = 0; k < 5; ++k) {
        float v[12];
#pragma unroll
        for (int t = 0; t < 12; ++t) v[t] = hq[k][rb + t][col];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float acc = 0.f;
#pragma unroll
          for (int t = 0; t < 11; ++t) acc += c_gauss[t] * v[j + t];
          f[j][k] = acc;
        }
        // one map at a time: its sums are complete before the next map's loads
        // (bounds the registers to 8 waves per SIMD)
        asm volatile("" : "+v"(f[0][k]), "+v"(f[1][k])::"memory");
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = rb + j;
        const float mu1 = f[j][0], mu2 = f[j][1];
        const float sigma1_sq = f[j][2] - mu1 * mu1;
        const float sigma2_sq = f[j][3] - mu2 * mu2;
        const float sigma12 = f[j][4] - mu1 * mu2;
        const float Cc = 2.f * mu1 * mu2 + C1;
        const float D = 2.f * sigma12 + C2;
        const float A = mu1 * mu1 + mu2 * mu2 + C1;
        const float Bb = sigma1_sq + sigma2_sq + C2;
        const int yy = y0 + r - SS_R, xx = x0 + col - SS_R;
        const bool in_img = xx >= 0 && yy >= 0 && xx < W && yy < H;
        float d0 = 0.f, d1 = 0.f, d2 = 0.f;
        if (in_img) {
          // the partial maps of clm_kernels/ssim.cu:240-262 from two
          // reciprocals; A >= C1 and Bb >= C2 - (rounding) > 0, so the
          // hardware reciprocal (within 1 ulp) is safe here
          const float rA = __builtin_amdgcn_rcpf(A), rB = __builtin_amdgcn_rcpf(Bb);
          const float rAB = rA * rB;
          const float CD = Cc * D;
          d0 = 2.f * rAB * (mu2 * D - mu2 * Cc + mu1 * CD * (rB - rA));
          d1 = -CD * rAB * rB;
          d2 = 2.f * Cc * rAB;
          if (r >= SS_R && r < SS_R + TL_T && col >= SS_R && col < SS_R + TL_T)
            m_acc += CD * rAB;
        }
        sdm[0][r][col] = g_ssim * d0;
        sdm[1][r][col] = g_ssim * d1;
        sdm[2][r][col] = g_ssim * d2;
      }
    }
    __syncthreads();
    // backward: horizontal pass (42 rows x 32 columns), two columns per item,
    // consecutive items on consecutive rows ...
    for (int o = tid; o < TL_D1 * (TL_T / 2); o += TL_THREADS) {
      const int cb = (o / TL_D1) * 2, r = o - (o / TL_D1) * TL_D1;
#pragma unroll
      for (int m = 0; m < 3; ++m) {
        float v[12];
#pragma unroll
        for (int t = 0; t < 12; ++t) v[t] = sdm[m][r][cb + t];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float q = 0.f;
#pragma unroll
          for (int t = 0; t < 11; ++t) q += c_gauss[t] * v[j + t];
          h2[m][r][cb + j] = q;
        }
      }
    }
    __syncthreads();
    // ... then vertical, two rows per item (threads below 512), and the
    // gradient of those pixels
    if (tid < TL_T * TL_T / 2) {
      float f[2][3];
#pragma unroll
      for (int m = 0; m < 3; ++m) {
        float v[12];
#pragma unroll
        for (int t = 0; t < 12; ++t) v[t] = h2[m][2 * rb2 + t][tx2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float q = 0.f;
#pragma unroll
          for (int t = 0; t < 11; ++t) q += c_gauss[t] * v[j + t];
          f[j][m] = q;
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (in2[j]) {
          const float d = x_own[j] - y_own[j];
          vimg[((py2 + j) * W + px2) * 3 + c] = f[j][0] + 2.f * x_own[j] * f[j][1] +
                                                y_own[j] * f[j][2] +
                                                (d > 0.f ? g_l1 : (d < 0.f ? -g_l1 : 0.f));
        }
      }
    }
  }
  const float l1 = tgs_wave_sum(l1_acc);
  const float ms = tgs_wave_sum(m_acc);
  const int lane = tid & 63, wave = tid >> 6;
  if (lane == 0) {
    red[0][wave] = l1;
    red[1][wave] = ms;
  }
  __syncthreads();
  if (tid == 0) {
    float a0 = 0.f, a1 = 0.f;
    for (int w = 0; w < TL_THREADS / 64; ++w) {
      a0 += red[0][w];
      a1 += red[1][w];
    }
    atomicAdd(&sums[2 * bidx + 0], (double)a0);
    atomicAdd(&sums[2 * bidx + 1], (double)a1);
  }
}

extern "C" int tgs_tide_loss(int32_t B, int32_t H, int32_t W, const float* images_hwc,
                             const float* gt_chw, float gt_div, float lambda_dssim, double* sums,
                             float* v_images_hwc, hipStream_t stream) {
  if ((int64_t)B * H * W == 0) return TGS_OK;
  TGS_CHECK_ARG(images_hwc && gt_chw && sums && v_images_hwc, "tide_loss: null pointer");
  TGS_CHECK_ARG((int64_t)H * W * 3 < (1ll << 31), "tide_loss: image too large");
  const float inv_n = 1.f / (float)((int64_t)3 * H * W);
  dim3 grid((W + TL_T - 1) / TL_T, (H + TL_T - 1) / TL_T, B);
  hipLaunchKernelGGL(tide_loss_kernel, grid, dim3(TL_THREADS), 0, stream, H, W, images_hwc, gt_chw,
                     gt_div,
                     1e-4f, 9e-4f, -lambda_dssim * inv_n, (1.f - lambda_dssim) * inv_n,
                     v_images_hwc, sums);
  TGS_RETURN_LAUNCH("tgs_tide_loss");
}
