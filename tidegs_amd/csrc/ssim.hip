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
// so dL/dSSIM-map is the constant -lambda/N and the forward and backward run
// in one streaming pass:
//   stats    mu, sigma (separable 11-tap window) giving SSIM and
//            g dm/dmu1, g dm/dsigma1^2, g dm/dsigma12 (zero off the image);
//   gradient G * (g dm): f0 + 2 x f1 + y f2, plus the L1 term.
// sums[2b] += sum|I-gt'|, sums[2b+1] += sum SSIM (double, caller-zeroed).
//
// One wavefront per (image, channel, strip of 44 output columns, band of
// LR_BAND output rows); lane L holds column x0 - 10 + L, so the strip's
// 64 columns cover the outputs and the 10-column halo on each side.  The
// wavefront walks the band's input rows top to bottom (LR_BAND + 20 of them:
// 10 rows of halo above and below) and keeps each stage's last 11 rows in
// registers, so no row is filtered twice:
//   input row r:   x, y into an 11-row LDS ring; horizontal window sums of
//                  x, y, x^2, y^2, xy at the lane's column -> register ring H;
//   stats row r-5: vertical window over H -> SSIM and the scaled partial maps
//                  (zero off the image), through LDS to the lanes' neighbours;
//                  horizontal window of the maps -> register ring Q;
//   output r-10:   vertical window over Q, plus the L1 term -> dL/dI.
// The three channel wavefronts of a strip and band share one workgroup (the
// HWC image rows they read and write are the same lines).  The step loop is
// unrolled by the ring length, so every ring index is a constant.
#define LR_OUT 44                 // output columns per strip
#define LR_BAND 123               // output rows per band (LR_BAND + 20 = 13 x 11)
#define LR_ROWS (LR_BAND + 4 * SS_R)
#define LR_RING 11
static_assert(LR_ROWS % LR_RING == 0, "band rows must fill whole ring periods");

__device__ __forceinline__ void lr_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ void __launch_bounds__(192) tide_loss_rows_kernel(int H, int W,
                                                             const float* __restrict__ images_hwc,
                                                             const float* __restrict__ gt_chw,
                                                             float gt_div, float C1, float C2,
                                                             float g_ssim, float g_l1,
                                                             float* __restrict__ v_images_hwc,
                                                             double* __restrict__ sums) {
  // per channel wavefront: ring of (x, y) rows and one row of scaled partial
  // maps, each padded by the window radius on both sides
  __shared__ float2 s_xy[3][LR_RING][64 + 2 * SS_R];
  __shared__ float4 s_dm[3][64 + 2 * SS_R];
  const int c = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int b = blockIdx.z;
  const int x0 = blockIdx.x * LR_OUT, y0 = blockIdx.y * LR_BAND;
  const int xi = x0 - 2 * SS_R + lane;
  const bool col_in = xi >= 0 && xi < W;
  const bool col_out = col_in && lane >= 2 * SS_R && lane < 2 * SS_R + LR_OUT;
  const int HW = H * W;
  const float* img = images_hwc + (int64_t)b * HW * 3 + c;
  const float* gtc = gt_chw + ((int64_t)b * 3 + c) * HW;
  float* vimg = v_images_hwc + (int64_t)b * HW * 3 + c;
  const float rdiv = 1.f / gt_div;
  float2(*xy)[64 + 2 * SS_R] = s_xy[c];
  float4* dm = s_dm[c];
  if (lane < 2 * SS_R) {
    const int e = lane < SS_R ? lane : 64 + lane;  // pads 0..4 and 69..73
#pragma unroll
    for (int k = 0; k < LR_RING; ++k) xy[k][e] = make_float2(0.f, 0.f);
    dm[e] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // raw image and target values of input row r at the lane's column, loaded
  // from clamped (always valid) addresses without a branch, so that a fixed
  // number of loads is in flight and the two-row prefetch really overlaps
  const int xc = min(max(xi, 0), W - 1);
  auto load_row = [&](int r, float& u, float& g) {
    const int pix = min(max(r, 0), H - 1) * W + xc;
    u = img[pix * 3];
    g = gtc[pix];
  };
  // the window's distinct weights (the taps mirror about the centre) in
  // VGPRs, so that every window product takes two VGPR sources (forms that
  // issue in pairs on gfx950)
  float wt[6];
#pragma unroll
  for (int t = 0; t < 6; ++t) asm volatile("v_mov_b32 %0, %1" : "=v"(wt[t]) : "s"(c_gauss[t]));
  auto wgt = [&](int t) { return wt[t < 6 ? t : 10 - t]; };

  float Hr[5][LR_RING];  // horizontal sums of the last 11 input rows
  float Qr[3][LR_RING];  // horizontal sums of the partial maps, last 11 stats rows
#pragma unroll
  for (int k = 0; k < 5; ++k)
#pragma unroll
    for (int t = 0; t < LR_RING; ++t) Hr[k][t] = 0.f;
#pragma unroll
  for (int k = 0; k < 3; ++k)
#pragma unroll
    for (int t = 0; t < LR_RING; ++t) Qr[k][t] = 0.f;
  const int ys = y0 - 2 * SS_R;  // first input row
  float u1, g1, u2, g2;          // raw inputs of the next two rows
  load_row(ys, u1, g1);
  load_row(ys + 1, u2, g2);
  float l1_acc = 0.f, m_acc = 0.f;

#pragma unroll 1
  for (int n0 = 0; n0 < LR_ROWS; n0 += LR_RING) {
#pragma unroll
    for (int p = 0; p < LR_RING; ++p) {
      const int n = n0 + p;
      const int ri = ys + n;
      // x and clamp(gt / gt_div, 0, 1) of row ri (zero off the image); the
      // division is rounded like a division: product plus one residual correction
      const bool ok = col_in && ri >= 0 && ri < H;
      float q = g1 * rdiv;
      q = fmaf(fmaf(-q, gt_div, g1), rdiv, q);
      const float u = ok ? u1 : 0.f, w = ok ? fminf(fmaxf(q, 0.f), 1.f) : 0.f;
      u1 = u2;
      g1 = g2;
      load_row(ri + 2, u2, g2);
      // input row ri: ring slot p
      xy[p][lane + SS_R] = make_float2(u, w);
      lr_wave_sync();
      {
        float wx[11], wy[11], xv[11], yv[11];
#pragma unroll
        for (int t = 0; t < 11; ++t) {
          const float2 v = xy[p][lane + t];
          xv[t] = v.x;
          yv[t] = v.y;
          wx[t] = wgt(t) * v.x;
          wy[t] = wgt(t) * v.y;
        }
        float h0 = wx[0], h1 = wy[0], h2 = wx[0] * xv[0], h3 = wy[0] * yv[0],
              h4 = wx[0] * yv[0];
#pragma unroll
        for (int t = 1; t < 11; ++t) {
          h0 += wx[t];
          h1 += wy[t];
          h2 = fmaf(wx[t], xv[t], h2);
          h3 = fmaf(wy[t], yv[t], h3);
          h4 = fmaf(wx[t], yv[t], h4);
        }
        Hr[0][p] = h0;
        Hr[1][p] = h1;
        Hr[2][p] = h2;
        Hr[3][p] = h3;
        Hr[4][p] = h4;
      }
      if (n >= 2 * SS_R) {
        // stats row rs = ri - 5 from input rows ri - 10 .. ri (slots p+1 .. p+11)
        const int rs = ri - SS_R;
        float f[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) {
          float acc = wgt(0) * Hr[k][(p + 1) % LR_RING];
#pragma unroll
          for (int t = 1; t < 11; ++t) acc = fmaf(wgt(t), Hr[k][(p + 1 + t) % LR_RING], acc);
          f[k] = acc;
        }
        const float mu1 = f[0], mu2 = f[1];
        const float sigma1_sq = f[2] - mu1 * mu1;
        const float sigma2_sq = f[3] - mu2 * mu2;
        const float sigma12 = f[4] - mu1 * mu2;
        const float Cc = 2.f * mu1 * mu2 + C1;
        const float D = 2.f * sigma12 + C2;
        const float A = mu1 * mu1 + mu2 * mu2 + C1;
        const float Bb = sigma1_sq + sigma2_sq + C2;
        float d0 = 0.f, d1 = 0.f, d2 = 0.f;
        if (col_in && rs >= 0 && rs < H) {
          // the partial maps of clm_kernels/ssim.cu:240-262 from two
          // reciprocals; A >= C1 and Bb >= C2 - (rounding) > 0, so the
          // hardware reciprocal (within 1 ulp) is safe here
          const float rA = __builtin_amdgcn_rcpf(A), rB = __builtin_amdgcn_rcpf(Bb);
          const float rAB = rA * rB;
          const float CD = Cc * D;
          d0 = 2.f * rAB * (mu2 * D - mu2 * Cc + mu1 * CD * (rB - rA));
          d1 = -CD * rAB * rB;
          d2 = 2.f * Cc * rAB;
          if (col_out && rs >= y0 && rs < y0 + LR_BAND) m_acc += CD * rAB;
        }
        dm[lane + SS_R] = make_float4(g_ssim * d0, g_ssim * d1, g_ssim * d2, 0.f);
        lr_wave_sync();
        float q0 = 0.f, q1 = 0.f, q2 = 0.f;
#pragma unroll
        for (int t = 0; t < 11; ++t) {
          const float4 v = dm[lane + t];
          q0 = fmaf(wgt(t), v.x, q0);
          q1 = fmaf(wgt(t), v.y, q1);
          q2 = fmaf(wgt(t), v.z, q2);
        }
        Qr[0][p] = q0;
        Qr[1][p] = q1;
        Qr[2][p] = q2;
      }
      if (n >= 4 * SS_R) {
        // output row ro = ri - 10 from stats rows ro - 5 .. ro + 5 (slots p+1 .. p+11)
        const int ro = ri - 2 * SS_R;
        float g3[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          float acc = wgt(0) * Qr[k][(p + 1) % LR_RING];
#pragma unroll
          for (int t = 1; t < 11; ++t) acc = fmaf(wgt(t), Qr[k][(p + 1 + t) % LR_RING], acc);
          g3[k] = acc;
        }
        if (col_out && ro < H) {
          const float2 v = xy[(p + 1) % LR_RING][lane + SS_R];  // x, y of row ro
          const float d = v.x - v.y;
          l1_acc += fabsf(d);
          vimg[(ro * W + xi) * 3] = g3[0] + 2.f * v.x * g3[1] + v.y * g3[2] +
                                    (d > 0.f ? g_l1 : (d < 0.f ? -g_l1 : 0.f));
        }
      }
      // every lane has read this step's rows before the next step writes
      lr_wave_sync();
    }
  }
  const float l1 = tgs_wave_sum(l1_acc);
  const float ms = tgs_wave_sum(m_acc);
  if (lane == 0) {
    atomicAdd(&sums[2 * b + 0], (double)l1);
    atomicAdd(&sums[2 * b + 1], (double)ms);
  }
}

extern "C" int tgs_tide_loss(int32_t B, int32_t H, int32_t W, const float* images_hwc,
                             const float* gt_chw, float gt_div, float lambda_dssim, double* sums,
                             float* v_images_hwc, hipStream_t stream) {
  if ((int64_t)B * H * W == 0) return TGS_OK;
  TGS_CHECK_ARG(images_hwc && gt_chw && sums && v_images_hwc, "tide_loss: null pointer");
  TGS_CHECK_ARG((int64_t)H * W * 3 < (1ll << 31), "tide_loss: image too large");
  const float inv_n = 1.f / (float)((int64_t)3 * H * W);
  TGS_CHECK_ARG(B <= 65535, "tide_loss: more than 65535 images");
  dim3 grid((W + LR_OUT - 1) / LR_OUT, (H + LR_BAND - 1) / LR_BAND, B);
  hipLaunchKernelGGL(tide_loss_rows_kernel, grid, dim3(192), 0, stream, H, W, images_hwc, gt_chw,
                     gt_div,
                     1e-4f, 9e-4f, -lambda_dssim * inv_n, (1.f - lambda_dssim) * inv_n,
                     v_images_hwc, sums);
  TGS_RETURN_LAUNCH("tgs_tide_loss");
}
