// Real spherical-harmonics basis (degree <= 4) and its gradient, evaluated on a
// unit direction.  The basis is the Sloan (JCGT 2013) polynomial form with the
// Condon-Shortley phase folded into the real harmonics, index k = l*l + l + m,
// exactly as gsplat's SH path uses it (gsplat/cuda/csrc/spherical_harmonics.cuh:11-92).
//
// sh_foreach(degree, x, y, z, f) calls f(k, Y_k, dY_k/dx, dY_k/dy, dY_k/dz) for
// every basis function up to `degree`, treating (x,y,z) as independent
// coordinates.  Callers evaluate colors (sum_k Y_k c_k) and the VJP
// (v_c_k = Y_k v_color; v_dir_n = sum_k <c_k, v_color> grad Y_k) in one pass,
// which is one thread per Gaussian for all channels instead of one thread per
// (Gaussian, channel).
#pragma once

#include "tgs_common.cuh"

namespace tgs_sh {
// l = 0, 1
constexpr float C0 = 0.28209479177387814f;   // 1 / (2 sqrt(pi))
constexpr float C1 = 0.48860251190291992f;   // sqrt(3 / (4 pi))
// l = 2
constexpr float C2a = 1.0925484305920792f;   // sqrt(15 / pi) / 2
constexpr float C2b = 0.94617469575756008f;  // 3 sqrt(5 / pi) / 4   (z^2 term)
constexpr float C2c = 0.31539156525252005f;  // sqrt(5 / pi) / 4
constexpr float C2d = 0.54627421529603959f;  // sqrt(15 / pi) / 4
// l = 3
constexpr float C3a = 0.59004358992664352f;  // sqrt(35 / (2 pi)) / 4
constexpr float C3b = 1.4453057213202771f;   // sqrt(105 / pi) / 4   (x2 -> 2.89 xyz)
constexpr float C3c = 0.45704579946446577f;  // sqrt(21 / (2 pi)) / 4
constexpr float C3d = 0.37317633259011546f;  // sqrt(7 / pi) / 4
// l = 4 (Sloan's factored recurrences)
constexpr float C4a = 0.62583573544917614f;  // 3 sqrt(35 / pi) / 16
constexpr float C4b = 1.7701307697799304f;   // 3 sqrt(35 / (2 pi)) / 8
constexpr float C4c = 3.3116114351514600f;
constexpr float C4d = 0.47308734787878000f;
constexpr float C4e = 4.6833258049010249f;
constexpr float C4f = 2.0071396306718676f;
constexpr float C4g = 1.9843134832984430f;
constexpr float C4h = 1.0062305898749053f;
}  // namespace tgs_sh

template <class F>
__device__ __forceinline__ void sh_foreach(int degree, float x, float y, float z, F&& f) {
  using namespace tgs_sh;
  f(0, C0, 0.f, 0.f, 0.f);
  if (degree < 1) return;
  f(1, -C1 * y, 0.f, -C1, 0.f);
  f(2, C1 * z, 0.f, 0.f, C1);
  f(3, -C1 * x, -C1, 0.f, 0.f);
  if (degree < 2) return;
  const float xx = x * x, yy = y * y, zz = z * z;
  const float xy = x * y, yz = y * z, xz = x * z;
  f(4, C2a * xy, C2a * y, C2a * x, 0.f);
  f(5, -C2a * yz, 0.f, -C2a * z, -C2a * y);
  f(6, C2b * zz - C2c, 0.f, 0.f, 2.f * C2b * z);
  f(7, -C2a * xz, -C2a * z, 0.f, -C2a * x);
  f(8, C2d * (xx - yy), 2.f * C2d * x, -2.f * C2d * y, 0.f);
  if (degree < 3) return;
  // fC1 = x^2 - y^2, fS1 = 2xy, fC2 = x^3 - 3xy^2, fS2 = 3x^2y - y^3
  const float fC1 = xx - yy, fS1 = 2.f * xy;
  const float fC2 = x * fC1 - y * fS1, fS2 = x * fS1 + y * fC1;
  const float t0c = -5.f * C3c * zz + C3c;  // -C3c (5z^2 - 1)
  f(9, -C3a * fS2, -C3a * 6.f * xy, -C3a * 3.f * fC1, 0.f);
  f(10, 2.f * C3b * xy * z, 2.f * C3b * yz, 2.f * C3b * xz, 2.f * C3b * xy);
  f(11, t0c * y, 0.f, t0c, -10.f * C3c * yz);
  f(12, z * (5.f * C3d * zz - 3.f * C3d), 0.f, 0.f, 15.f * C3d * zz - 3.f * C3d);
  f(13, t0c * x, t0c, 0.f, -10.f * C3c * xz);
  f(14, C3b * z * fC1, 2.f * C3b * xz, -2.f * C3b * yz, C3b * fC1);
  f(15, -C3a * fC2, -C3a * 3.f * fC1, C3a * 6.f * xy, 0.f);
  if (degree < 4) return;
  // Degree 4 in Sloan's factored form.
  const float fC3 = x * fC2 - y * fS2;  // x^4 - 6x^2y^2 + y^4
  const float fS3 = x * fS2 + y * fC2;  // 4x^3y - 4xy^3
  const float fC2x = 3.f * fC1, fC2y = -6.f * xy;
  const float fS2x = 6.f * xy, fS2y = 3.f * fC1;
  const float fC3x = 4.f * x * (xx - 3.f * yy), fC3y = 4.f * y * (yy - 3.f * xx);
  const float fS3x = 4.f * y * (3.f * xx - yy), fS3y = 4.f * x * (xx - 3.f * yy);
  const float d0 = z * (-C4e * zz + C4f);   // fTmp0D
  const float d0z = -3.f * C4e * zz + C4f;
  const float c1 = C4c * zz - C4d;          // fTmp1C
  const float c1z = 2.f * C4c * z;
  const float b2 = -C4b * z;                // fTmp2B
  const float p12 = z * (5.f * C3d * zz - 3.f * C3d);
  const float p12z = 15.f * C3d * zz - 3.f * C3d;
  const float p6 = C2b * zz - C2c, p6z = 2.f * C2b * z;
  f(16, C4a * fS3, C4a * fS3x, C4a * fS3y, 0.f);
  f(17, b2 * fS2, b2 * fS2x, b2 * fS2y, -C4b * fS2);
  f(18, c1 * fS1, c1 * 2.f * y, c1 * 2.f * x, c1z * fS1);
  f(19, d0 * y, 0.f, d0, d0z * y);
  f(20, C4g * z * p12 - C4h * p6, 0.f, 0.f, C4g * (p12 + z * p12z) - C4h * p6z);
  f(21, d0 * x, d0, 0.f, d0z * x);
  f(22, c1 * fC1, c1 * 2.f * x, -c1 * 2.f * y, c1z * fC1);
  f(23, b2 * fC2, b2 * fC2x, b2 * fC2y, -C4b * fC2);
  f(24, C4a * fC3, C4a * fC3x, C4a * fC3y, 0.f);
}

// colors[c] = sum_k Y_k(dir/|dir|) * coeffs[k*3 + c]  (3 channels)
__device__ __forceinline__ void sh_eval3(int degree, float dx, float dy, float dz,
                                         const float* __restrict__ coeffs, float out[3]) {
  float x = 0.f, y = 0.f, z = 0.f;
  if (degree >= 1) {
    const float inorm = 1.0f / sqrtf(dx * dx + dy * dy + dz * dz);
    x = dx * inorm;
    y = dy * inorm;
    z = dz * inorm;
  }
  float r = 0.f, g = 0.f, b = 0.f;
  sh_foreach(degree, x, y, z, [&](int k, float Y, float, float, float) {
    r += Y * coeffs[k * 3 + 0];
    g += Y * coeffs[k * 3 + 1];
    b += Y * coeffs[k * 3 + 2];
  });
  out[0] = r;
  out[1] = g;
  out[2] = b;
}

// VJP of sh_eval3.  Writes (ACCUM: adds to) v_coeffs[k*3+c] for
// k < (degree+1)^2 (entries above the degree are left to the caller) and
// returns v_dir (the gradient w.r.t. the un-normalised direction) when
// want_dir is set.  FAST_NORM normalises with the hardware reciprocal square
// root (1 ulp) instead of an IEEE square root and division.
template <bool ACCUM = false, bool FAST_NORM = false>
__device__ __forceinline__ void sh_vjp3(int degree, float dx, float dy, float dz,
                                        const float* __restrict__ coeffs, const float v_col[3],
                                        float* __restrict__ v_coeffs, bool want_dir,
                                        float v_dir[3]) {
  float x = 0.f, y = 0.f, z = 0.f, inorm = 0.f;
  if (degree >= 1) {
    const float n2 = dx * dx + dy * dy + dz * dz;
    inorm = FAST_NORM ? __builtin_amdgcn_rsqf(n2) : 1.0f / sqrtf(n2);
    x = dx * inorm;
    y = dy * inorm;
    z = dz * inorm;
  }
  float gx = 0.f, gy = 0.f, gz = 0.f;
  sh_foreach(degree, x, y, z, [&](int k, float Y, float Yx, float Yy, float Yz) {
    if (ACCUM) {
      v_coeffs[k * 3 + 0] += Y * v_col[0];
      v_coeffs[k * 3 + 1] += Y * v_col[1];
      v_coeffs[k * 3 + 2] += Y * v_col[2];
    } else {
      v_coeffs[k * 3 + 0] = Y * v_col[0];
      v_coeffs[k * 3 + 1] = Y * v_col[1];
      v_coeffs[k * 3 + 2] = Y * v_col[2];
    }
    if (want_dir && k > 0) {
      const float s = coeffs[k * 3 + 0] * v_col[0] + coeffs[k * 3 + 1] * v_col[1] +
                      coeffs[k * 3 + 2] * v_col[2];
      gx += s * Yx;
      gy += s * Yy;
      gz += s * Yz;
    }
  });
  v_dir[0] = v_dir[1] = v_dir[2] = 0.f;
  if (want_dir && degree >= 1) {
    // d(dir/|dir|)/d dir = (I - n n^T) / |dir|
    const float dot = gx * x + gy * y + gz * z;
    v_dir[0] = (gx - dot * x) * inorm;
    v_dir[1] = (gy - dot * y) * inorm;
    v_dir[2] = (gz - dot * z) * inorm;
  }
}
