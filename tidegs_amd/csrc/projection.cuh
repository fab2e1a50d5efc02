// EWA projection of one 3D Gaussian into one pinhole camera, and its VJP.
//
// Forward (gsplat fully_fused_projection_fwd.cu:18-129 with utils.cuh:10-73,
// 146-172, 234-312), written here in row-major form:
//   p_c   = R p + t                       cull if z < near or z > far
//   Sigma = (Rq S)(Rq S)^T,  Rq = rotmat(q / |q|), S = diag(scale)
//   Sig_c = R Sigma R^T
//   J     = [[fx/z, 0, -fx tx/z^2], [0, fy/z, -fy ty/z^2]],
//           tx = z clamp(x/z, +-1.3 W/(2 fx)), ty likewise
//   cov2d = J Sig_c J^T + eps2d I     (compensation = sqrt(det_orig/det_blur))
//   cull if det <= 0; conic = cov2d^-1
//   radius = ceil(3 sqrt(b + sqrt(max(0.01, b^2 - det)))), b = tr/2
//   cull if radius <= radius_clip or the 3-sigma box misses the image.
// Backward (fully_fused_projection_bwd.cu:199-366, utils.cuh:31-52,75-107,
// 174-232,242-301,314-344) is the exact VJP of the same chain, including the
// fov-clamp branch of J and the normalisation inside rotmat(q).
#pragma once

#include "tgs_common.cuh"

struct Cam {
  float R[3][3];
  float t[3];
  float fx, fy, cx, cy;
};

// viewmat: row-major [4,4] world-to-camera; K: row-major [3,3].
__device__ __forceinline__ Cam load_cam(const float* __restrict__ viewmat,
                                        const float* __restrict__ K) {
  Cam c;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
#pragma unroll
    for (int j = 0; j < 3; ++j) c.R[i][j] = viewmat[i * 4 + j];
    c.t[i] = viewmat[i * 4 + 3];
  }
  c.fx = K[0];
  c.cx = K[2];
  c.fy = K[4];
  c.cy = K[5];
  return c;
}

// Row-major rotation matrix of the normalised quaternion (w, x, y, z).
__device__ __forceinline__ m3 quat_to_rotmat(float w, float x, float y, float z) {
  const float inv = 1.0f / sqrtf(w * w + x * x + y * y + z * z);
  w *= inv;
  x *= inv;
  y *= inv;
  z *= inv;
  const float x2 = x * x, y2 = y * y, z2 = z * z;
  const float xy = x * y, xz = x * z, yz = y * z;
  const float wx = w * x, wy = w * y, wz = w * z;
  m3 R;
  R.m[0][0] = 1.f - 2.f * (y2 + z2);
  R.m[0][1] = 2.f * (xy - wz);
  R.m[0][2] = 2.f * (xz + wy);
  R.m[1][0] = 2.f * (xy + wz);
  R.m[1][1] = 1.f - 2.f * (x2 + z2);
  R.m[1][2] = 2.f * (yz - wx);
  R.m[2][0] = 2.f * (xz - wy);
  R.m[2][1] = 2.f * (yz + wx);
  R.m[2][2] = 1.f - 2.f * (x2 + y2);
  return R;
}

// Gradient w.r.t. the raw quaternion given G = dL/dR (row-major); accounts
// for the normalisation: v_q = (I - n n^T) v_n / |q|.
__device__ __forceinline__ void quat_to_rotmat_vjp(const float q[4], const m3& G, float v_q[4]) {
  const float inv = 1.0f / sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
  const float w = q[0] * inv, x = q[1] * inv, y = q[2] * inv, z = q[3] * inv;
  const float (&g)[3][3] = G.m;
  float vn[4];
  vn[0] = 2.f * (x * (g[2][1] - g[1][2]) + y * (g[0][2] - g[2][0]) + z * (g[1][0] - g[0][1]));
  vn[1] = 2.f * (-2.f * x * (g[1][1] + g[2][2]) + y * (g[0][1] + g[1][0]) +
                 z * (g[0][2] + g[2][0]) + w * (g[2][1] - g[1][2]));
  vn[2] = 2.f * (x * (g[0][1] + g[1][0]) - 2.f * y * (g[0][0] + g[2][2]) +
                 z * (g[1][2] + g[2][1]) + w * (g[0][2] - g[2][0]));
  vn[3] = 2.f * (x * (g[0][2] + g[2][0]) + y * (g[1][2] + g[2][1]) -
                 2.f * z * (g[0][0] + g[1][1]) + w * (g[1][0] - g[0][1]));
  const float dot = vn[0] * w + vn[1] * x + vn[2] * y + vn[3] * z;
  v_q[0] = (vn[0] - dot * w) * inv;
  v_q[1] = (vn[1] - dot * x) * inv;
  v_q[2] = (vn[2] - dot * y) * inv;
  v_q[3] = (vn[3] - dot * z) * inv;
}

// Sigma = (Rq S)(Rq S)^T
__device__ __forceinline__ m3 covar_from_quat_scale(const float q[4], const float s[3]) {
  const m3 Rq = quat_to_rotmat(q[0], q[1], q[2], q[3]);
  m3 M;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) M.m[i][j] = Rq.m[i][j] * s[j];
  return m3_mul_bt(M, M);
}

// covars6 = upper triangle (xx, xy, xz, yy, yz, zz)
__device__ __forceinline__ m3 covar_from_6(const float* __restrict__ c) {
  m3 S;
  S.m[0][0] = c[0];
  S.m[0][1] = S.m[1][0] = c[1];
  S.m[0][2] = S.m[2][0] = c[2];
  S.m[1][1] = c[3];
  S.m[1][2] = S.m[2][1] = c[4];
  S.m[2][2] = c[5];
  return S;
}

struct ProjResult {
  float mean2d[2];
  float depth;
  float conic[3];
  float comp;
  int radius;  // 0 = culled
};

// PACKED selects the radius rule of the packed projection
// (fully_fused_projection_packed_fwd.cu:111-119: sqrt(max(0.1, b^2 - det)))
// instead of the dense one (fully_fused_projection_fwd.cu:99-103: 0.01).
template <bool PACKED = false>
__device__ __forceinline__ ProjResult project_forward(const float p[3], const m3& Sigma,
                                                      const Cam& cam, int W, int H, float eps2d,
                                                      float near_plane, float far_plane,
                                                      float radius_clip) {
  ProjResult out;
  out.radius = 0;
  float pc[3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
    pc[i] = cam.R[i][0] * p[0] + cam.R[i][1] * p[1] + cam.R[i][2] * p[2] + cam.t[i];
  if (pc[2] < near_plane || pc[2] > far_plane) return out;

  m3 Rc;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) Rc.m[i][j] = cam.R[i][j];
  const m3 Sc = m3_mul_bt(m3_mul(Rc, Sigma), Rc);

  const float x = pc[0], y = pc[1], z = pc[2];
  const float lim_x = 1.3f * (0.5f * (float)W / cam.fx);
  const float lim_y = 1.3f * (0.5f * (float)H / cam.fy);
  const float rz = 1.f / z;
  const float rz2 = rz * rz;
  const float tx = z * fminf(lim_x, fmaxf(-lim_x, x * rz));
  const float ty = z * fminf(lim_y, fmaxf(-lim_y, y * rz));
  const float J00 = cam.fx * rz, J02 = -cam.fx * tx * rz2;
  const float J11 = cam.fy * rz, J12 = -cam.fy * ty * rz2;
  // JS = J Sc (2x3)
  float JS0[3], JS1[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    JS0[k] = J00 * Sc.m[0][k] + J02 * Sc.m[2][k];
    JS1[k] = J11 * Sc.m[1][k] + J12 * Sc.m[2][k];
  }
  float a = JS0[0] * J00 + JS0[2] * J02;
  float b = JS0[1] * J11 + JS0[2] * J12;
  float d = JS1[1] * J11 + JS1[2] * J12;
  const float det_orig = a * d - b * b;
  a += eps2d;
  d += eps2d;
  const float det = a * d - b * b;
  out.comp = sqrtf(fmaxf(0.f, det_orig / det));
  if (det <= 0.f) return out;
  const float inv_det = 1.f / det;
  out.conic[0] = d * inv_det;
  out.conic[1] = -b * inv_det;
  out.conic[2] = a * inv_det;

  const float bb = 0.5f * (a + d);
  const float v1 = bb + sqrtf(fmaxf(PACKED ? 0.1f : 0.01f, bb * bb - det));
  const float radius = ceilf(3.f * sqrtf(v1));
  if (radius <= radius_clip) return out;

  const float mx = cam.fx * x * rz + cam.cx;
  const float my = cam.fy * y * rz + cam.cy;
  if (mx + radius <= 0.f || mx - radius >= (float)W || my + radius <= 0.f ||
      my - radius >= (float)H)
    return out;
  out.mean2d[0] = mx;
  out.mean2d[1] = my;
  out.depth = z;
  out.radius = (int)radius;
  return out;
}

struct ProjGrad {
  float v_p[3];    // d/d world mean
  m3 v_Sigma;      // d/d world covariance (not symmetrised)
  m3 v_R;          // d/d viewmat rotation
  float v_t[3];    // d/d viewmat translation
};

// VJP of project_forward for a Gaussian that was not culled.
__device__ __forceinline__ void project_backward(const float p[3], const m3& Sigma,
                                                 const Cam& cam, int W, int H, float eps2d,
                                                 const float conic[3], float comp,
                                                 const float v_mean2d[2], float v_depth,
                                                 const float v_conic[3], bool has_v_comp,
                                                 float v_comp, bool want_cam, ProjGrad& out) {
  // conic = inverse(cov2d): G_cov = -P G_P P with the off-diagonal gradient
  // split evenly over the two symmetric entries.
  const float P00 = conic[0], P01 = conic[1], P11 = conic[2];
  const float G00 = v_conic[0], G01 = 0.5f * v_conic[1], G11 = v_conic[2];
  // T = G_P P
  const float T00 = G00 * P00 + G01 * P01, T01 = G00 * P01 + G01 * P11;
  const float T10 = G01 * P00 + G11 * P01, T11 = G01 * P01 + G11 * P11;
  float C00 = -(P00 * T00 + P01 * T10);
  float C01 = -(P00 * T01 + P01 * T11);
  float C10 = -(P01 * T00 + P11 * T10);
  float C11 = -(P01 * T01 + P11 * T11);
  if (has_v_comp) {
    // d comp / d cov2d = (1 - comp^2) P - eps2d det(P) I, scaled by 1/(2 comp)
    const float det_p = P00 * P11 - P01 * P01;
    const float v_sqr = v_comp * 0.5f / (comp + 1e-6f);
    const float one_m = 1.f - comp * comp;
    C00 += v_sqr * (one_m * P00 - eps2d * det_p);
    C01 += v_sqr * (one_m * P01);
    C10 += v_sqr * (one_m * P01);
    C11 += v_sqr * (one_m * P11 - eps2d * det_p);
  }

  float pc[3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
    pc[i] = cam.R[i][0] * p[0] + cam.R[i][1] * p[1] + cam.R[i][2] * p[2] + cam.t[i];
  m3 Rc;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) Rc.m[i][j] = cam.R[i][j];
  const m3 RS = m3_mul(Rc, Sigma);
  const m3 Sc = m3_mul_bt(RS, Rc);

  const float x = pc[0], y = pc[1], z = pc[2];
  const float fx = cam.fx, fy = cam.fy;
  const float lim_x = 1.3f * (0.5f * (float)W / fx);
  const float lim_y = 1.3f * (0.5f * (float)H / fy);
  const float rz = 1.f / z;
  const float rz2 = rz * rz;
  const float rz3 = rz2 * rz;
  const float tx = z * fminf(lim_x, fmaxf(-lim_x, x * rz));
  const float ty = z * fminf(lim_y, fmaxf(-lim_y, y * rz));
  float J[2][3] = {{fx * rz, 0.f, -fx * tx * rz2}, {0.f, fy * rz, -fy * ty * rz2}};
  const float Gc[2][2] = {{C00, C01}, {C10, C11}};

  // G_Sc = J^T Gc J
  m3 GSc;
  {
    float GJ[2][3];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int k = 0; k < 3; ++k) GJ[r][k] = Gc[r][0] * J[0][k] + Gc[r][1] * J[1][k];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int k = 0; k < 3; ++k) GSc.m[i][k] = J[0][i] * GJ[0][k] + J[1][i] * GJ[1][k];
  }
  // G_J = Gc J Sc^T + Gc^T J Sc
  float GJm[2][3];
  {
    float JS[2][3], JSt[2][3];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        JS[r][k] = J[r][0] * Sc.m[0][k] + J[r][1] * Sc.m[1][k] + J[r][2] * Sc.m[2][k];
        JSt[r][k] = J[r][0] * Sc.m[k][0] + J[r][1] * Sc.m[k][1] + J[r][2] * Sc.m[k][2];
      }
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int k = 0; k < 3; ++k)
        GJm[r][k] = Gc[r][0] * JSt[0][k] + Gc[r][1] * JSt[1][k] + Gc[0][r] * JS[0][k] +
                    Gc[1][r] * JS[1][k];
  }
  float gpc[3];
  gpc[0] = fx * rz * v_mean2d[0];
  gpc[1] = fy * rz * v_mean2d[1];
  gpc[2] = -(fx * x * v_mean2d[0] + fy * y * v_mean2d[1]) * rz2;
  if (x * rz <= lim_x && x * rz >= -lim_x)
    gpc[0] += -fx * rz2 * GJm[0][2];
  else
    gpc[2] += -fx * rz3 * GJm[0][2] * tx;
  if (y * rz <= lim_y && y * rz >= -lim_y)
    gpc[1] += -fy * rz2 * GJm[1][2];
  else
    gpc[2] += -fy * rz3 * GJm[1][2] * ty;
  gpc[2] += -fx * rz2 * GJm[0][0] - fy * rz2 * GJm[1][1] + 2.f * fx * tx * rz3 * GJm[0][2] +
            2.f * fy * ty * rz3 * GJm[1][2];
  gpc[2] += v_depth;

  // p_c = R p + t ; Sig_c = R Sigma R^T
#pragma unroll
  for (int j = 0; j < 3; ++j)
    out.v_p[j] = Rc.m[0][j] * gpc[0] + Rc.m[1][j] * gpc[1] + Rc.m[2][j] * gpc[2];
  // v_Sigma = R^T G_Sc R
  out.v_Sigma = m3_mul(m3_mul_at(Rc, GSc), Rc);
  if (want_cam) {
    // v_R = gpc p^T + G_Sc R Sigma^T + G_Sc^T R Sigma
    const m3 RSt = m3_mul_bt(Rc, Sigma);  // R Sigma^T
    const m3 A = m3_mul(GSc, RSt);
    const m3 B = m3_mul_at(GSc, RS);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
      for (int j = 0; j < 3; ++j) out.v_R.m[i][j] = gpc[i] * p[j] + A.m[i][j] + B.m[i][j];
      out.v_t[i] = gpc[i];
    }
  }
}

// Sigma = M M^T, M = Rq diag(s): gradients w.r.t. raw quaternion and scale.
__device__ __forceinline__ void covar_vjp_quat_scale(const float q[4], const float s[3],
                                                     const m3& vSigma, float v_q[4],
                                                     float v_s[3]) {
  const m3 Rq = quat_to_rotmat(q[0], q[1], q[2], q[3]);
  m3 M, Gsym;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      M.m[i][j] = Rq.m[i][j] * s[j];
      Gsym.m[i][j] = vSigma.m[i][j] + vSigma.m[j][i];
    }
  const m3 GM = m3_mul(Gsym, M);
  m3 GR;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    v_s[j] = Rq.m[0][j] * GM.m[0][j] + Rq.m[1][j] * GM.m[1][j] + Rq.m[2][j] * GM.m[2][j];
#pragma unroll
    for (int i = 0; i < 3; ++i) GR.m[i][j] = GM.m[i][j] * s[j];
  }
  quat_to_rotmat_vjp(q, GR, v_q);
}
