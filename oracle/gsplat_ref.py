"""CPU restatement of gsplat 1.0's projection and spherical-harmonics math.

Test oracle only (see ``oracle/__init__.py``).  All functions take torch CPU
tensors and a ``dtype`` (float32 mirrors the kernels, float64 is the
high-precision truth).

Restated from:
* ``gsplat/cuda/csrc/utils.cuh:10-73`` (quat -> rotmat, covariance),
  ``:146-172`` (perspective projection), ``:234-312`` (world->cam, inverse, blur)
* ``gsplat/cuda/csrc/fully_fused_projection_fwd.cu:18-129`` (fused forward, culls)
* ``gsplat/cuda/csrc/fully_fused_projection_bwd.cu:18-185`` and the VJPs at
  ``utils.cuh:31-52,75-107,174-232,242-301,314-344``
* ``gsplat/cuda/csrc/spherical_harmonics.cuh:11-352`` (SH basis and VJP)

Pins (tests/test_oracle_gsplat.py): covariance vs scipy Rotation; conic vs
numpy.linalg.inv; mean2d vs K @ p_c; radius vs the eigenvalue closed form;
backward vs torch.autograd of the forward in float64; SH basis vs
scipy.special spherical harmonics; SH backward vs autograd.
"""
from __future__ import annotations

import torch

# ---------------------------------------------------------------------------
# projection
# ---------------------------------------------------------------------------


def quat_to_rotmat(q: torch.Tensor) -> torch.Tensor:
    """Row-major rotation of the normalised (w, x, y, z) quaternion (utils.cuh:10-29)."""
    q = q / torch.sqrt((q * q).sum(-1, keepdim=True))
    w, x, y, z = q.unbind(-1)
    R = torch.stack([
        1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
        2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
        2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y),
    ], -1)
    return R.reshape(*q.shape[:-1], 3, 3)


def covar_from_quat_scale(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """Sigma = (R S)(R S)^T (utils.cuh:54-73)."""
    M = quat_to_rotmat(q) * s[..., None, :]
    return M @ M.transpose(-1, -2)


def covar_from_6(c: torch.Tensor) -> torch.Tensor:
    return torch.stack([c[..., 0], c[..., 1], c[..., 2],
                        c[..., 1], c[..., 3], c[..., 4],
                        c[..., 2], c[..., 4], c[..., 5]], -1).reshape(*c.shape[:-1], 3, 3)


def _cam_split(viewmats, Ks):
    R = viewmats[:, :3, :3]
    t = viewmats[:, :3, 3]
    fx, fy, cx, cy = Ks[:, 0, 0], Ks[:, 1, 1], Ks[:, 0, 2], Ks[:, 1, 2]
    return R, t, fx, fy, cx, cy


def project_core(means, Sigma, viewmats, Ks, W, H, eps2d):
    """Differentiable part of the projection for every (camera, Gaussian).

    Returns p_c [C,N,3], mean2d [C,N,2], cov2d (blurred) [C,N,2,2], det_blur,
    det_orig, conics [C,N,3], compensation [C,N].
    """
    R, t, fx, fy, cx, cy = _cam_split(viewmats, Ks)
    pc = torch.einsum("cij,nj->cni", R, means) + t[:, None, :]
    Sc = R[:, None] @ Sigma[None] @ R[:, None].transpose(-1, -2)
    x, y, z = pc.unbind(-1)
    lim_x = (1.3 * (0.5 * W / fx))[:, None]
    lim_y = (1.3 * (0.5 * H / fy))[:, None]
    rz = 1.0 / z
    rz2 = rz * rz
    tx = z * torch.minimum(lim_x, torch.maximum(-lim_x, x * rz))
    ty = z * torch.minimum(lim_y, torch.maximum(-lim_y, y * rz))
    fxb, fyb = fx[:, None], fy[:, None]
    zero = torch.zeros_like(z)
    J = torch.stack([fxb * rz, zero, -fxb * tx * rz2,
                     zero, fyb * rz, -fyb * ty * rz2], -1).reshape(*z.shape, 2, 3)
    cov2d = J @ Sc @ J.transpose(-1, -2)
    a, b, d = cov2d[..., 0, 0], cov2d[..., 0, 1], cov2d[..., 1, 1]
    det_orig = a * d - b * b
    a = a + eps2d
    d = d + eps2d
    det = a * d - b * b
    comp = torch.sqrt(torch.clamp(det_orig / det, min=0.0))
    inv = 1.0 / det
    conics = torch.stack([d * inv, -b * inv, a * inv], -1)
    mean2d = torch.stack([fxb * x * rz + cx[:, None], fyb * y * rz + cy[:, None]], -1)
    return pc, mean2d, a, b, d, det, conics, comp


def project_fwd(means, quats=None, scales=None, viewmats=None, Ks=None, W=0, H=0,
                eps2d=0.3, near_plane=0.01, far_plane=1e10, radius_clip=0.0, covars=None,
                dtype=torch.float64, packed=False):
    """gsplat fully_fused_projection forward (fwd.cu:18-129), dense [C, N] layout.

    ``packed`` applies the packed kernel's radius rule
    (fully_fused_projection_packed_fwd.cu:111-119: ``sqrt(max(0.1, b^2 - det))``
    instead of ``max(0.01, ...)``); every other quantity is the same.  Culled
    entries get radius 0 and zeros elsewhere.
    """
    means = means.to(dtype)
    viewmats = viewmats.to(dtype)
    Ks = Ks.to(dtype)
    Sigma = covar_from_6(covars.to(dtype)) if covars is not None else \
        covar_from_quat_scale(quats.to(dtype), scales.to(dtype))
    pc, mean2d, a, b, d, det, conics, comp = project_core(means, Sigma, viewmats, Ks, W, H, eps2d)
    z = pc[..., 2]
    ok = (z >= near_plane) & (z <= far_plane) & (det > 0)
    bb = 0.5 * (a + d)
    v1 = bb + torch.sqrt(torch.clamp(bb * bb - det, min=0.1 if packed else 0.01))
    radius = torch.ceil(3.0 * torch.sqrt(v1))
    ok &= ~(radius <= radius_clip)
    mx, my = mean2d[..., 0], mean2d[..., 1]
    ok &= ~((mx + radius <= 0) | (mx - radius >= W) | (my + radius <= 0) | (my - radius >= H))
    ok &= torch.isfinite(radius)
    radii = torch.where(ok, radius, torch.zeros_like(radius)).to(torch.int32)
    okf = ok[..., None]
    return (radii,
            torch.where(okf, mean2d, torch.zeros_like(mean2d)),
            torch.where(ok, z, torch.zeros_like(z)),
            torch.where(okf, conics, torch.zeros_like(conics)),
            torch.where(ok, comp, torch.zeros_like(comp)))


def _quat_rotmat_vjp(q, G):
    """dL/dq for R = rotmat(q/|q|) given G = dL/dR (utils.cuh:31-52)."""
    inv = 1.0 / torch.sqrt((q * q).sum(-1, keepdim=True))
    n = q * inv
    w, x, y, z = n.unbind(-1)
    g = lambda i, j: G[..., i, j]  # noqa: E731
    vw = 2 * (x * (g(2, 1) - g(1, 2)) + y * (g(0, 2) - g(2, 0)) + z * (g(1, 0) - g(0, 1)))
    vx = 2 * (-2 * x * (g(1, 1) + g(2, 2)) + y * (g(0, 1) + g(1, 0)) + z * (g(0, 2) + g(2, 0))
              + w * (g(2, 1) - g(1, 2)))
    vy = 2 * (x * (g(0, 1) + g(1, 0)) - 2 * y * (g(0, 0) + g(2, 2)) + z * (g(1, 2) + g(2, 1))
              + w * (g(0, 2) - g(2, 0)))
    vz = 2 * (x * (g(0, 2) + g(2, 0)) + y * (g(1, 2) + g(2, 1)) - 2 * z * (g(0, 0) + g(1, 1))
              + w * (g(1, 0) - g(0, 1)))
    vn = torch.stack([vw, vx, vy, vz], -1)
    return (vn - (vn * n).sum(-1, keepdim=True) * n) * inv


def project_bwd(means, quats, scales, viewmats, Ks, W, H, eps2d, radii, conics,
                v_means2d, v_depths, v_conics, compensations=None, v_compensations=None,
                covars=None, want_viewmats=False, dtype=torch.float64):
    """gsplat fully_fused_projection backward (bwd.cu:18-185), vectorised.

    Returns (v_means [N,3], v_quats [N,4] | None, v_scales [N,3] | None,
    v_covars [N,6] | None, v_viewmats [C,4,4] | None).
    """
    cvt = lambda t: None if t is None else t.to(dtype)  # noqa: E731
    means, viewmats, Ks = cvt(means), cvt(viewmats), cvt(Ks)
    conics, v_means2d, v_conics = cvt(conics), cvt(v_means2d), cvt(v_conics)
    v_depths = cvt(v_depths) if v_depths is not None else torch.zeros(radii.shape, dtype=dtype)
    if covars is not None:
        Sigma = covar_from_6(cvt(covars))
    else:
        quats, scales = cvt(quats), cvt(scales)
        Sigma = covar_from_quat_scale(quats, scales)
    live = (radii > 0)
    R, t, fx, fy, cx, cy = _cam_split(viewmats, Ks)

    # conic = inverse(cov2d): G_cov = -P G_P P
    P00, P01, P11 = conics.unbind(-1)
    G00, G01, G11 = v_conics[..., 0], 0.5 * v_conics[..., 1], v_conics[..., 2]
    T00 = G00 * P00 + G01 * P01
    T01 = G00 * P01 + G01 * P11
    T10 = G01 * P00 + G11 * P01
    T11 = G01 * P01 + G11 * P11
    C00 = -(P00 * T00 + P01 * T10)
    C01 = -(P00 * T01 + P01 * T11)
    C10 = -(P01 * T00 + P11 * T10)
    C11 = -(P01 * T01 + P11 * T11)
    if v_compensations is not None:
        comp = cvt(compensations)
        vcomp = cvt(v_compensations)
        det_p = P00 * P11 - P01 * P01
        v_sqr = vcomp * 0.5 / (comp + 1e-6)
        one_m = 1 - comp * comp
        C00 = C00 + v_sqr * (one_m * P00 - eps2d * det_p)
        C01 = C01 + v_sqr * (one_m * P01)
        C10 = C10 + v_sqr * (one_m * P01)
        C11 = C11 + v_sqr * (one_m * P11 - eps2d * det_p)
    Gc = torch.stack([C00, C01, C10, C11], -1).reshape(*C00.shape, 2, 2)

    pc = torch.einsum("cij,nj->cni", R, means) + t[:, None, :]
    RS = R[:, None] @ Sigma[None]
    Sc = RS @ R[:, None].transpose(-1, -2)
    x, y, z = pc.unbind(-1)
    fxb, fyb = fx[:, None], fy[:, None]
    lim_x = (1.3 * (0.5 * W / fx))[:, None]
    lim_y = (1.3 * (0.5 * H / fy))[:, None]
    rz = 1.0 / z
    rz2 = rz * rz
    rz3 = rz2 * rz
    tx = z * torch.minimum(lim_x, torch.maximum(-lim_x, x * rz))
    ty = z * torch.minimum(lim_y, torch.maximum(-lim_y, y * rz))
    zero = torch.zeros_like(z)
    J = torch.stack([fxb * rz, zero, -fxb * tx * rz2,
                     zero, fyb * rz, -fyb * ty * rz2], -1).reshape(*z.shape, 2, 3)
    GSc = J.transpose(-1, -2) @ Gc @ J
    GJ = Gc @ J @ Sc.transpose(-1, -2) + Gc.transpose(-1, -2) @ J @ Sc
    vm = v_means2d
    gx = fxb * rz * vm[..., 0]
    gy = fyb * rz * vm[..., 1]
    gz = -(fxb * x * vm[..., 0] + fyb * y * vm[..., 1]) * rz2
    in_x = (x * rz <= lim_x) & (x * rz >= -lim_x)
    in_y = (y * rz <= lim_y) & (y * rz >= -lim_y)
    gx = gx + torch.where(in_x, -fxb * rz2 * GJ[..., 0, 2], zero)
    gz = gz + torch.where(in_x, zero, -fxb * rz3 * GJ[..., 0, 2] * tx)
    gy = gy + torch.where(in_y, -fyb * rz2 * GJ[..., 1, 2], zero)
    gz = gz + torch.where(in_y, zero, -fyb * rz3 * GJ[..., 1, 2] * ty)
    gz = gz + (-fxb * rz2 * GJ[..., 0, 0] - fyb * rz2 * GJ[..., 1, 1]
               + 2 * fxb * tx * rz3 * GJ[..., 0, 2] + 2 * fyb * ty * rz3 * GJ[..., 1, 2])
    gz = gz + v_depths
    gpc = torch.stack([gx, gy, gz], -1)
    livef = live[..., None].to(dtype)
    gpc = gpc * livef
    GSc = GSc * livef[..., None]
    gpc = torch.nan_to_num(gpc) * livef
    GSc = torch.nan_to_num(GSc) * livef[..., None]

    v_means = torch.einsum("cij,cni->nj", R, gpc)
    v_Sigma = (R[:, None].transpose(-1, -2) @ GSc @ R[:, None]).sum(0)
    v_viewmats = None
    if want_viewmats:
        vR = torch.einsum("cni,nj->cij", gpc, means)
        vR = vR + (GSc @ (R[:, None] @ Sigma[None].transpose(-1, -2))).sum(1)
        vR = vR + (GSc.transpose(-1, -2) @ RS).sum(1)
        vt = gpc.sum(1)
        v_viewmats = torch.zeros(viewmats.shape, dtype=dtype)
        v_viewmats[:, :3, :3] = vR
        v_viewmats[:, :3, 3] = vt
    if covars is not None:
        vS = v_Sigma
        v_covars = torch.stack([vS[:, 0, 0], vS[:, 0, 1] + vS[:, 1, 0], vS[:, 0, 2] + vS[:, 2, 0],
                                vS[:, 1, 1], vS[:, 1, 2] + vS[:, 2, 1], vS[:, 2, 2]], -1)
        return v_means, None, None, v_covars, v_viewmats
    Rq = quat_to_rotmat(quats)
    M = Rq * scales[:, None, :]
    GM = (v_Sigma + v_Sigma.transpose(-1, -2)) @ M
    v_scales = (Rq * GM).sum(-2)
    GR = GM * scales[:, None, :]
    v_quats = _quat_rotmat_vjp(quats, GR)
    return v_means, v_quats, v_scales, None, v_viewmats


# ---------------------------------------------------------------------------
# spherical harmonics
# ---------------------------------------------------------------------------

_SH_C0 = 0.28209479177387814
_SH_C1 = 0.4886025119029199


def sh_basis(degree: int, n: torch.Tensor) -> torch.Tensor:
    """Real SH basis Y_k(n) for k < (degree+1)^2 at unit directions n [...,3]
    (spherical_harmonics.cuh:20-89, Sloan's polynomial form)."""
    x, y, z = n.unbind(-1)
    out = [torch.full_like(x, _SH_C0)]
    if degree >= 1:
        out += [-_SH_C1 * y, _SH_C1 * z, -_SH_C1 * x]
    if degree >= 2:
        z2 = z * z
        fC1 = x * x - y * y
        fS1 = 2 * x * y
        out += [0.5462742152960395 * fS1, -1.092548430592079 * z * y,
                0.9461746957575601 * z2 - 0.3153915652525201, -1.092548430592079 * z * x,
                0.5462742152960395 * fC1]
    if degree >= 3:
        fC2 = x * fC1 - y * fS1
        fS2 = x * fS1 + y * fC1
        t0 = -2.285228997322329 * z2 + 0.4570457994644658
        t1 = 1.445305721320277 * z
        out += [-0.5900435899266435 * fS2, t1 * fS1, t0 * y,
                z * (1.865881662950577 * z2 - 1.119528997770346), t0 * x, t1 * fC1,
                -0.5900435899266435 * fC2]
    if degree >= 4:
        fC3 = x * fC2 - y * fS2
        fS3 = x * fS2 + y * fC2
        d0 = z * (-4.683325804901025 * z2 + 2.007139630671868)
        c1 = 3.31161143515146 * z2 - 0.47308734787878
        b2 = -1.770130769779931 * z
        p12 = z * (1.865881662950577 * z2 - 1.119528997770346)
        p6 = 0.9461746957575601 * z2 - 0.3153915652525201
        out += [0.6258357354491763 * fS3, b2 * fS2, c1 * fS1, d0 * y,
                1.984313483298443 * z * p12 - 1.006230589874905 * p6, d0 * x, c1 * fC1,
                b2 * fC2, 0.6258357354491763 * fC3]
    return torch.stack(out, -1)


def _normalize(dirs):
    return dirs / torch.sqrt((dirs * dirs).sum(-1, keepdim=True))


def sh_fwd(degree: int, dirs: torch.Tensor, coeffs: torch.Tensor, dtype=torch.float64):
    """colors[...,c] = sum_k Y_k(dirs/|dirs|) coeffs[...,k,c] (compute_sh_fwd.cu:9-29)."""
    dirs, coeffs = dirs.to(dtype), coeffs.to(dtype)
    K = (degree + 1) ** 2
    n = _normalize(dirs) if degree >= 1 else dirs
    Y = sh_basis(degree, n)
    return (Y[..., :, None] * coeffs[..., :K, :]).sum(-2)


def sh_basis_grad(degree: int, n: torch.Tensor) -> torch.Tensor:
    """dY_k/d(x,y,z) treating the unit-vector components as independent,
    [..., K, 3] (the derivative polynomials of spherical_harmonics.cuh:94-352)."""
    x, y, z = n.unbind(-1)
    o, zz = torch.zeros_like(x), torch.ones_like(x)
    rows = [(o, o, o)]
    if degree >= 1:
        c = _SH_C1
        rows += [(o, -c * zz, o), (o, o, c * zz), (-c * zz, o, o)]
    if degree >= 2:
        a = 1.092548430592079
        rows += [(a * y, a * x, o), (o, -a * z, -a * y), (o, o, 2 * 0.9461746957575601 * z),
                 (-a * z, o, -a * x), (a * x, -a * y, o)]
    if degree >= 3:
        c3a, c3b, c3c = 0.5900435899266435, 1.445305721320277, 0.4570457994644658
        c12a, c12b = 1.865881662950577, 1.119528997770346
        fC1 = x * x - y * y
        t0 = -5 * c3c * z * z + c3c
        rows += [(-c3a * 6 * x * y, -c3a * 3 * fC1, o),
                 (2 * c3b * y * z, 2 * c3b * x * z, 2 * c3b * x * y),
                 (o, t0, -10 * c3c * y * z),
                 (o, o, 3 * c12a * z * z - c12b),
                 (t0, o, -10 * c3c * x * z),
                 (2 * c3b * x * z, -2 * c3b * y * z, c3b * fC1),
                 (-c3a * 3 * fC1, c3a * 6 * x * y, o)]
    if degree >= 4:
        fC1 = x * x - y * y
        fS1 = 2 * x * y
        fC2 = x * fC1 - y * fS1
        fS2 = x * fS1 + y * fC1
        C4a, C4b, C4c, C4d = 0.6258357354491763, 1.770130769779931, 3.31161143515146, 0.47308734787878
        C4e, C4f, C4g, C4h = 4.683325804901025, 2.007139630671868, 1.984313483298443, 1.006230589874905
        d0 = z * (-C4e * z * z + C4f)
        d0z = -3 * C4e * z * z + C4f
        c1 = C4c * z * z - C4d
        c1z = 2 * C4c * z
        b2 = -C4b * z
        p12 = z * (1.865881662950577 * z * z - 1.119528997770346)
        p12z = 3 * 1.865881662950577 * z * z - 1.119528997770346
        p6z = 2 * 0.9461746957575601 * z
        rows += [(C4a * 4 * y * (3 * x * x - y * y), C4a * 4 * x * (x * x - 3 * y * y), o),
                 (b2 * 6 * x * y, b2 * 3 * fC1, -C4b * fS2),
                 (c1 * 2 * y, c1 * 2 * x, c1z * fS1),
                 (o, d0, d0z * y),
                 (o, o, C4g * (p12 + z * p12z) - C4h * p6z),
                 (d0, o, d0z * x),
                 (c1 * 2 * x, -c1 * 2 * y, c1z * fC1),
                 (b2 * 3 * fC1, b2 * (-6 * x * y), -C4b * fC2),
                 (C4a * 4 * x * (x * x - 3 * y * y), C4a * 4 * y * (y * y - 3 * x * x), o)]
    return torch.stack([torch.stack(r, -1) for r in rows], -2)


def sh_bwd(degree: int, dirs, coeffs, v_colors, dtype=torch.float64):
    """VJP of sh_fwd (compute_sh_bwd.cu:68-99): v_coeffs [...,K,3] (zero above the
    degree) and v_dirs [...,3] (zero for degree 0)."""
    dirs, coeffs, v_colors = dirs.to(dtype), coeffs.to(dtype), v_colors.to(dtype)
    Kd = (degree + 1) ** 2
    v_coeffs = torch.zeros_like(coeffs)
    if degree == 0:
        v_coeffs[..., 0, :] = _SH_C0 * v_colors
        return v_coeffs, torch.zeros_like(dirs)
    norm = torch.sqrt((dirs * dirs).sum(-1, keepdim=True))
    n = dirs / norm
    Y = sh_basis(degree, n)
    v_coeffs[..., :Kd, :] = Y[..., :, None] * v_colors[..., None, :]
    s = (coeffs[..., :Kd, :] * v_colors[..., None, :]).sum(-1)      # [...,K]
    gY = sh_basis_grad(degree, n)                                     # [...,K,3]
    g = (s[..., None] * gY).sum(-2)
    v_dirs = (g - (g * n).sum(-1, keepdim=True) * n) / norm
    return v_coeffs, v_dirs
