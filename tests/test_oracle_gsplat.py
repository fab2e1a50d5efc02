"""Pins for the CPU oracle of the projection and SH math (oracle/gsplat_ref.py).

Each check compares the oracle with something independent of its own
formulas: scipy rotations, numpy matrix inverses / eigenvalues, the pinhole
closed form, torch.autograd of the forward, and scipy's spherical harmonics.
"""
import math

import numpy as np
import pytest
import torch
from scipy.spatial.transform import Rotation

from oracle import gsplat_ref as G
from tidegs_amd import scenes


def _rand_scene(n=300, C=2, seed=0, spread=1.0):
    g = torch.Generator().manual_seed(seed)
    means = torch.randn((n, 3), generator=g, dtype=torch.float64) * spread
    means[:, 2] += 4.0
    quats = torch.randn((n, 4), generator=g, dtype=torch.float64)
    scales = torch.exp(torch.randn((n, 3), generator=g, dtype=torch.float64) * 0.5 - 2.0)
    vms = []
    for c in range(C):
        vms.append(scenes.look_at((0.2 * c, 0.1 * c, -0.5 * c), (0.0, 0.0, 4.0),
                                  up=(0.0, -1.0, 0.0)).double())
    viewmats = torch.stack(vms)
    Ks = torch.tensor([[[120.0, 0, 64.0], [0, 110.0, 48.0], [0, 0, 1]]] * C, dtype=torch.float64)
    return means, quats, scales, viewmats, Ks


def test_rotmat_matches_scipy():
    q = torch.randn((64, 4), dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    R = G.quat_to_rotmat(q).numpy()
    qn = (q / q.norm(dim=1, keepdim=True)).numpy()
    ref = Rotation.from_quat(qn[:, [1, 2, 3, 0]]).as_matrix()  # scipy is (x,y,z,w)
    np.testing.assert_allclose(R, ref, atol=1e-12)


def test_covariance_closed_form():
    g = torch.Generator().manual_seed(2)
    q = torch.randn((32, 4), dtype=torch.float64, generator=g)
    s = torch.rand((32, 3), dtype=torch.float64, generator=g) + 0.1
    S = G.covar_from_quat_scale(q, s).numpy()
    qn = (q / q.norm(dim=1, keepdim=True)).numpy()
    R = Rotation.from_quat(qn[:, [1, 2, 3, 0]]).as_matrix()
    ref = R @ np.stack([np.diag(v ** 2) for v in s.numpy()]) @ np.transpose(R, (0, 2, 1))
    np.testing.assert_allclose(S, ref, atol=1e-12)


def test_projection_forward_closed_forms():
    means, quats, scales, viewmats, Ks = _rand_scene()
    W, H, eps = 128, 96, 0.3
    radii, m2d, depths, conics, comps = G.project_fwd(means, quats, scales, viewmats, Ks, W, H,
                                                      eps2d=eps)
    live = radii > 0
    assert live.sum() > 100
    R, t = viewmats[:, :3, :3], viewmats[:, :3, 3]
    pc = torch.einsum("cij,nj->cni", R, means) + t[:, None]
    proj = torch.einsum("cij,cnj->cni", Ks, pc)
    np.testing.assert_allclose(m2d[live].numpy(), (proj[..., :2] / proj[..., 2:])[live].numpy(),
                               rtol=1e-10, atol=1e-9)
    np.testing.assert_allclose(depths[live].numpy(), pc[..., 2][live].numpy(), rtol=1e-12)
    # conic = inverse of the blurred 2D covariance; compensation from determinants.
    Sigma = G.covar_from_quat_scale(quats, scales)
    for c in range(viewmats.shape[0]):
        for n in torch.nonzero(live[c]).flatten()[:50].tolist():
            x, y, z = pc[c, n].tolist()
            fx, fy = Ks[c, 0, 0].item(), Ks[c, 1, 1].item()
            limx, limy = 1.3 * 0.5 * W / fx, 1.3 * 0.5 * H / fy
            tx = z * min(limx, max(-limx, x / z))
            ty = z * min(limy, max(-limy, y / z))
            J = np.array([[fx / z, 0, -fx * tx / z ** 2], [0, fy / z, -fy * ty / z ** 2]])
            Sc = R[c].numpy() @ Sigma[n].numpy() @ R[c].numpy().T
            cov = J @ Sc @ J.T
            covb = cov + eps * np.eye(2)
            inv = np.linalg.inv(covb)
            np.testing.assert_allclose(conics[c, n].numpy(), [inv[0, 0], inv[0, 1], inv[1, 1]],
                                       rtol=1e-9, atol=1e-12)
            np.testing.assert_allclose(comps[c, n].item(),
                                       math.sqrt(np.linalg.det(cov) / np.linalg.det(covb)),
                                       rtol=1e-9)
            lam = np.linalg.eigvalsh(covb).max()
            r = math.ceil(3 * math.sqrt(lam))
            # b^2 - det >= 0.01 except for near-isotropic footprints
            assert abs(radii[c, n].item() - r) <= 1


def test_packed_projection_radius_rule():
    """Packed radius (fully_fused_projection_packed_fwd.cu:111-119): the same 3-sigma
    radius of the largest eigenvalue of the blurred 2D covariance, with the
    discriminant floored at 0.1 instead of 0.01; every other output equal."""
    means, quats, scales, viewmats, Ks = _rand_scene()
    W, H, eps = 128, 96, 0.3
    dense = G.project_fwd(means, quats, scales, viewmats, Ks, W, H, eps2d=eps)
    packed = G.project_fwd(means, quats, scales, viewmats, Ks, W, H, eps2d=eps, packed=True)
    rd, rp = dense[0], packed[0]
    both = (rd > 0) & (rp > 0)
    assert both.sum() > 100
    assert bool((rp[both] >= rd[both]).all())  # larger floor, never a smaller radius
    assert bool(((rd > 0) <= (rp > 0)).all())   # the packed set holds every dense survivor
    for k in range(1, 5):
        assert torch.equal(dense[k][both], packed[k][both])
    R, t = viewmats[:, :3, :3], viewmats[:, :3, 3]
    pc = torch.einsum("cij,nj->cni", R, means) + t[:, None]
    Sigma = G.covar_from_quat_scale(quats, scales)
    checked = 0
    for c in range(viewmats.shape[0]):
        for n in torch.nonzero(rp[c]).flatten()[:80].tolist():
            x, y, z = pc[c, n].tolist()
            fx, fy = Ks[c, 0, 0].item(), Ks[c, 1, 1].item()
            limx, limy = 1.3 * 0.5 * W / fx, 1.3 * 0.5 * H / fy
            tx = z * min(limx, max(-limx, x / z))
            ty = z * min(limy, max(-limy, y / z))
            J = np.array([[fx / z, 0, -fx * tx / z ** 2], [0, fy / z, -fy * ty / z ** 2]])
            covb = J @ (R[c].numpy() @ Sigma[n].numpy() @ R[c].numpy().T) @ J.T + eps * np.eye(2)
            lam = np.linalg.eigvalsh(covb)
            disc = (0.5 * (lam[1] - lam[0])) ** 2  # b^2 - det of the blurred covariance
            if disc >= 0.1:
                assert abs(rp[c, n].item() - math.ceil(3 * math.sqrt(lam[1]))) <= 1
                checked += 1
            else:
                bb = 0.5 * (lam[0] + lam[1])
                assert abs(rp[c, n].item() - math.ceil(3 * math.sqrt(bb + math.sqrt(0.1)))) <= 1
    assert checked > 20


def test_projection_culls():
    means = torch.tensor([[0.0, 0.0, -1.0], [0.0, 0.0, 0.005], [500.0, 0.0, 4.0],
                          [0.0, 0.0, 4.0]], dtype=torch.float64)
    quats = torch.tensor([[1.0, 0, 0, 0]] * 4, dtype=torch.float64)
    scales = torch.full((4, 3), 0.05, dtype=torch.float64)
    vm = torch.eye(4, dtype=torch.float64)[None]
    K = torch.tensor([[[100.0, 0, 50], [0, 100.0, 50], [0, 0, 1]]], dtype=torch.float64)
    radii, *_ = G.project_fwd(means, quats, scales, vm, K, 100, 100)
    assert radii[0].tolist()[:3] == [0, 0, 0] and radii[0, 3] > 0
    radii, *_ = G.project_fwd(means, quats, scales, vm, K, 100, 100, radius_clip=1e6)
    assert int(radii.abs().sum()) == 0


def _autograd_projection(means, quats, scales, viewmats, Ks, W, H, eps, radii, seed,
                         covars=None, with_comp=False):
    g = torch.Generator().manual_seed(seed)
    C, N = radii.shape
    live = (radii > 0).double()
    w_m = torch.randn((C, N, 2), generator=g, dtype=torch.float64) * live[..., None]
    w_d = torch.randn((C, N), generator=g, dtype=torch.float64) * live
    w_c = torch.randn((C, N, 3), generator=g, dtype=torch.float64) * live[..., None]
    w_k = torch.randn((C, N), generator=g, dtype=torch.float64) * live if with_comp else None
    leaves = [means.clone().requires_grad_(), viewmats.clone().requires_grad_()]
    if covars is not None:
        leaves.append(covars.clone().requires_grad_())
        Sigma = G.covar_from_6(leaves[2])
    else:
        leaves += [quats.clone().requires_grad_(), scales.clone().requires_grad_()]
        Sigma = G.covar_from_quat_scale(leaves[2], leaves[3])
    pc, m2d, a, b, d, det, conics, comp = G.project_core(leaves[0], Sigma, leaves[1], Ks, W, H, eps)
    L = (w_m * m2d).sum() + (w_d * pc[..., 2]).sum() + (w_c * conics).sum()
    if with_comp:
        L = L + (w_k * comp).sum()
    grads = torch.autograd.grad(L, leaves)
    return grads, (w_m, w_d, w_c, w_k)


@pytest.mark.parametrize("with_comp", [False, True])
def test_projection_backward_vs_autograd(with_comp):
    # spread 3 puts some Gaussians outside 1.3x the fov, exercising the clamp branch
    means, quats, scales, viewmats, Ks = _rand_scene(seed=3, spread=3.0)
    W, H, eps = 128, 96, 0.3
    radii, m2d, depths, conics, comps = G.project_fwd(means, quats, scales, viewmats, Ks, W, H,
                                                      eps2d=eps)
    R, t = viewmats[:, :3, :3], viewmats[:, :3, 3]
    pc = torch.einsum("cij,nj->cni", R, means) + t[:, None]
    clamped = ((pc[..., 0] / pc[..., 2]).abs() > 1.3 * 0.5 * W / Ks[:, None, 0, 0]) & (radii > 0)
    assert clamped.any(), "scene must exercise the fov clamp"
    grads, (w_m, w_d, w_c, w_k) = _autograd_projection(means, quats, scales, viewmats, Ks, W, H,
                                                       eps, radii, seed=4, with_comp=with_comp)
    v_means, v_quats, v_scales, _, v_vm = G.project_bwd(
        means, quats, scales, viewmats, Ks, W, H, eps, radii, conics, w_m, w_d, w_c,
        compensations=comps if with_comp else None, v_compensations=w_k,
        want_viewmats=True)
    # The reference's compensation VJP divides by (comp + 1e-6) (utils.cuh:336), so
    # with compensation it is the exact derivative only to ~1e-6 relative.
    rtol = 1e-5 if with_comp else 1e-7
    for got, ref in ((v_means, grads[0]), (v_quats, grads[2]), (v_scales, grads[3]),
                     (v_vm[:, :3, :], grads[1][:, :3, :])):
        atol = (1e-6 if with_comp else 1e-9) * float(ref.abs().max())
        np.testing.assert_allclose(got.numpy(), ref.numpy(), rtol=rtol, atol=atol)


def test_projection_backward_covars_vs_autograd():
    means, quats, scales, viewmats, Ks = _rand_scene(seed=5)
    covars6 = G.covar_from_quat_scale(quats, scales)[:, [0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2]]
    W, H, eps = 128, 96, 0.3
    radii, m2d, depths, conics, comps = G.project_fwd(means, None, None, viewmats, Ks, W, H,
                                                      eps2d=eps, covars=covars6)
    grads, (w_m, w_d, w_c, _) = _autograd_projection(means, None, None, viewmats, Ks, W, H, eps,
                                                     radii, seed=6, covars=covars6)
    v_means, _, _, v_cov, _ = G.project_bwd(means, None, None, viewmats, Ks, W, H, eps, radii,
                                            conics, w_m, w_d, w_c, covars=covars6)
    np.testing.assert_allclose(v_means.numpy(), grads[0].numpy(), rtol=1e-7, atol=1e-9)
    np.testing.assert_allclose(v_cov.numpy(), grads[2].numpy(), rtol=1e-7, atol=1e-9)


def _real_sh_scipy(l, m, n):
    import scipy.special as sp

    x, y, z = n[:, 0], n[:, 1], n[:, 2]
    polar = np.arccos(np.clip(z, -1, 1))
    azim = np.arctan2(y, x)
    Y = sp.sph_harm_y(l, abs(m), polar, azim)  # complex, Condon-Shortley phase
    if m > 0:
        return math.sqrt(2) * Y.real
    if m < 0:
        return math.sqrt(2) * Y.imag
    return Y.real


def test_sh_basis_matches_scipy():
    n = torch.randn((200, 3), dtype=torch.float64, generator=torch.Generator().manual_seed(7))
    n = n / n.norm(dim=1, keepdim=True)
    Y = G.sh_basis(4, n).numpy()
    for l in range(5):
        for m in range(-l, l + 1):
            k = l * l + l + m
            np.testing.assert_allclose(Y[:, k], _real_sh_scipy(l, m, n.numpy()), atol=1e-12,
                                       err_msg=f"l={l} m={m}")


@pytest.mark.parametrize("degree", [0, 1, 2, 3, 4])
def test_sh_backward_vs_autograd(degree):
    g = torch.Generator().manual_seed(8 + degree)
    dirs = torch.randn((100, 3), dtype=torch.float64, generator=g).requires_grad_()
    coeffs = torch.randn((100, 25, 3), dtype=torch.float64, generator=g).requires_grad_()
    v = torch.randn((100, 3), dtype=torch.float64, generator=g)
    col = G.sh_fwd(degree, dirs, coeffs)
    gd, gc = torch.autograd.grad((col * v).sum(), [dirs, coeffs], allow_unused=True)
    vc, vd = G.sh_bwd(degree, dirs.detach(), coeffs.detach(), v)
    np.testing.assert_allclose(vc.numpy(), gc.numpy(), atol=1e-12)
    if degree == 0:
        assert gd is None or float(gd.abs().max()) == 0.0
        assert float(vd.abs().max()) == 0.0
    else:
        np.testing.assert_allclose(vd.numpy(), gd.numpy(), rtol=1e-9, atol=1e-12)
