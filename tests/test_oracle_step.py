"""Pin for the composed step oracle (oracle/step_ref.py): its compact row
gradients equal central finite differences of its own float64 loss summed over
the cameras, through activations, SH clamp, projection and compositing."""
import numpy as np
import pytest
import torch

from oracle import raster_ref as R
from oracle import ssim_ref as S
from oracle import step_ref as SR
from tidegs_amd import scenes


def _tiny_scene():
    sc = scenes.small(seed=11, n=40, n_cams=2, W=40, H=28, log_scale_mu=-1.8)
    p = sc.params.double()
    p[:, 10] = p[:, 10] * 0.5 - 0.5   # moderate opacities keep alpha away from the clamps
    return sc, p


def _loss(p, sc):
    touched, grads, losses, _, _ = SR.batch_grads(p, sc.viewmats, sc.Ks, sc.gt, sc.width,
                                                  sc.height, raster_dtype=np.float64)
    return sum(l for l in losses if l is not None)


def test_step_oracle_matches_finite_differences():
    sc, p = _tiny_scene()
    touched, grads, losses, _, filters = SR.batch_grads(p, sc.viewmats, sc.Ks, sc.gt, sc.width,
                                                        sc.height, raster_dtype=np.float64)
    assert touched.numel() >= 20
    rng = np.random.default_rng(0)
    rows = rng.choice(touched.numel(), size=6, replace=False)
    cols = [0, 1, 2, 3, 5, 6, 8, 10, 11, 13, 20, 40]
    h = 1e-6
    fd, an = [], []
    for t in rows:
        r = int(touched[t])
        for c in cols:
            saved = float(p[r, c])
            p[r, c] = saved + h
            lp = _loss(p, sc)
            p[r, c] = saved - h
            lm = _loss(p, sc)
            p[r, c] = saved
            fd.append((lp - lm) / (2 * h))
            an.append(float(grads[t, c]))
    fd, an = np.array(fd), np.array(an)
    err = np.linalg.norm(fd - an) / np.linalg.norm(fd)
    assert err < 1e-5, err


# ---------------------------------------------------------------------------
# packed filters (fully_fused_projection_packed_fwd.cu:50-131)
# ---------------------------------------------------------------------------
def _brute_force_keep(row, vm, K, W, H, eps2d=0.3, near=0.01, far=1e10, radius_clip=0.0):
    """One (camera, row) decision of the packed rule from the eigenvalues of
    the blurred 2D covariance (numpy, float64, scalar code): in front of the
    near plane and behind the far plane, positive determinant, radius
    ceil(3 sqrt(max(lambda_max, (l1 + l2) / 2 + sqrt(0.1)))) above the clip,
    and the radius disc overlapping the image.  Returns (keep, radius, mean)."""
    import math

    from scipy.spatial.transform import Rotation

    row = np.asarray(row, np.float64)
    q = row[6:10]
    nq = np.linalg.norm(q)
    if not nq > 0:
        return False, None, None
    Rq = Rotation.from_quat([q[1], q[2], q[3], q[0]]).as_matrix()  # scipy: (x, y, z, w)
    S = np.diag(np.exp(row[3:6]))
    Sigma = Rq @ S @ S @ Rq.T
    R, t = np.asarray(vm[:3, :3], np.float64), np.asarray(vm[:3, 3], np.float64)
    pc = R @ row[0:3] + t
    x, y, z = pc
    if z < near or z > far:
        return False, None, None
    fx, fy, cx, cy = float(K[0, 0]), float(K[1, 1]), float(K[0, 2]), float(K[1, 2])
    limx, limy = 1.3 * 0.5 * W / fx, 1.3 * 0.5 * H / fy
    tx = z * min(limx, max(-limx, x / z))
    ty = z * min(limy, max(-limy, y / z))
    J = np.array([[fx / z, 0, -fx * tx / z ** 2], [0, fy / z, -fy * ty / z ** 2]])
    cov = J @ (R @ Sigma @ R.T) @ J.T + eps2d * np.eye(2)
    lam = np.linalg.eigvalsh(cov)
    if not lam[0] * lam[1] > 0:
        return False, None, None
    v = max(lam[1], 0.5 * (lam[0] + lam[1]) + math.sqrt(0.1))
    r = math.ceil(3.0 * math.sqrt(v))
    if r <= radius_clip:
        return False, r, None
    mx, my = fx * x / z + cx, fy * y / z + cy
    if mx + r <= 0 or mx - r >= W or my + r <= 0 or my - r >= H:
        return False, r, (mx, my)
    return True, r, (mx, my)


def _edge_case_table(seed=3):
    """Rows around one camera (identity pose, 160x120, f = 150) that hit every
    branch of the packed rule: behind the camera, inside the near plane,
    beyond a far plane of 40, a zero quaternion, tiny Gaussians that only the
    radius clip removes, and many rows straddling each image border."""
    g = torch.Generator().manual_seed(seed)
    W, H, f = 160, 120, 150.0
    rows = []

    def row(x, y, z, log_s=-2.5, q=(1.0, 0.0, 0.0, 0.0)):
        r = torch.zeros(59, dtype=torch.float64)
        r[0:3] = torch.tensor([x, y, z], dtype=torch.float64)
        r[3:6] = log_s
        r[6:10] = torch.tensor(q, dtype=torch.float64)
        return r

    rows += [row(0, 0, -1.0), row(0, 0, 0.005), row(0, 0, 55.0, log_s=0.0),
             row(0.1, 0.1, 3.0, q=(0, 0, 0, 0))]
    # tiny: the blur alone gives ceil(3 sqrt(0.3 + sqrt(0.1))) = 3, cut by a clip of 3
    rows += [row(0.2, -0.1, 4.0, log_s=-9.0), row(-0.3, 0.2, 6.0, log_s=-8.0)]
    # border straddlers: means just outside / inside each edge at several depths
    for _ in range(400):
        z = float(torch.rand((), generator=g)) * 8 + 1
        edge = int(torch.randint(4, (), generator=g))
        off = (float(torch.rand((), generator=g)) - 0.5) * 12.0  # pixels across the edge
        u = float(torch.rand((), generator=g)) * (W if edge < 2 else H)
        px = [-off, W + off, u, u][edge]
        py = [u, u, -off, H + off][edge]
        x, y = (px - W / 2) * z / f, (py - H / 2) * z / f
        ls = float(torch.randn((), generator=g)) * 0.7 - 3.0
        q = torch.randn(4, generator=g, dtype=torch.float64)
        rows.append(row(x, y, z, log_s=ls, q=tuple((q / q.norm()).tolist())))
    for _ in range(300):  # ordinary rows, some far away
        z = float(torch.rand((), generator=g)) * 60 + 0.5
        x, y = (torch.rand(2, generator=g, dtype=torch.float64) - 0.5) * z * 1.6
        q = torch.randn(4, generator=g, dtype=torch.float64)
        rows.append(row(float(x), float(y), z, log_s=float(torch.randn((), generator=g)) - 3.0,
                        q=tuple((q / q.norm()).tolist())))
    p = torch.stack(rows)
    vm = torch.eye(4, dtype=torch.float64)[None]
    K = torch.tensor([[[f, 0, W / 2], [0, f, H / 2], [0, 0, 1]]], dtype=torch.float64)
    return p, vm, K, W, H


@pytest.mark.parametrize("far,radius_clip", [(1e10, 0.0), (40.0, 0.0), (1e10, 3.0)])
def test_packed_filters_match_brute_force(far, radius_clip):
    """packed_filters equals the eigenvalue restatement of the packed rule on
    every row except where the decision sits within rounding of a boundary
    (flagged by packed_filter_ambiguous, which the brute force also respects:
    no flagged row may be needed to explain more than a handful of the 700)."""
    p, vm, K, W, H = _edge_case_table()
    got = SR.packed_filters(p, vm, K, W, H, far=far, radius_clip=radius_clip)[0].numpy()
    amb = SR.packed_filter_ambiguous(p, vm, K, W, H, far=far, radius_clip=radius_clip)[0].numpy()
    keep = np.array([_brute_force_keep(r.numpy(), vm[0].numpy(), K[0].numpy(), W, H, far=far,
                                       radius_clip=radius_clip)[0] for r in p])
    mine = np.zeros(p.shape[0], bool)
    mine[got] = True
    diff = np.nonzero(mine != keep)[0]
    assert np.all(amb[diff]), f"rows {diff[~amb[diff]]} differ off every boundary"
    assert diff.size <= 3 and amb.sum() <= 20
    # the explicit cases: behind, inside the near plane, zero quaternion
    assert not mine[0] and not mine[1] and not mine[3]
    assert mine[2] == (far > 55.0)
    if radius_clip > 0:
        assert not mine[4] and not mine[5]
    # the border straddlers take both decisions
    assert 50 < mine[6:406].sum() < 350


def test_packed_filter_ambiguity_covers_float32_rounding():
    """The float32 evaluation of the packed rule (torch, its own operation
    order) differs from the float64 one only on entries that
    packed_filter_ambiguous flags, and those are rare: the GPU's float32
    filters are then held exactly to the oracle's off that set."""
    sc = scenes.cfg3(seed=0, n=150_000, n_cams=16, with_gt=False)
    vm, K = sc.viewmats[[0, 9]], sc.Ks[[0, 9]]
    f64 = SR.packed_filters(sc.params, vm, K, sc.width, sc.height)
    f32 = SR.packed_filters(sc.params, vm, K, sc.width, sc.height, dtype=torch.float32)
    amb = SR.packed_filter_ambiguous(sc.params, vm, K, sc.width, sc.height)
    n_diff = 0
    for c in range(2):
        a = np.zeros(sc.n, bool)
        b = np.zeros(sc.n, bool)
        a[f64[c].numpy()] = True
        b[f32[c].numpy()] = True
        d = np.nonzero(a != b)[0]
        assert np.all(amb[c].numpy()[d]), d[~amb[c].numpy()[d]]
        n_diff += d.size
    frac = float(amb.double().mean())
    print(f"  float32 vs float64 filter differences: {n_diff}; ambiguous fraction {frac:.2e}")
    assert frac < 2e-3


def test_isect_inputs_override_reproduces_default():
    """batch_grads with the intersection step fed its own float32 (mean,
    radius, depth) values -- what the GPU parity tests pass in, with the GPU's
    values -- reproduces the default run exactly; render_projection gives
    those values."""
    sc, p = _tiny_scene()
    base = SR.batch_grads(p, sc.viewmats, sc.Ks, sc.gt, sc.width, sc.height)
    inputs = []
    for c, rows in enumerate(base[4]):
        radii, m2d, depths, rr = SR.render_projection(p, rows, sc.viewmats[c], sc.Ks[c],
                                                      sc.width, sc.height)
        assert torch.equal(radii, torch.where(radii > 0, torch.ceil(rr), 0).to(radii.dtype))
        inputs.append((m2d.float().numpy(), radii.numpy(), depths.float().numpy()))
    again = SR.batch_grads(p, sc.viewmats, sc.Ks, sc.gt, sc.width, sc.height,
                           filters=base[4], isect_inputs=inputs)
    assert torch.equal(base[0], again[0]) and torch.equal(base[1], again[1])
    assert base[2] == again[2]


def test_batch_row_grads_from_splat_grads_match_batch_grads():
    """batch_row_grads (row gradients from given splat gradients, the oracle
    half the GPU parity tests feed with the GPU's splat gradients) equals
    batch_grads when given the oracle's own splat gradients."""
    sc, p = _tiny_scene()
    W, H = sc.width, sc.height
    touched, grads, _, _, filters = SR.batch_grads(p, sc.viewmats, sc.Ks, sc.gt, W, H)
    per_cam = []
    for c, rows in enumerate(filters):
        f = SR._render_entries(p, rows, sc.viewmats[c], sc.Ks[c], W, H, 3, torch.float64)
        _, ids, flat = R.isect_tiles(f.m2d.float().numpy(), f.radii.numpy(),
                                     f.depths.float().numpy(), 16, -(-W // 16), -(-H // 16))
        offs = R.isect_offset_encode(ids, 1, -(-W // 16), -(-H // 16))
        splat = (f.m2d.numpy().reshape(-1, 2), f.conics[0].numpy(), f.colors.numpy(),
                 f.opac.numpy())
        img, alphas, last = R.rasterize_fwd(*splat, W, H, 16, offs, flat)
        _, v = S.tide_loss(img[0].transpose(2, 0, 1), sc.gt[c].numpy(), dtype=np.float64)
        v = np.ascontiguousarray(v.transpose(1, 2, 0))[None]
        per_cam.append(R.rasterize_bwd(*splat, W, H, 16, offs, flat, alphas, last, v)[:4])
    t2, g2 = SR.batch_row_grads(p, sc.viewmats, sc.Ks, W, H, filters, per_cam)
    assert torch.equal(touched, t2)
    assert torch.allclose(grads, g2, rtol=1e-12, atol=1e-18)
