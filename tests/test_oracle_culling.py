"""Pins of the block-culling oracle (oracle/culling_ref.py) on the CPU."""
import numpy as np

from oracle import culling_ref as K


def _blocks(seed, n, lo=-4.0, hi=4.0):
    rng = np.random.default_rng(seed)
    mins = rng.uniform(lo, hi, size=(n, 3)).astype(np.float32)
    ext = rng.uniform(0.05, 0.8, size=(n, 3)).astype(np.float32)
    return np.concatenate([mins, mins + ext], axis=1)


def test_subset_equals_full_reference_case():
    # tests/test_bounds_generation.py:140-170: identity view and projection
    b = _blocks(7, 128)
    c, r = K.spheres(b)
    p = K.planes(np.eye(4, dtype=np.float32), np.eye(4, dtype=np.float32))
    full = K.cull(c, r, p)
    assert K.cull(c, r, p, block_ids=np.arange(128)) == full
    assert K.cull(c, r, p, block_ids=sorted(set(range(128)))) == full


def test_identity_frustum_closed_form():
    # identity VP: planes are x>=-1, x<=1, ... so a sphere is kept iff every
    # |c_i| <= 1 + r (exactly, away from float32 ties)
    b = _blocks(3, 5000)
    c, r = K.spheres(b)
    p = K.planes(np.eye(4, dtype=np.float32), np.eye(4, dtype=np.float32))
    np.testing.assert_allclose(np.abs(p[:, :3]).sum(axis=1), 1.0)
    got = set(K.cull(c, r, p))
    margin = (1.0 + r.astype(np.float64))[:, None] - np.abs(c.astype(np.float64))
    want = set(np.nonzero((margin >= 0).all(axis=1))[0].tolist())
    tie = np.abs(margin).min(axis=1) < 1e-6
    assert {i for i in got ^ want if not tie[i]} == set()


def test_radii_and_centres_closed_form():
    b = np.float32([[0, 0, 0, 2, 2, 2], [-1, 3, 5, 1, 3, 9]])
    c, r = K.spheres(b)
    np.testing.assert_array_equal(c, np.float32([[1, 1, 1], [0, 3, 7]]))
    np.testing.assert_allclose(r, np.float32([np.sqrt(12) / 2 * 1.15, np.sqrt(20) / 2 * 1.15]),
                               rtol=1e-6)


def test_perspective_planes_and_float64_agreement():
    # OpenGL perspective, 90 degree fov, aspect 1: the side planes are
    # x = +-(-z) and y = +-(-z) (normals (1,0,-1)/sqrt2 ...), near/far along -z
    n_, f_ = 0.5, 50.0
    proj = np.float32([[1, 0, 0, 0], [0, 1, 0, 0],
                       [0, 0, -(f_ + n_) / (f_ - n_), -2 * f_ * n_ / (f_ - n_)], [0, 0, -1, 0]])
    p = K.planes(np.eye(4, dtype=np.float32), proj)
    s = np.float32(1 / np.sqrt(2))
    np.testing.assert_allclose(p[0], [s, 0, -s, 0], atol=1e-6)
    np.testing.assert_allclose(p[1], [-s, 0, -s, 0], atol=1e-6)
    np.testing.assert_allclose(p[4], [0, 0, -1, -n_], atol=1e-5)
    np.testing.assert_allclose(p[5], [0, 0, 1, f_], atol=1e-4)
    b = _blocks(11, 20000, lo=-40.0, hi=40.0)
    c, r = K.spheres(b)
    got = set(K.cull(c, r, p))
    sd = np.concatenate([c, np.ones((len(c), 1))], axis=1).astype(np.float64) @ \
        p.astype(np.float64).T
    margin = sd + r.astype(np.float64)[:, None]
    want = set(np.nonzero((margin >= 0).all(axis=1))[0].tolist())
    tie = np.abs(margin).min(axis=1) < 1e-4
    assert len(got) > 100
    assert {i for i in got ^ want if not tie[i]} == set()


def test_legacy_cone_closed_form():
    """The legacy cone + distance test on blocks whose answer is fixed by
    geometry: camera at the origin looking down +z (view row 2 = +z), reach
    50 (no scene radius): ahead within reach visible, ahead beyond it not,
    straight behind not, at the camera visible, and across the cosine -0.3
    boundary of a known direction."""
    view = np.eye(4, dtype=np.float32)
    cam = np.zeros(3, dtype=np.float32)
    s = np.sqrt(1.0 - 0.31 ** 2)
    centers = np.array([[0, 0, 10], [0, 0, 49], [0, 0, 51], [0, 0, -10], [0, 0, 0],
                        [s * 20, 0, -0.29 * 20], [s * 20, 0, -0.31 * 20], [40, 0, 0]],
                       dtype=np.float32)
    assert K.cone(centers, cam, view) == [0, 1, 4, 5, 7]
    # the reach scales with the margin and follows min(scene_radius / 2, 100)
    assert K.cone(centers, cam, view, margin=1.1) == [0, 1, 2, 4, 5, 7]
    assert K.cone(centers, cam, view, scene_radius=30.0) == [0, 4]
    assert K.cone(centers, cam, view, scene_radius=1000.0) == [0, 1, 2, 4, 5, 7]
