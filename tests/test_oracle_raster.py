"""Pins for the CPU oracle of tile intersection and rasterization.

* isect: a per-entry Python loop with np.float32 scalars and Python's sorted()
  on (camera, tile, depth bits, flatten id) tuples, decoded from the keys.
* offsets: a literal restatement of the per-intersection kernel loop.
* raster forward: a tile-free per-pixel compositor (depth-sorted list of the
  Gaussians whose tile rectangle covers the pixel's tile).
* raster backward: central finite differences of the float64 forward.
"""
import numpy as np
import pytest

from oracle import raster_ref as R


def _scene(seed, C=2, N=60, W=40, H=24, tile=16, depth_ties=False):
    rng = np.random.default_rng(seed)
    means2d = rng.uniform([-8, -8], [W + 8, H + 8], size=(C, N, 2)).astype(np.float32)
    radii = rng.integers(0, 14, size=(C, N)).astype(np.int32)
    radii[:, :5] = 0
    depths = rng.uniform(0.5, 9.0, size=(C, N)).astype(np.float32)
    if depth_ties:
        depths[:, 10:20] = depths[:, 10:11]
    tw, th = -(-W // tile), -(-H // tile)
    return means2d, radii, depths, tw, th


def _brute_isect(means2d, radii, depths, tile, tw, th):
    C, N = radii.shape
    tile_bits = int(tw * th).bit_length()
    rows = []
    counts = np.zeros((C, N), np.int32)
    for c in range(C):
        for n in range(N):
            r = int(radii[c, n])
            if r <= 0:
                continue
            ts = np.float32(tile)
            tr = np.float32(r) / ts
            tx = np.float32(means2d[c, n, 0]) / ts
            ty = np.float32(means2d[c, n, 1]) / ts
            x0 = int(min(max(0, np.floor(np.float32(tx - tr))), tw))
            y0 = int(min(max(0, np.floor(np.float32(ty - tr))), th))
            x1 = int(min(max(0, np.ceil(np.float32(tx + tr))), tw))
            y1 = int(min(max(0, np.ceil(np.float32(ty + tr))), th))
            for yy in range(y0, y1):
                for xx in range(x0, x1):
                    dbits = int(np.float32(depths[c, n]).view(np.uint32))
                    rows.append((c, yy * tw + xx, dbits, c * N + n))
                    counts[c, n] += 1
    rows.sort()
    return counts, rows, tile_bits


@pytest.mark.parametrize("seed,ties", [(0, False), (1, True), (2, False)])
def test_isect_matches_bruteforce(seed, ties):
    means2d, radii, depths, tw, th = _scene(seed, depth_ties=ties)
    tiles, ids, flat = R.isect_tiles(means2d, radii, depths, 16, tw, th)
    counts, rows, tile_bits = _brute_isect(means2d, radii, depths, 16, tw, th)
    np.testing.assert_array_equal(tiles, counts)
    assert len(rows) == ids.size
    dec = [(int(k) >> (32 + tile_bits), (int(k) >> 32) & ((1 << tile_bits) - 1),
            int(k) & 0xFFFFFFFF, int(f)) for k, f in zip(ids, flat)]
    assert dec == rows


def _kernel_offsets(ids, C, tw, th):
    n_tiles = tw * th
    bits = int(n_tiles).bit_length()
    total = C * n_tiles
    out = np.full(total, -7, np.int64)
    n = ids.size

    def bucket(k):
        hi = int(k) >> 32
        return (hi >> bits) * n_tiles + (hi & ((1 << bits) - 1))

    for idx in range(n):
        cur = bucket(ids[idx])
        if idx == 0:
            out[: cur + 1] = 0
        if idx == n - 1:
            out[cur + 1:] = n
        if idx > 0:
            prev = bucket(ids[idx - 1])
            if prev != cur:
                out[prev + 1: cur + 1] = idx
    return out.reshape(C, th, tw)


def test_offset_encode_matches_kernel_loop():
    means2d, radii, depths, tw, th = _scene(3)
    _, ids, _ = R.isect_tiles(means2d, radii, depths, 16, tw, th)
    np.testing.assert_array_equal(R.isect_offset_encode(ids, 2, tw, th),
                                  _kernel_offsets(ids, 2, tw, th))
    # leading and trailing empty tiles
    sub = ids[(ids >> 32) == (ids[ids.size // 2] >> 32)]
    np.testing.assert_array_equal(R.isect_offset_encode(sub, 2, tw, th),
                                  _kernel_offsets(sub, 2, tw, th))


def _splats(seed, N=45, W=40, H=24, C=1, D=3):
    rng = np.random.default_rng(seed)
    m = rng.uniform([0, 0], [W, H], size=(C, N, 2))
    # SPD conics from random 2x2 covariances (sigma 1.5..5 px)
    L = rng.normal(size=(C, N, 2, 2)) * 1.2
    cov = L @ np.swapaxes(L, -1, -2) + np.eye(2) * 2.0
    inv = np.linalg.inv(cov)
    con = np.stack([inv[..., 0, 0], inv[..., 0, 1], inv[..., 1, 1]], -1)
    col = rng.uniform(0, 1, size=(C, N, D))
    op = rng.uniform(0.05, 0.7, size=(C, N))
    dep = rng.uniform(1, 5, size=(C, N)).astype(np.float32)
    radii = np.ceil(3 * np.sqrt(np.linalg.eigvalsh(cov)[..., -1])).astype(np.int32)
    return m, con, col, op, dep, radii


def _tile_free_composite(m, con, col, op, dep, radii, W, H, tile, bg=None):
    C, N, D = col.shape
    tw = -(-W // tile)
    out = np.zeros((C, H, W, D))
    alp = np.zeros((C, H, W))
    last = np.zeros((C, H, W), np.int64)
    for c in range(C):
        for i in range(H):
            for j in range(W):
                t = (i // tile) * tw + (j // tile)
                ty_, tx_ = divmod(t, tw)
                cand = []
                for n in range(N):
                    r = radii[c, n]
                    if r <= 0:
                        continue
                    x0 = max(0, np.floor(np.float32(m[c, n, 0] / tile) - np.float32(r / tile)))
                    x1 = np.ceil(np.float32(m[c, n, 0] / tile) + np.float32(r / tile))
                    y0 = max(0, np.floor(np.float32(m[c, n, 1] / tile) - np.float32(r / tile)))
                    y1 = np.ceil(np.float32(m[c, n, 1] / tile) + np.float32(r / tile))
                    if x0 <= tx_ < x1 and y0 <= ty_ < y1:
                        cand.append((int(np.float32(dep[c, n]).view(np.uint32)), n))
                cand.sort()
                T, acc = 1.0, np.zeros(D)
                px, py = j + 0.5, i + 0.5
                for rank, (_, n) in enumerate(cand):
                    dx, dy = m[c, n, 0] - px, m[c, n, 1] - py
                    a, b, cc = con[c, n]
                    s = 0.5 * (a * dx * dx + cc * dy * dy) + b * dx * dy
                    al = min(0.999, op[c, n] * np.exp(-s))
                    if s < 0 or al < 1 / 255:
                        continue
                    nt = T * (1 - al)
                    if nt <= 1e-4:
                        break
                    acc += col[c, n] * al * T
                    last[c, i, j] = rank
                    T = nt
                alp[c, i, j] = 1 - T
                out[c, i, j] = acc + (T * bg[c] if bg is not None else 0)
    return out, alp


def _oracle_forward(m, con, col, op, dep, radii, W, H, tile, bg=None, dtype=np.float64):
    C = m.shape[0]
    tw, th = -(-W // tile), -(-H // tile)
    _, ids, flat = R.isect_tiles(m.astype(np.float32), radii, dep, tile, tw, th)
    offs = R.isect_offset_encode(ids, C, tw, th)
    colors, alphas, last = R.rasterize_fwd(m.reshape(-1, 2), con.reshape(-1, 3),
                                           col.reshape(-1, col.shape[-1]), op.reshape(-1), W, H,
                                           tile, offs, flat, backgrounds=bg, dtype=dtype)
    return colors, alphas, last, offs, flat


@pytest.mark.parametrize("use_bg", [False, True])
def test_raster_forward_matches_tile_free(use_bg):
    W, H, tile = 40, 24, 16
    m, con, col, op, dep, radii = _splats(5, W=W, H=H, C=2)
    m = m.astype(np.float32).astype(np.float64)
    bg = np.array([[0.2, 0.5, 0.9], [0.1, 0.1, 0.3]]) if use_bg else None
    colors, alphas, last, _, _ = _oracle_forward(m, con, col, op, dep, radii, W, H, tile, bg=bg)
    ref_c, ref_a = _tile_free_composite(m, con, col, op, dep, radii, W, H, tile, bg=bg)
    np.testing.assert_allclose(colors, ref_c, atol=1e-12)
    np.testing.assert_allclose(alphas, ref_a, atol=1e-12)


def test_raster_backward_matches_finite_differences():
    W, H, tile = 32, 20, 16
    m, con, col, op, dep, radii = _splats(9, N=25, W=W, H=H, C=1)
    m = m.astype(np.float32).astype(np.float64)
    rng = np.random.default_rng(10)
    wc = rng.normal(size=(1, H, W, 3))
    wa = rng.normal(size=(1, H, W))
    bg = np.array([[0.3, 0.6, 0.2]])
    tw, th = -(-W // tile), -(-H // tile)
    _, ids, flat = R.isect_tiles(m.astype(np.float32), radii, dep, tile, tw, th)
    offs = R.isect_offset_encode(ids, 1, tw, th)

    def loss(mm, cc, cl, oo):
        c, a, _ = R.rasterize_fwd(mm.reshape(-1, 2), cc.reshape(-1, 3), cl.reshape(-1, 3),
                                  oo.reshape(-1), W, H, tile, offs, flat, backgrounds=bg,
                                  dtype=np.float64)
        return float((c * wc).sum() + (a * wa).sum())

    c0, a0, last = R.rasterize_fwd(m.reshape(-1, 2), con.reshape(-1, 3), col.reshape(-1, 3),
                                   op.reshape(-1), W, H, tile, offs, flat, backgrounds=bg,
                                   dtype=np.float64)
    vm, vc, vcol, vo, _ = R.rasterize_bwd(m.reshape(-1, 2), con.reshape(-1, 3), col.reshape(-1, 3),
                                          op.reshape(-1), W, H, tile, offs, flat, a0, last, wc,
                                          v_alphas=wa, backgrounds=bg, dtype=np.float64)
    h = 1e-6
    params = [("m", m, vm.reshape(m.shape)), ("con", con, vc.reshape(con.shape)),
              ("col", col, vcol.reshape(col.shape)), ("op", op, vo.reshape(op.shape))]
    for name, arr, grad in params:
        fd = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            saved = arr[idx]
            arr[idx] = saved + h
            lp = loss(m, con, col, op)
            arr[idx] = saved - h
            lm = loss(m, con, col, op)
            arr[idx] = saved
            fd[idx] = (lp - lm) / (2 * h)
        err = np.linalg.norm(fd - grad) / max(np.linalg.norm(fd), 1e-30)
        assert err < 1e-5, (name, err)


def _one_tile(means2d, conics, opac):
    """One 16x16 tile holding every Gaussian, front to back in input order."""
    n = len(opac)
    return (np.asarray(means2d, np.float64), np.asarray(conics, np.float64),
            np.asarray(opac, np.float64), np.zeros((1, 1, 1), np.int32),
            np.arange(n, dtype=np.int32))


def test_decision_flips_identical_sets():
    """The same parameters on both sides flip nothing and flag nothing."""
    m, q, o, offs, flat = _one_tile([[5.3, 7.1], [9.0, 4.2], [8.0, 8.0]],
                                    [[0.5, 0.1, 0.7], [0.2, 0.0, 0.3], [1.0, 0.0, 1.0]],
                                    [0.6, 0.9, 0.4])
    flip, flag = R.decision_flips((m, q, o), (m, q, o), 16, 16, 16, offs, flat)
    assert not flip.any() and not flag.any()
    # a marked pixel flags the Gaussians composited there: at pixel (7, 7)
    # (centre (7.5, 7.5)) alpha = 0.6 exp(-1.354), 0.9 exp(-1.858) and
    # 0.4 exp(-0.25), all above 1/255
    mark = np.zeros((1, 16, 16), bool)
    mark[0, 7, 7] = True
    flip, flag = R.decision_flips((m, q, o), (m, q, o), 16, 16, 16, offs, flat,
                                  dtype=np.float64, mark=mark)
    assert not flip.any()
    np.testing.assert_array_equal(flag, [True, True, True])


def test_decision_flips_alpha_ring():
    """An isotropic Gaussian (conic (1, 0, 1)) at a pixel centre passes the
    alpha test where o exp(-r^2 / 2) >= 1/255, i.e. r^2 <= 2 ln(255 o): raising
    its opacity from o_a to o_b adds exactly the pixels with r^2 in
    (2 ln(255 o_a), 2 ln(255 o_b)] (values chosen away from pixel distances),
    and flags that Gaussian only; a second Gaussian far from the ring is not
    flagged."""
    c = (7.3, 8.6)
    o_a, o_b = 0.04, 0.3
    m = [list(c), [1.5, 1.5]]
    q = [[1.0, 0.0, 1.0], [4.0, 0.0, 4.0]]
    _, _, _, offs, flat = _one_tile(m, q, [o_a, 0.9])
    flip, flag = R.decision_flips((m, q, [o_a, 0.9]), (m, q, [o_b, 0.9]), 16, 16, 16,
                                  offs, flat, dtype=np.float64)
    j, i = np.meshgrid(np.arange(16) + 0.5, np.arange(16) + 0.5)
    r2 = (j - c[0]) ** 2 + (i - c[1]) ** 2
    lo, hi = 2 * np.log(255 * o_a), 2 * np.log(255 * o_b)
    assert np.abs(r2 - lo).min() > 1e-3 and np.abs(r2 - hi).min() > 1e-3
    want = (r2 > lo) & (r2 <= hi)
    assert want.sum() > 10
    np.testing.assert_array_equal(flip[0], want)
    np.testing.assert_array_equal(flag, [True, False])


def test_decision_flips_transmittance_stop():
    """Five Gaussians centred on pixel (8, 8) (alpha = opacity there): with
    opacities 0.95 the transmittance after three is 1.25e-4 and the fourth
    stops the pixel (6.25e-6 <= 1e-4), so three composite; with the third at
    0.5 and the fourth at 0.9 it is 1.25e-3 after three and 1.25e-4 after
    four, so the fifth stops it and four composite.  The centre pixel's decisions differ, and all
    four Gaussians composited under the second set are flagged; a pixel far
    from the stack (where no Gaussian passes the alpha test) is not flipped."""
    c = [8.5, 8.5]
    m = [c] * 5
    q = [[8.0, 0.0, 8.0]] * 5
    a = [0.95] * 5
    b = [0.95, 0.95, 0.5, 0.9, 0.95]
    _, _, _, offs, flat = _one_tile(m, q, a)
    flip, flag = R.decision_flips((m, q, a), (m, q, b), 16, 16, 16, offs, flat,
                                  dtype=np.float64)
    assert flip[0, 8, 8]
    assert not flip[0, 0, 0] and not flip[0, 15, 15]
    np.testing.assert_array_equal(flag, [True, True, True, True, False])
