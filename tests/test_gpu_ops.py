"""GPU parity of the gsplat / clm_kernels drop-in ops against the CPU oracle.

Tolerances: integer/index outputs bit-exact (isect ids, flatten ids,
offsets, sort); floating-point gradients within relative L2 <= 1e-4 of the
oracle (atomics reorder sums), forward values within
1e-4 relative.  Radii may differ by +-1 on a small fraction of Gaussians, as
gsplat's own test allows (test_basic.py:219-221).
"""
import numpy as np
import pytest
import torch

from oracle import gsplat_ref as G
from oracle import raster_ref as R
from oracle import ssim_ref as S
from tests.gpu_util import announce, rel_l2, to_np
from tidegs_amd import gsplat_ops as ops
from tidegs_amd import scenes
from tidegs_amd.clm_ops import FusedSSIMMap, fused_ssim

pytestmark = pytest.mark.gpu


def _proj_inputs(seed=0, n=3000, C=3, W=96, H=64):
    sc = scenes.small(seed=seed, n=n, n_cams=C, W=W, H=H)
    means, quats, scales, opac, sh = scenes.activations(sc.params)
    return sc, means.contiguous(), quats.contiguous(), scales.contiguous()


@pytest.mark.parametrize("calc_comp", [False, True])
def test_projection_fwd_bwd(gpu, calc_comp):
    announce(f"projection calc_comp={calc_comp}")
    sc, means, quats, scales = _proj_inputs()
    W, H = sc.width, sc.height
    dm = means.to(gpu).requires_grad_()
    dq = quats.to(gpu).requires_grad_()
    ds = scales.to(gpu).requires_grad_()
    dv = sc.viewmats.to(gpu).requires_grad_()
    radii, m2d, depths, conics, comps = ops.fully_fused_projection(
        dm, None, dq, ds, dv, sc.Ks.to(gpu), W, H, calc_compensations=calc_comp)
    o_radii, o_m2d, o_depths, o_conics, o_comps = G.project_fwd(
        means, quats, scales, sc.viewmats, sc.Ks, W, H)
    r_gpu, r_ref = to_np(radii), to_np(o_radii)
    assert (r_ref > 0).sum() > 1000
    same = r_gpu == r_ref
    assert same.mean() > 0.998, same.mean()
    assert np.abs(r_gpu - r_ref).max() <= 1 or same.mean() > 0.999
    both = (r_gpu > 0) & (r_ref > 0)
    assert rel_l2(to_np(m2d)[both], to_np(o_m2d)[both]) < 1e-6
    assert rel_l2(to_np(depths)[both], to_np(o_depths)[both]) < 1e-6
    assert rel_l2(to_np(conics)[both], to_np(o_conics)[both]) < 1e-5
    if calc_comp:
        assert rel_l2(to_np(comps)[both], to_np(o_comps)[both]) < 1e-5
    # backward with cotangents on entries live in both
    g = torch.Generator().manual_seed(1)
    live = torch.from_numpy(both)
    w_m = torch.randn(m2d.shape, generator=g) * live[..., None]
    w_d = torch.randn(depths.shape, generator=g) * live
    w_c = torch.randn(conics.shape, generator=g) * live[..., None]
    w_k = torch.randn(depths.shape, generator=g) * live if calc_comp else None
    L = (m2d * w_m.to(gpu)).sum() + (depths * w_d.to(gpu)).sum() + (conics * w_c.to(gpu)).sum()
    if calc_comp:
        L = L + (comps * w_k.to(gpu)).sum()
    L.backward()
    rad_both = torch.from_numpy(np.where(both, r_ref, 0))
    v_means, v_quats, v_scales, _, v_vm = G.project_bwd(
        means, quats, scales, sc.viewmats, sc.Ks, W, H, 0.3, rad_both, o_conics, w_m, w_d, w_c,
        compensations=o_comps if calc_comp else None, v_compensations=w_k, want_viewmats=True)
    assert rel_l2(to_np(dm.grad), v_means) < 1e-4
    assert rel_l2(to_np(dq.grad), v_quats) < 1e-4
    assert rel_l2(to_np(ds.grad), v_scales) < 1e-4
    assert rel_l2(to_np(dv.grad)[:, :3], to_np(v_vm)[:, :3]) < 1e-4


@pytest.mark.parametrize("calc_comp,sparse", [(False, False), (True, False), (False, True)])
def test_projection_packed(gpu, calc_comp, sparse):
    """fully_fused_projection(packed=True): entries camera-major and Gaussian-
    ascending, exactly the oracle's survivors under the packed radius rule;
    values as the dense projection; VJPs summed over a Gaussian's cameras (or
    per entry as COO tensors with sparse_grad)."""
    announce(f"projection packed calc_comp={calc_comp} sparse_grad={sparse}")
    sc, means, quats, scales = _proj_inputs(seed=4)
    W, H = sc.width, sc.height
    C = sc.n_cams
    dm = means.to(gpu).requires_grad_()
    dq = quats.to(gpu).requires_grad_()
    ds = scales.to(gpu).requires_grad_()
    cam_ids, g_ids, radii, m2d, depths, conics, comps = ops.fully_fused_projection(
        dm, None, dq, ds, sc.viewmats.to(gpu), sc.Ks.to(gpu), W, H, packed=True,
        sparse_grad=sparse, calc_compensations=calc_comp)
    o = G.project_fwd(means, quats, scales, sc.viewmats, sc.Ks, W, H, packed=True)
    o_radii = to_np(o[0])
    oc, on = np.nonzero(o_radii > 0)  # camera-major, ascending
    np.testing.assert_array_equal(to_np(cam_ids), oc)
    np.testing.assert_array_equal(to_np(g_ids), on)
    assert cam_ids.dtype == torch.int64 and radii.dtype == torch.int32 and oc.size > 1000
    r = to_np(radii)
    assert np.abs(r - o_radii[oc, on]).max() <= 1 and (r == o_radii[oc, on]).mean() > 0.998
    assert rel_l2(to_np(m2d), to_np(o[1])[oc, on]) < 1e-6
    assert rel_l2(to_np(depths), to_np(o[2])[oc, on]) < 1e-6
    assert rel_l2(to_np(conics), to_np(o[3])[oc, on]) < 1e-5
    if calc_comp:
        assert rel_l2(to_np(comps), to_np(o[4])[oc, on]) < 1e-5
    else:
        assert comps is None
    g = torch.Generator().manual_seed(5)
    w_m = torch.randn(m2d.shape, generator=g)
    w_d = torch.randn(depths.shape, generator=g)
    w_c = torch.randn(conics.shape, generator=g)
    w_k = torch.randn(depths.shape, generator=g) if calc_comp else None
    L = (m2d * w_m.to(gpu)).sum() + (depths * w_d.to(gpu)).sum() + (conics * w_c.to(gpu)).sum()
    if calc_comp:
        L = L + (comps * w_k.to(gpu)).sum()
    L.backward()
    # oracle: the same cotangents scattered to the dense [C, N] layout
    Nn = means.shape[0]
    dense = lambda w, k: torch.zeros((C, Nn) + k, dtype=w.dtype).index_put_(  # noqa: E731
        (torch.from_numpy(oc), torch.from_numpy(on)), w)
    live = torch.zeros((C, Nn), dtype=torch.int32)
    live[oc, on] = 1
    v_means, v_quats, v_scales, _, _ = G.project_bwd(
        means, quats, scales, sc.viewmats, sc.Ks, W, H, 0.3, live, o[3], dense(w_m, (2,)),
        dense(w_d, ()), dense(w_c, (3,)), compensations=o[4] if calc_comp else None,
        v_compensations=dense(w_k, ()) if calc_comp else None)
    gm, gq, gs = dm.grad, dq.grad, ds.grad
    if sparse:
        assert gm.is_sparse
        gm, gq, gs = gm.coalesce().to_dense(), gq.coalesce().to_dense(), gs.coalesce().to_dense()
    assert rel_l2(to_np(gm), v_means) < 1e-4
    assert rel_l2(to_np(gq), v_quats) < 1e-4
    assert rel_l2(to_np(gs), v_scales) < 1e-4


def test_projection_covars(gpu):
    announce("projection covars")
    sc, means, quats, scales = _proj_inputs(seed=1, C=2)
    W, H = sc.width, sc.height
    cov6 = G.covar_from_quat_scale(quats.double(), scales.double())[:, [0, 0, 0, 1, 1, 2],
                                                                    [0, 1, 2, 1, 2, 2]].float()
    dm = means.to(gpu).requires_grad_()
    dc = cov6.to(gpu).requires_grad_()
    radii, m2d, depths, conics, _ = ops.fully_fused_projection(
        dm, dc, None, None, sc.viewmats.to(gpu), sc.Ks.to(gpu), W, H)
    o_radii, o_m2d, o_depths, o_conics, _ = G.project_fwd(means, None, None, sc.viewmats, sc.Ks,
                                                          W, H, covars=cov6)
    both = (to_np(radii) > 0) & (to_np(o_radii) > 0) & (to_np(radii) == to_np(o_radii))
    assert rel_l2(to_np(conics)[both], to_np(o_conics)[both]) < 1e-5
    g = torch.Generator().manual_seed(2)
    live = torch.from_numpy(both)
    w_m = torch.randn(m2d.shape, generator=g) * live[..., None]
    w_c = torch.randn(conics.shape, generator=g) * live[..., None]
    ((m2d * w_m.to(gpu)).sum() + (conics * w_c.to(gpu)).sum()).backward()
    v_means, _, _, v_cov, _ = G.project_bwd(
        means, None, None, sc.viewmats, sc.Ks, W, H, 0.3, torch.from_numpy(np.where(both, 1, 0)),
        o_conics, w_m, None, w_c, covars=cov6)
    assert rel_l2(to_np(dm.grad), v_means) < 1e-4
    assert rel_l2(to_np(dc.grad), v_cov) < 1e-4


@pytest.mark.parametrize("degree,K", [(0, 16), (1, 16), (2, 9), (3, 16), (4, 25), (1, 4),
                                      (2, 12)])
def test_spherical_harmonics(gpu, degree, K):
    announce(f"sh degree={degree} K={K}")
    g = torch.Generator().manual_seed(degree)
    dirs = torch.randn((4097, 3), generator=g)
    coeffs = torch.randn((4097, K, 3), generator=g)
    masks = torch.rand(4097, generator=g) > 0.2
    v = torch.randn((4097, 3), generator=g)
    d_dirs = dirs.to(gpu).requires_grad_()
    d_coeffs = coeffs.to(gpu).requires_grad_()
    col = ops.spherical_harmonics(degree, d_dirs, d_coeffs, masks=masks.to(gpu))
    ref = G.sh_fwd(degree, dirs, coeffs) * masks[:, None]
    assert rel_l2(to_np(col), ref) < 1e-6
    (col * v.to(gpu)).sum().backward()
    vc, vd = G.sh_bwd(degree, dirs, coeffs, v * masks[:, None])
    assert rel_l2(to_np(d_coeffs.grad), vc) < 1e-6
    if degree > 0:
        assert rel_l2(to_np(d_dirs.grad), vd) < 1e-5
    else:
        assert float(d_dirs.grad.abs().max()) == 0.0


def _projected(gpu, seed=0, n=20000, C=2, W=200, H=120, log_scale_mu=-2.5):
    sc = scenes.small(seed=seed, n=n, n_cams=C, W=W, H=H, log_scale_mu=log_scale_mu)
    means, quats, scales, opac, sh = scenes.activations(sc.params)
    with torch.no_grad():
        radii, m2d, depths, conics, _ = ops.fully_fused_projection(
            means.to(gpu), None, quats.to(gpu), scales.to(gpu), sc.viewmats.to(gpu),
            sc.Ks.to(gpu), W, H)
    return sc, radii, m2d, depths, conics, opac


@pytest.mark.parametrize("C", [1, 3])
def test_isect_tiles_bit_exact(gpu, C):
    announce(f"isect C={C}")
    sc, radii, m2d, depths, conics, _ = _projected(gpu, seed=3, C=C)
    W, H, ts = sc.width, sc.height, 16
    tw, th = -(-W // ts), -(-H // ts)
    tiles, ids, flat = ops.isect_tiles(m2d, radii, depths, ts, tw, th)
    o_tiles, o_ids, o_flat = R.isect_tiles(to_np(m2d), to_np(radii), to_np(depths), ts, tw, th)
    assert ids.numel() > 10000
    np.testing.assert_array_equal(to_np(tiles), o_tiles)
    np.testing.assert_array_equal(to_np(ids), o_ids)
    np.testing.assert_array_equal(to_np(flat), o_flat)
    offs = ops.isect_offset_encode(ids, C, tw, th)
    np.testing.assert_array_equal(to_np(offs), R.isect_offset_encode(o_ids, C, tw, th))


@pytest.mark.parametrize("case", ["depth_ties", "negative_depth", "unsorted_cameras"])
def test_isect_tiles_paths_bit_exact(gpu, case):
    """isect_tiles on equal depths (ties broken by entry index: the reference's
    stable sort of (camera, tile, depth, entry) keys), on a negative depth
    (the reference sign-extends its bits into the key, which then sorts past
    every tile) and on packed camera ids out of order: bit-exact with the
    oracle in every case."""
    announce(f"isect paths {case}")
    sc, radii, m2d, depths, _, _ = _projected(gpu, seed=5, C=3)
    W, H, ts = sc.width, sc.height, 16
    tw, th = -(-W // ts), -(-H // ts)
    depths = depths.clone()
    if case == "depth_ties":
        depths = torch.round(depths * 4) / 4  # a few hundred distinct depths
    elif case == "negative_depth":
        vis = torch.nonzero(radii.reshape(-1) > 0).reshape(-1)
        depths.view(-1)[vis[::97]] *= -1.0
    if case == "unsorted_cameras":
        cam, gid = torch.nonzero(radii > 0, as_tuple=True)
        perm = torch.randperm(cam.numel(), generator=torch.Generator().manual_seed(1)).to(gpu)
        cam, gid = cam[perm], gid[perm]
        args = (m2d[cam, gid].contiguous(), radii[cam, gid].contiguous(),
                depths[cam, gid].contiguous())
        tiles, ids, flat = ops.isect_tiles(*args, ts, tw, th, packed=True, n_cameras=3,
                                           camera_ids=cam, gaussian_ids=gid)
        o_tiles, o_ids, o_flat = R.isect_tiles(*[to_np(a) for a in args], ts, tw, th,
                                               camera_ids=to_np(cam))
    else:
        tiles, ids, flat = ops.isect_tiles(m2d, radii, depths, ts, tw, th)
        o_tiles, o_ids, o_flat = R.isect_tiles(to_np(m2d), to_np(radii), to_np(depths), ts, tw,
                                               th)
    assert ids.numel() > 10000
    np.testing.assert_array_equal(to_np(tiles), o_tiles)
    np.testing.assert_array_equal(to_np(ids), o_ids)
    np.testing.assert_array_equal(to_np(flat), o_flat)


@pytest.mark.parametrize("n,shift", [(1, 0), (7, 0), (9, 1), (4096 + 5, 3), (200_003, 1)])
def test_isect_offset_encode_ragged(gpu, n, shift):
    """Offsets from sorted keys of every length class of the eight-keys-per-
    thread encoder (shorter than a thread's run, ragged tail) and from a key
    view that is not 32-byte aligned, with empty buckets before, between and
    after the runs; equal to the oracle's encoding."""
    announce(f"offset encode n={n} shift={shift}")
    C, tw, th = 3, 7, 5
    rng = np.random.default_rng(n)
    # buckets drawn sparsely so that many stay empty; keys sorted by bucket
    buckets = np.sort(rng.integers(1, C * tw * th - 1, size=n))
    tile_bits = int(tw * th).bit_length()
    cam, tile = buckets // (tw * th), buckets % (tw * th)
    keys = ((cam << (32 + tile_bits)) | (tile << 32) | rng.integers(0, 2**31, size=n)).astype(np.int64)
    buf = torch.zeros(n + shift, dtype=torch.int64)
    buf[shift:] = torch.from_numpy(keys)
    d = buf.to(gpu)[shift:]
    offs = ops.isect_offset_encode(d, C, tw, th)
    np.testing.assert_array_equal(to_np(offs), R.isect_offset_encode(keys, C, tw, th))


def test_isect_tiles_packed_and_empty(gpu):
    announce("isect packed + empty")
    sc, radii, m2d, depths, _, _ = _projected(gpu, seed=4, C=2)
    W, H, ts = sc.width, sc.height, 16
    tw, th = -(-W // ts), -(-H // ts)
    cam, gid = torch.nonzero(radii > 0, as_tuple=True)
    tiles, ids, flat = ops.isect_tiles(m2d[cam, gid].contiguous(), radii[cam, gid].contiguous(),
                                       depths[cam, gid].contiguous(), ts, tw, th, packed=True,
                                       n_cameras=2, camera_ids=cam, gaussian_ids=gid)
    o_tiles, o_ids, o_flat = R.isect_tiles(to_np(m2d[cam, gid]), to_np(radii[cam, gid]),
                                           to_np(depths[cam, gid]), ts, tw, th,
                                           camera_ids=to_np(cam))
    np.testing.assert_array_equal(to_np(ids), o_ids)
    np.testing.assert_array_equal(to_np(flat), o_flat)
    # nothing visible: empty outputs and all-zero offsets (isect_tiles.cu:298)
    z = torch.zeros_like(radii)
    tiles, ids, flat = ops.isect_tiles(m2d, z, depths, ts, tw, th)
    assert ids.numel() == 0 and int(tiles.abs().sum()) == 0
    offs = ops.isect_offset_encode(ids, 2, tw, th)
    assert offs.shape == (2, th, tw) and int(offs.abs().sum()) == 0


@pytest.mark.parametrize("n,begin,end", [(1, 0, 64), (100, 0, 46), (4097, 3, 40),
                                         (1_000_003, 0, 46), (70_000, 0, 64)])
def test_radix_sort_pairs_stable(gpu, n, begin, end):
    announce(f"radix n={n} bits=[{begin},{end})")
    rng = np.random.default_rng(n)
    keys = rng.integers(-2 ** 62, 2 ** 62, size=n, dtype=np.int64)
    keys[: n // 3] = keys[n // 3: 2 * (n // 3)]  # duplicates exercise stability
    vals = np.arange(n, dtype=np.int32)
    k, v = ops.radix_sort_pairs(torch.from_numpy(keys).to(gpu), torch.from_numpy(vals).to(gpu),
                                begin, end)
    span = end - begin
    masked = (keys.view(np.uint64) >> np.uint64(begin)) & np.uint64((1 << span) - 1 if span < 64
                                                                    else 2 ** 64 - 1)
    order = np.argsort(masked, kind="stable")
    np.testing.assert_array_equal(to_np(v), vals[order])
    np.testing.assert_array_equal(to_np(k), keys[order])


@pytest.mark.parametrize("segs,bits,vbytes", [
    ([0, 5000], 13, 4),
    ([0, 0, 4096, 4097, 4097, 90_000], 13, 4),   # empty segments, a one-key segment
    ([0, 1, 2, 3000, 3000], 32, 8),
    ([0, 300_000, 300_001, 1_000_000], 32, 8),
    ([0, 8192, 8192, 8192], 7, 4),
    ([0, 0, 4096, 4097, 70_000], 26, 4),          # three 9-bit passes (512 digits)
    ([0, 3, 50_000], 9, 8),                        # one 9-bit pass
])
def test_segmented_sort_pairs_u32(gpu, segs, bits, vbytes):
    """Each segment sorted stably on its own (numpy argsort kind='stable')."""
    import ctypes
    from tidegs_amd import _native as N
    announce(f"segmented sort segs={segs} bits={bits} vbytes={vbytes}")
    n = segs[-1]
    rng = np.random.default_rng(n + bits)
    keys = rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
    keys[: n // 3] = keys[n // 3: 2 * (n // 3)]  # duplicates exercise stability
    vdt = np.int32 if vbytes == 4 else np.int64
    vals = (np.arange(n, dtype=np.int64) * 3 + (1 << 40 if vbytes == 8 else 0)).astype(vdt)
    k = torch.from_numpy(keys.view(np.int32)).to(gpu)
    v = torch.from_numpy(vals).to(gpu)
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    lib = N.load()
    ws = torch.empty(lib.tgs_segmented_sort_workspace_size(n, len(segs) - 1), dtype=torch.uint8,
                     device=gpu)
    sel = ctypes.c_int(0)
    host = (ctypes.c_uint32 * len(segs))(*segs)
    N.call("tgs_segmented_sort_pairs_u32", N.ptr(k), N.ptr(v), N.ptr(k2), N.ptr(v2), vbytes, n,
           len(segs) - 1, host, 0, bits, N.ptr(ws), ws.numel(), ctypes.byref(sel),
           N.stream_handle())
    ko, vo = (k2, v2) if sel.value else (k, v)
    ko = to_np(ko).view(np.uint32)
    vo = to_np(vo)
    mask = np.uint32((1 << bits) - 1) if bits < 32 else np.uint32(0xffffffff)
    for a, b in zip(segs[:-1], segs[1:]):
        order = np.argsort(keys[a:b] & mask, kind="stable") + a
        np.testing.assert_array_equal(ko[a:b], keys[order])
        np.testing.assert_array_equal(vo[a:b], vals[order])


@pytest.mark.parametrize("segs,key_bits", [([0, 70_000], 25), ([0, 5000, 5000, 90_000, 131_073], 19),
                                           ([0, 40_000], 32), ([0, 1, 60_000, 60_000, 99_999], 27),
                                           ([0, 33_000], 18), ([0, 4096], 1), ([0, 2, 9000], 8),
                                           ([0, 12_345], 9)])
def test_segmented_sort_pairs_u32_range(gpu, segs, key_bits):
    """The range form sorts keys in [base, base + 2^bits - 1) into the same
    order as a full stable sort, with the 0xffffffff sentinels (culled depth
    entries) tied after them in input order and keys below the base first."""
    import ctypes
    from tidegs_amd import _native as N
    announce(f"segmented range sort segs={segs} bits={key_bits}")
    n = segs[-1]
    rng = np.random.default_rng(n + key_bits)
    base = 0x41200000 if key_bits < 32 else 0
    span = (1 << key_bits) - 1 if key_bits < 32 else 0xFFFFFFFF
    keys = (base + rng.integers(0, span, size=n, dtype=np.uint64)).astype(np.uint32)
    keys[: n // 4] = keys[n // 4: 2 * (n // 4)]  # duplicates exercise stability
    keys[rng.random(n) < 0.05] = 0xFFFFFFFF
    if key_bits < 32:
        keys[rng.random(n) < 0.01] = base - 7  # below the range: ranked as the base
    vals = np.arange(n, dtype=np.int64) * 5 + (1 << 40)
    k = torch.from_numpy(keys.view(np.int32)).to(gpu)
    v = torch.from_numpy(vals).to(gpu)
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    lib = N.load()
    ws = torch.empty(lib.tgs_segmented_sort_workspace_size(n, len(segs) - 1), dtype=torch.uint8,
                     device=gpu)
    sel = ctypes.c_int(0)
    host = (ctypes.c_uint32 * len(segs))(*segs)
    N.call("tgs_segmented_sort_pairs_u32_range", N.ptr(k), N.ptr(v), N.ptr(k2), N.ptr(v2), 8, n,
           len(segs) - 1, host, base, key_bits, N.ptr(ws), ws.numel(), ctypes.byref(sel),
           N.stream_handle())
    ko, vo = (k2, v2) if sel.value else (k, v)
    ko = to_np(ko).view(np.uint32)
    vo = to_np(vo)
    cap = np.uint64(span)
    rel = np.minimum(np.maximum(keys.astype(np.int64) - base, 0).astype(np.uint64), cap)
    for a, b in zip(segs[:-1], segs[1:]):
        order = np.argsort(rel[a:b], kind="stable") + a
        np.testing.assert_array_equal(ko[a:b], keys[order])
        np.testing.assert_array_equal(vo[a:b], vals[order])
        # the keys inside the range come out in their full stable order
        ins = np.flatnonzero((keys[a:b] >= base) & (keys[a:b] != 0xFFFFFFFF)) + a
        full = ins[np.argsort(keys[ins], kind="stable")]
        out_in = (ko[a:b] >= base) & (ko[a:b] != 0xFFFFFFFF)
        np.testing.assert_array_equal(vo[a:b][out_in], vals[full])


def _raster_case(gpu, seed, C=2, D=3, W=200, H=120, tile=16, packed=False):
    sc, radii, m2d, depths, conics, opac = _projected(gpu, seed=seed, C=C, W=W, H=H)
    tw, th = -(-W // tile), -(-H // tile)
    g = torch.Generator().manual_seed(seed)
    Nn = radii.shape[1]
    colors = torch.rand((C, Nn, D), generator=g).to(gpu)
    opacs = opac[None].repeat(C, 1).to(gpu).contiguous()
    if packed:
        cam, gid = torch.nonzero(radii > 0, as_tuple=True)
        m2d, conics, colors, opacs = (m2d[cam, gid].contiguous(), conics[cam, gid].contiguous(),
                                      colors[cam, gid].contiguous(), opacs[cam, gid].contiguous())
        _, ids, flat = ops.isect_tiles(m2d, radii[cam, gid].contiguous(),
                                       depths[cam, gid].contiguous(), tile, tw, th, packed=True,
                                       n_cameras=C, camera_ids=cam, gaussian_ids=gid)
    else:
        _, ids, flat = ops.isect_tiles(m2d, radii, depths, tile, tw, th)
    offs = ops.isect_offset_encode(ids, C, tw, th)
    return m2d, conics, colors, opacs, offs, flat


@pytest.mark.parametrize("D,tile,bg,packed,absgrad", [
    (3, 16, False, False, False), (3, 16, True, False, True), (1, 16, False, False, False),
    (4, 8, True, False, False), (5, 16, False, False, False), (32, 16, False, True, False),
    (3, 16, False, True, True), (33, 16, True, False, False), (64, 16, False, True, False),
    (65, 8, True, False, False)])
def test_rasterize_fwd_bwd(gpu, D, tile, bg, packed, absgrad):
    """Drop-in rasterize_to_pixels forward and backward against the oracle's
    restatement of rasterize_to_pixels_fwd/bwd.cu, over channel counts the
    kernels instantiate, padded ones (5) and ones run in 32-channel launches
    (33, 64, 65)."""
    announce(f"raster D={D} tile={tile} bg={bg} packed={packed} absgrad={absgrad}")
    C, W, H = 2, 200, 120
    m2d, conics, colors, opacs, offs, flat = _raster_case(gpu, seed=10 + D, C=C, D=D, W=W, H=H,
                                                          tile=tile, packed=packed)
    g = torch.Generator().manual_seed(D)
    bgs = torch.rand((C, D), generator=g).to(gpu) if bg else None
    leaves = [t.clone().requires_grad_() for t in (m2d, conics, colors, opacs)]
    if bg:
        bgs.requires_grad_()
    rc, ra = ops.rasterize_to_pixels(*leaves, W, H, tile, offs, flat, backgrounds=bgs,
                                     packed=packed, absgrad=absgrad)
    ref_c, ref_a, ref_last = R.rasterize_fwd(
        to_np(m2d).reshape(-1, 2), to_np(conics).reshape(-1, 3), to_np(colors).reshape(-1, D),
        to_np(opacs).reshape(-1), W, H, tile, to_np(offs), to_np(flat),
        backgrounds=to_np(bgs) if bg else None)
    assert rel_l2(to_np(rc), ref_c) < 1e-5
    assert rel_l2(to_np(ra)[..., 0], ref_a) < 1e-5
    wc = torch.randn(rc.shape, generator=g)
    wa = torch.randn(ra.shape, generator=g)
    ((rc * wc.to(gpu)).sum() + (ra * wa.to(gpu)).sum()).backward()
    # oracle backward from the GPU's own forward state
    _, _, last = R.rasterize_fwd(
        to_np(m2d).reshape(-1, 2), to_np(conics).reshape(-1, 3), to_np(colors).reshape(-1, D),
        to_np(opacs).reshape(-1), W, H, tile, to_np(offs), to_np(flat))
    vm, vc, vcol, vo, vabs = R.rasterize_bwd(
        to_np(m2d).reshape(-1, 2), to_np(conics).reshape(-1, 3), to_np(colors).reshape(-1, D),
        to_np(opacs).reshape(-1), W, H, tile, to_np(offs), to_np(flat), ref_a, ref_last,
        to_np(wc), v_alphas=to_np(wa)[..., 0], backgrounds=to_np(bgs) if bg else None,
        absgrad=absgrad)
    assert rel_l2(to_np(leaves[0].grad).reshape(-1, 2), vm) < 1e-4
    assert rel_l2(to_np(leaves[1].grad).reshape(-1, 3), vc) < 1e-4
    assert rel_l2(to_np(leaves[2].grad).reshape(-1, D), vcol) < 1e-4
    assert rel_l2(to_np(leaves[3].grad).reshape(-1), vo) < 1e-4
    if absgrad:
        assert rel_l2(to_np(leaves[0].absgrad).reshape(-1, 2), vabs) < 1e-4
    if bg:
        ref_vbg = (to_np(wc) * (1 - ref_a[..., None])).sum(axis=(1, 2))
        assert rel_l2(to_np(bgs.grad), ref_vbg) < 1e-5


@pytest.mark.parametrize("D,tile", [(3, 16), (4, 8)])
def test_rasterize_nonfinite_colour(gpu, D, tile):
    """A Gaussian with an infinite colour channel reaches only the pixels it
    composites, as in the reference (which adds c * alpha * T only there):
    everywhere else the forward stays finite and equal to the oracle's, and
    the backward's gradients are non-finite exactly where the oracle's are,
    equal elsewhere.  (The walks multiply colours by zero for Gaussians that
    fail the alpha test; a batch holding a non-finite colour takes the
    select form instead.)"""
    announce(f"raster non-finite colour D={D} tile={tile}")
    C, W, H = 2, 200, 120
    m2d, conics, colors, opacs, offs, flat = _raster_case(gpu, seed=91 + D, C=C, D=D, W=W, H=H,
                                                          tile=tile)
    # a visible Gaussian (projected conic) inside the frame that composites
    # into a few pixels (the first such candidate, by the oracle's forward)
    live = torch.nonzero((conics[..., 0] > 0) & (m2d[..., 0] > 20) & (m2d[..., 0] < W - 20) &
                         (m2d[..., 1] > 20) & (m2d[..., 1] < H - 20)).tolist()
    base = to_np(colors).copy()
    for cam, gid in live[len(live) // 2:]:
        colors_np = base.copy()
        colors_np[cam, gid, 1] = np.inf
        np_args = (to_np(m2d).reshape(-1, 2), to_np(conics).reshape(-1, 3),
                   colors_np.reshape(-1, D), to_np(opacs).reshape(-1), W, H, tile, to_np(offs),
                   to_np(flat))
        ref_c, ref_a, ref_last = R.rasterize_fwd(*np_args)
        fin = np.isfinite(ref_c)
        if 0 < (~fin).sum() and fin.mean() > 0.99:
            break
    else:
        pytest.fail("no Gaussian composites into a few pixels")
    colors = torch.from_numpy(colors_np).to(gpu)
    leaves = [t.clone().requires_grad_() for t in (m2d, conics, colors, opacs)]
    rc, ra = ops.rasterize_to_pixels(*leaves, W, H, tile, offs, flat)
    got = to_np(rc)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    assert rel_l2(got[fin], ref_c[fin]) < 1e-5
    assert rel_l2(to_np(ra)[..., 0], ref_a) < 1e-5
    g = torch.Generator().manual_seed(D)
    wc = torch.randn(rc.shape, generator=g)
    (rc * wc.to(gpu)).sum().backward()
    ref = R.rasterize_bwd(*np_args, ref_a, ref_last, to_np(wc))[:4]
    widths = (2, 3, D, 1)
    for leaf, r, w in zip(leaves, ref, widths):
        v, r = to_np(leaf.grad).reshape(-1, w), np.asarray(r).reshape(-1, w)
        f = np.isfinite(r)
        np.testing.assert_array_equal(np.isfinite(v), f)
        assert f.mean() > 0.99 and rel_l2(v[f], r[f]) < 1e-4


def test_fused_ssim(gpu):
    announce("fused_ssim")
    g = torch.Generator().manual_seed(0)
    a = torch.rand((2, 3, 67, 91), generator=g)
    b = torch.rand((2, 3, 67, 91), generator=g)
    da = a.to(gpu).requires_grad_()
    m = FusedSSIMMap.apply(0.01 ** 2, 0.03 ** 2, da, b.to(gpu), "same", True)
    rm, d1, d2, d3 = S.ssim_fwd(a.numpy(), b.numpy())
    assert rel_l2(to_np(m), rm) < 1e-5
    gm = torch.randn(m.shape, generator=g)
    (m * gm.to(gpu)).sum().backward()
    ref = S.ssim_bwd(a.numpy(), b.numpy(), gm.numpy(), d1, d2, d3)
    assert rel_l2(to_np(da.grad), ref) < 1e-5
    val = fused_ssim(a.to(gpu), b.to(gpu), padding="valid")
    assert abs(float(val) - float(rm[:, :, 5:-5, 5:-5].mean())) < 1e-5


@pytest.mark.parametrize("D,tile,bg", [(3, 16, True), (4, 16, False), (40, 8, True)])
def test_rasterize_masks(gpu, D, tile, bg):
    """Tile masks: a skipped tile's pixels hold the background (zero without
    one) with alpha 0 and pass no gradient; the other pixels and all gradients
    equal the oracle's with the skipped pixels' output gradients zeroed."""
    announce(f"raster masks D={D} tile={tile} bg={bg}")
    C, W, H = 2, 200, 120
    m2d, conics, colors, opacs, offs, flat = _raster_case(gpu, seed=70 + D, C=C, D=D, W=W, H=H,
                                                          tile=tile, packed=False)
    g = torch.Generator().manual_seed(7 + D)
    bgs = torch.rand((C, D), generator=g).to(gpu) if bg else None
    th, tw = offs.shape[1], offs.shape[2]
    masks = torch.rand((C, th, tw), generator=g) > 0.3
    leaves = [t.clone().requires_grad_() for t in (m2d, conics, colors, opacs)]
    rc, ra = ops.rasterize_to_pixels(*leaves, W, H, tile, offs, flat, backgrounds=bgs,
                                     masks=masks.to(gpu))
    ref_c, ref_a, ref_last = R.rasterize_fwd(
        to_np(m2d).reshape(-1, 2), to_np(conics).reshape(-1, 3), to_np(colors).reshape(-1, D),
        to_np(opacs).reshape(-1), W, H, tile, to_np(offs), to_np(flat),
        backgrounds=to_np(bgs) if bg else None)
    pm = masks.numpy().repeat(tile, 1).repeat(tile, 2)[:, :H, :W]
    exp_c = np.where(pm[..., None], ref_c, to_np(bgs)[:, None, None, :] if bg else 0.0)
    exp_a = np.where(pm, ref_a, 0.0)
    assert rel_l2(to_np(rc), exp_c) < 1e-5
    np.testing.assert_array_equal(to_np(ra)[..., 0][~pm], 0.0)
    assert rel_l2(to_np(ra)[..., 0], exp_a) < 1e-5
    wc = torch.randn(rc.shape, generator=g)
    wa = torch.randn(ra.shape, generator=g)
    ((rc * wc.to(gpu)).sum() + (ra * wa.to(gpu)).sum()).backward()
    wc_m = to_np(wc) * pm[..., None]
    wa_m = to_np(wa)[..., 0] * pm
    vm, vc, vcol, vo, _ = R.rasterize_bwd(
        to_np(m2d).reshape(-1, 2), to_np(conics).reshape(-1, 3), to_np(colors).reshape(-1, D),
        to_np(opacs).reshape(-1), W, H, tile, to_np(offs), to_np(flat), ref_a, ref_last,
        wc_m, v_alphas=wa_m, backgrounds=to_np(bgs) if bg else None)
    assert rel_l2(to_np(leaves[0].grad).reshape(-1, 2), vm) < 1e-4
    assert rel_l2(to_np(leaves[1].grad).reshape(-1, 3), vc) < 1e-4
    assert rel_l2(to_np(leaves[2].grad).reshape(-1, D), vcol) < 1e-4
    assert rel_l2(to_np(leaves[3].grad).reshape(-1), vo) < 1e-4


@pytest.mark.parametrize("B,H,W", [(1, 70, 130), (2, 37, 21)])
def test_tide_loss_kernel(gpu, B, H, W):
    """One-pass L1 + SSIM loss and gradient (tgs_tide_loss) against the oracle
    restatement of base_engine.py:464-488, per image of the batch."""
    announce(f"tide loss (L1 + SSIM) B={B} {H}x{W}")
    from tidegs_amd import _native as N

    g = torch.Generator().manual_seed(3 + B)
    img = torch.rand((B, H, W, 3), generator=g)
    gt = torch.rand((B, 3, H, W), generator=g) * 300 - 20
    d_img, d_gt = img.to(gpu), gt.to(gpu)  # keep the device copies alive
    sums = torch.zeros(2 * B, dtype=torch.float64, device=gpu)
    v = torch.empty((B, H, W, 3), device=gpu)
    N.call("tgs_tide_loss", B, H, W, N.ptr(d_img), N.ptr(d_gt), 255.0, 0.2, N.ptr(sums), N.ptr(v),
           N.stream_handle())
    sums = to_np(sums)
    n = 3 * H * W
    for bi in range(B):
        loss_ref, grad_ref = S.tide_loss(img[bi].permute(2, 0, 1).numpy(), gt[bi].numpy())
        loss = 0.8 * sums[2 * bi] / n + 0.2 * (1 - sums[2 * bi + 1] / n)
        assert abs(loss - loss_ref) < 1e-6
        assert rel_l2(to_np(v[bi]).transpose(2, 0, 1), grad_ref) < 1e-5


@pytest.mark.parametrize("form", [0, 1, 2, 3, 4, 5])
def test_valu_probe_sums(gpu, form):
    """tgs_valu_probe (bench.py's VALU-rate measurement kernel, in its own
    library bench_valu_probe.so) computes what it
    claims, per thread 8 chains from a_k = tid + k (u_k = 7 tid + k), summed,
    against the same recurrences in float64 / integers: 0 a_k <- a_k z with
    z = x - (tid mod 64) 1e-9 in float32; 1 a_k <- a_k x; 2 u_k <- u_k + 3 tid
    + 1 (low 16 bits summed); 3 u_k <- u_k ^ bits(x); 4 a_k <- fma(a_k, z, y),
    y = (tid mod 64) 1e-9; 5 a_k <- 2^-a_k from a_k = k / 10."""
    from bench import valu_probe

    blocks, iters, x = 3, 40, np.float32(0.999999)
    announce(f"valu probe form {form}: {blocks} blocks x {iters} rounds")
    out = torch.full((blocks * 256,), float("nan"), device=gpu)
    valu_probe(out, blocks, iters, form, torch.cuda.current_stream(gpu).cuda_stream)
    torch.cuda.synchronize(gpu)
    tid = np.arange(256)
    lane = (tid % 64).astype(np.float32)
    z = (x - lane * np.float32(1e-9)).astype(np.float64)
    y = (lane * np.float32(1e-9)).astype(np.float64)
    a = (tid[:, None] + np.arange(8)[None, :]).astype(np.float64)
    u = tid[:, None] * 7 + np.arange(8)[None, :]  # int64: no wrap at these sizes
    if form == 0:
        a = a * z[:, None] ** iters
    elif form == 1:
        a = a * float(x) ** iters
    elif form == 2:
        a = ((u + iters * (3 * tid[:, None] + 1)) & 0xffff).astype(np.float64)
    elif form == 3:
        bits = int(np.float32(x).view(np.uint32))
        a = ((u ^ bits if iters % 2 else u) & 0xffff).astype(np.float64)
    elif form == 4:
        for _ in range(iters):
            a = a * z[:, None] + y[:, None]
    else:
        a = np.tile(np.arange(8) * 0.1, (256, 1))
        for _ in range(iters):
            a = 2.0 ** -a
    ref = np.tile(a.sum(1), blocks)
    np.testing.assert_allclose(to_np(out), ref, rtol=1e-4 if form == 5 else 1e-5)
