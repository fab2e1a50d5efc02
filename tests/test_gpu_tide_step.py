"""GPU parity of the fused resident step (tidegs_amd.tide_step.TideStep) with
the CPU step oracle (oracle/step_ref.py), which restates TideGS's per-camera
loop.  Index work bit-exact (filters, touched rows, isect ids); compact
gradients within relative L2 <= 1e-4 per parameter group;
untouched rows of the table bitwise unchanged by the optimizer."""
import numpy as np
import pytest
import torch

from oracle import optim_ref as O
from oracle import raster_ref as R
from oracle import step_ref as SR
from tests.gpu_util import announce, rel_l2, to_np
from tidegs_amd import scenes
from tidegs_amd.tide_step import TideStep

pytestmark = pytest.mark.gpu

GROUPS = {"xyz": slice(0, 3), "scale": slice(3, 6), "rot": slice(6, 10), "opacity": slice(10, 11),
          "dc": slice(11, 14), "rest": slice(14, 59)}


def _scene(seed=0, n=3000, C=3, W=96, H=64):
    return scenes.small(seed=seed, n=n, n_cams=C, W=W, H=H, log_scale_mu=-2.3)


@pytest.mark.parametrize("with_bg,pitch", [(False, 59), (True, 59), (False, 64)])
def test_tide_step_grads_match_oracle(gpu, with_bg, pitch):
    announce(f"tide step grads bg={with_bg} row pitch={pitch}")
    sc = _scene(seed=1 if with_bg else 0)
    bgs = torch.tensor([[0.1, 0.5, 0.9], [1.0, 1.0, 1.0], [0.0, 0.2, 0.3]]) if with_bg else None
    params = sc.params.to(gpu).contiguous()
    if pitch == 64:
        params = scenes.padded_table(params)
    ts = TideStep(params, sc.width, sc.height, batch_size=sc.n_cams,
                  backgrounds=bgs.to(gpu) if with_bg else None)
    touched, grads, stats = ts.forward_backward(sc.viewmats, sc.Ks, sc.gt)
    o_touched, o_grads, o_losses, o_images, o_filters = SR.batch_grads(
        sc.params, sc.viewmats, sc.Ks, sc.gt, sc.width, sc.height, backgrounds=bgs)
    # filters and touched rows: exact
    np.testing.assert_array_equal(to_np(touched), to_np(o_touched))
    offs = to_np(ts.last["cam_offsets"])
    entries = to_np(ts.last["entries"])
    for c, f in enumerate(o_filters):
        np.testing.assert_array_equal(entries[offs[c]:offs[c + 1]], to_np(f))
    # rendered images and losses
    imgs = to_np(ts.last["images"])
    for c in range(sc.n_cams):
        assert rel_l2(imgs[c], o_images[c]) < 1e-5
    losses = stats.losses(sc.width, sc.height)
    np.testing.assert_allclose(losses, o_losses, rtol=1e-5)
    g = to_np(grads)
    og = to_np(o_grads)
    for name, sl in GROUPS.items():
        err = rel_l2(g[:, sl], og[:, sl])
        print(f"  grad {name}: rel_l2={err:.2e}")
        assert err < 1e-4, (name, err)


def test_counting_forward_matches_plain(gpu):
    """The forward variant that also counts each pixel's composited Gaussians
    (bench live-pair statistic) renders bit-identically to the plain one; its
    counts are zero exactly where nothing composites and bounded by the
    pixel's tile list."""
    announce("tide step counting forward")
    sc = _scene(seed=4)
    ts = TideStep(sc.params.to(gpu).contiguous(), sc.width, sc.height, batch_size=sc.n_cams)
    ts.forward_backward(sc.viewmats, sc.Ks, sc.gt)
    plain = {k: to_np(ts.last[k]).copy() for k in ("images", "alphas", "last_ids", "v_images")}
    ts.forward_backward(sc.viewmats, sc.Ks, sc.gt, count_pairs=True)
    for k, v in plain.items():
        np.testing.assert_array_equal(to_np(ts.last[k]), v, err_msg=k)
    n = to_np(ts.last["n_contrib"])
    alphas = plain["alphas"]
    assert ((n == 0) == (alphas == 0)).all()
    offs = to_np(ts.last["offsets"]).reshape(sc.n_cams, -1)
    n_isects = len(to_np(ts.last["flatten_ids"]))
    flat = offs.reshape(-1)
    ends = np.append(flat[1:], n_isects).reshape(offs.shape)
    per_tile = ends - offs  # list length of each (camera, tile)
    tw = offs.shape[1] // ((sc.height + 15) // 16)
    for c in range(sc.n_cams):
        ty, tx = np.divmod(np.arange(sc.height * sc.width), sc.width)
        lim = per_tile[c][(ty // 16) * tw + tx // 16].reshape(sc.height, sc.width)
        assert (n[c] <= lim).all()
    assert ts.last_live_pairs == int(n.sum())


@pytest.mark.parametrize("V,C", [(1, 1), (2047, 2), (2049, 3), (50_000, 16)])
def test_blocked_emit_matches_offset_emit(gpu, V, C):
    """tgs_tide_isect_emit_blocked (block area sums + scan + in-block prefix
    sums) writes the same keys and flatten ids as the per-entry form (count,
    int64 inclusive scan, emit), on random rectangles with empty ones and
    camera boundaries inside and across blocks."""
    announce(f"blocked isect emission V={V} C={C}")
    from tidegs_amd import _native as N
    lib = N.load()
    rng = np.random.default_rng(V + C)
    tw, th = 120, 68
    x0 = rng.integers(0, tw, V)
    y0 = rng.integers(0, th, V)
    x1 = np.minimum(x0 + rng.integers(0, 5, V), tw)  # width 0 gives empty rectangles
    y1 = np.minimum(y0 + rng.integers(0, 4, V), th)
    rc = (x0 | (x1 << 8) | (y0 << 16) | (y1 << 24)).astype(np.uint64)
    ids = rng.integers(0, 1 << 30, V).astype(np.uint64)
    rects = torch.from_numpy(((rc << np.uint64(32)) | ids).view(np.int64)).to(gpu)
    cuts = np.sort(rng.choice(np.arange(1, V), size=min(C - 1, V - 1), replace=False)) if V > 1 else []
    cam_off = torch.tensor(np.concatenate([[0], cuts, [V] * (C - len(cuts))]).astype(np.int32),
                           device=gpu)
    n_isects = int(((x1 - x0) * (y1 - y0)).sum())
    tile_bits = (tw * th).bit_length()
    s = N.stream_handle()
    tiles = torch.empty(V, dtype=torch.int32, device=gpu)
    cum = torch.empty(V, dtype=torch.int64, device=gpu)
    ws = torch.empty(lib.tgs_scan_workspace_size(V), dtype=torch.uint8, device=gpu)
    N.call("tgs_tide_isect_count", V, N.ptr(rects), N.ptr(tiles), s)
    N.call("tgs_inclusive_scan_i32_i64", N.ptr(tiles), N.ptr(cum), V, N.ptr(ws), ws.numel(), s)
    cap = max(n_isects, 1)
    k_ref = torch.empty(cap, dtype=torch.int32, device=gpu)
    f_ref = torch.empty(cap, dtype=torch.int32, device=gpu)
    N.call("tgs_tide_isect_emit", V, N.ptr(cam_off), C, N.ptr(rects), N.ptr(cum), tw, tile_bits,
           N.ptr(k_ref), N.ptr(f_ref), s)
    nb = lib.tgs_tide_isect_emit_blocks(V)
    sums = torch.empty(nb, dtype=torch.int32, device=gpu)
    base = torch.empty(nb, dtype=torch.int32, device=gpu)
    ws2 = torch.empty(lib.tgs_scan_workspace_size(nb), dtype=torch.uint8, device=gpu)
    N.call("tgs_tide_isect_block_sums", V, N.ptr(rects), N.ptr(sums), s)
    N.call("tgs_exclusive_scan_u32", N.ptr(sums), N.ptr(base), nb, N.ptr(ws2), ws2.numel(), s)
    k = torch.empty(cap, dtype=torch.int32, device=gpu)
    f = torch.empty(cap, dtype=torch.int32, device=gpu)
    N.call("tgs_tide_isect_emit_blocked", V, N.ptr(cam_off), C, N.ptr(rects), N.ptr(base), tw,
           tile_bits, N.ptr(k), N.ptr(f), s)
    assert int(cum[-1]) == n_isects
    np.testing.assert_array_equal(to_np(k)[:n_isects], to_np(k_ref)[:n_isects])
    np.testing.assert_array_equal(to_np(f)[:n_isects], to_np(f_ref)[:n_isects])


@pytest.mark.parametrize("V,C,big", [(3000, 4, 0.0), (20_000, 6, 0.02), (70_000, 16, 0.001)])
def test_emit_hist_then_hist0_sort(gpu, V, C, big):
    """tgs_tide_isect_emit_blocked_hist + tgs_segmented_sort_pairs_u32_hist0 (the
    emission counting the first pass's digit histogram) give the same sorted
    keys and flatten ids as a stable per-camera sort of the emitted keys on the
    tile bits (numpy), with empty cameras and rectangles spanning many sort
    tiles (counted by the global-atomic path)."""
    announce(f"emission histogram + hist0 sort V={V} C={C} big={big}")
    import ctypes
    from tidegs_amd import _native as N
    lib = N.load()
    rng = np.random.default_rng(V * 7 + C)
    tw, th = 120, 68
    x0 = rng.integers(0, tw, V)
    y0 = rng.integers(0, th, V)
    wide = rng.random(V) < big
    x1 = np.minimum(x0 + np.where(wide, rng.integers(20, 120, V), rng.integers(0, 5, V)), tw)
    y1 = np.minimum(y0 + np.where(wide, rng.integers(20, 68, V), rng.integers(0, 4, V)), th)
    rc = (x0 | (x1 << 8) | (y0 << 16) | (y1 << 24)).astype(np.uint64)
    ids = rng.integers(0, 1 << 30, V).astype(np.uint64)
    rects = torch.from_numpy(((rc << np.uint64(32)) | ids).view(np.int64)).to(gpu)
    cuts = np.sort(rng.choice(np.arange(1, V), size=C - 2, replace=False))
    cam = np.concatenate([[0], cuts[:1], cuts[:1], cuts[1:], [V]]).astype(np.int64)  # camera 1 empty
    cam_off = torch.tensor(cam.astype(np.int32), device=gpu)
    area = (x1 - x0) * (y1 - y0)
    isect_off = np.array([area[cam[c]:cam[c + 1]].sum() for c in range(C)]).cumsum()
    segs = [0] + [int(v) for v in isect_off]
    n_isects = segs[-1]
    tile_bits = (tw * th).bit_length()
    s = N.stream_handle()
    nb = lib.tgs_tide_isect_emit_blocks(V)
    sums = torch.empty(nb, dtype=torch.int32, device=gpu)
    base = torch.empty(nb, dtype=torch.int32, device=gpu)
    ws2 = torch.empty(lib.tgs_scan_workspace_size(nb), dtype=torch.uint8, device=gpu)
    N.call("tgs_tide_isect_block_sums", V, N.ptr(rects), N.ptr(sums), s)
    N.call("tgs_exclusive_scan_u32", N.ptr(sums), N.ptr(base), nb, N.ptr(ws2), ws2.numel(), s)
    k = torch.empty(n_isects, dtype=torch.int32, device=gpu)
    f = torch.empty(n_isects, dtype=torch.int32, device=gpu)
    N.call("tgs_tide_isect_emit_blocked", V, N.ptr(cam_off), C, N.ptr(rects), N.ptr(base), tw,
           tile_bits, N.ptr(k), N.ptr(f), s)
    k_in, f_in = to_np(k).view(np.uint32), to_np(f)
    hs = (ctypes.c_uint32 * (C + 1))(*segs)
    ws = torch.empty(lib.tgs_segmented_sort_workspace_size(n_isects, C), dtype=torch.uint8,
                     device=gpu)
    k2, f2 = torch.empty_like(k), torch.empty_like(f)
    N.call("tgs_tide_isect_emit_blocked_hist", V, N.ptr(cam_off), C, N.ptr(rects), N.ptr(base),
           tw, tile_bits, N.ptr(k), N.ptr(f), hs, N.ptr(ws), ws.numel() // 4, s)
    np.testing.assert_array_equal(to_np(k).view(np.uint32), k_in)
    sel = ctypes.c_int(0)
    N.call("tgs_segmented_sort_pairs_u32_hist0", N.ptr(k), N.ptr(f), N.ptr(k2), N.ptr(f2),
           n_isects, C, hs, 0, tile_bits, N.ptr(ws), ws.numel(), ctypes.byref(sel), s)
    ko, fo = (k2, f2) if sel.value else (k, f)
    ko, fo = to_np(ko).view(np.uint32), to_np(fo)
    tmask = np.uint32((1 << tile_bits) - 1)
    for a, b in zip(segs[:-1], segs[1:]):
        order = np.argsort(k_in[a:b] & tmask, kind="stable") + a
        np.testing.assert_array_equal(ko[a:b], k_in[order])
        np.testing.assert_array_equal(fo[a:b], f_in[order])


@pytest.mark.parametrize("V,C,big,tw,th", [(3000, 4, 0.0, 120, 68), (20_000, 6, 0.02, 120, 68),
                                           (70_000, 16, 0.001, 120, 68), (5000, 3, 0.01, 16, 9),
                                           (1, 1, 0.0, 120, 68)])
def test_fused_emission_sort_matches_stable_tile_sort(gpu, V, C, big, tw, th):
    """tgs_tide_isect_fused_count + scan + tgs_tide_isect_fused_scatter (the
    emission written in the order of the tile-bit sort's first pass) and the
    remaining pass give the stable per-camera sort of the emission
    (isect_tiles.cu:73-98 over the entries in the given order) on the tile
    bits, as numpy's stable argsort gives it: an empty camera, entries whose
    rectangles span several 4096-intersection chunks of a block (up to 120 x
    68 tiles), a grid whose tile bits fit one pass (16 x 9 tiles), one entry."""
    announce(f"fused emission + first tile pass V={V} C={C} big={big} grid={tw}x{th}")
    import ctypes
    from tidegs_amd import _native as N
    lib = N.load()
    rng = np.random.default_rng(V * 13 + C + tw)
    x0 = rng.integers(0, tw, V)
    y0 = rng.integers(0, th, V)
    wide = rng.random(V) < big
    x1 = np.minimum(x0 + np.where(wide, rng.integers(min(20, tw), tw + 1, V),
                                  rng.integers(0, 5, V)), tw)
    y1 = np.minimum(y0 + np.where(wide, rng.integers(min(20, th), th + 1, V),
                                  rng.integers(0, 4, V)), th)
    if big:  # entries whose rectangles span whole chunks
        x0[:3], y0[:3], x1[:3], y1[:3] = 0, 0, tw, th
    rc = (x0 | (x1 << 8) | (y0 << 16) | (y1 << 24)).astype(np.uint64)
    ids = rng.integers(0, 1 << 30, V).astype(np.uint64)
    rects = torch.from_numpy(((rc << np.uint64(32)) | ids).view(np.int64)).to(gpu)
    if C > 2:
        cuts = np.sort(rng.choice(np.arange(1, V), size=C - 2, replace=False))
        cam = np.concatenate([[0], cuts[:1], cuts[:1], cuts[1:], [V]]).astype(np.int64)  # cam 1 empty
    else:
        cam = np.linspace(0, V, C + 1).astype(np.int64)
    area = (x1 - x0) * (y1 - y0)
    segs = [0] + [int(v) for v in np.array([area[cam[c]:cam[c + 1]].sum()
                                             for c in range(C)]).cumsum()]
    n_isects = segs[-1]
    tile_bits = (tw * th).bit_length()
    s = N.stream_handle()
    co = (ctypes.c_uint32 * (C + 1))(*[int(v) for v in cam])
    words = int(lib.tgs_tide_isect_fused_hist_words(C, co, tile_bits))
    hist = torch.empty(max(words, 1), dtype=torch.int32, device=gpu)
    hscan = torch.empty_like(hist)
    ws = torch.empty(lib.tgs_scan_workspace_size(max(words, 1)), dtype=torch.uint8, device=gpu)
    N.call("tgs_tide_isect_fused_count", C, co, N.ptr(rects), tw, tile_bits, N.ptr(hist), words, s)
    N.call("tgs_exclusive_scan_u32", N.ptr(hist), N.ptr(hscan), words, N.ptr(ws), ws.numel(), s)
    k = torch.empty(max(n_isects, 1), dtype=torch.int32, device=gpu)
    f = torch.empty_like(k)
    N.call("tgs_tide_isect_fused_scatter", C, co, N.ptr(rects), tw, tile_bits, N.ptr(hscan), words,
           n_isects, N.ptr(k), N.ptr(f), s)
    w1 = int(lib.tgs_tide_isect_fused_digit_bits(tile_bits))
    if tile_bits > w1:
        k2, f2 = torch.empty_like(k), torch.empty_like(f)
        tws = torch.empty(lib.tgs_segmented_sort_workspace_size(n_isects, C), dtype=torch.uint8,
                          device=gpu)
        sel = ctypes.c_int(0)
        hs = (ctypes.c_uint32 * (C + 1))(*segs)
        N.call("tgs_segmented_sort_pairs_u32", N.ptr(k), N.ptr(f), N.ptr(k2), N.ptr(f2), 4,
               n_isects, C, hs, w1, tile_bits, N.ptr(tws), tws.numel(), ctypes.byref(sel), s)
        if sel.value:
            k, f = k2, f2
    ko, fo = to_np(k)[:n_isects].view(np.uint32), to_np(f)[:n_isects]
    # the emission in entry order (each rectangle row by row), then a stable
    # sort on the tile bits within each camera
    cam_of = np.zeros(V, np.int64)
    for c in range(C):
        cam_of[cam[c]:cam[c + 1]] = c
    e = np.repeat(np.arange(V), area)
    w = np.maximum(x1 - x0, 1)
    o = np.arange(len(e)) - np.repeat(np.cumsum(area) - area, area)
    tile = (y0[e] + o // w[e]) * tw + x0[e] + o % w[e]
    k_in = ((cam_of[e] << tile_bits) | tile).astype(np.uint32)
    f_in = ids[e].astype(np.uint32).view(np.int32)
    for a, b in zip(segs[:-1], segs[1:]):
        order = np.argsort(tile[a:b], kind="stable") + a
        np.testing.assert_array_equal(ko[a:b], k_in[order])
        np.testing.assert_array_equal(fo[a:b], f_in[order])
    # and the tile offsets of the sorted keys: each (camera, tile) bucket's
    # first intersection, empty buckets taking the next occupied one's start
    offs = torch.empty(C * tw * th, dtype=torch.int32, device=gpu)
    N.call("tgs_tide_offset_encode", n_isects, N.ptr(k), C, tw, th, tile_bits, N.ptr(offs), s)
    bucket = (ko >> tile_bits).astype(np.int64) * (tw * th) + (ko & ((1 << tile_bits) - 1))
    np.testing.assert_array_equal(
        to_np(offs), np.searchsorted(bucket, np.arange(C * tw * th)).astype(np.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("n,C,tw,th,fill", [
    (1, 1, 3, 2, "first"), (1, 2, 3, 2, "last"), (2, 1, 4, 4, "last"), (3, 3, 5, 1, "rand"),
    (5, 2, 120, 68, "first"), (1000, 4, 17, 9, "rand"), (65537, 16, 120, 68, "rand"),
    (200_000, 3, 120, 68, "sparse")])
def test_tide_offset_encode_matches_lower_bound(gpu, n, C, tw, th, fill):
    """tgs_tide_offset_encode on sorted camera | tile keys gives each bucket the
    index of its first key, and empty buckets the next occupied bucket's
    start (n_isects after the last key): isect_tiles.cu:234-301.  Key counts
    around powers of two (the search's probe width), every key in the first
    or the last bucket, a one-row grid, and keys confined to a few buckets."""
    announce(f"offset encode n={n} C={C} grid={tw}x{th} fill={fill}")
    from tidegs_amd import _native as N
    rng = np.random.default_rng(n + C * 7 + tw)
    tile_bits = (tw * th).bit_length()
    nb = C * tw * th
    if fill == "first":
        b = np.zeros(n, np.int64)
    elif fill == "last":
        b = np.full(n, nb - 1, np.int64)
    elif fill == "sparse":
        b = np.sort(rng.choice(rng.integers(0, nb, 7), n))
    else:
        b = np.sort(rng.integers(0, nb, n))
    keys = (((b // (tw * th)) << tile_bits) | (b % (tw * th))).astype(np.uint32)
    k = torch.from_numpy(keys.view(np.int32)).to(gpu)
    offs = torch.full((nb,), -7, dtype=torch.int32, device=gpu)
    N.call("tgs_tide_offset_encode", n, N.ptr(k), C, tw, th, tile_bits, N.ptr(offs),
           N.stream_handle())
    np.testing.assert_array_equal(to_np(offs), np.searchsorted(b, np.arange(nb)).astype(np.int32))


def test_tide_step_isect_bit_exact(gpu):
    announce("tide step isect")
    sc = _scene(seed=2)
    ts = TideStep(sc.params.to(gpu).contiguous(), sc.width, sc.height, batch_size=sc.n_cams,
                  keep_isect_ids=True)
    ts.forward_backward(sc.viewmats, sc.Ks, sc.gt)
    sp = to_np(ts.last["splats"])
    offs = to_np(ts.last["cam_offsets"])
    C = sc.n_cams
    cams = np.zeros(sp.shape[0], np.int64)
    for c in range(C):
        cams[offs[c]:offs[c + 1]] = c
    tw, th = -(-sc.width // 16), -(-sc.height // 16)
    _, o_ids, o_flat = R.isect_tiles(sp[:, 0:2], sp[:, 7].astype(np.int32), sp[:, 3], 16, tw, th,
                                     camera_ids=cams)
    # the batched key carries the camera id with bit_width(C) bits
    np.testing.assert_array_equal(to_np(ts.last["isect_ids"]), o_ids)
    np.testing.assert_array_equal(to_np(ts.last["flatten_ids"]), o_flat)
    np.testing.assert_array_equal(to_np(ts.last["offsets"]), R.isect_offset_encode(o_ids, C, tw, th))


def test_depth_sort_repair_keeps_reference_order(gpu, monkeypatch):
    """A depth-key range that misses projected keys (forced from the host: the
    range helper returns a base above the smallest keys and too few bits for
    the largest) makes the ranked depth sort tie those keys; the projection's
    own range check then re-sorts on all 32 bits and the intersections are
    still the reference's, bit for bit.  With the true range nothing is
    repaired and every projected key lies inside it."""
    announce("tide step depth sort repair")
    from tidegs_amd import tide_step as TS
    sc = _scene(seed=2)
    C = sc.n_cams
    tw, th = -(-sc.width // 16), -(-sc.height // 16)

    def run(ts):
        ts.forward_backward(sc.viewmats, sc.Ks, sc.gt)
        sp = to_np(ts.last["splats"])
        offs = to_np(ts.last["cam_offsets"])
        cams = np.zeros(sp.shape[0], np.int64)
        for c in range(C):
            cams[offs[c]:offs[c + 1]] = c
        _, o_ids, o_flat = R.isect_tiles(sp[:, 0:2], sp[:, 7].astype(np.int32), sp[:, 3], 16,
                                         tw, th, camera_ids=cams)
        np.testing.assert_array_equal(to_np(ts.last["isect_ids"]), o_ids)
        np.testing.assert_array_equal(to_np(ts.last["flatten_ids"]), o_flat)
        return sp

    ts = TideStep(sc.params.to(gpu).contiguous(), sc.width, sc.height, batch_size=C,
                  keep_isect_ids=True)
    sp = run(ts)
    assert ts.depth_sort_repairs == 0
    keys = sp[:, 3].view(np.uint32)[sp[:, 7] > 0].astype(np.int64)
    true_range = TS.depth_key_range(int(keys.min()), int(keys.max()))
    base, bits = true_range
    assert keys.min() >= base and keys.max() - base < (1 << bits) - 1

    def narrow(lo, hi):
        return lo + (hi - lo) // 4, max(1, ((hi - lo) // 4).bit_length())

    monkeypatch.setattr(TS, "depth_key_range", narrow)
    ts2 = TideStep(sc.params.to(gpu).contiguous(), sc.width, sc.height, batch_size=C,
                   keep_isect_ids=True)
    run(ts2)
    assert ts2.depth_sort_repairs == 1


@pytest.mark.parametrize("pitch", [59, 64])
def test_tide_step_optimizer_untouched_rows_bitwise(gpu, pitch):
    announce(f"tide step optimizer row pitch={pitch}")
    sc = _scene(seed=3, n=20000, C=2)
    params = sc.params.to(gpu).contiguous()
    if pitch == 64:
        params = scenes.padded_table(params)
    before = params.clone()
    ts = TideStep(params, sc.width, sc.height, batch_size=2, block_size=4096)
    touched, grads, stats = ts.forward_backward(sc.viewmats, sc.Ks, sc.gt)
    g = grads.clone()
    t = touched.long().clone()
    out = ts.optimizer_step(touched, grads)
    assert out["touched_rows"] == t.numel() and out["cold_rows"] == t.numel()
    mask = torch.ones(params.shape[0], dtype=torch.bool, device=gpu)
    mask[t] = False
    assert torch.equal(params[mask], before[mask])
    if pitch == 64:  # the padding columns keep their bits (zeros)
        assert not bool(params.as_strided((params.shape[0], 64), (64, 1))[:, 59:].any())
    # touched rows follow the closed-form first Adam step with TideGS's sqrt-mode
    # scaling (gaussian_model.py:855-888): lr*sqrt(bsz), betas^bsz, eps/sqrt(bsz)
    lr_groups = np.array([1.6e-4, 0.05, 5e-3, 1e-3, 2.5e-3, 2.5e-3 / 20.0]) * np.sqrt(2)
    # CACHE column order: xyz, scale, rot, opacity, dc, rest
    lr_cols = np.concatenate([[lr_groups[0]] * 3, [lr_groups[2]] * 3, [lr_groups[3]] * 4,
                              [lr_groups[1]], [lr_groups[4]] * 3, [lr_groups[5]] * 45])
    b1, b2 = 0.9 ** 2, 0.999 ** 2
    p_ref, _, _ = O.adam_rows(to_np(before)[to_np(t)].astype(np.float64),
                              to_np(g).astype(np.float64), 0.0, 0.0, lr_cols, b1, b2,
                              1e-15 / np.sqrt(2), 2.0, 1 - b1, np.sqrt(1 - b2))
    np.testing.assert_allclose(to_np(params)[to_np(t)], p_ref, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("optimizer,pitch,block_size", [("adam", 64, 1024), ("adam", 59, 1000),
                                                        ("sophia", 64, 1024)])
def test_fused_update_matches_two_launch_step(gpu, optimizer, pitch, block_size):
    """tgs_tide_project_bwd_update (projection backward with the optimizer
    update in the same launch) against tgs_tide_project_bwd +
    GPUResidentAdam/Sophia.step over the materialised gradient rows, on the
    same per-entry splat gradients (the rasterizer backward accumulates those
    with float atomics, so two separate steps differ in their last bits and
    Adam's normalised update amplifies that for near-zero gradients).  Three
    steps; parameters and moments agree (both kernels inline one update with
    pinned rounding, so they are expected bitwise equal; the bound allows a
    few ulps), the optimizer's stats are equal, and rows no
    camera sees keep their bits.  Blocks of 1000/1024 rows make wavefront runs
    cross resident blocks (the non-power-of-two size takes the layout search)."""
    announce(f"tide step fused update {optimizer} pitch={pitch} block={block_size}")
    from tidegs_amd import _native as N

    sc = _scene(seed=4, n=20000, C=3)

    def table():
        p = sc.params.to(gpu).contiguous()
        return scenes.padded_table(p) if pitch == 64 else p

    kw = dict(batch_size=3, block_size=block_size, optimizer=optimizer)
    fused = TideStep(table(), sc.width, sc.height, **kw)
    split = TideStep(table(), sc.width, sc.height, fuse_update=False, **kw)
    # evict every block, admit the second half, then all: the first half
    # lands in the slots after the second half's, so the block -> slot map is
    # not the identity
    for ts in (fused, split):
        blocks = list(ts.manager.loaded_blocks)
        ts.optimizer.set_resident_blocks([])
        ts.optimizer.set_resident_blocks(blocks[len(blocks) // 2:])
        ts.optimizer.set_resident_blocks(blocks)
    slots = [fused.optimizer.slot_of(b) for b in fused.manager.loaded_blocks]
    assert slots != sorted(slots) and sorted(slots) == list(range(len(slots)))
    before = fused.params.clone()
    idle = np.ones(sc.params.shape[0], dtype=bool)  # rows that no camera saw in any step
    s = N.stream_handle(gpu)
    vm = sc.viewmats.to(gpu, torch.float32).contiguous()  # alive across the launches
    Ks = sc.Ks.to(gpu, torch.float32).contiguous()
    for it in range(1, 4):
        touched, grads, stats = split.forward_backward(sc.viewmats, sc.Ks, sc.gt)
        L = split.last
        idle &= to_np(L["masks"])[: sc.params.shape[0]] == 0
        T = touched.numel()
        counts = fused.optimizer.launch_touch_counts(fused.gaussians, touched)
        torch.cuda.synchronize()
        args, fstats = fused.optimizer.fused_update_args(it, fused.gaussians, T, counts)
        N.call("tgs_tide_project_bwd_update", T, N.ptr(touched), N.ptr(L["visit_base"]),
               N.ptr(L["visits"]), N.ptr(L["masks"]), sc.n_cams, N.ptr(fused.params),
               fused.row_stride, N.ptr(vm), N.ptr(Ks), N.ptr(L["campos"]), sc.width, sc.height,
               fused.eps2d, fused.near, fused.far, 0.0, fused.sh_degree, N.ptr(L["splat_grads"]),
               *args, s)
        sstats = split.optimizer_step(touched, grads)
        assert fstats == sstats and fstats["touched_rows"] == T > 0
        pf, ps = to_np(fused.params), to_np(split.params)
        print(f"  step {it}: {int((pf != ps).sum())} of {pf.size} parameters differ")
        np.testing.assert_allclose(pf, ps, rtol=2e-6, atol=1e-9)
    of, os_ = fused.optimizer, split.optimizer
    np.testing.assert_allclose(to_np(of._exp_avg), to_np(os_._exp_avg), rtol=1e-5, atol=1e-12)
    np.testing.assert_allclose(to_np(of._exp_avg_sq), to_np(os_._exp_avg_sq), rtol=1e-5,
                               atol=1e-18)
    assert of.get_stats() == os_.get_stats()
    assert idle.any()
    np.testing.assert_array_equal(to_np(fused.params)[idle], to_np(before)[idle])
    if pitch == 64:  # the padding columns keep their bits (zeros)
        full = fused.params.as_strided((sc.params.shape[0], 64), (64, 1))
        assert not bool(full[:, 59:].any())
    # step() wires the same launch: one more batch each way, same bookkeeping
    fused._iteration = split._iteration
    a = fused.step(sc.viewmats, sc.Ks, sc.gt)
    b = split.step(sc.viewmats, sc.Ks, sc.gt)
    assert a.optimizer == b.optimizer and a.optimizer["touched_rows"] == a.touched_rows
    np.testing.assert_allclose(a.losses(sc.width, sc.height), b.losses(sc.width, sc.height),
                               rtol=1e-5)
    assert fused.last["grads"] is None and of.get_stats() == os_.get_stats()


def test_fused_step_trains(gpu):
    """End to end: repeated fused steps (forward, backward, update in the
    projection-backward launch) fit the targets: the batch loss falls and the
    table stays finite."""
    announce("tide step: 40 fused training steps")
    sc = _scene(seed=5, n=6000, C=3)
    ts = TideStep(sc.params.to(gpu).contiguous(), sc.width, sc.height, batch_size=sc.n_cams)
    losses = []
    for _ in range(40):
        st = ts.step(sc.viewmats, sc.Ks, sc.gt)
        losses.append(sum(st.losses(sc.width, sc.height)) / sc.n_cams)
    print(f"  loss {losses[0]:.5f} -> {losses[-1]:.5f}")
    assert bool(torch.isfinite(ts.params).all())
    assert losses[-1] < 0.97 * losses[0]
    assert sum(losses[-5:]) < sum(losses[:5])
