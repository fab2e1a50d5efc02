"""Shared helpers for the GPU parity tests."""
import numpy as np
import torch


def rel_l2(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64).ravel()
    ref = np.asarray(ref, dtype=np.float64).ravel()
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / den) if den > 0 else float(np.linalg.norm(got))


def to_np(t):
    return t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)


def clamp_marks(colors) -> np.ndarray:
    """Channels of fused-step splat records whose colour the projection
    clamped (clamp_min(SH + 0.5, 0)): stored as -0.0, given no colour
    gradient by the rasterizer backward."""
    c = np.asarray(colors)
    return np.signbit(c) & (c == 0)


def announce(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)


def check_isect_properties(ts, C, tw, th):
    """The fused step's intersection list equals gsplat's (isect_tiles.cu:14-227)
    bit for bit: with ``(key, flatten_id)`` strictly increasing, every entry
    contributing exactly the tiles of its rectangle, each once, and every key
    carrying its entry's camera, tile and depth bits, the list is the stable
    sort of the reference's emission.  Offsets are the run starts."""
    L = ts.last
    ids, fids = L["isect_ids"], L["flatten_ids"].long()
    sp = L["splats"]
    V = sp.shape[0]
    n = ids.numel()
    assert n == fids.numel() and n > 0
    inc = (ids[1:] > ids[:-1]) | ((ids[1:] == ids[:-1]) & (fids[1:] > fids[:-1]))
    assert bool(inc.all()), "intersections are not in (key, entry) order"
    tile_bits = (tw * th).bit_length()
    cam_offsets = L["cam_offsets"].long()
    cam_of_entry = torch.searchsorted(cam_offsets[1:], torch.arange(V, device=sp.device),
                                      right=True)
    # the rectangle of isect_tiles.cu:55-64 in float32
    r = sp[:, 7] / 16.0
    tx, ty = sp[:, 0] / 16.0, sp[:, 1] / 16.0
    x0 = torch.clamp(torch.floor(tx - r), 0, tw).long()
    x1 = torch.clamp(torch.ceil(tx + r), 0, tw).long()
    y0 = torch.clamp(torch.floor(ty - r), 0, th).long()
    y1 = torch.clamp(torch.ceil(ty + r), 0, th).long()
    live = sp[:, 7] > 0
    area = torch.where(live, (x1 - x0).clamp(min=0) * (y1 - y0).clamp(min=0), 0)
    assert torch.equal(torch.bincount(fids, minlength=V), area), "per-entry tile counts differ"
    cam = ids >> (32 + tile_bits)
    tile = (ids >> 32) & ((1 << tile_bits) - 1)
    dbits = ids & 0xFFFFFFFF
    assert torch.equal(cam, cam_of_entry[fids])
    e_dbits = sp[:, 3].contiguous().view(torch.int32).long() & 0xFFFFFFFF
    assert torch.equal(dbits, e_dbits[fids])
    t_x, t_y = tile % tw, tile // tw
    assert bool(((t_x >= x0[fids]) & (t_x < x1[fids]) & (t_y >= y0[fids]) &
                 (t_y < y1[fids])).all()), "intersection outside its entry's rectangle"
    bucket = cam * (tw * th) + tile
    want = torch.searchsorted(bucket, torch.arange(C * tw * th, device=sp.device)).to(torch.int32)
    assert torch.equal(L["offsets"].reshape(-1), want)
    return bucket
