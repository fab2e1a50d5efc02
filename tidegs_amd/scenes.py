"""Seeded synthetic scenes for the benchmark configurations.

The resident table is ``[N, 59]`` fp32 in TideGS's CACHE column order
(``storage/block_reader.py:35-44``, ``double_buffer_gpu.py:726-734``):
``xyz | log-scale | quat (w,x,y,z) | opacity logit | SH dc (3) | SH rest (45)``,
SH coefficient k / channel c at column ``11 + 3k + c``.

Cameras follow the OpenCV/Inria convention used by TideGS (x right, y down,
z forward; ``viewmat`` = world-to-camera, row-major).  Ground-truth images are
``[3, H, W]`` on a 0..255 scale, as ``camera.original_image`` is consumed by
``strategies/base_engine.py:476``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

ROW = 59
COL_XYZ = slice(0, 3)
COL_SCALE = slice(3, 6)
COL_ROT = slice(6, 10)
COL_OPAC = slice(10, 11)
COL_SH = slice(11, 59)
COL_DC = slice(11, 14)
COL_REST = slice(14, 59)


@dataclass
class Scene:
    params: torch.Tensor     # [N, 59] CACHE layout
    viewmats: torch.Tensor   # [C, 4, 4] world-to-camera, row-major
    Ks: torch.Tensor         # [C, 3, 3]
    width: int
    height: int
    gt: torch.Tensor         # [C, 3, H, W], 0..255
    name: str = ""

    @property
    def n(self) -> int:
        return self.params.shape[0]

    @property
    def n_cams(self) -> int:
        return self.viewmats.shape[0]

    def to(self, device) -> "Scene":
        return Scene(self.params.to(device), self.viewmats.to(device), self.Ks.to(device),
                     self.width, self.height, self.gt.to(device), self.name)

    def camtoworlds(self) -> torch.Tensor:
        return torch.linalg.inv(self.viewmats.double()).float()


def _gaussian_rows(g: torch.Generator, n: int, means: torch.Tensor, log_scale_mu: float,
                   log_scale_sigma: float) -> torch.Tensor:
    dev = means.device
    p = torch.empty((n, ROW), dtype=torch.float32, device=dev)
    p[:, COL_XYZ] = means
    p[:, COL_SCALE] = torch.randn((n, 3), generator=g, device=dev) * log_scale_sigma + log_scale_mu
    q = torch.randn((n, 4), generator=g, device=dev)
    p[:, COL_ROT] = q / q.norm(dim=1, keepdim=True)
    p[:, COL_OPAC] = torch.randn((n, 1), generator=g, device=dev)
    p[:, COL_SH] = torch.randn((n, 48), generator=g, device=dev) * 0.2
    return p


def look_at(eye, target, up=(0.0, 0.0, 1.0)) -> torch.Tensor:
    """World-to-camera [4,4] (OpenCV: z forward, y down) looking from eye at target."""
    eye = torch.tensor(eye, dtype=torch.float64)
    target = torch.tensor(target, dtype=torch.float64)
    up = torch.tensor(up, dtype=torch.float64)
    f = target - eye
    f = f / f.norm()
    r = torch.linalg.cross(f, up)
    if r.norm() < 1e-8:
        r = torch.linalg.cross(f, torch.tensor([0.0, 1.0, 0.0], dtype=torch.float64))
    r = r / r.norm()
    d = torch.linalg.cross(f, r)  # camera y (down)
    R = torch.stack([r, d, f], 0)
    w2c = torch.eye(4, dtype=torch.float64)
    w2c[:3, :3] = R
    w2c[:3, 3] = -R @ eye
    return w2c.float()


def _intrinsics(f: float, W: int, H: int) -> torch.Tensor:
    return torch.tensor([[f, 0.0, W / 2.0], [0.0, f, H / 2.0], [0.0, 0.0, 1.0]])


def padded_table(p: torch.Tensor, pitch: int = 64) -> torch.Tensor:
    """The same [N, 59] table stored at a row pitch of ``pitch`` floats (the
    extra columns zero): a [N, 59] view whose rows start on 256-byte
    boundaries at pitch 64, so that a row is exactly two cache lines."""
    out = torch.zeros((p.shape[0], pitch), dtype=p.dtype, device=p.device)
    out[:, :ROW] = p
    return out[:, :ROW]


BLOCK_ROWS = 4096  # rows per block of TideGS's block store (arguments/__init__.py:190)


def morton_codes(xyz: torch.Tensor) -> torch.Tensor:
    """30-bit Morton codes of ``xyz`` over its bounds, as the streaming
    initializer computes them (``storage/streaming_ply_init.py:154-168``: 10
    bits per axis, x in the lowest bit of each triple), as int64."""
    xyz = xyz.float()
    lo, hi = xyz.min(0).values, xyz.max(0).values
    q = ((xyz - lo) / (hi - lo + 1e-8) * 1023.0).to(torch.int64).clamp(0, 1023)

    def spread(v):
        v = (v | (v << 16)) & 0x030000FF
        v = (v | (v << 8)) & 0x0300F00F
        v = (v | (v << 4)) & 0x030C30C3
        return (v | (v << 2)) & 0x09249249

    return spread(q[:, 0]) | (spread(q[:, 1]) << 1) | (spread(q[:, 2]) << 2)


def block_layout(params: torch.Tensor, block_rows: int = BLOCK_ROWS, seed: int = 0) -> torch.Tensor:
    """The row order of a TideGS resident table, as a permutation of ``params``'
    rows.  The streaming initializer writes the base file's rows in stable
    Morton order (``storage/streaming_ply_init.py:359``), the block store and
    the working set move them in blocks of 4096 rows (``log_storage_manager.py
    :280-291``, ``gpu_working_set.py``), and a resident set holds its blocks in
    whatever slots its transitions gave them: rows in Morton order within each
    block, the blocks in a seeded random order.  The scene (its Gaussians,
    visible entries, intersections and pixels) is the same in any row order;
    what changes is how close in memory the Gaussians one tile touches lie."""
    # on the host: a one-off set-up step, kept out of the device's kernel stream
    order = torch.argsort(morton_codes(params[:, :3].cpu()), stable=True)
    n = order.numel()
    nb = -(-n // block_rows)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))
    idx = (perm[:, None] * block_rows + torch.arange(block_rows)[None]).flatten()
    return order[idx[idx < n]].to(params.device)


def cfg1(seed: int = 0, n: int = 10_000) -> Scene:
    """10k Gaussians, one 256x256 pinhole (fx=fy=256) at the origin looking +z."""
    g = torch.Generator().manual_seed(seed)
    xy = torch.rand((n, 2), generator=g) * 2 - 1
    z = torch.rand((n, 1), generator=g) * 4 + 2
    p = _gaussian_rows(g, n, torch.cat([xy, z], 1), -4.5, 0.5)
    W = H = 256
    gt = torch.rand((1, 3, H, W), generator=g) * 255.0
    return Scene(p, torch.eye(4)[None], _intrinsics(256.0, W, H)[None], W, H, gt, "cfg1")


def cfg2(seed: int = 0, n: int = 1_000_000) -> Scene:
    """1M Gaussians in x,y in [-10,10], depth 5..40, one 1920x1080 camera (f=1100)."""
    g = torch.Generator().manual_seed(seed)
    xy = torch.rand((n, 2), generator=g) * 20 - 10
    z = torch.rand((n, 1), generator=g) * 35 + 5
    p = _gaussian_rows(g, n, torch.cat([xy, z], 1), -4.5, 0.5)
    W, H = 1920, 1080
    gt = torch.rand((1, 3, H, W), generator=g) * 255.0
    return Scene(p, torch.eye(4)[None], _intrinsics(1100.0, W, H)[None], W, H, gt, "cfg2")


def orbit_cameras(n_cams: int, center=(0.0, 0.0, 10.0), radius: float = 70.0,
                  height: float = 35.0, arc_deg: float = 90.0):
    """Poses on a smooth arc around `center`, all looking at it."""
    mats = []
    for i in range(n_cams):
        a = math.radians(-arc_deg / 2 + arc_deg * (i / max(1, n_cams - 1)))
        eye = (center[0] + radius * math.cos(a), center[1] + radius * math.sin(a),
               center[2] + height)
        mats.append(look_at(eye, center))
    return torch.stack(mats, 0)


def cfg3(seed: int = 0, n: int = 4_000_000, n_cams: int = 16, width: int = 1920,
         height: int = 1080, with_gt: bool = True) -> Scene:
    """4M Gaussians in a 100x100x20 box (log-scales N(-3.5, 0.7)), 16 cameras on an
    orbit arc, 1920x1080, f=1100: the north-star training-step configuration."""
    g = torch.Generator().manual_seed(seed)
    xy = torch.rand((n, 2), generator=g) * 100 - 50
    z = torch.rand((n, 1), generator=g) * 20
    p = _gaussian_rows(g, n, torch.cat([xy, z], 1), -3.5, 0.7)
    vm = orbit_cameras(n_cams)
    Ks = _intrinsics(1100.0, width, height)[None].repeat(n_cams, 1, 1)
    gt = (torch.rand((n_cams, 3, height, width), generator=g) * 255.0 if with_gt
          else torch.empty((n_cams, 3, height, width)))
    return Scene(p, vm, Ks, width, height, gt, "cfg3")


def cfg4(seed: int = 0, n: int = 16_000_000, n_cams: int = 4, width: int = 1920,
         height: int = 1080, n_buildings: int = 3000, building_frac: float = 0.6,
         log_scale_mu: float = -1.3, log_scale_sigma: float = 0.5, distance: float = 260.0,
         with_gt: bool = True, device="cpu") -> Scene:
    """Dense aerial city: a 1 km x 1 km ground plane (z ~ N(0, 0.3)) holding
    ``1 - building_frac`` of the Gaussians, and ``n_buildings`` box-shaped
    clusters (footprint half-widths U[5, 15] m, log-normal heights with median
    20 m and log-sigma 0.6) holding the rest, spread uniformly inside each box
    with a building drawn in proportion to its volume.  ``n_cams`` oblique
    cameras (45 degrees down, ``distance`` m out and up) on a 10-degree heading
    step look at the centre, 1920x1080, f = 1100.  At the defaults a camera
    sees about 8M Gaussians and 19M intersections, 2.4k per tile on average,
    with the hottest tiles above 9k (p99) and 16k (max).

    The random streams are drawn on ``device`` (the 16M-row table takes about
    40 s on a few CPU cores, well under a second on a GPU); a scene is
    reproducible for a given seed and device type."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    n_b = int(n * building_frac)
    n_g = n - n_b

    def rand(*shape):
        return torch.rand(shape, generator=g, device=dev)

    ground = torch.cat([rand(n_g, 2) * 1000 - 500,
                        torch.randn((n_g, 1), generator=g, device=dev) * 0.3], 1)
    centre = rand(n_buildings, 2) * 960 - 480
    half = rand(n_buildings, 2) * 10 + 5
    heights = torch.exp(torch.randn((n_buildings,), generator=g, device=dev) * 0.6 +
                        math.log(20.0))
    cdf = torch.cumsum((half[:, 0] * half[:, 1] * heights).double(), 0)
    which = torch.searchsorted(cdf / cdf[-1], rand(n_b).double()).clamp_(max=n_buildings - 1)
    u = rand(n_b, 3)
    bxy = centre[which] + (u[:, :2] * 2 - 1) * half[which]
    bz = u[:, 2:3] * heights[which][:, None]
    means = torch.cat([ground, torch.cat([bxy, bz], 1)], 0)
    p = _gaussian_rows(g, n, means, log_scale_mu, log_scale_sigma)
    mats = []
    for i in range(n_cams):
        a = math.radians(-90.0 + 10.0 * i)
        eye = (distance * math.cos(a), distance * math.sin(a), distance)
        mats.append(look_at(eye, (0.0, 0.0, 0.0)))
    vm = torch.stack(mats, 0).to(dev)
    Ks = _intrinsics(1100.0, width, height)[None].repeat(n_cams, 1, 1).to(dev)
    gt = (rand(n_cams, 3, height, width) * 255.0 if with_gt
          else torch.empty((n_cams, 3, height, width), device=dev))
    return Scene(p, vm, Ks, width, height, gt, "cfg4")


@dataclass
class OptimizerCase:
    table: torch.Tensor   # [N, 59] parameters
    rows: torch.Tensor    # [T] int32, sorted ascending, distinct
    grads: torch.Tensor   # [T, 59]


def cfg5(seed: int = 0, n: int = 32_000_000, visible_frac: float = 0.3,
         grad_sigma: float = 1e-3, device="cpu") -> OptimizerCase:
    """Optimizer-only case: a resident ``[n, 59]`` table (N(0, 1) entries), a
    sorted ascending int32 set of ``visible_frac * n`` distinct rows and
    N(0, grad_sigma) gradients for those rows.  Generated on ``device`` (the
    full 32M-row case is 7.5 GB per array)."""
    g = torch.Generator(device=device).manual_seed(seed)
    table = torch.randn((n, ROW), generator=g, device=device)
    t = int(visible_frac * n)
    rows = torch.randperm(n, generator=g, device=device)[:t].sort().values.to(torch.int32)
    grads = torch.randn((t, ROW), generator=g, device=device) * grad_sigma
    return OptimizerCase(table, rows, grads)


def small(seed: int = 0, n: int = 2000, n_cams: int = 2, W: int = 96, H: int = 64,
          log_scale_mu: float = -2.5) -> Scene:
    """Small multi-camera scene for parity tests (oracle finishes in seconds)."""
    g = torch.Generator().manual_seed(seed)
    xy = torch.rand((n, 2), generator=g) * 4 - 2
    z = torch.rand((n, 1), generator=g) * 4 + 3
    p = _gaussian_rows(g, n, torch.cat([xy, z], 1), log_scale_mu, 0.5)
    mats = []
    for i in range(n_cams):
        eye = (0.3 * i, -0.2 * i, 0.0)
        mats.append(look_at(eye, (0.0, 0.0, 5.0), up=(0.0, -1.0, 0.0)))
    vm = torch.stack(mats, 0)
    Ks = _intrinsics(0.9 * W, W, H)[None].repeat(n_cams, 1, 1)
    gt = torch.rand((n_cams, 3, H, W), generator=g) * 255.0
    return Scene(p, vm, Ks, W, H, gt, "small")


def activations(params: torch.Tensor):
    """Split a CACHE-layout table into TideGS's activated inputs
    (base_gaussian_model.py:35-50): means, quats (normalised), scales (exp),
    opacities (sigmoid), SH coefficients [N,16,3]."""
    means = params[:, COL_XYZ]
    q = params[:, COL_ROT]
    quats = torch.nn.functional.normalize(q, dim=-1)
    scales = torch.exp(params[:, COL_SCALE])
    opac = torch.sigmoid(params[:, COL_OPAC]).squeeze(1)
    sh = params[:, COL_SH].reshape(-1, 16, 3)
    return means, quats, scales, opac, sh
