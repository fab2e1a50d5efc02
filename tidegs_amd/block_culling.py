"""Block frustum culling on the GPU (drop-in for ``storage/gaussian_block.py``'s
``FrustumCuller``, 6-plane mode).

Each 4096-Gaussian block is a bounding sphere (centre = midpoint of its xyz
bounds, radius = half the bounds diagonal x 1.15); a block is visible from a
camera when the signed distance of its centre to every one of the six
normalized frustum planes is at least -radius (``gaussian_block.py:264-532``).
The sphere table lives in HBM next to the block bounds that
``ResidentWorkingSet.stage_block_bounds`` produces, and one launch
(``tgs_cull_blocks``) tests all blocks against up to 32 cameras, setting one
bit per camera, with the reference's float32 operation order so the visible
lists are identical.  Plane extraction (a 4x4 product per camera) stays on the
host, as in the reference.
"""
from __future__ import annotations

import threading
import warnings
from typing import List, Sequence

import numpy as np
import torch

from . import _native as N

MAX_CAMERAS_PER_LAUNCH = 32


def extract_frustum_planes(view_matrix: np.ndarray, proj_matrix: np.ndarray,
                           coordinate_system: str = "opengl", validate: bool = True) -> np.ndarray:
    """(6,4) float32 planes, order left, right, bottom, top, near, far, each
    scaled to a unit normal (Gribb-Hartmann; gaussian_block.py:145-228)."""
    view = np.array(view_matrix, copy=True)
    if coordinate_system == "opencv":
        view = np.diag(np.float32([1, -1, -1, 1])) @ view
    vp = proj_matrix @ view
    planes = np.zeros((6, 4), dtype=np.float32)
    for k in range(6):
        row = k // 2  # x, y, z clip rows; even k adds, odd k subtracts
        planes[k] = vp[3, :] + vp[row, :] if k % 2 == 0 else vp[3, :] - vp[row, :]
    for k in range(6):
        length = np.sqrt(planes[k, 0] ** 2 + planes[k, 1] ** 2 + planes[k, 2] ** 2)
        if length > 1e-8:
            planes[k] /= length
        else:
            raise ValueError(f"Degenerate frustum plane {k}: normal length = {length}")
    if validate and coordinate_system == "opengl":
        if planes[4, 2] > 0 or planes[5, 2] < 0:
            warnings.warn(f"Suspicious plane orientations: near_z={planes[4, 2]:.3f}, "
                          f"far_z={planes[5, 2]:.3f}. Expected near_z < 0 and far_z > 0 for "
                          "OpenGL. Check projection matrix.")
    return planes


def camera_view_projection(R, T, fov_y: float, width=None, height=None,
                           scene_radius: float = 0.0):
    """(camera position, OpenGL view matrix, projection matrix) of a COLMAP-style
    camera (R, T) as TideStorageAdapter.get_visible_blocks builds them
    (storage/tide_storage_adapter.py:685-723)."""
    R = np.array(R).reshape(3, 3)
    T = np.array(T).reshape(3, 1)
    position = (-R @ T).flatten()
    view = np.eye(4, dtype=np.float32)
    view[:3, :3] = R.T
    view[:3, 3] = T.flatten()
    view = np.diag(np.float32([1, -1, -1, 1])) @ view
    aspect = width / height if (width is not None and height is not None) else 16.0 / 9.0
    near, far = 0.01, max(float(scene_radius) * 2.0, 1000.0)
    f = 1.0 / np.tan(fov_y / 2.0)
    proj = np.array([[f / aspect, 0, 0, 0], [0, f, 0, 0],
                     [0, 0, -(far + near) / (far - near), -2 * far * near / (far - near)],
                     [0, 0, -1, 0]], dtype=np.float32)
    return position, view, proj


class FrustumCuller:
    """GPU 6-plane block culling over ``block_bounds`` [num_blocks, 6]
    (min xyz, max xyz)."""

    def __init__(self, block_bounds, scene_radius: float | None = None, block_size: int = 4096,
                 verbose: bool = False, device="cuda"):
        self.device = torch.device(device)
        b = torch.as_tensor(np.asarray(block_bounds, dtype=np.float32) if not torch.is_tensor(
            block_bounds) else block_bounds, dtype=torch.float32)
        if b.dim() != 2 or b.shape[1] != 6:
            raise ValueError(f"block_bounds must be [num_blocks, 6], got {tuple(b.shape)}")
        self.bounds = b.to(self.device).contiguous()
        self.num_blocks = int(self.bounds.shape[0])
        self.scene_radius = scene_radius
        self.block_size = block_size
        self.verbose = bool(verbose)
        self._lock = threading.RLock()
        self.centers = torch.empty((self.num_blocks, 3), dtype=torch.float32, device=self.device)
        self.radii = torch.empty(self.num_blocks, dtype=torch.float32, device=self.device)
        self._spheres()
        # legacy scalar radius (the largest block radius), kept like the reference's
        self.block_radius = float(self.radii.max()) if self.num_blocks else 0.0

    def _spheres(self) -> None:
        N.call("tgs_cull_block_spheres", N.ptr(self.bounds), self.num_blocks, N.ptr(self.centers),
               N.ptr(self.radii), N.stream_handle(self.device))

    @property
    def block_bounds(self) -> np.ndarray:
        return self.bounds.cpu().numpy()

    @property
    def block_centers(self) -> np.ndarray:
        return self.centers.cpu().numpy()

    @property
    def block_radii(self) -> np.ndarray:
        return self.radii.cpu().numpy()

    def update_block_bounds(self, block_ids, block_bounds: np.ndarray) -> int:
        """Replace the bounds of ``block_ids`` (gaussian_block.py:315-339)."""
        ids = np.asarray(block_ids, dtype=np.int64)
        if ids.size == 0:
            return 0
        bounds = np.asarray(block_bounds, dtype=np.float32)
        if bounds.shape != (ids.size, 6):
            raise ValueError(f"Expected block_bounds shape {(ids.size, 6)}, got {bounds.shape}")
        with self._lock:
            idx = torch.from_numpy(ids).to(self.device)
            self.bounds.index_copy_(0, idx, torch.from_numpy(bounds).to(self.device))
            self._spheres()
            self.block_radius = max(self.block_radius, float(self.radii[idx].max()))
        return int(ids.size)

    def cull_masks(self, planes: np.ndarray, block_ids=None) -> torch.Tensor:
        """Device u32 masks: bit c of entry i = block (i, or block_ids[i]) is
        visible from camera c of ``planes`` [C, 6, 4] (C <= 32)."""
        planes = np.ascontiguousarray(planes, dtype=np.float32).reshape(-1, 6, 4)
        C = planes.shape[0]
        if not 1 <= C <= MAX_CAMERAS_PER_LAUNCH:
            raise ValueError(f"1..{MAX_CAMERAS_PER_LAUNCH} cameras per launch, got {C}")
        ids = None
        n = self.num_blocks
        if block_ids is not None:
            ids = torch.as_tensor(np.asarray(block_ids, dtype=np.int64)).to(self.device)
            n = int(ids.numel())
        masks = torch.empty(n, dtype=torch.int32, device=self.device)
        p = torch.from_numpy(planes).to(self.device)
        with self._lock:
            N.call("tgs_cull_blocks", N.ptr(self.centers), N.ptr(self.radii), N.ptr(ids), n,
                   N.ptr(p), C, N.ptr(masks), N.stream_handle(self.device))
        return masks

    def cull_batch(self, view_matrices: Sequence[np.ndarray],
                   projection_matrices: Sequence[np.ndarray]) -> List[List[int]]:
        """Visible block lists (ascending) of several cameras from one launch
        per 32 cameras."""
        planes = np.stack([extract_frustum_planes(v, p)
                           for v, p in zip(view_matrices, projection_matrices)])
        out: List[List[int]] = []
        for c0 in range(0, planes.shape[0], MAX_CAMERAS_PER_LAUNCH):
            part = planes[c0:c0 + MAX_CAMERAS_PER_LAUNCH]
            m = self.cull_masks(part).cpu().numpy().view(np.uint32)
            for c in range(part.shape[0]):
                out.append(np.nonzero(m & np.uint32(1 << c))[0].tolist())
        return out

    def cone_flags(self, camera_position, view_matrix, margin: float = 1.0) -> torch.Tensor:
        """Device uint8 flags of the legacy cone + distance test
        (gaussian_block.py:465-510) for every block: within
        min(scene_radius / 2, 100) * margin of the camera (50 * margin without
        a scene radius) and either at it or at a cosine > -0.3 from its
        forward axis (view row 2)."""
        max_view_distance = (min(self.scene_radius * 0.5, 100.0) if self.scene_radius is not None
                             else 50.0)
        threshold = max_view_distance * margin
        fwd = np.asarray(view_matrix, dtype=np.float64)[2, :3]
        fwd = fwd / (np.linalg.norm(fwd) + 1e-8)
        cam = np.asarray(camera_position, dtype=np.float64).reshape(3)
        flags = torch.empty(self.num_blocks, dtype=torch.uint8, device=self.device)
        with self._lock:
            N.call("tgs_cull_blocks_cone", N.ptr(self.centers), self.num_blocks, float(cam[0]),
                   float(cam[1]), float(cam[2]), float(fwd[0]), float(fwd[1]), float(fwd[2]),
                   float(threshold), N.ptr(flags), N.stream_handle(self.device))
        return flags

    def cull(self, camera_position, view_matrix, projection_matrix, margin: float = 1.0,
             use_6plane: bool = True) -> List[int]:
        """Visible blocks of one camera, ascending (gaussian_block.py:341-354);
        ``use_6plane=False`` runs the legacy cone + distance test."""
        if not use_6plane:
            flags = self.cone_flags(camera_position, view_matrix, margin)
            return torch.nonzero(flags).flatten().cpu().tolist()
        return self.cull_batch([view_matrix], [projection_matrix])[0]

    def cull_subset(self, camera_position, view_matrix, projection_matrix, block_ids,
                    margin: float = 1.0, use_6plane: bool = True) -> List[int]:
        """The 6-plane test on ``block_ids`` only, in their given order
        (gaussian_block.py:356-399); ``use_6plane=False`` keeps the ids the
        legacy full-scene test finds visible, in their given order."""
        if isinstance(block_ids, set):
            block_ids = sorted(block_ids)
        ids = np.asarray(block_ids, dtype=np.int64)
        if ids.size == 0:
            return []
        if np.any(ids < 0) or np.any(ids >= self.num_blocks):
            raise ValueError("block_ids contains an out-of-range block")
        if not use_6plane:
            flags = self.cone_flags(camera_position, view_matrix, margin).cpu().numpy()
            return ids[flags[ids] != 0].tolist()
        planes = extract_frustum_planes(view_matrix, projection_matrix)[None]
        m = self.cull_masks(planes, block_ids=ids).cpu().numpy()
        return ids[m != 0].tolist()

    def get_visibility_order(self, visible_blocks: List[int], camera_position) -> List[int]:
        """Visible blocks front to back by centre distance (gaussian_block.py:516-532);
        equal distances keep their input order."""
        if not visible_blocks:
            return []
        with self._lock:
            centers = self.centers[torch.as_tensor(visible_blocks, device=self.device)].cpu().numpy()
        diff = centers - camera_position
        dist_sq = np.sum(diff ** 2, axis=1)
        return [visible_blocks[i] for i in np.argsort(dist_sq, kind="stable")]
