"""Pin for the composed step oracle (oracle/step_ref.py): its compact row
gradients equal central finite differences of its own float64 loss summed over
the cameras, through activations, SH clamp, projection and compositing."""
import numpy as np
import pytest
import torch

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
