"""Drop-in for ``clm_kernels.fused_ssim`` (``clm_kernels/__init__.py:23-61``).

``fused_ssim(img1, img2, padding="same", train=True)`` returns the mean SSIM
(11x11 Gaussian window, sigma 1.5, C1 = 0.01^2, C2 = 0.03^2) and is
differentiable w.r.t. ``img1``; used inside TideGS's training loss
(``strategies/base_engine.py:472-488``).
"""
from __future__ import annotations

import torch

from . import _native as N

allowed_padding = ["same", "valid"]


class FusedSSIMMap(torch.autograd.Function):
    @staticmethod
    def forward(ctx, C1, C2, img1, img2, padding="same", train=True):
        img1 = img1.contiguous()
        img2 = img2.contiguous()
        N.require_cuda(img1, img2, names=["img1", "img2"])
        B, CH, H, W = img1.shape
        ssim_map = torch.empty_like(img1)
        if train:
            d1, d2, d3 = (torch.empty_like(img1) for _ in range(3))
        else:
            d1 = d2 = d3 = None
        N.call("tgs_fused_ssim_fwd", B, CH, H, W, float(C1), float(C2), N.ptr(img1), N.ptr(img2),
               N.ptr(ssim_map), N.ptr(d1), N.ptr(d2), N.ptr(d3), N.stream_handle())
        if padding == "valid":
            ssim_map = ssim_map[:, :, 5:-5, 5:-5]
        ctx.save_for_backward(img1.detach(), img2, d1, d2, d3)
        ctx.C1, ctx.C2, ctx.padding = C1, C2, padding
        return ssim_map

    @staticmethod
    def backward(ctx, opt_grad):
        img1, img2, d1, d2, d3 = ctx.saved_tensors
        if d1 is None:
            raise RuntimeError("fused_ssim backward needs train=True in the forward")
        dL_dmap = opt_grad
        if ctx.padding == "valid":
            dL_dmap = torch.zeros_like(img1)
            dL_dmap[:, :, 5:-5, 5:-5] = opt_grad
        dL_dmap = dL_dmap.contiguous()
        B, CH, H, W = img1.shape
        grad = torch.empty_like(img1)
        N.call("tgs_fused_ssim_bwd", B, CH, H, W, float(ctx.C1), float(ctx.C2), N.ptr(img1),
               N.ptr(img2), N.ptr(dL_dmap), N.ptr(d1), N.ptr(d2), N.ptr(d3), N.ptr(grad),
               N.stream_handle())
        return None, None, grad, None, None, None


def fused_ssim(img1, img2, padding="same", train=True):
    C1 = 0.01 ** 2
    C2 = 0.03 ** 2
    assert padding in allowed_padding
    ssim_map = FusedSSIMMap.apply(C1, C2, img1, img2, padding, train)
    return ssim_map.mean()
