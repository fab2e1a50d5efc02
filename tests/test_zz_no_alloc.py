"""The allocation-free radix sort (tgs_radix_sort_pairs_noalloc, the one entry
point that takes no workspace) against tgs_radix_sort_pairs with a workspace:
bit-identical keys and values on calls in a row, each smaller than the one
before (the scratch array keeps the previous call's contents, which must not
matter), from its 2^25-key maximum down; a size above the maximum is refused
on the host with an error text, before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from tests.gpu_util import announce
from tidegs_amd import _native as N

pytestmark = pytest.mark.gpu

MAX_KEYS = 1 << 25


def _sort(entry, keys, vals, begin, end, gpu):
    k, v = keys.clone(), vals.clone()
    k_alt, v_alt = torch.empty_like(k), torch.empty_like(v)
    sel = ctypes.c_int(-1)
    s = N.stream_handle(gpu)
    if entry == "noalloc":
        N.call("tgs_radix_sort_pairs_noalloc", N.ptr(k), N.ptr(v), N.ptr(k_alt), N.ptr(v_alt),
               k.numel(), begin, end, ctypes.byref(sel), s)
    else:
        ws = torch.empty(max(1, N.load().tgs_radix_sort_workspace_size(k.numel())),
                         dtype=torch.uint8, device=gpu)
        N.call("tgs_radix_sort_pairs", N.ptr(k), N.ptr(v), N.ptr(k_alt), N.ptr(v_alt), k.numel(),
               begin, end, N.ptr(ws), ws.numel(), ctypes.byref(sel), s)
    torch.cuda.synchronize()
    assert sel.value in (0, 1)
    return (k_alt, v_alt) if sel.value else (k, v)


def test_noalloc_sort_matches_workspace_sort(gpu):
    for n, begin, end, seed in ((MAX_KEYS, 0, 46, 1), (3_000_017, 0, 20, 2), (70_001, 3, 64, 3)):
        announce(f"radix sort without workspace: n={n} bits=[{begin},{end})")
        g = torch.Generator(device=gpu).manual_seed(seed)
        keys = torch.randint(-2 ** 62, 2 ** 62, (n,), generator=g, device=gpu, dtype=torch.int64)
        keys[: n // 3] = keys[n // 3: 2 * (n // 3)]  # duplicate keys exercise stability
        vals = torch.arange(n, dtype=torch.int32, device=gpu)
        ka, va = _sort("noalloc", keys, vals, begin, end, gpu)
        kb, vb = _sort("workspace", keys, vals, begin, end, gpu)
        assert torch.equal(ka, kb) and torch.equal(va, vb)
        span = end - begin
        digits = (ka >> begin) & ((1 << span) - 1) if span < 63 else ka
        if span < 63:
            assert bool((digits[1:] >= digits[:-1]).all())
        assert torch.equal(torch.sort(va.long()).values, torch.arange(n, device=gpu))


def test_noalloc_sort_refuses_more_than_its_maximum(gpu):
    announce("radix sort without workspace: oversize refused on the host")
    sel = ctypes.c_int(-1)
    with pytest.raises(RuntimeError, match="exceed the allocation-free maximum"):
        N.call("tgs_radix_sort_pairs_noalloc", None, None, None, None, MAX_KEYS + 1, 0, 46,
               ctypes.byref(sel), N.stream_handle(gpu))
    assert sel.value == 0
    # nothing was launched: the device is still fine for a small call
    keys = torch.tensor([5, 3, 9, 3, 1], dtype=torch.int64, device=gpu)
    vals = torch.arange(5, dtype=torch.int32, device=gpu)
    k, v = _sort("noalloc", keys, vals, 0, 8, gpu)
    assert k.tolist() == [1, 3, 3, 5, 9] and v.tolist() == [4, 1, 3, 0, 2]
