"""Benchmark of the TideGS per-iteration GPU step on one MI355X.

Workload: 4M resident Gaussians in a 100x100x20
box (log-scales N(-3.5, 0.7)), a batch of 16 cameras at 1920x1080 (f=1100)
on a smooth orbit arc, L1 + SSIM loss, full forward + backward and the fused
resident Adam over all 59 columns (TideGS sqrt-mode scaling for bsz 16).
Synthetic, seeded data; fp32 throughout.

Prints ONE JSON line: ms per train step, the roofline of the dominant kernel
(HIP events on the launch stream), per-stage times and the CPU baseline (the
oracle, timed on a bounded sample and extrapolated).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "ms/train-step (fwd+bwd+Adam) at 4M Gaussians, 16×1080p; bwd HBM GB/s"

# Algorithmic bytes per unit of work (fp32), see DESIGN.md "Measurement".
BYTES = {
    "visibility": lambda s: 40 * s["N"] + 4 * s["N"],
    "project_fwd": lambda s: s["T"] * (4 + 4 + 4 + 236) + s["V"] * (4 + 48 + 4 + 8),
    "raster_fwd": lambda s: s["C"] * s["P"] * 20 + s["I"] * 52,
    "raster_bwd": lambda s: s["C"] * s["P"] * 20 + s["I"] * 52 + s["V"] * 36,
    "project_bwd": lambda s: s["T"] * (4 + 4 + 4 + 236 + 236) + s["V"] * (4 + 36),
    "adam": lambda s: s["T"] * 1656,
}


def profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` at cfg3 from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summary (profiles/*_traffic.md), or None."""
    import re

    for f in sorted((ROOT / "profiles").glob("*_traffic.md")):
        m = re.search(rf"^traffic_bytes_per_launch {re.escape(kernel)}: (\d+)", f.read_text(),
                      re.M)
        if m:
            return int(m.group(1))
    return None


def cpu_baseline(width, height, frac_a=1 / 16, frac_b=1 / 8, seed=0):
    """Time the CPU oracle on one camera of the same workload with a random
    subset of the Gaussians at two subset sizes, fit t = t_pix + f * t_gauss,
    and extrapolate to 16 cameras x 4M Gaussians (single thread)."""
    import numpy as np
    import torch

    from oracle import step_ref as SR
    from tidegs_amd import scenes

    torch.set_num_threads(1)
    times = []
    sizes = []
    for frac in (frac_a, frac_b):
        n = int(4_000_000 * frac)
        sc = scenes.cfg3(seed=seed, n=n, n_cams=16, width=width, height=height)
        vm, K, gt = sc.viewmats[:1], sc.Ks[:1], sc.gt[:1]
        t0 = time.perf_counter()
        SR.batch_grads(sc.params, vm, K, gt, width, height, raster_dtype=np.float32,
                       proj_dtype=torch.float32)
        times.append(time.perf_counter() - t0)
        sizes.append(frac)
    slope = (times[1] - times[0]) / (sizes[1] - sizes[0])
    t_pix = max(0.0, times[0] - slope * sizes[0])
    per_cam_full = t_pix + slope * 1.0
    ms_step = per_cam_full * 16 * 1000.0
    return {
        "value": round(ms_step, 1),
        "unit": "ms/train-step (extrapolated)",
        "cores": 1,
        "kind": "port",
        "sample": (f"CPU oracle (oracle/step_ref.py, 1 thread) on 1 camera of the cfg3 workload "
                   f"with {int(4e6 * frac_a)} and {int(4e6 * frac_b)} random Gaussians: "
                   f"{times[0]:.1f}s and {times[1]:.1f}s; linear fit in the Gaussian count, "
                   f"x16 cameras"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--n", type=int, default=4_000_000)
    ap.add_argument("--cams", type=int, default=16)
    ap.add_argument("--width", type=int, default=1920)
    ap.add_argument("--height", type=int, default=1080)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-stage-timing", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run 3 plain device copies of MIB MiB (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the TideGS step is single-GPU; "
              "see DESIGN.md for how it would shard by camera). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from tidegs_amd import scenes
    from tidegs_amd.tide_step import TideStep

    dev = torch.device("cuda:0")
    sc = scenes.cfg3(seed=0, n=args.n, n_cams=args.cams, width=args.width, height=args.height,
                     with_gt=True).to(dev)
    ts = TideStep(sc.params.contiguous(), sc.width, sc.height, batch_size=args.cams)

    for _ in range(args.warmup):
        ts.step(sc.viewmats, sc.Ks, sc.gt)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        stats = ts.step(sc.viewmats, sc.Ks, sc.gt)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / args.steps

    if args.copy_calibration:
        src = torch.ones(args.copy_calibration * (1 << 20) // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # Per-stage kernel times from HIP events on the launch stream (separate
    # pass so the timed loop above carries no event overhead).
    stage_ms = {}
    if not args.no_stage_timing:
        reps = 3
        acc = {}
        for _ in range(reps):
            st = ts.step(sc.viewmats, sc.Ks, sc.gt, timing=True)
            for k, v in ts.stage_ms.items():
                acc[k] = acc.get(k, 0.0) + v
        stage_ms = {k: round(v / reps, 4) for k, v in acc.items()}
        stats = st
    C, P = args.cams, args.width * args.height
    Vvis = int(ts.last_visible_entries)
    shape = {"N": args.n, "C": C, "P": P, "V": stats.entries, "Vvis": Vvis, "I": stats.n_isects,
             "T": stats.touched_rows}
    kernels = {}
    for name, f in BYTES.items():
        if name in stage_ms and stage_ms[name] > 0:
            b = f(shape)
            kernels[name] = {"ms": stage_ms[name], "bytes": b,
                             "GBs": round(b / (stage_ms[name] * 1e-3) / 1e9, 1)}
    dominant = max(kernels, key=lambda k: kernels[k]["ms"]) if kernels else None
    roofline = None
    if dominant:
        d = kernels[dominant]
        default_cfg = (args.n, args.cams, args.width, args.height) == (4_000_000, 16, 1920, 1080)
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": d["GBs"], "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(d["GBs"] / HBM_PEAK_GBS, 4),
                    "traffic": profiled_traffic(dominant) if default_cfg else None}
    bwd_names = ("raster_bwd", "project_bwd")
    bwd_ms = sum(kernels[k]["ms"] for k in bwd_names if k in kernels)
    bwd_bytes = sum(kernels[k]["bytes"] for k in bwd_names if k in kernels)
    line = {
        "metric": METRIC,
        "value": round(ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded cfg3 scene, random-init Gaussians, random targets)",
        "config": {"workload": "cfg3: 4M Gaussians, 16 cams x 1920x1080, L1+SSIM, fwd+bwd+Adam",
                   "gaussians": args.n, "cameras": C, "width": args.width,
                   "height": args.height, "visible_entries": stats.entries,
                   "touched_rows": stats.touched_rows, "isects": stats.n_isects,
                   "isects_per_tile": round(stats.n_isects / (C * ts.tw * ts.th), 1)},
        "bwd_hbm_GBs": round(bwd_bytes / (bwd_ms * 1e-3) / 1e9, 1) if bwd_ms else None,
        "roofline": roofline,
        "stage_ms": stage_ms,
        "kernels": kernels,
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.width, args.height)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
