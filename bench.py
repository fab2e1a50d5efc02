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

# Algorithmic bytes per unit of work (fp32).  The compositing kernels use the
# per-camera figures of the hot-path scope table: backward 24 B per pixel
# (alpha, last id, dL/dcolour, dL/dalpha) + 40 B per intersection (flatten id
# and staged record) + 72 B per visible entry (the 9-float gradient record
# zero-filled and written); forward 20 B per pixel + 40 B per intersection +
# 4 B per tile.  The projection/optimizer kernels count what their algorithm
# moves (each touched row once; the scope table's 760 B per visible entry
# assumes a read-modify-write of the compact row per camera, which this
# design does not do).
BYTES = {
    "visibility": lambda s: 40 * s["N"] + 4 * s["N"],
    "project_fwd": lambda s: s["T"] * (4 + 4 + 4 + 236) + s["V"] * (4 + 48 + 4 + 8),
    "raster_fwd": lambda s: s["C"] * s["P"] * 20 + s["I"] * 40 + s["C"] * s["tiles"] * 4,
    "raster_bwd": lambda s: s["C"] * s["P"] * 24 + s["I"] * 40 + s["V"] * 72,
    "project_bwd": lambda s: s["T"] * (4 + 4 + 4 + 236 + 236) + s["V"] * (4 + 36),
    "adam": lambda s: s["T"] * 1656,
    # intersection stages, as this design's passes move them: the depth sort
    # of the V entries (per pass 4 B key + 8 B (rectangle, entry) read and
    # written, + the 4 B key read of its histogram), the per-block digit
    # counts of the tile sort's first pass (8 B rectangle read); the emission
    # fused with that first pass (8 B rectangle read per entry, 4 B key + 4 B
    # flatten id written per intersection), the tile sort's remaining passes
    # (8 B read + 8 B written per intersection, + 4 B histogram key read) and
    # the offset encode (4 B key read per intersection, 4 B per bucket written)
    "isect_scan": lambda s: s["V"] * (s["passes_d"] * (24 + 4) + 8),
    "isect_sort": lambda s: (8 * s["V"] + 8 * s["I"] + (s["passes_t"] - 1) * 20 * s["I"]
                             + 4 * s["I"] + 4 * s["buckets"]),
    # fused: the row read once, p/m/v written, m/v read; no gradient rows
    "project_bwd_update": lambda s: (s["T"] * (4 + 4 + 4 + 236 + 2 * 236 + 3 * 236)
                                     + s["V"] * (4 + 36)),
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


SIMDS = 1024  # 256 CUs x 4 SIMDs
XCDS = 8      # GRBM_GUI_ACTIVE sums the 8 XCDs' busy clocks


def source_sha16(rel: str) -> str:
    """First 16 hex digits of the SHA-256 of a repository file."""
    import hashlib

    return hashlib.sha256((ROOT / rel).read_bytes()).hexdigest()[:16]


def profiled_valu(kernel: str):
    """VALU counters of one launch of `kernel` at cfg3 from the committed
    rocprofv3 PMC summary (profiles/*_valu.md): SQ_INSTS_VALU (wave64
    instructions), SQ_ACTIVE_INST_VALU (VALU quad-cycles summed over waves),
    SQ_THREAD_CYCLES_VALU (active lanes x VALU instructions), GRBM_GUI_ACTIVE
    and the launch's duration in that run, or None.  The summary names the
    source file the kernel was built from and its hash at profiling time
    (``valu_source <kernel>: <file> <sha16>``); ``source_matches`` tells
    whether that file is unchanged since, i.e. whether the counts describe the
    kernel this run timed."""
    import re

    for f in sorted((ROOT / "profiles").glob("*_valu.md")):
        text = f.read_text()
        m = re.search(rf"^valu_counters {re.escape(kernel)}: (.*)$", text, re.M)
        if m:
            out = {k: float(v) for k, v in re.findall(r"(\w+)=([0-9.eE+-]+)", m.group(1))}
            src = re.search(rf"^valu_source {re.escape(kernel)}: (\S+) ([0-9a-f]{{16}})$", text,
                            re.M)
            out["source"] = f"{src.group(1)} {src.group(2)}" if src else None
            out["source_matches"] = bool(src) and (ROOT / src.group(1)).exists() and \
                source_sha16(src.group(1)) == src.group(2)
            return out
    return None


# tgs_valu_probe's instruction forms, in its `form` order
VALU_FORMS = ("mul_f32_vgpr", "mul_f32_sgpr", "add_u32_vgpr", "xor_b32_sgpr", "fma_f32_vgpr",
              "exp_f32")
# the probe is a measurement aid of this benchmark only: its own library,
# built from bench_valu_probe.hip beside this file, not part of libtidegs_amd.so
PROBE_SRC = ROOT / "bench_valu_probe.hip"
PROBE_LIB = ROOT / "bench_valu_probe.so"
_probe = None


def build_valu_probe() -> Path:
    """Compile bench_valu_probe.so for gfx950 (hipcc, the library's flags)."""
    import subprocess

    from tidegs_amd import build as B

    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [B._hipcc(), *B.HIPCC_FLAGS, "-shared", str(PROBE_SRC), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SRC.name}:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def valu_probe_lib():
    """The probe library (after torch, so that both share one HIP runtime);
    built here if missing."""
    global _probe
    if _probe is None:
        import ctypes

        import torch  # noqa: F401

        if not PROBE_LIB.exists():
            build_valu_probe()
        lib = ctypes.CDLL(str(PROBE_LIB))
        lib.tgs_valu_probe.restype = ctypes.c_int
        lib.tgs_valu_probe.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                       ctypes.c_int32, ctypes.c_void_p]
        _probe = lib
    return _probe


def valu_probe(out, blocks: int, iters: int, form: int, stream: int) -> None:
    """Launch tgs_valu_probe (8 * iters wave64 VALU instructions of one form
    per wavefront, 4 wavefronts per block) into out[blocks * 256]."""
    rc = valu_probe_lib().tgs_valu_probe(out.data_ptr(), blocks, iters, form, stream)
    if rc != 0:
        raise RuntimeError(f"tgs_valu_probe failed (code {rc})")


def valu_peak(dev, blocks: int = 8192, iters: int = 4096, form: int = 0) -> float:
    """Wave64 VALU instructions per second of a synthetic stream of one
    instruction form (tgs_valu_probe: 8 * iters per wavefront, 4 wavefronts
    per block), best of three timed launches.  Form 0, two-source FP32
    multiplies on VGPRs, is the fastest VALU issue rate on this machine: the
    VALU roofline's peak."""
    import torch

    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    valu_probe(out, blocks, 64, form, s)  # warm-up
    best = float("inf")
    for _ in range(3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        valu_probe(out, blocks, iters, form, s)
        b.record()
        b.synchronize()
        best = min(best, a.elapsed_time(b) * 1e-3)
    return blocks * 4 * iters * 8 / best


def valu_roofline(c: dict, live_pairs: int, event_ms: float, peak: float):
    """The compositing kernels are bound by instruction issue, not HBM.  frac =
    the kernel's VALU issue rate (the committed PMC pass's wave64 VALU
    instruction count per launch over this run's event time) / the fastest
    VALU issue rate on this machine (valu_peak: two-source FP32 on VGPRs).
    On gfx950 the issue rate depends on the instruction form: integer and
    bit operations, operands in SGPRs or literals, and three-source FMAs
    issue about half as often as that stream, transcendentals a quarter as
    often; so a kernel's own issue limit lies below the peak and frac
    understates how close it is to it.  Beside it: rocprof's VALU busy on a
    four-cycles-per-instruction basis (4 x SQ_ACTIVE_INST_VALU / (1024 SIMDs x
    XCD clock cycles), which exceeds 1 for two-cycle forms), and the lane
    work per live (Gaussian, pixel) pair (pairs counted by this run's forward)."""
    cycles = c["GRBM_GUI_ACTIVE"] / XCDS
    busy = 4.0 * c["SQ_ACTIVE_INST_VALU"] / (SIMDS * cycles)
    rate = c["SQ_INSTS_VALU"] / (event_ms * 1e-3)
    out = {"bound": "valu", "frac": round(rate / peak, 4),
           "measure": "VALU issue rate / two-source FP32 VGPR stream (tgs_valu_probe)",
           "counts_from": c.get("source"), "counts_match_source": c.get("source_matches"),
           "insts_per_launch": int(c["SQ_INSTS_VALU"]),
           "insts_per_s": round(rate / 1e9, 1) * 1e9, "peak_insts_per_s": round(peak / 1e9, 1) * 1e9,
           "busy_4cycle_basis": round(busy, 4),
           "profiled_clock_GHz": round(cycles / c["duration_ns"], 3),
           "profiled_ms": round(c["duration_ns"] * 1e-6, 3)}
    if live_pairs:
        out["live_pairs"] = int(live_pairs)
        out["lane_slots_per_live_pair"] = round(c["SQ_INSTS_VALU"] * 64 / live_pairs, 1)
        out["active_lane_insts_per_live_pair"] = round(c["SQ_THREAD_CYCLES_VALU"] / live_pairs, 1)
    return out


def _host_cpu():
    """(threads to use, nproc, CPU model): the box's CPU share (OMP_NUM_THREADS
    when set, else the affinity mask) and the lscpu model name."""
    import subprocess

    nproc = os.cpu_count() or 1
    try:
        share = len(os.sched_getaffinity(0))
    except AttributeError:
        share = nproc
    threads = int(os.environ.get("OMP_NUM_THREADS") or share)
    model = "unknown"
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                model = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return max(1, min(threads, share)), nproc, model


def _median_time(fn, repeats=3):
    """1 warm-up, then the median wall time of ``repeats`` runs (seconds)."""
    fn()
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_baseline(width, height, gpu_stats, seed=0):
    """The CPU oracle (oracle/step_ref.py + oracle/optim_ref.py) timed on the
    host cores: all threads of the box's CPU share, 1
    warm-up and the median of 3 repeats per sample.

    * cfg1 (10k Gaussians, one 256x256 camera, L1, Adam) runs in full.
    * cfg3: one camera at a time on seeded subsets of the 4M rows (4 samples
      over different cameras and subset sizes); a least-squares fit of the
      time in the sample's measured visible entries V and intersections I,
      t = c0 + cV V + cI I, is extrapolated to the GPU step's measured V and I
      of each of its 16 cameras, plus the Adam update of its touched rows
      (timed on a row sample, linear in the rows)."""
    import numpy as np
    import torch
    from scipy.optimize import nnls

    from oracle import optim_ref as O
    from oracle import raster_ref as R
    from oracle import step_ref as SR
    from tidegs_amd import scenes

    threads, nproc, model = _host_cpu()
    torch.set_num_threads(threads)
    f32 = dict(raster_dtype=np.float32, proj_dtype=torch.float32)
    # cfg1 in full: forward + backward + one Adam step at lr 1e-3
    c1 = scenes.cfg1(seed=seed)

    def cfg1_step():
        touched, grads, *_ = SR.batch_grads(c1.params, c1.viewmats, c1.Ks, c1.gt, c1.width,
                                            c1.height, lambda_dssim=0.0, **f32)
        p = c1.params[touched].double().numpy()
        O.adam_rows(p, grads.numpy(), 0.0, 0.0, 1e-3, 0.9, 0.999, 1e-15, 1.0, 0.1,
                    np.sqrt(0.001))

    cfg1_s = _median_time(cfg1_step)
    # cfg3 samples
    sc = scenes.cfg3(seed=seed, with_gt=False)
    g = torch.Generator().manual_seed(seed + 1)
    gt = torch.rand((3, height, width), generator=g) * 255.0
    rows_all = []
    samples = []
    for n_sub, cam in ((31_250, 0), (62_500, 5), (125_000, 10), (62_500, 15)):
        rows = torch.sort(torch.randperm(sc.n, generator=g)[:n_sub]).values
        params = sc.params[rows].contiguous()
        vm, K = sc.viewmats[cam:cam + 1], sc.Ks[cam:cam + 1]
        t = _median_time(lambda: SR.batch_grads(params, vm, K, gt[None], width, height, **f32))
        filt = SR.packed_filters(params, vm, K, width, height)[0]
        radii, m2d, depths, _ = SR.render_projection(params, filt, vm[0], K[0], width, height)
        tw, th = -(-width // 16), -(-height // 16)
        n_isect = R.isect_tiles(m2d.float().numpy()[None], radii.numpy()[None],
                                depths.float().numpy()[None], 16, tw, th)[1].size
        samples.append((t, filt.numel(), n_isect))
        rows_all.append(f"{n_sub} rows cam {cam}: V={filt.numel()} I={n_isect} {t:.2f}s")
    A = np.array([[1.0, v, i] for _, v, i in samples])
    coef, _ = nnls(A, np.array([s[0] for s in samples]))
    cams = [coef[0] + coef[1] * v + coef[2] * i
            for v, i in zip(gpu_stats.visible_per_camera, gpu_stats.isects_per_camera)]
    # Adam over the touched rows: float64 numpy on a 250k-row sample
    n_adam = 250_000
    p = np.random.default_rng(seed).standard_normal((n_adam, 59))
    gr = p * 1e-3
    adam_s = _median_time(lambda: O.adam_rows(p, gr, p * 0, p * 0, 1e-3, 0.9, 0.999, 1e-15, 16.0,
                                              0.1, np.sqrt(0.001)))
    adam_full = adam_s * gpu_stats.touched_rows / n_adam
    ms_step = (sum(cams) + adam_full) * 1000.0
    return {
        "value": round(ms_step, 1),
        "unit": "ms/train-step (extrapolated)",
        "cores": threads,
        "kind": "port",
        "nproc": nproc,
        "cpu_model": model,
        "sample": ("CPU oracle (oracle/step_ref.py, float32 projection and compositing; "
                   f"torch threads {threads}), 1 warm-up + median of 3 per sample, one camera "
                   f"per sample on seeded subsets of the cfg3 rows: {'; '.join(rows_all)}. "
                   f"Fit t = {coef[0]:.3g} s + {coef[1]:.3g} s*V + {coef[2]:.3g} s*I, summed over "
                   f"the 16 cameras' measured V and I ({sum(cams):.1f} s) + Adam over "
                   f"{gpu_stats.touched_rows} touched rows ({adam_full:.1f} s, from "
                   f"{n_adam} rows in {adam_s:.2f} s)"),
        "cfg1_full_ms": round(cfg1_s * 1000.0, 1),
    }


WORKLOADS = {
    "cfg3": "cfg3: 4M Gaussians, 16 cams x 1920x1080, L1+SSIM, fwd+bwd+Adam",
    "cfg3-dropin": "cfg3 through the drop-in gsplat/clm ops and GPUResidentAdam at TideGS's "
                   "per-camera call sites (engine.py:2255-2469, runtime.py:1762)",
    "cfg2": "cfg2: 1M Gaussians, 1 cam 1920x1080, rasterizer fwd+bwd",
    "cfg4": "cfg4: 16M-Gaussian aerial city, 4 oblique cams x 1920x1080, fwd+bwd+Adam",
    "cfg5": "cfg5: resident [32M,59] optimizer step, 30% rows visible",
    "init": "Morton-sorted base file from a 16M-vertex PLY (streaming initializer)",
    "resident": "resident-set swap: 4M-row working set of 4096-row blocks (half kept, half "
                "streamed in UNIFIED order), 30% of blocks packed for writeback + bounds",
}


def _stage_kernels(ts, stats, args, stage_ms, C, P):
    Vvis = int(ts.last_visible_entries)
    tile_bits = (ts.tw * ts.th).bit_length()
    shape = {"N": ts.params.shape[0], "C": C, "P": P, "V": stats.entries, "Vvis": Vvis,
             "I": stats.n_isects, "T": stats.touched_rows, "tiles": ts.tw * ts.th,
             "buckets": C * ts.tw * ts.th, "passes_d": (ts.last_depth_key_bits + 7) // 8,
             "passes_t": (tile_bits + 7) // 8}
    # the reference design's figures for the same stages (isect_tiles.cu:14-301
    # count + emit, 20 B per visible entry + 12 B per intersection, and cub's
    # LSD sort of 8 B key + 4 B value pairs, 24 B per intersection and pass
    # over the 32 + tile + camera bits in passes of 8)
    ref_passes = (32 + tile_bits + (C - 1).bit_length() + 7) // 8
    scope = {"isect_scan": 20 * stats.entries + 12 * stats.n_isects,
             "isect_sort": 24 * ref_passes * stats.n_isects}
    kernels = {}
    for name, f in BYTES.items():
        if name in stage_ms and stage_ms[name] > 0:
            b = f(shape)
            kernels[name] = {"ms": stage_ms[name], "bytes": b,
                             "GBs": round(b / (stage_ms[name] * 1e-3) / 1e9, 1)}
            if name in scope:
                kernels[name]["reference_design_bytes"] = scope[name]
    return kernels


def _tile_load(ts, stats):
    """Max and 99th percentile of the intersections per (camera, tile) of the
    step ``stats`` describes, from that step's bucket offsets."""
    import torch

    offs = ts.last["offsets"].reshape(-1).to(torch.int64)
    ends = torch.cat([offs[1:], offs.new_tensor([stats.n_isects])])
    per_tile = (ends - offs).double()
    return {"isects_per_tile_max": int(per_tile.max()),
            "isects_per_tile_p99": round(float(torch.quantile(per_tile, 0.99)), 1)}


def bench_step(args, dev):
    """Full TideGS step (cfg3, cfg4) or the rasterizer pair alone (cfg2).

    Every step (warm-up, timed, stage-timed and the pair-counting one) runs
    from the same scene state: the seeded scene as generated, with cold
    optimizer moments.  The resident table, the moments and the slot
    bookkeeping are snapshotted before the first step and put back before
    each step, outside its timed bracket, so that a step does the whole
    forward + backward + update of that one state however many steps ran
    before it, and the counts reported beside the time (visible entries,
    intersections, live pairs) and the profiles describe the step that was
    timed."""
    import torch

    from tidegs_amd import scenes
    from tidegs_amd.tide_step import TideStep

    if args.workload == "cfg3":
        sc = scenes.cfg3(seed=0, n=args.n, n_cams=args.cams, width=args.width,
                         height=args.height, with_gt=True).to(dev)
    elif args.workload == "cfg4":
        sc = scenes.cfg4(seed=0, device=dev)
    else:
        sc = scenes.cfg2(seed=0).to(dev)
    C = sc.n_cams
    if args.row_order == "blocks" and args.workload in ("cfg3", "cfg4"):
        # TideGS's resident row order: Morton order within 4096-row blocks
        sc.params = sc.params[scenes.block_layout(sc.params)]
    # the resident table in its MI355X layout: rows padded to 256 bytes
    table = scenes.padded_table(sc.params.contiguous())
    del sc.params
    ts = TideStep(table, sc.width, sc.height, batch_size=C, fuse_update=not args.split_update)
    snap = ts.snapshot()

    def one_step(**kw):
        """One step from the pinned state: (stats, wall seconds between two
        device synchronisations around the step alone)."""
        ts.restore(snap)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        st = ts.step(sc.viewmats, sc.Ks, sc.gt, **kw)
        torch.cuda.synchronize()
        return st, time.perf_counter() - t0

    for _ in range(args.warmup):
        one_step()
    wall = []
    for _ in range(args.steps):
        stats, dt = one_step()
        wall.append(dt)
    ms = sum(wall) * 1000.0 / args.steps

    if args.copy_calibration:
        src = torch.ones(args.copy_calibration * (1 << 20) // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # Per-stage kernel times from HIP events on the launch stream (separate
    # steps, so the timed ones above carry no event overhead).
    stage_ms = {}
    if not args.no_stage_timing or args.workload == "cfg2":
        reps = 3
        acc = {}
        for _ in range(reps):
            stats, _ = one_step(timing=True)
            for k, v in ts.stage_ms.items():
                acc[k] = acc.get(k, 0.0) + v
        stage_ms = {k: round(v / reps, 4) for k, v in acc.items()}
    # one more step, untimed, with the forward counting the composited
    # (Gaussian, pixel) pairs (its counting walk is slower than the plain one)
    stats, _ = one_step(count_pairs=True)
    tile_load = _tile_load(ts, stats)
    P = sc.width * sc.height
    kernels = _stage_kernels(ts, stats, args, stage_ms, C, P)
    default_cfg = (args.workload == "cfg3" and
                   (args.n, args.cams, args.width, args.height) == (4_000_000, 16, 1920, 1080))
    if args.workload == "cfg2":
        kernels = {k: v for k, v in kernels.items() if k in ("raster_fwd", "raster_bwd")}
        ms = sum(v["ms"] for v in kernels.values())
    dominant = max(kernels, key=lambda k: kernels[k]["ms"]) if kernels else None
    roofline = None
    if dominant:
        d = kernels[dominant]
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": d["GBs"], "peak": HBM_PEAK_GBS,
                    "unit": "GB/s", "frac": round(d["GBs"] / HBM_PEAK_GBS, 4),
                    "traffic": profiled_traffic(dominant) if default_cfg else None}
        # the compositing kernels are limited by VALU issue, not HBM
        valu = profiled_valu(dominant) if default_cfg else None
        if valu:
            # the compositing kernels are limited by VALU issue, not HBM: the
            # VALU roofline below is the one that bounds them
            roofline["limited_by"] = "valu"
            rates = {name: valu_peak(dev, form=f) for f, name in enumerate(VALU_FORMS)}
            roofline["valu"] = valu_roofline(valu, getattr(ts, "last_live_pairs", 0), d["ms"],
                                             rates[VALU_FORMS[0]])
            roofline["valu"]["form_insts_per_s"] = {k: round(v / 1e9, 1) * 1e9
                                                    for k, v in rates.items()}
    bwd_names = ("raster_bwd", "project_bwd", "project_bwd_update")
    bwd_ms = sum(kernels[k]["ms"] for k in bwd_names if k in kernels)
    bwd_bytes = sum(kernels[k]["bytes"] for k in bwd_names if k in kernels)
    metric = {"cfg3": METRIC,
              "cfg4": "ms/train-step (fwd+bwd+Adam) at 16M Gaussians (aerial city), 4×1080p",
              "cfg2": "ms/rasterizer fwd+bwd at 1M Gaussians, 1×1080p"}[args.workload]
    line = {
        "metric": metric,
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
        "data": f"synthetic (seeded {args.workload} scene, random-init Gaussians, random targets)",
        "config": {"workload": WORKLOADS[args.workload],
                   "gaussians": ts.params.shape[0], "cameras": C, "width": sc.width,
                   "height": sc.height, "visible_entries": stats.entries,
                   "touched_rows": stats.touched_rows, "isects": stats.n_isects,
                   "isects_per_tile": round(stats.n_isects / (C * ts.tw * ts.th), 1),
                   **tile_load, "scene_state": "seeded scene, restored before every step",
                   "row_order": ("Morton within 4096-row blocks, blocks in seeded random order "
                                 "(TideGS's block store)" if args.row_order == "blocks" and
                                 args.workload in ("cfg3", "cfg4") else "generator order (random)"),
                   "optimizer_update": "split" if args.split_update else "fused",
                   "live_pairs": int(getattr(ts, "last_live_pairs", 0))},
        "bwd_hbm_GBs": round(bwd_bytes / (bwd_ms * 1e-3) / 1e9, 1) if bwd_ms else None,
        "roofline": roofline,
        "stage_ms": stage_ms,
        # step time not covered by any stage bracket (host launch latency at
        # the step's start and its final synchronisation)
        "unbracketed_ms": round(ms - sum(stage_ms.values()), 3) if stage_ms else None,
        "kernels": kernels,
        "cpu_baseline": None,
    }
    if args.workload == "cfg3" and not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.width, args.height, stats)
    if default_cfg and not args.no_dropin:
        # the same step through the drop-in ops at TideGS's unchanged
        # per-camera call sites, in its own loop after the headline
        del ts, snap
        torch.cuda.empty_cache()
        d = bench_dropin(args, dev, steps=3, warmup=1)
        line["dropin"] = {"ms_per_step": d["ms_per_step"], "steps": d["steps"],
                          "warmup": d["warmup"], "workload": d["config"]["workload"],
                          "visible_entries": d["config"]["visible_entries"],
                          "isects": d["config"]["isects"]}
    return line


def bench_dropin(args, dev, steps=None, warmup=None):
    """cfg3 through the drop-in ops at TideGS's own call sites, camera by
    camera, as the reference's batch loop runs them
    (``strategies/base_engine.py:329-425`` filters,
    ``strategies/tide_engine/engine.py:2255-2469`` per camera,
    ``runtime.py:1762`` optimizer): the packed projection of all cameras for the
    filters and the touched rows, then per camera the gather + clone of the
    filter's rows, activations, ``fully_fused_projection``,
    ``spherical_harmonics``, ``isect_tiles``, ``isect_offset_encode``,
    ``rasterize_to_pixels``, L1 + ``fused_ssim`` loss, autograd backward and
    ``scatter_add_`` into the compact gradients, and finally
    ``GPUResidentAdam.step`` over the touched rows."""
    import math
    import types

    import torch

    from tidegs_amd import gsplat_ops as ops
    from tidegs_amd import scenes
    from tidegs_amd.clm_ops import fused_ssim
    from tidegs_amd.resident_optim import GPUResidentAdam
    from tidegs_amd.tide_step import _Manager

    sc = scenes.cfg3(seed=0, n=args.n, n_cams=args.cams, width=args.width, height=args.height,
                     with_gt=True).to(dev)
    if args.row_order == "blocks":
        sc.params = sc.params[scenes.block_layout(sc.params)]
    C, W, H = sc.n_cams, sc.width, sc.height
    n = sc.params.shape[0]
    # TideGS's GPU-resident component tensors
    comp = {"xyz": (0, 3), "scaling": (3, 6), "rotation": (6, 10), "opacity": (10, 11),
            "features_dc": (11, 14), "features_rest": (14, 59)}
    g = types.SimpleNamespace()
    for name, (a, b) in comp.items():
        setattr(g, "_" + name, sc.params[:, a:b].contiguous())
    del sc.params
    bsz = C
    lrs = torch.tensor([1.6e-4, 0.05, 5e-3, 1e-3, 2.5e-3, 2.5e-3 / 20.0]) * math.sqrt(bsz)
    g.optimizer = types.SimpleNamespace(
        columns_lr=lrs, param_groups=[{"betas": (0.9 ** bsz, 0.999 ** bsz),
                                       "eps": 1e-15 / math.sqrt(bsz)}])
    g.gpu_working_set_manager = _Manager(n, 4096, dev)
    opt = GPUResidentAdam(batch_size=bsz, block_size=4096,
                          capacity_blocks=len(g.gpu_working_set_manager.loaded_blocks),
                          device=str(dev))
    opt.set_resident_blocks(g.gpu_working_set_manager.loaded_blocks)
    vms, Ks = sc.viewmats.contiguous(), sc.Ks.contiguous()
    camtoworlds = torch.linalg.inv(vms)
    gts = [torch.clamp(sc.gt[c] / 255.0, 0.0, 1.0) for c in range(C)]
    tw, th = -(-W // 16), -(-H // 16)
    state = {"it": 0, "visible": 0, "isects": 0}

    def step():
        with torch.no_grad():
            quats = torch.nn.functional.normalize(g._rotation, dim=-1)
            out = ops.fully_fused_projection(g._xyz, None, quats, torch.exp(g._scaling), vms, Ks,
                                             W, H, packed=True)
            cam_ids, gauss_ids = out[0], out[1]
            counts = torch.bincount(cam_ids, minlength=C).tolist()
            filters = torch.split(gauss_ids, counts)
            touched = torch.unique(gauss_ids)
        grads = {name: torch.zeros((touched.numel(), b - a), device=dev)
                 for name, (a, b) in comp.items()}
        n_isect = 0
        for c in range(C):
            rows = filters[c]
            xyz = g._xyz[rows].clone().requires_grad_(True)
            op_raw = g._opacity[rows].clone().requires_grad_(True)
            sc_raw = g._scaling[rows].clone().requires_grad_(True)
            rot_raw = g._rotation[rows].clone().requires_grad_(True)
            shs = torch.cat([g._features_dc[rows], g._features_rest[rows]], 1)
            shs = shs.reshape(-1, 16, 3).requires_grad_(True)
            opac = torch.sigmoid(op_raw)
            scales = torch.exp(sc_raw)
            rots = torch.nn.functional.normalize(rot_raw, dim=-1)
            radii, m2d, depths, conics, _ = ops.fully_fused_projection(
                xyz, None, rots, scales, vms[c:c + 1], Ks[c:c + 1], W, H, packed=False)
            m2d.retain_grad()
            dirs = xyz[None] - camtoworlds[c:c + 1, None, :3, 3]
            colors = torch.clamp_min(ops.spherical_harmonics(3, dirs, shs[None]) + 0.5, 0.0)
            _, isect_ids, flat = ops.isect_tiles(m2d, radii, depths, 16, tw, th)
            offs = ops.isect_offset_encode(isect_ids, 1, tw, th)
            img, _ = ops.rasterize_to_pixels(m2d, conics, colors, opac.squeeze(1)[None], W, H,
                                             16, offs, flat)
            img = img[0].permute(2, 0, 1).contiguous()
            loss = 0.8 * (img - gts[c]).abs().mean() + \
                0.2 * (1.0 - fused_ssim(img[None], gts[c][None]))
            loss.backward()
            idx = torch.searchsorted(touched, rows)
            for name, t in (("xyz", xyz), ("opacity", op_raw), ("scaling", sc_raw),
                            ("rotation", rot_raw)):
                grads[name].index_add_(0, idx, t.grad)
            sg = shs.grad.reshape(-1, 48)
            grads["features_dc"].index_add_(0, idx, sg[:, :3])
            grads["features_rest"].index_add_(0, idx, sg[:, 3:])
            n_isect += isect_ids.numel()
        state["it"] += 1
        opt.step(state["it"], g, touched, grads)
        state["visible"], state["isects"], state["touched"] = sum(counts), n_isect, touched.numel()

    # every step from the same scene state, as in bench_step: the component
    # tensors and the optimizer state are put back before each step, outside
    # its timed bracket
    torch.cuda.synchronize()
    saved = {name: getattr(g, "_" + name).clone() for name in comp}
    opt_snap = opt.snapshot()

    def one_step():
        for name in comp:
            getattr(g, "_" + name).copy_(saved[name])
        opt.restore(opt_snap)
        state["it"] = 0
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    for _ in range(warmup):
        one_step()
    ms = sum(one_step() for _ in range(steps)) * 1000.0 / steps
    return {
        "metric": "ms/train-step (fwd+bwd+Adam) at 4M Gaussians, 16×1080p, drop-in ops at "
                  "TideGS's per-camera call sites",
        "value": round(ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded cfg3 scene, random-init Gaussians, random targets)",
        "config": {"workload": WORKLOADS["cfg3-dropin"], "gaussians": n, "cameras": C,
                   "width": W, "height": H, "visible_entries": state["visible"],
                   "touched_rows": state["touched"], "isects": state["isects"]},
        "roofline": None,
        "cpu_baseline": None,
    }


def bench_optimizer(args, dev):
    """cfg5: fused resident Adam and Sophia over a [32M, 59] CACHE-order table
    with 30% of the rows visible (sorted int32 ids).  The timed step is the
    whole GPUResidentAdam.step (host bookkeeping + one kernel); the kernel
    alone is timed with HIP events on its stream."""
    import torch

    from tidegs_amd import scenes
    from tidegs_amd.resident_optim import GPUResidentAdam, GPUResidentSophia
    from tidegs_amd.tide_step import _CACHE_COLS, _Manager, _TableGaussians

    n = 32_000_000 if args.n == 4_000_000 else args.n
    case = scenes.cfg5(seed=0, n=n, device=dev)
    # resident table and gradient rows in the padded layout (256-byte rows), as
    # the fused step keeps them
    case.table = scenes.padded_table(case.table)
    case.grads = scenes.padded_table(case.grads)
    torch.cuda.empty_cache()
    T = case.rows.numel()
    mgr = _Manager(n, 4096, dev)
    lrs = torch.tensor([1.6e-4, 0.05, 5e-3, 1e-3, 2.5e-3, 1.25e-4])
    comps = {name: case.grads[:, a:b] for name, (a, b) in _CACHE_COLS.items()}
    out = {}
    for kind, cls, kw, betas in (("adam", GPUResidentAdam, {}, (0.9, 0.999)),
                                 ("sophia", GPUResidentSophia, {"rho": 0.04}, (0.9, 0.99))):
        gs = _TableGaussians(case.table, mgr, lrs, betas, 1e-15)
        opt = cls(batch_size=1, block_size=4096, capacity_blocks=len(mgr.loaded_blocks),
                  device=str(dev), **kw)
        opt.set_resident_blocks(mgr.loaded_blocks)
        it = 0
        for _ in range(args.warmup):
            it += 1
            opt.step(it, gs, case.rows, comps)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            it += 1
            opt.step(it, gs, case.rows, comps)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1000.0 / args.steps
        evs = []
        opt.kernel_hooks = (lambda: evs.append([torch.cuda.Event(enable_timing=True)]) or
                            evs[-1][0].record(),
                            lambda: evs[-1].append(torch.cuda.Event(enable_timing=True)) or
                            evs[-1][1].record())
        for _ in range(3):
            it += 1
            opt.step(it, gs, case.rows, comps)
        opt.kernel_hooks = None
        torch.cuda.synchronize()
        k_ms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
        b = T * 1656
        out[kind] = {"ms_per_step": round(ms, 4), "kernel_ms": round(k_ms, 4), "bytes": b,
                     "GBs": round(b / (k_ms * 1e-3) / 1e9, 1)}
        del opt
        torch.cuda.empty_cache()
    a = out["adam"]
    return {
        "metric": "ms/optimizer-step (fused resident Adam) at [32M,59], 30% rows visible",
        "value": a["ms_per_step"],
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": a["ms_per_step"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) table, N(0,1e-3) gradients, sorted int32 rows)",
        "config": {"workload": WORKLOADS["cfg5"], "rows": n, "touched_rows": T},
        "roofline": {"kernel": "resident_optim (adam)", "bound": "hbm", "achieved": a["GBs"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(a["GBs"] / HBM_PEAK_GBS, 4),
                     "traffic": None},
        "optimizers": out,
        "cpu_baseline": None,
    }


def bench_resident(args, dev):
    """Resident-set materialization and writeback (the Triton movers of
    double_buffer_gpu.py / gpu_working_set.py): a 4M-row working set (padded
    256-byte rows) of 4096-row blocks drawn from a 16M-row scene.  One step =
    copy the kept half of the blocks from the previous buffer, unpack the
    streamed half from packed UNIFIED rows already in HBM (the H2D upload is
    PCIe and outside the step), rebuild the block-start table, pack 30% of the
    blocks for writeback and take their xyz bounds.  Kernels are timed with
    events on the launch stream."""
    import numpy as np
    import torch

    from tidegs_amd.working_set import BlockLayout, ResidentBuffer, ResidentWorkingSet

    bs = 4096
    rows = args.n
    n_blocks = -(-rows // bs)
    num_total = 4 * n_blocks * bs
    ws = ResidentWorkingSet(num_total, block_size=bs, device=dev, row_pitch=64)
    rng = np.random.default_rng(0)
    prev_ids = sorted(rng.choice(num_total // bs, n_blocks, replace=False).tolist())
    prev = ResidentBuffer()
    ws.allocate(prev, n_blocks * bs)
    prev.table.normal_()
    prev.table.as_strided((n_blocks * bs, 64), (64, 1))[:, 59:].zero_()
    prev.local_to_global_idx.copy_(torch.cat([torch.arange(b * bs, (b + 1) * bs)
                                              for b in prev_ids]))
    prev.block_to_local_slice = {b: slice(i * bs, (i + 1) * bs) for i, b in enumerate(prev_ids)}
    kept = sorted(rng.choice(prev_ids, n_blocks // 2, replace=False).tolist())
    fresh = sorted(set(range(num_total // bs)) - set(prev_ids))
    streamed = sorted(rng.choice(fresh, n_blocks - len(kept), replace=False).tolist())
    order = kept + streamed
    packed = torch.randn((len(streamed) * bs, 59), device=dev)
    dirty = sorted(rng.choice(order, int(0.3 * n_blocks), replace=False).tolist())
    tgt = ResidentBuffer()
    ws.allocate(tgt, len(order) * bs)
    tgt.block_to_local_slice = {b: slice(i * bs, (i + 1) * bs) for i, b in enumerate(order)}
    kept_rows, streamed_rows, dirty_rows = len(kept) * bs, len(streamed) * bs, len(dirty) * bs
    from tidegs_amd import _native as N

    def step():
        ws.copy_resident_blocks(prev, tgt, kept, tgt.block_to_local_slice)
        ws.unpack_streamed_rows(packed, BlockLayout.UNIFIED, tgt, kept_rows, block_ids=streamed)
        tgt._block_starts = ws.build_block_starts(tgt.block_to_local_slice)
        ws.stage_updated_blocks(tgt, dirty, to_host=False)
        ws.stage_block_bounds(tgt, dirty, to_host=False)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / args.steps

    # each kernel alone, events right around its launch (index arrays prebuilt)
    def i64(v):
        return torch.tensor(list(v), dtype=torch.int64, device=dev)

    kept_src = i64(prev.block_to_local_slice[b].start for b in kept)
    kept_dst = i64(tgt.block_to_local_slice[b].start for b in kept)
    streamed_ids = i64(streamed)
    dirty_src = i64(tgt.block_to_local_slice[b].start for b in dirty)
    dirty_cnt = i64([bs] * len(dirty))
    dirty_out = i64(range(0, len(dirty) * bs, bs))
    out = torch.empty((len(dirty) * bs, 59), device=dev)
    bounds = torch.empty((len(dirty), 6), device=dev)
    tid = torch.empty(num_total // bs, dtype=torch.int64, device=dev)
    order_ids = i64(order)
    order_starts = i64(tgt.block_to_local_slice[b].start for b in order)
    st = N.stream_handle(dev)
    launches = {
        "copy": lambda: N.call("tgs_ws_copy_rows", N.ptr(prev.table), 64,
                               N.ptr(prev.local_to_global_idx), N.ptr(kept_src), N.ptr(kept_dst),
                               len(kept), kept_rows, bs, N.ptr(tgt.table), 64,
                               N.ptr(tgt.local_to_global_idx), st),
        "unpack": lambda: N.call("tgs_ws_unpack_rows", N.ptr(packed), 1, streamed_rows,
                                 N.ptr(tgt.table), 64, kept_rows, N.ptr(streamed_ids),
                                 len(streamed), bs, N.ptr(tgt.local_to_global_idx), st),
        "starts": lambda: N.call("tgs_ws_build_block_starts", N.ptr(order_ids),
                                 N.ptr(order_starts), len(order), N.ptr(tid), tid.numel(), st),
        "pack": lambda: N.call("tgs_ws_pack_rows", N.ptr(tgt.table), 64, N.ptr(dirty_src),
                               N.ptr(dirty_cnt), N.ptr(dirty_out), len(dirty), bs, N.ptr(out), st),
        "bounds": lambda: N.call("tgs_ws_block_bounds", N.ptr(tgt.table), 64, N.ptr(dirty_src),
                                 N.ptr(dirty_cnt), len(dirty), bs, N.ptr(bounds), st),
    }
    # algorithmic bytes: 59 floats read + 59 written per row, +8 B id read/write
    byt = {"copy": kept_rows * (236 * 2 + 16), "unpack": streamed_rows * (236 * 2 + 8),
           "starts": 8 * (num_total // bs) + 16 * len(order),
           "pack": dirty_rows * 236 * 2, "bounds": dirty_rows * 12}
    stages = {}
    for k, fn in launches.items():
        times = []
        for _ in range(7):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b))
        k_ms = sorted(times)[len(times) // 2]
        stages[k] = {"ms": round(k_ms, 4), "bytes": byt[k],
                     "GBs": round(byt[k] / (k_ms * 1e-3) / 1e9, 1)}
    # streaming from the on-disk store: the streamed blocks' rows as a base
    # file (page cache warm after the write), read by the native parallel
    # reader into pinned staging, uploaded and unpacked (PCIe + host memory
    # bound; reported beside the HBM-resident step, never as its value)
    import tempfile

    from tidegs_amd.block_store import BlockStore, BlockStoreReader

    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as tmp:
        n_st = len(streamed)
        store = BlockStore(tmp, block_size=bs, num_blocks=n_st)
        store.write_base(packed)
        reader = BlockStoreReader(store, n_st * bs)
        ids = list(range(n_st))
        times = []
        for i in range(4):
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            ws.materialize(None, ids, set(), set(), True, reader)
            torch.cuda.synchronize()
            if i:
                times.append((time.perf_counter() - t1) * 1000.0)
        st_ms = sorted(times)[len(times) // 2]
        cpu_line = None
        if not args.no_cpu_baseline:
            # the reference's per-block seek + read + copy (oracle restatement),
            # one thread, the same blocks
            from oracle import block_store_ref as B

            paths = {f: str(p) for f, p in store.file_paths.items()}
            t1 = time.perf_counter()
            parts = [B.read_block(paths, (0, loc.offset, loc.size), b, bs, 59)
                     for b, loc in sorted(store.index.items())]
            np.concatenate(parts)
            cpu_s = time.perf_counter() - t1
            cpu_line = {"value": round(cpu_s * 1000.0, 2), "unit": "ms", "cores": 1,
                        "kind": "port",
                        "sample": f"oracle/block_store_ref.read_block over the {n_st} streamed "
                                  f"blocks ({n_st * bs * 236 / 1e6:.0f} MB, page cache warm) + "
                                  "concatenation, 1 thread; compare with stream_from_store.ms"}
        store.close()
    stream_store = {"blocks": n_st, "bytes": n_st * bs * 236, "ms": round(st_ms, 3),
                    "GBs": round(n_st * bs * 236 / (st_ms * 1e-3) / 1e9, 2)}
    # block frustum culling at billion-Gaussian scale: 250k blocks x 16 cameras
    from tidegs_amd.block_culling import FrustumCuller, camera_view_projection, \
        extract_frustum_planes

    mins = rng.uniform(-500, 500, (250_000, 3)).astype(np.float32)
    cb = np.concatenate([mins, mins + rng.uniform(1, 30, (250_000, 3)).astype(np.float32)], 1)
    culler = FrustumCuller(cb, device=dev)
    views, projs = [], []
    for i in range(16):
        a = 2 * np.pi * i / 16
        cpos = np.array([700 * np.cos(a), 700 * np.sin(a), 150.0])
        z = -cpos / np.linalg.norm(cpos)
        x = np.cross(z, [0.0, 0.0, 1.0])
        x /= np.linalg.norm(x)
        W = np.stack([x, np.cross(z, x), z])
        _, v, pm = camera_view_projection(W.T, -W @ cpos, np.deg2rad(60), 1920, 1080, 900)
        views.append(v)
        projs.append(pm)
    planes = np.stack([extract_frustum_planes(v, pm) for v, pm in zip(views, projs)])
    times = []
    for _ in range(7):
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record()
        culler.cull_masks(planes)
        a1.record()
        torch.cuda.synchronize()
        times.append(a0.elapsed_time(a1))
    t1 = time.perf_counter()
    lists = culler.cull_batch(views, projs)
    batch_ms = (time.perf_counter() - t1) * 1000.0
    cull_line = {"blocks": 250_000, "cameras": 16, "launch_ms": round(sorted(times)[3], 4),
                 "batch_lists_ms": round(batch_ms, 3),
                 "visible_per_camera": int(np.mean([len(x) for x in lists]))}
    if not args.no_cpu_baseline:
        from oracle import culling_ref as K

        c_, r_ = K.spheres(cb)
        t1 = time.perf_counter()
        for v, pm in zip(views, projs):
            K.cull(c_, r_, K.planes(v, pm))
        cull_line["cpu_oracle_ms"] = round((time.perf_counter() - t1) * 1000.0, 1)
    dom = max(("copy", "unpack", "pack"), key=lambda k: stages[k]["ms"])
    return {
        "metric": "ms/resident-set swap (copy kept + unpack streamed + pack dirty + bounds) "
                  "at a 4M-row working set",
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) rows, random block sets)",
        "config": {"workload": WORKLOADS["resident"], "rows": len(order) * bs,
                   "kept_blocks": len(kept), "streamed_blocks": len(streamed),
                   "dirty_blocks": len(dirty)},
        "roofline": {"kernel": f"ws_move_rows ({dom})", "bound": "hbm",
                     "achieved": stages[dom]["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(stages[dom]["GBs"] / HBM_PEAK_GBS, 4), "traffic": None},
        "stages": stages,
        "stream_from_store": stream_store,
        "block_culling": cull_line,
        "cpu_baseline": cpu_line,
    }


def bench_init(args, dev):
    """The streaming initializer (storage/streaming_ply_init.py) on a synthetic
    16M-vertex PLY (cfg4 scale: the aerial-city positions, 8-bit colours):
    host read, GPU passes (bounds, Morton codes, stable sort, bucket choice,
    per-bucket bounds, row packing, block bounds), D2H + file write.  The
    CPU baseline is the oracle's restatement of the reference's bucketed
    external sort on a 1M-vertex sample, scaled linearly to 16M."""
    import tempfile

    import numpy as np
    import torch

    from tidegs_amd import scenes
    from tidegs_amd.streaming_init import streaming_ply_to_ssd_base, write_binary_ply

    n = 16_000_000 if args.n == 4_000_000 else args.n
    rng = np.random.default_rng(0)
    xyz = scenes.cfg4(seed=0, n=n, device=torch.device("cpu")).params[:, 0:3].numpy()
    cols = {c: rng.integers(0, 256, n).astype(np.uint8) for c in ("red", "green", "blue")}
    runs = []
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as tmp:
        ply = os.path.join(tmp, "scene.ply")
        write_binary_ply(ply, xyz, cols)
        for i in range(min(max(1, args.steps), 2) + 1):
            t = {}
            t0 = time.perf_counter()
            streaming_ply_to_ssd_base(ply, os.path.join(tmp, "out"), block_size=4096,
                                      debug_fast_init_scales=True, device=dev, timings=t)
            t["total"] = time.perf_counter() - t0
            if i:
                runs.append(t)
    med = {k: sorted(r[k] for r in runs)[len(runs) // 2] for k in runs[0]}
    gpu_bytes = n * 430  # algorithmic bytes of the GPU passes per vertex
    cpu_line = None
    if not args.no_cpu_baseline:
        from oracle import streaming_init_ref as S

        m = 1_000_000
        v = np.empty(m, dtype=[("x", "<f4"), ("y", "<f4"), ("z", "<f4"), ("red", "u1"),
                               ("green", "u1"), ("blue", "u1")])
        for d, c in enumerate("xyz"):
            v[c] = xyz[:m, d]
        for c in ("red", "green", "blue"):
            v[c] = cols[c][:m]
        t0 = time.perf_counter()
        S.build_base(v, block_size=4096)
        cs = time.perf_counter() - t0
        cpu_line = {"value": round(cs * n / m * 1000.0, 1), "unit": "ms", "cores": 1,
                    "kind": "port",
                    "sample": f"oracle/streaming_init_ref.build_base (in-memory buckets, no temp "
                              f"files) on the first 1M of the {n // 1_000_000}M vertices: "
                              f"{cs:.2f} s, scaled x{n // m}"}
    return {
        "metric": "ms/base-file build (PLY -> Morton-sorted base_file.bin) at 16M vertices",
        "value": round(med["total"] * 1000.0, 2),
        "unit": "ms",
        "n_gpus": 1,
        "steps": len(runs),
        "warmup": 1,
        "ms_per_step": round(med["total"] * 1000.0, 2),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (cfg4 aerial-city positions, random 8-bit colours)",
        "config": {"workload": WORKLOADS["init"], "vertices": n, "block_size": 4096},
        "phases_ms": {k: round(v * 1000.0, 2) for k, v in med.items()},
        "roofline": {"kernel": "GPU passes (bounds, codes, sort, buckets, pack, block bounds)",
                     "bound": "hbm", "achieved": round(gpu_bytes / med["gpu"] / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gpu_bytes / med["gpu"] / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None},
        "cpu_baseline": cpu_line,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="cfg3",
                    help="cfg3 (default) is the headline step; the others are the "
                         "remaining BASELINE configurations")
    ap.add_argument("--n", type=int, default=4_000_000)
    ap.add_argument("--cams", type=int, default=16)
    ap.add_argument("--width", type=int, default=1920)
    ap.add_argument("--height", type=int, default=1080)
    ap.add_argument("--row-order", choices=("blocks", "random"), default="blocks",
                    help="cfg3/cfg4 resident row order: TideGS's (Morton order within 4096-row "
                         "blocks, the blocks in a seeded random slot order) or the generator's "
                         "own random order")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-stage-timing", action="store_true")
    ap.add_argument("--no-dropin", action="store_true",
                    help="cfg3: skip the drop-in call-site step timed after the headline")
    ap.add_argument("--split-update", action="store_true",
                    help="cfg3/cfg4: optimizer update as its own launch over materialised "
                         "gradient rows instead of inside the projection backward")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run 3 plain device copies of MIB MiB (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the TideGS step is single-GPU; "
              "a multi-GPU run would shard the cameras over ranks). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    dev = torch.device("cuda:0")
    if args.workload == "cfg5":
        line = bench_optimizer(args, dev)
    elif args.workload == "resident":
        line = bench_resident(args, dev)
    elif args.workload == "init":
        line = bench_init(args, dev)
    elif args.workload == "cfg3-dropin":
        line = bench_dropin(args, dev)
    else:
        line = bench_step(args, dev)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
