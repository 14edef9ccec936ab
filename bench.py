#!/usr/bin/env python3
"""Benchmark of the MI355X Gaussian-splatting rasterizer.

Metric: fwd+bwd iterations/s and forward FPS at 1M Gaussians,
SH degree 3, 1920x1080 (config 3: antialias, 8 orbit views), plus the HBM
roofline fraction.  A step is one view: GaussianModel.render -> L1 loss
against a seeded U(0,1) target -> backward to every raw parameter.  Inputs,
targets and parameters are resident in HBM before timing starts.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3]

Prints one JSON line.  The K timed steps run without instrumentation; a
second pass over the same K steps records HIP events on the launch stream
around every stage, for the stage breakdown and the ``roofline`` of the
dominant kernel (its algorithmic bytes per launch over its mean duration);
``cpu_baseline`` times the CPU oracle (C, OpenMP) on one fwd+bwd iteration
per view of the same workload.

Profiling helpers (used to produce profiles/):
    --copy-probe MB    after timing, stream MB megabytes through a plain
                       read-once/write-once kernel (gsx_debug_expf), the
                       calibration for rocprofv3's FETCH_SIZE / WRITE_SIZE
    --summarize-prof DIR --workload NAME
                       turn rocprofv3 csv output under DIR (kernel stats,
                       counter collections) into the text summary and the
                       traffic record bench.py reads; no GPU needed
"""

from __future__ import annotations

import argparse
import contextlib
import gc
import json
import math
import os
import platform
import sys
import time

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s


def _parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=24)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-stages", action="store_true",
                    help="print per-stage times to stderr")
    ap.add_argument("--train-steps", type=int, default=12,
                    help="also time GaussianTrainer.step (SH configs with a backward); 0 = off")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB")
    ap.add_argument("--layout", default="morton", choices=["morton", "creation"],
                    help="row order of the Gaussian table: 3D Morton order of the means "
                         "(spatial_order, the default) or the scene's creation order")
    ap.add_argument("--reference-suite", action="store_true",
                    help="time the reference's own published benchmark cases "
                         "(examples/benchmark.py) and print them as one JSON line")
    ap.add_argument("--summarize-prof", metavar="DIR", nargs="+")
    ap.add_argument("--workload", default="c3_1m_sh3_aa_1080p_8views")
    ap.add_argument("--command", default="", help="command line recorded in the summary")
    return ap.parse_args()


# stage name -> device kernel symbol prefix (as rocprofv3 reports it)
KERNEL_SYMBOL = {"raster_fwd": "k_raster_fwd", "raster_bwd": "k_raster_bwd",
                 "preprocess_fwd": "k_preprocess_fwd", "preprocess_bwd": "k_preprocess_bwd",
                 "photometric_fwd": "k_ssim_fwd", "photometric_bwd": "k_ssim_bwd",
                 "adam": "k_adam", "preprocess_bwd_adam": "k_preprocess_bwd_adam"}
COPY_PROBE_KERNEL = "k_debug_expf"


def algorithmic_bytes(N, D, P, C, Ka, sh_path, depth):
    """Compulsory HBM bytes per stage (the path's measurement contract): each
    tensor read or written once.  D is the number of (tile, Gaussian)
    duplicates binning writes; the rasterizers are charged one gather per
    duplicate.

        raster fwd   D (28 + 4C [+4 depth]) + P (4C + 8 [+4 depth])
        raster bwd   D (28 + 4C) + P (4C + 8) + N (24 + 4C)
        preprocess   N (44 + 12 Ka) + N (36 + 4 Cw)      Cw = C on the SH path
        binning      28 N + 44 D
        pre bwd      N (44 + 12 Ka + 24 + 4 Cw) + N (44 + 12 Ka)
        loss (L1)    12 C P
    """
    Cw = C if sh_path else 0
    dz = 4 if depth else 0
    raster_fwd = D * (28 + 4 * C + dz) + P * (4 * C + 8 + dz)
    raster_bwd = D * (28 + 4 * C) + P * (4 * C + 8) + N * (24 + 4 * C)
    pre_fwd = N * (44 + 12 * Ka) + N * (36 + 4 * Cw)
    binning = 28 * N + 44 * D
    pre_bwd = N * (44 + 12 * Ka + 24 + 4 * Cw) + N * (44 + 12 * Ka)
    fwd = pre_fwd + binning + raster_fwd
    bwd = raster_bwd + pre_bwd
    loss = 12 * C * P
    return dict(raster_fwd=raster_fwd, raster_bwd=raster_bwd, preprocess_fwd=pre_fwd,
                binning=binning, preprocess_bwd=pre_bwd, fwd=fwd, bwd=bwd, loss=loss,
                iter=fwd + bwd + loss)


def needed_bytes(Dn, N, P, C, depth):
    """The rasterizers' bytes when only the list entries a pixel can reach are
    charged: Dn = sum over tiles of the largest n_contrib (the backward
    replays exactly those; the forward reads at least those).  A secondary
    figure beside algorithmic_bytes, which charges every duplicate."""
    dz = 4 if depth else 0
    return dict(raster_fwd=Dn * (28 + 4 * C + dz) + P * (4 * C + 12 + dz),
                raster_bwd=Dn * (28 + 4 * C) + P * (4 * C + 8) + N * (24 + 4 * C))


def needed_entries(n_contrib, tile: int = 16) -> int:
    """Sum over 16x16 tiles of the largest n_contrib (the 1-based list
    position of a pixel's last composited Gaussian) in the tile."""
    import torch

    H, W = n_contrib.shape
    ty, tx = -(-H // tile), -(-W // tile)
    pad = torch.zeros((ty * tile, tx * tile), dtype=torch.int64, device=n_contrib.device)
    pad[:H, :W] = n_contrib
    return int(pad.view(ty, tile, tx, tile).amax(dim=(1, 3)).sum())


def _profiles_dir():
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def _traffic(kernel: str, workload: str):
    """HBM bytes per launch (FETCH + WRITE, calibrated) from the rocprofv3
    PMC runs recorded under profiles/, if present."""
    path = os.path.join(_profiles_dir(), f"traffic_{kernel}_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


# Nominal wave-level VALU issue rate: one wave64 instruction per SIMD every
# 4 cycles, 4 SIMDs x 256 CUs at 2.4 GHz.
VALU_PEAK_G = 256 * 4 * 2.4e9 / 4 / 1e9
# Rate a standalone probe measured on the box for the rasterizers' mix of
# fma / compare / multiply / select (dual-issue of independent VALU ops).
VALU_MEASURED_G = 732.3


def _issue(kernel: str, workload: str, mean_ms: float):
    """VALU issue rate of the kernel: wave-level VALU instructions per launch
    (rocprofv3 SQ_INSTS_VALU, recorded under profiles/) over its mean
    duration, against the nominal issue peak (and the measured mix rate),
    if recorded."""
    path = os.path.join(_profiles_dir(), f"valu_{kernel}_{workload}.json")
    if not os.path.exists(path) or not mean_ms or mean_ms != mean_ms:
        return None
    with open(path) as f:
        n = json.load(f).get("valu_instructions_per_launch")
    if not n:
        return None
    g = n / (mean_ms * 1e-3) / 1e9
    return {"bound": "valu", "valu_instructions": int(n), "achieved": round(g, 1),
            "peak": round(VALU_PEAK_G, 1), "unit": "G wave-instr/s",
            "frac": round(g / VALU_PEAK_G, 4),
            "measured_mix_peak": VALU_MEASURED_G,
            "frac_of_measured_mix": round(g / VALU_MEASURED_G, 4)}


def _read_csv(path):
    import csv

    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    return name.split("(")[0]


def summarize_prof(dirs, workload: str, command: str, out_dir: str | None = None):
    """rocprofv3 csv output under dirs -> <out_dir>/kernels_<workload>.md and,
    with counter runs present, <out_dir>/traffic_<kernel>_<workload>.json
    (out_dir: profiles/ by default)."""
    import glob

    out_dir = out_dir or _profiles_dir()
    os.makedirs(out_dir, exist_ok=True)

    def find(pattern):
        return sorted(p for d in dirs for p in glob.glob(os.path.join(d, "**", pattern),
                                                         recursive=True))

    stats = find("*kernel_stats.csv")
    if stats:
        rows = _read_csv(stats[0])
        rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
        total = sum(float(r["TotalDurationNs"]) for r in rows)
        lines = [f"# rocprofv3 kernel statistics: {workload}", "",
                 "Command (run from the repository root on the MI355X box):", "",
                 f"    {command}", "",
                 "| kernel | calls | avg us | min us | max us | total ms | % |",
                 "|---|---|---|---|---|---|---|"]
        for r in rows[:30]:
            lines.append(f"| `{_short(r['Name'])[:70]}` | {r['Calls']} | "
                         f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                         f"{float(r['MaxNs']) / 1e3:.2f} | "
                         f"{float(r['TotalDurationNs']) / 1e6:.3f} | "
                         f"{100.0 * float(r['TotalDurationNs']) / total:.1f} |")
        path = os.path.join(out_dir, f"kernels_{workload}.md")
        with open(path, "w") as f:
            f.write("\n".join(lines) + "\n")
        print(f"wrote {path}")
    counters = {}
    for path in find("*counter_collection.csv"):
        for r in _read_csv(path):
            counters.setdefault(r["Counter_Name"], []).append(
                (_short(r["Kernel_Name"]), float(r["Counter_Value"]), int(r["Grid_Size"])))
    if "FETCH_SIZE" in counters and "WRITE_SIZE" in counters:
        def is_kernel(name, sym):  # the symbol itself or an instantiation of it
            return name == sym or name.startswith(sym + "<")

        def per_kernel(cname, sym):
            v = [x[1] for x in counters[cname] if is_kernel(x[0], sym)]
            return sum(v) / len(v) if v else None

        probe = [x for x in counters["FETCH_SIZE"] if is_kernel(x[0], COPY_PROBE_KERNEL)]
        n_probe = max(x[2] for x in probe)  # grid = elements of the largest probe launch
        known_kib = 4.0 * n_probe / 1024.0
        f_probe = max(x[1] for x in probe)
        w_probe = max(x[1] for x in counters["WRITE_SIZE"]
                      if is_kernel(x[0], COPY_PROBE_KERNEL))
        f_scale, w_scale = known_kib / f_probe, known_kib / w_probe
        for stage, sym in KERNEL_SYMBOL.items():
            fk, wk = per_kernel("FETCH_SIZE", sym), per_kernel("WRITE_SIZE", sym)
            if fk is None or wk is None:
                continue
            rec = {"kernel": sym, "workload": workload,
                   "fetch_kib_per_launch_raw": round(fk, 1),
                   "write_kib_per_launch_raw": round(wk, 1),
                   "calibration": {"probe_kernel": COPY_PROBE_KERNEL,
                                   "probe_bytes_read": int(known_kib * 1024),
                                   "probe_bytes_written": int(known_kib * 1024),
                                   "fetch_scale": round(f_scale, 4),
                                   "write_scale": round(w_scale, 4)},
                   "hbm_bytes_per_launch": int((fk * f_scale + wk * w_scale) * 1024),
                   "command": command}
            path = os.path.join(out_dir, f"traffic_{stage}_{workload}.json")
            with open(path, "w") as f:
                json.dump(rec, f, indent=1)
            print(f"wrote {path}")


def cpu_baseline(scene, views, cfg_name: str):
    """One fwd+bwd iteration of the oracle per view, on the host cores."""
    import numpy as np

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import oracle as O

    threads = O.default_threads()
    if scene.features is not None:
        scales, opac, flags, sh = scene.scales, scene.opacities, 0, None
    else:
        scales, opac = scene.log_scales, scene.logit_opacities
        flags = O.LOG_SCALES | O.LOGIT_OPACITY
        sh = np.concatenate([scene.sh_dc, scene.sh_rest], 1)
    if scene.antialias:
        flags |= O.ANTIALIAS
    t_fwd = t_all = 0.0
    for view in views:
        cam = scene.cameras[view]
        f = cam.gsx_fields()
        oc = O.make_camera(f["R"], f["t"], f["center"], f["fx"], f["fy"], f["cx"], f["cy"],
                           f["lim_x"], f["lim_y"], f["znear"], f["width"], f["height"])
        target = scene.target(cam)
        t0 = time.perf_counter()
        pre = O.preprocess_fwd(oc, scene.means, scene.quats, scales, opac, sh=sh,
                               degree=scene.sh_degree, flags=flags, threads=threads)
        feats = pre["colors"] if sh is not None else scene.features
        ids, ranges, _, _ = O.bin_gaussians(pre["means2d"], pre["radii"], pre["depths"],
                                            cam.width, cam.height, threads=threads)
        r = O.raster_fwd(pre["means2d"], pre["conics"], pre["opac_eff"], feats, ids, ranges,
                         cam.width, cam.height, depths=pre["depths"] if scene.depth else None,
                         threads=threads)
        t1 = time.perf_counter()
        if scene.backward:
            g_img = (np.sign(r["image"] - target) / np.float32(target.size)).astype(np.float32)
            gr = O.raster_bwd(pre["means2d"], pre["conics"], pre["opac_eff"], feats, ids,
                              ranges, cam.width, cam.height, r["final_T"], r["n_contrib"],
                              g_img, threads=threads)
            O.preprocess_bwd(oc, scene.means, scene.quats, scales, opac,
                             pre["colors"] if sh is not None else None,
                             0 if sh is None else sh.shape[1], scene.sh_degree, flags,
                             gr["means2d"], gr["conics"], gr["opacities"],
                             gr["features"] if sh is not None else None, threads=threads)
        t2 = time.perf_counter()
        t_fwd += t1 - t0
        t_all += t2 - t0
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    k = len(views)
    what = "fwd+bwd iteration" if scene.backward else "forward"
    return {"value": round(k / t_all, 4), "unit": "it/s" if scene.backward else "frames/s",
            "cores": threads, "kind": "port",
            "sample": f"{k} x 1 {what} (views {views[0]}..{views[-1]} of {cfg_name}, full "
                      f"frames, loss L1 as on the GPU), C oracle + OpenMP on {threads} threads",
            "fwd_s_per_view": round(t_fwd / k, 3), "iter_s_per_view": round(t_all / k, 3),
            "cpu_model": cpu}


def dense_reference_cpu(scene, view: int, gpu_image):
    """C1's "reference compositing path": reference.py:16-74 restated as
    torch-CPU float32, every Gaussian at every pixel in one global depth
    order, chunked over Gaussians (the transmittance in front of a chunk
    carries over; a splat is kept while the product of the earlier
    1 - alpha factors exceeds 1e-4, as reference.py:64-69).  Projection and
    colours come from the CPU oracle.  Timed end to end (projection, sort,
    compositing) on the host's torch threads, and compared with the GPU image
    of the same view."""
    import numpy as np
    import torch

    from oracle import oracle as O

    cam = scene.cameras[view]
    f = cam.gsx_fields()
    oc = O.make_camera(f["R"], f["t"], f["center"], f["fx"], f["fy"], f["cx"], f["cy"],
                       f["lim_x"], f["lim_y"], f["znear"], f["width"], f["height"])
    flags = O.LOG_SCALES | O.LOGIT_OPACITY | (O.ANTIALIAS if scene.antialias else 0)
    sh = np.concatenate([scene.sh_dc, scene.sh_rest], 1)
    H, W = cam.height, cam.width
    chunk = 256
    threads = torch.get_num_threads()
    t0 = time.perf_counter()
    pre = O.preprocess_fwd(oc, scene.means, scene.quats, scene.log_scales,
                           scene.logit_opacities, sh=sh, degree=scene.sh_degree, flags=flags,
                           threads=O.default_threads())
    order = np.argsort(pre["depths"], kind="stable")
    live = pre["radii"][order] > 0
    order = order[live]  # culled Gaussians have alpha 0 everywhere (reference.py:62)
    m2 = torch.from_numpy(pre["means2d"][order])
    con = torch.from_numpy(pre["conics"][order])
    op = torch.from_numpy(pre["opac_eff"][order])
    col = torch.from_numpy(pre["colors"][order])
    xs = (torch.arange(W, dtype=torch.float32) + 0.5).repeat(H)
    ys = (torch.arange(H, dtype=torch.float32) + 0.5).repeat_interleave(W)
    T = torch.ones(H * W)
    acc = torch.zeros(H * W, col.shape[1])
    with torch.no_grad():
        for s in range(0, m2.shape[0], chunk):
            e = min(s + chunk, m2.shape[0])
            dx = m2[s:e, 0:1] - xs[None]
            dy = m2[s:e, 1:2] - ys[None]
            power = -0.5 * (con[s:e, 0:1] * dx * dx + con[s:e, 2:3] * dy * dy) \
                - con[s:e, 1:2] * dx * dy
            a = torch.clamp_max(op[s:e, None] * torch.exp(power), 0.99)
            a = torch.where((power > 0) | (a < 1.0 / 255.0), torch.zeros_like(a), a)
            om = 1.0 - a
            front = T[None] * torch.cat([torch.ones_like(om[:1]), torch.cumprod(om, 0)[:-1]], 0)
            keep = front > 1e-4
            acc += (a * front * keep).transpose(0, 1) @ col[s:e]
            T = T * torch.where(keep, om, torch.ones_like(om)).prod(0)
    image = acc.reshape(H, W, -1).numpy()  # background 0, as the GPU render
    sec = time.perf_counter() - t0
    diff = np.abs(image - gpu_image)
    return {"value": round(1.0 / sec, 4), "unit": "frames/s", "cores": threads,
            "kind": "port",
            "sample": f"1 forward of view {view} of {scene.name}: reference.py:16-74 as dense "
                      f"torch-CPU fp32 over {m2.shape[0]} live Gaussians x {H * W} pixels, "
                      f"chunks of {chunk} Gaussians; projection/SH by the C oracle",
            "max_abs_vs_gpu": float(diff.max()),
            "pixels_over_1e-3": int((diff.max(-1) > 1e-3).sum())}


@contextlib.contextmanager
def _no_gc():
    """Python's cyclic garbage collector off inside a timed region (as timeit
    does): a collection pass over the autograd objects of earlier steps can
    stall the host for tens of milliseconds at an arbitrary step."""
    gc.collect()
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def train_step(model, cams, targets, steps: int, warmup: int, antialias: bool,
               workload: str) -> dict:
    """Times GaussianTrainer.step (trainer.py:319-421): fused render forward and
    backward, L1 + D-SSIM, Adam over the six groups.  Density control, opacity
    reset and SH growth are outside the measured steps, so the table keeps
    its size; the step's own loss readback (float(loss)) is included."""
    import torch

    from mlx3d_amd.profiling import StageTimer
    from mlx3d_amd.splatting.trainer import GaussianTrainer, TrainerConfig

    big = 1 << 30
    # the table keeps the bench's row order (spatial_order would leave an
    # already sorted table as it is)
    cfg = TrainerConfig(densify_from=big, densify_until=big, opacity_reset_every=big,
                        sh_increase_every=big, antialias=antialias)
    tr = GaussianTrainer(model, cfg)
    nviews = len(cams)
    for i in range(max(warmup, nviews)):
        tr.step(cams[i % nviews], targets[i % nviews])
    with _no_gc():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            tr.step(cams[i % nviews], targets[i % nviews])
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / steps
    # stage breakdown from a second pass with stage events recorded
    timer = StageTimer()
    with timer, _no_gc():
        for i in range(steps):
            tr.step(cams[i % nviews], targets[i % nviews])
        torch.cuda.synchronize()
    N = model.num_gaussians
    P = cams[0].width * cams[0].height
    floats = sum(int(v[0].numel()) for v in model.params.values())  # per Gaussian
    # the fused preprocess VJP + Adam: parameters and both moments read and
    # written (24 B per float), the rasterizer's per-Gaussian cotangents and
    # the SH colours read (48 B per Gaussian)
    algo = {"photometric_fwd": 20 * P * 3, "photometric_bwd": 24 * P * 3,
            "adam": 28 * N * floats, "preprocess_bwd_adam": N * (24 * floats + 48)}
    stages = {}
    for name in ("preprocess_fwd", "binning", "raster_fwd", "photometric_fwd",
                 "photometric_bwd", "raster_bwd", "preprocess_bwd", "adam",
                 "preprocess_bwd_adam"):
        t = timer.mean_ms(name)
        if math.isnan(t):
            continue
        stages[name] = {"ms": round(t, 4)}
        if name in algo:
            gbs = algo[name] / (t * 1e-3) / 1e9
            stages[name].update({"GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                                 "algorithmic_bytes": int(algo[name]),
                                 "traffic": _traffic(name, workload)})
    return {"ms": round(ms, 4), "it_s": round(1e3 / ms, 3), "steps": steps,
            "what": "GaussianTrainer.step: render fwd+bwd, L1 + 0.2 D-SSIM, Adam (6 groups, "
                    "fused into the preprocess backward)",
            "stages": stages}


# The reference's published Apple-GPU figures (docs/benchmarks.md:17-22),
# per-call latency in ms, for the cases of examples/benchmark.py:44-85.
REFERENCE_PUBLISHED_MS = {
    "hard rasterizer 20480 faces @ 256px": 4.3,
    "hard rasterizer 20480 faces @ 512px": 6.2,
    "hard rasterizer 20480 faces @ 1024px": 17.9,
    "gaussian splatting 10000 splats @ 512px": 12.5,
    "gaussian splatting 100000 splats @ 720px": 100.0,
}


def reference_suite():
    """examples/benchmark.py:68-85 (and :44-56 for the mesh rasterizer) on
    this GPU: the same inputs (points N(0, 1) * 0.6 with U(0, 1) colours
    through GaussianModel.from_points at SH degree 0; a 20 480-face
    icosphere), cameras and outputs.  `latency_ms` is the reference's
    measure -- each call waits for its result, as mx.eval does -- averaged
    over 50 calls after 5 warmups; `pipelined_ms` is the same calls
    enqueued back to back.  Synthetic data from numpy's PCG64 (MLX's
    generator is not available), so the splat sets are statistically, not
    bitwise, the reference's."""
    import numpy as np
    import torch

    from mlx3d_amd import scenes
    from mlx3d_amd.cameras import Camera
    from mlx3d_amd.renderer import interpolate_face_attributes, rasterize_meshes
    from mlx3d_amd.splatting import GaussianModel

    dev = torch.device("cuda:0")
    rows = []

    def timed(name, fn, iters=50, warmup=5):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
            torch.cuda.synchronize()
        lat = (time.perf_counter() - t0) / iters * 1e3
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        pipe = (time.perf_counter() - t0) / iters * 1e3
        ref = REFERENCE_PUBLISHED_MS[name]
        rows.append({"case": name, "latency_ms": round(lat, 4), "fps": round(1e3 / lat, 1),
                     "pipelined_ms": round(pipe, 4), "reference_ms": ref,
                     "speedup_vs_reference": round(ref / lat, 1)})

    verts, faces = scenes.ico_sphere(level=5, radius=1.0)
    v = torch.as_tensor(verts, device=dev)
    f = torch.as_tensor(faces, device=dev)
    vc = 0.5 * v + 0.5
    for size in (256, 512, 1024):
        cam = Camera.look_at(eye=(2.2, 1.6, 2.2), at=(0, 0, 0), fov=45.0, width=size,
                             height=size)

        def hard(cam=cam):
            frag = rasterize_meshes(cam, v, f)
            return interpolate_face_attributes(frag, vc)

        with torch.no_grad():
            timed(f"hard rasterizer {faces.shape[0]} faces @ {size}px", hard)
    rng = np.random.default_rng(0)
    for n, size in ((10_000, 512), (100_000, 720)):
        pts = torch.as_tensor((rng.standard_normal((n, 3)) * 0.6).astype(np.float32), device=dev)
        col = torch.as_tensor(rng.random((n, 3), dtype=np.float32), device=dev)
        model = GaussianModel.from_points(pts, col, sh_degree=0)
        cam = Camera.look_at(eye=(0, 0, -3.0), at=(0, 0, 0), fov=60.0, width=size, height=size)
        with torch.no_grad():
            timed(f"gaussian splatting {n} splats @ {size}px",
                  lambda model=model, cam=cam: model.render(cam)["image"])
    return {"metric": "reference benchmark cases (examples/benchmark.py), per-call latency",
            "unit": "ms", "device": torch.cuda.get_device_name(dev), "rows": rows,
            "reference_device": "Apple-Silicon GPU (docs/benchmarks.md, chip not named)"}


def main():
    args = _parse()
    if args.reference_suite:
        sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
        from mlx3d_amd import _lib

        _lib.load()
        print(json.dumps(reference_suite()), flush=True)
        return
    if args.summarize_prof:
        summarize_prof(args.summarize_prof, args.workload, args.command)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: only --gpus 1 is supported (got --gpus {args.gpus}, WORLD_SIZE "
              f"{world}). This build measures the rasterizer on one MI355X; across GPUs the "
              "path would shard by view for multi-view training (by bands of tile rows for a "
              "single view), with the per-Gaussian gradients all-reduced once per step.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from mlx3d_amd import _lib, scenes
    from mlx3d_amd.profiling import StageTimer
    from mlx3d_amd.losses import l1_loss
    from mlx3d_amd.splatting import GaussianModel, render_gaussian_features, spatial_order

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    scene = scenes.make_scene(args.config)
    cams = scene.cameras
    nviews = len(cams)
    feat_mode = scene.features is not None
    cu = lambda a: torch.as_tensor(a).to(dev)  # noqa: E731
    if feat_mode:
        leaf = {k: cu(v) for k, v in dict(
            means=scene.means, quats=scene.quats, scales=scene.scales,
            opacities=scene.opacities, features=scene.features).items()}
        if args.layout == "morton":
            perm = spatial_order(leaf["means"])
            leaf = {k: v[perm].contiguous() for k, v in leaf.items()}
        leaf = {k: v.requires_grad_(scene.backward) for k, v in leaf.items()}
    else:
        model = GaussianModel({"means": cu(scene.means), "quats": cu(scene.quats),
                               "scales": cu(scene.log_scales),
                               "opacities": cu(scene.logit_opacities),
                               "sh_dc": cu(scene.sh_dc), "sh_rest": cu(scene.sh_rest)},
                              sh_degree=3)
        model.active_sh_degree = scene.sh_degree
        if args.layout == "morton":
            model.reorder_spatial()
        model.requires_grad_(scene.backward)
        leaf = model.params
    targets = [cu(scene.target(c)) for c in cams]
    torch.cuda.synchronize()

    def render_all(i):
        cam = cams[i % nviews]
        if feat_mode:
            return render_gaussian_features(cam, leaf["means"], leaf["quats"], leaf["scales"],
                                            leaf["opacities"], leaf["features"],
                                            antialias=scene.antialias, return_depth=scene.depth)
        return model.render(cam, antialias=scene.antialias, return_depth=scene.depth)

    def render(i):
        return render_all(i)["features" if feat_mode else "image"]

    def step(i):
        for p in leaf.values():
            p.grad = None
        if not scene.backward:
            with torch.no_grad():
                render(i)
            return
        img = render(i)
        loss = l1_loss(img, targets[i % nviews])
        loss.backward()

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # the timed steps run without instrumentation; a second pass over the
    # same steps records HIP events around every stage for the breakdown
    with _no_gc():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            step(i)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps

    # The stage pass covers every view equally often (a whole number of
    # passes over the views, at least K steps), so per-stage means and
    # medians weigh the views alike even when K is not a multiple of them.
    stage_steps = -(-args.steps // nviews) * nviews
    timer = StageTimer()
    with timer, _no_gc():
        for i in range(stage_steps):
            step(i)
        torch.cuda.synchronize()

    # forward-only frames per second over the same views
    with torch.no_grad(), _no_gc():
        torch.cuda.synchronize()
        f0 = time.perf_counter()
        for i in range(args.steps):
            render(i)
        torch.cuda.synchronize()
        f1 = time.perf_counter()
    ms_fwd = (f1 - f0) * 1e3 / args.steps

    if args.copy_probe > 0:  # counter calibration: reads and writes MB megabytes once
        n = args.copy_probe * (1 << 20) // 4
        src = torch.zeros(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(2):
            _lib.check(_lib.load().gsx_debug_expf(n, _lib.ptr(src), _lib.ptr(dst),
                                                  _lib.stream_handle(dev)), "copy probe")
        torch.cuda.synchronize()
        del src, dst

    N = scene.n
    P = cams[0].width * cams[0].height
    C = scene.channels
    Ka = 0 if feat_mode else (scene.sh_degree + 1) ** 2
    D = float(np.mean(timer.counters["duplicates"]))
    with torch.no_grad():  # outside the timed regions, one render per view
        Dn = float(np.mean([needed_entries(render_all(i)["n_contrib"])
                            for i in range(nviews)]))
    B = algorithmic_bytes(N, D, P, C, Ka, not feat_mode, scene.depth)
    Bn = needed_bytes(Dn, N, P, C, scene.depth)
    stages = {}
    for name in ("preprocess_fwd", "binning", "raster_fwd", "raster_bwd", "preprocess_bwd"):
        ms = timer.mean_ms(name)
        if not math.isnan(ms):
            med = timer.median_ms(name)
            gbs = B[name] / (ms * 1e-3) / 1e9
            stages[name] = {"ms": round(ms, 4), "median_ms": round(med, 4),
                            "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                            "frac_median": round(B[name] / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
            if name in Bn:
                stages[name]["frac_needed_entries"] = round(
                    Bn[name] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    kernels = [k for k in ("raster_fwd", "raster_bwd", "preprocess_fwd", "preprocess_bwd")
               if k in stages]
    dom = max(kernels, key=lambda k: stages[k]["ms"])
    achieved = stages[dom]["GB/s"]
    workload = scene.name
    fwd_gbs = B["fwd"] / (ms_fwd * 1e-3) / 1e9
    it_s = 1e3 / ms_step
    out = {
        "metric": "fwd+bwd iters/s, 1M Gaussians SH3 @1920x1080 (GaussianModel.render + L1 + "
                  "backward)" if scene.backward else "forward frames/s",
        "value": round(it_s, 3),
        "unit": "it/s" if scene.backward else "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy PCG64 scene, random-init parameters)",
        "config": {"workload": workload, "gaussians": N, "width": cams[0].width,
                   "height": cams[0].height, "views": nviews, "sh_degree": scene.sh_degree,
                   "channels": C, "antialias": scene.antialias, "depth": scene.depth,
                   "layout": args.layout,
                   "duplicates_mean": int(D), "needed_entries_mean": int(Dn)},
        "fwd_fps": round(1e3 / ms_fwd, 2),
        "fwd_ms": round(ms_fwd, 4),
        "fwd_hbm_roofline_frac": round(fwd_gbs / HBM_PEAK_GBS, 4),
        "iter_hbm_roofline_frac": round(B["iter"] / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "kernel": dom, "kernel_symbol": KERNEL_SYMBOL[dom],
                     "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": _traffic(dom, workload),
                     "algorithmic_bytes": int(B[dom]), "mean_ms": stages[dom]["ms"],
                     "median_ms": stages[dom]["median_ms"],
                     "frac_median": stages[dom]["frac_median"],
                     "bytes_formula": "bench.py algorithmic_bytes: every duplicate charged",
                     "frac_needed_entries": stages[dom].get("frac_needed_entries"),
                     "issue": _issue(dom, workload, stages[dom]["ms"])},
        "stages": stages,
    }
    if args.train_steps > 0 and scene.backward and not feat_mode:
        out["train_step"] = train_step(model, cams, targets, args.train_steps, args.warmup,
                                       scene.antialias, scene.name)
    if not args.no_cpu_baseline:
        print("bench: timing CPU oracle baseline ...", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(scene, list(range(nviews)), workload)
    else:
        out["cpu_baseline"] = None
    if args.config == 1 and not args.no_cpu_baseline:
        print("bench: timing the dense reference path on the CPU ...", file=sys.stderr,
              flush=True)
        with torch.no_grad():
            gpu_img = render(0).cpu().numpy()
        out["reference_path_cpu"] = dense_reference_cpu(scene, 0, gpu_img)
    if args.profile_stages:
        print(json.dumps(stages, indent=1), file=sys.stderr)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
