"""Benchmark of the gfx950 render path: fwd and fwd+bwd frames/s on the BASELINE workload.

A step is one forward + backward render of the workload (project -> rasterize -> MSE loss ->
backward through rasterize and project, the loss fused into the blends by
splax_amd.render_loss), with all inputs resident in HBM. The default workload is
config 2 (1,000,000 gaussians on 64 planes, one 1920x1080 camera).

The JSON line carries:
- value: forward+backward frames/s (whole job, one GPU; a frame is one rendered image, so a
  batched step of B cameras counts B); fwd_frames_per_s: forward only.
- roofline: the dominant kernel's algorithmic work per launch / its average launch duration,
  timed with HIP events on the launch stream inside the timed region (library timing, enabled
  for that kernel only: a blend kernel's events ride on its own dispatch, hipExtLaunchKernelGGL;
  a separate untimed pass with every stage bracketed gives stage_ms_per_step and picks the
  dominant stage).
  Blend work is the reference loop's pair count from the CPU oracle (26 Pc + 16 Pr FLOPs
  forward, 65 Qc + 16 Qr backward); depth range, emission, sort and bin bytes are
  12G + 32V + 104M + 16T.
- stages: every stage's average duration per call (HIP events around each stage, in an untimed
  pass) with its algorithmic bytes or FLOPs per call and the achieved rate against MI355X's peak
  (HBM 8 TB/s for projection, depth range, emission, sort, bins and the projection backward;
  FP32 157.3 TFLOP/s for the two blends). `work_per_call` / `frac` price the stage on the
  path's algorithmic bytes (projection 44 N + 40 G, depth range 8 G, emission 4 G + 32 V + 8 M,
  sort 64 M, bins 4 M + 16 T, projection backward 40 N + 80 G); `moved_per_call` /
  `frac_moved` on the bytes this build's kernels move (the fused projection's colour reads and
  record writes, the sort's positions and 16-bit key halves, the bins' 16-bit halves).
- resort_path_frames_per_s: forward+backward frames/s through the reference's own call shape,
  one library call per custom_vjp rule: project, rasterize (its own sort), the loss cotangent,
  a rasterize backward that sorts again (splat_rasterize_bwd), the projection backward; the
  value line's step keeps the forward's sorted lists and records instead.
- cpu_baseline: the CPU oracle (the C restatement of the reference kernels, "port") timed on the
  host on one full forward+backward frame of the same workload, OpenMP over `cores` threads
  (the host's share, at most 16), and again on one thread (`single_thread`), with the CPU model.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--n", type=int, default=None, help="override the gaussian count")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=None)
    ap.add_argument("--fwd-only", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="end with three plain 256 MiB device copies (counter calibration for "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE runs)")
    return ap.parse_args()


def profiled_traffic(kernel, config):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary, or None.

    profiles/<kernel>_config<k>_hbm_traffic.md holds a line
    `traffic_bytes_per_launch: <int>` (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the
    counter's reading for a copy of known size)."""
    path = ROOT / "profiles" / f"{kernel}_config{config}_hbm_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def oracle_leg(scene, threads):
    """Time the CPU oracle on one full fwd+bwd frame; also returns the reference loop counts."""
    import numpy as np

    from oracle import oracle as O

    O.set_threads(threads)
    s = scene
    q = np.roll(s.quats, -1, axis=-1)
    B = s.B
    vm = s.viewmats.reshape(-1, 4)
    t0 = time.perf_counter()
    xys, depths, radii, conics, nth, cum = O.project_fwd(
        s.means, s.scales, q, vm, s.opacities, n=s.n, total=B * s.n, img_shape=s.img_shape,
        f=s.f, c=s.c)
    img, Ts, fidx, fstats, M = O.rasterize_fwd(s.colors, s.opacities, s.opacities, s.background,
                                               xys, depths, radii, conics, cum, n=s.n, B=B,
                                               img_shape=s.img_shape)
    t1 = time.perf_counter()
    H, W = s.img_shape
    vout = (2.0 * (img.reshape(B, H, W, 3) - s.targets) / img.size).astype(np.float32)
    g = O.rasterize_bwd(s.colors, s.opacities, s.opacities, s.background, xys, depths, radii,
                        conics, cum, Ts, fidx, vout, n=s.n, B_out=B, B_geom=B,
                        img_shape=s.img_shape)
    O.project_bwd(s.means, s.scales, q, vm, radii, conics, g[2],
                  np.zeros(B * s.n, np.float32), g[3], n=s.n, B=B, f=s.f)
    t2 = time.perf_counter()
    counts = dict(G=B * s.n, V=int((radii > 0).sum()), M=int(M), Pc=int(fstats[0]),
                  Pr=int(fstats[1]), Qc=int(g[4][0]), Qr=int(g[4][1]))
    return (t1 - t0), (t2 - t0), counts


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# Work per call of each library stage: (bound, algorithmic work, work this build moves, unit)
# from the workload counts (G items, N gaussians, V visible items, M intersections, T tiles,
# Pc/Pr and Qc/Qr the contributing / rejected pixel-gaussian pairs of the forward / backward
# walk). Algorithmic bytes are the path's own (projection 44 N + 40 G, sort 64 M: four passes
# reading and writing 8-byte pairs, bins 4 M + 16 T). What this build moves: the step renders
# through splat_render_fwd, whose projection also reads the colours (12 B/gaussian) and writes the
# packed blend records (64 B/item), 56 N + 104 G; its sort reads 4 + 4 + 2 + 2 B per key for the
# digit counts and its scatters move 20 + 22 + 20 + 20 B per key (key, emission position, id; the
# pass over bits 8-15 writes the keys' 16-bit high halves, which the last two passes and the bin
# edges read), 94 M; the bins read those 16-bit halves, 2 M + 16 T.
def stage_work(counts, N, T):
    G, V, M = counts["G"], counts["V"], counts["M"]
    fwd_flops = 26 * counts["Pc"] + 16 * counts["Pr"]
    bwd_flops = 65 * counts["Qc"] + 16 * counts["Qr"]
    return {
        "project": ("hbm", 44 * N + 40 * G, 56 * N + 104 * G, "GB/s"),
        "minmax": ("hbm", 8 * G, 8 * G, "GB/s"),
        "emit": ("hbm", 4 * G + 32 * V + 8 * M, 4 * G + 32 * V + 8 * M, "GB/s"),
        "sort": ("hbm", 64 * M, 94 * M, "GB/s"),
        "bins": ("hbm", 4 * M + 16 * T, 2 * M + 16 * T, "GB/s"),
        "blend_fwd": ("valu", fwd_flops, fwd_flops, "TFLOP/s"),
        "blend_fwd_kernel": ("valu", fwd_flops, fwd_flops, "TFLOP/s"),
        "blend_bwd": ("valu", bwd_flops, bwd_flops, "TFLOP/s"),
        "blend_bwd_kernel": ("valu", bwd_flops, bwd_flops, "TFLOP/s"),
        "project_bwd": ("hbm", 40 * N + 80 * G, 40 * N + 80 * G, "GB/s"),
    }


def stage_rates(cal, cal_steps, counts, N, T):
    """Per-stage average ms per call and achieved rate against peak, from a pass with every stage
    bracketed by HIP events."""
    out = {}
    work = stage_work(counts, N, T) if counts else {}
    for name, (ms, calls) in cal.items():
        if not calls:
            continue
        per_call = ms / calls
        row = {"ms_per_call": round(per_call, 4), "calls_per_step": round(calls / cal_steps, 2)}
        if name in work:
            bound, w, moved, unit = work[name]
            scale = 1e12 if unit == "TFLOP/s" else 1e9
            rate = w / (per_call / 1e3) / scale
            peak = FP32_PEAK_TFLOPS if unit == "TFLOP/s" else HBM_PEAK_GBS
            row.update(bound=bound, work_per_call=int(w), achieved=round(rate, 2), unit=unit,
                       frac=round(rate / peak, 4))
            if moved != w:
                mrate = moved / (per_call / 1e3) / scale
                row.update(moved_per_call=int(moved), achieved_moved=round(mrate, 2),
                           frac_moved=round(mrate / peak, 4))
        out[name] = row
    return out


def resort_path_ms(scene, params, vm, bg, target, steps, warmup=2):
    """ms per fwd+bwd step through the reference's call shape (splax/_render.py:94-115 with the
    custom_vjp rules of splax/_project/_project.py and splax/_rasterize/_rasterize.py): one
    library call per rule, the rasterize backward sorting again (splat_rasterize_bwd, as the
    reference's _rasterize_bwd_warp does at splax/_rasterize/_kernels.py:422), the MSE and its
    image cotangent in torch (the caller's loss), per-camera colour / opacity rows summed in
    torch for a batch."""
    import torch

    from splax_amd import _ops

    B, n = scene.B, scene.n
    H, W = scene.img_shape
    dev = params[0].device
    means, scales, quats, colors, opac = (p.detach() for p in params)
    opac = opac.reshape(-1)
    vmf = vm.detach().reshape(-1, 4)
    tgt = target.reshape(B * H, W, 3)
    tf = torch.zeros((1, 4, 4), device=dev)
    tids = torch.full((1,), -1, device=dev, dtype=torch.int32)
    want_vm = vm.requires_grad

    def step():
        xys, depths, radii, conics, _, cum = _ops.project_fwd(
            means, scales, quats, vmf, opac, tf, tids, n=n, total=B * n, num_transforms=1,
            has_transforms=False, img_shape=(H, W), f=scene.f, c=scene.c, glob_scale=1.0,
            clip_thresh=0.01, quats_wxyz=True)
        img, Ts, fidx, _ = _ops.rasterize_fwd(colors, opac, opac, bg, xys, depths, radii,
                                              conics, cum, n=n, B=B, img_shape=(H, W))
        d = img - tgt
        loss = (d * d).mean()
        v_out = d * (2.0 / d.numel())
        vc, vo, vxy, vcon = _ops.rasterize_bwd(colors, opac, opac, bg, xys, depths, radii,
                                               conics, cum, Ts, fidx, v_out.reshape(-1, 3), n=n,
                                               B_out=B, B_geom=B, img_shape=(H, W))
        if B > 1:
            vc, vo = vc.reshape(B, n, 3).sum(0), vo.reshape(B, n).sum(0)
        _ops.project_bwd(means, scales, quats, vmf, radii, conics, vxy, None, vcon, tf, tids,
                         n=n, B=B, num_transforms=1, has_transforms=False, f=scene.f,
                         glob_scale=1.0, quats_wxyz=True, fold=B > 1, want_viewmat=want_vm)
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def bench_train(args):
    """Config 4: the full training step (render_log fwd+bwd over B=4 cameras with antialiasing,
    L1, fused Adam, one MCMC relocation), steps/s."""
    import numpy as np
    import torch

    from splax_amd import _lib, mcmc
    from splax_amd.scenes import make_scene
    from splax_amd.train import TrainStep, params_from_scene

    dev = torch.device("cuda:0")
    scene = make_scene(4, n=args.n)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    params = params_from_scene(scene, dev)
    H, W = scene.img_shape
    train = TrainStep(params, viewmats=t(scene.viewmats), targets=t(scene.targets),
                      background=t(scene.background), img_shape=(H, W), f=scene.f,
                      antialiased=True, seed=4)
    for _ in range(args.warmup):
        train()
    torch.cuda.synchronize()
    # breakdown pass: library stages plus events around the Adam and relocation launches
    ev = {k: [torch.cuda.Event(enable_timing=True) for _ in range(2)]
          for k in ("render_fwd_bwd", "adam", "relocate")}
    _lib.stage_times()
    _lib.set_stage_timing(True)
    cal_steps = 3
    part_ms = {k: 0.0 for k in ev}
    for _ in range(cal_steps):
        ev["render_fwd_bwd"][0].record()
        loss, grads = train.loss_and_grads()
        ev["render_fwd_bwd"][1].record()
        ev["adam"][0].record()
        train.opt.step(grads)
        ev["adam"][1].record()
        train.step_idx += 1
        ev["relocate"][0].record()
        reset = mcmc.relocate_((train.seed << 32) ^ train.step_idx, *train.params.values(),
                               train.binoms, train.min_opacity)
        train.opt.reset_rows(reset)
        ev["relocate"][1].record()
        torch.cuda.synchronize()
        for k, (a, b) in ev.items():
            part_ms[k] += a.elapsed_time(b)
    _lib.set_stage_timing(False)
    cal = _lib.stage_times()
    stage_ms_per_step = {k: round(v[0] / cal_steps, 4) for k, v in cal.items()}
    part_ms = {k: round(v / cal_steps, 4) for k, v in part_ms.items()}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        train()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    n = scene.n
    adam_bytes = 7 * 4 * 14 * n  # read p, g, mu, nu and write p, mu, nu for 14 floats/gaussian
    adam_s = part_ms["adam"] / 1e3
    out = {
        "metric": "config-4 training steps/sec (3M gaussians, 4 cameras 1600x1060, antialiased, "
                  "L1 + Adam + MCMC relocate)",
        "value": round(1e3 / ms, 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy PCG64, BASELINE.json config 4 distributions)",
        "config": {"workload": "config4", "gaussians": n, "cameras": scene.B,
                   "img_shape": [H, W], "loss": "l1", "antialiased": True,
                   "optimizer": "adam (5 groups, fused)", "relocate_every": 1,
                   "parallelism": "single-gpu"},
        "stage_ms_per_step": stage_ms_per_step,
        "stages": stage_rates(cal, cal_steps, None, n, 0),
        "part_ms_per_step": part_ms,
        "roofline": {"kernel": "adam_step", "bound": "hbm",
                     "achieved": round(adam_bytes / adam_s / 1e9, 1) if adam_s > 0 else None,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(adam_bytes / adam_s / 1e9 / HBM_PEAK_GBS, 4)
                     if adam_s > 0 else None,
                     "traffic": profiled_traffic("adam_step", 4), "work_per_launch": adam_bytes},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)
    if args.calibrate_copy:
        calibrate_copy(dev)


def calibrate_copy(dev):
    """Three plain 256 MiB device copies after the bench line: the FETCH_SIZE / WRITE_SIZE scale
    of the HBM traffic summaries under profiles/ comes from them."""
    import torch

    src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(the path shards by camera across GPUs by design, but no multi-GPU run is built)",
              file=sys.stderr)
        sys.exit(2)
    if args.config == 4:
        bench_train(args)
        return
    import numpy as np
    import torch

    import splax_amd
    from splax_amd import _lib
    from splax_amd.scenes import make_scene

    dev = torch.device("cuda:0")
    scene = make_scene(args.config, n=args.n)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    params = [t(scene.means), t(scene.scales), t(scene.quats), t(scene.colors),
              t(scene.opacities)]
    for p in params:
        p.requires_grad_(True)
    B = scene.B
    vm = t(scene.viewmats if B > 1 else scene.viewmats[0])
    if args.config == 3:
        vm.requires_grad_(True)  # config 3 differentiates the camera poses too
    bg = t(scene.background)
    target = t(scene.targets if B > 1 else scene.targets[0])
    H, W = scene.img_shape

    def forward():
        img, _ = splax_amd.render(*params, viewmat=vm, background=bg, img_shape=(H, W),
                                  f=scene.f, antialiased=scene.antialiased)
        return img

    one = target.new_ones(())  # the loss cotangent, made once (backward() would fill one per step)

    def step():
        for p in params:
            p.grad = None
        vm.grad = None
        # the MSE fused into the blends: the forward blend sums each tile's squared errors as
        # it writes the image, the backward blend forms each pixel's image cotangent (no loss
        # passes over the image: 30 us of GPU time as separate launches)
        loss, _ = splax_amd.render_loss(*params, target=target, loss="mse", viewmat=vm,
                                        background=bg, img_shape=(H, W), f=scene.f,
                                        antialiased=scene.antialiased)
        loss.backward(one)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # forward-only frames/s
    with torch.no_grad():
        for _ in range(2):
            forward()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            forward()
        torch.cuda.synchronize()
        fwd_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    # per-stage breakdown (untimed pass: every stage bracketed by events)
    _lib.stage_times()  # reset
    _lib.set_stage_timing(True)
    cal_steps = 3
    for _ in range(cal_steps):
        step()
    torch.cuda.synchronize()
    _lib.set_stage_timing(False)
    cal = _lib.stage_times()
    stage_ms_per_step = {k: round(v[0] / cal_steps, 4) for k, v in cal.items()}
    roof_stages = ("blend_bwd", "blend_fwd", "sort", "project")
    dom = max(roof_stages, key=lambda k: cal[k][0])
    # timed fwd+bwd region: only the dominant stage is timed, a blend by the events its kernel's
    # own dispatch carries (no marker packets between kernels), other stages by bracketing events
    timed = dom + "_kernel" if dom + "_kernel" in cal else dom
    _lib.stage_times()
    _lib.set_stage_timing([timed])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    _lib.set_stage_timing(False)
    stages = _lib.stage_times()
    resort_ms = resort_path_ms(scene, params, vm, bg, target, args.steps)

    counts = None
    cpu = None
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        cpu_fwd_s, cpu_s, counts = oracle_leg(scene, threads)
        cpu = {"value": round(B / cpu_s, 4), "unit": "frames/s", "cores": threads,
               "kind": "port",
               "sample": f"one full fwd+bwd step of config {args.config} "
                         f"({scene.n} gaussians, {B} frame(s) of {H}x{W}) by the C oracle; "
                         f"fwd alone {cpu_fwd_s:.2f} s",
               "cpu_model": cpu_model(), "host_logical_cpus": os.cpu_count()}
        # one thread as well (Warp's CPU device runs a launch on one thread), for frames up to
        # about 2M items (config 2 takes about 20 s there)
        if B * scene.n <= 2_000_000 and threads > 1:
            st_fwd_s, st_s, _ = oracle_leg(scene, 1)
            cpu["single_thread"] = {"value": round(B / st_s, 4), "unit": "frames/s",
                                    "cores": 1, "fwd_s": round(st_fwd_s, 3),
                                    "fwd_bwd_s": round(st_s, 3)}

    per_stage = {k: (v[0] / v[1] if v[1] else 0.0) for k, v in stages.items()}
    roofline = None
    if counts is not None:
        G, V, M = counts["G"], counts["V"], counts["M"]
        T = B * ((W + 15) // 16) * ((H + 15) // 16)
        cands = {
            "blend_bwd": ("valu", (65 * counts["Qc"] + 16 * counts["Qr"]) / 1e12, "TFLOP/s",
                          FP32_PEAK_TFLOPS),
            "blend_fwd": ("valu", (26 * counts["Pc"] + 16 * counts["Pr"]) / 1e12, "TFLOP/s",
                          FP32_PEAK_TFLOPS),
            "sort": ("hbm", 64 * M / 1e9, "GB/s", HBM_PEAK_GBS),
            "project": ("hbm", (44 * scene.n + 40 * G) / 1e9, "GB/s", HBM_PEAK_GBS),
        }
        bound, work, unit, peak = cands[dom]
        dur_s = per_stage[timed] / 1e3
        achieved = work / dur_s if dur_s > 0 else 0.0
        roofline = {"kernel": dom, "bound": bound, "achieved": round(achieved, 3),
                    "peak": peak, "unit": unit, "frac": round(achieved / peak, 4),
                    "traffic": profiled_traffic(dom, args.config),
                    "avg_launch_ms": round(per_stage[timed], 4), "timed": timed,
                    "work_per_launch": work * (1e12 if unit == "TFLOP/s" else 1e9)}

    # a frame is one rendered image: a batched step (config 3) renders B of them
    metric = "fwd and fwd+bwd frames/sec @1M gaussians 1080p; HBM GB/s & VALU % of peak"
    if args.config != 2 or args.n is not None:
        metric = f"fwd and fwd+bwd frames/sec, config {args.config} ({scene.n} gaussians, " \
                 f"{B} x {W}x{H})"
    out = {
        "metric": metric,
        "value": round(B * 1e3 / ms, 3),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "fwd_frames_per_s": round(B * 1e3 / fwd_ms, 3),
        "fwd_ms": round(fwd_ms, 4),
        "resort_path_frames_per_s": round(B * 1e3 / resort_ms, 3),
        "resort_path_ms": round(resort_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy PCG64, BASELINE.json config distributions)",
        "config": {"workload": f"config{args.config}", "gaussians": scene.n, "cameras": B,
                   "img_shape": [H, W], "loss": "mse", "viewmat_grads": args.config == 3,
                   "parallelism": "single-gpu"},
        "stage_ms_per_step": stage_ms_per_step,
        "stages": stage_rates(cal, cal_steps, counts, scene.n,
                              B * ((W + 15) // 16) * ((H + 15) // 16)),
        "counts": counts,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    if args.calibrate_copy:
        calibrate_copy(dev)


if __name__ == "__main__":
    main()
