"""Benchmark: one full cost -> matching -> matched-loss forward + backward step
of MaskMatchingFunction on the headline configuration (BASELINE.json
B=16, Q=200, 256x256 bf16 mask logits, G ~ U[5,100], C=133 +
no-object), synthetic inputs resident in HBM.

Prints ONE JSON line (rank 0).  `value` = milliseconds per step (lower is
better), timed with events around K uninstrumented steps.  `roofline` = the
dominant kernel's algorithmic bytes per launch over its average launch
duration, measured with HIP events that the library records on its launch
stream around each launch group during K further steps.  `cpu_baseline` = the float64
oracle (a port of the reference algorithm; the reference's own CPU path is not
buildable here) timed on a bounded sample of the same workload on this host.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="cfg3_dense_headline",
                    help="workload of the main line; cfg2_point_sampling_front_end runs only the "
                         "point-sampling front end")
    ap.add_argument("--cpu-sample-images", type=int, default=16,
                    help="images of the headline step the host oracle runs (16 = the whole step)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the per-config lines of the other BASELINE configurations")
    ap.add_argument("--other-steps", type=int, default=50)
    ap.add_argument("--other-warmup", type=int, default=5)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device copy of 512 MiB (3 launches), the reference "
                         "point for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="run only the read-only HBM stream over the headline logits' size "
                         "(ml_profile_stream_read) and print its GB/s")
    return ap.parse_args()


COPY_BYTES = 512 << 20


def copy_calibration():
    import torch
    src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "launches": 3}), flush=True)


READ_BYTES = 16 * 200 * 256 * 256 * 2  # the headline's bf16 logits, read once by the contraction


def read_ceiling(reps=20):
    """Practical HBM read ceiling: ml_profile_stream_read (16-byte loads, one
    contiguous chunk per workgroup, eight loads in flight per thread) over
    READ_BYTES, timed with HIP events on the launch stream; per grid size the
    best and median of `reps` launches."""
    import torch
    lib = prof_lib()
    src = torch.ones(READ_BYTES // 2, dtype=torch.bfloat16, device="cuda:0")
    out = torch.empty(8192, dtype=torch.int32, device="cuda:0")
    st = torch.cuda.current_stream()
    res = {}
    for grid in (1024, 2048, 4096):
        for _ in range(3):
            lib.ml_profile_stream_read(ctypes.c_void_p(src.data_ptr()), READ_BYTES,
                                       ctypes.c_void_p(out.data_ptr()), grid, ctypes.c_void_p(st.cuda_stream))
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            rc = lib.ml_profile_stream_read(ctypes.c_void_p(src.data_ptr()), READ_BYTES,
                                            ctypes.c_void_p(out.data_ptr()), grid,
                                            ctypes.c_void_p(st.cuda_stream))
            e1.record(st)
            if rc != 0:
                raise RuntimeError("ml_profile_stream_read failed")
            e1.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3)
        ts.sort()
        res[grid] = {"best_us": round(ts[0], 2), "median_us": round(ts[len(ts) // 2], 2),
                     "best_GBs": round(READ_BYTES / (ts[0] * 1e-6) / 1e9, 1),
                     "median_GBs": round(READ_BYTES / (ts[len(ts) // 2] * 1e-6) / 1e9, 1)}
    best = max(res.values(), key=lambda r: r["median_GBs"])
    return {"bytes": READ_BYTES, "grids": res, "median_GBs": best["median_GBs"],
            "best_GBs": best["best_GBs"]}


def load_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` on `workload` from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (scaled by the copy-kernel
    factor), or None if that profile is absent."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)[workload][kernel]
        return int(rec["fetch_bytes"] + rec["write_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def prof_lib():
    import mask_loss_amd
    lib = ctypes.CDLL(mask_loss_amd.HIP_LIBRARY)
    lib.ml_profile_enable.argtypes = [ctypes.c_int]
    lib.ml_profile_read.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64),
                                    ctypes.POINTER(ctypes.c_double)]
    lib.ml_profile_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                           ctypes.c_int, ctypes.c_void_p]
    return lib


def read_prof(lib, name):
    n = ctypes.c_int64(0)
    t = ctypes.c_double(0.0)
    if lib.ml_profile_read(name.encode(), ctypes.byref(n), ctypes.byref(t)) != 0:
        return 0, 0.0
    return n.value, t.value


def cpu_threads():
    """Host threads for the CPU baseline: OMP_NUM_THREADS when set (the GPU
    box's CPU share), else every core."""
    try:
        n = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        n = 0
    return max(1, n or os.cpu_count() or 1)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def total_cost_matrices(cfg, x, z, zc):
    """The fp32 total-cost matrices (L*B, Q, GT_out) of the step, as the
    reference's matcher receives them (src/cpu/matching.cpp:665-704)."""
    import mask_loss_amd
    k = cfg.kwargs
    sep = mask_loss_amd.mask_loss.pairwise_mask_loss_forward(
        z.detach(), x["mask_targets"], zc.detach(), x["cls_targets"], k["smooth"],
        k["sigmoid_scale"], k["dice_scale"], k["cls_scale"], k["background_index"],
        k["uncertainty_gamma"], k["uncertainty_gamma_min"], k["mask_focal_gamma"],
        -1.0 if k["mask_focal_alpha"] is None else k["mask_focal_alpha"], k["cls_focal_gamma"],
        -1.0 if k["cls_focal_alpha"] is None else k["cls_focal_alpha"],
        k["label_loss"] == "softmax", k["normalize_uncertainty"])
    total = ((sep[0] + sep[1]) + sep[2]).double().cpu().numpy()
    L, B, Q, G = total.shape
    return total.reshape(L * B, Q, G)


def cpu_matcher(total, threads):
    """The reference's CPU stage (src/cpu/matching.cpp:690-719: the
    assignment of every (layer, image) slice, at::parallel_for over slices):
    the C restatement with `threads` OpenMP threads on the GPU's cost
    matrices.  Milliseconds per step."""
    from oracle import assign as OA
    OA.assign_batch(total[:1], 1e30, 1, 0, nthreads=1)  # load the library first
    t0 = time.perf_counter()
    OA.assign_batch(total, 1e30, 1, 0, nthreads=threads)
    return (time.perf_counter() - t0) * 1e3


def cpu_baseline(cfg, x, z, zc, p2g_gpu, total, n_img, threads):
    """The whole step on the host: the float64 NumPy oracle (pairwise cost,
    matched-loss forward, backward) of n_img images with all of their
    queries, the images spread over `threads` threads (one BLAS thread each),
    plus the C assignment restatement on every image's GPU cost matrix with
    `threads` threads.  With n_img = B nothing is extrapolated."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import mask_oracle as O
    k = cfg.kwargs
    n_img = max(1, min(n_img, cfg.B))
    imgs = []
    for b in range(n_img):  # host copies outside the timed region
        imgs.append((z.detach()[:, b:b + 1].float().cpu().numpy().astype(np.float64),
                     zc.detach()[:, b:b + 1].float().cpu().numpy().astype(np.float64),
                     x["mask_targets"][b:b + 1].cpu().numpy(),
                     x["cls_targets"][b:b + 1].cpu().numpy(), p2g_gpu[:, b:b + 1]))

    def one(b):
        zb, zcb, tgt, ct, p2g = imgs[b]
        sep = O.pairwise_mask_loss_forward(zb, tgt, zcb, ct, k["smooth"], k["sigmoid_scale"],
                                           k["dice_scale"], k["cls_scale"], k["background_index"],
                                           k["uncertainty_gamma"], k["uncertainty_gamma_min"], 0.0,
                                           -1.0, 0.0, -1.0, True, True)
        O.matching_forward_losses(sep, p2g, zb, zcb, tgt.shape, force_cls=True,
                                  void_class_index=cfg.C, use_softmax=True)
        O.matching_backward(np.ones(1), np.ones(1), np.ones(1), zb, tgt, zcb, ct, p2g,
                            background_index=0, force_cls=True, void_class_index=cfg.C,
                            use_softmax=True)

    t0 = time.perf_counter()
    with threadpool_limits(limits=1):
        with ThreadPoolExecutor(threads) as ex:
            list(ex.map(one, range(n_img)))
    t_img = time.perf_counter() - t0
    t_match = cpu_matcher(total, threads)
    scale = cfg.B / n_img
    ms = t_img * scale * 1e3 + t_match
    sample = (f"float64 NumPy oracle on {n_img} of {cfg.B} images, all {cfg.Q} queries each "
              f"(cost + matched loss fwd/bwd, {threads} threads, {t_img:.1f} s wall)")
    sample += f" scaled x{scale:g}" if n_img < cfg.B else " (the whole step, not extrapolated)"
    sample += (f", plus the C assignment restatement on all {total.shape[0]} GPU cost "
               f"matrices with {threads} threads ({t_match:.1f} ms)")
    return {
        "value": round(ms, 1), "unit": "ms/step", "cores": threads, "kind": "port",
        "sample": sample, "cpu_model": cpu_model(), "cpu_count": os.cpu_count(),
        "matcher_ms": round(t_match, 2),
    }


def step_bytes_of(cfg, e, M):
    """Algorithmic HBM bytes of one step: logits read by the forward, matched
    logits read and all gradients written by the backward, the int64 label
    map once, class logits read twice and their gradient written once."""
    K = cfg.H * cfg.W
    LBQ = cfg.L * cfg.B * cfg.Q
    Ht, Wt = cfg.H * cfg.scale, cfg.W * cfg.scale
    return e * K * (LBQ + M + LBQ) + 8 * cfg.B * Ht * Wt + 12 * LBQ * (cfg.C + 1)


def make_step(cfg, dev):
    import torch
    from mask_loss_amd import synth
    from mask_loss_amd.functions import MaskMatchingFunction
    x = synth.make_torch(cfg, dev, logits_on_device_rng=True)
    z = x["mask_logits"].requires_grad_(True)
    zc = x["cls_logits"].requires_grad_(True)
    args = synth.call_args(cfg, dict(x, mask_logits=z, cls_logits=zc))
    state = {}
    # upstream gradients of the three per-layer means: ones(L) each, i.e. the
    # gradient of loss = sum of the layer means
    ones = [torch.ones(cfg.L, device=dev) for _ in range(3)]

    def step():
        z.grad = None
        zc.grad = None
        p2g, pr, m, d, c = MaskMatchingFunction.apply(*args)
        torch.autograd.backward((m, d, c), ones)
        state["p2g"] = p2g

    return x, z, zc, step, state


def time_steps(step, steps, warmup):
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def other_config(cfg, dev, steps, warmup, cpu=True):
    """ms/step, images/s and the step's fraction of the HBM / MFMA roofline for
    another BASELINE configuration (same step, fewer timed steps), and the
    reference's CPU stage (the assignment) timed on the host."""
    x, z, zc, step, state = make_step(cfg, dev)
    ms = time_steps(step, steps, warmup)
    cpu_m = None
    if cpu:
        threads = cpu_threads()
        cpu_m = {"matcher_ms": round(cpu_matcher(total_cost_matrices(cfg, x, z, zc), threads), 2),
                 "threads": threads, "kind": "port",
                 "what": "C restatement of the reference's assignment (src/cpu/matching.cpp:476-571, "
                         "690-719) on the step's GPU cost matrices"}
    M = int((state["p2g"] >= 0).sum().item())
    e = z.element_size()
    sb = step_bytes_of(cfg, e, M)
    t_hbm = sb / HBM_PEAK_GBS / 1e3  # us
    t_roof = t_hbm  # HBM binds in every configuration (the contraction's MFMA time is lower)
    return {"workload": cfg.name, "ms_per_step": round(ms, 4),
            "images_per_s": round(cfg.B * cfg.L / (ms * 1e-3), 1), "dtype": cfg.dtype,
            "matched": M, "step_algorithmic_bytes": sb, "hbm_floor_us": round(t_hbm, 1),
            "roofline_frac": round(t_roof / (ms * 1e3), 4), "steps": steps, "warmup": warmup,
            "cpu_matcher": cpu_m}


def point_front_end(dev, steps, warmup):
    """Point-sampling front end at configuration 2's shape: mask logits
    (1, 8, 100, 128, 128) float32 ~ N(0, 2), label maps (8, 512, 512) from the
    configuration's recipe, 12,544 points per image (torch.rand).  Times the
    bilinear point gather alone (HIP events on the launch stream) and one
    matcher front end: the point-sampled pairwise sigmoid-CE and dice costs
    (two calls, each sampling the logits and reading targets.max() back, as
    the reference's functions do); then configuration 2's Mask2Former-style
    step on the same points: sampling with its gradient, then the fused
    cost -> assignment -> loss forward and backward."""
    import dataclasses
    import numpy as np
    import torch
    from mask_loss_amd import synth
    from mask_loss_amd.functions import (pairwise_dice_loss_sampling_py,
                                         pairwise_sigmoid_cross_entropy_loss_sampling_py)
    ml = mask_loss_amd_module()
    cfg2 = [c for c in synth.CONFIGS if c.name == "cfg2_point_sampled"][0]
    cfg = dataclasses.replace(cfg2, H=128, W=128, scale=4)
    rng = np.random.Generator(np.random.PCG64(cfg.seed))
    labels, cls_t, _ = synth.make_targets(cfg, rng)
    t = torch.from_numpy(np.ascontiguousarray(labels)).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    z = torch.randn(cfg.L, cfg.B, cfg.Q, cfg.H, cfg.W, device=dev, generator=g) * cfg.sigma
    P = 12544
    coords = torch.rand(cfg.B, P, 2, device=dev, generator=g)
    # the gather alone
    for _ in range(warmup):
        ml.point_sample_masks(z, coords, False)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        ml.point_sample_masks(z, coords, False)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    gather_bytes = 4 * cfg.L * cfg.B * cfg.Q * (cfg.H * cfg.W + P)  # planes read once, samples written

    def both():
        pairwise_sigmoid_cross_entropy_loss_sampling_py(z, t, background_index=0, point_coords=coords)
        pairwise_dice_loss_sampling_py(z, t, smooth=1.0, background_index=0, point_coords=coords)

    ms = time_steps(both, steps, warmup)

    # the Mask2Former-style step of configuration 2 on these points: sampled
    # logits and point labels into the fused cost -> assignment -> loss, with
    # the backward through the sampling to the dense logits
    from mask_loss_amd.functions import MaskMatchingFunction, point_sample
    zd = z.clone().requires_grad_(True)
    lab = ml.point_labels(t, coords).view(cfg.B, 1, P)
    zc = torch.randn(cfg.L, cfg.B, cfg.Q, cfg.C + 1, device=dev, generator=g).requires_grad_(True)
    ct = torch.from_numpy(np.ascontiguousarray(cls_t)).to(dev)
    ones = [torch.ones(cfg.L, device=dev) for _ in range(3)]

    def match_step():
        zd.grad = None
        zc.grad = None
        zs = point_sample(zd.view(cfg.L * cfg.B, cfg.Q, cfg.H, cfg.W),
                          coords.repeat(cfg.L, 1, 1)).view(cfg.L, cfg.B, cfg.Q, 1, P)
        out = MaskMatchingFunction.apply(*synth.call_args(
            cfg, dict(mask_logits=zs, mask_targets=lab, cls_logits=zc, cls_targets=ct)))
        torch.autograd.backward(out[2:], ones)
        match_step.p2g = out[0]

    ms_match = time_steps(match_step, steps, warmup)
    matched = int((match_step.p2g >= 0).sum().item())
    return {"workload": "cfg2_point_sampling_front_end", "L": cfg.L, "B": cfg.B, "Q": cfg.Q,
            "H": cfg.H, "W": cfg.W, "Ht": cfg.H * cfg.scale, "Wt": cfg.W * cfg.scale, "points": P,
            "dtype": "float32", "ms_per_call": round(ms, 4),
            "images_per_s": round(cfg.B / (ms * 1e-3), 1),
            "point_sample": {"avg_us": round(us, 2), "algorithmic_bytes": gather_bytes,
                             "achieved_GBs": round(gather_bytes / (us * 1e-6) / 1e9, 1),
                             "frac_of_hbm_peak": round(gather_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
            "matching_step": {"what": "point_sample (autograd) + MaskMatchingFunction fwd/bwd on the "
                                      "sampled 1 x P map, gradient to the dense logits",
                              "ms_per_step": round(ms_match, 4),
                              "images_per_s": round(cfg.B / (ms_match * 1e-3), 1),
                              "matched": matched},
            "steps": steps, "warmup": warmup}


def mask_loss_amd_module():
    import mask_loss_amd
    return mask_loss_amd.mask_loss


def main():
    a = parse()
    if a.copy_calibration:
        copy_calibration()
        return
    if a.read_ceiling:
        print(json.dumps(read_ceiling()), flush=True)
        return
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1 "
                                   "(the step shards over images across GPUs, which is not "
                                   "built here)"}))
        sys.exit(2)
    import torch

    import mask_loss_amd
    from mask_loss_amd import synth

    if a.config == "cfg2_point_sampling_front_end":  # the front end alone (for profiling)
        print(json.dumps(point_front_end(torch.device("cuda:0"), a.steps, a.warmup)), flush=True)
        return
    cfg = synth.BY_NAME[a.config]
    dev = torch.device("cuda:0")
    x, z, zc, step, state = make_step(cfg, dev)
    # timed region: K steps, no instrumentation
    ms = time_steps(step, a.steps, a.warmup)
    # per-kernel breakdown: another K steps with the library's HIP events
    # recorded around each launch group on the launch stream (the events add
    # gaps between launches, so this pass is not the timed one)
    lib = prof_lib()
    lib.ml_profile_reset()
    lib.ml_profile_enable(1)
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    lib.ml_profile_enable(0)

    kernels = {}
    # finalize_early / assign_early / cost_rest: with images in the widest
    # column-tile class and another, the widest class's finalize and
    # assignment (on the side stream), and the other classes' contraction
    # (finalize and assign then cover the other images)
    for name in ["prep", "pair_cost", "cost_rest", "finalize", "assign", "finalize_early",
                 "assign_early", "prefill", "layer", "bwd_mask", "bwd_cls"]:
        n, t = read_prof(lib, name)
        if n:
            kernels[name] = {"launches": n, "avg_us": round(1e3 * t / n, 2)}
    lib.ml_profile_reset()

    p2g = state["p2g"]
    M = int((p2g >= 0).sum().item())
    e = z.element_size()
    K = cfg.H * cfg.W
    LBQ = cfg.L * cfg.B * cfg.Q
    Ht, Wt = cfg.H * cfg.scale, cfg.W * cfg.scale
    Cp = cfg.C + 1
    bytes_alg = {
        "pair_cost": e * K * LBQ + 2 * cfg.B * K,        # logits once + compact labels
        "bwd_mask": e * K * 2 * M,                       # matched rows: logits read, grads written
        # class logits, plus the gradient buffer zero-filled by the extra
        # workgroups of the same launch
        "assign": 4 * LBQ * Cp + e * K * LBQ,
    }

    step_bytes = step_bytes_of(cfg, e, M)
    dom = max(kernels, key=lambda k: kernels[k]["avg_us"])
    dom_bytes = bytes_alg.get(dom)
    achieved = dom_bytes / (kernels[dom]["avg_us"] * 1e-6) / 1e9 if dom_bytes else None
    roofline = {
        "kernel": dom,
        "bound": "hbm",
        "achieved": round(achieved, 1) if achieved else None,
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
        "traffic": load_traffic(cfg.name, dom),
        "algorithmic_bytes": dom_bytes,
        "avg_launch_us": kernels[dom]["avg_us"],
    }
    # the practical read ceiling of this box (a read-only 16-byte-load stream
    # over the headline logits' size), beside the published peak
    rc_ = read_ceiling(reps=10)
    roofline["practical_read_ceiling_GBs"] = rc_["median_GBs"]
    if achieved:
        roofline["frac_of_practical_read_ceiling"] = round(achieved / rc_["median_GBs"], 4)
    if dom_bytes is None:
        roofline["note"] = ("the dominant launch is bound by the serial float64 assignment chains "
                            "(one wave per image), not by HBM or MFMA")
    step_roof = {
        "algorithmic_bytes": step_bytes,
        "hbm_floor_us": round(step_bytes / HBM_PEAK_GBS / 1e3, 1),
        "frac": round(step_bytes / HBM_PEAK_GBS / 1e3 / (ms * 1e3), 4),
    }

    cpu = None
    if not a.no_cpu_baseline:
        cpu = cpu_baseline(cfg, x, z, zc, p2g.cpu().numpy(), total_cost_matrices(cfg, x, z, zc),
                           a.cpu_sample_images, cpu_threads())

    others = []
    if not a.no_other_configs:
        for oc in synth.CONFIGS:
            if oc.name != cfg.name:
                others.append(other_config(oc, dev, a.other_steps, a.other_warmup,
                                           cpu=not a.no_cpu_baseline))
        others.append(point_front_end(dev, a.other_steps, a.other_warmup))

    out = {
        "metric": "ms per cost+match+loss fwd/bwd step (B=16,Q=200,256²); % MFMA/HBM roofline",
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 4),
        "images_per_s": round(cfg.B * cfg.L / (ms * 1e-3), 1),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == "bfloat16" else "f32",
        "data": "synthetic (label maps from the NumPy recipe, logits from the device RNG)",
        "config": {"workload": cfg.name, "L": cfg.L, "B": cfg.B, "Q": cfg.Q, "H": cfg.H,
                   "W": cfg.W, "G": list(cfg.G), "C": cfg.C + 1, "matched": M,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "step_roofline": step_roof,
        "kernels": kernels,
        "cpu_baseline": cpu,
        "other_configs": others,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
