"""Benchmark: YOLOv8n-320 W8A8 images/s on one MI355X (bs=64 headline, bs=1 reported).

One step = one forward pass of the seeded YOLOv8n-320 network (CSP backbone
and PAN neck W8A8, detection head fp16, raw head output [B, 144, 2100]) over
one batch of synthetic U(0,1) images already resident in HBM.  The run is
replayed from a HIP graph; the timed region is bracketed by device
synchronisation and measured with HIP events on the stream the graph runs
on.

After the timed region a profiling pass times every launch of the same plan
with per-launch HIP events on the same stream; the kernel with the largest
total time is reported against its roofline (algorithmic ops or bytes per
launch over its average duration).  The CPU baseline times the oracle's
W8A8 network (a C port of the reference semantics) on the host cores over a
bounded sample of bs=1 images.

Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_INT8_OPS = 5.0e15      # dense int8 MFMA, MI355X
PEAK_FP16_FLOPS = 2.5e15    # dense fp16 MFMA
PEAK_HBM = 8.0e12           # bytes/s


def build_model(batch: int, imgsz: int = 320, seed: int = 4):
    from aexrt_amd import engine as E
    from aexrt_amd.runtime import NativeHipYoloModel
    from aexrt_amd.yolov8 import build_yolov8n

    g = build_yolov8n(batch=batch, imgsz=imgsz, seed=seed)
    replay = E.lower_graph(g)
    algo = E.w8a8_algo_map(replay, g.metadata["int8_convs"].split(","))
    data = E.build_aexrt_engine(g, precision="fp16", algo_overrides=algo, classes=80)
    model = NativeHipYoloModel(data)
    return g, model


def fill_input(model, batch: int, imgsz: int, seed: int = 4) -> None:
    import ctypes

    from aexrt_amd import _lib

    x = np.random.default_rng(seed).random((batch, 3, imgsz, imgsz), dtype=np.float32)
    # hipMemcpy of the HIP runtime the library is linked against (found
    # through the library's handle), kind 1 = host to device
    memcpy = _lib.lib().hipMemcpy
    memcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    memcpy.restype = ctypes.c_int
    rc = memcpy(ctypes.c_void_p(model.input_device_ptr), x.ctypes.data_as(ctypes.c_void_p), x.nbytes, 1)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy failed: {rc}")


def time_steps(model, steps: int, warmup: int, stream) -> float:
    import torch

    for _ in range(warmup):
        model.run_device(stream=stream)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        model.run_device(stream=stream)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def conv_work(params, int8: bool):
    """(ops, algorithmic HBM bytes) of one conv launch: in once, out once (fp16), weights once."""
    b, ic, ih, iw, oc, oh, ow, kh, kw = (int(v) for v in params[:9])
    ops = 2 * b * oh * ow * oc * ic * kh * kw
    in_bytes = b * ic * ih * iw * (2 if ic > 3 else 4)
    out_bytes = b * oc * oh * ow * 2
    w_bytes = oc * ic * kh * kw * (1 if int8 else 2)
    return ops, in_bytes + out_bytes + w_bytes


def profile_kernels(model, plan, reps: int = 5):
    """Per-launch average ms from HIP events (profiling pass on the model stream)."""
    model.set_profiling(True)
    totals = {}
    for _ in range(reps):
        model.run_device()
        for label, ms in model.profile_events():
            totals[label] = totals.get(label, 0.0) + ms
    model.set_profiling(False)
    return {k: v / reps for k, v in totals.items()}


TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "hbm_traffic_yolov8n320_bs64.md")


def measured_traffic(label: str, batch: int):
    """HBM bytes per launch of a step, from the committed rocprofv3 counter summary of this
    workload (FETCH_SIZE + WRITE_SIZE, calibrated against a copy of known size); None when the
    summary has no row for this step."""
    if batch != 64 or not os.path.exists(TRAFFIC_TABLE):
        return None
    with open(TRAFFIC_TABLE) as f:
        for line in f:
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 5 and cells[0] == label:
                return int(round((float(cells[3]) + float(cells[4])) * 1e6))
    return None


def roofline_for(prof: dict, replay, plans):
    """Dominant conv kernel and its roofline record."""
    best = None
    for label, ms in prof.items():
        if not label.startswith("cmd#") or "alg=" not in label:
            continue
        ci = int(label.split()[0][4:])
        if best is None or ms > best[1]:
            best = (ci, ms, label)
    if best is None:
        return None, None
    ci, ms, label = best
    cmd = replay["commands"][ci]
    int8 = "int8" in label
    ops, nbytes = conv_work(cmd["params"], int8)
    # "+ cmd#N": a sibling conv of the same input computed by the same launch
    # (its output channels appended); the input is read once for both
    for sib in label.split(" + cmd#")[1:]:
        p = replay["commands"][int(sib.split()[0])]["params"]
        s_ops, s_bytes = conv_work(p, int8)
        b, ic, ih, iw = (int(v) for v in p[:4])
        ops += s_ops
        nbytes += s_bytes - b * ic * ih * iw * (2 if ic > 3 else 4)
    secs = ms / 1e3
    peak_ops = PEAK_INT8_OPS if int8 else PEAK_FP16_FLOPS
    if ops / peak_ops >= nbytes / PEAK_HBM:
        achieved = ops / secs / 1e12
        rec = {"bound": "mfma", "achieved": round(achieved, 3), "peak": peak_ops / 1e12, "unit": "TFLOP/s",
               "frac": round(achieved / (peak_ops / 1e12), 4)}
    else:
        achieved = nbytes / secs / 1e9
        rec = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
               "frac": round(achieved / (PEAK_HBM / 1e9), 4)}
    rec["traffic"] = None
    rec["kernel"] = label
    rec["avg_ms"] = round(ms, 5)
    rec["ops_per_launch"] = ops
    rec["algorithmic_bytes_per_launch"] = nbytes
    return rec, ci


def int8_tops(prof: dict, replay) -> float:
    ops = 0
    secs = 0.0
    for label, ms in prof.items():
        if "alg=int8" not in label:
            continue
        ci = int(label.split()[0][4:])
        ops += conv_work(replay["commands"][ci]["params"], True)[0]
        secs += ms / 1e3
    return ops / secs / 1e12 if secs else 0.0


def cpu_baseline(graph_bs1, images_budget_s: float = 12.0):
    """Oracle W8A8 network on the host cores, bounded sample of bs=1 images."""
    import oracle.network as ON

    threads = max(1, min(16, os.cpu_count() or 1))
    names = graph_bs1.metadata["int8_convs"].split(",")
    rng = np.random.default_rng(4)
    x = rng.random((1, 3, 320, 320), dtype=np.float32)
    t0 = time.perf_counter()
    ON.run_graph(graph_bs1, x, int8_convs=names, threads=threads)
    one = time.perf_counter() - t0
    n = max(1, min(64, int(images_budget_s / max(one, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(n):
        ON.run_graph(graph_bs1, x, int8_convs=names, threads=threads)
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 3), "unit": "images/s", "cores": threads, "kind": "port",
            "sample": f"{n} YOLOv8n-320 W8A8 images at bs=1 (oracle C port, OpenMP over (n, oc), "
                      f"{dt:.1f} s)"}


CAL_ELEMS = 64 << 20  # fp32 elements of the counter-calibration copy (256 MiB read, 256 MiB written)


def pmc_pass(batch: int) -> int:
    """One pass for rocprofv3 --pmc: a negation of CAL_ELEMS fp32 values (known
    HBM traffic, the counters' scale), then one event-profiled forward of the
    network, every step launched on its own; prints the step labels in launch
    order so that aexrt_amd/profiling.py can match dispatches to steps."""
    import torch

    torch.cuda.init()
    g, model = build_model(batch)
    fill_input(model, batch, 320)
    model.run_device()
    torch.cuda.synchronize()
    a = torch.ones(CAL_ELEMS, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    torch.neg(a, out=b)
    torch.cuda.synchronize()
    del a, b
    model.set_profiling(True)
    model.run_device()
    labels = [lab for lab, _ in model.profile_events()]
    model.set_profiling(False)
    print(json.dumps({"pmc_pass": {"batch": batch, "calibration_bytes": CAL_ELEMS * 4, "steps": labels}}))
    model.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="one calibration copy and one profiled forward at --batch, for rocprofv3 --pmc")
    args = ap.parse_args()
    if args.pmc_pass:
        return pmc_pass(args.batch)
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU; multi-GPU runs are not part of this "
                                   "build (per-tensor amax would need a batch-wide max-reduce across GPUs)"}))
        return 2

    import torch

    from aexrt_amd import engine as E

    torch.cuda.init()
    # a created (non-default, default-priority) stream: graph capture is not
    # allowed on the legacy null stream
    stream = torch.cuda.Stream()
    results = {}
    plan_replay = {}
    for bs in (args.batch, 1):
        g, model = build_model(bs)
        fill_input(model, bs, 320)
        ms = time_steps(model, args.steps if bs == args.batch else max(args.steps, 100),
                        args.warmup, stream)
        replay = E.lower_graph(g)
        prof = profile_kernels(model, replay)
        results[bs] = dict(ms=ms, ips=bs / (ms / 1e3), prof=prof, graph=g, model=model, replay=replay)
        plan_replay[bs] = replay
    big = results[args.batch]
    roof, _ = roofline_for(big["prof"], big["replay"], None)
    if roof:
        roof["traffic"] = measured_traffic(roof["kernel"], args.batch)
    tops = int8_tops(big["prof"], big["replay"])
    line = {
        "metric": "YOLOv8n-320 W8A8 images/s (bs1, bs64); int8 conv TOPS vs MFMA peak",
        "value": round(big["ips"], 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(big["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "dtype_detail": "int8 MFMA with int32 accumulation on the 44 W8A8 convs; fp16 stem and head",
        "data": "synthetic U(0,1) images, seeded random He-init weights",
        "config": {"workload": f"YOLOv8n-320 W8A8 forward, batch {args.batch}", "global_batch": args.batch,
                   "imgsz": 320, "int8_convs": 44, "fp16_convs": 19, "parallelism": "single GPU"},
        "bs1_images_per_s": round(results[1]["ips"], 2),
        "bs1_ms": round(results[1]["ms"], 4),
        "int8_conv_tops": round(tops, 2),
        "int8_conv_frac_of_peak": round(tops / (PEAK_INT8_OPS / 1e12), 4),
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(results[1]["graph"])
    print(json.dumps(line))
    for r in results.values():
        r["model"].close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
