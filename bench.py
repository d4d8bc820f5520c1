"""Benchmark: YOLOv8n-320 W8A8 images/s on one MI355X (bs=64 headline, bs=1 reported).

One step = one forward pass of the seeded YOLOv8n-320 network (CSP backbone
and PAN neck W8A8, detection head fp16, raw head output [B, 144, 2100]) over
one batch of synthetic U(0,1) images already resident in HBM.  The run is
replayed from a HIP graph; the timed region is bracketed by device
synchronisation and measured with HIP events on the stream the graph runs
on.

The engine runs its measured kernel plan: the per-conv kernel/tile choices
and the schedule measured on an MI355X for this workload, committed as
aexrt_amd/tuned/yolov8n320.tune (AEXRT_HIP_TUNE_CACHE, no measurement at
load: AEXRT_HIP_AUTOTUNE=0); ``--retune`` measures them again instead and
``--save-tune-cache FILE`` writes what was used.

After the timed region a profiling pass times every launch of the same plan
with per-launch HIP events on the same stream.  Launches are grouped by the
kernel template instance that ran (the name a kernel trace reports); the
instance with the most time per step is reported against its roofline
(algorithmic ops or bytes per launch over its mean launch duration), and the
int8 and fp16 conv families against their MFMA peaks and the sum of their
per-layer rooflines.  The CPU baseline times the oracle's W8A8 network (a C
port of the reference semantics) on the host cores over a bounded sample of
bs=1 images.

Prints one JSON line.  Other modes: ``--trace-pass`` (graph replays only, for
``rocprofv3 --kernel-trace --stats``), ``--pmc-pass`` (one profiled forward
after a calibration copy, for ``rocprofv3 --pmc``), ``--configs`` (the
single-conv benchmark configurations, GPU and single-thread CPU, as JSON lines).
"""
from __future__ import annotations

import argparse
import re
import json
import os
import platform
import shutil
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_INT8_OPS = 5.0e15      # dense int8 MFMA, MI355X
PEAK_FP16_FLOPS = 2.5e15    # dense fp16 MFMA
PEAK_FP32_FLOPS = 157.3e12  # fp32 (vector and matrix)
PEAK_HBM = 8.0e12           # bytes/s

TUNE_FILE = os.path.join(ROOT, "aexrt_amd", "tuned", "yolov8n320.tune")
TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "hbm_traffic_yolov8n320_bs64.md")


def use_tune_plan(retune: bool, source: str | None = None) -> str | None:
    """Points AEXRT_HIP_TUNE_CACHE at a scratch copy of the committed plan (or of `source`; the
    runtime rewrites the file it is given after a measuring load).  Returns the scratch path."""
    path = os.path.join(tempfile.mkdtemp(prefix="aexrt_tune_"), "plan.tune")
    source = source or TUNE_FILE
    if os.path.exists(source) and not retune:
        shutil.copyfile(source, path)
        os.environ["AEXRT_HIP_AUTOTUNE"] = "0"
    else:
        os.environ.pop("AEXRT_HIP_AUTOTUNE", None)
    os.environ["AEXRT_HIP_TUNE_CACHE"] = path
    return path


def build_model(batch: int, imgsz: int = 320, seed: int = 4):
    from aexrt_amd import engine as E
    from aexrt_amd.runtime import NativeHipYoloModel
    from aexrt_amd.yolov8 import build_yolov8n

    g = build_yolov8n(batch=batch, imgsz=imgsz, seed=seed)
    replay = E.lower_graph(g)
    algo = E.w8a8_algo_map(replay, g.metadata["int8_convs"].split(","))
    data = E.build_aexrt_engine(g, precision="fp16", algo_overrides=algo, classes=80)
    model = NativeHipYoloModel(data)
    return g, model, replay


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
    """(ops, algorithmic HBM bytes) of one conv: input once, output once (fp16), weights once."""
    b, ic, ih, iw, oc, oh, ow, kh, kw = (int(v) for v in params[:9])
    ops = 2 * b * oh * ow * oc * ic * kh * kw
    in_bytes = b * ic * ih * iw * (2 if ic > 3 else 4)
    out_bytes = b * oc * oh * ow * 2
    w_bytes = oc * ic * kh * kw * (1 if int8 else 2)
    return ops, in_bytes + out_bytes + w_bytes


def parse_label(label: str):
    """(engine command index, kernel instance, int8, sibling command indices, fused 1x1 command
    indices) of a conv step label "cmd#N KIND ... alg=... kernel=<instance> <tile>[ + cmd#M]
    [ then 1x1 cmd#K]"; None for other steps."""
    if not label.startswith("cmd#") or " kernel=" not in label:
        return None
    ci = int(label.split()[0][4:])
    head, rest = label.split(" kernel=", 1)
    rest, *fused = rest.split(" then 1x1 cmd#")
    parts = rest.split(" + cmd#")
    instance = parts[0].split(" ")[0]
    sibs = [int(p.split()[0]) for p in parts[1:]]
    return ci, instance, "alg=int8" in head, sibs, [int(f.split()[0]) for f in fused]


def launch_work(label: str, replay):
    """(ops, algorithmic bytes) of one conv launch: every conv the label names (a sibling pair,
    a fused 1x1, a head branch of three convs or a level's two branches); HBM bytes are each
    distinct input read once, the outputs no conv of the launch reads written once, and every
    weight once (the intermediates a launch keeps on chip are neither)."""
    ci, _, int8, _, _ = parse_label(label)
    cmds = replay["commands"]
    tail = label.split(" kernel=", 1)[1]
    # "+ 2x upsample cmd#R": the launch also writes the nearest 2x upsample of its output (the
    # resize R it replaces), 4x the output's positions
    up = re.search(r" \+ 2x upsample cmd#(\d+)", tail)
    tail = tail[:up.start()] + tail[up.end():] if up else tail
    # "reading 2x upsample cmd#R": the conv reads that upsampled slice of its input from the resize
    # R's source, a quarter of the slice's positions
    rd = re.search(r" reading 2x upsample cmd#(\d+)", tail)
    tail = tail[:rd.start()] + tail[rd.end():] if rd else tail
    idx = [ci] + [int(m) for m in re.findall(r"cmd#(\d+)", tail)]
    ops = nbytes = 0
    if up:
        b, _, _, _, oc, oh, ow = (int(v) for v in cmds[ci]["params"][:7])
        nbytes += b * oc * 4 * oh * ow * 2
    if rd:
        b, c, h, w, oh, ow = (int(v) for v in cmds[int(rd.group(1))]["params"][:6])
        nbytes -= b * c * oh * ow * 2 - b * c * h * w * 2
    produced = {cmds[i]["output"] for i in idx}
    consumed = {cmds[i]["inputs"][0] for i in idx}
    inputs_seen = set()
    for i in idx:
        p = cmds[i]["params"]
        c_int8 = int8 and i == ci or (int8 and cmds[i]["inputs"][0] == cmds[ci]["inputs"][0])
        c_ops, _ = conv_work(p, c_int8)
        b, ic, ih, iw, oc, oh, ow, kh, kw = (int(v) for v in p[:9])
        ops += c_ops
        nbytes += oc * ic * kh * kw * (1 if c_int8 else 2)
        x = cmds[i]["inputs"][0]
        if x not in produced and x not in inputs_seen:
            inputs_seen.add(x)
            nbytes += b * ic * ih * iw * (2 if ic > 3 else 4)
        if cmds[i]["output"] not in consumed:
            nbytes += b * oc * oh * ow * 2
    return ops, nbytes


def profile_steps(model, reps: int = 5):
    """[(label, ms)] of one forward, each step's mean over `reps` event-profiled passes."""
    model.set_profiling(True)
    totals = {}
    order = []
    for _ in range(reps):
        model.run_device()
        for label, ms in model.profile_events():
            if label not in totals:
                order.append(label)
            totals[label] = totals.get(label, 0.0) + ms
    model.set_profiling(False)
    return [(lab, totals[lab] / reps) for lab in order]


def measured_traffic(instance: str, labels: list, batch: int):
    """HBM bytes per launch of a kernel instance (its launches' FETCH_SIZE + WRITE_SIZE from the
    committed counter summary, calibrated against a copy of known size); None without rows."""
    if batch != 64 or not os.path.exists(TRAFFIC_TABLE):
        return None
    rows = {}
    with open(TRAFFIC_TABLE) as f:
        for line in f:
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 5 and cells[0].startswith("cmd#"):
                try:
                    rows[cells[0].split()[0]] = float(cells[3]) + float(cells[4])
                except ValueError:
                    continue
    got = [rows.get(lab.split()[0]) for lab in labels]
    if not got or any(v is None for v in got):
        return None
    return int(round(sum(got) / len(got) * 1e6))


def roofline_record(ops: float, nbytes: float, secs: float, peak_ops: float, unit_ops: str):
    if ops / peak_ops >= nbytes / PEAK_HBM:
        achieved = ops / secs / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 3), "peak": peak_ops / 1e12, "unit": unit_ops,
                "frac": round(achieved / (peak_ops / 1e12), 4)}
    achieved = nbytes / secs / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "frac": round(achieved / (PEAK_HBM / 1e9), 4)}


def analyse(steps, replay, batch: int):
    """Dominant kernel instance (most time per step) with its roofline record, and the int8 and
    fp16 conv family records."""
    by_inst = {}
    fam = {True: dict(ops=0, bytes=0, secs=0.0, roof=0.0, n=0), False: dict(ops=0, bytes=0, secs=0.0, roof=0.0, n=0)}
    for label, ms in steps:
        p = parse_label(label)
        if p is None:
            continue
        _, inst, int8, _, _ = p
        ops, nbytes = launch_work(label, replay)
        e = by_inst.setdefault(inst, dict(ms=0.0, ops=0, bytes=0, labels=[], int8=int8))
        e["ms"] += ms
        e["ops"] += ops
        e["bytes"] += nbytes
        e["labels"].append(label)
        f = fam[int8]
        f["ops"] += ops
        f["bytes"] += nbytes
        f["secs"] += ms / 1e3
        f["n"] += 1
        f["roof"] += max(ops / (PEAK_INT8_OPS if int8 else PEAK_FP16_FLOPS), nbytes / PEAK_HBM)
    inst, e = max(by_inst.items(), key=lambda kv: kv[1]["ms"])
    n = len(e["labels"])
    rec = roofline_record(e["ops"], e["bytes"], e["ms"] / 1e3, PEAK_INT8_OPS if e["int8"] else PEAK_FP16_FLOPS,
                          "TOPS" if e["int8"] else "TFLOP/s")
    rec["traffic"] = measured_traffic(inst, e["labels"], batch)
    t_ms = trace_launch_ms(inst) if batch == 64 else None
    if t_ms:
        # the same algorithmic work over the kernel-trace mean duration (no event boundaries)
        per = (e["ops"] if rec["bound"] == "mfma" else e["bytes"]) / n
        ach = per / (t_ms / 1e3) / (1e12 if rec["bound"] == "mfma" else 1e9)
        rec["trace_avg_launch_ms"] = round(t_ms, 5)
        rec["achieved_trace"] = round(ach, 1)
        rec["frac_trace"] = round(ach / rec["peak"], 4)
    rec.update(kernel=inst, launches_per_step=n, ms_per_step=round(e["ms"], 5), avg_launch_ms=round(e["ms"] / n, 5),
               ops_per_launch=e["ops"] // n, algorithmic_bytes_per_launch=e["bytes"] // n,
               layers=[lab.split(" alg=")[0] for lab in e["labels"]])
    families = {}
    for int8, f in fam.items():
        if not f["n"]:
            continue
        peak = PEAK_INT8_OPS if int8 else PEAK_FP16_FLOPS
        tops = f["ops"] / f["secs"] / 1e12
        families["int8_convs" if int8 else "fp16_convs"] = {
            "launches": f["n"], "ops_per_step": f["ops"], "ms_per_step": round(f["secs"] * 1e3, 4),
            "achieved": round(tops, 2), "unit": "TOPS" if int8 else "TFLOP/s", "peak": peak / 1e12,
            "frac_of_peak": round(tops / (peak / 1e12), 4),
            "roofline_ms_per_step": round(f["roof"] * 1e3, 4),
            "frac_of_layer_rooflines": round(f["roof"] / f["secs"], 4)}
    ranking = sorted(((k, round(v["ms"], 4), len(v["labels"])) for k, v in by_inst.items()), key=lambda t: -t[1])
    return rec, families, ranking


def bandwidth_launches(steps, replay):
    """The HBM-bound launches that are not convs: the amax-slot clear (one fill of the slot words),
    the 2x nearest upsamples and the fused SPPF pools, each against 8 TB/s with its algorithmic
    bytes (fp16 tensors read once and written once; the fill writes its words)."""
    cmds = replay["commands"]
    groups = {}
    for label, ms in steps:
        kind = nbytes = None
        m = re.match(r"amax slots clear (\d+) words", label) or re.match(r"superblock sync clear (\d+) words", label)
        if m:
            kind, nbytes = ("slot clear" if label.startswith("amax") else "superblock sync clear"), int(m.group(1)) * 4
        elif label.startswith("cmd#") and " RESIZE" in label:
            n, c, h, w, oh, ow = (int(v) for v in cmds[int(label.split()[0][4:])]["params"][:6])
            kind, nbytes = "resize 2x nearest", n * c * (h * w + oh * ow) * 2
        elif label.startswith("cmd#") and " SPPF" in label:
            n, c, h, w = (int(v) for v in cmds[int(label.split()[0][4:])]["params"][:4])
            kind, nbytes = "SPPF three 5x5 pools", 4 * n * c * h * w * 2  # one read, three pooled maps written
        if kind is None:
            continue
        g = groups.setdefault(kind, dict(ms=0.0, bytes=0, n=0, layers=[]))
        g["ms"] += ms
        g["bytes"] += nbytes
        g["n"] += 1
        g["layers"].append(label.split(" alg=")[0])
    out = []
    for kind, g in groups.items():
        gbs = g["bytes"] / (g["ms"] / 1e3) / 1e9
        out.append({"launch": kind, "launches_per_step": g["n"], "algorithmic_bytes_per_launch": g["bytes"] // g["n"],
                    "avg_launch_ms": round(g["ms"] / g["n"], 5), "achieved": round(gbs, 1), "unit": "GB/s",
                    "peak": PEAK_HBM / 1e9, "frac": round(gbs / (PEAK_HBM / 1e9), 4), "layers": g["layers"]})
    return out


TRACE_TABLE = os.path.join(ROOT, "profiles", "kernel_stats_yolov8n320_bs64.md")


def trace_launch_ms(instance: str):
    """Mean duration per launch (ms) of a kernel instance in the committed kernel-trace summary (the
    rocprofv3 trace of this plan's graph replays), or None."""
    if not os.path.exists(TRACE_TABLE):
        return None
    want = instance.replace(" ", "")
    with open(TRACE_TABLE) as f:
        for line in f:
            cells = [c.strip().strip("`") for c in line.strip().strip("|").split("|")]
            if len(cells) == 4 and cells[0] and cells[0][0].isalpha():
                name = cells[0].split("::")[-1].replace(" ", "")
                # the trace names a template's defaulted trailing arguments too
                if name == want or name.startswith(want[:-1] + ","):
                    try:
                        return float(cells[3]) / 1e3
                    except ValueError:
                        return None
    return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_threads() -> int:
    """The host cores this GPU's job may use: the job's thread allowance (OMP_NUM_THREADS, set to
    the box's per-GPU CPU share) or, without one, every core."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return min(n, int(env))
    return n


def cpu_baseline(graph_bs1, images_budget_s: float = 12.0):
    """Oracle W8A8 network on the host cores, bounded sample of bs=1 images."""
    import oracle.network as ON

    threads = cpu_threads()
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
            "nproc": os.cpu_count(), "cpu_model": cpu_model(),
            "sample": f"{n} YOLOv8n-320 W8A8 images at bs=1 (oracle C port, OpenMP over (n, oc) on {threads} "
                      f"threads of {os.cpu_count()} cores, {dt:.1f} s)"}


CAL_ELEMS = 64 << 20  # fp32 elements of the counter-calibration copy (256 MiB read, 256 MiB written)


def pmc_pass(batch: int) -> int:
    """One pass for rocprofv3 --pmc: a negation of CAL_ELEMS fp32 values (known
    HBM traffic, the counters' scale), then one event-profiled forward of the
    network, every step launched on its own; prints the step labels in launch
    order so that aexrt_amd/profiling.py can match dispatches to steps."""
    import torch

    torch.cuda.init()
    g, model, _ = build_model(batch)
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


def trace_pass(batch: int, replays: int) -> int:
    """Graph replays of the plan only (one stream, steps in launch order), for a kernel trace:
    the trace holds `replays` dispatches of every step and nothing else of the network."""
    import torch

    os.environ.setdefault("AEXRT_HIP_LANES", "1")
    torch.cuda.init()
    g, model, _ = build_model(batch)
    fill_input(model, batch, 320)
    model.set_profiling(True)
    model.run_device()
    labels = [lab for lab, _ in model.profile_events()]
    model.set_profiling(False)
    torch.cuda.synchronize()
    for _ in range(replays):
        model.run_device()
    torch.cuda.synchronize()
    print(json.dumps({"trace_pass": {"batch": batch, "replays": replays, "profiled_passes": 2, "steps": labels}}))
    model.close()
    return 0


def _gpu_ms(fn, reps: int = 50, warmup: int = 5) -> float:
    """Mean ms of fn() over `reps` back-to-back calls on the current stream (HIP events)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def _cpu_ms(fn, reps: int = 3) -> float:
    """Median ms of fn() over `reps` runs after one warm-up."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    return float(np.median(ts))


def configs_bench() -> int:
    """The single-conv benchmark configurations and the C2f block: GPU time (HIP events over back-to-back
    launches of the op-level entry points, or graph replays of the engine) against each one's roofline,
    and the oracle on one host thread (the reference's CPU path is single threaded).  One JSON line each."""
    import torch

    import oracle as O
    import oracle.network as ON
    from aexrt_amd import kernels as K
    from aexrt_amd import packing
    from aexrt_amd import engine as E
    from aexrt_amd import workloads as WL
    from aexrt_amd.runtime import NativeHipYoloModel

    dev = torch.device("cuda:0")
    torch.cuda.init()
    out = []

    def emit(name, gpu_ms, ops, nbytes, peak, cpu_ms, cpu_note, extra=None):
        secs = gpu_ms / 1e3
        roof = max(ops / peak, nbytes / PEAK_HBM)
        rec = {"config": name, "gpu_ms": round(gpu_ms, 5), "gpu_tops": round(ops / secs / 1e12, 2),
               "frac_of_peak": round(ops / secs / peak, 4), "roofline_ms": round(roof * 1e3, 5),
               "frac_of_roofline": round(roof / secs, 4), "algorithmic_ops": ops, "algorithmic_bytes": nbytes,
               "cpu_ms_1thread": round(cpu_ms, 2), "cpu_note": cpu_note, "cpu_gpu_ratio": round(cpu_ms / gpu_ms, 1)}
        rec.update(extra or {})
        out.append(rec)
        print(json.dumps(rec), flush=True)

    def nhwc(a):
        return torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 3, 1)).astype(np.float16)).to(dev)

    # C1: fp32 3x3 64->64 @80x80, SiLU (the reference's fp32 path), seed 0
    x, w, b = WL.c1_case()
    desc = O.conv_desc(1, 64, 80, 80, 64, 3, 1, 1)
    xd, wd, bd = (torch.from_numpy(a).to(dev) for a in (x, w, b))
    yd = torch.empty((1, 64, 80, 80), dtype=torch.float32, device=dev)
    import ctypes
    from aexrt_amd import _lib
    dsc = _lib.ConvDesc.from_params(desc)
    L = _lib.lib()
    g1 = _gpu_ms(lambda: L.aexrt_hip_conv2d_f32(ctypes.byref(dsc), K.SILU, xd.data_ptr(), wd.data_ptr(),
                                                bd.data_ptr(), yd.data_ptr(), None), reps=100)
    c1 = _cpu_ms(lambda: O.cpu_conv2d(x, w, b, desc, silu=True, threads=1))
    ops, nb = conv_work(desc, False)
    emit("C1 fp32 3x3 64->64 @80x80 bs1", g1, ops, 64 * 80 * 80 * 4 * 2 + w.nbytes, PEAK_FP32_FLOPS, c1,
         "or_cpu_conv2d (the reference's cpu_conv2d loop), 1 thread", {"dtype": "fp32"})

    def int8_conv(n, c, h, wd_, oc, k, s, x_, wt, bb):
        d = O.conv_desc(n, c, h, wd_, oc, k, s, k // 2)
        alg = 51 if k == 1 else (53 if s == 2 else 52)
        pc = K.prepare_conv(d, alg, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True), bb, device=dev)
        xin = nhwc(x_)
        _, _, oh, ow = O.out_shape(d)
        y = torch.empty((n, oh, ow, oc), dtype=torch.float16, device=dev)
        return _gpu_ms(lambda: K.conv2d_int8(pc, xin, y)), d

    def fp16_conv(n, c, h, wd_, oc, k, s, x_, wt, bb):
        d = O.conv_desc(n, c, h, wd_, oc, k, s, k // 2)
        pc = K.prepare_conv(d, 5, K.SRC_RAW_F32, packing.fp16_round(wt), bb, device=dev)
        xin = nhwc(x_)
        _, _, oh, ow = O.out_shape(d)
        y = torch.empty((n, oh, ow, oc), dtype=torch.float16, device=dev)
        return _gpu_ms(lambda: K.conv2d(pc, xin, y, flags=K.SILU))

    # C2: W8A8 1x1 128->256 @40x40 with 1% outliers x8, per-16-output-channel weight scales, seed 1
    x2, w2, b2 = WL.c2_case()
    ms2, d2 = int8_conv(1, 128, 40, 40, 256, 1, 1, x2, w2, b2)
    c2 = _cpu_ms(lambda: O.w8a8_conv(x2, w2, b2, d2, silu=True, fp16_engine=True), reps=5)
    ops, nb = conv_work(d2, True)
    emit("C2 W8A8 1x1 128->256 @40x40 bs1", ms2, ops, nb, PEAK_INT8_OPS, c2,
         "oracle W8A8 chain (amax, quantize, int32 conv, dequant, SiLU), 1 thread",
         {"dtype": "int8", "gpu_includes": "amax pass + conv (the reference's whole int8 command)"})

    # C3: 3x3 s2 64x160x160 -> 128x80x80, W8A8 and fp16, batch 1 and 32, seed 2
    x3, w3, b3 = WL.c3_case(32)
    d31 = O.conv_desc(1, 64, 160, 160, 128, 3, 2, 1)
    c3_int8 = _cpu_ms(lambda: O.w8a8_conv(x3[:1], w3, b3, d31, silu=True, fp16_engine=True), reps=3)
    c3_fp16 = _cpu_ms(lambda: O.cpu_conv2d(x3[:1], packing.fp16_round(w3), b3, d31, silu=True, threads=1), reps=3)
    for n in (1, 32):
        ms_i8, d3 = int8_conv(n, 64, 160, 160, 128, 3, 2, x3[:n], w3, b3)
        ops, nb = conv_work(d3, True)
        emit(f"C3 W8A8 3x3 s2 64->128 @160->80 bs{n}", ms_i8, ops, nb, PEAK_INT8_OPS, c3_int8 * n,
             "oracle W8A8 chain, 1 thread" + ("" if n == 1 else f" (batch 1 time x {n})"),
             {"dtype": "int8", "gpu_includes": "amax pass + conv"})
        # the command's amax pass on its own: one read of the fp16 input, a few slot words written
        xin = nhwc(x3[:n])
        slots = K.new_slots(64, dev, stripes=16)
        ms_amax = _gpu_ms(lambda: K.amax_slots(xin, slots))
        amax_bytes = n * 64 * 160 * 160 * 2
        gbs = amax_bytes / (ms_amax / 1e3) / 1e9
        rec = {"config": f"C3 W8A8 amax pass (a1) 64x160x160 bs{n}", "gpu_ms": round(ms_amax, 5),
               "algorithmic_bytes": amax_bytes, "achieved": round(gbs, 1), "unit": "GB/s",
               "peak": PEAK_HBM / 1e9, "frac": round(gbs / (PEAK_HBM / 1e9), 4),
               "kernel": "amax_slots_nhwc_kernel", "dtype": "fp16 in"}
        out.append(rec)
        print(json.dumps(rec), flush=True)
        ms_f = fp16_conv(n, 64, 160, 160, 128, 3, 2, x3[:n], w3, b3)
        ops, nb = conv_work(d3, False)
        emit(f"C3 fp16 3x3 s2 64->128 @160->80 bs{n}", ms_f, ops, nb, PEAK_FP16_FLOPS, c3_fp16 * n,
             "or_cpu_conv2d on fp16-rounded operands, 1 thread" + ("" if n == 1 else f" (batch 1 time x {n})"),
             {"dtype": "fp16"})

    # C4: C2f fp16 @40x40 (cv1 1x1 128->128, split, two bottlenecks of two 3x3 64->64 with residual,
    # concat 4x64 -> 1x1 256->128, SiLU), seed 3; the plan's 3x3 convs on the direct kernel and on
    # Winograd F(2x2,3x3)
    g4 = WL.c2f_block(batch=1, c=128, dim=40, seed=3)
    x4 = np.random.default_rng(3).standard_normal((1, 128, 40, 40)).astype(np.float32)
    data4 = E.build_aexrt_engine(g4, precision="fp16")
    c4 = _cpu_ms(lambda: ON.run_graph(g4, x4, threads=1), reps=3)
    ops4 = sum(conv_work(c["params"], False)[0] for c in E.lower_graph(g4)["commands"] if c["kind"].startswith("CONV"))
    bytes4 = 128 * 40 * 40 * 2 * 2
    for wino in (False, True, "superblock"):
        if wino == "superblock":
            os.environ["AEXRT_HIP_C2F_SUPERBLOCK"] = "1"
        with NativeHipYoloModel(data4) as m:
            os.environ.pop("AEXRT_HIP_C2F_SUPERBLOCK", None)
            if wino is True:
                for info in m.conv_plan():
                    if info["desc"][7] == 3 and 40 in info["candidates"]:
                        m.override_conv_algorithm(info["command_index"], 40)
            m.run(x4)
            ms4 = _gpu_ms(lambda: m.run_device(), reps=100)
        form = {False: "direct 3x3", True: "Winograd F(2x2,3x3) 3x3", "superblock": "bottleneck superblocks"}[wino]
        emit(f"C4 C2f fp16 @40x40 bs1 ({form})", ms4, ops4, bytes4,
             PEAK_FP16_FLOPS, c4, "oracle network (fp16-stored values), 1 thread",
             {"dtype": "fp16", "gpu_includes": "the whole block (6 convs) as one engine, graph replay"})
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--retune", action="store_true", help="measure the kernel plan at load instead of the committed one")
    ap.add_argument("--save-tune-cache", help="write the kernel plan the run used to this file")
    ap.add_argument("--tune-plan", help="run this kernel plan file instead of the committed one")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="one calibration copy and one profiled forward at --batch, for rocprofv3 --pmc")
    ap.add_argument("--trace-pass", action="store_true", help="--steps graph replays at --batch, for a kernel trace")
    ap.add_argument("--configs", action="store_true", help="the single-conv benchmark configurations")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU; multi-GPU runs are not part of this "
                                   "build (per-tensor amax would need a batch-wide max-reduce across GPUs)"}))
        return 2
    plan = use_tune_plan(args.retune, args.tune_plan)
    if args.pmc_pass:
        return pmc_pass(args.batch)
    if args.trace_pass:
        return trace_pass(args.batch, args.steps)
    if args.configs:
        return configs_bench()

    import torch

    torch.cuda.init()
    # a created (non-default, default-priority) stream: graph capture is not
    # allowed on the legacy null stream
    stream = torch.cuda.Stream()
    results = {}
    for bs in (args.batch, 1):
        g, model, replay = build_model(bs)
        fill_input(model, bs, 320)
        ms = time_steps(model, args.steps if bs == args.batch else max(args.steps, 100), args.warmup, stream)
        steps = profile_steps(model)
        results[bs] = dict(ms=ms, ips=bs / (ms / 1e3), steps=steps, graph=g, model=model, replay=replay)
    big = results[args.batch]
    roof, families, ranking = analyse(big["steps"], big["replay"], args.batch)
    bw = bandwidth_launches(big["steps"], big["replay"])
    i8 = families.get("int8_convs", {})
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
                   "imgsz": 320, "int8_convs": 44, "fp16_convs": 19, "parallelism": "single GPU",
                   "kernel_plan": "committed measured plan" if os.environ.get("AEXRT_HIP_AUTOTUNE") == "0"
                   else "measured at load"},
        "bs1_images_per_s": round(results[1]["ips"], 2),
        "bs1_ms": round(results[1]["ms"], 4),
        "int8_conv_tops": i8.get("achieved"),
        "int8_conv_frac_of_peak": i8.get("frac_of_peak"),
        "roofline": roof,
        "families": families,
        "kernel_ranking_ms_per_step": ranking[:8],
        "bandwidth_bound_launches": bw,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(results[1]["graph"])
    for r in results.values():
        r["model"].close()
    if args.save_tune_cache and plan and os.path.exists(plan):
        shutil.copyfile(plan, args.save_tune_cache)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
