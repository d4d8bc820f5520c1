"""Per-step HBM traffic and dispatch durations from rocprofv3 output.

Inputs are the output directories of

* ``rocprofv3 --pmc FETCH_SIZE --output-format csv -d <fetch> -o run -- python3 bench.py --pmc-pass``
* ``rocprofv3 --pmc WRITE_SIZE --output-format csv -d <write> -o run -- python3 bench.py --pmc-pass``
* optionally ``rocprofv3 --kernel-trace --stats --output-format csv -d <trace> -o run -- python3 bench.py ...``

and the JSON line ``bench.py --pmc-pass`` printed.  In a pmc pass the
dispatch of the calibration kernel (a negation of a known number of fp32
values: bytes read = bytes written = ``calibration_bytes``) comes right before
the profiled forward, whose dispatches follow in step order, one per step.
The counters (KiB per dispatch) are scaled by what they read for the
calibration kernel, so that the reported MB are HBM bytes.

``python -m aexrt_amd.profiling --fetch DIR --write DIR --pass-log FILE [--trace DIR]``
prints a markdown table: step label, kernel, MB read, MB written, and, with a
kernel trace, the mean dispatch duration of that kernel instance and grid.
``--stats --trace DIR --pass-log FILE`` summarises a kernel trace of
``bench.py --trace-pass`` per kernel instance and per step; ``--mfma DIR
--pass-log FILE [--trace DIR --trace-log FILE]`` prints the executed MFMA
operations of a pmc pass per step and, with the trace, the MFMA rate.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import re
import statistics
from pathlib import Path
from typing import Dict, List, Optional


def _csv_in(d: str, suffix: str) -> str:
    hits = glob.glob(str(Path(d) / "**" / f"*{suffix}"), recursive=True)
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return sorted(hits)[0]


def load_dispatches(d: str) -> List[dict]:
    """Counter collection of one --pmc run: one record per dispatch, in dispatch order."""
    rows: Dict[int, dict] = {}
    with open(_csv_in(d, "counter_collection.csv"), newline="") as f:
        for r in csv.DictReader(f):
            k = int(r["Dispatch_Id"])
            e = rows.setdefault(k, {"id": k, "name": r["Kernel_Name"], "grid": int(r["Grid_Size"]), "counters": {}})
            c = r["Counter_Name"]
            e["counters"][c] = e["counters"].get(c, 0.0) + float(r["Counter_Value"])
    return [rows[k] for k in sorted(rows)]


def pass_info(log: str) -> dict:
    for line in Path(log).read_text().splitlines():
        line = line.strip()
        if line.startswith("{") and "pmc_pass" in line:
            return json.loads(line)["pmc_pass"]
    raise ValueError(f"no pmc_pass line in {log}")


def _steps_after_calibration(disp: List[dict], nsteps: int) -> tuple:
    cal = [i for i, d in enumerate(disp) if "neg" in d["name"]]
    if not cal:
        raise ValueError("calibration dispatch not found")
    i = cal[-1]
    steps = disp[i + 1:i + 1 + nsteps]
    if len(steps) != nsteps:
        raise ValueError("fewer dispatches after the calibration than profiled steps")
    return disp[i], steps


def short_name(kernel: str) -> str:
    k = re.sub(r"^void ", "", kernel).replace("(anonymous namespace)::", "")
    k = re.sub(r"\(.*$", "", k)
    return k.replace("aexrt::", "").replace("igemm::", "")


def traffic_table(fetch_dir: str, write_dir: str, pass_log: str, trace_dir: Optional[str] = None) -> List[dict]:
    info = pass_info(pass_log)
    labels = info["steps"]
    cal_bytes = float(info["calibration_bytes"])
    fd, wd = load_dispatches(fetch_dir), load_dispatches(write_dir)
    fcal, fsteps = _steps_after_calibration(fd, len(labels))
    wcal, wsteps = _steps_after_calibration(wd, len(labels))
    f_scale = cal_bytes / (fcal["counters"]["FETCH_SIZE"] * 1024.0)
    w_scale = cal_bytes / (wcal["counters"]["WRITE_SIZE"] * 1024.0)
    durations: Dict[tuple, List[float]] = {}
    if trace_dir:
        with open(_csv_in(trace_dir, "kernel_trace.csv"), newline="") as f:
            for r in csv.DictReader(f):
                grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
                key = (r["Kernel_Name"], grid)
                durations.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    rows = []
    for lab, fs, ws in zip(labels, fsteps, wsteps):
        if fs["name"] != ws["name"]:
            raise ValueError(f"dispatch order differs between the runs at {lab}")
        d = durations.get((fs["name"], fs["grid"]), [])
        rows.append(dict(step=lab, kernel=short_name(fs["name"]), grid=fs["grid"],
                         read_mb=fs["counters"]["FETCH_SIZE"] * 1024.0 * f_scale / 1e6,
                         write_mb=ws["counters"]["WRITE_SIZE"] * 1024.0 * w_scale / 1e6,
                         trace_us_mean=statistics.mean(d) if d else None, trace_n=len(d)))
    return [dict(f_scale=f_scale, w_scale=w_scale)] + rows


def trace_pass_info(log: str) -> dict:
    for line in Path(log).read_text().splitlines():
        line = line.strip()
        if line.startswith("{") and "trace_pass" in line:
            return json.loads(line)["trace_pass"]
    raise ValueError(f"no trace_pass line in {log}")


def kernel_stats(trace_dir: str, pass_log: str) -> dict:
    """Per-step kernel durations of a ``bench.py --trace-pass`` kernel trace.

    The trace ends with the pass's graph replays (one stream, steps in launch
    order): the last replays x steps dispatches are matched to the step
    labels in order.  Returns per-step mean duration, per-instance totals per
    replay, and the replays' wall time (first dispatch start to last end)."""
    info = trace_pass_info(pass_log)
    labels, reps = info["steps"], int(info["replays"])
    rows = []
    with open(_csv_in(trace_dir, "kernel_trace.csv"), newline="") as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    n = len(labels)
    tail = rows[-reps * n:]
    if len(tail) != reps * n:
        raise ValueError("fewer dispatches than replays x steps")
    per_step = []
    for i, lab in enumerate(labels):
        ds = [(tail[r * n + i][1] - tail[r * n + i][0]) / 1e3 for r in range(reps)]
        per_step.append(dict(step=lab, kernel=short_name(tail[i][2]), mean_us=statistics.mean(ds),
                             min_us=min(ds)))
    walls = [(tail[(r + 1) * n - 1][1] - tail[r * n][0]) / 1e3 for r in range(reps)]
    inst: Dict[str, dict] = {}
    for s in per_step:
        e = inst.setdefault(s["kernel"], dict(n=0, us=0.0))
        e["n"] += 1
        e["us"] += s["mean_us"]
    return dict(per_step=per_step, instances=inst, wall_us=statistics.median(walls),
                busy_us=sum(s["mean_us"] for s in per_step), replays=reps, batch=info["batch"])


def mfma_table(pmc_dir: str, pass_log: str) -> List[dict]:
    """Per-step executed MFMA operations of a ``bench.py --pmc-pass`` run with
    SQ_INSTS_VALU_MFMA_MOPS_I8 and SQ_INSTS_VALU_MFMA_MOPS_F16 (ops = MOPS x 512)."""
    info = pass_info(pass_log)
    labels = info["steps"]
    disp = load_dispatches(pmc_dir)
    _, steps = _steps_after_calibration(disp, len(labels))
    out = []
    for lab, d in zip(labels, steps):
        c = d["counters"]
        out.append(dict(step=lab, kernel=short_name(d["name"]),
                        ops_i8=c.get("SQ_INSTS_VALU_MFMA_MOPS_I8", 0.0) * 512,
                        ops_f16=c.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0) * 512))
    return out


def _print_stats(a) -> int:
    st = kernel_stats(a.trace, a.pass_log)
    print(f"{st['replays']} graph replays at batch {st['batch']} on one stream; replay wall time (first dispatch "
          f"start to last end, median) {st['wall_us']:.1f} us; sum of kernel durations {st['busy_us']:.1f} us\n")
    print("| kernel instance | launches per step | us per step | mean us per launch |")
    print("|---|---|---|---|")
    for k, e in sorted(st["instances"].items(), key=lambda kv: -kv[1]["us"]):
        print(f"| `{k}` | {e['n']} | {e['us']:.2f} | {e['us'] / e['n']:.2f} |")
    print("\n| step | kernel | mean us | min us |")
    print("|---|---|---|---|")
    for s in st["per_step"]:
        print(f"| {s['step']} | `{s['kernel'][:70]}` | {s['mean_us']:.2f} | {s['min_us']:.2f} |")
    return 0


PEAK_INT8_OPS = 5.0e15   # MI355X dense int8 MFMA, op/s
PEAK_FP16_FLOPS = 2.5e15  # MI355X dense fp16 MFMA, flop/s


def _print_mfma(a) -> int:
    """Executed MFMA ops per step with the step's mean duration from a
    ``--trace-pass`` kernel trace (``--trace DIR --trace-log FILE``): MFMA rate
    = executed ops / duration, as a fraction of the dense peak of its type."""
    rows = mfma_table(a.mfma, a.pass_log)
    dur = {}
    if a.trace and a.trace_log:
        for s in kernel_stats(a.trace, a.trace_log)["per_step"]:
            dur[s["step"]] = s["mean_us"]
    print("| step | kernel | int8 MFMA Gop | fp16 MFMA Gflop | trace mean us | MFMA rate T/s | of peak |")
    print("|---|---|---|---|---|---|---|")
    fam = {}
    for r in rows:
        us = dur.get(r["step"])
        key = "int8" if r["ops_i8"] else ("fp16" if r["ops_f16"] else "other")
        ops = r["ops_i8"] + r["ops_f16"]
        peak = PEAK_INT8_OPS if key == "int8" else PEAK_FP16_FLOPS
        rate = ops / (us * 1e-6) if us else None
        rc = f"{rate / 1e12:.1f}" if rate is not None else ""
        fc = f"{rate / peak:.4f}" if rate is not None and key != "other" else ""
        uc = f"{us:.2f}" if us is not None else ""
        print(f"| {r['step']} | `{r['kernel'][:60]}` | {r['ops_i8'] / 1e9:.3f} | {r['ops_f16'] / 1e9:.3f} | {uc} | {rc} | {fc} |")
        f = fam.setdefault(key, dict(ops=0.0, us=0.0, n=0))
        f["ops"] += ops
        f["us"] += us or 0.0
        f["n"] += 1
    print("\n| launches | count | executed MFMA Gop | trace us per step | MFMA rate T/s | of peak |")
    print("|---|---|---|---|---|---|")
    for k, f in fam.items():
        peak = PEAK_INT8_OPS if k == "int8" else PEAK_FP16_FLOPS
        rate = f["ops"] / (f["us"] * 1e-6) if f["us"] else 0.0
        fc = f"{rate / peak:.4f}" if k != "other" else ""
        print(f"| {k} | {f['n']} | {f['ops'] / 1e9:.2f} | {f['us']:.1f} | {rate / 1e12:.1f} | {fc} |")
    return 0


# Issue cycles of one wave64 VALU instruction on a SIMD (gfx950 measured with
# 8 waves per SIMD: fp32 add 2.5, most others 4.2, exp/rcp 8.2; 4 is the
# figure for the mix) and the part's SIMDs and clock, for the VALU-time column.
VALU_CYCLES = 4.0
SIMDS = 1024
CLOCK_HZ = 2.4e9
INSTS_COUNTERS = ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_VMEM_RD",
                  "SQ_INSTS_VMEM_WR")


def insts_table(pmc_dir: str, pass_log: str) -> List[dict]:
    """Per-step instruction counts of a ``bench.py --pmc-pass`` run with the INSTS_COUNTERS:
    per wave, and the VALU issue time if the step's VALU instructions were spread evenly
    over every SIMD (VALU_CYCLES each)."""
    info = pass_info(pass_log)
    labels = info["steps"]
    disp = load_dispatches(pmc_dir)
    _, steps = _steps_after_calibration(disp, len(labels))
    out = []
    for lab, d in zip(labels, steps):
        c = d["counters"]
        w = max(c.get("SQ_WAVES", 0.0), 1.0)
        valu = c.get("SQ_INSTS_VALU", 0.0)
        out.append(dict(step=lab, kernel=short_name(d["name"]), waves=w, valu=valu / w,
                        salu=c.get("SQ_INSTS_SALU", 0.0) / w, lds=c.get("SQ_INSTS_LDS", 0.0) / w,
                        vmem_rd=c.get("SQ_INSTS_VMEM_RD", 0.0) / w, vmem_wr=c.get("SQ_INSTS_VMEM_WR", 0.0) / w,
                        valu_us=valu * VALU_CYCLES / SIMDS / CLOCK_HZ * 1e6))
    return out


def _print_insts(a) -> int:
    rows = insts_table(a.insts, a.pass_log)
    print("| step | kernel | waves | VALU / wave | SALU / wave | LDS / wave | VMEM rd / wave | VMEM wr / wave "
          "| VALU issue us |")
    print("|---|---|---|---|---|---|---|---|---|")
    fam = {}
    for r in rows:
        print(f"| {r['step']} | `{r['kernel'][:60]}` | {r['waves']:.0f} | {r['valu']:.0f} | {r['salu']:.0f} | "
              f"{r['lds']:.0f} | {r['vmem_rd']:.0f} | {r['vmem_wr']:.0f} | {r['valu_us']:.2f} |")
        key = "int8" if "alg=int8" in r["step"] else ("fp16" if " alg=" in r["step"] else "other")
        fam[key] = fam.get(key, 0.0) + r["valu_us"]
    print("\n| launches | VALU issue us per step |")
    print("|---|---|")
    for k, v in fam.items():
        print(f"| {k} | {v:.1f} |")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--pass-log", required=True)
    ap.add_argument("--trace")
    ap.add_argument("--stats", action="store_true", help="kernel statistics of a bench.py --trace-pass trace")
    ap.add_argument("--mfma", help="MFMA counter run of bench.py --pmc-pass")
    ap.add_argument("--trace-log", help="log of the bench.py --trace-pass run the --trace directory holds")
    ap.add_argument("--insts", help="instruction counter run of bench.py --pmc-pass (INSTS_COUNTERS)")
    a = ap.parse_args()
    if a.stats:
        return _print_stats(a)
    if a.insts:
        return _print_insts(a)
    if a.mfma:
        return _print_mfma(a)
    t = traffic_table(a.fetch, a.write, a.pass_log, a.trace)
    print(f"counter scale (calibration bytes / counter bytes): FETCH_SIZE {t[0]['f_scale']:.4f}, "
          f"WRITE_SIZE {t[0]['w_scale']:.4f}\n")
    print("| step | kernel | grid | HBM read MB | HBM write MB | trace mean us (n) |")
    print("|---|---|---|---|---|---|")
    for r in t[1:]:
        tr = f"{r['trace_us_mean']:.2f} ({r['trace_n']})" if r["trace_us_mean"] is not None else ""
        print(f"| {r['step']} | `{r['kernel'][:60]}` | {r['grid']} | {r['read_mb']:.3f} | {r['write_mb']:.3f} | {tr} |")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
