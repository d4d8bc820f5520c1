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
    k = re.sub(r"^void ", "", kernel)
    k = re.sub(r"\(.*$", "", k)
    return k.replace("aexrt::", "").replace("(anonymous namespace)::", "").replace("igemm::", "")


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--pass-log", required=True)
    ap.add_argument("--trace")
    a = ap.parse_args()
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
