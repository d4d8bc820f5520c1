"""The conv_autotune program (per-device algorithm choice with a detection gate) on a real engine.

It must run the reference tool's flow end to end over the public C ABI and
emit a report, a JSON algo map {engine command index: algorithm} that the
compiler accepts as algo_overrides, and a C header table.
"""
from __future__ import annotations

import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

from aexrt_amd import engine as E
from aexrt_amd.runtime import NativeHipYoloModel
from aexrt_amd.yolov8 import build_yolov8n
from tests.test_gpu_model import _layer_check

pytestmark = pytest.mark.gpu

TOOL = Path(__file__).resolve().parents[1] / "aexrt_amd" / "conv_autotune"


def test_conv_autotune_emits_gated_algo_map(cuda, tmp_path):
    g = build_yolov8n(batch=1, imgsz=160, seed=4)
    eng = tmp_path / "y160.aexrt"
    eng.write_bytes(E.build_aexrt_engine(g, precision="fp16", classes=80))
    report, amap, hdr = tmp_path / "report.md", tmp_path / "map.json", tmp_path / "tuned.h"
    r = subprocess.run([str(TOOL), str(eng), "--runs", "3", "--warmup", "1", "--limit", "8", "--out", str(report),
                        "--emit-map", str(amap), "--emit-header", str(hdr)],
                       capture_output=True, text=True, timeout=240)
    print(r.stdout[-3000:], r.stderr[-2000:])
    assert r.returncode == 0, r.stderr
    assert "final gate PASS" in r.stdout
    text = report.read_text()
    assert "# conv_autotune report" in text and "final detection gate: PASS" in text
    m = {int(k): int(v) for k, v in json.loads(amap.read_text()).items()}
    plan = E.compile_plan(g, precision="fp16")
    kinds = {i: c["kind"] for i, c in enumerate(plan["replay"]["commands"])}
    assert all(kinds[k] in ("CONV", "CONV_SILU") for k in m)
    assert "kAexrtTunedConvCount" in hdr.read_text()
    # the map rebuilds into an engine (Winograd targets are refused by the compiler) whose every
    # conv matches the oracle fed the GPU's own layer inputs, on the algorithm the map chose
    # (conv_autotune.cpp:300-351 keeps a choice only when the detections pass its gate; here each
    # layer is held to the backend's parity bounds)
    overrides = {k: v for k, v in m.items() if v not in (40, 46)}
    data = E.build_aexrt_engine(g, precision="fp16", classes=80, algo_overrides=overrides)
    plan = E.compile_plan(g, precision="fp16", algo_overrides=overrides)
    x = np.random.default_rng(1).random((1, 3, 160, 160)).astype(np.float32)
    with NativeHipYoloModel(data) as model:
        model.run(x)
        current = {i["command_index"]: i["current_algorithm"] for i in model.conv_plan()}
        for k, v in overrides.items():
            assert current[k] == v, (k, v, current[k])
        checked, worst = _layer_check(model, g, plan, threads=8)
        assert checked == 63, checked
        assert worst <= 1.0
