"""CPU runs of the library's model-level host code under a stand-in HIP runtime.

``tests/hipstub`` builds a host-only ``libamdhip64.so.7`` (device memory is host memory, kernel
launches are counted and do nothing, events report 5 ns per launch between them, graphs and
streams are host objects).  A child process whose dynamic loader finds it first loads the
benchmarked YOLOv8n-320 W8A8 engine through the C ABI, runs it, reads the profile events and
the output and closes it: the engine parser, memory planning, weight preparation, step building
(sibling merges, head 1x1 fusions, head chains, bottleneck superblocks), the lane schedule,
graph capture and teardown all run on the CPU.  With load-time tuning on, every candidate
launcher, the isolated and in-network measurements, the lane choice, the chain and superblock
choices and the tune-cache write and re-read run too.  Kernels do not execute, so outputs are
not checked here (the GPU tests do that); the checks are that each path completes and that its
step list and counters are what the plan says.  With ``make -C aexrt_amd/csrc asan`` built, the
same runs also go through the host-AddressSanitizer build of the library.
"""
from __future__ import annotations

import glob
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
STUB_DIR = ROOT / "tests" / "hipstub"
STUB = STUB_DIR / "_build" / "libamdhip64.so.7"
LIB = ROOT / "aexrt_amd" / "libaexrt_hip.so"
ASAN_LIB = ROOT / "aexrt_amd" / "csrc" / "_build_asan" / "libaexrt_hip_asan.so"

CHILD = r"""
import json, os, sys
sys.path.insert(0, os.environ["AEXRT_ROOT"])
import numpy as np
import bench
from aexrt_amd import engine as E, workloads as WL
from aexrt_amd.runtime import NativeHipYoloModel
spec = json.loads(sys.argv[1])
if spec.get("plan", "committed") == "committed":
    bench.use_tune_plan(False)
else:
    os.environ.pop("AEXRT_HIP_AUTOTUNE", None)
    os.environ["AEXRT_HIP_TUNE_CACHE"] = spec["plan"]
for k, v in spec.get("env", {}).items():
    os.environ[k] = v
res = {}
if spec.get("model") == "c2f":
    g = WL.c2f_block(batch=1, c=128, dim=40, seed=3)
    model = NativeHipYoloModel(E.build_aexrt_engine(g, precision="fp16"))
    model.run(np.zeros((1, 128, 40, 40), np.float32))
elif spec.get("model") == "yolo160_concat_fp16":
    from aexrt_amd.yolov8 import build_yolov8n
    g = build_yolov8n(batch=1, imgsz=160, seed=4)
    model = NativeHipYoloModel(E.build_aexrt_engine(g, precision="fp16", classes=80, fuse_concat_min_h=-1))
    model.run(np.zeros((1, 3, 160, 160), np.float32))
else:
    g, model, _ = bench.build_model(spec["batch"])
    bench.fill_input(model, spec["batch"], 320)
    model.run_device()
    res["output_elements"] = int(np.asarray(model.output()).size)
model.set_profiling(True)
model.run_device()
res["labels"] = [label for label, _ in model.profile_events()]
model.set_profiling(False)
res["superblocks"] = model.counter("c2f_bottleneck_superblock_count")
model.close()
print("RESULT " + json.dumps(res), flush=True)
"""


@pytest.fixture(scope="module")
def stub():
    if not LIB.exists():
        pytest.skip("libaexrt_hip.so is not built")
    r = subprocess.run(["make", "-s", "-C", str(STUB_DIR)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return STUB


def _asan_runtime():
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def _run(spec, asan=False, timeout=600):
    env = dict(os.environ)
    env["LD_LIBRARY_PATH"] = str(STUB.parent) + os.pathsep + env.get("LD_LIBRARY_PATH", "")
    env["AEXRT_ROOT"] = str(ROOT)
    env.pop("AEXRT_HIP_LIBRARY", None)
    if asan:
        env["AEXRT_HIP_LIBRARY"] = str(ASAN_LIB)
        env["LD_PRELOAD"] = _asan_runtime()
        env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    r = subprocess.run([sys.executable, "-c", CHILD, json.dumps(spec)], capture_output=True, text=True,
                       env=env, timeout=timeout, cwd=str(ROOT))
    assert r.returncode == 0, (spec, r.returncode, r.stdout[-2000:], r.stderr[-4000:])
    line = [ln for ln in r.stdout.splitlines() if ln.startswith("RESULT ")]
    assert line, r.stdout[-2000:]
    res = json.loads(line[-1][len("RESULT "):])
    # with AEXRT_HIP_TUNE_LOG=1 the library prints each step's lane of the final schedule
    res["lanes"] = [int(ln.split()[4]) for ln in r.stderr.splitlines() if ln.startswith("aexrt step ")]
    return res


def _conv_labels(res):
    return [lab for lab in res["labels"] if lab.startswith("cmd#")]


@pytest.mark.parametrize("batch", [1, 2, 64])  # 2: no shape of the plan, every choice by rule
def test_committed_plan_loads_runs_and_closes(stub, batch):
    res = _run({"batch": batch})
    assert res["output_elements"] == batch * 144 * 2100  # output0 [B][A = 2100 anchors][4 * 16 + 80]
    assert res["labels"][0].startswith("amax slots clear")
    convs = _conv_labels(res)
    assert len(convs) > 40
    assert all(" kernel=" in lab and "not launchable" not in lab for lab in convs if "CONV" in lab)
    # the neck's two 2x upsamples are read from their sources by the convs over their concats
    folded = [lab for lab in convs if " reading 2x upsample" in lab]
    assert len(folded) == 2 and all("conv1x1_stream_kernel<" in lab and ",false,true>" in lab for lab in folded)
    assert not any(lab.endswith("RESIZE") for lab in convs)


@pytest.mark.parametrize("batch", [1, 64])
def test_committed_chain_tiles_are_applied(stub, batch):
    """Each head chain launch runs the tile its plan line records ("chain cmd <command> <dims> one|two":
    measured at load among the tiles the kernel offers)."""
    tiles = {}
    for key, fields in _plan_line("chain cmd "):
        _, _, cmd, dims, form = key.split()
        if int(dims.split("x")[0]) == batch:
            f = fields.split()
            tiles[(int(cmd), form)] = (int(f[4]), int(f[5]))
    res = _run({"batch": batch})
    chains = [lab for lab in _conv_labels(res) if "conv_chain" in lab]
    assert chains
    for lab in chains:
        cmd = int(lab.split()[0][len("cmd#"):])
        form = "two" if "conv_chain2_kernel" in lab else "one"
        tr, tc = tiles[(cmd, form)]
        assert f"> {tr}x{tc} then" in lab, (lab, tr, tc)


def test_upsample_fold_forms(stub):
    res = _run({"batch": 64, "env": {"AEXRT_HIP_FOLD_UPSAMPLE": "0"}})
    convs = _conv_labels(res)
    assert sum(lab.endswith("RESIZE") for lab in convs) == 2
    assert not any("2x upsample" in lab for lab in convs)
    # the producer form: the convs producing the upsamples' inputs write them too
    res = _run({"batch": 64, "env": {"AEXRT_HIP_FOLD_UPSAMPLE": "copy"}})
    convs = _conv_labels(res)
    folded = [lab for lab in convs if " + 2x upsample" in lab]
    assert len(folded) == 2 and all(",true>" in lab and ",false,true>" not in lab for lab in folded)
    assert not any(lab.endswith("RESIZE") for lab in convs)


def test_load_time_tuning_writes_a_plan_that_reloads(stub, tmp_path):
    plan = tmp_path / "plan.tune"
    log = {"AEXRT_HIP_TUNE_LOG": "1"}
    tuned = _run({"batch": 64, "plan": str(plan), "env": log})
    assert plan.exists() and "schedule 64x3x320x320" in plan.read_text()
    # the measured plan, read back without measuring, gives the same launches on the same lanes
    again = _run({"batch": 64, "plan": str(plan), "env": dict(log, AEXRT_HIP_AUTOTUNE="0")})
    assert again["labels"] == tuned["labels"]
    assert again["lanes"] == tuned["lanes"] and len(tuned["lanes"]) == len(tuned["labels"])


def _plan_line(prefix):
    text = (ROOT / "aexrt_amd" / "tuned" / "yolov8n320.tune").read_text()
    return [ln.split("\t") for ln in text.splitlines() if ln.startswith(prefix)]


def test_committed_lane_plan_is_applied(stub):
    (sched, fields), = _plan_line("schedule 64x3x320x320")
    (_, plan), = _plan_line("lanes 64x3x320x320")
    lanes = int(fields.split()[1])
    log = {"AEXRT_HIP_TUNE_LOG": "1"}
    res = _run({"batch": 64, "env": log})
    assert res["lanes"] == [int(c) for c in plan] and max(res["lanes"]) < lanes
    # the dependency rule instead (same lane count), and list scheduling over the steps' times
    for policy in ("0", "1"):
        other = _run({"batch": 64, "env": dict(log, AEXRT_HIP_LIST_SCHEDULE=policy)})
        assert other["labels"] == res["labels"] and len(other["lanes"]) == len(plan)
        assert max(other["lanes"]) < lanes and other["lanes"][:20] == [0] * 20  # the backbone is a chain


def test_forced_superblocks_build_one_launch_per_bottleneck(stub):
    res = _run({"batch": 64, "env": {"AEXRT_HIP_C2F_SUPERBLOCK": "1"}})
    assert res["superblocks"] > 0
    assert sum("(C2f bottleneck superblock)" in lab for lab in res["labels"]) == res["superblocks"]
    assert any(lab.startswith("superblock sync clear") for lab in res["labels"])
    fp16 = _run({"model": "c2f", "env": {"AEXRT_HIP_C2F_SUPERBLOCK": "1"}})
    assert fp16["superblocks"] == 2


def test_yolov8n_160_fused_concat_fp16_load_time_tuning(stub, tmp_path):
    """The load of the fp16 YOLOv8n-160 engine with its 13 fused concat + 1x1 commands, measuring
    every fp16 candidate at load (the GPU test of this engine is skipped: one of its loads aborted
    on the GPU with no cause shown); here, and under ASan below, it completes."""
    plan = tmp_path / "plan.tune"
    res = _run({"model": "yolo160_concat_fp16", "plan": str(plan)})
    assert plan.exists() and "schedule 1x3x160x160" in plan.read_text()
    assert len(_conv_labels(res)) > 50


def _asan_current():
    return ASAN_LIB.exists() and LIB.exists() and ASAN_LIB.stat().st_mtime >= LIB.stat().st_mtime


@pytest.mark.skipif(not _asan_current() or _asan_runtime() is None,
                    reason="host-ASan library not built, or older than libaexrt_hip.so (make -C aexrt_amd/csrc asan)")
def test_host_paths_under_address_sanitizer(stub, tmp_path):
    _run({"batch": 64}, asan=True)
    _run({"batch": 1, "plan": str(tmp_path / "plan.tune")}, asan=True)  # load-time tuning (bs 1: quicker)
    _run({"model": "yolo160_concat_fp16", "plan": str(tmp_path / "plan160.tune")}, asan=True)
    _run({"batch": 64, "env": {"AEXRT_HIP_C2F_SUPERBLOCK": "1"}}, asan=True)
