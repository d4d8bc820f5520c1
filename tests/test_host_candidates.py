"""CPU checks of the load-time kernel/tile candidates (host code only).

The model loader measures every candidate ``enumerate_conv_choices`` offers
for a conv shape and launches the fastest.  Here every conv of the
benchmarked networks goes through ``aexrt_hip_conv_candidates``: each
candidate must be accepted by its own launcher (which runs in probe mode: it
resolves the kernel instance and geometry, makes no HIP call and launches
nothing), the enumeration must stay below its cap (a count at the cap means
candidates were dropped unmeasured), and the streaming 1x1 int8 kernel must be
offered exactly where its launcher's conditions hold.  Run with
``AEXRT_HIP_LIBRARY`` pointing at the host-ASan build
(``make -C aexrt_amd/csrc asan``) and the clang ASan runtime preloaded, the
same paths are checked for memory errors.
"""
from __future__ import annotations

import pytest

from aexrt_amd import engine as E
from aexrt_amd import kernels as K
from aexrt_amd._lib import ConvDesc
from aexrt_amd.yolov8 import build_yolov8n

CAP = 256  # kMaxConvChoices in the library


def _network_convs(batch, imgsz=320):
    g = build_yolov8n(batch=batch, imgsz=imgsz, seed=4)
    names = g.metadata["int8_convs"].split(",")
    plan = E.compile_plan(g, precision="fp16", algo_overrides=E.w8a8_algo_map(E.lower_graph(g), names))
    for i, c in enumerate(plan["replay"]["commands"]):
        if c["kind"] not in ("CONV", "CONV_SILU"):
            continue
        params = list(c["params"][:16])
        alg = plan["plans"][i]["planned_kernel"]
        if alg not in E.INT8_KERNELS:
            alg = 5  # every fp16 plan id runs on the fp16 MFMA kernels (Winograd has no tiles)
        flags = K.SILU if c["kind"] == "CONV_SILU" else 0
        x_cstride = None
        if params[1] == 3:  # the network input: fp32 NCHW read by the stem conv as 8 channels
            params[1] = 8
            flags |= K.IN_NCHW_F32
            x_cstride = 3
        yield i, ConvDesc.from_params(params), alg, flags, x_cstride


def _check(desc, alg, flags, **kw):
    names = K.conv_candidates(desc, alg, flags, **kw)
    assert 0 < len(names) < CAP, (desc.as_list(), len(names))
    assert all(names), [k for k, n in enumerate(names) if not n]
    assert len(set(names)) == len(names), "duplicate candidates"
    return names


@pytest.mark.parametrize("batch", [1, 64])
def test_every_candidate_of_yolov8n_320_is_launchable(batch):
    total = 0
    for i, desc, alg, flags, xc in _network_convs(batch):
        names = _check(desc, alg, flags, x_cstride=xc)
        s1x1 = [n for n in names if n.startswith("conv1x1_stream_kernel")]
        one_by_one = desc.kernel_h == 1 and desc.kernel_w == 1
        assert bool(s1x1) == (alg == 51 and one_by_one and desc.in_channels % 16 == 0), (i, names)
        total += len(names)
    assert total > 1000


def test_streaming_1x1_candidates_follow_its_view_rules():
    d = ConvDesc.from_params([64, 128, 20, 20, 128, 20, 20, 1, 1, 1, 1, 0, 0, 1, 1, 1])
    dense = [n for n in _check(d, 51, K.SILU) if n.startswith("conv1x1_stream")]
    assert dense
    # output written into a channel slice of a wider concat root: still evenly strided
    sliced = [n for n in _check(d, 51, K.SILU, y_cstride=384) if n.startswith("conv1x1_stream")]
    assert sliced == dense
    # a residual add in the epilogue is not supported by the streaming kernel
    res = _check(d, 51, K.SILU | K.RESIDUAL, residual=True)
    assert not [n for n in res if n.startswith("conv1x1_stream")]
    # fp16 convs never take it
    assert not [n for n in _check(d, 5, K.SILU) if n.startswith("conv1x1_stream")]


def test_candidates_refuse_convs_without_tile_choice():
    d = ConvDesc.from_params([1, 64, 40, 40, 64, 40, 40, 3, 3, 1, 1, 1, 1, 1, 1, 1])
    with pytest.raises(RuntimeError, match="no tile choice"):
        K.conv_candidates(d, 40, K.SILU)
