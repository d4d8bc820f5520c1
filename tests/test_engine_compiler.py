"""CPU tests of the engine compiler and the container (no GPU)."""
from __future__ import annotations

import ctypes
import struct

import numpy as np
import pytest

from aexrt_amd import _lib
from aexrt_amd import engine as E
from aexrt_amd.graph import Graph, TensorSpec
from aexrt_amd.yolov8 import build_yolov8n

from engine_acceptance import reference_accepts


def _params(ic=128, oc=128, h=20, w=20, oh=20, ow=20, k=3, s=1, p=1, d=1, g=1, b=1):
    return [b, ic, h, w, oc, oh, ow, k, k, s, s, p, p, d, d, g]


# reference: tests/test_engine_fp16_winograd_plan.py:47-72
@pytest.mark.parametrize("params", [_params(), _params(ic=96, oc=64), _params(w=18, ow=18)])
def test_winograd_gate_accepts_aligned_even_outputs(params):
    assert E.uses_native_fp16_winograd(params)


@pytest.mark.parametrize("params", [_params(ic=80), _params(h=19, oh=19), _params(w=19, ow=19), _params(k=1, p=0),
                                    _params(s=2), _params(p=0), _params(d=2), _params(g=2)])
def test_winograd_gate_rejects(params):
    assert not E.uses_native_fp16_winograd(params)


def _conv_graph(c=64, dim=40, k=1, silu=False):
    g = Graph("one_conv")
    g.input("images", TensorSpec((1, c, dim, dim)))
    w = (np.arange(c * c * k * k, dtype=np.float32) / 1024.0).reshape(c, c, k, k)
    g.const("w", w)
    g.const("b", np.zeros((c,), np.float32))
    p = k // 2
    g.conv2d("c", "images", "w", "b", pads=(p, p, p, p))
    out = "c"
    if silu:
        g.sigmoid("s", "c")
        g.mul("m", "c", "s")
        out = "m"
    g.reshape("output0", out, (1, c, dim * dim))
    g.output("output0")
    return g


def test_fp16_conv1x1_plan_record_matches_reference_kat():
    # reference: tests/test_engine_fp16_1x1_plan.py:27-73 -> plan[2:6] == (45, 2, 1, 3), layout 4
    data = E.build_aexrt_engine(_conv_graph(), precision="fp16", classes=60)
    info = E.inspect_aexrt_engine(data)
    assert info["kernel_plan"][0][2:6] == (45, 2, 1, 3)
    assert info["packed_layout_counts"] == {4: 1}


def test_value_numbering_and_conv_record():
    plan = E.compile_plan(_conv_graph(), precision="fp16")
    replay = plan["replay"]
    assert replay["names"][:3] == ["images", "w", "b"]
    cmd = replay["commands"][0]
    assert cmd["kind"] == "CONV" and cmd["params"] == [1, 64, 40, 40, 64, 40, 40, 1, 1, 1, 1, 0, 0, 1, 1, 1]
    assert plan["plans"][0]["packed_value"] == 1


def test_silu_pattern_fuses_to_conv_silu():
    replay = E.lower_graph(_conv_graph(k=3, silu=True))
    kinds = [c["kind"] for c in replay["commands"]]
    assert kinds == ["CONV_SILU", "ALIAS"]


def test_yolov8n_plan_puts_backbone_and_neck_on_int8():
    g = build_yolov8n(batch=1)
    replay = E.lower_graph(g)
    algo = E.w8a8_algo_map(replay, g.metadata["int8_convs"].split(","))
    assert len(algo) == 44
    names = replay["names"]
    for i in algo:
        wname = names[replay["commands"][i]["inputs"][1]]
        assert not wname.startswith(("stem", "head"))
    plan = E.compile_plan(g, algo_overrides=algo)
    kernels = [p["planned_kernel"] for p in plan["plans"]]
    assert kernels.count(51) + kernels.count(52) + kernels.count(53) == 44
    layouts = [p["layout"] for p in plan["packed"]]
    assert layouts.count(8) == 44
    # int8 commands carry the DXIL bit like the reference's override (engine.py:1213-1214)
    assert all(plan["plans"][i]["flags"] & E.PLAN_FLAG_DXIL for i in algo)


def test_algo_override_refuses_winograd_and_non_conv():
    g = _conv_graph(k=3, silu=True)
    replay = E.lower_graph(g)
    plans = E.build_kernel_plan(replay, E.PRECISION_FLOAT16)
    assert E.apply_algo_overrides(replay, plans, {0: 40}) == [0]
    with pytest.raises(ValueError):
        E.apply_algo_overrides(replay, plans, {1: 52})


def test_int8_pergroup_flag_only_on_int8_commands():
    g = _conv_graph(k=3, silu=True)
    plan = E.compile_plan(g, algo_overrides={0: 52}, int8_pergroup=[0, 1])
    assert plan["plans"][0]["flags"] & E.PLAN_FLAG_INT8_PERGROUP
    assert not plan["plans"][1]["flags"] & E.PLAN_FLAG_INT8_PERGROUP


def _validate(data: bytes) -> bool:
    L = _lib.lib()
    buf = ctypes.create_string_buffer(data, len(data))
    return bool(L.aexrt_hip_validate_engine(buf, len(data)))


def test_native_loader_validates_and_fails_closed():
    g = _conv_graph(k=3, silu=True)
    data = E.build_aexrt_engine(g, algo_overrides={0: 52})
    assert _validate(data)
    bad = bytearray(data)
    bad[-1] ^= 0x5A
    assert not _validate(bytes(bad))
    assert "checksum" in _lib.last_error()
    # plan says int8 but the packed-weight section lacks the layout-8 record
    sections = E.engine_sections(g, algo_overrides={0: 52})
    sections[E.SECTION_PACKED_WEIGHTS] = E.encode_packed_weights([])
    assert not _validate(E.build_container(sections))
    assert "layout-8" in _lib.last_error()
    # truncated header
    assert not _validate(data[:40])


def test_inspect_reports_crc_mismatch():
    data = bytearray(E.build_aexrt_engine(_conv_graph()))
    data[-3] ^= 1
    with pytest.raises(ValueError, match="checksum"):
        E.inspect_aexrt_engine(bytes(data))


def _val(vid, shape, raw=b""):
    n = int(np.prod(shape))
    return dict(id=vid, name=f"v{vid}", flags=E.VALUE_CONSTANT if raw else 0, elements=n,
                shape4=tuple(([1] * (4 - len(shape))) + list(shape)), raw=raw, rank=len(shape))


def _concat_conv_replay(chans, oc, h, silu=1):
    ic = sum(chans)
    k = len(chans)
    values = [_val(i, (1, c, h, h)) for i, c in enumerate(chans)]
    wid = k
    values.append(_val(wid, (oc, ic, 1, 1), (np.arange(oc * ic, dtype=np.float32) / 1024.0).tobytes()))
    values.append(_val(k + 1, (oc,), np.zeros(oc, np.float32).tobytes()))
    values.append(_val(k + 2, (1, oc, h, h)))
    cmd = dict(kind="CONCAT_CONV1X1", kind_id=E.COMMAND_KIND["CONCAT_CONV1X1"], inputs=[*range(k), wid, k + 1],
               output=k + 2, params=[1, h, h, oc, silu, *chans])
    return dict(values=values, commands=[cmd]), wid


# reference: tests/test_engine_fp16_1x1_plan.py:165-206 (generic plan 1, no packed weight, flags 1)
@pytest.mark.parametrize("oc", [64, 68])
def test_concat_conv1x1_generic_plan_matches_reference_kat(oc):
    replay, _ = _concat_conv_replay([32, 32], oc, 20)
    plans = E.build_kernel_plan(replay, E.PRECISION_FLOAT16)
    p = plans[0]
    assert (p["planned_kernel"], p["precision"], p["packed_value"], p["flags"]) == (1, 2, E.NO_VALUE, 1)
    assert E.build_packed_weights(replay, plans, E.PRECISION_FLOAT16) == []


def test_concat_conv1x1_small_plans_zero():
    replay, _ = _concat_conv_replay([16, 16], 32, 8)
    assert E.build_kernel_plan(replay, E.PRECISION_FLOAT16)[0]["planned_kernel"] == 0


# reference: tests/test_engine_fp16_1x1_plan.py:318-360 ((1, 20, 20, 384 -> 256, silu, 3 x 128) is native)
def test_concat_conv1x1_native_fp16_plan_and_layout4_weight():
    replay, wid = _concat_conv_replay([128, 128, 128], 256, 20)
    assert E.uses_native_fp16_concat_conv1x1(replay["commands"][0])
    plans = E.build_kernel_plan(replay, E.PRECISION_FLOAT16)
    p = plans[0]
    assert (p["planned_kernel"], p["packed_value"], p["flags"]) == (3, wid, E.PLAN_FLAG_AUTHORITATIVE | E.PLAN_FLAG_DXIL)
    packed = E.build_packed_weights(replay, plans, E.PRECISION_FLOAT16)
    assert len(packed) == 1 and packed[0]["layout"] == 4
    assert (packed[0]["in_channels"], packed[0]["out_channels"], packed[0]["elements"]) == (384, 256, 384 * 256)
    # fp32 engines never take the native kernel
    assert E.build_kernel_plan(replay, E.PRECISION_FLOAT32)[0]["planned_kernel"] == 1


@pytest.mark.parametrize("threshold,count", [(None, 0), (-1, 13), (20, 4), (44, 1)])
def test_yolov8n_concat_conv1x1_fusion_thresholds(threshold, count):
    """yolo.py:473-488: fused by default; AEXRTC_UNFUSE_SMALL_CONCAT=1/2 keep only outputs taller than 20/44."""
    g = build_yolov8n(batch=1, imgsz=320, seed=4)
    r = E.lower_graph(g, fuse_concat_min_h=threshold)
    cc = [c for c in r["commands"] if c["kind"] == "CONCAT_CONV1X1"]
    assert len(cc) == count
    n_conv = sum(1 for c in r["commands"] if c["kind"] in ("CONV", "CONV_SILU"))
    assert n_conv + count == 63
    for c in cc:
        n, h, w, oc, silu, *chans = c["params"]
        out = r["values"][c["output"]]
        assert (n, oc, h, w) == tuple(out["shape4"]) and silu == 1
        assert chans == [r["values"][v]["shape4"][1] for v in c["inputs"][:-2]]
        assert r["values"][c["inputs"][-2]]["shape4"] == (oc, sum(chans), 1, 1)


def test_fused_engine_validates():
    g = build_yolov8n(batch=1, imgsz=160, seed=4)
    data = E.build_aexrt_engine(g, precision="fp16", classes=80, fuse_concat_min_h=-1)
    L = _lib.lib()
    buf = ctypes.create_string_buffer(data, len(data))
    assert L.aexrt_hip_validate_engine(buf, len(data))


def _engines():
    g1 = build_yolov8n(batch=1, imgsz=160, seed=4)
    r1 = E.lower_graph(g1)
    int8 = E.w8a8_algo_map(r1, g1.metadata["int8_convs"].split(","))
    return {
        "conv1x1_fp16": E.build_aexrt_engine(_conv_graph(), precision="fp16", classes=60),
        "conv3x3_silu_fp32": E.build_aexrt_engine(_conv_graph(k=3, silu=True), precision="fp32", classes=60),
        "conv3x3_int8": E.build_aexrt_engine(_conv_graph(k=3, silu=True), algo_overrides={0: 52}, classes=60),
        "yolov8n160_fp16": E.build_aexrt_engine(g1, precision="fp16", classes=80),
        "yolov8n160_w8a8": E.build_aexrt_engine(g1, precision="fp16", classes=80, algo_overrides=int8),
        "yolov8n160_w8a8_pg16": E.build_aexrt_engine(g1, precision="fp16", classes=80, algo_overrides=int8,
                                                     int8_pergroup=sorted(int8)),
        "yolov8n160_fused_concat": E.build_aexrt_engine(g1, precision="fp16", classes=80, fuse_concat_min_h=-1),
        "yolov8n320_bs2_w8a8": E.build_aexrt_engine(build_yolov8n(batch=2, imgsz=320, seed=4), precision="fp16",
                                                    classes=80, algo_overrides=int8),
    }


ENGINES = _engines()


@pytest.mark.parametrize("name", sorted(ENGINES))
def test_written_engines_pass_reference_acceptance(name):
    """Sections 1-9, a real arena size and every record rule of the reference loader
    (RT:17560-18593) and inspector (ENG:336-400)."""
    data = ENGINES[name]
    ok, why = reference_accepts(data)
    assert ok, why
    assert _validate(data), _lib.last_error()
    info = E.inspect_aexrt_engine(data)
    assert set(info["sections"]) == set(range(1, 10))
    mem = info["memory_plan"]
    assert mem["version"] == 2 and info["manifest"]["arena_nbytes"] == sum(mem["page_nbytes"]) > 0
    assert info["fusion_groups"] == [] and info["pipeline_cache_records"] == 0


def _arena_layout(data: bytes):
    """(page, offset, nbytes, born, last read) of every allocated value, from the engine bytes."""
    info = E.inspect_aexrt_engine(data)
    s = info["sections"][E.SECTION_MEMORY_PLAN]
    body = data[s["offset"]:s["offset"] + s["size"]]
    _, _, pages, nrec, _, _, _ = struct.unpack_from("<4IQII", body)
    at = 32 + 24 * pages
    return [struct.unpack_from("<6IQQ", body, at + 40 * i) for i in range(nrec)]


def test_memory_plan_keeps_live_values_apart_and_outputs_off_their_input_pages():
    """Overlapping byte ranges on one page only for values whose lifetimes do not overlap; no
    command writes a page it reads (page colouring)."""
    g = build_yolov8n(batch=1, imgsz=160, seed=4)
    replay = E.lower_graph(g)
    mem = E.plan_memory(replay)
    root = list(range(len(replay["values"])))
    for c in replay["commands"]:
        if c["kind"] in ("VIEW", "ALIAS"):
            root[c["output"]] = root[c["inputs"][0]]
    born, last = {}, {}
    for v in replay["values"]:
        if v["flags"] & E.VALUE_INPUT:
            born[v["id"]] = -1
    for i, c in enumerate(replay["commands"]):
        for x in c["inputs"]:
            last[root[x]] = max(last.get(root[x], -1), i)
        born.setdefault(root[c["output"]], i)
    last[root[replay["output_value"]]] = len(replay["commands"])
    recs = {v: r for v, r in mem["records"].items() if root[v] == v}
    for a in recs:
        for b in recs:
            if a >= b or recs[a][1] != recs[b][1]:
                continue
            _, _, oa, na = recs[a]
            _, _, ob, nb = recs[b]
            if oa < ob + nb and ob < oa + na:
                assert last.get(a, born[a]) < born[b] or last.get(b, born[b]) < born[a], (a, b)
    for c in replay["commands"]:
        if c["kind"] in ("VIEW", "ALIAS"):
            continue
        out_page = mem["records"][c["output"]][1]
        for x in c["inputs"]:
            if x in mem["records"]:
                assert mem["records"][x][1] != out_page
    assert mem["total_nbytes"] < sum(4 * replay["values"][v]["elements"] for v in recs)
    assert _arena_layout(ENGINES["yolov8n160_fp16"])


def _patched(data: bytes, section: int, fn) -> bytes:
    """Engine with one section payload replaced by fn(payload), CRCs and offsets rebuilt."""
    info = E.inspect_aexrt_engine(data)
    secs = {t: data[s["offset"]:s["offset"] + s["size"]] for t, s in info["sections"].items()}
    secs[section] = fn(secs[section])
    return E.build_container(secs)


def _set(fmt: str, at: int, *vals):
    def f(b: bytes) -> bytes:
        out = bytearray(b)
        struct.pack_into(fmt, out, at, *vals)
        return bytes(out)
    return f


def _toc_patch(data: bytes, index: int, field_at: int, value: int) -> bytes:
    out = bytearray(data)
    struct.pack_into("<I", out, 64 + 32 * index + field_at, value)
    return bytes(out)


def _mutations():
    base = ENGINES["conv3x3_int8"]
    secs = E.inspect_aexrt_engine(base)["sections"]
    order = sorted(secs)
    return {
        "duplicate section type": _toc_patch(base, order.index(9), 0, 8),
        "TOC reserved field": _toc_patch(base, 0, 28, 1),
        "missing memory plan": E.build_container({t: base[s["offset"]:s["offset"] + s["size"]]
                                                  for t, s in secs.items() if t != 7}),
        "arena_nbytes zero": _patched(base, 1, _set("<Q", 76, 0)),
        "manifest version": _patched(base, 1, _set("<I", 0, 2)),
        "manifest mode": _patched(base, 1, _set("<I", 12, 1)),
        "values reserved": _patched(base, 2, _set("<I", 4, 7)),
        "memory page flags": _patched(base, 7, _set("<I", 32 + 12, 0)),
        "memory total": _patched(base, 7, _set("<Q", 16, 1)),
        "memory record page dtype": _patched(base, 7, lambda b: _set("<I", 32 + 24 * struct.unpack_from(
            "<I", b, 8)[0] + 12, 2)(b)),
        "fusion plan version": _patched(base, 8, _set("<I", 0, 2)),
        "fusion plan command count": _patched(base, 8, _set("<I", 8, 99)),
        "pipeline cache version": _patched(base, 9, _set("<I", 0, 0)),
        "pipeline cache record without payload": _patched(
            base, 9, lambda b: struct.pack("<4I", 1, 1, 0, 0) + struct.pack("<IIQQQ", 1, 0, 5, 48, 0)),
        "kernel plan flags": _patched(base, 5, _set("<I", 8 + 20, 1 | 64)),
    }


MUTATIONS = _mutations()


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_mutated_engines_are_refused_like_the_reference(name):
    data = MUTATIONS[name]
    ok, _ = reference_accepts(data)
    assert not ok
    assert not _validate(data)


def _yolo_engine_sections(imgsz=160):
    g = build_yolov8n(batch=1, imgsz=imgsz, seed=4)
    return E.engine_sections(g, precision="fp16", classes=80)


def _mutate_command(sections, kind: str, fn):
    """Sections with the params of the first command of `kind` rewritten by fn(params) (same count)."""
    body = bytearray(sections[E.SECTION_COMMANDS])
    n = struct.unpack_from("<I", body, 0)[0]
    at = 8
    for _ in range(n):
        k, _, ni, npar, _, _ = struct.unpack_from("<6I", body, at)
        p_at = at + 24 + 4 * ni
        if k == E.COMMAND_KIND[kind]:
            params = list(struct.unpack_from(f"<{npar}I", body, p_at))
            struct.pack_into(f"<{npar}I", body, p_at, *fn(params))
            out = dict(sections)
            out[E.SECTION_COMMANDS] = bytes(body)
            return out
        at = p_at + 4 * npar
    raise AssertionError(f"no {kind} command")


def _with(params, **changes):
    out = list(params)
    for idx, v in changes.items():
        out[int(idx[1:])] = v
    return out


@pytest.mark.parametrize("kind,change", [
    ("RESIZE", dict(i1=64)),       # more channels than its input: the kernel would overrun the output root
    ("RESIZE", dict(i0=3)),        # more images than its input
    ("RESIZE", dict(i2=7)),        # input height that is not the input's
    ("MAXPOOL", dict(i0=2)),       # batch that is not the input's
    ("MAXPOOL", dict(i4=9)),       # output rows the 5x5/s1/p2 window does not produce
])
def test_loader_refuses_resize_and_maxpool_params_that_disagree_with_their_input(kind, change):
    """infer_dims checks RESIZE / MAXPOOL params against the input before anything is sized from
    them (aexrt_hip_validate_engine runs the same host-side shape inference as a load)."""
    base = _yolo_engine_sections()
    assert _validate(E.build_container(base)), _lib.last_error()
    bad = _mutate_command(base, kind, lambda p: _with(p, **change))
    assert not _validate(E.build_container(bad))
    assert kind in _lib.last_error()
