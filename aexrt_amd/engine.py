"""Engine compiler: Graph -> replay commands -> kernel plan -> packed weights
-> ``.aexrt`` container (the reference's ``aexrtc build``, src/aexrt/engine.py).

What is kept byte-compatible with the reference, because it is the drop-in
surface:
  * the container: 64-byte header, 32-byte TOC entries, 64-byte aligned
    sections, CRC32 per section, sections 1-9 present (docs/AEXRT_ENGINE.md:54-104;
    loader RT:17560-17599);
  * the record formats of sections 1-9: manifest, values, commands, constants,
    kernel plan, packed weights, Memory Plan V2, fusion plan, pipeline cache
    (docs/AEXRT_ENGINE.md:106-538);
  * command kinds and their u32 params (yolo.py:701-927), kernel ids
    (runtime enum RT:8881-8940), plan flags (engine.py:85-96), packed layouts
    2/3/4/5/8 (engine.py:59-71);
  * the kernel-plan rules (engine.py:1046-1109, 1945-2098), the algo-map
    override (engine.py:1112-1222) and the int8 per-group flag loop
    (engine.py:192-210).

The writer itself (_Section, the encoders, build_container) and the arena
placement (plan_memory) are this compiler's own.  Not emitted: the optional
physical dispatch and barrier plans (sections 10-11).  The fusion plan has no
groups and the pipeline cache no records.  The HIP runtime plans its own
NHWC memory at load (concat inputs placed as slices of their concat) and
ignores section 7, which describes the reference runtime's fp32 NCHW arena.
"""
from __future__ import annotations

import hashlib
import os
import struct
import zlib
from pathlib import Path
from typing import Any, Dict, Iterable, List, Optional, Sequence

import numpy as np

from . import packing
from .graph import Graph, TensorSpec, infer_value_specs

ENGINE_MAGIC = b"AEXRTENG"
ENGINE_VERSION = 1
ENGINE_HEADER_SIZE = 64
ENGINE_TOC_ENTRY_SIZE = 32
ENGINE_ALIGNMENT = 64

SECTION_MANIFEST = 1
SECTION_VALUES = 2
SECTION_COMMANDS = 3
SECTION_CONSTANTS = 4
SECTION_KERNEL_PLAN = 5
SECTION_PACKED_WEIGHTS = 6
SECTION_MEMORY_PLAN = 7
SECTION_FUSION_PLAN = 8
SECTION_PIPELINE_CACHE = 9
REQUIRED_SECTIONS = tuple(range(1, 10))

PRECISION_FLOAT32 = 1
PRECISION_FLOAT16 = 2

PLAN_FLAG_AUTHORITATIVE = 1 << 0
PLAN_FLAG_DXIL = 1 << 1
PLAN_FLAG_INPUT_FP16 = 1 << 2
PLAN_FLAG_OUTPUT_FP16 = 1 << 3
PLAN_FLAG_INT8_PERGROUP = 1 << 4

VALUE_INPUT = 1 << 0
VALUE_CONSTANT = 1 << 1
VALUE_ARENA = 1 << 2
VALUE_ALIAS = 1 << 3

NO_OFFSET = (1 << 64) - 1
NO_VALUE = (1 << 32) - 1

COMMAND_KIND = {
    "CONV": 1, "CONV_SILU": 2, "CONCAT_CONV1X1": 3, "VIEW": 4, "ALIAS": 5, "SLICE": 6, "CONCAT": 7,
    "RESIZE": 8, "MAXPOOL": 9, "UNARY": 10, "BINARY": 11, "MATMUL": 12, "TRANSPOSE": 13, "SOFTMAX": 14,
}
KIND_NAME = {v: k for k, v in COMMAND_KIND.items()}

INT8_KERNELS = (51, 52, 53)
WINOGRAD_KERNELS = (40, 46)


# ---------------------------------------------------------------------------
# lowering
# ---------------------------------------------------------------------------

def _shape4(shape: Sequence[int]) -> List[int]:
    s = [int(v) for v in shape]
    if len(s) > 4:
        raise NotImplementedError("replay tensors support rank <= 4")
    return [1] * (4 - len(s)) + s


def _numel(shape: Sequence[int]) -> int:
    return int(np.prod([int(v) for v in shape])) if len(shape) else 1


def _strides4(shape: Sequence[int]) -> List[int]:
    p = _shape4(shape)
    st = [1, 1, 1, 1]
    for i in range(2, -1, -1):
        st[i] = st[i + 1] * p[i + 1]
    return st


def conv_params(x: Sequence[int], w: Sequence[int], y: Sequence[int], attrs: Dict[str, Any]) -> List[int]:
    """16-u32 conv descriptor (yolo.py:929-939)."""
    pads = [int(v) for v in attrs.get("pads", [0, 0, 0, 0])]
    strides = [int(v) for v in attrs.get("strides", [1, 1])]
    dil = [int(v) for v in attrs.get("dilations", [1, 1])]
    return [int(x[0]), int(x[1]), int(x[2]), int(x[3]), int(y[1]), int(y[2]), int(y[3]), int(w[2]), int(w[3]),
            strides[0], strides[1], pads[0], pads[1], dil[0], dil[1], int(attrs.get("group", 1))]


def _silu_patterns(graph: Graph) -> Dict[int, int]:
    """conv node index -> mul node index for Conv -> Sigmoid -> Mul(conv, sigmoid) (yolo.py:599)."""
    consumers: Dict[str, List[int]] = {}
    for i, n in enumerate(graph.nodes):
        for v in n.inputs:
            consumers.setdefault(v, []).append(i)
    out: Dict[int, int] = {}
    for i, n in enumerate(graph.nodes):
        if n.op != "Conv" or len(n.outputs) != 1:
            continue
        y = n.outputs[0]
        users = consumers.get(y, [])
        if len(users) != 2 or y in graph.outputs:
            continue
        sig = [u for u in users if graph.nodes[u].op == "Sigmoid"]
        mul = [u for u in users if graph.nodes[u].op == "Mul"]
        if len(sig) != 1 or len(mul) != 1:
            continue
        s_out = graph.nodes[sig[0]].outputs[0]
        if consumers.get(s_out, []) != [mul[0]] or set(graph.nodes[mul[0]].inputs) != {y, s_out}:
            continue
        out[i] = mul[0]
    return out


def _concat_conv1x1_patterns(graph: Graph, silu: Dict[int, int]) -> Dict[int, int]:
    """concat node index -> conv node index for Concat immediately followed by the 1x1 conv that is
    the concat's only consumer (yolo.py:586-596, 624-659)."""
    uses: Dict[str, int] = {}
    for n in graph.nodes:
        for v in n.inputs:
            uses[v] = uses.get(v, 0) + 1
    out: Dict[int, int] = {}
    for i, n in enumerate(graph.nodes[:-1]):
        conv = graph.nodes[i + 1]
        if n.op != "Concat" or len(n.outputs) != 1 or uses.get(n.outputs[0], 0) != 1:
            continue
        if conv.op != "Conv" or not conv.inputs or conv.inputs[0] != n.outputs[0] or len(conv.inputs) < 2:
            continue
        w = graph.constants.get(conv.inputs[1])
        if w is None or np.asarray(w).ndim != 4 or tuple(np.asarray(w).shape[2:]) != (1, 1):
            continue
        out[i] = i + 1
    return out


def lower_graph(graph: Graph, *, fuse_concat_min_h: Optional[int] = None) -> Dict[str, Any]:
    """Graph -> replay dict {values, commands, input_value, output_value}.

    fuse_concat_min_h: None keeps every Concat + 1x1 conv separate (so that
    the int8 plan can claim the conv); otherwise a Concat feeding a 1x1 conv
    whose output is taller than fuse_concat_min_h rows becomes one
    CONCAT_CONV1X1 command (yolo.py:473-488: -1 fuses all, the reference's
    default; 20 / 44 are its AEXRTC_UNFUSE_SMALL_CONCAT=1 / 2 settings).
    """
    if len(graph.inputs) != 1 or len(graph.outputs) != 1:
        raise ValueError("the conv-path compiler takes one input and one output")
    specs = infer_value_specs(graph)
    silu = _silu_patterns(graph)
    skip = set()
    for ci, mi in silu.items():
        sig = [j for j in range(len(graph.nodes)) if graph.nodes[j].op == "Sigmoid"
               and graph.nodes[j].inputs == [graph.nodes[ci].outputs[0]]]
        skip.update(sig)
        skip.add(mi)
    fused: Dict[int, int] = {}
    if fuse_concat_min_h is not None:
        for ci, vi in _concat_conv1x1_patterns(graph, silu).items():
            y = graph.nodes[silu[vi]].outputs[0] if vi in silu else graph.nodes[vi].outputs[0]
            if int(specs[y].shape[2]) > fuse_concat_min_h:
                fused[ci] = vi
    fused_convs = set(fused.values())
    generated: Dict[str, np.ndarray] = {}
    raw_cmds: List[Dict[str, Any]] = []

    def conv_bias(n, w) -> str:
        if len(n.inputs) >= 3:
            return n.inputs[2]
        oc = specs[w].shape[0]
        b = f"__aexrt_zero_bias_{len(raw_cmds)}_{oc}"
        generated[b] = np.zeros((oc,), np.float32)
        specs[b] = TensorSpec((oc,), "float32")
        return b

    for i, n in enumerate(graph.nodes):
        if i in skip or i in fused_convs:
            continue
        op = n.op
        if i in fused:
            # CONCAT_CONV1X1 params: N, H, W, OC, silu, then the channels of
            # each concat input (yolo.py:771-779)
            vi = fused[i]
            conv = graph.nodes[vi]
            y = graph.nodes[silu[vi]].outputs[0] if vi in silu else conv.outputs[0]
            w = conv.inputs[1]
            b = conv_bias(conv, w)
            nb, oc, oh, ow = specs[y].shape
            params = [nb, oh, ow, oc, 1 if vi in silu else 0, *[int(specs[v].shape[1]) for v in n.inputs]]
            raw_cmds.append(dict(kind="CONCAT_CONV1X1", out=[y], ins=[*n.inputs, w, b], params=params))
            continue
        if op == "Conv":
            x, w = n.inputs[0], n.inputs[1]
            y = graph.nodes[silu[i]].outputs[0] if i in silu else n.outputs[0]
            b = conv_bias(n, w)
            params = conv_params(specs[x].shape, specs[w].shape, specs[y].shape, n.attrs)
            raw_cmds.append(dict(kind="CONV_SILU" if i in silu else "CONV", out=[y], ins=[x, w, b],
                                 params=params))
        elif op == "Split":
            src = n.inputs[0]
            shp = specs[src].shape
            axis = n.attrs.get("axis", 0) % len(shp)
            if axis != 1:
                raise NotImplementedError("only channel splits lower to VIEW")
            trailing = _numel(shp[2:])
            off = 0
            for o in n.outputs:
                c = specs[o].shape[1]
                raw_cmds.append(dict(kind="VIEW", out=[o], ins=[src], params=[off * trailing, c * trailing]))
                off += c
        elif op == "Concat":
            out = n.outputs[0]
            rank = len(specs[out].shape)
            axis = n.attrs.get("axis", 0) % rank
            sizes = [int(specs[v].shape[axis]) for v in n.inputs]
            sizes += [sizes[-1]] * (8 - len(sizes))
            params = [_numel(specs[out].shape), rank, axis + (4 - rank), len(n.inputs),
                      *_shape4(specs[out].shape), *sizes, 0, 0]
            raw_cmds.append(dict(kind="CONCAT", out=[out], ins=list(n.inputs), params=params))
        elif op == "MaxPool":
            src, out = n.inputs[0], n.outputs[0]
            nb, c, ih, iw = specs[src].shape
            _, _, oh, ow = specs[out].shape
            k = n.attrs["kernel_shape"]
            s = n.attrs.get("strides", k)
            p = n.attrs.get("pads", [0, 0, 0, 0])
            d = n.attrs.get("dilations", [1, 1])
            raw_cmds.append(dict(kind="MAXPOOL", out=[out], ins=[src],
                                 params=[nb, c, ih, iw, oh, ow, k[0], k[1], s[0], s[1], p[0], p[1], d[0]]))
        elif op == "Resize":
            src, out = n.inputs[0], n.outputs[0]
            nb, c, ih, iw = specs[src].shape
            _, _, oh, ow = specs[out].shape
            raw_cmds.append(dict(kind="RESIZE", out=[out], ins=[src], params=[nb, c, ih, iw, oh, ow]))
        elif op in ("Add", "Sub", "Mul", "Div"):
            a, b = n.inputs[:2]
            out = n.outputs[0]
            code = {"Add": 0, "Sub": 1, "Mul": 2, "Div": 3}[op]
            params = [_numel(specs[out].shape), code, len(specs[out].shape), 0, *_shape4(specs[out].shape),
                      *_shape4(specs[a].shape), *_shape4(specs[b].shape), *_strides4(specs[a].shape),
                      *_strides4(specs[b].shape)]
            raw_cmds.append(dict(kind="BINARY", out=[out], ins=[a, b], params=params))
        elif op == "Sigmoid":
            out = n.outputs[0]
            raw_cmds.append(dict(kind="UNARY", out=[out], ins=[n.inputs[0]], params=[2, _numel(specs[out].shape)]))
        elif op == "Reshape":
            out = n.outputs[0]
            raw_cmds.append(dict(kind="ALIAS", out=[out], ins=[n.inputs[0]], params=[0, _numel(specs[out].shape)]))
        else:
            raise NotImplementedError(f"cannot lower {op}")

    # value numbering: inputs, generated constants, then first appearance
    names: List[str] = []
    seen = set()

    def add(name: str) -> None:
        if name not in seen:
            seen.add(name)
            names.append(name)

    for name in graph.inputs:
        add(name)
    for name in generated:
        add(name)
    for c in raw_cmds:
        for v in c["ins"]:
            add(v)
        for v in c["out"]:
            add(v)
    vid = {name: i for i, name in enumerate(names)}
    values = []
    for name in names:
        shape = specs[name].shape
        flags = 0
        raw = b""
        if name in graph.inputs:
            flags |= VALUE_INPUT
        elif name in graph.constants or name in generated:
            flags |= VALUE_CONSTANT
            arr = graph.constants[name] if name in graph.constants else generated[name]
            raw = np.ascontiguousarray(arr, dtype=np.float32).tobytes()
        values.append(dict(id=vid[name], name=name, flags=flags, elements=_numel(shape), shape4=tuple(_shape4(shape)),
                           raw=raw, rank=len(shape)))
    commands = [dict(kind=c["kind"], kind_id=COMMAND_KIND[c["kind"]], output=vid[c["out"][0]],
                     inputs=[vid[v] for v in c["ins"]], params=[int(p) for p in c["params"]]) for c in raw_cmds]
    return dict(values=values, commands=commands, input_value=vid[next(iter(graph.inputs))],
                output_value=vid[graph.outputs[0]], names=names)


# ---------------------------------------------------------------------------
# kernel plan (engine.py:1046-1109 and the shape gates it calls)
# ---------------------------------------------------------------------------

def _p16(params):
    return tuple(int(v) for v in params[:16])


def uses_native_fp16_winograd(params) -> bool:
    """engine.py:1945-1963."""
    if len(params) < 16:
        return False
    _, ic, _, _, _, oh, ow, kh, kw, sh, sw, pt, pl, dh, dw, g = _p16(params)
    return (kh == kw == 3 and sh == sw == 1 and pt == pl == 1 and dh == dw == 1 and g == 1 and ic > 0
            and ic % 32 == 0 and oh > 0 and ow > 0 and oh % 2 == 0 and ow % 2 == 0)


_STRIDE1_39 = {(40, 40, 64, 64), (40, 40, 128, 64)}
_STRIDE1_40 = {(20, 20, 128, 64), (20, 20, 128, 128), (20, 20, 256, 64), (20, 20, 64, 64), (10, 10, 256, 64),
               (10, 10, 128, 128), (10, 10, 64, 64)}


def stable_conv_algorithm(params, silu: bool) -> int:
    """Shape table of engine.py:1966-2032 (kernel ids of the runtime enum)."""
    if len(params) < 16:
        return 0
    _, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, pt, pl, dh, dw, g = _p16(params)
    if kh == kw == sh == sw == dh == dw == 1 and pt == pl == 0 and g == 1 and ih == oh and iw == ow:
        return 1
    if (silu and (ic, ih, iw, oc, oh, ow) == (3, 320, 320, 32, 160, 160) and kh == kw == 6 and sh == sw == 2
            and pt == pl == 2 and dh == dw == g == 1):
        return 42
    if not silu or kh != 3 or kw != 3 or pt != 1 or pl != 1 or dh != 1 or dw != 1 or g != 1:
        return 0
    shape = (oh, ow, ic, oc)
    if sh == sw == 2 and ih >= oh * 2 - 1 and iw >= ow * 2 - 1:
        if shape in {(160, 160, 3, 16), (80, 80, 16, 32)}:
            return 24
        if shape == (40, 40, 128, 128):
            return 33
        if shape == (20, 20, 256, 256):
            return 32
        if ic >= 32 and oc >= 64 and oh * ow >= 100:
            return 24
        return 0
    if sh != 1 or sw != 1 or ih != oh or iw != ow:
        return 0
    if shape in _STRIDE1_39:
        return 39
    if shape in _STRIDE1_40:
        return 40
    if shape == (10, 10, 512, 64):
        return 28
    if shape == (20, 20, 64, 128):
        return 25
    if oh == ow == 10 and oc == 64:
        return 2
    if ic >= 64 and oc >= 64 and oh * ow <= 400:
        table = {(20, 20, 128, 64): 12, (20, 20, 64, 64): 10, (10, 10, 256, 64): 13, (10, 10, 128, 128): 11,
                 (10, 10, 256, 256): 46}
        if shape in table:
            return table[shape]
        if oh == ow == 20 and ic % 32 == 0 and oc % 16 == 0:
            return 7
        if oh == ow == 10 and ic % 32 == 0 and oc % 16 == 0:
            return 8
        return 5
    return 3 if oc >= 4 and oh * ow >= 100 else 2


_NATIVE_FP16_1X1 = {(1, 40, 40, 64, 64), (1, 40, 40, 128, 64), (1, 40, 40, 128, 128), (1, 40, 40, 256, 64),
                    (1, 20, 20, 128, 128), (1, 20, 20, 128, 64), (1, 20, 20, 256, 128), (1, 20, 20, 256, 256),
                    (1, 20, 20, 384, 256), (1, 20, 20, 512, 128), (1, 10, 10, 512, 512), (1, 10, 10, 256, 256)}


def uses_native_fp16_conv1x1(params) -> bool:
    """engine.py:1610-1640."""
    if len(params) < 16:
        return False
    b, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, pt, pl, dh, dw, g = _p16(params)
    return (kh == kw == sh == sw == dh == dw == g == 1 and pt == pl == 0 and ih == oh and iw == ow
            and (b, oh, ow, ic, oc) in _NATIVE_FP16_1X1)


def uses_measured_native_fp16(params) -> bool:
    """engine.py:2035-2056 (native fp16 3x3 s2, kernel 43)."""
    if len(params) < 16:
        return False
    _, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, pt, pl, dh, dw, g = _p16(params)
    if (kh != 3 or kw != 3 or sh != 2 or sw != 2 or pt != 1 or pl != 1 or dh != 1 or dw != 1 or g != 1
            or ic < 32 or ic % 4 or oc % 4 or ih < oh * 2 - 1 or iw < ow * 2 - 1):
        return False
    return (oh == ow == 10) or (oh == ow == 20 and oc <= 128)


def uses_native_fp16_position_pair_40x40_256x256(params) -> bool:
    """engine.py:2059-2079."""
    return len(params) >= 16 and _p16(params) == (1, 256, 40, 40, 256, 20, 20, 3, 3, 2, 2, 1, 1, 1, 1, 1)


def uses_native_fp16_pos2_40x40_64x64(params) -> bool:
    """engine.py:2082-2097."""
    if len(params) < 16:
        return False
    b, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, pt, pl, dh, dw, g = _p16(params)
    return (b >= 1 and (ic, ih, iw, oc, oh, ow) == (64, 40, 40, 64, 40, 40) and kh == kw == 3 and sh == sw == 1
            and pt == pl == 1 and dh == dw == 1 and g == 1)


_NATIVE_FP16_CONCAT_CONV1X1 = {
    (1, 80, 80, 64, 64, 1, (32, 32)), (1, 40, 40, 128, 128, 1, (64, 64)), (1, 40, 40, 512, 128, 1, (256, 256)),
    (1, 40, 40, 192, 128, 1, (64, 64, 64)), (1, 20, 20, 128, 128, 1, (64, 64)),
    (1, 20, 20, 256, 128, 1, (64, 64, 64, 64)), (1, 20, 20, 384, 256, 1, (128, 128, 128)),
    (1, 10, 10, 384, 256, 1, (128, 128, 128)),
}


def uses_native_fp16_concat_conv1x1(cmd) -> bool:
    """engine.py:1643-1670: the measured shapes of the native fp16 concat + 1x1 kernel."""
    k = len(cmd["inputs"]) - 2
    p = [int(v) for v in cmd["params"]]
    if k <= 0 or k > 8 or len(p) < 5 + k:
        return False
    ch = tuple(p[5:5 + k])
    return (p[0], p[1], p[2], sum(ch), p[3], p[4], ch) in _NATIVE_FP16_CONCAT_CONV1X1


def build_kernel_plan(replay: Dict[str, Any], precision: int) -> List[Dict[str, int]]:
    plans = []
    for index, cmd in enumerate(replay["commands"]):
        kind = cmd["kind"]
        kernel = 0
        packed_value = NO_VALUE
        winograd = False
        if kind in ("CONV", "CONV_SILU"):
            params = cmd["params"]
            kernel = stable_conv_algorithm(params, silu=kind == "CONV_SILU")
            winograd = precision == PRECISION_FLOAT16 and kernel in WINOGRAD_KERNELS and uses_native_fp16_winograd(params)
            if precision == PRECISION_FLOAT16 and uses_native_fp16_conv1x1(params):
                kernel = 45
            elif precision == PRECISION_FLOAT16 and kind == "CONV_SILU":
                if uses_native_fp16_position_pair_40x40_256x256(params):
                    kernel = 47
                elif uses_native_fp16_pos2_40x40_64x64(params):
                    kernel = 44
                elif uses_measured_native_fp16(params):
                    kernel = 43
            if len(cmd["inputs"]) >= 2 and (kernel in (32, 33, 34, 39, 43, 44, 45, 47) or winograd):
                packed_value = int(cmd["inputs"][1])
        elif kind == "CONCAT_CONV1X1":
            # engine.py:1080-1089: 3 = native fp16 (layout-4 weight), else 1 / 0
            p = cmd["params"]
            total_in = sum(int(v) for v in p[5:5 + max(0, len(cmd["inputs"]) - 2)])
            oc, spatial = int(p[3]), int(p[1]) * int(p[2])
            if precision == PRECISION_FLOAT16 and uses_native_fp16_concat_conv1x1(cmd):
                kernel = 3
                packed_value = int(cmd["inputs"][-2])
            else:
                kernel = 1 if total_in >= 64 and oc >= 64 and oc % 4 == 0 and spatial >= 100 else 0
        heavy = kind in ("CONV", "CONV_SILU", "CONCAT_CONV1X1", "MATMUL")
        flags = PLAN_FLAG_AUTHORITATIVE
        native_fp16 = (kind in ("CONV", "CONV_SILU") and (kernel in (43, 44, 45, 47) or winograd)) or (
            kind == "CONCAT_CONV1X1" and kernel == 3)
        if precision == PRECISION_FLOAT16 and (not heavy or native_fp16):
            flags |= PLAN_FLAG_DXIL
        plans.append(dict(command_index=index, kind_id=int(cmd["kind_id"]), planned_kernel=kernel,
                          precision=precision if heavy else PRECISION_FLOAT32, packed_value=packed_value,
                          flags=flags))
    return plans


def apply_algo_overrides(replay: Dict[str, Any], plans: List[Dict[str, int]], overrides: Dict[int, int]) -> List[int]:
    """Freezes per-command kernel choices (engine.py:1112-1222, no fusion groups here).

    Winograd targets are refused, as in the reference; packed kernels point
    packed_value at the raw weight; the DXIL bit follows the kernel family.
    Returns the indices that were skipped.
    """
    packed_kernels = {32, 33, 34, 39, 43, 44, 45, 47, 51, 52, 53, 54}
    skipped = []
    cmds = replay["commands"]
    for raw_index, kernel in dict(overrides).items():
        i, kernel = int(raw_index), int(kernel)
        if i < 0 or i >= len(plans):
            raise ValueError(f"algo override command index out of range: {i}")
        if cmds[i]["kind"] not in ("CONV", "CONV_SILU"):
            raise ValueError(f"algo override target is not a conv command: {i}")
        if kernel < 0 or kernel > 54:
            raise ValueError(f"algo override kernel id out of range: {kernel}")
        if kernel in WINOGRAD_KERNELS:
            skipped.append(i)
            continue
        rec = plans[i]
        prev = rec["planned_kernel"]
        rec["planned_kernel"] = kernel
        if kernel in packed_kernels and prev in packed_kernels:
            pass
        elif kernel in packed_kernels and len(cmds[i]["inputs"]) >= 2:
            rec["packed_value"] = int(cmds[i]["inputs"][1])
        else:
            rec["packed_value"] = NO_VALUE
        rec["flags"] = (rec["flags"] & ~PLAN_FLAG_DXIL) | PLAN_FLAG_AUTHORITATIVE
        if kernel in (43, 44, 45, 47, 51, 52, 53, 54):
            rec["flags"] |= PLAN_FLAG_DXIL
    return skipped


def int8_kernel_for(params) -> int:
    """51 / 52 / 53 by conv family (runtime enum RT:8935-8937)."""
    kh, sh = int(params[7]), int(params[9])
    if kh == 1:
        return 51
    return 53 if sh == 2 else 52


def int8_eligible(params) -> bool:
    """Reference eligibility (RT:9399-9422) plus in_channels % 16 == 0."""
    b, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, pt, pl, dh, dw, g = _p16(params)
    if g != 1 or ic % 16 or oc % 4:
        return False
    if kh == kw == 1:
        return sh == sw == 1 and pt == pl == 0 and dh == dw == 1 and oc % 8 == 0 and ih == oh and iw == ow
    if kh == kw == 3 and dh == dw == 1 and pt == pl == 1:
        if sh == sw == 2:
            return ih >= oh * 2 - 1 and iw >= ow * 2 - 1
        return sh == sw == 1 and ih == oh and iw == ow
    return False


def w8a8_algo_map(replay: Dict[str, Any], conv_names: Optional[Iterable[str]] = None) -> Dict[int, int]:
    """Algo map putting every eligible conv (or the named ones) on the int8 kernels."""
    wanted = None if conv_names is None else set(conv_names)
    names = replay.get("names")
    out = {}
    for i, cmd in enumerate(replay["commands"]):
        if cmd["kind"] not in ("CONV", "CONV_SILU") or not int8_eligible(cmd["params"]):
            continue
        if wanted is not None:
            wname = names[cmd["inputs"][1]] if names else ""
            if wname.rsplit(".w", 1)[0] not in wanted:
                continue
        out[i] = int8_kernel_for(cmd["params"])
    return out


# ---------------------------------------------------------------------------
# packed weights (engine.py:2099-2306)
# ---------------------------------------------------------------------------

def _weight_array(values, vid: int, shape) -> np.ndarray:
    return np.frombuffer(values[vid]["raw"], dtype="<f4").reshape(shape)


def build_packed_weights(replay: Dict[str, Any], plans: List[Dict[str, int]], precision: int) -> List[Dict[str, Any]]:
    values = replay["values"]
    packed: Dict[int, Dict[str, Any]] = {}

    def put(vid: int, layout: int, ic: int, oc: int, elements: int, data: bytes) -> None:
        prev = packed.get(vid)
        if prev is not None:
            if (prev["layout"], prev["in_channels"], prev["out_channels"]) != (layout, ic, oc):
                raise ValueError("weight already has an incompatible packed layout")
            return
        packed[vid] = dict(value_id=vid, layout=layout, in_channels=ic, out_channels=oc, elements=elements,
                           data=data)

    for cmd, plan in zip(replay["commands"], plans):
        if cmd["kind"] == "CONCAT_CONV1X1" and int(plan["planned_kernel"]) == 3:
            # engine.py:2157-2164: layout 4 over the concatenated input channels
            p = cmd["params"]
            ic = sum(int(v) for v in p[5:5 + len(cmd["inputs"]) - 2])
            oc = int(p[3])
            wid = int(cmd["inputs"][-2])
            w = _weight_array(values, wid, (oc, ic, 1, 1))
            put(wid, packing.PACKED_LAYOUT_CONV1X1_OC8_FP16, ic, oc, oc * ic, packing.pack_conv1x1_oc8_fp16(w))
            continue
        if cmd["kind"] not in ("CONV", "CONV_SILU"):
            continue
        p = cmd["params"]
        ic, oc, kh, kw = int(p[1]), int(p[4]), int(p[7]), int(p[8])
        wid = int(cmd["inputs"][1])
        kernel = int(plan["planned_kernel"])
        w = _weight_array(values, wid, (oc, ic, kh, kw))
        if kernel in INT8_KERNELS:
            put(wid, packing.PACKED_LAYOUT_CONV_INT8, ic, oc, oc * ic * kh * kw,
                packing.pack_conv_int8(w, fp16_engine=precision == PRECISION_FLOAT16))
            continue
        if precision == PRECISION_FLOAT16:
            if kernel == 45:
                put(wid, packing.PACKED_LAYOUT_CONV1X1_OC8_FP16, ic, oc, oc * ic, packing.pack_conv1x1_oc8_fp16(w))
            elif kernel == 40 and plan["flags"] & PLAN_FLAG_DXIL:
                put(wid, packing.PACKED_LAYOUT_WINOGRAD_F2X2_FP16, ic, oc, oc * ic * 16,
                    packing.pack_winograd_f2x2_fp16(w))
            elif kernel == 46 and plan["flags"] & PLAN_FLAG_DXIL:
                put(wid, packing.PACKED_LAYOUT_WINOGRAD_F2X2_FP32, ic, oc, oc * ic * 16,
                    packing.pack_winograd_f2x2_fp32(w))
        g = int(p[15])
        if kh != 3 or kw != 3 or not (int(p[9]) == 2 and int(p[10]) == 2 or kernel in (39, 44)) or g != 1 or oc % 4:
            continue
        if wid in packed:
            continue
        if precision == PRECISION_FLOAT16:
            put(wid, packing.PACKED_LAYOUT_CONV3X3_OC4_FP16, ic, oc, oc * ic * 9, packing.pack_conv3x3_oc4_fp16(w))
        else:
            arr = w.reshape(oc // 4, 4, ic, 9).transpose(0, 2, 3, 1).astype("<f4")
            put(wid, packing.PACKED_LAYOUT_CONV3X3_OC4, ic, oc, oc * ic * 9, arr.tobytes())
    return [packed[k] for k in sorted(packed)]


# ---------------------------------------------------------------------------
# memory plan (section 7)
# ---------------------------------------------------------------------------

def _align(v: int, a: int) -> int:
    return -(-int(v) // a) * a


STORAGE_DTYPE_FP32 = 1
STORAGE_LAYOUT_LINEAR_NCHW = 1
MEMORY_PLAN_V2 = 2
ARENA_ALIGNMENT = 256


def plan_memory(replay: Dict[str, Any], alignment: int = ARENA_ALIGNMENT) -> Dict[str, Any]:
    """Arena placement described by the Memory Plan V2 section (docs/AEXRT_ENGINE.md:234-308; the
    loader's checks RT:17891-17962).

    Every non-constant value lives in fp32 linear-NCHW storage, the reference runtime's default
    activation format (fp16 islands are a measured option there, ENG:211-246).  The placement
    is this compiler's own:

    * VIEW / ALIAS outputs take no storage of their own: they resolve to the allocation of their
      source at the element offset in params[0] (nested views add up);
    * pages are colours: the output of a command never shares a page with one of its inputs
      (a D3D12 resource cannot be read and written by one dispatch), colours chosen greedily
      in command order, smallest first;
    * within a page, a value takes the lowest-offset slot whose previous occupant was last read
      by an earlier command than the one that writes it (strictly earlier, so no command reads
      and writes one slot), else a new slot at the end; the graph output is held to the end.

    The alignment is halved until every alias offset is a multiple of it.
    Returns {alignment, pages: [nbytes], records: {value_id: (flags, page, offset, nbytes)},
    total_nbytes}.
    """
    values, commands = replay["values"], replay["commands"]
    n = len(values)
    root = list(range(n))
    elem_offset = [0] * n
    for c in commands:
        if c["kind"] in ("VIEW", "ALIAS"):
            src = int(c["inputs"][0])
            out = int(c["output"])
            root[out] = root[src]
            elem_offset[out] = elem_offset[src] + int(c["params"][0])
    is_const = [bool(v["flags"] & VALUE_CONSTANT) for v in values]
    aliased = [i for i in range(n) if root[i] != i]
    while alignment > 4 and any((elem_offset[i] * 4) % alignment for i in aliased):
        alignment //= 2

    born: Dict[int, int] = {}
    last_read: Dict[int, int] = {}
    for v in values:
        if v["flags"] & VALUE_INPUT:
            born[int(v["id"])] = -1
    for step, c in enumerate(commands):
        for i in c["inputs"]:
            if not is_const[int(i)]:
                r = root[int(i)]
                last_read[r] = max(last_read.get(r, -1), step)
        out = int(c["output"])
        if root[out] == out:
            born.setdefault(out, step)
    out_root = root[int(replay["output_value"])]
    last_read[out_root] = len(commands)

    colour: Dict[int, int] = {}
    for r, step in born.items():
        if step < 0:
            colour[r] = 0
    for c in commands:
        out = int(c["output"])
        if root[out] != out or out in colour:
            continue
        taken = {colour[root[int(i)]] for i in c["inputs"] if not is_const[int(i)] and root[int(i)] in colour}
        colour[out] = next(k for k in range(len(taken) + 1) if k not in taken)
    page_ids = {k: p for p, k in enumerate(sorted(set(colour.values())))}
    if len(page_ids) > 64:
        raise ValueError("memory plan needs more than the loader's 64 pages")

    slots: Dict[int, List[List[int]]] = {p: [] for p in page_ids.values()}  # [offset, size, free_after]
    place: Dict[int, tuple] = {}
    for r in sorted(born, key=lambda v: (born[v], v)):
        page = page_ids[colour[r]]
        nbytes = int(values[r]["elements"]) * 4
        start, end = born[r], last_read.get(r, born[r])
        size = _align(nbytes, alignment)
        chosen = None
        for slot in sorted(slots[page]):
            if slot[2] < start and slot[1] >= size:
                chosen = slot
                break
        if chosen is None:
            top = max((s[0] + s[1] for s in slots[page]), default=0)
            chosen = [top, size, end]
            slots[page].append(chosen)
        chosen[2] = end
        place[r] = (page, chosen[0])
    pages = [0] * len(page_ids)
    for p, ss in slots.items():
        pages[p] = max(s[0] + s[1] for s in ss)

    records: Dict[int, tuple] = {}
    for i in range(n):
        if is_const[i] or root[i] not in place:
            continue
        page, base = place[root[i]]
        flags = int(values[i]["flags"]) | VALUE_ARENA | (VALUE_ALIAS if root[i] != i else 0)
        records[i] = (flags, page, base + elem_offset[i] * 4, int(values[i]["elements"]) * 4)
    return dict(alignment=alignment, pages=pages, records=records, total_nbytes=sum(pages))


# ---------------------------------------------------------------------------
# sections and container
# ---------------------------------------------------------------------------
#
# Every section is a fixed header, then records; constants and packed
# weights end in a heap of 64-byte aligned payloads addressed by
# section-relative offsets (docs/AEXRT_ENGINE.md:54-233).  _Section does the
# layout for all of them; the functions below only list the fields.

class _Section:
    """One section payload: header fields, fixed- or variable-size records, then an optional
    payload heap (each payload 64-byte aligned, its offset patched into its record)."""

    def __init__(self, header_fmt: str, *header: Any) -> None:
        self.head = struct.pack(header_fmt, *header)
        self.records: List[tuple] = []   # (record_fmt, fields, payload or None, offset field index)

    def record(self, fmt: str, *fields: Any, payload: Optional[bytes] = None, at: int = -1) -> None:
        self.records.append((fmt, list(fields), payload, at))

    def raw(self, data: bytes) -> None:
        self.records.append((None, [data], None, -1))

    def tobytes(self) -> bytes:
        fixed = len(self.head) + sum(struct.calcsize(f) if f else len(v[0]) for f, v, _, _ in self.records)
        heap = bytearray()
        heap_base = _align(fixed, ENGINE_ALIGNMENT) if any(p is not None for *_, p, _ in self.records) else fixed
        chunks = [self.head]
        for fmt, fields, payload, at in self.records:
            if fmt is None:
                chunks.append(fields[0])
                continue
            if payload is not None:
                heap.extend(bytes(_align(len(heap), ENGINE_ALIGNMENT) - len(heap)))
                fields[at] = heap_base + len(heap)
                heap.extend(payload)
            chunks.append(struct.pack(fmt, *fields))
        chunks.append(bytes(heap_base - fixed))
        chunks.append(bytes(heap))
        return b"".join(chunks)


MANIFEST_U32_FIELDS = (
    "manifest_version", "runtime_target", "precision", "mode", "layout", "has_objectness", "channels", "anchors",
    "classes", "max_candidates", "max_detections", "graph_node_count", "value_count", "constant_count",
    "command_count", "input_value", "output_value")


def encode_manifest(**f: Any) -> bytes:
    """Section 1 (docs/AEXRT_ENGINE.md:106-125): 17 u32, input_elements, arena_nbytes, thresholds, digest."""
    f = dict(f, manifest_version=1, runtime_target=1, mode=2)
    s = _Section("<17I", *(int(f[k]) for k in MANIFEST_U32_FIELDS))
    s.record("<QQff32s", f["input_elements"], f["arena_nbytes"], f["conf_threshold"], f["iou_threshold"],
             bytes(f["source_hash"]))
    return s.tobytes()


def encode_values(replay: Dict[str, Any], memory: Optional[Dict[str, Any]] = None) -> bytes:
    """Section 2: <IIQ4IQQ> per value; arena values carry their memory-plan offset and size."""
    recs = (memory or {}).get("records", {})
    s = _Section("<II", len(replay["values"]), 0)
    for v in replay["values"]:
        flags, _, offset, nbytes = recs.get(int(v["id"]), (int(v["flags"]), 0, NO_OFFSET, 0))
        s.record("<IIQ4IQQ", v["id"], flags, v["elements"], *v["shape4"], offset, nbytes)
    return s.tobytes()


def encode_commands(replay: Dict[str, Any], plans: List[Dict[str, int]]) -> bytes:
    """Section 3: <6I> head (kind, output, #inputs, #params, kernel, precision), then the u32 lists."""
    s = _Section("<II", len(replay["commands"]), 0)
    for c, p in zip(replay["commands"], plans):
        words = [c["kind_id"], c["output"], len(c["inputs"]), len(c["params"]), p["planned_kernel"],
                 p["precision"], *c["inputs"], *c["params"]]
        s.raw(np.asarray(words, dtype="<u4").tobytes())
    return s.tobytes()


def fp16_constant_ids(replay: Dict[str, Any], precision: int) -> set:
    """Constants an fp16 engine stores as fp16: conv weights and biases (ENG:1299-1304)."""
    if precision != PRECISION_FLOAT16:
        return set()
    ids = set()
    for c in replay["commands"]:
        if c["kind"] in ("CONV", "CONV_SILU"):
            ids.update(int(v) for v in c["inputs"][1:3])
        elif c["kind"] == "CONCAT_CONV1X1":
            ids.update(int(v) for v in c["inputs"][-2:])
    return ids


def encode_constants(replay: Dict[str, Any], precision: int) -> bytes:
    """Section 4: <IIQQQ> (value, dtype, elements, offset, nbytes) per constant + payload heap."""
    half = fp16_constant_ids(replay, precision)
    consts = [v for v in replay["values"] if v["flags"] & VALUE_CONSTANT]
    s = _Section("<II", len(consts), 0)
    for v in consts:
        data = np.frombuffer(v["raw"], dtype="<f4")
        dtype = PRECISION_FLOAT16 if v["id"] in half else PRECISION_FLOAT32
        payload = (data.astype("<f2") if dtype == PRECISION_FLOAT16 else data).tobytes()
        s.record("<IIQQQ", v["id"], dtype, v["elements"], 0, len(payload), payload=payload, at=3)
    return s.tobytes()


def encode_kernel_plan(plans: List[Dict[str, int]]) -> bytes:
    """Section 5: count, plan version 1, then <6I> per command (ENG:2650-2663 record fields)."""
    s = _Section("<II", len(plans), 1)
    for p in plans:
        s.record("<6I", *(p[k] for k in ("command_index", "kind_id", "planned_kernel", "precision",
                                          "packed_value", "flags")))
    return s.tobytes()


def encode_packed_weights(packed: List[Dict[str, Any]]) -> bytes:
    """Section 6: <4IQQQ> (value, layout, ic, oc, elements, offset, nbytes) per weight + heap."""
    s = _Section("<II", len(packed), 0)
    for w in packed:
        s.record("<4IQQQ", w["value_id"], w["layout"], w["in_channels"], w["out_channels"], w["elements"], 0,
                 len(w["data"]), payload=w["data"], at=5)
    return s.tobytes()


def encode_memory_plan(memory: Dict[str, Any]) -> bytes:
    """Section 7, Memory Plan V2: <4IQII> header, <4IQ> per page, <6IQQ> per arena value."""
    recs = memory["records"]
    s = _Section("<4IQII", MEMORY_PLAN_V2, memory["alignment"], len(memory["pages"]), len(recs),
                 memory["total_nbytes"], 1, 0)
    for page, nbytes in enumerate(memory["pages"]):
        s.record("<4IQ", page, STORAGE_DTYPE_FP32, STORAGE_LAYOUT_LINEAR_NCHW, 1, nbytes)
    for vid in sorted(recs):
        flags, page, offset, nbytes = recs[vid]
        s.record("<6IQQ", vid, flags, page, STORAGE_DTYPE_FP32, STORAGE_LAYOUT_LINEAR_NCHW, 0, offset, nbytes)
    return s.tobytes()


def encode_fusion_plan(command_count: int) -> bytes:
    """Section 8: version 1, no groups, authoritative (docs/AEXRT_ENGINE.md:321-360).  Concat +
    1x1 fusion is a command kind (CONCAT_CONV1X1) here, not a group."""
    return _Section("<4I", 1, 0, command_count, 1).tobytes()


def encode_pipeline_cache() -> bytes:
    """Section 9: version 1 and no shader or PSO records, the valid empty cache of
    ``--no-pipeline-cache`` (docs/AEXRT_ENGINE.md:514-538).  HIP code objects live in the library."""
    return _Section("<4I", 1, 0, 0, 0).tobytes()


HEADER_FMT = "<8sIIIIQQQ16s"
TOC_FMT = "<IIQQII"
ENGINE_FLAG_VALID = 1


def build_container(sections: Dict[int, bytes]) -> bytes:
    """Header, TOC, then each section 64-byte aligned in type order, CRC32 per section."""
    items = sorted(sections.items())
    toc_bytes = ENGINE_TOC_ENTRY_SIZE * len(items)
    placed = []
    pos = ENGINE_HEADER_SIZE + toc_bytes
    for stype, payload in items:
        pos = _align(pos, ENGINE_ALIGNMENT)
        placed.append((stype, pos, payload))
        pos += len(payload)
    chunks = [struct.pack(HEADER_FMT, ENGINE_MAGIC, ENGINE_VERSION, ENGINE_HEADER_SIZE, len(items),
                          ENGINE_FLAG_VALID, pos, ENGINE_HEADER_SIZE, toc_bytes, bytes(16))]
    chunks += [struct.pack(TOC_FMT, t, 0, off, len(p), zlib.crc32(p) & 0xFFFFFFFF, 0) for t, off, p in placed]
    at = ENGINE_HEADER_SIZE + toc_bytes
    for _, off, p in placed:
        chunks += [bytes(off - at), p]
        at = off + len(p)
    return b"".join(chunks)


def _source_hash(replay: Dict[str, Any]) -> bytes:
    d = hashlib.sha256()
    for v in replay["values"]:
        d.update(struct.pack("<IQ", v["id"], v["elements"]))
        d.update(v["raw"])
    for c in replay["commands"]:
        d.update(c["kind"].encode("ascii"))
        d.update(struct.pack("<I", c["output"]))
    return d.digest()


def _precision_id(precision: str) -> int:
    p = str(precision).lower()
    if p in ("fp16", "float16", "half"):
        return PRECISION_FLOAT16
    if p in ("fp32", "float32", "float"):
        return PRECISION_FLOAT32
    raise ValueError(f"unsupported precision {precision}")


def compile_plan(graph: Graph, *, precision: str = "fp16", algo_overrides: Optional[Dict[int, int]] = None,
                 int8_pergroup: Optional[Sequence[int]] = None,
                 fuse_concat_min_h: Optional[int] = None) -> Dict[str, Any]:
    """Lowering + kernel plan + packed weights (everything but the bytes)."""
    prec = _precision_id(precision)
    replay = lower_graph(graph, fuse_concat_min_h=fuse_concat_min_h)
    plans = build_kernel_plan(replay, prec)
    if algo_overrides:
        apply_algo_overrides(replay, plans, algo_overrides)
    if int8_pergroup:
        pg = {int(i) for i in int8_pergroup}
        for p in plans:
            if p["command_index"] in pg and p["planned_kernel"] in INT8_KERNELS:
                p["flags"] |= PLAN_FLAG_INT8_PERGROUP
    packed = build_packed_weights(replay, plans, prec)
    return dict(replay=replay, plans=plans, packed=packed, precision=prec)


def engine_sections(graph: Graph, *, precision: str = "fp16", classes: Optional[int] = None,
                       algo_overrides: Optional[Dict[int, int]] = None,
                       int8_pergroup: Optional[Sequence[int]] = None, max_candidates: int = 512,
                       max_detections: int = 100, conf_threshold: float = 0.25,
                       iou_threshold: float = 0.45, fuse_concat_min_h: Optional[int] = None) -> Dict[int, bytes]:
    """Payloads of sections 1-9 by section type (what build_container lays out)."""
    plan = compile_plan(graph, precision=precision, algo_overrides=algo_overrides, int8_pergroup=int8_pergroup,
                        fuse_concat_min_h=fuse_concat_min_h)
    replay, plans, packed, prec = plan["replay"], plan["plans"], plan["packed"], plan["precision"]
    out_v = replay["values"][replay["output_value"]]
    out_shape = [d for d in out_v["shape4"]]
    rank = out_v["rank"]
    channels = int(out_shape[-2]) if rank == 3 else int(out_shape[1])
    anchors = int(out_shape[-1]) if rank == 3 else int(out_shape[2] * out_shape[3])
    ncls = int(classes) if classes is not None else max(channels - 64, 1)
    memory = plan_memory(replay)
    sections = {
        SECTION_VALUES: encode_values(replay, memory),
        SECTION_COMMANDS: encode_commands(replay, plans),
        SECTION_CONSTANTS: encode_constants(replay, prec),
        SECTION_KERNEL_PLAN: encode_kernel_plan(plans),
        SECTION_PACKED_WEIGHTS: encode_packed_weights(packed),
        SECTION_MEMORY_PLAN: encode_memory_plan(memory),
        SECTION_FUSION_PLAN: encode_fusion_plan(len(replay["commands"])),
        SECTION_PIPELINE_CACHE: encode_pipeline_cache(),
    }
    sections[SECTION_MANIFEST] = encode_manifest(
        precision=prec, layout=1, has_objectness=False, channels=channels, anchors=anchors, classes=ncls,
        max_candidates=max_candidates, max_detections=max_detections, graph_node_count=len(graph.nodes),
        value_count=len(replay["values"]),
        constant_count=sum(bool(v["flags"] & VALUE_CONSTANT) for v in replay["values"]),
        command_count=len(replay["commands"]), input_value=replay["input_value"],
        output_value=replay["output_value"], input_elements=replay["values"][replay["input_value"]]["elements"],
        arena_nbytes=memory["total_nbytes"], conf_threshold=conf_threshold, iou_threshold=iou_threshold,
        source_hash=_source_hash(replay))
    return sections


def build_aexrt_engine(graph: Graph, **kwargs: Any) -> bytes:
    """The .aexrt bytes of a graph (keyword arguments of engine_sections)."""
    return build_container(engine_sections(graph, **kwargs))


def save_aexrt_engine(graph: Graph, path, **kwargs) -> Dict[str, Any]:
    p = Path(path)
    if p.suffix.lower() != ".aexrt":
        raise ValueError("AEXRT engine output must use the .aexrt extension")
    data = build_aexrt_engine(graph, **kwargs)
    p.parent.mkdir(parents=True, exist_ok=True)
    p.write_bytes(data)
    return inspect_aexrt_engine(data)


def inspect_aexrt_engine(source) -> Dict[str, Any]:
    """Header, TOC (CRC, duplicates, reserved fields, sections 1-9 present), manifest, kernel plan,
    packed-layout counts, memory plan, fusion groups and pipeline-cache records; raises ValueError
    on an engine the reference's inspector refuses (ENG:336-400)."""
    data = bytes(source) if not isinstance(source, (str, os.PathLike)) else Path(source).read_bytes()
    if len(data) < ENGINE_HEADER_SIZE:
        raise ValueError("truncated AEXRT engine header")
    magic, version, hsize, count, flags, fsize, toc_off, toc_size, _ = struct.unpack_from(HEADER_FMT, data, 0)
    if magic != ENGINE_MAGIC or version != ENGINE_VERSION or hsize != ENGINE_HEADER_SIZE:
        raise ValueError("not an AEXRT engine")
    if fsize != len(data) or toc_size != count * ENGINE_TOC_ENTRY_SIZE or toc_off + toc_size > len(data):
        raise ValueError("AEXRT engine size mismatch")
    sections: Dict[int, Dict[str, int]] = {}
    for i in range(count):
        stype, sflags, off, size, crc, reserved = struct.unpack_from(TOC_FMT, data, toc_off + i * ENGINE_TOC_ENTRY_SIZE)
        if reserved or off + size > len(data):
            raise ValueError("invalid AEXRT section entry")
        if stype in sections:
            raise ValueError(f"duplicate AEXRT section {stype}")
        if zlib.crc32(data[off:off + size]) & 0xFFFFFFFF != crc:
            raise ValueError(f"AEXRT section {stype} checksum mismatch")
        sections[stype] = dict(offset=off, size=size, crc32=crc, flags=sflags)
    missing = [t for t in REQUIRED_SECTIONS if t not in sections]
    if missing:
        raise ValueError(f"AEXRT engine lacks sections {missing}")

    def body(t: int) -> bytes:
        s = sections[t]
        return data[s["offset"]:s["offset"] + s["size"]]

    info: Dict[str, Any] = dict(version=version, flags=flags, sections=sections, file_size=fsize)
    head = struct.unpack_from("<17I", body(SECTION_MANIFEST))
    info["manifest"] = {k: head[i] for i, k in enumerate(MANIFEST_U32_FIELDS)}
    info["manifest"]["input_elements"], info["manifest"]["arena_nbytes"] = struct.unpack_from(
        "<QQ", body(SECTION_MANIFEST), 68)
    plan = body(SECTION_KERNEL_PLAN)
    n = struct.unpack_from("<I", plan)[0]
    info["kernel_plan"] = [struct.unpack_from("<6I", plan, 8 + 24 * i) for i in range(n)]
    if any(not r[5] & PLAN_FLAG_AUTHORITATIVE or r[5] & ~0x1F for r in info["kernel_plan"]):
        raise ValueError("invalid AEXRT kernel-plan flags")
    pw = body(SECTION_PACKED_WEIGHTS)
    layouts = [struct.unpack_from("<4IQQQ", pw, 8 + 40 * i)[1] for i in range(struct.unpack_from("<I", pw)[0])]
    info["packed_layout_counts"] = {k: layouts.count(k) for k in sorted(set(layouts))}
    mem = body(SECTION_MEMORY_PLAN)
    if struct.unpack_from("<I", mem)[0] == MEMORY_PLAN_V2:
        _, align, pages, nrec, total, mflags, mres = struct.unpack_from("<4IQII", mem)
        if mflags != 1 or mres or total != info["manifest"]["arena_nbytes"]:
            raise ValueError("invalid AEXRT V2 memory-plan header")
        page_bytes = [struct.unpack_from("<4IQ", mem, 32 + 24 * p)[4] for p in range(pages)]
        if sum(page_bytes) != total:
            raise ValueError("invalid AEXRT V2 memory-page total")
        info["memory_plan"] = dict(version=2, alignment=align, page_nbytes=page_bytes, value_records=nrec)
    else:
        info["memory_plan"] = dict(version=1)
    fusion = body(SECTION_FUSION_PLAN)
    fver, groups, fcmds, fflags = struct.unpack_from("<4I", fusion)
    if fver != 1 or fcmds != info["manifest"]["command_count"] or not fflags & 1:
        raise ValueError("invalid AEXRT fusion plan")
    info["fusion_groups"] = [struct.unpack_from("<8I", fusion, 16 + 32 * g) for g in range(groups)]
    cver, ndxil, npso, _ = struct.unpack_from("<4I", body(SECTION_PIPELINE_CACHE))
    if cver != 1:
        raise ValueError("invalid AEXRT pipeline cache")
    info["pipeline_cache_records"] = ndxil + npso
    return info
