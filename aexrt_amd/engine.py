"""Engine compiler: Graph -> replay commands -> kernel plan -> packed weights
-> ``.aexrt`` container (the reference's ``aexrtc build``, src/aexrt/engine.py).

What is kept byte-compatible with the reference, because it is the drop-in
surface:
  * the container: 64-byte header, 32-byte TOC entries, 64-byte aligned
    sections, CRC32 per section (engine.py:3952-3985);
  * sections 1-6: manifest (engine.py:2556-2580), values (2583-2598),
    commands (2601-2617), constants (2620-2647), kernel plan (2650-2662),
    packed weights (2665-2690);
  * command kinds and their u32 params (yolo.py:701-927), kernel ids
    (runtime enum RT:8881-8940), plan flags (engine.py:85-96), packed layouts
    2/3/4/5/8 (engine.py:59-71);
  * the kernel-plan rules (engine.py:1046-1109, 1945-2098), the algo-map
    override (engine.py:1112-1222) and the int8 per-group flag loop
    (engine.py:192-210).

What is not emitted: the D3D12 memory plan, barrier plan, fusion plan,
physical dispatch plan and pipeline cache (sections 7-12).  The HIP runtime
plans its own memory (one buffer per value, concat inputs placed as slices
of their concat) and runs every command as its own kernel.
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
# sections and container
# ---------------------------------------------------------------------------

def _align(v: int, a: int) -> int:
    return (int(v) + a - 1) // a * a


def encode_manifest(**f: Any) -> bytes:
    out = bytearray()
    for v in (1, 1, f["precision"], 2, f["layout"], int(f["has_objectness"]), f["channels"], f["anchors"],
              f["classes"], f["max_candidates"], f["max_detections"], f["graph_node_count"], f["value_count"],
              f["constant_count"], f["command_count"], f["input_value"], f["output_value"]):
        out += struct.pack("<I", int(v))
    out += struct.pack("<QQff", f["input_elements"], f["arena_nbytes"], f["conf_threshold"], f["iou_threshold"])
    out += bytes(f["source_hash"])
    return bytes(out)


def encode_values(replay: Dict[str, Any]) -> bytes:
    out = bytearray(struct.pack("<II", len(replay["values"]), 0))
    for v in replay["values"]:
        out += struct.pack("<IIQ4IQQ", v["id"], v["flags"], v["elements"], *v["shape4"], NO_OFFSET, 0)
    return bytes(out)


def encode_commands(replay: Dict[str, Any], plans: List[Dict[str, int]]) -> bytes:
    out = bytearray(struct.pack("<II", len(replay["commands"]), 0))
    for c, p in zip(replay["commands"], plans):
        out += struct.pack("<6I", c["kind_id"], c["output"], len(c["inputs"]), len(c["params"]),
                           p["planned_kernel"], p["precision"])
        if c["inputs"]:
            out += struct.pack(f"<{len(c['inputs'])}I", *c["inputs"])
        if c["params"]:
            out += struct.pack(f"<{len(c['params'])}I", *c["params"])
    return bytes(out)


def encode_constants(replay: Dict[str, Any], precision: int) -> bytes:
    consts = [v for v in replay["values"] if v["flags"] & VALUE_CONSTANT]
    fp16_ids = set()
    if precision == PRECISION_FLOAT16:
        for c in replay["commands"]:
            if c["kind"] in ("CONV", "CONV_SILU") and len(c["inputs"]) >= 3:
                fp16_ids.update(int(v) for v in c["inputs"][1:3])
            elif c["kind"] == "CONCAT_CONV1X1" and len(c["inputs"]) >= 2:
                fp16_ids.update(int(v) for v in c["inputs"][-2:])
    rec = 32
    data_offset = _align(8 + len(consts) * rec, ENGINE_ALIGNMENT)
    out = bytearray(data_offset)
    struct.pack_into("<II", out, 0, len(consts), 0)
    cursor = data_offset
    for i, v in enumerate(consts):
        cursor = _align(cursor, ENGINE_ALIGNMENT)
        if cursor > len(out):
            out.extend(b"\0" * (cursor - len(out)))
        raw = v["raw"]
        prec = PRECISION_FLOAT16 if v["id"] in fp16_ids else PRECISION_FLOAT32
        if prec == PRECISION_FLOAT16:
            raw = np.frombuffer(raw, dtype="<f4").astype("<f2").tobytes()
        struct.pack_into("<IIQQQ", out, 8 + i * rec, v["id"], prec, v["elements"], cursor, len(raw))
        out.extend(raw)
        cursor += len(raw)
    return bytes(out)


def encode_kernel_plan(plans: List[Dict[str, int]]) -> bytes:
    out = bytearray(struct.pack("<II", len(plans), 1))
    for p in plans:
        out += struct.pack("<6I", p["command_index"], p["kind_id"], p["planned_kernel"], p["precision"],
                           p["packed_value"], p["flags"])
    return bytes(out)


def encode_packed_weights(packed: List[Dict[str, Any]]) -> bytes:
    rec = 40
    data_offset = _align(8 + len(packed) * rec, ENGINE_ALIGNMENT)
    out = bytearray(data_offset)
    struct.pack_into("<II", out, 0, len(packed), 0)
    cursor = data_offset
    for i, item in enumerate(packed):
        cursor = _align(cursor, ENGINE_ALIGNMENT)
        if cursor > len(out):
            out.extend(b"\0" * (cursor - len(out)))
        data = item["data"]
        struct.pack_into("<4IQQQ", out, 8 + i * rec, item["value_id"], item["layout"], item["in_channels"],
                         item["out_channels"], item["elements"], cursor, len(data))
        out.extend(data)
        cursor += len(data)
    return bytes(out)


def build_container(sections: Dict[int, bytes]) -> bytes:
    ordered = sorted(sections.items())
    toc_offset = ENGINE_HEADER_SIZE
    toc_size = len(ordered) * ENGINE_TOC_ENTRY_SIZE
    cursor = _align(toc_offset + toc_size, ENGINE_ALIGNMENT)
    entries, payloads = [], []
    for stype, payload in ordered:
        cursor = _align(cursor, ENGINE_ALIGNMENT)
        entries.append((stype, 0, cursor, len(payload), zlib.crc32(payload) & 0xFFFFFFFF, 0))
        payloads.append((cursor, payload))
        cursor += len(payload)
    out = bytearray(cursor)
    struct.pack_into("<8sIIIIQQQ16s", out, 0, ENGINE_MAGIC, ENGINE_VERSION, ENGINE_HEADER_SIZE, len(entries), 1,
                     cursor, toc_offset, toc_size, b"\0" * 16)
    for i, e in enumerate(entries):
        struct.pack_into("<IIQQII", out, toc_offset + i * ENGINE_TOC_ENTRY_SIZE, *e)
    for off, payload in payloads:
        out[off:off + len(payload)] = payload
    return bytes(out)


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


def build_aexrt_engine(graph: Graph, *, precision: str = "fp16", classes: Optional[int] = None,
                       algo_overrides: Optional[Dict[int, int]] = None,
                       int8_pergroup: Optional[Sequence[int]] = None, max_candidates: int = 512,
                       max_detections: int = 100, conf_threshold: float = 0.25,
                       iou_threshold: float = 0.45, fuse_concat_min_h: Optional[int] = None) -> bytes:
    plan = compile_plan(graph, precision=precision, algo_overrides=algo_overrides, int8_pergroup=int8_pergroup,
                        fuse_concat_min_h=fuse_concat_min_h)
    replay, plans, packed, prec = plan["replay"], plan["plans"], plan["packed"], plan["precision"]
    out_v = replay["values"][replay["output_value"]]
    out_shape = [d for d in out_v["shape4"]]
    rank = out_v["rank"]
    channels = int(out_shape[-2]) if rank == 3 else int(out_shape[1])
    anchors = int(out_shape[-1]) if rank == 3 else int(out_shape[2] * out_shape[3])
    ncls = int(classes) if classes is not None else max(channels - 64, 1)
    sections = {
        SECTION_VALUES: encode_values(replay),
        SECTION_COMMANDS: encode_commands(replay, plans),
        SECTION_CONSTANTS: encode_constants(replay, prec),
        SECTION_KERNEL_PLAN: encode_kernel_plan(plans),
        SECTION_PACKED_WEIGHTS: encode_packed_weights(packed),
    }
    sections[SECTION_MANIFEST] = encode_manifest(
        precision=prec, layout=1, has_objectness=False, channels=channels, anchors=anchors, classes=ncls,
        max_candidates=max_candidates, max_detections=max_detections, graph_node_count=len(graph.nodes),
        value_count=len(replay["values"]),
        constant_count=sum(bool(v["flags"] & VALUE_CONSTANT) for v in replay["values"]),
        command_count=len(replay["commands"]), input_value=replay["input_value"],
        output_value=replay["output_value"], input_elements=replay["values"][replay["input_value"]]["elements"],
        arena_nbytes=0, conf_threshold=conf_threshold, iou_threshold=iou_threshold,
        source_hash=_source_hash(replay))
    return build_container(sections)


def save_aexrt_engine(graph: Graph, path, **kwargs) -> Dict[str, Any]:
    p = Path(path)
    if p.suffix.lower() != ".aexrt":
        raise ValueError("AEXRT engine output must use the .aexrt extension")
    data = build_aexrt_engine(graph, **kwargs)
    p.parent.mkdir(parents=True, exist_ok=True)
    p.write_bytes(data)
    return inspect_aexrt_engine(data)


def inspect_aexrt_engine(source) -> Dict[str, Any]:
    """Header, TOC (with CRC check), manifest, kernel plan and packed-layout counts."""
    data = bytes(source) if not isinstance(source, (str, os.PathLike)) else Path(source).read_bytes()
    if len(data) < ENGINE_HEADER_SIZE:
        raise ValueError("truncated AEXRT engine header")
    magic, version, hsize, count, flags, fsize, toc_off, toc_size, _ = struct.unpack_from("<8sIIIIQQQ16s", data, 0)
    if magic != ENGINE_MAGIC or version != ENGINE_VERSION or hsize != ENGINE_HEADER_SIZE:
        raise ValueError("not an AEXRT engine")
    if fsize != len(data) or toc_size != count * ENGINE_TOC_ENTRY_SIZE:
        raise ValueError("AEXRT engine size mismatch")
    sections = {}
    for i in range(count):
        stype, _, off, size, crc, _ = struct.unpack_from("<IIQQII", data, toc_off + i * ENGINE_TOC_ENTRY_SIZE)
        if off + size > len(data):
            raise ValueError("AEXRT section out of range")
        if zlib.crc32(data[off:off + size]) & 0xFFFFFFFF != crc:
            raise ValueError(f"AEXRT section {stype} checksum mismatch")
        sections[stype] = dict(offset=off, size=size, crc32=crc)
    info: Dict[str, Any] = dict(version=version, sections=sections, file_size=fsize)
    if SECTION_MANIFEST in sections:
        s = sections[SECTION_MANIFEST]
        ints = struct.unpack_from("<17I", data, s["offset"])
        info["manifest"] = dict(precision=ints[2], layout=ints[4], channels=ints[6], anchors=ints[7],
                                classes=ints[8], value_count=ints[12], constant_count=ints[13],
                                command_count=ints[14], input_value=ints[15], output_value=ints[16],
                                input_elements=struct.unpack_from("<Q", data, s["offset"] + 68)[0])
    if SECTION_KERNEL_PLAN in sections:
        s = sections[SECTION_KERNEL_PLAN]
        n, _ = struct.unpack_from("<II", data, s["offset"])
        info["kernel_plan"] = [struct.unpack_from("<6I", data, s["offset"] + 8 + 24 * i) for i in range(n)]
    if SECTION_PACKED_WEIGHTS in sections:
        s = sections[SECTION_PACKED_WEIGHTS]
        n, _ = struct.unpack_from("<II", data, s["offset"])
        counts: Dict[int, int] = {}
        for i in range(n):
            rec = struct.unpack_from("<4IQQQ", data, s["offset"] + 8 + 40 * i)
            counts[rec[1]] = counts.get(rec[1], 0) + 1
        info["packed_layout_counts"] = counts
    return info
