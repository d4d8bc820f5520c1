"""CPU oracle for the AEXRT W8A8 convolution path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
(``aexrt_amd``) never imports it.

The arithmetic lives in ``aexrt_oracle.c`` (a C restatement of the
reference's shaders and CPU loops, built into ``liboracle.so`` by the
Makefile next to it); this module wraps it for numpy arrays in the
reference's NCHW layout.

Pinning status (what, besides retyping, holds each function in place):

* ``f32_to_f16``: every finite/inf/nan/subnormal boundary against
  ``numpy.float16`` (tests/test_oracle.py).
* ``amax`` / ``amax_slots``: brute force ``np.abs().max()`` per strip,
  including the reference's N>1 memory-strip grouping and the C%16 tail.
* ``quantize`` / ``quant_pack``: RNE ties at exact .5, +-amax -> +-127,
  amax == 0 -> zeros, byte layout of the NC/4HW4 pack against a numpy
  gather; ``amax/127`` vs ``127/amax`` planted-mistake check.
* ``weight_quant`` (layout 8): half-away rounding at exact .5 ties, the
  compiler's fp32 ``floor(|p| + 0.5)`` edge at |p| = 0.5 - 2^-25, zero rows
  (scale 1), clamp at +-127, fp16 pre-rounding, and a float64 closed form
  away from ties.
* ``conv_int8_acc``: int64 ``np.einsum`` over an explicit im2col.
* ``conv_int8_epilogue`` / ``conv_int8_pg`` / ``conv_int8_ksplit`` /
  ``conv_int8_dynamic``: the integer parts reduce to ``conv_int8_acc``
  (pg16 with one group == per-tensor; k-split sums == unsplit); the fp32
  epilogue is checked to 1e-6 against a float64 evaluation.  Bit patterns
  of the reference's fp32 epilogue depend on DXC/driver ``exp`` and
  contraction: parity unpinned beyond that tolerance.
* ``cpu_conv2d``: float64 direct convolution, and ``torch.nn.functional
  .conv2d`` on small cases.
* ``winograd_weight``: the reference's own known-answer test
  (tests/test_engine_fp16_winograd_plan.py:76-144) reproduced as golden
  vectors in tests/golden/winograd_f2x2_kat.npz.
* ``winograd_conv``: the Lavin-Gray identity -- equals direct convolution
  of the same (fp16-rounded) weights to fp32 rounding.
* ``maxpool`` / ``resize_nearest``: ``torch.nn.functional`` equivalents.
* ``quant_fused_pg16``: equals ``amax_slots`` + ``quant_pack(per_group)``
  at N = 1; at N > 1 every image is packed with image 0's group maxima
  (the reference's strip start has no image offset), checked as that
  composition.
* ``yolo_decode_nms_topk``: the reference's own known-answer vectors
  (tests/test_runtime.py:442-463 CPU path, 3412-3448 GPU path); the NMS
  invariants (kept same-class boxes overlap <= iou, every dropped box has
  an outranking overlap); equality with greedy NMS (the reference's CPU
  ``yolo_postprocess``) where no suppression chains exist, and a planted
  chain where the GPU's mark rule differs from greedy NMS.  The anchor-order
  append is one of the orders the reference's atomic counter can produce.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_int = ctypes.c_int


def build(force: bool = False) -> Path:
    """Compile liboracle.so with the Makefile beside this file."""
    src = _HERE / "aexrt_oracle.c"
    if force or not _LIB_PATH.exists() or _LIB_PATH.stat().st_mtime < src.stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(_HERE), "-B" if force else "liboracle.so"],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        build()
    L = ctypes.CDLL(str(_LIB_PATH))
    sig = {
        "or_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "or_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
        "or_round_f16_array": (None, [_f32p, _u64]),
        "or_amax_bits": (_u32, [_f32p, _u64]),
        "or_amax_slots": (None, [_f32p, _u32, _u32, _u32, _u32p]),
        "or_quantize": (None, [_f32p, _u64, ctypes.c_float, _i8p]),
        "or_quant_pack": (None, [_f32p, _u32, _u32, _u32, _u32p, _int, _u32p]),
        "or_quant_fused_pg16": (None, [_f32p, _u32, _u32, _u32, _u32p, _u32p]),
        "or_weight_quant": (None, [_f32p, _u32, _u32, _int, _i8p, _f32p]),
        "or_conv_int8_acc": (None, [_i8p, _i8p, _u32p, _i32p]),
        "or_conv_int8_acc_mt": (None, [_i8p, _i8p, _u32p, _i32p, _int]),
        "or_conv_int8_epilogue": (None, [_i32p, _u32, _u32, _u32, ctypes.c_float, _f32p, _f32p,
                                         _int, _f32p]),
        "or_conv_int8_pg": (None, [_u32p, _i8p, _u32p, _u32, _u32p, _f32p, _f32p, _int, _f32p]),
        "or_conv_int8_ksplit": (None, [_u32p, _i8p, _u32p, _u32, _u32p, _int, _u32, _f32p, _f32p,
                                       _int, _f32p]),
        "or_conv_int8_dynamic": (None, [_f32p, _i8p, _u32p, _u32, _f32p, _f32p, _int, _f32p]),
        "or_cpu_conv2d": (None, [_f32p, _f32p, _f32p, _f32p, _u32p, _int, _int]),
        "or_winograd_f2x2_weight": (None, [_f32p, _u32, _u32, _int, _f32p]),
        "or_winograd_f2x2_conv": (None, [_f32p, _f32p, _f32p, _u32p, _f32p]),
        "or_maxpool": (None, [_f32p, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _f32p, _u32, _u32]),
        "or_resize_nearest": (None, [_f32p, _u32, _u32, _u32, _u32, _f32p, _u32, _u32]),
        "or_yolo_decode_nms_topk": (_u32, [_f32p, _u32, _u32, _u32, _u32, _u32, ctypes.c_float, ctypes.c_float,
                                           _u32, _u32, _f32p, _u32p, _f32p]),
        "or_yolo_dfl_decode_nms_topk": (_u32, [_f32p, _u32, _u32, _u32p, _f32p, _u32, ctypes.c_float,
                                               ctypes.c_float, _u32, _u32, _f32p, _u32p, _f32p]),
        "or_post_exp": (ctypes.c_float, [ctypes.c_float]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def conv_desc(batch, in_c, in_h, in_w, out_c, k, stride, pad, dilation=1, groups=1) -> np.ndarray:
    """16-u32 conv descriptor in the reference's order (yolo.py:929-939)."""
    out_h = (in_h + 2 * pad - dilation * (k - 1) - 1) // stride + 1
    out_w = (in_w + 2 * pad - dilation * (k - 1) - 1) // stride + 1
    return np.array([batch, in_c, in_h, in_w, out_c, out_h, out_w, k, k, stride, stride,
                     pad, pad, dilation, dilation, groups], dtype=np.uint32)


def out_shape(desc) -> tuple[int, int, int, int]:
    d = [int(v) for v in desc]
    return (d[0], d[4], d[5], d[6])


def conv_family(desc) -> int:
    """Reference int8 family id: 1 (1x1), 3 (3x3 s1), 32 (3x3 s2)."""
    d = [int(v) for v in desc]
    if d[7] == 1:
        return 1
    return 32 if d[9] == 2 else 3


# --- fp16 -----------------------------------------------------------------

def round_f16(x) -> np.ndarray:
    a = _f32(x).copy()
    lib().or_round_f16_array(a.reshape(-1), a.size)
    return a


def f32_to_f16_bits(x: float) -> int:
    return int(lib().or_f32_to_f16(float(x)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().or_f16_to_f32(int(h)))


# --- a1/a2/a3 --------------------------------------------------------------

def amax(x) -> float:
    a = _f32(x).reshape(-1)
    return float(np.uint32(lib().or_amax_bits(a, a.size)).view(np.float32))


def amax_slots(x) -> np.ndarray:
    a = _f32(x)
    n, c, h, w = a.shape
    out = np.zeros(c // 16 + 1, dtype=np.uint32)
    lib().or_amax_slots(a.reshape(-1), n, c, h * w, out)
    return out


def quantize(x, amax_value: float) -> np.ndarray:
    a = _f32(x)
    q = np.empty(a.shape, dtype=np.int8)
    lib().or_quantize(a.reshape(-1), a.size, float(amax_value), q.reshape(-1))
    return q


def quant_pack(x, slots, per_group: bool = False) -> np.ndarray:
    a = _f32(x)
    n, c, h, w = a.shape
    out = np.zeros(n * (c // 4) * h * w, dtype=np.uint32)
    lib().or_quant_pack(a.reshape(-1), n, c, h * w, np.ascontiguousarray(slots, np.uint32),
                        int(per_group), out)
    return out


def quant_fused_pg16(x) -> tuple[np.ndarray, np.ndarray]:
    a = _f32(x)
    n, c, h, w = a.shape
    packed = np.zeros(n * (c // 4) * h * w, dtype=np.uint32)
    slots = np.zeros(c // 16 + 1, dtype=np.uint32)
    lib().or_quant_fused_pg16(a.reshape(-1), n, c, h * w, packed, slots)
    return packed, slots


def unpack_nc4hw4(packed, n, c, h, w) -> np.ndarray:
    """NC/4HW4 uint32 pack -> int8 NCHW (byte j of word icg = channel 4icg+j)."""
    b = np.ascontiguousarray(packed, np.uint32).view(np.int8).reshape(n, c // 4, h * w, 4)
    return b.transpose(0, 1, 3, 2).reshape(n, c, h, w).copy()


# --- a4 -------------------------------------------------------------------

def weight_quant(w, fp16_round: bool = True) -> tuple[np.ndarray, np.ndarray]:
    a = _f32(w)
    oc = a.shape[0]
    per = a.size // oc if oc else 0
    q = np.empty(a.shape, dtype=np.int8)
    s = np.empty(oc, dtype=np.float32)
    lib().or_weight_quant(a.reshape(-1), oc, per, int(fp16_round), q.reshape(-1), s)
    return q, s


# --- a5..a9 ---------------------------------------------------------------

def conv_int8_acc(qa, qw, desc, threads: int = 1) -> np.ndarray:
    d = np.ascontiguousarray(desc, np.uint32)
    acc = np.empty(out_shape(d), dtype=np.int32)
    lib().or_conv_int8_acc_mt(np.ascontiguousarray(qa, np.int8).reshape(-1),
                              np.ascontiguousarray(qw, np.int8).reshape(-1), d, acc.reshape(-1), int(threads))
    return acc


def conv_int8_epilogue(acc, amax_value, w_scale, bias, silu: bool) -> np.ndarray:
    acc = np.ascontiguousarray(acc, np.int32)
    n, oc, h, w = acc.shape
    y = np.empty(acc.shape, dtype=np.float32)
    lib().or_conv_int8_epilogue(acc.reshape(-1), n, oc, h * w, float(amax_value), _f32(w_scale),
                                _f32(bias), int(silu), y.reshape(-1))
    return y


def conv_int8_pg(packed, qw, desc, slots, w_scale, bias, silu: bool) -> np.ndarray:
    d = np.ascontiguousarray(desc, np.uint32)
    y = np.empty(out_shape(d), dtype=np.float32)
    lib().or_conv_int8_pg(np.ascontiguousarray(packed, np.uint32),
                          np.ascontiguousarray(qw, np.int8).reshape(-1), d, conv_family(d),
                          np.ascontiguousarray(slots, np.uint32), _f32(w_scale), _f32(bias),
                          int(silu), y.reshape(-1))
    return y


def conv_int8_ksplit(packed, qw, desc, slots, w_scale, bias, silu: bool,
                     per_group: bool = False, k_splits: int = 4) -> np.ndarray:
    d = np.ascontiguousarray(desc, np.uint32)
    y = np.empty(out_shape(d), dtype=np.float32)
    lib().or_conv_int8_ksplit(np.ascontiguousarray(packed, np.uint32),
                              np.ascontiguousarray(qw, np.int8).reshape(-1), d, conv_family(d),
                              np.ascontiguousarray(slots, np.uint32), int(per_group), k_splits,
                              _f32(w_scale), _f32(bias), int(silu), y.reshape(-1))
    return y


def conv_int8_dynamic(x, qw, desc, w_scale, bias, silu: bool) -> np.ndarray:
    d = np.ascontiguousarray(desc, np.uint32)
    y = np.empty(out_shape(d), dtype=np.float32)
    lib().or_conv_int8_dynamic(_f32(x).reshape(-1), np.ascontiguousarray(qw, np.int8).reshape(-1),
                               d, conv_family(d), _f32(w_scale), _f32(bias), int(silu),
                               y.reshape(-1))
    return y


def w8a8_conv(x, w, bias, desc, silu: bool = True, fp16_engine: bool = True):
    """The whole per-tensor chain: amax -> quantize -> int32 conv -> dequant.

    Returns (amax, q_activation NCHW int8, q_weight, w_scale, acc int32,
    y fp32).  ``x`` is the activation as the consumer reads it (fp16-stored
    values widened to fp32).
    """
    x = _f32(x)
    a = amax(x)
    qa = quantize(x, a)
    qw, ws = weight_quant(w, fp16_round=fp16_engine)
    b = round_f16(bias) if fp16_engine else _f32(bias)
    acc = conv_int8_acc(qa, qw, desc)
    y = conv_int8_epilogue(acc, a, ws, b, silu)
    return a, qa, qw, ws, acc, y


# --- a12/a13/a15 ------------------------------------------------------------

def cpu_conv2d(x, w, b, desc, silu: bool, threads: int = 1) -> np.ndarray:
    d = np.ascontiguousarray(desc, np.uint32)
    y = np.empty(out_shape(d), dtype=np.float32)
    lib().or_cpu_conv2d(_f32(x).reshape(-1), _f32(w).reshape(-1), _f32(b), y.reshape(-1), d,
                        int(silu), int(threads))
    return y


def winograd_weight(w, to_f16: bool = True) -> np.ndarray:
    a = _f32(w)
    oc, ic = a.shape[:2]
    u = np.empty((oc, ic, 4, 4), dtype=np.float32)
    lib().or_winograd_f2x2_weight(a.reshape(-1), oc, ic, int(to_f16), u.reshape(-1))
    return u


def winograd_conv(x, u, bias, desc) -> np.ndarray:
    d = np.ascontiguousarray(desc, np.uint32)
    y = np.empty(out_shape(d), dtype=np.float32)
    lib().or_winograd_f2x2_conv(_f32(x).reshape(-1), _f32(u).reshape(-1), _f32(bias), d,
                                y.reshape(-1))
    return y


def maxpool(x, k: int, s: int, p: int) -> np.ndarray:
    a = _f32(x)
    n, c, h, w = a.shape
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    y = np.empty((n, c, oh, ow), dtype=np.float32)
    lib().or_maxpool(a.reshape(-1), n, c, h, w, k, s, p, y.reshape(-1), oh, ow)
    return y


def resize_nearest(x, oh: int, ow: int) -> np.ndarray:
    a = _f32(x)
    n, c, h, w = a.shape
    y = np.empty((n, c, oh, ow), dtype=np.float32)
    lib().or_resize_nearest(a.reshape(-1), n, c, h, w, y.reshape(-1), oh, ow)
    return y


# --- YOLO postprocess ---------------------------------------------------------

def yolo_decode_nms_topk(out, *, layout: int = 1, classes: int, has_objectness: bool = False,
                         conf: float = 0.25, iou: float = 0.45, max_candidates: int = 512,
                         max_detections: int = 100) -> np.ndarray:
    """The reference's GPU postprocess of one output0 image ([C, A], or [A, C] for layout 2):
    [count, 6] float32 rows x1, y1, x2, y2, score, class, best first."""
    a = _f32(out)
    if a.ndim == 3:
        a = a[0]
    channels, anchors = (a.shape[1], a.shape[0]) if layout == 2 else a.shape
    cand = np.zeros(max_candidates * 6, np.float32)
    keep = np.zeros(max_candidates, np.uint32)
    dets = np.zeros(max_detections * 6, np.float32)
    n = lib().or_yolo_decode_nms_topk(a.reshape(-1), layout, anchors, channels, classes, int(has_objectness),
                                      float(conf), float(iou), max_candidates, max_detections, cand, keep, dets)
    return dets.reshape(max_detections, 6)[:n].copy()


def post_exp(x: float) -> float:
    return float(lib().or_post_exp(float(x)))


def yolo_dfl_decode_nms_topk(head, levels, *, classes: int, layout: int = 1, conf: float = 0.25,
                             iou: float = 0.45, max_candidates: int = 512, max_detections: int = 100) -> np.ndarray:
    """Raw Detect head [64 + classes, A] (layout 2: [A, 64 + classes]) of one image, levels = [(h, w, stride)]:
    the reference's head decode + NMS + top-k, [count, 6] rows x1, y1, x2, y2, score, class."""
    a = _f32(head)
    if a.ndim == 3:
        a = a[0]
    hw = np.array([[h, w] for h, w, _ in levels], np.uint32).reshape(-1)
    st = np.array([s for _, _, s in levels], np.float32)
    cand = np.zeros(max_candidates * 6, np.float32)
    keep = np.zeros(max_candidates, np.uint32)
    dets = np.zeros(max_detections * 6, np.float32)
    n = lib().or_yolo_dfl_decode_nms_topk(a.reshape(-1), layout, len(levels), hw, st, classes, float(conf),
                                          float(iou), max_candidates, max_detections, cand, keep, dets)
    return dets.reshape(max_detections, 6)[:n].copy()
