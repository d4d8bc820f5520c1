"""Host wrappers of the op-level C ABI (one function per hot-path kernel).

PyTorch tensors provide device memory and the stream; every computation runs
in libaexrt_hip.so.  Activation tensors are NHWC fp16 (``[N, H, W, C]``);
a channel slice ``t[..., c0:c1]`` is a valid view as long as ``c0`` is a
multiple of 8 (16 when the view carries amax slots).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _lib
from ._lib import ConvDesc, TensorView, check

SILU = 1
RESIDUAL = 2
OUT_F32 = 4
IN_NCHW_F32 = 8
INT8_PG16 = 16
INT8_DYNAMIC = 32

SRC_RAW_F32 = 0
SRC_RAW_F16 = 1
SRC_LAYOUT_OC4_F16 = 2
SRC_LAYOUT_WINO_F16 = 3
SRC_LAYOUT_OC8_F16 = 4
SRC_LAYOUT_WINO_F32 = 5
SRC_LAYOUT_INT8 = 8


def _stream(stream=None):
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(int(getattr(stream, "cuda_stream", stream) or 0))


def _ptr(t) -> Optional[int]:
    return None if t is None else int(t.data_ptr())


def view(t, slots=None) -> TensorView:
    """TensorView of an NHWC tensor (or channel slice) ``t`` of shape [N, H, W, C]."""
    if t.dim() != 4:
        raise ValueError("activation views are 4-D NHWC")
    if t.stride(3) != 1 or t.stride(1) != t.shape[2] * t.stride(2):
        raise ValueError("view must be NHWC with contiguous pixels (channel slices allowed)")
    stripes, stride = 0, 0
    if slots is not None and slots.dim() == 2:
        # striped slot array [stripes, groups]: producers spread their updates
        # over the rows, readers take the max over the rows
        if slots.stride(1) != 1:
            raise ValueError("slot rows must be contiguous")
        stripes, stride = slots.shape[0], slots.stride(0)
    return TensorView(data=t.data_ptr(), n_stride=t.stride(0), c_stride=t.stride(2), amax_stripes=stripes,
                      amax_slots=_ptr(slots), amax_stripe_stride=stride)


def new_slots(channels: int, device="cuda", stripes: int = 1):
    """Zeroed amax slots of a ``channels``-wide tensor: [groups], or [stripes, groups] when striped."""
    import torch

    g = (channels + 15) // 16
    shape = (g,) if stripes == 1 else (stripes, g)
    return torch.zeros(shape, dtype=torch.int32, device=device)


def slots_max(slots) -> np.ndarray:
    """Per-group slot bit patterns, max over the stripes of a striped slot array (host read)."""
    a = slots.detach().cpu().numpy().astype(np.int32).view(np.uint32)
    return a.max(axis=0) if a.ndim == 2 else a


def slots_amax(slots) -> float:
    """Per-tensor amax from a slot tensor (host read)."""
    a = slots_max(slots)
    return float(np.uint32(a.max() if a.size else 0).view(np.float32))


def amax_slots(x, slots, stream=None) -> None:
    n, h, w, c = x.shape
    v = view(x, slots)
    check(_lib.lib().aexrt_hip_amax_slots(ctypes.byref(v), n, h, w, c, _stream(stream)), "amax_slots")


def amax_nchw(x, stream=None):
    """Reference amax buffer (C/16 + 1 words) of an NCHW fp16/fp32 tensor."""
    import torch

    n, c, h, w = x.shape
    out = torch.empty(c // 16 + 1, dtype=torch.int32, device=x.device)
    check(_lib.lib().aexrt_hip_amax_nchw(x.data_ptr(), int(x.dtype == torch.float16), n, c, h * w,
                                          out.data_ptr(), _stream(stream)), "amax_nchw")
    return out


def quantize(x, slots, stream=None):
    import torch

    n, h, w, c = x.shape
    q = torch.empty((n, h, w, c), dtype=torch.int8, device=x.device)
    v = view(x, slots)
    check(_lib.lib().aexrt_hip_quantize(ctypes.byref(v), n, h, w, c, q.data_ptr(), _stream(stream)),
          "quantize")
    return q


def quant_pack_nchw(x, amax, per_group: bool = False, stream=None):
    import torch

    n, c, h, w = x.shape
    packed = torch.empty(n * (c // 4) * h * w, dtype=torch.int32, device=x.device)
    check(_lib.lib().aexrt_hip_quant_pack_nchw(x.data_ptr(), int(x.dtype == torch.float16), n, c, h * w,
                                                amax.data_ptr(), int(per_group), packed.data_ptr(),
                                                _stream(stream)), "quant_pack_nchw")
    return packed


def amax_strips_nhwc(x, stream=None):
    """pg16 group amax of an NHWC fp16 tensor: word s = the reference's amax[1 + s] (NCHW memory strip s)."""
    import torch

    n, h, w, c = x.shape
    out = torch.empty(c // 16, dtype=torch.int32, device=x.device)
    v = view(x)
    check(_lib.lib().aexrt_hip_amax_strips_nhwc(ctypes.byref(v), n, h, w, c, out.data_ptr(), _stream(stream)),
          "amax_strips_nhwc")
    return out


def quant_fused_pg16(x, stream=None):
    """The reference's fused pg16 amax + pack of an NCHW tensor: (packed words, amax buffer; amax[0] untouched = 0)."""
    import torch

    n, c, h, w = x.shape
    packed = torch.empty(n * (c // 4) * h * w, dtype=torch.int32, device=x.device)
    amax = torch.zeros(c // 16 + 1, dtype=torch.int32, device=x.device)
    check(_lib.lib().aexrt_hip_quant_fused_pg16(x.data_ptr(), int(x.dtype == torch.float16), n, c, h * w,
                                                 packed.data_ptr(), amax.data_ptr(), _stream(stream)),
          "quant_fused_pg16")
    return packed, amax


def conv2d_int8_pg16(pc: "PreparedConv", packed, amax, y, *, flags: int = SILU, stream=None) -> None:
    """pg16 conv on the reference's operands: packed NC/4HW4 words + amax buffer -> dense NCHW y."""
    d = ConvDesc.from_params(pc.params)
    check(_lib.lib().aexrt_hip_conv2d_int8_pg16(
        ctypes.byref(d), pc.algorithm, flags, packed.data_ptr(), amax.data_ptr(), pc.weight.data_ptr(),
        _ptr(pc.w_scale), pc.bias.data_ptr(), y.data_ptr(), _stream(stream)), "conv2d_int8_pg16")


def yolo_decode_nms_topk(out, *, classes: int, layout: int = 1, has_objectness: bool = False, conf: float = 0.25,
                         iou: float = 0.45, max_candidates: int = 512, max_detections: int = 100, stream=None):
    """YOLO postprocess of one output0 image on the device ([C, A] fp32, or [A, C] with layout 2).

    Returns the [count, 6] detections (x1, y1, x2, y2, score, class) as a device tensor."""
    import torch

    a = out[0] if out.dim() == 3 else out
    if a.dtype != torch.float32 or not a.is_contiguous():
        raise ValueError("output0 must be a contiguous fp32 tensor")
    channels, anchors = (a.shape[1], a.shape[0]) if layout == 2 else (a.shape[0], a.shape[1])
    dets = torch.zeros((max_detections, 6), dtype=torch.float32, device=a.device)
    count = torch.zeros(1, dtype=torch.int32, device=a.device)
    check(_lib.lib().aexrt_hip_yolo_decode_nms_topk(
        a.data_ptr(), layout, anchors, channels, classes, int(has_objectness), float(conf), float(iou),
        max_candidates, max_detections, dets.data_ptr(), count.data_ptr(), _stream(stream)), "yolo_decode_nms_topk")
    return dets[: int(count.item())]


def yolo_dfl_decode_nms_topk(head, levels, *, classes: int, layout: int = 1, conf: float = 0.25, iou: float = 0.45,
                             max_candidates: int = 512, max_detections: int = 100, stream=None):
    """YOLO postprocess of one raw Detect-head image on the device ([64 + classes, A] fp32, or [A, 64 + classes]
    with layout 2; levels = [(h, w, stride)]).  Returns the [count, 6] detections as a device tensor."""
    import torch

    a = head[0] if head.dim() == 3 else head
    if a.dtype != torch.float32 or not a.is_contiguous():
        raise ValueError("head must be a contiguous fp32 tensor")
    hw = (ctypes.c_uint32 * (2 * len(levels)))(*[int(v) for h, w, _ in levels for v in (h, w)])
    st = (ctypes.c_float * len(levels))(*[float(s) for _, _, s in levels])
    dets = torch.zeros((max_detections, 6), dtype=torch.float32, device=a.device)
    count = torch.zeros(1, dtype=torch.int32, device=a.device)
    check(_lib.lib().aexrt_hip_yolo_dfl_decode_nms_topk(
        a.data_ptr(), layout, len(levels), hw, st, classes, float(conf), float(iou), max_candidates, max_detections,
        dets.data_ptr(), count.data_ptr(), _stream(stream)), "yolo_dfl_decode_nms_topk")
    return dets[: int(count.item())]


def can_use_conv_int8(params: Sequence[int], kernel_elems: int) -> bool:
    d = ConvDesc.from_params(params)
    return bool(_lib.lib().aexrt_hip_can_use_conv_int8(ctypes.byref(d), kernel_elems))


def set_conv_tile(jn: int = 0, pw: int = 0, ksw: bool = False) -> None:
    """Force the igemm conv kernel's per-wave tile for later launches ((0, 0) = automatic)."""
    check(_lib.lib().aexrt_hip_set_conv_tile(jn, pw, 1 if ksw else 0), "set_conv_tile")


HALO_AUTO, HALO_OFF, HALO_FORCE, HALO_FORCE8, HALO_FORCE_WIDE, HALO_FORCE_M32, HALO_FORCE_M32_8 = 0, 1, 2, 3, 4, 5, 6
HALO_FORCE_M32_2G = 7


def set_conv3x3_halo(mode: int = HALO_AUTO, jn: int = 0, pw: int = 0, tr: int = 0, tc: int = 0, cc: int = 0) -> None:
    """Select the halo-tile kernel for 3x3 convs: automatic, off (implicit GEMM), or a forced tile
    (HALO_FORCE: 4 waves per block, HALO_FORCE8: 8 waves; HALO_FORCE_WIDE: the wide-tile fp16 kernel;
    HALO_FORCE_M32 / HALO_FORCE_M32_8: the 32x32-MFMA kernel with 4 / 8 waves per block (HALO_FORCE_M32_2G:
    8 waves in two groups of 4 with their own windows and barriers), jn 32-channel
    subtiles and pw 32-position subtiles)."""
    check(_lib.lib().aexrt_hip_set_conv3x3_halo(mode, jn, pw, tr, tc, cc), "set_conv3x3_halo")


STEM_AUTO, STEM_OFF, STEM_FORCE, STEM_FORCE_ONE = 0, 1, 2, 3


def set_conv_stem(mode: int = STEM_AUTO, tr: int = 0) -> None:
    """Select the kernel of the first conv on the fp32 NCHW input: automatic (band kernel when it
    fits), off (halo-tile kernel), or a forced band of ``tr`` output rows (STEM_FORCE: a grid of
    resident blocks walking runs of bands, STEM_FORCE_ONE: one band per block)."""
    check(_lib.lib().aexrt_hip_set_conv_stem(mode, tr), "set_conv_stem")


def set_conv1x1_stream(on: bool = False, jq: int = 0, pq: int = 0, one_tile: bool = False) -> None:
    """Force the streaming 1x1 int8 kernel (jq 16-channel subtiles per block, pq 16-position
    subtiles per wave; one_tile: a grid of one tile per block instead of a persistent one) onto
    every int8 1x1 conv launched without a measured choice; off restores the automatic choice."""
    mode = 0 if not on else (2 if one_tile else 1)
    check(_lib.lib().aexrt_hip_set_conv1x1_stream(mode, jq, pq), "set_conv1x1_stream")


def conv_weight_bytes(params: Sequence[int], algorithm: int) -> int:
    d = ConvDesc.from_params(params)
    n = ctypes.c_uint64()
    check(_lib.lib().aexrt_hip_conv_weight_bytes(ctypes.byref(d), algorithm, ctypes.byref(n)),
          "conv_weight_bytes")
    return int(n.value)


def pack_conv_weight(params: Sequence[int], algorithm: int, src_layout: int, src: bytes | np.ndarray):
    """Host repack of a weight payload; returns (packed bytes as uint8 array, scales or None)."""
    d = ConvDesc.from_params(params)
    raw = src.tobytes() if isinstance(src, np.ndarray) else bytes(src)
    nbytes = conv_weight_bytes(params, algorithm)
    out = np.zeros(nbytes, dtype=np.uint8)
    scales = np.zeros(d.out_channels, dtype=np.float32) if algorithm in (51, 52, 53) else None
    buf = ctypes.create_string_buffer(raw, len(raw))
    check(_lib.lib().aexrt_hip_pack_conv_weight(
        ctypes.byref(d), algorithm, src_layout, ctypes.cast(buf, ctypes.c_void_p), len(raw),
        out.ctypes.data, nbytes, None if scales is None else scales.ctypes.data), "pack_conv_weight")
    return out, scales


@dataclass
class PreparedConv:
    """Device-resident weights of one conv, ready for :func:`conv2d`."""

    params: list
    algorithm: int
    weight: object       # torch uint8 tensor (packed)
    w_scale: object      # torch float32 [OC] or None
    bias: object         # torch float32 [OC]


def prepare_conv(params, algorithm: int, src_layout: int, src, bias: np.ndarray, device="cuda") -> PreparedConv:
    import torch

    packed, scales = pack_conv_weight(params, algorithm, src_layout, src)
    w = torch.from_numpy(packed).to(device)
    ws = None if scales is None else torch.from_numpy(scales).to(device)
    b = torch.from_numpy(np.ascontiguousarray(bias, dtype=np.float32)).to(device)
    return PreparedConv(list(int(v) for v in params), algorithm, w, ws, b)


def conv2d(pc: PreparedConv, x, y, *, flags: int = SILU, x_slots=None, y_slots=None, residual=None,
           acc_out=None, stream=None) -> None:
    """Runs one conv: x and y are NHWC views (x may be dense fp32 NCHW with IN_NCHW_F32)."""
    d = ConvDesc.from_params(pc.params)
    if flags & IN_NCHW_F32:
        xv = TensorView(data=x.data_ptr(), n_stride=x.stride(0), c_stride=1, amax_stripes=0, amax_slots=None,
                        amax_stripe_stride=0)
    else:
        xv = view(x, x_slots)
    yv = view(y, y_slots)
    rv = view(residual) if residual is not None else None
    check(_lib.lib().aexrt_hip_conv2d(
        ctypes.byref(d), pc.algorithm, flags, ctypes.byref(xv), pc.weight.data_ptr(),
        _ptr(pc.w_scale), pc.bias.data_ptr(), None if rv is None else ctypes.byref(rv), ctypes.byref(yv),
        _ptr(acc_out), _stream(stream)), "conv2d")


def conv2d_upsampled_input(pc: PreparedConv, x, x_up, up_c0: int, y, *, flags: int = SILU, x_slots=None,
                           x_up_slots=None, y_slots=None, acc_out=None, stream=None) -> None:
    """int8 1x1 conv ``pc`` (per-tensor) over ``x`` ([N, H, W, C] NHWC view) whose channels [up_c0,
    up_c0 + C_up) are the nearest 2x upsample of ``x_up`` ([N, H/2, W/2, C_up]), read from x_up
    directly (x's memory there is not read); ``x_up_slots``: x_up's amax slots."""
    d = ConvDesc.from_params(pc.params)
    xv, uv, yv = view(x, x_slots), view(x_up, x_up_slots), view(y, y_slots)
    check(_lib.lib().aexrt_hip_conv2d_upsampled_input(
        ctypes.byref(d), pc.algorithm, flags, ctypes.byref(xv), ctypes.byref(uv), up_c0, x_up.shape[3],
        pc.weight.data_ptr(), _ptr(pc.w_scale), pc.bias.data_ptr(), ctypes.byref(yv), _ptr(acc_out),
        _stream(stream)), "conv2d_upsampled_input")


def conv2d_upsample_copy(pc: PreparedConv, x, y, y_up, *, flags: int = SILU, x_slots=None, y_slots=None,
                         y_up_slots=None, stream=None) -> None:
    """int8 1x1 conv ``pc`` (per-tensor) that also writes its output's nearest 2x upsample into the
    NHWC view ``y_up`` ([N, 2 OH, 2 OW, OC], e.g. a channel slice of a concat) and folds its amax into
    ``y_up_slots``: the resize after the conv, in the conv's launch."""
    d = ConvDesc.from_params(pc.params)
    xv, yv, uv = view(x, x_slots), view(y, y_slots), view(y_up, y_up_slots)
    check(_lib.lib().aexrt_hip_conv2d_upsample_copy(
        ctypes.byref(d), pc.algorithm, flags, ctypes.byref(xv), pc.weight.data_ptr(), _ptr(pc.w_scale),
        pc.bias.data_ptr(), ctypes.byref(yv), ctypes.byref(uv), _stream(stream)), "conv2d_upsample_copy")


def conv2d_fused_1x1(pc: PreparedConv, pc2: PreparedConv, x, y2, *, flags2: int = 0, y2_slots=None,
                     stream=None) -> None:
    """fp16 3x3 SiLU conv ``pc`` with the 1x1 conv ``pc2`` of its output fused into its epilogue:
    y2 = conv1x1(fp16(silu(conv3x3(x)))) (SiLU too with flags2 SILU, fp32 y2 with OUT_F32); the 3x3
    output is not stored."""
    d, d2 = ConvDesc.from_params(pc.params), ConvDesc.from_params(pc2.params)
    xv, yv = view(x), view(y2, y2_slots)
    check(_lib.lib().aexrt_hip_conv2d_fused_1x1(
        ctypes.byref(d), SILU, ctypes.byref(xv), pc.weight.data_ptr(), pc.bias.data_ptr(), ctypes.byref(d2), flags2,
        pc2.weight.data_ptr(), pc2.bias.data_ptr(), ctypes.byref(yv), _stream(stream)), "conv2d_fused_1x1")


def conv_chain3(pa: PreparedConv, pb: PreparedConv, pc: PreparedConv, x, y, *, flags_c: int = 0, tile=(0, 0),
                stream=None) -> None:
    """A detect-head branch in one launch: y = conv_c(fp16(silu(conv_b(fp16(silu(conv_a(x))))))) with
    a, b fp16 3x3 SiLU convs and c a 1x1 conv (SiLU with flags_c SILU, fp32 y with OUT_F32); the two
    intermediate maps stay in LDS.  tile = (rows, cols) of a block's output tile, (0, 0): chosen."""
    da, db, dc = (ConvDesc.from_params(p.params) for p in (pa, pb, pc))
    xv, yv = view(x), view(y)
    check(_lib.lib().aexrt_hip_conv_chain3(
        ctypes.byref(da), pa.weight.data_ptr(), pa.bias.data_ptr(), ctypes.byref(db), pb.weight.data_ptr(),
        pb.bias.data_ptr(), ctypes.byref(dc), flags_c, pc.weight.data_ptr(), pc.bias.data_ptr(), ctypes.byref(xv),
        ctypes.byref(yv), int(tile[0]), int(tile[1]), _stream(stream)), "conv_chain3")


def conv_pair(pa: PreparedConv, pb: PreparedConv, x, y, *, x_slots=None, y_slots=None, residual: bool = False,
              band_rows: int = 0, t_out=None, acc_a=None, acc_b=None, stream=None) -> None:
    """A C2f bottleneck in one launch: y = silu(conv_b(fp16(silu(conv_a(x))))) (+ x with residual), both
    3x3 C -> C convs on int8 (algorithm 52: x_slots hold x's amax; the intermediate is quantized with
    its own batch-global amax) or fp16; the intermediate stays on chip (t_out: an optional copy).
    acc_a / acc_b: optional int32 [N*H*W, C] sums of the two int8 convs."""
    d = ConvDesc.from_params(pa.params)
    xv, yv = view(x, x_slots), view(y, y_slots)
    check(_lib.lib().aexrt_hip_conv_pair(
        ctypes.byref(d), pa.algorithm, RESIDUAL if residual else 0, ctypes.byref(xv), pa.weight.data_ptr(),
        _ptr(pa.w_scale), pa.bias.data_ptr(), pb.weight.data_ptr(), _ptr(pb.w_scale), pb.bias.data_ptr(),
        ctypes.byref(yv), int(band_rows), _ptr(t_out), _ptr(acc_a), _ptr(acc_b), _stream(stream)), "conv_pair")


def conv_pair_barrier_timeouts() -> int:
    """Synchronizes the device; nonzero when an int8 pair launch's grid barrier wait timed out."""
    return int(_lib.lib().aexrt_hip_conv_pair_barrier_timeouts())


def conv2d_int8(pc: PreparedConv, x, y, *, flags: int = SILU, residual=None, stream=None) -> None:
    """The reference's int8 conv command on a plain fp16 NHWC input: dynamic below 4096 input
    elements, else the input's amax (strips with INT8_PG16) then the int8 conv."""
    d = ConvDesc.from_params(pc.params)
    xv, yv = view(x), view(y)
    rv = view(residual) if residual is not None else None
    check(_lib.lib().aexrt_hip_conv2d_int8(
        ctypes.byref(d), pc.algorithm, flags, ctypes.byref(xv), pc.weight.data_ptr(), _ptr(pc.w_scale),
        pc.bias.data_ptr(), None if rv is None else ctypes.byref(rv), ctypes.byref(yv), _stream(stream)),
        "conv2d_int8")


def conv2d_int8_noalloc(pc: PreparedConv, x, y, *, flags: int = SILU, residual=None, stream=None) -> None:
    """:func:`conv2d_int8` with the amax scratch in the library's static device array (no device
    allocation; in_channels <= 4096)."""
    d = ConvDesc.from_params(pc.params)
    xv, yv = view(x), view(y)
    rv = view(residual) if residual is not None else None
    check(_lib.lib().aexrt_hip_conv2d_int8_noalloc(
        ctypes.byref(d), pc.algorithm, flags, ctypes.byref(xv), pc.weight.data_ptr(), _ptr(pc.w_scale),
        pc.bias.data_ptr(), None if rv is None else ctypes.byref(rv), ctypes.byref(yv), _stream(stream)),
        "conv2d_int8_noalloc")


def fill_u32(t, value: int = 0, stream=None) -> None:
    check(_lib.lib().aexrt_hip_fill_u32(t.data_ptr(), t.numel(), value, _stream(stream)), "fill_u32")


def nchw_f32_to_nhwc(x, y, y_slots=None, stream=None) -> None:
    n, c, h, w = x.shape
    yv = view(y, y_slots)
    check(_lib.lib().aexrt_hip_nchw_f32_to_nhwc(x.data_ptr(), n, c, h * w, ctypes.byref(yv),
                                                 _stream(stream)), "nchw_f32_to_nhwc")


def nhwc_to_nchw_f32(x, stream=None):
    import torch

    n, h, w, c = x.shape
    y = torch.empty((n, c, h, w), dtype=torch.float32, device=x.device)
    xv = view(x)
    check(_lib.lib().aexrt_hip_nhwc_to_nchw_f32(ctypes.byref(xv), int(x.dtype == torch.float16), n, c, h * w,
                                                 y.data_ptr(), _stream(stream)), "nhwc_to_nchw_f32")
    return y


def copy(src, dst, dst_slots=None, stream=None) -> None:
    n, h, w, c = src.shape
    sv, dv = view(src), view(dst, dst_slots)
    check(_lib.lib().aexrt_hip_copy(ctypes.byref(sv), ctypes.byref(dv), n, h * w, c, _stream(stream)), "copy")


def maxpool(x, y, k: int, s: int, p: int, y_slots=None, stream=None) -> None:
    n, h, w, c = x.shape
    _, oh, ow, _ = y.shape
    xv, yv = view(x), view(y, y_slots)
    check(_lib.lib().aexrt_hip_maxpool(ctypes.byref(xv), ctypes.byref(yv), n, c, h, w, oh, ow, k, s, p,
                                        _stream(stream)), "maxpool")


def resize_nearest(x, y, y_slots=None, stream=None) -> None:
    n, h, w, c = x.shape
    _, oh, ow, _ = y.shape
    xv, yv = view(x), view(y, y_slots)
    check(_lib.lib().aexrt_hip_resize_nearest(ctypes.byref(xv), ctypes.byref(yv), n, c, h, w, oh, ow,
                                               _stream(stream)), "resize_nearest")


def sppf_maxpool(x, y1, y2, y3, slots=(None, None, None), stream=None) -> None:
    """y1 = maxpool5(x), y2 = maxpool5(y1), y3 = maxpool5(y2) (stride 1, pad 2) in one kernel."""
    n, h, w, c = x.shape
    xv = view(x)
    v1, v2, v3 = (view(t, sl) for t, sl in zip((y1, y2, y3), slots))
    check(_lib.lib().aexrt_hip_sppf_maxpool(ctypes.byref(xv), ctypes.byref(v1), ctypes.byref(v2), ctypes.byref(v3),
                                            n, c, h, w, _stream(stream)), "sppf_maxpool")


def add(a, b, y, y_slots=None, stream=None) -> None:
    n, h, w, c = a.shape
    av, bv, yv = view(a), view(b), view(y, y_slots)
    check(_lib.lib().aexrt_hip_add(ctypes.byref(av), ctypes.byref(bv), ctypes.byref(yv), n, h * w, c,
                                    _stream(stream)), "add")


def conv_candidates(desc: ConvDesc, algorithm: int, flags: int = SILU, *, x_cstride: Optional[int] = None,
                    y_cstride: Optional[int] = None, residual: bool = False, cap: int = 512) -> list[str]:
    """Kernel instance and tile of every candidate the model loader measures for one conv with
    dense NHWC views (channel strides ``x_cstride`` / ``y_cstride`` for channel slices); ``""``
    marks a candidate its launcher rejects.  With ``IN_NCHW_F32`` in flags the input is the
    network's fp32 NCHW tensor of ``x_cstride`` channels (desc.in_channels 8).  Host only: no
    kernel runs, no device is needed."""
    d = desc
    xc = x_cstride or d.in_channels
    yc = y_cstride or d.out_channels
    base = 1 << 20  # aligned placeholder addresses: nothing is dereferenced
    xv = TensorView(data=base, n_stride=d.in_h * d.in_w * xc, c_stride=xc, amax_stripes=0, amax_slots=base,
                    amax_stripe_stride=0)
    if flags & IN_NCHW_F32:
        xv.c_stride = 1
    yv = TensorView(data=base, n_stride=d.out_h * d.out_w * yc, c_stride=yc, amax_stripes=0, amax_slots=None,
                    amax_stripe_stride=0)
    rv = TensorView(data=base, n_stride=d.out_h * d.out_w * yc, c_stride=yc, amax_stripes=0, amax_slots=None,
                    amax_stripe_stride=0)
    name_len = 128
    buf = ctypes.create_string_buffer(name_len * cap)
    n = _lib.lib().aexrt_hip_conv_candidates(ctypes.byref(d), algorithm, flags, ctypes.byref(xv),
                                             ctypes.byref(rv) if residual else None, ctypes.byref(yv), buf,
                                             name_len, cap)
    if n == 0:
        raise RuntimeError(f"conv_candidates failed: {_lib.last_error()}")
    raw = buf.raw
    return [raw[i * name_len:(i + 1) * name_len].split(b"\0", 1)[0].decode() for i in range(min(n, cap))] + \
        [None] * max(0, n - cap)
