"""Build-time weight packing of the engine compiler (the reference's
``_add_packed_*`` helpers, src/aexrt/engine.py:2309-2553).

These produce the reference's packed-weight payloads byte for byte, so an
engine written here carries the same section-6 records as one written by the
reference compiler.  The gfx950 kernels consume their own operand layouts;
the runtime repacks these payloads at load time (see
``aexrt_hip_pack_conv_weight``).
"""
from __future__ import annotations

import numpy as np

PACKED_LAYOUT_CONV3X3_OC4 = 1
PACKED_LAYOUT_CONV3X3_OC4_FP16 = 2
PACKED_LAYOUT_WINOGRAD_F2X2_FP16 = 3
PACKED_LAYOUT_CONV1X1_OC8_FP16 = 4
PACKED_LAYOUT_WINOGRAD_F2X2_FP32 = 5
PACKED_LAYOUT_CONV_INT8 = 8

# Winograd F(2x2,3x3) filter transform G (engine.py:2369-2372).
WINOGRAD_G = np.array(((1.0, 0.0, 0.0), (0.5, 0.5, 0.5), (0.5, -0.5, 0.5), (0.0, 0.0, 1.0)),
                      dtype=np.float32)


def fp16_round(a: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest fp16 and widen back (RNE)."""
    return np.asarray(a, dtype=np.float32).astype("<f2").astype(np.float32)


def quantize_conv_int8(weight: np.ndarray, *, fp16_engine: bool) -> tuple[np.ndarray, np.ndarray]:
    """Per-output-channel symmetric int8 weights (engine.py:2418-2465).

    scale = max|w_oc| / 127 (1 for an all-zero row), inv = 1/scale in fp32,
    q = clamp(sign(p) * floor(|p| + 0.5), -127, 127) with p = w * inv in fp32
    -- the compiler's half-away-from-zero rounding, including its fp32
    evaluation of ``|p| + 0.5``.  fp16 engines round the source to fp16
    first.  Returns (q int8 shaped like ``weight``, scale fp32 [oc]).
    """
    w = np.asarray(weight, dtype=np.float32)
    oc = w.shape[0]
    if fp16_engine:
        w = fp16_round(w)
    rows = w.reshape(oc, -1)
    amax = np.abs(rows).max(axis=1) if rows.size else np.zeros(oc, np.float32)
    scale = np.where(amax > 0.0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    prod = (rows * inv[:, None]).astype(np.float32)
    mag = np.floor((np.abs(prod) + np.float32(0.5)).astype(np.float32))
    q = np.clip(np.sign(prod) * mag, -127.0, 127.0).astype(np.int8)
    return q.reshape(w.shape), scale


def pack_conv_int8(weight: np.ndarray, *, fp16_engine: bool) -> bytes:
    """Layout 8 payload: int8 [oc][ic][kk] followed by oc fp32 scales."""
    q, scale = quantize_conv_int8(weight, fp16_engine=fp16_engine)
    return q.tobytes(order="C") + scale.astype("<f4").tobytes(order="C")


def unpack_conv_int8(payload: bytes, out_channels: int, per_oc: int) -> tuple[np.ndarray, np.ndarray]:
    n = out_channels * per_oc
    q = np.frombuffer(payload, dtype=np.int8, count=n).reshape(out_channels, per_oc)
    s = np.frombuffer(payload, dtype="<f4", count=out_channels, offset=n)
    return q, s


def winograd_f2x2_transform(weight: np.ndarray) -> np.ndarray:
    """U = G g G^T on the fp16-rounded 3x3 source, fp32, [oc][ic][4][4]."""
    src = fp16_round(weight).reshape(weight.shape[0], weight.shape[1], 3, 3)
    return np.einsum("ak,oikl,bl->oiab", WINOGRAD_G, src, WINOGRAD_G, optimize=True)


def pack_winograd_f2x2_fp16(weight: np.ndarray) -> bytes:
    """Layout 3: fp16 U [oc][ic][4][4] (engine.py:2346-2379)."""
    return winograd_f2x2_transform(weight).astype("<f2").tobytes(order="C")


def pack_winograd_f2x2_fp32(weight: np.ndarray) -> bytes:
    """Layout 5: fp32 U [oc][ic][4][4] (engine.py:2382-2415)."""
    return winograd_f2x2_transform(weight).astype("<f4").tobytes(order="C")


def pack_conv1x1_oc8_fp16(weight: np.ndarray) -> bytes:
    """Layout 4: fp16 [oc/8][ic][8] (engine.py:2520-2553)."""
    w = np.asarray(weight, dtype=np.float32)
    oc, ic = w.shape[0], w.shape[1]
    return w.reshape(oc // 8, 8, ic).transpose(0, 2, 1).astype("<f2").tobytes(order="C")


def pack_conv3x3_oc4_fp16(weight: np.ndarray) -> bytes:
    """Layout 2: fp16 [oc/4][ic][9][4] (the runtime layout of kernel 43)."""
    w = np.asarray(weight, dtype=np.float32)
    oc, ic = w.shape[0], w.shape[1]
    return w.reshape(oc // 4, 4, ic, 9).transpose(0, 2, 3, 1).astype("<f2").tobytes(order="C")
