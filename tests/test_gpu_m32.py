"""Parity of the 32x32-MFMA 3x3 conv kernel on forced tiles, through the op-level C ABI.

int8: the int32 accumulators must equal the oracle's exactly (they are exact sums of int8
products whatever the tile), the stored fp16 outputs must be within one fp16 ulp of the
W8A8 oracle (with a fused residual add, one more of the sum), and the output amax slots must hold the max |y|
of what was stored.  fp16: within 1e-2 of the output range of the fp32 direct conv of the
fp16 operands.  Cases cover ragged row and column tiles, tiles wider than the image,
several channel chunks, stride 2, 80 output channels on a 96-channel block, several channel
blocks, fp32 output, SiLU + residual, and a residual written into a channel slice.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from aexrt_amd import kernels as K
from aexrt_amd import packing
from tests.helpers import group16_weight, he_weight, nhwc_to_nchw, tol_range
from tests.test_gpu_ops import FP16_TOL, FP32_TOL, _dev_nhwc, _run_fp16_residual, _run_int8, _u32

pytestmark = pytest.mark.gpu


def _ulp16(a):
    return np.spacing(np.abs(a).astype(np.float16)).astype(np.float64)


def _force(mq, nq, tr, tc, cc, nw=4):
    """nw 4 or 8 waves per block; 16: 8 waves in two groups of 4."""
    mode = {4: K.HALO_FORCE_M32, 8: K.HALO_FORCE_M32_8, 16: K.HALO_FORCE_M32_2G}[nw]
    K.set_conv3x3_halo(mode, nq, mq, tr, tc, cc)


def _slots_of(y, oc):
    g = (oc + 15) // 16
    return np.array([np.float32(np.abs(y[:, k * 16:(k + 1) * 16]).max()).view(np.uint32) for k in range(g)],
                    dtype=np.uint32)


# (n, c, h, w, oc, s, mq, nq, tr, tc, cc divisor, seed[, waves per block])
INT8_M32 = [
    (2, 64, 11, 13, 80, 1, 2, 3, 8, 13, 1, 301),     # 80 channels on a 96-channel block, ragged rows
    (2, 64, 11, 13, 80, 1, 1, 1, 4, 13, 2, 302),     # three channel blocks, two chunks
    (1, 32, 17, 15, 64, 2, 1, 2, 4, 8, 1, 303),      # stride 2, ragged columns
    (3, 16, 20, 20, 32, 1, 4, 1, 20, 20, 1, 304),    # one tile per image (400 positions of 512)
    (1, 128, 10, 10, 128, 1, 2, 2, 10, 10, 2, 305),  # 128 channels in two blocks, two chunks
    (2, 128, 20, 20, 256, 2, 1, 2, 10, 10, 2, 306),  # stride 2, four channel blocks, two chunks
    (1, 48, 9, 7, 32, 1, 2, 1, 9, 7, 3, 307),        # C = 48: three 16-channel chunks, padded k steps
    (2, 64, 20, 20, 64, 1, 2, 2, 20, 20, 2, 308, 8),  # 8 waves: one 20x20 image per tile
    (1, 32, 17, 15, 96, 2, 1, 3, 9, 8, 1, 309, 8),    # 8 waves, stride 2, 96 channels
    (2, 64, 20, 20, 64, 1, 2, 2, 10, 20, 2, 310, 16),   # two wave groups, each with its own tiles
    (3, 32, 17, 15, 96, 2, 1, 3, 4, 8, 1, 312, 16),     # two groups, stride 2, ragged tiles
    (1, 64, 8, 8, 64, 1, 1, 2, 8, 8, 1, 313, 16),       # one tile: the second group has none
]


@pytest.mark.parametrize("case", INT8_M32, ids=[f"c{t[1]}_{t[2]}x{t[3]}_oc{t[4]}_s{t[5]}_mq{t[6]}_nq{t[7]}_cc{t[1] // t[10]}"
                                                f"_w{t[12] if len(t) > 12 else 4}" for t in INT8_M32])
def test_m32_int8_conv(cuda, case):
    n, c, h, w, oc, s, mq, nq, tr, tc, ccd, seed = case[:12]
    nw = case[12] if len(case) > 12 else 4
    oh, ow = (h - 1) // s + 1, (w - 1) // s + 1
    _force(mq, nq, min(tr, oh), min(tc, ow), c // ccd, nw)
    try:
        r = _run_int8(cuda, n, c, h, w, oc, 3, s, seed)
        np.testing.assert_array_equal(r["acc"], r["acc_ref"])
        err = np.abs(r["y"].astype(np.float64) - r["y_ref"])
        assert (err <= _ulp16(r["y_ref"])).all(), float(err.max())
        np.testing.assert_array_equal(r["slots"], _slots_of(r["y"], oc))
        # fp32 output without activation
        r = _run_int8(cuda, n, c, h, w, oc, 3, s, seed + 50, silu=False, out_f32=True)
        np.testing.assert_array_equal(r["acc"], r["acc_ref"])
        err, allowed = tol_range(r["y_ref"], r["y"], FP32_TOL)
        assert err <= allowed, (err, allowed)
    finally:
        K.set_conv3x3_halo(K.HALO_AUTO)


def _run_int8_fused(cuda, n, c, h, w, oc, s, seed, residual):
    """The SiLU (and SiLU + residual) epilogue instances: no accumulator output."""
    import torch

    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, c, h, w)).astype(np.float16).astype(np.float32)
    wt = group16_weight(rng, oc, c, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, 3, s, 1)
    pc = K.prepare_conv(desc, 53 if s == 2 else 52, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True),
                        b, device=cuda)
    xd = _dev_nhwc(x, cuda)
    xs = K.new_slots(c, cuda)
    K.amax_slots(xd, xs)
    _, _, oh, ow = O.out_shape(desc)
    y = torch.full((n, oh, ow, oc), float("nan"), dtype=torch.float16, device=cuda)
    ys = K.new_slots(oc, cuda, stripes=16)
    rt = None
    flags = K.SILU
    if residual:
        rr = O.round_f16(rng.standard_normal((n, oc, oh, ow)).astype(np.float32))
        rt = _dev_nhwc(rr, cuda)
        flags |= K.RESIDUAL
    K.conv2d(pc, xd, y, flags=flags, x_slots=xs, y_slots=ys, residual=rt)
    torch.cuda.synchronize()
    *_, conv = O.w8a8_conv(x, wt, b, desc, silu=True, fp16_engine=True)
    got = nhwc_to_nchw(y.float().cpu().numpy())
    # within one fp16 ulp of the conv output, and with the residual one more of the sum
    bound = _ulp16(conv)
    y_ref = conv
    if residual:
        y_ref = O.round_f16(conv) + rr
        bound = bound + _ulp16(y_ref)
    return got, y_ref, bound, K.slots_max(ys)


@pytest.mark.parametrize("residual", [False, True], ids=["silu", "silu_residual"])
def test_m32_int8_fused_epilogues(cuda, residual):
    _force(2, 2, 10, 20, 32)
    try:
        got, y_ref, bound, slots = _run_int8_fused(cuda, 2, 64, 20, 20, 64, 1, 311 + residual, residual)
    finally:
        K.set_conv3x3_halo(K.HALO_AUTO)
    assert np.isfinite(got).all()
    err = np.abs(got.astype(np.float64) - y_ref)
    assert (err <= bound).all(), float(err.max())
    np.testing.assert_array_equal(slots, _slots_of(got, 64))


# (n, c, h, w, oc, s, mq, nq, tr, tc, cc divisor, silu, out_f32[, waves per block])
FP16_M32 = [
    (1, 64, 40, 40, 64, 1, 2, 2, 6, 40, 2, True, False),   # the head's 40x40 shape, two chunks
    (2, 64, 40, 40, 80, 1, 2, 3, 6, 40, 4, True, False),   # 80 channels on a 96-channel block
    (1, 80, 20, 20, 80, 1, 1, 1, 6, 20, 5, True, False),   # three channel blocks, five chunks
    (2, 128, 10, 10, 64, 1, 1, 1, 10, 10, 2, True, False),  # two channel blocks, two chunks
    (1, 48, 13, 11, 64, 2, 1, 2, 7, 6, 1, False, True),    # stride 2, fp32 output, no activation
    (1, 32, 9, 37, 32, 1, 4, 1, 13, 37, 1, True, False),   # tile wider than the map's rows
    (2, 64, 40, 40, 64, 1, 2, 2, 10, 40, 2, True, False, 8),  # 8 waves: the head's 40x40 shape
    (1, 64, 40, 40, 80, 1, 1, 3, 6, 40, 4, True, False, 8),   # 8 waves, 96-channel block
    (1, 48, 13, 11, 64, 2, 2, 1, 7, 11, 3, False, True, 8),   # 8 waves, stride 2, fp32 output
    (2, 64, 40, 40, 144, 1, 1, 3, 3, 40, 4, True, False, 16),  # two groups: the head's 144-channel sibling pair
    (1, 64, 40, 40, 64, 1, 2, 2, 6, 40, 4, True, False, 16),   # two groups, two subtiles per wave
]


@pytest.mark.parametrize("case", FP16_M32, ids=[f"c{t[1]}_{t[2]}x{t[3]}_oc{t[4]}_s{t[5]}_mq{t[6]}_nq{t[7]}_cc{t[1] // t[10]}"
                                                f"_w{t[13] if len(t) > 13 else 4}" for t in FP16_M32])
def test_m32_fp16_conv(cuda, case):
    import torch

    n, c, h, w, oc, s, mq, nq, tr, tc, ccd, silu, out_f32 = case[:13]
    nw = case[13] if len(case) > 13 else 4
    rng = np.random.default_rng(401 + c + h + oc)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    wt = he_weight(rng, oc, c, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, 3, s, 1)
    _, _, oh, ow = O.out_shape(desc)
    pc = K.prepare_conv(desc, 5, K.SRC_RAW_F32, wt, b, device=cuda)
    y = torch.full((n, oh, ow, oc), float("nan"), dtype=torch.float32 if out_f32 else torch.float16, device=cuda)
    slots = K.new_slots(oc, cuda)
    flags = (K.SILU if silu else 0) | (K.OUT_F32 if out_f32 else 0)
    _force(mq, nq, min(tr, oh), min(tc, ow), c // ccd, nw)
    try:
        K.conv2d(pc, _dev_nhwc(x, cuda), y, flags=flags, y_slots=slots)
    finally:
        K.set_conv3x3_halo(K.HALO_AUTO)
    torch.cuda.synchronize()
    got = nhwc_to_nchw(y.float().cpu().numpy())
    assert np.isfinite(got).all()
    y_ref = O.cpu_conv2d(x, O.round_f16(wt), b, desc, silu=silu)
    err, allowed = tol_range(y_ref, got, FP32_TOL if out_f32 else FP16_TOL)
    assert err <= allowed, (err, allowed)
    np.testing.assert_array_equal(_u32(slots), _slots_of(got, oc))


def test_m32_fp16_residual_into_channel_slice(cuda):
    _force(1, 1, 9, 7, 32)
    try:
        y_ref, got, slots = _run_fp16_residual(cuda, 2, 32, 9, 7, 421, tail=(48, 80), width=96)
    finally:
        K.set_conv3x3_halo(K.HALO_AUTO)
    err, allowed = tol_range(y_ref, got[:, 48:80], FP16_TOL)
    assert err <= allowed, (err, allowed)
    assert not got[:, :48].any() and not got[:, 80:].any()


def test_m32_forced_tile_that_does_not_fit_fails(cuda):
    import torch

    K.set_conv3x3_halo(K.HALO_FORCE_M32, 2, 2, 4, 16, 48)  # C = 64 is not a multiple of 48
    try:
        rng = np.random.default_rng(5)
        desc = O.conv_desc(1, 64, 8, 16, 64, 3, 1, 1)
        pc = K.prepare_conv(desc, 5, K.SRC_RAW_F32, he_weight(rng, 64, 64, 3), np.zeros(64, np.float32), device=cuda)
        x = torch.zeros((1, 8, 16, 64), dtype=torch.float16, device=cuda)
        y = torch.empty_like(x)
        with pytest.raises(RuntimeError):
            K.conv2d(pc, x, y)
    finally:
        K.set_conv3x3_halo(K.HALO_AUTO)
    with pytest.raises(RuntimeError):  # no instance: 4 position subtiles x 3 channel subtiles
        K.set_conv3x3_halo(K.HALO_FORCE_M32, 3, 4, 4, 16, 16)


# (n, c, h, w, oc, oc2, tile (mode, jn, pw, tr, tc, cc) or None, silu2, slice of a wider output)
FUSED = [
    (2, 64, 40, 40, 64, 64, (5, 2, 2, 6, 40, 32), False, None),   # the head's 40x40 box branch
    (1, 64, 40, 40, 64, 64, None, False, None),                   # the first tile that fits
    (2, 80, 20, 20, 80, 80, (5, 3, 1, 3, 20, 16), False, None),   # class branch: 80 channels, 96-channel block
    (2, 64, 10, 10, 64, 64, (6, 2, 1, 10, 10, 64), True, (16, 80, 96)),  # 8 waves, SiLU, into a channel slice
    (1, 80, 13, 11, 80, 64, (5, 3, 2, 13, 11, 16), False, None),  # ragged map, 1x1 to fewer channels
    (2, 80, 20, 20, 80, 80, (5, 3, 1, 3, 20, 16), "f32", None),   # fp32 output (the head's raw output)
    (2, 64, 40, 40, 64, 64, (7, 2, 1, 3, 40, 32), False, None),   # two wave groups
    (2, 80, 20, 20, 80, 80, (7, 3, 1, 3, 20, 16), "f32", None),   # two groups, fp32 output
]


@pytest.mark.parametrize("case", FUSED, ids=[f"c{t[1]}_{t[2]}x{t[3]}_oc{t[4]}_to{t[5]}_{'forced' if t[6] else 'auto'}"
                                             f"{'_' + (t[7] if isinstance(t[7], str) else 'silu') if t[7] else ''}"
                                             f"{'_slice' if t[8] else ''}" for t in FUSED])
def test_m32_fused_1x1(cuda, case):
    """A 3x3 SiLU conv with the following 1x1 conv in its epilogue: against the oracle's two convs
    with the 3x3 output rounded to fp16 in between (what the unfused pair stores and reads)."""
    import torch

    n, c, h, w, oc, oc2, tile, silu2, sl = case
    rng = np.random.default_rng(501 + c + h + oc2)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    wt = he_weight(rng, oc, c, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    w2 = he_weight(rng, oc2, oc, 1)
    b2 = packing.fp16_round(rng.uniform(-0.1, 0.1, oc2).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, 3, 1, 1)
    desc2 = O.conv_desc(n, oc, h, w, oc2, 1, 1, 0)
    pc = K.prepare_conv(desc, 5, K.SRC_RAW_F32, wt, b, device=cuda)
    pc2 = K.prepare_conv(desc2, 5, K.SRC_RAW_F32, w2, b2, device=cuda)
    lo, hi, width = sl if sl else (0, oc2, oc2)
    f32 = silu2 == "f32"
    silu2 = silu2 is True
    big = torch.zeros((n, h, w, width), dtype=torch.float32 if f32 else torch.float16, device=cuda)
    slots = K.new_slots(width, cuda)
    if tile:
        K.set_conv3x3_halo(*tile)
    try:
        K.conv2d_fused_1x1(pc, pc2, _dev_nhwc(x, cuda), big[..., lo:hi],
                           flags2=(K.SILU if silu2 else 0) | (K.OUT_F32 if f32 else 0), y2_slots=slots[lo // 16:hi // 16])
    finally:
        K.set_conv3x3_halo(K.HALO_AUTO)
    torch.cuda.synchronize()
    got = nhwc_to_nchw(big.float().cpu().numpy())
    y1 = O.round_f16(O.cpu_conv2d(x, O.round_f16(wt), b, desc, silu=True))
    y2 = O.cpu_conv2d(y1, O.round_f16(w2), b2, desc2, silu=silu2)
    assert np.isfinite(got).all()
    err, allowed = tol_range(y2, got[:, lo:hi], FP32_TOL if f32 else FP16_TOL)
    assert err <= allowed, (err, allowed)
    assert not got[:, :lo].any() and not got[:, hi:].any()
    np.testing.assert_array_equal(_u32(slots)[lo // 16:hi // 16], _slots_of(got[:, lo:hi], oc2))


def test_m32_fused_1x1_refuses_what_it_cannot_fuse(cuda):
    import torch

    rng = np.random.default_rng(7)
    desc = O.conv_desc(1, 64, 8, 8, 128, 3, 1, 1)  # 128 channels: no tile covers them all
    desc2 = O.conv_desc(1, 128, 8, 8, 64, 1, 1, 0)
    pc = K.prepare_conv(desc, 5, K.SRC_RAW_F32, he_weight(rng, 128, 64, 3), np.zeros(128, np.float32), device=cuda)
    pc2 = K.prepare_conv(desc2, 5, K.SRC_RAW_F32, he_weight(rng, 64, 128, 1), np.zeros(64, np.float32), device=cuda)
    x = torch.zeros((1, 8, 8, 64), dtype=torch.float16, device=cuda)
    y = torch.zeros((1, 8, 8, 64), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError):
        K.conv2d_fused_1x1(pc, pc2, x, y)
