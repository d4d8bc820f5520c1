"""Parity of the streaming 1x1 int8 conv kernel on forced tiles, through the op-level C ABI.

The int32 accumulators must equal the oracle's exactly (exact sums of int8 products whatever
the tile), the stored fp16 outputs must be within one fp16 ulp of the W8A8 oracle, and the
output amax slots must hold the max |y| of what was stored.  Cases cover ragged position
tails, channel counts that leave a padded k step (C = 16, 48), several channel blocks with an
empty half (OC 80 on 64-channel blocks), 1 to 8 input pieces per thread, two position subtiles
per wave, runs of several tiles per block (the double-buffered LDS tiles), fp32 output without
SiLU, the SiLU-only instance, and channel-slice input and output views (a concat root's
layout: positions evenly strided, channel stride wider than the conv).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from aexrt_amd import kernels as K
from aexrt_amd import packing
from tests.helpers import group16_weight, nchw_to_nhwc, nhwc_to_nchw, tol_range
from tests.test_gpu_ops import FP32_TOL, _run_int8, _u32

pytestmark = pytest.mark.gpu


def _ulp16(a):
    return np.spacing(np.abs(a).astype(np.float16)).astype(np.float64)


def _slots_of(y, oc):
    g = (oc + 15) // 16
    return np.array([np.float32(np.abs(y[:, k * 16:(k + 1) * 16]).max()).view(np.uint32) for k in range(g)],
                    dtype=np.uint32)


# (n, c, h, w, oc, jq, pq, seed)
S1X1_CASES = [
    (2, 32, 7, 9, 32, 2, 1, 401),       # ragged tail: 126 positions in two 64-position tiles
    (2, 48, 7, 9, 32, 2, 2, 402),       # C = 48: the k step's last 16 channels padded; 2 subtiles per wave
    (3, 16, 11, 13, 16, 1, 1, 403),     # C = 16, one 16-channel subtile
    (1, 96, 10, 10, 80, 4, 1, 404),     # OC 80 on 64-channel blocks: the second block is 3/4 empty
    (2, 192, 20, 20, 64, 4, 1, 405),    # three k steps, 3 of 4 piece rounds per thread
    (2, 128, 20, 20, 64, 4, 2, 409),    # 2 subtiles per wave, 4 pieces per thread
    (1, 384, 10, 10, 256, 8, 1, 406),   # six k steps, 8 pieces per thread, two channel blocks
    (48, 512, 20, 20, 128, 8, 1, 407),  # 128 KB of LDS: one block per CU, runs of 2 tiles per block
    (24, 32, 80, 80, 32, 2, 1, 408),    # 2400 tiles on at most 2048 resident blocks: runs of 2 tiles
]


@pytest.mark.parametrize("case", S1X1_CASES,
                         ids=[f"n{t[0]}_c{t[1]}_{t[2]}x{t[3]}_oc{t[4]}_jq{t[5]}_pq{t[6]}" for t in S1X1_CASES])
def test_s1x1_int8_conv(cuda, case):
    n, c, h, w, oc, jq, pq, seed = case
    K.set_conv1x1_stream(True, jq, pq)
    try:
        r = _run_int8(cuda, n, c, h, w, oc, 1, 1, seed)
        np.testing.assert_array_equal(r["acc"], r["acc_ref"])
        err = np.abs(r["y"].astype(np.float64) - r["y_ref"])
        assert (err <= _ulp16(r["y_ref"])).all(), float(err.max())
        np.testing.assert_array_equal(r["slots"], _slots_of(r["y"], oc))
        # fp32 output without activation
        r = _run_int8(cuda, n, c, h, w, oc, 1, 1, seed + 50, silu=False, out_f32=True)
        np.testing.assert_array_equal(r["acc"], r["acc_ref"])
        err, allowed = tol_range(r["y_ref"], r["y"], FP32_TOL)
        assert err <= allowed, (err, allowed)
    finally:
        K.set_conv1x1_stream(False)


# (n, c, h, w, oc, input root width, input channel offset, output root width, output offset, jq, pq, seed)
S1X1_SLICES = [
    (2, 64, 20, 20, 64, 128, 64, 192, 64, 4, 1, 421),    # second half of a root -> middle of a concat root
    (4, 128, 10, 10, 128, 384, 128, 256, 0, 8, 1, 422),  # middle third -> first half
    (3, 32, 9, 11, 48, 64, 0, 96, 48, 2, 2, 423),        # ragged tail, 48 of 96 output channels
]


@pytest.mark.parametrize("case", S1X1_SLICES,
                         ids=[f"c{t[1]}of{t[5]}_oc{t[4]}of{t[7]}_jq{t[9]}_pq{t[10]}" for t in S1X1_SLICES])
def test_s1x1_int8_silu_channel_slices(cuda, case):
    """The SiLU instance (no accumulator output) reading a channel slice of one root and writing
    a channel slice of another: the other channels of the output root stay untouched."""
    import torch

    n, c, h, w, oc, cw, c0, ow_, o0, jq, pq, seed = case
    rng = np.random.default_rng(seed)
    xr = rng.standard_normal((n, cw, h, w)).astype(np.float16).astype(np.float32)
    x = xr[:, c0:c0 + c]
    wt = group16_weight(rng, oc, c, 1)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, 1, 1, 0)
    pc = K.prepare_conv(desc, 51, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True), b, device=cuda)
    xroot = torch.from_numpy(nchw_to_nhwc(xr.astype(np.float16))).to(cuda)
    xv = xroot[..., c0:c0 + c]
    xs = K.new_slots(c, cuda)
    K.amax_slots(xv, xs)
    yroot = torch.full((n, h, w, ow_), 7.0, dtype=torch.float16, device=cuda)
    yv = yroot[..., o0:o0 + oc]
    ys = K.new_slots(oc, cuda)
    K.set_conv1x1_stream(True, jq, pq)
    try:
        K.conv2d(pc, xv, yv, flags=K.SILU, x_slots=xs, y_slots=ys)
        torch.cuda.synchronize()
    finally:
        K.set_conv1x1_stream(False)
    _, _, _, _, _, y_ref = O.w8a8_conv(x, wt, b, desc, silu=True, fp16_engine=True)
    got_root = yroot.float().cpu().numpy()
    got = nhwc_to_nchw(got_root[..., o0:o0 + oc])
    err = np.abs(got.astype(np.float64) - y_ref)
    assert (err <= _ulp16(y_ref)).all(), float(err.max())
    np.testing.assert_array_equal(_u32(ys), _slots_of(got, oc))
    rest = np.concatenate([got_root[..., :o0], got_root[..., o0 + oc:]], axis=3)
    assert (rest == 7.0).all()


def test_s1x1_rejects_tiles_without_instance(cuda):
    with pytest.raises(RuntimeError, match="set_conv1x1_stream"):
        K.set_conv1x1_stream(True, 3, 1)
    with pytest.raises(RuntimeError, match="set_conv1x1_stream"):
        K.set_conv1x1_stream(True, 8, 2)
    K.set_conv1x1_stream(False)


# (n, c, h, w, oc, upsample root width, channel offset there, jq or 0 for the first fitting tile, seed)
S1X1_UPSAMPLE = [
    (2, 192, 20, 20, 128, 192, 0, 4, 431),   # YOLO's top-down path at 20x20: 128 of the 192 concat channels
    (3, 512, 10, 10, 256, 384, 0, 4, 432),   # SPPF's conv at 10x10 feeding a 384-channel concat
    (2, 64, 7, 9, 32, 96, 48, 0, 433),       # ragged tail, a slice at a channel offset, first tile that fits
    (1, 32, 5, 6, 16, 16, 0, 1, 434),        # one 16-channel group, dense upsample view
]


@pytest.mark.parametrize("case", S1X1_UPSAMPLE,
                         ids=[f"n{t[0]}_c{t[1]}_{t[2]}x{t[3]}_oc{t[4]}_up{t[5]}at{t[6]}_jq{t[7]}" for t in S1X1_UPSAMPLE])
def test_s1x1_upsample_copy_equals_resize(cuda, case):
    """The conv with its output's nearest 2x upsample written in the same launch
    (aexrt_hip_conv2d_upsample_copy): y bit-identical to the plain conv's, the upsample
    view bit-identical to the resize kernel's output of y (the reference's RESIZE), its slots
    equal to the resize's, and the rest of the upsample root untouched."""
    import torch

    n, c, h, w, oc, uw, u0, jq, seed = case
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, c, h, w)).astype(np.float16).astype(np.float32)
    wt = group16_weight(rng, oc, c, 1)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, 1, 1, 0)
    pc = K.prepare_conv(desc, 51, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True), b, device=cuda)
    xd = torch.from_numpy(nchw_to_nhwc(x.astype(np.float16))).to(cuda)
    xs = K.new_slots(c, cuda, stripes=16)
    K.amax_slots(xd, xs)
    # the plain conv, then the resize kernel into a root of the same layout
    y_ref = torch.empty((n, h, w, oc), dtype=torch.float16, device=cuda)
    ys_ref = K.new_slots(oc, cuda, stripes=16)
    if jq:
        K.set_conv1x1_stream(True, jq, 1)
    try:
        K.conv2d(pc, xd, y_ref, flags=K.SILU, x_slots=xs, y_slots=ys_ref)
        up_ref = torch.full((n, 2 * h, 2 * w, uw), 5.0, dtype=torch.float16, device=cuda)
        us_ref = K.new_slots(uw, cuda, stripes=16)
        K.resize_nearest(y_ref, up_ref[..., u0:u0 + oc], y_slots=us_ref[:, u0 // 16:(u0 + oc) // 16])
        # the conv with the upsample copy
        y = torch.empty_like(y_ref)
        ys = K.new_slots(oc, cuda, stripes=16)
        up = torch.full_like(up_ref, 5.0)
        us = K.new_slots(uw, cuda, stripes=16)
        K.conv2d_upsample_copy(pc, xd, y, up[..., u0:u0 + oc], x_slots=xs, y_slots=ys,
                               y_up_slots=us[:, u0 // 16:(u0 + oc) // 16])
        torch.cuda.synchronize()
    finally:
        K.set_conv1x1_stream(False)
    if jq:
        # the same tile on both sides: the same kernel arithmetic, bit for bit
        assert torch.equal(y, y_ref)
        assert torch.equal(up, up_ref)
        np.testing.assert_array_equal(_u32(ys).max(axis=0), _u32(ys_ref).max(axis=0))
        np.testing.assert_array_equal(_u32(us).max(axis=0), _u32(us_ref).max(axis=0))
    # against the oracle: y within one fp16 ulp; the upsample is y repeated 2 x 2 bit for bit, with
    # the max |y| of each group in its slots, and the rest of its root untouched
    _, _, _, _, _, yo = O.w8a8_conv(x, wt, b, desc, silu=True, fp16_engine=True)
    got = nhwc_to_nchw(y.float().cpu().numpy())
    assert (np.abs(got.astype(np.float64) - yo) <= _ulp16(yo)).all()
    upn = up.float().cpu().numpy()
    np.testing.assert_array_equal(upn[..., u0:u0 + oc], np.repeat(np.repeat(nchw_to_nhwc(got), 2, axis=1), 2, axis=2))
    assert (upn[..., :u0] == 5.0).all() and (upn[..., u0 + oc:] == 5.0).all()
    np.testing.assert_array_equal(_u32(us).max(axis=0)[u0 // 16:(u0 + oc) // 16], _slots_of(got, oc))


def test_s1x1_upsample_copy_refuses_fp32_output(cuda):
    import torch

    desc = O.conv_desc(1, 32, 4, 4, 16, 1, 1, 0)
    rng = np.random.default_rng(1)
    pc = K.prepare_conv(desc, 51, K.SRC_LAYOUT_INT8,
                        packing.pack_conv_int8(group16_weight(rng, 16, 32, 1), fp16_engine=True),
                        np.zeros(16, np.float32), device=cuda)
    x = torch.zeros((1, 4, 4, 32), dtype=torch.float16, device=cuda)
    xs = K.new_slots(32, cuda)
    y = torch.zeros((1, 4, 4, 16), dtype=torch.float32, device=cuda)
    up = torch.zeros((1, 8, 8, 16), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="conv2d_upsample_copy"):
        K.conv2d_upsample_copy(pc, x, y, up, flags=K.OUT_F32, x_slots=xs)


# (n, upsample channels, other channels, h, w (of the conv), oc, slice offset, jq or 0, seed)
S1X1_UPSAMPLED_INPUT = [
    (2, 128, 64, 40, 40, 64, 0, 4, 441),    # YOLO's P3 top-down concat: upsample first, then the skip feature
    (3, 256, 128, 20, 20, 128, 0, 8, 442),  # the P4 one (256 + 128 channels)
    (2, 32, 48, 6, 10, 32, 48, 0, 443),     # the upsample as the last slice, a ragged tail, first tile that fits
    (1, 16, 16, 4, 4, 16, 16, 1, 444),      # one 16-channel group each
]


@pytest.mark.parametrize("case", S1X1_UPSAMPLED_INPUT,
                         ids=[f"n{t[0]}_up{t[1]}_c{t[2]}_{t[3]}x{t[4]}_oc{t[5]}_at{t[6]}_jq{t[7]}"
                              for t in S1X1_UPSAMPLED_INPUT])
def test_s1x1_upsampled_input_equals_resize_then_conv(cuda, case):
    """The conv over a concat whose upsampled slice it reads from the resize's source
    (aexrt_hip_conv2d_upsampled_input; the slice itself left unwritten) against the resize into
    the slice followed by the same conv: int32 accumulators equal (and equal to the oracle's),
    outputs and output slots bit-identical on the same tile; the slice's own slot words are not
    needed (they stay zero)."""
    import torch

    n, cu, cs, h, w, oc, u0, jq, seed = case
    c = cu + cs
    rng = np.random.default_rng(seed)
    src = rng.standard_normal((n, cu, h // 2, w // 2)).astype(np.float16).astype(np.float32)
    skip = rng.standard_normal((n, cs, h, w)).astype(np.float16).astype(np.float32)
    up = np.repeat(np.repeat(src, 2, axis=2), 2, axis=3)
    cat = np.concatenate([up, skip], axis=1) if u0 == 0 else np.concatenate([skip, up], axis=1)
    assert cat.shape[1] == c and (u0 == 0 or u0 == cs)
    wt = group16_weight(rng, oc, c, 1)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, 1, 1, 0)
    pc = K.prepare_conv(desc, 51, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True), b, device=cuda)
    # the source and the folded form's root in one allocation (the kernel reads both through one
    # buffer resource, as a model's arena holds them)
    arena = torch.empty(n * (h // 2) * (w // 2) * cu + n * h * w * c, dtype=torch.float16, device=cuda)
    src_d = arena[:n * (h // 2) * (w // 2) * cu].view(n, h // 2, w // 2, cu)
    src_d.copy_(torch.from_numpy(nchw_to_nhwc(src.astype(np.float16))).to(cuda))
    src_s = K.new_slots(cu, cuda, stripes=16)
    K.amax_slots(src_d, src_s)
    # the reference order: the skip feature and the resize into one root, then the conv over it
    root = torch.zeros((n, h, w, c), dtype=torch.float16, device=cuda)
    root_s = K.new_slots(c, cuda, stripes=16)
    s0 = 0 if u0 else cu  # the skip slice
    root[..., s0:s0 + cs] = torch.from_numpy(nchw_to_nhwc(skip.astype(np.float16))).to(cuda)
    K.amax_slots(root[..., s0:s0 + cs], root_s[:, s0 // 16:(s0 + cs) // 16])
    K.resize_nearest(src_d, root[..., u0:u0 + cu], y_slots=root_s[:, u0 // 16:(u0 + cu) // 16])
    y_ref = torch.empty((n, h, w, oc), dtype=torch.float16, device=cuda)
    ys_ref = K.new_slots(oc, cuda, stripes=16)
    acc_ref = torch.empty((n * h * w, oc), dtype=torch.int32, device=cuda)
    # the folded form: a root holding only the skip slice and its slots
    root2 = arena[n * (h // 2) * (w // 2) * cu:].view(n, h, w, c)
    root2.fill_(float("nan"))
    root2_s = K.new_slots(c, cuda, stripes=16)
    root2[..., s0:s0 + cs] = root[..., s0:s0 + cs]
    K.amax_slots(root2[..., s0:s0 + cs], root2_s[:, s0 // 16:(s0 + cs) // 16])
    y = torch.empty_like(y_ref)
    ys = K.new_slots(oc, cuda, stripes=16)
    acc = torch.empty_like(acc_ref)
    K.set_conv1x1_stream(True, jq or 1, 1)
    try:
        K.conv2d(pc, root, y_ref, flags=K.SILU, x_slots=root_s, y_slots=ys_ref, acc_out=acc_ref)
        if not jq:
            K.set_conv1x1_stream(False)
        K.conv2d_upsampled_input(pc, root2, src_d, u0, y, x_slots=root2_s, x_up_slots=src_s, y_slots=ys,
                                 acc_out=acc)
        torch.cuda.synchronize()
    finally:
        K.set_conv1x1_stream(False)
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_ref.cpu().numpy())
    _, _, _, _, acc_o, y_o = O.w8a8_conv(cat, wt, b, desc, silu=True, fp16_engine=True)
    np.testing.assert_array_equal(acc.cpu().numpy().reshape(n, h, w, oc), nchw_to_nhwc(acc_o))
    got = nhwc_to_nchw(y.float().cpu().numpy())
    assert (np.abs(got.astype(np.float64) - y_o) <= _ulp16(y_o)).all()
    np.testing.assert_array_equal(_u32(ys).max(axis=0), _slots_of(got, oc))
    if jq:
        assert torch.equal(y, y_ref)
    # the slice was never written nor its slots
    assert torch.isnan(root2[..., u0:u0 + cu]).all()
    assert not _u32(root2_s)[:, u0 // 16:(u0 + cu) // 16].any()
