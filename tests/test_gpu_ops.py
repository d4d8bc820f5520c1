"""GPU parity of every op-level kernel against the CPU oracle (through the C ABI).

int8 tensors, int32 accumulators and amax bit patterns must match exactly;
fp16 outputs within 1e-2 of the output range; fp32 outputs within 1e-4.
aexrt_hip_conv2d without AEXRT_HIP_CONV_INT8_DYNAMIC is the reference's
prequantized int8 kernel (RT:4614-4762), which its dispatcher runs on inputs of
at least 4096 elements (RT:21478-21479); the int8 cases here have that many.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from aexrt_amd import kernels as K
from aexrt_amd import packing
from tests.helpers import c2_input, group16_weight, he_weight, nchw_to_nhwc, nhwc_to_nchw, tol_range

pytestmark = pytest.mark.gpu

FP16_TOL = 1e-2
FP32_TOL = 1e-4


def _dev_nhwc(x_nchw: np.ndarray, cuda, pad_c: int = 0):
    import torch

    a = nchw_to_nhwc(x_nchw.astype(np.float16))
    if pad_c:
        a = np.concatenate([a, np.zeros(a.shape[:3] + (pad_c,), np.float16)], axis=3)
    return torch.from_numpy(a).to(cuda)


def _u32(t) -> np.ndarray:
    return t.detach().cpu().numpy().view(np.uint32)


def test_amax_slots_and_quantize_bit_exact_c2(cuda):
    import torch

    x = c2_input(seed=1)
    xd = _dev_nhwc(x, cuda)
    slots = K.new_slots(128, cuda)
    K.amax_slots(xd, slots)
    q = K.quantize(xd, slots)
    torch.cuda.synchronize()
    got_slots = _u32(slots)
    # per-16-channel group max, exact
    want = np.array([np.float32(np.abs(x[:, g * 16:(g + 1) * 16]).max()).view(np.uint32)
                     for g in range(8)], dtype=np.uint32)
    np.testing.assert_array_equal(got_slots, want)
    a = O.amax(x)
    assert np.float32(a).view(np.uint32) == got_slots.max()
    q_ref = O.quantize(x, a)
    np.testing.assert_array_equal(nhwc_to_nchw(q.cpu().numpy()), q_ref)


@pytest.mark.parametrize("n,c,h,w,f16", [(1, 128, 40, 40, True), (2, 48, 9, 7, False), (3, 24, 5, 5, True),
                                          (1, 8, 4, 4, False)])
def test_amax_nchw_reference_strips(cuda, n, c, h, w, f16):
    import torch

    rng = np.random.default_rng(7)
    x = rng.standard_normal((n, c, h, w)).astype(np.float32) * 3
    if f16:
        x = x.astype(np.float16).astype(np.float32)
    xd = torch.from_numpy(x.astype(np.float16 if f16 else np.float32)).to(cuda)
    got = _u32(K.amax_nchw(xd))
    np.testing.assert_array_equal(got, O.amax_slots(x))


@pytest.mark.parametrize("per_group", [False, True])
@pytest.mark.parametrize("n", [1, 2])
def test_quant_pack_nchw_reference_layout(cuda, per_group, n):
    import torch

    rng = np.random.default_rng(11 + n)
    x = (rng.standard_normal((n, 64, 12, 10)) * 2).astype(np.float16).astype(np.float32)
    slots = O.amax_slots(x)
    xd = torch.from_numpy(x.astype(np.float16)).to(cuda)
    sd = torch.from_numpy(slots.view(np.int32)).to(cuda)
    got = K.quant_pack_nchw(xd, sd, per_group=per_group).cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, O.quant_pack(x, slots, per_group=per_group))


INT8_CASES = [
    # (name, n, ic, h, w, oc, k, s, seed)
    ("c2_1x1_128_256_40", 1, 128, 40, 40, 256, 1, 1, 1),
    ("1x1_32_16_ragged", 3, 32, 7, 9, 16, 1, 1, 21),
    ("3x3s1_64_64_20_b2", 2, 64, 20, 20, 64, 3, 1, 22),
    ("3x3s1_48_32_odd", 1, 48, 11, 13, 32, 3, 1, 23),
    ("3x3s2_64_128_160", 1, 64, 160, 160, 128, 3, 2, 2),
    ("3x3s2_16_32_odd", 3, 16, 17, 15, 32, 3, 2, 24),
    ("3x3s1_256_256_10", 1, 256, 10, 10, 256, 3, 1, 25),
]


def _run_int8(cuda, n, ic, h, w, oc, k, s, seed, *, silu=True, out_f32=False, x=None, residual=False):
    import torch

    rng = np.random.default_rng(seed)
    if x is None:
        x = rng.standard_normal((n, ic, h, w)).astype(np.float16).astype(np.float32)
    r = None
    wt = group16_weight(rng, oc, ic, k)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, ic, h, w, oc, k, s, k // 2)
    alg = 51 if k == 1 else (53 if s == 2 else 52)
    pc = K.prepare_conv(desc, alg, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True), b,
                        device=cuda)
    xd = _dev_nhwc(x, cuda)
    xs = K.new_slots(ic, cuda)
    K.amax_slots(xd, xs)
    _, _, oh, ow = O.out_shape(desc)
    y = torch.empty((n, oh, ow, oc), dtype=torch.float32 if out_f32 else torch.float16, device=cuda)
    ys = K.new_slots(oc, cuda)
    acc = torch.empty((n * oh * ow, oc), dtype=torch.int32, device=cuda)
    flags = (K.SILU if silu else 0) | (K.OUT_F32 if out_f32 else 0)
    rd = None
    if residual:
        r = O.round_f16(rng.standard_normal((n, oc, oh, ow)).astype(np.float32))
        rd = _dev_nhwc(r, cuda)
        flags |= K.RESIDUAL
    K.conv2d(pc, xd, y, flags=flags, x_slots=xs, y_slots=ys, acc_out=acc, residual=rd)
    torch.cuda.synchronize()
    a, qa, qw, ws, acc_ref, y_ref = O.w8a8_conv(x, wt, b, desc, silu=silu, fp16_engine=True)
    if residual:
        y_ref = y_ref + r
    got_acc = nhwc_to_nchw(acc.cpu().numpy().reshape(n, oh, ow, oc))
    return dict(acc=got_acc, acc_ref=acc_ref, y=nhwc_to_nchw(y.float().cpu().numpy()), y_ref=y_ref,
                slots=_u32(ys), y_raw=y, qa=qa, a=a)


@pytest.mark.parametrize("case", INT8_CASES, ids=[c[0] for c in INT8_CASES])
def test_int8_conv_parity(cuda, case):
    _, n, ic, h, w, oc, k, s, seed = case
    r = _run_int8(cuda, n, ic, h, w, oc, k, s, seed)
    np.testing.assert_array_equal(r["acc"], r["acc_ref"])
    err, allowed = tol_range(r["y_ref"], r["y"], FP16_TOL)
    assert err <= allowed, (err, allowed)
    # epilogue amax slots == max |fp16 output| per 16-channel group
    y = r["y"]
    want = np.array([np.float32(np.abs(y[:, g * 16:(g + 1) * 16]).max()).view(np.uint32)
                     for g in range(oc // 16)], dtype=np.uint32)
    np.testing.assert_array_equal(r["slots"], want)


def test_int8_conv_fp32_output_and_linear(cuda):
    r = _run_int8(cuda, 1, 128, 40, 40, 256, 1, 1, 1, silu=False, out_f32=True, x=c2_input(1))
    np.testing.assert_array_equal(r["acc"], r["acc_ref"])
    err, allowed = tol_range(r["y_ref"], r["y"], FP32_TOL)
    assert err <= allowed, (err, allowed)


def test_striped_slots_producer_and_consumer(cuda):
    """Striped amax slots: producers spread over the copies, readers take the max over them."""
    import torch

    n, ic, h, w, oc = 2, 64, 12, 10, 48
    rng = np.random.default_rng(81)
    x = rng.standard_normal((n, ic, h, w)).astype(np.float16).astype(np.float32)
    wt = group16_weight(rng, oc, ic, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, ic, h, w, oc, 3, 1, 1)
    pc = K.prepare_conv(desc, 52, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True), b, device=cuda)
    xd = _dev_nhwc(x, cuda)
    # producer: amax over the input into 5 stripes
    xs = K.new_slots(ic, cuda, stripes=5)
    K.amax_slots(xd, xs)
    torch.cuda.synchronize()
    want = np.array([np.float32(np.abs(x[:, g * 16:(g + 1) * 16]).max()).view(np.uint32) for g in range(ic // 16)])
    np.testing.assert_array_equal(K.slots_max(xs), want)
    # consumer: each group's max sits in a different stripe, the rest hold smaller values
    striped = np.zeros((4, ic // 16), np.uint32)
    for g in range(ic // 16):
        striped[:, g] = (want[g].view(np.float32) * np.float32(0.5)).view(np.uint32)
        striped[g % 4, g] = want[g]
    xs4 = torch.from_numpy(striped.view(np.int32)).to(cuda)
    y = torch.empty((n, h, w, oc), dtype=torch.float16, device=cuda)
    ys = K.new_slots(oc, cuda, stripes=3)
    acc = torch.empty((n * h * w, oc), dtype=torch.int32, device=cuda)
    K.conv2d(pc, xd, y, flags=K.SILU, x_slots=xs4, y_slots=ys, acc_out=acc)
    torch.cuda.synchronize()
    _, _, _, _, acc_ref, y_ref = O.w8a8_conv(x, wt, b, desc, silu=True, fp16_engine=True)
    np.testing.assert_array_equal(nhwc_to_nchw(acc.cpu().numpy().reshape(n, h, w, oc)), acc_ref)
    got = nhwc_to_nchw(y.float().cpu().numpy())
    err, allowed = tol_range(y_ref, got, FP16_TOL)
    assert err <= allowed, (err, allowed)
    np.testing.assert_array_equal(
        K.slots_max(ys), [np.float32(np.abs(got[:, g * 16:(g + 1) * 16]).max()).view(np.uint32) for g in range(3)])
    # glue producer into a striped slice of a wider tensor's slots
    big = torch.zeros((n, h, w, 96), dtype=torch.float16, device=cuda)
    bs = K.new_slots(96, cuda, stripes=4)
    K.copy(xd, big[..., 32:96], dst_slots=bs[:, 2:6])
    torch.cuda.synchronize()
    m = K.slots_max(bs)
    assert m[0] == 0 and m[1] == 0
    np.testing.assert_array_equal(m[2:6], want)


def test_int8_conv_all_zero_input(cuda):
    """amax == 0 packs zeros: output is bias (then SiLU), accumulators zero.  4096 input elements:
    the smallest tensor the reference prequantizes (RT:21478-21479)."""
    x = np.zeros((2, 32, 8, 8), np.float32)
    r = _run_int8(cuda, 2, 32, 8, 8, 16, 3, 1, 5, x=x)
    assert not r["acc"].any()
    err, allowed = tol_range(r["y_ref"], r["y"], FP16_TOL)
    assert err <= max(allowed, 1e-3)


FP16_CASES = [
    ("stem_nchw_3_16_s2", 2, 3, 64, 64, 16, 3, 2, True),
    ("1x1_64_64", 1, 64, 20, 20, 64, 1, 1, False),
    ("3x3s1_80_80_head", 1, 80, 10, 10, 80, 3, 1, False),
    ("3x3s2_64_128_160", 1, 64, 160, 160, 128, 3, 2, False),
]


@pytest.mark.parametrize("case", FP16_CASES, ids=[c[0] for c in FP16_CASES])
def test_fp16_conv_parity(cuda, case):
    import torch

    _, n, ic, h, w, oc, k, s, nchw_in = case
    rng = np.random.default_rng(31)
    x = rng.standard_normal((n, ic, h, w)).astype(np.float32)
    wt = he_weight(rng, oc, ic, k)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, ic, h, w, oc, k, s, k // 2)
    _, _, oh, ow = O.out_shape(desc)
    y = torch.empty((n, oh, ow, oc), dtype=torch.float16, device=cuda)
    if nchw_in:
        # network input: fp32 NCHW staged to fp16 NHWC with channels padded to 8
        cp = (ic + 7) // 8 * 8
        xd = torch.zeros((n, h, w, cp), dtype=torch.float16, device=cuda)
        K.nchw_f32_to_nhwc(torch.from_numpy(x).to(cuda), xd[..., :ic])
        wpad = np.zeros((oc, cp, k, k), np.float32)
        wpad[:, :ic] = wt
        dpad = O.conv_desc(n, cp, h, w, oc, k, s, k // 2)
        pc = K.prepare_conv(dpad, 5, K.SRC_RAW_F32, wpad, b, device=cuda)
        K.conv2d(pc, xd, y, flags=K.SILU)
        x_ref = O.round_f16(x)
    else:
        pc = K.prepare_conv(desc, 5, K.SRC_RAW_F32, wt, b, device=cuda)
        x_ref = O.round_f16(x)
        xd = _dev_nhwc(x_ref, cuda)
        K.conv2d(pc, xd, y, flags=K.SILU)
    torch.cuda.synchronize()
    y_ref = O.cpu_conv2d(x_ref, O.round_f16(wt), b, desc, silu=True)
    err, allowed = tol_range(y_ref, nhwc_to_nchw(y.float().cpu().numpy()), FP16_TOL)
    assert err <= allowed, (err, allowed)


@pytest.mark.parametrize("n,h,w,oc,s", [(2, 64, 64, 16, 2), (1, 37, 29, 32, 2), (3, 20, 18, 24, 1),
                                         (1, 160, 160, 16, 2)])
def test_stem_conv_reads_fp32_nchw_input(cuda, n, h, w, oc, s):
    """The first conv reading the fp32 NCHW network input itself equals the
    staged path (fp16 NHWC copy, channels padded to 8) bit for bit."""
    import torch

    rng = np.random.default_rng(61 + h)
    ic, cp = 3, 8
    x = rng.standard_normal((n, ic, h, w)).astype(np.float32)
    wt = he_weight(rng, oc, ic, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    wpad = np.zeros((oc, cp, 3, 3), np.float32)
    wpad[:, :ic] = wt
    dpad = O.conv_desc(n, cp, h, w, oc, 3, s, 1)
    pc = K.prepare_conv(dpad, 5, K.SRC_RAW_F32, wpad, b, device=cuda)
    _, _, oh, ow = O.out_shape(dpad)
    xf = torch.from_numpy(x).to(cuda)
    staged = torch.zeros((n, h, w, cp), dtype=torch.float16, device=cuda)
    K.nchw_f32_to_nhwc(xf, staged[..., :ic])
    y0 = torch.empty((n, oh, ow, oc), dtype=torch.float16, device=cuda)
    y1 = torch.empty_like(y0)
    s0, s1 = K.new_slots(oc, cuda), K.new_slots(oc, cuda)
    K.conv2d(pc, staged, y0, flags=K.SILU, y_slots=s0)
    K.set_conv_stem(K.STEM_OFF)  # the halo-tile kernel: same k order as the staged path
    try:
        K.conv2d(pc, xf, y1, flags=K.SILU | K.IN_NCHW_F32, y_slots=s1)
    finally:
        K.set_conv_stem(K.STEM_AUTO)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    np.testing.assert_array_equal(_u32(s0), _u32(s1))
    desc = O.conv_desc(n, ic, h, w, oc, 3, s, 1)
    y_ref = O.cpu_conv2d(O.round_f16(x), O.round_f16(wt), b, desc, silu=True)
    err, allowed = tol_range(y_ref, nhwc_to_nchw(y1.float().cpu().numpy()), FP16_TOL)
    assert err <= allowed, (err, allowed)


@pytest.mark.parametrize("n,ic,h,w,oc,s", [(2, 3, 64, 64, 16, 2), (1, 3, 36, 28, 32, 2), (3, 3, 20, 20, 24, 1),
                                            (1, 3, 160, 160, 16, 2), (2, 3, 33, 40, 48, 2), (1, 1, 24, 16, 16, 2),
                                            (2, 2, 17, 12, 64, 1)])
@pytest.mark.parametrize("tr", [0, 1, 2, 4, 8])
def test_stem_band_kernel(cuda, n, ic, h, w, oc, s, tr):
    """The band kernel of the first conv (whole output rows per tile, k = c * 9 + tap in one
    MFMA) against the fp32 direct conv of the fp16-rounded operands, against the halo-tile
    kernel, and its amax slot against max|y| of what it stored."""
    import torch

    rng = np.random.default_rng(71 + h + ic)
    cp = 8
    x = rng.standard_normal((n, ic, h, w)).astype(np.float32)
    wt = he_weight(rng, oc, ic, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    wpad = np.zeros((oc, cp, 3, 3), np.float32)
    wpad[:, :ic] = wt
    dpad = O.conv_desc(n, cp, h, w, oc, 3, s, 1)
    pc = K.prepare_conv(dpad, 5, K.SRC_RAW_F32, wpad, b, device=cuda)
    _, _, oh, ow = O.out_shape(dpad)
    xf = torch.from_numpy(x).to(cuda)
    y_band = torch.full((n, oh, ow, oc), float("nan"), dtype=torch.float16, device=cuda)
    y_halo = torch.empty_like(y_band)
    s_band, s_halo = K.new_slots(oc, cuda), K.new_slots(oc, cuda)
    K.set_conv_stem(K.STEM_FORCE if tr else K.STEM_AUTO, tr)
    try:
        K.conv2d(pc, xf, y_band, flags=K.SILU | K.IN_NCHW_F32, y_slots=s_band)
        K.set_conv_stem(K.STEM_OFF)
        K.conv2d(pc, xf, y_halo, flags=K.SILU | K.IN_NCHW_F32, y_slots=s_halo)
    finally:
        K.set_conv_stem(K.STEM_AUTO)
    torch.cuda.synchronize()
    got = y_band.float().cpu().numpy()
    assert np.isfinite(got).all()  # every output position written
    desc = O.conv_desc(n, ic, h, w, oc, 3, s, 1)
    y_ref = O.cpu_conv2d(O.round_f16(x), O.round_f16(wt), b, desc, silu=True)
    err, allowed = tol_range(y_ref, nhwc_to_nchw(got), FP16_TOL)
    assert err <= allowed, (err, allowed)
    err_h, _ = tol_range(y_halo.float().cpu().numpy(), got, FP16_TOL)
    assert err_h <= allowed, (err_h, allowed)
    amax_stored = np.abs(got.reshape(-1, oc)).reshape(-1, (oc + 15) // 16, 16).max(axis=(0, 2)) \
        if oc % 16 == 0 else None
    slots = _u32(s_band).view(np.float32)
    if amax_stored is not None:
        np.testing.assert_array_equal(slots, amax_stored.astype(np.float32))
    assert float(slots.max()) == float(np.abs(got).max())


def test_stem_conv_nchw_input_rejects_unsupported(cuda):
    import torch

    rng = np.random.default_rng(62)
    wpad = np.zeros((16, 8, 3, 3), np.float32)
    wpad[:, :3] = he_weight(rng, 16, 3, 3)
    b = np.zeros(16, np.float32)
    dpad = O.conv_desc(1, 8, 16, 16, 16, 3, 2, 1)
    pc = K.prepare_conv(dpad, 5, K.SRC_RAW_F32, wpad, b, device=cuda)
    xf = torch.zeros((1, 3, 16, 16), dtype=torch.float32, device=cuda)
    y = torch.empty((1, 8, 8, 16), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="NCHW"):
        K.conv2d(pc, xf, y, flags=K.IN_NCHW_F32)  # no SiLU
    x5 = torch.zeros((1, 5, 16, 16), dtype=torch.float32, device=cuda)
    with pytest.raises(RuntimeError, match="NCHW"):
        K.conv2d(pc, x5, y, flags=K.SILU | K.IN_NCHW_F32)  # more than 4 channels


def test_fp16_conv_residual_into_channel_slice(cuda):
    """Bottleneck tail: y[..., 32:64] = silu(conv(x)) + r, written into a wider tensor."""
    import torch

    rng = np.random.default_rng(41)
    n, c, h, w = 2, 32, 12, 12
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    r = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    wt = he_weight(rng, c, c, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, c).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, c, 3, 1, 1)
    pc = K.prepare_conv(desc, 5, K.SRC_RAW_F32, wt, b, device=cuda)
    big = torch.zeros((n, h, w, 96), dtype=torch.float16, device=cuda)
    slots = K.new_slots(96, cuda)
    K.conv2d(pc, _dev_nhwc(x, cuda), big[..., 32:64], flags=K.SILU | K.RESIDUAL, residual=_dev_nhwc(r, cuda),
             y_slots=slots[2:4])
    torch.cuda.synchronize()
    y_ref = O.cpu_conv2d(x, O.round_f16(wt), b, desc, silu=True) + r
    got = nhwc_to_nchw(big.float().cpu().numpy())
    err, allowed = tol_range(y_ref, got[:, 32:64], FP16_TOL)
    assert err <= allowed
    assert not got[:, :32].any() and not got[:, 64:].any()
    s = _u32(slots)
    assert s[0] == 0 and s[1] == 0 and s[4] == 0 and s[5] == 0
    for g in (2, 3):
        assert s[g] == np.float32(np.abs(got[:, g * 16:(g + 1) * 16]).max()).view(np.uint32)


def _run_fp16_residual(cuda, n, c, h, w, seed, *, tail=(32, 64), width=96):
    """silu(conv3x3(x)) + r written into channels [tail) of a wider NHWC tensor."""
    import torch

    rng = np.random.default_rng(seed)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    r = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    wt = he_weight(rng, c, c, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, c).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, c, 3, 1, 1)
    pc = K.prepare_conv(desc, 5, K.SRC_RAW_F32, wt, b, device=cuda)
    big = torch.zeros((n, h, w, width), dtype=torch.float16, device=cuda)
    slots = K.new_slots(width, cuda)
    lo, hi = tail
    K.conv2d(pc, _dev_nhwc(x, cuda), big[..., lo:hi], flags=K.SILU | K.RESIDUAL, residual=_dev_nhwc(r, cuda),
             y_slots=slots[lo // 16:(hi + 15) // 16])
    torch.cuda.synchronize()
    y_ref = O.cpu_conv2d(x, O.round_f16(wt), b, desc, silu=True) + r
    return y_ref, nhwc_to_nchw(big.float().cpu().numpy()), _u32(slots)


# Every per-wave tile the igemm kernel is instantiated for: (jn, pw, ksw).
TILES = [(1, 1, False), (1, 2, False), (1, 4, False), (2, 1, False), (2, 2, False), (2, 4, False),
         (4, 1, False), (4, 2, False), (4, 4, False), (8, 1, False), (8, 2, False),
         (1, 1, True), (2, 1, True), (4, 1, True), (8, 1, True)]


@pytest.mark.parametrize("jn,pw,ksw", TILES, ids=[f"jn{t[0]}_pw{t[1]}{'_ksw' if t[2] else ''}" for t in TILES])
def test_conv_every_tile(cuda, jn, pw, ksw):
    """Each kernel instance on shapes with partial channel tiles, ragged
    position tails, k steps that straddle taps, fp32 output and a residual."""
    K.set_conv_tile(jn, pw, ksw)
    K.set_conv3x3_halo(K.HALO_OFF)  # the 3x3 cases below run on the implicit GEMM too
    try:
        # int8 3x3 s1: OC 80 = 5 channel subtiles, M = 286, C = 48 (taps straddle k steps)
        r = _run_int8(cuda, 2, 48, 11, 13, 80, 3, 1, 71)
        np.testing.assert_array_equal(r["acc"], r["acc_ref"])
        err, allowed = tol_range(r["y_ref"], r["y"], FP16_TOL)
        assert err <= allowed, (err, allowed)
        want = np.array([np.float32(np.abs(r["y"][:, g * 16:(g + 1) * 16]).max()).view(np.uint32)
                         for g in range(5)], dtype=np.uint32)
        np.testing.assert_array_equal(r["slots"], want)
        # int8 3x3 s2, fp32 output without activation
        r = _run_int8(cuda, 1, 32, 17, 15, 32, 3, 2, 72, silu=False, out_f32=True)
        np.testing.assert_array_equal(r["acc"], r["acc_ref"])
        err, allowed = tol_range(r["y_ref"], r["y"], FP32_TOL)
        assert err <= allowed, (err, allowed)
        # int8 1x1 with a long k (K = 384, 6 steps)
        r = _run_int8(cuda, 1, 384, 6, 5, 64, 1, 1, 73)
        np.testing.assert_array_equal(r["acc"], r["acc_ref"])
        # fp16 3x3, C = 24 (8-channel halves cross taps), residual into a channel slice
        y_ref, got, slots = _run_fp16_residual(cuda, 2, 24, 9, 7, 74, tail=(48, 72), width=96)
        err, allowed = tol_range(y_ref, got[:, 48:72], FP16_TOL)
        assert err <= allowed, (err, allowed)
        assert not got[:, :48].any() and not got[:, 72:].any()
    finally:
        K.set_conv_tile(0, 0, False)
        K.set_conv3x3_halo(K.HALO_AUTO)


def _halo_fits(c, h, w, s, jn, pw, tr, tc, cc, int8, nw=4):
    """Whether a forced halo tile fits a conv: the kernel's LDS holds the
    block's weights (C/cc chunks of ceil(9cc/64) 64-k steps, jn*16 channels)
    and two input windows ((tr-1)s+3 x (tc-1)s+3 pixels x cc channels)."""
    esz = 1 if int8 else 2
    if cc % (16 if int8 else 8) or c % cc or tr * tc > 16 * nw * pw:
        return False
    spc = (9 * cc + 63) // 64
    pixels = ((tr - 1) * s + 3) * ((tc - 1) * s + 3)
    npieces = pixels * cc // 8
    wbytes = (c // cc) * spc * esz * jn * 16 * 64
    tbytes = (pixels * cc * esz + 15) // 16 * 16
    return npieces <= 8 * 64 * nw and wbytes + 2 * tbytes <= 80 * 1024 - 2048


# Halo-tile kernel tiles: (jn, pw, tile columns (0 = whole output row), channel chunk divisor, waves)
HALO_TILES = [(1, 1, 16, 1, 4), (1, 2, 0, 1, 4), (1, 4, 16, 2, 4), (2, 1, 0, 2, 4), (2, 2, 16, 1, 4),
              (2, 4, 0, 2, 4), (4, 1, 16, 1, 4), (4, 2, 0, 2, 4), (4, 4, 16, 2, 4), (4, 4, 0, 1, 4),
              (1, 1, 16, 1, 8), (2, 2, 0, 2, 8), (4, 1, 0, 1, 8), (4, 2, 16, 2, 8)]


@pytest.mark.parametrize("jn,pw,tc,ccd,nw", HALO_TILES,
                         ids=[f"jn{t[0]}_pw{t[1]}_tc{t[2]}_cc{t[3]}_w{t[4]}" for t in HALO_TILES])
def test_halo_every_tile(cuda, jn, pw, tc, ccd, nw):
    """The halo-tile 3x3 kernel on forced tiles: ragged row/column tiles,
    several channel chunks, stride 2, fp32 output, SiLU + residual, fp16."""
    ran = 0

    def force(c, h, w, s, int8):
        nonlocal ran
        oh, ow = (h - 1) // s + 1, (w - 1) // s + 1
        cols = ow if tc == 0 else tc
        rows = max(1, min(oh, 16 * nw * pw // cols))
        cc = c // ccd
        K.set_conv3x3_halo(K.HALO_FORCE if nw == 4 else K.HALO_FORCE8, jn, pw, rows, cols, max(cc, 16))
        fits = cc >= 16 and _halo_fits(c, h, w, s, jn, pw, rows, cols, cc, int8, nw)
        ran += fits
        return fits

    try:
        # int8 s1: OC 80 = 5 channel subtiles, 11 x 13 map
        if force(64, 11, 13, 1, True):
            r = _run_int8(cuda, 2, 64, 11, 13, 80, 3, 1, 91)
            np.testing.assert_array_equal(r["acc"], r["acc_ref"])
            err, allowed = tol_range(r["y_ref"], r["y"], FP16_TOL)
            assert err <= allowed, (err, allowed)
            want = np.array([np.float32(np.abs(r["y"][:, g * 16:(g + 1) * 16]).max()).view(np.uint32)
                             for g in range(5)], dtype=np.uint32)
            np.testing.assert_array_equal(r["slots"], want)
        # int8 s2, fp32 output without activation
        if force(32, 17, 15, 2, True):
            r = _run_int8(cuda, 1, 32, 17, 15, 32, 3, 2, 92, silu=False, out_f32=True)
            np.testing.assert_array_equal(r["acc"], r["acc_ref"])
            err, allowed = tol_range(r["y_ref"], r["y"], FP32_TOL)
            assert err <= allowed, (err, allowed)
        # int8 SiLU + residual (the bottleneck's fused add)
        if force(16, 20, 20, 1, True):
            r = _run_int8(cuda, 2, 16, 20, 20, 16, 3, 1, 93, residual=True)
            np.testing.assert_array_equal(r["acc"], r["acc_ref"])
            err, allowed = tol_range(r["y_ref"], r["y"], FP16_TOL)
            assert err <= allowed, (err, allowed)
        # fp16, residual into a channel slice of a wider tensor
        if force(32, 9, 7, 1, False):
            y_ref, got, slots = _run_fp16_residual(cuda, 2, 32, 9, 7, 94, tail=(48, 80), width=96)
            err, allowed = tol_range(y_ref, got[:, 48:80], FP16_TOL)
            assert err <= allowed, (err, allowed)
            assert not got[:, :48].any() and not got[:, 80:].any()
    finally:
        K.set_conv3x3_halo(K.HALO_AUTO)
    assert ran >= 3


# 80-channel fp16 tiles: every output channel in one 8-wave block (jn 5, weights up to 128 KB)
HALO80 = [(1, 64, 40, 40, 1, 2, 8, 16, 32), (2, 80, 12, 20, 1, 2, 8, 16, 40), (1, 80, 9, 11, 1, 1, 5, 11, 80),
          (2, 64, 13, 7, 2, 2, 7, 4, 64), (1, 64, 10, 10, 1, 1, 8, 16, 64)]


@pytest.mark.parametrize("n,c,h,w,s,pw,tr,tc,cc", HALO80, ids=[f"c{t[1]}_{t[2]}x{t[3]}_s{t[4]}_pw{t[5]}_cc{t[8]}"
                                                             for t in HALO80])
def test_halo_all_80_channels_in_one_block(cuda, n, c, h, w, s, pw, tr, tc, cc):
    """fp16 3x3 convs with 80 output channels on the jn 5 halo tile: against the fp32 direct conv
    of the fp16 operands, with the amax slots of what was stored."""
    import torch

    oc = 80
    rng = np.random.default_rng(97 + c + h)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    wt = he_weight(rng, oc, c, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, 3, s, 1)
    _, _, oh, ow = O.out_shape(desc)
    pc = K.prepare_conv(desc, 5, K.SRC_RAW_F32, wt, b, device=cuda)
    y = torch.full((n, oh, ow, oc), float("nan"), dtype=torch.float16, device=cuda)
    slots = K.new_slots(oc, cuda)
    K.set_conv3x3_halo(K.HALO_FORCE8, 5, pw, min(tr, oh), min(tc, ow), cc)
    try:
        K.conv2d(pc, _dev_nhwc(x, cuda), y, flags=K.SILU, y_slots=slots)
    finally:
        K.set_conv3x3_halo(K.HALO_AUTO)
    torch.cuda.synchronize()
    got = nhwc_to_nchw(y.float().cpu().numpy())
    assert np.isfinite(got).all()
    y_ref = O.cpu_conv2d(x, O.round_f16(wt), b, desc, silu=True)
    err, allowed = tol_range(y_ref, got, FP16_TOL)
    assert err <= allowed, (err, allowed)
    want = np.array([np.float32(np.abs(got[:, g * 16:(g + 1) * 16]).max()).view(np.uint32) for g in range(5)],
                    dtype=np.uint32)
    np.testing.assert_array_equal(_u32(slots), want)


# Wide-tile fp16 kernel: (n, c, h, w, oc, s, jn, pw, tr, tc, cc, silu, out_f32)
WIDE = [(2, 80, 12, 20, 80, 1, 5, 2, 6, 20, 16, True, False), (1, 64, 40, 40, 80, 1, 5, 4, 6, 40, 16, True, False),
        (1, 64, 17, 23, 64, 1, 4, 2, 8, 16, 16, True, False), (2, 128, 10, 10, 80, 1, 5, 2, 10, 10, 16, True, False),
        (1, 256, 10, 10, 64, 1, 4, 4, 10, 10, 8, True, False), (2, 48, 13, 11, 64, 2, 4, 2, 7, 6, 24, False, True),
        (1, 24, 9, 7, 56, 1, 4, 4, 9, 7, 8, False, False)]


@pytest.mark.parametrize("case", WIDE, ids=[f"c{t[1]}_{t[2]}x{t[3]}_oc{t[4]}_s{t[5]}_jn{t[6]}_pw{t[7]}_cc{t[10]}"
                                            for t in WIDE])
def test_wide_tile_fp16_conv(cuda, case):
    """The wide-tile fp16 3x3 kernel (every output channel per wave, weights streamed per
    channel chunk) on forced tiles: ragged tiles, several chunks, stride 2, fp32 output."""
    import torch

    n, c, h, w, oc, s, jn, pw, tr, tc, cc, silu, out_f32 = case
    rng = np.random.default_rng(131 + c + h + oc)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    wt = he_weight(rng, oc, c, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, 3, s, 1)
    _, _, oh, ow = O.out_shape(desc)
    pc = K.prepare_conv(desc, 5, K.SRC_RAW_F32, wt, b, device=cuda)
    y = torch.full((n, oh, ow, oc), float("nan"), dtype=torch.float32 if out_f32 else torch.float16, device=cuda)
    slots = K.new_slots(oc, cuda)
    flags = (K.SILU if silu else 0) | (K.OUT_F32 if out_f32 else 0)
    K.set_conv3x3_halo(K.HALO_FORCE_WIDE, jn, pw, min(tr, oh), min(tc, ow), cc)
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
    g = (oc + 15) // 16
    want = np.array([np.float32(np.abs(got[:, k * 16:(k + 1) * 16]).max()).view(np.uint32) for k in range(g)],
                    dtype=np.uint32)
    np.testing.assert_array_equal(_u32(slots), want)


def test_halo_forced_tile_that_does_not_fit_fails(cuda):
    K.set_conv3x3_halo(K.HALO_FORCE, 1, 1, 4, 16, 48)  # C = 64 is not a multiple of 48
    try:
        with pytest.raises(RuntimeError):
            _run_int8(cuda, 1, 64, 8, 8, 16, 3, 1, 95)
    finally:
        K.set_conv3x3_halo(K.HALO_AUTO)
    r = _run_int8(cuda, 1, 64, 8, 8, 16, 3, 1, 95)
    np.testing.assert_array_equal(r["acc"], r["acc_ref"])


WINO_CASES = [
    ("64_64_20", 1, 64, 20, 20, 64),
    ("96_64_20x18", 1, 96, 20, 18, 64),
    ("32_48_b2_8x6", 2, 32, 8, 6, 48),
    ("64_64_40", 1, 64, 40, 40, 64),
]


@pytest.mark.parametrize("case", WINO_CASES, ids=[c[0] for c in WINO_CASES])
def test_winograd_parity(cuda, case):
    import torch

    _, n, ic, h, w, oc = case
    rng = np.random.default_rng(51)
    x = O.round_f16(rng.standard_normal((n, ic, h, w)).astype(np.float32))
    wt = he_weight(rng, oc, ic, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, ic, h, w, oc, 3, 1, 1)
    pc = K.prepare_conv(desc, 40, K.SRC_LAYOUT_WINO_F16, packing.pack_winograd_f2x2_fp16(wt), b, device=cuda)
    y = torch.empty((n, h, w, oc), dtype=torch.float16, device=cuda)
    K.conv2d(pc, _dev_nhwc(x, cuda), y, flags=K.SILU)
    torch.cuda.synchronize()
    u = O.winograd_weight(wt, to_f16=True)
    y_ref = O.winograd_conv(x, u, b, desc)
    err, allowed = tol_range(y_ref, nhwc_to_nchw(y.float().cpu().numpy()), FP16_TOL)
    assert err <= allowed, (err, allowed)


@pytest.mark.parametrize("n,c,h,w", [(2, 32, 10, 10), (1, 128, 20, 20), (3, 16, 13, 7), (1, 64, 1, 5)])
def test_sppf_maxpool_equals_three_pools(cuda, n, c, h, w):
    """The fused SPPF kernel writes exactly the three chained 5x5 pools (and
    their amax slots) into slices of one concat tensor."""
    import torch

    rng = np.random.default_rng(71 + h)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32) * 3)
    x[:, :, 0, 0] = -1e4  # a large negative corner pixel must not leak through the padding
    xd = _dev_nhwc(x, cuda)
    cat = torch.zeros((n, h, w, 4 * c), dtype=torch.float16, device=cuda)
    slots = K.new_slots(4 * c, cuda, stripes=8)
    g = c // 16
    K.sppf_maxpool(xd, cat[..., c:2 * c], cat[..., 2 * c:3 * c], cat[..., 3 * c:],
                   slots=(slots[:, g:2 * g], slots[:, 2 * g:3 * g], slots[:, 3 * g:]))
    torch.cuda.synchronize()
    got = nhwc_to_nchw(cat.float().cpu().numpy())
    p1 = O.maxpool(x, 5, 1, 2)
    p2 = O.maxpool(p1, 5, 1, 2)
    p3 = O.maxpool(p2, 5, 1, 2)
    np.testing.assert_array_equal(got[:, c:2 * c], p1)
    np.testing.assert_array_equal(got[:, 2 * c:3 * c], p2)
    np.testing.assert_array_equal(got[:, 3 * c:], p3)
    assert not got[:, :c].any()
    want = np.concatenate([np.zeros((n, c, h, w), np.float32), p1, p2, p3], axis=1)
    m = K.slots_max(slots)
    np.testing.assert_array_equal(m, [np.float32(np.abs(want[:, k * 16:(k + 1) * 16]).max()).view(np.uint32)
                                      for k in range(4 * g)])


def test_resize_nearest_general_scale(cuda):
    """Non-2x scales use the general kernel: floor(o * in / out) sources."""
    import torch

    rng = np.random.default_rng(72)
    x = O.round_f16(rng.standard_normal((2, 16, 5, 7)).astype(np.float32))
    up = torch.empty((2, 15, 14, 16), dtype=torch.float16, device=cuda)
    K.resize_nearest(_dev_nhwc(x, cuda), up)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(nhwc_to_nchw(up.float().cpu().numpy()), O.resize_nearest(x, 15, 14))


def test_glue_ops(cuda):
    import torch

    rng = np.random.default_rng(61)
    x = O.round_f16(rng.standard_normal((2, 64, 10, 10)).astype(np.float32))
    xd = _dev_nhwc(x, cuda)
    # maxpool k5 s1 p2 (SPPF)
    y = torch.empty_like(xd)
    ys = K.new_slots(64, cuda)
    K.maxpool(xd, y, 5, 1, 2, y_slots=ys)
    # nearest resize x2
    up = torch.empty((2, 20, 20, 64), dtype=torch.float16, device=cuda)
    K.resize_nearest(xd, up)
    # add
    s = torch.empty_like(xd)
    K.add(xd, y, s)
    # copy into a channel slice
    big = torch.zeros((2, 10, 10, 128), dtype=torch.float16, device=cuda)
    K.copy(xd, big[..., 64:])
    torch.cuda.synchronize()
    mp = O.maxpool(x, 5, 1, 2)
    np.testing.assert_array_equal(nhwc_to_nchw(y.float().cpu().numpy()), mp)
    np.testing.assert_array_equal(_u32(ys), [np.float32(np.abs(mp[:, g * 16:(g + 1) * 16]).max()).view(np.uint32)
                                             for g in range(4)])
    np.testing.assert_array_equal(nhwc_to_nchw(up.float().cpu().numpy()), O.resize_nearest(x, 20, 20))
    np.testing.assert_array_equal(nhwc_to_nchw(s.float().cpu().numpy()), O.round_f16(x + mp))
    np.testing.assert_array_equal(nhwc_to_nchw(big.float().cpu().numpy())[:, 64:], x)
    # layout round trip
    xf = torch.from_numpy(rng.standard_normal((1, 16, 5, 7)).astype(np.float32)).to(cuda)
    nh = torch.empty((1, 5, 7, 16), dtype=torch.float16, device=cuda)
    K.nchw_f32_to_nhwc(xf, nh)
    back = K.nhwc_to_nchw_f32(nh)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(back.cpu().numpy(), O.round_f16(xf.cpu().numpy()))
