"""Pins the CPU oracle before anything is compared against it.

Each check is chosen so that a plausible slip in the restatement (dropped
term, wrong index or sign, transposed operand, wrong rounding) fails: golden
vectors of the reference's own known-answer tests, brute force on small
inputs, closed-form special cases and library routines.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- fp16
def test_f16_conversion_matches_numpy_everywhere():
    rng = np.random.default_rng(0)
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                        6.1035156e-05, 6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08,
                        8.940697e-08, 1e-12, 0.5, 1.5, 2.5, 1.0009766, 1.00048828125],
                       dtype=np.float32)
    vals = np.concatenate([special, rng.standard_normal(20000).astype(np.float32) * 100,
                           (rng.random(20000).astype(np.float32) * 1e-4),
                           rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    vals = vals[np.isfinite(vals) | np.isinf(vals)]
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).astype(np.float32)
    got = O.round_f16(vals)
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all(), vals[~same][:8]


# ---------------------------------------------------------------- a1 amax
@pytest.mark.parametrize("shape", [(1, 32, 5, 7), (2, 48, 3, 3), (3, 24, 4, 4), (1, 8, 2, 2)])
def test_amax_slots_brute_force_strips(shape):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(shape).astype(np.float32)
    n, c, h, w = shape
    flat = x.reshape(-1)
    strip = 16 * n * h * w
    want = [np.abs(flat[g * strip:(g + 1) * strip]).max() for g in range(c // 16)]
    got = O.amax_slots(x).view(np.float32)
    assert got[0] == (max(want) if want else 0.0)
    np.testing.assert_array_equal(got[1:], np.array(want, dtype=np.float32))
    assert O.amax(x) == np.abs(x).max()


# ---------------------------------------------------------------- a2 quantize
def test_quantize_special_values():
    amax = 2.0
    s = np.float32(127.0) / np.float32(amax)
    # exact ties: x*s = k + 0.5 -> round half to even
    ties = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 126.5], dtype=np.float32) / s
    assert np.all((ties * s) == np.array([0.5, 1.5, 2.5, -0.5, -1.5, 126.5], np.float32))
    q = O.quantize(ties, amax)
    np.testing.assert_array_equal(q, [0, 2, 2, 0, -2, 126])
    # +-amax -> +-127, 0 -> 0
    np.testing.assert_array_equal(O.quantize(np.array([2.0, -2.0, 0.0], np.float32), amax), [127, -127, 0])
    # amax == 0 packs zero
    np.testing.assert_array_equal(O.quantize(np.array([0.0, 0.0], np.float32), 0.0), [0, 0])


def test_quantize_uses_127_over_amax_not_reciprocal_of_scale():
    # x * (127/amax) and x / (amax/127) round differently next to .5 ties;
    # the oracle must follow the reference's s = 127/amax (RT:3337) --
    # planted-mistake check on values built right at those ties.
    a = np.float32(3.7)
    s = np.float32(127.0) / a
    d = a / np.float32(127.0)
    xs = []
    for k in range(127):
        x = np.float32((k + 0.5) / float(s))
        for _ in range(4):
            x = np.nextafter(x, np.float32(-1))
        for _ in range(9):
            if np.rint(x * s) != np.rint(x / d):
                xs.append(x)
            x = np.nextafter(x, np.float32(200))
    x = np.array(xs, dtype=np.float32)
    assert x.size > 0
    right = np.rint(x * s).astype(np.int8)
    wrong = np.rint(x / d).astype(np.int8)
    assert (right != wrong).all()
    np.testing.assert_array_equal(O.quantize(x, a), right)


@pytest.mark.parametrize("per_group", [False, True])
def test_quant_pack_layout_against_numpy_gather(per_group):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((2, 32, 3, 5)) * 3).astype(np.float32)
    slots = O.amax_slots(x)
    packed = O.quant_pack(x, slots, per_group=per_group)
    q = O.unpack_nc4hw4(packed, 2, 32, 3, 5)
    if per_group:
        amax_c = np.repeat(slots[1:].view(np.float32), 16)
        s = (np.float32(127.0) / amax_c).astype(np.float32)[None, :, None, None]
        want = np.rint((x * s).astype(np.float32))
        want = (want.astype(np.int64) & 0xFF).astype(np.uint8).view(np.int8)
    else:
        want = O.quantize(x, slots.view(np.float32)[0])
    np.testing.assert_array_equal(q, want)


def test_fused_pg16_reduces_to_strip_amax_at_batch_one():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1, 32, 6, 6)).astype(np.float32)
    packed, slots = O.quant_fused_pg16(x)
    ref_slots = O.amax_slots(x)
    np.testing.assert_array_equal(slots[1:], ref_slots[1:])
    np.testing.assert_array_equal(packed, O.quant_pack(x, ref_slots, per_group=True))


# ---------------------------------------------------------------- a4 weights
def test_weight_quant_rounding_zero_rows_and_clamp():
    # row 0: scale = 2/127; w*inv hits exact .5 ties -> half away from zero
    s = np.float32(2.0) / np.float32(127.0)
    inv = np.float32(1.0) / s
    row0 = np.array([2.0, 0.5 / inv, -0.5 / inv, 1.5 / inv, -2.5 / inv, 0.0], np.float32)
    assert (row0[1] * inv) == np.float32(0.5) and (row0[4] * inv) == np.float32(-2.5)
    row1 = np.zeros(6, np.float32)
    w = np.stack([row0, row1])
    q, sc = O.weight_quant(w, fp16_round=False)
    np.testing.assert_array_equal(q[0], [127, 1, -1, 2, -3, 0])
    np.testing.assert_array_equal(q[1], 0)
    assert sc[0] == s and sc[1] == 1.0


def test_weight_quant_fp16_prerounding():
    w = np.array([[1.0, 1.0 + 2.0 ** -12, 0.333333343]], np.float32)
    q16, s16 = O.weight_quant(w, fp16_round=True)
    q32, s32 = O.weight_quant(w, fp16_round=False)
    assert s16[0] == np.float32(np.float16(1.0 + 2.0 ** -12)) / np.float32(127.0)
    assert s32[0] == np.float32(1.0 + 2.0 ** -12) / np.float32(127.0)


def test_weight_quant_matches_float64_closed_form_away_from_ties():
    rng = np.random.default_rng(6)
    w = rng.standard_normal((16, 72)).astype(np.float32)
    q, s = O.weight_quant(w, fp16_round=False)
    p = w.astype(np.float64) / (np.abs(w).max(axis=1, keepdims=True) / 127.0)
    safe = np.abs(np.abs(p) - np.floor(np.abs(p)) - 0.5) > 1e-3
    want = np.clip(np.sign(p) * np.floor(np.abs(p) + 0.5), -127, 127)
    np.testing.assert_array_equal(q[safe], want[safe])


# ---------------------------------------------------------------- a5 conv int8
def _im2col_acc(qa, qw, desc):
    n, c, h, w = qa.shape
    oc, _, kh, kw = qw.shape
    s, p = int(desc[9]), int(desc[11])
    oh, ow = int(desc[5]), int(desc[6])
    xp = np.zeros((n, c, h + 2 * p, w + 2 * p), np.int64)
    xp[:, :, p:p + h, p:p + w] = qa
    cols = np.zeros((n, c, kh, kw, oh, ow), np.int64)
    for ky in range(kh):
        for kx in range(kw):
            cols[:, :, ky, kx] = xp[:, :, ky:ky + s * oh:s, kx:kx + s * ow:s]
    return np.einsum("nckluv,ockl->nouv", cols, qw.astype(np.int64)).astype(np.int32)


@pytest.mark.parametrize("k,s", [(1, 1), (3, 1), (3, 2)])
def test_conv_int8_acc_equals_int64_einsum(k, s):
    rng = np.random.default_rng(7)
    qa = rng.integers(-127, 128, (2, 16, 9, 7), dtype=np.int8)
    qw = rng.integers(-127, 128, (8, 16, k, k), dtype=np.int8)
    desc = O.conv_desc(2, 16, 9, 7, 8, k, s, k // 2)
    np.testing.assert_array_equal(O.conv_int8_acc(qa, qw, desc), _im2col_acc(qa, qw, desc))


def test_conv_int8_acc_transposed_weight_is_caught():
    rng = np.random.default_rng(8)
    qa = rng.integers(-127, 128, (1, 16, 5, 5), dtype=np.int8)
    qw = rng.integers(-127, 128, (16, 16, 3, 3), dtype=np.int8)
    desc = O.conv_desc(1, 16, 5, 5, 16, 3, 1, 1)
    ref = _im2col_acc(qa, qw, desc)
    assert not np.array_equal(O.conv_int8_acc(qa, np.ascontiguousarray(qw.transpose(1, 0, 2, 3)), desc), ref)
    assert not np.array_equal(O.conv_int8_acc(qa, np.ascontiguousarray(qw[:, :, ::-1, ::-1]), desc), ref)


def test_epilogue_against_float64():
    rng = np.random.default_rng(9)
    acc = rng.integers(-200000, 200000, (1, 8, 4, 4), dtype=np.int32)
    ws = rng.random(8).astype(np.float32) * 0.01
    b = rng.uniform(-0.1, 0.1, 8).astype(np.float32)
    amax = 3.7
    y = O.conv_int8_epilogue(acc, amax, ws, b, silu=True)
    v = acc * (amax / 127.0) * ws[None, :, None, None].astype(np.float64) + b[None, :, None, None]
    ref = v / (1.0 + np.exp(-v))
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)
    y_lin = O.conv_int8_epilogue(acc, amax, ws, b, silu=False)
    np.testing.assert_allclose(y_lin, v, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- a6/a8/a9
def _chain_inputs(seed, n=1, c=32, h=6, w=6, oc=8, k=3, s=1):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    wt = rng.standard_normal((oc, c, k, k)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, oc).astype(np.float32)
    desc = O.conv_desc(n, c, h, w, oc, k, s, k // 2)
    qw, ws = O.weight_quant(wt, fp16_round=False)
    return x, qw, ws, b, desc


@pytest.mark.parametrize("k,s", [(1, 1), (3, 1), (3, 2)])
def test_pg16_equals_per_tensor_when_groups_share_amax(k, s):
    x, qw, ws, b, desc = _chain_inputs(10, k=k, s=s)
    # force every 16-channel group to the same amax
    x[:, :, 0, 0] = 0.0
    x[:, 0, 0, 0] = 5.0
    x[:, 16, 0, 0] = 5.0
    slots = O.amax_slots(x)
    assert len(set(slots.tolist())) == 1
    packed = O.quant_pack(x, slots, per_group=True)
    y_pg = O.conv_int8_pg(packed, qw, desc, slots, ws, b, silu=True)
    qa = O.quantize(x, 5.0)
    y_pt = O.conv_int8_epilogue(O.conv_int8_acc(qa, qw, desc), 5.0, ws, b, silu=True)
    np.testing.assert_allclose(y_pg, y_pt, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("k,s", [(1, 1), (3, 1), (3, 2)])
@pytest.mark.parametrize("per_group", [False, True])
def test_ksplit_sums_to_unsplit(k, s, per_group):
    x, qw, ws, b, desc = _chain_inputs(11, c=64, k=k, s=s)
    slots = O.amax_slots(x)
    packed = O.quant_pack(x, slots, per_group=per_group)
    y_ks = O.conv_int8_ksplit(packed, qw, desc, slots, ws, b, silu=False, per_group=per_group)
    if per_group:
        y_full = O.conv_int8_pg(packed, qw, desc, slots, ws, b, silu=False)
    else:
        a = slots.view(np.float32)[0]
        y_full = O.conv_int8_epilogue(O.conv_int8_acc(O.quantize(x, a), qw, desc), a, ws, b, silu=False)
    np.testing.assert_allclose(y_ks, y_full, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("k,s", [(1, 1), (3, 1), (3, 2)])
def test_dynamic_fallback_is_close_to_float_conv(k, s):
    x, qw, ws, b, desc = _chain_inputs(12, c=32, k=k, s=s)
    y = O.conv_int8_dynamic(x, qw, desc, ws, b, silu=False)
    wq = qw.astype(np.float32) * ws[:, None, None, None]
    ref = O.cpu_conv2d(x, wq, b, desc, silu=False)
    err = np.abs(y - ref).max()
    assert err <= 0.02 * (ref.max() - ref.min())


def test_dynamic_fallback_exact_when_inputs_are_grid_values():
    # every 4-channel group has amax 127 and integer values -> quantization is
    # exact, so the dynamic path equals the float conv of the int values.
    rng = np.random.default_rng(13)
    x = rng.integers(-120, 121, (1, 16, 5, 5)).astype(np.float32)
    x[:, :, :, :] = np.where(np.arange(16)[None, :, None, None] % 4 == 0, 127.0, x)
    qw = rng.integers(-127, 128, (8, 16, 1, 1), dtype=np.int8)
    ws = np.ones(8, np.float32)
    b = np.zeros(8, np.float32)
    desc = O.conv_desc(1, 16, 5, 5, 8, 1, 1, 0)
    y = O.conv_int8_dynamic(x, qw, desc, ws, b, silu=False)
    ref = np.einsum("nchw,oc->nohw", x.astype(np.float64), qw[:, :, 0, 0].astype(np.float64))
    np.testing.assert_allclose(y, ref, rtol=1e-6)


def _unpack_nc4(packed, n, c, h, w):
    """NC/4HW4 uint32 words -> int8 NCHW (channel 4*icg + j in byte j of word (n, icg, pos))."""
    b = np.asarray(packed, np.uint32).reshape(n, c // 4, h * w).view(np.uint8).reshape(n, c // 4, h * w, 4)
    return b.transpose(0, 1, 3, 2).reshape(n, c, h, w).view(np.int8)


@pytest.mark.parametrize("k,s", [(1, 1), (3, 1), (3, 2)])
def test_pg16_equals_float64_group_dequant_with_distinct_group_amax(k, s):
    """or_conv_int8_pg against the closed form of per-16-channel activation scales: each channel's
    quantized value times amax[1 + c/16]/127, each weight times its scale, a float64 convolution.
    The four groups have distinct maxima, so a wrong group index (c/4, c/16 + 1, ...) fails."""
    rng = np.random.default_rng(21)
    n, c, h, w, oc = 2, 64, 7, 6, 16
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    for g, m in enumerate((0.25, 3.0, 1.0, 9.5)):
        x[:, 16 * g:16 * (g + 1)] *= m / np.abs(x[:, 16 * g:16 * (g + 1)]).max()
    wt = rng.standard_normal((oc, c, k, k)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, oc).astype(np.float32)
    desc = O.conv_desc(n, c, h, w, oc, k, s, k // 2)
    qw, ws = O.weight_quant(wt, fp16_round=False)
    slots = O.amax_slots(x)
    group_amax = slots.view(np.float32)[1:]
    assert len(set(group_amax.tolist())) == 4
    packed = O.quant_pack(x, slots, per_group=True)
    y = O.conv_int8_pg(packed, qw, desc, slots, ws, b, silu=False)
    qa = _unpack_nc4(packed, n, c, h, w).astype(np.float64)
    xa = qa * (np.repeat(group_amax.astype(np.float64), 16) / 127.0)[None, :, None, None]
    wa = qw.astype(np.float64) * ws.astype(np.float64)[:, None, None, None]
    import torch
    ref = torch.nn.functional.conv2d(torch.from_numpy(xa), torch.from_numpy(wa), torch.from_numpy(b.astype(np.float64)),
                                     stride=s, padding=k // 2).numpy()
    np.testing.assert_allclose(y, ref, rtol=2e-5, atol=2e-5 * np.abs(ref).max())
    # the per-tensor scale for every group is far off (planted mistake)
    xt = qa * (float(group_amax.max()) / 127.0)
    wrong = torch.nn.functional.conv2d(torch.from_numpy(xt), torch.from_numpy(wa), stride=s, padding=k // 2).numpy()
    assert np.abs(wrong - ref).max() > 100 * np.abs(y - ref).max()


@pytest.mark.parametrize("k,s", [(1, 1), (3, 1), (3, 2)])
def test_dynamic_fallback_exact_with_power_of_two_group_scales(k, s):
    """Every 4-channel group holds integers times a group-specific 2^-e with 127 * 2^-e present in
    each of its windows (one pixel for 1x1, the 3x3 taps otherwise): 127/amax and amax/127 are
    exact powers of two, quantization is exact, and the dynamic conv equals the float64
    convolution of x.  A scale shared across groups, or taken over the wrong taps, is inexact."""
    rng = np.random.default_rng(22)
    n, c, h, w, oc = 1, 16, 6, 5, 8
    e = np.array([0, 3, 1, 5])  # group g values are ints * 2^-e[g]
    q = rng.integers(-126, 127, (n, c, h, w)).astype(np.float64)
    q[:, 0::4] = 127.0  # channel 4g holds the group's maximum at every position
    x = (q * (2.0 ** -np.repeat(e, 4))[None, :, None, None]).astype(np.float32)
    qw = rng.integers(-127, 128, (oc, c, k, k), dtype=np.int8)
    ws = np.full(oc, 0.5, np.float32)
    b = np.zeros(oc, np.float32)
    desc = O.conv_desc(n, c, h, w, oc, k, s, k // 2)
    y = O.conv_int8_dynamic(x, qw, desc, ws, b, silu=False)
    import torch
    ref = 0.5 * torch.nn.functional.conv2d(torch.from_numpy(x.astype(np.float64)),
                                           torch.from_numpy(qw.astype(np.float64)), stride=s, padding=k // 2).numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-6)


def test_network_int8_convs_below_4096_elements_take_the_dynamic_path():
    """oracle.network follows RT:21478-21479: an int8 conv whose input has fewer than 4096 elements
    is the dynamic conv, at 4096 and above the per-tensor chain."""
    from oracle import network as ON
    rng = np.random.default_rng(23)
    w = rng.standard_normal((16, 32, 3, 3)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, 16).astype(np.float32)
    attrs = dict(strides=[1, 1], pads=[1, 1, 1, 1])
    for shape, dynamic in (((1, 32, 11, 11), True), ((1, 32, 8, 16), False), ((2, 32, 8, 8), False)):
        x = O.round_f16(rng.standard_normal(shape).astype(np.float32))
        y = ON.conv_layer(x, w, b, attrs, int8=True, silu=True)
        desc = O.conv_desc(*shape, 16, 3, 1, 1)
        qw, ws = O.weight_quant(w, fp16_round=True)
        dyn = O.conv_int8_dynamic(x, qw, desc, ws, O.round_f16(b), True)
        pt = O.w8a8_conv(x, w, b, desc, silu=True, fp16_engine=True)[-1]
        assert np.array_equal(y, dyn if dynamic else pt), shape
        assert not np.array_equal(dyn, pt)


# ---------------------------------------------------------------- a15 cpu conv
@pytest.mark.parametrize("k,s,p", [(1, 1, 0), (3, 1, 1), (3, 2, 1), (6, 2, 2)])
def test_cpu_conv2d_against_torch(k, s, p):
    import torch

    rng = np.random.default_rng(14)
    x = rng.standard_normal((2, 8, 11, 9)).astype(np.float32)
    w = rng.standard_normal((6, 8, k, k)).astype(np.float32)
    b = rng.standard_normal(6).astype(np.float32)
    desc = O.conv_desc(2, 8, 11, 9, 6, k, s, p)
    y = O.cpu_conv2d(x, w, b, desc, silu=True)
    ref = torch.nn.functional.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                                     torch.from_numpy(b).double(), stride=s, padding=p)
    ref = (ref * torch.sigmoid(ref)).numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5)
    y4 = O.cpu_conv2d(x, w, b, desc, silu=True, threads=4)
    np.testing.assert_array_equal(y, y4)


# ---------------------------------------------------------------- a12 winograd
def test_winograd_weight_matches_reference_kat():
    g = np.load(GOLDEN / "winograd_f2x2_kat.npz")
    w = (np.arange(32 * 32 * 9, dtype=np.float32).reshape(32, 32, 3, 3) / 4096.0)
    u16 = O.winograd_weight(w, to_f16=True)
    np.testing.assert_array_equal(u16.astype(np.float16).view(np.uint16), g["expected_f16_bits"])
    u32 = O.winograd_weight(w, to_f16=False)
    np.testing.assert_array_equal(u32, g["expected_f32"])


def test_winograd_conv_equals_direct_conv_with_fp32_transform():
    rng = np.random.default_rng(15)
    x = rng.standard_normal((2, 16, 8, 10)).astype(np.float32)
    w = O.round_f16(rng.standard_normal((12, 16, 3, 3)).astype(np.float32))
    b = rng.uniform(-0.1, 0.1, 12).astype(np.float32)
    desc = O.conv_desc(2, 16, 8, 10, 12, 3, 1, 1)
    y = O.winograd_conv(x, O.winograd_weight(w, to_f16=False), b, desc)
    ref = O.cpu_conv2d(x, w, b, desc, silu=True)
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-4)


def test_winograd_conv_detects_swapped_output_transform():
    rng = np.random.default_rng(16)
    x = rng.standard_normal((1, 8, 4, 4)).astype(np.float32)
    w = rng.standard_normal((4, 8, 3, 3)).astype(np.float32)
    b = np.zeros(4, np.float32)
    desc = O.conv_desc(1, 8, 4, 4, 4, 3, 1, 1)
    u = O.winograd_weight(w, to_f16=False)
    ref = O.cpu_conv2d(x, O.round_f16(w), b, desc, silu=True)
    # a transposed U (rows/cols swapped) must not reproduce the direct conv
    y_bad = O.winograd_conv(x, np.ascontiguousarray(u.transpose(0, 1, 3, 2)), b, desc)
    assert np.abs(y_bad - ref).max() > 1e-2


# ---------------------------------------------------------------- glue
def test_maxpool_and_resize_against_torch():
    import torch

    rng = np.random.default_rng(17)
    x = rng.standard_normal((2, 4, 7, 9)).astype(np.float32)
    mp = O.maxpool(x, 5, 1, 2)
    ref = torch.nn.functional.max_pool2d(torch.from_numpy(x), 5, 1, 2).numpy()
    np.testing.assert_array_equal(mp, ref)
    up = O.resize_nearest(x, 14, 18)
    ref_up = torch.nn.functional.interpolate(torch.from_numpy(x), size=(14, 18), mode="nearest").numpy()
    np.testing.assert_array_equal(up, ref_up)


def test_fused_pg16_uses_image0_group_max_at_batch_gt_one():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((3, 32, 5, 4)).astype(np.float32)
    x[1:] *= 3.0
    packed, slots = O.quant_fused_pg16(x)
    s0 = O.amax_slots(x[:1])  # image 0's channel groups (N = 1: strips = groups)
    np.testing.assert_array_equal(slots[1:], s0[1:])
    for n in range(3):
        want = O.quant_pack(x[n:n + 1], s0, per_group=True)
        np.testing.assert_array_equal(packed.reshape(3, -1)[n], want)


# ---- YOLO postprocess ----------------------------------------------------------

def _scores_classes(d):
    return [round(float(v), 2) for v in d[:, 4]], [int(v) for v in d[:, 5]]


def test_yolo_post_reference_gpu_kat():
    """tests/test_runtime.py:3412-3448 of the reference (its GPU decode + NMS + top-k)."""
    out = np.zeros((6, 5), dtype="float32")
    out[:4, 0] = [10, 10, 10, 10]
    out[:4, 1] = [11, 10, 10, 10]
    out[:4, 2] = [50, 50, 8, 8]
    out[:4, 3] = [80, 80, 8, 8]
    out[:4, 4] = [70, 70, 8, 8]
    out[4:, 0] = [0.9, 0.1]
    out[4:, 1] = [0.8, 0.1]
    out[4:, 2] = [0.1, 0.7]
    out[4:, 3] = [0.2, 0.1]
    out[4:, 4] = [0.4, 0.2]
    d = O.yolo_decode_nms_topk(out, classes=2, conf=0.25, iou=0.5, max_candidates=8, max_detections=4)
    assert d.shape[0] == 3
    assert _scores_classes(d) == ([0.9, 0.7, 0.4], [0, 1, 0])
    np.testing.assert_array_equal(d[0, :4], np.float32([5, 5, 15, 15]))


def test_yolo_post_reference_cpu_kats():
    """tests/test_runtime.py:442-463 of the reference (channels first; channels last with objectness)."""
    out = np.zeros((1, 6, 4), dtype="float32")
    out[0, :4, 0] = [10, 10, 10, 10]
    out[0, :4, 1] = [11, 10, 10, 10]
    out[0, :4, 2] = [50, 50, 8, 8]
    out[0, :4, 3] = [80, 80, 8, 8]
    out[0, 4:, 0] = [0.9, 0.1]
    out[0, 4:, 1] = [0.8, 0.1]
    out[0, 4:, 2] = [0.1, 0.7]
    out[0, 4:, 3] = [0.2, 0.1]
    d = O.yolo_decode_nms_topk(out, classes=2, conf=0.25, iou=0.5)
    assert list(zip(_scores_classes(d)[1], _scores_classes(d)[0])) == [(0, 0.9), (1, 0.7)]
    out = np.zeros((1, 5, 7), dtype="float32")
    out[0, 0, :4] = [10, 10, 10, 10]
    out[0, 0, 4:] = [0.5, 0.9, 0.1]
    out[0, 1, :4] = [50, 50, 8, 8]
    out[0, 1, 4:] = [0.8, 0.1, 0.7]
    d = O.yolo_decode_nms_topk(out, layout=2, classes=2, has_objectness=True, conf=0.25, iou=0.5)
    assert list(zip(_scores_classes(d)[1], _scores_classes(d)[0])) == [(1, 0.56), (0, 0.45)]


def _greedy_nms_reference(out, classes, conf, iou):
    """The reference's CPU yolo_postprocess (src/aexrt/yolo.py:92-140, 996-1018), restated with numpy."""
    y = out
    boxes = y[:4].T.astype(np.float64)
    scores = y[4:4 + classes].T
    cls = np.argmax(scores, axis=1)
    sc = scores[np.arange(scores.shape[0]), cls]
    keep = sc >= conf
    b = boxes[keep]
    xyxy = np.stack([b[:, 0] - b[:, 2] / 2, b[:, 1] - b[:, 3] / 2, b[:, 0] + b[:, 2] / 2, b[:, 1] + b[:, 3] / 2], 1)
    sc, cls = sc[keep], cls[keep]
    res = []
    for c in np.unique(cls):
        idx = np.where(cls == c)[0]
        order = idx[np.argsort(-sc[idx], kind="stable")]
        while order.size:
            i = order[0]
            res.append((float(sc[i]), int(c)))
            rest = order[1:]
            x1 = np.maximum(xyxy[i, 0], xyxy[rest, 0]); y1 = np.maximum(xyxy[i, 1], xyxy[rest, 1])
            x2 = np.minimum(xyxy[i, 2], xyxy[rest, 2]); y2 = np.minimum(xyxy[i, 3], xyxy[rest, 3])
            inter = np.maximum(0, x2 - x1) * np.maximum(0, y2 - y1)
            a0 = (xyxy[i, 2] - xyxy[i, 0]) * (xyxy[i, 3] - xyxy[i, 1])
            a1 = (xyxy[rest, 2] - xyxy[rest, 0]) * (xyxy[rest, 3] - xyxy[rest, 1])
            order = rest[inter / np.maximum(a0 + a1 - inter, 1e-7) <= iou]
    return sorted(res, key=lambda t: -t[0])


def _pair_clusters(rng, n_pairs, classes):
    """Boxes in far-apart pairs (each pair overlapping or not): no suppression chains exist."""
    a = 2 * n_pairs
    out = np.zeros((4 + classes, a), np.float32)
    for k in range(n_pairs):
        cx, cy = 100.0 * (k % 10) + 50, 100.0 * (k // 10) + 50
        for m in range(2):
            j = 2 * k + m
            out[:4, j] = [cx + rng.uniform(-8, 8), cy + rng.uniform(-8, 8), rng.uniform(10, 30), rng.uniform(10, 30)]
            out[4:, j] = rng.uniform(0, 1, classes).astype(np.float32)
    return out


def test_yolo_post_equals_greedy_nms_without_chains():
    rng = np.random.default_rng(5)
    for trial in range(20):
        out = _pair_clusters(rng, 30, 3)
        d = O.yolo_decode_nms_topk(out, classes=3, conf=0.3, iou=0.3, max_candidates=512, max_detections=512)
        want = _greedy_nms_reference(out, 3, 0.3, 0.3)
        got = [(float(s), int(c)) for s, c in zip(d[:, 4], d[:, 5])]
        assert [c for _, c in got] == [c for _, c in want] and np.allclose([s for s, _ in got], [s for s, _ in want])


def test_yolo_post_mark_rule_differs_from_greedy_on_a_chain():
    """A > B > C in one class, A overlaps B, B overlaps C, A does not overlap C: greedy NMS keeps A and C,
    the reference's GPU mark rule drops C too (B outranks C and overlaps it, suppressed or not)."""
    out = np.zeros((5, 3), np.float32)
    out[:4, 0] = [10, 10, 10, 10]
    out[:4, 1] = [14, 10, 10, 10]  # IoU(A, B) = IoU(B, C) = 0.43, IoU(A, C) = 0.11
    out[:4, 2] = [18, 10, 10, 10]
    out[4, :] = [0.9, 0.8, 0.7]
    d = O.yolo_decode_nms_topk(out, classes=1, conf=0.25, iou=0.3)
    assert _scores_classes(d)[0] == [0.9]
    assert [s for s, _ in _greedy_nms_reference(out, 1, 0.25, 0.3)] == pytest.approx([0.9, 0.7])


def test_yolo_post_invariants_and_candidate_cap():
    rng = np.random.default_rng(9)
    out = np.zeros((4 + 5, 600), np.float32)
    out[:2] = rng.uniform(0, 320, (2, 600))
    out[2:4] = rng.uniform(10, 60, (2, 600))
    out[4:] = rng.uniform(0, 1, (5, 600))
    for cap in (64, 512):
        d = O.yolo_decode_nms_topk(out, classes=5, conf=0.2, iou=0.45, max_candidates=cap, max_detections=1000)
        assert np.all(np.diff(d[:, 4]) <= 0)
        for i in range(len(d)):
            for j in range(i + 1, len(d)):
                if d[i, 5] != d[j, 5]:
                    continue
                x1, y1 = max(d[i, 0], d[j, 0]), max(d[i, 1], d[j, 1])
                x2, y2 = min(d[i, 2], d[j, 2]), min(d[i, 3], d[j, 3])
                inter = max(0, x2 - x1) * max(0, y2 - y1)
                ai = (d[i, 2] - d[i, 0]) * (d[i, 3] - d[i, 1]); aj = (d[j, 2] - d[j, 0]) * (d[j, 3] - d[j, 1])
                assert inter / max(ai + aj - inter, 1e-7) <= 0.45 + 1e-6
        # only the first `cap` passing anchors (in anchor order) are candidates
        sc = out[4:].max(axis=0)
        first = np.where(sc >= 0.2)[0][:cap]
        assert set(np.round(d[:, 4], 6)) <= set(np.round(sc[first], 6))
    small = O.yolo_decode_nms_topk(out, classes=5, conf=0.2, iou=0.45, max_candidates=512, max_detections=7)
    assert small.shape[0] == 7


def test_post_exp_against_numpy():
    xs = np.concatenate([np.linspace(-87, 88.5, 20001, dtype=np.float32), np.float32([0, 1, -1, 0.5, -0.5])])
    got = np.array([O.post_exp(float(x)) for x in xs], np.float64)
    want = np.exp(xs.astype(np.float64))
    assert np.max(np.abs(got - want) / want) < 3e-7
    assert O.post_exp(0.0) == 1.0 and O.post_exp(-100.0) == 0.0 and O.post_exp(100.0) == float("inf")
    assert np.isnan(O.post_exp(float("nan")))


def _dfl_head(levels, classes, rng=None, onehot=None):
    a = sum(h * w for h, w, _ in levels)
    head = np.zeros((64 + classes, a), np.float32)
    if rng is not None:
        head[:] = rng.normal(0, 2, head.shape)
    if onehot is not None:
        head[:64] = 0
        for i in range(a):
            for d in range(4):
                head[16 * d + onehot[i][d], i] = 40.0
    return head


def test_dfl_decode_closed_form_boxes_and_grid():
    """One-hot bins give integer distances; the box is (grid centre -/+ distance) * stride per level."""
    levels = [(4, 6, 8.0), (2, 3, 16.0), (1, 2, 32.0)]
    a = sum(h * w for h, w, _ in levels)
    rng = np.random.default_rng(3)
    onehot = rng.integers(0, 16, (a, 4))
    head = _dfl_head(levels, 2, onehot=onehot)
    head[64:] = -5.0
    head[64 + 1, :] = np.linspace(0, 4, a)  # class 1 wins, scores increase with the anchor index
    d = O.yolo_dfl_decode_nms_topk(head, levels, classes=2, conf=0.0, iou=1.0, max_candidates=a, max_detections=a)
    assert d.shape[0] == a
    i = 0
    want = {}
    for h, w, s in levels:
        for pos in range(h * w):
            gx, gy = pos % w + 0.5, pos // w + 0.5
            l, t, r, b = onehot[i]
            sc = 1.0 / (1.0 + np.exp(-np.float64(head[65, i])))
            want[i] = ((gx - l) * s, (gy - t) * s, (gx + r) * s, (gy + b) * s, sc)
            i += 1
    # rank order = descending score = descending anchor index
    for rank, row in enumerate(d):
        wx = want[a - 1 - rank]
        np.testing.assert_array_equal(row[:4], np.float32(wx[:4]))
        assert abs(row[4] - wx[4]) < 2e-7 and row[5] == 1.0


def test_dfl_decode_matches_float64_softmax_expectation():
    levels = [(5, 5, 8.0), (3, 3, 16.0)]
    rng = np.random.default_rng(8)
    head = _dfl_head(levels, 3, rng=rng)
    d = O.yolo_dfl_decode_nms_topk(head, levels, classes=3, conf=0.0, iou=1.0, max_candidates=64, max_detections=64)
    # recompute every anchor in float64 and match rows by score
    a = head.shape[1]
    rows = {}
    i = 0
    for h, w, s in levels:
        for pos in range(h * w):
            lg = head[:64, i].astype(np.float64).reshape(4, 16)
            e = np.exp(lg - lg.max(axis=1, keepdims=True))
            dist = (e * np.arange(16)).sum(1) / e.sum(1)
            gx, gy = pos % w + 0.5, pos // w + 0.5
            sc = 1 / (1 + np.exp(-head[64:, i].astype(np.float64)))
            rows[i] = (np.array([(gx - dist[0]) * s, (gy - dist[1]) * s, (gx + dist[2]) * s, (gy + dist[3]) * s]),
                       sc.max(), int(sc.argmax()))
            i += 1
    assert d.shape[0] == a
    for row in d:
        k = min(rows, key=lambda j: abs(rows[j][1] - row[4]) + 10 * (rows[j][2] != row[5]))
        np.testing.assert_allclose(row[:4], rows[k][0], rtol=1e-5, atol=1e-4)
