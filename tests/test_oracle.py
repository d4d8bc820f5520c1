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
