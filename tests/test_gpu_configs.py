"""GPU parity at the benchmark configurations that are single convolutions, and of the
dynamic int8 kernel, through the op-level C ABI.

* C1: 1x64x80x80 fp32, 3x3 s1 p1 64->64, SiLU, seed 0 -- the reference's fp32 conv path
  (RT:1554-1622, CPU RT:20552-20580) on the GPU, against the oracle's cpu_conv2d.
* C3: 64x160x160 -> 128x80x80, 3x3 s2 p1, at batch 32, W8A8 and fp16, seed 2.
* a9: the dynamic int8 conv the reference runs on inputs of fewer than 4096 elements.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as O
from aexrt_amd import _lib
from aexrt_amd import kernels as K
from aexrt_amd import packing
from tests.helpers import he_weight, nchw_to_nhwc, nhwc_to_nchw, tol_range

pytestmark = pytest.mark.gpu

ORACLE_THREADS = 16


def _ulp16(a: np.ndarray) -> np.ndarray:
    """Spacing of fp16 at |a| (the larger of the two neighbouring gaps)."""
    return np.spacing(np.abs(a).astype(np.float16)).astype(np.float64)


def _within_ulp16(ref: np.ndarray, got: np.ndarray, ulps: float = 1.0):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = ulps * _ulp16(ref)
    worst = float((err / np.maximum(bound, 1e-30)).max()) if err.size else 0.0
    return worst <= 1.0, worst


def _conv_f32(cuda, x, w, b, desc, silu):
    import torch

    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(cuda)
    wd = torch.from_numpy(np.ascontiguousarray(w, np.float32)).to(cuda)
    bd = torch.from_numpy(np.ascontiguousarray(b, np.float32)).to(cuda)
    y = torch.empty(tuple(O.out_shape(desc)), dtype=torch.float32, device=cuda)
    d = _lib.ConvDesc.from_params(desc)
    _lib.check(_lib.lib().aexrt_hip_conv2d_f32(ctypes.byref(d), K.SILU if silu else 0, xd.data_ptr(), wd.data_ptr(),
                                               bd.data_ptr(), y.data_ptr(), None), "conv2d_f32")
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_c1_fp32_conv_matches_the_reference_cpu_path(cuda):
    """C1 on the GPU: within 1e-4 of the output range with SiLU, bit-exact without (the same
    accumulation order, every multiply and add rounded on its own)."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 64, 80, 80)).astype(np.float32)
    w = (rng.standard_normal((64, 64, 3, 3)) * np.sqrt(2.0 / 576)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, 64).astype(np.float32)
    desc = O.conv_desc(1, 64, 80, 80, 64, 3, 1, 1)
    ref = O.cpu_conv2d(x, w, b, desc, silu=True, threads=ORACLE_THREADS)
    got = _conv_f32(cuda, x, w, b, desc, silu=True)
    err, allowed = tol_range(ref, got, 1e-4)
    assert err <= allowed, (err, allowed)
    lin = _conv_f32(cuda, x, w, b, desc, silu=False)
    np.testing.assert_array_equal(lin, O.cpu_conv2d(x, w, b, desc, silu=False, threads=ORACLE_THREADS))


@pytest.mark.parametrize("n,c,h,w,oc,k,s,p,d,g", [
    (2, 8, 9, 11, 12, 3, 2, 1, 1, 1),     # stride 2, ragged dims, OC % 4 == 0
    (1, 8, 10, 10, 6, 3, 1, 2, 2, 2),     # dilation 2 with pad 2, 2 groups of 3 output channels
    (1, 3, 320, 320, 16, 6, 2, 2, 1, 1),  # 6x6 s2 p2 (the reference's stem conv shape)
    (3, 16, 5, 7, 16, 1, 1, 0, 1, 4),     # grouped 1x1
])
def test_fp32_conv_geometry_bit_exact(cuda, n, c, h, w, oc, k, s, p, d, g):
    rng = np.random.default_rng(n * 100 + c + k)
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    wt = rng.standard_normal((oc, c // g, k, k)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, oc).astype(np.float32)
    oh = (h + 2 * p - d * (k - 1) - 1) // s + 1
    ow = (w + 2 * p - d * (k - 1) - 1) // s + 1
    desc = np.array([n, c, h, w, oc, oh, ow, k, k, s, s, p, p, d, d, g], np.uint32)
    got = _conv_f32(cuda, x, wt, b, desc, silu=False)
    np.testing.assert_array_equal(got, O.cpu_conv2d(x, wt, b, desc, silu=False))
    import torch

    ref64 = torch.nn.functional.conv2d(torch.from_numpy(x.astype(np.float64)), torch.from_numpy(wt.astype(np.float64)),
                                       torch.from_numpy(b.astype(np.float64)), stride=s, padding=p, dilation=d,
                                       groups=g).numpy()
    np.testing.assert_allclose(got, ref64, rtol=1e-4, atol=1e-5)


C3_IMAGES = (0, 13, 31)


@pytest.fixture(scope="module")
def c3_operands():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((32, 64, 160, 160)).astype(np.float32)
    w = he_weight(rng, 128, 64, 3)
    b = rng.uniform(-0.1, 0.1, 128).astype(np.float32)
    return O.round_f16(x), w, packing.fp16_round(b)


def test_c3_stride2_batch32_w8a8(cuda, c3_operands):
    """C3 W8A8 at batch 32: amax over the whole batch and every quantized byte bit-exact; the int32
    accumulators of three images bit-exact; their fp16 outputs within one fp16 ulp."""
    import torch

    x, w, b = c3_operands
    desc = O.conv_desc(32, 64, 160, 160, 128, 3, 2, 1)
    pc = K.prepare_conv(desc, 53, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(w, fp16_engine=True), b, device=cuda)
    xd = torch.from_numpy(nchw_to_nhwc(x.astype(np.float16))).to(cuda)
    xs = K.new_slots(64, cuda)
    K.amax_slots(xd, xs)
    q = K.quantize(xd, xs)
    y = torch.empty((32, 80, 80, 128), dtype=torch.float16, device=cuda)
    acc = torch.empty((32 * 80 * 80, 128), dtype=torch.int32, device=cuda)
    K.conv2d(pc, xd, y, flags=K.SILU, x_slots=xs, acc_out=acc)
    torch.cuda.synchronize()
    a = O.amax(x)
    assert np.float32(a).view(np.uint32) == K.slots_max(xs).max()
    qa = O.quantize(x, a)
    np.testing.assert_array_equal(nhwc_to_nchw(q.cpu().numpy()), qa)
    qw, ws = O.weight_quant(w, fp16_round=True)
    sel = list(C3_IMAGES)
    d3 = O.conv_desc(len(sel), 64, 160, 160, 128, 3, 2, 1)
    acc_ref = O.conv_int8_acc(qa[sel], qw, d3, threads=ORACLE_THREADS)
    got_acc = nhwc_to_nchw(acc.cpu().numpy().reshape(32, 80, 80, 128)[sel])
    np.testing.assert_array_equal(got_acc, acc_ref)
    y_ref = O.conv_int8_epilogue(acc_ref, a, ws, b, silu=True)
    ok, worst = _within_ulp16(y_ref, nhwc_to_nchw(y.float().cpu().numpy()[sel]))
    assert ok, worst


def test_c3_stride2_batch32_fp16(cuda, c3_operands):
    """C3 fp16 at batch 32 (fp16 MFMA, fp32 accumulation): three images within 1e-2 of the range of
    the oracle's direct conv on the same fp16-rounded operands."""
    import torch

    x, w, b = c3_operands
    desc = O.conv_desc(32, 64, 160, 160, 128, 3, 2, 1)
    wf = packing.fp16_round(w)
    pc = K.prepare_conv(desc, 5, K.SRC_RAW_F32, wf, b, device=cuda)
    xd = torch.from_numpy(nchw_to_nhwc(x.astype(np.float16))).to(cuda)
    y = torch.empty((32, 80, 80, 128), dtype=torch.float16, device=cuda)
    K.conv2d(pc, xd, y, flags=K.SILU)
    torch.cuda.synchronize()
    sel = list(C3_IMAGES)
    ref = O.cpu_conv2d(x[sel], wf, b, O.conv_desc(len(sel), 64, 160, 160, 128, 3, 2, 1), silu=True,
                       threads=ORACLE_THREADS)
    err, allowed = tol_range(ref, nhwc_to_nchw(y.float().cpu().numpy()[sel]), 1e-2)
    assert err <= allowed, (err, allowed)


DYN_CASES = [
    # (name, n, c, h, w, oc, k, s) -- all but the last have fewer than 4096 input elements
    ("3x3s1_128_5x5", 1, 128, 5, 5, 128, 3, 1),
    ("3x3s2_32_7x7_b2", 2, 32, 7, 7, 64, 3, 2),
    ("1x1_64_6x5", 1, 64, 6, 5, 48, 1, 1),
    ("1x1_16_10x10", 2, 16, 10, 10, 32, 1, 1),
    ("3x3s1_256_5x5_6400", 1, 256, 5, 5, 64, 3, 1),
]


def _dyn_run(cuda, n, c, h, w, oc, k, s, *, silu, out_f32, residual, seed):
    import torch

    rng = np.random.default_rng(seed)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32) * 2.0)
    x[:, :4] *= 20.0  # one loud 4-channel group: per-group scales differ
    x = O.round_f16(x)
    wt = he_weight(rng, oc, c, k)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, k, s, k // 2)
    alg = 51 if k == 1 else (53 if s == 2 else 52)
    pc = K.prepare_conv(desc, alg, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True), b, device=cuda)
    xd = torch.from_numpy(nchw_to_nhwc(x.astype(np.float16))).to(cuda)
    _, _, oh, ow = O.out_shape(desc)
    y = torch.empty((n, oh, ow, oc), dtype=torch.float32 if out_f32 else torch.float16, device=cuda)
    ys = K.new_slots(oc, cuda, stripes=4)
    flags = K.INT8_DYNAMIC | (K.SILU if silu else 0) | (K.OUT_F32 if out_f32 else 0)
    r = None
    if residual:
        r = O.round_f16(rng.standard_normal((n, oc, oh, ow)).astype(np.float32))
        flags |= K.RESIDUAL
    K.conv2d(pc, xd, y, flags=flags, y_slots=ys,
             residual=None if r is None else torch.from_numpy(nchw_to_nhwc(r.astype(np.float16))).to(cuda))
    torch.cuda.synchronize()
    qw, ws = O.weight_quant(wt, fp16_round=True)
    ref = O.conv_int8_dynamic(x, qw, desc, ws, b, silu)
    return ref, r, nhwc_to_nchw(y.float().cpu().numpy()), K.slots_max(ys)


@pytest.mark.parametrize("case", DYN_CASES, ids=[c[0] for c in DYN_CASES])
def test_dynamic_int8_fp32_out_bit_exact(cuda, case):
    """Per (position, 4-channel group) scales, int32 dot4 partials, fp32 dequant accumulation in
    group order: without SiLU the fp32 output equals the oracle's bit for bit."""
    _, n, c, h, w, oc, k, s = case
    ref, _, got, _ = _dyn_run(cuda, n, c, h, w, oc, k, s, silu=False, out_f32=True, residual=False, seed=31)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("case", DYN_CASES, ids=[c[0] for c in DYN_CASES])
@pytest.mark.parametrize("residual", [False, True])
def test_dynamic_int8_fp16_silu_residual_and_slots(cuda, case, residual):
    _, n, c, h, w, oc, k, s = case
    ref, r, got, slots = _dyn_run(cuda, n, c, h, w, oc, k, s, silu=True, out_f32=False, residual=residual, seed=32)
    if residual:
        conv = O.round_f16(ref)
        ok, worst = _within_ulp16(conv + r, got, 1.0)
        ok2 = np.all(np.abs(got.astype(np.float64) - (conv + r)) <= _ulp16(conv) + _ulp16(conv + r))
        assert ok or ok2, worst
    else:
        ok, worst = _within_ulp16(ref, got)
        assert ok, worst
    want = [np.float32(np.abs(got[:, g * 16:(g + 1) * 16]).max()).view(np.uint32) for g in range(oc // 16)]
    np.testing.assert_array_equal(slots, want)


def _cmd_case(cuda, x, wt, b, k, s, *, pg16=False, silu=True):
    import torch

    n, c, h, w = x.shape
    oc = wt.shape[0]
    desc = O.conv_desc(n, c, h, w, oc, k, s, k // 2)
    alg = 51 if k == 1 else (53 if s == 2 else 52)
    pc = K.prepare_conv(desc, alg, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True), b, device=cuda)
    xd = torch.from_numpy(nchw_to_nhwc(x.astype(np.float16))).to(cuda)
    _, _, oh, ow = O.out_shape(desc)
    y = torch.empty((n, oh, ow, oc), dtype=torch.float16, device=cuda)
    K.conv2d_int8(pc, xd, y, flags=(K.SILU if silu else 0) | (K.INT8_PG16 if pg16 else 0))
    torch.cuda.synchronize()
    return desc, nhwc_to_nchw(y.float().cpu().numpy())


def test_int8_command_c2_per_tensor(cuda):
    """C2 (1x128x40x40 fp16 with 1% outliers x8, 1x1 128->256, per-16-output-channel weight scales)
    through the int8 command: the input's amax, quantize-on-load, int32 MFMA, dequant + bias + SiLU,
    within one fp16 ulp of the oracle's chain."""
    from tests.helpers import c2_input, group16_weight

    rng = np.random.default_rng(1)
    x = c2_input(seed=1)
    wt = group16_weight(rng, 256, 128, 1)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, 256).astype(np.float32))
    desc, got = _cmd_case(cuda, x, wt, b, 1, 1)
    y_ref = O.w8a8_conv(x, wt, b, desc, silu=True, fp16_engine=True)[-1]
    ok, worst = _within_ulp16(y_ref, got)
    assert ok, worst


def test_int8_command_pg16_strips_at_batch_two(cuda):
    """Plan flag 16 through the command: the reference's memory-strip amax (images mixed at N > 1),
    per-group pack scales, pg16 conv; within 1e-3 of the range of the oracle's pg16 chain."""
    from oracle import network as ON

    rng = np.random.default_rng(41)
    x = O.round_f16(rng.standard_normal((2, 64, 12, 12)).astype(np.float32))
    x[:, 16:32] *= 6.0
    x = O.round_f16(x)
    wt = he_weight(rng, 32, 64, 3)
    b = rng.uniform(-0.1, 0.1, 32).astype(np.float32)
    desc, got = _cmd_case(cuda, x, wt, packing.fp16_round(b), 3, 1, pg16=True)
    ref = ON.conv_layer(x, wt, b, dict(strides=[1, 1], pads=[1, 1, 1, 1]), int8=True, silu=True, pg16=True)
    err, allowed = tol_range(ref, got, 1e-3)
    assert err <= allowed, (err, allowed)


def test_int8_command_below_4096_elements_is_the_dynamic_conv(cuda):
    rng = np.random.default_rng(42)
    x = O.round_f16(rng.standard_normal((1, 128, 5, 5)).astype(np.float32))
    wt = he_weight(rng, 128, 128, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, 128).astype(np.float32))
    desc, got = _cmd_case(cuda, x, wt, b, 3, 1, pg16=True)
    qw, ws = O.weight_quant(wt, fp16_round=True)
    ok, worst = _within_ulp16(O.conv_int8_dynamic(x, qw, desc, ws, b, True), got)
    assert ok, worst
