"""The C2f bottleneck pair kernel (3x3 SiLU -> 3x3 SiLU (+ residual) in one launch,
csrc/conv_pair.h) against the oracle, through aexrt_hip_conv_pair.

int8: the first conv's accumulators are the oracle's exact int8 conv of x quantized with x's
per-tensor amax (RT:3314-3346, 4614-4762), its fp16 output (the intermediate, copied out for the
check) within one fp16 ulp of the oracle's epilogue; the second conv's accumulators are the
oracle's int8 conv of that intermediate quantized with ITS per-tensor amax over the whole batch
(the amax the workgroups exchange through the grid barrier, RT:3232-3257), bit for bit; y within
one fp16 ulp (two with the residual add) and its amax slots exactly max|y| per 16 channels.
fp16: against the oracle's two direct convs with the intermediate rounded to fp16, within 1e-2 of
the output range.  Every case also checks that no grid-barrier wait timed out.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from aexrt_amd import kernels as K
from aexrt_amd import packing
from tests.helpers import he_weight, nchw_to_nhwc, nhwc_to_nchw, tol_range
from tests.test_gpu_ops import FP16_TOL, _dev_nhwc

pytestmark = pytest.mark.gpu

# (batch, channels, h, w, band rows (0: chosen), residual)
CASES = [
    (2, 64, 20, 20, 0, True),     # the 20x20 bottleneck of YOLOv8n-320, chosen bands
    (2, 64, 20, 20, 5, False),    # four bands per image, no shortcut (the neck's C2f)
    (1, 128, 10, 10, 0, True),    # the 10x10 bottleneck: one band, 128 channels
    (3, 32, 40, 40, 10, True),    # the 40x40 bottleneck: 480-position bands (4 subtiles per wave)
    (1, 64, 13, 11, 4, True),     # ragged map, a partial last band
    (2, 32, 9, 30, 3, False),     # wide rows, three bands
    (64, 64, 20, 20, 5, True),    # the benchmark batch: 256 workgroups meet at the barrier
]


def _ulp16(a):
    return np.spacing(np.abs(a).astype(np.float16)).astype(np.float64)


def _case_id(t):
    return f"n{t[0]}_c{t[1]}_{t[2]}x{t[3]}_b{t[4]}{'_res' if t[5] else ''}"


@pytest.mark.parametrize("case", CASES, ids=[_case_id(t) for t in CASES])
def test_int8_pair_matches_the_oracle_bit_exact(cuda, case):
    import torch

    n, c, h, w, band, res = case
    rng = np.random.default_rng(900 + c + h + w + n)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    x[:, : c // 4] *= 4.0  # one channel group with a larger range
    wa, wb = he_weight(rng, c, c, 3), he_weight(rng, c, c, 3)
    ba, bb = (packing.fp16_round(rng.uniform(-0.1, 0.1, c).astype(np.float32)) for _ in range(2))
    desc = O.conv_desc(n, c, h, w, c, 3, 1, 1)
    pa = K.prepare_conv(desc, 52, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wa, fp16_engine=True), ba, device=cuda)
    pb = K.prepare_conv(desc, 52, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wb, fp16_engine=True), bb, device=cuda)
    xd = _dev_nhwc(x, cuda)
    xs = K.new_slots(c, cuda, stripes=16)
    K.amax_slots(xd, xs)
    wide = torch.full((n, h, w, 2 * c), float("nan"), dtype=torch.float16, device=cuda)
    y = wide[..., c:]  # the output in a channel slice of a wider tensor (a C2f concat)
    ys_all = K.new_slots(2 * c, cuda, stripes=16)
    ys = ys_all[:, c // 16:]
    t = torch.empty((n, h, w, c), dtype=torch.float16, device=cuda)
    acc_a = torch.empty((n * h * w, c), dtype=torch.int32, device=cuda)
    acc_b = torch.empty_like(acc_a)
    K.conv_pair(pa, pb, xd, y, x_slots=xs, y_slots=ys, residual=res, band_rows=band, t_out=t, acc_a=acc_a,
                acc_b=acc_b)
    assert K.conv_pair_barrier_timeouts() == 0
    # conv a: accumulators exact, the intermediate within one fp16 ulp
    amax_x = O.amax(x)
    qwa, swa = O.weight_quant(wa, fp16_round=True)
    acc_a_ref = O.conv_int8_acc(O.quantize(x, amax_x), qwa, desc, threads=8)
    got_a = acc_a.cpu().numpy().reshape(n, h, w, c).transpose(0, 3, 1, 2)
    assert np.array_equal(got_a, acc_a_ref), int(np.abs(got_a.astype(np.int64) - acc_a_ref).max())
    tt = nhwc_to_nchw(t.float().cpu().numpy())
    t_ref = O.conv_int8_epilogue(acc_a_ref, amax_x, swa, ba, silu=True)
    assert float((np.abs(tt - t_ref) / _ulp16(t_ref)).max()) <= 1.0
    # conv b: exact on the intermediate quantized with its own batch-global amax
    amax_t = O.amax(tt)
    qwb, swb = O.weight_quant(wb, fp16_round=True)
    acc_b_ref = O.conv_int8_acc(O.quantize(tt, amax_t), qwb, desc, threads=8)
    got_b = acc_b.cpu().numpy().reshape(n, h, w, c).transpose(0, 3, 1, 2)
    assert np.array_equal(got_b, acc_b_ref), int(np.abs(got_b.astype(np.int64) - acc_b_ref).max())
    conv_ref = O.conv_int8_epilogue(acc_b_ref, amax_t, swb, bb, silu=True)
    y_ref = O.round_f16(conv_ref) + x if res else conv_ref
    yy = nhwc_to_nchw(y.float().cpu().numpy())
    bound = _ulp16(y_ref) + (_ulp16(conv_ref) if res else 0.0)
    assert float((np.abs(yy - y_ref) / bound).max()) <= 1.0
    assert np.isnan(wide[..., :c].float().cpu().numpy()).all()  # nothing written outside the slice
    # y's slots: max|y| of each 16-channel group, exactly
    got_s = K.slots_max(ys)
    want = np.abs(yy).reshape(n, c // 16, 16, h * w).max(axis=(0, 2, 3)).astype(np.float32).view(np.uint32)
    np.testing.assert_array_equal(got_s, want)


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[3], CASES[4]], ids=[_case_id(t) for t in
                                                                            (CASES[0], CASES[2], CASES[3], CASES[4])])
def test_fp16_pair_matches_two_convs(cuda, case):
    import torch

    n, c, h, w, band, res = case
    rng = np.random.default_rng(950 + c + h)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    wa, wb = he_weight(rng, c, c, 3), he_weight(rng, c, c, 3)
    ba, bb = (packing.fp16_round(rng.uniform(-0.1, 0.1, c).astype(np.float32)) for _ in range(2))
    desc = O.conv_desc(n, c, h, w, c, 3, 1, 1)
    pa = K.prepare_conv(desc, 5, K.SRC_RAW_F32, wa, ba, device=cuda)
    pb = K.prepare_conv(desc, 5, K.SRC_RAW_F32, wb, bb, device=cuda)
    xd = _dev_nhwc(x, cuda)
    y = torch.empty((n, h, w, c), dtype=torch.float16, device=cuda)
    t = torch.empty_like(y)
    K.conv_pair(pa, pb, xd, y, residual=res, band_rows=band, t_out=t)
    torch.cuda.synchronize()
    t_ref = O.round_f16(O.cpu_conv2d(x, O.round_f16(wa), ba, desc, silu=True))
    err, allowed = tol_range(t_ref, nhwc_to_nchw(t.float().cpu().numpy()), FP16_TOL)
    assert err <= allowed, ("intermediate", err, allowed)
    y_ref = O.cpu_conv2d(t_ref, O.round_f16(wb), bb, desc, silu=True)
    if res:
        y_ref = O.round_f16(y_ref) + x
    err, allowed = tol_range(y_ref, nhwc_to_nchw(y.float().cpu().numpy()), FP16_TOL)
    assert err <= allowed, (err, allowed)


def test_pair_refuses_what_it_cannot_run(cuda):
    import torch

    rng = np.random.default_rng(3)
    # 48 channels: not a multiple of 32
    n, c, h, w = 1, 48, 10, 10
    desc = O.conv_desc(n, c, h, w, c, 3, 1, 1)
    pa = K.prepare_conv(desc, 5, K.SRC_RAW_F32, he_weight(rng, c, c, 3), np.zeros(c, np.float32), device=cuda)
    x = _dev_nhwc(O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32)), cuda)
    y = torch.empty((n, h, w, c), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        K.conv_pair(pa, pa, x, y)
    # a band of 20 rows at 40x40x64: 880 positions per block
    n, c, h, w = 1, 64, 40, 40
    desc = O.conv_desc(n, c, h, w, c, 3, 1, 1)
    pa = K.prepare_conv(desc, 5, K.SRC_RAW_F32, he_weight(rng, c, c, 3), np.zeros(c, np.float32), device=cuda)
    x = _dev_nhwc(O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32)), cuda)
    y = torch.empty((n, h, w, c), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="no band"):
        K.conv_pair(pa, pa, x, y, band_rows=20)
