"""The detect-head chain kernel (3x3 SiLU -> 3x3 SiLU -> 1x1 in one launch, csrc/conv_chain.h)
against the oracle's three convs with each intermediate rounded to fp16 (what the separate convs
store and read): whole-map tiles, tiles with recomputed borders, ragged maps with partial tiles,
fp16 and fp32 outputs, a channel slice of a wider output."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from aexrt_amd import kernels as K
from aexrt_amd import packing
from tests.helpers import he_weight, nhwc_to_nchw, tol_range
from tests.test_gpu_ops import FP16_TOL, FP32_TOL, _dev_nhwc

pytestmark = pytest.mark.gpu

# fp32 outputs: the fp32 tolerance for each of the two fp16 intermediates, whose roundings can
# fall on the other side of a tie point when the fp32 sums are added in another order (one fp16
# ulp, 2^-11 relative, carried through the next conv) — measured up to 1.3e-4 of the range
CHAIN_FP32_TOL = 2.5 * FP32_TOL

# (batch, in channels, h, w, branch channels, out channels, tile, output, output slice)
CASES = [
    (2, 256, 10, 10, 80, 80, (0, 0), "f32", None),    # the 10x10 class branch: one tile per image
    (2, 256, 10, 10, 64, 64, (0, 0), "f32", None),    # the 10x10 box branch
    (2, 128, 20, 20, 80, 80, (10, 10), "f32", None),  # 20x20: four tiles, borders recomputed
    (1, 64, 40, 40, 64, 64, (8, 8), "f16", None),     # 40x40 box branch, interior tiles
    (2, 64, 40, 40, 80, 80, (6, 8), "f16", None),     # partial last tile row
    (1, 64, 13, 11, 80, 64, (5, 4), "silu", None),    # ragged map, partial tiles, SiLU on the 1x1
    (1, 128, 13, 11, 80, 64, (5, 4), "silu", None),   # the same with a 16 KB window
    (2, 32, 9, 7, 48, 32, (0, 0), "f16", None),       # 48 channels in a 64-channel block
    (2, 128, 20, 20, 64, 64, (10, 10), "f32", (80, 144, 144)),  # box outputs in a 144-channel tensor
    (1, 64, 40, 40, 80, 80, (8, 12), "f16", None),    # 140-position regions: two subtiles per wave
    (2, 64, 24, 24, 64, 64, (12, 12), "f32", None),   # 196 and 144 positions
    # small tiles the load-time measurement offers (many blocks at batch 1, borders recomputed)
    (1, 256, 10, 10, 80, 80, (5, 5), "f32", None),
    (1, 256, 10, 10, 64, 64, (4, 4), "f32", None),    # ragged: tiles of 4, 4 and 2
    (1, 128, 20, 20, 80, 80, (3, 3), "f32", None),    # 25-position regions, 9-position tiles
    (1, 64, 40, 40, 64, 64, (14, 14), "f16", None),   # thirds of the map
]


# the cases of the two-group blocks (two groups of four waves splitting each chunk's k steps):
# one block subtile per wave and a window of at least 16 KB
KG2_CASES = [t for t in CASES if t[1] >= 128]


@pytest.mark.skip(reason="two-group chain blocks (KG = 2) switched off: a model load that ran them "
                         "aborted and no cause was shown; the library launches one group only")
@pytest.mark.parametrize("case", KG2_CASES, ids=[f"c{t[1]}_{t[2]}x{t[3]}_b{t[4]}_o{t[5]}_t{t[6][0]}x{t[6][1]}"
                                                 for t in KG2_CASES])
def test_chain_two_k_groups_matches_three_convs(cuda, case):
    """Kept skipped while the path is off.  No hook selects the two-group blocks, so the test
    fails rather than re-test the one-group form: a hook that selects them, and a check of the
    launched instance's name, come back with the path."""
    pytest.fail("no hook selects the two-group chain blocks")


@pytest.mark.parametrize("case", CASES, ids=[f"c{t[1]}_{t[2]}x{t[3]}_b{t[4]}_o{t[5]}_t{t[6][0]}x{t[6][1]}_{t[7]}"
                                             f"{'_slice' if t[8] else ''}" for t in CASES])
def test_chain_matches_three_convs(cuda, case):
    """One group of four waves per block (the library launches no other form)."""
    import torch

    n, c, h, w, cb, oc, tile, out, sl = case
    rng = np.random.default_rng(701 + c + h + cb + oc)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    wa, wb, wc = he_weight(rng, cb, c, 3), he_weight(rng, cb, cb, 3), he_weight(rng, oc, cb, 1)
    ba, bb, bc = (packing.fp16_round(rng.uniform(-0.1, 0.1, k).astype(np.float32)) for k in (cb, cb, oc))
    da, db, dc = O.conv_desc(n, c, h, w, cb, 3, 1, 1), O.conv_desc(n, cb, h, w, cb, 3, 1, 1), \
        O.conv_desc(n, cb, h, w, oc, 1, 1, 0)
    pa = K.prepare_conv(da, 5, K.SRC_RAW_F32, wa, ba, device=cuda)
    pb = K.prepare_conv(db, 5, K.SRC_RAW_F32, wb, bb, device=cuda)
    pc = K.prepare_conv(dc, 5, K.SRC_RAW_F32, wc, bc, device=cuda)
    f32, silu_c = out == "f32", out == "silu"
    lo, hi, width = sl if sl else (0, oc, oc)
    big = torch.zeros((n, h, w, width), dtype=torch.float32 if f32 else torch.float16, device=cuda)
    K.conv_chain3(pa, pb, pc, _dev_nhwc(x, cuda), big[..., lo:hi],
                  flags_c=(K.OUT_F32 if f32 else 0) | (K.SILU if silu_c else 0), tile=tile)
    torch.cuda.synchronize()
    got = nhwc_to_nchw(big.float().cpu().numpy())
    t1 = O.round_f16(O.cpu_conv2d(x, O.round_f16(wa), ba, da, silu=True))
    t2 = O.round_f16(O.cpu_conv2d(t1, O.round_f16(wb), bb, db, silu=True))
    ref = O.cpu_conv2d(t2, O.round_f16(wc), bc, dc, silu=silu_c)
    assert np.isfinite(got).all()
    err, allowed = tol_range(ref, got[:, lo:hi], CHAIN_FP32_TOL if f32 else FP16_TOL)
    assert err <= allowed, (err, allowed)
    assert not got[:, :lo].any() and not got[:, hi:].any()


def test_chain_agrees_with_the_separate_kernels(cuda):
    """The chain's output against the same three convs run one by one on this backend (fp16
    intermediates in memory): the fp32 sums differ only in their order."""
    import torch

    n, c, h, w, cb = 2, 128, 20, 20, 80
    rng = np.random.default_rng(77)
    x = _dev_nhwc(O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32)), cuda)
    descs = [O.conv_desc(n, c, h, w, cb, 3, 1, 1), O.conv_desc(n, cb, h, w, cb, 3, 1, 1),
             O.conv_desc(n, cb, h, w, cb, 1, 1, 0)]
    pcs = [K.prepare_conv(d, 5, K.SRC_RAW_F32, he_weight(rng, cb, int(d[1]), int(d[7])),
                          packing.fp16_round(rng.uniform(-0.1, 0.1, cb).astype(np.float32)), device=cuda)
           for d in descs]
    y = torch.empty((n, h, w, cb), dtype=torch.float32, device=cuda)
    K.conv_chain3(*pcs, x, y, flags_c=K.OUT_F32)
    t1 = torch.empty((n, h, w, cb), dtype=torch.float16, device=cuda)
    t2 = torch.empty_like(t1)
    y3 = torch.empty((n, h, w, cb), dtype=torch.float32, device=cuda)
    K.conv2d(pcs[0], x, t1, flags=K.SILU)
    K.conv2d(pcs[1], t1, t2, flags=K.SILU)
    K.conv2d(pcs[2], t2, y3, flags=K.OUT_F32)
    torch.cuda.synchronize()
    err, allowed = tol_range(y3.cpu().numpy(), y.cpu().numpy(), CHAIN_FP32_TOL)
    assert err <= allowed, (err, allowed)


def test_chain_refuses_what_it_cannot_run(cuda):
    import torch

    rng = np.random.default_rng(5)
    n, c, h, w = 1, 64, 10, 10
    x = _dev_nhwc(O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32)), cuda)

    def prep(cin, cout, k):
        return K.prepare_conv(O.conv_desc(n, cin, h, w, cout, k, 1, k // 2), 5, K.SRC_RAW_F32,
                              he_weight(rng, cout, cin, k), np.zeros(cout, np.float32), device=cuda)

    y = torch.empty((n, h, w, 128), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="96 channels"):
        K.conv_chain3(prep(c, 128, 3), prep(128, 128, 3), prep(128, 128, 1), x, y)
    with pytest.raises(RuntimeError, match="3x3"):
        K.conv_chain3(prep(c, 64, 1), prep(64, 64, 3), prep(64, 64, 1), x, y[..., :64])
    h = w = 40
    x40 = _dev_nhwc(O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32)), cuda)
    y40 = torch.empty((n, h, w, 64), dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="tile"):  # 400 positions per block
        K.conv_chain3(prep(c, 64, 3), prep(64, 64, 3), prep(64, 64, 1), x40, y40, tile=(20, 20))
