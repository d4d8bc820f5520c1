"""CPU model of the bottleneck-pair kernel's geometry: every LDS and buffer access in range.

The pair kernel (aexrt_amd/csrc/conv_pair.h, host side conv_pair.hip) keeps a weight ring, the
input window X, the grid G of the first conv's fp16 output and (int8) G quantized into the X
region in one block's LDS.  This test restates pair_geometry and the kernel's index arithmetic
(window staging, tap tables, operand reads of both convs, the epilogue writes, the optional
intermediate and accumulator outputs, the residual reads and the output stores) and checks for
the bottleneck shapes of YOLOv8n-320 at batch 1, 2 and 64 and a few ragged maps, every band
height the host offers, that each access lies inside its LDS region or buffer view, that the
float reciprocal divisions equal integer division, and that the launch's sync words stay inside
their area.  No GPU is used.
"""
from __future__ import annotations

import numpy as np
import pytest

KD, KKC, NT = 4, 4, 256
LDS_BUDGET = 152 * 1024
MAX_STEPS = 72
SYNC_WORDS, TOP, GEN, AMAX, STRIPES = 512, 128, 144, 192, 16


def vdiv(a, d):
    """small_div over an array: floor((a + 0.5) * (1 / d)) in float32, as the kernel computes it."""
    inv = np.float32(1) / np.float32(d)
    return ((np.asarray(a).astype(np.float32) + np.float32(0.5)) * inv).astype(np.int64)


def pair_geometry(N, C, H, W, tr, int8):
    if C % 32 or C > 128 or tr < 1:
        return None
    tr = min(tr, H)
    nq = C // 32
    ra = min(tr + 2, H)
    need = max(ra, tr) * W
    mq = 1 if need <= 128 else 2 if need <= 256 else 4 if need <= 512 else 0
    if not mq or nq * mq > 4:
        return None
    mw = W + 2
    xnpix, gnpix = (ra + 2) * mw, (tr + 2) * mw
    cpp = 16 if int8 else 8
    if (C // cpp) * xnpix > NT * (8 if int8 else 12):
        return None
    ks = 9 * C // (32 if int8 else 16)
    if ks > MAX_STEPS:
        return None
    xb = (C * (1 if int8 else 2) * xnpix + 15) // 16 * 16
    gb = C * 2 * gnpix
    ring = KD * KKC * 2 * C * 16
    if ring + xb + gb > LDS_BUDGET:
        return None
    return dict(N=N, C=C, H=H, W=W, TR=tr, nq=nq, mq=mq, nband=-(-H // tr), ks=ks, x_off=ring, g_off=ring + xb,
                lds=ring + xb + gb, xb=xb, cpp=cpp, int8=int8)


def check(h, x_cstride=None, y_cstride=None, r_cstride=None):
    C, H, W, TR, nq, mq, cpp, int8 = (h[k] for k in ("C", "H", "W", "TR", "nq", "mq", "cpp", "int8"))
    NOCB = nq * 32
    CB = KKC * 2 * NOCB * 16
    PT = KKC * 2 * NOCB // NT
    assert PT * NT * 16 == CB and h["x_off"] == KD * CB
    xcs, ycs, rcs = x_cstride or C, y_cstride or C, r_cstride or C
    x_img = ((H * W - 1) * xcs + C) * 2
    y_img = ((H * W - 1) * ycs + C) * 2
    r_img = ((H * W - 1) * rcs + C) * 2
    dense = H * W * C  # elements of one image of t_out / the accumulators
    MW = W + 2
    l32 = np.arange(64) & 31
    assert 2 * h["ks"] <= 2 * MAX_STEPS
    # ring: a chunk's A reads per lane
    for sl in range(KKC):
        for j in range(nq):
            assert (1 * NOCB + 31) * 16 + sl * (2 * NOCB * 16) + j * 512 + 16 <= CB
    for band in range(h["nband"]):
        r0 = band * TR
        TRr = min(TR, H - r0)
        a0, a1 = max(r0 - 1, 0), min(r0 + TRr + 1, H)
        RA = a1 - a0
        XNPIX, GNPIX = (RA + 2) * MW, (TRr + 2) * MW
        npos1, npos2 = RA * W, TRr * W
        assert npos1 <= 4 * mq * 32 and npos2 <= 4 * mq * 32
        npiece = (C // cpp) * XNPIX
        assert npiece <= NT * (8 if int8 else 12)
        assert h["x_off"] + npiece * 16 <= h["g_off"]
        e = np.arange(npiece)
        pl = vdiv(e, XNPIX)
        pix = e - pl * XNPIX
        pr = vdiv(pix, MW)
        assert (pl == e // XNPIX).all() and (pr == pix // MW).all()
        ih, iw = a0 - 1 + pr, pix - pr * MW - 1
        inside = (ih >= 0) & (ih < H) & (iw >= 0) & (iw < W)
        off = ((ih * W + iw) * xcs + pl * cpp) * 2 + (32 if int8 else 16)
        assert (off[inside] <= x_img).all()
        assert h["g_off"] + (C // 8) * GNPIX * 16 <= h["lds"]
        # tap planes inside the map
        k0 = np.arange(h["ks"]) * (32 if int8 else 16)
        assert ((k0 % C) // cpp + 1 < C // cpp).all()
        # operand reads and epilogue writes of every lane's subtiles (offsets grow with the
        # channel, so the last 4-channel quad bounds each one)
        pos = (np.arange(4)[:, None, None] + 4 * np.arange(mq)[None, :, None]) * 32 + l32[None, None, :]
        p1 = np.minimum(pos, npos1 - 1).ravel()
        r1 = vdiv(p1, W)
        assert (r1 == p1 // W).all()
        c1 = p1 - r1 * W
        assert ((r1 + 2) * MW + c1 + 2 < XNPIX).all()  # bottom-right tap in X
        gp = (r1 + a0 - (r0 - 1)) * MW + c1 + 1
        assert ((gp >= 0) & (gp < GNPIX)).all()
        assert (((a0 + r1) * W + c1) * C + C <= dense).all()
        p2 = np.minimum(pos, npos2 - 1).ravel()
        r2 = vdiv(p2, W)
        assert (r2 == p2 // W).all()
        c2 = p2 - r2 * W
        assert ((r2 + 2) * MW + c2 + 2 < GNPIX).all()  # bottom-right tap in G
        px = (r0 + r2) * W + c2
        assert ((px * ycs + C) * 2 <= y_img).all() and ((px * rcs + C) * 2 <= r_img).all()
        assert (((r0 * W + p2) * C + C) <= dense).all()
        # int8: G quantized into the X region
        if int8:
            nq16 = (C // 16) * GNPIX
            assert h["x_off"] + nq16 * 16 <= h["g_off"]
            e = np.arange(nq16)
            plq = vdiv(e, GNPIX)
            assert (plq == e // GNPIX).all() and (2 * plq + 1 < C // 8).all()
    # sync words: per-XCD counters, top, generation, amax copies
    assert 7 * 16 < TOP < GEN < AMAX and AMAX + (STRIPES - 1) * 16 < SYNC_WORDS


SHAPES = [(32, 40), (64, 20), (128, 10)]  # the bottleneck maps of YOLOv8n-320


@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("batch", [1, 2, 64])
def test_pair_accesses_stay_in_bounds(int8, batch):
    seen = 0
    for C, hw in SHAPES:
        for parts in range(1, hw + 1):
            tr = -(-hw // parts)
            h = pair_geometry(batch, C, hw, hw, tr, int8)
            if h is None:
                continue
            check(h)
            check(h, x_cstride=C * 3, y_cstride=C * 4, r_cstride=C * 3)  # channel slices of concat roots
            seen += 1
    assert seen >= 6


def test_pair_accesses_on_ragged_maps():
    for (C, H, W) in [(64, 13, 11), (32, 9, 30), (128, 7, 5), (64, 40, 40)]:
        for int8 in (True, False):
            n = 0
            for tr in range(1, H + 1):
                h = pair_geometry(2, C, H, W, tr, int8)
                if h:
                    check(h)
                    n += 1
            assert n > 0, (C, H, W, int8)


def test_pair_geometry_model_catches_a_planted_overflow():
    h = pair_geometry(2, 64, 20, 20, 5, True)
    with pytest.raises(AssertionError):
        check(dict(h, g_off=h["x_off"] + 16 * 64))
