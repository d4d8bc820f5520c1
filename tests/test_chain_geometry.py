"""CPU model of the head-branch chain kernel's geometry: every LDS and buffer access in range.

The chain kernel (aexrt_amd/csrc/conv_chain.h, host side conv_chain.hip) keeps a weight ring,
the input window X and the grid G of the first conv's output in one block's LDS and addresses
them with per-tile index arithmetic.  This test restates that arithmetic (make_chain_params,
chain_tile, chain_block's X staging, tap tables, operand reads, epilogue writes, the k-group
reduction and the output offsets) and checks, for every tile of every head level of YOLOv8n-160
and -320 at batch 1, 2 and 64, one and two k groups, and both launch forms (one branch, two
branches sharing the block size and the larger LDS), that:
  - every LDS byte a thread writes or reads lies inside its region and the block's dynamic
    LDS, and dynamic plus static LDS fits the CU's 160 KB;
  - every buffer offset of a live load or store lies inside its view;
  - the float reciprocal divisions (small_div) equal integer division over their ranges;
  - the two-group reduction's 16 KB fits the window region and the tap tables fit their arrays.
No GPU is used.  The two-group form stays switched off in the library; this check is the
host-side bounds evidence for both forms.
"""
from __future__ import annotations

import numpy as np
import pytest

KD, KKC, NT = 4, 4, 256          # ring slots, k steps per chunk, threads of one group
LDS_BUDGET = 156 * 1024          # kChainLdsBudget: dynamic LDS of a block
STATIC_LDS = 3 * 128 * 4 + 2 * 2 * 160 * 4  # l_bias_a, l_bias, l_bias2, l_tap_a, l_tap_b
LDS_CU = 160 * 1024
MAX_STEPS = 160


def chain_nq(*ocs):
    m = max(ocs)
    return 2 if m <= 64 else 3 if m <= 96 else 0


def region_extent(n, t):
    return max(min(o + t + 1, n) - max(o - 1, 0) for o in range(0, n, t))


def chain_lds(C, H, W, nq, tr, tc):
    tr, tc = min(tr, H), min(tc, W)
    r1h, r1w = region_extent(H, tr), region_extent(W, tc)
    if r1h * r1w > 256 or tr * tc > 256:
        return None
    xp = (C // 8) * (r1h + 2) * (r1w + 2)
    xb = (xp + 63) // 64 * 64 * 16
    gb = nq * 4 * (tr + 2) * (tc + 2) * 16
    ring = KD * KKC * 2 * nq * 32 * 16
    total = ring + xb + gb
    if total > LDS_BUDGET:
        return None
    return total, xb


def chain_tile(C, H, W, nq, tr=0, tc=0):
    if tr > 0 and tc > 0:
        return (min(tr, H), min(tc, W)) if chain_lds(C, H, W, nq, tr, tc) else None
    for t in [(H, W), ((H + 1) // 2, W), ((H + 1) // 2, (W + 1) // 2), (8, 8), (6, 8), (4, 8)]:
        if chain_lds(C, H, W, nq, *t):
            return min(t[0], H), min(t[1], W)
    return None


def small_div(a, inv):
    return int((np.float32(a) + np.float32(0.5)) * inv)


def make_params(N, C, H, W, oca, ocb, occ, tr, tc, kg_wanted):
    """make_chain_params: tile, LDS layout, chunk counts; None when the branch does not fit."""
    nq = chain_nq(oca, ocb, occ)
    assert nq, "chain_shape_error refuses > 96 channels"
    t = chain_tile(C, H, W, nq, tr, tc)
    if t is None:
        return None
    TR, TC = t
    lds, xb = chain_lds(C, H, W, nq, TR, TC)
    ka, kb = 9 * C // 16, 9 * oca // 16
    mq = 1 if region_extent(H, TR) * region_extent(W, TC) <= 128 and TR * TC <= 128 else 2
    kg = 2 if kg_wanted == 2 and mq == 1 and xb >= 4 * 16 * 64 * 4 else 1
    ring = KD * KKC * 2 * nq * 32 * 16
    return dict(N=N, C=C, H=H, W=W, oca=oca, ocb=ocb, occ=occ, nq=nq, TR=TR, TC=TC, lds=lds, xb=xb,
                x_off=ring, g_off=ring + xb, ka=ka, kb=kb, nchunk_a=-(-ka // KKC),
                nchunk=-(-ka // KKC) + -(-kb // KKC), mq=mq, kg=kg,
                ntc=-(-W // TC), tpi=-(-H // TR) * -(-W // TC))


def check_block_geometry(h, kg, x_cstride=None, y_cstride=None, out_f32=True):
    C, H, W, nq, mq = h["C"], h["H"], h["W"], h["nq"], h["mq"]
    NOCB = nq * 32
    CB = KKC * 2 * NOCB * 16
    PT = KKC * 2 * NOCB // NT
    KS = KKC // kg
    lds = h["lds"]
    x_off, g_off = h["x_off"], h["g_off"]
    xcs = x_cstride or C
    ycs = y_cstride or h["occ"]
    esz = 4 if out_f32 else 2
    x_img = ((H * W - 1) * xcs + C) * 2
    y_img = ((H * W - 1) * ycs + h["occ"]) * esz
    assert lds + STATIC_LDS <= LDS_CU
    assert kg == 1 or mq == 1
    # tap tables: [chunk][hi][k step], read as KS ints at grp * KS
    for ks in (h["ka"], h["kb"]):
        nch = -(-ks // KKC)
        assert nch * 2 * KKC <= 2 * MAX_STEPS
    # ring: a chunk's LDS-DMA writes (first 4 waves) and the A reads of both groups
    assert (PT * NT) * 16 == CB
    for grp in range(kg):
        for sl in range(KS):
            for hi in (0, 1):
                for j in range(nq):
                    top = (hi * NOCB + 31) * 16 + grp * KS * (2 * NOCB * 16) + sl * (2 * NOCB * 16) + j * 512 + 16
                    assert top <= CB
    # the two-group reduction: 4 waves x MQ x 16 floats x 64 lanes through the window region
    if kg == 2:
        assert 4 * mq * 16 * 64 * 4 <= h["xb"]
    lanes = np.arange(64)
    l32, hi = lanes & 31, lanes >> 5
    for t in range(h["tpi"]):
        trow, tcol = divmod(t, h["ntc"])
        oh0, ow0 = trow * h["TR"], tcol * h["TC"]
        TRr, TCr = min(h["TR"], H - oh0), min(h["TC"], W - ow0)
        GW, GNPIX = TCr + 2, (TRr + 2) * (TCr + 2)
        r1r, r1c = max(oh0 - 1, 0), max(ow0 - 1, 0)
        R1H, R1W = min(oh0 + TRr + 1, H) - r1r, min(ow0 + TCr + 1, W) - r1c
        XW = R1W + 2
        XNPIX = (R1H + 2) * XW
        npos1, npos2 = R1H * R1W, TRr * TCr
        assert npos1 <= 256 and npos2 <= 256
        # X staging: every wave loads 64 pieces from e0 = wave * 64 in steps of the block's threads
        npiece = (C // 8) * XNPIX
        assert npiece * 16 <= h["xb"]
        top = 0
        for e0 in range(0, npiece, 64):
            top = max(top, x_off + (e0 + 64) * 16)
        assert top <= g_off, ("X staging past its region", top, g_off)
        inv_npix, inv_xw = np.float32(1.0) / np.float32(XNPIX), np.float32(1.0) / np.float32(XW)
        for e in range(-(-npiece // 64) * 64):
            pl = small_div(e, inv_npix)
            pix = e - pl * XNPIX
            pr = small_div(pix, inv_xw)
            assert pl == e // XNPIX and pr == pix // XW
            ih, iw = r1r - 1 + pr, r1c - 1 + (pix - pr * XW)
            if e < npiece and 0 <= ih < H and 0 <= iw < W:
                assert ((ih * W + iw) * xcs + pl * 8) * 2 + 16 <= x_img
        # G zeroing and the LDS end
        assert g_off + nq * 4 * GNPIX * 16 <= lds
        # tap offsets of conv a over X and conv b over G: plane and pixel inside the map
        for (cin, ks, npix, w, region) in ((C, h["ka"], XNPIX, XW, npiece), (h["oca"], h["kb"], GNPIX, GW,
                                                                            nq * 4 * GNPIX)):
            nch = -(-ks // KKC)
            for e in range(nch * 2 * KKC):
                c, r = divmod(e, 2 * KKC)
                hh, sl = divmod(r, KKC)
                k0 = 16 * min(c * KKC + sl, ks - 1)
                tap, c0 = divmod(k0, cin)
                plane = (c0 >> 3) + hh
                assert plane < cin // 8
                to = (plane * npix + (tap // 3) * w + tap % 3) * 16
                # largest position offset of a subtile read (clamped to the region)
                assert to // 16 < region
        # per-lane position offsets of both groups' subtiles (lw = wave & 3)
        inv_r1w, inv_tc = np.float32(1.0) / np.float32(R1W), np.float32(1.0) / np.float32(TCr)
        for lw in range(4):
            for q in range(mq):
                pos = (lw + 4 * q) * 32 + l32
                for p1 in np.minimum(pos, npos1 - 1):
                    r1 = small_div(int(p1), inv_r1w)
                    assert r1 == p1 // R1W
                    # largest tap offset: bottom-right tap of the last plane of the chunk
                    pix = r1 * XW + (p1 - r1 * R1W) + 2 * XW + 2
                    assert pix < XNPIX
                for p2 in np.minimum(pos, npos2 - 1):
                    r2 = small_div(int(p2), inv_tc)
                    assert r2 == p2 // TCr
                    c2 = p2 - r2 * TCr
                    assert (r2 * GW + c2) + 2 * GW + 2 < GNPIX
                    yo = ((oh0 + r2) * W + ow0 + c2) * ycs
                    for oc0 in range(0, h["occ"], 4):
                        assert (yo + oc0 + 4) * esz <= y_img
                # epilogue a: the grid pixel of every in-region position, for the grp-0 writers
                dr, dc = r1r - (oh0 - 1), r1c - (ow0 - 1)
                for p in pos[pos < npos1]:
                    r = small_div(int(p), inv_r1w)
                    gp = (r + dr) * GW + (p - r * R1W) + dc
                    assert 0 <= gp < GNPIX


HEADS = {  # input channels and map size of each head level
    320: [(64, 40), (128, 20), (256, 10)],
    160: [(64, 20), (128, 10), (256, 5)],
}
BRANCHES = [(64, 64, 64), (80, 80, 80)]  # box (reg_max 16 x 4) and class (80) branches


@pytest.mark.parametrize("imgsz", [160, 320])
@pytest.mark.parametrize("batch", [1, 2, 64])
@pytest.mark.parametrize("kg", [1, 2])
def test_chain_accesses_stay_in_bounds_on_yolov8n_heads(imgsz, batch, kg):
    seen = 0
    for C, hw in HEADS[imgsz]:
        # the rule's tile (0, 0), the tiles the load-time measurement tries (enumerate_chain_tiles),
        # and a ragged one
        for tile in [(0, 0), (hw, hw), ((hw + 1) // 2, hw), ((hw + 1) // 2, (hw + 1) // 2),
                     ((hw + 2) // 3, (hw + 2) // 3), (8, 8), (6, 8), (5, 5), (4, 4), (3, 3), (5, 4)]:
            # the two-branch launch takes the tile that fits the branch with more channels
            t = chain_tile(C, hw, hw, max(chain_nq(*br) for br in BRANCHES), *tile)
            if t is None:
                continue
            parts = [make_params(batch, C, hw, hw, *br, *t, kg) for br in BRANCHES]
            if any(p is None for p in parts):
                continue
            for p in parts:
                check_block_geometry(p, p["kg"])
                seen += 1
            # two branches in one launch: one tile (the larger branch's), the larger LDS for
            # both, blocks of each branch with their own layout; the same k groups
            p0, p1 = parts
            assert (p0["TR"], p0["TC"]) == (p1["TR"], p1["TC"])
            if p0["mq"] == p1["mq"]:
                assert max(p0["lds"], p1["lds"]) + STATIC_LDS <= LDS_CU
                assert p0["g_off"] + p0["nq"] * 4 * (p0["TR"] + 2) * (p0["TC"] + 2) * 16 <= max(p0["lds"], p1["lds"])
    assert seen >= 6


def test_chain_accesses_stay_in_bounds_on_ragged_and_sliced_maps():
    for (N, C, H, W, a, b, c, tr, tc) in [(2, 256, 10, 10, 80, 80, 80, 0, 0), (2, 128, 20, 20, 80, 80, 80, 10, 10),
                                          (1, 64, 13, 11, 80, 64, 64, 5, 4), (2, 32, 9, 7, 48, 32, 32, 0, 0),
                                          (1, 64, 40, 40, 80, 80, 80, 8, 12), (2, 64, 24, 24, 64, 64, 64, 12, 12)]:
        for kg in (1, 2):
            p = make_params(N, C, H, W, a, b, c, tr, tc, kg)
            assert p is not None
            check_block_geometry(p, p["kg"], x_cstride=C + 64, y_cstride=c + 16, out_f32=False)


def test_geometry_model_catches_a_planted_overflow():
    """The model itself must fail when the window region is one 64-piece group short."""
    p = make_params(64, 256, 10, 10, 80, 80, 80, 0, 0, 1)
    bad = dict(p, g_off=p["g_off"] - 64 * 16)
    with pytest.raises(AssertionError):
        check_block_geometry(bad, 1)
