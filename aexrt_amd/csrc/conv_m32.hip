// Host side of the 32x32-MFMA 3x3 conv (kernel in conv_m32.h): geometry,
// candidate tiles, forced tiles, launch.
#include <algorithm>
#include <atomic>
#include <cstdio>

#include "conv_m32.h"

namespace aexrt {

namespace m32 {
AEXRT_M32_FAMILIES(AEXRT_M32_EXTERN)
}  // namespace m32

namespace {

// dynamic LDS of one block (its static tables aside)
constexpr int kM32LdsBudget = 156 * 1024;

struct M32Tile {
    int mq, nq, np, TR, TC, CC;
    int nw = 4;  // waves per block
    int ng = 1;  // wave groups (2: two groups of 4 with their own windows and barriers)
};

bool m32_shape_ok(const ConvParams& p) {
    return p.KH == 3 && p.KW == 3 && p.P == 1 && (p.S == 1 || p.S == 2) && p.OH == (p.H - 1) / p.S + 1 &&
           p.OW == (p.W - 1) / p.S + 1 && p.H < 8192 && p.W < 8192 && p.loader == kLoaderNhwc && p.C % 16 == 0 &&
           p.x_cstride % 8 == 0;
}

// Fills the geometry of tile t into h; false when it does not fit the kernel.
bool m32_geometry(M32Params& h, const M32Tile& t, bool int8) {
    const ConvParams& p = h.c;
    const int cpp = int8 ? 16 : 8;
    const int ksub = int8 ? 32 : 16;
    if (t.CC < 16 || t.CC % 16 || p.C % t.CC || t.TR < 1 || t.TC < 1 || t.mq < 1 || t.nq < 1) return false;
    if (t.ng < 1 || t.nw % t.ng || t.TR * t.TC > t.nw / t.ng * 32 * t.mq) return false;
    h.TR = t.TR;
    h.TC = t.TC;
    h.IR = (t.TR - 1) * p.S + 3;
    h.ICOL = (t.TC - 1) * p.S + 3;
    h.NPIX = h.IR * h.ICOL;
    h.CC = t.CC;
    h.nch = p.C / t.CC;
    h.nks = (9 * t.CC + ksub - 1) / ksub;
    if (h.nks > kM32MaxSteps) return false;
    h.npiece = (t.CC / cpp) * h.NPIX;
    if (h.npiece > 64 * (t.nw / t.ng) * t.np) return false;
    h.ntc = (p.OW + t.TC - 1) / t.TC;
    h.tpi = ((p.OH + t.TR - 1) / t.TR) * h.ntc;
    const int64_t ntile = (int64_t)p.N * h.tpi;
    if (ntile > INT32_MAX / 2) return false;
    h.ntile = (int)ntile;
    const int nocb = t.nq * 32;
    h.wbytes = h.nch * h.nks * 2 * nocb * 16;
    h.tbytes = h.npiece * 16;
    if ((int64_t)h.wbytes + t.ng * 2 * h.tbytes > kM32LdsBudget) return false;
    h.c.ntn = (p.OCp + nocb - 1) / nocb;
    h.fd_npix = make_fastdiv((uint32_t)h.NPIX);
    h.fd_icol = make_fastdiv((uint32_t)h.ICOL);
    h.fd_tc = make_fastdiv((uint32_t)t.TC);
    h.fd_ntc = make_fastdiv((uint32_t)h.ntc);
    h.fd_tpi = make_fastdiv((uint32_t)h.tpi);
    h.fd_cc = make_fastdiv((uint32_t)t.CC);
    h.fd_nks = make_fastdiv((uint32_t)h.nks);
    h.fd_nocb = make_fastdiv((uint32_t)nocb);
    h.c.fd_ntn = make_fastdiv((uint32_t)h.c.ntn);
    return true;
}

// (mq, nq) tiles of 8 subtiles have no 8-round window instance (registers);
// 8-wave blocks exist for tiles of at most 4 subtiles
bool m32_instantiated(int mq, int nq, int np, int nw, int ng = 1) {
    if (np != 4 && np != 8) return false;
    if (ng == 2) {
        if (nw != 8) return false;
        if (np == 8) return (mq == 1 && nq <= 2) || (mq == 2 && nq == 1);
        return (mq == 1 && nq <= 3) || (mq == 2 && nq <= 2);
    }
    if (ng != 1) return false;
    if (nw == 8) {
        if (np == 8) return (mq == 1 && nq <= 2) || (mq == 2 && nq == 1);
        return (mq == 1 && nq <= 3) || (mq == 2 && nq <= 2);
    }
    if (nw != 4) return false;
    if (np == 8 && mq * nq == 8) return false;
    if (mq == 4) return nq == 1 || nq == 2;
    return (mq == 1 || mq == 2) && nq >= 1 && nq <= 4;
}

// Tiles with a fused-1x1 instance (conv_m32_f16_f2.hip).
bool m32_f2_instantiated(int mq, int nq, int np, int nw, int ng = 1) {
    if (ng == 2) return nw == 8 && mq == 1 && (nq == 2 || nq == 3) && (np == 4 || np == 8);
    if (ng != 1) return false;
    if (nw == 4) {
        if (np == 4) return (mq == 1 || mq == 2) && (nq == 2 || nq == 3);
        return np == 8 && ((mq <= 2 && nq == 2) || (mq == 1 && nq == 3));
    }
    if (nw == 8) {
        if (np == 4) return (mq == 1 && (nq == 2 || nq == 3)) || (mq == 2 && nq == 2);
        return np == 8 && mq == 1 && nq == 2;
    }
    return false;
}

// The fused 1x1 fits a tile of nq channel subtiles: its input is every output
// channel of the block (one channel tile), it reads k < 32 nq of its padded
// rows, and its output channels fit the block's second product.
bool m32_f2_ok(const ConvParams& p, int nq) {
    const ConvParams* f = p.fuse_1x1;
    if (!f) return true;
    const int nocb = nq * 32;
    return p.OCp <= nocb && f->C == p.OC && f->KH == 1 && f->KW == 1 && f->S == 1 && f->P == 0 && f->N == p.N &&
           f->H == p.OH && f->W == p.OW && f->OCp <= nocb && f->Kp >= nocb && f->OC % 4 == 0 && f->w && f->bias &&
           f->y && !(f->flags & ~(kConvSilu | kConvOutF32)) && !(p.flags & (kConvResidual | kConvOutF32)) &&
           (p.flags & kConvSilu);
}

// Smallest instantiated piece count that holds the window.
bool m32_fit(M32Params& h, M32Tile& t, bool int8) {
    const bool f2 = h.c.fuse_1x1 != nullptr;
    if (f2 && (int8 || !m32_f2_ok(h.c, t.nq))) return false;
    for (int np : {4, 8}) {
        if (f2 ? !m32_f2_instantiated(t.mq, t.nq, np, t.nw, t.ng) : !m32_instantiated(t.mq, t.nq, np, t.nw, t.ng))
            continue;
        t.np = np;
        M32Params hh = h;
        if (m32_geometry(hh, t, int8)) {
            h = hh;
            return true;
        }
    }
    return false;
}

std::atomic<bool> g_m32_forced{false};
std::atomic<uint64_t> g_m32_force{0};  // mq | nq << 8 | tr << 16 | tc << 32 | cc << 48
std::atomic<int> g_m32_force_nw{4};
std::atomic<int> g_m32_force_ng{1};

hipError_t m32_launch(const M32Params& h, bool int8, int epi, const M32Tile& t, hipStream_t s) {
    using m32::m32_launch_family;
    const bool f2 = h.c.fuse_1x1 != nullptr;
    if (LaunchProbe* pr = launch_probe()) {
        std::snprintf(pr->name, sizeof(pr->name), "conv3x3_m32_kernel<%s,%d,%d,%d,%d,%d%s> %dx%d cc%d",
                      int8 ? "true" : "false", t.mq, t.nq, t.np, epi, t.nw,
                      t.ng == 2 ? (f2 ? ",true,2" : ",false,2") : (f2 ? ",true" : ""), t.TR, t.TC, t.CC);
        return hipSuccess;
    }
    if (f2) {
        if (int8 || epi != 1) return hipErrorInvalidValue;
        M32Params hf = h;
        hf.c2 = *h.c.fuse_1x1;
        return m32::m32_launch_f2(hf, t.mq, t.nq, t.np, t.nw, t.ng, s);
    }
    if (int8) {
        if (epi == 1) return m32_launch_family<true, 1>(h, t.mq, t.nq, t.np, t.nw, t.ng, s);
        if (epi == 2) return m32_launch_family<true, 2>(h, t.mq, t.nq, t.np, t.nw, t.ng, s);
        return m32_launch_family<true, 0>(h, t.mq, t.nq, t.np, t.nw, t.ng, s);
    }
    if (epi == 1) return m32_launch_family<false, 1>(h, t.mq, t.nq, t.np, t.nw, t.ng, s);
    return m32_launch_family<false, 0>(h, t.mq, t.nq, t.np, t.nw, t.ng, s);
}

}  // namespace

int enumerate_m32_choices(const ConvParams& p, bool int8, ConvChoice* out, int cap) {
    if (!m32_shape_ok(p)) return 0;
    int n = 0;
    const int oc32 = (p.OCp + 31) / 32;
    // channel chunks: every CC = C / div (CC % 16 == 0) from the whole input down to 16 channels
    for (int div = 1; div <= p.C / 16 && n < cap; ++div) {
        if (p.C % div) continue;
        const int CC = p.C / div;
        if (CC % 16 || (div > 8 && CC != 16)) continue;
        for (int nq = 1; nq <= 4 && n < cap; ++nq) {
            if (nq > oc32 || (nq == 3 && oc32 != 3)) continue;  // 3 subtiles only for 65..96 channels
            for (int nwg : {4, 8, 16})  // waves per block x groups: 4 x 1, 8 x 1, 8 x 2
            for (int mq : {1, 2, 4}) {
                if (n >= cap) break;
                const int nw = nwg == 16 ? 8 : nwg, ng = nwg == 16 ? 2 : 1;
                if (p.fuse_1x1 ? !m32_f2_instantiated(mq, nq, 4, nw, ng) : !m32_instantiated(mq, nq, 4, nw, ng)) continue;
                const int npos = nw / ng * 32 * mq;
                const int tcs[4] = {p.OW, 32, 16, 8};
                for (int i = 0; i < 4 && n < cap; ++i) {
                    const int tc = tcs[i];
                    bool dup = false;
                    for (int k = 0; k < i; ++k) dup = dup || tcs[k] == tc;
                    if (dup || tc > p.OW || tc > npos || (tc < p.OW && i > 0 && p.OW <= npos)) continue;
                    const int TR = std::min(p.OH, npos / tc);
                    if (TR < 1) continue;
                    M32Params h{};
                    h.c = p;
                    M32Tile t{mq, nq, 4, TR, tc, CC, nw, ng};
                    if (!m32_fit(h, t, int8)) continue;
                    ConvChoice c;
                    c.kind = 5;
                    c.jn = nq;
                    c.pw = mq;
                    c.tr = TR;
                    c.tc = tc;
                    c.cc = CC;
                    c.nw = nw;
                    c.ksw = ng - 1;  // kind 5 keeps its wave groups (minus one) here
                    out[n++] = c;
                }
            }
        }
    }
    return n;
}

bool set_conv3x3_m32(bool on, int mq, int nq, int tr, int tc, int cc, int nw, int ng) {
    if (!on) {
        g_m32_forced.store(false);
        return true;
    }
    if (!m32_instantiated(mq, nq, 4, nw, ng) || tr < 1 || tr > 0xFFFF || tc < 1 || tc > 0xFFFF || cc < 16 || cc > 0xFFFF)
        return false;
    g_m32_force_nw.store(nw);
    g_m32_force_ng.store(ng);
    g_m32_force.store((uint64_t)mq | ((uint64_t)nq << 8) | ((uint64_t)tr << 16) | ((uint64_t)tc << 32) |
                      ((uint64_t)cc << 48));
    g_m32_forced.store(true);
    return true;
}

bool forced_m32_choice(ConvChoice& c) {
    if (!g_m32_forced.load(std::memory_order_relaxed)) return false;
    const uint64_t f = g_m32_force.load(std::memory_order_relaxed);
    c = ConvChoice{};
    c.kind = 5;
    c.pw = (int)(f & 0xFF);
    c.jn = (int)((f >> 8) & 0xFF);
    c.tr = (int)((f >> 16) & 0xFFFF);
    c.tc = (int)((f >> 32) & 0xFFFF);
    c.cc = (int)((f >> 48) & 0xFFFF);
    c.nw = g_m32_force_nw.load(std::memory_order_relaxed);
    c.ksw = g_m32_force_ng.load(std::memory_order_relaxed) - 1;
    return true;
}

// One batch slice of a conv with a kind-5 choice (views already inside
// 32-bit spans).  A choice that does not fit the conv is an error.
hipError_t launch_conv_m32(const ConvParams& p, bool int8, int epi, hipStream_t stream) {
    if (!m32_shape_ok(p) || p.choice.kind != 5) return hipErrorInvalidValue;
    M32Params h{};
    h.c = p;
    M32Tile t{p.choice.pw, p.choice.jn, 4, p.choice.tr, p.choice.tc, p.choice.cc, p.choice.nw, p.choice.ksw + 1};
    if (!m32_fit(h, t, int8)) return hipErrorInvalidValue;
    return m32_launch(h, int8, epi, t, stream);
}

}  // namespace aexrt
