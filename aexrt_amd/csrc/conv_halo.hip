// Host side of the halo-tile 3x3 conv (kernel in conv_halo.h): applicability,
// tile choice, launch geometry.
#include <algorithm>
#include <atomic>
#include <cmath>

#include <cstdio>
#include "conv_halo.h"

namespace aexrt {

namespace halo {
AEXRT_HALO_FAMILIES(AEXRT_HALO_EXTERN)
}  // namespace halo

namespace {

// 0: automatic; 1: never (implicit GEMM only); 2: forced tile (g_force).
std::atomic<int> g_halo_mode{0};
std::atomic<uint64_t> g_force{0};  // jn | pw << 8 | tr << 16 | tc << 32 | cc << 48 (8/8/16/16/16 bits)
std::atomic<int> g_force_nw{4};     // waves per block of the forced tile

// dynamic LDS of one block (static tables aside): two blocks fit a CU's 160 KB;
// 8-wave blocks may take most of a CU (one block per CU)
constexpr int kLdsBudget = 80 * 1024 - 2048;
constexpr int kLdsBudget8 = 152 * 1024;

struct HaloTile {
    int jn, pw, np, TR, TC, CC;
    int nw = 4;  // waves per block
};

int pow2_at_least(int v, int cap) {
    int r = 1;
    while (r < v && r < cap) r <<= 1;
    return r;
}

// Fills the geometry of tile t into h; false when it does not fit the kernel.
bool halo_geometry(HaloParams& h, const HaloTile& t, bool int8) {
    const ConvParams& p = h.c;
    const int esz = int8 ? 1 : 2;
    const int wq = int8 ? 1 : 2;
    // int8: a 16-k MFMA operand piece is 16 channels of one tap; fp16: 8
    if (t.CC < (int8 ? 16 : 8) || t.CC % (int8 ? 16 : 8) || p.C % t.CC || t.TR < 1 || t.TC < 1) return false;
    if (p.loader == kLoaderNchwF32 && t.CC != p.C) return false;
    if (t.TR * t.TC > 16 * t.nw * t.pw) return false;
    h.TR = t.TR;
    h.TC = t.TC;
    h.IR = (t.TR - 1) * p.S + 3;
    h.ICOL = (t.TC - 1) * p.S + 3;
    h.CC = t.CC;
    h.nch = p.C / t.CC;
    h.spc = (9 * t.CC + 63) / 64;
    if (h.spc > kHaloMaxSpc) return false;
    h.npieces = h.IR * h.ICOL * t.CC / 8;
    if (p.loader == kLoaderNchwF32) {
        // 16-byte quads of one channel row; every tile's first quad starts
        // at a multiple of 4 columns
        if ((t.TC * p.S) % 4) return false;
        h.icol4 = (h.ICOL + 3 + 3) / 4;
        h.npieces = p.c_real * h.IR * h.icol4;
        h.fd_icol4 = make_fastdiv((uint32_t)h.icol4);
        h.fd_rq = make_fastdiv((uint32_t)(h.IR * h.icol4));
    }
    if (h.npieces > 64 * t.nw * t.np) return false;
    h.ntc = (p.OW + t.TC - 1) / t.TC;
    h.tpi = ((p.OH + t.TR - 1) / t.TR) * h.ntc;
    const int64_t ntile = (int64_t)p.N * h.tpi;
    if (ntile > INT32_MAX / 2) return false;
    h.ntile = (int)ntile;
    h.wbytes = h.nch * h.spc * wq * t.jn * 16 * 64;
    // an MFMA operand read takes 16 bytes of 16 consecutive window pixels: a
    // pixel stride that is an odd multiple of 16 bytes spreads them over all
    // LDS banks, an even one folds them onto a quarter or half of the banks
    h.pstride = t.CC * esz;
    if ((h.pstride / 16) % 2 == 0) h.pstride += 16;
    h.tbytes = (h.IR * h.ICOL * h.pstride + 15) & ~15;
    if (h.wbytes + 2 * h.tbytes > (t.nw == 8 ? kLdsBudget8 : kLdsBudget) ||
        h.wbytes > 64 * t.nw * kHaloWeightRounds * 16)
        return false;
    h.c.ntn = (p.OCp / 16 + t.jn - 1) / t.jn;
    h.fd_cc8 = make_fastdiv((uint32_t)(t.CC / 8));
    h.fd_icol = make_fastdiv((uint32_t)h.ICOL);
    h.fd_tc = make_fastdiv((uint32_t)t.TC);
    h.fd_ntc = make_fastdiv((uint32_t)h.ntc);
    h.fd_tpi = make_fastdiv((uint32_t)h.tpi);
    h.fd_cc = make_fastdiv((uint32_t)t.CC);
    h.fd_spc = make_fastdiv((uint32_t)h.spc);
    h.c.fd_ntn = make_fastdiv((uint32_t)h.c.ntn);
    return true;
}

// Estimated duration (GPU clocks) of a launch with tile t.  Per tile and
// block: MFMA issue of one wave, LDS operand reads of the 4 waves, window
// staging (loads + int8 quantization), a fixed part per chunk (barrier,
// latency) and per tile (epilogue).  Blocks spread over 256 CUs; the input
// window traffic (with its halo, once per oc tile) and the output bound from
// below.
double halo_cost(const HaloParams& h, const HaloTile& t, bool int8) {
    const ConvParams& p = h.c;
    const int wq = int8 ? 1 : 2;
    const double steps = (double)h.nch * h.spc;
    const double t_mfma = steps * t.jn * t.pw * wq * 16.0;
    const double t_lds = steps * (t.jn + t.pw) * wq * 4 * 8.0;
    const double t_stage = h.nch * std::ceil(h.npieces / 256.0) * (int8 ? 110.0 : 24.0);
    const double t_tile = std::max(t_mfma, t_lds) + t_stage + h.nch * 350.0 + t.jn * t.pw * (int8 ? 160.0 : 120.0);
    const double blocks = (double)h.ntile * h.c.ntn;
    const double waves_of_blocks = std::ceil(blocks / 512.0);  // ~2 blocks per CU overlap
    const double compute = waves_of_blocks * t_tile;
    const double bytes = blocks * h.nch * h.npieces * 16.0 + (double)p.M * p.OC * 2.0;
    return std::max(compute, bytes / 2500.0) + 1500.0;
}

bool halo_shape_ok(const ConvParams& p, bool int8) {
    if (!(p.KH == 3 && p.KW == 3 && p.P == 1 && (p.S == 1 || p.S == 2) && p.OH == (p.H - 1) / p.S + 1 &&
          p.OW == (p.W - 1) / p.S + 1 && p.H < 8192 && p.W < 8192))
        return false;
    if (p.loader == kLoaderNchwF32)
        return !int8 && p.C == 8 && p.c_real >= 1 && p.c_real <= 4 && p.flags == kConvSilu;
    return p.loader == kLoaderNhwc && p.C % (int8 ? 16 : 8) == 0 && p.x_cstride % 8 == 0;
}

// Lowest-cost tile of the instantiated shapes.
bool choose_halo_tile(HaloParams& h, bool int8, HaloTile& best) {
    const ConvParams& p = h.c;
    double best_cost = 0.0;
    bool found = false;
    const int ocj = (p.OCp + 15) / 16;
    const bool nchw = p.loader == kLoaderNchwF32;
    for (int div = 1; div <= 8; div <<= 1) {
        if (p.C % div) break;
        const int CC = p.C / div;
        if (CC % (int8 ? 16 : 8) || CC > (int8 ? 128 : 64)) continue;
        for (int jn = 1; jn <= std::min(4, pow2_at_least(ocj, 4)); jn <<= 1) {
            for (int pw = nchw ? 2 : 1; pw <= 4; pw <<= 1) {
                // the whole row, or its width rounded up to 4 (the NCHW
                // loader needs TC * S % 4 == 0), or multiples of 16
                const int ow4 = (p.OW + 3) / 4 * 4;
                int tcs[7] = {p.OW, ow4, 16, 32, 48, 64, 80};
                for (int tc : tcs) {
                    if (tc > ow4 || (tc > p.OW && tc != ow4) || (tc < p.OW && tc > 64 * pw)) continue;
                    const int TR = std::min(p.OH, 64 * pw / tc);
                    if (TR < 1) continue;
                    for (int np : {4, 8}) {
                        const HaloTile t{jn, pw, np, TR, tc, CC};
                        HaloParams hh = h;
                        if (!halo_geometry(hh, t, int8)) continue;
                        if (np == 8 && hh.npieces <= 4 * 64 * t.nw) continue;
                        const double c = halo_cost(hh, t, int8);
                        if (!found || c < best_cost) {
                            best_cost = c;
                            best = t;
                            found = true;
                        }
                    }
                }
            }
        }
    }
    return found;
}

hipError_t halo_launch(const HaloParams& h, bool int8, int epi, const HaloTile& t, hipStream_t s) {
    using halo::halo_launch_family;
    if (LaunchProbe* pr = launch_probe()) {
        // the kernel template instance (as a trace names it), then the tile
        const bool nchw = h.c.loader == kLoaderNchwF32;
        std::snprintf(pr->name, sizeof(pr->name), "conv3x3_halo_kernel<%s,%d,%d,%d,%d,%s,%d> %dx%d cc%d",
                      int8 ? "true" : "false", t.jn, t.pw, t.np, nchw ? (int)igemm::kEpiSilu : epi,
                      nchw ? "true" : "false", nchw ? 4 : t.nw, t.TR, t.TC, t.CC);
        return hipSuccess;
    }
    if (h.c.loader == kLoaderNchwF32) return halo::halo_launch_nchw(h, t.jn, t.pw, t.np, s);
    if (int8) {
        if (epi == 1) return halo_launch_family<true, 1>(h, t.jn, t.pw, t.np, t.nw, s);
        if (epi == 2) return halo_launch_family<true, 2>(h, t.jn, t.pw, t.np, t.nw, s);
        return halo_launch_family<true, 0>(h, t.jn, t.pw, t.np, t.nw, s);
    }
    if (epi == 1) return halo_launch_family<false, 1>(h, t.jn, t.pw, t.np, t.nw, s);
    return halo_launch_family<false, 0>(h, t.jn, t.pw, t.np, t.nw, s);
}

}  // namespace

int enumerate_halo_choices(const ConvParams& p, bool int8, ConvChoice* out, int cap) {
    if (!halo_shape_ok(p, int8)) return 0;
    const bool nchw = p.loader == kLoaderNchwF32;
    const int ocj = (p.OCp + 15) / 16;
    const int ow4 = (p.OW + 3) / 4 * 4;
    int n = 0;
    for (int div = 1; div <= 8 && n < cap; div <<= 1) {
        if (p.C % div) break;
        const int CC = p.C / div;
        if (CC % (int8 ? 16 : 8) || CC > (int8 ? 128 : 64)) continue;
        for (int nw = 4; nw <= (nchw ? 4 : 8) && n < cap; nw <<= 1)
        for (int jn = 1; jn <= (ocj == 5 && nw == 8 && !int8 ? 5 : std::min(4, pow2_at_least(ocj, 4))) && n < cap;
             jn = jn == 4 ? 5 : jn << 1) {
            if (jn == 5 && ocj != 5) continue;
            for (int pw = nchw ? 2 : 1; pw <= (nw == 8 ? 2 : 4) && n < cap; pw <<= 1) {
                // fp16 tiles of 4-5 channel subtiles with 2 or more position
                // subtiles per wave need more than 256 registers and spill to
                // scratch memory (slow, and a first launch has to grow the
                // queue's scratch): not offered
                if (!int8 && jn >= 4 && pw >= (nchw ? 4 : 2)) continue;
                const int npos = 16 * nw * pw;  // positions of a tile
                const int tcs[7] = {p.OW, ow4, 16, 32, 48, 64, 80};
                for (int i = 0; i < 7 && n < cap; ++i) {
                    const int tc = tcs[i];
                    bool dup = false;
                    for (int k = 0; k < i; ++k) dup = dup || tcs[k] == tc;
                    if (dup || tc > ow4 || (tc > p.OW && tc != ow4) || (tc < p.OW && tc > npos)) continue;
                    const int TR = std::min(p.OH, npos / tc);
                    if (TR < 1) continue;
                    HaloParams hh{};
                    hh.c = p;
                    HaloTile t{jn, pw, 4, TR, tc, CC, nw};
                    if (!halo_geometry(hh, t, int8)) {
                        t.np = 8;
                        if (!halo_geometry(hh, t, int8)) continue;
                    }
                    ConvChoice c;
                    c.kind = 2;
                    c.jn = jn;
                    c.pw = pw;
                    c.tr = TR;
                    c.tc = tc;
                    c.cc = CC;
                    c.nw = nw;
                    out[n++] = c;
                }
            }
        }
    }
    return n;
}

bool set_conv3x3_halo(int mode, int jn, int pw, int tr, int tc, int cc) {
    if (mode == 0 || mode == 1) {
        g_halo_mode.store(mode);
        return true;
    }
    if (mode == 4) {
        // the wide-tile fp16 kernel: jn 4 or 5 channel subtiles, pw 2 or 4
        if (!(jn == 4 || jn == 5) || !(pw == 2 || pw == 4) || tr < 1 || tr > 0xFFFF || tc < 1 || tc > 0xFFFF ||
            cc < 8 || cc > 0xFFFF)
            return false;
        g_force.store((uint64_t)jn | ((uint64_t)pw << 8) | ((uint64_t)tr << 16) | ((uint64_t)tc << 32) |
                      ((uint64_t)cc << 48));
        g_halo_mode.store(4);
        return true;
    }
    // mode 2: 4 waves per block, mode 3: 8 waves (pw 1 or 2; jn 5 only with 8 waves)
    if ((mode != 2 && mode != 3) || !(jn == 1 || jn == 2 || jn == 4 || (jn == 5 && mode == 3)) ||
        !(pw == 1 || pw == 2 || pw == 4) ||
        (mode == 3 && pw == 4) || tr < 1 || tr > 0xFFFF || tc < 1 || tc > 0xFFFF || cc < 8 || cc > 0xFFFF)
        return false;
    g_force.store((uint64_t)jn | ((uint64_t)pw << 8) | ((uint64_t)tr << 16) | ((uint64_t)tc << 32) |
                  ((uint64_t)cc << 48));
    g_force_nw.store(mode == 3 ? 8 : 4);
    g_halo_mode.store(2);
    return true;
}

bool forced_wide_choice(ConvChoice& c) {
    if (g_halo_mode.load(std::memory_order_relaxed) != 4) return false;
    const uint64_t f = g_force.load(std::memory_order_relaxed);
    c = ConvChoice{};
    c.kind = 4;
    c.jn = (int)(f & 0xFF);
    c.pw = (int)((f >> 8) & 0xFF);
    c.tr = (int)((f >> 16) & 0xFFFF);
    c.tc = (int)((f >> 32) & 0xFFFF);
    c.cc = (int)((f >> 48) & 0xFFFF);
    return true;
}

// One batch slice of a conv (views already inside 32-bit spans).
// hipErrorNotSupported: the shape is not a halo-tile conv (the caller uses
// the implicit-GEMM kernel).
hipError_t launch_conv_halo(const ConvParams& p, bool int8, int epi, hipStream_t stream) {
    if (!halo_shape_ok(p, int8)) return hipErrorNotSupported;
    // the NCHW input has no other kernel; the tile modes apply to NHWC convs
    const int mode = p.loader == kLoaderNchwF32 ? 0 : g_halo_mode.load(std::memory_order_relaxed);
    if (mode == 1 && p.choice.kind != 2) return hipErrorNotSupported;
    HaloParams h{};
    h.c = p;
    HaloTile t{};
    if (mode == 2 || p.choice.kind == 2) {
        if (p.choice.kind == 2) {
            t.jn = p.choice.jn;
            t.pw = p.choice.pw;
            t.TR = p.choice.tr;
            t.TC = p.choice.tc;
            t.CC = p.choice.cc;
            t.nw = p.choice.nw;
        } else {
            const uint64_t f = g_force.load(std::memory_order_relaxed);
            t.jn = (int)(f & 0xFF);
            t.pw = (int)((f >> 8) & 0xFF);
            t.TR = (int)((f >> 16) & 0xFFFF);
            t.TC = (int)((f >> 32) & 0xFFFF);
            t.CC = (int)((f >> 48) & 0xFFFF);
            t.nw = g_force_nw.load(std::memory_order_relaxed);
        }
        // a forced tile that does not fit this conv is an error, not a
        // silent fallback (tests rely on the tile being used)
        t.np = 4;
        if (!halo_geometry(h, t, int8)) {
            t.np = 8;
            HaloParams h8 = h;
            if (!halo_geometry(h8, t, int8)) return hipErrorInvalidValue;
        }
    } else if (!choose_halo_tile(h, int8, t)) {
        return hipErrorNotSupported;
    }
    if (!halo_geometry(h, t, int8)) return hipErrorNotSupported;
    return halo_launch(h, int8, epi, t, stream);
}

}  // namespace aexrt
