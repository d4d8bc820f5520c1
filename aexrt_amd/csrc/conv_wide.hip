// Host side of the wide-tile fp16 3x3 conv (kernel in conv_wide.h):
// applicability, tile geometry, launch.
#include <algorithm>

#include <cstdio>
#include "conv_wide.h"

namespace aexrt {

namespace {

constexpr int kWideNPW = 4;                 // window pieces per thread
constexpr int kWideNWP = 8;                 // weight pieces per thread
constexpr int kWideLdsBudget = 150 * 1024;  // dynamic LDS of one block

bool wide_shape_ok(const ConvParams& p) {
    return p.loader == kLoaderNhwc && p.KH == 3 && p.KW == 3 && p.P == 1 && (p.S == 1 || p.S == 2) &&
           p.OH == (p.H - 1) / p.S + 1 && p.OW == (p.W - 1) / p.S + 1 && p.H < 8192 && p.W < 8192 && p.C % 8 == 0 &&
           p.x_cstride % 8 == 0 && p.OCp >= 49 && p.OCp <= 80 && !p.res && !p.acc_out &&
           (p.flags & ~(kConvSilu | kConvOutF32)) == 0 && p.C <= 2048;
}

}  // namespace

bool wide_geometry(WideParams& h, int jn, int pw, int tr, int tc, int cc) {
    const ConvParams& p = h.c;
    if (!(jn == 4 || jn == 5) || jn * 16 < p.OCp || !(pw == 2 || pw == 4) || cc < 8 || cc % 8 || p.C % cc ||
        tr < 1 || tc < 1 || tr * tc > 64 * pw)
        return false;
    const int R = jn * 16;
    h.TR = tr;
    h.TC = tc;
    h.IR = (tr - 1) * p.S + 3;
    h.ICOL = (tc - 1) * p.S + 3;
    h.CC = cc;
    h.nch = p.C / cc;
    h.spc = (9 * cc + 31) / 32;
    if (h.spc > kWideMaxSpc) return false;
    h.npieces = h.IR * h.ICOL * cc / 8;
    h.wpieces = h.spc * R * 4;
    if (h.npieces > 256 * kWideNPW || h.wpieces > 256 * kWideNWP) return false;
    h.ntc = (p.OW + tc - 1) / tc;
    h.tpi = ((p.OH + tr - 1) / tr) * h.ntc;
    const int64_t ntile = (int64_t)p.N * h.tpi;
    if (ntile > INT32_MAX / 2) return false;
    h.ntile = (int)ntile;
    h.pstride = cc * 2;
    h.tbytes = (h.IR * h.ICOL * h.pstride + 15) & ~15;
    h.wbytes = h.wpieces * 16;
    if (2 * (h.wbytes + h.tbytes) > kWideLdsBudget) return false;
    h.fd_cc8 = make_fastdiv((uint32_t)(cc / 8));
    h.fd_icol = make_fastdiv((uint32_t)h.ICOL);
    h.fd_tc = make_fastdiv((uint32_t)tc);
    h.fd_ntc = make_fastdiv((uint32_t)h.ntc);
    h.fd_tpi = make_fastdiv((uint32_t)h.tpi);
    h.fd_cc = make_fastdiv((uint32_t)cc);
    h.fd_spc4 = make_fastdiv((uint32_t)(R * 4));
    return true;
}

int enumerate_wide_choices(const ConvParams& p, ConvChoice* out, int cap) {
    if (!wide_shape_ok(p)) return 0;
    const int jn = p.OCp <= 64 ? 4 : 5;
    int n = 0;
    for (int cc : {8, 16, 24}) {
        for (int pw : {2, 4}) {
            const int npos = 64 * pw;
            const int tcs[4] = {p.OW, 16, 32, 48};
            for (int i = 0; i < 4 && n < cap; ++i) {
                const int tc = tcs[i];
                bool dup = false;
                for (int k = 0; k < i; ++k) dup = dup || tcs[k] == tc;
                if (dup || tc > p.OW || (tc < p.OW && tc > npos)) continue;
                const int tr = std::min(p.OH, npos / tc);
                WideParams h{};
                h.c = p;
                if (tr < 1 || !wide_geometry(h, jn, pw, tr, tc, cc)) continue;
                ConvChoice c;
                c.kind = 4;
                c.jn = jn;
                c.pw = pw;
                c.tr = tr;
                c.tc = tc;
                c.cc = cc;
                out[n++] = c;
            }
        }
    }
    return n;
}

namespace {

template <int JN, int PW, int EPI>
hipError_t wide_launch_cfg(WideParams h, hipStream_t stream) {
    const int lds_bytes = 2 * (h.wbytes + h.tbytes);
    auto kern = wide::conv3x3_wide_kernel<JN, PW, kWideNPW, kWideNWP, EPI>;
    int per_cu = 0, cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, (size_t)lds_bytes) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu < 1 ||
        cus < 1) {
        per_cu = 1;
        cus = 256;
    }
    const int groups0 = std::min(h.ntile, per_cu * cus);
    h.c.per = (h.ntile + groups0 - 1) / groups0;
    const int groups = (h.ntile + h.c.per - 1) / h.c.per;
    hipLaunchKernelGGL(kern, dim3((unsigned)groups), dim3(256), (size_t)lds_bytes, stream, h);
    return hipGetLastError();
}

}  // namespace

// One batch slice (views inside 32-bit spans), choice kind 4.
hipError_t launch_conv_wide(const ConvParams& p, int epi, hipStream_t stream) {
    if (!wide_shape_ok(p) || p.choice.kind != 4 || (epi != igemm::kEpiAny && epi != igemm::kEpiSilu))
        return hipErrorInvalidValue;
    WideParams h{};
    h.c = p;
    const ConvChoice& t = p.choice;
    if (!wide_geometry(h, t.jn, t.pw, t.tr, t.tc, t.cc)) return hipErrorInvalidValue;
    if (LaunchProbe* pr = launch_probe()) {
        // the kernel template instance (as a trace names it), then the tile
        std::snprintf(pr->name, sizeof(pr->name), "conv3x3_wide_kernel<%d,%d,%d,%d,%d> %dx%d cc%d", t.jn, t.pw,
                      kWideNPW, kWideNWP, epi == igemm::kEpiSilu ? (int)igemm::kEpiSilu : (int)igemm::kEpiAny, t.tr,
                      t.tc, t.cc);
        return hipSuccess;
    }
#define AEXRT_WIDE_CASE(J, P)                                                                    \
    if (t.jn == J && t.pw == P)                                                                  \
        return epi == igemm::kEpiSilu ? wide_launch_cfg<J, P, igemm::kEpiSilu>(h, stream)        \
                                      : wide_launch_cfg<J, P, igemm::kEpiAny>(h, stream);
    AEXRT_WIDE_CASE(4, 2) AEXRT_WIDE_CASE(4, 4) AEXRT_WIDE_CASE(5, 2) AEXRT_WIDE_CASE(5, 4)
#undef AEXRT_WIDE_CASE
    return hipErrorInvalidValue;
}

}  // namespace aexrt
