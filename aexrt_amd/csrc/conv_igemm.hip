// Host side of the implicit-GEMM conv (kernel in conv_igemm.h): per-wave tile
// choice, batch splitting for 32-bit view offsets, launch parameters.
#include <algorithm>
#include <atomic>

#include <cstdio>
#include "conv_igemm.h"

namespace aexrt {

namespace igemm {
AEXRT_IGEMM_FAMILIES(AEXRT_IGEMM_EXTERN)
}  // namespace igemm

namespace {

hipError_t launch_variant(bool int8, bool mc, int epi, const ConvParams& p, const ConvTile& t, hipStream_t s) {
    using igemm::launch_family;
    if (LaunchProbe* pr = launch_probe()) {
        // the kernel template instance (as a trace names it), then the tile
        std::snprintf(pr->name, sizeof(pr->name), "conv_mfma_kernel<%s,%d,%d,%s,%s,%d>", int8 ? "true" : "false",
                      t.jn, t.pw, t.ksw ? "true" : "false", mc ? "true" : "false", epi);
        return hipSuccess;
    }
    if (int8) {
        if (mc) {
            if (epi == 1) return launch_family<true, true, 1>(p, t, s);
            if (epi == 2) return launch_family<true, true, 2>(p, t, s);
            return launch_family<true, true, 0>(p, t, s);
        }
        if (epi == 1) return launch_family<true, false, 1>(p, t, s);
        if (epi == 2) return launch_family<true, false, 2>(p, t, s);
        return launch_family<true, false, 0>(p, t, s);
    }
    if (mc) return epi == 1 ? launch_family<false, true, 1>(p, t, s) : launch_family<false, true, 0>(p, t, s);
    return epi == 1 ? launch_family<false, false, 1>(p, t, s) : launch_family<false, false, 0>(p, t, s);
}

int pow2_at_least(int v, int cap) {
    int r = 1;
    while (r < v && r < cap) r <<= 1;
    return r;
}

// Byte span of an NHWC view of N images (0 when absent).
uint64_t view_span(int N, int64_t nstride, int32_t cstride, int HW, int C, int esz) {
    if (N <= 0) return 0;
    return (uint64_t)(((int64_t)(N - 1) * nstride + (int64_t)(HW - 1) * cstride + C) * esz);
}

}  // namespace

namespace {
thread_local LaunchProbe* g_probe = nullptr;
}  // namespace

void set_launch_probe(LaunchProbe* probe) { g_probe = probe; }
LaunchProbe* launch_probe() { return g_probe; }

void conv_kernel_name(const ConvParams& p, bool int8, char* out, size_t n) {
    LaunchProbe pr{};
    std::snprintf(pr.name, sizeof(pr.name), "none");
    LaunchProbe* prev = g_probe;
    g_probe = &pr;
    const hipError_t e = launch_conv_igemm(p, int8, nullptr);
    g_probe = prev;
    std::snprintf(out, n, "%s", e == hipSuccess ? pr.name : "not launchable");
}

namespace {
// jn * 100 + pw * 10 + ksw + 1, 0 = no override
std::atomic<int> g_tile_override{0};

bool tile_instantiated(const ConvTile& t) {
    if (t.ksw) return t.pw == 1 && (t.jn == 1 || t.jn == 2 || t.jn == 4 || t.jn == 8);
    switch (t.jn * 8 + t.pw) {
        case 9: case 10: case 12: case 17: case 18: case 20: case 33: case 34: case 36: case 65: case 66:
            return true;
    }
    return false;
}
}  // namespace

bool set_conv_tile_override(int jn, int pw, int ksw) {
    if (jn == 0 && pw == 0 && ksw == 0) {
        g_tile_override.store(0);
        return true;
    }
    const ConvTile t{jn, pw, ksw != 0};
    if (!tile_instantiated(t)) return false;
    g_tile_override.store(jn * 100 + pw * 10 + (ksw ? 1 : 0) + 1);
    return true;
}

// Tile choice.  A block is 4 waves x pw 16-position subtiles by jn
// 16-channel subtiles and walks a run of such tiles with its weights resident
// in LDS.  Cover all output channels (up to 128) so activations are read
// once, with as many positions per wave as the registers allow; maps too small
// to give every CU a tile shrink the position tile, then the channel tile, and
// finally let the 4 waves of a block split k (one position subtile per block).
ConvTile choose_conv_tile(int M, int OC, int Kp) {
    const int ov = g_tile_override.load(std::memory_order_relaxed);
    if (ov) return ConvTile{(ov - 1) / 100, ((ov - 1) / 10) % 10, ((ov - 1) % 10) != 0};
    const int ocj = (OC + 15) / 16;
    const int nks = Kp / 64;
    auto tiles = [&](int jn, int pw, bool ksw) {
        return (int64_t)((M + (ksw ? 16 : 64) * pw - 1) / ((ksw ? 16 : 64) * pw)) * ((ocj + jn - 1) / jn);
    };
    const int64_t want = 256;  // one tile per CU at least
    int jn = pow2_at_least(ocj, 8);
    int pw = jn >= 8 ? 2 : (jn >= 4 ? 4 : 4);
    while (pw > 1 && tiles(jn, pw, false) < want) pw >>= 1;
    while (jn > 1 && tiles(jn, pw, false) < want) jn >>= 1;
    if (tiles(jn, pw, false) >= want / 2 || nks < 4) return ConvTile{jn, pw, false};
    // small map: one position subtile per block, k split over the 4 waves
    jn = pow2_at_least(ocj, 8);
    while (jn > 1 && tiles(jn, 1, true) < want) jn >>= 1;
    return ConvTile{jn, 1, true};
}

int enumerate_conv_choices(const ConvParams& p, bool int8, ConvChoice* out, int cap) {
    // a fused 1x1 runs only in the 32x32-MFMA kernel's epilogue
    if (p.fuse_1x1) return p.loader == kLoaderNhwc ? enumerate_m32_choices(p, int8, out, cap) : 0;
    // an upsample copy of the output: the streaming 1x1 kernel only
    if (p.yup || p.xup) return int8 && p.KH == 1 && p.KW == 1 ? enumerate_s1x1_choices(p, int8, out, cap) : 0;
    int n = 0;
    const bool nchw = p.loader == kLoaderNchwF32;
    if (!nchw && p.Kp / 64 <= igemm::kMaxSteps) {
        static const ConvTile tiles[] = {{1, 1, false}, {1, 2, false}, {1, 4, false}, {2, 1, false}, {2, 2, false},
                                         {2, 4, false}, {4, 1, false}, {4, 2, false}, {4, 4, false}, {8, 1, false},
                                         {8, 2, false}, {1, 1, true},  {2, 1, true},  {4, 1, true},  {8, 1, true}};
        const int ocj = (p.OCp + 15) / 16;
        for (const ConvTile& t : tiles) {
            if (n >= cap) break;
            if (t.jn > 1 && t.jn / 2 >= ocj) continue;  // a channel tile past every channel
            if (t.ksw && p.Kp / 64 < 4) continue;
            ConvChoice c;
            c.kind = 1;
            c.jn = t.jn;
            c.pw = t.pw;
            c.ksw = t.ksw ? 1 : 0;
            out[n++] = c;
        }
    }
    if (n < cap && int8 && p.KH == 1 && p.KW == 1) n += enumerate_s1x1_choices(p, int8, out + n, cap - n);
    if (n < cap && nchw && !int8) n += enumerate_stem_choices(p, out + n, cap - n);
    if (n < cap && !nchw) n += enumerate_m32_choices(p, int8, out + n, cap - n);
    if (n < cap && !nchw && !int8) n += enumerate_wide_choices(p, out + n, cap - n);
    if (n < cap) n += enumerate_halo_choices(p, int8, out + n, cap - n);
    return n;
}

hipError_t launch_conv_igemm(const ConvParams& p0, bool int8, hipStream_t stream) {
    const bool nchw = p0.loader == kLoaderNchwF32;
    if ((p0.loader != kLoaderNhwc && !nchw) || p0.OC % 4 || p0.C % 8 || p0.Kp % 64 || p0.OCp % 16)
        return hipErrorInvalidValue;
    if (nchw && (int8 || p0.c_real < 1 || p0.c_real > 4 || p0.x_nstride != (int64_t)p0.c_real * p0.H * p0.W))
        return hipErrorInvalidValue;
    const ConvTile t = p0.choice.kind == 1 ? ConvTile{p0.choice.jn, p0.choice.pw, p0.choice.ksw != 0}
                                           : choose_conv_tile(p0.M, p0.OC, p0.Kp);
    if (p0.choice.kind == 1 && !tile_instantiated(t)) return hipErrorInvalidValue;
    const bool out_f32 = (p0.flags & kConvOutF32) != 0;
    const int HWi = p0.H * p0.W, HWo = p0.OH * p0.OW;
    // Images per launch: every view a launch touches must stay inside
    // kMaxViewBytes so the kernel can address it with 32-bit offsets.
    const uint64_t x_img = nchw ? (uint64_t)p0.x_nstride * 4
                                : std::max((uint64_t)p0.x_nstride * 2, (uint64_t)HWi * p0.x_cstride * 2);
    const uint64_t per_img = std::max({x_img, (uint64_t)p0.y_nstride * (out_f32 ? 4 : 2),
                                       p0.res ? (uint64_t)p0.r_nstride * 2 : 0,
                                       p0.acc_out ? (uint64_t)HWo * p0.OC * 4 : 0,
                                       p0.fuse_1x1 ? (uint64_t)p0.fuse_1x1->y_nstride *
                                                         ((p0.fuse_1x1->flags & kConvOutF32) ? 4 : 2)
                                                   : 0,
                                       p0.yup ? (uint64_t)p0.yup_nstride * 2 : 0,
                                       p0.xup ? (uint64_t)p0.xup_nstride * 2 : 0});
    if ((uint64_t)p0.OCp * p0.Kp * 2 > kMaxViewBytes || per_img == 0) return hipErrorInvalidValue;
    const int per_launch = (int)std::min<uint64_t>((uint64_t)p0.N, kMaxViewBytes / per_img);
    if (per_launch < 1) return hipErrorInvalidValue;
    const int nks = p0.Kp / 64;
    if (nks > igemm::kMaxSteps) return hipErrorInvalidValue;
    if (int8 && (p0.x_slots.p == nullptr ||
                 (int64_t)p0.x_slots.stripes * p0.x_nslots > igemm::kMaxSlotReads))
        return hipErrorInvalidValue;
    const bool mc = nks > igemm::chunk_steps_of(int8, t.jn, t.ksw);
    const int f = p0.flags & (kConvSilu | kConvResidual | kConvOutF32);
    // the int32 accumulator output (acc_out) is written by the run-time
    // flag variant only
    const int epi = p0.acc_out ? igemm::kEpiAny
                    : f == kConvSilu ? igemm::kEpiSilu
                    : (int8 && f == (kConvSilu | kConvResidual) ? igemm::kEpiSiluRes : igemm::kEpiAny);
    if (p0.fuse_1x1 && (p0.choice.kind != 5 || int8)) return hipErrorInvalidValue;
    // the upsample copy: a streaming 1x1 choice (measured, or forced)
    ConvChoice forced_up;
    if ((p0.yup || p0.xup) &&
        !(int8 && (p0.choice.kind == 6 || (p0.choice.kind == 0 && forced_s1x1_choice(forced_up)))))
        return hipErrorInvalidValue;
    for (int nb = 0; nb < p0.N; nb += per_launch) {
        ConvParams p = p0;
        ConvParams f2;  // the fused 1x1 on this slice of the batch
        if (p0.fuse_1x1) {
            f2 = *p0.fuse_1x1;
            f2.N = std::min(per_launch, p0.N - nb);
            f2.M = f2.N * HWo;
            const int esz2 = (f2.flags & kConvOutF32) ? 4 : 2;
            f2.y = static_cast<char*>(f2.y) + (int64_t)nb * f2.y_nstride * esz2;
            f2.y_bytes = (uint32_t)view_span(f2.N, f2.y_nstride, f2.y_cstride, HWo, f2.OC, esz2);
            if ((uint64_t)f2.OCp * f2.Kp * 2 > kMaxViewBytes || (uint64_t)f2.y_nstride * esz2 > kMaxViewBytes)
                return hipErrorInvalidValue;
            p.fuse_1x1 = &f2;
        }
        p.N = std::min(per_launch, p0.N - nb);
        p.M = p.N * HWo;
        p.x = nchw ? static_cast<const void*>(static_cast<const float*>(p0.x) + (int64_t)nb * p0.x_nstride)
                   : static_cast<const void*>(static_cast<const __half*>(p0.x) + (int64_t)nb * p0.x_nstride);
        p.y = static_cast<char*>(p0.y) + (int64_t)nb * p0.y_nstride * (out_f32 ? 4 : 2);
        if (p0.res) p.res = p0.res + (int64_t)nb * p0.r_nstride;
        if (p0.acc_out) p.acc_out = p0.acc_out + (int64_t)nb * HWo * p0.OC;
        if (p0.yup) {
            p.yup = static_cast<__half*>(p0.yup) + (int64_t)nb * p0.yup_nstride;
            p.yup_bytes = (uint32_t)view_span(p.N, p.yup_nstride, p.yup_cstride, 4 * HWo, p.OC, 2);
        }
        if (p0.xup) {
            p.xup = static_cast<const __half*>(p0.xup) + (int64_t)nb * p0.xup_nstride;
            p.xup_bytes = (uint32_t)view_span(p.N, p.xup_nstride, p.xup_cstride, HWi / 4, p.xup_cn, 2);
        }
        p.x_bytes = nchw ? (uint32_t)((uint64_t)p.N * p.x_nstride * 4)
                         : (uint32_t)view_span(p.N, p.x_nstride, p.x_cstride, HWi, p.C, 2);
        p.y_bytes = (uint32_t)view_span(p.N, p.y_nstride, p.y_cstride, HWo, p.OC, out_f32 ? 4 : 2);
        p.r_bytes = p.res ? (uint32_t)view_span(p.N, p.r_nstride, p.r_cstride, HWo, p.OC, 2) : 0u;
        p.ntn = (p.OCp / 16 + t.jn - 1) / t.jn;
        const int mtile = (t.ksw ? 16 : 64) * t.pw;
        p.npt = (p.M + mtile - 1) / mtile;
        p.fd_ntn = make_fastdiv((uint32_t)p.ntn);
        if (int8) {
            p.x_slot_bytes = ((p.x_slots.stripes - 1) * p.x_slots.stride + (uint32_t)p.x_nslots) * 4u;
            p.fd_ns = make_fastdiv((uint32_t)std::max(p.x_nslots, 1));
        }
        p.lin = 0;
        if (p.M < (1 << 24)) {
            if (!nchw && p.KH == 1 && p.KW == 1 && p.S == 1 && p.P == 0 && p.x_nstride == (int64_t)HWi * p.x_cstride &&
                p.x_cstride < (1 << 24))
                p.lin |= kLinX;
            if (p.y_nstride == (int64_t)HWo * p.y_cstride && p.y_cstride < (1 << 24) &&
                (!p.res || (p.r_nstride == (int64_t)HWo * p.r_cstride && p.r_cstride < (1 << 24))))
                p.lin |= kLinY;
        }
        p.fd_ohw = make_fastdiv((uint32_t)HWo);
        p.fd_ow = make_fastdiv((uint32_t)p.OW);
        p.fd_c = make_fastdiv((uint32_t)p.C);
        p.fd_kw = make_fastdiv((uint32_t)p.KW);
        hipError_t e = hipErrorNotSupported;
        if (p.choice.kind == 0 && int8 && p.KH == 1 && p.KW == 1) {
            ConvChoice forced;
            if (forced_s1x1_choice(forced)) {
                p.choice = forced;  // a forced tile that does not fit is an error
                e = launch_conv_s1x1(p, int8, epi, stream);
                if (e != hipSuccess) return e;
                continue;
            }
        }
        if (p.choice.kind == 6) {
            e = launch_conv_s1x1(p, int8, epi, stream);
            if (e != hipSuccess) return e;
            continue;
        }
        if (p.choice.kind == 0 && !nchw) {
            ConvChoice forced;
            if (forced_m32_choice(forced) && p.KH == 3 && p.KW == 3) {
                p.choice = forced;  // a forced tile that does not fit is an error
                e = launch_conv_m32(p, int8, epi, stream);
                if (e != hipSuccess) return e;
                continue;
            }
        }
        if (p.choice.kind == 5) {
            e = launch_conv_m32(p, int8, epi, stream);
            if (e != hipSuccess) return e;
            continue;
        }
        if (p.choice.kind == 0 && !int8 && !nchw) {
            ConvChoice forced;
            if (forced_wide_choice(forced)) {
                p.choice = forced;  // a forced wide tile that does not fit is an error
                e = launch_conv_wide(p, epi, stream);
                if (e != hipSuccess) return e;
                continue;
            }
        }
        if (p.choice.kind == 4) {
            e = launch_conv_wide(p, epi, stream);
            if (e != hipSuccess) return e;
            continue;
        }
        if (nchw && !int8 && (p.choice.kind == 0 || p.choice.kind == 3)) e = launch_conv_stem(p, stream);
        if (e == hipErrorNotSupported && p.choice.kind != 1 && p.choice.kind != 3)
            e = launch_conv_halo(p, int8, epi, stream);
        if (e == hipErrorNotSupported && !nchw && p.choice.kind != 2) e = launch_variant(int8, mc, epi, p, t, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace aexrt
