// Host side of the streaming 1x1 int8 conv (kernel in conv_s1x1.h): geometry,
// the forced tile, launch.
#include <algorithm>
#include <atomic>
#include <cstdio>

#include "conv_s1x1.h"

namespace aexrt {

namespace s1x1 {
AEXRT_S1X1_EXTERN(0)
AEXRT_S1X1_EXTERN(1)
}  // namespace s1x1

namespace {

// dynamic LDS of one block (its static arrays aside)
constexpr int kS1x1LdsBudget = 152 * 1024;

struct S1x1Tile {
    int jq, pq, np;
};

// int8 1x1 stride-1 convs on views whose positions are evenly strided, with
// the SiLU or run-time-flag epilogue and no residual.
// An upsample copy (yup) takes an fp16 output and a view of 4x the
// positions with 8-byte aligned channel groups; an upsampled input source
// (xup) whole 16-channel pieces of the input, an even map and the source's
// slots, and not both at once.
bool s1x1_shape_ok(const ConvParams& p, bool int8) {
    const bool up_ok = !p.yup || (!(p.flags & kConvOutF32) && p.yup_cstride % 4 == 0 && p.yup_cstride >= p.OC &&
                                  p.yup_nstride >= (int64_t)4 * p.OH * p.OW * p.yup_cstride);
    const bool xup_ok =
        !p.xup || (!p.yup && p.H % 2 == 0 && p.W % 2 == 0 && p.xup_c0 % 16 == 0 && p.xup_cn % 16 == 0 &&
                   p.xup_cn > 0 && p.xup_c0 + p.xup_cn <= p.C && p.xup_cstride % 8 == 0 && p.xup_cstride >= p.xup_cn &&
                   p.xup_nstride >= (int64_t)(p.H / 2) * (p.W / 2) * p.xup_cstride && p.xup_slots.p &&
                   p.xup_nslots == p.xup_cn / 16 &&
                   (int64_t)p.xup_slots.stripes * p.xup_nslots <= igemm::kMaxUpSlotReads);
    return int8 && p.loader == kLoaderNhwc && p.KH == 1 && p.KW == 1 && p.S == 1 && p.P == 0 && p.OH == p.H &&
           p.OW == p.W && p.C % 16 == 0 && p.x_cstride % 8 == 0 && (p.lin & kLinX) && (p.lin & kLinY) &&
           !(p.flags & kConvResidual) && p.res == nullptr && p.fuse_1x1 == nullptr && p.M < (1 << 24) && up_ok &&
           xup_ok;
}

bool s1x1_instantiated(int jq, int pq, int np, bool up) {
    if (jq != 1 && jq != 2 && jq != 4 && jq != 8) return false;
    if (np != 1 && np != 2 && np != 4 && np != 8) return false;
    if (pq == 1) return true;
    return !up && pq == 2 && jq <= 4 && np <= 4;
}

// Fills the geometry of tile (jq, pq) into h and the piece count into t.np;
// false when it does not fit a kernel instance or the LDS.
bool s1x1_geometry(S1x1Params& h, S1x1Tile& t) {
    const ConvParams& p = h.c;
    h.TP = 64 * t.pq;
    h.nks = p.Kp / 64;
    h.c16 = p.C / 16;
    h.npiece = h.TP * h.c16;
    const int need = (h.npiece + 255) / 256;
    t.np = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : need <= 8 ? 8 : 0;
    if (!t.np || !s1x1_instantiated(t.jq, t.pq, t.np, p.yup != nullptr || p.xup != nullptr)) return false;
    const int64_t ntile = ((int64_t)p.M + h.TP - 1) / h.TP;
    if (ntile > INT32_MAX / 2) return false;
    h.ntile = (int)ntile;
    const int ocb = 16 * t.jq;
    h.wbytes = h.nks * ocb * 64;
    h.tbytes = h.nks * h.TP * 64;
    if ((int64_t)h.wbytes + 2 * h.tbytes > kS1x1LdsBudget) return false;
    h.c.ntn = (p.OCp + ocb - 1) / ocb;
    h.c.fd_ntn = make_fastdiv((uint32_t)h.c.ntn);
    h.fd_c16 = make_fastdiv((uint32_t)h.c16);
    h.fd_hw = make_fastdiv((uint32_t)(p.OH * p.OW));
    h.fd_w = make_fastdiv((uint32_t)p.OW);
    if (p.xup) {
        h.fd_uns = make_fastdiv((uint32_t)std::max(p.xup_nslots, 1));
        h.xup_slot_bytes = ((p.xup_slots.stripes - 1) * p.xup_slots.stride + (uint32_t)p.xup_nslots) * 4u;
    }
    return true;
}

std::atomic<int> g_s1x1_force{0};  // jq | pq << 8 | one-tile-per-block << 16, 0 = off

hipError_t s1x1_launch(const S1x1Params& h, int epi, const S1x1Tile& t, hipStream_t s) {
    const bool up = h.c.yup != nullptr, xup = h.c.xup != nullptr;
    if (LaunchProbe* pr = launch_probe()) {
        std::snprintf(pr->name, sizeof(pr->name), "conv1x1_stream_kernel<%d,%d,%d,%d%s>%s", t.jq, t.pq, t.np, epi,
                      up ? ",true" : xup ? ",false,true" : "", h.one ? " one tile per block" : "");
        return hipSuccess;
    }
    if (epi == igemm::kEpiSilu) return s1x1::s1x1_launch_family<igemm::kEpiSilu>(h, t.jq, t.pq, t.np, up, xup, s);
    if (epi == igemm::kEpiAny) return s1x1::s1x1_launch_family<igemm::kEpiAny>(h, t.jq, t.pq, t.np, up, xup, s);
    return hipErrorInvalidValue;
}

}  // namespace

bool set_conv1x1_stream(int mode, int jq, int pq) {
    if (!mode) {
        g_s1x1_force.store(0);
        return true;
    }
    if ((mode != 1 && mode != 2) || !s1x1_instantiated(jq, pq, 1, false)) return false;
    g_s1x1_force.store(jq | (pq << 8) | (mode == 2 ? 1 << 16 : 0));
    return true;
}

bool forced_s1x1_choice(ConvChoice& c) {
    const int f = g_s1x1_force.load(std::memory_order_relaxed);
    if (!f) return false;
    c = ConvChoice{};
    c.kind = 6;
    c.jn = f & 0xFF;
    c.pw = (f >> 8) & 0xFF;
    c.ksw = (f >> 16) & 1;  // one tile per block
    return true;
}

int enumerate_s1x1_choices(const ConvParams& p, bool int8, ConvChoice* out, int cap) {
    // the launcher sets p.lin per batch slice; the strides decide it
    ConvParams q = p;
    q.lin = 0;
    if (p.KH == 1 && p.KW == 1 && p.S == 1 && p.P == 0 && p.M < (1 << 24) &&
        p.x_nstride == (int64_t)p.H * p.W * p.x_cstride && p.x_cstride < (1 << 24) &&
        p.y_nstride == (int64_t)p.OH * p.OW * p.y_cstride && p.y_cstride < (1 << 24))
        q.lin = kLinX | kLinY;
    if (!s1x1_shape_ok(q, int8)) return 0;
    const int ocj = (p.OCp + 15) / 16;
    int n = 0;
    for (int pq : {1, 2}) {
        if (pq > 1 && (p.yup || p.xup)) break;  // the upsample variants run on one-subtile tiles
        for (int jq : {1, 2, 4, 8}) {
            if (n >= cap) return n;
            if (jq > 1 && jq / 2 >= ocj) continue;  // a channel tile past every channel
            S1x1Params h{};
            h.c = q;
            S1x1Tile t{jq, pq, 0};
            if (!s1x1_geometry(h, t)) continue;
            ConvChoice c;
            c.kind = 6;
            c.jn = jq;
            c.pw = pq;
            out[n++] = c;
            // the same tile on a grid of one tile per block: the hardware refills
            // the CUs as blocks end, so loads and stores of different blocks
            // interleave instead of all blocks' phases lining up
            if (n < cap && (int64_t)h.ntile * h.c.ntn > 256) {
                c.ksw = 1;
                out[n++] = c;
            }
        }
    }
    return n;
}

// One batch slice of a conv with a kind-6 choice (views already inside
// 32-bit spans, p.lin set).  A choice that does not fit the conv is an error.
hipError_t launch_conv_s1x1(const ConvParams& p, bool int8, int epi, hipStream_t stream) {
    if (!s1x1_shape_ok(p, int8) || p.choice.kind != 6) return hipErrorInvalidValue;
    if (int8 && (p.x_slots.p == nullptr || (int64_t)p.x_slots.stripes * p.x_nslots > igemm::kMaxSlotReads))
        return hipErrorInvalidValue;
    S1x1Params h{};
    h.c = p;
    S1x1Tile t{p.choice.jn, p.choice.pw, 0};
    if (!s1x1_geometry(h, t)) return hipErrorInvalidValue;
    h.one = p.choice.ksw ? 1 : 0;
    if (p.xup) {
        // one buffer resource over the input view and the source: 32-bit offsets from the lower
        const uintptr_t xa = reinterpret_cast<uintptr_t>(p.x), ua = reinterpret_cast<uintptr_t>(p.xup);
        const uintptr_t lo = std::min(xa, ua), hi = std::max(xa + p.x_bytes, ua + p.xup_bytes);
        if (hi - lo > 0xFFFFFFF0ull) return hipErrorInvalidValue;
        h.xbase = reinterpret_cast<const void*>(lo);
        h.xspan = (uint32_t)(hi - lo);
        h.x_off0 = (uint32_t)(xa - lo);
        h.xup_off0 = (uint32_t)(ua - lo);
    }
    return s1x1_launch(h, epi, t, stream);
}

}  // namespace aexrt
