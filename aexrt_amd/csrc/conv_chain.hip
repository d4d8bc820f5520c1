// Host side of the detect-head chain kernel (conv_chain.h): shape checks,
// tile geometry, LDS layout, launch.
#include <algorithm>
#include <cstdio>

#include "conv_chain.h"

namespace aexrt {

namespace {

constexpr int kChainLdsBudget = 156 * 1024;  // dynamic LDS of one block (the static arrays take ~4 KB)

int chain_nq(const ConvParams& a, const ConvParams& b, const ConvParams& c) {
    const int oc = std::max({a.OC, b.OC, c.OC});
    return oc <= 64 ? 2 : oc <= 96 ? 3 : 0;
}

bool dense_fp16(const ConvParams& p) { return p.loader == kLoaderNhwc && p.x_cstride % 8 == 0; }

}  // namespace

// a: fp16 3x3 s1 p1 SiLU; b: the same over a's output; c: 1x1 s1 over b's
// output; every channel count <= 96, the 3x3 inputs in 16-channel steps.
const char* chain_shape_error(const ConvParams& a, const ConvParams& b, const ConvParams& c) {
    auto conv3 = [](const ConvParams& p) {
        return p.KH == 3 && p.KW == 3 && p.S == 1 && p.P == 1 && p.OH == p.H && p.OW == p.W && p.C % 16 == 0 &&
               p.flags == kConvSilu && p.res == nullptr && p.acc_out == nullptr;
    };
    if (!dense_fp16(a) || !conv3(a) || !conv3(b) || b.C != a.OC || b.N != a.N || b.H != a.H || b.W != a.W)
        return "chain: two fp16 3x3 stride-1 SiLU convs, the second over the first's output";
    if (c.KH != 1 || c.KW != 1 || c.S != 1 || c.P != 0 || c.C != b.OC || c.N != a.N || c.H != a.H || c.W != a.W ||
        (c.flags & ~(kConvSilu | kConvOutF32)) || c.res != nullptr || c.y_slots.p != nullptr || c.OC % 4)
        return "chain: a 1x1 stride-1 conv over the second conv's output (flags SILU, OUT_F32; no amax slots)";
    const int nq = chain_nq(a, b, c);
    if (!nq || c.Kp < nq * 32 || 9 * a.C / 16 > kChainMaxSteps || 9 * b.C / 16 > kChainMaxSteps)
        return "chain: at most 96 channels per conv and 9 * in_channels / 16 <= 160 k steps";
    return nullptr;
}

namespace {

// Largest extent of conv a's region (the tile plus a border of one, inside
// the map) over the tiles of a map of n positions cut into tiles of t.
int region_extent(int n, int t) {
    int m = 0;
    for (int o = 0; o < n; o += t) m = std::max(m, std::min(o + t + 1, n) - std::max(o - 1, 0));
    return m;
}

// LDS bytes of one block for tile (tr, tc): weight ring, largest window X,
// largest grid G; 0 when a region exceeds 256 positions or LDS.
int chain_lds(const ConvParams& a, int nq, int tr, int tc, int* x_bytes) {
    tr = std::min(tr, a.H);
    tc = std::min(tc, a.W);
    const int r1h = region_extent(a.H, tr), r1w = region_extent(a.W, tc);
    if (r1h * r1w > 256 || tr * tc > 256) return 0;
    const int64_t xp = (int64_t)(a.C / 8) * (r1h + 2) * (r1w + 2);
    const int64_t xb = (xp + 63) / 64 * 64 * 16;
    const int64_t gb = (int64_t)nq * 4 * (tr + 2) * (tc + 2) * 16;
    const int64_t ring = (int64_t)chain::kD * chain::kKC * 2 * nq * 32 * 16;
    const int64_t total = ring + xb + gb;
    if (total > kChainLdsBudget) return 0;
    if (x_bytes) *x_bytes = (int)xb;
    return (int)total;
}

}  // namespace

// Tile of the chain: the given one when it fits, else the largest of a few
// shapes (whole map, half rows, quarters, 8x8) that fits.
bool chain_tile(const ConvParams& a, const ConvParams& b, const ConvParams& c, int& tr, int& tc) {
    const int nq = chain_nq(a, b, c);
    if (!nq) return false;
    if (tr > 0 && tc > 0) return chain_lds(a, nq, tr, tc, nullptr) > 0;
    const int cand[][2] = {{a.H, a.W}, {(a.H + 1) / 2, a.W}, {(a.H + 1) / 2, (a.W + 1) / 2}, {8, 8}, {6, 8}, {4, 8}};
    for (const auto& t : cand)
        if (chain_lds(a, nq, t[0], t[1], nullptr) > 0) {
            tr = std::min(t[0], a.H);
            tc = std::min(t[1], a.W);
            return true;
        }
    return false;
}

namespace {

// Kernel parameters of one branch for tile (tr, tc) (fitted); its dynamic LDS
// bytes and position subtiles per wave.  False when it does not fit.
// k groups of the chain blocks: 1.  The two-group blocks (KG = 2) are
// switched off: a process that loaded a YOLOv8n-160 model with them (load-time
// tuning runs the chain on its 10x10 and 5x5 head maps) aborted, and no cause
// has been found; they are not launched until one is.
int chain_kgroups() { return 1; }

bool make_chain_params(const ConvParams& a, const ConvParams& b, const ConvParams& c, int tr, int tc, ChainParams& h,
                       int& lds, int& mq, int& kg) {
    if (chain_shape_error(a, b, c) || !chain_tile(a, b, c, tr, tc)) return false;
    const int nq = chain_nq(a, b, c);
    h = ChainParams{};
    h.a = a;
    h.b = b;
    h.c = c;
    h.TR = std::min(tr, a.H);
    h.TC = std::min(tc, a.W);
    h.ntc = (a.W + h.TC - 1) / h.TC;
    h.tpi = ((a.H + h.TR - 1) / h.TR) * h.ntc;
    const int64_t ntile = (int64_t)a.N * h.tpi;
    if (ntile > INT32_MAX / 2) return false;
    h.ntile = (int)ntile;
    h.ka = 9 * a.C / 16;
    h.kb = 9 * b.C / 16;
    h.nchunk_a = (h.ka + chain::kKC - 1) / chain::kKC;
    h.nchunk = h.nchunk_a + (h.kb + chain::kKC - 1) / chain::kKC;
    int xb = 0;
    lds = chain_lds(a, nq, h.TR, h.TC, &xb);
    if (!lds) return false;
    h.x_off = chain::kD * chain::kKC * 2 * nq * 32 * 16;
    h.g_off = h.x_off + xb;
    // one image's views (the kernel addresses each image from its own base)
    const int esz = (c.flags & kConvOutF32) ? 4 : 2;
    const uint64_t x_img = ((uint64_t)(a.H * a.W - 1) * a.x_cstride + a.C) * 2;
    const uint64_t y_img = ((uint64_t)(c.OH * c.OW - 1) * c.y_cstride + c.OC) * esz;
    if (x_img > kMaxViewBytes || y_img > kMaxViewBytes || (uint64_t)a.OCp * a.Kp * 2 > kMaxViewBytes ||
        (uint64_t)b.OCp * b.Kp * 2 > kMaxViewBytes || (uint64_t)c.OCp * c.Kp * 2 > kMaxViewBytes)
        return false;
    h.x_img = (uint32_t)x_img;
    h.y_img = (uint32_t)y_img;
    h.fd_tpi = make_fastdiv((uint32_t)h.tpi);
    h.fd_ntc = make_fastdiv((uint32_t)h.ntc);
    h.fd_cs16a = make_fastdiv((uint32_t)(a.C / 16));
    h.fd_cs16b = make_fastdiv((uint32_t)(b.C / 16));
    // one position subtile per wave when both regions have at most 128 positions
    mq = region_extent(a.H, h.TR) * region_extent(a.W, h.TC) <= 128 && h.TR * h.TC <= 128 ? 1 : 2;
    // two k groups of 4 waves each: one subtile per wave and a window large
    // enough to pass the partial sums of a 32-channel subtile (4 x 16 x 64 floats)
    kg = chain_kgroups() == 2 && mq == 1 && xb >= 4 * 16 * 64 * 4 ? 2 : 1;
    return true;
}

}  // namespace

hipError_t launch_conv_chain(const ConvParams& a, const ConvParams& b, const ConvParams& c, int tr, int tc,
                             hipStream_t stream) {
    ChainParams h{};
    int lds = 0, mq = 1, kg = 1;
    if (!make_chain_params(a, b, c, tr, tc, h, lds, mq, kg)) return hipErrorInvalidValue;
    const int nq = chain_nq(a, b, c);
    if (LaunchProbe* pr = launch_probe()) {
        std::snprintf(pr->name, sizeof(pr->name), "conv_chain_kernel<%d,%d,%d> %dx%d", nq, mq, kg, h.TR, h.TC);
        return hipSuccess;
    }
    const dim3 grid((unsigned)h.ntile), block(chain::kNT * kg);
#define AEXRT_CHAIN1(Q, M, G)                                                                                      \
    if (nq == Q && mq == M && kg == G) {                                                                           \
        hipLaunchKernelGGL((chain::conv_chain_kernel<Q, M, G>), grid, block, (size_t)lds, stream, h);               \
        return hipGetLastError();                                                                                  \
    }
    AEXRT_CHAIN1(2, 1, 1) AEXRT_CHAIN1(2, 2, 1) AEXRT_CHAIN1(3, 1, 1) AEXRT_CHAIN1(3, 2, 1)
#undef AEXRT_CHAIN1
    return hipErrorInvalidValue;
}

int enumerate_chain_tiles(const ConvParams* br0, const ConvParams* br1, int* tr, int* tc, int cap) {
    const ConvParams& a = br0[0];
    const int H = a.H, W = a.W;
    const int cand[][2] = {{H, W}, {(H + 1) / 2, W}, {(H + 1) / 2, (W + 1) / 2}, {(H + 2) / 3, (W + 2) / 3},
                           {8, 8}, {6, 8}, {5, 5}, {4, 4}, {3, 3}};
    int n = 0;
    for (const auto& t : cand) {
        const int r = std::min(t[0], H), c = std::min(t[1], W);
        if (r < 1 || c < 1) continue;
        bool seen = false;
        for (int k = 0; k < n; ++k) seen = seen || (tr[k] == r && tc[k] == c);
        if (seen || n >= cap) continue;
        ChainParams h0{}, h1{};
        int lds0 = 0, lds1 = 0, mq0 = 1, mq1 = 1, kg0 = 1, kg1 = 1;
        if (!make_chain_params(br0[0], br0[1], br0[2], r, c, h0, lds0, mq0, kg0)) continue;
        if (br1 && (!make_chain_params(br1[0], br1[1], br1[2], r, c, h1, lds1, mq1, kg1) || mq0 != mq1 ||
                    (int64_t)h0.ntile + h1.ntile > INT32_MAX))
            continue;
        tr[n] = r;
        tc[n] = c;
        ++n;
    }
    return n;
}

// Two branches over one input map in one launch, on one tile (the one that
// fits the branch with more channels).
hipError_t launch_conv_chain2(const ConvParams* br0, const ConvParams* br1, int tr, int tc, hipStream_t stream) {
    const ConvParams &a0 = br0[0], &b0 = br0[1], &c0 = br0[2], &a1 = br1[0], &b1 = br1[1], &c1 = br1[2];
    if (a0.x != a1.x || a0.N != a1.N || a0.H != a1.H || a0.W != a1.W || a0.C != a1.C) return hipErrorInvalidValue;
    const int nq0 = chain_nq(a0, b0, c0), nq1 = chain_nq(a1, b1, c1);
    if (!nq0 || !nq1) return hipErrorInvalidValue;
    if (tr <= 0 || tc <= 0) {
        tr = tc = 0;
        const bool big0 = nq0 >= nq1;
        if (!chain_tile(big0 ? a0 : a1, big0 ? b0 : b1, big0 ? c0 : c1, tr, tc)) return hipErrorInvalidValue;
    }
    ChainParams h0{}, h1{};
    int lds0 = 0, lds1 = 0, mq0 = 1, mq1 = 1, kg0 = 1, kg1 = 1;
    if (!make_chain_params(a0, b0, c0, tr, tc, h0, lds0, mq0, kg0) ||
        !make_chain_params(a1, b1, c1, tr, tc, h1, lds1, mq1, kg1) || mq0 != mq1 ||
        (int64_t)h0.ntile + h1.ntile > INT32_MAX)
        return hipErrorInvalidValue;
    const int kg = std::min(kg0, kg1);
    if (LaunchProbe* pr = launch_probe()) {
        std::snprintf(pr->name, sizeof(pr->name), "conv_chain2_kernel<%d,%d,%d,%d> %dx%d", nq0, nq1, mq0, kg, h0.TR,
                      h0.TC);
        return hipSuccess;
    }
    const dim3 grid((unsigned)(h0.ntile + h1.ntile)), block(chain::kNT * kg);
    const size_t lds = (size_t)std::max(lds0, lds1);
#define AEXRT_CHAIN2(Q0, Q1, M, G)                                                                                 \
    if (nq0 == Q0 && nq1 == Q1 && mq0 == M && kg == G) {                                                           \
        hipLaunchKernelGGL((chain::conv_chain2_kernel<Q0, Q1, M, G>), grid, block, lds, stream, h0, h1);          \
        return hipGetLastError();                                                                                  \
    }
    AEXRT_CHAIN2(2, 3, 1, 1) AEXRT_CHAIN2(3, 2, 1, 1) AEXRT_CHAIN2(2, 2, 1, 1) AEXRT_CHAIN2(3, 3, 1, 1)
    AEXRT_CHAIN2(2, 3, 2, 1) AEXRT_CHAIN2(3, 2, 2, 1) AEXRT_CHAIN2(2, 2, 2, 1) AEXRT_CHAIN2(3, 3, 2, 1)
#undef AEXRT_CHAIN2
    return hipErrorInvalidValue;
}

}  // namespace aexrt
