// Host side of the bottleneck-pair kernel (conv_pair.h): shape checks, band
// geometry and LDS layout, the residency check of the grid barrier, launch.
// Kernel instances: conv_pair_i8.hip and conv_pair_f16.hip.
#include <algorithm>
#include <cstdio>

#include "conv_pair.h"

namespace aexrt {

namespace pair {
template <bool INT8>
hipError_t pair_launch_family(const PairParams& h, int nq, int mq, int lds, hipStream_t s);
template <bool INT8>
int pair_resident_blocks(int nq, int mq, int lds);
extern template hipError_t pair_launch_family<true>(const PairParams&, int, int, int, hipStream_t);
extern template hipError_t pair_launch_family<false>(const PairParams&, int, int, int, hipStream_t);
extern template int pair_resident_blocks<true>(int, int, int);
extern template int pair_resident_blocks<false>(int, int, int);
}  // namespace pair

namespace {

constexpr int kPairLdsBudget = 152 * 1024;  // dynamic LDS of one block (the static arrays take ~2.5 KB)

bool conv3x3_same(const ConvParams& p) {
    return p.KH == 3 && p.KW == 3 && p.S == 1 && p.P == 1 && p.OH == p.H && p.OW == p.W && p.loader == kLoaderNhwc &&
           p.fuse_1x1 == nullptr;
}

}  // namespace

const char* pair_shape_error(const ConvParams& a, const ConvParams& b, bool int8) {
    if (!conv3x3_same(a) || !conv3x3_same(b))
        return "pair: two 3x3 stride-1 pad-1 convs of one map size, NHWC";
    const int C = a.C;
    if (a.OC != C || b.C != C || b.OC != C || b.N != a.N || b.H != a.H || b.W != a.W)
        return "pair: both convs C -> C channels over one map";
    if (C % 32 || C > 128) return "pair: C a multiple of 32, at most 128";
    if (a.flags != kConvSilu || (b.flags != kConvSilu && b.flags != (kConvSilu | kConvResidual)))
        return "pair: SiLU on both convs, an optional residual on the second, fp16 output";
    if ((b.flags & kConvResidual) && !b.res) return "pair: residual flag without a residual view";
    if (a.res || a.acc_out) return "pair: the first conv takes no residual (its sums: the acc_a argument)";
    if (b.acc_out && !int8) return "pair: accumulator output with int8 only";
    if (a.x_cstride % 8 || b.y_cstride % 4 || (b.res && b.r_cstride % 4)) return "pair: view strides";
    if (int8 && !a.x_slots.p) return "pair: int8 needs the input's amax slots";
    if ((uint64_t)a.OCp * a.Kp * 2 > kMaxViewBytes || (uint64_t)b.OCp * b.Kp * 2 > kMaxViewBytes)
        return "pair: weights too large";
    return nullptr;
}

namespace {

// Band geometry for tr output rows: kernel parameters (views per image,
// chunk counts, LDS layout), the dynamic LDS bytes and the position subtiles
// per wave; false when the band does not fit the kernel.
bool pair_geometry(const ConvParams& a, const ConvParams& b, bool int8, int tr, PairParams& h, int& lds, int& nq,
                   int& mq) {
    if (pair_shape_error(a, b, int8) || tr < 1) return false;
    const int C = a.C, H = a.H, W = a.W;
    tr = std::min(tr, H);
    nq = C / 32;
    const int ra = std::min(tr + 2, H);  // rows of conv a for the largest band
    const int need = std::max(ra, tr) * W;
    mq = need <= 128 ? 1 : need <= 256 ? 2 : need <= 512 ? 4 : 0;
    if (!mq || nq * mq > 4) return false;
    const int mw = W + 2;
    const int xnpix = (ra + 2) * mw, gnpix = (tr + 2) * mw;
    const int cpp = int8 ? 16 : 8;
    if ((C / cpp) * xnpix > pair::kNT * pair_max_pieces(int8)) return false;
    const int ksub = int8 ? 32 : 16;
    const int ks = 9 * C / ksub;
    if (ks > kPairMaxSteps) return false;
    const int64_t xb = ((int64_t)C * (int8 ? 1 : 2) * xnpix + 15) / 16 * 16;
    const int64_t gb = (int64_t)C * 2 * gnpix;
    const int64_t ring = (int64_t)pair::kD * pair::kKC * 2 * C * 16;
    if (ring + xb + gb > kPairLdsBudget) return false;
    h = PairParams{};
    h.a = a;
    h.b = b;
    h.TR = tr;
    h.nband = (H + tr - 1) / tr;
    const int64_t ntile = (int64_t)a.N * h.nband;
    if (ntile > INT32_MAX / 2) return false;
    h.ntile = (int)ntile;
    h.ka = h.kb = ks;
    h.nchunk_a = (ks + pair::kKC - 1) / pair::kKC;
    h.nchunk = 2 * h.nchunk_a;
    h.x_off = (int)ring;
    h.g_off = (int)(ring + xb);
    lds = (int)(ring + xb + gb);
    const int esz = 2;
    const uint64_t x_img = ((uint64_t)(H * W - 1) * a.x_cstride + C) * 2;
    const uint64_t y_img = ((uint64_t)(H * W - 1) * b.y_cstride + C) * esz;
    const uint64_t r_img = b.res ? ((uint64_t)(H * W - 1) * b.r_cstride + C) * 2 : 0;
    const uint64_t dense = (uint64_t)a.N * H * W * C * 4;  // the accumulator outputs
    if (x_img > kMaxViewBytes || y_img > kMaxViewBytes || r_img > kMaxViewBytes || dense > kMaxViewBytes)
        return false;
    h.x_img = (uint32_t)x_img;
    h.y_img = (uint32_t)y_img;
    h.r_img = (uint32_t)r_img;
    h.fd_nband = make_fastdiv((uint32_t)h.nband);
    if (int8) {
        h.a.x_slot_bytes = ((h.a.x_slots.stripes - 1) * h.a.x_slots.stride + (uint32_t)h.a.x_nslots) * 4u;
        h.a.fd_ns = make_fastdiv((uint32_t)std::max(h.a.x_nslots, 1));
        if ((int64_t)h.a.x_slots.stripes * h.a.x_nslots > igemm::kMaxSlotReads) return false;
    }
    return true;
}

}  // namespace

int enumerate_pair_bands(const ConvParams& a, const ConvParams& b, bool int8, int* out, int cap) {
    int n = 0;
    int last = -1;
    for (int parts = 1; parts <= a.H && n < cap; ++parts) {
        const int tr = (a.H + parts - 1) / parts;
        if (tr == last) continue;
        last = tr;
        PairParams h{};
        int lds = 0, nq = 0, mq = 0;
        if (!pair_geometry(a, b, int8, tr, h, lds, nq, mq)) continue;
        if (int8 && h.ntile > pair::pair_resident_blocks<true>(nq, mq, lds)) continue;
        if (h.nband > 64) break;
        out[n++] = tr;
    }
    return n;
}

hipError_t launch_conv_pair(const ConvParams& a, const ConvParams& b, bool int8, int tr, uint32_t* sync,
                            uint32_t* err, __half* t_out, int32_t* acc_a, hipStream_t stream) {
    if (tr <= 0) {
        int bands[16];
        const int nb = enumerate_pair_bands(a, b, int8, bands, 16);
        if (nb == 0) return hipErrorInvalidValue;
        // the band count that first gives every image's bands a quarter of the GPU, else the most
        tr = bands[nb - 1];
        for (int i = 0; i < nb; ++i)
            if ((int64_t)a.N * ((a.H + bands[i] - 1) / bands[i]) >= 64) {
                tr = bands[i];
                break;
            }
    }
    PairParams h{};
    int lds = 0, nq = 0, mq = 0;
    if (!pair_geometry(a, b, int8, tr, h, lds, nq, mq)) return hipErrorInvalidValue;
    if (int8 && (!sync || !err)) return hipErrorInvalidValue;
    if (!int8 && acc_a) return hipErrorInvalidValue;
    h.sync = sync;
    h.err = err;
    h.t_out = t_out;
    h.acc_a = acc_a;
    if (LaunchProbe* pr = launch_probe()) {
        std::snprintf(pr->name, sizeof(pr->name), "conv_pair_kernel<%s,%d,%d> %dx%d", int8 ? "true" : "false", nq, mq,
                      h.TR, a.W);
        return hipSuccess;
    }
    // every block of an int8 pair waits for all the others at the barrier:
    // the whole grid must be resident at once
    if (int8 && h.ntile > pair::pair_resident_blocks<true>(nq, mq, lds)) return hipErrorInvalidConfiguration;
    return int8 ? pair::pair_launch_family<true>(h, nq, mq, lds, stream)
                : pair::pair_launch_family<false>(h, nq, mq, lds, stream);
}

}  // namespace aexrt
