// fp32 direct convolution on NCHW tensors: the reference's fp32 conv entry
// points (aexrt_d3d12_conv2d_float32 / _silu_float32, native/aexrt.h:175-189,
// shader RT:1554-1622) and its CPU path cpu_conv2d (RT:20552-20580).
//
// Each output is acc = bias[oc], then += x * w over (input channel of the
// group, ky, kx) in that order, skipping taps outside the input, with every
// multiply and add rounded on its own (no fused multiply-add): the exact
// arithmetic of the reference's CPU loop.  SiLU is acc / (1 + e^-acc).
//
// A block covers 256 consecutive output positions of one image and KOC
// output channels: input reads are coalesced along the row, the weights of
// the block's channels are the same for every lane (scalar loads), and each
// input value loaded serves the KOC channels.
// Built with -ffp-contract=off (Makefile).
#include "common.h"
#include "kernels.h"

namespace aexrt {

namespace {

constexpr int kF32Threads = 256;
constexpr int kKoc = 4;

__global__ __launch_bounds__(kF32Threads) void conv_f32_kernel(F32ConvParams p) {
    const int64_t ohw = (int64_t)p.OH * p.OW;
    const int64_t pos = (int64_t)blockIdx.x * kF32Threads + threadIdx.x;
    const int noc = (p.OC + kKoc - 1) / kKoc;
    const int n = blockIdx.y / noc;
    const int oc0 = (blockIdx.y - n * noc) * kKoc;
    if (pos >= ohw) return;
    const int oh = (int)(pos / p.OW), ow = (int)(pos - (int64_t)(pos / p.OW) * p.OW);
    const int ocpg = p.OC / p.G, icpg = p.C / p.G;
    float acc[kKoc];
#pragma unroll
    for (int j = 0; j < kKoc; ++j) acc[j] = oc0 + j < p.OC ? p.bias[oc0 + j] : 0.0f;
    // all kKoc channels of the tile in one group (group size a multiple of
    // kKoc): each input value serves all of them; otherwise channel by channel
    const bool shared = ocpg % kKoc == 0;
#pragma unroll
    for (int jo = 0; jo < kKoc; ++jo) {
        if (shared && jo > 0) break;
        if (oc0 + jo >= p.OC) break;
        const int gid = (oc0 + jo) / ocpg;
        for (int icg = 0; icg < icpg; ++icg) {
            const int ic = gid * icpg + icg;
            const float* xc = p.x + ((int64_t)n * p.C + ic) * p.H * p.W;
            for (int ky = 0; ky < p.KH; ++ky) {
                const int iy = oh * p.SH + ky * p.DH - p.PT;
                if (iy < 0 || iy >= p.H) continue;
                for (int kx = 0; kx < p.KW; ++kx) {
                    const int ix = ow * p.SW + kx * p.DW - p.PL;
                    if (ix < 0 || ix >= p.W) continue;
                    const float xv = xc[(int64_t)iy * p.W + ix];
                    const int64_t wk = ((int64_t)icg * p.KH + ky) * p.KW + kx;
                    if (shared) {
#pragma unroll
                        for (int j = 0; j < kKoc; ++j)
                            if (oc0 + j < p.OC)
                                acc[j] = __fadd_rn(acc[j], __fmul_rn(xv, p.w[(int64_t)(oc0 + j) * icpg * p.KH * p.KW + wk]));
                    } else {
                        acc[jo] = __fadd_rn(acc[jo], __fmul_rn(xv, p.w[(int64_t)(oc0 + jo) * icpg * p.KH * p.KW + wk]));
                    }
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kKoc; ++j) {
        const int oc = oc0 + j;
        if (oc >= p.OC) break;
        float v = acc[j];
        if (p.silu) v = __fdiv_rn(v, __fadd_rn(1.0f, expf(-v)));
        p.y[((int64_t)n * p.OC + oc) * ohw + pos] = v;
    }
}

}  // namespace

hipError_t launch_conv_f32(const F32ConvParams& p, hipStream_t stream) {
    if (p.N <= 0 || p.C <= 0 || p.OC <= 0 || p.OH <= 0 || p.OW <= 0 || p.H <= 0 || p.W <= 0 || p.KH <= 0 ||
        p.KW <= 0 || p.SH <= 0 || p.SW <= 0 || p.DH <= 0 || p.DW <= 0 || p.G <= 0 || p.C % p.G || p.OC % p.G)
        return hipErrorInvalidValue;
    const int64_t ohw = (int64_t)p.OH * p.OW;
    const int64_t rows = (int64_t)p.N * ((p.OC + kKoc - 1) / kKoc);
    const int64_t blocks = (ohw + kF32Threads - 1) / kF32Threads;
    if (blocks > 0x7FFFFFFF || rows > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(conv_f32_kernel, dim3((unsigned)blocks, (unsigned)rows), dim3(kF32Threads), 0, stream, p);
    return hipGetLastError();
}

}  // namespace aexrt
