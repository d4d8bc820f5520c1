// Dynamic int8 convolution: the reference's fallback int8 conv
// (native/aexrt_d3d12_runtime.cpp:2952-3115), which quantizes in the kernel
// instead of reading a prequantized tensor.  The reference dispatches it for
// int8 convs whose input tensor has fewer than 4096 elements
// (RT:21478-21479, RT:24260-24317).
//
// Per output position and 4-channel input group g:
//   1x1: amax = max|x| over the 4 channels at the position;
//   3x3: amax = max|x| over the 4 channels at the 9 taps (zero padding
//        included), one scale for the 36 values;
//   s = 127/amax (0 when amax is 0), q = round_half_even(x*s) as a byte,
//   part = sum over the taps of dot4(q, w) in int32,
//   acc += float(part) * (amax/127), in group order, fp32;
// y = acc * w_scale[oc] + bias[oc], SiLU, (+ residual), fp16 or fp32 out.
//
// These convs see at most 4095 input elements, so the kernel is small and
// latency-bound: one block per output position; the block quantizes the
// position's patch once into LDS (C/4 scales, 9 x C/4 packed words) and each
// thread then computes output channels with v_dot4_i32_i8; max|y| goes to the
// output's amax slots through one LDS max per 16-channel group.  Every multiply
// and add of the fp32 chain is rounded on its own (no contraction), so the
// result equals a scalar restatement of the same formula bit for bit.
// Built with -ffp-contract=off (Makefile).
#include "common.h"
#include "kernels.h"

namespace aexrt {

namespace {

constexpr int kDynThreads = 256;

__global__ __launch_bounds__(kDynThreads) void conv_int8_dynamic_kernel(DynConvParams p) {
    extern __shared__ uint32_t lds[];
    const int G = p.C / 4;
    const int taps = p.K * p.K;
    const int OG = (p.OC + 15) / 16;
    uint32_t* l_ymax = lds;                              // [OG] max|y| per 16-channel output group
    float* l_inv = reinterpret_cast<float*>(lds + OG);  // [G]
    uint32_t* l_q = lds + OG + G;                        // [taps][G]
    for (int i = threadIdx.x; i < OG; i += blockDim.x) l_ymax[i] = 0u;
    const int pos = blockIdx.x;
    const int ohw = p.OH * p.OW;
    const int n = pos / ohw;
    const int r = pos - n * ohw;
    const int oh = r / p.OW, ow = r - (r / p.OW) * p.OW;
    const int pad = p.K == 3 ? 1 : 0;
    const __half* xn = p.x + (int64_t)n * p.x_nstride;
    for (int g = threadIdx.x; g < G; g += blockDim.x) {
        // the taps' values in registers: loops over the largest tap count with
        // constant indices (a runtime-indexed array would live in scratch memory)
        float v[9][4];
        float am = 0.0f;
#pragma unroll
        for (int t = 0; t < 9; ++t) {
            const int iy = oh * p.S + t / p.K - pad;
            const int ix = ow * p.S + t % p.K - pad;
            const bool in = t < taps && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float val = in ? __half2float(xn[(int64_t)(iy * p.W + ix) * p.x_cstride + g * 4 + c]) : 0.0f;
                v[t][c] = val;
                am = fmaxf(am, fabsf(val));
            }
        }
        const float s = am > 0.0f ? __fdiv_rn(127.0f, am) : 0.0f;
        l_inv[g] = __fdiv_rn(am, 127.0f);
#pragma unroll
        for (int t = 0; t < 9; ++t)
            if (t < taps) l_q[t * G + g] = pack4_q(v[t][0], v[t][1], v[t][2], v[t][3], s);
    }
    __syncthreads();
    const bool out_f32 = (p.flags & kConvOutF32) != 0;
    const bool do_res = (p.flags & kConvResidual) != 0;
    for (int oc = threadIdx.x; oc < p.OC; oc += blockDim.x) {
        const int8_t* wrow = p.w + (int64_t)oc * p.Kp;
        float acc = 0.0f;
        for (int g = 0; g < G; ++g) {
            int part = 0;
            for (int t = 0; t < taps; ++t) {
                const int wq = *reinterpret_cast<const int*>(wrow + t * p.C + g * 4);
                part = __builtin_amdgcn_sdot4((int)l_q[t * G + g], wq, part, false);
            }
            acc = __fadd_rn(acc, __fmul_rn((float)part, l_inv[g]));
        }
        float v = __fadd_rn(__fmul_rn(acc, p.w_scale[oc]), p.bias[oc]);
        if (p.flags & kConvSilu) v = silu(v);
        const int64_t yo = (int64_t)n * p.y_nstride + (int64_t)r * p.y_cstride + oc;
        if (out_f32) {
            if (do_res) v += __half2float(p.res[(int64_t)n * p.r_nstride + (int64_t)r * p.r_cstride + oc]);
            static_cast<float*>(p.y)[yo] = v;
        } else {
            if (do_res) {
                // fp16 conv output + fp16 residual, added in fp32 and rounded again
                v = __half2float(__float2half(v)) +
                    __half2float(p.res[(int64_t)n * p.r_nstride + (int64_t)r * p.r_cstride + oc]);
            }
            const __half h = __float2half(v);
            static_cast<__half*>(p.y)[yo] = h;
            v = __half2float(h);
        }
        if (p.y_slots.p && fabsf(v) > 0.0f) atomicMax(&l_ymax[oc / 16], f2u(fabsf(v)));
    }
    if (!p.y_slots.p) return;
    __syncthreads();
    for (int i = threadIdx.x; i < OG; i += blockDim.x)
        if (l_ymax[i]) slot_max(slot_copy(p.y_slots, blockIdx.x) + i, u2f(l_ymax[i]));
}

}  // namespace

hipError_t launch_conv_int8_dynamic(const DynConvParams& p, hipStream_t stream) {
    if (p.K != 1 && p.K != 3) return hipErrorInvalidValue;
    if (p.C % 16 || p.C <= 0 || p.OC <= 0 || p.N <= 0 || p.OH <= 0 || p.OW <= 0) return hipErrorInvalidValue;
    if (p.K == 1 && (p.S != 1 || p.OH != p.H || p.OW != p.W)) return hipErrorInvalidValue;
    if (p.K == 3 && (p.S < 1 || p.S > 2 || (p.OH - 1) * p.S + 1 > p.H + 1 || (p.OW - 1) * p.S + 1 > p.W + 1))
        return hipErrorInvalidValue;
    if (p.Kp < p.K * p.K * p.C) return hipErrorInvalidValue;
    const int64_t positions = (int64_t)p.N * p.OH * p.OW;
    if (positions > (1 << 30)) return hipErrorInvalidValue;
    const size_t lds = ((size_t)(p.C / 4) * (1 + p.K * p.K) + (p.OC + 15) / 16) * 4;
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(conv_int8_dynamic_kernel, dim3((unsigned)positions), dim3(kDynThreads), lds, stream, p);
    return hipGetLastError();
}

}  // namespace aexrt
