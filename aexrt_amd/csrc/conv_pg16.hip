// pg16 int8 convolution (per-16-input-channel activation scales) and the
// fused amax + pack of its input.
//
// The reference's pg16 conv (native/aexrt_d3d12_runtime.cpp:4770-4923) sums
// the int8 products of one 16-channel group exactly in int32, scales each
// group sum by amax[1 + g] / 127 into an fp32 accumulator, and finishes with
// the oc weight scale, the bias and SiLU.  One v_mfma_i32_16x16x64_i8 covers
// 64 input channels, i.e. four groups, and its sum would mix them.  Here the
// A operand (weights) is made block-diagonal instead: of the 16 A rows, row
// 4o + r carries output channel oc0 + 4o + j's weights of group r only (the
// lanes of the three other lane groups read zero), so row 4o + r of the
// product is the exact int32 sum of group r alone.  A lane of lane group grp
// then holds the four group sums of one (output channel, position); four
// MFMAs (j = 0..3) cover 16 output channels, and lane (grp, col) ends with
// channels oc0 + 4 grp + j of position col -- the fragment layout of the
// per-tensor kernels, so their epilogue and 8-byte NHWC stores are reused.
//
// The int32 group sums run over all taps of the kernel before the fp32
// scaling (exact integers; the reference scales per tap for 3x3 and per 8
// channels for 1x1, which differs only in fp32 rounding).  The MFMA work is
// 4x that of the per-tensor kernel; at these shapes the kernels are bound by
// memory latency and VALU, not by MFMA.
#include "conv_igemm.h"

namespace aexrt {

namespace {

using igemm::bload16;
using igemm::kOob;
using igemm::make_rsrc;
using igemm::quant8;
using igemm::rsrc_t;
using igemm::v2i;

constexpr int kPgWaves = 4;
constexpr int kPgMaxGroups = 256;  // in_channels <= 4096

// LOADER kLoaderNhwc: fp16 NHWC view quantized here with 127/amax_g (the
// reference's pack with per-group scales, RT:3330-3344); kLoaderPackedNc4: the
// reference's packed NC/4HW4 int8 ((n * C/4 + icg) * H*W + pixel words).
template <int KK, int LOADER>
__global__ __launch_bounds__(kPgWaves * 64) void conv_int8_pg16_kernel(ConvParams p) {
    __shared__ float l_gs[kPgMaxGroups];  // amax_g / 127
    __shared__ float l_qs[kPgMaxGroups];  // 127 / amax_g, 0 when amax_g is not > 0
    __shared__ float l_bias[16], l_scale[16];
    __shared__ uint32_t l_slots[1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int T = (p.C + 63) >> 6;  // 64-channel steps
    const int G = p.C >> 4;
    for (int g = tid; g < 4 * T; g += kPgWaves * 64) {
        uint32_t m = 0;
        if (g < G)
            for (uint32_t s = 0; s < p.x_slots.stripes; ++s) m = max(m, p.x_slots.p[s * p.x_slots.stride + g]);
        const float a = u2f(m);
        l_gs[g] = g < G ? a / 127.0f : 0.0f;
        l_qs[g] = a > 0.0f ? 127.0f / a : 0.0f;
    }
    const int oc0 = blockIdx.y * 16;
    if (tid < 16) {
        const int oc = oc0 + tid;
        l_bias[tid] = oc < p.OC ? p.bias[oc] : 0.0f;
        l_scale[tid] = oc < p.OC ? p.w_scale[oc] : 0.0f;
    }
    if (tid == 0) l_slots[0] = 0u;
    __syncthreads();

    const int m = (blockIdx.x * kPgWaves + wave) * 16 + col;
    const bool mok = m < p.M;
    const int mm = mok ? m : 0;
    const int n = (int)fdiv((uint32_t)mm, p.fd_ohw);
    const int pos = mm - n * p.OH * p.OW;
    const int oh = (int)fdiv((uint32_t)pos, p.fd_ow);
    const int ow = pos - oh * p.OW;
    const int iy0 = oh * p.S - p.P, ix0 = ow * p.S - p.P;
    const uint32_t plane = (uint32_t)(p.H * p.W);

    const rsrc_t rx = make_rsrc(p.x, p.x_bytes);
    const rsrc_t rw = make_rsrc(p.w, (uint32_t)p.OCp * (uint32_t)p.Kp);
    // element offset of (n, channel 0, pixel 0) in the input
    const uint32_t xbase = LOADER == kLoaderPackedNc4 ? (uint32_t)n * (uint32_t)(p.C >> 2) * plane
                                                      : (uint32_t)((int64_t)n * p.x_nstride);
    // A row col = 4 o + r: output channel oc0 + 4 o + j, group r of the step;
    // only lane group r loads it, every other lane reads zero
    const int wo = col >> 2;
    const bool wlane = (col & 3) == grp;

    typedef float v4f_t __attribute__((ext_vector_type(4)));
    v4f_t accf = {0.0f, 0.0f, 0.0f, 0.0f};  // channel oc0 + 4 grp + j
    for (int t = 0; t < T; ++t) {
        const int c0 = 64 * t + 16 * grp;  // this lane group's 16 channels
        const bool cok = c0 < p.C;
        v4i acc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int tap = 0; tap < KK; ++tap) {
            const int iy = iy0 + (KK == 9 ? tap / 3 : 0);
            const int ix = ix0 + (KK == 9 ? tap % 3 : 0);
            const bool ok = mok && cok && iy >= 0 && iy < p.H && ix >= 0 && ix < p.W;
            const uint32_t pix = (uint32_t)(iy * p.W + ix);
            v4i b;
            if constexpr (LOADER == kLoaderPackedNc4) {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    b[q] = __builtin_amdgcn_raw_buffer_load_b32(
                        rx, ok ? (xbase + (uint32_t)((c0 >> 2) + q) * plane + pix) * 4u : kOob, 0, 0);
            } else {
                const uint32_t e = xbase + pix * (uint32_t)p.x_cstride + (uint32_t)c0;
                const v4i lo = bload16(rx, ok ? e * 2u : kOob);
                const v4i hi = bload16(rx, ok ? (e + 8u) * 2u : kOob);
                const float s = l_qs[4 * t + grp];
                const v2i q0 = quant8(lo, s), q1 = quant8(hi, s);
                b = v4i{q0[0], q0[1], q1[0], q1[1]};
            }
            const uint32_t k = (uint32_t)(tap * p.C + c0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t oc = (uint32_t)(oc0 + 4 * wo + j);
                const v4i a = bload16(rw, wlane && cok ? oc * (uint32_t)p.Kp + k : kOob);
                acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[j], 0, 0, 0);
            }
        }
        // acc[j][r] = int32 sum of group 4t + r for channel oc0 + 4 grp + j
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) accf[j] = __builtin_fmaf((float)acc[j][r], l_gs[4 * t + r], accf[j]);
    }

    const bool do_silu = (p.flags & kConvSilu) != 0;
    const bool out_f32 = (p.flags & kConvOutF32) != 0;
    if (p.flags & kConvOutNchw) {
        // dense NCHW output of the reference (typed fp32 or fp16 storage)
        const rsrc_t ry = make_rsrc(p.y, p.y_bytes);
        const int ohw = p.OH * p.OW;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int lc = 4 * grp + j, oc = oc0 + lc;
            float v = __builtin_fmaf(accf[j], l_scale[lc], l_bias[lc]);
            if (do_silu) v = silu(v);
            const bool ok = mok && oc < p.OC;
            const uint32_t e = (uint32_t)((n * p.OC + oc) * ohw + pos);
            if (out_f32)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(v), ry, ok ? e * 4u : kOob, 0, 0);
            else
                __builtin_amdgcn_raw_buffer_store_b16(__half_as_short(__float2half(v)), ry, ok ? e * 2u : kOob, 0,
                                                      0);
        }
        return;
    }
    // NHWC view output: the per-tensor kernels' epilogue (scale, bias, SiLU,
    // residual, amax slots of the output)
    const rsrc_t ry = make_rsrc(p.y, p.y_bytes);
    const rsrc_t rr = make_rsrc(p.res, p.r_bytes);
    const rsrc_t racc = make_rsrc(nullptr, 0u);
    int yo[1], ro[1], mo[1];
    yo[0] = mok ? (int)((int64_t)n * p.y_nstride + (int64_t)pos * p.y_cstride) : -1;
    ro[0] = (int)((int64_t)n * p.r_nstride + (int64_t)pos * p.r_cstride);
    mo[0] = m;
    v2i rv[1][1];
    igemm::tile_residual<1, 1, igemm::kEpiAny>(p, rr, yo, ro, oc0, 1, grp, 1u, rv);
    const v4f_t accs[1][1] = {{accf}};
    float gmax[1] = {0.0f};
    igemm::tile_store<true, 1, 1, igemm::kEpiAny>(p, accs, yo, mo, rv, oc0, 1, grp, 1u, l_bias, l_scale, gmax, ry,
                                                  racc);
    igemm::flush_slots<1>(p, gmax, oc0, 1, 1u, out_f32, l_slots);
}

// a3: the reference's fused amax + pack (RT:4083-4149).  One block per
// (image n, 16-channel group g): the group max is taken over channels
// 16g..16g+15 of image 0's memory for every n (the reference's strip start
// carries no image offset), written to amax[1 + g] (every n writes the same
// value), and image n's four 4-channel planes of the group are packed with
// s = 127/max.  amax[0] is not written.
constexpr int kFusedThreads = 512;

template <typename T>
__device__ __forceinline__ float ld_f(const T* x, int64_t i) {
    if constexpr (sizeof(T) == 2) return __half2float(x[i]);
    else return x[i];
}

template <typename T>
__global__ __launch_bounds__(kFusedThreads) void quant_fused_pg16_kernel(const T* x, int C, int HW,
                                                                         uint32_t* packed, uint32_t* amax) {
    __shared__ float lm[kFusedThreads / 64];
    const int G = C >> 4;
    const int n = blockIdx.x / G, g = blockIdx.x - n * G;
    const int64_t b = (int64_t)g * 16 * HW;
    const int64_t span = (int64_t)16 * HW;
    float m = 0.0f;
    for (int64_t i = threadIdx.x; i < span; i += kFusedThreads) m = fmaxf(m, fabsf(ld_f(x, b + i)));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) lm[threadIdx.x >> 6] = m;
    __syncthreads();
    m = lm[0];
#pragma unroll
    for (int w = 1; w < kFusedThreads / 64; ++w) m = fmaxf(m, lm[w]);
    if (threadIdx.x == 0) amax[g + 1] = f2u(m);
    const int icg_count = C >> 2;
    const float s = 127.0f / m;
    const int64_t out0 = ((int64_t)n * icg_count + 4 * g) * HW;
    const int64_t in0 = out0 * 4;
    for (int e = threadIdx.x; e < 4 * HW; e += kFusedThreads) {
        const int il = e / HW, pp = e - il * HW;
        uint32_t v = 0u;
        if (m > 0.0f) {
            const int64_t base = in0 + (int64_t)il * 4 * HW + pp;
            v = pack4_q(ld_f(x, base), ld_f(x, base + HW), ld_f(x, base + 2 * HW), ld_f(x, base + 3 * HW), s);
        }
        packed[out0 + e] = v;
    }
}

template <int KK, int LOADER>
void launch_pg(const ConvParams& p, hipStream_t stream) {
    const dim3 grid((p.M + kPgWaves * 16 - 1) / (kPgWaves * 16), p.OCp / 16);
    hipLaunchKernelGGL((conv_int8_pg16_kernel<KK, LOADER>), grid, dim3(kPgWaves * 64), 0, stream, p);
}

uint64_t span_nhwc(int N, int64_t nstride, int32_t cstride, int HW, int C, int esz) {
    if (N <= 0) return 0;
    return (uint64_t)(((int64_t)(N - 1) * nstride + (int64_t)(HW - 1) * cstride + C) * esz);
}

}  // namespace

hipError_t launch_conv_int8_pg16(const ConvParams& p0, hipStream_t stream) {
    const bool packed = p0.loader == kLoaderPackedNc4;
    const bool nchw_out = (p0.flags & kConvOutNchw) != 0;
    if ((p0.loader != kLoaderNhwc && !packed) || p0.C % 16 || p0.C > 16 * kPgMaxGroups || p0.OC % 4 ||
        p0.Kp % 64 || p0.OCp % 16 || p0.acc_out || !p0.x_slots.p || !(p0.KH == p0.KW) ||
        (p0.KH != 1 && p0.KH != 3) || (nchw_out && (p0.flags & kConvResidual)))
        return hipErrorInvalidValue;
    const bool out_f32 = (p0.flags & kConvOutF32) != 0;
    const int HWi = p0.H * p0.W, HWo = p0.OH * p0.OW;
    const uint64_t x_img = packed ? (uint64_t)p0.C * HWi
                                  : std::max((uint64_t)p0.x_nstride * 2, (uint64_t)HWi * p0.x_cstride * 2);
    const uint64_t y_img = nchw_out ? (uint64_t)p0.OC * HWo * (out_f32 ? 4 : 2)
                                    : std::max((uint64_t)p0.y_nstride, (uint64_t)HWo * p0.y_cstride) *
                                          (out_f32 ? 4 : 2);
    const uint64_t per_img = std::max({x_img, y_img, p0.res ? (uint64_t)p0.r_nstride * 2 : 0});
    if ((uint64_t)p0.OCp * p0.Kp > kMaxViewBytes || per_img == 0) return hipErrorInvalidValue;
    const int per_launch = (int)std::min<uint64_t>((uint64_t)p0.N, kMaxViewBytes / per_img);
    if (per_launch < 1) return hipErrorInvalidValue;
    for (int nb = 0; nb < p0.N; nb += per_launch) {
        ConvParams p = p0;
        p.N = std::min(per_launch, p0.N - nb);
        p.M = p.N * HWo;
        if (packed) {
            p.x = static_cast<const uint8_t*>(p0.x) + (int64_t)nb * p0.C * HWi;
            p.x_bytes = (uint32_t)((uint64_t)p.N * p.C * HWi);
        } else {
            p.x = static_cast<const __half*>(p0.x) + (int64_t)nb * p0.x_nstride;
            p.x_bytes = (uint32_t)span_nhwc(p.N, p.x_nstride, p.x_cstride, HWi, p.C, 2);
        }
        const int esz = out_f32 ? 4 : 2;
        if (nchw_out) {
            p.y = static_cast<char*>(p0.y) + (int64_t)nb * p0.OC * HWo * esz;
            p.y_bytes = (uint32_t)((uint64_t)p.N * p.OC * HWo * esz);
        } else {
            p.y = static_cast<char*>(p0.y) + (int64_t)nb * p0.y_nstride * esz;
            p.y_bytes = (uint32_t)span_nhwc(p.N, p.y_nstride, p.y_cstride, HWo, p.OC, esz);
        }
        if (p0.res) {
            p.res = p0.res + (int64_t)nb * p0.r_nstride;
            p.r_bytes = (uint32_t)span_nhwc(p.N, p.r_nstride, p.r_cstride, HWo, p.OC, 2);
        }
        p.fd_ohw = make_fastdiv((uint32_t)HWo);
        p.fd_ow = make_fastdiv((uint32_t)p.OW);
        if (p.KH == 1) {
            if (packed) launch_pg<1, kLoaderPackedNc4>(p, stream);
            else launch_pg<1, kLoaderNhwc>(p, stream);
        } else {
            if (packed) launch_pg<9, kLoaderPackedNc4>(p, stream);
            else launch_pg<9, kLoaderNhwc>(p, stream);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_quant_fused_pg16(const void* x, bool f16, int N, int C, int HW, uint32_t* packed,
                                   uint32_t* amax, hipStream_t stream) {
    if (!x || !packed || !amax || N < 1 || C < 16 || C % 16 || HW < 1) return hipErrorInvalidValue;
    const int64_t blocks = (int64_t)N * (C / 16);
    if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
    if (f16)
        hipLaunchKernelGGL(quant_fused_pg16_kernel<__half>, dim3((unsigned)blocks), dim3(kFusedThreads), 0, stream,
                           static_cast<const __half*>(x), C, HW, packed, amax);
    else
        hipLaunchKernelGGL(quant_fused_pg16_kernel<float>, dim3((unsigned)blocks), dim3(kFusedThreads), 0, stream,
                           static_cast<const float*>(x), C, HW, packed, amax);
    return hipGetLastError();
}

}  // namespace aexrt
