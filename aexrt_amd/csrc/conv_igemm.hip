// Implicit-GEMM convolution on gfx950 MFMA: the W8A8 int8 convolution
// (reference kernels 51/52/53) and the fp16 convolution it falls back to
// (reference kernels 5/43/45 and the fp16 stem/head convs).
//
// GEMM view: M = N*OH*OW output positions (batch folded into M), N = output
// channels, K = KH*KW*C ordered (ky, kx, c) with c fastest, so that NHWC
// activations give contiguous K runs.  Weights are repacked at load to
// [OCp][Kp] (OCp = OC rounded up to 16, Kp = K rounded up to 64, zero padded),
// i.e. one K-contiguous row per output channel.
//
// int8: the activation tile is quantized while it is staged into LDS
// (q = rne(x * 127/amax) & 0xFF, the reference's pack pass RT:3314-3346, done
// by the consumer instead of a separate dispatch), the contraction runs on
// v_mfma_i32_16x16x64_i8 with exact int32 accumulation, and the epilogue
// dequantizes as float(acc) * (amax/127) * w_scale[oc] + bias[oc]
// (RT:4669-4674) before SiLU.  fp16: v_mfma_f32_16x16x32_f16, fp32
// accumulation, + bias, SiLU.
//
// Every epilogue rounds to the stored type and folds max|y| of each
// 16-channel group into the output tensor's amax slots (one atomicMax per
// wave and group), so the next int8 consumer needs no separate amax pass.
#include "common.h"
#include "kernels.h"

namespace aexrt {

namespace {

constexpr int BK = 64;  // K elements per pipeline stage

template <bool INT8>
struct Elem;
template <>
struct Elem<true> { static constexpr int bytes = 1; };
template <>
struct Elem<false> { static constexpr int bytes = 2; };

// XCD-aware tile order: workgroups are dealt round-robin over the 8 XCDs, so
// block b runs on XCD b % 8.  Give each XCD a contiguous run of tiles (all
// N-tiles of an M-tile together) so the input rows of a tile are fetched
// into one L2 only.
__device__ __forceinline__ int xcd_remap(int b, int nb) {
    const int full = (nb / 8) * 8;
    if (b >= full) return b;
    return (b % 8) * (nb / 8) + b / 8;
}

template <bool INT8, int BM, int BN, int WM, int WN, int LOADER>
__global__ __launch_bounds__(64 * WM * WN) void conv_igemm_kernel(ConvParams p) {
    constexpr int NT = 64 * WM * WN;
    constexpr int ESZ = Elem<INT8>::bytes;
    constexpr int ROWB = BK * ESZ + 16;  // padded LDS row (bytes)
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int SI = TM / 16, SJ = TN / 16;
    constexpr int KC = BK / 8;  // 8-element A chunks per row
    static_assert(NT % KC == 0 && BM % (NT / KC) == 0, "A tile split");
    constexpr int CA = BM / (NT / KC);  // A chunks per thread
    constexpr int BCPR = BK * ESZ / 16;  // 16-byte B chunks per row
    constexpr int BCH = BN * BCPR;       // B chunks per stage
    constexpr int CB = (BCH + NT - 1) / NT;

    __shared__ __attribute__((aligned(16))) uint8_t smem[2][(BM + BN) * ROWB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    const int ntn = (p.OC + BN - 1) / BN;
    const int nb = gridDim.x;
    const int t = xcd_remap(blockIdx.x, nb);
    const int m0 = (t / ntn) * BM;
    const int n0 = (t % ntn) * BN;

    // Input amax over the view's slots -> quantization scale.
    float s_q = 0.0f, in_scale = 0.0f;
    if constexpr (INT8) {
        uint32_t am = 0;
        for (int i = 0; i < p.x_nslots; ++i) am = max(am, p.x_slots[i]);
        const float a = u2f(am);
        if (a > 0.0f) {
            s_q = 127.0f / a;
            in_scale = a / 127.0f;
        }
    }

    // Per-thread A rows: fixed chunk column kc, rows r = tid/KC + i*(NT/KC).
    const int kc = tid % KC;
    const int OHW = p.OH * p.OW;
    int row_ih[CA], row_iw[CA];
    int64_t row_base[CA];
#pragma unroll
    for (int i = 0; i < CA; ++i) {
        const int m = m0 + tid / KC + i * (NT / KC);
        if (m < p.M) {
            const int n = m / OHW;
            const int rem = m - n * OHW;
            const int oh = rem / p.OW;
            const int ow = rem - oh * p.OW;
            row_ih[i] = oh * p.S - p.P;
            row_iw[i] = ow * p.S - p.P;
            row_base[i] = (int64_t)n * p.x_nstride;
        } else {
            row_ih[i] = -(1 << 28);  // never in bounds
            row_iw[i] = 0;
            row_base[i] = 0;
        }
    }

    // Staging registers for one stage.
    uint4 areg[CA];
    uint4 breg[CB];

    auto load_a = [&](int ks) {
        const int k = ks * BK + kc * 8;
#pragma unroll
        for (int i = 0; i < CA; ++i) areg[i] = make_uint4(0, 0, 0, 0);
        if (k >= p.K) return;
        if constexpr (LOADER == kLoaderNhwc) {
            const int tap = k / p.C;
            const int c = k - tap * p.C;
            const int ky = tap / p.KW;
            const int kx = tap - ky * p.KW;
            const __half* xb = reinterpret_cast<const __half*>(p.x);
#pragma unroll
            for (int i = 0; i < CA; ++i) {
                const int ih = row_ih[i] + ky, iw = row_iw[i] + kx;
                if ((unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W) {
                    const __half* src = xb + row_base[i] + ((int64_t)ih * p.W + iw) * p.x_cstride + c;
                    areg[i] = *reinterpret_cast<const uint4*>(src);
                }
            }
        } else {
            // fp32 NCHW gather (network input); K order (ky, kx, c), any C.
            const float* xf = reinterpret_cast<const float*>(p.x);
            const int64_t plane = (int64_t)p.H * p.W;
#pragma unroll
            for (int i = 0; i < CA; ++i) {
                _Float16 v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int kk = k + e;
                    float val = 0.0f;
                    if (kk < p.K) {
                        const int tap = kk / p.C;
                        const int c = kk - tap * p.C;
                        const int ky = tap / p.KW;
                        const int kx = tap - ky * p.KW;
                        const int ih = row_ih[i] + ky, iw = row_iw[i] + kx;
                        if ((unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W)
                            val = xf[row_base[i] + c * plane + (int64_t)ih * p.W + iw];
                    }
                    v[e] = (_Float16)val;
                }
                areg[i] = *reinterpret_cast<uint4*>(v);
            }
        }
    };

    auto load_b = [&](int ks) {
        const uint8_t* wb = reinterpret_cast<const uint8_t*>(p.w);
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const int c = tid + j * NT;
            breg[j] = make_uint4(0, 0, 0, 0);
            if (c < BCH) {
                const int r = n0 + c / BCPR;
                const int off = c % BCPR;
                if (r < p.OCp)
                    breg[j] = *reinterpret_cast<const uint4*>(
                        wb + ((int64_t)r * p.Kp + (int64_t)ks * BK) * ESZ + off * 16);
            }
        }
    };

    auto store_stage = [&](int buf) {
        uint8_t* sa = smem[buf];
        uint8_t* sb = smem[buf] + BM * ROWB;
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int r = tid / KC + i * (NT / KC);
            if constexpr (INT8) {
                const __half2* h = reinterpret_cast<const __half2*>(&areg[i]);
                float2 f0 = __half22float2(h[0]), f1 = __half22float2(h[1]);
                float2 f2 = __half22float2(h[2]), f3 = __half22float2(h[3]);
                uint2 q;
                q.x = pack4_q(f0.x, f0.y, f1.x, f1.y, s_q);
                q.y = pack4_q(f2.x, f2.y, f3.x, f3.y, s_q);
                *reinterpret_cast<uint2*>(sa + r * ROWB + kc * 8) = q;
            } else {
                *reinterpret_cast<uint4*>(sa + r * ROWB + kc * 16) = areg[i];
            }
        }
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const int c = tid + j * NT;
            if (c < BCH) {
                const int r = c / BCPR;
                const int off = c % BCPR;
                *reinterpret_cast<uint4*>(sb + r * ROWB + off * 16) = breg[j];
            }
        }
    };

    typedef typename std::conditional<INT8, v4i, v4f>::type acc_t;
    acc_t acc[SI][SJ];
#pragma unroll
    for (int i = 0; i < SI; ++i)
#pragma unroll
        for (int j = 0; j < SJ; ++j) acc[i][j] = acc_t{0, 0, 0, 0};

    const int nks = p.Kp / BK;
    load_a(0);
    load_b(0);
    store_stage(0);
    __syncthreads();

    const int lr = lane & 15;
    const int lg = lane >> 4;
    for (int ks = 0; ks < nks; ++ks) {
        const int buf = ks & 1;
        if (ks + 1 < nks) {
            load_a(ks + 1);
            load_b(ks + 1);
        }
        const uint8_t* sa = smem[buf];
        const uint8_t* sb = smem[buf] + BM * ROWB;
        if constexpr (INT8) {
            v4i a[SI], b[SJ];
#pragma unroll
            for (int i = 0; i < SI; ++i)
                a[i] = *reinterpret_cast<const v4i*>(sa + (wm * TM + i * 16 + lr) * ROWB + lg * 16);
#pragma unroll
            for (int j = 0; j < SJ; ++j)
                b[j] = *reinterpret_cast<const v4i*>(sb + (wn * TN + j * 16 + lr) * ROWB + lg * 16);
#pragma unroll
            for (int i = 0; i < SI; ++i)
#pragma unroll
                for (int j = 0; j < SJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                v8h a[SI], b[SJ];
#pragma unroll
                for (int i = 0; i < SI; ++i)
                    a[i] = *reinterpret_cast<const v8h*>(sa + (wm * TM + i * 16 + lr) * ROWB + h * 64 + lg * 16);
#pragma unroll
                for (int j = 0; j < SJ; ++j)
                    b[j] = *reinterpret_cast<const v8h*>(sb + (wn * TN + j * 16 + lr) * ROWB + h * 64 + lg * 16);
#pragma unroll
                for (int i = 0; i < SI; ++i)
#pragma unroll
                    for (int j = 0; j < SJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
        }
        if (ks + 1 < nks) {
            store_stage(buf ^ 1);
            __syncthreads();
        }
    }

    // Epilogue.  16x16 MFMA result layout: lane holds column (lane & 15) and
    // rows 4*(lane >> 4) + r of its sub-tile in register r.
    const bool do_silu = p.flags & kConvSilu;
    const bool do_res = p.flags & kConvResidual;
    const bool out_f32 = p.flags & kConvOutF32;
#pragma unroll
    for (int j = 0; j < SJ; ++j) {
        const int col = n0 + wn * TN + j * 16 + lr;
        const bool col_ok = col < p.OC;
        float ws = 0.0f, bs = 0.0f;
        if (col_ok) {
            bs = p.bias[col];
            if constexpr (INT8) ws = p.w_scale[col];
        }
        float gmax = 0.0f;
#pragma unroll
        for (int i = 0; i < SI; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + wm * TM + i * 16 + lg * 4 + r;
                if (!col_ok || m >= p.M) continue;
                float v;
                if constexpr (INT8) {
                    const int32_t a = acc[i][j][r];
                    if (p.acc_out) p.acc_out[(int64_t)m * p.OC + col] = a;
                    v = (float)a * in_scale;
                    v = v * ws;
                    v = v + bs;
                } else {
                    v = acc[i][j][r] + bs;
                }
                if (do_silu) v = silu(v);
                const int n = m / OHW;
                const int pos = m - n * OHW;
                if (do_res) {
                    const __half* rp = p.res + (int64_t)n * p.r_nstride + (int64_t)pos * p.r_cstride + col;
                    v = v + __half2float(*rp);
                }
                const int64_t yo = (int64_t)n * p.y_nstride + (int64_t)pos * p.y_cstride + col;
                if (out_f32) {
                    reinterpret_cast<float*>(p.y)[yo] = v;
                    gmax = fmaxf(gmax, fabsf(v));
                } else {
                    const __half h = __float2half(v);
                    reinterpret_cast<__half*>(p.y)[yo] = h;
                    gmax = fmaxf(gmax, fabsf(__half2float(h)));
                }
            }
        }
        if (p.y_slots) {
            gmax = wave_max(gmax);
            const int g = (n0 + wn * TN + j * 16) / 16;
            if (lane == 0 && n0 + wn * TN + j * 16 < p.OC) atomicMax(p.y_slots + g, f2u(gmax));
        }
    }
}

template <bool INT8, int BM, int BN, int WM, int WN, int LOADER>
hipError_t launch_cfg(const ConvParams& p, hipStream_t stream) {
    const int tiles = ((p.M + BM - 1) / BM) * ((p.OC + BN - 1) / BN);
    hipLaunchKernelGGL((conv_igemm_kernel<INT8, BM, BN, WM, WN, LOADER>), dim3(tiles),
                       dim3(64 * WM * WN), 0, stream, p);
    return hipGetLastError();
}

template <bool INT8, int LOADER>
hipError_t launch_any(const ConvParams& p, hipStream_t stream) {
    if (p.OC <= 16) return launch_cfg<INT8, 128, 16, 4, 1, LOADER>(p, stream);
    if (p.OC <= 32) return launch_cfg<INT8, 128, 32, 4, 1, LOADER>(p, stream);
    const int tiles128 = ((p.M + 127) / 128) * ((p.OC + 63) / 64);
    if (tiles128 < 512) return launch_cfg<INT8, 64, 64, 2, 2, LOADER>(p, stream);
    return launch_cfg<INT8, 128, 64, 2, 2, LOADER>(p, stream);
}

}  // namespace

hipError_t launch_conv_igemm(const ConvParams& p, bool int8, hipStream_t stream) {
    if (int8) {
        if (p.loader != kLoaderNhwc) return hipErrorInvalidValue;
        return launch_any<true, kLoaderNhwc>(p, stream);
    }
    if (p.loader == kLoaderNchwF32) return launch_any<false, kLoaderNchwF32>(p, stream);
    return launch_any<false, kLoaderNhwc>(p, stream);
}

}  // namespace aexrt
