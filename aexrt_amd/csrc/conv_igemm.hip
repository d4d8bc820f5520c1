// Implicit-GEMM convolution on gfx950 MFMA: the W8A8 int8 convolution
// (reference kernels 51/52/53) and the fp16 convolution it falls back to
// (reference kernels 5/43/45 and the fp16 stem/head convs).
//
// GEMM view: M = N*OH*OW output positions (batch folded into M), N = output
// channels, K = KH*KW*C ordered (ky, kx, c) with c fastest, so that NHWC
// activations give contiguous K runs.  Weights are repacked at load to
// [OCp][Kp] (OCp = OC rounded up to 16, Kp = K rounded up to 64, zero padded),
// one K-contiguous row per output channel.
//
// int8: the activation tile is quantized while it is staged into LDS
// (q = rne(x * 127/amax) & 0xFF, the reference's pack pass RT:3314-3346, done
// by the consumer instead of a separate dispatch), the contraction runs on
// v_mfma_i32_16x16x64_i8 with exact int32 accumulation, and the epilogue
// dequantizes as float(acc) * (amax/127) * w_scale[oc] + bias[oc]
// (RT:4669-4674) before SiLU.  fp16: v_mfma_f32_16x16x32_f16, fp32
// accumulation, + bias, SiLU.
//
// Pipeline per block: a whole K chunk (128-256 elements) of the A and B tiles
// is fetched with every load of the chunk in flight at once, quantized /
// staged into LDS, and consumed by 2-8 MFMA k-steps per wave; the next
// chunk's loads are issued before the current chunk's MFMAs.  The epilogue
// goes register -> LDS -> 16-byte coalesced stores, adds the residual there
// (a bottleneck's "x + cv2(cv1(x))", RT's BINARY add fused) and folds max|y|
// of each 16-channel group into the output tensor's amax slots.
//
// Split-K (small M, e.g. 10x10 layers at batch 1): blocks of one output tile
// split the K chunks, write exact int32 (fp32 for fp16) partial tiles to a
// workspace, and the last block to arrive sums the partials in split order
// and runs the epilogue; it also re-arms the tile's arrival counter, so the
// workspace needs no clearing between runs (graph replays included).
#include "common.h"
#include "kernels.h"

namespace aexrt {

namespace {

template <bool INT8>
struct Elem;
template <>
struct Elem<true> { static constexpr int bytes = 1; };
template <>
struct Elem<false> { static constexpr int bytes = 2; };

// XCD-aware tile order: workgroups are dealt round-robin over the 8 XCDs, so
// block b runs on XCD b % 8.  Give each XCD a contiguous run of tiles so the
// input rows of neighbouring tiles are fetched into one L2.
__device__ __forceinline__ int xcd_remap(int b, int nb) {
    const int full = (nb / 8) * 8;
    if (b >= full) return b;
    return (b % 8) * (nb / 8) + b / 8;
}

template <bool INT8, int BM, int BN, int WM, int WN, int KCH>
__global__ __launch_bounds__(256) void conv_igemm_kernel(ConvParams p) {
    constexpr int NT = 256;
    static_assert(WM * WN == 4, "4 waves");
    constexpr int ESZ = Elem<INT8>::bytes;
    constexpr int ROWB = KCH * ESZ + 16;  // padded LDS row (bytes)
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int SI = TM / 16, SJ = TN / 16;
    constexpr int KCC = KCH / 8;          // 8-element A chunks per row
    static_assert(NT % KCC == 0 && BM % (NT / KCC) == 0, "A tile split");
    constexpr int CA = BM / (NT / KCC);   // A chunks (rows) per thread
    constexpr int BCPR = KCH * ESZ / 16;  // 16-byte B chunks per row
    constexpr int BCH = BN * BCPR;
    constexpr int CB = (BCH + NT - 1) / NT;
    constexpr int AB_BYTES = (BM + BN) * ROWB;
    // epilogue staging reuses the A/B LDS: fp16 always fits, fp32 only for
    // tiles the host launches with fp32 output (F32_OK)
    constexpr int OUT_ROW16 = BN * 2 + 16;
    constexpr int OUT_ROW32 = BN * 4 + 16;
    constexpr int LDS_BYTES = AB_BYTES > BM * OUT_ROW16 ? AB_BYTES : BM * OUT_ROW16;
    constexpr bool F32_OK = BM * OUT_ROW32 <= LDS_BYTES;

    __shared__ __attribute__((aligned(16))) uint8_t smem[LDS_BYTES];
    __shared__ uint32_t lslots[BN / 16];
    __shared__ int last_flag;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 15, lg = lane >> 4;

    const int ntn = (p.OC + BN - 1) / BN;
    const int ntiles = gridDim.x;
    const int tile = xcd_remap(blockIdx.x, ntiles);
    const int m0 = (tile / ntn) * BM;
    const int n0 = (tile % ntn) * BN;
    const int split = blockIdx.y;

    // K chunks of this block
    const int nchunks = (p.Kp + KCH - 1) / KCH;
    const int cps = (nchunks + p.ksplit - 1) / p.ksplit;
    const int c_begin = split * cps;
    const int c_end = min(nchunks, c_begin + cps);

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

    // Per-thread A rows: fixed chunk column kc, rows tid/KCC + i*(NT/KCC).
    const int kc = tid % KCC;
    const int OHW = p.OH * p.OW;
    int rowpix[CA];       // pixel index of (n, oh*S-P, ow*S-P)
    uint32_t rowhw[CA];   // (ih0 + 32768) << 16 | (iw0 + 32768)
#pragma unroll
    for (int i = 0; i < CA; ++i) {
        const int m = m0 + tid / KCC + i * (NT / KCC);
        if (m < p.M) {
            const int n = m / OHW;
            const int rem = m - n * OHW;
            const int oh = rem / p.OW;
            const int ow = rem - oh * p.OW;
            const int ih0 = oh * p.S - p.P, iw0 = ow * p.S - p.P;
            rowpix[i] = (n * p.H + ih0) * p.W + iw0;
            rowhw[i] = ((uint32_t)(ih0 + 32768) << 16) | (uint32_t)(iw0 + 32768);
        } else {
            rowpix[i] = 0;
            rowhw[i] = 0u;  // ih0 = -32768: never in bounds
        }
    }

    uint4 areg[CA];
    uint4 breg[CB];
    const __half* xb = reinterpret_cast<const __half*>(p.x);
    const uint8_t* wb = reinterpret_cast<const uint8_t*>(p.w);

    auto load_chunk = [&](int ch) {
        const int k = ch * KCH + kc * 8;
#pragma unroll
        for (int i = 0; i < CA; ++i) areg[i] = make_uint4(0, 0, 0, 0);
        if (k < p.K) {
            const int tap = k / p.C;
            const int c = k - tap * p.C;
            const int ky = tap / p.KW;
            const int kx = tap - ky * p.KW;
            const int koff = ky * p.W + kx;
#pragma unroll
            for (int i = 0; i < CA; ++i) {
                const int ih = (int)(rowhw[i] >> 16) - 32768 + ky;
                const int iw = (int)(rowhw[i] & 0xffffu) - 32768 + kx;
                if ((unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W)
                    areg[i] = *reinterpret_cast<const uint4*>(xb + (int64_t)(rowpix[i] + koff) * p.x_cstride + c);
            }
        }
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const int cidx = tid + j * NT;
            breg[j] = make_uint4(0, 0, 0, 0);
            if (cidx < BCH) {
                const int r = n0 + cidx / BCPR;
                const int kel = ch * KCH + (cidx % BCPR) * (16 / ESZ);
                if (r < p.OCp && kel < p.Kp)
                    breg[j] = *reinterpret_cast<const uint4*>(wb + ((int64_t)r * p.Kp + kel) * ESZ);
            }
        }
    };

    auto store_chunk = [&]() {
        uint8_t* sa = smem;
        uint8_t* sb = smem + BM * ROWB;
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int r = tid / KCC + i * (NT / KCC);
            if constexpr (INT8) {
                const __half2* h = reinterpret_cast<const __half2*>(&areg[i]);
                const float2 f0 = __half22float2(h[0]), f1 = __half22float2(h[1]);
                const float2 f2 = __half22float2(h[2]), f3 = __half22float2(h[3]);
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
            const int cidx = tid + j * NT;
            if (cidx < BCH)
                *reinterpret_cast<uint4*>(sb + (cidx / BCPR) * ROWB + (cidx % BCPR) * 16) = breg[j];
        }
    };

    typedef typename std::conditional<INT8, v4i, v4f>::type acc_t;
    acc_t acc[SI][SJ];
#pragma unroll
    for (int i = 0; i < SI; ++i)
#pragma unroll
        for (int j = 0; j < SJ; ++j) acc[i][j] = acc_t{0, 0, 0, 0};

    if (c_begin < c_end) {
        load_chunk(c_begin);
        store_chunk();
        __syncthreads();
    }
    for (int ch = c_begin; ch < c_end; ++ch) {
        const bool more = ch + 1 < c_end;
        if (more) load_chunk(ch + 1);
        const uint8_t* sa = smem;
        const uint8_t* sb = smem + BM * ROWB;
        const int ksteps = (min(KCH, p.Kp - ch * KCH) + 63) / 64;
        for (int kk = 0; kk < ksteps; ++kk) {
            if constexpr (INT8) {
                v4i a[SI], b[SJ];
#pragma unroll
                for (int i = 0; i < SI; ++i)
                    a[i] = *reinterpret_cast<const v4i*>(sa + (wm * TM + i * 16 + lr) * ROWB + kk * 64 + lg * 16);
#pragma unroll
                for (int j = 0; j < SJ; ++j)
                    b[j] = *reinterpret_cast<const v4i*>(sb + (wn * TN + j * 16 + lr) * ROWB + kk * 64 + lg * 16);
#pragma unroll
                for (int i = 0; i < SI; ++i)
#pragma unroll
                    for (int j = 0; j < SJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
            } else {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    v8h a[SI], b[SJ];
                    const int off = kk * 128 + h * 64 + lg * 16;
#pragma unroll
                    for (int i = 0; i < SI; ++i)
                        a[i] = *reinterpret_cast<const v8h*>(sa + (wm * TM + i * 16 + lr) * ROWB + off);
#pragma unroll
                    for (int j = 0; j < SJ; ++j)
                        b[j] = *reinterpret_cast<const v8h*>(sb + (wn * TN + j * 16 + lr) * ROWB + off);
#pragma unroll
                    for (int i = 0; i < SI; ++i)
#pragma unroll
                        for (int j = 0; j < SJ; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        __syncthreads();
        if (more) {
            store_chunk();
            __syncthreads();
        }
    }

    // ---- split-K: exchange partial tiles through the workspace ----------
    if (p.ksplit > 1) {
        int32_t* ws = reinterpret_cast<int32_t*>(p.ws);
        const int64_t slice = (int64_t)ntiles * BM * BN;
        int32_t* mine = ws + (int64_t)split * slice + (int64_t)tile * BM * BN;
#pragma unroll
        for (int i = 0; i < SI; ++i)
#pragma unroll
            for (int j = 0; j < SJ; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = wm * TM + i * 16 + lg * 4 + r;
                    const int col = wn * TN + j * 16 + lr;
                    int32_t v;
                    if constexpr (INT8) v = acc[i][j][r];
                    else v = __float_as_int(acc[i][j][r]);
                    mine[row * BN + col] = v;
                }
        __threadfence();
        __syncthreads();
        if (tid == 0) {
            const uint32_t prev = atomicAdd(p.counters + tile, 1u);
            last_flag = prev == (uint32_t)(p.ksplit - 1);
        }
        __syncthreads();
        if (!last_flag) return;
        __threadfence();
        if (tid == 0) p.counters[tile] = 0u;  // re-arm for the next run
#pragma unroll
        for (int i = 0; i < SI; ++i)
#pragma unroll
            for (int j = 0; j < SJ; ++j) acc[i][j] = acc_t{0, 0, 0, 0};
        for (int s = 0; s < p.ksplit; ++s) {
            const int32_t* part = ws + (int64_t)s * slice + (int64_t)tile * BM * BN;
#pragma unroll
            for (int i = 0; i < SI; ++i)
#pragma unroll
                for (int j = 0; j < SJ; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int row = wm * TM + i * 16 + lg * 4 + r;
                        const int col = wn * TN + j * 16 + lr;
                        const int32_t v = part[row * BN + col];
                        if constexpr (INT8) acc[i][j][r] += v;
                        else acc[i][j][r] += __int_as_float(v);
                    }
        }
    }

    // ---- epilogue: registers -> LDS (dequant, bias, activation, rounding) ----
    const bool do_silu = p.flags & kConvSilu;
    const bool do_res = p.flags & kConvResidual;
    const bool out_f32 = F32_OK && (p.flags & kConvOutF32);
    const int OUT_ROW = out_f32 ? OUT_ROW32 : OUT_ROW16;
    uint8_t* stage = smem;
#pragma unroll
    for (int j = 0; j < SJ; ++j) {
        const int lcol = wn * TN + j * 16 + lr;
        const int col = n0 + lcol;
        const bool col_ok = col < p.OC;
        float ws = 0.0f, bs = 0.0f;
        if (col_ok) {
            bs = p.bias[col];
            if constexpr (INT8) ws = p.w_scale[col];
        }
#pragma unroll
        for (int i = 0; i < SI; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int lrow = wm * TM + i * 16 + lg * 4 + r;
                float v;
                if constexpr (INT8) {
                    const int32_t a = acc[i][j][r];
                    if (p.acc_out && col_ok && m0 + lrow < p.M) p.acc_out[(int64_t)(m0 + lrow) * p.OC + col] = a;
                    v = (float)a * in_scale;
                    v = v * ws;
                    v = v + bs;
                } else {
                    v = acc[i][j][r] + bs;
                }
                if (do_silu) v = silu(v);
                if (out_f32) *reinterpret_cast<float*>(stage + lrow * OUT_ROW + lcol * 4) = v;
                else *reinterpret_cast<__half*>(stage + lrow * OUT_ROW + lcol * 2) = __float2half(v);
            }
        }
    }
    if (tid < BN / 16) lslots[tid] = 0u;
    __syncthreads();

    // ---- LDS -> global, 8 channels (16 B of fp16 / 32 B of fp32) per item ----
    constexpr int QPR = BN / 8;           // 8-channel items per row
    for (int it = tid; it < BM * QPR; it += NT) {
        const int lrow = it / QPR;
        const int q = it - lrow * QPR;
        const int col0 = n0 + q * 8;
        const int m = m0 + lrow;
        if (m >= p.M || col0 >= p.OC) continue;
        float gmax = 0.0f;
        const int n = m / OHW;
        const int pos = m - n * OHW;
        const int64_t yo = (int64_t)n * p.y_nstride + (int64_t)pos * p.y_cstride + col0;
        float v[8];
        if (out_f32) {
            const float4* s4 = reinterpret_cast<const float4*>(stage + lrow * OUT_ROW + q * 32);
            const float4 a = s4[0], b = s4[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const uint4 u = *reinterpret_cast<const uint4*>(stage + lrow * OUT_ROW + q * 16);
            const __half2* h = reinterpret_cast<const __half2*>(&u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float2 f = __half22float2(h[e]);
                v[2 * e] = f.x;
                v[2 * e + 1] = f.y;
            }
        }
        if (do_res) {
            const uint4 ru = *reinterpret_cast<const uint4*>(p.res + (int64_t)n * p.r_nstride +
                                                             (int64_t)pos * p.r_cstride + col0);
            const __half2* rh = reinterpret_cast<const __half2*>(&ru);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float2 f = __half22float2(rh[e]);
                v[2 * e] += f.x;
                v[2 * e + 1] += f.y;
            }
        }
        if (out_f32) {
            float4* y4 = reinterpret_cast<float4*>(reinterpret_cast<float*>(p.y) + yo);
            y4[0] = make_float4(v[0], v[1], v[2], v[3]);
            y4[1] = make_float4(v[4], v[5], v[6], v[7]);
#pragma unroll
            for (int e = 0; e < 8; ++e) gmax = fmaxf(gmax, fabsf(v[e]));
        } else {
            uint4 o;
            __half2* oh = reinterpret_cast<__half2*>(&o);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                oh[e] = __floats2half2_rn(v[2 * e], v[2 * e + 1]);
                const float2 f = __half22float2(oh[e]);
                gmax = fmaxf(gmax, fmaxf(fabsf(f.x), fabsf(f.y)));
            }
            *reinterpret_cast<uint4*>(reinterpret_cast<__half*>(p.y) + yo) = o;
        }
        if (p.y_slots) atomicMax(&lslots[q >> 1], f2u(gmax));
    }
    if (p.y_slots) {
        __syncthreads();
        if (tid < BN / 16 && n0 + tid * 16 < p.OC && lslots[tid]) slot_max(p.y_slots + (n0 / 16) + tid, u2f(lslots[tid]));
    }
}

template <bool INT8, int BM, int BN, int WM, int WN, int KCH>
hipError_t launch_cfg(const ConvParams& p, hipStream_t stream) {
    const int tiles = ((p.M + BM - 1) / BM) * ((p.OC + BN - 1) / BN);
    hipLaunchKernelGGL((conv_igemm_kernel<INT8, BM, BN, WM, WN, KCH>), dim3(tiles, p.ksplit), dim3(256), 0, stream,
                       p);
    return hipGetLastError();
}

// Tile configs by output channels.  BN covers all channels up to 128 so the
// input tile is read once per output position; K chunks are as large as the
// 64 KB LDS budget and the 16-rows-per-thread staging allow.
template <bool INT8>
hipError_t launch_any(const ConvParams& p, hipStream_t stream) {
    constexpr int K1 = INT8 ? 256 : 128;  // BM + BN <= 224
    constexpr int K2 = INT8 ? 128 : 64;   // BM + BN = 256
    switch (conv_block_n(p.OC, (p.flags & kConvOutF32) != 0)) {
        case 16: return launch_cfg<INT8, 128, 16, 4, 1, K1>(p, stream);
        case 32: return launch_cfg<INT8, 128, 32, 4, 1, K1>(p, stream);
        case 64: return launch_cfg<INT8, 128, 64, 2, 2, K1>(p, stream);
        case 80: return launch_cfg<INT8, 128, 80, 4, 1, K1>(p, stream);
        default: return launch_cfg<INT8, 128, 128, 2, 2, K2>(p, stream);
    }
}

}  // namespace

int conv_block_m() { return 128; }

// Output channels per block: all of them up to 80, else 128 (64 for fp32
// output, whose staging would not fit a 128-wide tile).
int conv_block_n(int oc, bool out_f32) {
    if (oc <= 16) return 16;
    if (oc <= 32) return 32;
    if (oc <= 64) return 64;
    if (oc <= 80) return 80;
    return out_f32 ? 64 : 128;
}

int conv_chunk_k(bool int8, int oc, bool out_f32) {
    const bool big = conv_block_n(oc, out_f32) == 128;
    return int8 ? (big ? 128 : 256) : (big ? 64 : 128);
}

hipError_t launch_conv_igemm(const ConvParams& p, bool int8, hipStream_t stream) {
    if (p.loader != kLoaderNhwc || p.ksplit < 1 || (p.ksplit > 1 && (!p.ws || !p.counters)))
        return hipErrorInvalidValue;
    if (int8) return launch_any<true>(p, stream);
    return launch_any<false>(p, stream);
}

}  // namespace aexrt
