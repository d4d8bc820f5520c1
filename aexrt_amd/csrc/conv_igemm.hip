// Implicit-GEMM convolution on gfx950 MFMA: the W8A8 int8 convolution
// (reference kernels 51/52/53) and the fp16 convolution it falls back to
// (reference kernels 5/43/45 and the fp16 stem/head convs).
//
// GEMM view: out[oc][m] = sum_k W[oc][k] * A[k][m], m = (n, oh, ow) over the
// batch-folded output positions, k = (ky, kx, c) with c fastest so that NHWC
// activations give contiguous k runs.  Weights are repacked at load to
// [OCp][Kp] (OCp = OC rounded up to 16, Kp = K rounded up to 64, zero padded).
//
// The weights are the MFMA's A operand (16 output channels per 16x16 tile)
// and the activations its B operand (16 output positions per tile), so every
// lane ends up holding 4 consecutive output channels of one position: one
// 8-byte NHWC store per lane and tile, no LDS transpose.  Operands go from
// memory straight into MFMA registers: a lane loads the 16 consecutive k of
// its operand row with two 16-byte buffer loads (8 channels of one input
// pixel each); taps that fall into the zero padding get an out-of-range
// buffer offset and read as zero.  There is no LDS staging and no barrier in
// the main loop; each wave owns a 16*PW position x 16*JN channel tile.  For
// maps too small to fill the GPU, the four waves of a block instead split the
// k steps of one tile (KSW) and add their partial tiles through LDS.
//
// int8: the activation fragment is quantized in registers right after its
// load (q = rne(x * 127/amax) & 0xFF, the reference's pack pass RT:3314-3346,
// done by the consumer instead of a separate dispatch), the contraction runs
// on v_mfma_i32_16x16x64_i8 with exact int32 accumulation, and the epilogue
// dequantizes as float(acc) * (amax/127) * w_scale[oc] + bias[oc]
// (RT:4669-4674) before SiLU.  fp16: v_mfma_f32_16x16x32_f16, fp32
// accumulation, + bias, SiLU.  The epilogue adds the residual of a fused
// bottleneck add (RT's BINARY add) and folds max|y| of each 16-channel group
// into the output tensor's amax slots.
#include <algorithm>
#include <atomic>

#include "common.h"
#include "kernels.h"

namespace aexrt {

namespace {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Offset for loads that must read zero: beyond every buffer's num_records
// (<= kMaxViewBytes) even after the compiler folds a small immediate into it.
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    // raw buffer, stride 0, range-checked against num_records (gfx9 dword3)
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4i bload16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// XCD-aware tile order: workgroups are dealt round-robin over the 8 XCDs, so
// block b runs on XCD b % 8.  Give each XCD a contiguous run of tiles so the
// input rows of neighbouring tiles (3x3 halos, the oc tiles of one position
// tile) are fetched into one L2.
__device__ __forceinline__ int xcd_remap(int b, int nb) {
    const int full = (nb / 8) * 8;
    if (b >= full) return b;
    return (b % 8) * (nb / 8) + b / 8;
}

// 8 fp16 -> 8 int8 of the reference quantizer.  x * s is rounded to fp32 and
// then to an integer by adding 1.5 * 2^23: for |x * s| < 2^22 the sum's low
// mantissa bits are exactly rne(x * s) in two's complement, so its low byte
// is the reference's q & 0xFF.  |x| <= amax bounds |x * s| by 127 (+1 ulp);
// NaN keeps a zero low byte, as the saturating float->int cast gives 0.
// Contraction stays off: one fma would round x * s + 1.5 * 2^23 once and
// change the ties.
__device__ __forceinline__ v2i quant8(v4i raw, float s) {
#pragma clang fp contract(off)
    _Float16 h[8];
    __builtin_memcpy(h, &raw, 16);
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = __float_as_uint(((float)h[i] * s) + 12582912.0f);
    v2i o;
    o[0] = (int)((b[0] & 0xFFu) | ((b[1] & 0xFFu) << 8) | ((b[2] & 0xFFu) << 16) | (b[3] << 24));
    o[1] = (int)((b[4] & 0xFFu) | ((b[5] & 0xFFu) << 8) | ((b[6] & 0xFFu) << 16) | (b[7] << 24));
    return o;
}

template <bool INT8>
struct Frag;
template <>
struct Frag<true> {
    static constexpr int wq = 1;  // 16-byte weight pieces per lane and k step
    static constexpr int esz = 1;
};
template <>
struct Frag<false> {
    static constexpr int wq = 2;
    static constexpr int esz = 2;
};

// k steps (64 k each) per weight chunk staged in LDS: 16 KB per buffer, at
// least 4 steps when the 4 waves split the steps of a chunk.
template <bool INT8, int JN, bool KSW>
constexpr int chunk_steps() {
    constexpr int kc = 16384 / (JN * 16 * 64 * Frag<INT8>::esz);
    constexpr int k1 = kc < 1 ? 1 : kc;
    return KSW ? (k1 < 4 ? 4 : k1) : k1;
}

template <bool INT8, int JN, int PW, bool KSW>
__global__ __launch_bounds__(256) void conv_mfma_kernel(ConvParams p) {
    constexpr int WQ = Frag<INT8>::wq;
    constexpr int ESZ = Frag<INT8>::esz;
    constexpr int R = JN * 16;                       // weight rows of the block
    constexpr int KC = chunk_steps<INT8, JN, KSW>();
    constexpr int CH_BYTES = KC * WQ * R * 64;       // one staged weight chunk
    constexpr int ST = CH_BYTES / (256 * 16);        // 16-byte pieces per thread
    static_assert(ST >= 1 && CH_BYTES % (256 * 16) == 0, "chunk split");
    constexpr int RED_BYTES = KSW ? 4 * JN * PW * 4 * 64 * 4 : 0;
    constexpr int LDS_BYTES = 2 * CH_BYTES > RED_BYTES ? 2 * CH_BYTES : RED_BYTES;
    typedef typename std::conditional<INT8, v4i, v4f>::type acc_t;

    // weight chunks: [buf][ks][h][row][64 B]; after the k loop the KSW
    // partial tiles reuse the same memory
    __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];
    __shared__ float l_bias[R], l_scale[R];
    __shared__ uint32_t l_amax, l_slots[JN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 15;  // position within a 16-position subtile
    const int grp = lane >> 4;  // k group (16 k each) / output channel quad

    const int tile = xcd_remap(blockIdx.x, gridDim.x);
    const int mt = (int)fdiv((uint32_t)tile, p.fd_ntn);
    const int n0 = (tile - mt * p.ntn) * R;
    const int pb = KSW ? mt * (16 * PW) : (mt * 4 + wave) * (16 * PW);
    // 16-channel subtiles of this tile that hold real (padded) channels
    const int jmax = min(JN, (p.OCp - n0) >> 4);

    const rsrc_t rx = make_rsrc(p.x, p.x_bytes);
    const rsrc_t rw = make_rsrc(p.w, (uint32_t)p.OCp * (uint32_t)p.Kp * ESZ);

    // ---- block set-up: per-channel constants, input amax, slot partials ----
    if (tid < R) {
        const int oc = n0 + tid;
        l_bias[tid] = oc < p.OC ? p.bias[oc] : 0.0f;
        if constexpr (INT8) l_scale[tid] = oc < p.OC ? p.w_scale[oc] : 0.0f;
    }
    if (tid < JN) l_slots[tid] = 0u;
    if constexpr (INT8) {
        if (tid == 0) l_amax = 0u;
        __syncthreads();
        uint32_t am = 0;
        for (int i = tid; i < p.x_nslots; i += 256) am = max(am, p.x_slots[i]);
        if (am) atomicMax(&l_amax, am);
    }

    // ---- weight chunk staging: global -> registers -> LDS ----
    const int nks = p.Kp >> 6;
    const int nch = (nks + KC - 1) / KC;
    v4i wst[ST];
    auto stage_load = [&](int c) {
#pragma unroll
        for (int i = 0; i < ST; ++i) {
            const int e = tid + i * 256;  // 16-byte piece of the chunk
            const int g = e & 3;
            const int row = (e >> 2) % R;
            const int kh = (e >> 2) / R;  // ks * WQ + h
            const int ks = kh / WQ, h = kh % WQ;
            const int s = c * KC + ks;
            const int oc = n0 + row;
            if (s < nks && oc < p.OCp)
                wst[i] = bload16(rw, (uint32_t)(oc * p.Kp + s * 64) * ESZ + g * 16 * ESZ + h * 16);
            else
                wst[i] = v4i{0, 0, 0, 0};
        }
    };
    auto stage_store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < ST; ++i)
            *reinterpret_cast<v4i*>(lds + buf * CH_BYTES + (tid + i * 256) * 16) = wst[i];
    };

    // ---- activation fragments: direct to registers ----
    int xo[PW], ih0[PW], iw0[PW];
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        const int m = pb + q * 16 + col;
        if (m < p.M) {
            const int n = (int)fdiv((uint32_t)m, p.fd_ohw);
            const int rem = m - n * p.OH * p.OW;
            const int oh = (int)fdiv((uint32_t)rem, p.fd_ow);
            const int ow = rem - oh * p.OW;
            ih0[q] = oh * p.S - p.P;
            iw0[q] = ow * p.S - p.P;
            xo[q] = n * (int)p.x_nstride + (ih0[q] * p.W + iw0[q]) * p.x_cstride;
        } else {
            ih0[q] = -0x40000000;  // every tap out of range
            iw0[q] = 0;
            xo[q] = 0;
        }
    }
    // a[q][h] = 8 channels (16 B fp16) of position subtile q at
    // k = s*64 + grp*16 + h*8; taps in the zero padding read as zero
    auto load_act = [&](int s, v4i (&a)[PW][2]) {
        const int kb = s * 64 + grp * 16;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = kb + h * 8;
            const int tap = (int)fdiv((uint32_t)k, p.fd_c);
            const int c = k - tap * p.C;
            const int ky = (int)fdiv((uint32_t)tap, p.fd_kw);
            const int kx = tap - ky * p.KW;
            const bool kok = k < p.K;
            const int toff = (ky * p.W + kx) * p.x_cstride + c;
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                const int ih = ih0[q] + ky, iw = iw0[q] + kx;
                const bool ok = kok && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
                a[q][h] = bload16(rx, ok ? (uint32_t)(xo[q] + toff) * 2u : kOob);
            }
        }
    };

    acc_t acc[JN][PW];
#pragma unroll
    for (int j = 0; j < JN; ++j)
#pragma unroll
        for (int q = 0; q < PW; ++q) acc[j][q] = acc_t{0, 0, 0, 0};

    float s_q = 0.0f;
    auto mma_step = [&](const v4i (&a)[PW][2], const uint8_t* wl) {
        // wl: this k step's [h][row][64 B] weights in LDS
        if constexpr (INT8) {
            v4i b[PW];
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                const v2i lo = quant8(a[q][0], s_q), hi = quant8(a[q][1], s_q);
                b[q] = v4i{lo[0], lo[1], hi[0], hi[1]};
            }
#pragma unroll
            for (int j = 0; j < JN; ++j) {
                if (j >= jmax) continue;
                const v4i w = *reinterpret_cast<const v4i*>(wl + (j * 16 + col) * 64 + grp * 16);
#pragma unroll
                for (int q = 0; q < PW; ++q)
                    acc[j][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, b[q], acc[j][q], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < JN; ++j) {
                if (j >= jmax) continue;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const v8h w = *reinterpret_cast<const v8h*>(wl + (h * R + j * 16 + col) * 64 + grp * 16);
#pragma unroll
                    for (int q = 0; q < PW; ++q) {
                        v8h xb;
                        __builtin_memcpy(&xb, &a[q][h], 16);
                        acc[j][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, xb, acc[j][q], 0, 0, 0);
                    }
                }
            }
        }
    };

    // ---- main loop over weight chunks, act fragments one step ahead ----
    const int sstep = KSW ? 4 : 1;
    int s = KSW ? wave : 0;
    v4i a_cur[PW][2];
    stage_load(0);
    if (s < nks) load_act(s, a_cur);
    stage_store(0);
    __syncthreads();
    if constexpr (INT8) {
        const float am = u2f(l_amax);
        if (am > 0.0f) s_q = 127.0f / am;
    }
    for (int c = 0; c < nch; ++c) {
        const bool more_w = c + 1 < nch;
        if (more_w) stage_load(c + 1);
        const int s_end = min(nks, (c + 1) * KC);
        const uint8_t* wbuf = lds + (c & 1) * CH_BYTES;
        for (; s < s_end; s += sstep) {
            v4i a_nxt[PW][2];
            const bool more_a = s + sstep < nks;
            if (more_a) load_act(s + sstep, a_nxt);
            mma_step(a_cur, wbuf + (s - c * KC) * WQ * R * 64);
            if (more_a) {
#pragma unroll
                for (int q = 0; q < PW; ++q) {
                    a_cur[q][0] = a_nxt[q][0];
                    a_cur[q][1] = a_nxt[q][1];
                }
            }
        }
        if (more_w) {
            stage_store((c + 1) & 1);
            __syncthreads();
        }
    }

    if constexpr (KSW) {
        // partial tiles of the 4 waves -> LDS; wave w finishes subtiles j % 4 == w
        int32_t* red = reinterpret_cast<int32_t*>(lds);
        __syncthreads();  // every wave is done reading the weight chunks
#pragma unroll
        for (int j = 0; j < JN; ++j)
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int32_t v;
                    if constexpr (INT8) v = acc[j][q][r];
                    else v = __float_as_int(acc[j][q][r]);
                    red[((wave * JN + j) * PW * 4 + q * 4 + r) * 64 + lane] = v;
                }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < JN; ++j) {
            if ((j & 3) != wave) continue;
#pragma unroll
            for (int q = 0; q < PW; ++q)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (INT8) {
                        int32_t t = 0;
#pragma unroll
                        for (int w = 0; w < 4; ++w) t += red[((w * JN + j) * PW * 4 + q * 4 + r) * 64 + lane];
                        acc[j][q][r] = t;
                    } else {
                        float t = 0.0f;
#pragma unroll
                        for (int w = 0; w < 4; ++w)
                            t += __int_as_float(red[((w * JN + j) * PW * 4 + q * 4 + r) * 64 + lane]);
                        acc[j][q][r] = t;
                    }
                }
        }
    }

    // ---- epilogue: dequant, bias, activation, residual, store, amax ----
    float in_scale = 0.0f;
    if constexpr (INT8) {
        const float am = u2f(l_amax);
        if (am > 0.0f) in_scale = am / 127.0f;
    }
    const bool do_silu = p.flags & kConvSilu;
    const bool do_res = p.flags & kConvResidual;
    const bool out_f32 = p.flags & kConvOutF32;
    const rsrc_t ry = make_rsrc(p.y, p.y_bytes);
    const rsrc_t rr = make_rsrc(p.res, p.r_bytes);
    int yo[PW], ro[PW];
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        const int m = pb + q * 16 + col;
        if (m < p.M) {
            const int n = (int)fdiv((uint32_t)m, p.fd_ohw);
            const int pos = m - n * p.OH * p.OW;
            yo[q] = n * (int)p.y_nstride + pos * p.y_cstride;
            ro[q] = n * (int)p.r_nstride + pos * p.r_cstride;
        } else {
            yo[q] = -1;
            ro[q] = 0;
        }
    }
#pragma unroll
    for (int j = 0; j < JN; ++j) {
        if (j >= jmax) continue;
        if (KSW && (j & 3) != wave) continue;
        const int lc = j * 16 + grp * 4;  // block-local channel of this lane's quad
        const int oc0 = n0 + lc;
        const bool oc_ok = oc0 < p.OC;  // OC % 4 == 0: the quad is all in or all out
        // residual fragments first, so their latency overlaps the arithmetic
        v2i rv[PW];
#pragma unroll
        for (int q = 0; q < PW; ++q)
            rv[q] = do_res ? __builtin_amdgcn_raw_buffer_load_b64(
                                 rr, oc_ok && yo[q] >= 0 ? (uint32_t)(ro[q] + oc0) * 2u : kOob, 0, 0)
                           : v2i{0, 0};
        float bv[4], wv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            bv[r] = l_bias[lc + r];
            wv[r] = INT8 ? l_scale[lc + r] : 0.0f;
        }
        float gmax = 0.0f;
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            if (!oc_ok || yo[q] < 0) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
#pragma clang fp contract(off)
                float t;
                if constexpr (INT8) {
                    t = (float)acc[j][q][r] * in_scale;
                    t = t * wv[r];
                    t = t + bv[r];
                } else {
                    t = acc[j][q][r] + bv[r];
                }
                if (do_silu) t = silu(t);
                v[r] = t;
            }
            if constexpr (INT8) {
                if (p.acc_out)
                    *reinterpret_cast<int4*>(p.acc_out + (int64_t)(pb + q * 16 + col) * p.OC + oc0) =
                        make_int4(acc[j][q][0], acc[j][q][1], acc[j][q][2], acc[j][q][3]);
            }
            __half2 rh[2];
            __builtin_memcpy(rh, &rv[q], 8);
            if (out_f32) {
                if (do_res) {
                    const float2 r0 = __half22float2(rh[0]), r1 = __half22float2(rh[1]);
                    v[0] += r0.x; v[1] += r0.y; v[2] += r1.x; v[3] += r1.y;
                }
                v4i o;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    o[r] = __float_as_int(v[r]);
                    gmax = fmaxf(gmax, fabsf(v[r]));
                }
                __builtin_amdgcn_raw_buffer_store_b128(o, ry, (uint32_t)(yo[q] + oc0) * 4u, 0, 0);
            } else {
                __half2 oh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                if (do_res) {
                    // fp16 conv output + fp16 residual, added in fp32 and
                    // rounded again: the reference's separate BINARY add
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const float2 a = __half22float2(oh[e]), b = __half22float2(rh[e]);
                        oh[e] = __floats2half2_rn(a.x + b.x, a.y + b.y);
                    }
                }
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float2 f = __half22float2(oh[e]);
                    gmax = fmaxf(gmax, fmaxf(fabsf(f.x), fabsf(f.y)));
                }
                v2i o;
                __builtin_memcpy(&o, oh, 8);
                __builtin_amdgcn_raw_buffer_store_b64(o, ry, (uint32_t)(yo[q] + oc0) * 2u, 0, 0);
            }
        }
        if (p.y_slots) {
            gmax = wave_max(gmax);
            if (lane == 0 && gmax > 0.0f) atomicMax(&l_slots[j], f2u(gmax));
        }
    }
    // one global amax update per 16-channel group and block
    if (p.y_slots) {
        __syncthreads();
        if (tid < jmax && n0 + tid * 16 < p.OC && l_slots[tid]) slot_max(p.y_slots + (n0 >> 4) + tid, u2f(l_slots[tid]));
    }
}

template <bool INT8, int JN, int PW, bool KSW>
hipError_t launch_cfg(const ConvParams& p, int blocks, hipStream_t stream) {
    hipLaunchKernelGGL((conv_mfma_kernel<INT8, JN, PW, KSW>), dim3(blocks), dim3(256), 0, stream, p);
    return hipGetLastError();
}

template <bool INT8>
hipError_t launch_any(const ConvParams& p, const ConvTile& t, int blocks, hipStream_t stream) {
    if (t.ksw) {
        switch (t.jn) {
            case 1: return launch_cfg<INT8, 1, 1, true>(p, blocks, stream);
            case 2: return launch_cfg<INT8, 2, 1, true>(p, blocks, stream);
            case 4: return launch_cfg<INT8, 4, 1, true>(p, blocks, stream);
            case 8: return launch_cfg<INT8, 8, 1, true>(p, blocks, stream);
        }
        return hipErrorInvalidValue;
    }
    switch (t.jn * 8 + t.pw) {
        case 1 * 8 + 1: return launch_cfg<INT8, 1, 1, false>(p, blocks, stream);
        case 1 * 8 + 2: return launch_cfg<INT8, 1, 2, false>(p, blocks, stream);
        case 1 * 8 + 4: return launch_cfg<INT8, 1, 4, false>(p, blocks, stream);
        case 2 * 8 + 1: return launch_cfg<INT8, 2, 1, false>(p, blocks, stream);
        case 2 * 8 + 2: return launch_cfg<INT8, 2, 2, false>(p, blocks, stream);
        case 2 * 8 + 4: return launch_cfg<INT8, 2, 4, false>(p, blocks, stream);
        case 4 * 8 + 1: return launch_cfg<INT8, 4, 1, false>(p, blocks, stream);
        case 4 * 8 + 2: return launch_cfg<INT8, 4, 2, false>(p, blocks, stream);
        case 4 * 8 + 4: return launch_cfg<INT8, 4, 4, false>(p, blocks, stream);
        case 8 * 8 + 1: return launch_cfg<INT8, 8, 1, false>(p, blocks, stream);
        case 8 * 8 + 2: return launch_cfg<INT8, 8, 2, false>(p, blocks, stream);
    }
    return hipErrorInvalidValue;
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
// 16-channel subtiles; its weight chunks are staged once in LDS for all 4
// waves, each wave streams its own positions.  Cover all output channels (up
// to 128) so activations are read once, take the most positions per wave that
// still gives >= 2 blocks per CU, and for maps too small for that shrink the
// channel tile, then let the 4 waves of a block split k (one position subtile
// per block).
ConvTile choose_conv_tile(int M, int OC, int Kp) {
    const int ov = g_tile_override.load(std::memory_order_relaxed);
    if (ov) return ConvTile{(ov - 1) / 100, ((ov - 1) / 10) % 10, ((ov - 1) % 10) != 0};
    const int ocj = (OC + 15) / 16;
    const int nks = Kp / 64;
    const int64_t want = 512;
    auto blocks = [&](int jn, int pw, bool ksw) {
        return (int64_t)((M + (ksw ? 16 : 64) * pw - 1) / ((ksw ? 16 : 64) * pw)) * ((ocj + jn - 1) / jn);
    };
    const int jn0 = pow2_at_least(ocj, 8);
    for (int pw = 4; pw >= 1; pw >>= 1) {
        const ConvTile t{jn0, pw, false};
        if (tile_instantiated(t) && blocks(jn0, pw, false) >= want) return t;
    }
    int jn = jn0;
    while (jn > 1 && blocks(jn, 1, false) < want) jn >>= 1;
    if (blocks(jn, 1, false) >= want / 2 || nks < 4) return ConvTile{jn, 1, false};
    // small map: one position subtile per block, k split over the 4 waves
    jn = jn0;
    while (jn > 1 && blocks(jn, 1, true) < want) jn >>= 1;
    return ConvTile{jn, 1, true};
}

hipError_t launch_conv_igemm(const ConvParams& p0, bool int8, hipStream_t stream) {
    if (p0.loader != kLoaderNhwc || p0.OC % 4 || p0.C % 8 || p0.Kp % 64 || p0.OCp % 16) return hipErrorInvalidValue;
    const ConvTile t = choose_conv_tile(p0.M, p0.OC, p0.Kp);
    const bool out_f32 = (p0.flags & kConvOutF32) != 0;
    const int HWi = p0.H * p0.W, HWo = p0.OH * p0.OW;
    // Images per launch: every view a launch touches must stay inside
    // kMaxViewBytes so the kernel can address it with 32-bit offsets.
    const uint64_t per_img = std::max({(uint64_t)p0.x_nstride * 2, (uint64_t)p0.y_nstride * (out_f32 ? 4 : 2),
                                       p0.res ? (uint64_t)p0.r_nstride * 2 : 0,
                                       p0.acc_out ? (uint64_t)HWo * p0.OC * 4 : 0,
                                       (uint64_t)HWi * p0.x_cstride * 2});
    if ((uint64_t)p0.OCp * p0.Kp * 2 > kMaxViewBytes || per_img == 0) return hipErrorInvalidValue;
    const int per_launch = (int)std::min<uint64_t>((uint64_t)p0.N, kMaxViewBytes / per_img);
    if (per_launch < 1) return hipErrorInvalidValue;
    for (int nb = 0; nb < p0.N; nb += per_launch) {
        ConvParams p = p0;
        p.N = std::min(per_launch, p0.N - nb);
        p.M = p.N * HWo;
        p.x = static_cast<const __half*>(p0.x) + (int64_t)nb * p0.x_nstride;
        p.y = static_cast<char*>(p0.y) + (int64_t)nb * p0.y_nstride * (out_f32 ? 4 : 2);
        if (p0.res) p.res = p0.res + (int64_t)nb * p0.r_nstride;
        if (p0.acc_out) p.acc_out = p0.acc_out + (int64_t)nb * HWo * p0.OC;
        p.x_bytes = (uint32_t)view_span(p.N, p.x_nstride, p.x_cstride, HWi, p.C, 2);
        p.y_bytes = (uint32_t)view_span(p.N, p.y_nstride, p.y_cstride, HWo, p.OC, out_f32 ? 4 : 2);
        p.r_bytes = p.res ? (uint32_t)view_span(p.N, p.r_nstride, p.r_cstride, HWo, p.OC, 2) : 0u;
        p.ntn = (p.OCp / 16 + t.jn - 1) / t.jn;
        const int mtile = (t.ksw ? 16 : 64) * t.pw;
        const int mtiles = (p.M + mtile - 1) / mtile;
        p.fd_ntn = make_fastdiv((uint32_t)p.ntn);
        p.fd_ohw = make_fastdiv((uint32_t)HWo);
        p.fd_ow = make_fastdiv((uint32_t)p.OW);
        p.fd_c = make_fastdiv((uint32_t)p.C);
        p.fd_kw = make_fastdiv((uint32_t)p.KW);
        const int64_t blocks = (int64_t)mtiles * p.ntn;
        if (blocks > INT32_MAX) return hipErrorInvalidValue;
        const hipError_t e = int8 ? launch_any<true>(p, t, (int)blocks, stream)
                                  : launch_any<false>(p, t, (int)blocks, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace aexrt
