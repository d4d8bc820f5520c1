// Implicit-GEMM convolution kernel on gfx950 MFMA: the W8A8 int8 convolution
// (reference kernels 51/52/53) and the fp16 convolution it falls back to
// (reference kernels 5/43/45 and the fp16 stem/head convs).  Included by the
// instance files conv_i8*.hip / conv_f16*.hip; the host side (tile choice,
// batch splitting) is conv_igemm.hip.
//
// GEMM view: out[oc][m] = sum_k W[oc][k] * A[k][m], m = (n, oh, ow) over the
// batch-folded output positions, k = (ky, kx, c) with c fastest so that NHWC
// activations give contiguous k runs.  Weights are repacked at load to
// [OCp][Kp] (OCp = OC rounded up to 16, Kp = K rounded up to 64, zero padded).
//
// The weights are the MFMA's A operand (16 output channels per 16x16 tile)
// and the activations its B operand (16 output positions per tile), so every
// lane ends up holding 4 consecutive output channels of one position: one
// 8-byte NHWC store per lane and tile, no LDS transpose.  Activations go from
// memory straight into MFMA registers: a lane loads the 16 consecutive k of
// its operand row with two 16-byte buffer loads (8 channels of one input
// pixel each); taps in the zero padding get an out-of-range buffer offset and
// read as zero, so every load is issued unconditionally and the compiler can
// keep a fixed number of them in flight.  The block's weights are staged in
// LDS (once, when they fit one 16 KB chunk) and shared by its 4 waves.
//
// A block keeps one output-channel tile and walks a contiguous run of
// position tiles (4 waves x PW 16-position subtiles each); neighbouring
// tiles share their 3x3 halo rows in L2.  For maps too small to fill the GPU
// the 4 waves of a block instead split the k steps of one tile (KSW) and add
// their partial tiles through LDS.
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
#pragma once
#include <algorithm>
#include <atomic>

#include "common.h"
#include "kernels.h"

namespace aexrt {
namespace igemm {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Offset for loads that must read zero: beyond every buffer's num_records
// (<= kMaxViewBytes) even after the compiler folds a small immediate into it.
constexpr uint32_t kOob = 0x80000000u;
// Largest k-step count (64 k each) of one conv: the per-block tap table.
constexpr int kMaxSteps = 128;
// Largest stripes x slots of an int8 input view (8 slot loads per lane).
constexpr int kMaxSlotReads = 512;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    // raw buffer, stride 0, range-checked against num_records (gfx9 dword3)
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4i bload16(rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

using ::aexrt::xcd_remap;

// fp32 product of the fp16 in the low / high half of h2 and s, rounded once:
// v_fma_mix with a -0 addend is exactly RN(x * s) (x converted exactly).
__device__ __forceinline__ float mul_f16lo(uint32_t h2, float s) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s), "v"(0x80000000u));
    return r;
}
__device__ __forceinline__ float mul_f16hi(uint32_t h2, float s) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s), "v"(0x80000000u));
    return r;
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
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        b[2 * i] = __float_as_uint(mul_f16lo((uint32_t)raw[i], s) + 12582912.0f);
        b[2 * i + 1] = __float_as_uint(mul_f16hi((uint32_t)raw[i], s) + 12582912.0f);
    }
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

// ---- input scale of an int8 conv -------------------------------------------
// The stripes x slots of the input view are spread over the lanes of each
// wave (8 loads per lane, issued early), then reduced: amax = max over all
// copies and groups, the reference's per-tensor activation scale.
__device__ __forceinline__ void in_slot_loads(const ConvParams& p, int lane, uint32_t (&raw)[kMaxSlotReads / 64]) {
    const rsrc_t rs = make_rsrc(p.x_slots.p, p.x_slot_bytes);
    const int ns = p.x_nslots;
    const int tot = (int)p.x_slots.stripes * ns;
#pragma unroll
    for (int r = 0; r < kMaxSlotReads / 64; ++r) {
        const int e = lane + r * 64;
        const int c = (int)fdiv((uint32_t)e, p.fd_ns);
        raw[r] = __builtin_amdgcn_raw_buffer_load_b32(
            rs, e < tot ? ((uint32_t)c * p.x_slots.stride + (uint32_t)(e - c * ns)) * 4u : kOob, 0, 0);
    }
}
// Slot words of an upsampled input source (ConvParams::xup): up to
// kMaxUpSlotReads (stripes x groups), spread over the lanes as above.
constexpr int kMaxUpSlotReads = 256;
__device__ __forceinline__ void up_slot_loads(const ConvParams& p, uint32_t slot_bytes, FastDiv fd_ns, int lane,
                                              uint32_t (&raw)[kMaxUpSlotReads / 64]) {
    const rsrc_t rs = make_rsrc(p.xup_slots.p, slot_bytes);
    const int ns = p.xup_nslots;
    const int tot = (int)p.xup_slots.stripes * ns;
#pragma unroll
    for (int r = 0; r < kMaxUpSlotReads / 64; ++r) {
        const int e = lane + r * 64;
        const int c = (int)fdiv((uint32_t)e, fd_ns);
        raw[r] = __builtin_amdgcn_raw_buffer_load_b32(
            rs, e < tot ? ((uint32_t)c * p.xup_slots.stride + (uint32_t)(e - c * ns)) * 4u : kOob, 0, 0);
    }
}
// s_q = 127 / amax (quantizer), in_scale = amax / 127 (dequant); both 0 for
// an all-zero input, whose quantized values are then all 0.
__device__ __forceinline__ void in_slot_scale(const uint32_t (&raw)[kMaxSlotReads / 64], float& s_q,
                                              float& in_scale, uint32_t also = 0u) {
    uint32_t am = also;  // also: slot words of further input channels this lane read
#pragma unroll
    for (int r = 0; r < kMaxSlotReads / 64; ++r) am = max(am, raw[r]);
    const float a_max = u2f(wave_umax(am));
    s_q = 0.0f;
    in_scale = 0.0f;
    if (a_max > 0.0f) {
        s_q = 127.0f / a_max;
        in_scale = a_max / 127.0f;
    }
}

// ---- output side of a tile, shared by the conv kernels ---------------------
// A lane holds, for each 16-channel subtile j and 16-position subtile q,
// acc[j][q][r] = channel n0 + 16j + 4*grp + r of one output position; yo[q]
// is that position's element offset in the output view (-1: none), ro[q] in
// the residual view, mo[q] its row in acc_out.  jmask: subtiles this wave
// stores.  Every lane issues every load/store (invalid ones at the
// out-of-range offset, which the hardware drops), so the number of memory
// operations in flight is the same on all paths.

enum Epi : int {
    kEpiAny = 0,      // flags read at run time (fp32 output, no SiLU, ...)
    kEpiSilu = 1,     // SiLU, fp16 output
    kEpiSiluRes = 2,  // SiLU, + residual, fp16 output
};

template <int EPI>
__device__ __forceinline__ bool epi_res(const ConvParams& p) {
    return EPI == kEpiSiluRes || (EPI == kEpiAny && (p.flags & kConvResidual));
}

template <int JN, int PW, int EPI>
__device__ __forceinline__ void tile_residual(const ConvParams& p, const rsrc_t& rr, const int (&yo)[PW],
                                              const int (&ro)[PW], int n0, int jmax, int grp, uint32_t jmask,
                                              v2i (&rv)[JN][PW]) {
    if (!epi_res<EPI>(p)) return;
#pragma unroll
    for (int j = 0; j < JN; ++j)
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const int oc0 = n0 + j * 16 + grp * 4;
            const bool ok = j < jmax && ((jmask >> j) & 1u) && oc0 < p.OC && yo[q] >= 0;
            rv[j][q] = __builtin_amdgcn_raw_buffer_load_b64(rr, ok ? (uint32_t)(ro[q] + oc0) * 2u : kOob, 0, 0);
        }
}

// Output values of one lane's 4 channels: dequant (int8), bias, SiLU and the
// residual (fp16 conv output + fp16 residual added in fp32, the reference's
// separate BINARY add; with fp32 output the residual is added unrounded).
template <bool INT8, int EPI, typename AccT>
__device__ __forceinline__ void epi_values(const ConvParams& p, const AccT& acc, const float (&bv)[4],
                                           const float (&wv)[4], const v2i& rv, float (&v)[4]) {
    const bool do_silu = EPI != kEpiAny || (p.flags & kConvSilu);
    const bool do_res = epi_res<EPI>(p);
    const bool out_f32 = EPI == kEpiAny && (p.flags & kConvOutF32);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float t;
        if constexpr (INT8) t = __builtin_fmaf((float)acc[r], wv[r], bv[r]);
        else t = acc[r] + bv[r];
        if (do_silu) t = silu(t);
        v[r] = t;
    }
    if (do_res) {
        __half2 rh[2];
        __builtin_memcpy(rh, &rv, 8);
        const float2 r0 = __half22float2(rh[0]), r1 = __half22float2(rh[1]);
        if (out_f32) {
            v[0] += r0.x; v[1] += r0.y; v[2] += r1.x; v[3] += r1.y;
        } else {
            v[0] = __half2float(__float2half(v[0])) + r0.x;
            v[1] = __half2float(__float2half(v[1])) + r0.y;
            v[2] = __half2float(__float2half(v[2])) + r1.x;
            v[3] = __half2float(__float2half(v[3])) + r1.y;
        }
    }
}

// Dequant (int8: one fma with the factor amax/127 * w_scale[oc] in l_scale),
// bias, SiLU, residual, store, and the running max|y| per channel subtile
// (fp32 before rounding: fp16 rounding is monotone, so it commutes with max).
template <bool INT8, int JN, int PW, int EPI, typename AccT>
__device__ __forceinline__ void tile_store(const ConvParams& p, const AccT (&acc)[JN][PW], const int (&yo)[PW],
                                           const int (&mo)[PW], const v2i (&rv)[JN][PW], int n0, int jmax,
                                           int grp, uint32_t jmask, const float* l_bias, const float* l_scale,
                                           float (&gmax)[JN], const rsrc_t& ry, const rsrc_t& racc) {
    const bool do_silu = EPI != kEpiAny || (p.flags & kConvSilu);
    const bool do_res = epi_res<EPI>(p);
    const bool out_f32 = EPI == kEpiAny && (p.flags & kConvOutF32);
#pragma unroll
    for (int j = 0; j < JN; ++j) {
        if (j >= jmax || !((jmask >> j) & 1u)) continue;
        const int lc = j * 16 + grp * 4;  // block-local channel of this lane's quad
        const int oc0 = n0 + lc;
        const bool oc_ok = oc0 < p.OC;  // OC % 4 == 0: the quad is all in or all out
        float bv[4], wv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            bv[r] = l_bias[lc + r];
            wv[r] = INT8 ? l_scale[lc + r] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const bool ok = oc_ok && yo[q] >= 0;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float t;
                if constexpr (INT8) t = __builtin_fmaf((float)acc[j][q][r], wv[r], bv[r]);
                else t = acc[j][q][r] + bv[r];
                if (do_silu) t = silu(t);
                v[r] = t;
            }
            if constexpr (INT8) {
                if (p.acc_out) {
                    const v4i av{(int)acc[j][q][0], (int)acc[j][q][1], (int)acc[j][q][2], (int)acc[j][q][3]};
                    __builtin_amdgcn_raw_buffer_store_b128(av, racc, ok ? (uint32_t)(mo[q] * p.OC + oc0) * 4u : kOob,
                                                           0, 0);
                }
            }
            __half2 rh[2];
            __builtin_memcpy(rh, &rv[j][q], 8);
            if (out_f32) {
                if (do_res) {
                    const float2 r0 = __half22float2(rh[0]), r1 = __half22float2(rh[1]);
                    v[0] += r0.x; v[1] += r0.y; v[2] += r1.x; v[3] += r1.y;
                }
                v4i o;
#pragma unroll
                for (int r = 0; r < 4; ++r) o[r] = __float_as_int(v[r]);
                const float m4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
                gmax[j] = fmaxf(gmax[j], ok ? m4 : 0.0f);
                __builtin_amdgcn_raw_buffer_store_b128(o, ry, ok ? (uint32_t)(yo[q] + oc0) * 4u : kOob, 0, 0);
            } else {
                __half2 oh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                if (do_res) {
                    // fp16 conv output + fp16 residual, added in fp32 and
                    // rounded again: the reference's separate BINARY add
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const float2 fa = __half22float2(oh[e]), fb = __half22float2(rh[e]);
                        v[2 * e] = fa.x + fb.x;
                        v[2 * e + 1] = fa.y + fb.y;
                        oh[e] = __floats2half2_rn(v[2 * e], v[2 * e + 1]);
                    }
                }
                const float m4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
                gmax[j] = fmaxf(gmax[j], ok ? m4 : 0.0f);
                v2i o;
                __builtin_memcpy(&o, oh, 8);
                __builtin_amdgcn_raw_buffer_store_b64(o, ry, ok ? (uint32_t)(yo[q] + oc0) * 2u : kOob, 0, 0);
            }
        }
    }
}

// Block-wide end of a conv launch: one atomic per 16-channel group into this
// block's copy of the output slots (no read first: with the copies striped
// over the blocks the atomics hardly contend, and one without a return value
// ends the block without waiting for its round trip).
template <int JN>
__device__ __forceinline__ void flush_slots(const ConvParams& p, float (&gmax)[JN], int n0, int jmax, uint32_t jmask,
                                            bool out_f32, uint32_t* l_slots) {
    if (!p.y_slots.p) return;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < JN; ++j) {
        if (j >= jmax || !((jmask >> j) & 1u)) continue;
        // the stored values are fp16 (fp32 for fp32 output)
        const float g = wave_max(out_f32 ? gmax[j] : __half2float(__float2half(gmax[j])));
        if (lane == 0 && g > 0.0f) atomicMax(&l_slots[j], f2u(g));
    }
    __syncthreads();
    const int tid = threadIdx.x;
    if (tid < jmax && n0 + tid * 16 < p.OC && l_slots[tid])
        atomicMax(slot_copy(p.y_slots, blockIdx.x) + (n0 >> 4) + tid, l_slots[tid]);
}

// MC: the weights span more than one chunk (staged chunk by chunk, double
// buffered); otherwise they are staged once for all tiles of the block.
template <bool INT8, int JN, int PW, bool KSW, bool MC, int EPI>
__global__ __launch_bounds__(256) void conv_mfma_kernel(ConvParams p) {
    constexpr int WQ = Frag<INT8>::wq;
    constexpr int ESZ = Frag<INT8>::esz;
    constexpr int R = JN * 16;                       // weight rows of the block
    constexpr int KC = chunk_steps<INT8, JN, KSW>();
    constexpr int CH_BYTES = KC * WQ * R * 64;       // one staged weight chunk
    constexpr int NBUF = MC ? 2 : 1;
    constexpr int ST = CH_BYTES / (256 * 16);        // 16-byte pieces per thread
    static_assert(ST >= 1 && CH_BYTES % (256 * 16) == 0, "chunk split");
    constexpr int RED_BYTES = KSW ? 4 * JN * PW * 4 * 64 * 4 : 0;
    constexpr int LDS_BYTES = NBUF * CH_BYTES > RED_BYTES ? NBUF * CH_BYTES : RED_BYTES;
    constexpr int TPOS = (KSW ? 16 : 64) * PW;       // output positions per tile
    constexpr int D = PW == 1 ? 4 : 2;               // k iterations of activations in flight
    typedef typename std::conditional<INT8, v4i, v4f>::type acc_t;

    // weight chunks: [buf][ks][h][row][64 B]; a KSW block (one tile) reuses
    // the memory for its partial tiles after the k loop
    __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];
    // tap table: (k step, k group, half) -> element offset of the tap and
    // channel, and ky | kx << 8 | (k < K) << 16
    __shared__ int2 l_tap[kMaxSteps * 8];
    __shared__ float l_bias[R], l_scale[R];
    __shared__ uint32_t l_slots[JN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 15;  // position within a 16-position subtile
    const int grp = lane >> 4;  // k group (16 k each) / output channel quad

    const int b = xcd_remap(blockIdx.x, gridDim.x);
    const int pg = (int)fdiv((uint32_t)b, p.fd_ntn);
    const int n0 = (b - pg * p.ntn) * R;
    const int pt0 = pg * p.per;
    const int ntl = min(p.per, p.npt - pt0);
    // 16-channel subtiles of this tile that hold real (padded) channels
    const int jmax = min(JN, (p.OCp - n0) >> 4);
    const int nks = p.Kp >> 6;
    const int nch = (nks + KC - 1) / KC;

    const rsrc_t rx = make_rsrc(p.x, p.x_bytes);
    const rsrc_t rw = make_rsrc(p.w, (uint32_t)p.OCp * (uint32_t)p.Kp * ESZ);

    // ---- activation fragments ----------------------------------------------
    // Position data of the tile most recently loaded for (loads go in tile
    // order, so it changes at most once per tile).
    int pos_tl = -1;
    int xo[PW], ih0[PW], iw0[PW];
    auto set_tile = [&](int tl) {
        const int pb = (pt0 + tl) * TPOS + (KSW ? 0 : wave * 16 * PW);
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const int m = pb + q * 16 + col;
            const bool mok = m < p.M;
            if (p.lin & kLinX) {
                // 1x1 s1 on a dense view: input pixel m, no padding taps
                ih0[q] = mok ? 0 : -0x40000000;
                iw0[q] = 0;
                xo[q] = (int)__umul24((uint32_t)m, (uint32_t)p.x_cstride);
            } else {
                const int n = (int)fdiv((uint32_t)m, p.fd_ohw);
                const int rem = m - n * p.OH * p.OW;
                const int oh = (int)fdiv((uint32_t)rem, p.fd_ow);
                const int ow = rem - oh * p.OW;
                ih0[q] = mok ? oh * p.S - p.P : -0x40000000;  // out of range for every tap
                iw0[q] = ow * p.S - p.P;
                xo[q] = n * (int)p.x_nstride + ((oh * p.S - p.P) * p.W + iw0[q]) * p.x_cstride;
            }
        }
        pos_tl = tl;
    };
    // a[q][h] = 8 channels (16 B fp16) of position subtile q of flattened
    // iteration i (tile i / nit, k step s0 + (i % nit) * sstep) at
    // k = s*64 + grp*16 + h*8.  Always issues its 2*PW loads.
    const int sstep = KSW ? 4 : 1;
    const int s0 = KSW ? wave : 0;
    const int nit = (nks + sstep - 1) / sstep;  // iterations per tile
    const int total = ntl * nit;
    // Tap of (k step s, half h) of this lane's k group: element offset of the
    // tap and channel, and ky | kx << 8 | (k < K) << 16.
    auto tap_of = [&](int s, int h) {
        const int k = s * 64 + grp * 16 + h * 8;
        const int tap = (int)fdiv((uint32_t)k, p.fd_c);
        const int c = k - tap * p.C;
        const int ky = (int)fdiv((uint32_t)tap, p.fd_kw);
        const int kx = tap - ky * p.KW;
        return k < p.K ? make_int2((ky * p.W + kx) * p.x_cstride + c, ky | (kx << 8) | (1 << 16)) : make_int2(0, 0);
    };
    // direct: compute the taps instead of reading the block's LDS table (the
    // prologue's loads go out before the table exists)
    auto load_act = [&](int i, v4i (&a)[PW][2], bool direct) {
        const int tl = (int)fdiv((uint32_t)i, p.fd_nit);
        const int s = s0 + (i - tl * nit) * sstep;
        const bool iok = i < total && s < nks;
        if (tl != pos_tl) set_tile(tl);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int2 e = direct ? tap_of(min(s, nks - 1), h) : l_tap[(min(s, nks - 1) * 4 + grp) * 2 + h];
            const int ky = e.y & 0xFF, kx = (e.y >> 8) & 0xFF;
            const bool kok = iok && (e.y >> 16) != 0;
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                const int ih = ih0[q] + ky, iw = iw0[q] + kx;
                const bool ok = kok && (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
                a[q][h] = bload16(rx, ok ? (uint32_t)(xo[q] + e.x) * 2u : kOob);
            }
        }
    };

    // ---- weight chunk staging: global -> registers -> LDS ------------------
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
            wst[i] = bload16(rw, s < nks && oc < p.OCp
                                     ? (uint32_t)(oc * p.Kp + s * 64) * ESZ + g * 16 * ESZ + h * 16
                                     : kOob);
        }
    };
    auto stage_store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < ST; ++i)
            *reinterpret_cast<v4i*>(lds + buf * CH_BYTES + (tid + i * 256) * 16) = wst[i];
    };

    // ---- prologue: every independent load goes out first (slots, per-channel
    // constants, weights, the first activations), then the waits, in issue
    // order, so the block pays one memory latency before its first MFMA ----
    uint32_t slot_raw[kMaxSlotReads / 64];
    if constexpr (INT8) in_slot_loads(p, lane, slot_raw);
    const rsrc_t rb = make_rsrc(p.bias, (uint32_t)p.OC * 4u);
    const rsrc_t rsc = make_rsrc(p.w_scale, INT8 ? (uint32_t)p.OC * 4u : 0u);
    const uint32_t cofs = tid < R && n0 + tid < p.OC ? (uint32_t)(n0 + tid) * 4u : kOob;
    const float bias_v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, cofs, 0, 0));
    float scale_v = 0.0f;
    if constexpr (INT8) scale_v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsc, cofs, 0, 0));
    stage_load(0);
    v4i a[D][PW][2];
#pragma unroll
    for (int d = 0; d < D; ++d) load_act(d, a[d], true);
    // tap table for the later iterations (ALU only)
    for (int e = tid; e < nks * 8; e += 256) {
        const int s = e >> 3, g = (e >> 1) & 3, h = e & 1;
        const int k = s * 64 + g * 16 + h * 8;
        const int tap = (int)fdiv((uint32_t)k, p.fd_c);
        const int c = k - tap * p.C;
        const int ky = (int)fdiv((uint32_t)tap, p.fd_kw);
        const int kx = tap - ky * p.KW;
        l_tap[e] = k < p.K ? make_int2((ky * p.W + kx) * p.x_cstride + c, ky | (kx << 8) | (1 << 16))
                           : make_int2(0, 0);
    }
    if (tid < JN) l_slots[tid] = 0u;
    float s_q = 0.0f, in_scale = 0.0f;
    if constexpr (INT8) in_slot_scale(slot_raw, s_q, in_scale);
    if (tid < R) {
        l_bias[tid] = bias_v;
        // dequant factor amax/127 * w_scale[oc], applied as one fma (the
        // reference multiplies twice; the two differ in the last fp32 bit at
        // most, far inside the fp16 output's rounding)
        if constexpr (INT8) l_scale[tid] = in_scale * scale_v;
    }
    stage_store(0);
    __syncthreads();
    if constexpr (MC) stage_load(1 < nch ? 1 : 0);

    acc_t acc[JN][PW];
#pragma unroll
    for (int j = 0; j < JN; ++j)
#pragma unroll
        for (int q = 0; q < PW; ++q) acc[j][q] = acc_t{0, 0, 0, 0};

    auto mma_step = [&](const v4i (&af)[PW][2], const uint8_t* wl) {
        // wl: this k step's [h][row][64 B] weights in LDS
        if constexpr (INT8) {
            v4i bq[PW];
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                const v2i lo = quant8(af[q][0], s_q), hi = quant8(af[q][1], s_q);
                bq[q] = v4i{lo[0], lo[1], hi[0], hi[1]};
            }
            // every subtile runs, also past the conv's channels (zero weights
            // there, never stored): no branches between the MFMAs
#pragma unroll
            for (int j = 0; j < JN; ++j) {
                const v4i w = *reinterpret_cast<const v4i*>(wl + (j * 16 + col) * 64 + grp * 16);
#pragma unroll
                for (int q = 0; q < PW; ++q)
                    acc[j][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, bq[q], acc[j][q], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < JN; ++j) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const v8h w = *reinterpret_cast<const v8h*>(wl + (h * R + j * 16 + col) * 64 + grp * 16);
#pragma unroll
                    for (int q = 0; q < PW; ++q) {
                        v8h xb;
                        __builtin_memcpy(&xb, &af[q][h], 16);
                        acc[j][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, xb, acc[j][q], 0, 0, 0);
                    }
                }
            }
        }
    };

    // ---- epilogue of one tile ------------------------------------------------
    const bool out_f32 = EPI == kEpiAny && (p.flags & kConvOutF32);
    const rsrc_t ry = make_rsrc(p.y, p.y_bytes);
    const rsrc_t rr = make_rsrc(p.res, p.r_bytes);
    const rsrc_t racc = make_rsrc(p.acc_out, p.acc_out ? (uint32_t)p.M * (uint32_t)p.OC * 4u : 0u);
    // KSW: wave w finishes channel subtiles j % 4 == w
    const uint32_t jmask = KSW ? (0x11111111u << wave) : 0xFFFFFFFFu;
    float gmax[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j) gmax[j] = 0.0f;
    int yo[PW], ro[PW], mo[PW];
    v2i rv[JN][PW];
    // output offsets and residual fragments of tile tl; issued before the
    // next tile's activation loads so that waiting for them leaves those in
    // flight
    auto epilogue_loads = [&](int tl) {
        const int pb = (pt0 + tl) * TPOS + (KSW ? 0 : wave * 16 * PW);
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const int m = pb + q * 16 + col;
            if (p.lin & kLinY) {
                // dense output (and residual) views: position m
                yo[q] = m < p.M ? (int)__umul24((uint32_t)m, (uint32_t)p.y_cstride) : -1;
                ro[q] = (int)__umul24((uint32_t)m, (uint32_t)p.r_cstride);
            } else {
                const int n = (int)fdiv((uint32_t)m, p.fd_ohw);
                const int pos = m - n * p.OH * p.OW;
                yo[q] = m < p.M ? n * (int)p.y_nstride + pos * p.y_cstride : -1;
                ro[q] = n * (int)p.r_nstride + pos * p.r_cstride;
            }
            mo[q] = m;
        }
        tile_residual<JN, PW, EPI>(p, rr, yo, ro, n0, jmax, grp, jmask, rv);
    };
    auto epilogue = [&](int) {
        tile_store<INT8, JN, PW, EPI>(p, acc, yo, mo, rv, n0, jmax, grp, jmask, l_bias, l_scale, gmax, ry, racc);
    };

    // ---- main loop ----------------------------------------------------------
    // Iteration i = tl * nit + it handles k step s0 + it * sstep of tile tl.
    // D iterations of activation fragments are in flight, across tile
    // boundaries: after iteration i's MFMAs its registers are refilled for
    // iteration i + D.  With MC, weight chunk gc (counting chunk boundaries)
    // sits in LDS buffer gc & 1 and the next one is fetched into registers
    // while it is in use; every wave reaches a boundary in the same iteration.
    constexpr int IPC = KC / (KSW ? 4 : 1);  // iterations per chunk
    // rounds of D iterations with no early exit (a single loop latch keeps the
    // compiler's count of loads in flight exact); the padding iterations only
    // issue out-of-range loads
    const int total_pad = (total + D - 1) / D * D;
    int tl = 0, it = 0, gc = 0;
    for (int ib = 0; ib < total_pad; ib += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int i = ib + d;
            const bool live = i < total;
            if constexpr (MC) {
                if (live && i > 0 && it % IPC == 0) {
                    ++gc;
                    stage_store(gc & 1);
                    __syncthreads();
                    if (gc + 1 < ntl * nch) stage_load((gc + 1) % nch);
                }
            }
            const int s = s0 + it * sstep;
            if (live && s < nks)
                mma_step(a[d], lds + (MC ? (gc & 1) * CH_BYTES : 0) + (s - (it / IPC) * KC) * WQ * R * 64);
            const bool tile_end = live && it == nit - 1;
            if (tile_end) epilogue_loads(tl);
            load_act(i + D, a[d], false);
            if (tile_end) {
                if constexpr (KSW) {
                    // partial tiles of the 4 waves -> LDS (the block's only
                    // tile: its weights are no longer needed); wave w
                    // finishes subtiles j % 4 == w
                    int32_t* red = reinterpret_cast<int32_t*>(lds);
                    __syncthreads();
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
                                    for (int w = 0; w < 4; ++w)
                                        t += red[((w * JN + j) * PW * 4 + q * 4 + r) * 64 + lane];
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
                epilogue(tl);
#pragma unroll
                for (int j = 0; j < JN; ++j)
#pragma unroll
                    for (int q = 0; q < PW; ++q) acc[j][q] = acc_t{0, 0, 0, 0};
                ++tl;
                it = 0;
            } else if (live) {
                ++it;
            }
        }
    }

    flush_slots<JN>(p, gmax, n0, jmax, jmask, out_f32, l_slots);
}

// Blocks of one kernel instance the GPU holds at once (occupancy x CUs),
// queried once per instance and device.
template <bool INT8, int JN, int PW, bool KSW, bool MC, int EPI>
int resident_blocks() {
    static std::atomic<int> cached[16];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 512;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, conv_mfma_kernel<INT8, JN, PW, KSW, MC, EPI>, 256, 0) !=
            hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu < 1 ||
        cus < 1)
        return 512;
    v = per_cu * cus;
    cached[dev].store(v, std::memory_order_relaxed);
    return v;
}

// Grid: a k-split block owns one tile; otherwise the position tiles of each
// channel tile are cut into contiguous runs so that every resident block
// slot gets one run (a single wave of blocks).
template <bool INT8, int JN, int PW, bool KSW, bool MC, int EPI>
hipError_t launch_cfg(ConvParams p, hipStream_t stream) {
    int groups = p.npt;
    if (!KSW) {
        const int cap = resident_blocks<INT8, JN, PW, KSW, MC, EPI>();
        if ((int64_t)p.npt * p.ntn > cap) groups = std::max(1, cap / p.ntn);
    }
    p.per = (p.npt + groups - 1) / groups;
    groups = (p.npt + p.per - 1) / p.per;
    const int64_t blocks = (int64_t)groups * p.ntn;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    const int nit = KSW ? (p.Kp / 64 + 3) / 4 : p.Kp / 64;
    p.fd_nit = make_fastdiv((uint32_t)nit);
    hipLaunchKernelGGL((conv_mfma_kernel<INT8, JN, PW, KSW, MC, EPI>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       p);
    return hipGetLastError();
}

// Every tile shape of one (INT8, MC, EPI) kernel family.
template <bool INT8, bool MC, int EPI>
hipError_t launch_family(const ConvParams& p, const ConvTile& t, hipStream_t stream) {
    if (t.ksw) {
        switch (t.jn) {
            case 1: return launch_cfg<INT8, 1, 1, true, MC, EPI>(p, stream);
            case 2: return launch_cfg<INT8, 2, 1, true, MC, EPI>(p, stream);
            case 4: return launch_cfg<INT8, 4, 1, true, MC, EPI>(p, stream);
            case 8: return launch_cfg<INT8, 8, 1, true, MC, EPI>(p, stream);
        }
        return hipErrorInvalidValue;
    }
    switch (t.jn * 8 + t.pw) {
        case 1 * 8 + 1: return launch_cfg<INT8, 1, 1, false, MC, EPI>(p, stream);
        case 1 * 8 + 2: return launch_cfg<INT8, 1, 2, false, MC, EPI>(p, stream);
        case 1 * 8 + 4: return launch_cfg<INT8, 1, 4, false, MC, EPI>(p, stream);
        case 2 * 8 + 1: return launch_cfg<INT8, 2, 1, false, MC, EPI>(p, stream);
        case 2 * 8 + 2: return launch_cfg<INT8, 2, 2, false, MC, EPI>(p, stream);
        case 2 * 8 + 4: return launch_cfg<INT8, 2, 4, false, MC, EPI>(p, stream);
        case 4 * 8 + 1: return launch_cfg<INT8, 4, 1, false, MC, EPI>(p, stream);
        case 4 * 8 + 2: return launch_cfg<INT8, 4, 2, false, MC, EPI>(p, stream);
        case 4 * 8 + 4: return launch_cfg<INT8, 4, 4, false, MC, EPI>(p, stream);
        case 8 * 8 + 1: return launch_cfg<INT8, 8, 1, false, MC, EPI>(p, stream);
        case 8 * 8 + 2: return launch_cfg<INT8, 8, 2, false, MC, EPI>(p, stream);
    }
    return hipErrorInvalidValue;
}

// k steps per weight chunk of a tile shape (host side of chunk_steps).
inline int chunk_steps_of(bool int8, int jn, bool ksw) {
    const int kc = std::max(1, 16384 / (jn * 16 * 64 * (int8 ? 1 : 2)));
    return ksw ? std::max(kc, 4) : kc;
}

// Each (INT8, MC, EPI) family is instantiated in a translation unit of its
// own (conv_i8*.hip, conv_f16*.hip), so the instances build in parallel.
#define AEXRT_IGEMM_FAMILIES(X) \
    X(true, false, 0) X(true, false, 1) X(true, false, 2) X(true, true, 0) X(true, true, 1) X(true, true, 2) \
    X(false, false, 0) X(false, false, 1) X(false, true, 0) X(false, true, 1)
#define AEXRT_IGEMM_EXTERN(I, M, E) \
    extern template hipError_t launch_family<I, M, E>(const ConvParams&, const ConvTile&, hipStream_t);
#define AEXRT_IGEMM_INSTANCE(I, M, E) \
    template hipError_t launch_family<I, M, E>(const ConvParams&, const ConvTile&, hipStream_t);

}  // namespace igemm
}  // namespace aexrt
