// A C2f bottleneck in one launch: conv a (3x3 s1 p1 SiLU, C -> C) and conv b
// (3x3 s1 p1 SiLU, C -> C, + the pair's input as residual when the
// bottleneck has its shortcut), the C2f "bottleneck superblock" of the
// reference (fusion kind 1, src/aexrt/engine.py:75-76; shader
// ensure_c2f_bottleneck_tiled_pipeline, native/aexrt_d3d12_runtime.cpp:
// 12205-12563), on int8 (W8A8, per-tensor activation scales, exact int32
// sums) or fp16 MFMA.
//
// A block owns a band of TR output rows (whole width) of one image.  Conv a
// runs over the band plus one row above and below (its rows inside the
// image), reading the input window X (those rows plus one more on each side,
// one column of zero padding left and right) from LDS; its fp16 SiLU output
// goes to the grid G in LDS (zero outside the image), and conv b runs over
// the band from G.  Neighbouring bands recompute their shared rows of a.
//
// int8: conv b quantizes a's output with the per-tensor amax of the whole
// intermediate tensor, every image (RT:3232-3257), a grid-wide dependency.
// Each block folds max|a| of the values it computed into a striped word and
// the grid meets in a barrier: per-XCD arrival counters, a counter of XCDs,
// and a generation word the waiting blocks poll with plain (relaxed) atomic
// loads, one acquire fence after the wait.  Every block of the grid must be
// resident at once: the host sizes the grid and refuses a launch that the
// GPU cannot hold; the wait is bounded (about a second) and sets an error
// word instead of spinning forever.  The recomputed rows of a are the same
// values in both blocks (same inputs, same arithmetic), so the max over
// everything computed is the max of the tensor.
//
//   prologue  input scale (int8); biases; X staged through registers
//             (quantized once for int8); G zeroed; tap tables; the first
//             weight chunks of a in flight
//   conv a    k steps in chunks of KKC through an LDS ring of KD slots (the
//             chunk loads go straight to LDS, KD - 1 in flight); B operands
//             from X
//   epi a     bias + SiLU -> fp16 -> G; max|a|
//   barrier   (int8) fold max|a|, the residual loads of the band issued,
//             grid barrier, amax of a; G quantized into the X region
//   conv b    the ring continues with b's weights (its first chunks were in
//             flight during the barrier); B operands from G
//   epi b     bias + SiLU (+ residual) -> y, max|y| into y's amax slots
//
// MFMA: v_mfma_i32_32x32x32_i8 / v_mfma_f32_32x32x16_f16, weights as the A
// operand (32 output channels), 32 positions as B; a lane's 16 outputs are
// channels 8 j4 + 4 (lane / 32) + r of position lane % 32.  LDS layouts as
// in the 32x32-MFMA conv kernel: weights [k step][half][oc][16 B], maps
// [channel piece][pixel][16 B]; every operand read is one conflict-free
// ds_read_b128 per lane.
#pragma once
#include "conv_igemm.h"

namespace aexrt {

constexpr int kPairMaxSteps = 72;      // k steps of one conv: 9 * C / KSUB (fp16 at C = 128)
// window pieces per thread (int8 pieces take two 16-byte loads)
constexpr int pair_max_pieces(bool int8) { return int8 ? 8 : 12; }
constexpr int kPairStripes = 16;       // copies of the intermediate's amax word
// words of a pair launch's sync area (uint32): arrival counters of the 8 XCD
// groups (a 64-byte line each), the counter of groups, the generation, the
// amax copies of the intermediate (a line each); cleared at run start
constexpr int kPairSyncWords = 512;
constexpr int kPairTop = 128, kPairGen = 144, kPairAmax = 192;
static_assert(kPairSyncWords == kPairSyncWordsHost, "sync area size");

struct PairParams {
    ConvParams a, b;        // a: x -> t, b: t -> y (b.res: the residual view, b.acc_out its accumulators)
    int TR;                 // output rows of a band (whole width)
    int nband, ntile;       // bands per image, N * nband
    int ka, kb;             // k steps of a and b
    int nchunk_a, nchunk;   // weight chunks of a, of a and b
    int x_off, g_off;       // LDS offsets of X and G (after the ring)
    uint32_t x_img, y_img, r_img;  // bytes of one image's input, output, residual views
    uint32_t* sync;         // int8: kPairSyncWords words, zero at launch (generation excepted)
    uint32_t* err;          // int8: set to 1 when a barrier wait times out
    __half* t_out;          // optional: the intermediate, dense NHWC [N][H][W][C] (for checks)
    int32_t* acc_a;         // optional: a's int32 sums [N*H*W][C] (int8)
    FastDiv fd_nband;
};

namespace pair {

using igemm::kOob;
using igemm::make_rsrc;
using igemm::quant8;
using igemm::rsrc_t;
using igemm::v2i;
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kKC = 4;   // k steps per weight chunk
constexpr int kD = 4;    // ring slots
constexpr int kNT = 256;
constexpr uint32_t kSpinLimit = 1u << 20;

__device__ __forceinline__ int small_div(int a, float inv) { return (int)(((float)a + 0.5f) * inv); }

// Grid barrier of the blocks of one launch (thread 0 of each block; the
// caller's __syncthreads around it).  Returns false after a timed-out wait.
__device__ __forceinline__ bool grid_barrier(uint32_t* sync, uint32_t* err) {
    const uint32_t nb = gridDim.x;
    const uint32_t g = __hip_atomic_load(&sync[kPairGen], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t x = blockIdx.x & 7u;
    const uint32_t nx = nb < 8u ? nb : 8u;
    const uint32_t gs = nb / 8u + (x < nb % 8u ? 1u : 0u);
    bool last = false;
    if (__hip_atomic_fetch_add(&sync[x * 16u], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gs - 1u) {
        __hip_atomic_store(&sync[x * 16u], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = __hip_atomic_fetch_add(&sync[kPairTop], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nx - 1u;
        if (last) __hip_atomic_store(&sync[kPairTop], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    bool ok = true;
    if (last) {
        __builtin_amdgcn_s_waitcnt(0);
        __hip_atomic_store(&sync[kPairGen], g + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        uint32_t it = 0;
        while (__hip_atomic_load(&sync[kPairGen], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g) {
            if (++it > kSpinLimit) {
                ok = false;
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return ok;
}

template <bool INT8, int NQ, int MQ>
__global__ __launch_bounds__(kNT) void conv_pair_kernel(PairParams h) {
    constexpr int NOCB = NQ * 32;             // channels of a, b and the input (C == NOCB)
    constexpr int CB = kKC * 2 * NOCB * 16;   // LDS bytes of one weight chunk
    constexpr int PT = kKC * 2 * NOCB / kNT;  // chunk loads per thread
    static_assert((kKC * 2 * NOCB) % kNT == 0, "a chunk is whole loads of every thread");
    constexpr int KSUB = INT8 ? 32 : 16;      // k of one MFMA step
    constexpr int CPP = INT8 ? 16 : 8;        // channels of one 16-byte map piece
    typedef typename std::conditional<INT8, v16i, v16f>::type acc_t;
    const ConvParams& pa = h.a;
    const ConvParams& pb = h.b;
    constexpr int C = NOCB;

    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ __attribute__((aligned(16))) float l_bias_a[NOCB], l_bias_b[NOCB], l_scale_a[NOCB], l_scale_b[NOCB];
    __shared__ __attribute__((aligned(16))) int l_tap_a[2 * kPairMaxSteps], l_tap_b[2 * kPairMaxSteps];
    __shared__ uint32_t l_slots[NQ * 2];
    __shared__ float l_red[kNT / 64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // ---- band geometry (block-uniform) --------------------------------------
    const int blk = xcd_remap(blockIdx.x, gridDim.x);
    const int n = (int)fdiv((uint32_t)blk, h.fd_nband);
    const int band = blk - n * h.nband;
    const int H = pa.H, W = pa.W;
    const int r0 = band * h.TR;
    const int TRr = min(h.TR, H - r0);
    const int a0 = max(r0 - 1, 0), a1 = min(r0 + TRr + 1, H);
    const int RA = a1 - a0;
    const int MW = W + 2;                       // pixels of a map row (X and G)
    const int XNPIX = (RA + 2) * MW, GNPIX = (TRr + 2) * MW;
    const int npos1 = RA * W, npos2 = TRr * W;

    const rsrc_t rx = make_rsrc(static_cast<const uint8_t*>(pa.x) + (int64_t)n * pa.x_nstride * 2, h.x_img);
    const rsrc_t rwa = make_rsrc(pa.w, (uint32_t)pa.OCp * (uint32_t)pa.Kp * (INT8 ? 1u : 2u));
    const rsrc_t rwb = make_rsrc(pb.w, (uint32_t)pb.OCp * (uint32_t)pb.Kp * (INT8 ? 1u : 2u));

    // ---- input scale (int8), per-channel constants --------------------------
    uint32_t slot_raw[igemm::kMaxSlotReads / 64];
    if constexpr (INT8) igemm::in_slot_loads(pa, lane, slot_raw);
    const rsrc_t rba = make_rsrc(pa.bias, (uint32_t)pa.OC * 4u);
    const rsrc_t rbb = make_rsrc(pb.bias, (uint32_t)pb.OC * 4u);
    const rsrc_t rsa = make_rsrc(pa.w_scale, INT8 ? (uint32_t)pa.OC * 4u : 0u);
    const rsrc_t rsb = make_rsrc(pb.w_scale, INT8 ? (uint32_t)pb.OC * 4u : 0u);
    const uint32_t cofs = tid < NOCB ? (uint32_t)tid * 4u : kOob;
    const float bias_a = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rba, cofs, 0, 0));
    const float bias_b = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rbb, cofs, 0, 0));
    const float wsc_a = INT8 ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsa, cofs, 0, 0)) : 0.0f;
    const float wsc_b = INT8 ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsb, cofs, 0, 0)) : 0.0f;

    // ---- window X: piece e = plane * XNPIX + pixel (plane = CPP channels);
    // this thread's pieces e = tid + k * 256 loaded into registers ----------
    const int npiece = (C / CPP) * XNPIX;
    constexpr int MAXP = pair_max_pieces(INT8);
    v4i xr[MAXP][INT8 ? 2 : 1];
    {
        const float inv_npix = 1.0f / (float)XNPIX, inv_mw = 1.0f / (float)MW;
#pragma unroll
        for (int k = 0; k < MAXP; ++k) {
            const int e = tid + k * kNT;
            const int pl = small_div(e, inv_npix);
            const int pix = e - pl * XNPIX;
            const int pr = small_div(pix, inv_mw);
            const int ih = a0 - 1 + pr, iw = pix - pr * MW - 1;
            const bool ok = e < npiece && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
            const uint32_t off = (uint32_t)((ih * W + iw) * pa.x_cstride + pl * CPP) * 2u;
            xr[k][0] = igemm::bload16(rx, ok ? off : kOob);
            if constexpr (INT8) xr[k][1] = igemm::bload16(rx, ok ? off + 16u : kOob);
        }
    }

    // ---- weight ring: chunk g (a's chunks, then b's) into slot g % kD -------
    int w_sl[PT];
    uint32_t w_a[PT], w_b[PT];
#pragma unroll
    for (int i = 0; i < PT; ++i) {
        const int e = i * kNT + tid;
        const int sl = e / (2 * NOCB);
        const int rem = e - sl * (2 * NOCB);
        const int half = rem / NOCB;
        const int row = rem - half * NOCB;
        w_sl[i] = sl;
        // byte offset of 16 bytes of k step sl, half `half` of weight row `row`
        w_a[i] = row < pa.OCp ? (uint32_t)row * (uint32_t)pa.Kp * (INT8 ? 1u : 2u) + (uint32_t)(32 * sl + 16 * half) : kOob;
        w_b[i] = row < pb.OCp ? (uint32_t)row * (uint32_t)pb.Kp * (INT8 ? 1u : 2u) + (uint32_t)(32 * sl + 16 * half) : kOob;
    }
    auto issue = [&](int g) {
        const bool isb = g >= h.nchunk_a;  // block-uniform
        const int s0 = (isb ? g - h.nchunk_a : g) * kKC;
        const int left = (isb ? h.kb : h.ka) - s0;
        uint8_t* const slot = lds + (g & (kD - 1)) * CB;
#pragma unroll
        for (int i = 0; i < PT; ++i) {
            const uint32_t base = isb ? w_b[i] : w_a[i];
            const bool ok = w_sl[i] < left && base != kOob;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(isb ? rwb : rwa, (lds_ptr_t)(slot + (i * kNT + wave * 64) * 16), 16,
                                                      ok ? base + (uint32_t)s0 * 32u : kOob, 0, 0, 0);
        }
    };
#pragma unroll
    for (int d = 0; d < kD - 1; ++d)
        if (d < h.nchunk) issue(d);

    // ---- G zeroed (fp16, [C / 8][GNPIX][16 B]), tap tables ------------------
    {
        uint8_t* const gb = lds + h.g_off;
        const int ng = (C / 8) * GNPIX;
        for (int e = tid; e < ng; e += kNT) *reinterpret_cast<v4i*>(gb + e * 16) = v4i{0, 0, 0, 0};
    }
    // k step s (one tap, KSUB channels), half hh: byte offset of its plane
    // and tap relative to the position's (0, 0) tap pixel; [s][hh]
    auto tap_table = [&](int* tab, int ks, int npix, int cpp) {
        for (int e = tid; e < 2 * ks; e += kNT) {
            const int s = e >> 1, hh = e & 1;
            const int k0 = s * KSUB, tap = k0 / C, c0 = k0 - tap * C;
            tab[e] = ((c0 / cpp + hh) * npix + (tap / 3) * MW + tap % 3) * 16;
        }
    };
    tap_table(l_tap_a, h.ka, XNPIX, CPP);
    // conv b reads G as fp16 pieces (fp16) or the quantized G (int8: CPP 16)
    tap_table(l_tap_b, h.kb, GNPIX, CPP);
    if (tid < NQ * 2) l_slots[tid] = 0u;

    // ---- X: wait for the window loads (the weight chunks may stay in
    // flight), quantize (int8) and store ----------------------------------------
    float s_q = 0.0f, in_scale = 0.0f;
    if constexpr (INT8) igemm::in_slot_scale(slot_raw, s_q, in_scale);
    if (tid < NOCB) {
        l_bias_a[tid] = bias_a;
        l_bias_b[tid] = bias_b;
        l_scale_a[tid] = in_scale * wsc_a;
        l_scale_b[tid] = wsc_b;  // times the intermediate's scale after the barrier
    }
    {
        uint8_t* const xb = lds + h.x_off;
#pragma unroll
        for (int k = 0; k < MAXP; ++k) {
            const int e = tid + k * kNT;
            if (e < npiece) {
                v4i v;
                if constexpr (INT8) {
                    const v2i lo = quant8(xr[k][0], s_q), hq = quant8(xr[k][1], s_q);
                    v = v4i{lo[0], lo[1], hq[0], hq[1]};
                } else {
                    v = xr[k][0];
                }
                *reinterpret_cast<v4i*>(xb + e * 16) = v;
            }
        }
    }

    // ---- per-lane positions of this wave's subtiles (w, w + 4, ...) ---------
    const int lw = wave;
    int bofs_a[MQ], bofs_b[MQ];
    const int myq1 = min(MQ, max(0, ((npos1 + 31) >> 5) - lw + 3) >> 2);
    const int myq2 = min(MQ, max(0, ((npos2 + 31) >> 5) - lw + 3) >> 2);
    {
        const float inv_w = 1.0f / (float)W;
#pragma unroll
        for (int q = 0; q < MQ; ++q) {
            const int pos = (lw + 4 * q) * 32 + l32;
            const int p1 = min(pos, npos1 - 1);
            const int r1 = small_div(p1, inv_w);
            bofs_a[q] = (r1 * MW + (p1 - r1 * W)) * 16;
            const int p2 = min(pos, npos2 - 1);
            const int r2 = small_div(p2, inv_w);
            bofs_b[q] = (r2 * MW + (p2 - r2 * W)) * 16;
        }
    }
    const int abase = (hi * NOCB + l32) * 16;

    acc_t acc[MQ][NQ];
#pragma unroll
    for (int q = 0; q < MQ; ++q)
#pragma unroll
        for (int j = 0; j < NQ; ++j) acc[q][j] = acc_t{};

    // chunk c complete in every wave (in-order completion: the loads after
    // it are the at most kD - 2 later chunks'), then the slot of c - 1 refilled
    auto ring_wait = [&](int c) {
        __builtin_amdgcn_sched_barrier(0);
        if (c + kD - 2 < h.nchunk) {
            constexpr int vm = PT * (kD - 2);
            static_assert(vm < 64, "vmcnt field");
            __builtin_amdgcn_s_waitcnt((vm & 15) | ((vm >> 4) << 14) | 0x0070);  // vmcnt(vm) lgkmcnt(0)
        } else {
            __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (c + kD - 1 < h.nchunk) issue(c + kD - 1);
    };
    // chunks [cb, ce) of one conv over a map with its tap table
    auto conv = [&](int cb, int ce, int ks, const uint8_t* map, const int* taps, const int (&bofs)[MQ], int myq) {
        for (int c = cb; c < ce; ++c) {
            ring_wait(c);
            const int s0 = (c - cb) * kKC;
            const uint8_t* const ws = lds + (c & (kD - 1)) * CB + abase;
            v4i A[kKC][NQ], B[kKC][MQ];
#pragma unroll
            for (int sl = 0; sl < kKC; ++sl) {
                const int s = min(s0 + sl, ks - 1);  // past the last step: zero weights, any map read in range
                const int to = taps[2 * s + hi];
#pragma unroll
                for (int j = 0; j < NQ; ++j)
                    A[sl][j] = *reinterpret_cast<const v4i*>(ws + sl * (2 * NOCB * 16) + j * 512);
#pragma unroll
                for (int q = 0; q < MQ; ++q) B[sl][q] = *reinterpret_cast<const v4i*>(map + bofs[q] + to);
            }
#pragma unroll
            for (int sl = 0; sl < kKC; ++sl) {
#pragma unroll
                for (int q = 0; q < MQ; ++q) {
                    if (q >= myq) break;  // wave-uniform
#pragma unroll
                    for (int j = 0; j < NQ; ++j) {
                        if constexpr (INT8)
                            acc[q][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[sl][j], B[sl][q], acc[q][j], 0, 0, 0);
                        else
                            acc[q][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, A[sl][j]),
                                                                               __builtin_bit_cast(v8h, B[sl][q]),
                                                                               acc[q][j], 0, 0, 0);
                    }
                }
            }
        }
    };

    // ---- conv a ------------------------------------------------------------
    conv(0, h.nchunk_a, h.ka, lds + h.x_off, l_tap_a, bofs_a, myq1);
    // epilogue a: fp16(silu(acc * scale + bias)) -> G; max|a| over the values
    float tmax = 0.0f;
    {
        uint8_t* const gb = lds + h.g_off;
        const int dr = a0 - (r0 - 1);  // G row of a's first row
        const float inv_w = 1.0f / (float)W;
        const rsrc_t rt = make_rsrc(h.t_out, h.t_out ? (uint32_t)((uint64_t)pa.N * H * W * C * 2u) : 0u);
        const rsrc_t racc = make_rsrc(h.acc_a, h.acc_a ? (uint32_t)((uint64_t)pa.N * H * W * C * 4u) : 0u);
#pragma unroll
        for (int q = 0; q < MQ; ++q) {
            const int pos = (lw + 4 * q) * 32 + l32;
            const bool live = q < myq1 && pos < npos1;
            const int r = small_div(min(pos, npos1 - 1), inv_w);
            const int cpos = min(pos, npos1 - 1) - r * W;
            const int gp = (r + dr) * MW + cpos + 1;
            const uint32_t m = (uint32_t)(((n * H + a0 + r) * W) + cpos);  // position in the image batch
            // rows of a this band owns (the recomputed neighbour rows are stored by their owner)
            const bool own = live && a0 + r >= r0 && a0 + r < r0 + TRr;
#pragma unroll
            for (int j = 0; j < NQ; ++j)
#pragma unroll
                for (int j4 = 0; j4 < 4; ++j4) {
                    const int lc = j * 32 + j4 * 8 + hi * 4;
                    float bv[4], wv[4], v[4];
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        bv[rr] = l_bias_a[lc + rr];
                        wv[rr] = l_scale_a[lc + rr];
                    }
                    const typename std::conditional<INT8, v4i, v4f>::type a4{
                        acc[q][j][4 * j4], acc[q][j][4 * j4 + 1], acc[q][j][4 * j4 + 2], acc[q][j][4 * j4 + 3]};
                    igemm::epi_values<INT8, igemm::kEpiSilu>(pa, a4, bv, wv, v2i{0, 0}, v);
                    const __half2 o0 = __floats2half2_rn(v[0], v[1]), o1 = __floats2half2_rn(v[2], v[3]);
                    const __half2 oh[2] = {o0, o1};
                    v2i o;
                    __builtin_memcpy(&o, oh, 8);
                    if (live) {
                        *reinterpret_cast<v2i*>(gb + ((j * 4 + j4) * GNPIX + gp) * 16 + hi * 8) = o;
                        tmax = fmaxf(tmax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
                    }
                    if (h.t_out)
                        __builtin_amdgcn_raw_buffer_store_b64(o, rt, own ? (m * (uint32_t)C + (uint32_t)lc) * 2u : kOob,
                                                              0, 0);
                    if constexpr (INT8) {
                        if (h.acc_a)
                            __builtin_amdgcn_raw_buffer_store_b128(
                                v4i{(int)a4[0], (int)a4[1], (int)a4[2], (int)a4[3]}, racc,
                                own ? (m * (uint32_t)C + (uint32_t)lc) * 4u : kOob, 0, 0);
                    }
                }
#pragma unroll
            for (int j = 0; j < NQ; ++j) acc[q][j] = acc_t{};
        }
    }

    // ---- output side: residual loads of the band (in flight during the barrier)
    const rsrc_t rr = make_rsrc(pb.res ? static_cast<const uint8_t*>(static_cast<const void*>(pb.res)) +
                                             (int64_t)n * pb.r_nstride * 2
                                       : nullptr,
                                pb.res ? h.r_img : 0u);
    int yo[MQ], ro[MQ];
    {
        const float inv_w = 1.0f / (float)W;
#pragma unroll
        for (int q = 0; q < MQ; ++q) {
            const int pos = (lw + 4 * q) * 32 + l32;
            const int p2 = min(pos, npos2 - 1);
            const int r2 = small_div(p2, inv_w);
            const int pix = (r0 + r2) * W + (p2 - r2 * W);
            const bool ok = q < myq2 && pos < npos2;
            yo[q] = ok ? pix * pb.y_cstride : -1;
            ro[q] = ok ? pix * pb.r_cstride : -1;
        }
    }
    v2i rv[MQ][NQ][4];
#pragma unroll
    for (int q = 0; q < MQ; ++q)
#pragma unroll
        for (int j = 0; j < NQ; ++j)
#pragma unroll
            for (int j4 = 0; j4 < 4; ++j4) {
                const int lc = j * 32 + j4 * 8 + hi * 4;
                rv[q][j][j4] = __builtin_amdgcn_raw_buffer_load_b64(
                    rr, pb.res && ro[q] >= 0 ? (uint32_t)(ro[q] + lc) * 2u : kOob, 0, 0);
            }

    if constexpr (INT8) {
        // ---- max|a| of the block -> one of the striped words; the grid barrier;
        // the intermediate's amax and scale ----------------------------------
        const float wm = wave_max(tmax);
        if (lane == 0) l_red[wave] = wm;
        __syncthreads();  // also: every wave's G writes before the quantization below
        if (tid == 0) {
            const float bm = fmaxf(fmaxf(l_red[0], l_red[1]), fmaxf(l_red[2], l_red[3]));
            // the stored values are fp16: the max of their magnitudes
            const uint32_t bits = f2u(__half2float(__float2half(bm)));
            uint32_t* const word = h.sync + kPairAmax + (blockIdx.x % kPairStripes) * 16u;
            // a returning atomic, its value waited for: performed before this
            // block's arrival at the barrier
            const uint32_t old = __hip_atomic_fetch_max(word, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("" ::"v"(old));
            __builtin_amdgcn_s_waitcnt(0);
            (void)grid_barrier(h.sync, h.err);  // a timed-out wait has set the error word
        }
        __syncthreads();
        uint32_t am = 0u;
        if (lane < kPairStripes)
            am = __hip_atomic_load(h.sync + kPairAmax + lane * 16u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float t_amax = u2f(wave_umax(am));
        const float s_t = t_amax > 0.0f ? 127.0f / t_amax : 0.0f;
        const float in_t = t_amax > 0.0f ? t_amax / 127.0f : 0.0f;
        if (tid < NOCB) l_scale_b[tid] = in_t * wsc_b;
        // G (fp16) quantized into the X region (int8 [C / 16][GNPIX][16 B])
        {
            const uint8_t* const gb = lds + h.g_off;
            uint8_t* const qb = lds + h.x_off;
            const int nq16 = (C / 16) * GNPIX;
            const float inv_g = 1.0f / (float)GNPIX;
            for (int e = tid; e < nq16; e += kNT) {
                const int pl = small_div(e, inv_g);
                const int px = e - pl * GNPIX;
                const v4i lo = *reinterpret_cast<const v4i*>(gb + ((2 * pl) * GNPIX + px) * 16);
                const v4i hq = *reinterpret_cast<const v4i*>(gb + ((2 * pl + 1) * GNPIX + px) * 16);
                const v2i q0 = quant8(lo, s_t), q1 = quant8(hq, s_t);
                *reinterpret_cast<v4i*>(qb + e * 16) = v4i{q0[0], q0[1], q1[0], q1[1]};
            }
        }
        // (conv b's first ring barrier orders these writes before its reads)
    }

    // ---- conv b --------------------------------------------------------------
    conv(h.nchunk_a, h.nchunk, h.kb, INT8 ? lds + h.x_off : lds + h.g_off, l_tap_b, bofs_b, myq2);

    // ---- epilogue b -----------------------------------------------------------
    const bool out_f32 = (pb.flags & kConvOutF32) != 0;
    const rsrc_t ry = make_rsrc(static_cast<uint8_t*>(pb.y) + (int64_t)n * pb.y_nstride * (out_f32 ? 4 : 2), h.y_img);
    const rsrc_t racc = make_rsrc(pb.acc_out, pb.acc_out ? (uint32_t)((uint64_t)pb.N * H * W * C * 4u) : 0u);
    float gmax[NQ * 2];
#pragma unroll
    for (int j = 0; j < NQ * 2; ++j) gmax[j] = 0.0f;
#pragma unroll
    for (int q = 0; q < MQ; ++q) {
        const bool ok = yo[q] >= 0;
        const int pos = (lw + 4 * q) * 32 + l32;
        const int p2 = min(pos, npos2 - 1);
        const uint32_t m = (uint32_t)((n * H + r0) * W + p2);
#pragma unroll
        for (int j = 0; j < NQ; ++j)
#pragma unroll
            for (int j4 = 0; j4 < 4; ++j4) {
                const int lc = j * 32 + j4 * 8 + hi * 4;
                float bv[4], wv[4], v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    bv[r] = l_bias_b[lc + r];
                    wv[r] = l_scale_b[lc + r];
                }
                const typename std::conditional<INT8, v4i, v4f>::type a4{
                    acc[q][j][4 * j4], acc[q][j][4 * j4 + 1], acc[q][j][4 * j4 + 2], acc[q][j][4 * j4 + 3]};
                igemm::epi_values<INT8, igemm::kEpiAny>(pb, a4, bv, wv, rv[q][j][j4], v);
                if constexpr (INT8) {
                    if (pb.acc_out)
                        __builtin_amdgcn_raw_buffer_store_b128(v4i{(int)a4[0], (int)a4[1], (int)a4[2], (int)a4[3]},
                                                               racc, ok ? (m * (uint32_t)C + (uint32_t)lc) * 4u : kOob,
                                                               0, 0);
                }
                const float m4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
                gmax[(j * 32 + j4 * 8) >> 4] = fmaxf(gmax[(j * 32 + j4 * 8) >> 4], ok ? m4 : 0.0f);
                if (out_f32) {
                    const v4i o{__float_as_int(v[0]), __float_as_int(v[1]), __float_as_int(v[2]), __float_as_int(v[3])};
                    __builtin_amdgcn_raw_buffer_store_b128(o, ry, ok ? (uint32_t)(yo[q] + lc) * 4u : kOob, 0, 0);
                } else {
                    const __half2 oh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                    v2i o;
                    __builtin_memcpy(&o, oh, 8);
                    __builtin_amdgcn_raw_buffer_store_b64(o, ry, ok ? (uint32_t)(yo[q] + lc) * 2u : kOob, 0, 0);
                }
            }
    }
    // max|y| per 16-channel group into this block's copy of y's slots
    if (pb.y_slots.p) {
#pragma unroll
        for (int g = 0; g < NQ * 2; ++g) {
            const float v = wave_max(out_f32 ? gmax[g] : __half2float(__float2half(gmax[g])));
            if (lane == 0 && v > 0.0f) atomicMax(&l_slots[g], f2u(v));
        }
        __syncthreads();
        if (tid < NQ * 2 && l_slots[tid]) atomicMax(slot_copy(pb.y_slots, blockIdx.x) + tid, l_slots[tid]);
    }
}

}  // namespace pair
}  // namespace aexrt
