// 3x3 convolution (pad 1, stride 1 or 2) on gfx950's 32x32 MFMA tiles: the
// arithmetic of the halo-tile kernel (int8 W8A8 with exact int32
// accumulation, or fp16 with fp32 accumulation) with the LDS operands laid
// out so that one MFMA operand read is a contiguous 1 KB per wave.
//
// A 32x32 MFMA (v_mfma_f32_32x32x16_f16 / v_mfma_i32_32x32x32_i8) reads a
// 32-row A and a 32-column B fragment of 1 KB each for 32 output channels x
// 32 positions, half the operand bytes per multiply-add of the 16x16 shape;
// a wave holding MQ x NQ such tiles reads (MQ + NQ) KB of LDS per k step for
// MQ * NQ MFMAs.  LDS bandwidth (about 128 B/clk per CU) is what bounds the
// 16x16 kernels; with MQ = NQ = 2 the operand reads of 4 waves match it.
//
// LDS layouts (16-byte pieces: 8 fp16 or 16 int8 channels of one pixel/tap):
//   weights [chunk][k step][half][oc][16 B]: the lanes of an A read (oc =
//     lane % 32, half = lane / 32) touch 64 consecutive pieces;
//   window  [plane][pixel][16 B], plane = channel / piece: the lanes of a B
//     read (32 positions, two channel planes) touch two runs of consecutive
//     pixels (unit stride for stride-1 convs).
// Both are conflict-free for ds_read_b128.
//
// The block's weights for all input channels are loaded into LDS once
// (directly, buffer_load ... lds) and stay resident while the block walks a
// run of position tiles; each (tile, chunk of CC channels) iteration stages
// the input window of the chunk (IR x ICOL pixels, zero outside the image)
// through registers (quantized once there for int8), double-buffered with
// one barrier per iteration.  The NW (4 or 8) waves split the tile's
// positions (MQ 32-position subtiles each) and share the block's NQ
// 32-channel subtiles.
//
// NG = 2 (8 waves): the waves form two groups of 4 with a window
// double-buffer each and a barrier of their own (a counter in LDS), sharing
// the block's resident weights; group g takes tiles g, g + 2, ... of the
// block's run.  With one barrier per block all waves are in the same phase
// (MFMAs, then the epilogue's VALU, then staging), so the matrix cores idle
// during the epilogue; two groups drift apart and one group's MFMAs run
// beside the other's epilogue and staging.
#pragma once
#include "conv_igemm.h"

namespace aexrt {

// k steps of one chunk (the table of tap offsets).
constexpr int kM32MaxSteps = 96;

struct M32Params {
    ConvParams c;          // views, weights, flags; c.ntn / c.per / c.fd_ntn are this launch's
    int TR, TC;            // output rows x columns of a position tile
    int IR, ICOL, NPIX;    // its input window: rows, columns, pixels
    int CC, nch;           // channels per chunk (C % CC == 0, CC % 16 == 0), chunks
    int nks;               // MFMA k steps per chunk: ceil(9 * CC / KSUB), the last zero-padded
    int npiece;            // 16-byte window pieces of one chunk: (CC / CPP) * NPIX
    int ntc, tpi, ntile;   // position tiles per row band, per image, in all
    int wbytes;            // LDS bytes of the resident weights (all chunks)
    int tbytes;            // LDS bytes of one window buffer
    FastDiv fd_npix, fd_icol, fd_tc, fd_ntc, fd_tpi, fd_cc, fd_nks, fd_nocb;
    // fused 1x1 conv (F2 instances): fp16 weights [OCp][Kp] over this conv's
    // output channels, bias, flags, output view and slots; its input is this
    // conv's fp16 output, which is not stored
    ConvParams c2;
};

namespace m32 {

using igemm::bload16;
using igemm::kOob;
using igemm::make_rsrc;
using igemm::quant8;
using igemm::rsrc_t;
using igemm::v2i;
using igemm::xcd_remap;
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Barrier of the waves of one group: each wave adds one to the group's LDS
// counter after its LDS writes and waits until the counter reaches target.
// The wait is bounded (about a second), so a wave can never spin forever.
__device__ __forceinline__ void group_barrier(uint32_t* ctr, uint32_t target) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    for (uint32_t it = 0; it < (1u << 22); ++it) {
        if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

template <bool INT8, int MQ, int NQ, int NP, int EPI, int NW, bool F2 = false, int NG = 1>
__global__ __launch_bounds__(NW * 64) void conv3x3_m32_kernel(M32Params h) {
    static_assert(!F2 || (!INT8 && EPI == igemm::kEpiSilu), "the fused 1x1 follows an fp16 SiLU conv");
    static_assert(NG == 1 || (NG == 2 && NW == 8), "two wave groups of 4");
    constexpr int NT = NW * 64;           // threads of the block
    constexpr int NWG = NW / NG;          // waves of a group
    constexpr int NTG = NWG * 64;         // threads of a group
    constexpr int ESZ = INT8 ? 1 : 2;
    constexpr int KSUB = INT8 ? 32 : 16;  // k of one MFMA
    constexpr int CPP = 16 / ESZ;         // channels of one 16-byte piece
    constexpr int NOCB = NQ * 32;         // output channels of the block
    constexpr int NL = INT8 ? 2 : 1;      // 16-byte fp16 loads per piece
    typedef typename std::conditional<INT8, v16i, v16f>::type acc_t;
    const ConvParams& p = h.c;

    // [weights: wbytes][window buffer 0: tbytes][window buffer 1: tbytes]
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    // k step * 2 + half -> byte offset of the piece's plane and tap in the
    // window, relative to the output position's (0, 0) tap pixel
    __shared__ int l_toff[2 * kM32MaxSteps];
    __shared__ float l_bias[NOCB], l_scale[NOCB];
    __shared__ uint32_t l_slots[NOCB / 16];
    __shared__ float l_bias2[F2 ? NOCB : 1];
    __shared__ uint32_t l_slots2[F2 ? NOCB / 16 : 1];
    __shared__ uint32_t l_gbar[NG];  // group barrier counters

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hi = lane >> 5;
    const int grp_id = NG == 1 ? 0 : wave / NWG;  // wave-uniform
    const int gwave = wave - grp_id * NWG;         // wave within its group
    const int gtid = tid - grp_id * NTG;           // thread within its group

    const int b = xcd_remap(blockIdx.x, gridDim.x);
    const int pg = (int)fdiv((uint32_t)b, p.fd_ntn);
    const int n0 = (b - pg * p.ntn) * NOCB;
    const int pt0 = pg * p.per;
    const int ntl = min(p.per, h.ntile - pt0);
    const int S = p.S;
    const rsrc_t rx = make_rsrc(p.x, p.x_bytes);
    const rsrc_t rw = make_rsrc(p.w, (uint32_t)p.OCp * (uint32_t)p.Kp * ESZ);

    // ---- window pieces of this thread: e = gtid + k * NTG -> plane e / NPIX,
    // pixel (ir, ic); LDS place e * 16 of its group's buffers (the same for
    // every tile and chunk) ----
    int prc[NP], prel[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) {
        const int e = gtid + k * NTG;
        const int pl = (int)fdiv((uint32_t)e, h.fd_npix);
        const int pix = e - pl * h.NPIX;
        const int ir = (int)fdiv((uint32_t)pix, h.fd_icol);
        const int ic = pix - ir * h.ICOL;
        prc[k] = e < h.npiece ? (ir | (ic << 16)) : 0x7FFF;  // row 0x7FFF fails every bounds test
        prel[k] = (ir * p.W + ic) * p.x_cstride + pl * CPP;
    }
    // this group's tiles: lt-th of the group -> tl = grp_id + lt * NG of the block's run
    const int ntl_g = NG == 1 ? ntl : (ntl - grp_id + NG - 1) / NG;
    auto tile_pos = [&](int lt, int& n, int& oh0, int& ow0) {
        const int ti = pt0 + grp_id + lt * NG;
        n = (int)fdiv((uint32_t)ti, h.fd_tpi);
        const int rem = ti - n * h.tpi;
        const int tr = (int)fdiv((uint32_t)rem, h.fd_ntc);
        oh0 = tr * h.TR;
        ow0 = (rem - tr * h.ntc) * h.TC;
    };
    v4i pf[NP][NL];
    // loads of (tile tl, chunk ch) into pf, all issued (out of range when
    // !live: the first row is moved off the image)
    auto window_loads = [&](int tl, int ch, bool live) {
        int n, oh0, ow0;
        tile_pos(tl, n, oh0, ow0);
        const int ihb = live ? oh0 * S - 1 : -0x40000000;
        const int iwb = ow0 * S - 1;
        const int gbase = n * (int)p.x_nstride + ((oh0 * S - 1) * p.W + iwb) * p.x_cstride + ch * h.CC;
#pragma unroll
        for (int k = 0; k < NP; ++k) {
            const int ih = ihb + (prc[k] & 0xFFFF), iw = iwb + (prc[k] >> 16);
            const bool ok = (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
            const uint32_t off = (uint32_t)(gbase + prel[k]) * 2u;
#pragma unroll
            for (int u = 0; u < NL; ++u) pf[k][u] = bload16(rx, ok ? off + 16u * u : kOob);
        }
    };
    window_loads(0, 0, ntl_g > 0);

    // ---- input scale, per-channel constants --------------------------------
    uint32_t slot_raw[igemm::kMaxSlotReads / 64];
    if constexpr (INT8) igemm::in_slot_loads(p, lane, slot_raw);
    const rsrc_t rb = make_rsrc(p.bias, (uint32_t)p.OC * 4u);
    const rsrc_t rsc = make_rsrc(p.w_scale, INT8 ? (uint32_t)p.OC * 4u : 0u);
    const uint32_t cofs = tid < NOCB && n0 + tid < p.OC ? (uint32_t)(n0 + tid) * 4u : kOob;
    const float bias_v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, cofs, 0, 0));
    float scale_v = 0.0f;
    if constexpr (INT8) scale_v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsc, cofs, 0, 0));
    float bias2_v = 0.0f;
    if constexpr (F2) {
        const rsrc_t rb2 = make_rsrc(h.c2.bias, (uint32_t)h.c2.OC * 4u);
        bias2_v = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(rb2, tid < NOCB && tid < h.c2.OC ? (uint32_t)tid * 4u : kOob, 0, 0));
    }

    // ---- weights: piece (chunk, k step, half, oc row) at LDS byte
    // (((ch * nks + ks) * 2 + half) * NOCB + row) * 16, written by the loads
    // directly (lane l of a wave's 64 pieces lands at the wave's base + 16 l;
    // 2 * NOCB is a multiple of 64, so no wave's pieces straddle the end) ----
    {
        const int wpieces = h.wbytes >> 4;
        for (int e0 = wave * 64; e0 < wpieces; e0 += NT) {
            const uint32_t e = (uint32_t)(e0 + lane);
            const int rest = (int)(e / (uint32_t)NOCB);
            const int row = (int)e - rest * NOCB;
            const int cks = rest >> 1, hf = rest & 1;
            const int ch = (int)fdiv((uint32_t)cks, h.fd_nks);
            const int ks = cks - ch * h.nks;
            const int kl = ks * KSUB + hf * CPP;  // chunk-local k = tap * CC + c
            const int tap = (int)fdiv((uint32_t)kl, h.fd_cc);
            const int k = tap * p.C + ch * h.CC + (kl - tap * h.CC);
            const bool ok = tap < 9 && n0 + row < p.OCp;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(lds + e0 * 16), 16,
                                                      ok ? (uint32_t)((n0 + row) * p.Kp + k) * ESZ : kOob, 0, 0, 0);
        }
    }

    // ---- tables (ALU only while the loads are in flight) -------------------
    for (int e = tid; e < 2 * h.nks; e += NT) {
        const int kl = (e >> 1) * KSUB + (e & 1) * CPP;
        const int tap = (int)fdiv((uint32_t)kl, h.fd_cc);
        int off = 0;  // padding k: any in-window address, zero weights
        if (tap < 9) {
            const int ky = tap / 3, kx = tap - (tap / 3) * 3;
            off = (((kl - tap * h.CC) / CPP) * h.NPIX + ky * h.ICOL + kx) * 16;
        }
        l_toff[e] = off;
    }
    // step-0 tap offset of this lane's half (the table's first entries)
    int t0;
    {
        const int kl = hi * CPP;
        const int tap = (int)fdiv((uint32_t)kl, h.fd_cc);
        const int ky = tap / 3, kx = tap - (tap / 3) * 3;
        t0 = (((kl - tap * h.CC) / CPP) * h.NPIX + ky * h.ICOL + kx) * 16;
    }
    // window byte offset of each position subtile's output position; its
    // place (r, c) in the tile, or -1 past the tile
    int bofs[MQ], prc_out[MQ];
    const int tpos = h.TR * h.TC;
#pragma unroll
    for (int q = 0; q < MQ; ++q) {
        const int pl = (gwave * MQ + q) * 32 + l32;
        const int pc = min(pl, tpos - 1);
        const int r = (int)fdiv((uint32_t)pc, h.fd_tc);
        const int c = pc - r * h.TC;
        bofs[q] = ((r * S) * h.ICOL + c * S) * 16;
        prc_out[q] = pl < tpos ? (r | (c << 16)) : -1;
    }
    const int abase = (hi * NOCB + l32) * 16;  // this lane's A piece in a k step's [half][oc] block
    if (tid < NOCB / 16) l_slots[tid] = 0u;
    if (tid < NG) l_gbar[tid] = 0u;
    if constexpr (F2) {
        if (tid < NOCB / 16) l_slots2[tid] = 0u;
        if (tid < NOCB) l_bias2[tid] = bias2_v;
    }
    float s_q = 0.0f, in_scale = 0.0f;
    if constexpr (INT8) igemm::in_slot_scale(slot_raw, s_q, in_scale);
    if (tid < NOCB) {
        l_bias[tid] = bias_v;
        if constexpr (INT8) l_scale[tid] = in_scale * scale_v;
    }
    // the weight loads into LDS complete before any wave passes the first
    // barrier; every load issued so far is needed by the first iteration
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    // two groups: the weights and tables written by all waves are complete
    // before either group reads them (one group's barrier does not cover
    // the other's loads)
    if constexpr (NG == 2) __syncthreads();

    const int jmax = min(NQ * 2, (p.OCp - n0) >> 4);  // 16-channel groups of the block with channels
    float gmax[NQ * 2], gmax2[F2 ? NQ * 2 : 1];
#pragma unroll
    for (int g = 0; g < NQ * 2; ++g) gmax[g] = 0.0f;
#pragma unroll
    for (int g = 0; g < (F2 ? NQ * 2 : 1); ++g) gmax2[g] = 0.0f;
    int yo[MQ], ro[MQ], mo[MQ], yo2[F2 ? MQ : 1];
    auto out_pos = [&](int tl, bool valid) {
        int n, oh0, ow0;
        tile_pos(tl, n, oh0, ow0);
#pragma unroll
        for (int q = 0; q < MQ; ++q) {
            const int oh = oh0 + (prc_out[q] & 0xFFFF), ow = ow0 + (prc_out[q] >> 16);
            const bool ok = valid && prc_out[q] >= 0 && oh < p.OH && ow < p.OW;
            const int pos = oh * p.OW + ow;
            yo[q] = ok ? n * (int)p.y_nstride + pos * p.y_cstride : -1;
            ro[q] = n * (int)p.r_nstride + pos * p.r_cstride;
            mo[q] = n * p.OH * p.OW + pos;
            if constexpr (F2) yo2[q] = ok ? n * (int)h.c2.y_nstride + pos * h.c2.y_cstride : -1;
        }
    };

    const bool out_f32 = EPI == igemm::kEpiAny && (p.flags & kConvOutF32);
    const bool do_res = igemm::epi_res<EPI>(p);
    const rsrc_t ry = make_rsrc(p.y, p.y_bytes);
    const rsrc_t rr = make_rsrc(p.res, p.r_bytes);
    const rsrc_t racc = make_rsrc(p.acc_out, p.acc_out ? (uint32_t)p.M * (uint32_t)p.OC * 4u : 0u);
    const rsrc_t rw2 = make_rsrc(F2 ? h.c2.w : nullptr, F2 ? (uint32_t)h.c2.OCp * (uint32_t)h.c2.Kp * 2u : 0u);
    const rsrc_t ry2 = make_rsrc(F2 ? h.c2.y : nullptr, F2 ? h.c2.y_bytes : 0u);
    const bool silu2 = F2 && (h.c2.flags & kConvSilu);
    const bool out2_f32 = F2 && (h.c2.flags & kConvOutF32);

    acc_t acc[MQ][NQ];
#pragma unroll
    for (int q = 0; q < MQ; ++q)
#pragma unroll
        for (int j = 0; j < NQ; ++j) acc[q][j] = acc_t{};
    v2i rv[MQ][NQ][4];

    const int wstep = 2 * NOCB * 16;  // LDS bytes of one k step's weights
    uint8_t* const win = lds + h.wbytes + grp_id * 2 * h.tbytes;
    const int total = ntl_g * h.nch;
    int tl = 0, ch = 0;
    for (int i = 0; i < total; ++i) {
        uint8_t* const tb = win + (i & 1) * h.tbytes;
        // this iteration's window -> LDS (int8: quantized once here)
#pragma unroll
        for (int k = 0; k < NP; ++k) {
            const int e = gtid + k * NTG;
            if (e < h.npiece) {
                if constexpr (INT8) {
                    const v2i lo = quant8(pf[k][0], s_q), hq = quant8(pf[k][1], s_q);
                    *reinterpret_cast<v4i*>(tb + e * 16) = v4i{lo[0], lo[1], hq[0], hq[1]};
                } else {
                    *reinterpret_cast<v4i*>(tb + e * 16) = pf[k][0];
                }
            }
        }
        const bool tile_end = ch == h.nch - 1;
        out_pos(tl, tile_end);
        if (do_res) {
#pragma unroll
            for (int q = 0; q < MQ; ++q)
#pragma unroll
                for (int j = 0; j < NQ; ++j)
#pragma unroll
                    for (int j4 = 0; j4 < 4; ++j4) {
                        const int oc0 = n0 + j * 32 + j4 * 8 + hi * 4;
                        const bool ok = oc0 < p.OC && yo[q] >= 0;
                        rv[q][j][j4] =
                            __builtin_amdgcn_raw_buffer_load_b64(rr, ok ? (uint32_t)(ro[q] + oc0) * 2u : kOob, 0, 0);
                    }
        }
        int ntl_ = tl, nch_ = ch + 1;
        if (nch_ == h.nch) {
            nch_ = 0;
            ++ntl_;
        }
        window_loads(min(ntl_, ntl_g - 1), nch_, ntl_ < ntl_g);
        if constexpr (NG == 1) __syncthreads();
        else group_barrier(&l_gbar[grp_id], (uint32_t)(i + 1) * NWG);

        // k steps of the chunk, software-pipelined two steps deep: the LDS
        // operands of step s + 2 are read before the MFMAs of step s (every
        // fetch is issued, past the last step it re-reads the last one, so
        // the count of reads in flight is the same on every path)
        const uint8_t* const wb = lds + ch * h.nks * wstep + abase;
        int tn = t0;
        auto fetch = [&](int s, v4i (&A)[NQ], v4i (&B)[MQ]) {
            const int toff = tn;
            tn = l_toff[min(s + 1, h.nks - 1) * 2 + hi];
#pragma unroll
            for (int j = 0; j < NQ; ++j) A[j] = *reinterpret_cast<const v4i*>(wb + s * wstep + j * 512);
#pragma unroll
            for (int q = 0; q < MQ; ++q) B[q] = *reinterpret_cast<const v4i*>(tb + bofs[q] + toff);
        };
        auto mma = [&](const v4i (&A)[NQ], const v4i (&B)[MQ]) {
#pragma unroll
            for (int q = 0; q < MQ; ++q)
#pragma unroll
                for (int j = 0; j < NQ; ++j) {
                    if constexpr (INT8)
                        acc[q][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[j], B[q], acc[q][j], 0, 0, 0);
                    else
                        acc[q][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, A[j]),
                                                                           __builtin_bit_cast(v8h, B[q]),
                                                                           acc[q][j], 0, 0, 0);
                }
        };
        const int last = h.nks - 1;
        v4i A0[NQ], B0[MQ], A1[NQ], B1[MQ], A2[NQ], B2[MQ];
        fetch(0, A0, B0);
        fetch(min(1, last), A1, B1);
        int s = 0;
        for (; s + 3 <= h.nks; s += 3) {
            fetch(s + 2, A2, B2);
            __builtin_amdgcn_sched_barrier(0);
            mma(A0, B0);
            __builtin_amdgcn_sched_barrier(0);
            fetch(min(s + 3, last), A0, B0);
            __builtin_amdgcn_sched_barrier(0);
            mma(A1, B1);
            __builtin_amdgcn_sched_barrier(0);
            fetch(min(s + 4, last), A1, B1);
            __builtin_amdgcn_sched_barrier(0);
            mma(A2, B2);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (s < h.nks) mma(A0, B0);
        if (s + 1 < h.nks) mma(A1, B1);

        // ---- epilogue at a tile's end: lane l holds, for position subtile q
        // and channel subtile j, channels 8 j4 + 4 hi + r (r < 4) of position
        // (wave * MQ + q) * 32 + l % 32 in acc[q][j][4 j4 + r] ----
        if (F2 && tile_end) {
            // fused 1x1: y1 = fp16(silu(acc + bias)) is the B operand of a
            // second product over the block's channels, out = W2 y1 + bias2.
            // k step k2 of that product takes channels 16 k2 + 8 hi .. + 7 of
            // y1 in a lane: four of them the lane holds (rows 8 j4 + 4 hi + r
            // of subtile k2 / 2, j4 = 2 (k2 % 2) + hi), four its partner lane
            // (lane ^ 32) does.
            // The W2 rows of an output subtile (all its k steps) are loaded
            // together, one subtile ahead: the first before y1 is formed, the
            // next ones under the current subtile's products and stores (loaded
            // at their use, each product would wait out a load of its own).
            v4i a2c[NQ * 2], a2n[NQ * 2];
            auto w2_loads = [&](int j2, v4i (&a)[NQ * 2]) {
                const int row2 = j2 * 32 + l32;
#pragma unroll
                for (int k2 = 0; k2 < NQ * 2; ++k2)
                    a[k2] = bload16(rw2, row2 < h.c2.OCp ? (uint32_t)(row2 * h.c2.Kp + k2 * 16 + hi * 8) * 2u : kOob);
            };
            w2_loads(0, a2c);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < MQ; ++q) {
                v4i b2[NQ * 2];
#pragma unroll
                for (int j = 0; j < NQ; ++j) {
                    uint32_t h2[4][2];
#pragma unroll
                    for (int j4 = 0; j4 < 4; ++j4) {
                        const int lc = j * 32 + j4 * 8 + hi * 4;
                        float v[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) v[r] = silu(acc[q][j][4 * j4 + r] + l_bias[lc + r]);
                        const __half2 a = __floats2half2_rn(v[0], v[1]), c = __floats2half2_rn(v[2], v[3]);
                        __builtin_memcpy(&h2[j4][0], &a, 4);
                        __builtin_memcpy(&h2[j4][1], &c, 4);
                    }
#pragma unroll
                    for (int m = 0; m < 2; ++m) b2[2 * j + m] = half_swap_operand(h2[2 * m], h2[2 * m + 1]);
                }
#pragma unroll
                for (int j2 = 0; j2 < NQ; ++j2) {
                    if (j2 + 1 < NQ) w2_loads(j2 + 1, a2n);
                    else if (q + 1 < MQ) w2_loads(0, a2n);
                    __builtin_amdgcn_sched_barrier(0);
                    v16f acc2{};
#pragma unroll
                    for (int k2 = 0; k2 < NQ * 2; ++k2)
                        acc2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a2c[k2]),
                                                                      __builtin_bit_cast(v8h, b2[k2]), acc2, 0, 0, 0);
#pragma unroll
                    for (int j4 = 0; j4 < 4; ++j4) {
                        const int oc0 = j2 * 32 + j4 * 8 + hi * 4;
                        float v[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            v[r] = acc2[4 * j4 + r] + l_bias2[oc0 + r];
                            if (silu2) v[r] = silu(v[r]);
                        }
                        const bool ok = oc0 < h.c2.OC && yo2[q] >= 0;
                        const float m4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
                        gmax2[j2 * 2 + (j4 >> 1)] = fmaxf(gmax2[j2 * 2 + (j4 >> 1)], ok ? m4 : 0.0f);
                        if (out2_f32) {
                            const v4i o{__float_as_int(v[0]), __float_as_int(v[1]), __float_as_int(v[2]),
                                        __float_as_int(v[3])};
                            __builtin_amdgcn_raw_buffer_store_b128(o, ry2, ok ? (uint32_t)(yo2[q] + oc0) * 4u : kOob,
                                                                   0, 0);
                        } else {
                            const __half2 oh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                            v2i o;
                            __builtin_memcpy(&o, oh, 8);
                            __builtin_amdgcn_raw_buffer_store_b64(o, ry2, ok ? (uint32_t)(yo2[q] + oc0) * 2u : kOob,
                                                                  0, 0);
                        }
                    }
#pragma unroll
                    for (int k2 = 0; k2 < NQ * 2; ++k2) a2c[k2] = a2n[k2];
                }
            }
#pragma unroll
            for (int q = 0; q < MQ; ++q)
#pragma unroll
                for (int j = 0; j < NQ; ++j) acc[q][j] = acc_t{};
        } else if (tile_end) {
#pragma unroll
            for (int q = 0; q < MQ; ++q)
#pragma unroll
                for (int j = 0; j < NQ; ++j)
#pragma unroll
                    for (int j4 = 0; j4 < 4; ++j4) {
                        const int lc = j * 32 + j4 * 8 + hi * 4;
                        const int oc0 = n0 + lc;
                        float bv[4], wv[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            bv[r] = l_bias[lc + r];
                            wv[r] = INT8 ? l_scale[lc + r] : 0.0f;
                        }
                        typedef typename std::conditional<INT8, v4i, v4f>::type a4_t;
                        const a4_t a4{acc[q][j][4 * j4], acc[q][j][4 * j4 + 1], acc[q][j][4 * j4 + 2],
                                      acc[q][j][4 * j4 + 3]};
                        float v[4];
                        igemm::epi_values<INT8, EPI>(p, a4, bv, wv, rv[q][j][j4], v);
                        const bool ok = oc0 < p.OC && yo[q] >= 0;
                        const float m4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
                        gmax[j * 2 + (j4 >> 1)] = fmaxf(gmax[j * 2 + (j4 >> 1)], ok ? m4 : 0.0f);
                        if (out_f32) {
                            const v4i o{__float_as_int(v[0]), __float_as_int(v[1]), __float_as_int(v[2]),
                                        __float_as_int(v[3])};
                            __builtin_amdgcn_raw_buffer_store_b128(o, ry, ok ? (uint32_t)(yo[q] + oc0) * 4u : kOob, 0,
                                                                   0);
                        } else {
                            const __half2 oh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                            v2i o;
                            __builtin_memcpy(&o, oh, 8);
                            __builtin_amdgcn_raw_buffer_store_b64(o, ry, ok ? (uint32_t)(yo[q] + oc0) * 2u : kOob, 0,
                                                                  0);
                        }
                        if constexpr (INT8 && EPI == igemm::kEpiAny) {
                            // int32 accumulators (acc_out; a zero-byte view drops them)
                            const v4i av{(int)a4[0], (int)a4[1], (int)a4[2], (int)a4[3]};
                            __builtin_amdgcn_raw_buffer_store_b128(
                                av, racc, ok ? (uint32_t)(mo[q] * p.OC + oc0) * 4u : kOob, 0, 0);
                        }
                    }
#pragma unroll
            for (int q = 0; q < MQ; ++q)
#pragma unroll
                for (int j = 0; j < NQ; ++j) acc[q][j] = acc_t{};
        }
        tl = ntl_;
        ch = nch_;
    }

    if constexpr (F2) {
        const int jmax2 = min(NQ * 2, h.c2.OCp >> 4);
        igemm::flush_slots<NQ * 2>(h.c2, gmax2, 0, jmax2, 0xFFFFFFFFu, out2_f32, l_slots2);
    } else {
        igemm::flush_slots<NQ * 2>(p, gmax, n0, jmax, 0xFFFFFFFFu, out_f32, l_slots);
    }
}

// Blocks of one instance the GPU holds at once with lds_bytes of dynamic LDS.
template <bool INT8, int MQ, int NQ, int NP, int EPI, int NW, bool F2, int NG>
int m32_resident_blocks(int lds_bytes) {
    int per_cu = 0, cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, conv3x3_m32_kernel<INT8, MQ, NQ, NP, EPI, NW, F2, NG>, NW * 64,
                                                     (size_t)lds_bytes) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu < 1 ||
        cus < 1)
        return 256;
    return per_cu * cus;
}

// Persistent grid: every resident block slot gets one contiguous run of
// position tiles of one channel tile.
template <bool INT8, int MQ, int NQ, int NP, int EPI, int NW, bool F2 = false, int NG = 1>
hipError_t m32_launch_cfg(M32Params h, hipStream_t stream) {
    const int lds_bytes = h.wbytes + NG * 2 * h.tbytes;
    const int cap = m32_resident_blocks<INT8, MQ, NQ, NP, EPI, NW, F2, NG>(lds_bytes);
    int groups = h.ntile;
    if ((int64_t)h.ntile * h.c.ntn > cap) groups = std::max(1, cap / h.c.ntn);
    h.c.per = (h.ntile + groups - 1) / groups;
    groups = (h.ntile + h.c.per - 1) / h.c.per;
    const int64_t blocks = (int64_t)groups * h.c.ntn;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((conv3x3_m32_kernel<INT8, MQ, NQ, NP, EPI, NW, F2, NG>), dim3((unsigned)blocks), dim3(NW * 64),
                       (size_t)lds_bytes, stream, h);
    return hipGetLastError();
}

// Every (MQ, NQ, NP, NW, NG) of one (INT8, EPI) family.
template <bool INT8, int EPI>
hipError_t m32_launch_family(const M32Params& h, int mq, int nq, int np, int nw, int ng, hipStream_t stream) {
    // 8 waves in two groups of 4 (their own window buffers and barriers)
#define AEXRT_M32_CASE2G(M, N, P) \
    if (nw == 8 && ng == 2 && mq == M && nq == N && np == P) return m32_launch_cfg<INT8, M, N, P, EPI, 8, false, 2>(h, stream);
    AEXRT_M32_CASE2G(1, 1, 4) AEXRT_M32_CASE2G(1, 2, 4) AEXRT_M32_CASE2G(1, 3, 4) AEXRT_M32_CASE2G(2, 1, 4)
    AEXRT_M32_CASE2G(2, 2, 4) AEXRT_M32_CASE2G(1, 1, 8) AEXRT_M32_CASE2G(1, 2, 8) AEXRT_M32_CASE2G(2, 1, 8)
#undef AEXRT_M32_CASE2G
    if (ng != 1) return hipErrorInvalidValue;
#define AEXRT_M32_CASE(M, N, P) \
    if (nw == 4 && mq == M && nq == N && np == P) return m32_launch_cfg<INT8, M, N, P, EPI, 4>(h, stream);
    AEXRT_M32_CASE(1, 1, 4) AEXRT_M32_CASE(1, 2, 4) AEXRT_M32_CASE(1, 3, 4) AEXRT_M32_CASE(1, 4, 4)
    AEXRT_M32_CASE(2, 1, 4) AEXRT_M32_CASE(2, 2, 4) AEXRT_M32_CASE(2, 3, 4) AEXRT_M32_CASE(2, 4, 4)
    AEXRT_M32_CASE(4, 1, 4) AEXRT_M32_CASE(4, 2, 4)
    AEXRT_M32_CASE(1, 1, 8) AEXRT_M32_CASE(1, 2, 8) AEXRT_M32_CASE(1, 3, 8) AEXRT_M32_CASE(1, 4, 8)
    AEXRT_M32_CASE(2, 1, 8) AEXRT_M32_CASE(2, 2, 8) AEXRT_M32_CASE(2, 3, 8) AEXRT_M32_CASE(4, 1, 8)
#undef AEXRT_M32_CASE
    // 8 waves: two per SIMD, so one wave's epilogue and window staging overlap
    // another's MFMAs, for the same weights in LDS
#define AEXRT_M32_CASE8(M, N, P) \
    if (nw == 8 && mq == M && nq == N && np == P) return m32_launch_cfg<INT8, M, N, P, EPI, 8>(h, stream);
    AEXRT_M32_CASE8(1, 1, 4) AEXRT_M32_CASE8(1, 2, 4) AEXRT_M32_CASE8(1, 3, 4) AEXRT_M32_CASE8(2, 1, 4)
    AEXRT_M32_CASE8(2, 2, 4) AEXRT_M32_CASE8(1, 1, 8) AEXRT_M32_CASE8(1, 2, 8) AEXRT_M32_CASE8(2, 1, 8)
#undef AEXRT_M32_CASE8
    return hipErrorInvalidValue;
}

// fp16 SiLU 3x3 convs with a fused 1x1 (F2): tiles whose block covers
// every output channel (nq 2 or 3: up to 64 / 96 channels).
hipError_t m32_launch_f2(const M32Params& h, int mq, int nq, int np, int nw, int ng, hipStream_t stream);

#define AEXRT_M32_FAMILIES(X) X(true, 0) X(true, 1) X(true, 2) X(false, 0) X(false, 1)
#define AEXRT_M32_EXTERN(I, E) \
    extern template hipError_t m32_launch_family<I, E>(const M32Params&, int, int, int, int, int, hipStream_t);
#define AEXRT_M32_INSTANCE(I, E) \
    template hipError_t m32_launch_family<I, E>(const M32Params&, int, int, int, int, int, hipStream_t);

}  // namespace m32
}  // namespace aexrt
