// Wide-tile fp16 3x3 convolution (pad 1, stride 1 or 2) on gfx950 MFMA, for
// convs whose weights are too large to stay resident in LDS next to the
// input windows (the fp16 detection head: 64..256 input channels, 64 or 80
// output channels, 10x10 .. 40x40 maps).
//
// Every wave holds all output channels of the conv (JN 16-channel subtiles,
// JN * 16 >= OC) for PW 16-position subtiles, so the input is read once and
// each LDS operand read feeds JN or PW MFMAs.  A block (4 waves) owns TR x TC
// output positions of one image and walks its channels in chunks of CC: per
// chunk, the input window ((TR-1)S+3 x (TC-1)S+3 pixels x CC channels) and
// the chunk's weights (all output channels x 9 taps x CC channels) are staged
// from global memory through registers into LDS, double buffered, while the
// previous chunk is computed.  k inside a chunk is tap * CC + c in steps of
// 32 (one v_mfma_f32_16x16x32_f16 per subtile pair and step; 9 * CC is
// rounded up to 32 with zero weights).  Every iteration issues the same loads
// and stores (out of range when idle), so the compiler's wait counts leave the
// epilogue stores in flight.
//
// Epilogue: bias, optional SiLU, fp16 or fp32 output, max|y| folded into the
// output's amax slots.  No residual, no int32 accumulator output.
#pragma once
#include "conv_igemm.h"

namespace aexrt {

struct WideParams {
    ConvParams c;
    int TR, TC;      // output rows x columns of a position tile
    int IR, ICOL;    // its input window
    int CC;          // channels per chunk (C % CC == 0, CC % 8 == 0)
    int nch;         // chunks: C / CC
    int spc;         // 32-k steps per chunk: ceil(9 * CC / 32)
    int npieces;     // 16-byte pieces of one window: IR * ICOL * CC / 8
    int wpieces;     // 16-byte pieces of one chunk's weights: spc * R * 4
    int ntc, tpi, ntile;
    int tbytes;      // LDS bytes of one window buffer
    int wbytes;      // LDS bytes of one weight buffer
    int pstride;     // LDS bytes per window pixel: CC * 2
    FastDiv fd_cc8, fd_icol, fd_tc, fd_ntc, fd_tpi, fd_cc, fd_spc4;
};

constexpr int kWideMaxSpc = 72;  // 9 * 256 / 32

namespace wide {

using igemm::bload16;
using igemm::kOob;
using igemm::make_rsrc;
using igemm::rsrc_t;
using igemm::v2i;
using igemm::xcd_remap;

template <int JN, int PW, int NPW, int NWP, int EPI>
__global__ __launch_bounds__(256) void conv3x3_wide_kernel(WideParams h) {
    constexpr int R = JN * 16;  // output channels held by every wave
    const ConvParams& p = h.c;

    // [weights 0][weights 1][window 0][window 1]
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    // (k step, k group) -> byte offset of the tap and channels inside the
    // window, relative to the output position's (0, 0) tap
    __shared__ int l_toff[kWideMaxSpc * 4];
    __shared__ float l_bias[R];
    __shared__ uint32_t l_slots[JN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 15;
    const int grp = lane >> 4;

    const int b = xcd_remap(blockIdx.x, gridDim.x);
    const int pt0 = b * p.per;
    const int ntl = min(p.per, h.ntile - pt0);
    const int S = p.S;

    const rsrc_t rx = make_rsrc(p.x, p.x_bytes);
    const rsrc_t rw = make_rsrc(p.w, (uint32_t)p.OCp * (uint32_t)p.Kp * 2u);
    const rsrc_t rb = make_rsrc(p.bias, (uint32_t)p.OC * 4u);
    const float bias_v =
        __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, tid < p.OC && tid < R ? (uint32_t)tid * 4u : kOob, 0, 0));

    // ---- staging of one (tile, chunk): window pieces and weight pieces -------
    // window piece k of this thread: e = tid + 256 k -> pixel (ir, ic), 8-channel group
    int prc[NPW], prel[NPW], plds[NPW];
#pragma unroll
    for (int k = 0; k < NPW; ++k) {
        const int e = tid + k * 256;
        const int pix = (int)fdiv((uint32_t)e, h.fd_cc8);
        const int cp = e - pix * (h.CC >> 3);
        const int ir = (int)fdiv((uint32_t)pix, h.fd_icol);
        const int ic = pix - ir * h.ICOL;
        prc[k] = e < h.npieces ? (ir | (ic << 16)) : 0x7FFF;
        prel[k] = (ir * p.W + ic) * p.x_cstride + cp * 8;
        plds[k] = pix * h.pstride + cp * 16;
    }
    // weight piece k: e = tid + 256 k -> (step s, row oc, group g); LDS
    // [s][row][g][16 B], k = 32 s + 8 g (+0..7) = tap * CC + c
    int wrel[NWP];  // element offset inside the conv's [OCp][Kp] weights at chunk 0, or -1
#pragma unroll
    for (int k = 0; k < NWP; ++k) {
        const int e = tid + k * 256;
        const int s = (int)fdiv((uint32_t)e, h.fd_spc4);  // e / (R * 4)
        const int rg = e - s * R * 4;
        const int row = rg >> 2, g = rg & 3;
        const int kk = s * 32 + g * 8;
        const int tap = (int)fdiv((uint32_t)kk, h.fd_cc);
        const int c = kk - tap * h.CC;
        const bool ok = e < h.wpieces && tap < 9 && row < p.OCp;
        wrel[k] = ok ? row * p.Kp + tap * p.C + c : -1;
    }
    auto tile_pos = [&](int tl, int& n, int& oh0, int& ow0) {
        const int ti = pt0 + tl;
        n = (int)fdiv((uint32_t)ti, h.fd_tpi);
        const int rem = ti - n * h.tpi;
        const int tr = (int)fdiv((uint32_t)rem, h.fd_ntc);
        oh0 = tr * h.TR;
        ow0 = (rem - tr * h.ntc) * h.TC;
    };
    v4i pf[NPW], wf[NWP];
    auto stage_loads = [&](int tl, int ch, bool live) {
        int n, oh0, ow0;
        tile_pos(tl, n, oh0, ow0);
        const int ihb = live ? oh0 * S - 1 : -0x40000000;
        const int iwb = ow0 * S - 1;
        const int gbase = n * (int)p.x_nstride + ((oh0 * S - 1) * p.W + iwb) * p.x_cstride + ch * h.CC;
#pragma unroll
        for (int k = 0; k < NPW; ++k) {
            const int ih = ihb + (prc[k] & 0xFFFF), iw = iwb + (prc[k] >> 16);
            const bool ok = (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
            pf[k] = bload16(rx, ok ? (uint32_t)(gbase + prel[k]) * 2u : kOob);
        }
#pragma unroll
        for (int k = 0; k < NWP; ++k)
            wf[k] = bload16(rw, live && wrel[k] >= 0 ? (uint32_t)(wrel[k] + ch * h.CC) * 2u : kOob);
    };
    stage_loads(0, 0, ntl > 0);

    // ---- output side -----------------------------------------------------------
    const bool out_f32 = EPI == igemm::kEpiAny && (p.flags & kConvOutF32);
    const bool do_silu = EPI != igemm::kEpiAny || (p.flags & kConvSilu);
    const rsrc_t ry = make_rsrc(p.y, p.y_bytes);
    // the prologue issues an iteration's stores too (all dropped), so both
    // edges into the loop carry the same VMEM sequence
#pragma unroll
    for (int d = 0; d < JN * PW; ++d) __builtin_amdgcn_raw_buffer_store_b128(v4i{0, 0, 0, 0}, ry, kOob, 0, 0);

    // ---- tables --------------------------------------------------------------------
    for (int e = tid; e < h.spc * 4; e += 256) {
        const int kk = e * 8;  // (s * 4 + g) * 8
        const int tap = (int)fdiv((uint32_t)kk, h.fd_cc);
        int off = 0;  // padding k: any in-window address, zero weights
        if (tap < 9) {
            const int ky = tap / 3, kx = tap - (tap / 3) * 3;
            off = (ky * h.ICOL + kx) * h.pstride + (kk - tap * h.CC) * 2;
        }
        l_toff[e] = off;
    }
    int bofs[PW], prc_out[PW];
    const int tpos = h.TR * h.TC;
#pragma unroll
    for (int q = 0; q < PW; ++q) {
        const int pl = (wave * PW + q) * 16 + col;
        const int pc = min(pl, tpos - 1);
        const int r = (int)fdiv((uint32_t)pc, h.fd_tc);
        const int c = pc - r * h.TC;
        bofs[q] = ((r * S) * h.ICOL + c * S) * h.pstride;
        prc_out[q] = pl < tpos ? (r | (c << 16)) : -1;
    }
    if (tid < JN) l_slots[tid] = 0u;
    if (tid < R) l_bias[tid] = bias_v;

    float gmax[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j) gmax[j] = 0.0f;
    int yo[PW];
    auto out_pos = [&](int tl, bool valid) {
        int n, oh0, ow0;
        tile_pos(tl, n, oh0, ow0);
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const int oh = oh0 + (prc_out[q] & 0xFFFF), ow = ow0 + (prc_out[q] >> 16);
            const bool ok = valid && prc_out[q] >= 0 && oh < p.OH && ow < p.OW;
            yo[q] = ok ? n * (int)p.y_nstride + (oh * p.OW + ow) * p.y_cstride : -1;
        }
    };

    // accumulators; at a tile's end they are overwritten with the packed
    // outputs (fp16: .xy, fp32: all four), stored, and cleared
    v4f acc[JN][PW];
#pragma unroll
    for (int j = 0; j < JN; ++j)
#pragma unroll
        for (int q = 0; q < PW; ++q) acc[j][q] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    uint8_t* const wbase = lds;
    uint8_t* const tbase = lds + 2 * h.wbytes;
    const int total = ntl * h.nch;
    int tl = 0, ch = 0;
    for (int i = 0; i < total; ++i) {
        uint8_t* const wb = wbase + (i & 1) * h.wbytes;
        uint8_t* const tb = tbase + (i & 1) * h.tbytes;
#pragma unroll
        for (int k = 0; k < NPW; ++k)
            if (tid + k * 256 < h.npieces) *reinterpret_cast<v4i*>(tb + plds[k]) = pf[k];
#pragma unroll
        for (int k = 0; k < NWP; ++k)
            if (tid + k * 256 < h.wpieces) *reinterpret_cast<v4i*>(wb + (tid + k * 256) * 16) = wf[k];
        const bool tile_end = ch == h.nch - 1;
        out_pos(tl, tile_end);
        int ntl_ = tl, nch_ = ch + 1;
        if (nch_ == h.nch) {
            nch_ = 0;
            ++ntl_;
        }
        stage_loads(min(ntl_, ntl - 1), nch_, ntl_ < ntl);
        __syncthreads();

        // k steps of the chunk, software-pipelined: the LDS operands of step
        // s + 1 are read before the MFMAs of step s
        auto fetch = [&](int s, v8h (&A)[JN], v8h (&B)[PW]) {
            const int toff = l_toff[s * 4 + grp];
#pragma unroll
            for (int j = 0; j < JN; ++j)
                A[j] = *reinterpret_cast<const v8h*>(wb + ((s * R + j * 16 + col) * 4 + grp) * 16);
#pragma unroll
            for (int q = 0; q < PW; ++q) B[q] = *reinterpret_cast<const v8h*>(tb + bofs[q] + toff);
        };
        auto mma = [&](const v8h (&A)[JN], const v8h (&B)[PW]) {
#pragma unroll
            for (int j = 0; j < JN; ++j)
#pragma unroll
                for (int q = 0; q < PW; ++q)
                    acc[j][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[j], B[q], acc[j][q], 0, 0, 0);
        };
        v8h A0[JN], B0[PW], A1[JN], B1[PW];
        fetch(0, A0, B0);
        int s = 0;
        for (; s + 2 <= h.spc; s += 2) {
            fetch(s + 1, A1, B1);
            __builtin_amdgcn_sched_barrier(0);
            mma(A0, B0);
            __builtin_amdgcn_sched_barrier(0);
            if (s + 2 < h.spc) fetch(s + 2, A0, B0);
            __builtin_amdgcn_sched_barrier(0);
            mma(A1, B1);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (s < h.spc) mma(A0, B0);

        // ---- epilogue values at a tile's end; the stores on every iteration ----
        if (tile_end) {
#pragma unroll
            for (int j = 0; j < JN; ++j) {
                const int lc = j * 16 + grp * 4;
                const bool oc_ok = lc < p.OC;
#pragma unroll
                for (int q = 0; q < PW; ++q) {
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float t = acc[j][q][r] + (oc_ok ? l_bias[lc + r] : 0.0f);
                        v[r] = do_silu ? silu(t) : t;
                    }
                    const float m4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
                    gmax[j] = fmaxf(gmax[j], oc_ok && yo[q] >= 0 ? m4 : 0.0f);
                    if (out_f32) {
                        acc[j][q] = v4f{v[0], v[1], v[2], v[3]};
                    } else {
                        __half2 oh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                        float packed[2];
                        __builtin_memcpy(packed, oh, 8);
                        acc[j][q][0] = packed[0];
                        acc[j][q][1] = packed[1];
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < JN; ++j) {
            const int oc0 = j * 16 + grp * 4;
            const bool oc_ok = oc0 < p.OC;
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                const bool ok = oc_ok && yo[q] >= 0;
                const v4i o = __builtin_bit_cast(v4i, acc[j][q]);
                if (out_f32)
                    __builtin_amdgcn_raw_buffer_store_b128(o, ry, ok ? (uint32_t)(yo[q] + oc0) * 4u : kOob, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b64(v2i{o[0], o[1]}, ry, ok ? (uint32_t)(yo[q] + oc0) * 2u : kOob,
                                                          0, 0);
            }
        }
        if (tile_end) {
#pragma unroll
            for (int j = 0; j < JN; ++j)
#pragma unroll
                for (int q = 0; q < PW; ++q) acc[j][q] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
        tl = ntl_;
        ch = nch_;
    }

    igemm::flush_slots<JN>(p, gmax, 0, min(JN, p.OCp >> 4), 0xFFFFFFFFu, out_f32, l_slots);
}

}  // namespace wide

// Geometry of a wide tile (host); false when it does not fit the kernel.
// jn: channel subtiles of every wave; pw: position subtiles per wave.
bool wide_geometry(WideParams& h, int jn, int pw, int tr, int tc, int cc);
int enumerate_wide_choices(const ConvParams& p, ConvChoice* out, int cap);
hipError_t launch_conv_wide(const ConvParams& p, int epi, hipStream_t stream);

}  // namespace aexrt
