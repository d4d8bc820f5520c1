// A detect-head branch in one launch: 3x3 SiLU conv (a) -> 3x3 SiLU conv (b)
// -> 1x1 conv (c), fp16 NHWC in, fp16 or fp32 out, with the two
// intermediate maps kept in LDS (rounded to fp16 there, as the three
// separate convs store them) and never written to memory.
//
// A block owns one output tile (TR x TC positions of one image).  The 3x3
// conv b over the tile reads conv a's output over the tile plus a one-pixel
// border (the grid G, zero outside the image), which conv a computes from
// the input window X (G's in-image part plus one more pixel, zero outside
// the image): neighbouring tiles recompute their shared border of conv a.
//
//   prologue  biases -> LDS; X -> LDS (buffer_load ... lds, zeros outside the
//             image); G zeroed; tap tables
//   conv a    k steps of a in chunks of KC; the chunks' weights stream
//             through an LDS ring of D slots (loads of D - 1 chunks in
//             flight, one barrier per chunk); B operands from X
//   epilogue  bias + SiLU -> fp16 -> G (in-image positions only)
//   conv b    the ring continues with b's weights; B operands from G
//   epilogue  bias + SiLU -> fp16 -> the 1x1 conv c in registers (the
//             32x32-MFMA fused-1x1 scheme: a lane's outputs and its partner
//             lane's are the k slices of c's B operand) -> bias (+ SiLU) ->
//             y
//
// The MFMA is v_mfma_f32_32x32x16_f16 with the weights as the A operand
// (32 output channels) and 32 positions as B.  The 4 waves split the
// positions of a region (subtiles w, w + 4, ...; at most MQ each) and share
// the NQ 32-channel subtiles; weights and X/G use the LDS layouts of the
// 32x32-MFMA conv kernel (weights [k step][half][oc][16 B], maps
// [channel / 8][pixel][16 B]), so every operand read is one conflict-free
// ds_read_b128 per lane.
#pragma once
#include "conv_igemm.h"

namespace aexrt {

constexpr int kChainMaxSteps = 160;  // k steps of one 3x3 conv: 9 * C / 16

struct ChainParams {
    ConvParams a, b, c;  // a: x -> t1, b: t1 -> t2, c: t2 -> y (t1, t2 never stored)
    int TR, TC;          // output tile: rows x columns
    int ntc, tpi;        // tiles per tile row, per image
    int ntile;           // N * tpi
    int ka, kb;          // k steps of a (9 * a.C / 16) and of b (9 * b.C / 16)
    int nchunk_a, nchunk;  // weight chunks of a, of a and b
    int x_off, g_off;    // LDS byte offsets of the window X and the grid G (after the ring)
    uint32_t x_img, y_img;  // bytes of one image's input / output view
    FastDiv fd_tpi, fd_ntc;
    FastDiv fd_cs16a, fd_cs16b;  // 16-channel steps of a's and b's input (a.C / 16, b.C / 16)
};

namespace chain {

using igemm::bload16;
using igemm::kOob;
using igemm::make_rsrc;
using igemm::rsrc_t;
using igemm::v2i;
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kKC = 4;   // k steps per weight chunk
constexpr int kD = 4;    // ring slots (chunks in flight + the one computed)
constexpr int kNT = 256;

// floor(a / d) for 0 <= a < 2^20 and d >= 1, from inv = 1 / d (float,
// correctly rounded): (a + 0.5) / d lies at least 0.5 / d from an integer,
// and the two roundings move the product by less than (a / d) 2^-22, which is
// below 0.5 / d while a < 2^21.
__device__ __forceinline__ int small_div(int a, float inv) { return (int)(((float)a + 0.5f) * inv); }

// MQ: position subtiles per wave and region (regions of up to 128 MQ
// positions); with MQ = 1 the operands of the next chunk are read from LDS
// while the MFMAs of the current one run.  blk: the block's tile; lds: the
// dynamic LDS [ring: kD * CB][X][G]; the biases (128 floats each) and the
// tap tables in LDS too.  KG = 2: 8 waves, two groups of 4 over the same
// positions, group g taking k steps 2g, 2g + 1 of every chunk (two waves per
// SIMD issue into the matrix core); group 1's partial sums are added into
// group 0's through the window's LDS at each conv's end, and group 0 runs the
// epilogues.
template <int NQ, int MQ, int KG>
__device__ __forceinline__ void chain_block(const ChainParams& h, int blk, uint8_t* lds,
                                            float* l_bias_a, float* l_bias, float* l_bias2, int* l_tap_a,
                                            int* l_tap_b) {
    constexpr int NOCB = NQ * 32;                // output channels of the block (every channel of a, b, c)
    constexpr int CB = kKC * 2 * NOCB * 16;      // LDS bytes of one weight chunk
    constexpr int PT = kKC * 2 * NOCB / kNT;     // chunk loads per thread
    static_assert((kKC * 2 * NOCB) % kNT == 0, "a chunk is whole loads of every thread");
    static_assert(KG == 1 || (KG == 2 && MQ == 1), "two k groups with one position subtile per wave");
    constexpr int NT = kNT * KG;  // threads of the block
    constexpr int KS = kKC / KG;  // k steps of a chunk per group
    const ConvParams& pa = h.a;
    const ConvParams& pb = h.b;
    const ConvParams& pc = h.c;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int hi = lane >> 5;
    const int grp = KG == 1 ? 0 : wave >> 2;  // k group (wave-uniform)
    const int lw = wave & 3;                  // wave within its group: position subtiles lw, lw + 4, ...

    // ---- tile geometry (block-uniform) --------------------------------------
    const int n = (int)fdiv((uint32_t)blk, h.fd_tpi);
    const int t = blk - n * h.tpi;
    const int trow = (int)fdiv((uint32_t)t, h.fd_ntc);
    const int H = pa.H, W = pa.W;
    const int oh0 = trow * h.TR, ow0 = (t - trow * h.ntc) * h.TC;
    const int TRr = min(h.TR, H - oh0), TCr = min(h.TC, W - ow0);
    // G: rows oh0 - 1 .. oh0 + TRr, columns ow0 - 1 .. ow0 + TCr
    const int GW = TCr + 2, GNPIX = (TRr + 2) * GW;
    // conv a's region R1 = G inside the image; X = R1 plus a one-pixel border
    const int r1r = max(oh0 - 1, 0), r1c = max(ow0 - 1, 0);
    const int R1H = min(oh0 + TRr + 1, H) - r1r, R1W = min(ow0 + TCr + 1, W) - r1c;
    const int XW = R1W + 2, XNPIX = (R1H + 2) * XW;
    const int npos1 = R1H * R1W, npos2 = TRr * TCr;

    const rsrc_t rx = make_rsrc(static_cast<const uint8_t*>(pa.x) + (int64_t)n * pa.x_nstride * 2, h.x_img);
    const rsrc_t rwa = make_rsrc(pa.w, (uint32_t)pa.OCp * (uint32_t)pa.Kp * 2u);
    const rsrc_t rwb = make_rsrc(pb.w, (uint32_t)pb.OCp * (uint32_t)pb.Kp * 2u);

    // ---- biases -> LDS (loads straight into LDS: no register waits) ---------
    if (wave < 2) {
        const uint32_t row = (uint32_t)(wave * 64 + lane);
        const rsrc_t ra = make_rsrc(pa.bias, (uint32_t)pa.OC * 4u);
        const rsrc_t rb = make_rsrc(pb.bias, (uint32_t)pb.OC * 4u);
        const rsrc_t rc = make_rsrc(pc.bias, (uint32_t)pc.OC * 4u);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(l_bias_a + wave * 64), 4, row * 4u, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(l_bias + wave * 64), 4, row * 4u, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (lds_ptr_t)(l_bias2 + wave * 64), 4, row * 4u, 0, 0, 0);
    }

    // ---- window X -> LDS: piece e = plane * XNPIX + pixel, plane = 8 channels
    {
        const int npiece = (pa.C / 8) * XNPIX;
        const float inv_npix = 1.0f / (float)XNPIX, inv_xw = 1.0f / (float)XW;
        uint8_t* const xb = lds + h.x_off;
        for (int e0 = wave * 64; e0 < npiece; e0 += NT) {
            const int e = e0 + lane;
            const int pl = small_div(e, inv_npix);
            const int pix = e - pl * XNPIX;
            const int pr = small_div(pix, inv_xw);
            const int ih = r1r - 1 + pr, iw = r1c - 1 + (pix - pr * XW);
            const bool ok = e < npiece && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
            const uint32_t off = (uint32_t)((ih * W + iw) * pa.x_cstride + pl * 8) * 2u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(xb + e0 * 16), 16, ok ? off : kOob, 0, 0, 0);
        }
    }

    // ---- weight ring: chunk g (a's chunks, then b's) into slot g % kD -------
    // piece e = i * kNT + tid of a chunk: k step sl, half, weight row; the
    // per-lane part of its byte offset in a's and b's weights (kOob past the
    // rows), fixed for every chunk
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
        w_a[i] = row < pa.OCp ? (uint32_t)(row * pa.Kp + 16 * sl + 8 * half) * 2u : kOob;
        w_b[i] = row < pb.OCp ? (uint32_t)(row * pb.Kp + 16 * sl + 8 * half) * 2u : kOob;
    }
    auto issue = [&](int g) {
        if (tid >= kNT) return;  // the chunk loads are the first 4 waves'
        const bool isb = g >= h.nchunk_a;  // block-uniform
        const int s0 = (isb ? g - h.nchunk_a : g) * kKC;
        const int left = (isb ? h.kb : h.ka) - s0;  // k steps of the conv from this chunk on
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

    // ---- G zeroed, tap tables (ALU while the loads are in flight) -----------
    {
        uint8_t* const gb = lds + h.g_off;
        const int ng = NQ * 4 * GNPIX;
        for (int e = tid; e < ng; e += NT) *reinterpret_cast<v4i*>(gb + e * 16) = v4i{0, 0, 0, 0};
    }
    // k step s (k = tap * C + c, 16 channels of one tap), half hi: byte offset
    // of its plane and tap relative to the position's (0, 0) tap pixel in a map
    // of npix pixels, w per row (past the last step the last one's: its
    // weights are zero).  Tables [chunk][hi][k step of the chunk], one 16-byte
    // read per chunk and lane instead of the arithmetic per k step.
    auto tap_table = [&](int* tab, int C, int ks, int npix, int w) {
        const int nchunk = (ks + kKC - 1) / kKC;
        for (int e = tid; e < nchunk * 2 * kKC; e += NT) {
            const int c = e / (2 * kKC), r = e - c * (2 * kKC), hh = r / kKC, sl = r - hh * kKC;
            const int k0 = 16 * min(c * kKC + sl, ks - 1), tap = k0 / C, c0 = k0 - tap * C;
            tab[e] = (((c0 >> 3) + hh) * npix + (tap / 3) * w + tap % 3) * 16;
        }
    };
    tap_table(l_tap_a, pa.C, h.ka, XNPIX, XW);
    tap_table(l_tap_b, pb.C, h.kb, GNPIX, GW);
    // this wave's position subtiles: window / grid byte offset of each
    // position (clamped to the region), conv b's output offsets
    int bofs_a[MQ], bofs_b[MQ], yo[MQ];
    const int myq1 = min(MQ, max(0, ((npos1 + 31) >> 5) - lw + 3) >> 2);
    const int myq2 = min(MQ, max(0, ((npos2 + 31) >> 5) - lw + 3) >> 2);
    {
        const float inv_r1w = 1.0f / (float)R1W, inv_tc = 1.0f / (float)TCr;
#pragma unroll
        for (int q = 0; q < MQ; ++q) {
            const int pos = (lw + 4 * q) * 32 + l32;
            const int p1 = min(pos, npos1 - 1);
            const int r1 = small_div(p1, inv_r1w);
            bofs_a[q] = (r1 * XW + (p1 - r1 * R1W)) * 16;
            const int p2 = min(pos, npos2 - 1);
            const int r2 = small_div(p2, inv_tc);
            const int c2 = p2 - r2 * TCr;
            bofs_b[q] = (r2 * GW + c2) * 16;
            yo[q] = pos < npos2 ? ((oh0 + r2) * pc.OW + ow0 + c2) * pc.y_cstride : -1;
        }
    }
    const int abase = (hi * NOCB + l32) * 16;

    v16f acc[MQ][NQ];
#pragma unroll
    for (int q = 0; q < MQ; ++q)
#pragma unroll
        for (int j = 0; j < NQ; ++j) acc[q][j] = v16f{};

    // chunk c's loads are complete in every wave and its slot may be read
    // (and the slot of chunk c - 1 refilled); in-order load completion: the
    // loads issued after chunk c's are the (at most kD - 2) later chunks'.
    // A plain s_barrier after the waits (LDS writes: lgkmcnt(0)): a
    // workgroup fence would wait for every load in flight, the later chunks'
    // too, since LDS-DMA loads count as LDS writes.
    auto ring_wait = [&](int c) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads and writes done
        if (c + kD - 2 < h.nchunk && grp == 0) {  // group 1 issues no chunk loads
            // s_waitcnt vmcnt(PT * (kD - 2)) lgkmcnt(0): vmcnt bits 3:0 and 15:14, expcnt 7
            constexpr int vm = PT * (kD - 2);
            static_assert(vm < 64, "vmcnt field");
            __builtin_amdgcn_s_waitcnt((vm & 15) | ((vm >> 4) << 14) | 0x0070);
        } else {
            __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (c + kD - 1 < h.nchunk) issue(c + kD - 1);
    };
    // the operands of chunk c's k steps over a map (X or G) with its tap table
    // (this group's KS of the chunk's kKC k steps: steps grp * KS + i)
    struct Ops {
        v4i A[KS][NQ], B[KS][MQ];
    };
    typedef int vks __attribute__((ext_vector_type(KS)));
    auto fetch = [&](int c, int s0, int ks, const uint8_t* map, const int* taps, const int (&bofs)[MQ], Ops& o) {
        const uint8_t* const ws = lds + (c & (kD - 1)) * CB + abase + grp * KS * (2 * NOCB * 16);
        const vks tt = *reinterpret_cast<const vks*>(taps + ((s0 / kKC) * 2 + hi) * kKC + grp * KS);
        (void)ks;
#pragma unroll
        for (int sl = 0; sl < KS; ++sl) {
            const int to = tt[sl];
#pragma unroll
            for (int j = 0; j < NQ; ++j) o.A[sl][j] = *reinterpret_cast<const v4i*>(ws + sl * (2 * NOCB * 16) + j * 512);
#pragma unroll
            for (int q = 0; q < MQ; ++q) o.B[sl][q] = *reinterpret_cast<const v4i*>(map + bofs[q] + to);
        }
    };
    auto mma = [&](int s0, int ks, int myq, const Ops& o) {
#pragma unroll
        for (int sl = 0; sl < KS; ++sl) {
            if (s0 + grp * KS + sl >= ks) break;  // wave-uniform
#pragma unroll
            for (int q = 0; q < MQ; ++q) {
                if (q >= myq) break;  // wave-uniform
#pragma unroll
                for (int j = 0; j < NQ; ++j)
                    acc[q][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, o.A[sl][j]),
                                                                       __builtin_bit_cast(v8h, o.B[sl][q]), acc[q][j],
                                                                       0, 0, 0);
            }
        }
    };
    // one k step: the MFMAs of step sl of `cur` (every one, straight-line: past
    // the last k step the weights are zero, and a wave past the region
    // computes clamped positions it never stores), then the operand reads of
    // step sl of the next chunk into `nxt`, so that the reads run while the
    // matrix core works
    auto mma_fetch = [&](const Ops& cur, int cn, int s0n, int ks, const uint8_t* map, const int* taps,
                         const int (&bofs)[MQ], Ops& nxt, bool more) {
        const uint8_t* const ws = lds + (cn & (kD - 1)) * CB + abase + grp * KS * (2 * NOCB * 16);
        vks tt{};
        if (more) tt = *reinterpret_cast<const vks*>(taps + ((s0n / kKC) * 2 + hi) * kKC + grp * KS);
        (void)ks;
#pragma unroll
        for (int sl = 0; sl < KS; ++sl) {
#pragma unroll
            for (int q = 0; q < MQ; ++q)
#pragma unroll
                for (int j = 0; j < NQ; ++j)
                    acc[q][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, cur.A[sl][j]),
                                                                       __builtin_bit_cast(v8h, cur.B[sl][q]), acc[q][j],
                                                                       0, 0, 0);
            if (more) {  // block-uniform
                const int to = tt[sl];
#pragma unroll
                for (int j = 0; j < NQ; ++j)
                    nxt.A[sl][j] = *reinterpret_cast<const v4i*>(ws + sl * (2 * NOCB * 16) + j * 512);
#pragma unroll
                for (int q = 0; q < MQ; ++q) nxt.B[sl][q] = *reinterpret_cast<const v4i*>(map + bofs[q] + to);
            }
        }
    };
    // chunks [cb, ce) of one conv (k steps from (c - cb) * kKC)
    auto conv = [&](int cb, int ce, int ks, const uint8_t* map, const int* toff, const int (&bofs)[MQ], int myq) {
        if constexpr (MQ == 1) {
            // the next chunk's barrier, then this chunk's MFMAs interleaved with
            // the next chunk's operand reads
            Ops o0, o1;
            ring_wait(cb);
            fetch(cb, 0, ks, map, toff, bofs, o0);
            for (int c = cb; c < ce; c += 2) {
                if (c + 1 < ce) ring_wait(c + 1);
                mma_fetch(o0, c + 1, (c + 1 - cb) * kKC, ks, map, toff, bofs, o1, c + 1 < ce);
                if (c + 1 < ce) {
                    if (c + 2 < ce) ring_wait(c + 2);
                    mma_fetch(o1, c + 2, (c + 2 - cb) * kKC, ks, map, toff, bofs, o0, c + 2 < ce);
                }
            }
        } else {
            for (int c = cb; c < ce; ++c) {
                Ops o;
                ring_wait(c);
                fetch(c, (c - cb) * kKC, ks, map, toff, bofs, o);
                mma((c - cb) * kKC, ks, myq, o);
            }
        }
    };

    // group 1's partial sums added into group 0's, one 32-channel subtile at a
    // time through the window region (free after conv a's last chunk): 4 waves
    // x MQ x 16 floats x 64 lanes per pass
    auto reduce_groups = [&]() {
        if constexpr (KG == 2) {
            float* const red = reinterpret_cast<float*>(lds + h.x_off);
            auto bar = [] {
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
            };
#pragma unroll
            for (int j = 0; j < NQ; ++j) {
                bar();  // every wave done reading the window / the previous pass
                if (grp == 1) {
#pragma unroll
                    for (int q = 0; q < MQ; ++q)
#pragma unroll
                        for (int r = 0; r < 16; ++r) red[((lw * MQ + q) * 16 + r) * 64 + lane] = acc[q][j][r];
                }
                bar();
                if (grp == 0) {
#pragma unroll
                    for (int q = 0; q < MQ; ++q)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[q][j][r] += red[((lw * MQ + q) * 16 + r) * 64 + lane];
                }
            }
        }
    };

    // ---- conv a --------------------------------------------------------------
    conv(0, h.nchunk_a, h.ka, lds + h.x_off, l_tap_a, bofs_a, myq1);
    reduce_groups();
    // epilogue a: fp16(silu(acc + bias)) -> G at the position's grid pixel
    {
        uint8_t* const gb = lds + h.g_off;
        const int dr = r1r - (oh0 - 1), dc = r1c - (ow0 - 1);
        const float inv_r1w = 1.0f / (float)R1W;
#pragma unroll
        for (int q = 0; q < MQ; ++q) {
            const int pos = (lw + 4 * q) * 32 + l32;
            if (grp == 0 && q < myq1 && pos < npos1) {
                const int r = small_div(pos, inv_r1w);
                const int gp = (r + dr) * GW + (pos - r * R1W) + dc;
#pragma unroll
                for (int j = 0; j < NQ; ++j)
#pragma unroll
                    for (int j4 = 0; j4 < 4; ++j4) {
                        const int lc = j * 32 + j4 * 8 + hi * 4;
                        const __half2 o0 = __floats2half2_rn(silu(acc[q][j][4 * j4] + l_bias_a[lc]),
                                                             silu(acc[q][j][4 * j4 + 1] + l_bias_a[lc + 1]));
                        const __half2 o1 = __floats2half2_rn(silu(acc[q][j][4 * j4 + 2] + l_bias_a[lc + 2]),
                                                             silu(acc[q][j][4 * j4 + 3] + l_bias_a[lc + 3]));
                        const __half2 oh[2] = {o0, o1};
                        v2i o;
                        __builtin_memcpy(&o, oh, 8);
                        *reinterpret_cast<v2i*>(gb + ((j * 4 + j4) * GNPIX + gp) * 16 + hi * 8) = o;
                    }
            }
#pragma unroll
            for (int j = 0; j < NQ; ++j) acc[q][j] = v16f{};
        }
    }
    // ---- conv b (its first barrier orders the G writes before its reads) -----
    conv(h.nchunk_a, h.nchunk, h.kb, lds + h.g_off, l_tap_b, bofs_b, myq2);
    reduce_groups();
    if (grp != 0) return;  // the 1x1 and the stores: group 0

    // ---- epilogue b + the 1x1 conv c -------------------------------------------
    // y1 = fp16(silu(acc + bias_b)) is the B operand of c: k step k2 of c takes
    // channels 16 k2 + 8 hi .. + 7 of y1 in a lane, four of them the lane holds
    // (rows 8 j4 + 4 hi + r of subtile k2 / 2, j4 = 2 (k2 % 2) + hi) and four
    // its partner lane (lane ^ 32) does.
    const rsrc_t rw2 = make_rsrc(pc.w, (uint32_t)pc.OCp * (uint32_t)pc.Kp * 2u);
    const rsrc_t ry = make_rsrc(static_cast<uint8_t*>(pc.y) + (int64_t)n * pc.y_nstride *
                                    ((pc.flags & kConvOutF32) ? 4 : 2), h.y_img);
    const bool silu2 = (pc.flags & kConvSilu) != 0;
    const bool out_f32 = (pc.flags & kConvOutF32) != 0;
#pragma unroll
    for (int q = 0; q < MQ; ++q) {
        if (q >= myq2) break;  // wave-uniform
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
                const __half2 x0 = __floats2half2_rn(v[0], v[1]), x1 = __floats2half2_rn(v[2], v[3]);
                __builtin_memcpy(&h2[j4][0], &x0, 4);
                __builtin_memcpy(&h2[j4][1], &x1, 4);
            }
#pragma unroll
            for (int m = 0; m < 2; ++m) b2[2 * j + m] = half_swap_operand(h2[2 * m], h2[2 * m + 1]);
        }
#pragma unroll
        for (int j2 = 0; j2 < NQ; ++j2) {
            const int row2 = j2 * 32 + l32;
            v4i a2[NQ * 2];
#pragma unroll
            for (int k2 = 0; k2 < NQ * 2; ++k2)
                a2[k2] = bload16(rw2, row2 < pc.OCp ? (uint32_t)(row2 * pc.Kp + k2 * 16 + hi * 8) * 2u : kOob);
            v16f acc2{};
#pragma unroll
            for (int k2 = 0; k2 < NQ * 2; ++k2)
                acc2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a2[k2]),
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
                const bool ok = oc0 < pc.OC && yo[q] >= 0;
                if (out_f32) {
                    const v4i o{__float_as_int(v[0]), __float_as_int(v[1]), __float_as_int(v[2]), __float_as_int(v[3])};
                    __builtin_amdgcn_raw_buffer_store_b128(o, ry, ok ? (uint32_t)(yo[q] + oc0) * 4u : kOob, 0, 0);
                } else {
                    const __half2 oh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                    v2i o;
                    __builtin_memcpy(&o, oh, 8);
                    __builtin_amdgcn_raw_buffer_store_b64(o, ry, ok ? (uint32_t)(yo[q] + oc0) * 2u : kOob, 0, 0);
                }
            }
        }
    }
}

// One branch: one block per tile.
template <int NQ, int MQ, int KG>
__global__ __launch_bounds__(kNT * KG) void conv_chain_kernel(ChainParams h) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ __attribute__((aligned(16))) float l_bias_a[128], l_bias[128], l_bias2[128];
    __shared__ __attribute__((aligned(16))) int l_tap_a[2 * kChainMaxSteps], l_tap_b[2 * kChainMaxSteps];
    const int blk = xcd_remap(blockIdx.x, gridDim.x);
    chain_block<NQ, MQ, KG>(h, blk, lds, l_bias_a, l_bias, l_bias2, l_tap_a, l_tap_b);
}

// Two branches over one input (the head level's box and class branches): the
// first h0.ntile blocks run branch 0, the rest branch 1, so both fill the GPU
// together.
template <int NQ0, int NQ1, int MQ, int KG>
__global__ __launch_bounds__(kNT * KG) void conv_chain2_kernel(ChainParams h0, ChainParams h1) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ __attribute__((aligned(16))) float l_bias_a[128], l_bias[128], l_bias2[128];
    __shared__ __attribute__((aligned(16))) int l_tap_a[2 * kChainMaxSteps], l_tap_b[2 * kChainMaxSteps];
    const int blk = xcd_remap(blockIdx.x, gridDim.x);
    if (blk < h0.ntile)
        chain_block<NQ0, MQ, KG>(h0, blk, lds, l_bias_a, l_bias, l_bias2, l_tap_a, l_tap_b);
    else
        chain_block<NQ1, MQ, KG>(h1, blk - h0.ntile, lds, l_bias_a, l_bias, l_bias2, l_tap_a,
                             l_tap_b);
}

}  // namespace chain
}  // namespace aexrt
