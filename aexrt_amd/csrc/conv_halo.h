// Halo-tile 3x3 convolution (pad 1, stride 1 or 2) on gfx950 MFMA: the same
// arithmetic as the implicit-GEMM kernel (int8 W8A8 with exact int32
// accumulation, or fp16 with fp32 accumulation), with the activations staged
// through LDS instead of being loaded per tap.
//
// A position tile is TR output rows x TC output columns of one image.  For
// each chunk of CC input channels the block loads the tile's input window
// (IR = (TR-1)*S + 3 rows x ICOL = (TC-1)*S + 3 columns, zero outside the
// image) once with 16-byte loads, quantizes it once (int8) and stores it in
// LDS as [row][col][CC]; the 9 taps of every output position then read their
// MFMA operands from there.  The implicit-GEMM kernel reads (and quantizes)
// every input element 9 times (once per tap), which makes its 3x3 layers
// VALU-bound; here each element is loaded and quantized (1 + halo) times.
//
// k order inside a chunk: k = tap * CC + c (tap = ky*3 + kx), padded to
// whole 64-k steps with zero weights; the block's weights for all chunks
// are gathered from the [OCp][Kp] (k = tap * C + c) layout into LDS once
// and stay resident while the block walks its run of position tiles.  The
// NW (4 or 8) waves of a block share the oc tile (JN 16-channel subtiles) and
// its weights in LDS (8 waves halve the LDS per wave for more waves per CU), and split
// the position tile (PW 16-position subtiles each).  The input of the next
// (tile, chunk) is loaded into registers while the current one is computed;
// two LDS tile buffers need one barrier per chunk.
//
// NCHW: the window is read from the fp32 NCHW network input (c_real <= 4
// channels) in 16-byte quads of 4 columns of one channel row, rounded to
// fp16 and scattered into the 8-channel zero-padded pixels of the LDS window,
// so the first conv runs without a separate layout-conversion pass (fp16
// only, CC = 8).  Quads start at columns that are multiples of 4 (TC * S % 4
// == 0 keeps that the same for every tile), so a quad is either wholly left
// of the image or starts inside it.
#pragma once
#include "conv_igemm.h"

namespace aexrt {

// Geometry of one halo-tile launch (host-computed).
struct HaloParams {
    ConvParams c;    // views, weights, flags; c.ntn / c.per / c.fd_ntn are this launch's
    int TR, TC;      // output rows x columns of a position tile
    int IR, ICOL;    // its input window
    int CC;          // channels per chunk (C % CC == 0, CC % 16 == 0)
    int nch;         // chunks: C / CC
    int spc;         // 64-k steps per chunk: ceil(9 * CC / 64)
    int npieces;     // 16-byte input pieces of one window: IR * ICOL * CC / 8
    int ntc;         // position tiles per image row band
    int tpi;         // position tiles per image
    int ntile;       // N * tpi
    int wbytes;      // LDS bytes of the resident weights
    int tbytes;      // LDS bytes of one window buffer
    int pstride;     // LDS bytes per window pixel: CC * element size, + 16 when that is an even multiple of 16
    FastDiv fd_cc8, fd_icol, fd_tc, fd_ntc, fd_tpi, fd_cc, fd_spc;
    int icol4;                // NCHW: column quads of a window row: (ICOL + 3 + 3) / 4
    FastDiv fd_icol4, fd_rq;  // NCHW: / icol4, / (IR * icol4)
};

// Largest k-step count of one chunk (table of tap offsets).
constexpr int kHaloMaxSpc = 32;
// 16-byte weight pieces per thread: the block's weights are at most
// 64 * NW * kHaloWeightRounds * 16 bytes (64 KB with 4 waves, 128 KB with 8).
constexpr int kHaloWeightRounds = 16;

namespace halo {

using igemm::bload16;
using igemm::Frag;
using igemm::kOob;
using igemm::make_rsrc;
using igemm::quant8;
using igemm::rsrc_t;
using igemm::v2i;
using igemm::xcd_remap;
typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <bool INT8, int JN, int PW, int NP, int EPI, bool NCHW = false, int NW = 4>
__global__ __launch_bounds__(NW * 64) void conv3x3_halo_kernel(HaloParams h) {
    constexpr int NT = NW * 64;  // threads of the block
    const ConvParams& p = h.c;
    constexpr int WQ = Frag<INT8>::wq;   // MFMAs (and weight pieces) per 64-k step
    constexpr int ESZ = Frag<INT8>::esz;
    constexpr int R = JN * 16;           // output channels of the block
    constexpr int PIECE = 8 * ESZ;       // LDS bytes of one 8-channel input piece
    static_assert(JN >= 1 && JN <= 8, "JN must be 1..8");
    static_assert(!(NCHW && INT8), "the NCHW input loader is fp16 only");
    typedef typename std::conditional<INT8, v4i, v4f>::type acc_t;

    // [weights: wbytes][window buffer 0: tbytes][window buffer 1: tbytes]
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    // (k step, k group, half) -> byte offset of the tap and channels inside
    // the window, relative to the output position's (0, 0) tap
    __shared__ int l_toff[kHaloMaxSpc * 4 * WQ];
    __shared__ float l_bias[R], l_scale[R];
    __shared__ uint32_t l_slots[JN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15;
    const int grp = lane >> 4;
    const int gsw = grp ^ ((col >> 2) & 3);  // LDS slot of k group grp in weight row col (mod 16)

    const int b = xcd_remap(blockIdx.x, gridDim.x);
    const int pg = (int)fdiv((uint32_t)b, p.fd_ntn);
    const int n0 = (b - pg * p.ntn) * R;
    const int pt0 = pg * p.per;
    const int ntl = min(p.per, h.ntile - pt0);
    const int jmax = min(JN, (p.OCp - n0) >> 4);
    const int S = p.S;

    const rsrc_t rx = make_rsrc(p.x, p.x_bytes);
    const int plane = p.H * p.W;  // NCHW: elements of one channel plane
    const rsrc_t rw = make_rsrc(p.w, (uint32_t)p.OCp * (uint32_t)p.Kp * ESZ);

    // ---- prologue loads: input scale, per-channel constants ----------------
    uint32_t slot_raw[igemm::kMaxSlotReads / 64];
    if constexpr (INT8) igemm::in_slot_loads(p, lane, slot_raw);
    const rsrc_t rb = make_rsrc(p.bias, (uint32_t)p.OC * 4u);
    const rsrc_t rsc = make_rsrc(p.w_scale, INT8 ? (uint32_t)p.OC * 4u : 0u);
    const uint32_t cofs = tid < R && n0 + tid < p.OC ? (uint32_t)(n0 + tid) * 4u : kOob;
    const float bias_v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, cofs, 0, 0));
    float scale_v = 0.0f;
    if constexpr (INT8) scale_v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsc, cofs, 0, 0));


    // ---- input windows -----------------------------------------------------
    // Piece k of this thread: e = tid + k * NT -> window pixel (ir, ic) and
    // 8-channel group; its LDS place is plds[k] = pixel * pstride + group * PIECE.
    // Pieces past the window get a row that fails every bounds test.
    // NCHW pieces: e -> channel c, window row ir, column quad q4 (columns
    // 4 q4 - 3 .. 4 q4 relative to the window's first column), packed as
    // ir | q4 << 12 | c << 24 in prc.
    int prc[NP], prel[NP], plds[NCHW ? 1 : NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) {
        const int e = tid + k * NT;
        if constexpr (NCHW) {
            const int c = (int)fdiv((uint32_t)e, h.fd_rq);
            const int rem = e - c * h.IR * h.icol4;
            const int ir = (int)fdiv((uint32_t)rem, h.fd_icol4);
            const int q4 = rem - ir * h.icol4;
            prc[k] = e < h.npieces ? (ir | (q4 << 12) | (c << 24)) : 0xFFF;
            prel[k] = c * plane + ir * p.W + 4 * q4;
        } else {
            const int pix = (int)fdiv((uint32_t)e, h.fd_cc8);
            const int cp = e - pix * (h.CC >> 3);
            const int ir = (int)fdiv((uint32_t)pix, h.fd_icol);
            const int ic = pix - ir * h.ICOL;
            prc[k] = e < h.npieces ? (ir | (ic << 16)) : 0x7FFF;
            prel[k] = (ir * p.W + ic) * p.x_cstride + cp * 8;
            plds[k] = pix * h.pstride + cp * PIECE;
        }
    }
    int pvalid[NCHW ? NP : 1];  // NCHW: columns of the quad inside the image (0..4)
    // tile tl of this block -> image, first output row and column
    auto tile_pos = [&](int tl, int& n, int& oh0, int& ow0) {
        const int ti = pt0 + tl;
        n = (int)fdiv((uint32_t)ti, h.fd_tpi);
        const int rem = ti - n * h.tpi;
        const int tr = (int)fdiv((uint32_t)rem, h.fd_ntc);
        oh0 = tr * h.TR;
        ow0 = (rem - tr * h.ntc) * h.TC;
    };
    v4i pf[NP];
    // loads of (tile tl, chunk ch) into pf, all NP issued (out of range when
    // !live: the first row is moved off the image)
    auto window_loads = [&](int tl, int ch, bool live) {
        int n, oh0, ow0;
        tile_pos(tl, n, oh0, ow0);
        const int ihb = live ? oh0 * S - 1 : -0x40000000;
        const int iwb = ow0 * S - 1;
        if constexpr (NCHW) {
            // quads start at column ow0 * S - 4 + 4 q4 (a multiple of 4)
            const int ws = ow0 * S - 4;
            const int gbase = n * (int)p.x_nstride + (oh0 * S - 1) * p.W + ws;
#pragma unroll
            for (int k = 0; k < NP; ++k) {
                const int ih = ihb + (prc[k] & 0xFFF), c0 = ws + 4 * ((prc[k] >> 12) & 0xFFF);
                const bool ok = (unsigned)ih < (unsigned)p.H && c0 >= 0 && c0 < p.W;
                pvalid[k] = ok ? min(4, p.W - c0) : 0;
                pf[k] = bload16(rx, ok ? (uint32_t)(gbase + prel[k]) * 4u : kOob);
            }
        } else {
            const int gbase = n * (int)p.x_nstride + ((oh0 * S - 1) * p.W + iwb) * p.x_cstride + ch * h.CC;
#pragma unroll
            for (int k = 0; k < NP; ++k) {
                const int ih = ihb + (prc[k] & 0xFFFF), iw = iwb + (prc[k] >> 16);
                const bool ok = (unsigned)ih < (unsigned)p.H && (unsigned)iw < (unsigned)p.W;
                pf[k] = bload16(rx, ok ? (uint32_t)(gbase + prel[k]) * 2u : kOob);
            }
        }
    };
    window_loads(0, 0, true);

    // ---- weights: [chunk * spc + s][h][row][64 B], gathered ----------------
    // 16-byte piece e: LDS slot e & 3 of row (e >> 2) % R, (gs, h) from the
    // rest.  Slot g' of a row holds k group g = g' ^ ((row >> 2) & 3) (chunk-
    // local k = g * 16 + h * 8 = tap * CC + c): the 16 rows an MFMA operand
    // read covers then spread one k group over all LDS banks.  The loads write LDS
    // directly (buffer_load ... lds: lane l of a wave's 64 pieces lands at
    // the wave's base + 16 l), so the weights take no registers and no LDS
    // store instructions; rounds past the image (a multiple of 64 pieces)
    // are skipped whole.
    const int wpieces = h.wbytes >> 4;
#pragma unroll
    for (int r = 0; r < kHaloWeightRounds; ++r) {
        const int e0 = r * NT + wave * 64;  // wave-uniform
        if (e0 < wpieces) {
            const uint32_t e = (uint32_t)(e0 + lane);
            const int row = (int)((e >> 2) % (uint32_t)R);
            const int g4 = (int)(e & 3u) ^ ((row >> 2) & 3);
            const int gsh = (int)((e >> 2) / (uint32_t)R);
            const int gs = gsh / WQ, hh = gsh - (gsh / WQ) * WQ;
            const int ch = (int)fdiv((uint32_t)gs, h.fd_spc);
            const int kk = ((gs - ch * h.spc) * 4 + g4) * 16 + hh * 8;
            const int tap = (int)fdiv((uint32_t)kk, h.fd_cc);
            const int k = tap * p.C + ch * h.CC + (kk - tap * h.CC);
            const bool ok = tap < 9 && n0 + row < p.OCp;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(lds + e0 * 16), 16,
                                                      ok ? (uint32_t)((n0 + row) * p.Kp + k) * ESZ : kOob, 0, 0, 0);
        }
    }

    // ---- output side -------------------------------------------------------
    const bool out_f32 = EPI == igemm::kEpiAny && (p.flags & kConvOutF32);
    const bool do_res = igemm::epi_res<EPI>(p);
    const rsrc_t ry = make_rsrc(p.y, p.y_bytes);
    const rsrc_t rr = make_rsrc(p.res, p.r_bytes);
    const rsrc_t racc = make_rsrc(p.acc_out, p.acc_out ? (uint32_t)p.M * (uint32_t)p.OC * 4u : 0u);
    // Every iteration issues the same VMEM operations after its window loads:
    // the tile's stores, out of range unless the tile ends there.  The loop
    // waits for a window load with a count of the operations issued after it,
    // which the compiler only gets exact when both edges into the loop header
    // carry the same sequence, so the prologue issues the stores of an
    // iteration too, all out of range (dropped).
#pragma unroll
    for (int d = 0; d < JN * PW * (EPI == igemm::kEpiAny && INT8 ? 2 : 1); ++d)
        __builtin_amdgcn_raw_buffer_store_b64(v2i{0, 0}, ry, kOob, 0, 0);

    // ---- tables (ALU only while the loads are in flight) -------------------
    for (int e = tid; e < h.spc * 4 * WQ; e += NT) {
        // e = (s * 4 + grp) * WQ + hh -> chunk-local k = (s * 4 + grp) * 16 + hh * 8
        const int kk = (e / WQ) * 16 + (e - (e / WQ) * WQ) * 8;
        const int tap = (int)fdiv((uint32_t)kk, h.fd_cc);
        int off = 0;  // padding k: any in-window address, zero weights
        if (tap < 9) {
            const int ky = tap / 3, kx = tap - (tap / 3) * 3;
            off = (ky * h.ICOL + kx) * h.pstride + (kk - tap * h.CC) * ESZ;
        }
        l_toff[e] = off;
    }
    // tap offsets of this lane's k groups at k step 0 (the table's first row)
    int t0[WQ];
#pragma unroll
    for (int hh = 0; hh < WQ; ++hh) {
        const int kk = grp * 16 + hh * 8;
        const int tap = (int)fdiv((uint32_t)kk, h.fd_cc);
        const int ky = tap / 3, kx = tap - (tap / 3) * 3;
        t0[hh] = (ky * h.ICOL + kx) * h.pstride + (kk - tap * h.CC) * ESZ;
    }
    // window byte offset of each position subtile's output position; output
    // position (r, c) of the tile, or -1 past the tile
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
    float s_q = 0.0f, in_scale = 0.0f;
    if constexpr (INT8) igemm::in_slot_scale(slot_raw, s_q, in_scale);
    if (tid < R) {
        l_bias[tid] = bias_v;
        if constexpr (INT8) l_scale[tid] = in_scale * scale_v;
    }
    if constexpr (NCHW) {
        // the padding channels of the window pixels are never written
        for (int e = tid; e < (2 * h.tbytes) >> 4; e += NT)
            *reinterpret_cast<v4i*>(lds + h.wbytes + e * 16) = v4i{0, 0, 0, 0};
        __syncthreads();  // zeros land before any thread's first window stores
    }

    float gmax[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j) gmax[j] = 0.0f;
    int yo[PW], ro[PW], mo[PW];
    v2i rv[JN][PW];
    // output offsets of tile tl (all -1 unless valid)
    auto out_pos = [&](int tl, bool valid) {
        int n, oh0, ow0;
        tile_pos(tl, n, oh0, ow0);
#pragma unroll
        for (int q = 0; q < PW; ++q) {
            const int oh = oh0 + (prc_out[q] & 0xFFFF), ow = ow0 + (prc_out[q] >> 16);
            const bool ok = valid && prc_out[q] >= 0 && oh < p.OH && ow < p.OW;
            const int pos = oh * p.OW + ow;
            yo[q] = ok ? n * (int)p.y_nstride + pos * p.y_cstride : -1;
            ro[q] = n * (int)p.r_nstride + pos * p.r_cstride;
            mo[q] = n * p.OH * p.OW + pos;
        }
    };

    acc_t acc[JN][PW];
#pragma unroll
    for (int j = 0; j < JN; ++j)
#pragma unroll
        for (int q = 0; q < PW; ++q) acc[j][q] = acc_t{0, 0, 0, 0};
    // packed outputs of the last finished tile (fp16: .xy; fp32: all four)
    v4i ov[JN][PW];

    // the weight loads into LDS complete before any wave passes the first
    // barrier (a wave with no window piece to store would not otherwise wait
    // for them); every load issued so far is needed by the first iteration
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    const int wstep = WQ * R * 64;  // LDS bytes of one k step's weights
    uint8_t* const win = lds + h.wbytes;
    const int total = ntl * h.nch;
    int tl = 0, ch = 0;
    for (int i = 0; i < total; ++i) {
        uint8_t* const tb = win + (i & 1) * h.tbytes;
        // this iteration's window -> LDS (int8: quantized once here)
#pragma unroll
        for (int k = 0; k < NP; ++k) {
            const int e = tid + k * NT;
            if (e < h.npieces) {
                if constexpr (INT8) {
                    *reinterpret_cast<v2i*>(tb + plds[k]) = quant8(pf[k], s_q);
                } else if constexpr (NCHW) {
                    // channel c of window pixels 4 q4 - 3 + j (those inside
                    // the window; columns past the image are zero)
                    const int ir = prc[k] & 0xFFF, q4 = (prc[k] >> 12) & 0xFFF, c = prc[k] >> 24;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int ic = 4 * q4 - 3 + j;
                        if (ic >= 0 && ic < h.ICOL) {
                            const __half v = __float2half(j < pvalid[k] ? __int_as_float(pf[k][j]) : 0.0f);
                            *reinterpret_cast<__half*>(tb + (ir * h.ICOL + ic) * h.pstride + c * 2) = v;
                        }
                    }
                } else {
                    *reinterpret_cast<v4i*>(tb + plds[k]) = pf[k];
                }
            }
        }
        const bool tile_end = ch == h.nch - 1;
        // output offsets and residual of the tile, issued before the next
        // window's loads so the epilogue's wait leaves those in flight
        out_pos(tl, tile_end);
        if constexpr (EPI != igemm::kEpiSilu) {
#pragma unroll
            for (int j = 0; j < JN; ++j)
#pragma unroll
                for (int q = 0; q < PW; ++q) {
                    const int oc0 = n0 + j * 16 + grp * 4;
                    const bool ok = do_res && j < jmax && oc0 < p.OC && yo[q] >= 0;
                    rv[j][q] = __builtin_amdgcn_raw_buffer_load_b64(rr, ok ? (uint32_t)(ro[q] + oc0) * 2u : kOob, 0, 0);
                }
        }
        int ntl_ = tl, nch_ = ch + 1;
        if (nch_ == h.nch) {
            nch_ = 0;
            ++ntl_;
        }
        window_loads(min(ntl_, ntl - 1), nch_, ntl_ < ntl);
        __syncthreads();

        // k steps of the chunk, software-pipelined: the LDS operands of step
        // s + 1 are read before the MFMAs of step s (scheduling barriers keep
        // the compiler from sinking the reads next to their MFMAs)
        const uint8_t* const wb = lds + ch * h.spc * wstep;
        // tap offsets of the step being fetched are in tn; the fetch reads
        // those of the next step from the table, one step ahead of their use
        int tn[WQ];
#pragma unroll
        for (int hh = 0; hh < WQ; ++hh) tn[hh] = t0[hh];
        auto fetch = [&](int s, v4i (&A)[WQ][JN], v4i (&B)[WQ][PW]) {
            const int sn = min(s + 1, h.spc - 1);
#pragma unroll
            for (int hh = 0; hh < WQ; ++hh) {
                const int toff = tn[hh];
                tn[hh] = l_toff[(sn * 4 + grp) * WQ + hh];
#pragma unroll
                for (int j = 0; j < JN; ++j)
                    A[hh][j] = *reinterpret_cast<const v4i*>(wb + s * wstep + (hh * R + j * 16 + col) * 64 + gsw * 16);
#pragma unroll
                for (int q = 0; q < PW; ++q) B[hh][q] = *reinterpret_cast<const v4i*>(tb + bofs[q] + toff);
            }
        };
        // every subtile runs, also past the conv's channels (zero weights there,
        // never stored): no branches between the MFMAs
        auto mma = [&](const v4i (&A)[WQ][JN], const v4i (&B)[WQ][PW]) {
#pragma unroll
            for (int hh = 0; hh < WQ; ++hh)
#pragma unroll
                for (int j = 0; j < JN; ++j) {
#pragma unroll
                    for (int q = 0; q < PW; ++q) {
                        if constexpr (INT8)
                            acc[j][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[hh][j], B[hh][q], acc[j][q], 0, 0, 0);
                        else
                            acc[j][q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, A[hh][j]),
                                                                               __builtin_bit_cast(v8h, B[hh][q]),
                                                                               acc[j][q], 0, 0, 0);
                    }
                }
        };
        v4i A0[WQ][JN], B0[WQ][PW], A1[WQ][JN], B1[WQ][PW];
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

        // ---- epilogue: values (VALU, at a tile's end), then the stores,
        // issued on every iteration (out of range unless at a tile's end) ----
        if (tile_end) {
#pragma unroll
            for (int j = 0; j < JN; ++j) {
                const int lc = j * 16 + grp * 4;
                float bv[4], wv[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    bv[r] = l_bias[lc + r];
                    wv[r] = INT8 ? l_scale[lc + r] : 0.0f;
                }
                const bool oc_ok = j < jmax && n0 + lc < p.OC;
#pragma unroll
                for (int q = 0; q < PW; ++q) {
                    float v[4];
                    igemm::epi_values<INT8, EPI>(p, acc[j][q], bv, wv, rv[j][q], v);
                    const float m4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
                    gmax[j] = fmaxf(gmax[j], oc_ok && yo[q] >= 0 ? m4 : 0.0f);
                    if (out_f32) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) ov[j][q][r] = __float_as_int(v[r]);
                    } else {
                        __half2 oh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                        __builtin_memcpy(&ov[j][q], oh, 8);
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < JN; ++j) {
            const int oc0 = n0 + j * 16 + grp * 4;
            const bool oc_ok = j < jmax && oc0 < p.OC;
#pragma unroll
            for (int q = 0; q < PW; ++q) {
                const bool ok = oc_ok && yo[q] >= 0;
                if (out_f32)
                    __builtin_amdgcn_raw_buffer_store_b128(ov[j][q], ry, ok ? (uint32_t)(yo[q] + oc0) * 4u : kOob, 0,
                                                           0);
                else
                    __builtin_amdgcn_raw_buffer_store_b64(v2i{ov[j][q][0], ov[j][q][1]}, ry,
                                                          ok ? (uint32_t)(yo[q] + oc0) * 2u : kOob, 0, 0);
                if constexpr (INT8 && EPI == igemm::kEpiAny) {
                    // int32 accumulators (acc_out; a zero-byte view drops them)
                    const v4i av{(int)acc[j][q][0], (int)acc[j][q][1], (int)acc[j][q][2], (int)acc[j][q][3]};
                    __builtin_amdgcn_raw_buffer_store_b128(av, racc, ok ? (uint32_t)(mo[q] * p.OC + oc0) * 4u : kOob,
                                                           0, 0);
                }
            }
        }
        if (tile_end) {
#pragma unroll
            for (int j = 0; j < JN; ++j)
#pragma unroll
                for (int q = 0; q < PW; ++q) acc[j][q] = acc_t{0, 0, 0, 0};
        }
        tl = ntl_;
        ch = nch_;
    }

    igemm::flush_slots<JN>(p, gmax, n0, jmax, 0xFFFFFFFFu, out_f32, l_slots);
}

// Blocks of one instance the GPU holds at once with lds_bytes of dynamic LDS.
template <bool INT8, int JN, int PW, int NP, int EPI, bool NCHW, int NW>
int halo_resident_blocks(int lds_bytes) {
    int per_cu = 0, cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, conv3x3_halo_kernel<INT8, JN, PW, NP, EPI, NCHW, NW>, NW * 64,
                                                     (size_t)lds_bytes) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu < 1 ||
        cus < 1)
        return 256;
    return per_cu * cus;
}

// Persistent grid: every resident block slot gets one contiguous run of
// position tiles of one oc tile.
template <bool INT8, int JN, int PW, int NP, int EPI, bool NCHW = false, int NW = 4>
hipError_t halo_launch_cfg(HaloParams h, hipStream_t stream) {
    const int lds_bytes = h.wbytes + 2 * h.tbytes;
    const int cap = halo_resident_blocks<INT8, JN, PW, NP, EPI, NCHW, NW>(lds_bytes);
    int groups = h.ntile;
    if ((int64_t)h.ntile * h.c.ntn > cap) groups = std::max(1, cap / h.c.ntn);
    h.c.per = (h.ntile + groups - 1) / groups;
    groups = (h.ntile + h.c.per - 1) / h.c.per;
    const int64_t blocks = (int64_t)groups * h.c.ntn;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((conv3x3_halo_kernel<INT8, JN, PW, NP, EPI, NCHW, NW>), dim3((unsigned)blocks), dim3(NW * 64),
                       (size_t)lds_bytes, stream, h);
    return hipGetLastError();
}

// Every (JN, PW, NP, NW) of one (INT8, EPI) family.
template <bool INT8, int EPI>
hipError_t halo_launch_family(const HaloParams& h, int jn, int pw, int np, int nw, hipStream_t stream) {
#define AEXRT_HALO_CASE(J, P, N) \
    if (nw == 4 && jn == J && pw == P && np == N) return halo_launch_cfg<INT8, J, P, N, EPI, false, 4>(h, stream);
    AEXRT_HALO_CASE(1, 1, 4) AEXRT_HALO_CASE(1, 2, 4) AEXRT_HALO_CASE(1, 4, 4)
    AEXRT_HALO_CASE(2, 1, 4) AEXRT_HALO_CASE(2, 2, 4) AEXRT_HALO_CASE(2, 4, 4)
    AEXRT_HALO_CASE(4, 1, 4) AEXRT_HALO_CASE(4, 2, 4) AEXRT_HALO_CASE(4, 4, 4)
    AEXRT_HALO_CASE(1, 1, 8) AEXRT_HALO_CASE(1, 2, 8) AEXRT_HALO_CASE(1, 4, 8)
    AEXRT_HALO_CASE(2, 1, 8) AEXRT_HALO_CASE(2, 2, 8) AEXRT_HALO_CASE(2, 4, 8)
    AEXRT_HALO_CASE(4, 1, 8) AEXRT_HALO_CASE(4, 2, 8) AEXRT_HALO_CASE(4, 4, 8)
#undef AEXRT_HALO_CASE
    // 8 waves: the block's weights shared by twice the positions
#define AEXRT_HALO_CASE8(J, P, N) \
    if (nw == 8 && jn == J && pw == P && np == N) return halo_launch_cfg<INT8, J, P, N, EPI, false, 8>(h, stream);
    AEXRT_HALO_CASE8(1, 1, 4) AEXRT_HALO_CASE8(1, 2, 4) AEXRT_HALO_CASE8(2, 1, 4) AEXRT_HALO_CASE8(2, 2, 4)
    AEXRT_HALO_CASE8(4, 1, 4) AEXRT_HALO_CASE8(4, 2, 4) AEXRT_HALO_CASE8(1, 1, 8) AEXRT_HALO_CASE8(1, 2, 8)
    AEXRT_HALO_CASE8(2, 1, 8) AEXRT_HALO_CASE8(2, 2, 8) AEXRT_HALO_CASE8(4, 1, 8) AEXRT_HALO_CASE8(4, 2, 8)
    // every output channel of an 80-channel conv in one block (weights up to
    // 128 KB, one block per CU)
    if constexpr (!INT8) {
        AEXRT_HALO_CASE8(5, 1, 4) AEXRT_HALO_CASE8(5, 2, 4) AEXRT_HALO_CASE8(5, 1, 8) AEXRT_HALO_CASE8(5, 2, 8)
    }
#undef AEXRT_HALO_CASE8
    return hipErrorInvalidValue;
}

// The first conv on the fp32 NCHW input (fp16, SiLU).
hipError_t halo_launch_nchw(const HaloParams& h, int jn, int pw, int np, hipStream_t stream);

#define AEXRT_HALO_FAMILIES(X) X(true, 0) X(true, 1) X(true, 2) X(false, 0) X(false, 1)
#define AEXRT_HALO_EXTERN(I, E) \
    extern template hipError_t halo_launch_family<I, E>(const HaloParams&, int, int, int, int, hipStream_t);
#define AEXRT_HALO_INSTANCE(I, E) \
    template hipError_t halo_launch_family<I, E>(const HaloParams&, int, int, int, int, hipStream_t);

}  // namespace halo
}  // namespace aexrt
