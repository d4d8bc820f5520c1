// Streaming 1x1 int8 convolution on gfx950 MFMA: the reference's W8A8 1x1
// conv (kernel 51, RT:4614-4762; per-tensor activation scale, per-oc weight
// scale, exact int32 sums, dequant + bias + SiLU) for NHWC views whose
// positions are evenly strided (dense images or channel slices of a concat
// root).
//
// A 1x1 conv over M positions is a GEMM with a short k (C <= 512 channels),
// so what bounds it is moving and quantizing the activations, not the
// multiply.  A block of 4 waves owns OCB = 16 JQ output channels and walks a
// contiguous run of position tiles of TP = 64 PQ positions:
//   - its weights ([k step][oc][64 B], 16-byte slots swizzled per 4 rows so
//     the 16 lanes of an operand read hit distinct banks) go from memory
//     straight into LDS once;
//   - a tile's fp16 input (TP positions x C channels) is loaded with every
//     load of the tile in flight at once (16 channels of one position per
//     32 B piece), quantized once by the thread that loaded it and stored as
//     int8 [k step][position][64 B] in one of two LDS tile buffers;
//   - the 4 waves split the tile's positions (PQ 16-position subtiles each)
//     and all read the block's weights: per 64-channel k step a wave reads
//     its B fragments and JQ A fragments (1 KB each, conflict-free) and
//     issues JQ x PQ v_mfma_i32_16x16x64_i8;
//   - the loads of tile t+1 are issued before tile t's MFMAs and epilogue,
//     so the memory latency of a tile overlaps the previous tile's work, with
//     one barrier per tile; a launch whose blocks own one tile each gets one
//     tile buffer (half the LDS, twice the resident blocks for small maps).
// UP: the epilogue also writes each output value to the 2 x 2 positions of
// the output's nearest 2x upsample (p.yup, e.g. a channel slice of a concat
// that a resize of this conv's output used to fill) and folds the block's
// maxima into that view's slots too: the resize's values and amax without
// its launch or its re-read of this output.
// XUP: the input pieces of channels [xup_c0, xup_c0 + xup_cn) are loaded
// from p.xup at the position's (y / 2, x / 2): the conv reads a nearest 2x
// upsample (a concat slice a resize would fill) straight from its source,
// through one buffer resource over both views (xbase, byte offsets x_off0,
// xup_off0); the source's amax slots are read with the input's.
// Every iteration issues the same memory operations (the epilogue's stores,
// then the next tile's loads; out-of-range offsets when there is nothing to
// do) and the prologue issues an iteration's stores as dropped ones, so the
// compiler's counts of loads in flight are exact on both edges into the loop
// and a tile's quantization waits for its own loads only, not for the stores
// issued after them.
#pragma once
#include "conv_igemm.h"

namespace aexrt {

// Geometry of one streaming 1x1 launch (host-computed).
struct S1x1Params {
    ConvParams c;  // views, weights, flags; c.ntn / c.per / c.fd_ntn are this launch's
    int TP;        // positions of a tile: 64 * PQ
    int nks;       // 64-channel k steps: Kp / 64
    int c16;       // 16-channel input pieces of one position: C / 16
    int npiece;    // pieces of one tile: TP * c16
    int ntile;     // position tiles: ceil(M / TP)
    int wbytes;    // LDS bytes of the block's weights: nks * OCB * 64
    int tbytes;    // LDS bytes of one int8 tile: nks * TP * 64
    FastDiv fd_c16;
    FastDiv fd_hw, fd_w;  // UP, XUP: positions of an image, columns
    // XUP: one resource over the input and the upsampled source
    const void* xbase;
    uint32_t xspan, x_off0, xup_off0;
    uint32_t xup_slot_bytes;
    FastDiv fd_uns;
    int one;  // one tile per block (a grid of every tile) instead of a persistent grid
};

namespace s1x1 {

using igemm::bload16;
using igemm::kOob;
using igemm::make_rsrc;
using igemm::quant8;
using igemm::rsrc_t;
using igemm::v2i;
using igemm::xcd_remap;
typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int JQ, int PQ, int NP, int EPI, bool UP = false, bool XUP = false>
__global__ __launch_bounds__(256) void conv1x1_stream_kernel(S1x1Params h) {
    constexpr int OCB = JQ * 16;  // output channels of the block
    constexpr int TP = PQ * 64;   // positions of a tile
    const ConvParams& p = h.c;

    // [weights: wbytes][tile buffer 0: tbytes][tile buffer 1: tbytes]
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    // read 4 at a time in the epilogue
    __shared__ __attribute__((aligned(16))) float l_bias[OCB];
    __shared__ __attribute__((aligned(16))) float l_scale[OCB];
    __shared__ uint32_t l_slots[JQ];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15;
    const int grp = lane >> 4;
    // LDS slot of k group grp in a 64-byte row r with (r >> 2) & 3 == (col >> 2) & 3
    const int gsw = grp ^ ((col >> 2) & 3);

    const int b = xcd_remap(blockIdx.x, gridDim.x);
    const int pg = (int)fdiv((uint32_t)b, p.fd_ntn);
    const int n0 = (b - pg * p.ntn) * OCB;
    const int pt0 = pg * p.per;
    const int ntl = min(p.per, h.ntile - pt0);
    const int jmax = min(JQ, (p.OCp - n0) >> 4);

    const rsrc_t rx = XUP ? make_rsrc(h.xbase, h.xspan) : make_rsrc(p.x, p.x_bytes);
    const rsrc_t rw = make_rsrc(p.w, (uint32_t)p.OCp * (uint32_t)p.Kp);

    // ---- prologue loads: input scale, per-channel constants ----------------
    uint32_t slot_raw[igemm::kMaxSlotReads / 64];
    igemm::in_slot_loads(p, lane, slot_raw);
    uint32_t up_raw[XUP ? igemm::kMaxUpSlotReads / 64 : 1];
    if constexpr (XUP) igemm::up_slot_loads(p, h.xup_slot_bytes, h.fd_uns, lane, up_raw);
    const rsrc_t rb = make_rsrc(p.bias, (uint32_t)p.OC * 4u);
    const rsrc_t rsc = make_rsrc(p.w_scale, (uint32_t)p.OC * 4u);
    const uint32_t cofs = tid < OCB && n0 + tid < p.OC ? (uint32_t)(n0 + tid) * 4u : kOob;
    const float bias_v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, cofs, 0, 0));
    const float scale_v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsc, cofs, 0, 0));

    // ---- input pieces of this thread: e = tid + k * 256 -> position e / c16
    // of the tile, channels 16 (e % c16) .. + 15; byte offset relative to the
    // tile's first position, and LDS place in a tile buffer ----
    int ppos[NP];
    uint32_t poff[NP];
    int plds[NP];
    uint32_t pup[XUP ? NP : 1];  // XUP: the piece's channel in the source, ~0 for the input's own
#pragma unroll
    for (int k = 0; k < NP; ++k) {
        const int e = tid + k * 256;
        const int pos = (int)fdiv((uint32_t)e, h.fd_c16);
        const int c = e - pos * h.c16;
        ppos[k] = e < h.npiece ? pos : 0x40000000;  // past every tile's last position
        poff[k] = (XUP ? h.x_off0 : 0u) + ((uint32_t)pos * (uint32_t)p.x_cstride + (uint32_t)c * 16u) * 2u;
        plds[k] = ((c >> 2) * TP + pos) * 64 + (((c & 3) ^ ((pos >> 2) & 3)) << 4);
        if constexpr (XUP) {
            const int cu = c * 16 - p.xup_c0;
            pup[k] = cu >= 0 && cu < p.xup_cn ? (uint32_t)cu : 0xFFFFFFFFu;
        }
    }
    v4i pf[NP][2];
    // all loads of tile tl (out of range when !live or past the map)
    auto tile_loads = [&](int tl, bool live) {
        const int m0 = (pt0 + tl) * TP;
        const uint32_t base = (uint32_t)m0 * (uint32_t)p.x_cstride * 2u;
#pragma unroll
        for (int k = 0; k < NP; ++k) {
            const int m = m0 + ppos[k];
            const bool ok = live && m < p.M;
            uint32_t off = base + poff[k];
            if constexpr (XUP) {
                // position m = (n, y, x) of the input -> (n, y / 2, x / 2) of the source
                const uint32_t n = fdiv((uint32_t)m, h.fd_hw);
                const uint32_t r = (uint32_t)m - n * (uint32_t)(p.H * p.W);
                const uint32_t yy = fdiv(r, h.fd_w);
                const uint32_t xx = r - yy * (uint32_t)p.W;
                const uint32_t uo = h.xup_off0 + (n * (uint32_t)p.xup_nstride +
                                                  ((yy >> 1) * (uint32_t)(p.W >> 1) + (xx >> 1)) * (uint32_t)p.xup_cstride +
                                                  pup[k]) * 2u;
                off = pup[k] != 0xFFFFFFFFu ? uo : off;
            }
            off = ok ? off : kOob;
            pf[k][0] = bload16(rx, off);
            pf[k][1] = bload16(rx, off + 16u);
        }
    };
    tile_loads(0, true);

    // ---- weights -> LDS: piece e = (k step s, row, slot) at LDS e * 16 holds
    // k group slot ^ ((row >> 2) & 3) of output channel n0 + row; lane l of a
    // wave's 64 pieces lands at the wave's base + 16 l ----
    {
        const int wpieces = h.wbytes >> 4;
        for (int e0 = wave * 64; e0 < wpieces; e0 += 256) {
            const uint32_t e = (uint32_t)(e0 + lane);
            const int s = (int)(e / (uint32_t)(OCB * 4));
            const int rem = (int)(e % (uint32_t)(OCB * 4));
            const int row = rem >> 2;
            const int g = (rem & 3) ^ ((row >> 2) & 3);
            const bool ok = n0 + row < p.OCp;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rw, (lds_ptr_t)(lds + e0 * 16), 16,
                ok ? (uint32_t)(n0 + row) * (uint32_t)p.Kp + (uint32_t)(s * 64 + g * 16) : kOob, 0, 0, 0);
        }
    }

    // ---- output side ---------------------------------------------------------
    const bool out_f32 = EPI == igemm::kEpiAny && (p.flags & kConvOutF32);
    const bool acc_on = EPI == igemm::kEpiAny && p.acc_out != nullptr;
    const rsrc_t ry = make_rsrc(p.y, p.y_bytes);
    const rsrc_t racc = make_rsrc(p.acc_out, acc_on ? (uint32_t)p.M * (uint32_t)p.OC * 4u : 0u);
    const rsrc_t ryu = make_rsrc(UP ? p.yup : nullptr, UP ? p.yup_bytes : 0u);
    constexpr int NST = JQ * PQ * ((EPI == igemm::kEpiAny ? 2 : 1) + (UP ? 4 : 0));  // stores of one tile
    // the stores of an iteration, dropped: both edges into the loop then
    // carry the same memory operations after the first tile's loads
#pragma unroll
    for (int d = 0; d < NST; ++d) __builtin_amdgcn_raw_buffer_store_b64(v2i{0, 0}, ry, kOob, 0, 0);

    if (tid < JQ) l_slots[tid] = 0u;
    // everything issued so far: the weights (no register tracks them) and
    // the first tile are needed before the first barrier
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    float s_q = 0.0f, in_scale = 0.0f;
    uint32_t up_am = 0u;
    if constexpr (XUP) {
#pragma unroll
        for (int r = 0; r < igemm::kMaxUpSlotReads / 64; ++r) up_am = max(up_am, up_raw[r]);
    }
    igemm::in_slot_scale(slot_raw, s_q, in_scale, up_am);
    if (tid < OCB) {
        l_bias[tid] = bias_v;
        // dequant factor amax/127 * w_scale[oc] (one fma in the epilogue)
        l_scale[tid] = in_scale * scale_v;
    }

    uint8_t* const tiles = lds + h.wbytes;
    // quantize the loaded tile into buffer buf (int8, one piece per 16 channels)
    auto tile_store = [&](int buf) {
        uint8_t* const tb = tiles + buf * h.tbytes;
#pragma unroll
        for (int k = 0; k < NP; ++k) {
            if (tid + k * 256 < h.npiece) {
                const v2i lo = quant8(pf[k][0], s_q), hq = quant8(pf[k][1], s_q);
                *reinterpret_cast<v4i*>(tb + plds[k]) = v4i{lo[0], lo[1], hq[0], hq[1]};
            }
        }
    };
    tile_store(0);
    tile_loads(1, 1 < ntl);

    float gmax[JQ];
#pragma unroll
    for (int j = 0; j < JQ; ++j) gmax[j] = 0.0f;
    const int wstep = OCB * 64;  // LDS bytes of one k step's weights
    const int tstep = TP * 64;   // LDS bytes of one k step of a tile
    const uint8_t* const wl = lds + col * 64 + gsw * 16;

    for (int i = 0; i < ntl; ++i) {
        __syncthreads();
        const uint8_t* const tb = tiles + (i & 1) * h.tbytes + (wave * PQ * 16 + col) * 64 + gsw * 16;
        v4i acc[JQ][PQ];
#pragma unroll
        for (int j = 0; j < JQ; ++j)
#pragma unroll
            for (int q = 0; q < PQ; ++q) acc[j][q] = v4i{0, 0, 0, 0};
        for (int s = 0; s < h.nks; ++s) {
            v4i B[PQ];
#pragma unroll
            for (int q = 0; q < PQ; ++q) B[q] = *reinterpret_cast<const v4i*>(tb + s * tstep + q * 1024);
#pragma unroll
            for (int j = 0; j < JQ; ++j) {
                const v4i A = *reinterpret_cast<const v4i*>(wl + s * wstep + j * 1024);
#pragma unroll
                for (int q = 0; q < PQ; ++q)
                    acc[j][q] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B[q], acc[j][q], 0, 0, 0);
            }
        }

        // ---- epilogue: lane holds channels n0 + 16 j + 4 grp + r of position
        // m = tile base + (wave * PQ + q) * 16 + col in acc[j][q][r] ----
        const int mb = (pt0 + i) * TP + wave * PQ * 16 + col;
#pragma unroll
        for (int j = 0; j < JQ; ++j) {
            const int lc = j * 16 + grp * 4;
            const int oc0 = n0 + lc;
            const bool oc_ok = j < jmax && oc0 < p.OC;
            const v4f bv4 = *reinterpret_cast<const v4f*>(&l_bias[lc]);
            const v4f wv4 = *reinterpret_cast<const v4f*>(&l_scale[lc]);
            const float bv[4] = {bv4[0], bv4[1], bv4[2], bv4[3]};
            const float wv[4] = {wv4[0], wv4[1], wv4[2], wv4[3]};
#pragma unroll
            for (int q = 0; q < PQ; ++q) {
                const int m = mb + q * 16;
                const bool ok = oc_ok && m < p.M;
                float v[4];
                igemm::epi_values<true, EPI>(p, acc[j][q], bv, wv, v2i{0, 0}, v);
                const float m4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
                gmax[j] = fmaxf(gmax[j], ok ? m4 : 0.0f);
                const uint32_t yoff = (uint32_t)m * (uint32_t)p.y_cstride + (uint32_t)oc0;
                if (out_f32) {
                    const v4i o{__float_as_int(v[0]), __float_as_int(v[1]), __float_as_int(v[2]),
                                __float_as_int(v[3])};
                    __builtin_amdgcn_raw_buffer_store_b128(o, ry, ok ? yoff * 4u : kOob, 0, 0);
                } else {
                    const __half2 oh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                    v2i o;
                    __builtin_memcpy(&o, oh, 8);
                    __builtin_amdgcn_raw_buffer_store_b64(o, ry, ok ? yoff * 2u : kOob, 0, 0);
                }
                if constexpr (UP) {
                    // position m = (n, y, x) -> (n, 2y + dy, 2x + dx), dy, dx in {0, 1}
                    const uint32_t n = fdiv((uint32_t)m, h.fd_hw);
                    const uint32_t r = (uint32_t)m - n * (uint32_t)(p.OH * p.OW);
                    const uint32_t yy = fdiv(r, h.fd_w);
                    const uint32_t xx = r - yy * (uint32_t)p.OW;
                    const uint32_t ucs = (uint32_t)p.yup_cstride;
                    const uint32_t u0 = n * (uint32_t)p.yup_nstride + ((2u * yy) * (2u * p.OW) + 2u * xx) * ucs + oc0;
                    const uint32_t drow = 2u * p.OW * ucs;
                    const __half2 uh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                    v2i uo;
                    __builtin_memcpy(&uo, uh, 8);
                    __builtin_amdgcn_raw_buffer_store_b64(uo, ryu, ok ? u0 * 2u : kOob, 0, 0);
                    __builtin_amdgcn_raw_buffer_store_b64(uo, ryu, ok ? (u0 + ucs) * 2u : kOob, 0, 0);
                    __builtin_amdgcn_raw_buffer_store_b64(uo, ryu, ok ? (u0 + drow) * 2u : kOob, 0, 0);
                    __builtin_amdgcn_raw_buffer_store_b64(uo, ryu, ok ? (u0 + drow + ucs) * 2u : kOob, 0, 0);
                }
                if constexpr (EPI == igemm::kEpiAny) {
                    // int32 accumulators (acc_out; a zero-byte view drops them)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        acc[j][q], racc, ok && acc_on ? ((uint32_t)m * (uint32_t)p.OC + (uint32_t)oc0) * 4u : kOob,
                        0, 0);
                }
            }
        }

        // ---- next tile: quantize into the other buffer (its last readers
        // passed this iteration's barrier; a launch whose blocks have one tile
        // each has no second buffer), then issue the one after ----
        if (i + 1 < ntl) tile_store((i + 1) & 1);
        tile_loads(i + 2, i + 2 < ntl);
    }

    igemm::flush_slots<JQ>(p, gmax, n0, jmax, 0xFFFFFFFFu, out_f32, l_slots);
    if constexpr (UP) {
        // the upsample holds the same values: the same maxima (l_slots as
        // reduced above, read by the threads that read them there)
        if (p.yup_slots.p && tid < jmax && n0 + tid * 16 < p.OC && l_slots[tid])
            atomicMax(slot_copy(p.yup_slots, blockIdx.x) + (n0 >> 4) + tid, l_slots[tid]);
    }
}

// Blocks of one instance the GPU holds at once with lds_bytes of dynamic LDS.
template <int JQ, int PQ, int NP, int EPI, bool UP, bool XUP>
int s1x1_resident_blocks(int lds_bytes) {
    int per_cu = 0, cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, conv1x1_stream_kernel<JQ, PQ, NP, EPI, UP, XUP>, 256,
                                                     (size_t)lds_bytes) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu < 1 ||
        cus < 1)
        return 256;
    return per_cu * cus;
}

// Persistent grid: every resident block slot gets one contiguous run of
// position tiles of one channel tile.
template <int JQ, int PQ, int NP, int EPI, bool UP = false, bool XUP = false>
hipError_t s1x1_launch_cfg(S1x1Params h, hipStream_t stream) {
    // one tile buffer when the single-buffer footprint already gives every
    // tile its own resident block
    int lds_bytes = h.wbytes + h.tbytes;
    int cap = h.one ? INT32_MAX : s1x1_resident_blocks<JQ, PQ, NP, EPI, UP, XUP>(lds_bytes);
    if ((int64_t)h.ntile * h.c.ntn > cap) {
        lds_bytes = h.wbytes + 2 * h.tbytes;
        cap = s1x1_resident_blocks<JQ, PQ, NP, EPI, UP, XUP>(lds_bytes);
    }
    int groups = h.ntile;
    if ((int64_t)h.ntile * h.c.ntn > cap) groups = std::max(1, cap / h.c.ntn);
    h.c.per = (h.ntile + groups - 1) / groups;
    groups = (h.ntile + h.c.per - 1) / h.c.per;
    const int64_t blocks = (int64_t)groups * h.c.ntn;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((conv1x1_stream_kernel<JQ, PQ, NP, EPI, UP, XUP>), dim3((unsigned)blocks), dim3(256),
                       (size_t)lds_bytes, stream, h);
    return hipGetLastError();
}

// Every (JQ, PQ, NP) of one epilogue family; with the upsample copy (up) or
// an upsampled input source (xup), the one-subtile-per-wave tiles (PQ 1).
template <int EPI>
hipError_t s1x1_launch_family(const S1x1Params& h, int jq, int pq, int np, bool up, bool xup, hipStream_t stream) {
#define AEXRT_S1X1_XUP_CASE(J, N) \
    if (jq == J && pq == 1 && np == N) return s1x1_launch_cfg<J, 1, N, EPI, false, true>(h, stream);
    if (xup) {
        if (up) return hipErrorInvalidValue;
        AEXRT_S1X1_XUP_CASE(1, 1) AEXRT_S1X1_XUP_CASE(1, 2) AEXRT_S1X1_XUP_CASE(1, 4) AEXRT_S1X1_XUP_CASE(1, 8)
        AEXRT_S1X1_XUP_CASE(2, 1) AEXRT_S1X1_XUP_CASE(2, 2) AEXRT_S1X1_XUP_CASE(2, 4) AEXRT_S1X1_XUP_CASE(2, 8)
        AEXRT_S1X1_XUP_CASE(4, 1) AEXRT_S1X1_XUP_CASE(4, 2) AEXRT_S1X1_XUP_CASE(4, 4) AEXRT_S1X1_XUP_CASE(4, 8)
        AEXRT_S1X1_XUP_CASE(8, 1) AEXRT_S1X1_XUP_CASE(8, 2) AEXRT_S1X1_XUP_CASE(8, 4) AEXRT_S1X1_XUP_CASE(8, 8)
        return hipErrorInvalidValue;
    }
#undef AEXRT_S1X1_XUP_CASE
#define AEXRT_S1X1_UP_CASE(J, N) \
    if (jq == J && pq == 1 && np == N) return s1x1_launch_cfg<J, 1, N, EPI, true>(h, stream);
    if (up) {
        AEXRT_S1X1_UP_CASE(1, 1) AEXRT_S1X1_UP_CASE(1, 2) AEXRT_S1X1_UP_CASE(1, 4) AEXRT_S1X1_UP_CASE(1, 8)
        AEXRT_S1X1_UP_CASE(2, 1) AEXRT_S1X1_UP_CASE(2, 2) AEXRT_S1X1_UP_CASE(2, 4) AEXRT_S1X1_UP_CASE(2, 8)
        AEXRT_S1X1_UP_CASE(4, 1) AEXRT_S1X1_UP_CASE(4, 2) AEXRT_S1X1_UP_CASE(4, 4) AEXRT_S1X1_UP_CASE(4, 8)
        AEXRT_S1X1_UP_CASE(8, 1) AEXRT_S1X1_UP_CASE(8, 2) AEXRT_S1X1_UP_CASE(8, 4) AEXRT_S1X1_UP_CASE(8, 8)
        return hipErrorInvalidValue;
    }
#undef AEXRT_S1X1_UP_CASE
#define AEXRT_S1X1_CASE(J, P, N) \
    if (jq == J && pq == P && np == N) return s1x1_launch_cfg<J, P, N, EPI>(h, stream);
    AEXRT_S1X1_CASE(1, 1, 1) AEXRT_S1X1_CASE(1, 1, 2) AEXRT_S1X1_CASE(1, 1, 4) AEXRT_S1X1_CASE(1, 1, 8)
    AEXRT_S1X1_CASE(2, 1, 1) AEXRT_S1X1_CASE(2, 1, 2) AEXRT_S1X1_CASE(2, 1, 4) AEXRT_S1X1_CASE(2, 1, 8)
    AEXRT_S1X1_CASE(4, 1, 1) AEXRT_S1X1_CASE(4, 1, 2) AEXRT_S1X1_CASE(4, 1, 4) AEXRT_S1X1_CASE(4, 1, 8)
    AEXRT_S1X1_CASE(8, 1, 1) AEXRT_S1X1_CASE(8, 1, 2) AEXRT_S1X1_CASE(8, 1, 4) AEXRT_S1X1_CASE(8, 1, 8)
    AEXRT_S1X1_CASE(1, 2, 1) AEXRT_S1X1_CASE(1, 2, 2) AEXRT_S1X1_CASE(1, 2, 4)
    AEXRT_S1X1_CASE(2, 2, 1) AEXRT_S1X1_CASE(2, 2, 2) AEXRT_S1X1_CASE(2, 2, 4)
    AEXRT_S1X1_CASE(4, 2, 1) AEXRT_S1X1_CASE(4, 2, 2) AEXRT_S1X1_CASE(4, 2, 4)
#undef AEXRT_S1X1_CASE
    return hipErrorInvalidValue;
}

#define AEXRT_S1X1_EXTERN(E) \
    extern template hipError_t s1x1_launch_family<E>(const S1x1Params&, int, int, int, bool, bool, hipStream_t);
#define AEXRT_S1X1_INSTANCE(E) \
    template hipError_t s1x1_launch_family<E>(const S1x1Params&, int, int, int, bool, bool, hipStream_t);

}  // namespace s1x1
}  // namespace aexrt
