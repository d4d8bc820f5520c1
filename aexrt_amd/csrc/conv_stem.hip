// Band kernel for the network's first conv: 3x3, pad 1, stride 1 or 2, over
// the fp32 NCHW network input with at most 3 channels (fp16 MFMA, bias, SiLU,
// fp16 NHWC output and its amax slots).
//
// The conv is HBM-bound (the input is read once, the output written once,
// 27 multiply-adds per output channel), so the kernel is laid out for
// streaming: a tile is TR whole output rows of one image; its input rows
// ((TR - 1) * S + 3 rows of every channel, each a contiguous fp32 row) are
// read with 16-byte loads, rounded to fp16 and stored unpadded in LDS as
// [channel][row][column] (the zero column left and right of the image sits
// in the row's padding).  The loads of the next tile are in flight while the
// current one is computed, and a block walks a contiguous run of tiles so
// that the rows two bands share are read back from L2.
//
// The contraction is a single v_mfma_f32_16x16x32_f16 per 16 positions and
// 16 output channels: k = c * 9 + ky * 3 + kx (27 of the 32 k, the rest
// zero).  A lane's 8 k of the B operand are 8 fp16 reads from the LDS window
// at per-lane constant offsets; the A operand (weights) is gathered once per
// block from the [OCp][Kp] (k = tap * C + c) layout the other fp16 kernels
// use.  The general halo-tile kernel pads the input to 8 channels instead
// (72 of 128 k, four MFMAs and a 16-byte LDS pixel per position).
#include <cstdio>
#include "conv_igemm.h"

namespace aexrt {

struct StemParams {
    ConvParams c;
    int TR;        // output rows per tile (band)
    int IR;        // input rows of a band: (TR - 1) * S + 3
    int RP;        // LDS row pitch in fp16 elements: W + 8 (image column x at x + 4)
    int plane;     // LDS elements of one channel: IR * RP
    int tbytes;    // LDS bytes of one window buffer
    int q4;        // 16-byte quads of one input row: W / 4
    int npieces;   // quads of one window: c_real * IR * q4
    int nband;     // bands per image
    int ntile;     // N * nband
    int npos;      // output positions of a band: TR * OW
    FastDiv fd_q4, fd_ir, fd_nband, fd_ow;
};

namespace stem {

using igemm::kOob;
using igemm::make_rsrc;
using igemm::rsrc_t;
using igemm::v2i;

// SW: position subtiles (16 positions) per wave and band, an upper bound of
// ceil(TR * OW / 64); every iteration issues exactly NP loads and SW * JN
// stores (out of range when idle), so the wait for the next band's loads
// leaves this band's stores in flight.
template <int JN, int NP, int SW>
__global__ __launch_bounds__(256) void conv3x3_stem_kernel(StemParams h) {
    const ConvParams& p = h.c;
    // [window buffer 0][window buffer 1]
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ uint32_t l_slots[JN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int col = lane & 15;
    const int grp = lane >> 4;

    const int b = igemm::xcd_remap(blockIdx.x, gridDim.x);
    const int t0 = b * p.per;
    const int nt = min(p.per, h.ntile - t0);
    const int S = p.S;
    const int HW = p.H * p.W;

    const rsrc_t rx = make_rsrc(p.x, p.x_bytes);
    const rsrc_t ry = make_rsrc(p.y, p.y_bytes);

    // ---- window quads of this thread: channel c, band row r, quad q ----------
    int grel[NP], lrel[NP], prow[NP];
#pragma unroll
    for (int k = 0; k < NP; ++k) {
        const int e = tid + k * 256;
        const int cr = (int)fdiv((uint32_t)e, h.fd_q4);  // c * IR + r
        const int q = e - cr * h.q4;
        const int c = (int)fdiv((uint32_t)cr, h.fd_ir);
        const int r = cr - c * h.IR;
        grel[k] = c * HW + r * p.W + 4 * q;
        lrel[k] = (c * h.plane + r * h.RP + 4 + 4 * q) * 2;
        prow[k] = e < h.npieces ? r : -0x40000000;  // fails every row test past the window
    }
    // two bands of loads in flight: band i is loaded into pf[i & 1] while
    // bands i - 1 and i - 2 are computed
    v4f pf0[NP], pf1[NP];
    // loads of band t (all NP issued; out of range when !live)
    auto window_loads = [&](v4f (&pf)[NP], int t, bool live) {
        const int n = (int)fdiv((uint32_t)t, h.fd_nband);
        const int row0 = (t - n * h.nband) * h.TR * S - 1;
        const int gbase = n * (int)p.x_nstride + row0 * p.W;
#pragma unroll
        for (int k = 0; k < NP; ++k) {
            const int row = row0 + prow[k];
            const bool ok = live && (unsigned)row < (unsigned)p.H;
            pf[k] = __builtin_bit_cast(v4f, igemm::bload16(rx, ok ? (uint32_t)(gbase + grel[k]) * 4u : kOob));
        }
    };
    // the prologue issues the stores of two iterations too (all dropped), so
    // both edges into the loop carry the same VMEM sequence: band loads, the
    // stores of the band two back, the next band's loads, the stores of the
    // band one back
    window_loads(pf0, t0, nt > 0);
#pragma unroll
    for (int d = 0; d < SW * JN; ++d) __builtin_amdgcn_raw_buffer_store_b64(v2i{0, 0}, ry, kOob, 0, 0);
    window_loads(pf1, t0 + 1, nt > 1);
#pragma unroll
    for (int d = 0; d < SW * JN; ++d) __builtin_amdgcn_raw_buffer_store_b64(v2i{0, 0}, ry, kOob, 0, 0);

    // ---- per-block constants ------------------------------------------------
    // A operand: lane (oc = j * 16 + col, grp) holds k = 8 * grp + e.  The
    // padding k (k >= 9 * c_real) have zero weights and read the position's
    // own (0, 0) tap, a finite value of its window.
    v8h wa[JN];
    const __half* wg = static_cast<const __half*>(p.w);
    int koff[8];  // LDS byte offset of k relative to the position's window origin
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int k = 8 * grp + e;
        const int c = k / 9, tap = k - (k / 9) * 9;
        const int ky = tap / 3, kx = tap - (tap / 3) * 3;
        const bool kok = c < p.c_real;
        koff[e] = (kok ? c * h.plane + ky * h.RP + kx + 3 : 3) * 2;
#pragma unroll
        for (int j = 0; j < JN; ++j) {
            const int oc = j * 16 + col;
            wa[j][e] = kok && oc < p.OC ? (_Float16)__half2float(wg[(size_t)oc * p.Kp + tap * p.C + c]) : (_Float16)0.0f;
        }
    }
    // bias as the MFMA's accumulator input: lane (position, grp) holds oc 4 grp + r
    v4f bias[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int oc = j * 16 + 4 * grp + r;
            bias[j][r] = oc < p.OC ? p.bias[oc] : 0.0f;
        }
    // band-relative geometry of this lane's position in each of its subtiles:
    // window byte offset, output element offset, output row (-1: none)
    const int nsub = (h.npos + 15) >> 4;
    int wofs[SW], yrel[SW], orow[SW];
#pragma unroll
    for (int s = 0; s < SW; ++s) {
        const int pi = (wave + 4 * s) * 16 + col;
        const int pc = min(pi, h.npos - 1);
        const int r = (int)fdiv((uint32_t)pc, h.fd_ow);
        const int ow = pc - r * p.OW;
        wofs[s] = (r * S * h.RP + ow * S) * 2;
        yrel[s] = (r * p.OW + ow) * p.y_cstride;
        orow[s] = pi < h.npos ? r : -0x40000000;
    }
    // zero columns (image column -1 and W) of every row of both buffers
    for (int e = tid; e < 2 * p.c_real * h.IR; e += 256) {
        const int bsel = e / (p.c_real * h.IR), cr = e - bsel * p.c_real * h.IR;
        const int c = cr / h.IR, r = cr - (cr / h.IR) * h.IR;
        __half* row = reinterpret_cast<__half*>(lds + bsel * h.tbytes) + c * h.plane + r * h.RP;
        row[3] = __float2half(0.0f);
        row[p.W + 4] = __float2half(0.0f);
    }
    if (tid < JN) l_slots[tid] = 0u;

    float gmax[JN];
#pragma unroll
    for (int j = 0; j < JN; ++j) gmax[j] = 0.0f;
    v2i ov[SW][JN];

    // band i of the block (i may be one past the last band: then it is
    // computed from stale data and every store is dropped)
    auto band = [&](int i, v4f (&pf)[NP]) {
        const bool live = i < nt;
        uint8_t* const buf = lds + (i & 1) * h.tbytes;
        // this band's window -> LDS (fp32 -> fp16)
#pragma unroll
        for (int k = 0; k < NP; ++k) {
            if (prow[k] >= 0) {
                const __half2 hv[2] = {__floats2half2_rn(pf[k][0], pf[k][1]), __floats2half2_rn(pf[k][2], pf[k][3])};
                v2i v;
                __builtin_memcpy(&v, hv, 8);
                *reinterpret_cast<v2i*>(buf + lrel[k]) = v;
            }
        }
        const int t = min(t0 + i, h.ntile - 1);
        window_loads(pf, min(t0 + i + 2, h.ntile - 1), i + 2 < nt);
        __syncthreads();

        const int n = (int)fdiv((uint32_t)t, h.fd_nband);
        const int oh0 = (t - n * h.nband) * h.TR;
        const int ybase = n * (int)p.y_nstride + oh0 * p.OW * p.y_cstride;
#pragma unroll
        for (int s = 0; s < SW; ++s) {
            if (wave + 4 * s < nsub) {  // wave-uniform
                const uint8_t* const pw = buf + wofs[s];
                v8h bx;
#pragma unroll
                for (int e = 0; e < 8; ++e) bx[e] = *reinterpret_cast<const _Float16*>(pw + koff[e]);
                const bool pok = live && orow[s] >= 0 && oh0 + orow[s] < p.OH;
#pragma unroll
                for (int j = 0; j < JN; ++j) {
                    const v4f acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa[j], bx, bias[j], 0, 0, 0);
                    float v[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[q] = silu(acc[q]);
                    const float m4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
                    gmax[j] = fmaxf(gmax[j], pok && j * 16 + 4 * grp < p.OC ? m4 : 0.0f);
                    const __half2 oh[2] = {__floats2half2_rn(v[0], v[1]), __floats2half2_rn(v[2], v[3])};
                    __builtin_memcpy(&ov[s][j], oh, 8);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < SW; ++s) {
            const bool pok = live && wave + 4 * s < nsub && orow[s] >= 0 && oh0 + orow[s] < p.OH;
#pragma unroll
            for (int j = 0; j < JN; ++j) {
                const int oc0 = j * 16 + 4 * grp;
                const bool ok = pok && oc0 < p.OC;
                __builtin_amdgcn_raw_buffer_store_b64(ov[s][j], ry, ok ? (uint32_t)(ybase + yrel[s] + oc0) * 2u : kOob,
                                                      0, 0);
            }
        }
    };
    for (int i = 0; i < nt; i += 2) {
        band(i, pf0);
        band(i + 1, pf1);
    }
    igemm::flush_slots<JN>(p, gmax, 0, min(JN, p.OCp >> 4), 0xFFFFFFFFu, false, l_slots);
}

template <int JN, int NP, int SW>
hipError_t stem_launch_cfg(StemParams h, bool one_per_block, hipStream_t stream) {
    const int lds_bytes = 2 * h.tbytes;
    int groups = h.ntile;
    if (!one_per_block) {
        int per_cu = 0, cus = 0, dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, conv3x3_stem_kernel<JN, NP, SW>, 256,
                                                         (size_t)lds_bytes) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu < 1 ||
            cus < 1) {
            per_cu = 2;
            cus = 256;
        }
        groups = std::min(h.ntile, per_cu * cus);
    }
    h.c.per = (h.ntile + groups - 1) / groups;
    groups = (h.ntile + h.c.per - 1) / h.c.per;
    hipLaunchKernelGGL((conv3x3_stem_kernel<JN, NP, SW>), dim3((unsigned)groups), dim3(256), (size_t)lds_bytes, stream,
                       h);
    return hipGetLastError();
}

}  // namespace stem

namespace {
// 0 automatic, 1 never (halo-tile kernel), 2 forced band rows (g_stem_tr) on
// a grid of resident blocks, 3 the same with one band per block
std::atomic<int> g_stem_mode{0};
std::atomic<int> g_stem_tr{4};
constexpr int kStemLdsBudget = 64 * 1024;
constexpr int kStemMaxNP = 12;  // window quads per thread
constexpr int kStemMaxSW = 12;  // position subtiles per wave
}  // namespace

bool stem_shape_ok(const ConvParams& p) {
    return p.loader == kLoaderNchwF32 && p.c_real >= 1 && p.c_real <= 3 && p.C == 8 && p.KH == 3 && p.KW == 3 &&
           p.P == 1 && (p.S == 1 || p.S == 2) && p.OH == (p.H - 1) / p.S + 1 && p.OW == (p.W - 1) / p.S + 1 &&
           p.W % 4 == 0 && p.W <= 4096 && p.flags == kConvSilu && p.OCp <= 64 && p.Kp >= 9 * p.C &&
           p.x_nstride == (int64_t)p.c_real * p.H * p.W;
}

// Geometry of a band of tr output rows; false when it does not fit.
static bool stem_geometry(StemParams& h, int tr) {
    const ConvParams& p = h.c;
    if (tr < 1) return false;
    h.TR = std::min(tr, p.OH);
    h.IR = (h.TR - 1) * p.S + 3;
    h.RP = p.W + 8;
    h.plane = h.IR * h.RP;
    h.tbytes = (p.c_real * h.plane * 2 + 15) & ~15;
    h.q4 = p.W / 4;
    h.npieces = p.c_real * h.IR * h.q4;
    if (2 * h.tbytes > kStemLdsBudget || h.npieces > 256 * kStemMaxNP ||
        (h.TR * p.OW + 15) / 16 > 4 * kStemMaxSW)
        return false;
    h.nband = (p.OH + h.TR - 1) / h.TR;
    const int64_t ntile = (int64_t)p.N * h.nband;
    if (ntile > INT32_MAX / 2) return false;
    h.ntile = (int)ntile;
    h.npos = h.TR * p.OW;
    h.fd_q4 = make_fastdiv((uint32_t)h.q4);
    h.fd_ir = make_fastdiv((uint32_t)h.IR);
    h.fd_nband = make_fastdiv((uint32_t)h.nband);
    h.fd_ow = make_fastdiv((uint32_t)p.OW);
    return true;
}

int enumerate_stem_choices(const ConvParams& p, ConvChoice* out, int cap) {
    if (!stem_shape_ok(p)) return 0;
    int n = 0;
    for (int tr : {1, 2, 4, 8}) {
        for (int one = 0; one <= 1 && n < cap; ++one) {
            StemParams h{};
            h.c = p;
            if (!stem_geometry(h, tr) || (tr > 1 && h.TR < tr)) continue;
            ConvChoice c;
            c.kind = 3;
            c.tr = tr;
            c.pw = one;
            c.jn = (p.OCp + 15) / 16;
            out[n++] = c;
        }
    }
    return n;
}

bool set_conv_stem(int mode, int tr) {
    if (mode < 0 || mode > 3 || (mode >= 2 && (tr < 1 || tr > 64))) return false;
    if (mode >= 2) g_stem_tr.store(tr);
    g_stem_mode.store(mode);
    return true;
}

// hipErrorNotSupported: not a stem-shaped conv, or the stem kernel is off
// (the caller runs the halo-tile kernel).
hipError_t launch_conv_stem(const ConvParams& p, hipStream_t stream) {
    const int mode = g_stem_mode.load(std::memory_order_relaxed);
    if (!stem_shape_ok(p) || (mode == 1 && p.choice.kind != 3)) return hipErrorNotSupported;
    StemParams h{};
    h.c = p;
    int tr = 4;
    bool one = false;
    if (p.choice.kind == 3) {
        tr = p.choice.tr;
        one = p.choice.pw != 0;
    } else if (mode >= 2) {
        tr = g_stem_tr.load(std::memory_order_relaxed);
        one = mode == 3;
    }
    if (!stem_geometry(h, tr)) return mode >= 2 || p.choice.kind == 3 ? hipErrorInvalidValue : hipErrorNotSupported;
    const int np = (h.npieces + 255) / 256;
    const int sw = ((h.npos + 15) / 16 + 3) / 4;
    const int jn = (p.OCp + 15) / 16;
    if (LaunchProbe* pr = launch_probe()) {
        // the instance the cases below pick (as a trace names it), then the band
        int J = 0, N = 0;
        for (int j : {1, 2, 4})
            for (int n : {4, 8, 12})
                if (!J && jn <= j && np <= n && sw <= n) J = j, N = n;
        if (!J) return hipErrorInvalidValue;
        std::snprintf(pr->name, sizeof(pr->name), "conv3x3_stem_kernel<%d,%d,%d> tr%d%s", J, N, N, tr,
                      one ? " one" : "");
        return hipSuccess;
    }
#define AEXRT_STEM_CASE(J, N, W) \
    if (jn <= J && np <= N && sw <= W) return stem::stem_launch_cfg<J, N, W>(h, one, stream);
    AEXRT_STEM_CASE(1, 4, 4) AEXRT_STEM_CASE(1, 8, 8) AEXRT_STEM_CASE(1, 12, 12)
    AEXRT_STEM_CASE(2, 4, 4) AEXRT_STEM_CASE(2, 8, 8) AEXRT_STEM_CASE(2, 12, 12)
    AEXRT_STEM_CASE(4, 4, 4) AEXRT_STEM_CASE(4, 8, 8) AEXRT_STEM_CASE(4, 12, 12)
#undef AEXRT_STEM_CASE
    return hipErrorInvalidValue;
}

}  // namespace aexrt
