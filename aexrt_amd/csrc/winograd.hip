// Winograd F(2x2,3x3) 3x3 s1 p1 convolution + bias + SiLU on fp16 MFMA
// (reference kernels 40/46, RT:2480-2631).
//
// Per 2x2 output tile the 4x4 input patch d is transformed to V = B^T d B
// (RT:2533-2548), the 16 transform points become 16 independent GEMMs
// M_r[tile][oc] = sum_c V_r[tile][c] * U_r[c][oc] with U = G g G^T prepared
// by the compiler (packed layout 3), and the output is A^T M A + bias
// (RT:2612-2619).  A block owns 32 tiles x 32 output channels; each wave
// computes the same 16x16 (tile, oc) sub-block for all 16 points, so after
// the K loop every lane holds all 16 points of its (tile, oc) pairs and the
// output transform runs in registers.  V is staged in LDS per 32-channel
// chunk; U ([16][OCp][Cp] fp16, repacked at load) streams from L2.
#include "common.h"
#include "kernels.h"

namespace aexrt {

namespace {

constexpr int WT = 32;       // tiles per block
constexpr int WN = 32;       // output channels per block
constexpr int WKC = 32;      // channels per K chunk
constexpr int VROW = WKC + 8;  // padded LDS row (halves)

// 4x4 input patch -> V = B^T d B for one channel (RT:2533-2548).
__device__ __forceinline__ void input_transform(const float (&d)[4][4], float (&v)[16]) {
    float t[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        t[i][0] = d[i][0] - d[i][2];
        t[i][1] = d[i][1] + d[i][2];
        t[i][2] = -d[i][1] + d[i][2];
        t[i][3] = d[i][1] - d[i][3];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[0 * 4 + j] = t[0][j] - t[2][j];
        v[1 * 4 + j] = t[1][j] + t[2][j];
        v[2 * 4 + j] = -t[1][j] + t[2][j];
        v[3 * 4 + j] = t[1][j] - t[3][j];
    }
}

// Bias, activation, residual, store and amax of one output tile: m[r] holds
// the 16 transform points of (tile T, channel oc); out = A^T M A (RT:2612-2619).
__device__ __forceinline__ void output_tile(const ConvParams& p, const float (&mr)[16], int T, int oc, int tiles_w,
                                            int tiles_img, float& gmax) {
    float r0[4], r1[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        r0[q] = mr[0 * 4 + q] + mr[1 * 4 + q] + mr[2 * 4 + q];
        r1[q] = mr[1 * 4 + q] - mr[2 * 4 + q] - mr[3 * 4 + q];
    }
    float o[4];
    o[0] = r0[0] + r0[1] + r0[2];
    o[1] = r0[1] - r0[2] - r0[3];
    o[2] = r1[0] + r1[1] + r1[2];
    o[3] = r1[1] - r1[2] - r1[3];
    const int n = T / tiles_img;
    const int rem = T - n * tiles_img;
    const int ty = rem / tiles_w;
    const int tx = rem - ty * tiles_w;
    const float bs = p.bias[oc];
    const bool do_silu = p.flags & kConvSilu;
    const bool do_res = p.flags & kConvResidual;
    const bool out_f32 = p.flags & kConvOutF32;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float v = o[q] + bs;
        if (do_silu) v = silu(v);
        const int oy = ty * 2 + (q >> 1), ox = tx * 2 + (q & 1);
        const int64_t pos = (int64_t)oy * p.OW + ox;
        const int64_t yo = (int64_t)n * p.y_nstride + pos * p.y_cstride + oc;
        if (out_f32) {
            if (do_res) v = v + __half2float(p.res[(int64_t)n * p.r_nstride + pos * p.r_cstride + oc]);
            reinterpret_cast<float*>(p.y)[yo] = v;
            gmax = fmaxf(gmax, fabsf(v));
        } else {
            __half h = __float2half(v);
            if (do_res)  // fp16 conv output + fp16 residual, the reference's separate add
                h = __float2half(__half2float(h) + __half2float(p.res[(int64_t)n * p.r_nstride + pos * p.r_cstride + oc]));
            reinterpret_cast<__half*>(p.y)[yo] = h;
            gmax = fmaxf(gmax, fabsf(__half2float(h)));
        }
    }
}

// Large maps: a block owns 32 tiles x 32 output channels; each wave computes
// the same 16x16 (tile, oc) sub-block for all 16 points, so after the K loop
// every lane holds all 16 points of its (tile, oc) pairs and the output
// transform runs in registers.  V is staged in LDS per 32-channel chunk by
// all 256 threads; U ([16][OCp][Cp] fp16, repacked at load) streams from L2.
__global__ __launch_bounds__(256) void winograd_f2x2_kernel(ConvParams p) {
    __shared__ __attribute__((aligned(16))) _Float16 vs[16][WT][VROW];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wt = wave >> 1, wn = wave & 1;
    const int lr = lane & 15, lg = lane >> 4;

    const int tiles_w = p.OW / 2, tiles_h = p.OH / 2;
    const int tiles_img = tiles_w * tiles_h;
    const int ttot = p.N * tiles_img;
    const int ntn = (p.OC + WN - 1) / WN;
    const int t0 = (blockIdx.x / ntn) * WT;
    const int n0 = (blockIdx.x % ntn) * WN;

    // transform unit of this thread: tile tl, channels c4..c4+3 of the chunk
    const int tl = tid >> 3;
    const int c4 = (tid & 7) * 4;
    const int T = t0 + tl;
    int y0 = 0, x0 = 0;
    int64_t xbase = 0;
    const bool t_ok = T < ttot;
    if (t_ok) {
        const int n = T / tiles_img;
        const int rem = T - n * tiles_img;
        const int ty = rem / tiles_w;
        const int tx = rem - ty * tiles_w;
        y0 = ty * 2 - 1;
        x0 = tx * 2 - 1;
        xbase = (int64_t)n * p.x_nstride;
    }
    const __half* xh = reinterpret_cast<const __half*>(p.x);
    const _Float16* U = reinterpret_cast<const _Float16*>(p.w);
    const int oc_b = n0 + wn * 16 + lr;
    const bool oc_b_ok = oc_b < p.OCp;

    v4f acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = v4f{0, 0, 0, 0};

    const int Cp = p.Kp;
    for (int cb = 0; cb < Cp; cb += WKC) {
        // B operands for all 16 points (independent of LDS, issue first).
        v8h b[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            if (oc_b_ok)
                b[r] = *reinterpret_cast<const v8h*>(U + ((int64_t)r * p.OCp + oc_b) * Cp + cb + lg * 8);
            else
                b[r] = v8h{0, 0, 0, 0, 0, 0, 0, 0};
        }
        // Input transform of 4 channels of one tile.
        float d[4][4][4];
        const int c = cb + c4;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int iy = y0 + i, ix = x0 + j;
                float2 lo = make_float2(0.f, 0.f), hi = make_float2(0.f, 0.f);
                if (t_ok && c < p.C && (unsigned)iy < (unsigned)p.H && (unsigned)ix < (unsigned)p.W) {
                    const __half2* src = reinterpret_cast<const __half2*>(
                        xh + xbase + ((int64_t)iy * p.W + ix) * p.x_cstride + c);
                    lo = __half22float2(src[0]);
                    hi = __half22float2(src[1]);
                }
                d[i][j][0] = lo.x; d[i][j][1] = lo.y; d[i][j][2] = hi.x; d[i][j][3] = hi.y;
            }
        __syncthreads();  // previous chunk's MFMAs are done with vs
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float dq[4][4], v[16];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) dq[i][j] = d[i][j][q];
            input_transform(dq, v);
#pragma unroll
            for (int r = 0; r < 16; ++r) vs[r][tl][c4 + q] = (_Float16)v[r];
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const v8h a = *reinterpret_cast<const v8h*>(&vs[r][wt * 16 + lr][lg * 8]);
            acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[r], acc[r], 0, 0, 0);
        }
    }

    // Lane has tiles t0 + wt*16 + lg*4 + i (i = 0..3) of output channel
    // n0 + wn*16 + lr; point r = 4*row + col.
    const int oc = n0 + wn * 16 + lr;
    float gmax = 0.0f;
    if (oc < p.OC) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int Ti = t0 + wt * 16 + lg * 4 + i;
            if (Ti >= ttot) continue;
            float mr[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) mr[r] = acc[r][i];
            output_tile(p, mr, Ti, oc, tiles_w, tiles_img, gmax);
        }
    }
    if (p.y_slots.p) {
        gmax = wave_max(gmax);
        const int g = (n0 + wn * 16) / 16;
        if (lane == 0 && n0 + wn * 16 < p.OC && gmax > 0.0f) slot_max(slot_copy(p.y_slots, blockIdx.x) + g, gmax);
    }
}

// Small maps: a block owns 16 tiles x 16 output channels and its 4 waves
// split the 32-channel chunks (wave w takes chunks w, w+4, ...), each
// transforming its own chunk into a private LDS region, so the K loop needs
// no block barrier.  The partial point sums meet in LDS; wave w then runs the
// output transform of tiles 4*lg + w.
__global__ __launch_bounds__(256) void winograd_f2x2_ksplit_kernel(ConvParams p) {
    constexpr int ST = 16;  // tiles per block
    __shared__ __attribute__((aligned(16))) uint8_t lds[4 * 16 * ST * VROW * 2 > 4 * 16 * 4 * 64 * 4
                                                             ? 4 * 16 * ST * VROW * 2
                                                             : 4 * 16 * 4 * 64 * 4];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    _Float16 (*vs)[ST][VROW] = reinterpret_cast<_Float16 (*)[ST][VROW]>(lds + wave * 16 * ST * VROW * 2);

    const int tiles_w = p.OW / 2, tiles_h = p.OH / 2;
    const int tiles_img = tiles_w * tiles_h;
    const int ttot = p.N * tiles_img;
    const int ntn = (p.OC + 15) / 16;
    const int t0 = (blockIdx.x / ntn) * ST;
    const int n0 = (blockIdx.x % ntn) * 16;

    // transform unit of this lane: tile tl, channels c4..c4+3 (+16) of the chunk
    const int tl = lane >> 2;
    const int c4 = (lane & 3) * 4;
    const int T = t0 + tl;
    int y0 = 0, x0 = 0;
    int64_t xbase = 0;
    const bool t_ok = T < ttot;
    if (t_ok) {
        const int n = T / tiles_img;
        const int rem = T - n * tiles_img;
        const int ty = rem / tiles_w;
        const int tx = rem - ty * tiles_w;
        y0 = ty * 2 - 1;
        x0 = tx * 2 - 1;
        xbase = (int64_t)n * p.x_nstride;
    }
    const __half* xh = reinterpret_cast<const __half*>(p.x);
    const _Float16* U = reinterpret_cast<const _Float16*>(p.w);
    const int oc_b = n0 + lr;
    const bool oc_b_ok = oc_b < p.OCp;

    v4f acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = v4f{0, 0, 0, 0};

    const int Cp = p.Kp;
    for (int cb = wave * WKC; cb < Cp; cb += 4 * WKC) {
        v8h b[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            if (oc_b_ok)
                b[r] = *reinterpret_cast<const v8h*>(U + ((int64_t)r * p.OCp + oc_b) * Cp + cb + lg * 8);
            else
                b[r] = v8h{0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int c = cb + half * 16 + c4;
            float d[4][4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int iy = y0 + i, ix = x0 + j;
                    float2 lo = make_float2(0.f, 0.f), hi = make_float2(0.f, 0.f);
                    if (t_ok && c < p.C && (unsigned)iy < (unsigned)p.H && (unsigned)ix < (unsigned)p.W) {
                        const __half2* src = reinterpret_cast<const __half2*>(
                            xh + xbase + ((int64_t)iy * p.W + ix) * p.x_cstride + c);
                        lo = __half22float2(src[0]);
                        hi = __half22float2(src[1]);
                    }
                    d[i][j][0] = lo.x; d[i][j][1] = lo.y; d[i][j][2] = hi.x; d[i][j][3] = hi.y;
                }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float dq[4][4], v[16];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) dq[i][j] = d[i][j][q];
                input_transform(dq, v);
#pragma unroll
                for (int r = 0; r < 16; ++r) vs[r][tl][half * 16 + c4 + q] = (_Float16)v[r];
            }
        }
        // the region is private to this wave: LDS operations of one wave
        // complete in order, only the compiler must not move them
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const v8h a = *reinterpret_cast<const v8h*>(&vs[r][lr][lg * 8]);
            acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[r], acc[r], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();
    }

    // partial sums of the 4 waves: red[wave][r][i][lane]
    float* red = reinterpret_cast<float*>(lds);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[((wave * 16 + r) * 4 + i) * 64 + lane] = acc[r][i];
    __syncthreads();

    // wave w finishes tile row i = w: tiles t0 + lg*4 + w, channel n0 + lr
    const int oc = n0 + lr;
    const int Ti = t0 + lg * 4 + wave;
    float gmax = 0.0f;
    if (oc < p.OC && Ti < ttot) {
        float mr[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float t = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w) t += red[((w * 16 + r) * 4 + wave) * 64 + lane];
            mr[r] = t;
        }
        output_tile(p, mr, Ti, oc, tiles_w, tiles_img, gmax);
    }
    if (p.y_slots.p) {
        gmax = wave_max(gmax);
        if (lane == 0 && n0 < p.OC && gmax > 0.0f) slot_max(slot_copy(p.y_slots, blockIdx.x) + n0 / 16, gmax);
    }
}

}  // namespace

// The 32x32 block tile when it yields at least one block per CU, else the
// k-split 16x16 tile (maps of 10x10 / 20x20 at small batch).
hipError_t launch_winograd_f2x2(const ConvParams& p, hipStream_t stream) {
    const int64_t ttot = (int64_t)p.N * (p.OH / 2) * (p.OW / 2);
    const int64_t big = ((ttot + WT - 1) / WT) * ((p.OC + WN - 1) / WN);
    if (big >= 256 || p.Kp < 4 * WKC) {
        hipLaunchKernelGGL(winograd_f2x2_kernel, dim3((unsigned)big), dim3(256), 0, stream, p);
    } else {
        const int64_t small = ((ttot + 15) / 16) * ((p.OC + 15) / 16);
        hipLaunchKernelGGL(winograd_f2x2_ksplit_kernel, dim3((unsigned)small), dim3(256), 0, stream, p);
    }
    return hipGetLastError();
}

}  // namespace aexrt
