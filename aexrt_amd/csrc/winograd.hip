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
            float t[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                t[i][0] = d[i][0][q] - d[i][2][q];
                t[i][1] = d[i][1][q] + d[i][2][q];
                t[i][2] = -d[i][1][q] + d[i][2][q];
                t[i][3] = d[i][1][q] - d[i][3][q];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                vs[0 * 4 + j][tl][c4 + q] = (_Float16)(t[0][j] - t[2][j]);
                vs[1 * 4 + j][tl][c4 + q] = (_Float16)(t[1][j] + t[2][j]);
                vs[2 * 4 + j][tl][c4 + q] = (_Float16)(-t[1][j] + t[2][j]);
                vs[3 * 4 + j][tl][c4 + q] = (_Float16)(t[1][j] - t[3][j]);
            }
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const v8h a = *reinterpret_cast<const v8h*>(&vs[r][wt * 16 + lr][lg * 8]);
            acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[r], acc[r], 0, 0, 0);
        }
    }

    // Output transform: lane has tiles t0 + wt*16 + lg*4 + i (i = 0..3) of
    // output channel n0 + wn*16 + lr; point r = 4*row + col.
    const int oc = n0 + wn * 16 + lr;
    const bool oc_ok = oc < p.OC;
    const float bs = oc_ok ? p.bias[oc] : 0.0f;
    const bool do_silu = p.flags & kConvSilu;
    const bool do_res = p.flags & kConvResidual;
    const bool out_f32 = p.flags & kConvOutF32;
    float gmax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int Ti = t0 + wt * 16 + lg * 4 + i;
        if (!oc_ok || Ti >= ttot) continue;
        float r0[4], r1[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            r0[q] = acc[0 * 4 + q][i] + acc[1 * 4 + q][i] + acc[2 * 4 + q][i];
            r1[q] = acc[1 * 4 + q][i] - acc[2 * 4 + q][i] - acc[3 * 4 + q][i];
        }
        float o[4];
        o[0] = r0[0] + r0[1] + r0[2];
        o[1] = r0[1] - r0[2] - r0[3];
        o[2] = r1[0] + r1[1] + r1[2];
        o[3] = r1[1] - r1[2] - r1[3];
        const int n = Ti / tiles_img;
        const int rem = Ti - n * tiles_img;
        const int ty = rem / tiles_w;
        const int tx = rem - ty * tiles_w;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float v = o[q] + bs;
            if (do_silu) v = silu(v);
            const int oy = ty * 2 + (q >> 1), ox = tx * 2 + (q & 1);
            const int64_t pos = (int64_t)oy * p.OW + ox;
            if (do_res) v = v + __half2float(p.res[(int64_t)n * p.r_nstride + pos * p.r_cstride + oc]);
            const int64_t yo = (int64_t)n * p.y_nstride + pos * p.y_cstride + oc;
            if (out_f32) {
                reinterpret_cast<float*>(p.y)[yo] = v;
                gmax = fmaxf(gmax, fabsf(v));
            } else {
                const __half h = __float2half(v);
                reinterpret_cast<__half*>(p.y)[yo] = h;
                gmax = fmaxf(gmax, fabsf(__half2float(h)));
            }
        }
    }
    if (p.y_slots) {
        gmax = wave_max(gmax);
        const int g = (n0 + wn * 16) / 16;
        if (lane == 0 && n0 + wn * 16 < p.OC) slot_max(p.y_slots + g, gmax);
    }
}

}  // namespace

hipError_t launch_winograd_f2x2(const ConvParams& p, hipStream_t stream) {
    const int ttot = p.N * (p.OH / 2) * (p.OW / 2);
    const int blocks = ((ttot + WT - 1) / WT) * ((p.OC + WN - 1) / WN);
    hipLaunchKernelGGL(winograd_f2x2_kernel, dim3(blocks), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace aexrt
