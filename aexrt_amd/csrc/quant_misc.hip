// Activation amax / quantization kernels and the glue ops of the replay
// stream (copy for concat, maxpool, nearest resize, add, layout changes).
//
// All of them are HBM-bound streaming kernels: 16-byte vector accesses along
// the contiguous channel dimension of NHWC views, grid-stride loops sized to
// the CU count, and amax reductions that go wave shuffle -> LDS -> one
// atomicMax per block and 16-channel group (never one workgroup per group, so
// low-channel / large-plane tensors still fill the chip).
#include "common.h"
#include "kernels.h"

namespace aexrt {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxSlots = 128;  // up to 2048 channels per view

inline int grid_for(int64_t work, int max_blocks = 256 * 16) {
    int64_t g = (work + kThreads - 1) / kThreads;
    if (g < 1) g = 1;
    if (g > max_blocks) g = max_blocks;
    return (int)g;
}

// Grid for a chunk loop over C/8 chunk columns: the grid stride (blocks x
// 256) is made a multiple of the column count so each thread keeps one
// column.
inline int grid_cols(int64_t chunks, int C) {
    const int cc = C / 8 > 0 ? C / 8 : 1;
    int a = cc, b = kThreads;
    while (b) {
        const int t = a % b;
        a = b;
        b = t;
    }
    const int r = cc / a;
    // 4 blocks per CU: enough to keep HBM busy with the grid-stride loops,
    // and few enough that the blocks' slot updates (one per group) stay cheap
    int g = grid_for(chunks, 256 * 4);
    g = (g + r - 1) / r * r;
    return g;
}

__device__ __forceinline__ void slots_init(uint32_t* s, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) s[i] = 0u;
    __syncthreads();
}

// Block maxima -> this block's copy of the slot array.
__device__ __forceinline__ void slots_flush(const uint32_t* s, int n, const SlotRef& ref) {
    __syncthreads();
    uint32_t* g = slot_copy(ref, blockIdx.x);
    for (int i = threadIdx.x; i < n; i += blockDim.x)
        if (s[i]) slot_max(g + i, u2f(s[i]));
}

// Per-thread running max of one 16-channel group.  The host sizes grids so
// that the grid stride is a multiple of the chunk columns C/8, which pins
// every thread to one chunk column (and so one group) for its whole loop;
// the block then folds one value per thread into LDS.
struct GroupMax {
    float v = 0.0f;
    int g = -1;
    __device__ __forceinline__ void add(int group, float m, uint32_t* ls) {
        if (g == group || g < 0) {
            g = group;
            v = fmaxf(v, m);
        } else {
            atomicMax(&ls[g], f2u(v));
            g = group;
            v = m;
        }
    }
    __device__ __forceinline__ void flush(uint32_t* ls) {
        if (g >= 0) atomicMax(&ls[g], f2u(v));
    }
};

// Element e of a chunk loop over (n, pos, 8-channel chunk) NHWC views:
// e = (n * HW + pos) * CC + cc.  The divisions are by launch constants.
struct ChunkDivs {
    FastDiv cc;   // C / 8
    FastDiv hw;   // pixels per image
    FastDiv ow;   // output row width (maxpool / resize)
    FastDiv oh;   // output rows (resize)
};

inline ChunkDivs chunk_divs(int C, int HW, int OW = 1, int OH = 1) {
    return ChunkDivs{make_fastdiv((uint32_t)(C / 8)), make_fastdiv((uint32_t)HW), make_fastdiv((uint32_t)OW),
                     make_fastdiv((uint32_t)OH)};
}

__device__ __forceinline__ void chunk_split(uint32_t e, int CC, int HW, const ChunkDivs& d, int& n, int& pp,
                                            int& cc) {
    const uint32_t pix = fdiv(e, d.cc);
    cc = (int)(e - pix * (uint32_t)CC);
    n = (int)fdiv(pix, d.hw);
    pp = (int)(pix - (uint32_t)n * (uint32_t)HW);
}

__device__ __forceinline__ float max8_abs(const uint4& v) {
    const __half2* h = reinterpret_cast<const __half2*>(&v);
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float2 f = __half22float2(h[i]);
        m = fmaxf(m, fmaxf(fabsf(f.x), fabsf(f.y)));
    }
    return m;
}

// ---- amax --------------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void amax_slots_nhwc_kernel(
    const __half* x, int64_t nstride, int32_t cstride, int HW, int C, int chunks, ChunkDivs dv,
    SlotRef slots, int strip_n) {
    __shared__ uint32_t ls[kMaxSlots];
    const int CC = C / 8;
    const int G = C / 16;
    slots_init(ls, G);
    GroupMax gm;
    const int step = gridDim.x * blockDim.x;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < chunks; e += step) {
        int n, pp, cc;
        chunk_split((uint32_t)e, CC, HW, dv, n, pp, cc);
        const uint4 v = *reinterpret_cast<const uint4*>(x + n * nstride + (int64_t)pp * cstride + cc * 8);
        // strip_n > 0: the reference's NCHW memory strip of (n, group)
        gm.add(strip_n ? (n * G + (cc >> 1)) / strip_n : cc >> 1, max8_abs(v), ls);
    }
    gm.flush(ls);
    slots_flush(ls, G, slots);
}

// Reference amax buffer over NCHW memory (RT:3219-3259): slot 0 = max over the
// scanned strips, slot 1+g = strip g of 16*N*HW elements.
template <typename T>
__global__ __launch_bounds__(kThreads) void amax_strips_kernel(const T* x, int64_t strip, int G,
                                                             uint32_t* slots) {
    __shared__ uint32_t ls[kMaxSlots + 1];
    slots_init(ls, G + 1);
    const int64_t total = strip * G;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    GroupMax gm;
    float all = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        float v;
        if constexpr (sizeof(T) == 2) v = __half2float(reinterpret_cast<const __half*>(x)[i]);
        else v = reinterpret_cast<const float*>(x)[i];
        const float a = fabsf(v);
        gm.add(1 + (int)(i / strip), a, ls);
        all = fmaxf(all, a);
    }
    gm.flush(ls);
    if (G > 0) atomicMax(&ls[0], f2u(all));
    slots_flush(ls, G + 1, SlotRef{slots, 1u, 0u});
}

__device__ __forceinline__ float slots_amax(const SlotRef& r, int n) {
    uint32_t am = 0;
    for (uint32_t c = 0; c < r.stripes; ++c)
        for (int i = 0; i < n; ++i) am = max(am, r.p[c * r.stride + i]);
    return u2f(am);
}

// ---- quantize -----------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void quantize_nhwc_kernel(
    const __half* x, int64_t nstride, int32_t cstride, int HW, int C, int chunks, ChunkDivs dv,
    SlotRef slots, int nslots, int8_t* q) {
    const float a = slots_amax(slots, nslots);
    const float s = a > 0.0f ? 127.0f / a : 0.0f;
    const int CC = C / 8;
    const int step = gridDim.x * blockDim.x;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < chunks; e += step) {
        int n, pp, cc;
        chunk_split((uint32_t)e, CC, HW, dv, n, pp, cc);
        const int pix = n * HW + pp;
        const uint4 v = *reinterpret_cast<const uint4*>(x + n * nstride + (int64_t)pp * cstride + cc * 8);
        uint2 o = make_uint2(0u, 0u);
        if (a > 0.0f) {
            const __half2* h = reinterpret_cast<const __half2*>(&v);
            float2 f0 = __half22float2(h[0]), f1 = __half22float2(h[1]);
            float2 f2 = __half22float2(h[2]), f3 = __half22float2(h[3]);
            o.x = pack4_q(f0.x, f0.y, f1.x, f1.y, s);
            o.y = pack4_q(f2.x, f2.y, f3.x, f3.y, s);
        }
        *reinterpret_cast<uint2*>(q + (int64_t)pix * C + cc * 8) = o;
    }
}

// Reference NC/4HW4 pack (RT:3314-3346).
template <typename T>
__global__ __launch_bounds__(kThreads) void quant_pack_nchw_kernel(const T* x, int C, int HW,
                                                                 int64_t total4, const uint32_t* slots,
                                                                 int per_group, uint32_t* packed) {
    const int icg_count = C / 4;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total4; idx += step) {
        const int pos = (int)(idx % HW);
        const int64_t t = idx / HW;
        const int icg = (int)(t % icg_count);
        const int64_t n = t / icg_count;
        const float a = u2f(per_group ? slots[icg / 4 + 1] : slots[0]);
        if (!(a > 0.0f)) {
            packed[idx] = 0u;
            continue;
        }
        const float s = 127.0f / a;
        const int64_t base = ((n * icg_count + icg) * 4) * HW + pos;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (sizeof(T) == 2) v[j] = __half2float(reinterpret_cast<const __half*>(x)[base + j * HW]);
            else v[j] = reinterpret_cast<const float*>(x)[base + j * HW];
        }
        packed[idx] = pack4_q(v[0], v[1], v[2], v[3], s);
    }
}

// ---- glue -------------------------------------------------------------------------

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step) p[i] = v;
}

__global__ __launch_bounds__(kThreads) void copy_nhwc_kernel(
    const __half* src, int64_t s_nstride, int32_t s_cstride, __half* dst, int64_t d_nstride,
    int32_t d_cstride, int HW, int C, int chunks, ChunkDivs dv, SlotRef dst_slots) {
    __shared__ uint32_t ls[kMaxSlots];
    const int G = dst_slots.p ? C / 16 : 0;
    slots_init(ls, G);
    GroupMax gm;
    const int CC = C / 8;
    const int step = gridDim.x * blockDim.x;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < chunks; e += step) {
        int n, pp, cc;
        chunk_split((uint32_t)e, CC, HW, dv, n, pp, cc);
        const uint4 v = *reinterpret_cast<const uint4*>(src + n * s_nstride + (int64_t)pp * s_cstride + cc * 8);
        *reinterpret_cast<uint4*>(dst + n * d_nstride + (int64_t)pp * d_cstride + cc * 8) = v;
        if (G) gm.add(cc >> 1, max8_abs(v), ls);
    }
    if (G) gm.flush(ls);
    if (G) slots_flush(ls, G, dst_slots);
}

// KS > 0: window size fixed at compile time (every tap load in flight at
// once); KS == 0: runtime k.
template <int KS>
__global__ __launch_bounds__(kThreads) void maxpool_nhwc_kernel(
    const __half* x, int64_t x_nstride, int32_t x_cstride, __half* y, int64_t y_nstride,
    int32_t y_cstride, int H, int W, int C, int OH, int OW, int kr, int s, int pad, int chunks, ChunkDivs dv,
    SlotRef y_slots) {
    __shared__ uint32_t ls[kMaxSlots];
    const int G = y_slots.p ? C / 16 : 0;
    slots_init(ls, G);
    GroupMax gm;
    const int CC = C / 8;
    const int OHW = OH * OW;
    const int step = gridDim.x * blockDim.x;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < chunks; e += step) {
        int n, pp, cc;
        chunk_split((uint32_t)e, CC, OHW, dv, n, pp, cc);
        const int oy = (int)fdiv((uint32_t)pp, dv.ow), ox = pp - oy * OW;
        const __half* xb = x + n * x_nstride + cc * 8;
        float m[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) m[i] = -INFINITY;
        // Every tap loads (from a clamped in-image pixel) and padding taps
        // become -inf by a select: no load sits under a branch, so all of
        // them are in flight at once instead of one latency per tap.
        auto tap = [&](int ry, int rx) {
            const int iy = oy * s + ry - pad, ix = ox * s + rx - pad;
            const bool ok = (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W;
            const int cy = min(max(iy, 0), H - 1), cx = min(max(ix, 0), W - 1);
            const uint4 v = *reinterpret_cast<const uint4*>(xb + ((int64_t)cy * W + cx) * x_cstride);
            const __half2* h = reinterpret_cast<const __half2*>(&v);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float2 f = __half22float2(h[i]);
                m[2 * i] = fmaxf(m[2 * i], ok ? f.x : -INFINITY);
                m[2 * i + 1] = fmaxf(m[2 * i + 1], ok ? f.y : -INFINITY);
            }
        };
        if constexpr (KS > 0) {
#pragma unroll
            for (int ry = 0; ry < KS; ++ry)
#pragma unroll
                for (int rx = 0; rx < KS; ++rx) tap(ry, rx);
        } else {
            for (int ry = 0; ry < kr; ++ry)
                for (int rx = 0; rx < kr; ++rx) tap(ry, rx);
        }
        uint4 o;
        __half2* oh = reinterpret_cast<__half2*>(&o);
#pragma unroll
        for (int i = 0; i < 4; ++i) oh[i] = __floats2half2_rn(m[2 * i], m[2 * i + 1]);
        *reinterpret_cast<uint4*>(y + n * y_nstride + (int64_t)pp * y_cstride + cc * 8) = o;
        if (G) gm.add(cc >> 1, max8_abs(o), ls);
    }
    if (G) gm.flush(ls);
    if (G) slots_flush(ls, G, y_slots);
}

__global__ __launch_bounds__(kThreads) void resize_nearest_nhwc_kernel(
    const __half* x, int64_t x_nstride, int32_t x_cstride, __half* y, int64_t y_nstride,
    int32_t y_cstride, int H, int W, int C, int OH, int OW, int chunks, ChunkDivs dv, SlotRef y_slots) {
    __shared__ uint32_t ls[kMaxSlots];
    const int G = y_slots.p ? C / 16 : 0;
    slots_init(ls, G);
    GroupMax gm;
    const int CC = C / 8;
    const int OHW = OH * OW;
    const int step = gridDim.x * blockDim.x;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < chunks; e += step) {
        int n, pp, cc;
        chunk_split((uint32_t)e, CC, OHW, dv, n, pp, cc);
        const int oy = (int)fdiv((uint32_t)pp, dv.ow), ox = pp - oy * OW;
        // floor(o * in / out), as the reference's nearest resize
        const int iy = (int)fdiv((uint32_t)(oy * H), dv.oh), ix = (int)fdiv((uint32_t)(ox * W), dv.ow);
        const uint4 v = *reinterpret_cast<const uint4*>(
            x + n * x_nstride + ((int64_t)iy * W + ix) * x_cstride + cc * 8);
        *reinterpret_cast<uint4*>(y + n * y_nstride + (int64_t)pp * y_cstride + cc * 8) = v;
        if (G) gm.add(cc >> 1, max8_abs(v), ls);
    }
    if (G) gm.flush(ls);
    if (G) slots_flush(ls, G, y_slots);
}

// Nearest 2x upsample: one thread per input (pixel, 8-channel chunk), one
// 16-byte load and its four output copies, no loop (every load of the grid in
// flight at once).  max|y| = max|x| of the chunk.
__global__ __launch_bounds__(kThreads) void resize2x_nhwc_kernel(
    const __half* x, int64_t x_nstride, int32_t x_cstride, __half* y, int64_t y_nstride, int32_t y_cstride,
    int H, int W, int C, int chunks, ChunkDivs dv, SlotRef y_slots) {
    __shared__ uint32_t ls[kMaxSlots];
    const int G = y_slots.p ? C / 16 : 0;
    slots_init(ls, G);
    const int CC = C / 8;
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < chunks) {
        int n, pp, cc;
        chunk_split((uint32_t)e, CC, H * W, dv, n, pp, cc);
        const int iy = (int)fdiv((uint32_t)pp, dv.ow), ix = pp - iy * W;
        const uint4 v = *reinterpret_cast<const uint4*>(x + n * x_nstride + (int64_t)pp * x_cstride + cc * 8);
        __half* yb = y + n * y_nstride + ((int64_t)(2 * iy) * (2 * W) + 2 * ix) * y_cstride + cc * 8;
        *reinterpret_cast<uint4*>(yb) = v;
        *reinterpret_cast<uint4*>(yb + y_cstride) = v;
        *reinterpret_cast<uint4*>(yb + (int64_t)(2 * W) * y_cstride) = v;
        *reinterpret_cast<uint4*>(yb + (int64_t)(2 * W + 1) * y_cstride) = v;
        if (G) atomicMax(&ls[cc >> 1], f2u(max8_abs(v)));
    }
    if (G) slots_flush(ls, G, y_slots);
}

// SPPF's three chained 5x5 / stride 1 / pad 2 max pools in one pass: with
// -inf padding, pool5(pool5(x)) = pool9(x) and pool5(pool5(pool5(x))) =
// pool13(x) (every window of the composition lies inside the image together
// with a path of in-image 5x5 windows).  A block owns one (image, 8-channel
// chunk) plane: the plane goes to LDS, a horizontal pass takes the row maxima
// over +-2, +-4 and +-6 columns, a vertical pass the column maxima of those
// over +-2, +-4 and +-6 rows.  Max is exact in fp16.
__device__ __forceinline__ uint4 hmax8(uint4 a, uint4 b) {
    // packed fp16 maximum (maxnum: a NaN operand yields the other, as fmaxf)
    const v8h m = __builtin_elementwise_max(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b));
    return __builtin_bit_cast(uint4, m);
}

__global__ __launch_bounds__(kThreads) void sppf_maxpool_nhwc_kernel(
    const __half* x, int64_t x_nstride, int32_t x_cstride, __half* y1, __half* y2, __half* y3, int64_t y_nstride,
    int32_t y_cstride, int H, int W, int C, SlotRef s1, SlotRef s2, SlotRef s3) {
    extern __shared__ uint4 sp[];  // [4][H*W]: plane, row maxima over +-2, +-4, +-6
    __shared__ uint32_t lm[3];
    const int HW = H * W;
    const int CC = C / 8;
    // the CC blocks of one image on one XCD: each reads 16 bytes of every
    // pixel's channels, so the others' parts of the lines hit its L2
    const int b = xcd_remap(blockIdx.x, gridDim.x);
    const int n = b / CC, cc = b - n * CC;
    const int tid = threadIdx.x;
    if (tid < 3) lm[tid] = 0u;
    const __half* xb = x + n * x_nstride + cc * 8;
    for (int p = tid; p < HW; p += kThreads) sp[p] = *reinterpret_cast<const uint4*>(xb + (int64_t)p * x_cstride);
    __syncthreads();
    for (int p = tid; p < HW; p += kThreads) {
        const int r = p / W, c = p - r * W;
        uint4 m = sp[p];
        for (int d = 1; d <= 6; ++d) {
            if (c - d >= 0) m = hmax8(m, sp[p - d]);
            if (c + d < W) m = hmax8(m, sp[p + d]);
            if (d == 2) sp[HW + p] = m;
            if (d == 4) sp[2 * HW + p] = m;
        }
        sp[3 * HW + p] = m;
    }
    __syncthreads();
    float g1 = 0.0f, g2 = 0.0f, g3 = 0.0f;
    __half* o1 = y1 + n * y_nstride + cc * 8;
    __half* o2 = y2 + n * y_nstride + cc * 8;
    __half* o3 = y3 + n * y_nstride + cc * 8;
    for (int p = tid; p < HW; p += kThreads) {
        const int r = p / W;
        uint4 m1 = sp[HW + p], m2 = sp[2 * HW + p], m3 = sp[3 * HW + p];
        for (int d = 1; d <= 6; ++d) {
            if (d <= 2) {
                if (r - d >= 0) m1 = hmax8(m1, sp[HW + p - d * W]);
                if (r + d < H) m1 = hmax8(m1, sp[HW + p + d * W]);
            }
            if (d <= 4) {
                if (r - d >= 0) m2 = hmax8(m2, sp[2 * HW + p - d * W]);
                if (r + d < H) m2 = hmax8(m2, sp[2 * HW + p + d * W]);
            }
            if (r - d >= 0) m3 = hmax8(m3, sp[3 * HW + p - d * W]);
            if (r + d < H) m3 = hmax8(m3, sp[3 * HW + p + d * W]);
        }
        *reinterpret_cast<uint4*>(o1 + (int64_t)p * y_cstride) = m1;
        *reinterpret_cast<uint4*>(o2 + (int64_t)p * y_cstride) = m2;
        *reinterpret_cast<uint4*>(o3 + (int64_t)p * y_cstride) = m3;
        g1 = fmaxf(g1, max8_abs(m1));
        g2 = fmaxf(g2, max8_abs(m2));
        g3 = fmaxf(g3, max8_abs(m3));
    }
    g1 = wave_max(g1);
    g2 = wave_max(g2);
    g3 = wave_max(g3);
    if ((tid & 63) == 0) {
        if (g1 > 0.0f) atomicMax(&lm[0], f2u(g1));
        if (g2 > 0.0f) atomicMax(&lm[1], f2u(g2));
        if (g3 > 0.0f) atomicMax(&lm[2], f2u(g3));
    }
    __syncthreads();
    if (tid < 3) {
        const SlotRef& sr = tid == 0 ? s1 : (tid == 1 ? s2 : s3);
        if (sr.p && lm[tid]) slot_max(slot_copy(sr, b) + (cc >> 1), u2f(lm[tid]));
    }
}

__global__ __launch_bounds__(kThreads) void add_nhwc_kernel(
    const __half* a, int64_t a_nstride, int32_t a_cstride, const __half* b, int64_t b_nstride,
    int32_t b_cstride, __half* y, int64_t y_nstride, int32_t y_cstride, int HW, int C, int chunks,
    ChunkDivs dv, SlotRef y_slots) {
    __shared__ uint32_t ls[kMaxSlots];
    const int G = y_slots.p ? C / 16 : 0;
    slots_init(ls, G);
    GroupMax gm;
    const int CC = C / 8;
    const int step = gridDim.x * blockDim.x;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < chunks; e += step) {
        int n, pp, cc;
        chunk_split((uint32_t)e, CC, HW, dv, n, pp, cc);
        const uint4 va = *reinterpret_cast<const uint4*>(a + n * a_nstride + (int64_t)pp * a_cstride + cc * 8);
        const uint4 vb = *reinterpret_cast<const uint4*>(b + n * b_nstride + (int64_t)pp * b_cstride + cc * 8);
        const __half2* ha = reinterpret_cast<const __half2*>(&va);
        const __half2* hb = reinterpret_cast<const __half2*>(&vb);
        uint4 o;
        __half2* ho = reinterpret_cast<__half2*>(&o);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float2 fa = __half22float2(ha[i]), fb = __half22float2(hb[i]);
            ho[i] = __floats2half2_rn(fa.x + fb.x, fa.y + fb.y);
        }
        *reinterpret_cast<uint4*>(y + n * y_nstride + (int64_t)pp * y_cstride + cc * 8) = o;
        if (G) gm.add(cc >> 1, max8_abs(o), ls);
    }
    if (G) gm.flush(ls);
    if (G) slots_flush(ls, G, y_slots);
}

__global__ __launch_bounds__(kThreads) void nchw_f32_to_nhwc_f16_kernel(
    const float* x, __half* y, int64_t y_nstride, int32_t y_cstride, int C, int HW, int64_t total,
    SlotRef y_slots) {
    __shared__ uint32_t ls[kMaxSlots];
    const int G = y_slots.p ? C / 16 : 0;
    slots_init(ls, G);
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        // i enumerates (n, pos, c) so that the fp16 stores are contiguous
        const int c = (int)(i % C);
        const int64_t t = i / C;
        const int64_t pos = t % HW;
        const int64_t n = t / HW;
        const __half h = __float2half(x[(n * C + c) * HW + pos]);
        y[n * y_nstride + pos * y_cstride + c] = h;
        if (G) atomicMax(&ls[c >> 4], f2u(fabsf(__half2float(h))));
    }
    if (G) slots_flush(ls, G, y_slots);
}

// One thread per (pixel, 8-channel group): reads up to 8 fp32 planes
// (coalesced across the pixels of a wave) and writes one 16-byte fp16 chunk,
// zero-filling the channels past C.
__global__ __launch_bounds__(kThreads) void nchw_f32_to_nhwc8_kernel(const float* x, __half* y, int C, int Cp,
                                                                    int HW, int total) {
    const int G = Cp / 8;
    const int step = gridDim.x * blockDim.x;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        const int pix = i / G;
        const int g = i - pix * G;
        const int n = pix / HW;
        const int pos = pix - n * HW;
        const float* src = x + ((int64_t)n * C + g * 8) * HW + pos;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (g * 8 + e < C) ? src[(int64_t)e * HW] : 0.0f;
        uint4 o;
        __half2* oh = reinterpret_cast<__half2*>(&o);
#pragma unroll
        for (int e = 0; e < 4; ++e) oh[e] = __floats2half2_rn(v[2 * e], v[2 * e + 1]);
        *reinterpret_cast<uint4*>(y + (int64_t)pix * Cp + g * 8) = o;
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void nhwc_to_nchw_f32_kernel(const T* x, int64_t x_nstride,
                                                                   int32_t x_cstride, float* y, int C,
                                                                   int HW, int64_t total) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        const int64_t pos = i % HW;
        const int64_t t = i / HW;
        const int c = (int)(t % C);
        const int64_t n = t / C;
        const int64_t src = n * x_nstride + pos * x_cstride + c;
        float v;
        if constexpr (sizeof(T) == 2) v = __half2float(reinterpret_cast<const __half*>(x)[src]);
        else v = reinterpret_cast<const float*>(x)[src];
        y[i] = v;
    }
}

}  // namespace

hipError_t launch_amax_slots_nhwc(const __half* x, int64_t nstride, int32_t cstride, int N, int HW, int C,
                                  SlotRef slots, hipStream_t stream) {
    if (C % 16 != 0 || C / 16 > kMaxSlots) return hipErrorInvalidValue;
    const int64_t chunks = (int64_t)N * HW * (C / 8);
    if (chunks >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(amax_slots_nhwc_kernel, dim3(grid_cols(chunks, C)), dim3(kThreads), 0, stream, x,
                       nstride, cstride, HW, C, (int)chunks, chunk_divs(C, HW), slots, 0);
    return hipGetLastError();
}

hipError_t launch_amax_strips_nhwc(const __half* x, int64_t nstride, int32_t cstride, int N, int HW, int C,
                                   uint32_t* slots, hipStream_t stream) {
    if (C % 16 != 0 || C / 16 > kMaxSlots || N < 1) return hipErrorInvalidValue;
    const int64_t chunks = (int64_t)N * HW * (C / 8);
    if (chunks >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(amax_slots_nhwc_kernel, dim3(grid_cols(chunks, C)), dim3(kThreads), 0, stream, x,
                       nstride, cstride, HW, C, (int)chunks, chunk_divs(C, HW), SlotRef{slots, 1u, 0u}, N);
    return hipGetLastError();
}

hipError_t launch_amax_strips_nchw(const void* x, bool f16, int N, int C, int HW, uint32_t* slots,
                                   hipStream_t stream) {
    const int G = C / 16;
    if (G > kMaxSlots) return hipErrorInvalidValue;
    const int64_t strip = (int64_t)16 * N * HW;
    const int grid = grid_for(strip * (G > 0 ? G : 1));
    if (f16)
        hipLaunchKernelGGL(amax_strips_kernel<__half>, dim3(grid), dim3(kThreads), 0, stream,
                           reinterpret_cast<const __half*>(x), strip, G, slots);
    else
        hipLaunchKernelGGL(amax_strips_kernel<float>, dim3(grid), dim3(kThreads), 0, stream,
                           reinterpret_cast<const float*>(x), strip, G, slots);
    return hipGetLastError();
}

hipError_t launch_quantize_nhwc(const __half* x, int64_t nstride, int32_t cstride, int N, int HW, int C,
                                SlotRef slots, int nslots, int8_t* q, hipStream_t stream) {
    if (C % 8 != 0) return hipErrorInvalidValue;
    const int64_t chunks = (int64_t)N * HW * (C / 8);
    if (chunks >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(quantize_nhwc_kernel, dim3(grid_cols(chunks, C)), dim3(kThreads), 0, stream, x, nstride,
                       cstride, HW, C, (int)chunks, chunk_divs(C, HW), slots, nslots, q);
    return hipGetLastError();
}

hipError_t launch_quant_pack_nchw(const void* x, bool f16, int N, int C, int HW, const uint32_t* slots,
                                  bool per_group, uint32_t* packed, hipStream_t stream) {
    if (C % 4 != 0) return hipErrorInvalidValue;
    const int64_t total4 = (int64_t)N * (C / 4) * HW;
    const int grid = grid_for(total4);
    if (f16)
        hipLaunchKernelGGL(quant_pack_nchw_kernel<__half>, dim3(grid), dim3(kThreads), 0, stream,
                           reinterpret_cast<const __half*>(x), C, HW, total4, slots, (int)per_group, packed);
    else
        hipLaunchKernelGGL(quant_pack_nchw_kernel<float>, dim3(grid), dim3(kThreads), 0, stream,
                           reinterpret_cast<const float*>(x), C, HW, total4, slots, (int)per_group, packed);
    return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(n)), dim3(kThreads), 0, stream, p, n, v);
    return hipGetLastError();
}

hipError_t launch_copy_nhwc(const __half* src, int64_t s_nstride, int32_t s_cstride, __half* dst,
                            int64_t d_nstride, int32_t d_cstride, int N, int HW, int C, SlotRef dst_slots,
                            hipStream_t stream) {
    if (C % 8 != 0 || (dst_slots.p && (C % 16 != 0 || C / 16 > kMaxSlots))) return hipErrorInvalidValue;
    const int64_t chunks = (int64_t)N * HW * (C / 8);
    if (chunks >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(copy_nhwc_kernel, dim3(grid_cols(chunks, C)), dim3(kThreads), 0, stream, src, s_nstride,
                       s_cstride, dst, d_nstride, d_cstride, HW, C, (int)chunks, chunk_divs(C, HW), dst_slots);
    return hipGetLastError();
}

hipError_t launch_maxpool_nhwc(const __half* x, int64_t x_nstride, int32_t x_cstride, __half* y,
                               int64_t y_nstride, int32_t y_cstride, int N, int H, int W, int C, int OH,
                               int OW, int k, int s, int pad, SlotRef y_slots, hipStream_t stream) {
    if (C % 8 != 0 || (y_slots.p && (C % 16 != 0 || C / 16 > kMaxSlots))) return hipErrorInvalidValue;
    const int64_t chunks = (int64_t)N * OH * OW * (C / 8);
    if (chunks >= INT32_MAX) return hipErrorInvalidValue;
    const ChunkDivs dv = chunk_divs(C, OH * OW, OW);
    if (k == 5)
        hipLaunchKernelGGL(maxpool_nhwc_kernel<5>, dim3(grid_cols(chunks, C)), dim3(kThreads), 0, stream, x,
                           x_nstride, x_cstride, y, y_nstride, y_cstride, H, W, C, OH, OW, k, s, pad, (int)chunks,
                           dv, y_slots);
    else
        hipLaunchKernelGGL(maxpool_nhwc_kernel<0>, dim3(grid_cols(chunks, C)), dim3(kThreads), 0, stream, x,
                           x_nstride, x_cstride, y, y_nstride, y_cstride, H, W, C, OH, OW, k, s, pad, (int)chunks,
                           dv, y_slots);
    return hipGetLastError();
}

hipError_t launch_resize_nearest_nhwc(const __half* x, int64_t x_nstride, int32_t x_cstride, __half* y,
                                      int64_t y_nstride, int32_t y_cstride, int N, int H, int W, int C,
                                      int OH, int OW, SlotRef y_slots, hipStream_t stream) {
    if (C % 8 != 0 || (y_slots.p && (C % 16 != 0 || C / 16 > kMaxSlots))) return hipErrorInvalidValue;
    const int64_t chunks = (int64_t)N * OH * OW * (C / 8);
    if (chunks >= INT32_MAX || (int64_t)OH * H >= INT32_MAX || (int64_t)OW * W >= INT32_MAX)
        return hipErrorInvalidValue;
    if (OH == 2 * H && OW == 2 * W) {
        const int64_t in_chunks = (int64_t)N * H * W * (C / 8);
        hipLaunchKernelGGL(resize2x_nhwc_kernel, dim3((unsigned)((in_chunks + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, stream, x, x_nstride, x_cstride, y, y_nstride, y_cstride, H, W, C,
                           (int)in_chunks, chunk_divs(C, H * W, W), y_slots);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(resize_nearest_nhwc_kernel, dim3(grid_cols(chunks, C)), dim3(kThreads), 0, stream, x,
                       x_nstride, x_cstride, y, y_nstride, y_cstride, H, W, C, OH, OW, (int)chunks,
                       chunk_divs(C, OH * OW, OW, OH), y_slots);
    return hipGetLastError();
}

bool sppf_fits(int H, int W) { return H >= 1 && W >= 1 && (int64_t)H * W * 64 <= 96 * 1024; }

hipError_t launch_sppf_maxpool_nhwc(const __half* x, int64_t x_nstride, int32_t x_cstride, __half* y1, __half* y2,
                                    __half* y3, int64_t y_nstride, int32_t y_cstride, int N, int H, int W, int C,
                                    SlotRef s1, SlotRef s2, SlotRef s3, hipStream_t stream) {
    if (C % 8 != 0 || !sppf_fits(H, W) || ((s1.p || s2.p || s3.p) && C % 16 != 0)) return hipErrorInvalidValue;
    const int64_t blocks = (int64_t)N * (C / 8);
    if (blocks >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(sppf_maxpool_nhwc_kernel, dim3((unsigned)blocks), dim3(kThreads),
                       (size_t)H * W * 64, stream, x, x_nstride, x_cstride, y1, y2, y3, y_nstride, y_cstride, H, W,
                       C, s1, s2, s3);
    return hipGetLastError();
}

hipError_t launch_add_nhwc(const __half* a, int64_t a_nstride, int32_t a_cstride, const __half* b,
                           int64_t b_nstride, int32_t b_cstride, __half* y, int64_t y_nstride, int32_t y_cstride,
                           int N, int HW, int C, SlotRef y_slots, hipStream_t stream) {
    if (C % 8 != 0 || (y_slots.p && (C % 16 != 0 || C / 16 > kMaxSlots))) return hipErrorInvalidValue;
    const int64_t chunks = (int64_t)N * HW * (C / 8);
    if (chunks >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(add_nhwc_kernel, dim3(grid_cols(chunks, C)), dim3(kThreads), 0, stream, a, a_nstride,
                       a_cstride, b, b_nstride, b_cstride, y, y_nstride, y_cstride, HW, C, (int)chunks,
                       chunk_divs(C, HW), y_slots);
    return hipGetLastError();
}

hipError_t launch_nchw_f32_to_nhwc_f16(const float* x, __half* y, int64_t y_nstride, int32_t y_cstride, int N,
                                       int C, int HW, SlotRef y_slots, hipStream_t stream) {
    if (y_slots.p && (C % 16 != 0 || C / 16 > kMaxSlots)) return hipErrorInvalidValue;
    const int64_t total = (int64_t)N * C * HW;
    hipLaunchKernelGGL(nchw_f32_to_nhwc_f16_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream, x, y,
                       y_nstride, y_cstride, C, HW, total, y_slots);
    return hipGetLastError();
}

hipError_t launch_nchw_f32_to_nhwc8(const float* x, __half* y, int N, int C, int HW, hipStream_t stream) {
    const int Cp = (C + 7) / 8 * 8;
    const int64_t total = (int64_t)N * HW * (Cp / 8);
    if (total >= INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(nchw_f32_to_nhwc8_kernel, dim3(grid_for(total)), dim3(kThreads), 0, stream, x, y, C, Cp, HW,
                       (int)total);
    return hipGetLastError();
}

hipError_t launch_nhwc_to_nchw_f32(const void* x, bool f16, int64_t x_nstride, int32_t x_cstride, float* y,
                                   int N, int C, int HW, hipStream_t stream) {
    const int64_t total = (int64_t)N * C * HW;
    if (f16)
        hipLaunchKernelGGL(nhwc_to_nchw_f32_kernel<__half>, dim3(grid_for(total)), dim3(kThreads), 0, stream,
                           reinterpret_cast<const __half*>(x), x_nstride, x_cstride, y, C, HW, total);
    else
        hipLaunchKernelGGL(nhwc_to_nchw_f32_kernel<float>, dim3(grid_for(total)), dim3(kThreads), 0, stream,
                           reinterpret_cast<const float*>(x), x_nstride, x_cstride, y, C, HW, total);
    return hipGetLastError();
}

}  // namespace aexrt
