// YOLO output0 postprocess: decode + confidence filter, class-wise NMS and
// top-k, as the reference runs it on the GPU after the network
// (native/aexrt_d3d12_runtime.cpp:15300-15356 decode/filter, 15637-15691 NMS
// mark, 15693-15735 top-k; recorded at 27104-27219).
//
// The reference uses three dispatches and appends candidates with an atomic
// counter, so their order (and which ones survive the max_candidates cap) is
// whatever order its threads ran in.  Here one 1024-thread block does all of
// it in LDS: anchors are scored in chunks of 1024, compacted with a block
// scan in anchor order (one of the orders the reference can produce, and a
// deterministic one), then every candidate is marked and ranked.  output0 is
// small (84 x 2100 floats at 320x320) and read once; the pairwise NMS over
// at most max_candidates boxes is the only quadratic step.
//
// Two decoders feed the same NMS and top-k:
// * decoded output0 ([4 (+1 objectness) + classes][anchors]: cx, cy, w, h,
//   scores), RT:15300-15356;
// * the raw Detect head ([64 + classes][anchors]: 4 x 16 DFL bin logits, then
//   class logits; anchors level by level), the post-conv part of the
//   reference's fused head decode (RT:15465-15636): score = sigmoid(logit),
//   per side the softmax expectation of the 16 bins, box = (anchor centre -/+
//   distance) x stride.
//
// Arithmetic follows the reference's expressions one operation at a time
// (no contraction): x1 = cx - 0.5 w, IoU = inter / max(area_a + area_b -
// inter, 1e-7) with IEEE division, strict-greater class argmax (first max
// wins), a candidate passes unless score < conf.  exp is post_exp below (the
// reference's comes from its shader compiler and driver), so that results
// are reproducible bit for bit on the host.
#include "common.h"
#include "kernels.h"

namespace aexrt {

namespace {

constexpr int kPostThreads = 1024;
constexpr int kPostWaves = kPostThreads / 64;
constexpr int kDflBins = 16;

struct PostParams {
    const float* out;  // element (channel ch, anchor a) at out[ch * ch_stride + a * a_stride]
    int ch_stride, a_stride;
    int anchors, classes, has_obj;
    float conf, iou;
    int max_cand, max_det;
    float* dets;       // [max_det][6]: x1, y1, x2, y2, score, class
    uint32_t* count;   // detections written
    // raw-head decode: level l covers anchors [lev_off[l], lev_off[l+1]) of a
    // grid lev_w[l] wide, stride lev_stride[l]
    int nlev;
    int lev_off[kYoloMaxLevels + 1];
    int lev_w[kYoloMaxLevels];
    float lev_stride[kYoloMaxLevels];
};

// e^x in fp32: Cody-Waite reduction x = k ln2 + r with ln2 split into a
// 16-bit head (k * head is exact) and a tail, |r| <= ln2/2, e^r by its
// degree-7 Taylor polynomial (truncation < 6e-9 relative) in Horner form,
// scaled by 2^k.  Below -87 it returns 0 (the true value is under 2e-38),
// above 88.5 infinity.
__device__ __forceinline__ float post_exp(float x) {
#pragma clang fp contract(off)
    if (x != x) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.5f) return __builtin_inff();
    const float k = __builtin_rintf(x * 1.44269504f);
    const float r = (x - k * 0.693145751953125f) - k * 1.42860677e-06f;
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return __builtin_ldexpf(p, (int)k);
}

__device__ __forceinline__ float post_sigmoid(float x) {
#pragma clang fp contract(off)
    return 1.0f / (1.0f + post_exp(-x));
}

__device__ __forceinline__ float box_iou(const float* a, const float* b) {
#pragma clang fp contract(off)
    const float x1 = fmaxf(a[0], b[0]);
    const float y1 = fmaxf(a[1], b[1]);
    const float x2 = fminf(a[2], b[2]);
    const float y2 = fminf(a[3], b[3]);
    const float iw = fmaxf(0.0f, x2 - x1);
    const float ih = fmaxf(0.0f, y2 - y1);
    const float inter = iw * ih;
    const float area_a = fmaxf(0.0f, a[2] - a[0]) * fmaxf(0.0f, a[3] - a[1]);
    const float area_b = fmaxf(0.0f, b[2] - b[0]) * fmaxf(0.0f, b[3] - b[1]);
    return inter / fmaxf(area_a + area_b - inter, 1e-7f);
}

// j outranks i: higher score, or equal score and earlier candidate
__device__ __forceinline__ bool outranks(float sj, int j, float si, int i) { return sj > si || (sj == si && j < i); }

template <bool DFL>
__global__ __launch_bounds__(kPostThreads) void yolo_decode_nms_topk_kernel(PostParams p) {
#pragma clang fp contract(off)
    extern __shared__ float l_cand[];  // [max_cand][6], then keep flags [max_cand]
    uint32_t* l_keep = reinterpret_cast<uint32_t*>(l_cand + 6 * p.max_cand);
    __shared__ uint32_t l_wsum[kPostWaves];
    __shared__ uint32_t l_total;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) l_total = 0;
    __syncthreads();
    const int cls_off = p.has_obj ? 5 : 4;
    // ---- decode + filter, compacted in anchor order ----
    for (int a0 = 0; a0 < p.anchors; a0 += kPostThreads) {
        const int a = a0 + tid;
        bool pass = false;
        float best = 0.0f;
        int best_cls = 0;
        if (a < p.anchors && p.classes > 0) {
            const float* col = p.out + (int64_t)a * p.a_stride;
            if constexpr (DFL) {
                const int c0 = 4 * kDflBins;
                best = post_sigmoid(col[(int64_t)c0 * p.ch_stride]);
                for (int c = 1; c < p.classes; ++c) {
                    const float s = post_sigmoid(col[(int64_t)(c0 + c) * p.ch_stride]);
                    if (s > best) {
                        best = s;
                        best_cls = c;
                    }
                }
            } else {
                const float obj = p.has_obj ? col[4 * (int64_t)p.ch_stride] : 1.0f;
                best = obj * col[(int64_t)cls_off * p.ch_stride];
                for (int c = 1; c < p.classes; ++c) {
                    const float s = obj * col[(int64_t)(cls_off + c) * p.ch_stride];
                    if (s > best) {
                        best = s;
                        best_cls = c;
                    }
                }
            }
            pass = !(best < p.conf);
        }
        const uint64_t m = __ballot(pass);
        const uint32_t below = (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
        if (lane == 0) l_wsum[wave] = (uint32_t)__popcll(m);
        __syncthreads();
        uint32_t off = l_total;
        for (int w = 0; w < wave; ++w) off += l_wsum[w];
        const uint32_t idx = off + below;
        if (pass && idx < (uint32_t)p.max_cand) {
            const float* col = p.out + (int64_t)a * p.a_stride;
            float* c = l_cand + 6 * idx;
            if constexpr (DFL) {
                // side d: softmax expectation of bins 16d..16d+15
                float dist[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    float m = -3.402823e38f;
                    for (int b = 0; b < kDflBins; ++b) m = fmaxf(m, col[(int64_t)(d * kDflBins + b) * p.ch_stride]);
                    float sum = 0.0f, acc = 0.0f;
                    for (int b = 0; b < kDflBins; ++b) {
                        const float e = post_exp(col[(int64_t)(d * kDflBins + b) * p.ch_stride] - m);
                        sum = sum + e;
                        acc = acc + e * (float)b;
                    }
                    dist[d] = acc / fmaxf(sum, 1e-20f);
                }
                int l = 0;
                while (l + 1 < p.nlev && a >= p.lev_off[l + 1]) ++l;
                const int pos = a - p.lev_off[l];
                const int gy = pos / p.lev_w[l];
                const float ax = (float)(pos - gy * p.lev_w[l]) + 0.5f, ay = (float)gy + 0.5f;
                const float st = p.lev_stride[l];
                c[0] = (ax - dist[0]) * st;
                c[1] = (ay - dist[1]) * st;
                c[2] = (ax + dist[2]) * st;
                c[3] = (ay + dist[3]) * st;
            } else {
                const float cx = col[0], cy = col[p.ch_stride], w = col[2 * (int64_t)p.ch_stride],
                            h = col[3 * (int64_t)p.ch_stride];
                const float hw = 0.5f * w, hh = 0.5f * h;
                c[0] = cx - hw;
                c[1] = cy - hh;
                c[2] = cx + hw;
                c[3] = cy + hh;
            }
            c[4] = best;
            c[5] = (float)best_cls;
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t t = l_total;
            for (int w = 0; w < kPostWaves; ++w) t += l_wsum[w];
            l_total = t;
        }
        __syncthreads();
    }
    const int count = (int)min(l_total, (uint32_t)p.max_cand);
    // ---- NMS mark: dropped when a same-class candidate that outranks it overlaps it ----
    for (int i = tid; i < count; i += kPostThreads) {
        const float* ci = l_cand + 6 * i;
        uint32_t keep = 1u;
        for (int j = 0; j < count; ++j) {
            if (j == i) continue;
            const float* cj = l_cand + 6 * j;
            if (cj[5] != ci[5]) continue;
            if (outranks(cj[4], j, ci[4], i) && box_iou(ci, cj) > p.iou) {
                keep = 0u;
                break;
            }
        }
        l_keep[i] = keep;
    }
    __syncthreads();
    // ---- top-k: a kept candidate's rank among the kept ones is its slot ----
    uint32_t kept = 0;
    for (int i = tid; i < count; i += kPostThreads) {
        if (!l_keep[i]) continue;
        ++kept;
        const float* ci = l_cand + 6 * i;
        int rank = 0;
        for (int j = 0; j < count; ++j)
            if (j != i && l_keep[j] && outranks(l_cand[6 * j + 4], j, ci[4], i)) ++rank;
        if (rank < p.max_det)
            for (int k = 0; k < 6; ++k) p.dets[6 * rank + k] = ci[k];
    }
    // ranks of the kept candidates are 0..K-1, so the count is min(K, max_det)
    uint32_t ws = kept;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ws += (uint32_t)__shfl_xor((int)ws, o, 64);
    if (lane == 0) l_wsum[wave] = ws;
    __syncthreads();
    if (tid == 0) {
        uint32_t k = 0;
        for (int w = 0; w < kPostWaves; ++w) k += l_wsum[w];
        p.count[0] = min(k, (uint32_t)p.max_det);
    }
}

}  // namespace

hipError_t launch_yolo_decode_nms_topk(const float* out, int ch_stride, int a_stride, int anchors, int classes,
                                       int has_objectness, float conf, float iou, int max_candidates,
                                       int max_detections, float* dets, uint32_t* count, hipStream_t stream,
                                       const YoloLevels* levels) {
    if ((!out && anchors > 0) || !dets || !count || anchors < 0 || classes < 0 || max_candidates < 1 ||
        max_candidates > kYoloMaxCandidates || max_detections < 1)
        return hipErrorInvalidValue;
    PostParams p{};
    p.out = out;
    p.ch_stride = ch_stride;
    p.a_stride = a_stride;
    p.anchors = anchors;
    p.classes = classes;
    p.has_obj = has_objectness ? 1 : 0;
    p.conf = conf;
    p.iou = iou;
    p.max_cand = max_candidates;
    p.max_det = max_detections;
    p.dets = dets;
    p.count = count;
    if (levels) {
        // raw Detect head: the levels must tile the anchors exactly
        if (has_objectness || levels->n < 1 || levels->n > kYoloMaxLevels) return hipErrorInvalidValue;
        int off = 0;
        for (int l = 0; l < levels->n; ++l) {
            if (levels->h[l] < 1 || levels->w[l] < 1) return hipErrorInvalidValue;
            p.lev_off[l] = off;
            p.lev_w[l] = levels->w[l];
            p.lev_stride[l] = levels->stride[l];
            off += levels->h[l] * levels->w[l];
        }
        p.lev_off[levels->n] = off;
        p.nlev = levels->n;
        if (off != anchors) return hipErrorInvalidValue;
    }
    const size_t lds = (size_t)max_candidates * 7 * sizeof(float);
    if (levels)
        hipLaunchKernelGGL(yolo_decode_nms_topk_kernel<true>, dim3(1), dim3(kPostThreads), lds, stream, p);
    else
        hipLaunchKernelGGL(yolo_decode_nms_topk_kernel<false>, dim3(1), dim3(kPostThreads), lds, stream, p);
    return hipGetLastError();
}

}  // namespace aexrt
