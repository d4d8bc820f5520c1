// Op-level C ABI of libaexrt_hip.so: argument validation, host-side weight
// repack, and dispatch of one hot-path kernel per call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/aexrt_hip.h"
#include "internal.h"
#include "kernels.h"

namespace aexrt {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
const char* last_error() { return g_last_error.c_str(); }

bool check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return false;
}

bool is_int8_algorithm(uint32_t a) { return a == 51u || a == 52u || a == 53u; }
bool is_winograd_algorithm(uint32_t a) { return a == 40u || a == 46u; }

static inline uint32_t round_up(uint32_t v, uint32_t m) { return (v + m - 1u) / m * m; }

// Reference int8 eligibility, native/aexrt_d3d12_runtime.cpp:9399-9422, plus
// in_channels % 16 == 0: amax is tracked per 16-channel group here, and the
// reference itself only scans C/16 full groups (9406 + 21631-21640), so a
// C % 16 tail would be quantized against a partial amax.
bool can_use_int8(const AexrtConv2DDesc& d, uint32_t kernel_elems) {
    if (d.groups != 1 || (d.in_channels % 4u) != 0 || (d.out_channels % 4u) != 0) return false;
    if ((d.in_channels % 16u) != 0) return false;
    if (kernel_elems == 1u) {
        if (d.kernel_h != 1 || d.kernel_w != 1 || d.stride_h != 1 || d.stride_w != 1 || d.pad_top != 0 ||
            d.pad_left != 0 || d.dilation_h != 1 || d.dilation_w != 1)
            return false;
        return (d.out_channels % 8u) == 0 && d.in_h == d.out_h && d.in_w == d.out_w;
    }
    if (kernel_elems == 9u) {
        if (d.kernel_h != 3 || d.kernel_w != 3 || d.dilation_h != 1 || d.dilation_w != 1 || d.pad_top != 1 ||
            d.pad_left != 1)
            return false;
        if (d.stride_h == 2 && d.stride_w == 2)
            return d.in_h >= d.out_h * 2u - 1u && d.in_w >= d.out_w * 2u - 1u;
        if (d.stride_h != 1 || d.stride_w != 1) return false;
        return d.in_h == d.out_h && d.in_w == d.out_w;
    }
    return false;
}

uint32_t int8_kernel_elems(uint32_t algorithm) { return algorithm == 51u ? 1u : 9u; }

bool winograd_shape_ok(const AexrtConv2DDesc& d) {
    return d.kernel_h == 3 && d.kernel_w == 3 && d.stride_h == 1 && d.stride_w == 1 && d.pad_top == 1 &&
           d.pad_left == 1 && d.dilation_h == 1 && d.dilation_w == 1 && d.groups == 1 &&
           (d.in_channels % 4u) == 0 && (d.out_h % 2u) == 0 && (d.out_w % 2u) == 0 && d.in_h == d.out_h &&
           d.in_w == d.out_w;
}

bool generic_shape_ok(const AexrtConv2DDesc& d) {
    if (d.groups != 1 || d.dilation_h != 1 || d.dilation_w != 1) return false;
    if (d.stride_h != d.stride_w || d.pad_top != d.pad_left || d.kernel_h == 0 || d.kernel_w == 0) return false;
    const int64_t oh = ((int64_t)d.in_h + 2 * d.pad_top - d.kernel_h) / d.stride_h + 1;
    const int64_t ow = ((int64_t)d.in_w + 2 * d.pad_left - d.kernel_w) / d.stride_w + 1;
    return oh == d.out_h && ow == d.out_w;
}

WeightGeom weight_geom(const AexrtConv2DDesc& d, uint32_t algorithm) {
    WeightGeom g{};
    g.ocp = round_up(d.out_channels, 16u);
    if (is_winograd_algorithm(algorithm)) {
        g.kp = round_up(d.in_channels, 32u);
        g.elem_bytes = 2;
        g.nbytes = 16ull * g.ocp * g.kp * 2ull;
    } else {
        const uint32_t k = d.kernel_h * d.kernel_w * d.in_channels;
        g.kp = round_up(k, 64u);
        g.elem_bytes = is_int8_algorithm(algorithm) ? 1 : 2;
        g.nbytes = (uint64_t)g.ocp * g.kp * g.elem_bytes;
    }
    return g;
}

// Half-away-from-zero round (std::round), the reference's weight rounding
// (engine.py:2454-2455, native/aexrt_d3d12_runtime.cpp:21736).
static inline float round_half_away(float v) { return std::round(v); }

// Per output channel quantization of an fp32 weight (the runtime fallback of
// native/aexrt_d3d12_runtime.cpp:21716-21741 for engines without layout 8).
static void quantize_weight_host(const float* w, uint32_t oc, uint32_t per_oc, int8_t* q, float* scale) {
    for (uint32_t o = 0; o < oc; ++o) {
        const float* row = w + (uint64_t)o * per_oc;
        float amax = 0.0f;
        for (uint32_t i = 0; i < per_oc; ++i) amax = std::max(amax, std::fabs(row[i]));
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / s;
        scale[o] = s;
        for (uint32_t i = 0; i < per_oc; ++i) {
            float v = round_half_away(row[i] * inv);
            v = std::min(127.0f, std::max(-127.0f, v));
            q[(uint64_t)o * per_oc + i] = (int8_t)v;
        }
    }
}

static inline float half_bits_to_float(uint16_t h) {
    _Float16 v;
    std::memcpy(&v, &h, 2);
    return (float)v;
}
static inline uint16_t float_to_half_bits(float f) {
    _Float16 v = (_Float16)f;
    uint16_t h;
    std::memcpy(&h, &v, 2);
    return h;
}

// Expands any supported source layout to fp32 [oc][ic][kh][kw].
static bool source_to_f32(const AexrtConv2DDesc& d, uint32_t layout, const void* src, uint64_t nbytes,
                          std::vector<float>& out) {
    const uint32_t oc = d.out_channels, ic = d.in_channels, kk = d.kernel_h * d.kernel_w;
    const uint64_t elems = (uint64_t)oc * ic * kk;
    out.assign(elems, 0.0f);
    if (layout == AEXRT_HIP_SRC_RAW_F32) {
        if (nbytes < elems * 4) return false;
        std::memcpy(out.data(), src, elems * 4);
        return true;
    }
    const uint16_t* h = static_cast<const uint16_t*>(src);
    if (layout == AEXRT_HIP_SRC_RAW_F16) {
        if (nbytes < elems * 2) return false;
        for (uint64_t i = 0; i < elems; ++i) out[i] = half_bits_to_float(h[i]);
        return true;
    }
    if (layout == AEXRT_HIP_SRC_LAYOUT_OC4_F16) {  // [oc/4][ic][9][4]
        if (kk != 9 || oc % 4 || nbytes < elems * 2) return false;
        for (uint32_t o = 0; o < oc; ++o)
            for (uint32_t c = 0; c < ic; ++c)
                for (uint32_t k = 0; k < 9; ++k)
                    out[((uint64_t)o * ic + c) * 9 + k] =
                        half_bits_to_float(h[(((uint64_t)(o / 4) * ic + c) * 9 + k) * 4 + (o % 4)]);
        return true;
    }
    if (layout == AEXRT_HIP_SRC_LAYOUT_OC8_F16) {  // [oc/8][ic][8]
        if (kk != 1 || oc % 8 || nbytes < elems * 2) return false;
        for (uint32_t o = 0; o < oc; ++o)
            for (uint32_t c = 0; c < ic; ++c)
                out[(uint64_t)o * ic + c] = half_bits_to_float(h[((uint64_t)(o / 8) * ic + c) * 8 + (o % 8)]);
        return true;
    }
    return false;
}

// Sync words of the op-level pair entry (and its barrier-timeout word after
// them), one allocation per device kept for the process; overlapping int8
// pair calls on one device share them and race.
constexpr uint32_t kPairSyncWordsAbi = 512;
static_assert(kPairSyncWordsAbi == (uint32_t)kPairSyncWordsHost, "sync area size");

static uint32_t* pair_sync_words() {
    static std::mutex mu;
    static std::map<int, uint32_t*> per_dev;
    int dev = 0;
    if (!check_hip(hipGetDevice(&dev), "conv_pair: current device")) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    auto it = per_dev.find(dev);
    if (it != per_dev.end()) return it->second;
    void* p = nullptr;
    if (!check_hip(hipMalloc(&p, (kPairSyncWordsAbi + 64) * 4), "conv_pair: sync allocation") ||
        !check_hip(hipMemset(p, 0, (kPairSyncWordsAbi + 64) * 4), "conv_pair: sync clear"))
        return nullptr;
    per_dev[dev] = static_cast<uint32_t*>(p);
    return static_cast<uint32_t*>(p);
}

}  // namespace aexrt

using namespace aexrt;

extern "C" {

uint32_t aexrt_hip_abi_version(void) { return 2u; }

const char* aexrt_hip_get_last_error(void) { return last_error(); }

int aexrt_hip_can_use_conv_int8(const AexrtConv2DDesc* desc, uint32_t kernel_elems) {
    return desc && can_use_int8(*desc, kernel_elems) ? 1 : 0;
}

int aexrt_hip_set_conv_tile(int32_t jn, int32_t pw, int32_t ksw) {
    if (!set_conv_tile_override(jn, pw, ksw)) {
        set_error("set_conv_tile: no kernel instance for this tile");
        return 0;
    }
    return 1;
}

int aexrt_hip_set_conv3x3_halo(int32_t mode, int32_t jn, int32_t pw, int32_t tr, int32_t tc, int32_t cc) {
    if (mode == 5 || mode == 6 || mode == 7) {
        if (!set_conv3x3_m32(true, pw, jn, tr, tc, cc, mode == 5 ? 4 : 8, mode == 7 ? 2 : 1)) {
            set_error("set_conv3x3_halo: no 32x32-MFMA kernel instance for this tile");
            return 0;
        }
        return 1;
    }
    set_conv3x3_m32(false, 0, 0, 0, 0, 0, 4, 1);
    if (!set_conv3x3_halo(mode, jn, pw, tr, tc, cc)) {
        set_error("set_conv3x3_halo: bad mode or no kernel instance for this tile");
        return 0;
    }
    return 1;
}

int aexrt_hip_set_conv_stem(int32_t mode, int32_t tr) {
    if (!set_conv_stem(mode, tr)) {
        set_error("set_conv_stem: bad mode or band rows");
        return 0;
    }
    return 1;
}

int aexrt_hip_set_conv1x1_stream(int32_t mode, int32_t jq, int32_t pq) {
    if (!set_conv1x1_stream(mode, jq, pq)) {
        set_error("set_conv1x1_stream: no kernel instance for this tile");
        return 0;
    }
    return 1;
}

int aexrt_hip_conv_weight_bytes(const AexrtConv2DDesc* desc, uint32_t algorithm, uint64_t* out_nbytes) {
    if (!desc || !out_nbytes) {
        set_error("conv_weight_bytes: null argument");
        return 0;
    }
    *out_nbytes = weight_geom(*desc, algorithm).nbytes;
    return 1;
}

int aexrt_hip_pack_conv_weight(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t src_layout,
                               const void* src, uint64_t src_nbytes, void* dst, uint64_t dst_nbytes,
                               float* scale_out) {
    if (!desc || !src || !dst) {
        set_error("pack_conv_weight: null argument");
        return 0;
    }
    const AexrtConv2DDesc& d = *desc;
    const WeightGeom g = weight_geom(d, algorithm);
    if (dst_nbytes < g.nbytes) {
        set_error("pack_conv_weight: destination too small");
        return 0;
    }
    std::memset(dst, 0, g.nbytes);
    const uint32_t oc = d.out_channels, ic = d.in_channels, kh = d.kernel_h, kw = d.kernel_w, kk = kh * kw;
    if (is_int8_algorithm(algorithm)) {
        if (!scale_out) {
            set_error("pack_conv_weight: int8 needs scale_out");
            return 0;
        }
        std::vector<int8_t> q((uint64_t)oc * ic * kk);
        if (src_layout == AEXRT_HIP_SRC_LAYOUT_INT8) {
            const uint64_t need = q.size() + 4ull * oc;
            if (src_nbytes < need) {
                set_error("pack_conv_weight: layout 8 payload too small");
                return 0;
            }
            std::memcpy(q.data(), src, q.size());
            std::memcpy(scale_out, static_cast<const uint8_t*>(src) + q.size(), 4ull * oc);
        } else {
            std::vector<float> w;
            if (!source_to_f32(d, src_layout, src, src_nbytes, w)) {
                set_error("pack_conv_weight: unsupported source layout for int8");
                return 0;
            }
            quantize_weight_host(w.data(), oc, ic * kk, q.data(), scale_out);
        }
        int8_t* out = static_cast<int8_t*>(dst);
        for (uint32_t o = 0; o < oc; ++o)
            for (uint32_t c = 0; c < ic; ++c)
                for (uint32_t k = 0; k < kk; ++k)
                    out[(uint64_t)o * g.kp + (uint64_t)k * ic + c] = q[((uint64_t)o * ic + c) * kk + k];
        return 1;
    }
    uint16_t* out = static_cast<uint16_t*>(dst);
    if (is_winograd_algorithm(algorithm)) {
        // U as [16][OCp][Cp] fp16 from layout 3 (fp16) / 5 (fp32) [oc][ic][4][4].
        if (src_layout == AEXRT_HIP_SRC_LAYOUT_WINO_F16 || src_layout == AEXRT_HIP_SRC_LAYOUT_WINO_F32) {
            const uint64_t elems = (uint64_t)oc * ic * 16;
            const bool f16 = src_layout == AEXRT_HIP_SRC_LAYOUT_WINO_F16;
            if (src_nbytes < elems * (f16 ? 2 : 4)) {
                set_error("pack_conv_weight: Winograd payload too small");
                return 0;
            }
            for (uint32_t o = 0; o < oc; ++o)
                for (uint32_t c = 0; c < ic; ++c)
                    for (uint32_t r = 0; r < 16; ++r) {
                        const uint64_t si = ((uint64_t)o * ic + c) * 16 + r;
                        const float v = f16 ? half_bits_to_float(static_cast<const uint16_t*>(src)[si])
                                            : static_cast<const float*>(src)[si];
                        out[((uint64_t)r * g.ocp + o) * g.kp + c] = float_to_half_bits(v);
                    }
            return 1;
        }
        // Raw 3x3 weights: U = G g G^T on the fp16-rounded source.
        std::vector<float> w;
        if (kk != 9 || !source_to_f32(d, src_layout, src, src_nbytes, w)) {
            set_error("pack_conv_weight: unsupported source layout for Winograd");
            return 0;
        }
        static const float G[4][3] = {{1.f, 0.f, 0.f}, {.5f, .5f, .5f}, {.5f, -.5f, .5f}, {0.f, 0.f, 1.f}};
        for (uint32_t o = 0; o < oc; ++o)
            for (uint32_t c = 0; c < ic; ++c) {
                float gg[3][3], t[3][4];
                for (int i = 0; i < 9; ++i)
                    gg[i / 3][i % 3] = half_bits_to_float(float_to_half_bits(w[((uint64_t)o * ic + c) * 9 + i]));
                for (int k = 0; k < 3; ++k)
                    for (int b = 0; b < 4; ++b) t[k][b] = gg[k][0] * G[b][0] + gg[k][1] * G[b][1] + gg[k][2] * G[b][2];
                for (int a = 0; a < 4; ++a)
                    for (int b = 0; b < 4; ++b) {
                        const float u = G[a][0] * t[0][b] + G[a][1] * t[1][b] + G[a][2] * t[2][b];
                        out[((uint64_t)(a * 4 + b) * g.ocp + o) * g.kp + c] = float_to_half_bits(u);
                    }
            }
        return 1;
    }
    std::vector<float> w;
    if (!source_to_f32(d, src_layout, src, src_nbytes, w)) {
        set_error("pack_conv_weight: unsupported source layout for fp16 conv");
        return 0;
    }
    for (uint32_t o = 0; o < oc; ++o)
        for (uint32_t c = 0; c < ic; ++c)
            for (uint32_t k = 0; k < kk; ++k)
                out[(uint64_t)o * g.kp + (uint64_t)k * ic + c] = float_to_half_bits(w[((uint64_t)o * ic + c) * kk + k]);
    return 1;
}

int aexrt_hip_conv2d(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags, const AexrtHipTensorView* x,
                     const void* weight, const float* w_scale, const float* bias, const AexrtHipTensorView* residual,
                     const AexrtHipTensorView* y, int32_t* acc_out, void* stream) {
    if (!desc || !x || !y || !weight || !bias || !x->data || !y->data) {
        set_error("conv2d: null argument");
        return 0;
    }
    std::string why;
    ConvParams p{};
    if (!build_conv_params(*desc, algorithm, flags, *x, weight, w_scale, bias, residual, *y, acc_out, p, why)) {
        set_error("conv2d: " + why);
        return 0;
    }
    return launch_conv(p, algorithm, static_cast<hipStream_t>(stream)) ? 1 : 0;
}

int aexrt_hip_conv2d_upsample_copy(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                                   const AexrtHipTensorView* x, const void* weight, const float* w_scale,
                                   const float* bias, const AexrtHipTensorView* y, const AexrtHipTensorView* y_up,
                                   void* stream) {
    if (!desc || !x || !y || !y_up || !weight || !bias || !x->data || !y->data || !y_up->data) {
        set_error("conv2d_upsample_copy: null argument");
        return 0;
    }
    if (!is_int8_algorithm(algorithm) || (flags & (AEXRT_HIP_CONV_INT8_PG16 | AEXRT_HIP_CONV_INT8_DYNAMIC))) {
        set_error("conv2d_upsample_copy: a per-tensor int8 1x1 conv (algorithm 51/52/53)");
        return 0;
    }
    if (!slot_ref_ok(*y_up) || y_up->c_stride <= 0 || y_up->n_stride <= 0 ||
        reinterpret_cast<uintptr_t>(y_up->data) % 8) {
        set_error("conv2d_upsample_copy: bad upsample view");
        return 0;
    }
    std::string why;
    ConvParams p{};
    if (!build_conv_params(*desc, algorithm, flags, *x, weight, w_scale, bias, nullptr, *y, nullptr, p, why)) {
        set_error("conv2d_upsample_copy: " + why);
        return 0;
    }
    p.yup = y_up->data;
    p.yup_nstride = y_up->n_stride;
    p.yup_cstride = (int32_t)y_up->c_stride;
    p.yup_slots = slot_ref(y_up);
    // the streaming 1x1 kernel: a forced tile, else the first that fits
    ConvChoice forced;
    if (!forced_s1x1_choice(forced)) {
        std::vector<ConvChoice> all(kMaxConvChoices);
        if (enumerate_conv_choices(p, true, all.data(), kMaxConvChoices) == 0) {
            set_error("conv2d_upsample_copy: no streaming 1x1 tile fits this conv and view");
            return 0;
        }
        p.choice = all[0];
    }
    return launch_conv(p, algorithm, static_cast<hipStream_t>(stream)) ? 1 : 0;
}

int aexrt_hip_conv2d_upsampled_input(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                                     const AexrtHipTensorView* x, const AexrtHipTensorView* x_up, uint32_t up_c0,
                                     uint32_t up_channels, const void* weight, const float* w_scale,
                                     const float* bias, const AexrtHipTensorView* y, int32_t* acc_out, void* stream) {
    if (!desc || !x || !x_up || !y || !weight || !bias || !x->data || !x_up->data || !y->data) {
        set_error("conv2d_upsampled_input: null argument");
        return 0;
    }
    if (!is_int8_algorithm(algorithm) || (flags & (AEXRT_HIP_CONV_INT8_PG16 | AEXRT_HIP_CONV_INT8_DYNAMIC))) {
        set_error("conv2d_upsampled_input: a per-tensor int8 1x1 conv (algorithm 51/52/53)");
        return 0;
    }
    if (!slot_ref_ok(*x_up) || !x_up->amax_slots || x_up->c_stride <= 0 || x_up->n_stride <= 0 ||
        reinterpret_cast<uintptr_t>(x_up->data) % 16 || up_channels == 0 || up_channels % 16 || up_c0 % 16) {
        set_error("conv2d_upsampled_input: bad source view (16-byte aligned, amax slots, 16-channel groups)");
        return 0;
    }
    std::string why;
    ConvParams p{};
    if (!build_conv_params(*desc, algorithm, flags, *x, weight, w_scale, bias, nullptr, *y, acc_out, p, why)) {
        set_error("conv2d_upsampled_input: " + why);
        return 0;
    }
    {
        // the kernel reads both views through one 32-bit buffer resource
        const uintptr_t xa = reinterpret_cast<uintptr_t>(x->data), ua = reinterpret_cast<uintptr_t>(x_up->data);
        const uintptr_t xe = xa + (uintptr_t)(desc->batch * x->n_stride) * 2;
        const uintptr_t ue = ua + (uintptr_t)(desc->batch * x_up->n_stride) * 2;
        if (std::max(xe, ue) - std::min(xa, ua) > 0xFFFFFFF0ull) {
            set_error("conv2d_upsampled_input: x and x_up must lie within one 4 GB span (e.g. one arena)");
            return 0;
        }
    }
    p.xup = x_up->data;
    p.xup_nstride = x_up->n_stride;
    p.xup_cstride = (int32_t)x_up->c_stride;
    p.xup_c0 = (int32_t)up_c0;
    p.xup_cn = (int32_t)up_channels;
    p.xup_slots = slot_ref(x_up);
    p.xup_nslots = (int32_t)(up_channels / 16);
    ConvChoice forced;
    if (!forced_s1x1_choice(forced)) {
        std::vector<ConvChoice> all(kMaxConvChoices);
        if (enumerate_conv_choices(p, true, all.data(), kMaxConvChoices) == 0) {
            set_error("conv2d_upsampled_input: no streaming 1x1 tile fits this conv and its source");
            return 0;
        }
        p.choice = all[0];
    }
    return launch_conv(p, algorithm, static_cast<hipStream_t>(stream)) ? 1 : 0;
}

uint32_t aexrt_hip_conv_candidates(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                                   const AexrtHipTensorView* x, const AexrtHipTensorView* residual,
                                   const AexrtHipTensorView* y, char* names, uint32_t name_len, uint32_t cap) {
    if (!desc || !x || !y || !x->data || !y->data || (cap && (!names || name_len < 2))) {
        set_error("conv_candidates: null argument");
        return 0;
    }
    if (is_winograd_algorithm(algorithm) ||
        (flags & (AEXRT_HIP_CONV_INT8_PG16 | AEXRT_HIP_CONV_INT8_DYNAMIC))) {
        set_error("conv_candidates: Winograd, pg16 and dynamic int8 convs have one kernel each, no tile choice");
        return 0;
    }
    // the launchers check the pointers only for presence and alignment: any
    // aligned non-null placeholder stands in for the weights
    static const float placeholder[4] __attribute__((aligned(16))) = {0, 0, 0, 0};
    const bool int8 = is_int8_algorithm(algorithm);
    std::string why;
    ConvParams p{};
    if (!build_conv_params(*desc, algorithm, flags, *x, placeholder, int8 ? placeholder : nullptr, placeholder,
                           residual, *y, nullptr, p, why)) {
        set_error("conv_candidates: " + why);
        return 0;
    }
    std::vector<ConvChoice> all(kMaxConvChoices);
    const int n = enumerate_conv_choices(p, int8, all.data(), kMaxConvChoices);
    const uint32_t out_n = std::min<uint32_t>((uint32_t)n, cap);
    for (uint32_t i = 0; i < out_n; ++i) {
        LaunchProbe probe{};
        ConvParams q = p;
        q.choice = all[i];
        set_launch_probe(&probe);
        const hipError_t e = launch_conv_igemm(q, int8, nullptr);
        set_launch_probe(nullptr);
        char* dst = names + (size_t)i * name_len;
        if (e != hipSuccess) probe.name[0] = '\0';
        std::snprintf(dst, name_len, "%s", probe.name);
    }
    return (uint32_t)n;
}

int aexrt_hip_conv_pair(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags, const AexrtHipTensorView* x,
                        const void* weight_a, const float* w_scale_a, const float* bias_a, const void* weight_b,
                        const float* w_scale_b, const float* bias_b, const AexrtHipTensorView* y, uint32_t band_rows,
                        void* t_out, int32_t* acc_a, int32_t* acc_b, void* stream) {
    if (!desc || !x || !y || !x->data || !y->data || !weight_a || !weight_b || !bias_a || !bias_b) {
        set_error("conv_pair: null argument");
        return 0;
    }
    if (flags & ~(uint32_t)AEXRT_HIP_CONV_RESIDUAL) {
        set_error("conv_pair: the only flag is AEXRT_HIP_CONV_RESIDUAL (both convs apply SiLU, fp16 output)");
        return 0;
    }
    const bool int8 = is_int8_algorithm(algorithm);
    if ((int8 && algorithm != 52u) || is_winograd_algorithm(algorithm) || (!int8 && (acc_a || acc_b))) {
        set_error("conv_pair: algorithm 52 (int8) or an fp16 MFMA id; accumulators with int8 only");
        return 0;
    }
    if (band_rows > 4096) {
        set_error("conv_pair: band_rows 0 (chosen) or at most 4096");
        return 0;
    }
    std::string why;
    ConvParams pa{}, pb{};
    AexrtHipTensorView t{};  // the intermediate's view (its pointer is never used)
    t.data = y->data;
    t.n_stride = int64_t(desc->out_h) * desc->out_w * desc->out_channels;
    t.c_stride = (int32_t)desc->out_channels;
    t.amax_slots = x->amax_slots;  // read by the kernel only through the barrier's amax words
    if (!build_conv_params(*desc, algorithm, AEXRT_HIP_CONV_SILU, *x, weight_a, w_scale_a, bias_a, nullptr, t, nullptr,
                           pa, why) ||
        !build_conv_params(*desc, algorithm, AEXRT_HIP_CONV_SILU | (flags & AEXRT_HIP_CONV_RESIDUAL), t, weight_b,
                           w_scale_b, bias_b, (flags & AEXRT_HIP_CONV_RESIDUAL) ? x : nullptr, *y, acc_b, pb, why)) {
        set_error("conv_pair: " + why);
        return 0;
    }
    if (const char* e = pair_shape_error(pa, pb, int8)) {
        set_error(e);
        return 0;
    }
    uint32_t* sync = nullptr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int8) {
        sync = pair_sync_words();
        if (!sync || !check_hip(launch_fill_u32(sync, kPairSyncWordsAbi, 0u, s), "conv_pair: clear sync words"))
            return 0;
    }
    const hipError_t e = launch_conv_pair(pa, pb, int8, (int)band_rows, sync, sync ? sync + kPairSyncWordsAbi : nullptr,
                                          static_cast<__half*>(t_out), acc_a, s);
    if (e == hipErrorInvalidConfiguration) {
        set_error("conv_pair: the grid of this batch and band height does not fit the GPU at once");
        return 0;
    }
    if (e == hipErrorInvalidValue) {
        set_error("conv_pair: no band of this height fits the kernel (LDS, positions per block, views)");
        return 0;
    }
    return check_hip(e, "conv_pair") ? 1 : 0;
}

uint32_t aexrt_hip_conv_pair_barrier_timeouts(void) {
    uint32_t* sync = pair_sync_words();
    if (!sync) return 0xFFFFFFFFu;
    uint32_t err = 0;
    if (!check_hip(hipDeviceSynchronize(), "conv_pair: sync") ||
        !check_hip(hipMemcpy(&err, sync + kPairSyncWordsAbi, 4, hipMemcpyDeviceToHost), "conv_pair: read error word"))
        return 0xFFFFFFFFu;
    return err;
}

int aexrt_hip_conv2d_fused_1x1(const AexrtConv2DDesc* desc, uint32_t flags, const AexrtHipTensorView* x,
                               const void* weight, const float* bias, const AexrtConv2DDesc* desc2, uint32_t flags2,
                               const void* weight2, const float* bias2, const AexrtHipTensorView* y2, void* stream) {
    if (!desc || !desc2 || !x || !y2 || !weight || !bias || !weight2 || !bias2 || !x->data || !y2->data) {
        set_error("conv2d_fused_1x1: null argument");
        return 0;
    }
    const AexrtConv2DDesc& d = *desc;
    const AexrtConv2DDesc& d2 = *desc2;
    if (flags != AEXRT_HIP_CONV_SILU || (flags2 & ~(AEXRT_HIP_CONV_SILU | AEXRT_HIP_CONV_OUT_F32)) ||
        d2.kernel_h != 1 || d2.kernel_w != 1 ||
        d2.stride_h != 1 || d2.pad_top != 0 || d2.batch != d.batch || d2.in_channels != d.out_channels ||
        d2.in_h != d.out_h || d2.in_w != d.out_w) {
        set_error("conv2d_fused_1x1: an fp16 SiLU conv followed by a 1x1 s1 conv of its output (flags2: SILU, "
                  "OUT_F32)");
        return 0;
    }
    // the intermediate is never stored: a dense view of its shape over y2's
    // memory stands in for it in the parameter checks
    AexrtHipTensorView mid{};
    mid.data = y2->data;
    mid.c_stride = (int32_t)d.out_channels;
    mid.n_stride = int64_t(d.out_h) * d.out_w * d.out_channels;
    std::string why;
    ConvParams p{}, p2{};
    if (!build_conv_params(d, 5u, flags, *x, weight, nullptr, bias, nullptr, mid, nullptr, p, why) ||
        !build_conv_params(d2, 5u, flags2, mid, weight2, nullptr, bias2, nullptr, *y2, nullptr, p2, why)) {
        set_error("conv2d_fused_1x1: " + why);
        return 0;
    }
    p.fuse_1x1 = &p2;
    ConvChoice c{};
    if (!forced_m32_choice(c)) {
        ConvChoice all[64];
        if (enumerate_m32_choices(p, false, all, 64) < 1) {
            set_error("conv2d_fused_1x1: no 32x32-MFMA tile covers every output channel of this conv");
            return 0;
        }
        c = all[0];
    }
    p.choice = c;
    return check_hip(launch_conv_igemm(p, false, static_cast<hipStream_t>(stream)), "conv2d_fused_1x1") ? 1 : 0;
}

int aexrt_hip_conv_chain3(const AexrtConv2DDesc* desc_a, const void* weight_a, const float* bias_a,
                          const AexrtConv2DDesc* desc_b, const void* weight_b, const float* bias_b,
                          const AexrtConv2DDesc* desc_c, uint32_t flags_c, const void* weight_c, const float* bias_c,
                          const AexrtHipTensorView* x, const AexrtHipTensorView* y, uint32_t tile_rows,
                          uint32_t tile_cols, void* stream) {
    if (!desc_a || !desc_b || !desc_c || !weight_a || !weight_b || !weight_c || !bias_a || !bias_b || !bias_c || !x ||
        !y || !x->data || !y->data) {
        set_error("conv_chain3: null argument");
        return 0;
    }
    if (tile_rows > 4096 || tile_cols > 4096 || (tile_rows == 0) != (tile_cols == 0)) {
        set_error("conv_chain3: tile rows and columns both 0 (chosen) or both in 1..4096");
        return 0;
    }
    // the intermediates are never stored: dense views of their shapes over
    // y's memory stand in for them in the parameter checks
    const AexrtConv2DDesc& a = *desc_a;
    const AexrtConv2DDesc& b = *desc_b;
    AexrtHipTensorView t1{}, t2{};
    t1.data = t2.data = y->data;
    t1.c_stride = (int32_t)a.out_channels;
    t1.n_stride = int64_t(a.out_h) * a.out_w * a.out_channels;
    t2.c_stride = (int32_t)b.out_channels;
    t2.n_stride = int64_t(b.out_h) * b.out_w * b.out_channels;
    std::string why;
    ConvParams pa{}, pb{}, pc{};
    if (!build_conv_params(a, 5u, AEXRT_HIP_CONV_SILU, *x, weight_a, nullptr, bias_a, nullptr, t1, nullptr, pa, why) ||
        !build_conv_params(b, 5u, AEXRT_HIP_CONV_SILU, t1, weight_b, nullptr, bias_b, nullptr, t2, nullptr, pb, why) ||
        !build_conv_params(*desc_c, 5u, flags_c, t2, weight_c, nullptr, bias_c, nullptr, *y, nullptr, pc, why)) {
        set_error("conv_chain3: " + why);
        return 0;
    }
    if (const char* e = chain_shape_error(pa, pb, pc)) {
        set_error(std::string("conv_chain3: ") + e);
        return 0;
    }
    int tr = (int)tile_rows, tc = (int)tile_cols;
    if (!chain_tile(pa, pb, pc, tr, tc)) {
        set_error("conv_chain3: the tile does not fit the kernel (at most 256 positions per region, LDS)");
        return 0;
    }
    return check_hip(launch_conv_chain(pa, pb, pc, tr, tc, static_cast<hipStream_t>(stream)), "conv_chain3") ? 1 : 0;
}

int aexrt_hip_conv2d_f32(const AexrtConv2DDesc* desc, uint32_t flags, const float* x, const float* weight,
                         const float* bias, float* y, void* stream) {
    if (!desc || !x || !weight || !bias || !y) {
        set_error("conv2d_f32: null argument");
        return 0;
    }
    const AexrtConv2DDesc& d = *desc;
    if (d.batch == 0 || d.in_channels == 0 || d.out_channels == 0 || d.in_h == 0 || d.in_w == 0 || d.out_h == 0 ||
        d.out_w == 0 || d.kernel_h == 0 || d.kernel_w == 0 || d.groups == 0 || d.stride_h == 0 || d.stride_w == 0 ||
        d.dilation_h == 0 || d.dilation_w == 0 || d.in_channels % d.groups || d.out_channels % d.groups ||
        (flags & ~AEXRT_HIP_CONV_SILU)) {
        set_error("conv2d_f32: invalid descriptor or flags (SILU only)");
        return 0;
    }
    const uint32_t dims[] = {d.batch, d.in_channels, d.in_h, d.in_w, d.out_channels, d.out_h, d.out_w,
                             d.kernel_h, d.kernel_w, d.stride_h, d.stride_w, d.pad_top, d.pad_left,
                             d.dilation_h, d.dilation_w, d.groups};
    for (uint32_t v : dims)
        if (v > 0x7FFFFFFu) {
            set_error("conv2d_f32: descriptor value out of range");
            return 0;
        }
    F32ConvParams p{};
    p.x = x, p.w = weight, p.bias = bias, p.y = y;
    p.N = (int)d.batch, p.C = (int)d.in_channels, p.H = (int)d.in_h, p.W = (int)d.in_w;
    p.OC = (int)d.out_channels, p.OH = (int)d.out_h, p.OW = (int)d.out_w, p.KH = (int)d.kernel_h;
    p.KW = (int)d.kernel_w, p.SH = (int)d.stride_h, p.SW = (int)d.stride_w, p.PT = (int)d.pad_top;
    p.PL = (int)d.pad_left, p.DH = (int)d.dilation_h, p.DW = (int)d.dilation_w, p.G = (int)d.groups;
    p.silu = (flags & AEXRT_HIP_CONV_SILU) ? 1 : 0;
    return check_hip(launch_conv_f32(p, static_cast<hipStream_t>(stream)), "conv2d_f32") ? 1 : 0;
}

int aexrt_hip_conv2d_int8_pg16(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                               const uint32_t* packed, const uint32_t* amax, const void* weight, const float* w_scale,
                               const float* bias, void* y, void* stream) {
    if (!desc || !packed || !amax || !weight || !w_scale || !bias || !y) {
        set_error("conv2d_int8_pg16: null argument");
        return 0;
    }
    const AexrtConv2DDesc& d = *desc;
    if (!is_int8_algorithm(algorithm) || !generic_shape_ok(d) || !can_use_int8(d, int8_kernel_elems(algorithm)) ||
        (algorithm == 52u && d.stride_h != 1) || (algorithm == 53u && d.stride_h != 2)) {
        set_error("conv2d_int8_pg16: descriptor is not eligible for the int8 kernel id");
        return 0;
    }
    if (d.batch == 0 || d.in_channels % 16 || d.in_channels > 4096 || d.out_h == 0 || d.out_w == 0 ||
        (flags & ~(AEXRT_HIP_CONV_SILU | AEXRT_HIP_CONV_OUT_F32))) {
        set_error("conv2d_int8_pg16: needs in_channels % 16 == 0 (<= 4096) and flags SILU / OUT_F32 only");
        return 0;
    }
    const int64_t m = (int64_t)d.batch * d.out_h * d.out_w;
    if (m > INT32_MAX / 2) {
        set_error("conv2d_int8_pg16: too many output positions");
        return 0;
    }
    const WeightGeom g = weight_geom(d, algorithm);
    ConvParams p{};
    p.x = packed;
    p.loader = kLoaderPackedNc4;
    p.x_slots = SlotRef{const_cast<uint32_t*>(amax) + 1, 1u, 0u};
    p.x_nslots = (int)(d.in_channels / 16);
    p.w = weight;
    p.Kp = (int)g.kp;
    p.OCp = (int)g.ocp;
    p.w_scale = w_scale;
    p.bias = bias;
    p.y = y;
    p.N = (int)d.batch;
    p.H = (int)d.in_h;
    p.W = (int)d.in_w;
    p.C = (int)d.in_channels;
    p.OH = (int)d.out_h;
    p.OW = (int)d.out_w;
    p.OC = (int)d.out_channels;
    p.KH = (int)d.kernel_h;
    p.KW = (int)d.kernel_w;
    p.S = (int)d.stride_h;
    p.P = (int)d.pad_top;
    p.K = p.KH * p.KW * p.C;
    p.M = (int)m;
    p.flags = (int)(flags & (AEXRT_HIP_CONV_SILU | AEXRT_HIP_CONV_OUT_F32)) | kConvPg16 | kConvOutNchw;
    return check_hip(launch_conv_int8_pg16(p, static_cast<hipStream_t>(stream)), "conv2d_int8_pg16") ? 1 : 0;
}

int aexrt_hip_yolo_decode_nms_topk(const float* output, uint32_t layout, uint32_t anchors, uint32_t channels,
                                   uint32_t classes, uint32_t has_objectness, float conf_threshold,
                                   float iou_threshold, uint32_t max_candidates, uint32_t max_detections,
                                   float* detections, uint32_t* count, void* stream) {
    const uint32_t cls_off = has_objectness ? 5u : 4u;
    if ((!output && anchors) || !detections || !count || anchors > 0x7FFFFFFFu || channels > 0xFFFFFFu ||
        channels < classes + cls_off || max_candidates < 1 || max_candidates > (uint32_t)kYoloMaxCandidates ||
        max_detections < 1 || max_detections > 0x7FFFFFFFu || uint64_t(anchors) * channels > 0x7FFFFFFFull) {
        set_error("yolo_decode_nms_topk: bad arguments (need channels >= classes + 4 (+1 objectness), "
                  "1 <= max_candidates <= 2048, max_detections >= 1)");
        return 0;
    }
    // layout 2: channels last ([A][C]); otherwise channels first ([C][A])
    const bool last = layout == 2u;
    return check_hip(launch_yolo_decode_nms_topk(output, last ? 1 : (int)anchors, last ? (int)channels : 1,
                                                 (int)anchors, (int)classes, (int)has_objectness, conf_threshold,
                                                 iou_threshold, (int)max_candidates, (int)max_detections, detections,
                                                 count, static_cast<hipStream_t>(stream)),
                     "yolo_decode_nms_topk")
               ? 1
               : 0;
}

int aexrt_hip_yolo_dfl_decode_nms_topk(const float* head, uint32_t layout, uint32_t num_levels,
                                       const uint32_t* level_hw, const float* level_strides, uint32_t classes,
                                       float conf_threshold, float iou_threshold, uint32_t max_candidates,
                                       uint32_t max_detections, float* detections, uint32_t* count, void* stream) {
    if (!level_hw || !level_strides || num_levels < 1 || num_levels > (uint32_t)kYoloMaxLevels || classes < 1 ||
        classes > 0xFFFFu || !detections || !count || max_candidates < 1 ||
        max_candidates > (uint32_t)kYoloMaxCandidates || max_detections < 1 || max_detections > 0x7FFFFFFFu) {
        set_error("yolo_dfl_decode_nms_topk: bad arguments (1..4 levels, classes >= 1, "
                  "1 <= max_candidates <= 2048, max_detections >= 1)");
        return 0;
    }
    YoloLevels lv{};
    lv.n = (int)num_levels;
    uint64_t anchors = 0;
    for (uint32_t l = 0; l < num_levels; ++l) {
        if (level_hw[2 * l] == 0 || level_hw[2 * l + 1] == 0 || level_hw[2 * l] > 0xFFFFu ||
            level_hw[2 * l + 1] > 0xFFFFu) {
            set_error("yolo_dfl_decode_nms_topk: empty or oversized level grid");
            return 0;
        }
        lv.h[l] = (int)level_hw[2 * l];
        lv.w[l] = (int)level_hw[2 * l + 1];
        lv.stride[l] = level_strides[l];
        anchors += uint64_t(lv.h[l]) * lv.w[l];
    }
    const uint64_t channels = 64u + classes;
    if (!head || anchors * channels > 0x7FFFFFFFull) {
        set_error("yolo_dfl_decode_nms_topk: null head or head too large");
        return 0;
    }
    const bool last = layout == 2u;
    return check_hip(launch_yolo_decode_nms_topk(head, last ? 1 : (int)anchors, last ? (int)channels : 1, (int)anchors,
                                                 (int)classes, 0, conf_threshold, iou_threshold, (int)max_candidates,
                                                 (int)max_detections, detections, count,
                                                 static_cast<hipStream_t>(stream), &lv),
                     "yolo_dfl_decode_nms_topk")
               ? 1
               : 0;
}

int aexrt_hip_amax_strips_nhwc(const AexrtHipTensorView* x, uint32_t batch, uint32_t height, uint32_t width,
                               uint32_t channels, uint32_t* out, void* stream) {
    if (!x || !x->data || !out || channels % 16 || x->c_stride % 8 || x->n_stride % 8 || batch == 0) {
        set_error("amax_strips_nhwc: bad view (need C % 16 == 0, 8-element strides, an output)");
        return 0;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!check_hip(launch_fill_u32(out, channels / 16, 0u, s), "amax_strips_nhwc zero")) return 0;
    return check_hip(launch_amax_strips_nhwc(static_cast<const __half*>(x->data), x->n_stride, x->c_stride,
                                             (int)batch, (int)(height * width), (int)channels, out, s),
                     "amax_strips_nhwc")
               ? 1
               : 0;
}

int aexrt_hip_quant_fused_pg16(const void* x, uint32_t is_f16, uint32_t batch, uint32_t channels, uint32_t plane,
                               uint32_t* packed, uint32_t* amax, void* stream) {
    if (!x || !packed || !amax || channels % 16 || channels == 0 || batch == 0 || plane == 0) {
        set_error("quant_fused_pg16: null argument or channels % 16 != 0");
        return 0;
    }
    return check_hip(launch_quant_fused_pg16(x, is_f16 != 0, (int)batch, (int)channels, (int)plane, packed, amax,
                                             static_cast<hipStream_t>(stream)),
                     "quant_fused_pg16")
               ? 1
               : 0;
}

int aexrt_hip_amax_slots(const AexrtHipTensorView* x, uint32_t batch, uint32_t height, uint32_t width,
                         uint32_t channels, void* stream) {
    if (!x || !x->data || !x->amax_slots || channels % 16 || x->c_stride % 8 || x->n_stride % 8 ||
        !slot_ref_ok(*x)) {
        set_error("amax_slots: bad view (need slots, C % 16 == 0, 8-element strides)");
        return 0;
    }
    return check_hip(launch_amax_slots_nhwc(static_cast<const __half*>(x->data), x->n_stride, x->c_stride,
                                            (int)batch, (int)(height * width), (int)channels, slot_ref(x),
                                            static_cast<hipStream_t>(stream)),
                     "amax_slots")
               ? 1
               : 0;
}

int aexrt_hip_amax_nchw(const void* x, uint32_t is_f16, uint32_t batch, uint32_t channels, uint32_t plane,
                        uint32_t* out, void* stream) {
    if (!x || !out) {
        set_error("amax_nchw: null argument");
        return 0;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!check_hip(launch_fill_u32(out, channels / 16 + 1, 0u, s), "amax_nchw zero")) return 0;
    return check_hip(launch_amax_strips_nchw(x, is_f16 != 0, (int)batch, (int)channels, (int)plane, out, s),
                     "amax_nchw")
               ? 1
               : 0;
}

int aexrt_hip_quantize(const AexrtHipTensorView* x, uint32_t batch, uint32_t height, uint32_t width,
                       uint32_t channels, int8_t* q, void* stream) {
    if (!x || !x->data || !x->amax_slots || !q || channels % 16 || x->c_stride % 8 || x->n_stride % 8 ||
        !slot_ref_ok(*x)) {
        set_error("quantize: bad view (need slots, C % 16 == 0, 8-element strides)");
        return 0;
    }
    return check_hip(launch_quantize_nhwc(static_cast<const __half*>(x->data), x->n_stride, x->c_stride,
                                          (int)batch, (int)(height * width), (int)channels, slot_ref(x),
                                          (int)(channels / 16), q, static_cast<hipStream_t>(stream)),
                     "quantize")
               ? 1
               : 0;
}

int aexrt_hip_quant_pack_nchw(const void* x, uint32_t is_f16, uint32_t batch, uint32_t channels, uint32_t plane,
                              const uint32_t* amax, uint32_t per_group, uint32_t* packed, void* stream) {
    if (!x || !amax || !packed || channels % 4) {
        set_error("quant_pack_nchw: bad arguments");
        return 0;
    }
    return check_hip(launch_quant_pack_nchw(x, is_f16 != 0, (int)batch, (int)channels, (int)plane, amax,
                                            per_group != 0, packed, static_cast<hipStream_t>(stream)),
                     "quant_pack_nchw")
               ? 1
               : 0;
}

int aexrt_hip_fill_u32(uint32_t* dst, uint64_t count, uint32_t value, void* stream) {
    if (!dst && count) {
        set_error("fill_u32: null destination");
        return 0;
    }
    return check_hip(launch_fill_u32(dst, (int64_t)count, value, static_cast<hipStream_t>(stream)), "fill_u32")
               ? 1
               : 0;
}

int aexrt_hip_nchw_f32_to_nhwc(const float* x, uint32_t batch, uint32_t channels, uint32_t plane,
                               const AexrtHipTensorView* y, void* stream) {
    if (!x || !y || !y->data || !slot_ref_ok(*y)) {
        set_error("nchw_f32_to_nhwc: null argument or bad slot stripes");
        return 0;
    }
    return check_hip(launch_nchw_f32_to_nhwc_f16(x, static_cast<__half*>(y->data), y->n_stride, y->c_stride,
                                                 (int)batch, (int)channels, (int)plane, slot_ref(y),
                                                 static_cast<hipStream_t>(stream)),
                     "nchw_f32_to_nhwc")
               ? 1
               : 0;
}

int aexrt_hip_nhwc_to_nchw_f32(const AexrtHipTensorView* x, uint32_t is_f16, uint32_t batch, uint32_t channels,
                               uint32_t plane, float* y, void* stream) {
    if (!x || !x->data || !y) {
        set_error("nhwc_to_nchw_f32: null argument");
        return 0;
    }
    return check_hip(launch_nhwc_to_nchw_f32(x->data, is_f16 != 0, x->n_stride, x->c_stride, y, (int)batch,
                                             (int)channels, (int)plane, static_cast<hipStream_t>(stream)),
                     "nhwc_to_nchw_f32")
               ? 1
               : 0;
}

static bool vec_view_ok(const AexrtHipTensorView* v) {
    return v && v->data && (reinterpret_cast<uintptr_t>(v->data) % 16) == 0 && v->c_stride % 8 == 0 &&
           v->n_stride % 8 == 0 && slot_ref_ok(*v);
}

int aexrt_hip_copy(const AexrtHipTensorView* src, const AexrtHipTensorView* dst, uint32_t batch, uint32_t plane,
                   uint32_t channels, void* stream) {
    if (!vec_view_ok(src) || !vec_view_ok(dst) || channels % 8) {
        set_error("copy: views need 16-byte alignment and C % 8 == 0");
        return 0;
    }
    return check_hip(launch_copy_nhwc(static_cast<const __half*>(src->data), src->n_stride, src->c_stride,
                                      static_cast<__half*>(dst->data), dst->n_stride, dst->c_stride, (int)batch,
                                      (int)plane, (int)channels, slot_ref(dst), static_cast<hipStream_t>(stream)),
                     "copy")
               ? 1
               : 0;
}

int aexrt_hip_maxpool(const AexrtHipTensorView* x, const AexrtHipTensorView* y, uint32_t batch, uint32_t channels,
                      uint32_t in_h, uint32_t in_w, uint32_t out_h, uint32_t out_w, uint32_t kernel, uint32_t stride,
                      uint32_t pad, void* stream) {
    if (!vec_view_ok(x) || !vec_view_ok(y) || channels % 8 || stride == 0) {
        set_error("maxpool: views need 16-byte alignment and C % 8 == 0");
        return 0;
    }
    return check_hip(launch_maxpool_nhwc(static_cast<const __half*>(x->data), x->n_stride, x->c_stride,
                                         static_cast<__half*>(y->data), y->n_stride, y->c_stride, (int)batch,
                                         (int)in_h, (int)in_w, (int)channels, (int)out_h, (int)out_w, (int)kernel,
                                         (int)stride, (int)pad, slot_ref(y), static_cast<hipStream_t>(stream)),
                     "maxpool")
               ? 1
               : 0;
}

int aexrt_hip_sppf_maxpool(const AexrtHipTensorView* x, const AexrtHipTensorView* y1, const AexrtHipTensorView* y2,
                           const AexrtHipTensorView* y3, uint32_t batch, uint32_t channels, uint32_t h, uint32_t w,
                           void* stream) {
    if (!vec_view_ok(x) || !vec_view_ok(y1) || !vec_view_ok(y2) || !vec_view_ok(y3) || channels % 8 ||
        y1->n_stride != y2->n_stride || y1->n_stride != y3->n_stride || y1->c_stride != y2->c_stride ||
        y1->c_stride != y3->c_stride || !sppf_fits((int)h, (int)w)) {
        set_error("sppf_maxpool: 16-byte aligned views, C % 8 == 0, outputs with one geometry, plane fits LDS");
        return 0;
    }
    return check_hip(launch_sppf_maxpool_nhwc(static_cast<const __half*>(x->data), x->n_stride, x->c_stride,
                                              static_cast<__half*>(y1->data), static_cast<__half*>(y2->data),
                                              static_cast<__half*>(y3->data), y1->n_stride, y1->c_stride,
                                              (int)batch, (int)h, (int)w, (int)channels, slot_ref(y1), slot_ref(y2),
                                              slot_ref(y3), static_cast<hipStream_t>(stream)),
                     "sppf_maxpool")
               ? 1
               : 0;
}

int aexrt_hip_resize_nearest(const AexrtHipTensorView* x, const AexrtHipTensorView* y, uint32_t batch,
                             uint32_t channels, uint32_t in_h, uint32_t in_w, uint32_t out_h, uint32_t out_w,
                             void* stream) {
    if (!vec_view_ok(x) || !vec_view_ok(y) || channels % 8) {
        set_error("resize: views need 16-byte alignment and C % 8 == 0");
        return 0;
    }
    return check_hip(launch_resize_nearest_nhwc(static_cast<const __half*>(x->data), x->n_stride, x->c_stride,
                                                static_cast<__half*>(y->data), y->n_stride, y->c_stride,
                                                (int)batch, (int)in_h, (int)in_w, (int)channels, (int)out_h,
                                                (int)out_w, slot_ref(y), static_cast<hipStream_t>(stream)),
                     "resize")
               ? 1
               : 0;
}

int aexrt_hip_add(const AexrtHipTensorView* a, const AexrtHipTensorView* b, const AexrtHipTensorView* y,
                  uint32_t batch, uint32_t plane, uint32_t channels, void* stream) {
    if (!vec_view_ok(a) || !vec_view_ok(b) || !vec_view_ok(y) || channels % 8) {
        set_error("add: views need 16-byte alignment and C % 8 == 0");
        return 0;
    }
    return check_hip(launch_add_nhwc(static_cast<const __half*>(a->data), a->n_stride, a->c_stride,
                                     static_cast<const __half*>(b->data), b->n_stride, b->c_stride,
                                     static_cast<__half*>(y->data), y->n_stride, y->c_stride, (int)batch,
                                     (int)plane, (int)channels, slot_ref(y), static_cast<hipStream_t>(stream)),
                     "add")
               ? 1
               : 0;
}

}  // extern "C"
