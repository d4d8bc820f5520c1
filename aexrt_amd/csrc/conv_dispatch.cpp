// Conv dispatch: maps a reference algorithm id and descriptor onto one of the
// three gfx950 kernels (int8 MFMA, fp16 MFMA, fp16 Winograd) and checks
// every assumption the kernel makes about shapes, views and alignment before
// anything is launched.
#include <cstdint>
#include <string>

#include "internal.h"

namespace aexrt {

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) % 16) == 0; }

bool build_conv_params(const AexrtConv2DDesc& d, uint32_t algorithm, uint32_t flags, const AexrtHipTensorView& x,
                       const void* weight, const float* w_scale, const float* bias,
                       const AexrtHipTensorView* residual, const AexrtHipTensorView& y, int32_t* acc_out,
                       ConvParams& p, std::string& why) {
    if (!generic_shape_ok(d)) {
        why = "unsupported conv geometry (groups/dilation/asymmetric stride or pad, or inconsistent out size)";
        return false;
    }
    if (d.batch == 0 || d.in_channels == 0 || d.out_channels == 0 || d.out_h == 0 || d.out_w == 0) {
        why = "empty convolution";
        return false;
    }
    const bool int8 = is_int8_algorithm(algorithm);
    const bool wino = is_winograd_algorithm(algorithm);
    const bool out_f32 = (flags & AEXRT_HIP_CONV_OUT_F32) != 0;
    // fp32 NCHW input read by the conv itself: x->n_stride = c_real * H * W
    // elements per image, c_real <= 4 channels read as in_channels = 8 (the
    // weights are packed for 8 channels, the missing ones zero)
    const bool nchw = (flags & AEXRT_HIP_CONV_IN_NCHW_F32) != 0;
    int c_real = 0;
    if (nchw) {
        const int64_t plane = int64_t(d.in_h) * d.in_w;
        c_real = plane > 0 ? (int)(x.n_stride / plane) : 0;
        if (int8 || wino || d.in_channels != 8 || d.kernel_h != 3 || d.kernel_w != 3 || d.pad_top != 1 ||
            (d.stride_h != 1 && d.stride_h != 2) || c_real < 1 || c_real > 4 || x.n_stride != c_real * plane ||
            reinterpret_cast<uintptr_t>(x.data) % 4 || !(flags & AEXRT_HIP_CONV_SILU) ||
            (flags & (AEXRT_HIP_CONV_RESIDUAL | AEXRT_HIP_CONV_OUT_F32))) {
            why = "fp32 NCHW input: fp16 3x3 pad-1 SiLU conv with in_channels 8, n_stride = c*H*W (c <= 4), "
                  "fp16 output, no residual";
            return false;
        }
    }
    if (int8) {
        if (!can_use_int8(d, int8_kernel_elems(algorithm))) {
            why = "descriptor is not eligible for the planned int8 kernel";
            return false;
        }
        if ((algorithm == 52u && d.stride_h != 1) || (algorithm == 53u && d.stride_h != 2)) {
            why = "int8 kernel id does not match the stride";
            return false;
        }
        const bool dynamic = (flags & AEXRT_HIP_CONV_INT8_DYNAMIC) != 0;
        if ((!dynamic && !x.amax_slots) || !w_scale) {
            why = "int8 conv needs the input amax slots and the weight scales";
            return false;
        }
        if (dynamic && (acc_out || (flags & AEXRT_HIP_CONV_INT8_PG16) || nchw)) {
            why = "dynamic int8 conv: no acc_out, not with pg16, NHWC input";
            return false;
        }
    } else if (flags & AEXRT_HIP_CONV_INT8_DYNAMIC) {
        why = "the dynamic int8 flag needs an int8 algorithm";
        return false;
    }
    if (wino) {
        if (!winograd_shape_ok(d)) {
            why = "Winograd F(2x2,3x3) needs 3x3 s1 p1, C % 4 == 0 and even output dims";
            return false;
        }
        if (!(flags & AEXRT_HIP_CONV_SILU)) {
            why = "Winograd kernels always apply SiLU (reference kernels 40/46)";
            return false;
        }
        if (!aligned16(x.data) || x.c_stride % 4 || x.n_stride % 4) {
            why = "Winograd input view must be 8-byte aligned with 4-element strides";
            return false;
        }
    } else {
        if (!nchw && (d.in_channels % 8 || !aligned16(x.data) || x.c_stride % 8 ||
                      x.n_stride != int64_t(d.in_h) * d.in_w * x.c_stride)) {
            why = "NHWC input view must be 16-byte aligned, C % 8 == 0, c_stride % 8 == 0 and n_stride == H*W*c_stride";
            return false;
        }
        if (d.out_channels % 8 || !aligned16(y.data) || y.c_stride % (out_f32 ? 4 : 8) ||
            y.n_stride % (out_f32 ? 4 : 8)) {
            why = "output view must be 16-byte aligned with OC % 8 == 0 and 16-byte aligned strides";
            return false;
        }
        if ((flags & AEXRT_HIP_CONV_RESIDUAL) && residual &&
            (!aligned16(residual->data) || residual->c_stride % 8 || residual->n_stride % 8)) {
            why = "residual view must be 16-byte aligned with 8-element strides";
            return false;
        }
    }
    if (!slot_ref_ok(x) || !slot_ref_ok(y)) {
        why = "striped amax slots need a stride with stripes * stride < 2^31";
        return false;
    }
    if (!nchw && (uint32_t)x.c_stride < d.in_channels) {
        why = "input c_stride smaller than in_channels";
        return false;
    }
    if ((uint32_t)y.c_stride < d.out_channels) {
        why = "output c_stride smaller than out_channels";
        return false;
    }
    if ((flags & AEXRT_HIP_CONV_RESIDUAL) && (!residual || !residual->data)) {
        why = "residual flag without a residual view";
        return false;
    }
    if (acc_out && !int8) {
        why = "acc_out is only produced by int8 kernels";
        return false;
    }
    const bool pg16 = (flags & AEXRT_HIP_CONV_INT8_PG16) != 0;
    if (pg16 && (!int8 || acc_out || nchw || d.in_channels > 4096)) {
        why = "pg16 (per-group activation scales) needs an int8 algorithm, in_channels <= 4096, no acc_out and an "
              "NHWC input";
        return false;
    }
    const WeightGeom g = weight_geom(d, algorithm);
    p = ConvParams{};
    p.x = x.data;
    p.x_nstride = x.n_stride;
    p.x_cstride = nchw ? 8 : x.c_stride;
    p.loader = nchw ? kLoaderNchwF32 : kLoaderNhwc;
    p.c_real = c_real;
    p.x_slots = slot_ref(x);
    p.x_nslots = (int)(d.in_channels / 16);
    p.w = weight;
    p.Kp = (int)g.kp;
    p.OCp = (int)g.ocp;
    p.w_scale = w_scale;
    p.bias = bias;
    p.y = y.data;
    p.y_nstride = y.n_stride;
    p.y_cstride = y.c_stride;
    p.y_slots = slot_ref(y);
    if (residual && (flags & AEXRT_HIP_CONV_RESIDUAL)) {
        p.res = static_cast<const __half*>(residual->data);
        p.r_nstride = residual->n_stride;
        p.r_cstride = residual->c_stride;
    }
    p.acc_out = acc_out;
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
    const int64_t m = (int64_t)d.batch * d.out_h * d.out_w;
    if (m > INT32_MAX / 2) {
        why = "too many output positions for one launch";
        return false;
    }
    p.M = (int)m;
    p.flags = (int)(flags & (AEXRT_HIP_CONV_SILU | AEXRT_HIP_CONV_RESIDUAL | AEXRT_HIP_CONV_OUT_F32));
    if (pg16) p.flags |= kConvPg16;
    if (flags & AEXRT_HIP_CONV_INT8_DYNAMIC) p.flags |= kConvDynamic;
    return true;
}

DynConvParams dynamic_params(const ConvParams& p) {
    DynConvParams q{};
    q.x = static_cast<const __half*>(p.x);
    q.x_nstride = p.x_nstride;
    q.x_cstride = p.x_cstride;
    q.w = static_cast<const int8_t*>(p.w);
    q.Kp = p.Kp;
    q.w_scale = p.w_scale;
    q.bias = p.bias;
    q.y = p.y;
    q.y_nstride = p.y_nstride;
    q.y_cstride = p.y_cstride;
    q.res = p.res;
    q.r_nstride = p.r_nstride;
    q.r_cstride = p.r_cstride;
    q.y_slots = p.y_slots;
    q.N = p.N, q.H = p.H, q.W = p.W, q.C = p.C, q.OH = p.OH, q.OW = p.OW, q.OC = p.OC, q.K = p.KH, q.S = p.S;
    q.flags = p.flags & (kConvSilu | kConvResidual | kConvOutF32);
    return q;
}

bool launch_conv(const ConvParams& p, uint32_t algorithm, hipStream_t stream) {
    if (is_winograd_algorithm(algorithm)) return check_hip(launch_winograd_f2x2(p, stream), "winograd conv");
    if (p.flags & kConvPg16) return check_hip(launch_conv_int8_pg16(p, stream), "int8 pg16 conv");
    if (p.flags & kConvDynamic) return check_hip(launch_conv_int8_dynamic(dynamic_params(p), stream), "int8 dynamic conv");
    return check_hip(launch_conv_igemm(p, is_int8_algorithm(algorithm), stream),
                     is_int8_algorithm(algorithm) ? "int8 conv" : "fp16 conv");
}

}  // namespace aexrt
