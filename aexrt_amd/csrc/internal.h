// Host-side internals shared by the op-level C ABI and the model runtime.
#pragma once
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/aexrt_hip.h"
#include "kernels.h"

namespace aexrt {

void set_error(const std::string& msg);
const char* last_error();
bool check_hip(hipError_t e, const char* what);

bool is_int8_algorithm(uint32_t algorithm);
bool is_winograd_algorithm(uint32_t algorithm);
uint32_t int8_kernel_elems(uint32_t algorithm);
bool can_use_int8(const AexrtConv2DDesc& d, uint32_t kernel_elems);
bool winograd_shape_ok(const AexrtConv2DDesc& d);
bool generic_shape_ok(const AexrtConv2DDesc& d);

// The (possibly striped) slot array of a view; p == nullptr when it has none.
inline SlotRef slot_ref(const AexrtHipTensorView& v) {
    const uint32_t stripes = v.amax_stripes ? v.amax_stripes : 1u;
    return SlotRef{v.amax_slots, stripes, stripes > 1 ? (uint32_t)v.amax_stripe_stride : 0u};
}
inline SlotRef slot_ref(const AexrtHipTensorView* v) { return v ? slot_ref(*v) : SlotRef{nullptr, 1u, 0u}; }
// A striped view needs a stride that fits the kernels' 32-bit slot arithmetic.
inline bool slot_ref_ok(const AexrtHipTensorView& v) {
    return v.amax_stripes <= 1 || (v.amax_stripe_stride > 0 && v.amax_stripe_stride <= 0x7FFFFFFFull &&
                                   (uint64_t)v.amax_stripes * v.amax_stripe_stride <= 0x7FFFFFFFull);
}

// Geometry of a repacked conv weight.
struct WeightGeom {
    uint32_t ocp;        // output channels rounded up to 16
    uint32_t kp;         // K rounded up to 64 (igemm) / C rounded up to 32 (Winograd)
    uint32_t elem_bytes;
    uint64_t nbytes;
};
WeightGeom weight_geom(const AexrtConv2DDesc& d, uint32_t algorithm);

// Validates one convolution and fills the kernel parameters.
bool build_conv_params(const AexrtConv2DDesc& d, uint32_t algorithm, uint32_t flags, const AexrtHipTensorView& x,
                       const void* weight, const float* w_scale, const float* bias,
                       const AexrtHipTensorView* residual, const AexrtHipTensorView& y, int32_t* acc_out,
                       ConvParams& p, std::string& why);
bool launch_conv(const ConvParams& p, uint32_t algorithm, hipStream_t stream);
// Kernel parameters of the dynamic int8 conv for a conv built with
// AEXRT_HIP_CONV_INT8_DYNAMIC.
DynConvParams dynamic_params(const ConvParams& p);
// The reference dispatches int8 convs whose input has fewer than this many
// elements to the dynamic kernel (native/aexrt_d3d12_runtime.cpp:21478-21479).
constexpr uint64_t kInt8PrequantMinElements = 4096;

// The reference's int8 conv command on a plain fp16 NHWC input (dynamic
// below 4096 elements, else amax into `scratch` + pg16 or per-tensor conv);
// scratch holds int8_command_scratch_words(C) uint32 (unused by the dynamic
// kernel).
uint64_t int8_command_scratch_words(uint32_t in_channels);
bool run_int8_command(const AexrtConv2DDesc& d, uint32_t algorithm, uint32_t flags, const AexrtHipTensorView& x,
                      const void* weight, const float* w_scale, const float* bias, const AexrtHipTensorView* residual,
                      const AexrtHipTensorView& y, uint32_t* scratch, uint64_t scratch_words, hipStream_t stream);

}  // namespace aexrt
