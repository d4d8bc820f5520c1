// The reference's int8 conv command (the int8 block of record_replay_conv,
// native/aexrt_d3d12_runtime.cpp:23935-24318) on NHWC device views: the
// caller passes a plain fp16 activation tensor, and the command chooses the
// quantization the reference would:
//   * fewer than 4096 input elements (RT:21478-21479): the dynamic kernel,
//     per (position, 4 channels) scales computed in the conv;
//   * plan flag 16 (AEXRT_HIP_CONV_INT8_PG16): the reference's strip amax of
//     the input (RT:3219-3259) into scratch, then the pg16 conv;
//   * otherwise: the per-tensor amax of the input (16-channel slots, striped)
//     into scratch, then the prequantized conv that quantizes on load.
// The scratch is the amax words: stripes x C/16 uint32, cleared by a fill
// kernel before every use.  The library allocates it once per device and
// keeps it for the process; calls that overlap on one device share it and
// race.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <vector>

#include "internal.h"

namespace aexrt {

namespace {

constexpr uint32_t kCmdStripes = 16;  // slot copies the amax pass spreads its atomics over

struct DeviceScratch {
    uint32_t* words = nullptr;
    uint64_t count = 0;
};

std::mutex g_scratch_mutex;
std::map<int, DeviceScratch> g_scratch;     // current scratch per device
std::vector<void*> g_retired;               // smaller scratch of earlier calls (kept: a stream may still use it)

// The library's scratch of this device, at least `words` uint32 (hipMalloc
// on first use and when a larger conv needs more).
uint32_t* library_scratch(uint64_t words) {
    int dev = 0;
    if (!check_hip(hipGetDevice(&dev), "conv2d_int8: current device")) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    DeviceScratch& s = g_scratch[dev];
    if (s.count >= words) return s.words;
    void* p = nullptr;
    if (!check_hip(hipMalloc(&p, words * 4), "conv2d_int8: scratch allocation")) return nullptr;
    if (s.words) g_retired.push_back(s.words);
    s.words = static_cast<uint32_t*>(p);
    s.count = words;
    return s.words;
}

}  // namespace

uint64_t int8_command_scratch_words(uint32_t in_channels) { return uint64_t(kCmdStripes) * ((in_channels + 15) / 16); }

bool run_int8_command(const AexrtConv2DDesc& d, uint32_t algorithm, uint32_t flags, const AexrtHipTensorView& x,
                      const void* weight, const float* w_scale, const float* bias, const AexrtHipTensorView* residual,
                      const AexrtHipTensorView& y, uint32_t* scratch, uint64_t scratch_words, hipStream_t stream) {
    const uint32_t allowed = AEXRT_HIP_CONV_SILU | AEXRT_HIP_CONV_RESIDUAL | AEXRT_HIP_CONV_OUT_F32 |
                             AEXRT_HIP_CONV_INT8_PG16;
    if (!is_int8_algorithm(algorithm) || (flags & ~allowed)) {
        set_error("conv2d_int8: an int8 algorithm (51/52/53) and flags SILU / RESIDUAL / OUT_F32 / INT8_PG16");
        return false;
    }
    if (d.in_channels % 16 || d.in_channels == 0) {
        set_error("conv2d_int8: in_channels % 16 == 0 (amax is kept per 16 channels)");
        return false;
    }
    const uint64_t elements = uint64_t(d.batch) * d.in_channels * d.in_h * d.in_w;
    const uint32_t groups = d.in_channels / 16;
    AexrtHipTensorView xv = x;
    xv.amax_slots = nullptr;
    xv.amax_stripes = 0;
    xv.amax_stripe_stride = 0;
    std::string why;
    ConvParams p{};
    if (elements < kInt8PrequantMinElements) {
        if (!build_conv_params(d, algorithm, (flags & ~AEXRT_HIP_CONV_INT8_PG16) | AEXRT_HIP_CONV_INT8_DYNAMIC, xv,
                               weight, w_scale, bias, residual, y, nullptr, p, why)) {
            set_error("conv2d_int8: " + why);
            return false;
        }
        return launch_conv(p, algorithm, stream);
    }
    const bool pg16 = (flags & AEXRT_HIP_CONV_INT8_PG16) != 0;
    const uint32_t stripes = pg16 ? 1u : kCmdStripes;
    if (!scratch || scratch_words < uint64_t(stripes) * groups) {
        set_error("conv2d_int8: scratch smaller than the input's amax words");
        return false;
    }
    xv.amax_slots = scratch;
    xv.amax_stripes = stripes;
    xv.amax_stripe_stride = stripes > 1 ? groups : 0;
    if (!build_conv_params(d, algorithm, flags, xv, weight, w_scale, bias, residual, y, nullptr, p, why)) {
        set_error("conv2d_int8: " + why);
        return false;
    }
    const __half* xd = static_cast<const __half*>(x.data);
    const int N = (int)d.batch, HW = (int)(d.in_h * d.in_w), C = (int)d.in_channels;
    if (!check_hip(launch_fill_u32(scratch, uint64_t(stripes) * groups, 0u, stream), "conv2d_int8: clear amax"))
        return false;
    const hipError_t e = pg16 ? launch_amax_strips_nhwc(xd, x.n_stride, x.c_stride, N, HW, C, scratch, stream)
                              : launch_amax_slots_nhwc(xd, x.n_stride, x.c_stride, N, HW, C,
                                                       SlotRef{scratch, stripes, groups}, stream);
    if (!check_hip(e, "conv2d_int8: amax pass")) return false;
    return launch_conv(p, algorithm, stream);
}

}  // namespace aexrt

// ---- allocation-free variant -------------------------------------------------
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc): the amax
// words live in this file-scope array instead of library-allocated memory.
// Each device holds its own copy until the process ends.  It covers convs of
// up to kNoAllocMaxChannels input channels (16 stripes x C/16 words).
namespace aexrt {
namespace {
constexpr uint32_t kNoAllocMaxChannels = 4096;
constexpr uint64_t kNoAllocWords = uint64_t(kCmdStripes) * (kNoAllocMaxChannels / 16);  // 16 KiB
}  // namespace
}  // namespace aexrt

static __device__ __align__(256) uint32_t scratch[aexrt::kNoAllocWords];

namespace aexrt {
namespace {

std::mutex g_symbol_mutex;
std::map<int, uint32_t*> g_scratch_ptr;  // device -> address of `scratch` on that device

// The device address of `scratch` on the current device, looked up once per
// device with that device current.  Host code uses this pointer, never the
// array's name (a host-side stand-in).
uint32_t* static_scratch() {
    int dev = 0;
    if (!check_hip(hipGetDevice(&dev), "conv2d_int8_noalloc: current device")) return nullptr;
    std::lock_guard<std::mutex> lock(g_symbol_mutex);
    auto it = g_scratch_ptr.find(dev);
    if (it != g_scratch_ptr.end()) return it->second;
    void* p = nullptr;
    if (!check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "conv2d_int8_noalloc: scratch address") || !p)
        return nullptr;
    g_scratch_ptr[dev] = static_cast<uint32_t*>(p);
    return static_cast<uint32_t*>(p);
}

}  // namespace
}  // namespace aexrt

using namespace aexrt;

extern "C" {

int aexrt_hip_conv2d_int8_noalloc(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags,
                                  const AexrtHipTensorView* x, const void* weight, const float* w_scale,
                                  const float* bias, const AexrtHipTensorView* residual, const AexrtHipTensorView* y,
                                  void* stream) {
    if (!desc || !x || !y || !weight || !w_scale || !bias || !x->data || !y->data) {
        set_error("conv2d_int8_noalloc: null argument");
        return 0;
    }
    if (desc->in_channels > kNoAllocMaxChannels) {
        set_error("conv2d_int8_noalloc: at most 4096 input channels (its static amax scratch is 16 KiB per device)");
        return 0;
    }
    uint32_t* s = static_scratch();
    if (!s) return 0;
    return run_int8_command(*desc, algorithm, flags, *x, weight, w_scale, bias, residual, *y, s, kNoAllocWords,
                            static_cast<hipStream_t>(stream))
               ? 1
               : 0;
}

int aexrt_hip_conv2d_int8(const AexrtConv2DDesc* desc, uint32_t algorithm, uint32_t flags, const AexrtHipTensorView* x,
                          const void* weight, const float* w_scale, const float* bias,
                          const AexrtHipTensorView* residual, const AexrtHipTensorView* y, void* stream) {
    if (!desc || !x || !y || !weight || !w_scale || !bias || !x->data || !y->data) {
        set_error("conv2d_int8: null argument");
        return 0;
    }
    const uint64_t words = int8_command_scratch_words(desc->in_channels);
    uint32_t* scratch = library_scratch(words);
    if (!scratch) return 0;
    return run_int8_command(*desc, algorithm, flags, *x, weight, w_scale, bias, residual, *y, scratch, words,
                            static_cast<hipStream_t>(stream))
               ? 1
               : 0;
}

}  // extern "C"
