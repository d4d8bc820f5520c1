// Shared device helpers for the gfx950 kernels of the W8A8 conv path.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "kernels.h"

namespace aexrt {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Activation amax is kept per 16-channel group ("slot") of every tensor as the
// bit pattern of a non-negative float, so that an unsigned atomicMax orders
// the values.  A view or concat over 16-aligned channel ranges takes the max
// of its slots; the per-tensor amax is the max over all slots.
constexpr int kAmaxGroup = 16;

// The slot copy a workgroup's maxima go to.
__device__ __forceinline__ uint32_t* slot_copy(const SlotRef& r, uint32_t block) {
    return r.p + (block % r.stripes) * r.stride;
}

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// A 16-byte MFMA operand gathered across the wave's two lane halves: every
// lane passes two dword pairs x and y; lane l < 32 gets {x of lane l, x of
// lane l + 32} and lane l + 32 gets {y of lane l, y of lane l + 32}.
// v_permlane32_swap exchanges the upper 32 lanes of its first operand with
// the lower 32 lanes of its second (a VALU op, no LDS round trip).
__device__ __forceinline__ v4i half_swap_operand(const uint32_t (&x)[2], const uint32_t (&y)[2]) {
    const auto a = __builtin_amdgcn_permlane32_swap(x[0], y[0], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(x[1], y[1], false, false);
    return v4i{(int)a[0], (int)b[0], (int)a[1], (int)b[1]};
}

// Max of the slot bit patterns over a wave: slots order as unsigned integers
// (a NaN pattern wins over every finite value, as in the atomicMax producers).
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, kWave));
    return v;
}

// Per-tensor quantizer of the reference's pack pass: s = 127/amax (IEEE fp32
// division, computed once by the caller), q = round-half-even(x * s), kept as
// the low byte of the saturated int32 (the D3D float->int cast saturates; the
// clamp makes the conversion defined for any input, NaN included).
__device__ __forceinline__ int32_t quant_int(float x, float s) {
    const float p = x * s;
    float r = __builtin_rintf(p);
    r = fminf(fmaxf(r, -2147483648.0f), 2147483520.0f);
    return (int32_t)r;
}

__device__ __forceinline__ uint32_t pack4_q(float a, float b, float c, float d, float s) {
    return ((uint32_t)quant_int(a, s) & 0xFFu) | (((uint32_t)quant_int(b, s) & 0xFFu) << 8) |
           (((uint32_t)quant_int(c, s) & 0xFFu) << 16) | (((uint32_t)quant_int(d, s) & 0xFFu) << 24);
}

// SiLU v * sigmoid(v) = v / (1 + e^-v) with the hardware exp2 and reciprocal
// (1 ulp each); the reference's HLSL division is itself a 2.5-ulp operation,
// and both round to the same fp16 except at rare ties.
__device__ __forceinline__ float silu(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// Folds a non-negative value into an amax slot.  Slots only grow during a
// run, so a value that does not exceed what is already visible cannot change
// the slot and its atomic is skipped (the value read is one the slot held at
// some point, never more than its current content).  Every wave of a layer
// targets the same few slots; without the check those atomics serialize in
// L2 and dominate the layer's run time.
__device__ __forceinline__ void slot_max(uint32_t* slot, float v) {
    const uint32_t b = f2u(v);
    const uint32_t seen = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (b > seen) atomicMax(slot, b);
}

// XCD-aware block order: workgroups are dealt round-robin over the 8 XCDs,
// so block b runs on XCD b % 8.  Give each XCD a contiguous range of logical
// blocks so the lines that neighbouring blocks share are fetched into one L2.
__device__ __forceinline__ int xcd_remap(int b, int nb) {
    const int full = (nb / 8) * 8;
    if (b >= full) return b;
    return (b % 8) * (nb / 8) + b / 8;
}

}  // namespace aexrt
