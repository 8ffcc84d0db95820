// Device-side helpers shared by the gfx950 kernels: fp16 vector types, the fused activation, the
// launch-error plumbing used by every extern "C" launcher.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "vkhip.h"

namespace vkhip {

    // Cache policy (buffer instruction aux bits) of the streaming accesses of the conv epilogues:
    // the residual, read once, and the output, written once per layer. NT (non-temporal, bit 1) on
    // the residual load keeps it from evicting the operand tiles that the other workgroups of the
    // launch re-read from L2. The output stays cached: the next layer reads it, and with NT stores
    // it would miss the last-level cache (measured: NT on both costs ResNet-50 b64 4%).
#ifndef VKHIP_STREAM_LOAD
#define VKHIP_STREAM_LOAD 2
#endif
#ifndef VKHIP_STREAM_STORE
#define VKHIP_STREAM_STORE 0
#endif
    constexpr int kStreamLoad  = VKHIP_STREAM_LOAD;
    constexpr int kStreamStore = VKHIP_STREAM_STORE;

    typedef _Float16 half_t;
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    typedef _Float16 half8 __attribute__((ext_vector_type(8)));
    typedef float    float4v __attribute__((ext_vector_type(4)));
    typedef float    float16v __attribute__((ext_vector_type(16)));

    // t / 6 in three VALU operations instead of the ~10 of a general fp32 division: q = t * (1/6),
    // then one fma-based correction with the exact remainder t - 6q (Markstein's method). It equals
    // the correctly rounded t / 6.f for every fp32 t whose quotient is a normal number; below that
    // (|t / 6| < 2^-126) the two may differ in the last subnormal bit, and both round to the same
    // signed zero in the fp16 stores every caller makes. q is kept when it is exact (r = 0: also
    // keeps the sign of -0) and for an infinite t (the correction would be inf - inf). Checked exhaustively over all 2^32 inputs by tests/test_div6.py.
    __device__ __forceinline__ float div6(float t) {
        constexpr float kInv6 = 1.0f / 6.0f;
        const float     q     = t * kInv6;
        const float     r     = __builtin_fmaf(-q, 6.0f, t);
        const float     q2    = __builtin_fmaf(r, kInv6, q);
        return (r == 0.f || q2 != q2) ? q : q2;
    }

    // fp32 -> fp16 bits with the reference codec's rounding (include/vknn/dtype.h:121-157): half away
    // from zero on the dropped mantissa bits (a carry may ripple into the exponent), subnormals
    // likewise, overflow to infinity, NaN kept quiet. The reference's GPU path converts conv weights
    // this way (src/backend/vulkan/ops/conv.cpp:364-437), so every weight blob packed here does too
    // (ref_half), and the input pack uses it for the reference host codec's bit-exact NC4HW4 image.
    __host__ __device__ inline uint16_t ref_half_bits(float v) {
        const uint32_t bits = __builtin_bit_cast(uint32_t, v);
        const uint32_t sign = (bits >> 16) & 0x8000u;
        const uint32_t fexp = (bits >> 23) & 0xFFu;
        const uint32_t man  = bits & 0x7FFFFFu;
        if (fexp == 0xFFu) return (uint16_t) (sign | 0x7C00u | (man ? 0x200u : 0u));
        const int e = (int) fexp - 112;
        if (e >= 31) return (uint16_t) (sign | 0x7C00u);
        if (e > 0) return (uint16_t) ((sign | ((uint32_t) e << 10) | (man >> 13)) + ((man >> 12) & 1u));
        if (e < -10) return (uint16_t) sign;
        const uint32_t full = man | 0x800000u;
        const uint32_t sh   = (uint32_t) (14 - e);
        return (uint16_t) (sign | ((full >> sh) + ((full >> (sh - 1)) & 1u)));
    }
    __host__ __device__ inline half_t ref_half(float v) { return __builtin_bit_cast(half_t, ref_half_bits(v)); }

    // Fused activation (codes = vknn ActType). The formulas follow the reference's applyAct
    // (src/backend/cpu/cpu_backend.cpp:33-72): HardSwish = v*clamp(v+3,0,6)/6, SiLU = v/(1+e^-v).
    __device__ __forceinline__ float apply_act(float v, int act, float lo, float hi) {
        switch (act) {
            case VKHIP_ACT_RELU: return v > 0.f ? v : 0.f;
            case VKHIP_ACT_RELU6: return v < 0.f ? 0.f : (v > 6.f ? 6.f : v);
            case VKHIP_ACT_CLIP: return v < lo ? lo : (v > hi ? hi : v);
            case VKHIP_ACT_HARDSWISH: {
                float c = fminf(fmaxf(v + 3.f, 0.f), 6.f);
                return div6(v * c);
            }
            // v / (1 + e^-v) with the hardware reciprocal (1 ulp) instead of an IEEE division: a
            // fraction of the instructions, and the result is stored as fp16
            case VKHIP_ACT_SILU: return v * __builtin_amdgcn_rcpf(1.f + __expf(-v));
            case VKHIP_ACT_HARDSIGMOID: return fminf(fmaxf(lo * v + hi, 0.f), 1.f);
            default: return v;
        }
    }

    // 4 fp16 lanes <-> 4 fp32 values. The fp32 -> fp16 conversion is v_cvt_f16_f32 under the
    // default round-to-nearest-even mode.
    __device__ __forceinline__ float4v h4_to_f4(half4 h) {
        float4v r;
        r.x = (float) h.x; r.y = (float) h.y; r.z = (float) h.z; r.w = (float) h.w;
        return r;
    }
    __device__ __forceinline__ half4 f4_to_h4(float4v f) {
        half4 r;
        r.x = (half_t) f.x; r.y = (half_t) f.y; r.z = (half_t) f.z; r.w = (half_t) f.w;
        return r;
    }
    __device__ __forceinline__ half4 u2_as_h4(uint2 u) {
        half4 h;
        __builtin_memcpy(&h, &u, 8);
        return h;
    }
    __device__ __forceinline__ uint2 h4_as_u2(half4 h) {
        uint2 u;
        __builtin_memcpy(&u, &h, 8);
        return u;
    }

    // Host-side error recording (defined in runtime.hip).
    int  set_error(int code, const char *fmt, ...);
    int  check_launch(const char *what);
    hipStream_t resolve_stream(vkhip_stream_t s);

    inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
    inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

} // namespace vkhip
