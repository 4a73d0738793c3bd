// Device helpers shared by the MoE kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "moe_internal.hpp"

namespace moehip {

constexpr int kWave = 64;

// bf16 -> f32 is a 16-bit shift (crates/metal-backend/src/shaders/affine.metal:9-10).
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
}

// One scalar of a scale/bias/dense array of dtype T (0 F32, 1 F16, 30 BF16)
// (affine.metal:6-12, common.metal val()).
template <int T>
__device__ __forceinline__ float load_scalar(const void *p, uint64_t i) {
    if constexpr (T == 0) {
        return reinterpret_cast<const float *>(p)[i];
    } else if constexpr (T == 30) {
        return bf16_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
    } else {
        return f16_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
    }
}

// Raw (untyped) buffer resource over `bytes` bytes at p (gfx9 descriptor word
// 3): loads through it take a scalar base and a 32-bit offset, and return 0
// past `bytes`.
constexpr int kRsrcWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *p, uint32_t bytes = 0xffffffffu) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, bytes, kRsrcWord3);
}

// Raw bits of one such scalar, converted later by raw_to_f32: lets a caller
// issue every load before the first conversion waits on one.
template <int T>
__device__ __forceinline__ uint32_t load_raw(const void *p, uint64_t i) {
    if constexpr (T == 0)
        return reinterpret_cast<const uint32_t *>(p)[i];
    else
        return reinterpret_cast<const uint16_t *>(p)[i];
}
template <int T>
__device__ __forceinline__ float raw_to_f32(uint32_t r) {
    if constexpr (T == 0)
        return __uint_as_float(r);
    else if constexpr (T == 30)
        return bf16_to_f32(r);
    else
        return f16_to_f32(r);
}

// ---- cross-lane reductions: DPP within 16-lane rows, gfx950 permlane swaps
// across rows (no LDS round trips, no SGPR round trips).  All lanes of the
// wave must be active.  dpp_ctrl codes (gfx9 DPP): quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror, row_mirror, row_ror:4, row_ror:8.
constexpr int kDppQuad1 = 0xB1;
constexpr int kDppQuad2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
constexpr int kDppRor4 = 0x124;
constexpr int kDppRor8 = 0x128;

// LDS writes of this wave are complete and visible to its other lanes.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ uint32_t readlane_u(uint32_t v, int l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
// v[l] op v[l ^ 16] and v[l] op v[l ^ 32] (v_permlane16/32_swap: each returns
// the value and its partner across the row / half-wave boundary).
__device__ __forceinline__ float add_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    return __int_as_float(r[0]) + __int_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    return __int_as_float(r[0]) + __int_as_float(r[1]);
}
__device__ __forceinline__ uint32_t max_xor16_u(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap((int)v, (int)v, false, false);
    return max((uint32_t)r[0], (uint32_t)r[1]);
}
__device__ __forceinline__ uint32_t max_xor32_u(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap((int)v, (int)v, false, false);
    return max((uint32_t)r[0], (uint32_t)r[1]);
}
__device__ __forceinline__ uint32_t min_xor16_u(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap((int)v, (int)v, false, false);
    return min((uint32_t)r[0], (uint32_t)r[1]);
}
__device__ __forceinline__ uint32_t min_xor32_u(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap((int)v, (int)v, false, false);
    return min((uint32_t)r[0], (uint32_t)r[1]);
}

// Sum over aligned groups of `width` lanes (a power of two <= 64, uniform);
// every lane of a group receives its group's sum.  After each step the
// partial is uniform inside the group reduced so far, so the mirrors pair
// each lane with the other half.
__device__ __forceinline__ float subwave_sum(float v, int width) {
    if (width >= 2) v += dpp_f<kDppQuad1>(v);
    if (width >= 4) v += dpp_f<kDppQuad2>(v);
    if (width >= 8) v += dpp_f<kDppHalfMirror>(v);
    if (width >= 16) v += dpp_f<kDppMirror>(v);
    if (width >= 32) v = add_xor16(v);
    if (width >= 64) v = add_xor32(v);
    return v;
}
// Wave sum, identical in every lane (lane 0's association order).
__device__ __forceinline__ float wave_sum(float v) { return readlane_f(subwave_sum(v, kWave), 0); }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u<kDppQuad1>(v));
    v = max(v, dpp_u<kDppQuad2>(v));
    v = max(v, dpp_u<kDppHalfMirror>(v));
    v = max(v, dpp_u<kDppMirror>(v));
    return max_xor32_u(max_xor16_u(v));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, dpp_u<kDppQuad1>(v));
    v = min(v, dpp_u<kDppQuad2>(v));
    v = min(v, dpp_u<kDppHalfMirror>(v));
    v = min(v, dpp_u<kDppMirror>(v));
    return min_xor32_u(min_xor16_u(v));
}
// Order-preserving key of a non-NaN float (unsigned compare = float compare;
// -0 is folded onto +0 so the two still tie, as under float `>`).
__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t b = __float_as_uint(f + 0.0f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float funkey(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// Max over the wave of non-NaN floats (NaN inputs must be pre-filtered).
__device__ __forceinline__ float wave_max(float v) { return funkey(wave_max_u32(fkey(v))); }

// Byte N of a word as float: one v_cvt_f32_ubyteN (written out because the
// compiler otherwise emits a bit-field extract plus v_cvt_f32_ubyte0 for
// bytes 1-3).
template <int N>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
    float r;
    if constexpr (N == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (N == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (N == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// Codes of one packed word as floats, low bits first (affine.metal:17-19,
// checkpoint.rs:183-191).  4-bit words are split into even/odd nibble bytes so
// each code converts with one v_cvt_f32_ubyteN.
template <int BITS>
__device__ __forceinline__ void unpack_word(uint32_t w, float *c) {
    if constexpr (BITS == 4) {
        uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
        c[0] = ubyte_f32<0>(lo);  // code 0 (bits 0-3)
        c[1] = ubyte_f32<0>(hi);  // code 1 (bits 4-7)
        c[2] = ubyte_f32<1>(lo);
        c[3] = ubyte_f32<1>(hi);
        c[4] = ubyte_f32<2>(lo);
        c[5] = ubyte_f32<2>(hi);
        c[6] = ubyte_f32<3>(lo);
        c[7] = ubyte_f32<3>(hi);
    } else if constexpr (BITS == 8) {
        c[0] = ubyte_f32<0>(w);
        c[1] = ubyte_f32<1>(w);
        c[2] = ubyte_f32<2>(w);
        c[3] = ubyte_f32<3>(w);
    } else {  // 2-bit: four 2-bit codes per byte
        uint32_t b0 = w & 0x03030303u, b1 = (w >> 2) & 0x03030303u;
        uint32_t b2 = (w >> 4) & 0x03030303u, b3 = (w >> 6) & 0x03030303u;
#pragma unroll
        for (int byte = 0; byte < 4; byte++) {
            int sh = byte;
            float v0, v1, v2, v3;
            if (sh == 0) {
                v0 = ubyte_f32<0>(b0); v1 = ubyte_f32<0>(b1);
                v2 = ubyte_f32<0>(b2); v3 = ubyte_f32<0>(b3);
            } else if (sh == 1) {
                v0 = ubyte_f32<1>(b0); v1 = ubyte_f32<1>(b1);
                v2 = ubyte_f32<1>(b2); v3 = ubyte_f32<1>(b3);
            } else if (sh == 2) {
                v0 = ubyte_f32<2>(b0); v1 = ubyte_f32<2>(b1);
                v2 = ubyte_f32<2>(b2); v3 = ubyte_f32<2>(b3);
            } else {
                v0 = ubyte_f32<3>(b0); v1 = ubyte_f32<3>(b1);
                v2 = ubyte_f32<3>(b2); v3 = ubyte_f32<3>(b3);
            }
            c[byte * 4 + 0] = v0;
            c[byte * 4 + 1] = v1;
            c[byte * 4 + 2] = v2;
            c[byte * 4 + 3] = v3;
        }
    }
}

// sum_j code_j * x[j] over one packed word (the per-word product of
// affine.metal:60-63).
template <int BITS>
__device__ __forceinline__ float word_dot(uint32_t w, const float *x) {
    constexpr int P = 32 / BITS;
    float c[P];
    unpack_word<BITS>(w, c);
    float d = 0.f;
#pragma unroll
    for (int j = 0; j < P; j++) d = fmaf(c[j], x[j], d);
    return d;
}

// e^x from the hardware base-2 exponential (v_exp_f32, 1 ulp): x*log2(e) is
// split into its rounded product t and that product's rounding error (an
// FMA recovers it, plus the low part of log2(e)), and
// 2^(t + err) = 2^t * (1 + err*ln 2) to first order.  About 1.5 ulp; exact
// 0 at -inf, +inf at +inf, NaN at NaN.  Used where routing needs many
// exponentials (the softmax denominator).
__device__ __forceinline__ float exp_fast(float x) {
    constexpr float kLog2e = 1.44269502162933349609375f;   // log2(e) rounded to float
    constexpr float kLog2eLo = 1.925963033500011e-8f;      // log2(e) - kLog2e
    constexpr float kLn2 = 0.693147180559945309417f;
    const float t = x * kLog2e;
    const float err = __builtin_isfinite(t) ? fmaf(x, kLog2e, -t) + x * kLog2eLo : 0.f;
    return __builtin_amdgcn_exp2f(t) * fmaf(err, kLn2, 1.0f);
}

__device__ __forceinline__ float silu_mul(float a, float b) {
    // activation kernel (elementwise.metal:8-17): a/(1+exp(-a))*b
    return a / (1.0f + __expf(-a)) * b;
}

}  // namespace moehip
