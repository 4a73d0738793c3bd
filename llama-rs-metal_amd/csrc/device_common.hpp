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

// Sum over the 64 lanes of a wave (butterfly; every lane gets the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
// Sum over aligned groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float subwave_sum(float v, int width) {
    for (int o = width >> 1; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Byte N of a word as float (selects to v_cvt_f32_ubyteN).
template <int N>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
    return (float)((v >> (8 * N)) & 0xffu);
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

__device__ __forceinline__ float silu_mul(float a, float b) {
    // activation kernel (elementwise.metal:8-17): a/(1+exp(-a))*b
    return a / (1.0f + __expf(-a)) * b;
}

}  // namespace moehip
