// Lane-row products shared by the fused decode (k_decode.hip) and the
// batched decode (k_batched.hip).
//
// Weight layout "chunk32": lane (sub, cl) of a wave owns 32 consecutive
// elements (chunk cl) of row `sub`; a row of `in` elements spans in/32 lanes
// (a power of two <= 64), so one wave instruction covers 64/(in/32) rows and
// every lane issues one 8/16/32-byte load per affine row (2/4/8-bit), all
// coalesced.  Each chunk lies inside one quantization group (group >= 32).
// The activations a lane multiplies against stay in registers.
#pragma once
#include "route.hpp"

namespace moehip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 32 consecutive weight elements of one row as raw words.
template <int BITS, int T>
struct Chunk32 {
    static constexpr int BYTES = BITS ? 4 * BITS : (T == 0 ? 128 : 64);
    static constexpr int NW = BYTES / 4;
    uint32_t w[NW];
    __device__ __forceinline__ void load(const void *base, uint64_t chunk) {
        const uint8_t *p = reinterpret_cast<const uint8_t *>(base) + chunk * BYTES;
        if constexpr (NW >= 4) {
#pragma unroll
            for (int i = 0; i < NW / 4; i++) {
                const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p) + i);
                w[4 * i + 0] = v[0];
                w[4 * i + 1] = v[1];
                w[4 * i + 2] = v[2];
                w[4 * i + 3] = v[3];
            }
        } else {
            const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
            w[0] = v[0];
            w[1] = v[1];
        }
    }
    // sum_j value_j * x[j]; for affine rows value_j is the raw code.
    __device__ __forceinline__ float dot(const float *x) const {
        float d = 0.f;
        if constexpr (BITS) {
            constexpr int P = 32 / BITS;
#pragma unroll
            for (int i = 0; i < NW; i++) d += word_dot<BITS>(w[i], x + i * P);
        } else if constexpr (T == 0) {
#pragma unroll
            for (int j = 0; j < 32; j++) d = fmaf(__uint_as_float(w[j]), x[j], d);
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float lo = T == 30 ? bf16_to_f32(w[i] & 0xffffu) : f16_to_f32(w[i] & 0xffffu);
                const float hi = T == 30 ? bf16_to_f32(w[i] >> 16) : f16_to_f32(w[i] >> 16);
                d = fmaf(lo, x[2 * i], d);
                d = fmaf(hi, x[2 * i + 1], d);
            }
        }
        return d;
    }
};

// One lane's share of `R` rows, split into a load phase and an arithmetic
// phase so a caller can put several row sets (and its activation loads) in
// flight before the first wait.  Loads are unconditional: a load under a
// branch, or a conversion next to its load, makes the compiler wait for it
// before the next row's loads issue.  An absent row (!ok[f]) re-reads row 0
// and contributes 0.
template <int BITS, int T, int R>
struct LaneRows {
    Chunk32<BITS, T> c[R];
    uint32_t sr[R], br[R];
    bool ok[R];
    __device__ __forceinline__ void load(const WDesc &w, const uint64_t *grow, const bool *okv,
                                         uint32_t cl, uint32_t C) {
#pragma unroll
        for (int f = 0; f < R; f++) {
            ok[f] = okv[f];
            const uint64_t row = okv[f] ? grow[f] : 0u;
            c[f].load(w.data, row * C + cl);
            if constexpr (BITS) {
                const uint64_t g = (row * w.in + (uint64_t)cl * 32) >> w.gshift;
                sr[f] = load_raw<T>(w.scales, g);
                br[f] = load_raw<T>(w.biases, g);
            }
        }
    }
    // Marks the raw words as changed: inside a loop over inputs this keeps the
    // compiler from hoisting the code conversions out of the loop, which would
    // hold every converted code of every row in registers.
    __device__ __forceinline__ void pin() {
#pragma unroll
        for (int f = 0; f < R; f++)
#pragma unroll
            for (int i = 0; i < Chunk32<BITS, T>::NW; i++) asm volatile("" : "+v"(c[f].w[i]));
    }
    __device__ __forceinline__ void dot(const float *x, float xsum, float *res) const {
#pragma unroll
        for (int f = 0; f < R; f++) {
            float v;
            if constexpr (BITS)
                v = raw_to_f32<T>(sr[f]) * c[f].dot(x) + raw_to_f32<T>(br[f]) * xsum;
            else
                v = c[f].dot(x);
            res[f] = ok[f] ? v : 0.f;
        }
    }
    // The same products for 4-bit rows from the input's limbs (XLimbs); cs:
    // the rows' code sums (code_sums4), fixed over the inputs
    template <typename XL>
    __device__ __forceinline__ void dot_limbs(const XL &xl, float xsum, const uint32_t *cs,
                                              float *res) const {
        static_assert(BITS == 4, "limb products take 4-bit codes");
#pragma unroll
        for (int f = 0; f < R; f++) {
            const float v = raw_to_f32<T>(sr[f]) * xl.dot4(c[f].w, cs[f]) + raw_to_f32<T>(br[f]) * xsum;
            res[f] = ok[f] ? v : 0.f;
        }
    }
    template <typename XL>
    __device__ __forceinline__ void code_sums4(uint32_t *cs) const {
#pragma unroll
        for (int f = 0; f < R; f++) cs[f] = XL::code_sum4(c[f].w);
    }
};

// A lane's 32-element input chunk as six 4-bit limbs, for 4-bit codes on
// the integer dot-product unit (v_dot8_u32_u4: eight code x limb products
// per instruction, against one conversion and one FMA per code in
// Chunk32::dot).  With 2^e > max|x| over the chunk, X_j = round(x_j 2^(22-e))
// + 2^22 lies in [0, 2^23): the FMA x_j 2^(22-e) + 3 * 2^22 leaves it in the
// float's mantissa bits (the exponent bit above them is 0 in [2^23, 2^24)).
// W[l][i] holds nibble l of X_8i .. X_8i+7 in code order, so
// sum_j c_j X_j = sum_l 16^l udot8(codes, W[l]) exactly; the 2^22 offset is
// taken off with sum_j c_j.  One rounding of the exact integer sum
// (2^-23 of the chunk maximum per input, the F32 FMA chain's order of
// error).  A non-finite input makes the chunk's scale NaN.  Chunks whose
// maximum lies below 2^-106 (subnormals included) take e = -105, so 2^(22-e)
// stays finite and every X_j still fits: their error is 2^-128 per input.
struct XLimbs {
    uint32_t W[6][4];
    float scale;  // 2^(e - 22)
    __device__ __forceinline__ void build(const float *x) {
        float m = 0.f;
#pragma unroll
        for (int j = 0; j < 32; j++) m = fmaxf(m, fabsf(x[j]));
        const int e = max(__builtin_amdgcn_frexp_expf(m), -105);
        const float up = __builtin_amdgcn_ldexpf(1.0f, 22 - e);
        scale = __builtin_isfinite(m) ? __builtin_amdgcn_ldexpf(1.0f, e - 22) : __builtin_nanf("");
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t X[8];
#pragma unroll
            for (int j = 0; j < 8; j++) X[j] = __float_as_uint(fmaf(x[8 * i + j], up, 12582912.0f));
            // bytes k of the even (E) and odd (O) elements: E_k = (X0, X2, X4, X6) byte k
            uint32_t E[3], O[3];
#pragma unroll
            for (int par = 0; par < 2; par++) {
                const uint32_t a = X[par], b = X[par + 2], c = X[par + 4], d = X[par + 6];
                const uint32_t ab01 = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
                const uint32_t cd01 = __builtin_amdgcn_perm(d, c, 0x05010400u);
                const uint32_t ab23 = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
                const uint32_t cd23 = __builtin_amdgcn_perm(d, c, 0x07030602u);
                uint32_t *B = par ? O : E;
                B[0] = __builtin_amdgcn_perm(cd01, ab01, 0x05040100u);  // a0 b0 c0 d0
                B[1] = __builtin_amdgcn_perm(cd01, ab01, 0x07060302u);  // a1 b1 c1 d1
                B[2] = __builtin_amdgcn_perm(cd23, ab23, 0x05040100u);  // a2 b2 c2 d2
            }
#pragma unroll
            for (int k = 0; k < 3; k++) {
                // nibble 2n <- element 2n, nibble 2n + 1 <- element 2n + 1
                W[2 * k][i] = (E[k] & 0x0f0f0f0fu) | ((O[k] << 4) & 0xf0f0f0f0u);
                W[2 * k + 1][i] = ((E[k] >> 4) & 0x0f0f0f0fu) | (O[k] & 0xf0f0f0f0u);
            }
        }
    }
    // sum_j c_j of 32 4-bit codes (the offset term of dot4)
    static __device__ __forceinline__ uint32_t code_sum4(const uint32_t *w) {
        uint32_t cs = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) cs = __builtin_amdgcn_udot8(w[i], 0x11111111u, cs, false);
        return cs;
    }
    // sum_j c_j x_j for the chunk's 32 4-bit codes (4 words, code j of word i
    // multiplies element 8i + j); cs = code_sum4(w)
    __device__ __forceinline__ float dot4(const uint32_t *w, uint32_t cs) const {
        uint32_t P[6];
#pragma unroll
        for (int l = 0; l < 6; l++) {
            uint32_t acc = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_udot8(w[i], W[l][i], acc, false);
            P[l] = acc;  // <= 32 * 15 * 15
        }
        const uint32_t lo = P[0] + (P[1] << 4) + (P[2] << 8);                       // < 2^21
        const int32_t hi = (int32_t)(P[3] + (P[4] << 4) + (P[5] << 8)) - (int32_t)(cs << 10);
        return ((float)lo + (float)hi * 4096.0f) * scale;  // (sum c X - 2^22 sum c) 2^(e-22)
    }
};

// Issue point: every load above it issues before the arithmetic below it.
__device__ __forceinline__ void loads_issued() { __builtin_amdgcn_sched_barrier(0); }

template <int BITS, int T, int R>
__device__ __forceinline__ void lane_rows_dot(const WDesc &w, const uint64_t *grow, const bool *ok,
                                              uint32_t cl, uint32_t C, const float *x, float xsum,
                                              float *res) {
    LaneRows<BITS, T, R> L;
    L.load(w, grow, ok, cl, C);
    loads_issued();
    L.dot(x, xsum, res);
}

// Single row of any kind (wave-uniform switch on the weight's kind).
template <int ST>
__device__ __forceinline__ float lane_row_dot_any(const WDesc &w, uint64_t grow, uint32_t cl,
                                                  uint32_t C, const float *x, float xsum) {
    const bool ok = true;
    float r = 0.f;
    switch (w.bits) {
    case 2: lane_rows_dot<2, ST, 1>(w, &grow, &ok, cl, C, x, xsum, &r); break;
    case 4: lane_rows_dot<4, ST, 1>(w, &grow, &ok, cl, C, x, xsum, &r); break;
    case 8: lane_rows_dot<8, ST, 1>(w, &grow, &ok, cl, C, x, xsum, &r); break;
    default:
        if (w.type == 0)
            lane_rows_dot<0, 0, 1>(w, &grow, &ok, cl, C, x, xsum, &r);
        else if (w.type == 1)
            lane_rows_dot<0, 1, 1>(w, &grow, &ok, cl, C, x, xsum, &r);
        else
            lane_rows_dot<0, 30, 1>(w, &grow, &ok, cl, C, x, xsum, &r);
    }
    return r;
}

// This lane's 32-element slice of the (optionally RMS-normalised) input,
// loaded first (load) and normalised once the caller's other loads are in
// flight (finish).  RMSNorm (crates/metal-backend/src/shaders/
// elementwise.metal:31-46): the sum of squares is reduced over the `width`
// lanes that span the row.
struct XChunk {
    float xr[32];
    float nw[32];
    __device__ __forceinline__ void load(const float *__restrict__ x,
                                         const float *__restrict__ norm_w, uint32_t cl) {
        const float4 *src = reinterpret_cast<const float4 *>(x + (uint64_t)cl * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 v = src[i];
            xr[4 * i + 0] = v.x;
            xr[4 * i + 1] = v.y;
            xr[4 * i + 2] = v.z;
            xr[4 * i + 3] = v.w;
        }
        if (norm_w) {
            const float4 *wv = reinterpret_cast<const float4 *>(norm_w + (uint64_t)cl * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 v = wv[i];
                nw[4 * i + 0] = v.x;
                nw[4 * i + 1] = v.y;
                nw[4 * i + 2] = v.z;
                nw[4 * i + 3] = v.w;
            }
        }
    }
    // Normalises in place (when norm_w) and returns the slice's sum.
    __device__ __forceinline__ float finish(const float *norm_w, float eps, uint32_t h, int width) {
        if (norm_w) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < 32; j++) ss += xr[j] * xr[j];
            ss = subwave_sum(ss, width);
            const float inv = 1.0f / sqrtf(ss / (float)h + eps);
#pragma unroll
            for (int j = 0; j < 32; j++) xr[j] = xr[j] * inv * nw[j];
        }
        float xsum = 0.f;
#pragma unroll
        for (int j = 0; j < 32; j++) xsum += xr[j];
        return xsum;
    }
};

constexpr int kGateFR = 4;    // routed ff indices per sub-wave in decode_gateup

// Reduce-scatter of four (gate, up) partial pairs over an lpr-lane sub-wave
// (lpr >= 16): two exchange steps halve the set per step (xor 1, xor 2 via
// quad_perm), then the remaining pair is summed over the lanes sharing
// lane & 3 (row_ror 4 and 8, then permlane xor 16 / 32).  Lane cl < 4 of the
// sub-wave ends with the sums of pair f = 2*(cl & 1) + ((cl >> 1) & 1).
__device__ __forceinline__ int rs4_index(uint32_t cl) { return 2 * (cl & 1) + ((cl >> 1) & 1); }
__device__ __forceinline__ void rs4_pairs(const float *g, const float *u, int lane, uint32_t lpr,
                                          float &go, float &uo) {
    const bool b0 = lane & 1, b1 = (lane >> 1) & 1;
    float g2[2], u2[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const float sg = b0 ? g[i] : g[i + 2], kg = b0 ? g[i + 2] : g[i];
        const float su = b0 ? u[i] : u[i + 2], ku = b0 ? u[i + 2] : u[i];
        g2[i] = kg + dpp_f<kDppQuad1>(sg);
        u2[i] = ku + dpp_f<kDppQuad1>(su);
    }
    const float sg = b1 ? g2[0] : g2[1], kg = b1 ? g2[1] : g2[0];
    const float su = b1 ? u2[0] : u2[1], ku = b1 ? u2[1] : u2[0];
    go = kg + dpp_f<kDppQuad2>(sg);
    uo = ku + dpp_f<kDppQuad2>(su);
    go += dpp_f<kDppRor4>(go);
    uo += dpp_f<kDppRor4>(uo);
    go += dpp_f<kDppRor8>(go);
    uo += dpp_f<kDppRor8>(uo);
    if (lpr >= 32) {
        go = add_xor16(go);
        uo = add_xor16(uo);
    }
    if (lpr >= 64) {
        go = add_xor32(go);
        uo = add_xor32(uo);
    }
}

// Reduce-scatter of two (routed, shared) partial pairs over an lpr-lane
// sub-wave (lpr >= 16): lane cl < 2 ends with pair f = cl & 1.
__device__ __forceinline__ void rs2_pairs(const float *r, const float *sh, int lane, uint32_t lpr,
                                          float &ro, float &so) {
    const bool b0 = lane & 1;
    ro = (b0 ? r[1] : r[0]) + dpp_f<kDppQuad1>(b0 ? r[0] : r[1]);
    so = (b0 ? sh[1] : sh[0]) + dpp_f<kDppQuad1>(b0 ? sh[0] : sh[1]);
    ro += dpp_f<kDppQuad2>(ro);
    so += dpp_f<kDppQuad2>(so);
    ro += dpp_f<kDppRor4>(ro);
    so += dpp_f<kDppRor4>(so);
    ro += dpp_f<kDppRor8>(ro);
    so += dpp_f<kDppRor8>(so);
    if (lpr >= 32) {
        ro = add_xor16(ro);
        so = add_xor16(so);
    }
    if (lpr >= 64) {
        ro = add_xor32(ro);
        so = add_xor32(so);
    }
}

// Writes silu(g)*u of the kGateFR rows of one sub-wave item.
__device__ __forceinline__ void gateup_epilogue(const float *g, const float *u, int lane,
                                                uint32_t lpr, uint32_t rpi, uint32_t sub,
                                                uint32_t cl, uint32_t item, uint32_t nrows,
                                                float *act_row) {
    static_assert(kGateFR == 4, "reduce-scatter layout assumes four rows per sub-wave");
    if (lpr >= 16) {
        float gv, uv;
        rs4_pairs(g, u, lane, lpr, gv, uv);
        if (cl < 4) {
            const uint32_t j = (item * kGateFR + rs4_index(cl)) * rpi + sub;
            // activation (elementwise.metal:8-17)
            if (j < nrows) act_row[j] = gv / (1.0f + expf(-gv)) * uv;
        }
    } else {
#pragma unroll
        for (int f = 0; f < kGateFR; f++) {
            const float gv = subwave_sum(g[f], (int)lpr), uv = subwave_sum(u[f], (int)lpr);
            const uint32_t j = (item * kGateFR + f) * rpi + sub;
            if (j < nrows && cl == 0) act_row[j] = gv / (1.0f + expf(-gv)) * uv;
        }
    }
}
}  // namespace moehip
