// Prefill-sized MoE products on the bf16 matrix cores (v_mfma_f32_32x32x16_bf16).
//
// Token-batched replacement of the reference's per-token expert loop
// (crates/model-runtime/src/execute.rs:208-233): after dispatch, every expert
// runs one grouped GEMM over its contiguous segment of (token, k) pairs.
//
//   to_bf16        x (F32, optionally RMS-normalised) -> bf16 rows
//   tile_schedule  segment sizes -> list of (expert, first pair) M-tiles
//   mfma ROUTER    logits[t, e] = x_t . R_e                   (one segment: all tokens)
//   mfma GATEUP    act[p, j] = silu(x_t . G_e[j]) * (x_t . U_e[j])  (bf16 out)
//   mfma DOWN      y[p, r]  = w_p * (act_p . D_e[r])           (bf16 out)
//   combine16      out[t] = sum_k y[pos(t, k)] (+ shared, + residual)
//
// Block tile 128 pairs x 128 weight rows x 128 K, 4 waves in a 2x2 layout,
// each wave 2x2 MFMA tiles of 32x32.  Weight rows (packed affine codes or
// dense) are dequantised once per block into an LDS tile of bf16; activation
// rows stream straight from global memory into the A operands.  Within a
// 128-wide K block, lane half h feeds k = 64h + 8j + [0, 8) at MFMA step j to
// both operands, so each lane's A row segment is one contiguous 128-byte load.
#include "rowdot.hpp"

namespace moehip {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef uint32_t u32x4m __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kLdsRow = kBK + 8;  // bf16 per LDS row (16-byte pad against bank conflicts)

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

enum { MODE_ROUTER = 0, MODE_GATEUP = 1, MODE_DOWN = 2 };

struct MfmaArgs {
    WDesc w, w2;               // B weights (w2: up for GATEUP)
    const uint16_t *a_rows;    // bf16 A source: xb16 [T, in] (ROUTER/GATEUP) or act16 [P, in]
    const uint32_t *perm;      // GATEUP: pair order; DOWN: pair of each position
    const uint32_t *offsets;   // [E+1] segment offsets (ROUTER: nullptr)
    const uint32_t *tiles;     // [2*max_tiles] (expert, first position); ROUTER: nullptr
    const uint32_t *ntiles;    // number of valid tiles (device)
    const float *route_w;      // DOWN: routing weight of each pair [T*K]
    const float *bias;         // ROUTER: optional logit bias [T, E]
    float *out_f32;            // ROUTER: logits [T, E]
    uint16_t *out_bf16;        // GATEUP: act16 [P, ff]; DOWN: y16 [P, h]
    uint32_t k;                // experts per token (GATEUP: token = perm / k)
    uint32_t m_total;          // ROUTER: number of tokens
};

// ---- B tile: dequantise 64 consecutive K values of one weight row to bf16 --
template <int BITS, int T>
__device__ __forceinline__ void load_b_half(const WDesc &w, uint64_t grow, uint32_t k0, bool ok,
                                            uint32_t *dst /* 32 words = 64 bf16 */) {
    if (!ok) {
#pragma unroll
        for (int i = 0; i < 32; i++) dst[i] = 0u;
        return;
    }
    const uint64_t e0 = grow * w.in + k0;
    if constexpr (BITS == 0) {
        if constexpr (T == 30) {  // bf16 already
            const u32x4m *p = reinterpret_cast<const u32x4m *>(reinterpret_cast<const uint16_t *>(w.data) + e0);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const u32x4m v = __builtin_nontemporal_load(p + i);
                dst[4 * i] = v[0]; dst[4 * i + 1] = v[1]; dst[4 * i + 2] = v[2]; dst[4 * i + 3] = v[3];
            }
        } else if constexpr (T == 1) {
            const u32x4m *p = reinterpret_cast<const u32x4m *>(reinterpret_cast<const uint16_t *>(w.data) + e0);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const u32x4m v = __builtin_nontemporal_load(p + i);
#pragma unroll
                for (int q = 0; q < 4; q++)
                    dst[4 * i + q] = pack_bf16(f16_to_f32(v[q] & 0xffffu), f16_to_f32(v[q] >> 16));
            }
        } else {
            const u32x4m *p = reinterpret_cast<const u32x4m *>(reinterpret_cast<const float *>(w.data) + e0);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const u32x4m v = __builtin_nontemporal_load(p + i);
                dst[2 * i] = pack_bf16(__uint_as_float(v[0]), __uint_as_float(v[1]));
                dst[2 * i + 1] = pack_bf16(__uint_as_float(v[2]), __uint_as_float(v[3]));
            }
        }
    } else {
        constexpr int NW = 2 * BITS;  // packed words for 64 codes
        constexpr int P = 32 / BITS;
        uint32_t words[NW];
        const u32x4m *p = reinterpret_cast<const u32x4m *>(reinterpret_cast<const uint32_t *>(w.data) + e0 / P);
#pragma unroll
        for (int i = 0; i < NW / 4; i++) {
            const u32x4m v = __builtin_nontemporal_load(p + i);
            words[4 * i] = v[0]; words[4 * i + 1] = v[1]; words[4 * i + 2] = v[2]; words[4 * i + 3] = v[3];
        }
        // two 32-code chunks, each inside one group (group >= 32)
        float s[2], b[2];
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const uint64_t g = (e0 + 32 * c) >> w.gshift;
            s[c] = load_scalar<T>(w.scales, g);
            b[c] = load_scalar<T>(w.biases, g);
        }
#pragma unroll
        for (int i = 0; i < NW; i++) {
            float cv[P];
            unpack_word<BITS>(words[i], cv);
            const int c = (i * P) / 32;
#pragma unroll
            for (int j = 0; j < P; j += 2)
                dst[(i * P + j) / 2] = pack_bf16(fmaf(cv[j], s[c], b[c]), fmaf(cv[j + 1], s[c], b[c]));
        }
    }
}

template <int MODE, int BITS, int T>
__global__ __launch_bounds__(256) void grouped_mfma_kernel(MfmaArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t Bs[kBN * kLdsRow];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv & 1, wn = wv >> 1;
    // ---- tile -> (expert, first position, end) ----
    uint32_t e = 0, m0, seg_end;
    if constexpr (MODE == MODE_ROUTER) {
        m0 = blockIdx.x * kBM;
        seg_end = a.m_total;
        if (m0 >= seg_end) return;
    } else {
        if (blockIdx.x >= *a.ntiles) return;
        e = a.tiles[2 * blockIdx.x];
        m0 = a.tiles[2 * blockIdx.x + 1];
        seg_end = a.offsets[e + 1];
    }
    const uint32_t in = a.w.in, out = a.w.out;
    const uint32_t n0 = blockIdx.y * (MODE == MODE_GATEUP ? kBN / 2 : kBN);
    // ---- this lane's two A rows ----
    const uint16_t *arow[2];
    bool aok[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const uint32_t pos = m0 + 64 * wm + 32 * s + (lane & 31);
        aok[s] = pos < seg_end;
        uint64_t src = 0;
        if (aok[s]) {
            if constexpr (MODE == MODE_GATEUP) src = a.perm[pos] / a.k;
            else src = pos;
        }
        arow[s] = a.a_rows + src * in + 64 * (lane >> 5);
    }
    // ---- this thread's B row (dequantised into LDS) ----
    const int br = tid >> 1, bh = tid & 1;
    uint64_t bgrow = 0;
    bool bok;
    bool second = false;  // GATEUP: this row comes from the up weights
    if constexpr (MODE == MODE_GATEUP) {
        const int q = br >> 5;  // 32-row blocks alternate gate / up
        const uint32_t n = n0 + (q >> 1) * 32 + (br & 31);
        bok = n < out;
        bgrow = (uint64_t)e * out + n;
        second = (q & 1) != 0;
    } else {
        const uint32_t n = n0 + br;
        bok = n < out;
        bgrow = (uint64_t)e * out + n;
    }
    f32x16 acc[2][2];
#pragma unroll
    for (int s = 0; s < 2; s++)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[s][t][r] = 0.f;

    for (uint32_t kb = 0; kb < in; kb += kBK) {
        // A fragments: 2 rows x 128 bytes per lane
        u32x4m af[2][8];
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const u32x4m *p = reinterpret_cast<const u32x4m *>(arow[s] + kb);
#pragma unroll
            for (int j = 0; j < 8; j++) af[s][j] = aok[s] ? p[j] : u32x4m{0u, 0u, 0u, 0u};
        }
        // B: 64 values of one row per thread -> LDS
        uint32_t bv[32];
        load_b_half<BITS, T>(second ? a.w2 : a.w, bgrow, kb + 64 * bh, bok, bv);
        u32x4m *bd = reinterpret_cast<u32x4m *>(Bs + br * kLdsRow + 64 * bh);
#pragma unroll
        for (int i = 0; i < 8; i++) bd[i] = u32x4m{bv[4 * i], bv[4 * i + 1], bv[4 * i + 2], bv[4 * i + 3]};
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 8; j++) {
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int col = 64 * wn + 32 * t + (lane & 31);
                const u32x4m b = *reinterpret_cast<const u32x4m *>(Bs + col * kLdsRow + 64 * (lane >> 5) + 8 * j);
#pragma unroll
                for (int s = 0; s < 2; s++)
                    acc[s][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, af[s][j]), __builtin_bit_cast(bf16x8, b), acc[s][t], 0, 0, 0);
            }
        }
        __syncthreads();
    }
    // ---- epilogue: acc[s][t][r] is row 64wm+32s+8(r/4)+4(lane/32)+(r%4), col 64wn+32t+lane%32 ----
#pragma unroll
    for (int s = 0; s < 2; s++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const uint32_t pos = m0 + 64 * wm + 32 * s + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (pos >= seg_end) continue;
            if constexpr (MODE == MODE_GATEUP) {
                const uint32_t n = n0 + 32 * wn + (lane & 31);
                if (n < out) {
                    const float g = acc[s][0][r], u = acc[s][1][r];
                    // activation (elementwise.metal:8-17)
                    const float act = g / (1.0f + expf(-g)) * u;
                    a.out_bf16[(uint64_t)pos * out + n] = (uint16_t)(pack_bf16(act, 0.f) & 0xffffu);
                }
            } else {
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const uint32_t n = n0 + 64 * wn + 32 * t + (lane & 31);
                    if (n >= out) continue;
                    const float v = acc[s][t][r];
                    if constexpr (MODE == MODE_ROUTER) {
                        const uint64_t o = (uint64_t)pos * out + n;
                        a.out_f32[o] = a.bias ? v + a.bias[o] : v;
                    } else {
                        const float wk = a.route_w[a.perm[pos]];
                        a.out_bf16[(uint64_t)pos * out + n] = (uint16_t)(pack_bf16(v * wk, 0.f) & 0xffffu);
                    }
                }
            }
        }
    }
}

// x (F32 [T, h]) -> bf16, optionally RMS-normalised first
// (elementwise.metal:31-46 / tensor_core::rms_norm, lib.rs:64-70).
__global__ __launch_bounds__(64) void to_bf16_kernel(const float *__restrict__ x,
                                                     const float *__restrict__ norm_w, float eps,
                                                     uint32_t h, uint16_t *__restrict__ y,
                                                     float *__restrict__ xn) {
    const uint64_t row = blockIdx.x;
    const float *xr = x + row * h;
    float inv = 1.f;
    if (norm_w) {
        float ss = 0.f;
        for (uint32_t i = threadIdx.x; i < h; i += 64) ss += xr[i] * xr[i];
        ss = wave_sum(ss);
        inv = 1.0f / sqrtf(ss / (float)h + eps);
    }
    for (uint32_t i = 2 * threadIdx.x; i < h; i += 128) {
        float v0 = xr[i], v1 = xr[i + 1];
        if (norm_w) {
            v0 = v0 * inv * norm_w[i];
            v1 = v1 * inv * norm_w[i + 1];
            if (xn) {
                xn[row * h + i] = v0;
                xn[row * h + i + 1] = v1;
            }
        }
        reinterpret_cast<uint32_t *>(y + row * h)[i / 2] = pack_bf16(v0, v1);
    }
}

// Same conversion with 8 elements per thread (two 16-byte loads, one 16-byte
// bf16 store), a block of up to 256 threads per row; h % 8 == 0.
__global__ __launch_bounds__(256) void to_bf16v_kernel(const float *__restrict__ x,
                                                      const float *__restrict__ norm_w, float eps,
                                                      uint32_t h, uint16_t *__restrict__ y,
                                                      float *__restrict__ xn) {
    __shared__ float part[4];
    const uint64_t row = blockIdx.x;
    const float *xr = x + row * h;
    float inv = 1.f;
    if (norm_w) {
        float ss = 0.f;
        for (uint32_t i = threadIdx.x; i < h; i += blockDim.x) ss += xr[i] * xr[i];
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
        __syncthreads();
        ss = 0.f;
        for (uint32_t w = 0; w < blockDim.x / 64; w++) ss += part[w];
        inv = 1.0f / sqrtf(ss / (float)h + eps);
    }
    for (uint32_t i = 8 * threadIdx.x; i < h; i += 8 * blockDim.x) {
        const float4 a = *reinterpret_cast<const float4 *>(xr + i);
        const float4 b = *reinterpret_cast<const float4 *>(xr + i + 4);
        float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        if (norm_w) {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = v[j] * inv * norm_w[i + j];
            if (xn) {
                float4 *d = reinterpret_cast<float4 *>(xn + row * h + i);
                d[0] = make_float4(v[0], v[1], v[2], v[3]);
                d[1] = make_float4(v[4], v[5], v[6], v[7]);
            }
        }
        *reinterpret_cast<u32x4m *>(y + row * h + i) =
            u32x4m{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7])};
    }
}

// Tile list: M-tiles of `tm` positions over every non-empty expert segment.
__global__ __launch_bounds__(64) void tile_schedule_kernel(const uint32_t *__restrict__ offsets,
                                                           uint32_t E, uint32_t tm,
                                                           uint32_t *__restrict__ tiles,
                                                           uint32_t *__restrict__ ntiles) {
    const int lane = threadIdx.x;
    uint32_t base = 0;
    for (uint32_t e0 = 0; e0 < E; e0 += 64) {
        const uint32_t e = e0 + lane;
        uint32_t nt = 0, beg = 0;
        if (e < E) {
            beg = offsets[e];
            nt = (offsets[e + 1] - beg + tm - 1) / tm;
        }
        // exclusive prefix of nt over the wave
        uint32_t incl = nt;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        const uint32_t first = base + incl - nt;
        for (uint32_t i = 0; i < nt; i++) {
            tiles[2 * (first + i)] = e;
            tiles[2 * (first + i) + 1] = beg + i * tm;
        }
        base += __shfl(incl, 63, 64);
    }
    if (lane == 0) *ntiles = base;
}

// out[t, i] = sum_k w[t,k] * y16[pos[t*K+k], i] (+ sh_out[t, i]/(1+exp(-sh_gate[t]))) (+ resid[t, i])
__global__ __launch_bounds__(256) void combine16_kernel(const uint16_t *__restrict__ y16,
                                                        const uint32_t *__restrict__ pos,
                                                        const float *__restrict__ wts,
                                                        uint32_t K, const float *__restrict__ sh_out,
                                                        const float *__restrict__ sh_gate,
                                                        const float *__restrict__ resid,
                                                        float *__restrict__ out, uint32_t h) {
    const uint32_t t = blockIdx.y;
    for (uint32_t i = 2 * (blockIdx.x * 256 + threadIdx.x); i < h; i += 2 * 256 * gridDim.x) {
        float v0 = 0.f, v1 = 0.f;
        // mix (elementwise.metal:47-57): sum over k ascending of w[k] * y_k
        for (uint32_t k = 0; k < K; k++) {
            const uint32_t w = reinterpret_cast<const uint32_t *>(y16 + (uint64_t)pos[(uint64_t)t * K + k] * h)[i / 2];
            const float wk = wts[(uint64_t)t * K + k];
            v0 += bf16_lo(w) * wk;
            v1 += bf16_hi(w) * wk;
        }
        const uint64_t o = (uint64_t)t * h + i;
        if (sh_out) {
            const float d = 1.0f + expf(-sh_gate[t]);
            v0 = v0 + sh_out[o] / d;
            v1 = v1 + sh_out[o + 1] / d;
        }
        if (resid) {
            v0 = resid[o] + v0;
            v1 = resid[o + 1] + v1;
        }
        out[o] = v0;
        out[o + 1] = v1;
    }
}

// ------------------------------------------------------------------ host --
bool mfma_supported(const WDesc &w) {
    if (w.in % kBK) return false;
    if (w.bits == 0) return w.type == 0 || w.type == 1 || w.type == 30;
    return (w.bits == 2 || w.bits == 4 || w.bits == 8) && (w.type == 0 || w.type == 1 || w.type == 30);
}

template <int MODE>
struct MfmaLaunch {
    Prof *p;
    const char *name;
    hipStream_t s;
    const MfmaArgs &a;
    dim3 grid;
    template <int BITS, int T>
    hipError_t operator()() {
        return launch_kernel(p, name, grouped_mfma_kernel<MODE, BITS, T>, grid, dim3(256), 0, s, a);
    }
};

hipError_t launch_to_bf16(Prof *p, hipStream_t s, const float *x, const float *norm_w, float eps,
                          uint32_t tokens, uint32_t h, uint16_t *y, float *xn) {
    const bool vec = h % 8 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) |
                                     reinterpret_cast<uintptr_t>(xn)) & 15u) == 0;
    if (vec) {
        const uint32_t threads = h / 8 < 256 ? ((h / 8 + 63) / 64) * 64 : 256;
        return launch_kernel(p, "to_bf16", to_bf16v_kernel, dim3(tokens), dim3(threads), 0, s, x,
                             norm_w, eps, h, y, xn);
    }
    return launch_kernel(p, "to_bf16", to_bf16_kernel, dim3(tokens), dim3(64), 0, s, x, norm_w, eps,
                         h, y, xn);
}

hipError_t launch_mfma_router(Prof *p, hipStream_t s, const WDesc &r, const uint16_t *xb16,
                              uint32_t tokens, const float *bias, float *logits) {
    MfmaArgs a{};
    a.w = r;
    a.a_rows = xb16;
    a.bias = bias;
    a.out_f32 = logits;
    a.m_total = tokens;
    dim3 grid((tokens + kBM - 1) / kBM, (r.out + kBN - 1) / kBN);
    return dispatch_kind(r, MfmaLaunch<MODE_ROUTER>{p, "mfma_router", s, a, grid});
}

hipError_t launch_mfma_experts(Prof *p, hipStream_t s, const WDesc &gate, const WDesc &up,
                               const WDesc &down, const uint16_t *xb16, const uint32_t *offsets,
                               const uint32_t *perm, const float *route_w, uint32_t k,
                               uint32_t pairs, uint32_t *tiles, uint32_t *ntiles,
                               uint16_t *act16, uint16_t *y16) {
    const uint32_t E = gate.experts;
    hipError_t e = launch_kernel(p, "tile_schedule", tile_schedule_kernel, dim3(1), dim3(64), 0, s,
                                 offsets, E, gemm_tile_rows(), tiles, ntiles);
    if (e != hipSuccess) return e;
    e = launch_grouped_gemm(p, s, 0, gate, up, xb16, perm, offsets, tiles, ntiles, nullptr, k, act16);
    if (e != hipSuccess) return e;
    return launch_grouped_gemm(p, s, 1, down, down, act16, perm, offsets, tiles, ntiles, route_w, k, y16);
}

// Same combine with 8 columns per thread (16-byte row loads, all K rows of a
// group of up to 8 issued before the accumulation; the sum still runs over k
// ascending).  One block of h/8 threads per token; h % 8 == 0.
constexpr uint32_t kCombKMax = 8;
__global__ __launch_bounds__(256) void combine16v_kernel(const uint16_t *__restrict__ y16,
                                                         const uint32_t *__restrict__ pos,
                                                         const float *__restrict__ wts, uint32_t K,
                                                         const float *__restrict__ sh_out,
                                                         const float *__restrict__ sh_gate,
                                                         const float *__restrict__ resid,
                                                         float *__restrict__ out, uint32_t h) {
    const uint32_t t = blockIdx.y;
    const uint32_t i = 8 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= h) return;
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = 0.f;
    // mix (elementwise.metal:47-57): sum over k ascending of w[k] * y_k
    for (uint32_t k0 = 0; k0 < K; k0 += kCombKMax) {
        const uint32_t n = min(kCombKMax, K - k0);
        u32x4m r[kCombKMax];
        float w[kCombKMax];
#pragma unroll
        for (uint32_t k = 0; k < kCombKMax; k++) {
            if (k < n) {
                const uint64_t pk = (uint64_t)t * K + k0 + k;
                r[k] = *reinterpret_cast<const u32x4m *>(y16 + (uint64_t)pos[pk] * h + i);
                w[k] = wts[pk];
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kCombKMax; k++) {
            if (k < n) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    v[2 * q] += bf16_lo(r[k][q]) * w[k];
                    v[2 * q + 1] += bf16_hi(r[k][q]) * w[k];
                }
            }
        }
    }
    const uint64_t o = (uint64_t)t * h + i;
    if (sh_out) {
        const float d = 1.0f + expf(-sh_gate[t]);
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = v[j] + sh_out[o + j] / d;
    }
    if (resid) {
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = resid[o + j] + v[j];
    }
    float4 *dst = reinterpret_cast<float4 *>(out + o);
    dst[0] = make_float4(v[0], v[1], v[2], v[3]);
    dst[1] = make_float4(v[4], v[5], v[6], v[7]);
}

hipError_t launch_combine16(Prof *p, hipStream_t s, const uint16_t *y16, const uint32_t *pos,
                            const float *wts, uint32_t k, const float *sh_out, const float *sh_gate,
                            const float *resid, float *out, uint32_t tokens, uint32_t h) {
    const bool vec = h % 8 == 0 && (reinterpret_cast<uintptr_t>(y16) & 15u) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
    if (vec) {
        const uint32_t threads = h / 8 < 256 ? ((h / 8 + 63) / 64) * 64 : 256;
        dim3 grid((h / 8 + threads - 1) / threads, tokens);
        return launch_kernel(p, "combine16", combine16v_kernel, grid, dim3(threads), 0, s, y16, pos,
                             wts, k, sh_out, sh_gate, resid, out, h);
    }
    dim3 grid((h / 2 + 255) / 256, tokens);
    return launch_kernel(p, "combine16", combine16_kernel, grid, dim3(256), 0, s, y16, pos, wts, k,
                         sh_out, sh_gate, resid, out, h);
}

}  // namespace moehip
