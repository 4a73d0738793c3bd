// Prefill (token-batched) pieces around the grouped MFMA GEMMs of k_gemm.hip.
//
// Token-batched replacement of the reference's per-token expert loop
// (crates/model-runtime/src/execute.rs:208-233): after dispatch every expert's
// (token, k) pairs form one contiguous segment, and each segment runs one GEMM.
//
//   to_bf16        x (F32, optionally RMS-normalised) -> bf16 rows (the GEMMs' A)
//   tile_schedule  segment sizes -> list of (expert, first pair) M-tiles (the
//                  dispatch kernel writes the same list itself where the
//                  experts fit its LDS; this kernel serves the other cases)
//   identity_schedule  one segment of all rows (the shared expert on the grouped GEMM)
//   combine16      out[t] = sum_k w[t, k] * y[pos(t, k)] (+ shared, + residual)

#include "rowdot.hpp"

namespace moehip {

typedef uint32_t u32x4m __attribute__((ext_vector_type(4)));
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

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

// The schedule of one segment of all T rows (the shared expert's products
// on the grouped GEMM): offsets {0, T}, M-tiles (0, tm i), their count.
__global__ __launch_bounds__(256) void identity_schedule_kernel(uint32_t T, uint32_t tm,
                                                                uint32_t *__restrict__ offsets,
                                                                uint32_t *__restrict__ tiles,
                                                                uint32_t *__restrict__ ntiles) {
    const uint32_t n = (T + tm - 1) / tm;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        tiles[2 * i] = 0;
        tiles[2 * i + 1] = i * tm;
    }
    if (threadIdx.x == 0) {
        offsets[0] = 0;
        offsets[1] = T;
        *ntiles = n;
    }
}

// The shared expert's gate input of token t: the sum of ks partial sums over
// K ranges, in range order.
__device__ __forceinline__ float gate_input(const float *g, uint32_t ks, uint32_t tokens, uint32_t t) {
    float v = g[t];
    for (uint32_t r = 1; r < ks; r++) v += g[(uint64_t)r * tokens + t];
    return v;
}

// The shared expert's output element o: F32 (sh_out) or bf16 (sh16).
__device__ __forceinline__ float shared_value(const float *sh_out, const uint16_t *sh16, uint64_t o) {
    return sh16 ? __uint_as_float((uint32_t)sh16[o] << 16) : sh_out[o];
}

// out[t, i] = sum_k w[t,k] * y16[pos[t*K+k], i] (+ sh[t, i]/(1+exp(-sh_gate[t]))) (+ resid[t, i])
__global__ __launch_bounds__(256) void combine16_kernel(const uint16_t *__restrict__ y16,
                                                        const uint32_t *__restrict__ pos,
                                                        const float *__restrict__ wts,
                                                        uint32_t K, const float *__restrict__ sh_out,
                                                        const uint16_t *__restrict__ sh16,
                                                        const float *__restrict__ sh_gate,
                                                        const float *__restrict__ resid,
                                                        float *__restrict__ out, uint32_t h, uint32_t gks) {
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
        if (sh_out || sh16) {
            const float d = 1.0f + expf(-gate_input(sh_gate, gks, gridDim.y, t));
            v0 = v0 + shared_value(sh_out, sh16, o) / d;
            v1 = v1 + shared_value(sh_out, sh16, o + 1) / d;
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

hipError_t launch_tile_schedule(Prof *p, hipStream_t s, const uint32_t *offsets, uint32_t experts,
                                uint32_t tm, uint32_t *tiles, uint32_t *ntiles) {
    return launch_kernel(p, "tile_schedule", tile_schedule_kernel, dim3(1), dim3(64), 0, s, offsets,
                         experts, tm, tiles, ntiles);
}

hipError_t launch_mfma_experts(Prof *p, hipStream_t s, const WDesc &gate, const WDesc &up,
                               const WDesc &down, const PackedW &pg, const PackedW &pu,
                               const PackedW &pd, const uint16_t *xb16, uint32_t tokens,
                               const uint32_t *offsets, const uint32_t *perm, uint32_t k,
                               uint32_t *tiles, uint32_t *ntiles, uint16_t *act16, uint16_t *y16,
                               const SharedSeg *sh_gu, const SharedSeg *sh_dn) {
    hipError_t e = launch_grouped_gemm(p, s, 0, gate, up, pg, pu, xb16, tokens, perm, offsets, tiles, ntiles, k,
                                       act16, nullptr, sh_gu);
    if (e != hipSuccess) return e;
    const uint64_t rows = (uint64_t)tokens * k + (sh_dn ? tokens : 0u);
    return launch_grouped_gemm(p, s, 1, down, down, pd, pd, act16, rows, perm, offsets, tiles, ntiles, k, y16,
                               nullptr, sh_dn);
}

// Same combine with 8 columns per thread (16-byte row loads, all K rows of a
// group of up to 8 issued before the accumulation; the sum still runs over k
// ascending).  One block of h/8 threads per token; h % 8 == 0.
constexpr uint32_t kCombKMax = 8;
__global__ __launch_bounds__(256) void combine16v_kernel(const uint16_t *__restrict__ y16,
                                                         const uint32_t *__restrict__ pos,
                                                         const float *__restrict__ wts, uint32_t K,
                                                         const float *__restrict__ sh_out,
                                                         const uint16_t *__restrict__ sh16,
                                                         const float *__restrict__ sh_gate,
                                                         const float *__restrict__ resid,
                                                         float *__restrict__ out, uint32_t h, uint32_t gks) {
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
    if (sh16) {
        const float d = 1.0f + expf(-gate_input(sh_gate, gks, gridDim.y, t));
        const u32x4m r = *reinterpret_cast<const u32x4m *>(sh16 + o);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            v[2 * q] = v[2 * q] + bf16_lo(r[q]) / d;
            v[2 * q + 1] = v[2 * q + 1] + bf16_hi(r[q]) / d;
        }
    } else if (sh_out) {
        const float d = 1.0f + expf(-gate_input(sh_gate, gks, gridDim.y, t));
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
                            const float *wts, uint32_t k, const float *sh_out, const uint16_t *sh16,
                            const float *sh_gate, const float *resid, float *out, uint32_t tokens,
                            uint32_t h, uint32_t gate_ks) {
    const bool vec = h % 8 == 0 &&
                     ((reinterpret_cast<uintptr_t>(y16) | reinterpret_cast<uintptr_t>(out) |
                       reinterpret_cast<uintptr_t>(sh16)) & 15u) == 0;
    if (vec) {
        const uint32_t threads = h / 8 < 256 ? ((h / 8 + 63) / 64) * 64 : 256;
        dim3 grid((h / 8 + threads - 1) / threads, tokens);
        return launch_kernel(p, "combine16", combine16v_kernel, grid, dim3(threads), 0, s, y16, pos,
                             wts, k, sh_out, sh16, sh_gate, resid, out, h, gate_ks);
    }
    dim3 grid((h / 2 + 255) / 256, tokens);
    return launch_kernel(p, "combine16", combine16_kernel, grid, dim3(256), 0, s, y16, pos, wts, k,
                         sh_out, sh16, sh_gate, resid, out, h, gate_ks);
}

hipError_t launch_identity_schedule(Prof *p, hipStream_t s, uint32_t rows, uint32_t tm, uint32_t *offsets,
                                    uint32_t *tiles, uint32_t *ntiles) {
    return launch_kernel(p, "identity_schedule", identity_schedule_kernel, dim3(1), dim3(256), 0, s, rows,
                         tm, offsets, tiles, ntiles);
}

}  // namespace moehip
