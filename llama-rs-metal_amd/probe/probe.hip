// Measurement and synthetic-data helpers of bench.py (libmoe_probe.so).  Not
// part of the MoE path or of include/moe_hip.h:
//   probe_mfma_peak   an MFMA-only loop: the dense bf16 (v_mfma_f32_32x32x16_bf16)
//                     or F32 (v_mfma_f32_32x32x2_f32) matrix-core rate of this GPU,
//                     the peaks the prefill fractions are priced against
//   probe_hbm_read    a streaming read of a buffer far larger than the 256 MB
//                     Infinity Cache: the HBM read rate decode is priced against
//   probe_synth_*     the seeded synthetic weights of the benchmark
//                     configurations, generated on the GPU: the LCG stream of
//                     hip_backend.synth.normal (the reference fixture LCG,
//                     crates/llama-rs/tests/common/mod.rs:86-97) through
//                     Box-Muller, and the affine quantizer of
//                     hip_backend.synth.quantize_affine, so multi-GB expert
//                     tensors need no host generation or upload
// Every function returns a hipError_t (0 = success) and synchronises before
// returning.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint64_t kLcgA = 6364136223846793005ull;  // s = s * A + 1

// ------------------------------------------------------------- MFMA peak --
constexpr int kChains = 4;  // independent accumulators per wave

__global__ __launch_bounds__(256) void mfma_bf16_kernel(int iters, float *out) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    bf16x8 a, b;
    for (int i = 0; i < 8; i++) {
        a[i] = (__bf16)(float)((t + i) & 7);
        b[i] = (__bf16)(float)((t * 3 + i) & 7);
    }
    f32x16 acc[kChains] = {};
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int c = 0; c < kChains; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < kChains; c++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += acc[c][r];
    out[t] = s;
}

__global__ __launch_bounds__(256) void mfma_f32_kernel(int iters, float *out) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const float a = (float)(t & 7), b = (float)((t * 3) & 7);
    f32x16 acc[kChains] = {};
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int c = 0; c < kChains; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[c], 0, 0, 0);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < kChains; c++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += acc[c][r];
    out[t] = s;
}

// -------------------------------------------------------------- HBM read --
constexpr int kReadUnroll = 8;  // 16-byte loads in flight per thread

__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4 *__restrict__ p, uint64_t n16,
                                                       uint32_t *out) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + (kReadUnroll - 1) * stride < n16; i += kReadUnroll * stride) {
        u32x4 v[kReadUnroll];
#pragma unroll
        for (int u = 0; u < kReadUnroll; u++) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < kReadUnroll; u++) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    for (; i < n16; i += stride) {
        const u32x4 v = p[i];
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    out[(uint64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

// ------------------------------------------------------ synthetic weights --
// LCG state after `steps` more steps from s (jump-ahead by squaring:
// s_{k+m} = A^m s_k + c_m with c_{2m} = c_m (A^m + 1)).
__device__ uint64_t lcg_skip(uint64_t s, uint64_t steps) {
    uint64_t a = kLcgA, c = 1, am = 1, cm = 0;
    while (steps) {
        if (steps & 1) {
            am *= a;
            cm = cm * a + c;
        }
        c *= a + 1;
        a *= a;
        steps >>= 1;
    }
    return am * s + cm;
}

// Values 2j, 2j + 1 of the stream come from states 2j + 1 and 2j + 2 after
// the seed: u = ((s >> 32) + 0.5) / 2^32 (exact in double, then rounded to
// float), Box-Muller in float, mean + std * z.  The host generator evaluates
// Box-Muller in double; in float the values agree to about 1e-6 relative
// (a double evaluation costs ~250 FP64 operations per value, minutes for the
// 48-layer stack's weights).
__device__ __forceinline__ void normal_pair(uint64_t &s, float mean, float sd, float &z0, float &z1) {
    s = s * kLcgA + 1;
    const float u1 = (float)(((double)(s >> 32) + 0.5) * (1.0 / 4294967296.0));
    s = s * kLcgA + 1;
    const float u2 = (float)(((double)(s >> 32) + 0.5) * (1.0 / 4294967296.0));
    const float r = sqrtf(-2.0f * logf(u1)), t = 6.28318530717958647692f * u2;
    float sn, cs;
    sincosf(t, &sn, &cs);
    z0 = mean + sd * (r * cs);
    z1 = mean + sd * (r * sn);
}

__global__ __launch_bounds__(256) void synth_normal_kernel(float *out, uint64_t n, uint64_t seed,
                                                           float mean, float sd) {
    // thread: 64 consecutive values (32 pairs) from one jump-ahead
    const uint64_t j0 = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 64;
    if (j0 >= n) return;
    uint64_t s = lcg_skip(seed, j0);
    for (uint64_t j = j0; j < j0 + 64 && j < n; j += 2) {
        float z0, z1;
        normal_pair(s, mean, sd, z0, z1);
        out[j] = z0;
        if (j + 1 < n) out[j + 1] = z1;
    }
}

// value rounded to the scale dtype (0 F32, 1 F16, 30 BF16, round to nearest
// even), with its stored 16-bit pattern
__device__ __forceinline__ float round_scale(float v, uint32_t type, uint16_t *bits) {
    if (type == 30) {
        uint32_t b = __float_as_uint(v);
        b += 0x7fffu + ((b >> 16) & 1u);
        *bits = (uint16_t)(b >> 16);
        return __uint_as_float((uint32_t)*bits << 16);
    }
    if (type == 1) {
        const __half h = __float2half_rn(v);
        *bits = __half_as_ushort(h);
        return __half2float(h);
    }
    *bits = 0;
    return v;
}

// One thread per quantization group: the group's normal values, then
// scale = (max - min) / (2^bits - 1) and bias = min rounded to the scale
// dtype, codes rint((w - bias) / scale) clamped, packed low bits first.
template <int BITS, int GROUP>
__global__ __launch_bounds__(256) void synth_affine_kernel(uint32_t *codes, void *scales, void *biases,
                                                           uint64_t groups, uint32_t type, uint64_t seed,
                                                           float mean, float sd) {
    constexpr uint32_t bits = BITS, group = GROUP;
    const uint64_t g = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    float w[GROUP];
    uint64_t s = lcg_skip(seed, g * group);
#pragma unroll
    for (uint32_t i = 0; i < group; i += 2) normal_pair(s, mean, sd, w[i], w[i + 1]);
    float mn = w[0], mx = w[0];
#pragma unroll
    for (uint32_t i = 1; i < group; i++) {
        mn = fminf(mn, w[i]);
        mx = fmaxf(mx, w[i]);
    }
    const uint32_t qmax = (1u << bits) - 1u;
    uint16_t sb, bb;
    const float sc = round_scale((mx - mn) / (float)qmax, type, &sb);
    const float bi = round_scale(mn, type, &bb);
    if (type == 0) {
        reinterpret_cast<float *>(scales)[g] = sc;
        reinterpret_cast<float *>(biases)[g] = bi;
    } else {
        reinterpret_cast<uint16_t *>(scales)[g] = sb;
        reinterpret_cast<uint16_t *>(biases)[g] = bb;
    }
    constexpr uint32_t per_word = 32 / bits;
    uint32_t *dst = codes + g * group / per_word;
#pragma unroll
    for (uint32_t wd = 0; wd < group / per_word; wd++) {
        uint32_t word = 0;
#pragma unroll
        for (uint32_t k = 0; k < per_word; k++) {
            float q = sc > 0.f ? rintf((w[wd * per_word + k] - bi) / sc) : 0.f;
            q = fminf(fmaxf(q, 0.f), (float)qmax);
            word |= ((uint32_t)q & qmax) << (k * bits);
        }
        dst[wd] = word;
    }
}

int cus() {
    int dev = 0, n = 256;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    return n;
}

}  // namespace

extern "C" {

// kind 0: bf16 (v_mfma_f32_32x32x16_bf16, 32768 FLOP each); kind 1: F32
// (v_mfma_f32_32x32x2_f32, 4096 FLOP each).  Eight 4-wave blocks per CU;
// the best of `reps` timed launches after one warm-up.
int probe_mfma_peak(int kind, int iters, int reps, double *tflops) {
    const uint32_t blocks = (uint32_t)cus() * 8, threads = 256;
    float *out = nullptr;
    hipError_t e = hipMalloc(&out, (size_t)blocks * threads * sizeof(float));
    if (e != hipSuccess) return e;
    hipEvent_t a = nullptr, b = nullptr;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    double best = 0.0;
    for (int r = 0; r <= reps && e == hipSuccess; r++) {
        (void)hipEventRecord(a, nullptr);
        if (kind == 0)
            hipLaunchKernelGGL(mfma_bf16_kernel, dim3(blocks), dim3(threads), 0, nullptr, iters, out);
        else
            hipLaunchKernelGGL(mfma_f32_kernel, dim3(blocks), dim3(threads), 0, nullptr, iters, out);
        (void)hipEventRecord(b, nullptr);
        e = hipEventSynchronize(b);
        if (e == hipSuccess) e = hipGetLastError();
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, a, b);
        const double flop = (double)blocks * (threads / 64) * iters * kChains * (kind == 0 ? 32768.0 : 4096.0);
        if (r > 0 && ms > 0.f && flop / (ms * 1e-3) / 1e12 > best) best = flop / (ms * 1e-3) / 1e12;
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    (void)hipFree(out);
    *tflops = best;
    return e;
}

// Streaming read of `bytes` (a multiple of 16) of fresh device memory, the
// best of `reps` timed passes after one warm-up pass; GB/s of bytes read.
int probe_hbm_read(uint64_t bytes, int reps, double *gbps) {
    void *buf = nullptr;
    uint32_t *out = nullptr;
    const uint32_t blocks = (uint32_t)cus() * 16, threads = 256;
    hipError_t e = hipMalloc(&buf, bytes);
    if (e == hipSuccess) e = hipMalloc(&out, (size_t)blocks * threads * 4);
    if (e == hipSuccess) e = hipMemset(buf, 1, bytes);
    hipEvent_t a = nullptr, b = nullptr;
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    double best = 0.0;
    for (int r = 0; r <= reps && e == hipSuccess; r++) {
        (void)hipEventRecord(a, nullptr);
        hipLaunchKernelGGL(hbm_read_kernel, dim3(blocks), dim3(threads), 0, nullptr,
                           static_cast<const u32x4 *>(buf), bytes / 16, out);
        (void)hipEventRecord(b, nullptr);
        e = hipEventSynchronize(b);
        if (e == hipSuccess) e = hipGetLastError();
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, a, b);
        if (r > 0 && ms > 0.f && bytes / (ms * 1e-3) / 1e9 > best) best = bytes / (ms * 1e-3) / 1e9;
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    if (out) (void)hipFree(out);
    if (buf) (void)hipFree(buf);
    *gbps = best;
    return e;
}

// n values of the stream hip_backend.synth.normal(seed, n, mean, std) draws
// (Box-Muller in float) into device memory.
int probe_synth_normal(float *out, uint64_t n, uint64_t seed, float mean, float sd) {
    const uint64_t threads = (n + 63) / 64;
    hipLaunchKernelGGL(synth_normal_kernel, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, nullptr, out,
                       n, seed, mean, sd);
    hipError_t e = hipGetLastError();
    return e != hipSuccess ? e : hipDeviceSynchronize();
}

// hip_backend.synth.quantize_affine of probe_synth_normal's values (bits,
// group, scale_type) into device memory: codes (n * bits / 8 bytes), scales
// and biases (n / group values of the scale type).
int probe_synth_affine(void *codes, void *scales, void *biases, uint64_t n, uint32_t bits, uint32_t group,
                       uint32_t scale_type, uint64_t seed, float mean, float sd) {
    if ((bits != 2 && bits != 4 && bits != 8) || (group != 32 && group != 64 && group != 128) || n % group)
        return hipErrorInvalidValue;
    const uint64_t groups = n / group;
    const dim3 grid((uint32_t)((groups + 255) / 256)), block(256);
    uint32_t *c = static_cast<uint32_t *>(codes);
#define SYNTH_CASE(B, G)                                                                                \
    if (bits == B && group == G)                                                                        \
        hipLaunchKernelGGL((synth_affine_kernel<B, G>), grid, block, 0, nullptr, c, scales, biases, groups, \
                           scale_type, seed, mean, sd);
    SYNTH_CASE(2, 32) SYNTH_CASE(2, 64) SYNTH_CASE(2, 128)
    SYNTH_CASE(4, 32) SYNTH_CASE(4, 64) SYNTH_CASE(4, 128)
    SYNTH_CASE(8, 32) SYNTH_CASE(8, 64) SYNTH_CASE(8, 128)
#undef SYNTH_CASE
    hipError_t e = hipGetLastError();
    return e != hipSuccess ? e : hipDeviceSynchronize();
}

}  // extern "C"
