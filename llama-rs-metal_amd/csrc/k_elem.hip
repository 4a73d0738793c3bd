// Element-wise epilogues of the MoE block
// (crates/metal-backend/src/shaders/elementwise.metal) and the combine that
// replaces mix + gate_scalar + add in the token-batched path.
#include "device_common.hpp"

namespace moehip {

constexpr int kEw = 256;

static inline dim3 ew_grid(uint64_t n) {
    uint64_t b = (n + kEw - 1) / kEw;
    if (b > 65535u * 16u) b = 65535u * 16u;
    return dim3((uint32_t)(b ? b : 1));
}

// activation (elementwise.metal:8-17): y = a/(1+exp(-a))*b; exact in-place allowed.
__global__ void swiglu_kernel(const float *a, const float *b, float *y, uint64_t n) {
    for (uint64_t i = blockIdx.x * (uint64_t)kEw + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kEw) {
        const float v = a[i];
        y[i] = v / (1.0f + expf(-v)) * b[i];
    }
}

// mix (elementwise.metal:47-57): y[i] = sum_{k ascending} x[k*n+i]*w[k].
__global__ void mix_kernel(const float *__restrict__ x, const float *__restrict__ w, uint32_t k,
                           uint64_t n, float *__restrict__ y) {
    for (uint64_t i = blockIdx.x * (uint64_t)kEw + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kEw) {
        float v = 0.f;
        for (uint32_t kk = 0; kk < k; kk++) v += x[(uint64_t)kk * n + i] * w[kk];
        y[i] = v;
    }
}

// gate_scalar (elementwise.metal:65-72): y = x/(1+exp(-g[0])).
__global__ void gate_scalar_kernel(const float *x, const float *g, float *y, uint64_t n) {
    const float d = 1.0f + expf(-g[0]);
    for (uint64_t i = blockIdx.x * (uint64_t)kEw + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kEw)
        y[i] = x[i] / d;
}

// add (elementwise.metal:1-7).
__global__ void add_kernel(const float *a, const float *b, float *y, uint64_t n) {
    for (uint64_t i = blockIdx.x * (uint64_t)kEw + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kEw)
        y[i] = a[i] + b[i];
}

__global__ void copy_kernel(const float *__restrict__ s, float *__restrict__ d, uint64_t n) {
    for (uint64_t i = blockIdx.x * (uint64_t)kEw + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kEw)
        d[i] = s[i];
}

// norm (elementwise.metal:31-46): one wave per head,
// y[head*n + i] = x[head*stride + i] * rsqrt(mean(x^2) + eps) * w[i].
template <int T>
__global__ __launch_bounds__(64) void norm_kernel(const float *__restrict__ x, const void *w,
                                                  float *__restrict__ y, uint32_t n,
                                                  uint32_t stride, float eps) {
    const uint32_t head = blockIdx.x;
    const int lane = threadIdx.x;
    const float *xr = x + (uint64_t)head * stride;
    float s = 0.f;
    for (uint32_t i = lane; i < n; i += 64) {
        const float v = xr[i];
        s += v * v;
    }
    s = wave_sum(s);
    const float inv = 1.0f / sqrtf(s / (float)n + eps);
    for (uint32_t i = lane; i < n; i += 64)
        y[(uint64_t)head * n + i] = xr[i] * inv * load_scalar<T>(w, i);
}

// out[t, i] = sum_k w[t,k] * yexp[pos[t*K+k]*h + i]          (mix, k ascending)
//           + sh_out[t, i] / (1 + exp(-sh_gate[t]))             (gate_scalar + add)
//           + resid[t, i]                                      (residual add)
__global__ void combine_kernel(const float *__restrict__ yexp, const uint32_t *__restrict__ pos,
                               const float *__restrict__ w, uint32_t K,
                               const float *__restrict__ sh_out, const float *__restrict__ sh_gate,
                               const float *__restrict__ resid, float *__restrict__ out,
                               uint32_t tokens, uint32_t h) {
    const uint32_t t = blockIdx.y;
    for (uint32_t i = blockIdx.x * kEw + threadIdx.x; i < h; i += gridDim.x * kEw) {
        float v = 0.f;
        for (uint32_t k = 0; k < K; k++)
            v += yexp[(uint64_t)pos[(uint64_t)t * K + k] * h + i] * w[(uint64_t)t * K + k];
        if (sh_out) v = v + sh_out[(uint64_t)t * h + i] / (1.0f + expf(-sh_gate[t]));
        if (resid) v = resid[(uint64_t)t * h + i] + v;
        out[(uint64_t)t * h + i] = v;
    }
}

#define EW_LAUNCH(name, kern, n, ...) \
    return launch_kernel(p, name, kern, ew_grid(n), dim3(kEw), 0, s, __VA_ARGS__);

hipError_t launch_swiglu(Prof *p, hipStream_t s, const float *a, const float *b, float *y,
                         uint64_t n) {
    EW_LAUNCH("swiglu", swiglu_kernel, n, a, b, y, n)
}
hipError_t launch_mix(Prof *p, hipStream_t s, const float *x, const float *w, uint32_t k,
                      uint64_t n, float *y) {
    EW_LAUNCH("mix", mix_kernel, n, x, w, k, n, y)
}
hipError_t launch_gate_scalar(Prof *p, hipStream_t s, const float *x, const float *g, float *y,
                              uint64_t n) {
    EW_LAUNCH("gate_scalar", gate_scalar_kernel, n, x, g, y, n)
}
hipError_t launch_add(Prof *p, hipStream_t s, const float *a, const float *b, float *y,
                      uint64_t n) {
    EW_LAUNCH("add", add_kernel, n, a, b, y, n)
}
hipError_t launch_copy(Prof *p, hipStream_t s, const float *src, float *dst, uint64_t n) {
    EW_LAUNCH("copy", copy_kernel, n, src, dst, n)
}

hipError_t launch_norm(Prof *p, hipStream_t s, const float *x, const void *w, uint32_t wtype,
                       float *y, uint32_t heads, uint32_t n, uint32_t stride, float eps) {
    auto kern = wtype == 0 ? norm_kernel<0> : wtype == 1 ? norm_kernel<1> : norm_kernel<30>;
    return launch_kernel(p, "norm", kern, dim3(heads), dim3(64), 0, s, x, w, y, n, stride, eps);
}

hipError_t launch_combine(Prof *p, hipStream_t s, const float *yexp, const uint32_t *pos,
                          const float *w, uint32_t k, const float *sh_out, const float *sh_gate,
                          const float *resid, float *out, uint32_t tokens, uint32_t h) {
    dim3 grid((h + kEw - 1) / kEw, tokens);
    return launch_kernel(p, "combine", combine_kernel, grid, dim3(kEw), 0, s, yexp, pos, w, k,
                         sh_out, sh_gate, resid, out, tokens, h);
}

// Keeps the stream busy for `ticks` of the 100 MHz constant clock: the
// launches queued behind it are all enqueued before the GPU reaches them, so
// per-launch events measure GPU time and not host enqueue gaps.  Bounded
// twice: by the clock and by an iteration count (each s_sleep 127 lasts
// 127*64 shader cycles, over 3 us at 2.4 GHz).
__global__ __launch_bounds__(64) void hold_kernel(uint64_t ticks, uint32_t max_iters) {
    const uint64_t t0 = wall_clock64();
    for (uint32_t i = 0; i < max_iters && wall_clock64() - t0 < ticks; i++)
        __builtin_amdgcn_s_sleep(127);
}

hipError_t launch_hold(hipStream_t s, uint32_t microseconds) {
    return launch_kernel(nullptr, "hold", hold_kernel, dim3(1), dim3(64), 0, s,
                         (uint64_t)microseconds * 100u, microseconds / 2u + 2u);
}

}  // namespace moehip
