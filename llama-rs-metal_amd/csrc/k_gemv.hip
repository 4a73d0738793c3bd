// Generic products behind Batch::matmul and Batch::expert_matmul
// (crates/metal-backend/src/apple/ops/matrix.rs:63-205).  One wave per
// (output row, selection, token); correct for every dtype, bit width, group
// size and shape the reference accepts.  The hot MoE shapes use the fused
// decode kernels (k_decode.hip) or the grouped kernels instead.
#include "rowdot.hpp"

namespace moehip {

template <int BITS, int T>
__global__ __launch_bounds__(256) void gemv_kernel(WDesc w, const float *__restrict__ x,
                                                   uint64_t x_sel_stride,
                                                   const uint32_t *__restrict__ ids,
                                                   float *__restrict__ y, uint32_t tokens) {
    const int lane = threadIdx.x & 63;
    const uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t sel = blockIdx.y, t = blockIdx.z;
    if (r >= w.out) return;
    float *yo = y + ((uint64_t)sel * tokens + t) * w.out + r;
    const uint32_t expert = ids ? ids[sel] : 0u;
    if (expert >= w.experts) {  // affine.metal:91 / matrix.metal:56-60
        if (lane == 0) *yo = 0.f;
        return;
    }
    const float *xv = x + (uint64_t)sel * x_sel_stride + (uint64_t)t * w.in;
    const float acc = row_dot_generic<BITS, T>(w, (uint64_t)expert * w.out + r, xv, lane);
    if (lane == 0) *yo = acc;
}

// One output row (the shared-expert gate scalar x . w_g, [h] reshaped to
// [h, 1]): one wave per token, four tokens per block.
template <int BITS, int T>
__global__ __launch_bounds__(256) void gemv_row1_kernel(WDesc w, const float *__restrict__ x,
                                                        float *__restrict__ y, uint32_t tokens) {
    const int lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= tokens) return;
    const float acc = row_dot_generic<BITS, T>(w, 0, x + (uint64_t)t * w.in, lane);
    if (lane == 0) y[t] = acc;
}

struct GemvLaunch {
    Prof *p;
    hipStream_t s;
    const WDesc &w;
    const float *x;
    uint64_t xs;
    const uint32_t *ids;
    uint32_t nsel;
    float *y;
    uint32_t tokens;
    template <int BITS, int T>
    hipError_t operator()() {
        // (a selected expert id may lie past the single expert: the generic
        // kernel then writes 0, as affine.metal:91 does)
        if (w.out == 1 && nsel == 1 && w.experts == 1 && ids == nullptr)
            return launch_kernel(p, "gemv_row1", gemv_row1_kernel<BITS, T>, dim3((tokens + 3) / 4), dim3(256), 0,
                                 s, w, x, y, tokens);
        dim3 grid((w.out + 3) / 4, nsel, tokens);
        return launch_kernel(p, "gemv_generic", gemv_kernel<BITS, T>, grid, dim3(256), 0, s, w, x, xs,
                             ids, y, tokens);
    }
};

hipError_t launch_gemv(Prof *p, hipStream_t s, const WDesc &w, const float *x,
                       uint64_t x_sel_stride, const uint32_t *ids, uint32_t nsel, float *y,
                       uint32_t tokens) {
    if (w.out == 0 || nsel == 0 || tokens == 0) return hipSuccess;
    hipError_t e = hipSuccess;
    if (nsel == 1 && w.out == 1 && w.experts == 1 && ids == nullptr) {
        e = dispatch_kind(w, GemvLaunch{p, s, w, x, x_sel_stride, ids, 1, y, tokens});
    } else if (nsel == 1) {
        // grid.z is limited to 65535: split long token runs (matmul only).
        for (uint32_t t0 = 0; t0 < tokens && e == hipSuccess; t0 += 65535u) {
            const uint32_t n = tokens - t0 < 65535u ? tokens - t0 : 65535u;
            e = dispatch_kind(w, GemvLaunch{p, s, w, x + (uint64_t)t0 * w.in, x_sel_stride, ids, 1,
                                            y + (uint64_t)t0 * w.out, n});
        }
    } else {
        e = dispatch_kind(w, GemvLaunch{p, s, w, x, x_sel_stride, ids, nsel, y, tokens});
    }
    return e;
}

}  // namespace moehip
