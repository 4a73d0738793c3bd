// Grouped expert products on VALU: experts iterate over their dispatched
// segment (perm order) so each expert row is fetched from HBM once per layer
// and re-used from cache for every token routed to it.  Generic in dtype,
// bit width and shape (the bf16 MFMA kernels cover prefill-sized segments).
#include "rowdot.hpp"

namespace moehip {

// act[p, j] = silu(x_t . G_e[j]) * (x_t . U_e[j]) for p in expert e's segment
// (the per-token sequence expert_matmul(gate) / expert_matmul(up) / swiglu of
// crates/model-runtime/src/execute.rs:222-224, regrouped by expert).
template <int BITS, int T>
__global__ __launch_bounds__(256) void grouped_gateup_kernel(WDesc g, WDesc u,
                                                             const float *__restrict__ x,
                                                             const uint32_t *__restrict__ offsets,
                                                             const uint32_t *__restrict__ perm,
                                                             uint32_t K, float *__restrict__ act) {
    const uint32_t e = blockIdx.x;
    const uint32_t j = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const uint32_t beg = offsets[e], end = offsets[e + 1];
    if (beg == end || j >= g.out) return;
    const uint64_t grow = (uint64_t)e * g.out + j;
    for (uint32_t p = beg; p < end; p++) {
        const uint32_t t = perm[p] / K;
        const float *xt = x + (uint64_t)t * g.in;
        const float gv = row_dot_generic<BITS, T>(g, grow, xt, lane);
        const float uv = row_dot_generic<BITS, T>(u, grow, xt, lane);
        if (lane == 0) act[(uint64_t)p * g.out + j] = gv / (1.0f + expf(-gv)) * uv;
    }
}

// yexp[p, r] = D_e[r] . act[p]  (expert_matmul(down, per_expert_input),
// execute.rs:225, regrouped by expert).
template <int BITS, int T>
__global__ __launch_bounds__(256) void grouped_down_kernel(WDesc d, const float *__restrict__ act,
                                                           const uint32_t *__restrict__ offsets,
                                                           float *__restrict__ yexp) {
    const uint32_t e = blockIdx.x;
    const uint32_t r = blockIdx.y * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const uint32_t beg = offsets[e], end = offsets[e + 1];
    if (beg == end || r >= d.out) return;
    const uint64_t grow = (uint64_t)e * d.out + r;
    for (uint32_t p = beg; p < end; p++) {
        const float v = row_dot_generic<BITS, T>(d, grow, act + (uint64_t)p * d.in, lane);
        if (lane == 0) yexp[(uint64_t)p * d.out + r] = v;
    }
}

struct GateUpLaunch {
    Prof *p;
    hipStream_t s;
    const WDesc &g, &u;
    const float *x;
    const uint32_t *offsets, *perm;
    uint32_t K, E;
    float *act;
    template <int BITS, int T>
    hipError_t operator()() {
        dim3 grid(E, (g.out + 3) / 4);
        return launch_kernel(p, "grouped_gateup_valu", grouped_gateup_kernel<BITS, T>, grid,
                             dim3(256), 0, s, g, u, x, offsets, perm, K, act);
    }
};

struct DownLaunch {
    Prof *p;
    hipStream_t s;
    const WDesc &d;
    const float *act;
    const uint32_t *offsets;
    uint32_t E;
    float *yexp;
    template <int BITS, int T>
    hipError_t operator()() {
        dim3 grid(E, (d.out + 3) / 4);
        return launch_kernel(p, "grouped_down_valu", grouped_down_kernel<BITS, T>, grid, dim3(256),
                             0, s, d, act, offsets, yexp);
    }
};

hipError_t launch_grouped_gateup(Prof *p, hipStream_t s, const WDesc &gate, const WDesc &up,
                                 const float *x, const uint32_t *offsets, const uint32_t *perm,
                                 uint32_t k, uint32_t experts, float *act) {
    return dispatch_kind(gate, GateUpLaunch{p, s, gate, up, x, offsets, perm, k, experts, act});
}

hipError_t launch_grouped_down(Prof *p, hipStream_t s, const WDesc &down, const float *act,
                               const uint32_t *offsets, uint32_t experts, uint32_t pairs,
                               float *yexp) {
    (void)pairs;
    return dispatch_kind(down, DownLaunch{p, s, down, act, offsets, experts, yexp});
}

}  // namespace moehip
