// Exact top-k routing for one token on one wave (device side).
#pragma once
#include "device_common.hpp"

namespace moehip {

// (value, index) pair order of the reference's selection scan: a candidate
// wins over another when its logit is strictly greater, or equal with a
// lower index (sampling.metal:19-28 scans ascending j with strict `>`).
__device__ __forceinline__ void better_of(float &v, uint32_t &j, float ov, uint32_t oj) {
    if (ov > v || (ov == v && oj < j)) {
        v = ov;
        j = oj;
    }
}

// Wave-wide argmax under better_of; every lane receives the winner.
// NaN never enters (candidates are filtered by `v > -inf` before).
__device__ __forceinline__ void wave_argmax(float &v, uint32_t &j) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(v, o, kWave);
        const uint32_t oj = __shfl_xor(j, o, kWave);
        better_of(v, j, ov, oj);
    }
}

// route (crates/metal-backend/src/shaders/sampling.metal:1-36) for one token,
// executed by one full wave.  `vals` is this wave's private LDS copy of the
// logits (E floats); lane l owns indices l, l+64, ...  Selected entries are
// overwritten with -inf, which removes them exactly as the reference's
// `used` test does: an entry equal to -inf can never win a strict `>` scan.
//   mx  = max(x) ignoring NaN (Metal max = fmax)
//   den = sum exp(x - mx)          (parallel order: equal up to rounding)
//   w_k = exp(x_best - mx) / den; exhausted pool -> id 0, score -inf
//   normalize: w_k /= sum_k w_k  (k order, as the reference)
// Lane 0 writes ids[0..K) and weights[0..K).
__device__ __forceinline__ void route_one_wave(float *vals, const float *__restrict__ logits,
                                               uint32_t E, uint32_t K, int normalize,
                                               uint32_t *ids, float *weights, int lane) {
    float mx = -INFINITY;
    for (uint32_t j = lane; j < E; j += kWave) {
        const float v = logits[j];
        vals[j] = v;
        mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    float den = 0.f;
    for (uint32_t j = lane; j < E; j += kWave) den += expf(vals[j] - mx);
    den = wave_sum(den);
    float selected = 0.f;
    for (uint32_t k = 0; k < K; k++) {
        float bv = -INFINITY;
        uint32_t bj = 0xffffffffu;
        for (uint32_t j = lane; j < E; j += kWave) {
            const float v = vals[j];
            if (v > bv) {
                bv = v;
                bj = j;
            }
        }
        wave_argmax(bv, bj);
        const bool none = bj == 0xffffffffu;
        const uint32_t best = none ? 0u : bj;
        const float score = none ? -INFINITY : bv;
        if ((best & (kWave - 1)) == (uint32_t)lane) vals[best] = -INFINITY;
        if (lane == 0) {
            const float wk = expf(score - mx) / den;
            ids[k] = best;
            weights[k] = wk;
            selected += wk;
        }
    }
    if (normalize && lane == 0)
        for (uint32_t k = 0; k < K; k++) weights[k] /= selected;
}

}  // namespace moehip
