// Exact top-k routing for one token on one wave (device side).
#pragma once
#include "device_common.hpp"

namespace moehip {

// route (crates/metal-backend/src/shaders/sampling.metal:1-36) for one token,
// executed by one full wave (K <= 64):
//   mx  = max(x) ignoring NaN (Metal max = fmax)
//   den = sum exp(x - mx)          (parallel order: equal up to rounding)
//   K passes; each takes the unused j with the largest logit, ties to the
//   lower j (the reference's strict `>` scan over ascending j); -inf and NaN
//   never win; an exhausted pool yields id 0 with score -inf
//   w_k = exp(x_best - mx) / den;  normalize: w_k /= sum_k w_k
// Lane l holds logits l, l+64, ... in registers and keeps its local best
// under the scan order.  A pass is a wave max of the bests' order keys and a
// wave min of the indices holding that key (both fused DPP/permlane integer
// reductions); only the winning lane rescans its slots.  Lane k records pass
// k, and the K weights are computed in parallel after the loop; lanes 0..K-1
// write ids[k] and weights[k].
template <int R>
__device__ __forceinline__ void route_wave_regs(const float *__restrict__ logits, uint32_t E,
                                                uint32_t K, int normalize, uint32_t *ids,
                                                float *weights, int lane) {
    float v[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const uint32_t j = lane + kWave * i;
        v[i] = j < E ? logits[j] : -INFINITY;
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < R; i++) m = fmaxf(m, v[i]);
    const float mx = wave_max(m);
    float den = 0.f;
#pragma unroll
    for (int i = 0; i < R; i++)
        if (lane + kWave * i < E) den += expf(v[i] - mx);
    den = wave_sum(den);
    // local best: strict > over ascending slots (= ascending j); NaN never wins
    float bv = -INFINITY;
    int bi = R;
#pragma unroll
    for (int i = 0; i < R; i++)
        if (v[i] > bv) {
            bv = v[i];
            bi = i;
        }
    uint32_t my_id = 0;
    float my_score = -INFINITY;
    for (uint32_t k = 0; k < K; k++) {
        const uint32_t key = bi < R ? fkey(bv) : 0u;  // 0: no candidate in this lane
        const uint32_t M = wave_max_u32(key);
        const uint32_t mine = (bi < R && key == M) ? (uint32_t)(lane + kWave * bi) : 0xffffffffu;
        const uint32_t best = wave_min_u32(mine);
        if (best != 0xffffffffu) {
            if ((uint32_t)lane == k) {
                my_id = best;
                my_score = funkey(M);
            }
            if ((best & (kWave - 1)) == (uint32_t)lane) {
                const int slot = (int)(best >> 6);
#pragma unroll
                for (int i = 0; i < R; i++)
                    if (i == slot) v[i] = -INFINITY;
                bv = -INFINITY;
                bi = R;
#pragma unroll
                for (int i = 0; i < R; i++)
                    if (v[i] > bv) {
                        bv = v[i];
                        bi = i;
                    }
            }
        }
        // exhausted pool: id 0, score -inf (my_id/my_score keep their defaults)
    }
    float wk = (uint32_t)lane < K ? expf(my_score - mx) / den : 0.f;
    if (normalize) wk = wk / wave_sum(wk);
    if ((uint32_t)lane < K) {
        ids[lane] = my_id;
        weights[lane] = wk;
    }
}

// Same selection for E > 1024 with the logits in this wave's LDS slice
// `vals` (E floats); a selected entry is overwritten with -inf, which removes
// it exactly as the reference's `used` test does (an entry equal to -inf can
// never win a strict `>` scan).
__device__ __forceinline__ void route_wave_lds(float *vals, const float *__restrict__ logits,
                                               uint32_t E, uint32_t K, int normalize,
                                               uint32_t *ids, float *weights, int lane) {
    float m = -INFINITY;
    for (uint32_t j = lane; j < E; j += kWave) {
        const float x = logits[j];
        vals[j] = x;
        m = fmaxf(m, x);
    }
    const float mx = wave_max(m);
    float den = 0.f;
    for (uint32_t j = lane; j < E; j += kWave) den += expf(vals[j] - mx);
    den = wave_sum(den);
    float selected = 0.f;
    for (uint32_t k = 0; k < K; k++) {
        float bv = -INFINITY;
        uint32_t bj = 0xffffffffu;
        for (uint32_t j = lane; j < E; j += kWave) {
            const float x = vals[j];
            if (x > bv) {
                bv = x;
                bj = j;
            }
        }
        const float M = wave_max(bv);
        const bool cand = bj != 0xffffffffu && bv == M;
        const uint32_t best0 = wave_min_u32(cand ? bj : 0xffffffffu);
        const bool none = best0 == 0xffffffffu;
        const uint32_t best = none ? 0u : best0;
        const float score = none ? -INFINITY : M;
        if (!none && (best & (kWave - 1)) == (uint32_t)lane) vals[best] = -INFINITY;
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

// Routing of one token by one wave; `vals` (E floats of LDS) is only used
// when E > 1024 or K > 64.
__device__ __forceinline__ void route_one_wave(float *vals, const float *__restrict__ logits,
                                               uint32_t E, uint32_t K, int normalize,
                                               uint32_t *ids, float *weights, int lane) {
    if (K > (uint32_t)kWave || E > 1024)
        route_wave_lds(vals, logits, E, K, normalize, ids, weights, lane);
    else if (E <= 64)
        route_wave_regs<1>(logits, E, K, normalize, ids, weights, lane);
    else if (E <= 128)
        route_wave_regs<2>(logits, E, K, normalize, ids, weights, lane);
    else if (E <= 256)
        route_wave_regs<4>(logits, E, K, normalize, ids, weights, lane);
    else if (E <= 512)
        route_wave_regs<8>(logits, E, K, normalize, ids, weights, lane);
    else
        route_wave_regs<16>(logits, E, K, normalize, ids, weights, lane);
}

}  // namespace moehip
