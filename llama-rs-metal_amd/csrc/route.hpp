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
        if (lane + kWave * i < E) den += exp_fast(v[i] - mx);
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
    float wk = (uint32_t)lane < K ? exp_fast(my_score - mx) / den : 0.f;
    if (normalize) wk = wk / wave_sum(wk);
    if ((uint32_t)lane < K) {
        ids[lane] = my_id;
        weights[lane] = wk;
    }
}

// LDS scratch of one routing wave.
struct RouteLds {
    alignas(16) uint64_t ck[64];  // composite keys of the surviving candidates
    uint32_t sj[64];  // selected ids by rank
    float sv[64];     // selected logits by rank
};

// Composite selection key of element j with value key k = fkey(v): larger =
// earlier in the reference's scan order (logit descending, index ascending);
// E < 65536.
__device__ __forceinline__ uint64_t ckey(uint32_t k, uint32_t j) {
    return ((uint64_t)k << 16) | (uint64_t)(0xffffu - j);
}
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Lane `lane` holds elements j = R*lane + i (i < R): two 16-byte loads per
// lane when R is a multiple of 4 and the row is aligned and whole.
template <int R>
__device__ __forceinline__ void load_logits(const float *__restrict__ logits, uint32_t E, int lane,
                                            float *v) {
    const uint32_t j0 = (uint32_t)R * lane;
    if constexpr (R % 4 == 0) {
        if ((reinterpret_cast<uintptr_t>(logits) & 15u) == 0 && (uint64_t)R * kWave <= E) {
#pragma unroll
            for (int q = 0; q < R / 4; q++) {
                const float4 f = reinterpret_cast<const float4 *>(logits + j0)[q];
                v[4 * q + 0] = f.x;
                v[4 * q + 1] = f.y;
                v[4 * q + 2] = f.z;
                v[4 * q + 3] = f.w;
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < R; i++) v[i] = j0 + i < E ? logits[j0 + i] : -INFINITY;
}

// Candidate ranking shared by the two selections below (K <= 64):
//  1. key_i = fkey(v_i) for v_i > -inf (0 for -inf, NaN and padding, which
//     never win the reference's strict `>` scan); kb = the lane's best key;
//  2. t = the largest 16-bit key prefix that at least K lane bests reach
//     (binary search over ballots): at least K elements have key >= t, so
//     every top-K element does;
//  3. the elements with key >= max(t, 1) are compacted into LDS and each is
//     ranked against the others under the composite order (key descending,
//     index ascending).
// Returns the candidate count `total` (> 64: nothing ranked; the caller runs
// route_wave_regs), and for lane < total its composite key `mine` and rank `r`.
template <int R>
__device__ __forceinline__ uint32_t rank_candidates(RouteLds *L, const float *v, uint32_t K,
                                                    int lane, uint64_t &mine, uint32_t &r) {
    uint32_t key[R], kb = 0;
#pragma unroll
    for (int i = 0; i < R; i++) {
        key[i] = v[i] > -INFINITY ? fkey(v[i]) : 0u;
        kb = max(kb, key[i]);
    }
    uint32_t t = 0;
#pragma unroll
    for (int b = 31; b >= 16; b--) {
        const uint32_t c = t | (1u << b);
        if ((uint32_t)__popcll(__ballot(kb >= c)) >= K) t = c;
    }
    const uint32_t tq = t ? t : 1u;
    uint32_t total = 0, pos[R];
    bool q[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
        q[i] = key[i] >= tq;
        const uint64_t bm = __ballot(q[i]);
        pos[i] = total + lanes_below(bm);
        total += (uint32_t)__popcll(bm);
    }
    if (total > (uint32_t)kWave) return total;
#pragma unroll
    for (int i = 0; i < R; i++)
        if (q[i]) L->ck[pos[i]] = ckey(key[i], (uint32_t)R * lane + i);
    if (total & 1u) L->ck[total] = 0ull;  // pad to whole pairs (odd total < 64); 0 ranks last
    wave_lds_sync();
    mine = (uint32_t)lane < total ? L->ck[lane] : 0ull;
    r = 0;
    for (uint32_t c = 0; c < total; c += 2) {
        const ulonglong2 p = *reinterpret_cast<const ulonglong2 *>(&L->ck[c]);
        r += (p.x > mine ? 1u : 0u) + (p.y > mine ? 1u : 0u);
    }
    return total;
}

// Full selection (ids and weights) without K serial passes.  Returns false
// (nothing written) when more than 64 candidates survive; the caller then
// runs route_wave_regs.
template <int R>
__device__ __forceinline__ bool route_wave_rank(RouteLds *L, const float *__restrict__ logits,
                                                uint32_t E, uint32_t K, int normalize,
                                                uint32_t *ids, float *weights, int lane) {
    float v[R];
    load_logits<R>(logits, E, lane, v);
    uint64_t mine;
    uint32_t r;
    const uint32_t total = rank_candidates<R>(L, v, K, lane, mine, r);
    if (total > (uint32_t)kWave) return false;
    if ((uint32_t)lane < total && r < K) {
        L->sj[r] = 0xffffu - (uint32_t)(mine & 0xffffu);
        L->sv[r] = funkey((uint32_t)(mine >> 16));
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < R; i++) m = fmaxf(m, v[i]);
    const float mx = wave_max(m);
    float den = 0.f;
#pragma unroll
    for (int i = 0; i < R; i++)
        if ((uint32_t)R * lane + i < E) den += exp_fast(v[i] - mx);
    den = wave_sum(den);
    wave_lds_sync();
    float score = -INFINITY;  // ranks beyond the candidates: id 0, score -inf
    uint32_t id = 0;
    if ((uint32_t)lane < K && (uint32_t)lane < total) {
        score = L->sv[lane];
        id = L->sj[lane];
    }
    float wk = (uint32_t)lane < K ? exp_fast(score - mx) / den : 0.f;
    if (normalize) wk = wk / wave_sum(wk);
    if ((uint32_t)lane < K) {
        ids[lane] = id;
        weights[lane] = wk;
    }
    return true;
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
    for (uint32_t j = lane; j < E; j += kWave) den += exp_fast(vals[j] - mx);
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
            const float wk = exp_fast(score - mx) / den;
            ids[k] = best;
            weights[k] = wk;
            selected += wk;
        }
    }
    if (normalize && lane == 0)
        for (uint32_t k = 0; k < K; k++) weights[k] /= selected;
}

// Routing of one token by one wave (LDS scratch `L`); `vals` (E floats of
// LDS) is only used when E > 1024 or K > 64.
template <int R>
__device__ __forceinline__ void route_regs(RouteLds *L, const float *__restrict__ logits,
                                           uint32_t E, uint32_t K, int normalize, uint32_t *ids,
                                           float *weights, int lane) {
    if (!route_wave_rank<R>(L, logits, E, K, normalize, ids, weights, lane))
        route_wave_regs<R>(logits, E, K, normalize, ids, weights, lane);
}
__device__ __forceinline__ void route_one_wave(RouteLds *L, float *vals,
                                               const float *__restrict__ logits, uint32_t E,
                                               uint32_t K, int normalize, uint32_t *ids,
                                               float *weights, int lane) {
    if (K > (uint32_t)kWave || E > 1024)
        route_wave_lds(vals, logits, E, K, normalize, ids, weights, lane);
    else if (E <= 64)
        route_regs<1>(L, logits, E, K, normalize, ids, weights, lane);
    else if (E <= 128)
        route_regs<2>(L, logits, E, K, normalize, ids, weights, lane);
    else if (E <= 256)
        route_regs<4>(L, logits, E, K, normalize, ids, weights, lane);
    else if (E <= 512)
        route_regs<8>(L, logits, E, K, normalize, ids, weights, lane);
    else
        route_regs<16>(L, logits, E, K, normalize, ids, weights, lane);
}

// Only the id selected by pass `want` (want < K <= 64) of the same routing;
// no weights.  Every lane returns it.  `after_load` runs once the logits are
// in registers and before the selection arithmetic: a caller issues its other
// loads there, so the logits do not wait behind them and they arrive during
// the selection.
template <int R, typename F>
__device__ __forceinline__ uint32_t route_id_regs(RouteLds *L, const float *__restrict__ logits,
                                                  uint32_t E, uint32_t K, uint32_t want, int lane,
                                                  F &&after_load) {
    float v[R];
    load_logits<R>(logits, E, lane, v);
#pragma unroll
    for (int i = 0; i < R; i++) asm volatile("" : "+v"(v[i]));
    asm volatile("" ::: "memory");
    after_load();
    uint64_t mine;
    uint32_t r;
    const uint32_t total = rank_candidates<R>(L, v, K, lane, mine, r);
    if (total <= (uint32_t)kWave) {
        const uint64_t hit = __ballot((uint32_t)lane < total && r == want);
        if (!hit) return 0u;  // exhausted pool: id 0
        return readlane_u(0xffffu - (uint32_t)(mine & 0xffffu), __ffsll((unsigned long long)hit) - 1);
    }
    route_wave_regs<R>(logits, E, K, 0, L->sj, L->sv, lane);
    wave_lds_sync();
    return L->sj[want];
}
template <typename F>
__device__ __forceinline__ uint32_t route_one_id(RouteLds *L, float *vals,
                                                 const float *__restrict__ logits, uint32_t E,
                                                 uint32_t K, uint32_t want, int lane, F &&after_load) {
    if (E > 1024) {
        after_load();
        route_wave_lds(vals, logits, E, K, 0, L->sj, L->sv, lane);
        wave_lds_sync();
        return L->sj[want];
    }
    if (E <= 64) return route_id_regs<1>(L, logits, E, K, want, lane, after_load);
    if (E <= 128) return route_id_regs<2>(L, logits, E, K, want, lane, after_load);
    if (E <= 256) return route_id_regs<4>(L, logits, E, K, want, lane, after_load);
    if (E <= 512) return route_id_regs<8>(L, logits, E, K, want, lane, after_load);
    return route_id_regs<16>(L, logits, E, K, want, lane, after_load);
}

}  // namespace moehip
