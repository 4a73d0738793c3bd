// Row dot products over any dense or affine weight (generic layout: the 64
// lanes of a wave stride over the packed words of one row).  Used by the
// op-level products and the grouped VALU path.
#pragma once
#include "device_common.hpp"

namespace moehip {

// Dot of global row `grow` (= expert*out + r) of `w` with x[0..in), summed
// over the wave.  Affine rows use the reference's per-word factorisation
// scale*sum(code*x) + bias*sum(x) (crates/metal-backend/src/shaders/affine.metal:49-66);
// dense rows follow the GEMV macro (crates/metal-backend/src/shaders/matrix.metal:8-38).
template <int BITS, int T>
__device__ __forceinline__ float row_dot_generic(const WDesc &w, uint64_t grow,
                                                 const float *__restrict__ x, int lane) {
    float acc = 0.f;
    if constexpr (BITS == 0) {
        const uint64_t base = grow * w.in;
        // eight independent loads per lane in flight (a lone wave per row is
        // latency-bound otherwise)
        constexpr int U = 8;
        uint32_t i = lane;
        for (; i + (U - 1) * kWave < w.in; i += U * kWave) {
            float wv[U], xv[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                wv[u] = load_scalar<T>(w.data, base + i + u * kWave);
                xv[u] = x[i + u * kWave];
            }
#pragma unroll
            for (int u = 0; u < U; u++) acc += wv[u] * xv[u];
        }
        for (; i < w.in; i += kWave) acc += load_scalar<T>(w.data, base + i) * x[i];
    } else {
        constexpr int P = 32 / BITS;
        const uint32_t row_words = w.in / P;
        const uint32_t *wr = reinterpret_cast<const uint32_t *>(w.data) + grow * row_words;
        const uint64_t elem0 = grow * w.in;
        // four words per lane per round, their loads issued together
        constexpr int U = 4;
        uint32_t wi = lane;
        for (; wi + (U - 1) * kWave < row_words; wi += U * kWave) {
            uint32_t wv[U], sr[U], br[U];
            float xs[U][P];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const uint32_t wu = wi + u * kWave;
                wv[u] = wr[wu];
                const uint64_t g = (elem0 + (uint64_t)wu * P) >> w.gshift;
                sr[u] = load_raw<T>(w.scales, g);
                br[u] = load_raw<T>(w.biases, g);
#pragma unroll
                for (int j = 0; j < P; j++) xs[u][j] = x[(uint64_t)wu * P + j];
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                float xsum = 0.f;
#pragma unroll
                for (int j = 0; j < P; j++) xsum += xs[u][j];
                acc += raw_to_f32<T>(sr[u]) * word_dot<BITS>(wv[u], xs[u]) + raw_to_f32<T>(br[u]) * xsum;
            }
        }
        for (; wi < row_words; wi += kWave) {
            const float *xx = x + (uint64_t)wi * P;
            float xs[P];
            float xsum = 0.f;
#pragma unroll
            for (int j = 0; j < P; j++) {
                xs[j] = xx[j];
                xsum += xs[j];
            }
            const float d = word_dot<BITS>(wr[wi], xs);
            const uint64_t g = (elem0 + (uint64_t)wi * P) >> w.gshift;
            acc += load_scalar<T>(w.scales, g) * d + load_scalar<T>(w.biases, g) * xsum;
        }
    }
    return wave_sum(acc);
}

// Instantiate `body.template operator()<BITS, T>()` for the weight's kind.
template <typename F>
__host__ hipError_t dispatch_kind(const WDesc &w, F &&body) {
    switch (w.bits) {
    case 0:
        if (w.type == 0) return body.template operator()<0, 0>();
        if (w.type == 1) return body.template operator()<0, 1>();
        if (w.type == 30) return body.template operator()<0, 30>();
        break;
    case 2:
        if (w.type == 0) return body.template operator()<2, 0>();
        if (w.type == 1) return body.template operator()<2, 1>();
        if (w.type == 30) return body.template operator()<2, 30>();
        break;
    case 4:
        if (w.type == 0) return body.template operator()<4, 0>();
        if (w.type == 1) return body.template operator()<4, 1>();
        if (w.type == 30) return body.template operator()<4, 30>();
        break;
    case 8:
        if (w.type == 0) return body.template operator()<8, 0>();
        if (w.type == 1) return body.template operator()<8, 1>();
        if (w.type == 30) return body.template operator()<8, 30>();
        break;
    default:
        break;
    }
    return hipErrorInvalidValue;
}

}  // namespace moehip
