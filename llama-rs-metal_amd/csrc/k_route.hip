// Routing (Batch::route, crates/metal-backend/src/apple/ops/sampling.rs:21-44)
// and token -> expert dispatch (counts, exclusive scan, stable permutation).
#include "route.hpp"

namespace moehip {

// One wave per token; each wave keeps a private LDS copy of its logits row.
__global__ __launch_bounds__(64) void route_kernel(const float *__restrict__ logits, uint32_t E,
                                                   uint32_t K, int normalize,
                                                   uint32_t *__restrict__ ids,
                                                   float *__restrict__ weights) {
    extern __shared__ float vals[];
    __shared__ RouteLds L;
    const uint32_t t = blockIdx.x;
    route_one_wave(&L, vals, logits + (uint64_t)t * E, E, K, normalize, ids + (uint64_t)t * K,
                   weights + (uint64_t)t * K, threadIdx.x);
}

hipError_t launch_route(Prof *p, hipStream_t s, const float *logits, uint32_t experts, uint32_t k,
                        int normalize, uint32_t tokens, uint32_t *ids, float *weights) {
    // LDS copy of the logits only where the selection keeps one (route_one_wave)
    const size_t lds = (experts > 1024 || k > 64) ? experts * sizeof(float) : 0;
    return launch_kernel(p, "route", route_kernel, dim3(tokens), dim3(64), lds, s, logits, experts,
                         k, normalize, ids, weights);
}

// Routing of router products split over K: logits[t, j] = sum_s part[s, t, j]
// (s ascending) + bias[t, j], written out and routed by the token's wave.
__global__ __launch_bounds__(64) void route_sum_kernel(const float *__restrict__ parts,
                                                       uint32_t nsplit, const float *__restrict__ bias,
                                                       uint32_t E, uint32_t K, int normalize,
                                                       float *__restrict__ logits,
                                                       uint32_t *__restrict__ ids,
                                                       float *__restrict__ weights) {
    extern __shared__ __attribute__((aligned(16))) float lg[];  // E logits of this token
    __shared__ RouteLds L;
    const uint32_t t = blockIdx.x;
    const uint64_t row = (uint64_t)t * E, stride = (uint64_t)gridDim.x * E;
    for (uint32_t j = threadIdx.x; j < E; j += kWave) {
        float v = parts[row + j];
        for (uint32_t s = 1; s < nsplit; s++) v += parts[s * stride + row + j];
        if (bias) v += bias[row + j];
        logits[row + j] = v;
        lg[j] = v;
    }
    wave_lds_sync();
    route_one_wave(&L, lg, lg, E, K, normalize, ids + (uint64_t)t * K, weights + (uint64_t)t * K,
                   threadIdx.x);
}

hipError_t launch_route_sum(Prof *p, hipStream_t s, const float *parts, uint32_t nsplit,
                            const float *bias, uint32_t experts, uint32_t k, int normalize,
                            uint32_t tokens, float *logits, uint32_t *ids, float *weights) {
    return launch_kernel(p, "route", route_sum_kernel, dim3(tokens), dim3(64),
                         experts * sizeof(float), s, parts, nsplit, bias, experts, k, normalize,
                         logits, ids, weights);
}

// ---------------------------------------------------------------- dispatch --
// Pass 1: per-expert counts.  LDS histogram per block, then one global
// atomic per touched expert; the totals are independent of atomic order.
constexpr int kDispThreads = 256;
constexpr int kDispItems = 8;

__global__ __launch_bounds__(kDispThreads) void zero_u32_kernel(uint32_t *p, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        p[i] = 0u;
}

__global__ __launch_bounds__(kDispThreads) void dispatch_count_kernel(
    const uint32_t *__restrict__ ids, uint32_t pairs, uint32_t E, uint32_t *__restrict__ counts) {
    extern __shared__ uint32_t hist[];
    for (uint32_t e = threadIdx.x; e < E; e += kDispThreads) hist[e] = 0u;
    __syncthreads();
    const uint32_t base = blockIdx.x * kDispThreads * kDispItems;
    for (int i = 0; i < kDispItems; i++) {
        const uint32_t p = base + i * kDispThreads + threadIdx.x;
        if (p < pairs) {
            const uint32_t e = ids[p];
            if (e < E) atomicAdd(&hist[e], 1u);
        }
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e < E; e += kDispThreads)
        if (hist[e]) atomicAdd(&counts[e], hist[e]);
}

// Pass 2: one block per expert.  The block sums counts[0..e) for its offset,
// then scans all pairs in ascending order and compacts those routed to e with
// a block-wide exclusive scan, so perm is ordered by (expert, token, k) with
// no dependence on scheduling.
__global__ __launch_bounds__(kDispThreads) void dispatch_place_kernel(
    const uint32_t *__restrict__ ids, uint32_t pairs, uint32_t E,
    const uint32_t *__restrict__ counts, uint32_t *__restrict__ offsets,
    uint32_t *__restrict__ perm, uint32_t *__restrict__ pos) {
    __shared__ uint32_t wsum[kDispThreads / 64];
    __shared__ uint32_t total;
    const uint32_t e = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // offset of expert e
    uint32_t part = 0;
    for (uint32_t i = tid; i < e; i += kDispThreads) part += counts[i];
    for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o, 64);
    if (lane == 0) wsum[wv] = part;
    __syncthreads();
    const uint32_t off = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    const uint32_t cnt = counts[e];
    if (tid == 0) {
        offsets[e] = off;
        if (e == E - 1) offsets[E] = off + cnt;
    }
    __syncthreads();
    if (cnt == 0) return;
    uint32_t running = 0;
    for (uint32_t base = 0; base < pairs && running < cnt; base += kDispThreads * kDispItems) {
        // each thread owns kDispItems consecutive pairs
        const uint32_t p0 = base + tid * kDispItems;
        uint32_t mine = 0, mask = 0;
#pragma unroll
        for (int i = 0; i < kDispItems; i++) {
            const uint32_t p = p0 + i;
            if (p < pairs && ids[p] == e) {
                mask |= 1u << i;
                mine++;
            }
        }
        // block exclusive scan of `mine`
        uint32_t incl = mine;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        if (lane == 63) wsum[wv] = incl;
        __syncthreads();
        uint32_t before = 0;
        for (int w = 0; w < wv; w++) before += wsum[w];
        const uint32_t excl = running + before + incl - mine;
        if (tid == 0) total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
        uint32_t at = off + excl;
#pragma unroll
        for (int i = 0; i < kDispItems; i++) {
            if (mask & (1u << i)) {
                perm[at] = p0 + i;
                pos[p0 + i] = at;
                at++;
            }
        }
        __syncthreads();
        running += total;
        __syncthreads();
    }
}

// Single-pass dispatch: every block histograms all pairs (and those before
// its chunk) in LDS, scans the counts over experts, and places its chunk of
// kPlaceChunk pairs.  Within a wave, the rank of a pair among the earlier
// lanes routed to the same expert comes from ballots over the bits of the
// expert id; per-wave, per-expert running counts (LDS) carry it across the
// wave's rounds and a per-expert prefix over the waves across the block.  So
// perm is ordered by pair index within every expert, as in the two-pass path.
// With `tiles`, block 0 (which holds every expert's count and offset after
// its scan) also writes the work list that tile_schedule_kernel would: the
// (expert, first position) of every run of tm pairs, experts ascending, and
// their count.
constexpr int kPlaceThreads = 1024;
constexpr int kPlaceWaves = kPlaceThreads / 64;
constexpr int kPlaceRounds = 4;
constexpr uint32_t kPlaceChunk = kPlaceWaves * kPlaceRounds * 64;
constexpr int kHistLoads = 8;  // id loads in flight per thread while histogramming

__global__ __launch_bounds__(kPlaceThreads) void dispatch_kernel(
    const uint32_t *__restrict__ ids, uint32_t pairs, uint32_t E, uint32_t *__restrict__ counts,
    uint32_t *__restrict__ offsets, uint32_t *__restrict__ perm, uint32_t *__restrict__ pos,
    uint32_t tm, uint32_t *__restrict__ tiles, uint32_t *__restrict__ ntiles, uint32_t per_chunk) {
    extern __shared__ uint32_t sm[];
    // cw: [kPlaceWaves][E]; hist (per_chunk): [gridDim.x][E], the counts of
    // every chunk, so each id costs one LDS atomic (otherwise the pairs
    // before this chunk are counted a second time into base)
    uint32_t *all = sm, *base = sm + E, *cw = sm + 2 * E, *hist = cw + kPlaceWaves * E;
    __shared__ uint32_t wsum[kPlaceWaves], tsum[kPlaceWaves];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t c0 = blockIdx.x * kPlaceChunk;
    const uint32_t nsm = (2 + kPlaceWaves) * E + (per_chunk ? gridDim.x * E : 0u);
    for (uint32_t i = tid; i < nsm; i += kPlaceThreads) sm[i] = 0u;
    __syncthreads();
    // counts of all pairs, and of the pairs before this chunk (kHistLoads
    // loads issued before their atomics)
    for (uint32_t b0 = 0; b0 < pairs; b0 += kPlaceThreads * kHistLoads) {
        uint32_t v[kHistLoads];
#pragma unroll
        for (int i = 0; i < kHistLoads; i++) {
            const uint32_t p = b0 + (uint32_t)(i * kPlaceThreads + tid);
            v[i] = p < pairs ? ids[p] : E;
        }
#pragma unroll
        for (int i = 0; i < kHistLoads; i++) {
            if (v[i] < E) {
                const uint32_t p = b0 + (uint32_t)(i * kPlaceThreads + tid);
                if (per_chunk) {
                    atomicAdd(&hist[(p / kPlaceChunk) * E + v[i]], 1u);
                } else {
                    atomicAdd(&all[v[i]], 1u);
                    if (p < c0) atomicAdd(&base[v[i]], 1u);
                }
            }
        }
    }
    __syncthreads();
    if (per_chunk) {
        for (uint32_t e = tid; e < E; e += kPlaceThreads) {
            uint32_t acc = 0, before = 0;
            for (uint32_t c = 0; c < gridDim.x; c++) {
                if (c == blockIdx.x) before = acc;
                acc += hist[c * E + e];
            }
            all[e] = acc;
            base[e] = before;
        }
        __syncthreads();
    }
    // exclusive scan over experts: thread t owns experts [t*per, t*per + per)
    const uint32_t per = (E + kPlaceThreads - 1) / kPlaceThreads;
    const uint32_t e0 = min(E, (uint32_t)tid * per), e1 = min(E, e0 + per);
    uint32_t part = 0;
    for (uint32_t e = e0; e < e1; e++) part += all[e];
    uint32_t incl = part;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
    }
    if (lane == 63) wsum[wv] = incl;
    __syncthreads();
    uint32_t run = incl - part, total = 0;
    for (int w = 0; w < kPlaceWaves; w++) {
        if (w < wv) run += wsum[w];
        total += wsum[w];
    }
    for (uint32_t e = e0; e < e1; e++) {
        const uint32_t c = all[e];
        if (blockIdx.x == 0) {
            counts[e] = c;
            offsets[e] = run;
        }
        base[e] += run;
        run += c;
    }
    if (blockIdx.x == 0 && tid == 0) offsets[E] = total;
    if (tiles && blockIdx.x == 0) {  // uniform over the block
        // block 0 places the first chunk, so base[e] now holds offsets[e]
        uint32_t tpart = 0;
        for (uint32_t e = e0; e < e1; e++) tpart += (all[e] + tm - 1) / tm;
        uint32_t tincl = tpart;
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t v = __shfl_up(tincl, o, 64);
            if (lane >= o) tincl += v;
        }
        if (lane == 63) tsum[wv] = tincl;
        __syncthreads();
        uint32_t first = tincl - tpart, ttotal = 0;
        for (int w = 0; w < kPlaceWaves; w++) {
            if (w < wv) first += tsum[w];
            ttotal += tsum[w];
        }
        for (uint32_t e = e0; e < e1; e++) {
            const uint32_t nt = (all[e] + tm - 1) / tm;
            for (uint32_t i = 0; i < nt; i++) {
                tiles[2 * (first + i)] = e;
                tiles[2 * (first + i) + 1] = base[e] + i * tm;
            }
            first += nt;
        }
        if (tid == 0) *ntiles = ttotal;
    }
    // ranks inside this chunk: wave wv takes pairs c0 + 64*(kPlaceRounds*wv + r) + lane
    const int bits = 32 - __clz((int)E);  // distinguishes 0..E (E marks an absent pair)
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t pe[kPlaceRounds], pr[kPlaceRounds];
#pragma unroll
    for (int r = 0; r < kPlaceRounds; r++) {
        const uint32_t p = c0 + 64u * (kPlaceRounds * wv + r) + lane;
        uint32_t e = p < pairs ? ids[p] : E;
        if (e > E) e = E;
        uint64_t same = ~0ull;
        for (int b = 0; b < bits; b++) {
            const bool bit = (e >> b) & 1u;
            const uint64_t m = __ballot(bit);
            same &= bit ? m : ~m;
        }
        const uint32_t c = e < E ? cw[wv * E + e] : 0u;
        // the group's last lane advances the running count (a wave's LDS
        // operations execute in order, so every lane above read the old value)
        if (e < E && (same >> lane) == 1ull) cw[wv * E + e] = c + (uint32_t)__popcll(same);
        pe[r] = e;
        pr[r] = c + (uint32_t)__popcll(same & below);
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += kPlaceThreads) {
        uint32_t acc = 0;
        for (int w = 0; w < kPlaceWaves; w++) {
            const uint32_t t = cw[w * E + e];
            cw[w * E + e] = acc;
            acc += t;
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kPlaceRounds; r++) {
        if (pe[r] < E) {
            const uint32_t p = c0 + 64u * (kPlaceRounds * wv + r) + lane;
            const uint32_t q = base[pe[r]] + cw[wv * E + pe[r]] + pr[r];
            perm[q] = p;
            pos[p] = q;
        }
    }
}

hipError_t launch_dispatch(Prof *p, hipStream_t s, const uint32_t *ids, uint32_t pairs,
                           uint32_t experts, uint32_t *counts, uint32_t *offsets, uint32_t *perm,
                           uint32_t *pos, uint32_t tm, uint32_t *tiles, uint32_t *ntiles) {
    const size_t lds = (size_t)(2 + kPlaceWaves) * experts * sizeof(uint32_t);
    if (lds <= 48 * 1024) {
        const uint32_t nb = pairs ? (pairs + kPlaceChunk - 1) / kPlaceChunk : 1u;
        const size_t lds_chunks = lds + (size_t)nb * experts * sizeof(uint32_t);
        const uint32_t per_chunk = lds_chunks <= 64 * 1024 ? 1u : 0u;
        return launch_kernel(p, "dispatch", dispatch_kernel, dim3(nb), dim3(kPlaceThreads),
                             per_chunk ? lds_chunks : lds, s, ids, pairs, experts, counts, offsets, perm,
                             pos, tm, tiles, ntiles, per_chunk);
    }
    if (tiles) {
        hipError_t e = launch_dispatch(p, s, ids, pairs, experts, counts, offsets, perm, pos);
        return e != hipSuccess ? e : launch_tile_schedule(p, s, offsets, experts, tm, tiles, ntiles);
    }
    const uint32_t zb = (experts + kDispThreads - 1) / kDispThreads;
    hipError_t e = launch_kernel(p, "dispatch_zero", zero_u32_kernel, dim3(zb), dim3(kDispThreads), 0,
                                 s, counts, experts);
    if (e != hipSuccess) return e;
    const uint32_t per_block = kDispThreads * kDispItems;
    const uint32_t nb = (pairs + per_block - 1) / per_block;
    if (nb) {
        e = launch_kernel(p, "dispatch_count", dispatch_count_kernel, dim3(nb), dim3(kDispThreads),
                          experts * sizeof(uint32_t), s, ids, pairs, experts, counts);
        if (e != hipSuccess) return e;
    }
    return launch_kernel(p, "dispatch_place", dispatch_place_kernel, dim3(experts),
                         dim3(kDispThreads), 0, s, ids, pairs, experts, counts, offsets, perm, pos);
}

// ------------------------------------------------- route + dispatch, fused --
// Routing of the T tokens (one wave per token, kRdWaves tokens per block), and
// in the block that finishes last the dispatch of all T*K pairs and the
// schedule of tm-pair work items (what dispatch_kernel and
// tile_schedule_kernel produce, in one launch instead of three).  Every block
// publishes its ids with a device-scope release and counts itself on
// `arrive`; the block whose increment completes the count reads all ids after
// an acquire and returns the counter to zero for the next launch.  No block
// waits for another.  Pair placement is stable: wave w takes a contiguous
// span of pairs, ranks inside a 64-pair round come from ballots over the
// expert id bits, per-wave running counts carry them across rounds, and a
// prefix over the waves orders the spans.
constexpr int kRdWaves = 4;
constexpr int kRdThreads = kRdWaves * 64;

__global__ __launch_bounds__(kRdThreads) void route_dispatch_kernel(
    const float *__restrict__ logits, uint32_t T, uint32_t E, uint32_t K, int normalize,
    uint32_t *ids, float *__restrict__ weights, uint32_t *arrive, uint32_t tm,
    uint32_t *__restrict__ counts, uint32_t *__restrict__ offsets, uint32_t *__restrict__ perm,
    uint32_t *__restrict__ pos, uint32_t *__restrict__ tiles, uint32_t *__restrict__ ntiles) {
    extern __shared__ uint32_t cw[];  // [kRdWaves][E]: per-wave expert counts, then bases
    __shared__ RouteLds L[kRdWaves];
    __shared__ uint32_t wsum[2][kRdWaves];
    __shared__ uint32_t last;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t t = blockIdx.x * kRdWaves + wv;
    if (t < T)
        route_one_wave(&L[wv], nullptr, logits + (uint64_t)t * E, E, K, normalize,
                       ids + (uint64_t)t * K, weights + (uint64_t)t * K, lane);
    __threadfence();
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
               gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    if (tid == 0) __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    const uint32_t pairs = T * K;
    const uint32_t span = (pairs + kRdThreads - 1) / kRdThreads * 64;
    const uint32_t p0 = min(pairs, wv * span), p1 = min(pairs, p0 + span);
    for (uint32_t i = tid; i < kRdWaves * E; i += kRdThreads) cw[i] = 0u;
    __syncthreads();
    for (uint32_t q = p0 + lane; q < p1; q += 64) {
        const uint32_t e = ids[q];
        if (e < E) atomicAdd(&cw[wv * E + e], 1u);
    }
    __syncthreads();
    // scan over experts (thread tid owns [e0, e1)) of pair and work-item counts
    const uint32_t per = (E + kRdThreads - 1) / kRdThreads;
    const uint32_t e0 = min(E, (uint32_t)tid * per), e1 = min(E, e0 + per);
    uint32_t part = 0, tpart = 0;
    for (uint32_t e = e0; e < e1; e++) {
        uint32_t c = 0;
        for (int w = 0; w < kRdWaves; w++) c += cw[w * E + e];
        part += c;
        tpart += (c + tm - 1) / tm;
    }
    uint32_t incl = part, tincl = tpart;
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(incl, o, 64), tv = __shfl_up(tincl, o, 64);
        if (lane >= o) {
            incl += v;
            tincl += tv;
        }
    }
    if (lane == 63) {
        wsum[0][wv] = incl;
        wsum[1][wv] = tincl;
    }
    __syncthreads();
    uint32_t run = incl - part, trun = tincl - tpart, total = 0, ttotal = 0;
    for (int w = 0; w < kRdWaves; w++) {
        if (w < wv) {
            run += wsum[0][w];
            trun += wsum[1][w];
        }
        total += wsum[0][w];
        ttotal += wsum[1][w];
    }
    for (uint32_t e = e0; e < e1; e++) {
        uint32_t c = 0;
        for (int w = 0; w < kRdWaves; w++) {
            const uint32_t v = cw[w * E + e];
            cw[w * E + e] = run + c;
            c += v;
        }
        counts[e] = c;
        offsets[e] = run;
        const uint32_t nt = (c + tm - 1) / tm;
        for (uint32_t i = 0; i < nt; i++) {
            tiles[2 * (trun + i)] = e;
            tiles[2 * (trun + i) + 1] = run + i * tm;
        }
        trun += nt;
        run += c;
    }
    if (tid == 0) {
        offsets[E] = total;
        *ntiles = ttotal;
    }
    __syncthreads();
    const int bits = 32 - __clz((int)E);  // distinguishes 0..E (E marks an absent pair)
    const uint64_t below = (1ull << lane) - 1ull;
    for (uint32_t b = p0; b < p1; b += 64) {
        const uint32_t q = b + lane;
        uint32_t e = q < p1 ? ids[q] : E;
        if (e > E) e = E;
        uint64_t same = ~0ull;
        for (int i = 0; i < bits; i++) {
            const bool bit = (e >> i) & 1u;
            const uint64_t m = __ballot(bit);
            same &= bit ? m : ~m;
        }
        const uint32_t c = e < E ? cw[wv * E + e] : 0u;
        // the group's last lane advances the running base (the wave's LDS
        // operations execute in order, so every lane read the old value)
        if (e < E && (same >> lane) == 1ull) cw[wv * E + e] = c + (uint32_t)__popcll(same);
        if (e < E) {
            const uint32_t at = c + (uint32_t)__popcll(same & below);
            perm[at] = q;
            pos[q] = at;
        }
    }
}

bool route_dispatch_fits(uint32_t experts, uint32_t k, uint32_t tokens) {
    // route_one_wave keeps no LDS copy of the logits for these sizes
    return tokens > 0 && experts <= 1024 && k <= (uint32_t)kWave;
}

hipError_t launch_route_dispatch(Prof *p, hipStream_t s, const float *logits, uint32_t experts,
                                 uint32_t k, int normalize, uint32_t tokens, uint32_t *ids,
                                 float *weights, uint32_t *arrive, uint32_t tm, uint32_t *counts,
                                 uint32_t *offsets, uint32_t *perm, uint32_t *pos, uint32_t *tiles,
                                 uint32_t *ntiles) {
    if (!route_dispatch_fits(experts, k, tokens)) return hipErrorInvalidValue;
    const uint32_t nb = (tokens + kRdWaves - 1) / kRdWaves;
    return launch_kernel(p, "route_dispatch", route_dispatch_kernel, dim3(nb), dim3(kRdThreads),
                         (size_t)kRdWaves * experts * sizeof(uint32_t), s, logits, tokens, experts, k,
                         normalize, ids, weights, arrive, tm, counts, offsets, perm, pos, tiles,
                         ntiles);
}

}  // namespace moehip
