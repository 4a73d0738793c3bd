// Batched decode: T >= 2 tokens whose expert segments are too short for the
// bf16 MFMA path (config 3: 8 to 64 tokens over 512 experts).  The fused
// decode's lane layout (lanerows.hpp) runs over work entries of at most
// kSegTokens rows of input: a wave loads its weight rows once and applies
// them to every input row of its entry, so every expert row is read from HBM
// once per layer and per entry and the activations come from L2.
//
//   seg_gateup  gate and up rows + SwiGLU (activation,
//               crates/metal-backend/src/shaders/elementwise.metal:8-17):
//               routed experts over their dispatched pairs, or the shared
//               expert over all tokens -> act [pair or token, ff]
//   seg_rows    plain row products of input row p -> out[p, row]: the router
//               (Batch::matmul(router), execute.rs:220, with the logit bias
//               added), the routed down rows (expert_matmul(down),
//               execute.rs:225), the shared expert's down rows and its gate
//               input row (execute.rs:228-230)
//
// Entries: either the dispatch's segments cut into runs of kSegTokens pairs
// (tile_schedule: (expert, first pair); the run ends at the segment end), or
// runs of seg_run(n) rows over [0, n) of a single weight.
#include "lanerows.hpp"
#include "rowdot.hpp"

namespace moehip {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kSegTokens = 8;  // pairs per work entry over the dispatched segments
// Input rows per entry over all tokens (router, shared expert): the weights
// are small, so more waves beat re-reads at a few tokens; from 48 tokens on,
// runs of 4 (config 3 at 64 tokens: 271.5 -> 262.4 us per step; at 8 tokens
// runs of 4 cost 72.8 -> 75.6 us).
__host__ __device__ inline uint32_t seg_run(uint32_t n) { return n >= 48 ? 4u : 2u; }
constexpr int kSegGateItems = 2;    // kGateFR-row items of gate (and of up) rows per wave
constexpr int kSegRowsFR = 4;       // row instructions per wave in seg_rows

struct SegArgs {
    WDesc w, w2;              // weights (w2: the up rows of seg_gateup)
    const float *in;          // input rows [*, w.in]
    const uint32_t *perm;     // seg_gateup over dispatched pairs: input row perm[p] / k
    uint32_t k;
    const uint32_t *tiles;    // entries (expert, first p), or nullptr: runs over [0, n)
    const uint32_t *ntiles;   // entry count (device), with tiles
    const uint32_t *offsets;  // segment ends offsets[e + 1], with tiles
    uint32_t n;               // without tiles: input rows
    uint32_t run;             // without tiles: input rows per entry (seg_run(n))
    const float *bias;        // seg_rows: added to out[p, row] (or nullptr)
    float *out;               // [p, w.out]
};

// Work entry i: expert e and input rows [beg, end).
__device__ __forceinline__ bool seg_entry(const SegArgs &a, uint32_t i, uint32_t &e, uint32_t &beg,
                                          uint32_t &end) {
    if (a.tiles) {
        if (i >= *a.ntiles) return false;
        e = a.tiles[2 * i];
        beg = a.tiles[2 * i + 1];
        end = min(a.offsets[e + 1], beg + kSegTokens);
    } else {
        e = 0;
        beg = i * a.run;
        if (beg >= a.n) return false;
        end = min(a.n, beg + a.run);
    }
    return true;
}

// Lanes per row: the kernels are specialised for rows of 2048 (64 lanes) and
// 512 (16 lanes) elements; 0 reads it from the weight at run time.
template <int LPR>
__device__ __forceinline__ uint32_t lanes_per_row(const WDesc &w) {
    if constexpr (LPR) return (uint32_t)LPR;
    else return w.in / 32;
}

// This lane's 32-element chunk of one input row, and the chunk's sum.
struct InChunk {
    float v[32];
    __device__ __forceinline__ void load(const float *__restrict__ row, uint32_t cl) {
        const float4 *src = reinterpret_cast<const float4 *>(row + (uint64_t)cl * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 q = src[i];
            v[4 * i] = q.x;
            v[4 * i + 1] = q.y;
            v[4 * i + 2] = q.z;
            v[4 * i + 3] = q.w;
        }
    }
    __device__ __forceinline__ float sum() const {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 32; j++) s += v[j];
        return s;
    }
};

// Runs `body(chunk, p)` for p in [beg, end), the chunk of input row row_of(p)
// loaded one row ahead (two buffers in turn).
template <typename RowOf, typename Body>
__device__ __forceinline__ void over_inputs(const float *in, uint32_t width, uint32_t cl, uint32_t beg,
                                            uint32_t end, RowOf row_of, Body body) {
    InChunk A, B;
    A.load(in + (uint64_t)row_of(beg) * width, cl);
#pragma unroll 1
    for (uint32_t p = beg; p < end; p += 2) {
        B.load(in + (uint64_t)row_of(min(p + 1, end - 1)) * width, cl);
        body(A, p);
        if (p + 1 < end) {
            A.load(in + (uint64_t)row_of(min(p + 2, end - 1)) * width, cl);
            body(B, p + 1);
        }
    }
}

// grid: x = row groups of kSegGateItems * kGateFR * rpi ff rows, y = entries.
template <int BITS, int ST, int LPR>
__global__ __launch_bounds__(64) void seg_gateup_kernel(SegArgs a) {
    const int lane = threadIdx.x;
    uint32_t e, beg, end;
    if (!seg_entry(a, blockIdx.y, e, beg, end)) return;
    const uint32_t in = a.w.in, ff = a.w.out;
    const uint32_t lpr = lanes_per_row<LPR>(a.w), rpi = 64u / lpr, sub = lane / lpr, cl = lane % lpr;
    LaneRows<BITS, ST, kGateFR> Lg[kSegGateItems], Lu[kSegGateItems];
#pragma unroll
    for (int q = 0; q < kSegGateItems; q++) {
        const uint32_t item = blockIdx.x * kSegGateItems + q;
        uint64_t rows[kGateFR];
        bool ok[kGateFR];
#pragma unroll
        for (int f = 0; f < kGateFR; f++) {
            const uint32_t j = (item * kGateFR + f) * rpi + sub;
            ok[f] = j < ff;
            rows[f] = (uint64_t)e * ff + j;
        }
        Lg[q].load(a.w, rows, ok, cl, lpr);
        Lu[q].load(a.w2, rows, ok, cl, lpr);
    }
    loads_issued();
    // 4-bit codes: the rows' code sums, once per entry (the limb products' offset)
    uint32_t csg[kSegGateItems][kGateFR], csu[kSegGateItems][kGateFR];
    if constexpr (BITS == 4) {
#pragma unroll
        for (int q = 0; q < kSegGateItems; q++) {
            Lg[q].template code_sums4<XLimbs>(csg[q]);
            Lu[q].template code_sums4<XLimbs>(csu[q]);
        }
    }
    over_inputs(a.in, in, cl, beg, end, [&](uint32_t p) { return a.perm ? a.perm[p] / a.k : p; },
                [&](const InChunk &X, uint32_t p) {
                    const float xs = X.sum();
                    // 4-bit codes: the input's limbs, shared by all the wave's rows
                    XLimbs xl;
                    if constexpr (BITS == 4) xl.build(X.v);
#pragma unroll
                    for (int q = 0; q < kSegGateItems; q++) {
                        Lg[q].pin();
                        Lu[q].pin();
                        const uint32_t item = blockIdx.x * kSegGateItems + q;
                        float g[kGateFR], u[kGateFR];
                        if constexpr (BITS == 4) {
                            Lg[q].dot_limbs(xl, xs, csg[q], g);
                            Lu[q].dot_limbs(xl, xs, csu[q], u);
                        } else {
                            Lg[q].dot(X.v, xs, g);
                            Lu[q].dot(X.v, xs, u);
                        }
                        gateup_epilogue(g, u, lane, lpr, rpi, sub, cl, item, ff, a.out + (uint64_t)p * ff);
                    }
                });
}

// Same as over_inputs for rows that span fewer than 64 lanes (rpi > 1
// sub-waves need the same chunk): each input row is loaded once per wave
// (lane l: float4s l, l + 64, ...), written to one of the wave's two LDS
// slots (float4 i of chunk c at i * C + c) and read back per sub-wave; the
// next row's loads are in flight while the current row is multiplied.
// NPL: float4s per lane when the width is a compile-time multiple of 256
// (every lane loads the same count, so the loads stay unconditional and in
// registers; a per-lane bound made the compiler wait on each load and keep
// the row in scratch); 0 for a run-time width.
template <int NPL, typename RowOf, typename Body>
__device__ __forceinline__ void over_inputs_staged(float4 *slots, const float *in, uint32_t width,
                                                   int lane, uint32_t cl, uint32_t beg, uint32_t end,
                                                   RowOf row_of, Body body) {
    constexpr int kMaxPerLane = NPL ? NPL : 8;  // width <= 2048
    const uint32_t C = width / 32, n4 = width / 4;
    f32x4 nx[kMaxPerLane];  // a plain vector type: HIP's float4 struct kept the row in scratch
    auto fetch = [&](uint32_t p) {
        const f32x4 *src = reinterpret_cast<const f32x4 *>(in + (uint64_t)row_of(p) * width);
#pragma unroll
        for (int j = 0; j < kMaxPerLane; j++)
            if (NPL || (uint32_t)(lane + 64 * j) < n4) nx[j] = src[lane + 64 * j];
    };
    fetch(beg);
#pragma unroll 1
    for (uint32_t p = beg; p < end; p++) {
        f32x4 *slot = reinterpret_cast<f32x4 *>(slots) + (p & 1) * n4;
#pragma unroll
        for (int j = 0; j < kMaxPerLane; j++) {
            const uint32_t w4 = lane + 64 * j;
            if (NPL || w4 < n4) slot[(w4 % 8) * C + w4 / 8] = nx[j];
        }
        if (p + 1 < end) fetch(p + 1);
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's slot writes landed
        __builtin_amdgcn_wave_barrier();
        InChunk X;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const f32x4 v = slot[i * C + cl];
            X.v[4 * i] = v[0];
            X.v[4 * i + 1] = v[1];
            X.v[4 * i + 2] = v[2];
            X.v[4 * i + 3] = v[3];
        }
        body(X, p);
    }
}

// grid: x = row groups of kSegRowsFR * rpi rows, y = entries.
template <int BITS, int ST, int LPR>
__global__ __launch_bounds__(64) void seg_rows_kernel(SegArgs a) {
    const int lane = threadIdx.x;
    uint32_t e, beg, end;
    if (!seg_entry(a, blockIdx.y, e, beg, end)) return;
    const uint32_t in = LPR ? (uint32_t)LPR * 32u : a.w.in, out = a.w.out;
    const uint32_t lpr = lanes_per_row<LPR>(a.w), rpi = 64u / lpr, sub = lane / lpr, cl = lane % lpr;
    uint64_t rows[kSegRowsFR];
    bool ok[kSegRowsFR];
    uint32_t r[kSegRowsFR];
#pragma unroll
    for (int f = 0; f < kSegRowsFR; f++) {
        r[f] = (blockIdx.x * kSegRowsFR + f) * rpi + sub;
        ok[f] = r[f] < out;
        rows[f] = (uint64_t)e * out + r[f];
    }
    LaneRows<BITS, ST, kSegRowsFR> L;
    L.load(a.w, rows, ok, cl, lpr);
    loads_issued();
    auto body = [&](const InChunk &X, uint32_t p) {
        L.pin();  // convert the codes per input row: all rows' would not fit
        float res[kSegRowsFR];
        L.dot(X.v, X.sum(), res);
#pragma unroll
        for (int f = 0; f < kSegRowsFR; f++) {
            const float v = subwave_sum(res[f], (int)lpr);
            if (cl == 0 && ok[f]) {
                const uint64_t o = (uint64_t)p * out + r[f];
                a.out[o] = a.bias ? v + a.bias[o] : v;
            }
        }
    };
    if constexpr (LPR != 64) {
        // rows of fewer than 64 lanes (the run-time width is never 64: those
        // rows take LPR 64): the input rows through the wave's LDS slots
        extern __shared__ float4 slots[];  // 2 x in / 4
        constexpr int kNpl = LPR * 32 % 256 == 0 ? LPR * 32 / 256 : 0;
        over_inputs_staged<kNpl>(slots, a.in, in, lane, cl, beg, end, [](uint32_t p) { return p; }, body);
    } else {
        over_inputs(a.in, in, cl, beg, end, [](uint32_t p) { return p; }, body);
    }
}

// ------------------------------------------------------------------ host --
static bool chunk_rows_ok(const WDesc &w) {
    if (w.in % 32) return false;
    const uint32_t c = w.in / 32;
    if (c < 1 || c > 64 || (c & (c - 1))) return false;
    if (w.bits == 0) return w.type == 0 || w.type == 1 || w.type == 30;
    return (w.bits == 2 || w.bits == 4 || w.bits == 8) && (w.type == 0 || w.type == 1 || w.type == 30);
}

bool seg_supported(const WDesc &w) { return chunk_rows_ok(w); }

uint32_t seg_max_entries(uint32_t pairs, uint32_t experts) {
    if (experts == 0) return (pairs + seg_run(pairs) - 1) / seg_run(pairs);
    return (pairs + kSegTokens - 1) / kSegTokens + (experts < pairs ? experts : pairs);
}
uint32_t seg_tokens() { return kSegTokens; }

template <int MODE>  // 0: seg_rows, 1: seg_gateup
struct SegLaunch {
    Prof *p;
    hipStream_t s;
    const SegArgs &a;
    uint32_t entries;
    const char *name;
    template <int BITS, int T, int LPR>
    hipError_t go() {
        const uint32_t rpi = 64u / (a.w.in / 32);
        if constexpr (MODE == 1) {
            const uint32_t per = kSegGateItems * kGateFR * rpi;
            return launch_kernel(p, name, seg_gateup_kernel<BITS, T, LPR>,
                                 dim3((a.w.out + per - 1) / per, entries), dim3(64), 0, s, a);
        } else {
            const uint32_t per = kSegRowsFR * rpi;
            // two input-row slots per wave when rows span fewer than 64 lanes
            const size_t lds = LPR != 64 ? 2 * (size_t)a.w.in * 4 : 0;
            return launch_kernel(p, name, seg_rows_kernel<BITS, T, LPR>,
                                 dim3((a.w.out + per - 1) / per, entries), dim3(64), lds, s, a);
        }
    }
    template <int BITS, int T>
    hipError_t operator()() {
        switch (a.w.in / 32) {
        case 64: return go<BITS, T, 64>();
        case 16: return go<BITS, T, 16>();
        default: return go<BITS, T, 0>();
        }
    }
};

hipError_t launch_seg_gateup(Prof *p, hipStream_t s, const char *name, const WDesc &gate,
                             const WDesc &up, const float *x, const uint32_t *perm, uint32_t k,
                             const uint32_t *tiles, const uint32_t *ntiles, const uint32_t *offsets,
                             uint32_t n, uint32_t entries, float *act) {
    if (entries == 0) return hipSuccess;
    if (gate.bits != up.bits || gate.type != up.type) return hipErrorInvalidValue;
    SegArgs a{};
    a.w = gate;
    a.w2 = up;
    a.in = x;
    a.perm = perm;
    a.k = k;
    a.tiles = tiles;
    a.ntiles = ntiles;
    a.offsets = offsets;
    a.n = n;
    a.run = seg_run(n);
    a.out = act;
    return dispatch_kind(gate, SegLaunch<1>{p, s, a, entries, name});
}

hipError_t launch_seg_rows(Prof *p, hipStream_t s, const char *name, const WDesc &w,
                           const float *in, const uint32_t *tiles, const uint32_t *ntiles,
                           const uint32_t *offsets, uint32_t n, uint32_t entries, const float *bias,
                           float *out) {
    if (entries == 0) return hipSuccess;
    SegArgs a{};
    a.w = w;
    a.w2 = w;
    a.in = in;
    a.tiles = tiles;
    a.ntiles = ntiles;
    a.offsets = offsets;
    a.n = n;
    a.run = seg_run(n);
    a.bias = bias;
    a.out = out;
    return dispatch_kind(w, SegLaunch<0>{p, s, a, entries, name});
}

}  // namespace moehip
