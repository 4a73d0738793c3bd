// Fused single-token MoE decode: three launches per layer.
//
//   decode_pre     router GEMV (+logit bias) and the shared expert's scalar
//                  gate input.
//   decode_gateup  every one-wave block re-derives its selection pass of the
//                  top-k routing from the logits (exact), then streams that
//                  expert's gate/up rows; blocks of the shared expert (no
//                  routing) stream theirs; all write SwiGLU activations.
//   decode_down    down rows of the K routed experts and the shared expert,
//                  weighted combine, sigmoid shared gate and residual.
//
// The lane layout and row products are in lanerows.hpp.
#include "lanerows.hpp"

namespace moehip {

// Per-wave phase stamps (s_memrealtime, a 100 MHz clock shared by the whole
// device) in the measurement build only (build.py --timeline defines
// MOE_TIMELINE): slot ranges decode_pre [0, 4096), decode_gateup [4096,
// 10240), decode_down [10240, 16384), eight stamps per slot.  Every lane
// stores the same value to the same address (no branch around the store, so
// the measured code is scheduled as in the normal build).
#ifdef MOE_TIMELINE
constexpr uint32_t kStampSlots = 16384;
__device__ uint64_t moe_stamps[kStampSlots * 8];
#define MOE_STAMP(slot, k) \
    (moe_stamps[min((uint32_t)(slot), kStampSlots - 1) * 8 + (k)] = __builtin_amdgcn_s_memrealtime())
#else
#define MOE_STAMP(slot, k) ((void)0)
#endif
constexpr uint32_t kStampPre = 0, kStampGate = 4096, kStampDown = 10240;

struct DecodeKArgs {
    WDesc router, gate, up, down, sg, su, sd, sgi;
    uint32_t has_shared, k, normalize;
    uint32_t h, ff, ffs, E;
    uint32_t lpr_h, lpr_f;  // lanes per row along h / along ff (powers of two <= 64)
    uint32_t n_router_waves, n_shared_waves, n_gate_waves_per_expert;
    const float *x, *norm_w, *logit_bias, *resid;
    float eps;
    float *out, *logits;
    uint32_t *ids;
    float *weights, *act, *sh_act, *sh_gate;
};

constexpr int kDownFR = 2;    // output rows per sub-wave in decode_down
constexpr int kPreFR = 2;     // router rows per sub-wave in decode_pre (one input slice each)

// ------------------------------------------------------------------ pre --
// One wave per block: kPreFR router rows per sub-wave (and the shared
// expert's scalar gate row).
template <int BR, int TR>
__device__ __forceinline__ void router_item(const DecodeKArgs &a, uint32_t wave_id, uint32_t sub,
                                            uint32_t cl, XChunk &X) {
    // router GEMV rows (Batch::matmul(router), crates/model-runtime/src/execute.rs:220)
    const uint32_t lpr = a.lpr_h, rpi = 64u / lpr;
    uint64_t e[kPreFR];
    bool ok[kPreFR];
#pragma unroll
    for (int f = 0; f < kPreFR; f++) {
        e[f] = ((uint64_t)wave_id * kPreFR + f) * rpi + sub;
        ok[f] = e[f] < a.E;
    }
    LaneRows<BR, TR, kPreFR> L;
    L.load(a.router, e, ok, cl, a.h / 32);
    // the logit bias loads with the rows (no bias: a dummy read of x[0]), so
    // its latency is not added after the products
    const float *bsrc = a.logit_bias ? a.logit_bias : a.x;
    float bias[kPreFR];
#pragma unroll
    for (int f = 0; f < kPreFR; f++) bias[f] = bsrc[a.logit_bias && ok[f] ? e[f] : 0u];
    loads_issued();
    const float xsum = X.finish(a.norm_w, a.eps, a.h, (int)lpr);
    float v[kPreFR];
    L.dot(X.xr, xsum, v);
#pragma unroll
    for (int f = 0; f < kPreFR; f++) {
        const float r = subwave_sum(v[f], (int)lpr);
        if (ok[f] && cl == 0) a.logits[e[f]] = a.logit_bias ? r + bias[f] : r;
    }
}

template <int ST>
__global__ __launch_bounds__(64) void decode_pre_kernel(DecodeKArgs a) {
    const int lane = threadIdx.x;
    const uint32_t wave_id = blockIdx.x;
    const uint32_t lpr = a.lpr_h, sub = lane / lpr, cl = lane % lpr;
    MOE_STAMP(kStampPre + wave_id, 0);
    XChunk X;
    X.load(a.x, a.norm_w, cl);
    if (wave_id < a.n_router_waves) {
        const WDesc &r = a.router;
        switch (r.bits) {
        case 2: router_item<2, ST>(a, wave_id, sub, cl, X); break;
        case 4: router_item<4, ST>(a, wave_id, sub, cl, X); break;
        case 8: router_item<8, ST>(a, wave_id, sub, cl, X); break;
        default:
            if (r.type == 0)
                router_item<0, 0>(a, wave_id, sub, cl, X);
            else if (r.type == 1)
                router_item<0, 1>(a, wave_id, sub, cl, X);
            else
                router_item<0, 30>(a, wave_id, sub, cl, X);
        }
        MOE_STAMP(kStampPre + wave_id, 1);
        return;
    }
    if (a.has_shared && wave_id == a.n_router_waves) {
        // shared-expert gate input [h] -> scalar (matmul(shared_gate [h,1]),
        // execute.rs:230; weight reshaped [h] -> [h,1], loader.rs:194)
        const float xsum = X.finish(a.norm_w, a.eps, a.h, (int)lpr);
        float v = 0.f;
        if (sub == 0) v = lane_row_dot_any<ST>(a.sgi, 0, cl, a.h / 32, X.xr, xsum);
        v = subwave_sum(v, (int)lpr);
        if (lane == 0) a.sh_gate[0] = v;
        MOE_STAMP(kStampPre + wave_id, 1);
    }
}

// --------------------------------------------------------------- gate/up --
template <int BS, int ST>
__device__ __forceinline__ void shared_item(const DecodeKArgs &a, uint32_t item, uint32_t sub,
                                            uint32_t cl, XChunk &X) {
    // shared expert gate/up + SwiGLU (encode_dense, execute.rs:258-264)
    const uint32_t lpr = a.lpr_h, rpi = 64u / lpr;
    uint64_t rows[kGateFR];
    bool ok[kGateFR];
#pragma unroll
    for (int f = 0; f < kGateFR; f++) {
        rows[f] = ((uint64_t)item * kGateFR + f) * rpi + sub;
        ok[f] = rows[f] < a.ffs;
    }
    LaneRows<BS, ST, kGateFR> Lg, Lu;
    Lg.load(a.sg, rows, ok, cl, a.h / 32);
    Lu.load(a.su, rows, ok, cl, a.h / 32);
    loads_issued();
    const float xsum = X.finish(a.norm_w, a.eps, a.h, (int)lpr);
    float g[kGateFR], u[kGateFR];
    Lg.dot(X.xr, xsum, g);
    Lu.dot(X.xr, xsum, u);
    gateup_epilogue(g, u, (int)(sub * lpr + cl), lpr, rpi, sub, cl, item, a.ffs, a.sh_act);
}

// One wave per block.  Waves [0, K*items) route the token (exactly, from the
// logits) and then compute kGateFR*rpi SwiGLU outputs of one selected expert;
// the next waves compute the shared expert's and need no routing, so their
// loads overlap the others' routing; the last wave derives the ids and
// weights the down kernel reads (the full selection, off the other waves'
// path).
template <int BITS, int ST>
__global__ __launch_bounds__(64) void decode_gateup_kernel(DecodeKArgs a) {
    extern __shared__ float route_vals[];  // E floats (routing with E > 1024 only)
    __shared__ uint32_t s_ids[64];
    __shared__ float s_w[64];
    __shared__ RouteLds route_lds;
    const int lane = threadIdx.x;
    const uint32_t lpr = a.lpr_h, rpi = 64u / lpr, sub = lane / lpr, cl = lane % lpr;
    const uint32_t wave_id = blockIdx.x;
    const uint32_t routed_waves = a.k * a.n_gate_waves_per_expert;
    const uint32_t shared_waves = a.has_shared ? a.n_shared_waves : 0u;
    MOE_STAMP(kStampGate + wave_id, 0);
    XChunk X;
    if (wave_id >= routed_waves + shared_waves) {
        // route (sampling.metal:1-36): all K ids and weights
        route_one_wave(&route_lds, route_vals, a.logits, a.E, a.k, (int)a.normalize, s_ids, s_w, lane);
        __syncthreads();
        if (lane < a.k) {
            a.ids[lane] = s_ids[lane];
            a.weights[lane] = s_w[lane];
        }
        MOE_STAMP(kStampGate + wave_id, 4);
        return;
    }
    if (wave_id >= routed_waves) {
        X.load(a.x, a.norm_w, cl);
        const uint32_t item = wave_id - routed_waves;
        switch (a.sg.bits) {
        case 2: shared_item<2, ST>(a, item, sub, cl, X); break;
        case 4: shared_item<4, ST>(a, item, sub, cl, X); break;
        default: shared_item<8, ST>(a, item, sub, cl, X); break;
        }
        MOE_STAMP(kStampGate + wave_id, 4);
        return;
    }
    // the id of this wave's selection pass kk of the same routing; the input
    // slice loads issue once the logits have arrived (before them, the
    // logits waited behind them)
    const uint32_t kk = wave_id / a.n_gate_waves_per_expert;
    const uint32_t item = wave_id % a.n_gate_waves_per_expert;
    const uint32_t e = route_one_id(&route_lds, route_vals, a.logits, a.E, a.k, kk, lane,
                                    [&]() { X.load(a.x, a.norm_w, cl); });  // < E by construction
    MOE_STAMP(kStampGate + wave_id, 1);
    uint64_t rows[kGateFR];
    bool ok[kGateFR];
#pragma unroll
    for (int f = 0; f < kGateFR; f++) {
        const uint32_t j = (item * kGateFR + f) * rpi + sub;
        ok[f] = j < a.ff;
        rows[f] = (uint64_t)e * a.ff + j;
    }
    LaneRows<BITS, ST, kGateFR> Lg, Lu;
    Lg.load(a.gate, rows, ok, cl, a.h / 32);
    Lu.load(a.up, rows, ok, cl, a.h / 32);
    loads_issued();
    MOE_STAMP(kStampGate + wave_id, 2);
    const float xsum = X.finish(a.norm_w, a.eps, a.h, (int)lpr);
    float g[kGateFR], u[kGateFR];
    Lg.dot(X.xr, xsum, g);
    Lu.dot(X.xr, xsum, u);
    MOE_STAMP(kStampGate + wave_id, 3);
    gateup_epilogue(g, u, lane, lpr, rpi, sub, cl, item, a.ff, a.act + (uint64_t)kk * a.ff);
    MOE_STAMP(kStampGate + wave_id, 4);
}

// ------------------------------------------------------------------ down --
// Block = nw waves over `rows_per_block` output rows; wave w takes experts
// w, w+nw, ... of the K routed experts plus the shared one (index K); all of
// a wave's weight loads are issued before its arithmetic, its expert's
// activation row reaches every sub-wave through the wave's LDS slot
// (staged_row), and the waves' partial sums meet in LDS.
constexpr int kDownMaxWaves = 16;
constexpr int kDownMaxPerWave = 2;
constexpr size_t kDownSlotBytes = 48 * 1024;  // beside the 16 KiB combine arrays

// This wave's activation row (ff floats) into xr: with a slot, through the
// wave's own LDS slot -- lane l loads float4s l, l + 64, ... once and every
// sub-wave reads its chunk from LDS (float4 i of chunk c at slot i * C + c,
// so a sub-wave's 16 lanes read consecutive slots); the direct loads fetched
// the row once per sub-wave (64 / lpr times).  Without a slot (rows too long
// for the block's LDS), direct loads.
// With a slot and ff a multiple of 256 the row is fetched first (fetch_row,
// every lane the same number of 16-byte loads, issued back to back: a caller
// issues them before its expert-id load) and written to the slot later; the
// loop of the general form waited for each load before its LDS write.
typedef float f32x4v __attribute__((ext_vector_type(4)));
constexpr int kRowLoadsMax = 8;  // ff <= 2048
struct RowRegs {
    f32x4v v[kRowLoadsMax];
};
__device__ __forceinline__ bool row_in_regs(uint32_t ff) { return ff % 256 == 0 && ff / 256 <= kRowLoadsMax; }
__device__ __forceinline__ void fetch_row(const float *src, uint32_t ff, int lane, RowRegs &r) {
    const f32x4v *s4 = reinterpret_cast<const f32x4v *>(src);
    const uint32_t nper = ff / 256;
#pragma unroll
    for (int j = 0; j < kRowLoadsMax; j++)
        if ((uint32_t)j < nper) r.v[j] = s4[lane + 64 * j];
}

template <bool SLOTS>
__device__ __forceinline__ void staged_row(float4 *slot, const float *src, uint32_t ff, int lane,
                                           uint32_t cl, float *xr, const RowRegs *pre = nullptr) {
    if constexpr (!SLOTS) {
        XChunk X;
        X.load(src, nullptr, cl);
#pragma unroll
        for (int j = 0; j < 32; j++) xr[j] = X.xr[j];
        return;
    }
    const uint32_t C = ff / 32, n4 = ff / 4;
    if (pre) {
        f32x4v *s = reinterpret_cast<f32x4v *>(slot);
        const uint32_t nper = ff / 256;
#pragma unroll
        for (int j = 0; j < kRowLoadsMax; j++) {
            const uint32_t w4 = lane + 64 * j;
            if ((uint32_t)j < nper) s[(w4 % 8) * C + w4 / 8] = pre->v[j];
        }
    } else {
        const float4 *s4 = reinterpret_cast<const float4 *>(src);
        for (uint32_t w4 = lane; w4 < n4; w4 += 64) slot[(w4 % 8) * C + w4 / 8] = s4[w4];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 v = slot[i * C + cl];
        xr[4 * i + 0] = v.x;
        xr[4 * i + 1] = v.y;
        xr[4 * i + 2] = v.z;
        xr[4 * i + 3] = v.w;
    }
}

template <int BITS, int ST, int BS, bool SLOTS>
__device__ __forceinline__ void down_wave(const DecodeKArgs &a, uint32_t wv, uint32_t nw,
                                          uint32_t row0, uint32_t sub, uint32_t cl, uint32_t rpi,
                                          float4 *slot, float *acc_r, float *acc_s) {
    const uint32_t n_exp = a.k + (a.has_shared ? 1u : 0u);
    const uint32_t C = a.ff / 32;
#pragma unroll
    for (int q = 0; q < kDownMaxPerWave; q++) {
        const uint32_t kk = wv + q * nw;
        if (kk >= n_exp) break;
        uint64_t rows[kDownFR];
        bool ok[kDownFR];
        float part[kDownFR];
        XChunk X;  // this expert's SwiGLU activations (no norm)
        if (kk < a.k) {
            // the activation row does not depend on the expert id: its loads
            // issue behind the id's, before the wait for it
            const uint32_t e = a.ids[kk];
            const float wk = a.weights[kk];
            const bool pre = SLOTS && row_in_regs(a.ff);
            RowRegs rr;
            if (pre) fetch_row(a.act + (uint64_t)kk * a.ff, a.ff, (int)(threadIdx.x & 63), rr);
#pragma unroll
            for (int f = 0; f < kDownFR; f++) {
                const uint32_t r = row0 + f * rpi + sub;
                ok[f] = r < a.h;
                rows[f] = (uint64_t)e * a.h + r;
            }
            LaneRows<BITS, ST, kDownFR> L;
            L.load(a.down, rows, ok, cl, C);
            loads_issued();
            MOE_STAMP(kStampDown + blockIdx.x * nw + wv, 1 + q);
            staged_row<SLOTS>(slot, a.act + (uint64_t)kk * a.ff, a.ff, (int)(threadIdx.x & 63), cl, X.xr,
                              pre ? &rr : nullptr);
            L.dot(X.xr, X.finish(nullptr, 0.f, 0, 0), part);
#pragma unroll
            for (int f = 0; f < kDownFR; f++) acc_r[f] += part[f] * wk;
        } else {
            const bool pre = SLOTS && row_in_regs(a.ff);
            RowRegs rr;
            if (pre) fetch_row(a.sh_act, a.ff, (int)(threadIdx.x & 63), rr);
#pragma unroll
            for (int f = 0; f < kDownFR; f++) {
                const uint32_t r = row0 + f * rpi + sub;
                ok[f] = r < a.h;
                rows[f] = r;
            }
            LaneRows<BS, ST, kDownFR> L;
            L.load(a.sd, rows, ok, cl, C);
            loads_issued();
            staged_row<SLOTS>(slot, a.sh_act, a.ff, (int)(threadIdx.x & 63), cl, X.xr, pre ? &rr : nullptr);
            L.dot(X.xr, X.finish(nullptr, 0.f, 0, 0), part);
#pragma unroll
            for (int f = 0; f < kDownFR; f++) acc_s[f] += part[f];
        }
    }
}

template <int BITS, int ST, bool SLOTS>
__global__ __launch_bounds__(64 * kDownMaxWaves) void decode_down_kernel(DecodeKArgs a) {
    __shared__ float red_r[kDownMaxWaves][128];
    __shared__ float red_s[kDownMaxWaves][128];
    extern __shared__ float4 dslot[];  // [waves][ff / 4] with SLOTS
    const int lane = threadIdx.x & 63;
    const uint32_t wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint32_t lpr = a.lpr_f, rpi = 64u / lpr, sub = lane / lpr, cl = lane % lpr;
    const uint32_t rows_per_block = rpi * kDownFR;
    const uint32_t row0 = blockIdx.x * rows_per_block;
    float4 *slot = SLOTS ? dslot + wv * (a.ff / 4) : nullptr;
    const uint32_t stamp = kStampDown + blockIdx.x * nw + wv;
    MOE_STAMP(stamp, 0);
    // issued first: needed only after the LDS combine
    const float shared_gate = a.has_shared ? a.sh_gate[0] : 0.f;
    float acc_r[kDownFR], acc_s[kDownFR];
#pragma unroll
    for (int f = 0; f < kDownFR; f++) acc_r[f] = acc_s[f] = 0.f;
    switch (a.has_shared ? a.sd.bits : BITS) {
    case 2: down_wave<BITS, ST, 2, SLOTS>(a, wv, nw, row0, sub, cl, rpi, slot, acc_r, acc_s); break;
    case 4: down_wave<BITS, ST, 4, SLOTS>(a, wv, nw, row0, sub, cl, rpi, slot, acc_r, acc_s); break;
    default: down_wave<BITS, ST, 8, SLOTS>(a, wv, nw, row0, sub, cl, rpi, slot, acc_r, acc_s); break;
    }
    MOE_STAMP(stamp, 3);
    static_assert(kDownFR == 2, "reduce-scatter layout assumes two rows per sub-wave");
    if (lpr >= 16) {
        float r, sh;
        rs2_pairs(acc_r, acc_s, lane, lpr, r, sh);
        if (cl < 2) {
            red_r[wv][cl * rpi + sub] = r;
            red_s[wv][cl * rpi + sub] = sh;
        }
    } else {
#pragma unroll
        for (int f = 0; f < kDownFR; f++) {
            const float r = subwave_sum(acc_r[f], (int)lpr), sh = subwave_sum(acc_s[f], (int)lpr);
            if (cl == 0) {
                red_r[wv][f * rpi + sub] = r;
                red_s[wv][f * rpi + sub] = sh;
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < rows_per_block) {
        const uint32_t i = threadIdx.x, row = row0 + i;
        if (row < a.h) {
            // mix (elementwise.metal:47-57), then shared / (1+exp(-g)) and add
            // (gate_scalar + add, execute.rs:231-232), then the residual
            // (execute.rs:236)
            float v = 0.f, sv = 0.f;
            for (uint32_t w = 0; w < nw; w++) {
                v += red_r[w][i];
                sv += red_s[w][i];
            }
            if (a.has_shared) v = v + sv / (1.0f + expf(-shared_gate));
            if (a.resid) v = a.resid[row] + v;
            a.out[row] = v;
        }
    }
    MOE_STAMP(stamp, 4);
}

// ------------------------------------------------------------------ host --
static bool pow2_chunks(uint32_t n) {
    if (n % 32) return false;
    const uint32_t c = n / 32;
    return c >= 1 && c <= 64 && (c & (c - 1)) == 0;
}
static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool decode_supported(const DecodeArgs &a) {
    const WDesc &g = a.gate;
    if (g.bits == 0 || a.up.bits != g.bits || a.down.bits != g.bits) return false;
    if (a.up.type != g.type || a.down.type != g.type) return false;
    const uint32_t st = g.type;
    if (!pow2_chunks(g.in) || !pow2_chunks(g.out)) return false;
    if (a.router.bits && a.router.type != st) return false;
    if (a.router.out > 4096 || a.k == 0 || a.k > 64 || a.k > a.router.out) return false;
    // the down kernel covers at most kDownMaxWaves * kDownMaxPerWave experts
    if (a.k + (a.has_shared ? 1u : 0u) > (uint32_t)(kDownMaxWaves * kDownMaxPerWave)) return false;
    if (a.has_shared) {
        if (a.sg.bits == 0 || a.su.bits != a.sg.bits || a.sd.bits != a.sg.bits) return false;
        if (a.sg.type != st || a.su.type != st || a.sd.type != st) return false;
        if (a.sg.out != g.out) return false;  // shared ff == routed ff (same down layout)
        if (a.sgi.bits && a.sgi.type != st) return false;
    }
    const WDesc *all[] = {&a.router, &a.gate, &a.up, &a.down, &a.sg, &a.su, &a.sd, &a.sgi};
    const int n = a.has_shared ? 8 : 4;
    for (int i = 0; i < n; i++)
        if (!aligned16(all[i]->data)) return false;
    if (!aligned16(a.x) || !aligned16(a.act) || !aligned16(a.sh_act)) return false;
    if (a.norm_w && !aligned16(a.norm_w)) return false;
    return true;
}

template <int BITS, int ST>
static hipError_t launch_decode_t(Prof *p, hipStream_t s, const DecodeKArgs &k) {
    const uint32_t pre_waves = k.n_router_waves + (k.has_shared ? 1 : 0);
    hipError_t e = launch_kernel(p, "decode_pre", decode_pre_kernel<ST>, dim3(pre_waves), dim3(64), 0,
                                 s, k);
    if (e != hipSuccess) return e;
    // routed waves, shared-expert waves, and the wave that writes ids and weights
    const uint32_t gate_waves = k.k * k.n_gate_waves_per_expert + (k.has_shared ? k.n_shared_waves : 0) + 1;
    const size_t lds = k.E > 1024 ? (size_t)k.E * sizeof(float) : 0;
    e = launch_kernel(p, "decode_gateup", decode_gateup_kernel<BITS, ST>, dim3(gate_waves), dim3(64),
                      lds, s, k);
    if (e != hipSuccess) return e;
    const uint32_t rows_per_block = (64u / k.lpr_f) * kDownFR;
    const uint32_t n_exp = k.k + (k.has_shared ? 1u : 0u);
    const uint32_t nw = n_exp < (uint32_t)kDownMaxWaves ? n_exp : (uint32_t)kDownMaxWaves;
    // one activation-row slot per wave when they fit beside the combine arrays
    const size_t slots = (size_t)nw * k.ff * 4;
    const dim3 grid((k.h + rows_per_block - 1) / rows_per_block), block(64 * nw);
    if (slots <= kDownSlotBytes)
        return launch_kernel(p, "decode_down", decode_down_kernel<BITS, ST, true>, grid, block, slots, s, k);
    return launch_kernel(p, "decode_down", decode_down_kernel<BITS, ST, false>, grid, block, 0, s, k);
}

hipError_t launch_decode(Prof *p, hipStream_t s, const DecodeArgs &a) {
    DecodeKArgs k{};
    k.router = a.router; k.gate = a.gate; k.up = a.up; k.down = a.down;
    k.sg = a.sg; k.su = a.su; k.sd = a.sd; k.sgi = a.sgi;
    k.has_shared = a.has_shared; k.k = a.k; k.normalize = a.normalize;
    k.h = a.gate.in; k.ff = a.gate.out; k.ffs = a.has_shared ? a.sg.out : 0; k.E = a.router.out;
    k.lpr_h = k.h / 32; k.lpr_f = k.ff / 32;
    const uint32_t rpi_h = 64u / k.lpr_h;
    k.n_router_waves = (k.E + rpi_h * kPreFR - 1) / (rpi_h * kPreFR);
    k.n_shared_waves = (k.ffs + rpi_h * kGateFR - 1) / (rpi_h * kGateFR);
    k.n_gate_waves_per_expert = (k.ff + rpi_h * kGateFR - 1) / (rpi_h * kGateFR);
    k.x = a.x; k.norm_w = a.norm_w; k.eps = a.eps; k.logit_bias = a.logit_bias; k.resid = a.resid;
    k.out = a.out; k.logits = a.logits; k.ids = a.ids; k.weights = a.weights; k.act = a.act;
    k.sh_act = a.sh_act; k.sh_gate = a.sh_gate;
    const uint32_t st = a.gate.type;
#define DEC_CASE(B, T) if (a.gate.bits == B && st == T) return launch_decode_t<B, T>(p, s, k);
    DEC_CASE(2, 0) DEC_CASE(2, 1) DEC_CASE(2, 30)
    DEC_CASE(4, 0) DEC_CASE(4, 1) DEC_CASE(4, 30)
    DEC_CASE(8, 0) DEC_CASE(8, 1) DEC_CASE(8, 30)
#undef DEC_CASE
    return hipErrorInvalidValue;
}

}  // namespace moehip

#ifdef MOE_TIMELINE
// Copies the phase stamps out (the measurement build's only export beyond
// the C ABI).
extern "C" int moe_timeline_read(void *dst, size_t bytes) {
    if (bytes > sizeof(moehip::moe_stamps)) return (int)hipErrorInvalidValue;
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(moehip::moe_stamps), bytes, 0, hipMemcpyDeviceToHost);
}
extern "C" int moe_timeline_clear(void) {
    static uint64_t zeros[moehip::kStampSlots * 8];
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(moehip::moe_stamps), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
}
#endif
