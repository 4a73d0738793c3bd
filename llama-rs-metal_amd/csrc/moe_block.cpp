// moe_block: one MoE block over T tokens behind the C ABI, plus profiling and
// graph capture.  The composition follows crates/model-runtime/src/execute.rs:200-236
// (router -> route -> gate/up -> swiglu -> down -> mix -> shared expert ->
// sigmoid gate -> add -> residual), with three interchangeable executions:
//   MOE_PATH_OPS      the reference's own per-token op sequence (14 ops per token)
//   MOE_PATH_GROUPED  token-batched: route all tokens, dispatch by expert,
//                     grouped expert products, one combine
//   MOE_PATH_AUTO     fused 3-kernel decode for one token; bf16 MFMA for
//                     prefill-sized segments; the batched decode
//                     (k_batched.hip) for a few tokens; grouped otherwise
#include "abi_common.hpp"

namespace {

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct WsLayout {
    uint64_t logits, ids, weights, counts, offsets, perm, pos, act, yexp, sh_act, sh_up, sh_gate,
        sh_out, xnorm, gates, ups, eo, proj, sgv, xb16, act16, y16, tiles, ntiles, sh_sched, total;
};

inline uint64_t al64(uint64_t n) { return (n + 63) & ~63ull; }

WsLayout ws_layout(uint64_t T, uint64_t E, uint64_t K, uint64_t h, uint64_t ff, uint64_t ffs) {
    WsLayout L{};
    uint64_t o = 0;
    auto take = [&](uint64_t &field, uint64_t n) {
        field = o;
        o += al64(n ? n : 1);
    };
    take(L.logits, T * E);
    take(L.ids, T * K);
    take(L.weights, T * K);
    take(L.counts, E);
    take(L.offsets, E + 1);
    take(L.perm, T * K);
    take(L.pos, T * K);
    take(L.act, T * K * ff);
    take(L.yexp, T * K * h);
    take(L.sh_act, T * ffs);
    take(L.sh_up, T * ffs);
    take(L.sh_gate, T);
    take(L.sh_out, T * h);
    take(L.xnorm, T * h);
    take(L.gates, K * ff);
    take(L.ups, K * ff);
    take(L.eo, K * h);
    take(L.proj, h);
    take(L.sgv, 1);
    // bf16 MFMA path (two bf16 per 4-byte element); with a shared expert its
    // T rows follow the T * K routed pairs in act16 and y16 (it runs as one
    // more segment of the routed GEMMs where its kind allows)
    take(L.xb16, (T * h + 1) / 2);
    take(L.act16, (T * K * ff + T * (ffs > ff ? ffs : ff) * (ffs ? 1 : 0) + 1) / 2);
    take(L.y16, (T * K * h + (ffs ? T * h : 0) + 1) / 2);
    take(L.tiles, 2 * ((T * K + 7) / 8 + E + 1));  // MFMA tiles of 128 pairs, batched runs of 8
    take(L.ntiles, 1);
    // the shared expert's one-segment schedule on the MFMA path: offsets [2],
    // M-tiles of 128 rows [2 * ceil(T / 128)], their count
    take(L.sh_sched, 3 + 2 * ((T + 127) / 128));
    L.total = o;
    return L;
}

struct Dims {
    uint64_t h, ff, E, K, ffs;
};

// Shape contract of the MoE binding (crates/model-runtime/src/loader.rs:172-203).
moe_status check_block(moe_gpu *g, const moe_block_weights *w, Dims &d) {
    if (!w) return shape(g, "missing block weights");
    moe_status st;
    if ((st = check_weight(g, &w->router, "router")) || (st = check_weight(g, &w->gate, "expert gates")) ||
        (st = check_weight(g, &w->up, "expert ups")) || (st = check_weight(g, &w->down, "expert downs")))
        return st;
    const moe_weight &r = w->router, &ga = w->gate, &u = w->up, &dn = w->down;
    if (r.ndims != 2 || ga.ndims != 3 || u.ndims != 3 || dn.ndims != 3)
        return shape(g, "MoE routing dimensions");
    d.h = r.dims[0];
    d.E = r.dims[1];
    d.K = w->experts_used;
    if (d.K == 0 || d.K > d.E) return shape(g, "MoE routing dimensions");
    if (ga.dims[0] != d.h || ga.dims[2] != d.E) return shape(g, "expert gates dimensions");
    d.ff = ga.dims[1];
    if (u.dims[0] != d.h || u.dims[1] != d.ff || u.dims[2] != d.E) return shape(g, "expert ups dimensions");
    if (dn.dims[0] != d.ff || dn.dims[1] != d.h || dn.dims[2] != d.E)
        return shape(g, "expert downs dimensions");
    d.ffs = 0;
    if (w->has_shared) {
        if ((st = check_weight(g, &w->shared_gate, "shared gate")) ||
            (st = check_weight(g, &w->shared_up, "shared up")) ||
            (st = check_weight(g, &w->shared_down, "shared down")) ||
            (st = check_weight(g, &w->shared_gate_inp, "shared expert gate")))
            return st;
        const moe_weight &sg = w->shared_gate, &su = w->shared_up, &sd = w->shared_down,
                         &gi = w->shared_gate_inp;
        if (sg.ndims != 2 || sg.dims[0] != d.h) return shape(g, "shared gate dimensions");
        d.ffs = sg.dims[1];
        if (su.ndims != 2 || su.dims[0] != d.h || su.dims[1] != d.ffs) return shape(g, "shared up dimensions");
        if (sd.ndims != 2 || sd.dims[0] != d.ffs || sd.dims[1] != d.h)
            return shape(g, "shared down dimensions");
        if (gi.dims[0] != d.h || (gi.ndims == 2 && gi.dims[1] != 1) || gi.ndims > 2)
            return shape(g, "shared expert gate dimensions");
    }
    if (d.E > 16384) return shape(g, "more than 16384 experts");
    // optional packed copies: sized for their weight, owned, disjoint from it
    const moe_packed_weight *pk[6] = {&w->gate_packed,        &w->up_packed,        &w->down_packed,
                                      &w->shared_gate_packed, &w->shared_up_packed, &w->shared_down_packed};
    const moe_weight *pw[6] = {&w->gate, &w->up, &w->down, &w->shared_gate, &w->shared_up, &w->shared_down};
    for (int i = 0; i < 6; i++) {
        if (i >= 3 && !w->has_shared && (pk[i]->data.ptr || pk[i]->scales.ptr || pk[i]->biases.ptr))
            return shape(g, "packed shared expert weights without a shared expert");
        if (!pk[i]->data.ptr && !pk[i]->scales.ptr && !pk[i]->biases.ptr) continue;
        uint64_t db = 0, sb = 0;
        if (!pack_layout(wdesc(*pw[i]), &db, &sb) || pk[i]->data.bytes != db || pk[i]->scales.bytes != sb ||
            pk[i]->biases.bytes != sb)
            return shape(g, "packed expert weight: no packed form, or sizes");
        if ((st = check_own(g, {rng(pk[i]->data), rng(pk[i]->scales), rng(pk[i]->biases)}))) return st;
    }
    if (!w->gate_packed.data.ptr != !w->up_packed.data.ptr)
        return shape(g, "packed expert weights: gate and up together");
    if (!w->shared_gate_packed.data.ptr != !w->shared_up_packed.data.ptr)
        return shape(g, "packed shared expert weights: gate and up together");
    return MOE_OK;
}

PackedW packed(const moe_packed_weight &p) {
    return PackedW{p.data.ptr, p.scales.ptr, p.biases.ptr};
}

float *fp(const moe_buffer &b, uint64_t off = 0) { return static_cast<float *>(b.ptr) + off; }
uint32_t *up32(const moe_buffer &b, uint64_t off = 0) { return static_cast<uint32_t *>(b.ptr) + off; }
bool has(const moe_buffer &b) { return b.ptr != nullptr && b.len != 0; }

WDesc gate_inp_desc(const moe_weight &w) {
    WDesc d = wdesc(w);
    d.out = 1;  // [h] reshaped [h, 1] (loader.rs:194)
    d.experts = 1;
    return d;
}

#define TRY(expr)                                       \
    do {                                                \
        hipError_t e_ = (expr);                         \
        if (e_ != hipSuccess) return gpu_err(g, e_, #expr); \
    } while (0)

// Work forked onto the gpu's side stream (the shared expert) joins the main
// stream on every exit: at join() on success, else when the guard goes out of
// scope after a failed launch, so a capture never ends with the side stream
// still forked and eager work on the side stream is ordered before the main
// stream's later work.
struct SideFork {
    moe_gpu *g;
    hipStream_t main;
    bool open = false;
    // mark() records the fork point on the main stream; enter() makes the
    // side stream start from it.  Main-stream work queued between the two
    // does not gate the side stream, but is queued ahead of it.
    hipError_t mark() { return hipEventRecord(g->ev_fork, main); }
    hipError_t enter() {
        const hipError_t e = hipStreamWaitEvent(g->side, g->ev_fork, 0);
        open = e == hipSuccess;
        return e;
    }
    hipError_t fork() {
        const hipError_t e = mark();
        return e == hipSuccess ? enter() : e;
    }
    hipError_t join() {
        if (!open) return hipSuccess;
        open = false;
        hipError_t e = hipEventRecord(g->ev_join, g->side);
        return e == hipSuccess ? hipStreamWaitEvent(main, g->ev_join, 0) : e;
    }
    ~SideFork() { (void)join(); }
};

// The reference's per-token op sequence (execute.rs:208-233 and encode_dense :251-267).
moe_status run_ops(moe_gpu *g, const moe_block_weights *w, const Dims &d, const float *xin,
                   const float *xres, float *out, uint64_t T, const moe_block_io *io,
                   const WsLayout &L, float *ws, float *logits, uint32_t *ids, float *wts) {
    Prof *p = &g->prof;
    hipStream_t s = g->stream;
    const WDesc R = wdesc(w->router), G = wdesc(w->gate), U = wdesc(w->up), D = wdesc(w->down);
    const uint32_t K = (uint32_t)d.K;
    float *gates = ws + L.gates, *ups = ws + L.ups, *eo = ws + L.eo, *proj = ws + L.proj;
    for (uint64_t t = 0; t < T; t++) {
        const float *xt = xin + t * d.h;
        float *lt = logits + t * d.E;
        uint32_t *it = ids + t * K;
        float *wt = wts + t * K;
        TRY(launch_gemv(p, s, R, xt, 0, nullptr, 1, lt, 1));
        if (has(io->logit_bias)) TRY(launch_add(p, s, lt, fp(io->logit_bias, t * d.E), lt, d.E));
        TRY(launch_route(p, s, lt, (uint32_t)d.E, K, w->normalize ? 1 : 0, 1, it, wt));
        TRY(launch_gemv(p, s, G, xt, 0, it, K, gates, 1));
        TRY(launch_gemv(p, s, U, xt, 0, it, K, ups, 1));
        TRY(launch_swiglu(p, s, gates, ups, gates, K * d.ff));
        TRY(launch_gemv(p, s, D, gates, d.ff, it, K, eo, 1));
        TRY(launch_mix(p, s, eo, wt, K, d.h, proj));
        if (w->has_shared) {
            float *sg = ws + L.sh_act, *su = ws + L.sh_up, *so = ws + L.sh_out, *sgv = ws + L.sgv;
            TRY(launch_gemv(p, s, wdesc(w->shared_gate), xt, 0, nullptr, 1, sg, 1));
            TRY(launch_gemv(p, s, wdesc(w->shared_up), xt, 0, nullptr, 1, su, 1));
            TRY(launch_swiglu(p, s, sg, su, sg, d.ffs));
            TRY(launch_gemv(p, s, wdesc(w->shared_down), sg, 0, nullptr, 1, so, 1));
            TRY(launch_gemv(p, s, gate_inp_desc(w->shared_gate_inp), xt, 0, nullptr, 1, sgv, 1));
            TRY(launch_gate_scalar(p, s, so, sgv, so, d.h));
            TRY(launch_add(p, s, proj, so, proj, d.h));
        }
        if (io->residual)
            TRY(launch_add(p, s, xres + t * d.h, proj, out + t * d.h, d.h));
        else
            TRY(launch_copy(p, s, proj, out + t * d.h, d.h));
    }
    return MOE_OK;
}

moe_status run_grouped(moe_gpu *g, const moe_block_weights *w, const Dims &d, const float *xin,
                       const float *xres, float *out, uint64_t T, const moe_block_io *io,
                       const WsLayout &L, float *ws, float *logits, uint32_t *ids, float *wts) {
    Prof *p = &g->prof;
    hipStream_t s = g->stream;
    const uint32_t K = (uint32_t)d.K, E = (uint32_t)d.E;
    const WDesc G = wdesc(w->gate), U = wdesc(w->up), D = wdesc(w->down);
    uint32_t *counts = reinterpret_cast<uint32_t *>(ws + L.counts);
    uint32_t *offsets = reinterpret_cast<uint32_t *>(ws + L.offsets);
    uint32_t *perm = reinterpret_cast<uint32_t *>(ws + L.perm);
    uint32_t *pos = reinterpret_cast<uint32_t *>(ws + L.pos);
    float *act = ws + L.act, *yexp = ws + L.yexp;
    TRY(launch_gemv(p, s, wdesc(w->router), xin, 0, nullptr, 1, logits, (uint32_t)T));
    if (has(io->logit_bias)) TRY(launch_add(p, s, logits, fp(io->logit_bias), logits, T * d.E));
    TRY(launch_route(p, s, logits, E, K, w->normalize ? 1 : 0, (uint32_t)T, ids, wts));
    TRY(launch_dispatch(p, s, ids, (uint32_t)(T * K), E, counts, offsets, perm, pos));
    TRY(launch_grouped_gateup(p, s, G, U, xin, offsets, perm, K, E, act));
    TRY(launch_grouped_down(p, s, D, act, offsets, E, (uint32_t)(T * K), yexp));
    const float *so = nullptr, *sgv = nullptr;
    if (w->has_shared) {
        float *sg = ws + L.sh_act, *su = ws + L.sh_up, *sout = ws + L.sh_out, *sgt = ws + L.sh_gate;
        TRY(launch_gemv(p, s, wdesc(w->shared_gate), xin, 0, nullptr, 1, sg, (uint32_t)T));
        TRY(launch_gemv(p, s, wdesc(w->shared_up), xin, 0, nullptr, 1, su, (uint32_t)T));
        TRY(launch_swiglu(p, s, sg, su, sg, T * d.ffs));
        TRY(launch_gemv(p, s, wdesc(w->shared_down), sg, 0, nullptr, 1, sout, (uint32_t)T));
        TRY(launch_gemv(p, s, gate_inp_desc(w->shared_gate_inp), xin, 0, nullptr, 1, sgt, (uint32_t)T));
        so = sout;
        sgv = sgt;
    }
    TRY(launch_combine(p, s, yexp, pos, wts, K, so, sgv, io->residual ? xres : nullptr, out,
                       (uint32_t)T, (uint32_t)d.h));
    return MOE_OK;
}

// Batched decode (k_batched.hip): several tokens whose expert segments are
// too short for the MFMA path.  Same composition as run_grouped; every
// product streams its weight rows once per run of seg_tokens() inputs.
bool batched_ok(const moe_block_weights *w) {
    const WDesc G = wdesc(w->gate), U = wdesc(w->up), D = wdesc(w->down);
    if (!seg_supported(wdesc(w->router)) || !seg_supported(G) || !seg_supported(U) ||
        !seg_supported(D) || G.bits != U.bits || G.type != U.type)
        return false;
    if (w->has_shared) {
        const WDesc SG = wdesc(w->shared_gate), SU = wdesc(w->shared_up);
        if (!seg_supported(SG) || !seg_supported(SU) || !seg_supported(wdesc(w->shared_down)) ||
            !seg_supported(gate_inp_desc(w->shared_gate_inp)) || SG.bits != SU.bits ||
            SG.type != SU.type)
            return false;
    }
    return true;
}

moe_status run_batched(moe_gpu *g, const moe_block_weights *w, const Dims &d, const float *xin,
                       const float *xres, float *out, uint64_t T, const moe_block_io *io,
                       const WsLayout &L, float *ws, float *logits, uint32_t *ids, float *wts) {
    Prof *p = &g->prof;
    hipStream_t s = g->stream;
    const uint32_t K = (uint32_t)d.K, E = (uint32_t)d.E, t32 = (uint32_t)T;
    uint32_t *counts = reinterpret_cast<uint32_t *>(ws + L.counts);
    uint32_t *offsets = reinterpret_cast<uint32_t *>(ws + L.offsets);
    uint32_t *perm = reinterpret_cast<uint32_t *>(ws + L.perm);
    uint32_t *pos = reinterpret_cast<uint32_t *>(ws + L.pos);
    uint32_t *tiles = reinterpret_cast<uint32_t *>(ws + L.tiles);
    uint32_t *ntiles = reinterpret_cast<uint32_t *>(ws + L.ntiles);
    float *act = ws + L.act, *yexp = ws + L.yexp;
    const uint32_t runs = seg_max_entries(t32, 0), entries = seg_max_entries(t32 * K, E);
    const float *bias = has(io->logit_bias) ? fp(io->logit_bias) : nullptr;
    // the shared expert needs only the input: it runs on the side stream,
    // concurrently with the routed chain, and joins before the combine.  Its
    // fork point precedes the router, but the router is queued first: a
    // replayed graph then starts the router ahead of the shared expert's
    // kernels (config 3 at 8/32/64 tokens: 78.7/173.4/273.2 ->
    // 71.0/166.0/271.3 us, against queuing the shared expert first)
    const float *so = nullptr, *sgv = nullptr;
    SideFork side{g, s};
    if (w->has_shared) TRY(side.mark());
    TRY(launch_seg_rows(p, s, "seg_router", wdesc(w->router), xin, nullptr, nullptr, nullptr, t32, runs,
                        bias, logits));
    if (w->has_shared) {
        float *sh = ws + L.sh_act, *sout = ws + L.sh_out, *sgt = ws + L.sh_gate;
        hipStream_t ss = g->side;
        TRY(side.enter());
        TRY(launch_seg_gateup(p, ss, "seg_shared_gateup", wdesc(w->shared_gate), wdesc(w->shared_up), xin,
                              nullptr, 1, nullptr, nullptr, nullptr, t32, runs, sh));
        TRY(launch_seg_rows(p, ss, "seg_shared_down", wdesc(w->shared_down), sh, nullptr, nullptr, nullptr,
                            t32, runs, nullptr, sout));
        TRY(launch_seg_rows(p, ss, "seg_shared_gate", gate_inp_desc(w->shared_gate_inp), xin, nullptr,
                            nullptr, nullptr, t32, runs, nullptr, sgt));
        so = sout;
        sgv = sgt;
    }
    if (route_dispatch_fits(E, K, t32)) {
        TRY(launch_route_dispatch(p, s, logits, E, K, w->normalize ? 1 : 0, t32, ids, wts, g->arrive,
                                  seg_tokens(), counts, offsets, perm, pos, tiles, ntiles));
    } else {
        TRY(launch_route(p, s, logits, E, K, w->normalize ? 1 : 0, t32, ids, wts));
        TRY(launch_dispatch(p, s, ids, t32 * K, E, counts, offsets, perm, pos, seg_tokens(), tiles, ntiles));
    }
    TRY(launch_seg_gateup(p, s, "seg_gateup", wdesc(w->gate), wdesc(w->up), xin, perm, K, tiles, ntiles,
                          offsets, 0, entries, act));
    TRY(launch_seg_rows(p, s, "seg_down", wdesc(w->down), act, tiles, ntiles, offsets, 0, entries,
                        nullptr, yexp));
    TRY(side.join());
    TRY(launch_combine(p, s, yexp, pos, wts, K, so, sgv, io->residual ? xres : nullptr, out, t32,
                       (uint32_t)d.h));
    return MOE_OK;
}

// The shared expert runs on the grouped bf16 GEMM too when its kinds allow
// (gate and up of one kind; K of both products a multiple of 128).
bool shared_mfma_ok(const moe_block_weights *w) {
    if (!w->has_shared) return false;
    const WDesc SG = wdesc(w->shared_gate), SU = wdesc(w->shared_up), SD = wdesc(w->shared_down);
    return gemm_supported(SG) && gemm_supported(SU) && gemm_supported(SD) && SG.bits == SU.bits &&
           SG.type == SU.type && SG.gshift == SU.gshift;
}

bool mfma_path_ok(const moe_block_weights *w, const Dims &d) {
    const WDesc G = wdesc(w->gate), U = wdesc(w->up), D = wdesc(w->down);
    return gemm_supported(G) && gemm_supported(U) && gemm_supported(D) && G.bits == U.bits &&
           G.type == U.type && d.h % 128 == 0 && d.ff % 128 == 0;
}

// bf16 MFMA grouped path (prefill-sized expert segments).
moe_status run_mfma(moe_gpu *g, const moe_block_weights *w, const Dims &d, const float *xraw,
                    const float *nw, float eps, float *out, uint64_t T, const moe_block_io *io,
                    const WsLayout &L, float *ws, float *logits, uint32_t *ids, float *wts) {
    Prof *p = &g->prof;
    hipStream_t s = g->stream;
    const uint32_t K = (uint32_t)d.K, E = (uint32_t)d.E;
    uint16_t *xb16 = reinterpret_cast<uint16_t *>(ws + L.xb16);
    uint16_t *act16 = reinterpret_cast<uint16_t *>(ws + L.act16);
    uint16_t *y16 = reinterpret_cast<uint16_t *>(ws + L.y16);
    uint32_t *counts = reinterpret_cast<uint32_t *>(ws + L.counts);
    uint32_t *offsets = reinterpret_cast<uint32_t *>(ws + L.offsets);
    uint32_t *perm = reinterpret_cast<uint32_t *>(ws + L.perm);
    uint32_t *pos = reinterpret_cast<uint32_t *>(ws + L.pos);
    uint32_t *tiles = reinterpret_cast<uint32_t *>(ws + L.tiles);
    uint32_t *ntiles = reinterpret_cast<uint32_t *>(ws + L.ntiles);
    float *xn = nw ? ws + L.xnorm : nullptr;
    const float *xin = nw ? xn : xraw;  // F32 input of the router and the VALU products
    const WDesc R = wdesc(w->router);
    const float *bias = has(io->logit_bias) ? fp(io->logit_bias) : nullptr;
    // The shared expert as one more segment of the routed experts' GEMMs
    // (its rows after the T * K pairs of act16 / y16) when its weights are of
    // their kind and width; its gate input then comes from the router's own
    // pass over x when it is a dense F32 row (gate_ks partial sums in sh_act).
    const bool fold = w->has_shared &&
                      gemm_shared_fold_ok(wdesc(w->gate), wdesc(w->up), wdesc(w->down), wdesc(w->shared_gate),
                                          wdesc(w->shared_up), wdesc(w->shared_down), T, K);
    const WDesc GI = fold ? gate_inp_desc(w->shared_gate_inp) : WDesc{};
    bool gate_in_router = fold && GI.bits == 0 && GI.type == 0 && aligned16(GI.data) &&
                          f32mm_supported(R, xin);
    float *gparts = ws + L.sh_act;  // [ks][T] (T * ffs floats, unused by the folded path)
    uint32_t gate_ks = 1;
    // the router product stays F32 (the routing is exact given the logits);
    // only the expert products run in bf16.  `x16`: the router also rounds x
    // to bf16 for them (one pass over x where there is no norm to apply).
    auto router = [&](uint16_t *x16) -> moe_status {
        if (f32mm_supported(R, xin)) {
            // partial sums of the K ranges staged in y16, free until the down GEMM
            float *parts = reinterpret_cast<float *>(y16);
            const uint64_t part_floats = (uint64_t)T * K * d.h / 2;
            const uint32_t ks = f32mm_ksplit(R, (uint32_t)T, part_floats);
            // the gate row's K range fits the router's LDS, and its partial sums sh_act
            if (gate_in_router &&
                (d.h / ks > f32mm_gate_max() || (uint64_t)ks * f32mm_columns(R) > d.ffs))
                gate_in_router = false;
            const float *grow = gate_in_router ? static_cast<const float *>(GI.data) : nullptr;
            float *gout = gate_in_router ? gparts : nullptr;
            gate_ks = gate_in_router ? ks * f32mm_columns(R) : 1u;
            if (ks > 1) {
                TRY(launch_f32mm(p, s, "router_f32", R, xin, (uint32_t)T, ks, nullptr, parts, x16, grow, gout));
                TRY(launch_route_sum(p, s, parts, ks, bias, E, K, w->normalize ? 1 : 0, (uint32_t)T,
                                     logits, ids, wts));
            } else {
                TRY(launch_f32mm(p, s, "router_f32", R, xin, (uint32_t)T, 1, bias, logits, x16, grow, gout));
                TRY(launch_route(p, s, logits, E, K, w->normalize ? 1 : 0, (uint32_t)T, ids, wts));
            }
        } else {
            TRY(launch_gemv(p, s, R, xin, 0, nullptr, 1, logits, (uint32_t)T));
            if (bias) TRY(launch_add(p, s, logits, bias, logits, T * d.E));
            TRY(launch_route(p, s, logits, E, K, w->normalize ? 1 : 0, (uint32_t)T, ids, wts));
        }
        return MOE_OK;
    };
    const bool router_rounds = !nw && f32mm_supported(R, xin);
    if (router_rounds) {
        const moe_status st = router(xb16);
        if (st != MOE_OK) return st;
    } else {
        TRY(launch_to_bf16(p, s, xraw, nw, eps, (uint32_t)T, (uint32_t)d.h, xb16, xn));
    }
    if (fold) {
        // one stream: router, dispatch, the GEMMs over the routed segments
        // and the shared segment, the combine
        if (!router_rounds) {
            const moe_status st = router(nullptr);
            if (st != MOE_OK) return st;
        }
        const float *sgv = gparts;
        if (!gate_in_router) {
            float *sgt = ws + L.sh_gate;
            TRY(launch_gemv(p, s, gate_inp_desc(w->shared_gate_inp), xin, 0, nullptr, 1, sgt, (uint32_t)T));
            sgv = sgt;
            gate_ks = 1;
        }
        TRY(launch_dispatch(p, s, ids, (uint32_t)(T * K), E, counts, offsets, perm, pos, gemm_tile_rows(), tiles,
                            ntiles));
        const uint32_t base = (uint32_t)(T * K);
        const SharedSeg sh_gu{wdesc(w->shared_gate), wdesc(w->shared_up), packed(w->shared_gate_packed),
                              packed(w->shared_up_packed), (uint32_t)T, base};
        const SharedSeg sh_dn{wdesc(w->shared_down), wdesc(w->shared_down), packed(w->shared_down_packed),
                              packed(w->shared_down_packed), (uint32_t)T, base};
        TRY(launch_mfma_experts(p, s, wdesc(w->gate), wdesc(w->up), wdesc(w->down), packed(w->gate_packed),
                                packed(w->up_packed), packed(w->down_packed), xb16, (uint32_t)T, offsets, perm, K,
                                tiles, ntiles, act16, y16, &sh_gu, &sh_dn));
        TRY(launch_combine16(p, s, y16, pos, wts, K, nullptr, y16 + (uint64_t)base * d.h, sgv,
                             io->residual ? xraw : nullptr, out, (uint32_t)T, (uint32_t)d.h, gate_ks));
        return MOE_OK;
    }
    // The shared expert needs only the input: on the side stream from here,
    // alongside the router product (when that does not produce the bf16
    // input), routing and dispatch, joined before the combine.  Its gate/up
    // and down run on the grouped bf16 GEMM as one segment of all T rows
    // (bf16 output, as the routed experts'); kinds the GEMM does not take keep
    // the per-token products.
    const float *so = nullptr, *sgv = nullptr;
    const uint16_t *so16 = nullptr;
    SideFork side{g, s};
    if (w->has_shared) {
        float *sgt = ws + L.sh_gate;
        hipStream_t ss = g->side;
        TRY(side.fork());
        if (shared_mfma_ok(w)) {
            uint32_t *soff = reinterpret_cast<uint32_t *>(ws + L.sh_sched), *stiles = soff + 2;
            uint32_t *snt = stiles + 2 * ((T + 127) / 128);
            uint16_t *sact16 = reinterpret_cast<uint16_t *>(ws + L.sh_act);
            uint16_t *sy16 = reinterpret_cast<uint16_t *>(ws + L.sh_out);
            const PackedW none{};
            TRY(launch_identity_schedule(p, ss, (uint32_t)T, gemm_tile_rows(), soff, stiles, snt));
            TRY(launch_grouped_gemm(p, ss, 0, wdesc(w->shared_gate), wdesc(w->shared_up), none, none, xb16, T,
                                    nullptr, soff, stiles, snt, 1, sact16, "gemm_shared_gateup"));
            TRY(launch_grouped_gemm(p, ss, 1, wdesc(w->shared_down), wdesc(w->shared_down), none, none, sact16,
                                    T, nullptr, soff, stiles, snt, 1, sy16, "gemm_shared_down"));
            so16 = sy16;
        } else {
            float *sg = ws + L.sh_act, *su = ws + L.sh_up, *sout = ws + L.sh_out;
            TRY(launch_gemv(p, ss, wdesc(w->shared_gate), xin, 0, nullptr, 1, sg, (uint32_t)T));
            TRY(launch_gemv(p, ss, wdesc(w->shared_up), xin, 0, nullptr, 1, su, (uint32_t)T));
            TRY(launch_swiglu(p, ss, sg, su, sg, T * d.ffs));
            TRY(launch_gemv(p, ss, wdesc(w->shared_down), sg, 0, nullptr, 1, sout, (uint32_t)T));
            so = sout;
        }
        TRY(launch_gemv(p, ss, gate_inp_desc(w->shared_gate_inp), xin, 0, nullptr, 1, sgt, (uint32_t)T));
        sgv = sgt;
    }
    if (!router_rounds) {
        const moe_status st = router(nullptr);
        if (st != MOE_OK) return st;
    }
    TRY(launch_dispatch(p, s, ids, (uint32_t)(T * K), E, counts, offsets, perm, pos,
                        gemm_tile_rows(), tiles, ntiles));
    TRY(launch_mfma_experts(p, s, wdesc(w->gate), wdesc(w->up), wdesc(w->down), packed(w->gate_packed),
                            packed(w->up_packed), packed(w->down_packed), xb16, (uint32_t)T, offsets, perm,
                            K, tiles, ntiles, act16, y16));
    TRY(side.join());
    TRY(launch_combine16(p, s, y16, pos, wts, K, so, so16, sgv, io->residual ? xraw : nullptr, out,
                         (uint32_t)T, (uint32_t)d.h));
    return MOE_OK;
}

}  // namespace

extern "C" {

moe_status moe_pack_size(const moe_weight *w, uint64_t *data_bytes, uint64_t *sb_bytes) {
    if (!w || !data_bytes || !sb_bytes || w->ndims == 0 || w->ndims > 3 || w->bits == 0 ||
        (w->group_size != 32 && w->group_size != 64 && w->group_size != 128))
        return MOE_ERR_SHAPE;
    for (uint32_t i = 0; i < w->ndims; i++)
        if (w->dims[i] == 0 || !fits_u32(w->dims[i])) return MOE_ERR_SHAPE;
    return pack_layout(wdesc(*w), data_bytes, sb_bytes) ? MOE_OK : MOE_ERR_SHAPE;
}

moe_status moe_pack_weight(moe_gpu *g, const moe_weight *w, moe_packed_weight out) {
    moe_status st = need_batch(g);
    if (st) return st;
    if ((st = check_weight(g, w, "pack weight"))) return st;
    uint64_t db = 0, sb = 0;
    if (moe_pack_size(w, &db, &sb) != MOE_OK) return shape(g, "pack weight: no packed form");
    if (out.data.bytes != db || out.scales.bytes != sb || out.biases.bytes != sb)
        return shape(g, "pack weight: packed region sizes");
    if ((st = check_own(g, {rng(out.data), rng(out.scales), rng(out.biases)}))) return st;
    if ((st = check_alias(g, weight_ranges(*w), {rng(out.data), rng(out.scales), rng(out.biases)}, false)))
        return st;
    return launched(g, launch_pack_weight(&g->prof, g->stream, wdesc(*w), const_cast<void *>(out.data.ptr),
                                          const_cast<void *>(out.scales.ptr), const_cast<void *>(out.biases.ptr)),
                    "pack weight");
}

moe_status moe_block_workspace(const moe_block_weights *w, uint64_t tokens, uint64_t *elems) {
    if (!w || !elems || tokens == 0) return MOE_ERR_SHAPE;
    const uint64_t h = w->router.dims[0], E = w->router.dims[1], K = w->experts_used;
    const uint64_t ff = w->gate.dims[1], ffs = w->has_shared ? w->shared_gate.dims[1] : 0;
    *elems = ws_layout(tokens, E, K, h, ff, ffs).total;
    return MOE_OK;
}

moe_status moe_block_workspace_layout(const moe_block_weights *w, uint64_t tokens,
                                      moe_block_layout *out) {
    if (!w || !out || tokens == 0) return MOE_ERR_SHAPE;
    const uint64_t h = w->router.dims[0], E = w->router.dims[1], K = w->experts_used;
    const uint64_t ff = w->gate.dims[1], ffs = w->has_shared ? w->shared_gate.dims[1] : 0;
    const WsLayout L = ws_layout(tokens, E, K, h, ff, ffs);
    *out = moe_block_layout{L.logits, L.ids,   L.weights, L.counts, L.offsets,        L.perm,       L.pos,
                            L.tiles,  L.ntiles, L.xb16,   gemm_tile_rows(), seg_tokens(), L.total};
    return MOE_OK;
}

moe_status moe_block(moe_gpu *g, const moe_block_weights *w, moe_buffer x, moe_buffer out,
                     uint64_t tokens, const moe_block_io *io) {
    return abi::block_entry(g, w, x, out, tokens, io, false);
}

}  // extern "C"

namespace abi {

moe_status block_entry(moe_gpu *g, const moe_block_weights *w, moe_buffer x, moe_buffer out,
                       uint64_t tokens, const moe_block_io *io, bool scratch) {
    moe_status st = need_batch(g);
    if (st) return st;
    if (!io) return shape(g, "missing block io");
    Dims d{};
    if ((st = check_block(g, w, d))) return st;
    if (tokens == 0 || tokens > 65535) return shape(g, "tokens must be in [1, 65535]");
    const uint64_t T = tokens;
    if (x.len != T * d.h || out.len != T * d.h) return shape(g, "block input/output length");
    const WsLayout L = ws_layout(T, d.E, d.K, d.h, d.ff, d.ffs);
    if (scratch && io->workspace.len < L.total)
        return shape(g, "the block needs " + std::to_string(L.total * 4) +
                            " bytes of workspace, more than the no-allocation scratch (" +
                            std::to_string(io->workspace.len * 4) + " bytes)");
    if (io->workspace.len < L.total) return shape(g, "workspace too small");
    if (has(io->logit_bias) && io->logit_bias.len != T * d.E) return shape(g, "logit bias length");
    if (has(io->logits_out) && io->logits_out.len != T * d.E) return shape(g, "logits output length");
    if (has(io->ids_out) && io->ids_out.len != T * d.K) return shape(g, "ids output length");
    if (has(io->weights_out) && io->weights_out.len != T * d.K) return shape(g, "weights output length");
    if (has(io->norm_weight) &&
        (io->norm_weight.len != d.h || !std::isfinite(io->norm_eps) || io->norm_eps <= 0.f))
        return shape(g, "norm");
    if (io->path > MOE_PATH_MFMA) return shape(g, "unknown path");
    if (io->path == MOE_PATH_MFMA && !mfma_path_ok(w, d))
        return shape(g, "MFMA path needs hidden and ff multiples of 128 and supported weight kinds");
    // ownership
    std::vector<Range> reads{rng(x)};
    std::vector<Range> writes{rng(out), rng(io->workspace)};
    if ((st = check_own(g, {rng(x), rng(out)}))) return st;
    // the no-allocation scratch is the library's own device array, not a
    // registered allocation
    if (!scratch && (st = check_own(g, {rng(io->workspace)}))) return st;
    const moe_buffer *opt_in[] = {&io->logit_bias, &io->norm_weight};
    const moe_buffer *opt_out[] = {&io->logits_out, &io->ids_out, &io->weights_out};
    for (auto b : opt_in)
        if (has(*b)) {
            if ((st = check_own(g, {rng(*b)}))) return st;
            reads.push_back(rng(*b));
        }
    for (auto b : opt_out)
        if (has(*b)) {
            if ((st = check_own(g, {rng(*b)}))) return st;
            writes.push_back(rng(*b));
        }
    const moe_weight *ws_list[] = {&w->router, &w->gate, &w->up, &w->down, &w->shared_gate,
                                   &w->shared_up, &w->shared_down, &w->shared_gate_inp};
    for (int i = 0; i < (w->has_shared ? 8 : 4); i++)
        for (const Range &r : weight_ranges(*ws_list[i])) reads.push_back(r);
    // out may be exactly x (in-place residual stream); everything else is disjoint
    for (size_t i = 0; i < writes.size(); i++) {
        for (size_t j = i + 1; j < writes.size(); j++)
            if (overlaps(writes[i], writes[j])) return shape(g, "overlapping GPU outputs");
        for (size_t r = 0; r < reads.size(); r++)
            if (overlaps(writes[i], reads[r]) && !(i == 0 && r == 0 && same(writes[i], reads[r])))
                return shape(g, "GPU input/output alias");
    }

    float *ws = fp(io->workspace);
    float *logits = has(io->logits_out) ? fp(io->logits_out) : ws + L.logits;
    uint32_t *ids = has(io->ids_out) ? up32(io->ids_out) : reinterpret_cast<uint32_t *>(ws + L.ids);
    float *wts = has(io->weights_out) ? fp(io->weights_out) : ws + L.weights;
    const float *xraw = fp(x);
    float *o = fp(out);
    const float *nw = has(io->norm_weight) ? fp(io->norm_weight) : nullptr;

    // fused single-token decode
    if (io->path == MOE_PATH_AUTO && T == 1) {
        DecodeArgs a{};
        a.router = wdesc(w->router);
        a.gate = wdesc(w->gate);
        a.up = wdesc(w->up);
        a.down = wdesc(w->down);
        a.has_shared = w->has_shared;
        if (w->has_shared) {
            a.sg = wdesc(w->shared_gate);
            a.su = wdesc(w->shared_up);
            a.sd = wdesc(w->shared_down);
            a.sgi = gate_inp_desc(w->shared_gate_inp);
        }
        a.k = (uint32_t)d.K;
        a.normalize = w->normalize ? 1 : 0;
        a.x = xraw;
        a.norm_w = nw;
        a.eps = io->norm_eps;
        a.logit_bias = has(io->logit_bias) ? fp(io->logit_bias) : nullptr;
        a.resid = io->residual ? xraw : nullptr;
        a.out = o;
        a.logits = logits;
        a.ids = ids;
        a.weights = wts;
        a.act = ws + L.act;
        a.sh_act = ws + L.sh_act;
        a.sh_gate = ws + L.sh_gate;
        if (decode_supported(a)) return launched(g, launch_decode(&g->prof, g->stream, a), "decode");
    }

    const bool mean_seg_16 = T * d.K >= 16 * d.E;  // mean expert segment >= 16 pairs
    if (io->path == MOE_PATH_MFMA || (io->path == MOE_PATH_AUTO && mean_seg_16 && mfma_path_ok(w, d)))
        return run_mfma(g, w, d, xraw, nw, io->norm_eps, o, T, io, L, ws, logits, ids, wts);

    const float *xin = xraw;
    if (nw) {
        float *xn = ws + L.xnorm;
        // Batch::norm over T rows (execute.rs:197)
        hipError_t e = launch_norm(&g->prof, g->stream, xraw, nw, MOE_F32, xn, (uint32_t)T,
                                   (uint32_t)d.h, (uint32_t)d.h, io->norm_eps);
        if (e != hipSuccess) return gpu_err(g, e, "norm");
        xin = xn;
    }
    if (io->path == MOE_PATH_OPS)
        return run_ops(g, w, d, xin, xraw, o, T, io, L, ws, logits, ids, wts);
    if (io->path == MOE_PATH_AUTO && batched_ok(w) && aligned16(xin) && aligned16(ws))
        return run_batched(g, w, d, xin, xraw, o, T, io, L, ws, logits, ids, wts);
    return run_grouped(g, w, d, xin, xraw, o, T, io, L, ws, logits, ids, wts);
}

}  // namespace abi

extern "C" {

// ============================================================ profiling ==
moe_status moe_profile_enable(moe_gpu *g, int enable) {
    if (!g) return MOE_ERR_SHAPE;
    g->prof.enabled = enable != 0;
    return MOE_OK;
}

moe_status moe_profile_count(moe_gpu *g, uint32_t *n) {
    if (!g || !n) return MOE_ERR_SHAPE;
    (void)hipSetDevice(g->device);
    prof_collect(&g->prof, g->stream);
    *n = (uint32_t)g->prof.entries.size();
    return MOE_OK;
}

moe_status moe_profile_get(moe_gpu *g, uint32_t index, char *name, size_t cap, uint64_t *launches,
                           double *seconds) {
    if (!g) return MOE_ERR_SHAPE;
    (void)hipSetDevice(g->device);
    prof_collect(&g->prof, g->stream);
    if (index >= g->prof.entries.size()) return shape(g, "profile index");
    const ProfEntry &e = g->prof.entries[index];
    if (name && cap) std::snprintf(name, cap, "%s", e.name.c_str());
    if (launches) *launches = e.launches;
    if (seconds) *seconds = e.seconds;
    return MOE_OK;
}

moe_status moe_profile_reset(moe_gpu *g) {
    if (!g) return MOE_ERR_SHAPE;
    (void)hipSetDevice(g->device);
    prof_collect(&g->prof, g->stream);
    g->prof.entries.clear();
    return MOE_OK;
}

moe_status moe_profile_hold(moe_gpu *g, uint32_t microseconds) {
    moe_status st = need_batch(g);
    if (st) return st;
    if (g->capturing) return shape(g, "hold inside a graph capture");
    if (microseconds > 100000u) return shape(g, "hold longer than 100 ms");
    return launched(g, launch_hold(g->stream, microseconds), "hold");
}

// ================================================================ graphs ==
moe_status moe_graph_begin(moe_gpu *g) {
    moe_status st = need_no_batch(g);
    if (st) return st;
    if (g->prof.enabled) return shape(g, "disable profiling before capturing a graph");
    hipError_t e = hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return gpu_err(g, e, "begin capture");
    g->in_batch = true;
    g->capturing = true;
    return MOE_OK;
}

moe_status moe_graph_end(moe_gpu *g, moe_graph **out) {
    if (!g || !out) return MOE_ERR_SHAPE;
    if (!g->capturing) return shape(g, "no graph capture in progress");
    (void)hipSetDevice(g->device);
    g->capturing = false;
    g->in_batch = false;
    moe_graph *gr = new moe_graph();
    hipError_t e = hipStreamEndCapture(g->stream, &gr->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&gr->exec, gr->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        moe_graph_destroy(gr);
        return gpu_err(g, e, "graph");
    }
    *out = gr;
    return MOE_OK;
}

moe_status moe_graph_launch(moe_gpu *g, moe_graph *gr) {
    moe_status st = need_batch(g);
    if (st) return st;
    if (!gr || g->capturing) return shape(g, "graph launch");
    return launched(g, hipGraphLaunch(gr->exec, g->stream), "graph launch");
}

void moe_graph_destroy(moe_graph *gr) {
    if (!gr) return;
    if (gr->exec) (void)hipGraphExecDestroy(gr->exec);
    if (gr->graph) (void)hipGraphDestroy(gr->graph);
    delete gr;
}

}  // extern "C"
