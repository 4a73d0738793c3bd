// Internal interfaces between the C ABI (moe_abi.cpp) and the kernel files.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <tuple>

namespace moehip {

// Kernel-side view of one weight tensor (dims [in, out, experts]).
// bits == 0: dense elements of `type` (0 F32, 1 F16, 30 BF16).
// bits in {2,4,8}: packed u32 codes; `type` is the scale/bias dtype.
struct WDesc {
    const void *data;
    const void *scales;
    const void *biases;
    uint32_t bits;
    uint32_t type;
    uint32_t in;
    uint32_t out;
    uint32_t experts;
    uint32_t gshift;  // log2(group_size); 0 for dense
};

// Launch-side profiling hook.  While profiling is enabled on the gpu,
// prof_launch hands out a start/stop event pair that launch_kernel passes to
// hipExtLaunchKernel: the events then carry the dispatch's own begin and end
// timestamps (the kernel's execution, as a kernel trace reports it, without
// the packet-processing time of separately recorded events).  Null events
// when profiling is off.
struct Prof;
struct ProfEvents {
    hipEvent_t start, stop;
};
ProfEvents prof_launch(Prof *p, const char *name);

// kernel<<<grid, block, lds, s>>>(args...), timed under `name` when profiling.
template <typename... KArgs, typename... Args>
hipError_t launch_kernel(Prof *p, const char *name, void (*kernel)(KArgs...), dim3 grid,
                         dim3 block, size_t lds, hipStream_t s, Args... args) {
    static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count");
    std::tuple<KArgs...> vals{static_cast<KArgs>(args)...};
    void *ptrs[sizeof...(KArgs) > 0 ? sizeof...(KArgs) : 1];
    std::apply([&ptrs](auto &...v) {
        size_t i = 0;
        ((ptrs[i++] = static_cast<void *>(&v)), ...);
    }, vals);
    const ProfEvents ev = prof_launch(p, name);
    if (ev.start)
        return hipExtLaunchKernel(reinterpret_cast<const void *>(kernel), grid, block, ptrs, lds, s,
                                  ev.start, ev.stop, 0);
    return hipLaunchKernel(reinterpret_cast<const void *>(kernel), grid, block, ptrs, lds, s);
}

// Work buffers of the fused/grouped MoE block (all device pointers).
struct BlockBufs {
    float *logits;    // [T, E]
    uint32_t *ids;    // [T, K]
    float *weights;   // [T, K]
    uint32_t *counts; // [E]
    uint32_t *offsets;// [E+1]
    uint32_t *perm;   // [T*K]
    uint32_t *pos;    // [T*K]
    float *act;       // [T*K, ff]  (F32 SwiGLU outputs in perm order)
    float *yexp;      // [T*K, h]   expert outputs in perm order (grouped path)
    float *sh_act;    // [T, ffs]
    float *sh_gate;   // [T]
    float *sh_out;    // [T, h]
    float *xnorm;     // [T, h] RMSNorm'ed input (when a norm weight is given)
    uint16_t *xb16;   // [T, h] bf16 copy of the block input (MFMA path)
    uint16_t *act16;  // [T*K, ff] bf16 SwiGLU outputs (MFMA path)
    uint32_t *tiles;  // MFMA tile schedule
};

// ---- generic products (k_gemv.hip) ----
// y[(sel*tokens + t)*out + r] = W_expert(sel) row r . x_sel_t
//   matmul:        nsel = 1, ids = nullptr, x_sel_stride = 0
//   expert_matmul: nsel = nids, tokens = 1, x_sel_stride = per_expert ? in : 0
hipError_t launch_gemv(Prof *p, hipStream_t s, const WDesc &w, const float *x,
                       uint64_t x_sel_stride, const uint32_t *ids, uint32_t nsel, float *y,
                       uint32_t tokens);

// ---- routing + dispatch (k_route.hip) ----
hipError_t launch_hold(hipStream_t s, uint32_t microseconds);
hipError_t launch_route_sum(Prof *p, hipStream_t s, const float *parts, uint32_t nsplit,
                            const float *bias, uint32_t experts, uint32_t k, int normalize,
                            uint32_t tokens, float *logits, uint32_t *ids, float *weights);
// out[t, r] = x_t . W_r in F32 on the F32 matrix cores (k_f32mm.hip; the
// prefill router product and moe_matmul at >= 4 tokens), W 2-D: K split
// into `ksplit` ranges (f32mm_ksplit picks it for a partial buffer of
// `part_floats`); with ksplit 1 `out` receives the products (+ bias), else
// the partial sums [ksplit, tokens, out] (launch_route_sum adds the
// router's).  Profiled under `name`.
bool f32mm_supported(const WDesc &w, const float *x);
uint32_t f32mm_ksplit(const WDesc &w, uint32_t tokens, uint64_t part_floats);
// xb16 (optional, [tokens, in]): x rounded to bf16, written on the way.
// grow: a dense F32 row (16-byte aligned) whose product with every token's x
// the router also forms, one partial sum per K range and column of 128
// outputs: gout[(kr * f32mm_columns(w) + c) * tokens + t]; a K range
// (w.in / ksplit) of at most f32mm_gate_max() values
uint32_t f32mm_gate_max();
uint32_t f32mm_columns(const WDesc &w);
hipError_t launch_f32mm(Prof *p, hipStream_t s, const char *name, const WDesc &w, const float *x,
                        uint32_t tokens, uint32_t ksplit, const float *bias, float *out,
                        uint16_t *xb16 = nullptr, const float *grow = nullptr, float *gout = nullptr);
hipError_t launch_route(Prof *p, hipStream_t s, const float *logits, uint32_t experts, uint32_t k,
                        int normalize, uint32_t tokens, uint32_t *ids, float *weights);
// With `tiles` it also writes the work list of tm-pair runs that
// launch_tile_schedule would (in the same launch where the experts fit LDS).
hipError_t launch_dispatch(Prof *p, hipStream_t s, const uint32_t *ids, uint32_t pairs,
                           uint32_t experts, uint32_t *counts, uint32_t *offsets, uint32_t *perm,
                           uint32_t *pos, uint32_t tm = 0, uint32_t *tiles = nullptr,
                           uint32_t *ntiles = nullptr);
// launch_route, launch_dispatch and launch_tile_schedule (work items of tm
// pairs) in one launch; `arrive` is a device word that is zero before the
// launch and is zero again after it.
bool route_dispatch_fits(uint32_t experts, uint32_t k, uint32_t tokens);
hipError_t launch_route_dispatch(Prof *p, hipStream_t s, const float *logits, uint32_t experts,
                                 uint32_t k, int normalize, uint32_t tokens, uint32_t *ids,
                                 float *weights, uint32_t *arrive, uint32_t tm, uint32_t *counts,
                                 uint32_t *offsets, uint32_t *perm, uint32_t *pos, uint32_t *tiles,
                                 uint32_t *ntiles);

// ---- element-wise (k_elem.hip) ----
hipError_t launch_swiglu(Prof *p, hipStream_t s, const float *a, const float *b, float *y,
                         uint64_t n);
hipError_t launch_mix(Prof *p, hipStream_t s, const float *x, const float *w, uint32_t k,
                      uint64_t n, float *y);
hipError_t launch_gate_scalar(Prof *p, hipStream_t s, const float *x, const float *g, float *y,
                              uint64_t n);
hipError_t launch_add(Prof *p, hipStream_t s, const float *a, const float *b, float *y,
                      uint64_t n);
hipError_t launch_norm(Prof *p, hipStream_t s, const float *x, const void *w, uint32_t wtype,
                       float *y, uint32_t heads, uint32_t n, uint32_t stride, float eps);
hipError_t launch_copy(Prof *p, hipStream_t s, const float *src, float *dst, uint64_t n);
// out[t, i] = sum_k w[t,k] * yexp[pos[t*K+k], i] (+ sigmoid(sh_gate[t]) * sh_out[t, i])
//             (+ resid[t, i])
hipError_t launch_combine(Prof *p, hipStream_t s, const float *yexp, const uint32_t *pos,
                          const float *w, uint32_t k, const float *sh_out, const float *sh_gate,
                          const float *resid, float *out, uint32_t tokens, uint32_t h);

// ---- grouped expert products on VALU (k_grouped.hip) ----
// act[p, j] = silu(x_t . G_e[j]) * (x_t . U_e[j]) for every dispatched pair p
// (perm order), t = perm[p] / K, e = expert of the segment holding p.
hipError_t launch_grouped_gateup(Prof *p, hipStream_t s, const WDesc &gate, const WDesc &up,
                                 const float *x, const uint32_t *offsets, const uint32_t *perm,
                                 uint32_t k, uint32_t experts, float *act);
// yexp[p, r] = D_e[r] . act[p]
hipError_t launch_grouped_down(Prof *p, hipStream_t s, const WDesc &down, const float *act,
                               const uint32_t *offsets, uint32_t experts, uint32_t pairs,
                               float *yexp);

// ---- prefill around the bf16 MFMA GEMMs (k_mfma.hip) ----
hipError_t launch_to_bf16(Prof *p, hipStream_t s, const float *x, const float *norm_w, float eps,
                          uint32_t tokens, uint32_t h, uint16_t *y, float *xn);
// An affine expert weight repacked in MFMA tile order (k_pack.hip): for
// expert e, 32-row tile t (rows past `out` zero) and K step kb (64 values),
// the 32 rows' codes form one block of 256*BITS bytes in which lane
// l = 32h + r holds row r's codes 32h .. 32h + 31 at byte 4*BITS*l; for each
// pair of K steps p, the tile's scales (and biases) form one block of
// 32 rows x (128 >> gshift) 16-bit values, row-major.  Null data: no copy.
struct PackedW {
    const void *data, *scales, *biases;
};
// One more segment of the grouped GEMM after the routed experts' (the
// shared expert): its weights (w2: up, for gate/up), their packed copies
// (null data: none), and its rows [base, base + rows) of the output and, for
// the down product, of the A rows (the gate/up product reads A row r - base,
// i.e. the token's own row).
struct SharedSeg {
    WDesc w, w2;
    PackedW pk, pk2;
    uint32_t rows, base;
};
// Byte sizes of the packed copy (false: no packed form -- affine weights with
// 16-bit scales, in % 128 == 0, offsets below 2^32 only).
bool pack_layout(const WDesc &w, uint64_t *data_bytes, uint64_t *sb_bytes);
hipError_t launch_pack_weight(Prof *p, hipStream_t s, const WDesc &w, void *data, void *scales,
                              void *biases);
// tiles / ntiles: the work list of gemm_tile_rows()-pair M-tiles, written by
// launch_dispatch (or launch_tile_schedule) over the same offsets.
// sh_gu / sh_dn: the shared expert as one more segment of the gate/up and
// down GEMMs (null: none); its rows follow the T*k routed pairs in act16 and y16.
hipError_t launch_mfma_experts(Prof *p, hipStream_t s, const WDesc &gate, const WDesc &up,
                               const WDesc &down, const PackedW &pg, const PackedW &pu,
                               const PackedW &pd, const uint16_t *xb16, uint32_t tokens,
                               const uint32_t *offsets, const uint32_t *perm, uint32_t k,
                               uint32_t *tiles, uint32_t *ntiles, uint16_t *act16, uint16_t *y16,
                               const SharedSeg *sh_gu = nullptr, const SharedSeg *sh_dn = nullptr);
// Grouped expert GEMM over the dispatched segments (k_gemm.hip): down = 0 for
// gate/up + SwiGLU (w = gate, w2 = up, a_rows = xb16, out = act16), 1 for the
// down product (w = w2 = down, a_rows = act16, out = y16; the combine applies
// the routing weights).  a_rows_n: rows of a_rows (tokens, or pairs for the
// down product).  tiles/ntiles: M-tiles of gemm_tile_rows() pairs from
// tile_schedule.
bool gemm_supported(const WDesc &w);
uint32_t gemm_tile_rows();  // pairs per work item (the M-tiles tile_schedule emits)
// Whether the shared expert (sg/su/sd) can run as that segment of the routed
// experts' affine GEMMs (g/u/d) over T tokens x K: the same code width,
// scale type and group, the same intermediate width, and every offset within
// 32 bits.
bool gemm_shared_fold_ok(const WDesc &g, const WDesc &u, const WDesc &d, const WDesc &sg, const WDesc &su,
                         const WDesc &sd, uint64_t T, uint64_t K);
// pk, pk2: packed copies of w, w2 (PackedW with null data: none).
// perm null: pair p is row p of a_rows (one segment of all rows, the shared
// expert).  sh: the shared expert as one more segment (null: none).  `name`:
// the profile name (null: gemm_gateup / gemm_down).
hipError_t launch_grouped_gemm(Prof *p, hipStream_t s, int down, const WDesc &w, const WDesc &w2,
                               const PackedW &pk, const PackedW &pk2, const uint16_t *a_rows,
                               uint64_t a_rows_n, const uint32_t *perm, const uint32_t *offsets,
                               const uint32_t *tiles, const uint32_t *ntiles, uint32_t k,
                               uint16_t *out, const char *name = nullptr, const SharedSeg *sh = nullptr);
// offsets {0, rows}, the M-tiles of tm rows over them, and their count
hipError_t launch_identity_schedule(Prof *p, hipStream_t s, uint32_t rows, uint32_t tm, uint32_t *offsets,
                                    uint32_t *tiles, uint32_t *ntiles);
// the shared expert's output as F32 (sh_out) or bf16 (sh16), or neither; its
// gate input sh_gate[t], or the sum of gate_ks partial sums sh_gate[kr * tokens + t]
hipError_t launch_combine16(Prof *p, hipStream_t s, const uint16_t *y16, const uint32_t *pos,
                            const float *wts, uint32_t k, const float *sh_out, const uint16_t *sh16,
                            const float *sh_gate, const float *resid, float *out, uint32_t tokens,
                            uint32_t h, uint32_t gate_ks = 1);

// ---- batched decode (k_batched.hip) ----
// Row products over work entries of at most seg_tokens() input rows: entries
// from tile_schedule over the dispatch's segments (tiles, ntiles, offsets),
// or, with tiles == nullptr, runs over the n input rows of one weight.
// `entries` bounds the grid (seg_max_entries); surplus entries exit.
bool seg_supported(const WDesc &w);  // whole 32-element chunks, in / 32 a power of two <= 64
uint32_t seg_tokens();
uint32_t seg_max_entries(uint32_t pairs, uint32_t experts);  // experts 0: runs over `pairs` rows
hipError_t launch_seg_gateup(Prof *p, hipStream_t s, const char *name, const WDesc &gate,
                             const WDesc &up, const float *x, const uint32_t *perm, uint32_t k,
                             const uint32_t *tiles, const uint32_t *ntiles, const uint32_t *offsets,
                             uint32_t n, uint32_t entries, float *act);
hipError_t launch_seg_rows(Prof *p, hipStream_t s, const char *name, const WDesc &w,
                           const float *in, const uint32_t *tiles, const uint32_t *ntiles,
                           const uint32_t *offsets, uint32_t n, uint32_t entries, const float *bias,
                           float *out);
// (expert, first position) of every run of `tm` pairs of the non-empty
// segments, and their count (k_mfma.hip)
hipError_t launch_tile_schedule(Prof *p, hipStream_t s, const uint32_t *offsets, uint32_t experts,
                                uint32_t tm, uint32_t *tiles, uint32_t *ntiles);

// ---- fused single-token decode (k_decode.hip) ----
struct DecodeArgs {
    WDesc router, gate, up, down, sg, su, sd, sgi;
    uint32_t has_shared, k, normalize;
    const float *x;          // [h] block input
    const float *norm_w;     // [h] RMSNorm weight or nullptr
    float eps;
    const float *logit_bias; // [E] or nullptr
    const float *resid;      // [h] or nullptr
    float *out;              // [h]
    float *logits;           // [E]
    uint32_t *ids;           // [K]
    float *weights;          // [K]
    float *act;              // [K, ff]
    float *sh_act;           // [ffs]
    float *sh_gate;          // [1]
};
bool decode_supported(const DecodeArgs &a);
hipError_t launch_decode(Prof *p, hipStream_t s, const DecodeArgs &a);

}  // namespace moehip
