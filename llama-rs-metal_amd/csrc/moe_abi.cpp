// C ABI of the MI355X MoE backend (declared in include/moe_hip.h).
//
// Host-side mirror of metal_backend's Gpu / Batch (crates/metal-backend/src/apple.rs,
// apple/commands.rs, apple/memory.rs, apple/ops/*.rs): the same shape checks,
// ownership and alias rules and error kinds, in front of HIP kernels on one
// stream.  Every check runs before anything is enqueued.
#include "abi_common.hpp"

namespace moehip {

static hipEvent_t prof_event(Prof *p) {
    if (!p->pool.empty()) {
        hipEvent_t e = p->pool.back();
        p->pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

ProfEvents prof_launch(Prof *p, const char *name) {
    if (!p || !p->enabled) return ProfEvents{nullptr, nullptr};
    size_t idx = p->entries.size();
    for (size_t i = 0; i < p->entries.size(); i++)
        if (p->entries[i].name == name) idx = i;
    if (idx == p->entries.size()) p->entries.push_back(ProfEntry{name, 0, 0.0});
    hipEvent_t a = prof_event(p), b = prof_event(p);
    if (!a || !b) {
        if (a) p->pool.push_back(a);
        if (b) p->pool.push_back(b);
        return ProfEvents{nullptr, nullptr};
    }
    p->pending.push_back(Prof::Pending{idx, a, b});
    return ProfEvents{a, b};
}

void prof_collect(Prof *p, hipStream_t s) {
    if (p->pending.empty()) return;
    (void)hipStreamSynchronize(s);
    for (auto &q : p->pending) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, q.a, q.b) == hipSuccess) {
            p->entries[q.entry].launches++;
            p->entries[q.entry].seconds += ms * 1e-3;
        }
        p->pool.push_back(q.a);
        p->pool.push_back(q.b);
    }
    p->pending.clear();
}

}  // namespace moehip

// ================================================================= device ==
extern "C" {

moe_status moe_gpu_create(int device, moe_gpu **out) {
    if (!out) return MOE_ERR_SHAPE;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0)
        return MOE_ERR_UNAVAILABLE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return MOE_ERR_UNAVAILABLE;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return MOE_ERR_UNAVAILABLE;
    if (hipSetDevice(device) != hipSuccess) return MOE_ERR_UNAVAILABLE;
    moe_gpu *g = new moe_gpu();
    g->device = device;
    g->name = prop.name[0] ? prop.name : prop.gcnArchName;
    if (hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&g->side, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&g->ev_begin) != hipSuccess || hipEventCreate(&g->ev_end) != hipSuccess ||
        hipEventCreateWithFlags(&g->ev_fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&g->ev_join, hipEventDisableTiming) != hipSuccess ||
        hipMalloc(reinterpret_cast<void **>(&g->arrive), 256) != hipSuccess ||
        hipMemset(g->arrive, 0, 256) != hipSuccess) {
        if (g->arrive) (void)hipFree(g->arrive);
        delete g;
        return MOE_ERR_GPU;
    }
    // this device's address of the no-allocation scratch (checked; without it
    // only moe_block_noalloc is unavailable)
    if (noalloc_scratch_address(device, &g->scratch) != hipSuccess) g->scratch = nullptr;
    *out = g;
    return MOE_OK;
}

void moe_gpu_destroy(moe_gpu *g) {
    if (!g) return;
    (void)hipSetDevice(g->device);
    (void)hipStreamSynchronize(g->stream);
    (void)hipStreamSynchronize(g->side);
    for (auto &a : g->allocs)
        if (a.second.owned) (void)hipFree(reinterpret_cast<void *>(a.first));
    for (auto &q : g->prof.pending) {
        (void)hipEventDestroy(q.a);
        (void)hipEventDestroy(q.b);
    }
    for (auto e : g->prof.pool) (void)hipEventDestroy(e);
    (void)hipFree(g->arrive);
    (void)hipEventDestroy(g->ev_begin);
    (void)hipEventDestroy(g->ev_end);
    (void)hipEventDestroy(g->ev_fork);
    (void)hipEventDestroy(g->ev_join);
    (void)hipStreamDestroy(g->side);
    (void)hipStreamDestroy(g->stream);
    delete g;
}

moe_status moe_gpu_name(const moe_gpu *g, char *buf, size_t cap) {
    if (!g || !buf || cap == 0) return MOE_ERR_SHAPE;
    std::snprintf(buf, cap, "%s", g->name.c_str());
    return MOE_OK;
}

uint64_t moe_allocated_bytes(const moe_gpu *g) { return g ? g->live : 0; }

const char *moe_last_error(const moe_gpu *g) { return g ? g->err.c_str() : "no gpu"; }

uint64_t moe_last_error_bytes(const moe_gpu *g) { return g ? g->err_bytes : 0; }

const char *moe_version(void) { return "moe-hip 0.1 (gfx950)"; }

// ================================================================= memory ==
moe_status moe_zeros(moe_gpu *g, uint64_t n, moe_buffer *out) {
    moe_status st = need_no_batch(g);
    if (st) return st;
    if (!out) return shape(g, "null output");
    if (n == 0 || !fits_u32(n)) return fail_alloc(g, elem_bytes(n), "allocation size");
    void *p = nullptr;
    st = alloc_bytes(g, n * 4, &p);
    if (st) return st;
    hipError_t e = hipMemset(p, 0, n * 4);
    if (e != hipSuccess) return gpu_err(g, e, "zero fill");
    *out = moe_buffer{p, n};
    return MOE_OK;
}

moe_status moe_upload(moe_gpu *g, const float *data, uint64_t n, moe_buffer *out) {
    moe_status st = need_no_batch(g);
    if (st) return st;
    if (!out || !data) return shape(g, "null pointer");
    if (n == 0 || !fits_u32(n)) return fail_alloc(g, elem_bytes(n), "allocation size");
    void *p = nullptr;
    st = alloc_bytes(g, n * 4, &p);
    if (st) return st;
    hipError_t e = hipMemcpy(p, data, n * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return gpu_err(g, e, "upload");
    *out = moe_buffer{p, n};
    return MOE_OK;
}

moe_status moe_upload_bytes(moe_gpu *g, const void *data, uint64_t bytes, moe_region *out) {
    moe_status st = need_no_batch(g);
    if (st) return st;
    if (!out || !data) return shape(g, "null pointer");
    if (bytes == 0) return fail_alloc(g, 0, "allocation size");
    void *p = nullptr;
    st = alloc_bytes(g, (bytes + 3) & ~3ull, &p);
    if (st) return st;
    hipError_t e = hipMemcpy(p, data, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) return gpu_err(g, e, "upload");
    *out = moe_region{p, bytes};
    return MOE_OK;
}

moe_status moe_read(moe_gpu *g, moe_buffer b, float *out) {
    moe_status st = need_no_batch(g);
    if (st) return st;
    if ((st = check_own(g, {rng(b)}))) return st;
    if (!out) return shape(g, "null host pointer");
    hipError_t e = hipStreamSynchronize(g->stream);
    if (e == hipSuccess) e = hipMemcpy(out, b.ptr, b.len * 4, hipMemcpyDeviceToHost);
    return launched(g, e, "read");
}

moe_status moe_write(moe_gpu *g, moe_buffer b, const float *data) {
    moe_status st = need_no_batch(g);
    if (st) return st;
    if ((st = check_own(g, {rng(b)}))) return st;
    if (!data) return shape(g, "null host pointer");
    hipError_t e = hipStreamSynchronize(g->stream);
    if (e == hipSuccess) e = hipMemcpy(b.ptr, data, b.len * 4, hipMemcpyHostToDevice);
    return launched(g, e, "write");
}

moe_status moe_clear(moe_gpu *g, moe_buffer b) {
    moe_status st = need_no_batch(g);
    if (st) return st;
    if ((st = check_own(g, {rng(b)}))) return st;
    hipError_t e = hipStreamSynchronize(g->stream);
    if (e == hipSuccess) e = hipMemset(b.ptr, 0, b.len * 4);
    return launched(g, e, "clear");
}

moe_status moe_release(moe_gpu *g, const void *base) {
    moe_status st = need_no_batch(g);
    if (st) return st;
    auto it = g->allocs.find(reinterpret_cast<uintptr_t>(base));
    if (it == g->allocs.end() || !it->second.owned)
        return shape(g, "release of memory this gpu did not allocate");
    (void)hipStreamSynchronize(g->stream);
    (void)hipStreamSynchronize(g->side);
    hipError_t e = hipFree(const_cast<void *>(base));
    g->live -= it->second.bytes;
    g->allocs.erase(it);
    return launched(g, e, "free");
}

moe_status moe_register(moe_gpu *g, void *base, uint64_t bytes) {
    if (!g) return MOE_ERR_SHAPE;
    if (!base || bytes == 0) return shape(g, "empty registration");
    Range r{reinterpret_cast<uintptr_t>(base), reinterpret_cast<uintptr_t>(base) + bytes};
    for (auto &a : g->allocs)
        if (overlaps(r, Range{a.first, a.first + a.second.bytes}))
            return shape(g, "registration overlaps an existing allocation");
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, base) != hipSuccess || attr.type != hipMemoryTypeDevice ||
        attr.device != g->device)
        return shape(g, "not device memory of this gpu");
    g->allocs[r.lo] = Alloc{bytes, false};
    return MOE_OK;
}

moe_status moe_unregister(moe_gpu *g, const void *base) {
    if (!g) return MOE_ERR_SHAPE;
    auto it = g->allocs.find(reinterpret_cast<uintptr_t>(base));
    if (it == g->allocs.end() || it->second.owned) return shape(g, "not a registered region");
    g->allocs.erase(it);
    return MOE_OK;
}

moe_status moe_view(moe_buffer b, uint64_t start, uint64_t len, moe_buffer *out) {
    // Buffer::view (apple.rs:51-63)
    if (!out) return MOE_ERR_SHAPE;
    if (start > UINT64_MAX - len) return MOE_ERR_SHAPE;  // view overflow
    if (start + len > b.len || len == 0) return MOE_ERR_SHAPE;  // view bounds
    *out = moe_buffer{static_cast<float *>(b.ptr) + start, len};
    return MOE_OK;
}

moe_status moe_copy(moe_gpu *g, moe_buffer src, moe_buffer dst) {
    moe_status st = need_batch(g);
    if (st) return st;
    if ((st = check_own(g, {rng(src), rng(dst)}))) return st;
    if (src.len != dst.len) return shape(g, "copy");
    if ((st = check_alias(g, {rng(src)}, {rng(dst)}, false))) return st;
    return launched(g, launch_copy(&g->prof, g->stream, (const float *)src.ptr, (float *)dst.ptr, src.len),
                    "copy");
}

// ================================================================== batch ==
moe_status moe_batch_begin(moe_gpu *g) {
    moe_status st = need_no_batch(g);
    if (st) return st;
    hipError_t e = hipEventRecord(g->ev_begin, g->stream);
    if (e != hipSuccess) return gpu_err(g, e, "batch begin");
    g->in_batch = true;
    return MOE_OK;
}

moe_status moe_batch_finish(moe_gpu *g, double *seconds) {
    moe_status st = need_batch(g);
    if (st) return st;
    if (g->capturing) return shape(g, "batch is capturing a graph; use moe_graph_end");
    g->in_batch = false;
    hipError_t e = hipEventRecord(g->ev_end, g->stream);
    if (e == hipSuccess) e = hipEventSynchronize(g->ev_end);
    if (e == hipSuccess) e = hipGetLastError();
    if (e != hipSuccess) return gpu_err(g, e, "batch");
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, g->ev_begin, g->ev_end);
    if (seconds) *seconds = ms * 1e-3;
    return MOE_OK;
}

// ================================================================== ops ==
moe_status moe_matmul(moe_gpu *g, const moe_weight *w, moe_buffer x, moe_buffer y,
                      uint64_t tokens) {
    moe_status st = need_batch(g);
    if (st) return st;
    if ((st = check_weight(g, w, "matmul"))) return st;
    // matrix.rs:64-75
    if (w->ndims != 2 || tokens == 0 || x.len != w->dims[0] * tokens || y.len != w->dims[1] * tokens)
        return shape(g, "matmul shape");
    if (!fits_u32(tokens)) return shape(g, "dimension exceeds u32");
    if ((st = check_own(g, {rng(x), rng(y)}))) return st;
    std::vector<Range> reads = weight_ranges(*w);
    reads.push_back(rng(x));
    if ((st = check_alias(g, reads, {rng(y)}, false))) return st;
    WDesc d = wdesc(*w);
    // 4 tokens or more: a tiled F32 product, as the reference switches to
    // affine_mm / gemm_simd (matrix.rs:77-123); fewer: one GEMV per token
    if (tokens >= 4 && f32mm_supported(d, (const float *)x.ptr))
        return launched(g, launch_f32mm(&g->prof, g->stream, "matmul_f32", d, (const float *)x.ptr,
                                        (uint32_t)tokens, 1, nullptr, (float *)y.ptr),
                        "matmul");
    return launched(g, launch_gemv(&g->prof, g->stream, d, (const float *)x.ptr, 0, nullptr, 1,
                                   (float *)y.ptr, (uint32_t)tokens),
                    "matmul");
}

moe_status moe_expert_matmul(moe_gpu *g, const moe_weight *w, moe_buffer x, moe_buffer ids,
                             moe_buffer y, int per_expert_input) {
    moe_status st = need_batch(g);
    if (st) return st;
    if ((st = check_weight(g, w, "expert matmul"))) return st;
    // matrix.rs:157-166
    if (w->ndims != 3 || x.len != w->dims[0] * (per_expert_input ? ids.len : 1) ||
        y.len != w->dims[1] * ids.len || ids.len == 0)
        return shape(g, "expert matmul");
    if (w->dims[2] < ids.len) return shape(g, "expert count");
    if ((st = check_own(g, {rng(x), rng(ids), rng(y)}))) return st;
    std::vector<Range> reads = weight_ranges(*w);
    reads.push_back(rng(x));
    reads.push_back(rng(ids));
    if ((st = check_alias(g, reads, {rng(y)}, false))) return st;
    WDesc d = wdesc(*w);
    return launched(g, launch_gemv(&g->prof, g->stream, d, (const float *)x.ptr,
                                   per_expert_input ? w->dims[0] : 0, (const uint32_t *)ids.ptr,
                                   (uint32_t)ids.len, (float *)y.ptr, 1),
                    "expert matmul");
}

moe_status moe_route(moe_gpu *g, moe_buffer logits, moe_buffer ids, moe_buffer weights,
                     int normalize) {
    moe_status st = need_batch(g);
    if (st) return st;
    // sampling.rs:28-30
    if (ids.len != weights.len || ids.len == 0 || ids.len > logits.len) return shape(g, "routing");
    if (logits.len > 16384) return shape(g, "routing: more than 16384 experts");
    if ((st = check_own(g, {rng(logits), rng(ids), rng(weights)}))) return st;
    if ((st = check_alias(g, {rng(logits)}, {rng(ids), rng(weights)}, false))) return st;
    return launched(g, launch_route(&g->prof, g->stream, (const float *)logits.ptr,
                                    (uint32_t)logits.len, (uint32_t)ids.len, normalize ? 1 : 0, 1,
                                    (uint32_t *)ids.ptr, (float *)weights.ptr),
                    "route");
}

moe_status moe_route_tokens(moe_gpu *g, moe_buffer logits, moe_buffer ids, moe_buffer weights,
                            uint64_t tokens, int normalize) {
    moe_status st = need_batch(g);
    if (st) return st;
    if (tokens == 0 || logits.len % tokens || ids.len % tokens || ids.len != weights.len)
        return shape(g, "routing");
    const uint64_t E = logits.len / tokens, K = ids.len / tokens;
    if (K == 0 || K > E) return shape(g, "routing");
    if (E > 16384 || !fits_u32(tokens)) return shape(g, "routing: size limit");
    if ((st = check_own(g, {rng(logits), rng(ids), rng(weights)}))) return st;
    if ((st = check_alias(g, {rng(logits)}, {rng(ids), rng(weights)}, false))) return st;
    return launched(g, launch_route(&g->prof, g->stream, (const float *)logits.ptr, (uint32_t)E,
                                    (uint32_t)K, normalize ? 1 : 0, (uint32_t)tokens,
                                    (uint32_t *)ids.ptr, (float *)weights.ptr),
                    "route");
}

moe_status moe_dispatch(moe_gpu *g, moe_buffer ids, uint64_t tokens, uint64_t k,
                        uint64_t experts, moe_buffer counts, moe_buffer offsets, moe_buffer perm,
                        moe_buffer pos) {
    moe_status st = need_batch(g);
    if (st) return st;
    if (tokens == 0 || k == 0 || experts == 0 || ids.len != tokens * k || counts.len != experts ||
        offsets.len != experts + 1 || perm.len != tokens * k || pos.len != tokens * k)
        return shape(g, "dispatch");
    if (experts > 16384 || !fits_u32(tokens * k)) return shape(g, "dispatch: size limit");
    if ((st = check_own(g, {rng(ids), rng(counts), rng(offsets), rng(perm), rng(pos)}))) return st;
    if ((st = check_alias(g, {rng(ids)}, {rng(counts), rng(offsets), rng(perm), rng(pos)}, false)))
        return st;
    return launched(g, launch_dispatch(&g->prof, g->stream, (const uint32_t *)ids.ptr,
                                       (uint32_t)(tokens * k), (uint32_t)experts,
                                       (uint32_t *)counts.ptr, (uint32_t *)offsets.ptr,
                                       (uint32_t *)perm.ptr, (uint32_t *)pos.ptr),
                    "dispatch");
}

static moe_status binary(moe_gpu *g, const char *name, moe_buffer a, moe_buffer b, moe_buffer y,
                         bool inplace) {
    moe_status st = need_batch(g);
    if (st) return st;
    // elementwise.rs:3-21
    if (a.len != b.len || a.len != y.len) return shape(g, name);
    if ((st = check_own(g, {rng(a), rng(b), rng(y)}))) return st;
    return check_alias(g, {rng(a), rng(b)}, {rng(y)}, inplace);
}

moe_status moe_swiglu(moe_gpu *g, moe_buffer a, moe_buffer b, moe_buffer y) {
    moe_status st = binary(g, "activation", a, b, y, true);
    if (st) return st;
    return launched(g, launch_swiglu(&g->prof, g->stream, (const float *)a.ptr, (const float *)b.ptr,
                                     (float *)y.ptr, y.len),
                    "swiglu");
}

moe_status moe_add(moe_gpu *g, moe_buffer a, moe_buffer b, moe_buffer y) {
    moe_status st = binary(g, "add", a, b, y, true);
    if (st) return st;
    return launched(g, launch_add(&g->prof, g->stream, (const float *)a.ptr, (const float *)b.ptr,
                                  (float *)y.ptr, y.len),
                    "add");
}

moe_status moe_gate_scalar(moe_gpu *g, moe_buffer x, moe_buffer gt, moe_buffer y) {
    moe_status st = need_batch(g);
    if (st) return st;
    // elementwise.rs:79-82
    if (x.len != y.len || gt.len != 1) return shape(g, "scalar gate");
    if ((st = check_own(g, {rng(x), rng(gt), rng(y)}))) return st;
    if ((st = check_alias(g, {rng(x), rng(gt)}, {rng(y)}, true))) return st;
    return launched(g, launch_gate_scalar(&g->prof, g->stream, (const float *)x.ptr,
                                          (const float *)gt.ptr, (float *)y.ptr, y.len),
                    "gate_scalar");
}

moe_status moe_mix(moe_gpu *g, moe_buffer x, moe_buffer w, moe_buffer y) {
    moe_status st = need_batch(g);
    if (st) return st;
    // elementwise.rs:92-95
    if (x.len != w.len * y.len || w.len == 0 || y.len == 0) return shape(g, "mix");
    if ((st = check_own(g, {rng(x), rng(w), rng(y)}))) return st;
    if ((st = check_alias(g, {rng(x), rng(w)}, {rng(y)}, false))) return st;
    return launched(g, launch_mix(&g->prof, g->stream, (const float *)x.ptr, (const float *)w.ptr,
                                  (uint32_t)w.len, y.len, (float *)y.ptr),
                    "mix");
}

moe_status moe_norm(moe_gpu *g, moe_buffer x, const moe_weight *w, moe_buffer y, uint64_t heads,
                    uint64_t stride, float eps) {
    moe_status st = need_batch(g);
    if (st) return st;
    if (!w) return shape(g, "norm");
    // attention.rs:12-31
    if (w->bits) return shape(g, "RMSNorm weights must be floating point");
    if ((st = check_weight(g, w, "norm"))) return st;
    const uint64_t n = w->dims[0];
    if (w->ndims != 1 || heads == 0 || stride < n || x.len < (heads - 1) * stride + n ||
        y.len != heads * n || !std::isfinite(eps) || eps <= 0.f)
        return shape(g, "norm");
    if (!fits_u32(heads) || !fits_u32(stride)) return shape(g, "dimension exceeds u32");
    if ((st = check_own(g, {rng(x), rng(y)}))) return st;
    if ((st = check_alias(g, {rng(x), rng(w->data)}, {rng(y)}, false))) return st;
    return launched(g, launch_norm(&g->prof, g->stream, (const float *)x.ptr, w->data.ptr, w->dtype,
                                   (float *)y.ptr, (uint32_t)heads, (uint32_t)n, (uint32_t)stride,
                                   eps),
                    "norm");
}

}  // extern "C"
