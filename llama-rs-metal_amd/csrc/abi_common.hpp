// Host-side state and checks shared by the C ABI translation units.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/moe_hip.h"
#include "moe_internal.hpp"

namespace moehip {

struct ProfEntry {
    std::string name;
    uint64_t launches = 0;
    double seconds = 0.0;
};
struct Prof {
    bool enabled = false;
    std::vector<ProfEntry> entries;
    struct Pending {
        size_t entry;
        hipEvent_t a, b;
    };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> pool;
};
void prof_collect(Prof *p, hipStream_t s);
// Device address of this device's no-allocation scratch array (looked up
// once per device; the device must be current).
hipError_t noalloc_scratch_address(int device, void **out);

}  // namespace moehip

using namespace moehip;

struct Alloc {
    uint64_t bytes;
    bool owned;  // allocated by this library (freed on release/destroy)
};

struct moe_gpu {
    int device = 0;
    hipStream_t stream = nullptr;
    // second stream for work independent of the routing (the shared expert),
    // forked from and joined back into `stream` with these events
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    // device word of the fused route + dispatch launch: zero between launches
    uint32_t *arrive = nullptr;
    // this device's copy of the no-allocation scratch array (moe_noalloc.cpp),
    // null when its address could not be obtained
    void *scratch = nullptr;
    std::map<uintptr_t, Alloc> allocs;
    uint64_t live = 0;
    bool in_batch = false;
    bool capturing = false;
    hipEvent_t ev_begin = nullptr, ev_end = nullptr;
    std::string err;
    uint64_t err_bytes = 0;  // requested bytes of the last allocation error
    std::string name;
    Prof prof;
};

struct moe_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace abi {

inline moe_status fail(moe_gpu *g, moe_status st, const std::string &msg) {
    if (g) {
        g->err = msg;
        g->err_bytes = 0;
    }
    return st;
}
// Error::Allocation(usize) carries the requested byte count
// (crates/metal-backend/src/lib.rs:12-13, apple/memory.rs:9-17).
inline moe_status fail_alloc(moe_gpu *g, uint64_t bytes, const std::string &msg) {
    fail(g, MOE_ERR_ALLOCATION, msg);
    if (g) g->err_bytes = bytes;
    return MOE_ERR_ALLOCATION;
}
// n elements of 4 bytes, saturating (the reference's checked_mul(4) failure
// reports usize::MAX, memory.rs:26)
inline uint64_t elem_bytes(uint64_t n) { return n > UINT64_MAX / 4 ? UINT64_MAX : n * 4; }
inline moe_status shape(moe_gpu *g, const std::string &msg) { return fail(g, MOE_ERR_SHAPE, msg); }
inline moe_status gpu_err(moe_gpu *g, hipError_t e, const char *what) {
    return fail(g, MOE_ERR_GPU, std::string(what) + ": " + hipGetErrorString(e));
}

// ---------------------------------------------------------------- ranges --
struct Range {
    uintptr_t lo, hi;  // [lo, hi)
    bool empty() const { return hi <= lo; }
};
inline Range rng(const moe_buffer &b) {
    uintptr_t p = reinterpret_cast<uintptr_t>(b.ptr);
    return Range{p, p + b.len * 4};
}
inline Range rng(const moe_region &r) {
    uintptr_t p = reinterpret_cast<uintptr_t>(r.ptr);
    return Range{p, p + r.bytes};
}
inline bool overlaps(const Range &a, const Range &b) {
    return !a.empty() && !b.empty() && a.lo < b.hi && b.lo < a.hi;
}
inline bool same(const Range &a, const Range &b) { return a.lo == b.lo && a.hi == b.hi; }

// Gpu::own (apple/memory.rs:3-8): the view must lie inside one allocation of this gpu.
inline bool owns(const moe_gpu *g, const Range &r) {
    if (r.empty()) return false;
    auto it = g->allocs.upper_bound(r.lo);
    if (it == g->allocs.begin()) return false;
    --it;
    return r.lo >= it->first && r.hi <= it->first + it->second.bytes;
}

// commands.rs:109-150: outputs may not overlap each other or any input,
// except an exact in-place operand where the kernel allows it.
inline moe_status check_alias(moe_gpu *g, const std::vector<Range> &reads, const std::vector<Range> &writes,
                       bool inplace) {
    for (size_t i = 0; i < writes.size(); i++) {
        for (size_t j = i + 1; j < writes.size(); j++)
            if (overlaps(writes[i], writes[j])) return shape(g, "overlapping GPU outputs");
        for (const Range &r : reads)
            if (overlaps(writes[i], r) && !(inplace && same(writes[i], r)))
                return shape(g, "GPU input/output alias");
    }
    return MOE_OK;
}

inline moe_status check_own(moe_gpu *g, std::initializer_list<Range> rs) {
    for (const Range &r : rs)
        if (!owns(g, r)) return shape(g, "buffer belongs to a different engine");
    return MOE_OK;
}

inline bool fits_u32(uint64_t v) { return v <= 0xffffffffull; }

inline uint32_t scalar_bytes(uint32_t t) { return t == MOE_F32 ? 4 : 2; }
inline bool float_type(uint32_t t) { return t == MOE_F32 || t == MOE_F16 || t == MOE_BF16; }

// Tensor::new validation (crates/model-format/src/checkpoint.rs:88-130) plus
// ownership of every region and the u32 limits of the kernels
// (apple.rs:143-152).
inline moe_status check_weight(moe_gpu *g, const moe_weight *w, const char *what) {
    if (!w) return shape(g, std::string(what) + ": missing weight");
    if (w->ndims == 0 || w->ndims > 3) return shape(g, std::string(what) + ": tensor dimensions");
    uint64_t n = 1;
    for (uint32_t d = 0; d < w->ndims; d++) {
        if (w->dims[d] == 0) return shape(g, std::string(what) + ": tensor dimensions");
        if (n > UINT64_MAX / w->dims[d]) return shape(g, std::string(what) + ": tensor size overflow");
        n *= w->dims[d];
        if (!fits_u32(w->dims[d])) return shape(g, "dimension exceeds u32");
    }
    if (w->bits == 0) {
        if (!float_type(w->dtype)) return shape(g, std::string(what) + ": unsupported dtype");
        if (w->data.bytes != n * scalar_bytes(w->dtype))
            return shape(g, std::string(what) + ": tensor byte length");
        return check_own(g, {rng(w->data)});
    }
    if ((w->bits != 2 && w->bits != 4 && w->bits != 8) ||
        (w->group_size != 32 && w->group_size != 64 && w->group_size != 128))
        return shape(g, std::string(what) + ": unsupported MLX affine bits/group_size");
    if (!float_type(w->scale_type) || w->dims[0] % w->group_size)
        return shape(g, std::string(what) + ": affine scale type/group alignment");
    const uint64_t sb = (n / w->group_size) * scalar_bytes(w->scale_type);
    if (w->data.bytes != n * w->bits / 8 || w->scales.bytes != sb || w->biases.bytes != sb)
        return shape(g, std::string(what) + ": affine packed/scale/bias length");
    return check_own(g, {rng(w->data), rng(w->scales), rng(w->biases)});
}

inline uint32_t log2u(uint32_t v) {
    uint32_t s = 0;
    while ((1u << s) < v) s++;
    return s;
}

inline WDesc wdesc(const moe_weight &w) {
    WDesc d{};
    d.data = w.data.ptr;
    d.scales = w.scales.ptr;
    d.biases = w.biases.ptr;
    d.bits = w.bits;
    d.type = w.bits ? w.scale_type : w.dtype;
    d.in = (uint32_t)w.dims[0];
    d.out = w.ndims > 1 ? (uint32_t)w.dims[1] : 1u;
    d.experts = w.ndims > 2 ? (uint32_t)w.dims[2] : 1u;
    d.gshift = w.bits ? log2u(w.group_size) : 0;
    return d;
}

inline std::vector<Range> weight_ranges(const moe_weight &w) {
    std::vector<Range> v{rng(w.data)};
    if (w.bits) {
        v.push_back(rng(w.scales));
        v.push_back(rng(w.biases));
    }
    return v;
}

inline moe_status need_batch(moe_gpu *g) {
    if (!g) return MOE_ERR_SHAPE;
    if (!g->in_batch) return shape(g, "no open batch");
    (void)hipSetDevice(g->device);
    return MOE_OK;
}
inline moe_status need_no_batch(moe_gpu *g) {
    if (!g) return MOE_ERR_SHAPE;
    if (g->in_batch) return shape(g, "GPU memory access while a batch is open");
    (void)hipSetDevice(g->device);
    return MOE_OK;
}
inline moe_status launched(moe_gpu *g, hipError_t e, const char *what) {
    if (e != hipSuccess) return gpu_err(g, e, what);
    return MOE_OK;
}

inline moe_status alloc_bytes(moe_gpu *g, uint64_t bytes, void **out) {
    if (bytes == 0 || bytes / 4 > 0xffffffffull * 64) return fail_alloc(g, bytes, "allocation size");
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess || !p)
        return fail_alloc(g, bytes, "allocation of " + std::to_string(bytes) + " bytes failed");
    g->allocs[reinterpret_cast<uintptr_t>(p)] = Alloc{bytes, true};
    g->live += bytes;
    *out = p;
    return MOE_OK;
}

// moe_block's checks and dispatch over the paths (moe_block.cpp).  With
// `scratch`, io->workspace is the library's no-allocation scratch array
// (moe_noalloc.cpp) rather than a buffer this gpu owns.
moe_status block_entry(moe_gpu *g, const moe_block_weights *w, moe_buffer x, moe_buffer out,
                       uint64_t tokens, const moe_block_io *io, bool scratch);

}  // namespace abi
using namespace abi;

