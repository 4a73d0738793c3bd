// moe_block_noalloc: moe_block with its workspace in a file-scope device
// array instead of a caller buffer, for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc).  No counterpart in the reference.
//
// `scratch` below has one copy per GPU, each at its own device address.  In
// host code its name is only a stand-in: noalloc_scratch_address looks the
// address up once per device (with that device current, from
// moe_gpu_create), and every host use -- the kernels' workspace argument --
// goes through that address.  Every call on one GPU shares the array and
// finds the previous call's contents in it; no kernel of the block reads a
// workspace word it has not written in the same call, so nothing needs
// clearing between calls.  Calls that overlap on one GPU (other streams,
// other moe_gpu handles of the same device) race on the array.
#include <mutex>

#include "abi_common.hpp"

static __device__ __align__(256) uint8_t scratch[MOE_NOALLOC_SCRATCH_BYTES];

namespace moehip {

hipError_t noalloc_scratch_address(int device, void **out) {
    static std::mutex mu;
    static std::map<int, void *> by_device;
    std::lock_guard<std::mutex> lock(mu);
    auto it = by_device.find(device);
    if (it != by_device.end()) {
        *out = it->second;
        return hipSuccess;
    }
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return e != hipSuccess ? e : hipErrorInvalidSymbol;
    by_device[device] = p;
    *out = p;
    return hipSuccess;
}

}  // namespace moehip

extern "C" moe_status moe_block_noalloc(moe_gpu *g, const moe_block_weights *w, moe_buffer x,
                                        moe_buffer out, uint64_t tokens, const moe_block_io *io) {
    if (!g) return MOE_ERR_SHAPE;
    if (!io) return shape(g, "missing block io");
    if (io->workspace.ptr || io->workspace.len) return shape(g, "moe_block_noalloc takes no workspace");
    if (!g->scratch) return fail(g, MOE_ERR_GPU, "no-allocation scratch unavailable on this device");
    moe_block_io with = *io;
    with.workspace = moe_buffer{g->scratch, MOE_NOALLOC_SCRATCH_BYTES / 4};
    return block_entry(g, w, x, out, tokens, &with, true);
}
