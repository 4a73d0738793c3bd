// The affine grouped GEMMs of launches that carry the shared expert as one
// more segment (gemm_kernels.hpp, affine_gemm_kernel with SH = true), in a
// translation unit of their own so they compile beside the routed-only
// kernels of k_gemm.hip.
#include "gemm_kernels.hpp"

namespace moehip {

namespace {

template <int MODE>
struct LaunchShared {
    Prof *p;
    hipStream_t s;
    const gemm::Args &a, &ash;
    uint32_t blocks;
    const char *name;
    template <int BITS, int T>
    hipError_t operator()() {
        if constexpr (BITS != 0)
            return launch_kernel(p, name, gemm::affine_gemm_kernel<MODE, BITS, T, true>, dim3(blocks),
                                 dim3(gemm::kAfThreads), 0, s, a, ash);
        return hipErrorInvalidValue;  // the shared segment runs on affine weights only
    }
};

}  // namespace

hipError_t launch_affine_shared(Prof *p, hipStream_t s, int down, const WDesc &w, const gemm::Args &a,
                                const gemm::Args &ash, uint32_t blocks, const char *name) {
    if (down) return dispatch_kind(w, LaunchShared<gemm::DOWN>{p, s, a, ash, blocks, name});
    return dispatch_kind(w, LaunchShared<gemm::GATEUP>{p, s, a, ash, blocks, name});
}

}  // namespace moehip
