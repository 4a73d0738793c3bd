// Grouped expert GEMMs of the prefill path: launch selection and argument
// set-up (the kernels and their design are in gemm_kernels.hpp).
#include "gemm_kernels.hpp"

namespace moehip {

namespace gemm {

template <int MODE>
struct Launch {
    Prof *p;
    hipStream_t s;
    const Args &a, &ash;
    uint32_t blocks;
    bool affine;  // affine_gemm_kernel (affine_blocks blocks)
    uint32_t affine_blocks;
    const char *name;
    template <int BITS, int T>
    hipError_t operator()() {
        if constexpr (BITS != 0) {
            if (affine)
                return launch_kernel(p, name, affine_gemm_kernel<MODE, BITS, T, false>, dim3(affine_blocks),
                                     dim3(kAfThreads), 0, s, a, ash);
        }
        return launch_kernel(p, name, grouped_gemm_kernel<MODE, BITS, T>, dim3(blocks), dim3(kThreads),
                             kLdsBytes, s, a);
    }
};

}  // namespace gemm

bool gemm_supported(const WDesc &w) {
    if (w.in % (2 * gemm::kTK)) return false;  // whole pairs of K steps
    if (w.bits == 0) return w.type == 0 || w.type == 1 || w.type == 30;
    return (w.bits == 2 || w.bits == 4 || w.bits == 8) && (w.type == 0 || w.type == 1 || w.type == 30);
}

uint32_t gemm_tile_rows() { return gemm::kTM; }

// Persistent grid: `per_cu` blocks on every CU (a multiple of 8 so each XCD
// gets the same number).
static uint32_t gemm_blocks(int per_cu = gemm::kBlocksPerCu) {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    return (uint32_t)((cus * per_cu + 7) / 8 * 8);
}

// affine_gemm_kernel addresses its operands with 32-bit buffer offsets.
static bool affine_fits(const WDesc &w, uint64_t a_rows_n) {
    if (w.bits == 0) return false;
    const uint64_t elems = (uint64_t)w.experts * w.out * w.in;
    const uint64_t groups = elems >> w.gshift;
    return elems < (1ull << 32) && groups * 4 < (1ull << 32) && a_rows_n * w.in * 2 < (1ull << 32);
}

// Allows the kernel's dynamic LDS size (above the default per-launch limit).
template <int MODE>
struct SetLds {
    template <int BITS, int T>
    hipError_t operator()() {
        return hipFuncSetAttribute((const void *)gemm::grouped_gemm_kernel<MODE, BITS, T>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, gemm::kLdsBytes);
    }
};

static bool same_kind(const WDesc &a, const WDesc &b) {
    return a.bits == b.bits && a.type == b.type && a.gshift == b.gshift;
}

bool gemm_shared_fold_ok(const WDesc &g, const WDesc &u, const WDesc &d, const WDesc &sg, const WDesc &su,
                         const WDesc &sd, uint64_t T, uint64_t K) {
    const uint64_t pairs = T * K + T;  // act16 rows: the routed pairs, then the shared rows
    return g.bits != 0 && same_kind(g, u) && same_kind(g, sg) && same_kind(g, su) && same_kind(d, sd) &&
           sg.out == g.out && su.out == g.out && sg.in == g.in && sd.in == d.in && sd.out == d.out &&
           affine_fits(g, T) && affine_fits(u, T) && affine_fits(sg, T) && affine_fits(su, T) &&
           affine_fits(d, pairs) && affine_fits(sd, pairs) && pairs < (1ull << 31);
}

hipError_t launch_grouped_gemm(Prof *p, hipStream_t s, int down, const WDesc &w, const WDesc &w2,
                               const PackedW &pk, const PackedW &pk2, const uint16_t *a_rows,
                               uint64_t a_rows_n, const uint32_t *perm, const uint32_t *offsets,
                               const uint32_t *tiles, const uint32_t *ntiles, uint32_t k,
                               uint16_t *out, const char *name, const SharedSeg *sh) {
    if (!name) name = down ? "gemm_down" : "gemm_gateup";
    gemm::Args a{};
    a.w = w;
    a.w2 = w2;
    a.a_rows = a_rows;
    a.perm = perm;
    a.offsets = offsets;
    a.tiles = tiles;
    a.ntiles = ntiles;
    a.out = out;
    a.k = k;
    const uint32_t blocks = gemm_blocks();
    const bool affine = affine_fits(w, a_rows_n) && affine_fits(w2, a_rows_n) && w2.bits == w.bits &&
                        w2.type == w.type && w2.gshift == w.gshift;
    const uint32_t affine_blocks = gemm_blocks(gemm::kAfBlocksPerCu);
    // the packed copies are read when both operands have one (16-bit scales)
    if (affine && w.type != 0 && pk.data && pk2.data) {
        a.pk = pk;
        a.pk2 = pk2;
    }
    // the shared expert: same kernel, its own weights; the gate/up product
    // reads the token's row (position - base), the down product its own rows
    gemm::Args ash = a;
    if (sh) {
        if (!affine || !same_kind(sh->w, w) || !same_kind(sh->w2, w) || sh->w.out != w.out ||
            sh->w.in != w.in || !affine_fits(sh->w, a_rows_n) || !affine_fits(sh->w2, a_rows_n))
            return hipErrorInvalidValue;
        ash.w = sh->w;
        ash.w2 = sh->w2;
        ash.pk = ash.pk2 = PackedW{};
        if (w.type != 0 && sh->pk.data && sh->pk2.data) {
            ash.pk = sh->pk;
            ash.pk2 = sh->pk2;
        }
        ash.perm = nullptr;
        ash.a_base = down ? 0u : sh->base;
        a.sh_mt = ash.sh_mt = (sh->rows + gemm::kTM - 1) / gemm::kTM;
        a.sh_base = ash.sh_base = sh->base;
        a.sh_rows = ash.sh_rows = sh->rows;
    }
    hipError_t e;
    if (down) {
        a.n_tiles_n = affine ? (w.out + 64 * gemm::kAfWaves - 1) / (64 * gemm::kAfWaves) : (w.out + gemm::kTN - 1) / gemm::kTN;
        if (!affine && (e = dispatch_kind(w, SetLds<gemm::DOWN>{})) != hipSuccess) return e;
        e = affine && a.sh_mt ? launch_affine_shared(p, s, 1, w, a, ash, affine_blocks, name)
                              : dispatch_kind(w, gemm::Launch<gemm::DOWN>{p, s, a, ash, blocks, affine, affine_blocks, name});
    } else {
        a.n_tiles_n = affine ? (w.out + 32 * gemm::kAfWaves - 1) / (32 * gemm::kAfWaves) : (w.out + gemm::kTN / 2 - 1) / (gemm::kTN / 2);
        if (!affine && (e = dispatch_kind(w, SetLds<gemm::GATEUP>{})) != hipSuccess) return e;
        e = affine && a.sh_mt ? launch_affine_shared(p, s, 0, w, a, ash, affine_blocks, name)
                              : dispatch_kind(w, gemm::Launch<gemm::GATEUP>{p, s, a, ash, blocks, affine, affine_blocks, name});
    }
    return e;
}

}  // namespace moehip
