// MFMA tile-order copy of an affine expert weight (the layout is described at
// PackedW in moe_internal.hpp).  The bf16-MFMA expert GEMM's B operand wants
// one weight row per lane pair, so from the row-major tensor every code load
// of a K step reads 32 bytes of 32 rows and every scale load a few bytes of
// 32 rows; from this copy each is one contiguous run.  The copy is made once,
// when the weights are prepared; the kernels here are plain gathers.
#include "moe_internal.hpp"

namespace moehip {

namespace {

constexpr uint32_t kPackThreads = 256;

// Codes: word q of the copy is word i of lane l of block (e, tile, kb); the
// lane's 32 codes 32h .. 32h + 31 of step kb are BITS consecutive words of
// row r of the row-major tensor (32 codes never straddle a word).
template <int BITS>
__global__ __launch_bounds__(kPackThreads) void pack_codes_kernel(const uint32_t *__restrict__ src,
                                                                  uint32_t *__restrict__ dst, uint32_t out,
                                                                  uint32_t in, uint32_t ntile, uint32_t nk,
                                                                  uint64_t words) {
    for (uint64_t q = (uint64_t)blockIdx.x * kPackThreads + threadIdx.x; q < words;
         q += (uint64_t)gridDim.x * kPackThreads) {
        const uint64_t blk = q / (64 * BITS);
        const uint32_t within = (uint32_t)(q % (64 * BITS));
        const uint32_t l = within / BITS, i = within % BITS;
        const uint32_t kb = (uint32_t)(blk % nk);
        const uint64_t et = blk / nk;
        const uint32_t tile = (uint32_t)(et % ntile);
        const uint64_t e = et / ntile;
        const uint32_t r = tile * 32 + (l & 31);
        uint32_t v = 0;
        if (r < out) {
            const uint64_t k0 = (uint64_t)kb * 64 + 32 * (l >> 5);
            v = src[((e * out + r) * in + k0) * BITS / 32 + i];
        }
        dst[q] = v;
    }
}

// Scales or biases: value q of the copy is group g of row rl of block
// (e, tile, p), i.e. group p * g2 + g of row tile * 32 + rl.
__global__ __launch_bounds__(kPackThreads) void pack_groups_kernel(const uint16_t *__restrict__ src,
                                                                   uint16_t *__restrict__ dst, uint32_t out,
                                                                   uint32_t row_groups, uint32_t ntile,
                                                                   uint32_t np, uint32_t g2, uint64_t n) {
    for (uint64_t q = (uint64_t)blockIdx.x * kPackThreads + threadIdx.x; q < n;
         q += (uint64_t)gridDim.x * kPackThreads) {
        const uint64_t blk = q / (32 * g2);
        const uint32_t within = (uint32_t)(q % (32 * g2));
        const uint32_t rl = within / g2, g = within % g2;
        const uint32_t pp = (uint32_t)(blk % np);
        const uint64_t et = blk / np;
        const uint32_t tile = (uint32_t)(et % ntile);
        const uint64_t e = et / ntile;
        const uint32_t r = tile * 32 + rl;
        dst[q] = r < out ? src[(e * out + r) * row_groups + pp * g2 + g] : (uint16_t)0;
    }
}

uint32_t grid_for(uint64_t n) {
    const uint64_t b = (n + kPackThreads - 1) / kPackThreads;
    return (uint32_t)(b < 65536 ? (b ? b : 1) : 65536);
}

}  // namespace

bool pack_layout(const WDesc &w, uint64_t *data_bytes, uint64_t *sb_bytes) {
    if ((w.bits != 2 && w.bits != 4 && w.bits != 8) || (w.type != 1 && w.type != 30)) return false;
    if (w.gshift < 5 || w.gshift > 7 || w.in % 128) return false;
    const uint64_t ntile = (w.out + 31) / 32, nk = w.in / 64;
    const uint64_t db = (uint64_t)w.experts * ntile * nk * 256 * w.bits;
    const uint64_t sb = (uint64_t)w.experts * ntile * (nk / 2) * 32 * (128u >> w.gshift) * 2;
    // the GEMM addresses both with 32-bit byte offsets
    if (db >= (1ull << 32) || sb >= (1ull << 32)) return false;
    *data_bytes = db;
    *sb_bytes = sb;
    return true;
}

hipError_t launch_pack_weight(Prof *p, hipStream_t s, const WDesc &w, void *data, void *scales,
                              void *biases) {
    uint64_t db = 0, sb = 0;
    if (!pack_layout(w, &db, &sb)) return hipErrorInvalidValue;
    const uint32_t ntile = (w.out + 31) / 32, nk = w.in / 64;
    const uint64_t words = db / 4;
    const uint32_t *src = static_cast<const uint32_t *>(w.data);
    uint32_t *dst = static_cast<uint32_t *>(data);
    hipError_t e;
    switch (w.bits) {
    case 2:
        e = launch_kernel(p, "pack_codes", pack_codes_kernel<2>, dim3(grid_for(words)), dim3(kPackThreads), 0,
                          s, src, dst, w.out, w.in, ntile, nk, words);
        break;
    case 4:
        e = launch_kernel(p, "pack_codes", pack_codes_kernel<4>, dim3(grid_for(words)), dim3(kPackThreads), 0,
                          s, src, dst, w.out, w.in, ntile, nk, words);
        break;
    default:
        e = launch_kernel(p, "pack_codes", pack_codes_kernel<8>, dim3(grid_for(words)), dim3(kPackThreads), 0,
                          s, src, dst, w.out, w.in, ntile, nk, words);
        break;
    }
    if (e != hipSuccess) return e;
    const uint32_t row_groups = w.in >> w.gshift, g2 = 128u >> w.gshift;
    const uint64_t n = sb / 2;
    e = launch_kernel(p, "pack_groups", pack_groups_kernel, dim3(grid_for(n)), dim3(kPackThreads), 0, s,
                      static_cast<const uint16_t *>(w.scales), static_cast<uint16_t *>(scales), w.out,
                      row_groups, ntile, nk / 2, g2, n);
    if (e != hipSuccess) return e;
    return launch_kernel(p, "pack_groups", pack_groups_kernel, dim3(grid_for(n)), dim3(kPackThreads), 0, s,
                         static_cast<const uint16_t *>(w.biases), static_cast<uint16_t *>(biases), w.out,
                         row_groups, ntile, nk / 2, g2, n);
}

}  // namespace moehip
