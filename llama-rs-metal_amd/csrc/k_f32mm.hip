// F32 products on the F32 matrix cores (v_mfma_f32_32x32x2_f32):
// y[t, r] = x_t . W_r (+ bias), W dims [in, out] (dense F32/F16/BF16 or
// affine 2/4/8-bit).  Two callers:
//  - the router product of the prefill path, Batch::matmul(router)
//    (crates/model-runtime/src/execute.rs:220).  The routing is exact given
//    the logits, so the logits themselves must be F32 products: bf16
//    operands change the selected experts of about 1-2% of the tokens of a
//    4096-token prefill;
//  - moe_matmul at 4 tokens or more, where the reference switches from its
//    GEMV kernels to tiled F32 GEMMs (affine_mm, gemm_simd / gemm_simd_wide,
//    crates/metal-backend/src/apple/ops/matrix.rs:77-123).
// Both operands stay F32: x as given, and the weights decoded to F32 exactly
// as Tensor::decode does (w = code * scale + bias, one product and one sum,
// crates/model-format/src/checkpoint.rs:164-196; F16/BF16 widened exactly).
// The products are the oracle's; only the summation order differs.
//
// Block = kWaves waves; wave w owns the 32x32 tile of 32 tokens x experts
// e0 + 32w .. +31 (rows r of W), over one of `ksplit` K ranges, in iterations of 64 K
// values.  The block's 32 token rows of an iteration reach LDS through
// coalesced loads (8 threads per 128-byte row segment), shared by the four
// waves; each lane loads its own expert row's 32 weight values of the
// iteration (one 16-byte load at 4 bits).  Lane (i = l % 32, h = l / 32)
// feeds x[i][32h + s] and R[e][32h + s], s = 0..31, to MFMA s of both lane
// halves (the same permutation of K on both operands).  x and the weights
// are loaded two iterations ahead, in a loop without branches; one barrier
// per iteration.  Token and expert rows past the ends are clamped for the
// loads and not stored.  With `xb16`, the blocks of the first expert column
// also store x rounded to bf16 (to nearest even) for the bf16 expert GEMMs,
// from the same staging registers: every (token, K range) is staged by
// exactly one of them, so x is read once for both products.  With `grow`
// (a dense F32 row: the shared expert's gate input, [h] reshaped [h, 1],
// crates/model-runtime/src/loader.rs:194), the same blocks also form x . grow
// from those registers, one partial sum per token, K range and expert column
// (each column takes every `columns`-th iteration) in gout[kr][column][t]
// (execute.rs:230 without a second pass over x).
#include <type_traits>

#include "rowdot.hpp"

namespace moehip {

namespace f32mm {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;

constexpr int kWaves = 4;                // expert tiles of 32 per block
constexpr int kThreads = 64 * kWaves;
constexpr int kIter = 64;                // K values per iteration (32 per lane half)
constexpr int kRow = kIter + 4;          // LDS floats per token row (16-byte pad: no bank conflicts)
constexpr uint32_t kTargetWaves = 2048;  // 2 per SIMD on 256 CUs
constexpr uint32_t kGateMax = 4096;      // K values of a range whose gate row is staged in LDS

// One lane's 32 weight values of one iteration, raw (as loaded).
template <int BITS, int T>
struct WRaw {
    static constexpr int NW = BITS == 0 ? (T == 0 ? 32 : 16) : BITS;
    uint32_t w[NW];
    uint32_t s, b;
};

template <int BITS, int T>
__device__ __forceinline__ void load_w(const WDesc &r, uint64_t el, WRaw<BITS, T> &o) {
    // el: the first of the lane's 32 consecutive values (a multiple of 32,
    // so they share one quantization group)
    constexpr int NW = WRaw<BITS, T>::NW;
    const uint8_t *base = reinterpret_cast<const uint8_t *>(r.data);
    const uint64_t byte = BITS ? el * BITS / 8 : el * (T == 0 ? 4 : 2);
    if constexpr (NW >= 4) {
#pragma unroll
        for (int v = 0; v < NW / 4; v++) {
            const u32x4 a = reinterpret_cast<const u32x4 *>(base + byte)[v];
#pragma unroll
            for (int i = 0; i < 4; i++) o.w[4 * v + i] = a[i];
        }
    } else {
        const u32x2 a = *reinterpret_cast<const u32x2 *>(base + byte);
        o.w[0] = a[0];
        o.w[1] = a[1];
    }
    if constexpr (BITS != 0) {
        o.s = load_raw<T>(r.scales, el >> r.gshift);
        o.b = load_raw<T>(r.biases, el >> r.gshift);
    }
}

// Values 16j .. 16j + 15 of the lane's 32 as F32: dense values widened
// exactly; affine values decoded as code * scale + bias with two roundings
// (no fused multiply-add), the values Tensor::decode produces.
template <int BITS, int T>
__device__ __forceinline__ void decode_w(const WRaw<BITS, T> &o, int j, float *v) {
    if constexpr (BITS == 0 && T == 0) {
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = __uint_as_float(o.w[16 * j + i]);
    } else if constexpr (BITS == 0) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[2 * i] = raw_to_f32<T>(o.w[8 * j + i] & 0xffffu);
            v[2 * i + 1] = raw_to_f32<T>(o.w[8 * j + i] >> 16);
        }
    } else {
        float c[16];
        constexpr int P = 32 / BITS;  // codes per word
#pragma unroll
        for (int i = 0; i < 16 / P; i++) unpack_word<BITS>(o.w[(16 / P) * j + i], c + P * i);
        const float s = raw_to_f32<T>(o.s), b = raw_to_f32<T>(o.b);
#pragma unroll
        for (int i = 0; i < 16; i++) {
#pragma clang fp contract(off)
            v[i] = c[i] * s + b;
        }
    }
}

template <int BITS, int T, bool GATE>
__global__ __launch_bounds__(kThreads) void f32mm_kernel(WDesc r, const float *__restrict__ x,
                                                              uint32_t tokens, uint32_t ksplit,
                                                              const float *__restrict__ bias,
                                                              float *__restrict__ out,
                                                              uint16_t *__restrict__ xb16,
                                                              const float *__restrict__ grow,
                                                              float *__restrict__ gout) {
    __shared__ __attribute__((aligned(16))) float xs[2][32 * kRow];
    __shared__ __attribute__((aligned(16))) float gs[GATE ? kGateMax : 4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t i = lane & 31, hf = lane >> 5;
    const uint32_t h = r.in, E = r.out;
    const uint32_t t0 = blockIdx.x * 32, e0 = (blockIdx.y * kWaves + wv) * 32;
    const uint32_t kr = blockIdx.z, klen = h / ksplit, kbeg = kr * klen;
    const uint32_t iters = klen / kIter;  // even
    // x staging: thread -> token row tid / 8, 16-byte chunks tid % 8 and
    // tid % 8 + 8 of the row's 64 values (8 threads read 128 contiguous bytes)
    const uint32_t srow = tid >> 3, sch = tid & 7;
    const f32x4 *xg = reinterpret_cast<const f32x4 *>(x + (uint64_t)min(t0 + srow, tokens - 1) * h + kbeg) + sch;
    // weights: lane (i, hf) holds values 32hf .. 32hf + 31 of the iteration of
    // expert e0 + i (clamped; rows past E are never stored)
    const uint64_t wel = (uint64_t)min(e0 + i, E - 1) * h + kbeg + 32 * hf;
    f32x16 acc = {};
    f32x4 xr[2][2];  // native vectors: HIP's float4 struct would stay in scratch
    WRaw<BITS, T> wr[2];
    // shared-gate row (GATE): the block's K range of it goes to LDS once
    // (klen <= kGateMax, checked on the host); in the iterations its expert
    // column takes, every thread multiplies the x values it stages with the
    // matching gate values (no loads in the loop; the branch is uniform), and
    // every column stores its partial sums
    float gsum = 0.f;
    if constexpr (GATE) {
        for (uint32_t k = 4 * tid; k < klen; k += 4 * kThreads)
            *reinterpret_cast<f32x4 *>(&gs[k]) = *reinterpret_cast<const f32x4 *>(grow + kbeg + k);
        __syncthreads();  // before the first staging reads it
    }
    auto gload_x = [&](int q, uint32_t it) __attribute__((always_inline)) {
        xr[q][0] = xg[it * (kIter / 4)];
        xr[q][1] = xg[it * (kIter / 4) + 8];
    };
    // bf16 copy of x: this thread's 2 x 4 values of iteration `it` of its row
    const bool copy = xb16 && blockIdx.y == 0 && t0 + srow < tokens;
    uint16_t *xbrow = copy ? xb16 + (uint64_t)(t0 + srow) * h + kbeg + 4 * sch : nullptr;
    auto put_x = [&](int q, int buf, uint32_t it) __attribute__((always_inline)) {
        float *d = &xs[buf][srow * kRow + 4 * sch];
        *reinterpret_cast<f32x4 *>(d) = xr[q][0];
        *reinterpret_cast<f32x4 *>(d + 32) = xr[q][1];
        if (copy && it < iters) {
            *reinterpret_cast<bf16x4 *>(xbrow + it * kIter) = __builtin_convertvector(xr[q][0], bf16x4);
            *reinterpret_cast<bf16x4 *>(xbrow + it * kIter + 32) = __builtin_convertvector(xr[q][1], bf16x4);
        }
        if constexpr (GATE) {
            // expert column y takes the iterations it % columns == y (uniform:
            // the columns share the work, so no block's span grows by all of it)
            if (it < iters && it % gridDim.y == blockIdx.y) {
                const uint32_t k0 = it * kIter + 4 * sch;
                const f32x4 g0 = *reinterpret_cast<const f32x4 *>(&gs[k0]);
                const f32x4 g1 = *reinterpret_cast<const f32x4 *>(&gs[k0 + 32]);
#pragma unroll
                for (int c = 0; c < 4; c++) gsum += xr[q][0][c] * g0[c];
#pragma unroll
                for (int c = 0; c < 4; c++) gsum += xr[q][1][c] * g1[c];
            }
        }
    };
    // one iteration: MFMA s of half j multiplies x[i][32hf + 16j + s] with
    // R[e][32hf + 16j + s] (the same permutation of K on both operands)
    auto compute = [&](int q, int buf) __attribute__((always_inline)) {
        const float *xrow = &xs[buf][i * kRow + 32 * hf];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            float wv16[16];
            decode_w<BITS, T>(wr[q], j, wv16);
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const f32x4 xv = *reinterpret_cast<const f32x4 *>(xrow + 16 * j + 4 * v);
#pragma unroll
                for (int c = 0; c < 4; c++)
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xv[c], wv16[4 * v + c], acc, 0, 0, 0);
            }
        }
    };
    // prologue: x of iteration 0 in LDS buffer 0, x of 1 in register stage 1,
    // weights of 0 and 1 in weight stages 0 and 1
    gload_x(0, 0);
    gload_x(1, min(1u, iters - 1));
    load_w<BITS, T>(r, wel, wr[0]);
    load_w<BITS, T>(r, wel + (uint64_t)min(1u, iters - 1) * kIter, wr[1]);
    put_x(0, 0, 0);
    __syncthreads();
    // Iteration it (stage Q = it % 2): load x of it + 2 into register stage Q
    // (its x of `it` went to LDS one iteration earlier); multiply LDS buffer
    // Q with weight stage Q; load the weights of it + 2 into weight stage Q;
    // store x of it + 1 (register stage Q ^ 1, loaded one iteration earlier)
    // into LDS buffer Q ^ 1; one barrier.  Indices past the last iteration
    // are clamped, so every load is in bounds, and the loop has no branches:
    // the compiler's in-order wait counts then keep the newest loads in
    // flight across the store.
    auto iteration = [&](uint32_t it, auto qc) __attribute__((always_inline)) {
        constexpr int Q = decltype(qc)::value;
        gload_x(Q, min(it + 2, iters - 1));
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
        compute(Q, Q);
        load_w<BITS, T>(r, wel + (uint64_t)min(it + 2, iters - 1) * kIter, wr[Q]);
        put_x(Q ^ 1, Q ^ 1, it + 1);  // x of iteration it + 1 (loaded one iteration earlier)
        __syncthreads();
    };
    for (uint32_t it = 0; it < iters; it += 2) {
        iteration(it, std::integral_constant<int, 0>{});
        iteration(it + 1, std::integral_constant<int, 1>{});
    }
    if constexpr (GATE) {
        // the 8 threads of a token row hold its partial sums
        gsum += __shfl_xor(gsum, 1, 64);
        gsum += __shfl_xor(gsum, 2, 64);
        gsum += __shfl_xor(gsum, 4, 64);
        if (sch == 0 && t0 + srow < tokens) gout[((uint64_t)kr * gridDim.y + blockIdx.y) * tokens + t0 + srow] = gsum;
    }
    // acc[q] = C[8(q/4) + 4(lane/32) + (q%4)][lane%32]: token row, expert column
    const uint32_t e = e0 + i;
    if (e >= E) return;
#pragma unroll
    for (int q = 0; q < 16; q++) {
        const uint32_t t = t0 + 8 * (q >> 2) + 4 * hf + (q & 3);
        if (t >= tokens) continue;
        const uint64_t o = (uint64_t)t * E + e;
        if (ksplit == 1)
            out[o] = bias ? acc[q] + bias[o] : acc[q];
        else
            out[(uint64_t)kr * tokens * E + o] = acc[q];
    }
}

struct Launch {
    Prof *p;
    hipStream_t s;
    const char *name;
    const WDesc &r;
    const float *x;
    uint32_t tokens, ksplit;
    const float *bias;
    float *out;
    uint16_t *xb16;
    const float *grow;
    float *gout;
    template <int BITS, int T>
    hipError_t operator()() {
        const dim3 grid((tokens + 31) / 32, (r.out + 32 * kWaves - 1) / (32 * kWaves), ksplit);
        if (grow)
            return launch_kernel(p, name, f32mm_kernel<BITS, T, true>, grid, dim3(kThreads), 0, s, r, x, tokens,
                                 ksplit, bias, out, xb16, grow, gout);
        return launch_kernel(p, name, f32mm_kernel<BITS, T, false>, grid, dim3(kThreads), 0, s, r, x, tokens,
                             ksplit, bias, out, xb16, grow, gout);
    }
};

}  // namespace f32mm

uint32_t f32mm_gate_max() { return f32mm::kGateMax; }
uint32_t f32mm_columns(const WDesc &w) { return (w.out + 32 * f32mm::kWaves - 1) / (32 * f32mm::kWaves); }

bool f32mm_supported(const WDesc &r, const float *x) {
    const bool kind = r.bits == 0 ? (r.type == 0 || r.type == 1 || r.type == 30)
                                  : (r.bits == 2 || r.bits == 4 || r.bits == 8) &&
                                        (r.type == 0 || r.type == 1 || r.type == 30);
    // an even number of iterations per K range; 16-byte operand loads (rows
    // of a multiple of 128 values start 16-byte aligned)
    return kind && r.in % (2 * f32mm::kIter) == 0 && r.experts == 1 &&
           ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(r.data)) & 15u) == 0;
}

uint32_t f32mm_ksplit(const WDesc &r, uint32_t tokens, uint64_t part_floats) {
    const uint64_t waves = (uint64_t)((tokens + 31) / 32) * ((r.out + 31) / 32);
    uint32_t ks = 1;
    // K ranges of an even number of iterations, until the grid holds
    // kTargetWaves waves, while the partial sums fit their buffer
    while (ks < 16 && waves * ks < f32mm::kTargetWaves && r.in % (2 * ks * 2 * f32mm::kIter) == 0 &&
           (uint64_t)(2 * ks) * tokens * r.out <= part_floats)
        ks *= 2;
    return ks;
}

hipError_t launch_f32mm(Prof *p, hipStream_t s, const char *name, const WDesc &r, const float *x,
                        uint32_t tokens, uint32_t ksplit, const float *bias, float *out, uint16_t *xb16,
                        const float *grow, float *gout) {
    if (tokens == 0 || ksplit == 0 || r.in % (ksplit * 2 * f32mm::kIter)) return hipErrorInvalidValue;
    if (grow && (!gout || (reinterpret_cast<uintptr_t>(grow) & 15u) || r.in / ksplit > f32mm::kGateMax))
        return hipErrorInvalidValue;
    return dispatch_kind(r, f32mm::Launch{p, s, name, r, x, tokens, ksplit, bias, out, xb16, grow, gout});
}

}  // namespace moehip
