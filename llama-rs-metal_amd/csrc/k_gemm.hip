// Grouped expert GEMMs of the prefill path on the bf16 matrix cores
// (v_mfma_f32_32x32x16_bf16), with the MLX-affine weights dequantised on the
// fly.  Token-batched replacement of the reference's per-token expert loop
// (crates/model-runtime/src/execute.rs:208-233): after dispatch every
// expert's (token, k) pairs form one contiguous segment, and each segment
// runs one GEMM against that expert's weights.
//
//   GATEUP  act[p, j] = silu(x_t . G_e[j]) * (x_t . U_e[j])   t = perm[p] / K
//           (activation, crates/metal-backend/src/shaders/elementwise.metal:8-17)
//   DOWN    y[p, r]   = act_p . D_e[r]   (the combine applies the routing weights)
//   ROUTER  logits[t, e] = x_t . R_e (+ bias), the router product
//           (Batch::matmul(router), crates/model-runtime/src/execute.rs:220);
//           one segment of all tokens, its K split into ksplit ranges whose
//           F32 partial sums the routing kernel adds in range order
//
// Work item = kTM pairs of one expert x one 128-row N-tile over the full K
// (ROUTER: over one of its K ranges).
// Blocks are persistent: the items are split into eight contiguous ranges,
// one per XCD (workgroup b runs on XCD b % 8), and the blocks of an XCD walk
// their range together, so the tiles that share an expert's weights and a
// segment's activation rows run side by side on one L2.
//
// Per 64-wide K step, double-buffered in LDS: the block's threads load the
// A tile (kTM rows x 128 bytes of bf16, rows gathered through perm for
// GATEUP) and the B tile (128 weight rows x 64 codes, dequantised once per
// block: w = code * scale + bias in F32, rounded to bf16); the global loads
// are issued two steps ahead (two register stages) so their latency hides
// behind two steps of matrix-core work.  Waves in a kWM x 2 layout each own
// a 64x64 sub-tile (2x2 MFMA tiles of 32x32).  Inside a K step lane half h of every
// wave feeds k = 32h + 8j + [0, 8) at MFMA step j to both operands (a
// permutation of K applied to A and B alike), so each fragment is one
// 16-byte LDS read.
#include <type_traits>

#include "rowdot.hpp"

namespace moehip {

namespace gemm {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Block layout: kWM x kWN waves, each owning kMT x kNT MFMA tiles of 32x32.
constexpr int kWM = 2, kWN = 2;          // waves along M / along N
constexpr int kMT = 2, kNT = 2;          // 32x32 tiles per wave along M / along N
constexpr int kTM = 32 * kMT * kWM;      // pairs per work item
constexpr int kTN = 32 * kNT * kWN;      // weight rows per tile
constexpr int kTK = 64;                  // K per step
constexpr int kRowBytes = kTK * 2 + 16;  // LDS row: kTK bf16 + 16-byte pad (bank spread)
constexpr int kATile = kTM * kRowBytes;  // one A stage
constexpr int kBTile = kTN * kRowBytes;  // one B stage
constexpr int kLdsBytes = 2 * kATile + 2 * kBTile;  // A and B, double-buffered
constexpr int kThreads = 64 * kWM * kWN;
constexpr int kMaxBlocksPerCu = 2;      // occupancy target (LDS and VGPRs allowing)
constexpr int kBlocksPerCu = kLdsBytes * kMaxBlocksPerCu <= 160 * 1024 ? kMaxBlocksPerCu
                             : kLdsBytes * 2 <= 160 * 1024            ? 2 : 1;
constexpr int kBVals = kTN * kTK / kThreads;  // weight values one thread dequantises per step
constexpr int kAChunksPerRow = kTK * 2 / 16;  // 16-byte chunks of one A row per step
constexpr int kAChunks = kTM * kAChunksPerRow / kThreads;  // A chunks one thread stages per step
constexpr int kARowsPerPass = kThreads / kAChunksPerRow;   // A rows one pass covers
constexpr int kXcds = 8;

enum { GATEUP = 1, DOWN = 2, ROUTER = 3 };
static_assert(kNT % 2 == 0, "gate/up columns pair up inside a wave");
static_assert(kBVals == 16 || kBVals == 32 || kBVals == 64, "whole words of codes per thread");
static_assert(kTM * kAChunksPerRow % kThreads == 0, "whole A chunks per thread");
static_assert(kTK == 32 || kTK == 64, "K step");

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Byte N of v as float: one v_cvt_f32_ubyteN (the compiler otherwise splits
// masked nibble extractions into a bit-field extract plus a conversion).
template <int N>
__device__ __forceinline__ float cvt_ubyte(uint32_t v) {
    float r;
    if constexpr (N == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (N == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (N == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// The codes of one packed word (low bits first) as floats: the word is split
// into byte-aligned code planes (one mask per plane), then each code converts
// with one instruction.
template <int BITS>
__device__ __forceinline__ void codes_f32(uint32_t w, float *c) {
    constexpr int P = 32 / BITS;        // codes per word
    constexpr int PLANES = 8 / BITS;    // codes per byte
    constexpr uint32_t kMask = BITS == 8 ? 0xffffffffu : BITS == 4 ? 0x0f0f0f0fu : 0x03030303u;
#pragma unroll
    for (int pl = 0; pl < PLANES; pl++) {
        const uint32_t v = (w >> (BITS * pl)) & kMask;  // code pl of every byte
        c[pl] = cvt_ubyte<0>(v);
        c[pl + PLANES] = cvt_ubyte<1>(v);
        c[pl + 2 * PLANES] = cvt_ubyte<2>(v);
        c[pl + 3 * PLANES] = cvt_ubyte<3>(v);
    }
    static_assert(P == 4 * PLANES, "four bytes per word");
}

struct Args {
    WDesc w, w2;               // B weights (w2: up for GATEUP)
    const uint16_t *a_rows;    // GATEUP: xb16 [T, in]; DOWN: act16 [P, in]
    const uint32_t *perm;      // pair order (GATEUP: token = perm / k; DOWN: routing weight index)
    const uint32_t *offsets;   // [E+1] segment offsets
    const uint32_t *tiles;     // [2*max_tiles] (expert, first position)
    const uint32_t *ntiles;    // number of valid M-tiles (device)
    uint16_t *out;             // GATEUP: act16 [P, ff]; DOWN: y16 [P, h]
    float *out_f32;            // ROUTER: logits [T, E] (ksplit 1) or partials [ksplit, T, E]
    const float *bias;         // ROUTER with ksplit 1: optional logit bias [T, E]
    uint32_t k;                // experts per token
    uint32_t n_tiles_n;        // N-tiles per M-tile
    uint32_t m_total;          // ROUTER: tokens
    uint32_t ksplit;           // ROUTER: K ranges (nk / ksplit is even)
};

// Per-thread source of kBVals consecutive K values of one weight row: the code
// (or dense) pointer of the row's first K step and, for affine weights, the
// row's first element index (its scale/bias group follows from it).
template <int BITS, int T>
struct BSrc {
    const uint8_t *data;   // bytes of K step 0 of this thread's 32 values
    const void *scales, *biases;
    uint64_t elem0;        // element index of K step 0 (affine group = elem >> gshift)
    uint32_t gshift;
    static constexpr uint32_t kStepBytes = BITS ? kTK * BITS / 8 : kTK * (T == 0 ? 4 : 2);
};

// Raw words of one K step (kBVals values) of a weight row plus the raw bits of
// its group's scale and bias; converted to bf16 only when stored to LDS, so
// the loads have no consumer before the next K step.
template <int BITS, int T>
struct BStage {
    static constexpr int NW = kBVals * (BITS ? BITS : (T == 0 ? 32 : 16)) / 32;  // source words
    uint32_t w[NW];
    uint32_t s, b;
    __device__ __forceinline__ void load(const BSrc<BITS, T> &src, uint32_t kb) {
        const uint8_t *p = src.data + (uint64_t)kb * BSrc<BITS, T>::kStepBytes;
        if constexpr (NW >= 4) {
#pragma unroll
            for (int i = 0; i < NW / 4; i++) {
                const u32x4 v = reinterpret_cast<const u32x4 *>(p)[i];
                w[4 * i] = v[0];
                w[4 * i + 1] = v[1];
                w[4 * i + 2] = v[2];
                w[4 * i + 3] = v[3];
            }
        } else if constexpr (NW == 2) {
            const u32x2 v = *reinterpret_cast<const u32x2 *>(p);
            w[0] = v[0];
            w[1] = v[1];
        } else {
            w[0] = *reinterpret_cast<const uint32_t *>(p);
        }
        if constexpr (BITS) {
            // kBVals values lie in one group (group >= 32)
            const uint64_t g = (src.elem0 + (uint64_t)kb * kTK) >> src.gshift;
            if constexpr (T == 0) {
                s = reinterpret_cast<const uint32_t *>(src.scales)[g];
                b = reinterpret_cast<const uint32_t *>(src.biases)[g];
            } else {
                s = reinterpret_cast<const uint16_t *>(src.scales)[g];
                b = reinterpret_cast<const uint16_t *>(src.biases)[g];
            }
        }
    }
    __device__ __forceinline__ static float scalar(uint32_t raw) {
        if constexpr (T == 0) return __uint_as_float(raw);
        else if constexpr (T == 30) return bf16_to_f32(raw);
        else return f16_to_f32(raw);
    }
    __device__ __forceinline__ void to_bf16(uint32_t *o /* kBVals / 2 words */) const {
        if constexpr (BITS) {
            constexpr int P = 32 / BITS;
            const float sf = scalar(s), bf = scalar(b);
#pragma unroll
            for (int i = 0; i < NW; i++) {
                float c[P];
                codes_f32<BITS>(w[i], c);
#pragma unroll
                for (int j = 0; j < P; j += 2)
                    o[(i * P + j) / 2] = pack_bf16(fmaf(c[j], sf, bf), fmaf(c[j + 1], sf, bf));
            }
        } else if constexpr (T == 30) {
#pragma unroll
            for (int i = 0; i < kBVals / 2; i++) o[i] = w[i];
        } else if constexpr (T == 1) {
#pragma unroll
            for (int i = 0; i < kBVals / 2; i++)
                o[i] = pack_bf16(f16_to_f32(w[i] & 0xffffu), f16_to_f32(w[i] >> 16));
        } else {
#pragma unroll
            for (int i = 0; i < kBVals / 2; i++) o[i] = pack_bf16(__uint_as_float(w[2 * i]), __uint_as_float(w[2 * i + 1]));
        }
    }
};

template <int BITS, int T>
__device__ __forceinline__ BSrc<BITS, T> make_bsrc(const WDesc &w, uint64_t grow, uint32_t k0) {
    BSrc<BITS, T> r;
    const uint64_t e0 = grow * w.in + k0;
    if constexpr (BITS)
        r.data = reinterpret_cast<const uint8_t *>(w.data) + e0 * BITS / 8;
    else
        r.data = reinterpret_cast<const uint8_t *>(w.data) + e0 * (T == 0 ? 4 : 2);
    r.scales = w.scales;
    r.biases = w.biases;
    r.elem0 = e0;
    r.gshift = w.gshift;
    return r;
}

template <int MODE, int BITS, int T>
__global__ __launch_bounds__(kThreads, kBlocksPerCu) void grouped_gemm_kernel(Args a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv % kWM, wn = wv / kWM;  // wave's row group and column group
    const uint32_t in = a.w.in, out = a.w.out;
    const uint32_t nk = in / kTK;
    // ---- this block's share of the work items ----
    const uint32_t n_tiles_m = MODE == ROUTER ? (a.m_total + kTM - 1) / kTM : 0;
    const uint32_t items = MODE == ROUTER ? n_tiles_m * a.n_tiles_n * a.ksplit : *a.ntiles * a.n_tiles_n;
    const uint32_t xcd = blockIdx.x % kXcds, q = blockIdx.x / kXcds, nq = gridDim.x / kXcds;
    const uint32_t per_xcd = (items + kXcds - 1) / kXcds;
    const uint32_t lo = xcd * per_xcd, hi = min(items, lo + per_xcd);
    // A staging: thread -> rows tid/kAChunksPerRow + kARowsPerPass*i, 16-byte chunk
    // tid%kAChunksPerRow of the K slice
    const int ac = tid % kAChunksPerRow, ar = tid / kAChunksPerRow;
    // B staging: thread -> tile row, kBVals values at kBVals*(quarter)
    constexpr int kBPerRow = kTK / kBVals;
    const int br = tid / kBPerRow, bq = tid % kBPerRow;

    for (uint32_t item = lo + q; item < hi; item += nq) {
        uint32_t mt, nt, e, m0, seg_end, ks = 0, kbeg = 0, kend = nk;
        if constexpr (MODE == ROUTER) {
            // consecutive items: M-tiles sharing one (K range, N-tile) of the router
            mt = item % n_tiles_m;
            const uint32_t rest = item / n_tiles_m;
            nt = rest % a.n_tiles_n;
            ks = rest / a.n_tiles_n;
            e = 0;
            m0 = mt * kTM;
            seg_end = a.m_total;
            kbeg = ks * (nk / a.ksplit);
            kend = kbeg + nk / a.ksplit;
        } else {
            mt = item / a.n_tiles_n;
            nt = item % a.n_tiles_n;
            e = a.tiles[2 * mt];
            m0 = a.tiles[2 * mt + 1];
            seg_end = a.offsets[e + 1];
        }
        // a wave whose rows all lie past the segment only loads and
        // dequantises (with one or two 64-row wave groups along M the first
        // rows are always live: no branch)
        const bool half_live = kMT * kWM <= 2 || m0 + 32 * kMT * (uint32_t)wm < seg_end;
        // A rows of this thread.  Rows past the segment read the segment's
        // first row instead: a C row depends only on its own A row, and those
        // rows are never stored.
        const uint16_t *asrc[kAChunks];
#pragma unroll
        for (int i = 0; i < kAChunks; i++) {
            uint32_t pos = m0 + ar + kARowsPerPass * i;
            if (pos >= seg_end) pos = m0;
            const uint64_t src = MODE == GATEUP ? a.perm[pos] / a.k : pos;
            asrc[i] = a.a_rows + src * in + 8 * ac;
        }
        // B row of this thread (rows past `out` read row 0 of the expert:
        // their C columns are never stored)
        BSrc<BITS, T> bsrc;
        {
            uint32_t j;
            bool second = false;  // GATEUP: the row comes from the up weights
            if constexpr (MODE == GATEUP) {
                const int q32 = br >> 5;  // 32-row groups alternate gate / up
                j = nt * (kTN / 2) + (q32 >> 1) * 32 + (br & 31);
                second = (q32 & 1) != 0;  // tile rows 32(2i+1).. are up rows
            } else {
                j = nt * kTN + br;
            }
            if (j >= out) j = 0;
            const uint64_t grow = (uint64_t)e * out + j;
            bsrc = second ? make_bsrc<BITS, T>(a.w2, grow, kBVals * bq)
                          : make_bsrc<BITS, T>(a.w, grow, kBVals * bq);
        }

        f32x16 acc[kMT][kNT];
#pragma unroll
        for (int s = 0; s < kMT; s++)
#pragma unroll
            for (int t = 0; t < kNT; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[s][t][r] = 0.f;

        // Two register stages: the global loads for step kb + 2 are issued in
        // iteration kb, stored to LDS in iteration kb + 1, used in kb + 2.
        u32x4 av[2][kAChunks];
        BStage<BITS, T> bs[2];
        auto load_step = [&](int st, uint32_t kb) {
#pragma unroll
            for (int i = 0; i < kAChunks; i++) av[st][i] = *reinterpret_cast<const u32x4 *>(asrc[i] + kb * kTK);
            bs[st].load(bsrc, kb);
        };
        auto store_step = [&](int st, int buf) {
            uint8_t *At = lds + buf * kATile;
            uint8_t *Bt = lds + 2 * kATile + buf * kBTile;
#pragma unroll
            for (int i = 0; i < kAChunks; i++)
                *reinterpret_cast<u32x4 *>(At + (ar + kARowsPerPass * i) * kRowBytes + 16 * ac) = av[st][i];
            uint32_t o[kBVals / 2];
            bs[st].to_bf16(o);
            u32x4 *bd = reinterpret_cast<u32x4 *>(Bt + br * kRowBytes + 2 * kBVals * bq);
#pragma unroll
            for (int i = 0; i < kBVals / 8; i++) bd[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
        };
        // One K step on LDS buffer ST: loads for kb + 2 into stage ST, MFMAs
        // on buffer ST, stage ST^1 (loaded one step earlier) -> buffer ST^1.
        // No branches around loads or stores: past the last step the loads
        // re-read step nk - 1 and the store fills the idle buffer, so the
        // compiler's wait counts let the just-issued loads stay in flight
        // across the store.
        auto iter = [&](uint32_t kb, auto st_c) {
            constexpr int ST = decltype(st_c)::value;
            load_step(ST, min(kb + 2, kend - 1));
            __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
            if (half_live) {
                const uint8_t *At = lds + ST * kATile;
                const uint8_t *Bt = lds + 2 * kATile + ST * kBTile;
                const int h = lane >> 5;
#pragma unroll
                for (int j = 0; j < kTK / 16; j++) {
                    const int koff = ((kTK / 2) * h + 8 * j) * 2;
                    bf16x8 af[kMT], bf[kNT];
#pragma unroll
                    for (int s = 0; s < kMT; s++)
                        af[s] = *reinterpret_cast<const bf16x8 *>(At + (32 * (kMT * wm + s) + (lane & 31)) * kRowBytes + koff);
#pragma unroll
                    for (int t = 0; t < kNT; t++)
                        bf[t] = *reinterpret_cast<const bf16x8 *>(Bt + (32 * (kNT * wn + t) + (lane & 31)) * kRowBytes + koff);
#pragma unroll
                    for (int s = 0; s < kMT; s++)
#pragma unroll
                        for (int t = 0; t < kNT; t++)
                            acc[s][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s], bf[t], acc[s][t], 0, 0, 0);
                }
            }
            store_step(ST ^ 1, ST ^ 1);  // may interleave with the MFMAs above
            __syncthreads();
        };
        load_step(0, kbeg);
        load_step(1, kbeg + 1);
        store_step(0, 0);
        __syncthreads();
        for (uint32_t kb = kbeg; kb < kend; kb += 2) {  // the range is even (in % 128 == 0)
            iter(kb, std::integral_constant<int, 0>{});
            iter(kb + 1, std::integral_constant<int, 1>{});
        }
        // ---- epilogue: acc[s][t][r] = C[32(kMT wm + s) + 8(r/4) + 4(lane/32) + (r%4)]
        //                             [32(kNT wn + t) + lane%32]
        if (!half_live) continue;
#pragma unroll
        for (int s = 0; s < kMT; s++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t pos = m0 + 32 * (kMT * wm + s) + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (pos >= seg_end) continue;
                if constexpr (MODE == GATEUP) {
                    // B rows 32(2i) .. are gate columns, 32(2i+1) .. the same up columns
#pragma unroll
                    for (int t = 0; t < kNT; t += 2) {
                        const uint32_t j = nt * (kTN / 2) + 32 * ((kNT * wn + t) / 2) + (lane & 31);
                        if (j < out) {
                            // activation (elementwise.metal:8-17) with the base-2
                            // exponential and a hardware reciprocal (the result is
                            // rounded to bf16)
                            const float g = acc[s][t][r], u = acc[s][t + 1][r];
                            const float act = g * __builtin_amdgcn_rcpf(1.0f + exp_fast(-g)) * u;
                            a.out[(uint64_t)pos * out + j] = (uint16_t)(pack_bf16(act, 0.f) & 0xffffu);
                        }
                    }
                } else if constexpr (MODE == ROUTER) {
#pragma unroll
                    for (int t = 0; t < kNT; t++) {
                        const uint32_t n = nt * kTN + 32 * (kNT * wn + t) + (lane & 31);
                        if (n >= out) continue;
                        if (a.ksplit == 1) {
                            const uint64_t o = (uint64_t)pos * out + n;
                            a.out_f32[o] = a.bias ? acc[s][t][r] + a.bias[o] : acc[s][t][r];
                        } else {
                            a.out_f32[((uint64_t)ks * a.m_total + pos) * out + n] = acc[s][t][r];
                        }
                    }
                } else {
#pragma unroll
                    for (int t = 0; t < kNT; t++) {
                        const uint32_t n = nt * kTN + 32 * (kNT * wn + t) + (lane & 31);
                        if (n < out)
                            a.out[(uint64_t)pos * out + n] = (uint16_t)(pack_bf16(acc[s][t][r], 0.f) & 0xffffu);
                    }
                }
            }
        }
    }
}

template <int MODE>
struct Launch {
    Prof *p;
    hipStream_t s;
    const Args &a;
    uint32_t blocks;
    template <int BITS, int T>
    hipError_t operator()() {
        return launch_kernel(p, MODE == DOWN ? "gemm_down" : MODE == ROUTER ? "gemm_router" : "gemm_gateup",
                             grouped_gemm_kernel<MODE, BITS, T>, dim3(blocks), dim3(kThreads),
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

// Persistent grid: kBlocksPerCu blocks on every CU (a multiple of 8 so each
// XCD gets the same number).
static uint32_t gemm_blocks() {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess)
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    return (uint32_t)((cus * gemm::kBlocksPerCu + 7) / 8 * 8);
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

hipError_t launch_grouped_gemm(Prof *p, hipStream_t s, int down, const WDesc &w, const WDesc &w2,
                               const uint16_t *a_rows, const uint32_t *perm, const uint32_t *offsets,
                               const uint32_t *tiles, const uint32_t *ntiles, uint32_t k,
                               uint16_t *out) {
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
    hipError_t e;
    if (down) {
        a.n_tiles_n = (w.out + gemm::kTN - 1) / gemm::kTN;
        if ((e = dispatch_kind(w, SetLds<gemm::DOWN>{})) != hipSuccess) return e;
        e = dispatch_kind(w, gemm::Launch<gemm::DOWN>{p, s, a, blocks});
    } else {
        a.n_tiles_n = (w.out + gemm::kTN / 2 - 1) / (gemm::kTN / 2);
        if ((e = dispatch_kind(w, SetLds<gemm::GATEUP>{})) != hipSuccess) return e;
        e = dispatch_kind(w, gemm::Launch<gemm::GATEUP>{p, s, a, blocks});
    }
    return e;
}

uint32_t gemm_router_ksplit(const WDesc &r, uint32_t tokens, uint64_t part_floats) {
    const uint32_t nk = r.in / gemm::kTK;
    const uint32_t tiles = (tokens + gemm::kTM - 1) / gemm::kTM * ((r.out + gemm::kTN - 1) / gemm::kTN);
    uint32_t ks = 1;
    // about two items per block of the persistent grid, each over an even
    // number of K steps, while the partial sums fit their buffer
    while (ks < 16 && tiles * ks * 2 < gemm_blocks() && nk % (4 * ks) == 0 &&
           (uint64_t)(2 * ks) * tokens * r.out <= part_floats)
        ks *= 2;
    return ks;
}

hipError_t launch_gemm_router(Prof *p, hipStream_t s, const WDesc &r, const uint16_t *xb16,
                              uint32_t tokens, uint32_t ksplit, const float *bias, float *out) {
    gemm::Args a{};
    a.w = r;
    a.w2 = r;
    a.a_rows = xb16;
    a.out_f32 = out;
    a.bias = bias;
    a.m_total = tokens;
    a.ksplit = ksplit;
    a.n_tiles_n = (r.out + gemm::kTN - 1) / gemm::kTN;
    hipError_t e;
    if ((e = dispatch_kind(r, SetLds<gemm::ROUTER>{})) != hipSuccess) return e;
    return dispatch_kind(r, gemm::Launch<gemm::ROUTER>{p, s, a, gemm_blocks()});
}

}  // namespace moehip
