// Device side of the grouped expert GEMMs, shared by k_gemm.hip (the
// launches over the routed experts) and k_gemm_shared.hip (the launches
// that carry the shared expert as one more segment).
//
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
// (The router product stays F32: k_f32mm.hip.)
//
// Work item = kTM pairs of one expert x one N-tile (128 weight rows for
// grouped_gemm, 64 per wave for affine_gemm) over the full K.
// Blocks are persistent: the items are split into eight contiguous ranges,
// one per XCD (workgroup b runs on XCD b % 8), and the blocks of an XCD walk
// their range together, so the tiles that share an expert's weights and a
// segment's activation rows run side by side on one L2.
//
// Two kernels share that schedule.  affine_gemm_kernel (GATEUP and DOWN over
// 2/4/8-bit affine weights, the prefill hot path) keeps the weights out of
// LDS: each of its four waves owns all kTM rows and 64 weight rows of the
// tile, loads its own codes into registers and dequantises them straight
// into MFMA operands (every weight value once per block), while the A tile
// reaches LDS by buffer DMA (buffer_load_dwordx4 ... lds), 16-byte chunks
// XOR-swizzled so the fragment reads are conflict-free.  Two such blocks
// share a CU; the four waves share one A stage, so per multiply-add half the
// A bytes of two-wave blocks move into the CU.  grouped_gemm_kernel (dense
// weights, and tensors whose offsets exceed 32 bits) stages both operands
// through LDS:
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
#pragma once
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

enum { GATEUP = 1, DOWN = 2 };
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
    const uint32_t *perm;      // pair order (GATEUP: token = perm / k; null: pair p is row p)
    const uint32_t *offsets;   // [E+1] segment offsets
    const uint32_t *tiles;     // [2*max_tiles] (expert, first position)
    const uint32_t *ntiles;    // number of valid M-tiles (device)
    uint16_t *out;             // GATEUP: act16 [P, ff]; DOWN: y16 [P, h]
    uint32_t k;                // experts per token
    uint32_t n_tiles_n;        // N-tiles per M-tile
    PackedW pk, pk2;           // affine GATEUP/DOWN: MFMA tile-order copies of w, w2 (or nulls)
    uint32_t a_base;           // perm null: pair p reads row p - a_base of a_rows
    // one more segment after the routed ones (the shared expert; affine_gemm_kernel
    // only): sh_mt M-tiles over positions [sh_base, sh_base + sh_rows), whose
    // weights and A rows the kernel's second Args describes
    uint32_t sh_mt, sh_base, sh_rows;
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
    const uint32_t items = *a.ntiles * a.n_tiles_n;
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
        const uint32_t mt = item / a.n_tiles_n, nt = item % a.n_tiles_n, kbeg = 0, kend = nk;
        const uint32_t e = a.tiles[2 * mt], m0 = a.tiles[2 * mt + 1];
        const uint32_t seg_end = a.offsets[e + 1];
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
            const uint64_t src = MODE == GATEUP && a.perm ? a.perm[pos] / a.k : pos;
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

// ------------------------------------------------------ affine_gemm ----
constexpr int kAfWaves = 4;                  // waves per block, sharing one A stage
constexpr int kAfThreads = 64 * kAfWaves;
constexpr int kAfBlocksPerCu = 2;            // 2 x 32 KiB of LDS, 2 waves per SIMD
constexpr int kAfNT = 2;            // 32-row weight tiles per wave
constexpr int kAfATile = kTM * kTK * 2;  // one A stage: kTM rows x 128 bytes
constexpr int kEpiRow = 32 * 2 + 16;             // staged gate/up epilogue row: 32 bf16 + pad
constexpr int kEpiBytes = 32 * kEpiRow;           // a wave's staging area: one 32-row slice

typedef __attribute__((address_space(3))) void *lds_ptr_t;
// Position of 16-byte chunk c of A-tile row r inside the row: chunks are
// XOR-permuted so the 32 rows one fragment read touches spread over the banks.
__device__ __forceinline__ uint32_t a_chunk(uint32_t r, uint32_t c) { return c ^ ((r ^ (r >> 3)) & 7u); }

// One lane's codes (32 consecutive K values) of its kAfNT weight rows for one
// K step, with the raw bits of their groups' scales and biases (F32 scales).
template <int BITS>
struct AfStage {
    uint32_t w[kAfNT][BITS];
    uint32_t s[kAfNT], b[kAfNT];
};
// 16-bit scales and biases of one lane's rows for two K steps: the 8 bytes
// from the (even) group holding the pair's first element.
struct AfScales {
    uint32_t s[kAfNT][2], b[kAfNT][2];
};

// The 8 codes k = 8j .. 8j + 7 of a lane's 32, as floats.
template <int BITS>
__device__ __forceinline__ void codes8(const uint32_t *w, int j, float *c) {
    if constexpr (BITS == 4) {
        codes_f32<4>(w[j], c);
    } else if constexpr (BITS == 8) {
        codes_f32<8>(w[2 * j], c);
        codes_f32<8>(w[2 * j + 1], c + 4);
    } else {
        float t[16];
        codes_f32<2>(w[j >> 1] >> (16 * (j & 1)), t);
#pragma unroll
        for (int i = 0; i < 8; i++) c[i] = t[i];
    }
}

// One work item with NS live 32-row slices of A (rows past the segment end
// are neither loaded nor multiplied).  Wave wv owns weight rows
// [64 wv, 64 wv + 64) of the N-tile (GATEUP: 32 gate rows and the 32 up rows
// of the same outputs); lane half h feeds K values 32h + 8j + [0, 8) at MFMA
// step j to both operands.  GS = log2(group size) for 16-bit scales, whose
// scale and bias loads then cover two K steps; 0 for F32 scales (one load
// per step).
template <int MODE, int NS>
__device__ __forceinline__ void affine_store(const Args &a, const f32x16 (&acc)[NS][kAfNT], uint32_t nt,
                                             uint32_t m0, uint32_t seg_end, uint32_t out, int h, int l32,
                                             int wv, uint8_t *stage);

template <int MODE, int BITS, int T, int NS, int GS, bool PK>
__device__ __forceinline__ void affine_item(const Args &a, uint8_t *abuf, uint32_t nt, uint32_t e,
                                            uint32_t m0, uint32_t seg_end, int lane, int wv) {
    static_assert(!PK || GS != 0, "packed copies carry 16-bit scales");
    const int h = lane >> 5, l32 = lane & 31;
    const uint32_t in = a.w.in, out = a.w.out, nk = in / kTK;
    static_assert((4 * NS) % kAfWaves == 0, "the live rows split evenly over the waves' DMA");
    constexpr int ND = 4 * NS / kAfWaves;  // DMA instructions per wave and step (8 rows each)
    // A: DMA instruction i of wave wv fills tile rows 8 kAfWaves i + 8wv .. +7, lane
    // (row, chunk position) = (lane / 8, lane % 8); byte offsets below 2^32
    // (checked on the host).  Rows past the segment re-read its first row.
    const uint32_t drow = 8 * wv + (lane >> 3), dpos = lane & 7;
    uint32_t aoff[ND];
#pragma unroll
    for (int i = 0; i < ND; i++) {
        const uint32_t r = 8 * kAfWaves * i + drow;
        uint32_t pos = m0 + r;
        if (pos >= seg_end) pos = m0;
        const uint32_t src = MODE == GATEUP && a.perm ? a.perm[pos] / a.k : pos - a.a_base;
        aoff[i] = src * in * 2 + (a_chunk(r, dpos) << 4);
    }
    // B: weight row n of tile t; rows past `out` read row 0 (never stored)
    uint32_t el0[kAfNT];  // element index of the lane's codes at K step 0 (< 2^32, host-checked)
    // PK: byte offsets of the lane's codes at K step 0 and of its scales at
    // step pair 0 in the packed copies (< 2^32, host-checked)
    constexpr uint32_t kG2 = GS ? 128u >> GS : 1u;  // groups per row and step pair
    uint32_t pko[kAfNT], pks[kAfNT];
    const uint32_t ntile = (out + 31) / 32;
#pragma unroll
    for (int t = 0; t < kAfNT; t++) {
        uint32_t n = MODE == GATEUP ? nt * (32 * kAfWaves) + 32 * wv + l32 : nt * (64 * kAfWaves) + 64 * wv + 32 * t + l32;
        const uint32_t tile = (e * ntile + n / 32);
        pko[t] = tile * nk * (256 * BITS) + lane * (4 * BITS);
        pks[t] = tile * (nk / 2) * (32 * kG2 * 2) + l32 * (kG2 * 2);
        if (n >= out) n = 0;
        el0[t] = (e * out + n) * in + 32 * h;
    }
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(a.a_rows);
    const void *wd[kAfNT] = {PK ? a.pk.data : a.w.data, PK ? (MODE == GATEUP ? a.pk2.data : a.pk.data)
                                                              : (MODE == GATEUP ? a.w2.data : a.w.data)};
    const void *ws[kAfNT] = {PK ? a.pk.scales : a.w.scales, PK ? (MODE == GATEUP ? a.pk2.scales : a.pk.scales)
                                                                  : (MODE == GATEUP ? a.w2.scales : a.w.scales)};
    const void *wb[kAfNT] = {PK ? a.pk.biases : a.w.biases, PK ? (MODE == GATEUP ? a.pk2.biases : a.pk.biases)
                                                                  : (MODE == GATEUP ? a.w2.biases : a.w.biases)};
    const __amdgpu_buffer_rsrc_t rw[kAfNT] = {buffer_rsrc(wd[0]), buffer_rsrc(wd[1])};
    // scale / bias arrays with their true sizes: the two-step loads may run
    // past the last group, and the hardware returns 0 there
    const uint32_t sb_bytes =
        PK ? (uint32_t)((uint64_t)a.w.experts * ntile * (nk / 2) * (32 * kG2 * 2))
           : (uint32_t)(((uint64_t)a.w.experts * out * in >> a.w.gshift) * (T == 0 ? 4 : 2));
    const __amdgpu_buffer_rsrc_t rs[kAfNT] = {buffer_rsrc(ws[0], sb_bytes), buffer_rsrc(ws[1], sb_bytes)};
    const __amdgpu_buffer_rsrc_t rb[kAfNT] = {buffer_rsrc(wb[0], sb_bytes), buffer_rsrc(wb[1], sb_bytes)};
    const uint32_t gshift = a.w.gshift;

    f32x16 acc[NS][kAfNT];
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
        for (int t = 0; t < kAfNT; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[s][t][r] = 0.f;

    auto dma = [&](uint32_t buf, uint32_t kb) {
        uint8_t *dst = abuf + buf * kAfATile + 8 * wv * (kTK * 2);
#pragma unroll
        for (int i = 0; i < ND; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(dst + 8 * kAfWaves * i * (kTK * 2)), 16, aoff[i],
                                                     kb * (kTK * 2), 0, 0);
    };
    auto load_b = [&](AfStage<BITS> &st, uint32_t kb) {
#pragma unroll
        for (int t = 0; t < kAfNT; t++) {
            const uint32_t vo = PK ? pko[t] : el0[t] / (8 / BITS), so = kb * (PK ? 256 * BITS : 8 * BITS);
            if constexpr (BITS == 2) {
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rw[t], vo, so, 0);
                st.w[t][0] = v[0];
                st.w[t][1] = v[1];
            } else {
#pragma unroll
                for (int i = 0; i < BITS / 4; i++) {
                    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw[t], vo + 16 * i, so, 0);
                    st.w[t][4 * i] = v[0];
                    st.w[t][4 * i + 1] = v[1];
                    st.w[t][4 * i + 2] = v[2];
                    st.w[t][4 * i + 3] = v[3];
                }
            }
            if constexpr (GS == 0) {
                const uint32_t g = (el0[t] + kb * kTK) >> gshift;  // 32 codes lie in one group
                st.s[t] = __builtin_amdgcn_raw_buffer_load_b32(rs[t], g * 4, 0, 0);
                st.b[t] = __builtin_amdgcn_raw_buffer_load_b32(rb[t], g * 4, 0, 0);
            }
        }
    };
    // Two-step scales (kb even): 8 bytes from group (row start + 64 kb) >> GS
    // rounded down to even, so the load is 4-byte aligned (for GS 5 and 6 the
    // group is already even: in % 128 == 0).  Within them lane half h finds
    // step kb + s's group at element (64 s + 32 h) >> GS for GS 5 and 6; for
    // GS 7 one group spans the two steps, at element (row start + 64 kb) >> 7
    // mod 2.
    auto load_sb = [&](AfScales &sc2, uint32_t kb) {
        if constexpr (GS != 0) {
#pragma unroll
            for (int t = 0; t < kAfNT; t++) {
                if constexpr (PK) {
                    // the tile's block for step pair kb / 2: this row's kG2 values
                    const uint32_t so = (kb / 2) * (32 * kG2 * 2);
                    if constexpr (GS == 5) {
                        const u32x2 vs = __builtin_amdgcn_raw_buffer_load_b64(rs[t], pks[t], so, 0);
                        const u32x2 vb = __builtin_amdgcn_raw_buffer_load_b64(rb[t], pks[t], so, 0);
                        sc2.s[t][0] = vs[0];
                        sc2.s[t][1] = vs[1];
                        sc2.b[t][0] = vb[0];
                        sc2.b[t][1] = vb[1];
                    } else if constexpr (GS == 6) {
                        sc2.s[t][0] = __builtin_amdgcn_raw_buffer_load_b32(rs[t], pks[t], so, 0);
                        sc2.b[t][0] = __builtin_amdgcn_raw_buffer_load_b32(rb[t], pks[t], so, 0);
                    } else {
                        sc2.s[t][0] = __builtin_amdgcn_raw_buffer_load_b16(rs[t], pks[t], so, 0);
                        sc2.b[t][0] = __builtin_amdgcn_raw_buffer_load_b16(rb[t], pks[t], so, 0);
                    }
                } else {
                    const uint32_t g = ((el0[t] - 32 * h + kb * kTK) >> GS) & ~1u;
                    const u32x2 vs = __builtin_amdgcn_raw_buffer_load_b64(rs[t], g * 2, 0, 0);
                    const u32x2 vb = __builtin_amdgcn_raw_buffer_load_b64(rb[t], g * 2, 0, 0);
                    sc2.s[t][0] = vs[0];
                    sc2.s[t][1] = vs[1];
                    sc2.b[t][0] = vb[0];
                    sc2.b[t][1] = vb[1];
                }
            }
        }
    };
    // raw 16-bit value (in the low half) of step kb + s of weight tile t from
    // a two-step load
    auto pick = [&](const uint32_t *pair, int t, int s, uint32_t kb) -> uint32_t {
        if constexpr (GS == 5) return pair[s] >> (16 * h);
        else if constexpr (GS == 6) return pair[0] >> (16 * s);
        else if constexpr (PK) return pair[0];
        else return pair[0] >> (16 * (((el0[t] - 32 * h + kb * kTK) >> 7) & 1));
    };
    auto compute = [&](const uint8_t *cur, const AfStage<BITS> &sc, const AfScales &sc2, int s2, uint32_t kb) {
        float sf[kAfNT], bf[kAfNT];
#pragma unroll
        for (int t = 0; t < kAfNT; t++) {
            if constexpr (GS == 0) {
                sf[t] = BStage<BITS, T>::scalar(sc.s[t]);
                bf[t] = BStage<BITS, T>::scalar(sc.b[t]);
            } else {
                sf[t] = BStage<BITS, T>::scalar(pick(sc2.s[t], t, s2, kb) & 0xffffu);
                bf[t] = BStage<BITS, T>::scalar(pick(sc2.b[t], t, s2, kb) & 0xffffu);
            }
        }
#pragma unroll
        for (int j = 0; j < kTK / 16; j++) {
            bf16x8 bfr[kAfNT], afr[NS];
#pragma unroll
            for (int s = 0; s < NS; s++) {
                const uint32_t R = 32 * s + l32;
                afr[s] = *reinterpret_cast<const bf16x8 *>(cur + R * (kTK * 2) + (a_chunk(R, 4 * h + j) << 4));
            }
#pragma unroll
            for (int t = 0; t < kAfNT; t++) {
                // w = code * scale + bias in F32, rounded to bf16
                float c[8];
                codes8<BITS>(sc.w[t], j, c);
                u32x4 o;
#pragma unroll
                for (int i = 0; i < 4; i++) o[i] = pack_bf16(fmaf(c[2 * i], sf[t], bf[t]), fmaf(c[2 * i + 1], sf[t], bf[t]));
                bfr[t] = __builtin_bit_cast(bf16x8, o);
            }
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
                for (int t = 0; t < kAfNT; t++)
                    acc[s][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afr[s], bfr[t], acc[s][t], 0, 0, 0);
        }
    };
    // Step kb: wait for this wave's DMA into stage kb & 1 and its weight loads
    // (issued one step earlier), then the barrier makes the other wave's DMA
    // visible and retires both waves' reads of the other stage, which the
    // DMA for kb + 1 then refills.  Past the last step the loads repeat step
    // nk - 1 into the idle stage.
    __builtin_amdgcn_s_waitcnt(0);  // the previous item's last DMA landed
    __builtin_amdgcn_s_barrier();   // and both waves finished reading both stages
    if (MODE == DOWN && BITS == 4 && nk % 4 == 0) {
        // (The down product only: config 4 same-box A/B, down 159.8 -> 151.8 us;
        // gate/up 254.7 -> 262.3 us, so it keeps the one-step loop below.  With
        // 8-bit codes the fourth stage spills.)
        // Weights two steps ahead: a ring of four register stages (step kb in
        // stage kb % 4) and two scale pairs (steps 2p, 2p + 1 in pair p % 2).
        // Step kb: wait only for this wave's DMA of A step kb (issued one step
        // earlier; the weight and scale loads issued after it may stay in
        // flight), barrier, DMA of step kb + 1, weights of kb + 2 and on even
        // steps the scales of pair kb / 2 + 1, then the MFMAs of step kb.  The
        // compiler's own waits cover the register stages.
        constexpr int NB = kAfNT * (BITS == 8 ? 2 : 1) + (GS == 0 ? 2 * kAfNT : 0);  // loads per load_b
        constexpr int NSB = GS == 0 ? 0 : 2 * kAfNT;                                 // loads per load_sb
        AfStage<BITS> b4[4];
        AfScales s2[2];
        dma(0, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_b(b4[0], 0);
        load_sb(s2[0], 0);
        load_b(b4[1], 1);
        auto step = [&](uint32_t kb, auto qc) __attribute__((always_inline)) {
            constexpr int Q = decltype(qc)::value;  // kb % 4
            constexpr int N = NB + (Q & 1 ? NSB : 0);  // loads issued after this step's DMA
            // s_waitcnt vmcnt(N), expcnt and lgkmcnt untouched (gfx9 encoding)
            __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
            __builtin_amdgcn_s_barrier();
            dma((Q + 1) & 1, min(kb + 1, nk - 1));
            // the DMA issues before the loads the wait count above leaves in flight
            __builtin_amdgcn_sched_barrier(0);
            load_b(b4[(Q + 2) & 3], min(kb + 2, nk - 1));
            if constexpr ((Q & 1) == 0) load_sb(s2[((Q >> 1) + 1) & 1], min(kb + 2, nk - 2));
            compute(abuf + (Q & 1) * kAfATile, b4[Q], s2[(Q >> 1) & 1], Q & 1, kb & ~1u);
        };
        for (uint32_t kb = 0; kb < nk; kb += 4) {
            step(kb, std::integral_constant<int, 0>{});
            step(kb + 1, std::integral_constant<int, 1>{});
            step(kb + 2, std::integral_constant<int, 2>{});
            step(kb + 3, std::integral_constant<int, 3>{});
        }
        affine_store<MODE>(a, acc, nt, m0, seg_end, out, h, l32, wv, abuf + 2 * kAfATile + wv * kEpiBytes);
        return;
    }
    AfStage<BITS> bs0, bs1;
    AfScales sb;
    dma(0, 0);
    load_b(bs0, 0);
    load_sb(sb, 0);
    // even step: its scales are element s = 0 of the pair loaded one step
    // earlier; odd step: element 1, and the next pair is loaded (the compiler
    // keeps the old pair live until the odd step's compute has read it)
    for (uint32_t kb = 0; kb < nk; kb += 2) {  // nk is even (in % 128 == 0)
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_s_barrier();
        dma(1, kb + 1);
        load_b(bs1, kb + 1);
        compute(abuf, bs0, sb, 0, kb);
        const AfScales cur = sb;
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_s_barrier();
        const uint32_t kn = min(kb + 2, nk - 1);
        dma(0, kn);
        load_b(bs0, kn);
        load_sb(sb, min(kb + 2, nk - 2));
        compute(abuf + kAfATile, bs1, cur, 1, kb);
    }
    affine_store<MODE>(a, acc, nt, m0, seg_end, out, h, l32, wv, abuf + 2 * kAfATile + wv * kEpiBytes);
}

// acc[s][t][r] = C[32 s + 8 (r / 4) + 4 h + r % 4][this wave's column 32 t + l32]
//
// GATEUP with out % 8 == 0: each 32-row slice of activations goes through
// the wave's own LDS staging area (`stage`, kEpiBytes) as bf16 and leaves in
// 16-byte row chunks, one global_store_dwordx4 per 8 outputs instead of one
// 16-bit store per output (config 4: gate/up 250.5 -> 245.1 us).  The down
// product keeps the per-output stores: its staged form spilled and ran
// slower.  Staged rows are kEpiRow bytes apart, so the lane halves, which write
// rows 4 apart, land 16 banks apart.
template <int MODE>
__device__ __forceinline__ float affine_out(const f32x16 (&acc)[kAfNT], int t, int r) {
    if constexpr (MODE == GATEUP) {
        // activation (elementwise.metal:8-17), base-2 exponential and
        // hardware reciprocal; the result is rounded to bf16
        const float g = acc[0][r], u = acc[1][r];
        return g * __builtin_amdgcn_rcpf(1.0f + exp_fast(-g)) * u;
    } else {
        return acc[t][r];
    }
}

template <int MODE, int NS>
__device__ __forceinline__ void affine_store(const Args &a, const f32x16 (&acc)[NS][kAfNT], uint32_t nt,
                                             uint32_t m0, uint32_t seg_end, uint32_t out, int h, int l32,
                                             int wv, uint8_t *stage) {
    const uint32_t col0 = MODE == GATEUP ? nt * (32 * kAfWaves) + 32 * wv : nt * (64 * kAfWaves) + 64 * wv;
    if (MODE == GATEUP && out % 8 == 0) {
        constexpr int kRow = kEpiRow;
        constexpr int kChunksPerRow = 4;               // 16-byte chunks per row
        constexpr int kRowsPerPass = 64 / kChunksPerRow;
        const int lane = 32 * h + l32;
        const int crow = lane / kChunksPerRow, cch = lane % kChunksPerRow;
#pragma unroll
        for (int s = 0; s < NS; s++) {
            if (m0 + 32 * s >= seg_end) break;  // uniform: no live row in this slice or after
#pragma unroll
            for (int r = 0; r < 16; r++)
                *reinterpret_cast<uint16_t *>(stage + (8 * (r >> 2) + 4 * h + (r & 3)) * kRow + 2 * l32) =
                    (uint16_t)(pack_bf16(affine_out<MODE>(acc[s], 0, r), 0.f) & 0xffffu);
            wave_lds_sync();
#pragma unroll
            for (int i = 0; i < 32 / kRowsPerPass; i++) {
                const int R = kRowsPerPass * i + crow;
                const u32x4 v = *reinterpret_cast<const u32x4 *>(stage + R * kRow + 16 * cch);
                const uint32_t pos = m0 + 32 * s + R, n = col0 + 8 * cch;
                if (pos < seg_end && n < out)
                    *reinterpret_cast<u32x4 *>(a.out + (uint64_t)pos * out + n) = v;
            }
            wave_lds_sync();  // the next slice reuses the area
        }
        return;
    }
#pragma unroll
    for (int s = 0; s < NS; s++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const uint32_t pos = m0 + 32 * s + 8 * (r >> 2) + 4 * h + (r & 3);
            if (pos >= seg_end) continue;
#pragma unroll
            for (int t = 0; t < (MODE == GATEUP ? 1 : kAfNT); t++) {
                const uint32_t n = col0 + 32 * t + l32;
                if (n < out) a.out[(uint64_t)pos * out + n] = (uint16_t)(pack_bf16(affine_out<MODE>(acc[s], t, r), 0.f) & 0xffffu);
            }
        }
    }
}

template <int MODE, int BITS, int T, int GS, bool PK>
__device__ __forceinline__ void affine_live(const Args &a, uint8_t *abuf, uint32_t nt, uint32_t e,
                                            uint32_t m0, uint32_t seg_end, uint32_t live, int lane,
                                            int wv) {
    if (live > 96) affine_item<MODE, BITS, T, 4, GS, PK>(a, abuf, nt, e, m0, seg_end, lane, wv);
    else if (live > 64) affine_item<MODE, BITS, T, 3, GS, PK>(a, abuf, nt, e, m0, seg_end, lane, wv);
    else if (live > 32) affine_item<MODE, BITS, T, 2, GS, PK>(a, abuf, nt, e, m0, seg_end, lane, wv);
    else affine_item<MODE, BITS, T, 1, GS, PK>(a, abuf, nt, e, m0, seg_end, lane, wv);
}

// Affine GATEUP / DOWN products: same persistent XCD-range schedule as
// grouped_gemm_kernel, kAfWaves waves per block, at most 256 VGPRs per lane so
// two waves share a SIMD.
// M-tile position p of the item order when sh shared-expert M-tiles are
// spread evenly over r + sh positions (shared tile j at position
// floor((2j + 1)(r + sh) / (2 sh)), so every XCD range holds its share;
// the routed tiles keep their order): returns the shared tile's index and
// sets `shared`, or the routed tile's index.
__device__ __forceinline__ uint32_t tile_at(uint32_t p, uint32_t r, uint32_t sh, bool &shared) {
    shared = false;
    if (sh == 0) return p;
    const uint64_t m = (uint64_t)r + sh;
    const int64_t num = 2 * (int64_t)sh * (p + 1) - (int64_t)m;  // shared positions <= p: ceil(num / 2m)
    const uint32_t c = num <= 0 ? 0u : (uint32_t)min((uint64_t)sh, ((uint64_t)num + 2 * m - 1) / (2 * m));
    if (c > 0 && (uint64_t)(2 * c - 1) * m / (2 * sh) == p) {
        shared = true;
        return c - 1;
    }
    return p - c;
}

// SH: the launch carries the shared expert's segment (a.sh_mt > 0).  Without
// it the item loop has no per-item choice between the two argument blocks.
template <int MODE, int BITS, int T, bool SH>
__global__ __attribute__((amdgpu_flat_work_group_size(kAfThreads, kAfThreads), amdgpu_waves_per_eu(2, 2)))
void affine_gemm_kernel(Args a, Args ash) {
    static_assert(MODE == GATEUP || MODE == DOWN, "affine_gemm_kernel: expert products only");
    static_assert(BITS == 2 || BITS == 4 || BITS == 8, "affine_gemm_kernel: affine weights only");
    __shared__ __attribute__((aligned(16))) uint8_t abuf[2 * kAfATile + kAfWaves * kEpiBytes];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t routed = *a.ntiles;
    const uint32_t items = (routed + (SH ? a.sh_mt : 0u)) * a.n_tiles_n;
    const uint32_t xcd = blockIdx.x % kXcds, q = blockIdx.x / kXcds, nq = gridDim.x / kXcds;
    const uint32_t per_xcd = (items + kXcds - 1) / kXcds;
    const uint32_t lo = xcd * per_xcd, hi = min(items, lo + per_xcd);
    for (uint32_t item = lo + q; item < hi; item += nq) {
        const uint32_t nt = item % a.n_tiles_n;
        bool sh = false;
        const uint32_t mt = SH ? tile_at(item / a.n_tiles_n, routed, a.sh_mt, sh) : item / a.n_tiles_n;
        // the shared expert's tiles: expert 0 of its own weights
        const Args &aa = SH && sh ? ash : a;
        const uint32_t e = sh ? 0u : a.tiles[2 * mt];
        const uint32_t m0 = sh ? a.sh_base + kTM * mt : a.tiles[2 * mt + 1];
        const uint32_t seg_end = sh ? a.sh_base + a.sh_rows : a.offsets[e + 1];
        const uint32_t live = min(seg_end - m0, (uint32_t)kTM);
        if constexpr (T == 0) {
            affine_live<MODE, BITS, T, 0, false>(aa, abuf, nt, e, m0, seg_end, live, lane, wv);
        } else if (aa.pk.data) {
            if (aa.w.gshift == 5) affine_live<MODE, BITS, T, 5, true>(aa, abuf, nt, e, m0, seg_end, live, lane, wv);
            else if (aa.w.gshift == 6) affine_live<MODE, BITS, T, 6, true>(aa, abuf, nt, e, m0, seg_end, live, lane, wv);
            else affine_live<MODE, BITS, T, 7, true>(aa, abuf, nt, e, m0, seg_end, live, lane, wv);
        } else {
            if (aa.w.gshift == 5) affine_live<MODE, BITS, T, 5, false>(aa, abuf, nt, e, m0, seg_end, live, lane, wv);
            else if (aa.w.gshift == 6) affine_live<MODE, BITS, T, 6, false>(aa, abuf, nt, e, m0, seg_end, live, lane, wv);
            else affine_live<MODE, BITS, T, 7, false>(aa, abuf, nt, e, m0, seg_end, live, lane, wv);
        }
    }
}


}  // namespace gemm

// Launches affine_gemm_kernel over the routed segments plus the shared
// expert's segment (a.sh_mt > 0; its weights in ash), for the weight kind of
// w (k_gemm_shared.hip).
hipError_t launch_affine_shared(Prof *p, hipStream_t s, int down, const WDesc &w, const gemm::Args &a,
                                const gemm::Args &ash, uint32_t blocks, const char *name);

}  // namespace moehip
