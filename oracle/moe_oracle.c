/*
 * moe_oracle.c -- CPU oracle for the MoE layer.  TEST INFRASTRUCTURE ONLY:
 * only tests/, the smoke check and bench.py's cpu_baseline leg may load it,
 * as the checker or the timed CPU baseline.  Never part of the product path.
 *
 * Plain C restatement of the reference's CPU semantics
 * (posedonYT/llama-rs-metal); each function cites the file:line it follows.
 * Build: see oracle/Makefile (gcc, -ffp-contract=off so float sums are the
 * plain sequential mul-then-add the reference's Rust iterators perform).
 */
#include "moe_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* Loops over at least this many elements run on the OpenMP threads (the
 * all-core CPU baseline); smaller ones stay on one thread. */
#define ORC_PAR_MIN 65536

void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int orc_threads(void) { return omp_get_max_threads(); }

/* ---------------------------------------------------------------- dtypes -- */

/* IEEE binary16 -> binary32, exact (the `half` crate's to_f32,
 * crates/model-format/src/quantization.rs:4-6). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while (!(man & 0x400));
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* bf16 -> f32 is a 16-bit left shift (crates/metal-backend/src/shaders/affine.metal:9-10,
 * crates/model-format/src/quantization.rs:29-31). */
float orc_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* f32 -> bf16, round to nearest even; NaN stays a quiet NaN. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

/* f32 -> f16, round to nearest even, with overflow to inf and subnormals. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
    uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00;           /* NaN */
    if (a >= 0x477ff000u) return sign | 0x7c00;          /* rounds to >= 65520 -> inf */
    if (a < 0x33000001u) return sign;                    /* < 2^-25 (+tie) -> 0 */
    int e = (int)(a >> 23) - 127;
    uint32_t m = (a & 0x7fffffu) | 0x800000u;
    if (e < -14) { /* subnormal result */
        int shift = -14 - e + 13;
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return sign | (uint16_t)q;
    }
    uint32_t q = ((uint32_t)(e + 15) << 10) | ((m >> 13) & 0x3ff);
    uint32_t rem = m & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) q++;
    return sign | (uint16_t)q;
}

static float scalar_at(const void *p, uint64_t i, uint32_t type) {
    if (type == ORC_F32) return ((const float *)p)[i];
    if (type == ORC_BF16) return orc_bf16_to_f32(((const uint16_t *)p)[i]);
    return orc_f16_to_f32(((const uint16_t *)p)[i]);
}

static uint64_t elements(const orc_weight *w) {
    uint64_t n = 1;
    for (uint32_t d = 0; d < w->ndims; d++) n *= w->dims[d];
    return n;
}

/* Tensor::new affine/dense validation (crates/model-format/src/checkpoint.rs:88-130). */
int orc_weight_validate(const orc_weight *w) {
    if (w->ndims == 0 || w->ndims > 3) return -1;
    for (uint32_t d = 0; d < w->ndims; d++)
        if (w->dims[d] == 0) return -1;
    if (w->bits == 0)
        return (w->dtype == ORC_F32 || w->dtype == ORC_F16 || w->dtype == ORC_BF16) ? 0 : -1;
    if (w->bits != 2 && w->bits != 4 && w->bits != 8) return -2;
    if (w->group_size != 32 && w->group_size != 64 && w->group_size != 128) return -2;
    if (w->scale_type != ORC_F32 && w->scale_type != ORC_F16 && w->scale_type != ORC_BF16)
        return -3;
    if (w->dims[0] % w->group_size != 0) return -3;
    return 0;
}

/* Tensor::decode, affine branch (checkpoint.rs:164-196): element i reads
 * word i/(32/bits), shifts by (i % (32/bits))*bits, masks, and applies
 * code*scale[i/g] + bias[i/g].  Dense branch: dequantize() F32/F16/BF16
 * (quantization.rs:26-31). */
int orc_weight_decode_rows(const orc_weight *w, uint64_t row0, uint64_t nrows, float *out) {
    if (orc_weight_validate(w)) return -1;
    uint64_t in = w->dims[0];
    uint64_t n = elements(w);
    if ((row0 + nrows) * in > n) return -1;
    uint64_t i0 = row0 * in, i1 = (row0 + nrows) * in;
    /* elements are independent: threads split the range (same values as one
     * thread) */
    if (w->bits == 0) {
#pragma omp parallel for schedule(static) if (i1 - i0 >= ORC_PAR_MIN)
        for (uint64_t i = i0; i < i1; i++) out[i - i0] = scalar_at(w->data, i, w->dtype);
        return 0;
    }
    const uint32_t *words = (const uint32_t *)w->data;
    uint32_t per_word = 32 / w->bits;
    uint32_t mask = (1u << w->bits) - 1;
#pragma omp parallel for schedule(static) if (i1 - i0 >= ORC_PAR_MIN)
    for (uint64_t i = i0; i < i1; i++) {
        uint32_t value = words[i / per_word];
        uint32_t code = (value >> ((uint32_t)(i % per_word) * w->bits)) & mask;
        uint64_t g = i / w->group_size;
        out[i - i0] = (float)code * scalar_at(w->scales, g, w->scale_type) +
                      scalar_at(w->biases, g, w->scale_type);
    }
    return 0;
}

/* ----------------------------------------------------------- tensor-core -- */

/* tensor_core::matvec (crates/tensor-core/src/lib.rs:80-85): rows of `in`
 * elements, each a sequential f32 sum of products.  Rows are independent:
 * threads split them, and every row's sum keeps its sequential order, so the
 * result is the single-thread result bit for bit. */
void orc_matvec(const float *w, const float *x, uint64_t rows, uint64_t in, float *y) {
#pragma omp parallel for schedule(static) if (rows * in >= ORC_PAR_MIN)
    for (uint64_t r = 0; r < rows; r++) {
        const float *row = w + r * in;
        float s = 0.0f;
        for (uint64_t i = 0; i < in; i++) s += row[i] * x[i];
        y[r] = s;
    }
}

/* tensor_core::softmax (lib.rs:71-79). */
void orc_softmax(const float *x, uint64_t n, float *y) {
    float m = -INFINITY;
    for (uint64_t i = 0; i < n; i++) m = fmaxf(m, x[i]);
    float s = 0.0f;
    for (uint64_t i = 0; i < n; i++) {
        y[i] = expf(x[i] - m);
        s += y[i];
    }
    for (uint64_t i = 0; i < n; i++) y[i] /= s;
}

/* tensor_core::silu (lib.rs:86-88). */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* tensor_core::rms_norm (lib.rs:64-70): scale = 1/sqrt(mean(x^2)+eps), y = x*w*scale. */
void orc_rms_norm(const float *x, const float *w, uint64_t n, float eps, float *y) {
    float ss = 0.0f;
    for (uint64_t i = 0; i < n; i++) ss += x[i] * x[i];
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (uint64_t i = 0; i < n; i++) y[i] = x[i] * w[i] * scale;
}

/* --------------------------------------------------------------- routing -- */

/* route (crates/metal-backend/src/shaders/sampling.metal:1-36):
 *  mx = max over logits (NaN ignored, Metal max = fmax);
 *  den = sequential sum of exp(x_j - mx);
 *  K passes, each taking the unused j with the largest logit under a strict
 *  `>` scan over ascending j (ties -> lower index; -inf and NaN never win;
 *  an exhausted pool yields id 0 with score -inf);
 *  w_k = exp(score - mx)/den; optional renormalisation by the k-ordered sum. */
void orc_route(const float *x, uint32_t n, uint32_t k, int normalize, uint32_t *ids,
               float *weights) {
    float mx = -INFINITY;
    for (uint32_t j = 0; j < n; j++) mx = fmaxf(mx, x[j]);
    float den = 0.0f;
    for (uint32_t j = 0; j < n; j++) den += expf(x[j] - mx);
    float selected = 0.0f;
    for (uint32_t kk = 0; kk < k; kk++) {
        uint32_t best = 0;
        float score = -INFINITY;
        for (uint32_t j = 0; j < n; j++) {
            int used = 0;
            for (uint32_t s = 0; s < kk; s++)
                if (ids[s] == j) used = 1;
            if (!used && x[j] > score) {
                score = x[j];
                best = j;
            }
        }
        ids[kk] = best;
        weights[kk] = expf(score - mx) / den;
        selected += weights[kk];
    }
    if (normalize)
        for (uint32_t kk = 0; kk < k; kk++) weights[kk] /= selected;
}

/* ----------------------------------------------------------- elementwise -- */

/* activation (elementwise.metal:8-17): y = a/(1+exp(-a))*b. */
void orc_swiglu(const float *a, const float *b, float *y, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        float v = a[i];
        y[i] = v / (1.0f + expf(-v)) * b[i];
    }
}

/* mix (elementwise.metal:47-57): y[i] = sum_{k ascending} x[k*n+i]*w[k]. */
void orc_mix(const float *x, const float *w, uint32_t k, uint64_t n, float *y) {
    for (uint64_t i = 0; i < n; i++) {
        float v = 0.0f;
        for (uint32_t kk = 0; kk < k; kk++) v += x[(uint64_t)kk * n + i] * w[kk];
        y[i] = v;
    }
}

/* gate_scalar (elementwise.metal:65-72): y = x/(1+exp(-g[0])). */
void orc_gate_scalar(const float *x, const float *g, float *y, uint64_t n) {
    float d = 1.0f + expf(-g[0]);
    for (uint64_t i = 0; i < n; i++) y[i] = x[i] / d;
}

/* add (elementwise.metal:1-7). */
void orc_add(const float *a, const float *b, float *y, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) y[i] = a[i] + b[i];
}

/* ------------------------------------------------------------ products -- */

/* Batch::matmul (crates/metal-backend/src/apple/ops/matrix.rs:63-148):
 * dims [in, out]; y[t*out + r] = matvec(decode(W), x[t*in..]).  Same values as
 * the reference test's tensor_core::matvec(&tensor.decode(), x)
 * (crates/metal-backend/tests/affine.rs:70-74). */
static int em_rows(const float *w, uint64_t rows, uint64_t in, const float *xs, uint64_t ld,
                   const uint64_t *src, const uint64_t *dst, uint64_t np, float *y,
                   uint64_t ystride);

int orc_matmul(const orc_weight *w, const float *x, float *y, uint64_t tokens) {
    if (orc_weight_validate(w) || w->ndims != 2 || tokens == 0) return -1;
    uint64_t in = w->dims[0], out = w->dims[1];
    float *dec = (float *)malloc(sizeof(float) * in * out);
    uint64_t *idx = (uint64_t *)malloc(sizeof(uint64_t) * tokens);
    int rc = dec && idx ? 0 : -2;
    if (rc == 0) {
        orc_weight_decode_rows(w, 0, out, dec);
        /* every token's rows are orc_matvec's sums, several tokens at a time */
        for (uint64_t t = 0; t < tokens; t++) idx[t] = t;
        rc = em_rows(dec, out, in, x, in, idx, idx, tokens, y, out);
    }
    free(dec);
    free(idx);
    return rc;
}

/* Batch::expert_matmul (matrix.rs:149-205) with the kernel semantics of
 * affine_expert_* (affine.metal:83-94) and expert_mv (matrix.metal:39-64):
 * dims [in, out, E]; y[k*out + r] = matvec(expert ids[k]) applied to x (or to
 * x[k*in..] when per_expert_input); an id >= E yields zeros. */
int orc_expert_matmul(const orc_weight *w, const float *x, const uint32_t *ids, uint32_t nids,
                      float *y, int per_expert_input) {
    if (orc_weight_validate(w) || w->ndims != 3) return -1;
    uint64_t in = w->dims[0], out = w->dims[1], e_count = w->dims[2];
    if (e_count < nids) return -1; /* matrix.rs:164-166 */
    float *dec = (float *)malloc(sizeof(float) * in * out);
    if (!dec) return -2;
    for (uint32_t k = 0; k < nids; k++) {
        float *yk = y + (uint64_t)k * out;
        if (ids[k] >= e_count) {
            memset(yk, 0, sizeof(float) * out);
            continue;
        }
        orc_weight_decode_rows(w, (uint64_t)ids[k] * out, out, dec);
        orc_matvec(dec, per_expert_input ? x + (uint64_t)k * in : x, out, in, yk);
    }
    free(dec);
    return 0;
}

/* -------------------------------------------------------------- dispatch -- */

/* Stable counting sort of pairs p = t*K+k by expert id.  Ascending p within
 * an expert gives the (token, k) order.  No reference counterpart: the
 * reference runs experts per token (crates/model-runtime/src/execute.rs:208). */
int orc_dispatch(const uint32_t *ids, uint32_t tokens, uint32_t k, uint32_t experts,
                 uint32_t *counts, uint32_t *offsets, uint32_t *perm, uint32_t *pos) {
    uint64_t pairs = (uint64_t)tokens * k;
    for (uint32_t e = 0; e < experts; e++) counts[e] = 0;
    for (uint64_t p = 0; p < pairs; p++) {
        if (ids[p] >= experts) return -1;
        counts[ids[p]]++;
    }
    offsets[0] = 0;
    for (uint32_t e = 0; e < experts; e++) offsets[e + 1] = offsets[e] + counts[e];
    uint32_t *cursor = (uint32_t *)malloc(sizeof(uint32_t) * (experts ? experts : 1));
    if (!cursor) return -2;
    memcpy(cursor, offsets, sizeof(uint32_t) * experts);
    for (uint64_t p = 0; p < pairs; p++) {
        uint32_t at = cursor[ids[p]]++;
        perm[at] = (uint32_t)p;
        if (pos) pos[p] = at;
    }
    free(cursor);
    return 0;
}

/* ------------------------------------------------------------ MoE block -- */

static int dense_matvec(const orc_weight *w, const float *x, float *y, float *scratch) {
    /* one token through a 2-D weight, decode then matvec (matrix.rs:63) */
    uint64_t in = w->dims[0], out = w->ndims > 1 ? w->dims[1] : 1;
    if (orc_weight_decode_rows(w, 0, out, scratch)) return -1;
    orc_matvec(scratch, x, out, in, y);
    return 0;
}

/* MoE block per token, in the order of execute.rs:208-233:
 *   routes = router . norm                       (:220, matrix.rs:63)
 *   ids, weights = route(routes, K, normalize)    (:221)
 *   gates/ups = expert_matmul(gate/up, norm, ids) (:222-223)
 *   gates = swiglu(gates, ups)                    (:224)
 *   expert_out = expert_matmul(down, gates, ids, per_expert_input) (:225)
 *   projected = mix(expert_out, weights)          (:226)
 *   shared = encode_dense(shared, norm)           (:228, :251-267)
 *   sg = shared_gate . norm; shared /= 1+exp(-sg) (:230-231)
 *   projected += shared                           (:232) */
int orc_moe_block(const orc_moe *m, const float *x, uint32_t tokens, const float *logit_bias,
                  const float *logits_in, float *out, float *logits_out, uint32_t *ids_out,
                  float *w_out) {
    uint64_t h = m->gate.dims[0], ff = m->gate.dims[1], E = m->gate.dims[2];
    uint32_t K = m->k;
    if (m->router.dims[0] != h || m->router.dims[1] != E || K == 0 || K > E) return -1;
    if (m->up.dims[0] != h || m->up.dims[1] != ff || m->down.dims[0] != ff ||
        m->down.dims[1] != h)
        return -1;
    uint64_t ffs = m->has_shared ? m->sh_gate.dims[1] : 0;
    uint64_t scratch_n = h * E;
    if (h * ff > scratch_n) scratch_n = h * ff;
    if (m->has_shared && h * ffs > scratch_n) scratch_n = h * ffs;
    float *scratch = (float *)malloc(sizeof(float) * scratch_n);
    float *routes = (float *)malloc(sizeof(float) * E);
    uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * K);
    float *wts = (float *)malloc(sizeof(float) * K);
    float *gates = (float *)malloc(sizeof(float) * K * ff);
    float *ups = (float *)malloc(sizeof(float) * K * ff);
    float *eo = (float *)malloc(sizeof(float) * K * h);
    float *sg = (float *)malloc(sizeof(float) * (ffs ? ffs : 1));
    float *su = (float *)malloc(sizeof(float) * (ffs ? ffs : 1));
    float *so = (float *)malloc(sizeof(float) * h);
    int rc = 0;
    if (!scratch || !routes || !ids || !wts || !gates || !ups || !eo || !sg || !su || !so) {
        rc = -2;
        goto done;
    }
    for (uint32_t t = 0; t < tokens; t++) {
        const float *norm = x + (uint64_t)t * h;
        float *proj = out + (uint64_t)t * h;
        if (logits_in) {
            memcpy(routes, logits_in + (uint64_t)t * E, sizeof(float) * E);
        } else {
            if (dense_matvec(&m->router, norm, routes, scratch)) { rc = -1; goto done; }
            if (logit_bias)
                for (uint64_t e = 0; e < E; e++) routes[e] += logit_bias[(uint64_t)t * E + e];
        }
        if (logits_out) memcpy(logits_out + (uint64_t)t * E, routes, sizeof(float) * E);
        orc_route(routes, (uint32_t)E, K, (int)m->normalize, ids, wts);
        if (ids_out) memcpy(ids_out + (uint64_t)t * K, ids, sizeof(uint32_t) * K);
        if (w_out) memcpy(w_out + (uint64_t)t * K, wts, sizeof(float) * K);
        if (orc_expert_matmul(&m->gate, norm, ids, K, gates, 0) ||
            orc_expert_matmul(&m->up, norm, ids, K, ups, 0)) { rc = -1; goto done; }
        orc_swiglu(gates, ups, gates, K * ff);
        if (orc_expert_matmul(&m->down, gates, ids, K, eo, 1)) { rc = -1; goto done; }
        orc_mix(eo, wts, K, h, proj);
        if (m->has_shared) {
            if (dense_matvec(&m->sh_gate, norm, sg, scratch) ||
                dense_matvec(&m->sh_up, norm, su, scratch)) { rc = -1; goto done; }
            orc_swiglu(sg, su, sg, ffs);
            if (dense_matvec(&m->sh_down, sg, so, scratch)) { rc = -1; goto done; }
            float g;
            orc_weight gi = m->sh_gate_inp;
            gi.ndims = 2;
            gi.dims[1] = 1; /* [h] reshaped to [h, 1] (crates/model-runtime/src/loader.rs:194) */
            if (dense_matvec(&gi, norm, &g, scratch)) { rc = -1; goto done; }
            orc_gate_scalar(so, &g, so, h);
            orc_add(proj, so, proj, h);
        }
    }
done:
    free(scratch); free(routes); free(ids); free(wts); free(gates); free(ups); free(eo);
    free(sg); free(su); free(so);
    return rc;
}

/* ------------------------------------------------- expert-major block -- */

/* Eight input rows advance together through one weight row: lane l of the
 * vector is input l's running sum.  Each lane is its own sequential
 * mul-then-add sum from 0 in ascending i -- the sum orc_matvec forms for
 * that input alone -- so the values are the same bit for bit (vector
 * arithmetic is element-wise IEEE; -ffp-contract=off forbids fusing). */
#define EM_LANES 8
typedef float em_vec __attribute__((vector_size(4 * EM_LANES)));

__attribute__((target_clones("avx2", "default"), noinline)) static void em_kernel(
    const float *w, uint64_t r0, uint64_t r1, uint64_t in, const em_vec *xt, uint64_t nj,
    const uint64_t *dst, float *y, uint64_t ystride) {
    uint64_t r = r0;
    /* four rows at a time: four independent sums per lane share the loads */
    for (; r + 4 <= r1; r += 4) {
        const float *w0 = w + r * in, *w1 = w0 + in, *w2 = w1 + in, *w3 = w2 + in;
        em_vec a0 = {0}, a1 = {0}, a2 = {0}, a3 = {0};
        for (uint64_t i = 0; i < in; i++) {
            const em_vec v = xt[i];
            a0 += w0[i] * v;
            a1 += w1[i] * v;
            a2 += w2[i] * v;
            a3 += w3[i] * v;
        }
        for (uint64_t l = 0; l < nj; l++) {
            float *yl = y + dst[l] * ystride + r;
            yl[0] = a0[l];
            yl[1] = a1[l];
            yl[2] = a2[l];
            yl[3] = a3[l];
        }
    }
    for (; r < r1; r++) {
        const float *wr = w + r * in;
        em_vec acc = {0};
        for (uint64_t i = 0; i < in; i++) acc += wr[i] * xt[i];
        for (uint64_t l = 0; l < nj; l++) y[dst[l] * ystride + r] = acc[l];
    }
}

/* y[dst[j]*ystride + r] = sum_i w[r*in+i] * xs[src[j]*ld + i] for rows r of
 * the decoded weight w (rows x in, row-major) and inputs j < np: one
 * orc_matvec per input, evaluated eight inputs at a time (same values). */
static int em_rows(const float *w, uint64_t rows, uint64_t in, const float *xs, uint64_t ld,
                   const uint64_t *src, const uint64_t *dst, uint64_t np, float *y,
                   uint64_t ystride) {
    const uint64_t nb = (np + EM_LANES - 1) / EM_LANES, rc = 32, nr = (rows + rc - 1) / rc;
    int bad = 0;
#pragma omp parallel if (rows * in * np >= ORC_PAR_MIN)
    {
        em_vec *xt = (em_vec *)aligned_alloc(sizeof(em_vec), sizeof(em_vec) * (in ? in : 1));
        if (!xt) {
#pragma omp atomic write
            bad = 1;
        }
#pragma omp for schedule(dynamic, 1)
        for (uint64_t task = 0; task < nb * nr; task++) {
            if (!xt) continue;
            const uint64_t b = task / nr, r0 = (task % nr) * rc;
            const uint64_t r1 = r0 + rc < rows ? r0 + rc : rows;
            const uint64_t j0 = b * EM_LANES, nj = np - j0 < EM_LANES ? np - j0 : EM_LANES;
            for (uint64_t i = 0; i < in; i++)
                for (uint64_t l = 0; l < EM_LANES; l++)
                    xt[i][l] = l < nj ? xs[src[j0 + l] * ld + i] : 0.0f;
            em_kernel(w, r0, r1, in, xt, nj, dst + j0, y, ystride);
        }
        free(xt);
    }
    return bad ? -2 : 0;
}

/* orc_moe_block evaluated expert by expert (same outputs bit for bit; test
 * infrastructure for all-token parity at prefill sizes).  Every token is
 * routed first (router decoded once, each token's logits the same
 * sequential sums, plus the bias, then orc_route); the (token, k) pairs of a
 * chunk of tokens are sorted by expert (orc_dispatch); each expert's
 * gate/up/down are decoded once per chunk and applied to all its pairs,
 * each (pair, row) product the sum orc_matvec forms; each token then mixes
 * its K rows in k order and adds the gated shared expert exactly as
 * orc_moe_block does (execute.rs:208-233,251-267). */
int orc_moe_block_em(const orc_moe *m, const float *x, uint32_t tokens, const float *logit_bias,
                     const float *logits_in, float *out, float *logits_out, uint32_t *ids_out,
                     float *w_out) {
    const uint64_t h = m->gate.dims[0], ff = m->gate.dims[1], E = m->gate.dims[2];
    const uint32_t K = m->k;
    if (m->router.dims[0] != h || m->router.dims[1] != E || K == 0 || K > E) return -1;
    if (m->up.dims[0] != h || m->up.dims[1] != ff || m->down.dims[0] != ff ||
        m->down.dims[1] != h)
        return -1;
    if (orc_weight_validate(&m->router) || orc_weight_validate(&m->gate) ||
        orc_weight_validate(&m->up) || orc_weight_validate(&m->down))
        return -1;
    const uint64_t ffs = m->has_shared ? m->sh_gate.dims[1] : 0;
    const uint32_t CH = 4096;  /* tokens per chunk (bounds the per-pair buffers) */
    const uint64_t ct = tokens < CH ? tokens : CH;
    uint64_t wmax = h * E;
    if (h * ff > wmax) wmax = h * ff;
    if (h * ffs > wmax) wmax = h * ffs;
    float *routes = (float *)malloc(sizeof(float) * ((uint64_t)tokens * E + 1));
    uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * ((uint64_t)tokens * K + 1));
    float *wts = (float *)malloc(sizeof(float) * ((uint64_t)tokens * K + 1));
    float *wg = (float *)malloc(sizeof(float) * wmax);
    float *wu = (float *)malloc(sizeof(float) * wmax);
    float *wd = (float *)malloc(sizeof(float) * wmax);
    float *gi = (float *)malloc(sizeof(float) * (h + 1));
    float *g = (float *)malloc(sizeof(float) * (ct * K * (ff > ffs ? ff : ffs) + 1));
    float *u = (float *)malloc(sizeof(float) * (ct * K * (ff > ffs ? ff : ffs) + 1));
    float *eo = (float *)malloc(sizeof(float) * (ct * K * h + 1));
    float *sg = (float *)malloc(sizeof(float) * (ct + 1));
    uint64_t *src = (uint64_t *)malloc(sizeof(uint64_t) * (ct * K + tokens + 1));
    uint64_t *dst = (uint64_t *)malloc(sizeof(uint64_t) * (ct * K + tokens + 1));
    uint32_t *counts = (uint32_t *)malloc(sizeof(uint32_t) * (E + 1));
    uint32_t *offsets = (uint32_t *)malloc(sizeof(uint32_t) * (E + 2));
    uint32_t *perm = (uint32_t *)malloc(sizeof(uint32_t) * (ct * K + 1));
    int rc = 0;
    if (!routes || !ids || !wts || !wg || !wu || !wd || !gi || !g || !u || !eo || !sg || !src ||
        !dst || !counts || !offsets || !perm) {
        rc = -2;
        goto done;
    }
    /* router (execute.rs:220) and routing (:221) of every token */
    if (logits_in) {
        memcpy(routes, logits_in, sizeof(float) * (uint64_t)tokens * E);
    } else {
        if (orc_weight_decode_rows(&m->router, 0, E, wg)) { rc = -1; goto done; }
        for (uint64_t t = 0; t < tokens; t++) src[t] = dst[t] = t;
        if ((rc = em_rows(wg, E, h, x, h, src, dst, tokens, routes, E))) goto done;
        if (logit_bias)
            for (uint64_t i = 0; i < (uint64_t)tokens * E; i++) routes[i] += logit_bias[i];
    }
    if (logits_out) memcpy(logits_out, routes, sizeof(float) * (uint64_t)tokens * E);
    for (uint64_t t = 0; t < tokens; t++)
        orc_route(routes + t * E, (uint32_t)E, K, (int)m->normalize, ids + t * K, wts + t * K);
    if (ids_out) memcpy(ids_out, ids, sizeof(uint32_t) * (uint64_t)tokens * K);
    if (w_out) memcpy(w_out, wts, sizeof(float) * (uint64_t)tokens * K);
    for (uint64_t t0 = 0; t0 < tokens; t0 += CH) {
        const uint64_t nt = tokens - t0 < CH ? tokens - t0 : CH;
        if ((rc = orc_dispatch(ids + t0 * K, (uint32_t)nt, K, (uint32_t)E, counts, offsets, perm,
                               NULL)))
            goto done;
        for (uint64_t e = 0; e < E; e++) {
            const uint64_t n = counts[e], o = offsets[e];
            if (!n) continue;
            /* expert_matmul gate/up (:222-223): pair j of the segment reads its
             * token's row; swiglu (:224); down on the pair's own row (:225) into
             * the token's k-th slot of eo */
            if (orc_weight_decode_rows(&m->gate, e * ff, ff, wg) ||
                orc_weight_decode_rows(&m->up, e * ff, ff, wu) ||
                orc_weight_decode_rows(&m->down, e * h, h, wd)) { rc = -1; goto done; }
            for (uint64_t j = 0; j < n; j++) {
                src[j] = t0 + perm[o + j] / K;
                dst[j] = j;
            }
            if ((rc = em_rows(wg, ff, h, x, h, src, dst, n, g, ff)) ||
                (rc = em_rows(wu, ff, h, x, h, src, dst, n, u, ff)))
                goto done;
            orc_swiglu(g, u, g, n * ff);
            for (uint64_t j = 0; j < n; j++) {
                src[j] = j;
                dst[j] = perm[o + j];
            }
            if ((rc = em_rows(wd, h, ff, g, ff, src, dst, n, eo, h))) goto done;
        }
        /* mix (:226) */
        for (uint64_t t = 0; t < nt; t++)
            orc_mix(eo + t * K * h, wts + (t0 + t) * K, K, h, out + (t0 + t) * h);
        if (!m->has_shared) continue;
        /* shared expert (:228, :251-267), its sigmoid gate (:230-231), add (:232) */
        if (orc_weight_decode_rows(&m->sh_gate, 0, ffs, wg) ||
            orc_weight_decode_rows(&m->sh_up, 0, ffs, wu) ||
            orc_weight_decode_rows(&m->sh_down, 0, h, wd) ||
            orc_weight_decode_rows(&m->sh_gate_inp, 0, 1, gi)) { rc = -1; goto done; }
        for (uint64_t t = 0; t < nt; t++) {
            src[t] = t0 + t;
            dst[t] = t;
        }
        if ((rc = em_rows(wg, ffs, h, x, h, src, dst, nt, g, ffs)) ||
            (rc = em_rows(wu, ffs, h, x, h, src, dst, nt, u, ffs)) ||
            (rc = em_rows(gi, 1, h, x, h, src, dst, nt, sg, 1)))
            goto done;
        orc_swiglu(g, u, g, nt * ffs);
        for (uint64_t t = 0; t < nt; t++) src[t] = t;
        if ((rc = em_rows(wd, h, ffs, g, ffs, src, dst, nt, eo, h))) goto done;
        for (uint64_t t = 0; t < nt; t++) {
            float *so = eo + t * h, *proj = out + (t0 + t) * h;
            orc_gate_scalar(so, sg + t, so, h);
            orc_add(proj, so, proj, h);
        }
    }
done:
    free(routes); free(ids); free(wts); free(wg); free(wu); free(wd); free(gi); free(g);
    free(u); free(eo); free(sg); free(src); free(dst); free(counts); free(offsets); free(perm);
    return rc;
}

/* RMSNorm -> MoE -> residual per layer (execute.rs:197,236).  The block is
 * the expert-major evaluation (the same values as orc_moe_block). */
int orc_moe_stack(const orc_moe *layers, const float *const *norm_w, uint32_t nlayers,
                  float eps, float *hidden, uint32_t tokens) {
    uint64_t h = layers[0].gate.dims[0];
    float *norm = (float *)malloc(sizeof(float) * h * tokens);
    float *proj = (float *)malloc(sizeof(float) * h * tokens);
    int rc = (norm && proj) ? 0 : -2;
    for (uint32_t l = 0; l < nlayers && rc == 0; l++) {
        for (uint32_t t = 0; t < tokens; t++)
            orc_rms_norm(hidden + t * h, norm_w[l], h, eps, norm + t * h);
        rc = orc_moe_block_em(&layers[l], norm, tokens, NULL, NULL, proj, NULL, NULL, NULL);
        if (rc == 0) orc_add(hidden, proj, hidden, h * tokens);
    }
    free(norm);
    free(proj);
    return rc;
}

/* ------------------------------------------------------- synthetic data -- */

/* LCG of crates/llama-rs/tests/common/mod.rs:86-97 (s = s*6364136223846793005+1),
 * uniform u = ((s>>32)+0.5)/2^32 in (0,1), Box-Muller pairs in double. */
void orc_normal(uint64_t seed, uint64_t n, float mean, float std, float *out) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (uint64_t i = 0; i < n; i += 2) {
        s = s * 6364136223846793005ULL + 1ULL;
        double u1 = ((double)(s >> 32) + 0.5) / 4294967296.0;
        s = s * 6364136223846793005ULL + 1ULL;
        double u2 = ((double)(s >> 32) + 0.5) / 4294967296.0;
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + std * (r * cos(two_pi * u2)));
        if (i + 1 < n) out[i + 1] = (float)(mean + std * (r * sin(two_pi * u2)));
    }
}

static float round_to(float v, uint32_t type, uint16_t *bits16) {
    if (type == ORC_BF16) {
        *bits16 = orc_f32_to_bf16(v);
        return orc_bf16_to_f32(*bits16);
    }
    if (type == ORC_F16) {
        *bits16 = orc_f32_to_f16(v);
        return orc_f16_to_f32(*bits16);
    }
    return v;
}

int orc_quantize_affine(const float *w, uint64_t n, uint32_t bits, uint32_t group,
                        uint32_t scale_type, uint32_t *packed, void *scales, void *biases) {
    if ((bits != 2 && bits != 4 && bits != 8) || group == 0 || n % group || n % (32 / bits))
        return -1;
    uint32_t per_word = 32 / bits, qmax = (1u << bits) - 1;
    memset(packed, 0, sizeof(uint32_t) * (n / per_word));
    for (uint64_t g = 0; g < n / group; g++) {
        const float *v = w + g * group;
        float mn = v[0], mx = v[0];
        for (uint32_t i = 1; i < group; i++) {
            mn = fminf(mn, v[i]);
            mx = fmaxf(mx, v[i]);
        }
        uint16_t sb = 0, bb = 0;
        float s = round_to((mx - mn) / (float)qmax, scale_type, &sb);
        float b = round_to(mn, scale_type, &bb);
        if (scale_type == ORC_F32) {
            ((float *)scales)[g] = s;
            ((float *)biases)[g] = b;
        } else {
            ((uint16_t *)scales)[g] = sb;
            ((uint16_t *)biases)[g] = bb;
        }
        for (uint32_t i = 0; i < group; i++) {
            float q = s > 0.0f ? nearbyintf((v[i] - b) / s) : 0.0f;
            if (q < 0.0f) q = 0.0f;
            if (q > (float)qmax) q = (float)qmax;
            uint64_t idx = g * group + i;
            packed[idx / per_word] |= ((uint32_t)q & qmax) << ((idx % per_word) * bits);
        }
    }
    return 0;
}

/* Pattern of crates/metal-backend/tests/affine.rs:3-45: code(i) = (i*37 + i/13) & mask;
 * group scales/biases alternate 0.125/-0.5 (even) and 0.25/-0.25 (odd), stored
 * with the same F16/BF16 bit patterns the reference test writes. */
int orc_affine_pattern(uint64_t n, uint32_t bits, uint32_t group, uint32_t scale_type,
                       uint32_t *packed, void *scales, void *biases) {
    if ((bits != 2 && bits != 4 && bits != 8) || n % group) return -1;
    uint32_t per_word = 32 / bits, mask = (1u << bits) - 1;
    memset(packed, 0, sizeof(uint32_t) * (n / per_word));
    for (uint64_t i = 0; i < n; i++)
        packed[i / per_word] |= ((uint32_t)(i * 37 + i / 13) & mask) << ((i % per_word) * bits);
    for (uint64_t g = 0; g < n / group; g++) {
        int alt = (g % 2) == 1;
        if (scale_type == ORC_F32) {
            ((float *)scales)[g] = alt ? 0.25f : 0.125f;
            ((float *)biases)[g] = alt ? -0.25f : -0.5f;
        } else if (scale_type == ORC_F16) {
            ((uint16_t *)scales)[g] = alt ? 0x3400 : 0x3000;
            ((uint16_t *)biases)[g] = alt ? 0xb400 : 0xb800;
        } else {
            ((uint16_t *)scales)[g] = alt ? 0x3e80 : 0x3e00;
            ((uint16_t *)biases)[g] = alt ? 0xbe80 : 0xbf00;
        }
    }
    return 0;
}
