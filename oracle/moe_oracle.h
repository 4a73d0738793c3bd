/*
 * moe_oracle.h -- CPU oracle for the MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * CPU semantics for the mixture-of-experts path (posedonYT/llama-rs-metal).
 * Only the test suite, the smoke check and the CPU-baseline leg of the
 * benchmark may load it, and only as the checker / the timed CPU baseline.
 * The HIP product path never links or calls it.
 *
 * Every function names the reference file:line it restates.  Paths are
 * relative to the reference repository root.
 *
 * Pinning status (what fixes each function independently of this code):
 *   orc_f16_to_f32 / orc_bf16_to_f32  bit-pattern KATs from
 *       crates/metal-backend/tests/affine.rs:16-27 + exhaustive IEEE checks
 *   orc_weight_decode_rows   KAT crates/model-format/tests/mlx.rs:99 and the
 *       affine.rs:3-45 pattern checked against an independent numpy decode
 *   orc_matvec / orc_softmax / orc_silu / orc_rms_norm   float64 numpy closed
 *       forms (crates/tensor-core/src/lib.rs:64-88)
 *   orc_route   KAT affine.rs:96-112 (logits [1,4,3,2], K=2 -> ids [1,2]) and
 *       brute force over all tie patterns on tiny E (stable sort)
 *   orc_dispatch   invariants (bijection, segment lengths, stable order) and a
 *       numpy stable argsort
 *   orc_moe_block   composition of the above; checked against an independent
 *       float64 numpy restatement on the config-1 fixture
 *   orc_moe_block_em   equal to orc_moe_block bit for bit (dense, affine,
 *       shared expert, ties, bias, logits_in, several token chunks)
 *   orc_normal / orc_quantize_affine   this build's own synthetic-input tools
 *       (no reference counterpart); LCG constants follow
 *       crates/llama-rs/tests/common/mod.rs:86-97.
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* DType ids: crates/model-format/src/dtype.rs:5-15 */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 30 };

/* A weight tensor exactly as the reference binds it
 * (crates/model-format/src/checkpoint.rs:63-86):
 *   dims[0] = in (contiguous), dims[1] = out, dims[2] = experts (3-D only).
 *   bits == 0: dense elements of `dtype`.
 *   bits in {2,4,8}: packed little-endian u32 codes (low bits first),
 *   scales/biases of `scale_type`, one per `group_size` elements along in. */
typedef struct {
    const void *data;
    const void *scales;
    const void *biases;
    uint32_t dtype;
    uint32_t bits;
    uint32_t group_size;
    uint32_t scale_type;
    uint32_t ndims;
    uint32_t pad_;
    uint64_t dims[3];
} orc_weight;

/* Threads of the parallel loops (decode, matvec): 1 gives the scalar
 * single-thread baseline; results do not depend on it. */
void orc_set_threads(int n);
int orc_threads(void);

float orc_f16_to_f32(uint16_t h);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
uint16_t orc_f32_to_f16(float f);

/* Validation of Tensor::new (checkpoint.rs:88-130).  0 = ok. */
int orc_weight_validate(const orc_weight *w);
/* Tensor::decode (checkpoint.rs:164-196), restricted to rows
 * [row0, row0+nrows) of `dims[0]` elements each. */
int orc_weight_decode_rows(const orc_weight *w, uint64_t row0, uint64_t nrows, float *out);

/* tensor_core ops (crates/tensor-core/src/lib.rs) */
void orc_matvec(const float *w, const float *x, uint64_t rows, uint64_t in, float *y);
void orc_softmax(const float *x, uint64_t n, float *y);
float orc_silu(float x);
void orc_rms_norm(const float *x, const float *w, uint64_t n, float eps, float *y);

/* Routing (crates/metal-backend/src/shaders/sampling.metal:1-36) */
void orc_route(const float *logits, uint32_t n, uint32_t k, int normalize,
               uint32_t *ids, float *weights);

/* Element-wise epilogues (crates/metal-backend/src/shaders/elementwise.metal) */
void orc_swiglu(const float *a, const float *b, float *y, uint64_t n);
void orc_mix(const float *x, const float *w, uint32_t k, uint64_t n, float *y);
void orc_gate_scalar(const float *x, const float *g, float *y, uint64_t n);
void orc_add(const float *a, const float *b, float *y, uint64_t n);

/* Batch::matmul / Batch::expert_matmul semantics on the CPU
 * (crates/metal-backend/src/apple/ops/matrix.rs:63-205). */
int orc_matmul(const orc_weight *w, const float *x, float *y, uint64_t tokens);
int orc_expert_matmul(const orc_weight *w, const float *x, const uint32_t *ids,
                      uint32_t nids, float *y, int per_expert_input);

/* Token -> expert dispatch: stable counting sort of (token, k) pairs by
 * expert.  perm holds pair indices t*K+k ordered by (expert, t, k); pos is
 * its inverse.  No reference counterpart (the reference loops tokens). */
int orc_dispatch(const uint32_t *ids, uint32_t tokens, uint32_t k, uint32_t experts,
                 uint32_t *counts, uint32_t *offsets, uint32_t *perm, uint32_t *pos);

/* One MoE block (crates/model-runtime/src/execute.rs:208-233,251-267). */
typedef struct {
    orc_weight router;      /* [h, E] */
    orc_weight gate, up;    /* [h, ff, E] */
    orc_weight down;        /* [ff, h, E] */
    orc_weight sh_gate, sh_up; /* [h, ffs] */
    orc_weight sh_down;     /* [ffs, h] */
    orc_weight sh_gate_inp; /* [h] or [h, 1] */
    uint32_t has_shared;
    uint32_t k;
    uint32_t normalize;
    uint32_t pad_;
} orc_moe;

/* out[T,h].  logit_bias[T,E] may be NULL; it is added to the router logits
 * before routing (benchmark skew harness).  If `logits_in` is non-NULL the
 * router product is skipped and those logits (already biased) are routed
 * instead -- this is how GPU-produced logits are fed to the oracle so that
 * routing parity is judged on identical logits.  logits_out/ids_out/w_out
 * may be NULL. */
int orc_moe_block(const orc_moe *m, const float *x, uint32_t tokens, const float *logit_bias,
                  const float *logits_in, float *out, float *logits_out, uint32_t *ids_out,
                  float *w_out);

/* orc_moe_block evaluated expert by expert: every token routed first, the
 * pairs of each chunk of 4096 tokens sorted by expert, each expert decoded
 * once per chunk for all its pairs.  Same arguments and the same outputs bit
 * for bit (each product is the same sequential sum); used where the
 * per-token form is too slow (all tokens at prefill sizes). */
int orc_moe_block_em(const orc_moe *m, const float *x, uint32_t tokens, const float *logit_bias,
                     const float *logits_in, float *out, float *logits_out, uint32_t *ids_out,
                     float *w_out);

/* MoE-only stack step: hidden += moe(rms_norm(hidden, norm_w, eps)) per layer
 * (execute.rs:197,236; tensor-core/src/lib.rs:64-70). */
int orc_moe_stack(const orc_moe *layers, const float *const *norm_w, uint32_t nlayers,
                  float eps, float *hidden, uint32_t tokens);

/* Synthetic inputs: reference fixture LCG (crates/llama-rs/tests/common/mod.rs:86-97)
 * feeding Box-Muller in double. */
void orc_normal(uint64_t seed, uint64_t n, float mean, float std, float *out);
/* Affine quantizer (this build's own): per group min/max, scale=(max-min)/(2^b-1),
 * bias=min, both rounded to scale_type; code = clamp(rint((w-bias)/scale)). */
int orc_quantize_affine(const float *w, uint64_t n, uint32_t bits, uint32_t group,
                        uint32_t scale_type, uint32_t *packed, void *scales, void *biases);
/* Deterministic pattern of crates/metal-backend/tests/affine.rs:3-45. */
int orc_affine_pattern(uint64_t n, uint32_t bits, uint32_t group, uint32_t scale_type,
                       uint32_t *packed, void *scales, void *biases);

#ifdef __cplusplus
}
#endif
#endif
