/*
 * moe_hip.h -- C ABI of the MI355X (gfx950) mixture-of-experts backend.
 *
 * This is the drop-in boundary a `hip-backend` crate binds in place of the
 * reference's `metal-backend` for the MoE path of posedonYT/llama-rs-metal.
 * Each declaration names the reference interface it replaces (paths relative
 * to the reference repository root).  Plain pointers and sizes only.
 *
 * Conventions (all mirror metal-backend):
 *  - Every call returns a moe_status; the codes map 1:1 onto
 *    metal_backend::Error (crates/metal-backend/src/lib.rs:5-14).
 *  - A moe_buffer is a view of 4-byte elements (F32 values, or u32 expert ids
 *    stored bitwise as the reference's scratch slots do,
 *    crates/model-runtime/src/workspace.rs:43-50) inside device memory owned
 *    by the moe_gpu that allocated or registered it
 *    (crates/metal-backend/src/apple.rs:38-64, apple/memory.rs:3-8).
 *  - Ops are stream ordered: each op sees every earlier op's writes, as the
 *    reference's per-dispatch buffer barrier guarantees
 *    (crates/metal-backend/src/apple/commands.rs:185).  Shapes, ownership
 *    and aliasing are checked before anything is enqueued
 *    (commands.rs:109-150); a failed check enqueues nothing.
 *  - Ops may only be issued between moe_batch_begin and moe_batch_finish
 *    (the Batch borrow, crates/metal-backend/src/apple/commands.rs:81-99).
 *  - One moe_gpu is used by one host thread at a time (the reference's Rc
 *    handles are !Send, crates/metal-backend/src/apple.rs:214-222).
 *  - The library never frees memory it did not allocate.
 */
#ifndef MOE_HIP_H
#define MOE_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* metal_backend::Error (crates/metal-backend/src/lib.rs:5-14). */
typedef enum {
    MOE_OK = 0,
    MOE_ERR_UNAVAILABLE = 1, /* Error::Unavailable: no usable gfx950 device      */
    MOE_ERR_GPU = 2,         /* Error::Gpu: a HIP call or kernel launch failed   */
    MOE_ERR_SHAPE = 3,       /* Error::Shape: invalid shape, ownership or alias  */
    MOE_ERR_ALLOCATION = 4   /* Error::Allocation: device allocation failed      */
} moe_status;

/* DType ids (crates/model-format/src/dtype.rs:5-15). */
enum { MOE_F32 = 0, MOE_F16 = 1, MOE_BF16 = 30 };

/* Gpu (crates/metal-backend/src/apple.rs:125-164): one device, one stream,
 * and the registry of allocations it owns. */
typedef struct moe_gpu moe_gpu;

/* Buffer (apple.rs:38-64): `ptr` is the device address of element 0,
 * `len` the number of 4-byte elements. */
typedef struct {
    void *ptr;
    uint64_t len;
} moe_buffer;

/* A byte region of device memory (weights.rs:142-204 uploads tensor bytes
 * region by region). */
typedef struct {
    const void *ptr;
    uint64_t bytes;
} moe_region;

/* Weight + AffineWeight (apple.rs:65-115; model_format::Tensor
 * crates/model-format/src/checkpoint.rs:63-86).
 *   dims[0] = in (contiguous), dims[1] = out, dims[2] = experts.
 *   bits == 0: dense `dtype` elements in `data`.
 *   bits in {2,4,8}: `data` holds packed little-endian u32 codes (low bits
 *   first), `scales`/`biases` one `scale_type` value per `group_size`
 *   elements along `in`; w = code*scale + bias. */
typedef struct {
    moe_region data;
    moe_region scales;
    moe_region biases;
    uint32_t dtype;
    uint32_t bits;
    uint32_t group_size;
    uint32_t scale_type;
    uint32_t ndims;
    uint32_t reserved;
    uint64_t dims[3];
} moe_weight;

/* ------------------------------------------------------------ device -- */

/* Gpu::new (apple.rs:165-211).  Fails with MOE_ERR_UNAVAILABLE when no
 * gfx950 device is visible. */
moe_status moe_gpu_create(int device, moe_gpu **out);
void moe_gpu_destroy(moe_gpu *gpu);
/* Gpu::name (apple.rs:131). */
moe_status moe_gpu_name(const moe_gpu *gpu, char *buf, size_t cap);
/* Gpu::allocated_bytes (apple/memory.rs:73-75). */
uint64_t moe_allocated_bytes(const moe_gpu *gpu);
/* Human-readable text of the last error on this gpu (the String payload of
 * metal_backend::Error). */
const char *moe_last_error(const moe_gpu *gpu);
/* The byte count of Error::Allocation(usize) (crates/metal-backend/src/lib.rs:12-13):
 * the requested size when the last error on this gpu was MOE_ERR_ALLOCATION
 * (UINT64_MAX when the element count overflowed, as the reference's
 * checked_mul failure reports usize::MAX, apple/memory.rs:26), else 0. */
uint64_t moe_last_error_bytes(const moe_gpu *gpu);

/* ------------------------------------------------------------ memory -- */

/* Gpu::zeros (apple/memory.rs:25-27): n zeroed 4-byte elements. */
moe_status moe_zeros(moe_gpu *gpu, uint64_t n, moe_buffer *out);
/* Gpu::upload (memory.rs:28-43). */
moe_status moe_upload(moe_gpu *gpu, const float *data, uint64_t n, moe_buffer *out);
/* Gpu::upload_region (apple/weights.rs:142-204): raw bytes (weights). */
moe_status moe_upload_bytes(moe_gpu *gpu, const void *data, uint64_t bytes, moe_region *out);
/* Gpu::read (memory.rs:44-60); waits for all enqueued work first. */
moe_status moe_read(moe_gpu *gpu, moe_buffer b, float *out);
/* Copy host bytes into an owned buffer (stream ordered, then waits). */
moe_status moe_write(moe_gpu *gpu, moe_buffer b, const float *data);
/* Gpu::clear (memory.rs:61-72). */
moe_status moe_clear(moe_gpu *gpu, moe_buffer b);
/* Drop of the last Storage handle (apple.rs:31-37): frees an allocation
 * made by moe_zeros/moe_upload/moe_upload_bytes, by its base pointer. */
moe_status moe_release(moe_gpu *gpu, const void *base);
/* Adopt caller-owned device memory into this gpu's ownership registry so it
 * passes the ownership check (the no-copy wrap of mapped checkpoint bytes,
 * apple/weights.rs:142-204, is the reference's nearest analogue).  The
 * library never frees it; moe_unregister forgets it. */
moe_status moe_register(moe_gpu *gpu, void *base, uint64_t bytes);
moe_status moe_unregister(moe_gpu *gpu, const void *base);
/* Buffer::view (apple.rs:51-63): element offset and length. */
moe_status moe_view(moe_buffer b, uint64_t start, uint64_t len, moe_buffer *out);

/* ------------------------------------------------------------- batch -- */

/* Gpu::batch (apple/commands.rs:81-99): opens the op sequence. */
moe_status moe_batch_begin(moe_gpu *gpu);
/* Batch::finish (commands.rs:215-224): waits for completion and returns the
 * GPU seconds between the batch's first and last op (hipEvent timing). */
moe_status moe_batch_finish(moe_gpu *gpu, double *gpu_seconds);

/* --------------------------------------------- Batch ops (MoE surface) -- */

/* Batch::matmul (crates/metal-backend/src/apple/ops/matrix.rs:63-148):
 * y[t*out + r] = sum_i W[r, i] * x[t*in + i], W dims [in, out]. */
moe_status moe_matmul(moe_gpu *gpu, const moe_weight *w, moe_buffer x, moe_buffer y,
                      uint64_t tokens);
/* Batch::expert_matmul (matrix.rs:149-205): W dims [in, out, E];
 * y[k*out + r] = expert ids[k] row r . (per_expert_input ? x[k*in..] : x);
 * an id >= E produces zeros (affine.metal:90-91, matrix.metal:56-60). */
moe_status moe_expert_matmul(moe_gpu *gpu, const moe_weight *w, moe_buffer x, moe_buffer ids,
                             moe_buffer y, int per_expert_input);
/* Batch::route (crates/metal-backend/src/apple/ops/sampling.rs:21-44):
 * exact top-k of one logits row; ids bit-exact with ties to the lower index. */
moe_status moe_route(moe_gpu *gpu, moe_buffer logits, moe_buffer ids, moe_buffer weights,
                     int normalize);
/* Batch::swiglu (apple/ops/elementwise.rs:25-27): y = a/(1+exp(-a))*b. */
moe_status moe_swiglu(moe_gpu *gpu, moe_buffer a, moe_buffer b, moe_buffer y);
/* Batch::mix (elementwise.rs:92-105): y[i] = sum_k x[k*n+i]*w[k]. */
moe_status moe_mix(moe_gpu *gpu, moe_buffer x, moe_buffer w, moe_buffer y);
/* Batch::gate_scalar (elementwise.rs:79-91): y = x/(1+exp(-g[0])). */
moe_status moe_gate_scalar(moe_gpu *gpu, moe_buffer x, moe_buffer g, moe_buffer y);
/* Batch::add (elementwise.rs:22-24). */
moe_status moe_add(moe_gpu *gpu, moe_buffer a, moe_buffer b, moe_buffer y);
/* Batch::norm (crates/metal-backend/src/apple/ops/attention.rs:3-45): RMSNorm
 * of `heads` rows of w.dims[0] elements spaced `stride` apart. */
moe_status moe_norm(moe_gpu *gpu, moe_buffer x, const moe_weight *w, moe_buffer y,
                    uint64_t heads, uint64_t stride, float eps);

/* ---------------------------------------- token-batched MoE additions -- */

/* route for each of `tokens` rows of logits[T, E] -> ids[T, K], weights[T, K]
 * (same per-row semantics as moe_route; the reference calls route once per
 * token, crates/model-runtime/src/execute.rs:208-221). */
moe_status moe_route_tokens(moe_gpu *gpu, moe_buffer logits, moe_buffer ids, moe_buffer weights,
                            uint64_t tokens, int normalize);
/* Token -> expert dispatch (no reference counterpart; it replaces the
 * per-token loop of execute.rs:208): counts[E], offsets[E+1] (exclusive scan),
 * perm[T*K] = pair indices t*K+k ordered by (expert, t, k), pos = inverse of
 * perm.  Deterministic, bit-exact. */
moe_status moe_dispatch(moe_gpu *gpu, moe_buffer ids, uint64_t tokens, uint64_t k,
                        uint64_t experts, moe_buffer counts, moe_buffer offsets, moe_buffer perm,
                        moe_buffer pos);

/* A copy of an affine expert weight in MFMA tile order (no reference
 * counterpart: the Metal kernels read the row-major tensor).  The bf16 MFMA
 * prefill path wants one weight row per lane pair, so from the row-major
 * tensor each of its code loads reads 32 bytes of 32 rows; from this copy it
 * reads one contiguous 256*bits-byte block, and each scale load one block of
 * the tile's groups.  Layout, for expert e, 32-row tile t (rows past dims[1]
 * zero) and K step kb of 64 values: data block (e, t, kb) of 256*bits bytes,
 * lane l = 32h + r holding row r's codes 32h .. 32h+31 at byte 4*bits*l;
 * scales (and biases) block (e, t, p) for the pair of steps p: 32 rows x
 * (128/group_size) values, row-major.  All-null regions: no copy. */
typedef struct {
    moe_region data;
    moe_region scales;
    moe_region biases;
} moe_packed_weight;

/* FeedForward::Moe (crates/model-runtime/src/lib.rs:46-56) as bound by the
 * loader (crates/model-runtime/src/loader.rs:172-203).  has_shared = 0 admits
 * layers without a shared expert (Qwen3-30B-A3B style). */
typedef struct {
    moe_weight router;          /* [h, E] */
    moe_weight gate;            /* [h, ff, E] */
    moe_weight up;              /* [h, ff, E] */
    moe_weight down;            /* [ff, h, E] */
    moe_weight shared_gate;     /* [h, ffs] */
    moe_weight shared_up;       /* [h, ffs] */
    moe_weight shared_down;     /* [ffs, h] */
    moe_weight shared_gate_inp; /* [h] (reshaped [h, 1], loader.rs:194) */
    uint32_t has_shared;
    uint32_t experts_used;      /* K, ModelConfig::experts_used (model-format/src/config.rs:42) */
    uint32_t normalize;         /* ModelConfig::normalize_expert_weights (config.rs:47) */
    uint32_t reserved;
    /* optional MFMA tile-order copies of gate/up/down (moe_pack_weight); the
     * bf16 MFMA path reads them when present (gate and up together) */
    moe_packed_weight gate_packed;
    moe_packed_weight up_packed;
    moe_packed_weight down_packed;
    /* the same for the shared expert's gate/up/down: the bf16 MFMA path runs
     * the shared expert as one more segment of the routed experts' GEMMs when
     * its weights are of the routed experts' kind and width */
    moe_packed_weight shared_gate_packed;
    moe_packed_weight shared_up_packed;
    moe_packed_weight shared_down_packed;
} moe_block_weights;

/* Byte sizes of the packed copy of w (the codes; the scales and the biases
 * each).  No reference counterpart.  MOE_ERR_SHAPE when w has no packed form:
 * it must be affine with F16/BF16 scales, dims[0] a multiple of 128, and
 * every byte offset of the copy below 2^32. */
moe_status moe_pack_size(const moe_weight *w, uint64_t *data_bytes, uint64_t *sb_bytes);
/* Batch op: writes the packed copy of w into `out`, whose regions must be
 * owned by this gpu, not overlap w, and have the sizes above.  No reference
 * counterpart (weight preparation for the prefill path). */
moe_status moe_pack_weight(moe_gpu *gpu, const moe_weight *w, moe_packed_weight out);

/* Path selection for moe_block. */
enum {
    MOE_PATH_AUTO = 0,   /* fused decode for one token; bf16 MFMA when the mean expert
                            segment holds >= 16 pairs; otherwise the batched decode
                            (weight rows streamed once per run of 8 inputs) where the
                            shapes allow it, else VALU grouped */
    MOE_PATH_OPS = 1,     /* the reference's per-token op sequence (execute.rs:208-233) */
    MOE_PATH_GROUPED = 2, /* dispatch + grouped expert products on VALU (F32) */
    MOE_PATH_MFMA = 3     /* dispatch + grouped expert products on bf16 MFMA */
};

typedef struct {
    moe_buffer workspace;   /* required: >= moe_block_workspace(...) elements */
    moe_buffer logit_bias;  /* optional [T, E], added to the router logits before routing */
    moe_buffer logits_out;  /* optional [T, E] router logits after the bias */
    moe_buffer ids_out;     /* optional [T, K] selected expert ids (u32) */
    moe_buffer weights_out; /* optional [T, K] routing weights */
    moe_buffer norm_weight; /* optional [h] F32: x is RMSNorm'ed with it first */
    float norm_eps;
    uint32_t residual;      /* 1: out = x + block(norm(x)) (execute.rs:236) */
    uint32_t path;          /* MOE_PATH_* */
    uint32_t reserved;
} moe_block_io;

/* Number of 4-byte workspace elements moe_block needs for `tokens`. */
moe_status moe_block_workspace(const moe_block_weights *w, uint64_t tokens, uint64_t *elems);

/* Where moe_block keeps its routing and dispatch inside the workspace, as
 * element offsets (no reference counterpart: the reference's scratch slots,
 * crates/model-runtime/src/workspace.rs:43-50, hold one token's routing and
 * there is no dispatch).  After a moe_block call over T tokens on a path
 * that dispatches (every path except the fused single-token decode):
 *   counts[E], offsets[E+1], perm[T*K], pos[T*K]  u32, as moe_dispatch writes;
 *   tiles[2*n], ntiles[1]  u32: the work list (expert, first position) of every
 *   run of `tile_pairs_mfma` (bf16 MFMA path) or `tile_pairs_batched` (batched
 *   decode) pairs of the non-empty segments, experts ascending, and its
 *   length n (not written by the VALU grouped path);
 *   xb16[T*h]  bf16 (two per element): the bf16 MFMA path's copy of the
 *   block input (RMS-normalised when io->norm_weight is given), rounded to
 *   nearest even.
 * logits/ids/weights hold the routing when the io struct gives no outputs. */
typedef struct {
    uint64_t logits, ids, weights;
    uint64_t counts, offsets, perm, pos;
    uint64_t tiles, ntiles, xb16;
    uint64_t tile_pairs_mfma, tile_pairs_batched;
    uint64_t total; /* = moe_block_workspace */
} moe_block_layout;
moe_status moe_block_workspace_layout(const moe_block_weights *w, uint64_t tokens,
                                      moe_block_layout *out);
/* One MoE block over T tokens: out[T, h] from x[T, h] (execute.rs:200-234,
 * token-batched). */
moe_status moe_block(moe_gpu *gpu, const moe_block_weights *w, moe_buffer x, moe_buffer out,
                     uint64_t tokens, const moe_block_io *io);

/* moe_block without a workspace argument.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * block's scratch is a file-scope device array of MOE_NOALLOC_SCRATCH_BYTES
 * on every GPU the library runs on, held until the process ends;
 * io->workspace must be empty, and a shape whose workspace
 * (moe_block_workspace) exceeds the array fails with MOE_ERR_SHAPE.  The call
 * allocates nothing.  Every call on one GPU shares that GPU's array: calls on
 * one moe_gpu are stream ordered, but calls that overlap on one GPU (other
 * streams, other moe_gpu handles of the same device) race. */
#define MOE_NOALLOC_SCRATCH_BYTES (64ull << 20)
moe_status moe_block_noalloc(moe_gpu *gpu, const moe_block_weights *w, moe_buffer x, moe_buffer out,
                             uint64_t tokens, const moe_block_io *io);

/* ------------------------------------------------------ measurement -- */

/* Per-kernel timing (the analogue of LLAMA_METAL_PROFILE,
 * crates/metal-backend/src/apple/commands.rs:187-209): while enabled, every
 * kernel this library launches is bracketed by hipEvents on its stream and
 * its duration accumulated under the kernel's name. */
moe_status moe_profile_enable(moe_gpu *gpu, int enable);
/* Number of distinct kernels recorded; then name/count/total seconds by index.
 * Reading synchronizes the stream. */
moe_status moe_profile_count(moe_gpu *gpu, uint32_t *n);
moe_status moe_profile_get(moe_gpu *gpu, uint32_t index, char *name, size_t cap,
                           uint64_t *launches, double *seconds);
moe_status moe_profile_reset(moe_gpu *gpu);
/* Inside an open batch (not a capture): occupy the stream for `microseconds`
 * (<= 100000) so that the launches enqueued next are all queued before the
 * GPU reaches them and profiled durations exclude host enqueue gaps.  No
 * counterpart in the reference (Metal command buffers are committed whole);
 * a measurement aid for moe_profile_*. */
moe_status moe_profile_hold(moe_gpu *gpu, uint32_t microseconds);

/* Stream capture of a batch into a replayable HIP graph (launch-bound decode
 * loops).  moe_graph_begin opens a batch in capture mode; moe_graph_end
 * closes it and instantiates the graph; moe_graph_launch replays it on the
 * gpu's stream (call inside moe_batch_begin/finish to time it). */
typedef struct moe_graph moe_graph;
moe_status moe_graph_begin(moe_gpu *gpu);
moe_status moe_graph_end(moe_gpu *gpu, moe_graph **out);
moe_status moe_graph_launch(moe_gpu *gpu, moe_graph *graph);
void moe_graph_destroy(moe_graph *graph);

/* Device-to-device copy of `elems` 4-byte elements (bench plumbing). */
moe_status moe_copy(moe_gpu *gpu, moe_buffer src, moe_buffer dst);

/* Library version string. */
const char *moe_version(void);

#ifdef __cplusplus
}
#endif
#endif
