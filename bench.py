#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X.

Workload ("config 2"): Qwen3-Next-shaped MoE layer
decode at batch 1 -- hidden 2048, 512 experts, top-10 renormalised softmax
routing, expert ff 512 with SwiGLU, shared expert ff 512 with a sigmoid gate;
routed and shared expert weights MLX-affine 4-bit g64 with bf16 scales and
biases, F32 router.  A step is one MoE layer applied to one token.

Cold-HBM protocol: 8 distinct layers (each with all 512 experts resident,
~7.3 GB in total, far beyond the 256 MB Infinity Cache) are rotated step by
step, every step on a fresh N(0,1) token.  Steps are captured into a HIP graph
of 64 steps and replayed; the timed region is bracketed by stream
synchronisation (hipEvents on the library's stream measure it).

Further legs: config 4 prefill (4096 tokens on the bf16 MFMA path; skip with
--no-prefill); config 3, the same layers with 8-bit g64 routers and shared
experts and hot-set routing, at 1, 8, 32 and 64 concurrent tokens (skip with
--no-batched); config 5, the 48-layer MoE-only stack (RMSNorm, MoE block,
residual) at the config-2 shapes with 2-bit g32 and 8-bit g128 experts, 256
decode steps each (skip with --no-stack).

Output: one JSON line (see the driver contract) with the dominant kernel's
roofline (algorithmic bytes / its hipEvent-measured average duration) and the
CPU oracle timed on this host's cores.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "llama-rs-metal_amd")
sys.path.insert(0, PKG)

import numpy as np  # noqa: E402

from hip_backend import BF16, BlockWeights, Gpu, Tensor, synth  # noqa: E402

METRIC = ("MoE-layer tokens/s + achieved HBM GB/s (decode b=1) and MFMA util (prefill)")
H, E, K, FF, FFS, BITS, GROUP = 2048, 512, 10, 512, 512, 4, 64
# affine matrix bytes = out*in*bits/8 + 2*(out*in/group)*2 (bf16 scales + biases)
MAT_BYTES = FF * H * BITS // 8 + 2 * (FF * H // GROUP) * 2          # 589,824
EXPERT_BYTES_PER_TOKEN = K * 3 * MAT_BYTES + 3 * MAT_BYTES          # 19,464,192
ROUTER_BYTES = H * E * 4 + H * 4                                    # F32 router + gate row
GATEUP_BYTES = K * 2 * MAT_BYTES + 2 * MAT_BYTES                    # decode_gateup per launch (routed + shared gate/up)
HBM_PEAK = 8.0e12
CHUNK = 64       # steps per captured graph
HOLD_US = 40000  # stream hold before a profiled batch (covers its host enqueue)
LAYERS = 8       # distinct weight sets rotated


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_layer_tensors(seed):
    """Host tensors of one config-2 layer (router F32 N(0,0.02); shared expert
    quantised from N(0,0.02); routed experts uniform 4-bit codes with
    N(0,0.02)-sized group scales -- see hip_backend.synth.random_affine)."""
    s = seed * 100
    router = Tensor.dense([H, E], synth.normal(s + 1, H * E, 0.0, 0.02))
    experts = []
    for i, dims in enumerate(([H, FF, E], [H, FF, E], [FF, H, E])):
        n = int(np.prod(dims))
        experts.append(Tensor.affine(dims, *synth.random_affine(s + 2 + i, n, BITS, GROUP, BF16),
                                     BITS, GROUP, BF16))
    shared = []
    for i, dims in enumerate(([H, FFS], [H, FFS], [FFS, H])):
        n = int(np.prod(dims))
        shared.append(Tensor.affine(dims, *synth.quantize_affine(
            synth.normal(s + 5 + i, n, 0.0, 0.02), BITS, GROUP, BF16), BITS, GROUP, BF16))
    sgate = Tensor.dense([H], synth.normal(s + 8, H, 0.0, 0.02))
    return router, experts, shared, sgate


def upload_layer(gpu, tensors):
    router, experts, shared, sgate = tensors
    w = [gpu.weight_tensor(t) for t in [router, *experts]]
    sh = tuple(gpu.weight_tensor(t) for t in shared)
    return BlockWeights(w[0], w[1], w[2], w[3], K, True, sh, gpu.weight_tensor(sgate))


# ---- config 4: Qwen3-30B-A3B-shaped prefill (bf16 MFMA grouped GEMM) ----
P_T, P_H, P_E, P_K, P_FF = 4096, 2048, 128, 8, 768
PREFILL_FLOPS = 2 * P_T * P_K * 3 * P_H * P_FF          # 309,237,645,312 expert FLOPs
ROUTER_FLOPS = 2 * P_T * P_H * P_E
MFMA_PEAK = 2.5e15


def zipf_bias(tokens, experts, seed, s=1.1):
    rng = np.random.Generator(np.random.PCG64(seed))
    rank = np.empty(experts, np.float64)
    rank[rng.permutation(experts)] = np.arange(1, experts + 1)
    return np.broadcast_to((-s * np.log(rank)).astype(np.float32), (tokens, experts)).copy()


def bench_prefill(gpu, iters=10, packed=True):
    """Config 4: one MoE layer over 4096 tokens, Zipf(1.1)-skewed routing.
    With `packed`, the expert weights also get their MFMA tile-order copies
    (moe_pack_weight, made once before timing), which the MFMA path reads."""
    s = 600 * 100
    router = Tensor.affine([P_H, P_E], *synth.random_affine(s + 1, P_H * P_E, 4, 64, BF16), 4, 64,
                           BF16)
    ex = [Tensor.affine(d, *synth.random_affine(s + 2 + i, int(np.prod(d)), 4, 64, BF16), 4, 64,
                        BF16)
          for i, d in enumerate(([P_H, P_FF, P_E], [P_H, P_FF, P_E], [P_FF, P_H, P_E]))]
    w = [gpu.weight_tensor(t) for t in [router, *ex]]
    pk = [gpu.pack_weight(t) for t in w[1:]] if packed else None
    bw = BlockWeights(w[0], w[1], w[2], w[3], P_K, True, packed=pk)
    x = gpu.upload(synth.normal(6060, P_T * P_H))
    out = gpu.zeros(P_T * P_H)
    ws = gpu.zeros(bw.workspace_elems(P_T))
    bias = gpu.upload(zipf_bias(P_T, P_E, 4))
    ids = gpu.zeros(P_T * P_K)
    for _ in range(2):
        with gpu.batch() as b:
            b.moe_block(bw, x, out, P_T, ws, logit_bias=bias, ids_out=ids)
    gpu.profile_reset()
    gpu.profile(True)
    with gpu.batch() as b:
        b.hold(HOLD_US)  # every launch queued before the GPU starts: events time GPU work only
        b.moe_block(bw, x, out, P_T, ws, logit_bias=bias, ids_out=ids)
    prof = gpu.profile_read()
    gpu.profile(False)
    with gpu.batch() as b:
        for _ in range(iters):
            b.moe_block(bw, x, out, P_T, ws, logit_bias=bias, ids_out=ids)
    t = b.seconds / iters
    counts = np.bincount(gpu.read_u32(ids), minlength=P_E)
    k_us = {k: round(v[1] / v[0] * 1e6, 2) for k, v in prof.items()}
    expert_s = sum(v[1] / v[0] for k, v in prof.items() if k in ("gemm_gateup", "gemm_down"))
    for buf in (x, out, ws, bias, ids):
        gpu.release(buf)
    return {
        "workload": "config4: Qwen3-30B-A3B MoE layer prefill, 4096 tokens (h2048 E128 top8 "
                    "ff768, 4-bit g64 bf16, Zipf(1.1) router skew), path bf16 MFMA",
        "expert_weights": "MFMA tile-order copies (moe_pack_weight)" if packed else "row-major",
        "tokens_per_s": round(P_T / t, 1),
        "ms_per_layer": round(t * 1e3, 4),
        "expert_flops": PREFILL_FLOPS,
        "achieved_TFLOPs": round(PREFILL_FLOPS / t / 1e12, 2),
        "mfma_frac": round(PREFILL_FLOPS / t / MFMA_PEAK, 4),
        "expert_kernels_TFLOPs": round(PREFILL_FLOPS / expert_s / 1e12, 2) if expert_s else None,
        "expert_kernels_mfma_frac": round(PREFILL_FLOPS / expert_s / MFMA_PEAK, 4) if expert_s else None,
        "segment_max": int(counts.max()), "segment_min": int(counts.min()),
        "kernels_us": k_us,
    }


# ---- config 3: 8-bit g64 router and shared expert, decode at 1/8/32/64 tokens ----
C3_BATCHES = (1, 8, 32, 64)
C3_CHUNK, C3_REPS = 16, 8  # steps per captured graph, graph replays timed
MAT8_BYTES = FF * H + 2 * (FF * H // GROUP) * 2  # 8-bit g64 matrix with bf16 scales and biases


def hot_bias(tokens, seed, frac=0.2, hot=16, boost=8.0):
    """Config-3 skew: a seeded `frac` of the tokens gets +boost on `hot` experts."""
    rng = np.random.Generator(np.random.PCG64(seed))
    hot_ids = rng.choice(E, hot, replace=False)
    sel = rng.random(tokens) < frac
    b = np.zeros((tokens, E), np.float32)
    b[np.ix_(sel, hot_ids)] = boost
    return b


def c3_layers(gpu, layers):
    """Config-3 layers over the resident config-2 routed experts: 8-bit g64
    routers and shared experts (quantised from N(0, 0.02)), one per layer."""
    out = []
    for l, bw in enumerate(layers):
        s = 800 * 100 + 10 * l
        q8 = lambda seed, dims: Tensor.affine(dims, *synth.quantize_affine(
            synth.normal(seed, int(np.prod(dims)), 0.0, 0.02), 8, GROUP, BF16), 8, GROUP, BF16)
        router = gpu.weight_tensor(q8(s, [H, E]))
        shared = tuple(gpu.weight_tensor(q8(s + 1 + i, d))
                       for i, d in enumerate(([H, FFS], [H, FFS], [FFS, H])))
        sgate = gpu.weight_tensor(Tensor.dense([H], synth.normal(s + 5, H, 0.0, 0.02)))
        _, g, u, d, _, _ = bw.keep
        out.append(BlockWeights(router, g, u, d, K, True, shared, sgate))
    return out


def bench_batched(gpu, layers, T):
    """Config 3 at T concurrent tokens: C3_CHUNK steps over the rotated layers
    (fresh N(0,1) tokens and hot-set biases per step) captured into a graph
    and replayed.  Bytes per step: the distinct routed experts the step
    selects (3 matrices each) plus the 8-bit router and shared expert."""
    xs = gpu.upload(synth.normal(8000 + T, C3_CHUNK * T * H))
    outs = gpu.zeros(C3_CHUNK * T * H)
    bias = gpu.upload(np.concatenate([hot_bias(T, 8100 + 31 * T + j) for j in range(C3_CHUNK)]))
    ids = gpu.zeros(C3_CHUNK * T * K)
    ws = gpu.zeros(layers[0].workspace_elems(T))

    def issue(b, j, ids_out=None):
        b.moe_block(layers[j % len(layers)], xs.view(j * T * H, T * H), outs.view(j * T * H, T * H),
                    T, ws, logit_bias=bias.view(j * T * E, T * E), ids_out=ids_out)

    with gpu.batch() as b:
        for j in range(C3_CHUNK):
            issue(b, j, ids.view(j * T * K, T * K))
    sel = gpu.read_u32(ids).reshape(C3_CHUNK, T * K)
    distinct = [len(np.unique(r)) for r in sel]
    step_bytes = [dn * 3 * MAT_BYTES + 4 * MAT8_BYTES + H * 4 for dn in distinct]
    cap = gpu.capture()
    with cap as b:
        for j in range(C3_CHUNK):
            issue(b, j)
    with gpu.batch() as b:
        b.graph(cap.graph)
    with gpu.batch() as b:
        for _ in range(C3_REPS):
            b.graph(cap.graph)
    per_step = b.seconds / (C3_REPS * C3_CHUNK)
    for buf in (xs, outs, bias, ids, ws):
        gpu.release(buf)
    gbps = np.mean(step_bytes) / per_step / 1e9
    return {"tokens": T, "path": "fused decode" if T == 1 else "batched decode",
            "us_per_step": round(per_step * 1e6, 3), "tokens_per_s": round(T / per_step, 1),
            "distinct_experts_per_step": round(float(np.mean(distinct)), 1),
            "bytes_per_step": int(np.mean(step_bytes)),
            "achieved_GBps": round(gbps, 1), "hbm_frac": round(gbps * 1e9 / HBM_PEAK, 4)}


# ---- config 5: 48-layer MoE-only stack (RMSNorm, MoE block, residual) ----
STACK_LAYERS, STACK_STEPS, STACK_CHUNK = 48, 256, 8
STACK_VARIANTS = {"2bit_g32": (2, 32), "8bit_g128": (8, 128)}


def bench_stack(gpu, variant):
    """Config 5: 256 decode steps at batch 1, each a fresh N(0,1) hidden state
    through 48 layers of RMSNorm -> MoE block (config-2 shapes) -> residual.
    The routed and shared expert weights of one seeded random layer are
    uploaded 48 times (48 distinct HBM copies, all cold for the step); the
    routers (F32) and norm weights are distinct per layer."""
    bits, group = STACK_VARIANTS[variant]
    s = 700 * 100 + bits
    ex = [Tensor.affine(d, *synth.random_affine(s + i, int(np.prod(d)), bits, group, BF16), bits, group,
                        BF16)
          for i, d in enumerate(([H, FF, E], [H, FF, E], [FF, H, E]))]
    sh = [Tensor.affine(d, *synth.random_affine(s + 3 + i, int(np.prod(d)), bits, group, BF16), bits,
                        group, BF16)
          for i, d in enumerate(([H, FFS], [H, FFS], [FFS, H]))]
    sgate = Tensor.dense([H], synth.normal(s + 6, H, 0.0, 0.02))
    layers, norms = [], []
    for l in range(STACK_LAYERS):
        router = Tensor.dense([H, E], synth.normal(s + 10 + l, H * E, 0.0, 0.02))
        w = [gpu.weight_tensor(t) for t in [router, *ex]]
        layers.append(BlockWeights(w[0], w[1], w[2], w[3], K, True,
                                   tuple(gpu.weight_tensor(t) for t in sh), gpu.weight_tensor(sgate)))
        norms.append(gpu.upload((1.0 + 0.1 * synth.normal(s + 100 + l, H)).astype(np.float32)))
    resident = gpu.allocated_bytes()
    log(f"[bench] config-5 {variant}: {STACK_LAYERS} layers resident ({resident / 1e9:.1f} GB on the GPU)")
    xs = gpu.upload(synth.normal(s + 200, STACK_CHUNK * H))
    hs = gpu.zeros(STACK_CHUNK * H)
    ws = gpu.zeros(layers[0].workspace_elems(1))

    def step(b, j):
        h = hs.view(j * H, H)
        b.copy(xs.view(j * H, H), h)
        for l in range(STACK_LAYERS):
            b.moe_block(layers[l], h, h, 1, ws, norm_weight=norms[l], norm_eps=1e-6, residual=True)

    cap = gpu.capture()
    with cap as b:
        for j in range(STACK_CHUNK):
            step(b, j)
    with gpu.batch() as b:
        b.graph(cap.graph)
    with gpu.batch() as b:
        for _ in range(STACK_STEPS // STACK_CHUNK):
            b.graph(cap.graph)
    per_token = b.seconds / STACK_STEPS
    mat = lambda i, o: o * i * bits // 8 + 2 * (o * i // group) * 2
    token_bytes = STACK_LAYERS * ((K + 1) * (2 * mat(H, FF) + mat(FF, H)) + H * E * 4 + H * 4)
    del layers, norms
    expert_bytes = STACK_LAYERS * (K + 1) * (2 * mat(H, FF) + mat(FF, H))
    return {"variant": variant, "layers": STACK_LAYERS, "steps": STACK_STEPS,
            "expert_bytes_per_token": expert_bytes,
            "us_per_token": round(per_token * 1e6, 2), "tokens_per_s": round(1.0 / per_token, 1),
            "us_per_layer": round(per_token * 1e6 / STACK_LAYERS, 3),
            "bytes_per_token": token_bytes,
            "achieved_GBps": round(token_bytes / per_token / 1e9, 1),
            "hbm_frac": round(token_bytes / per_token / HBM_PEAK, 4),
            "weights": "one seeded random expert set uploaded 48 times; distinct F32 routers and norm weights"}


def cpu_baseline(tensors, budget_s):
    """The C oracle (single thread) on the same layer, bounded sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    router, experts, shared, sgate = tensors
    spec = oracle.MoeSpec(router, experts[0], experts[1], experts[2], K, True, tuple(shared), sgate)
    oracle.build() if not os.path.exists(oracle.LIB_PATH) else None
    n, t0 = 0, time.perf_counter()
    while True:
        x = synth.normal(900000 + n, H).reshape(1, H)
        oracle.moe_block(spec, x, 1)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 10000:
            break
    return {"value": n / el, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{n} config-2 decode tokens (layer 0 weights, seeds 900000+) through "
                      f"oracle/moe_oracle.c orc_moe_block, single thread, {el:.1f} s"}


COPY_BYTES = 256 << 20  # calibration copy: reads and writes 256 MiB


def traffic_probe(gpu, which):
    """Eager workload for HBM-traffic counters (rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE): a few launches of the named path, then a plain copy kernel of
    COPY_BYTES (reads COPY_BYTES, writes COPY_BYTES) whose counter readings
    calibrate the scale of the counters."""
    src = gpu.zeros(COPY_BYTES // 4)
    dst = gpu.zeros(COPY_BYTES // 4)
    if which == "decode":
        layers = [upload_layer(gpu, make_layer_tensors(500 + l)) for l in range(LAYERS)]
        xs = gpu.upload(synth.normal(4242, CHUNK * H))
        outs = gpu.zeros(CHUNK * H)
        ws = gpu.zeros(layers[0].workspace_elems(1))
        with gpu.batch() as b:
            for j in range(CHUNK):
                b.moe_block(layers[j % LAYERS], xs.view(j * H, H), outs.view(j * H, H), 1, ws)
        log(f"[probe] {CHUNK} eager config-2 decode steps done")
    else:
        bench_prefill(gpu, iters=1)
        log("[probe] config-4 prefill done")
    with gpu.batch() as b:
        for _ in range(4):
            b.copy(src, dst)
    log(f"[probe] 4 copies of {COPY_BYTES} bytes done")


def committed_traffic(kernel_prefix):
    """HBM bytes per launch of a kernel from the committed rocprofv3 --pmc
    summary (profiles/traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        kernels = json.load(f).get("kernels", {})
    for name, v in kernels.items():
        if name.startswith(kernel_prefix):
            return v.get("bytes_per_launch")
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=12800)
    ap.add_argument("--warmup", type=int, default=640)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-stack", action="store_true")
    ap.add_argument("--no-batched", action="store_true")
    ap.add_argument("--traffic-probe", choices=["decode", "prefill"], default=None,
                    help="short eager workload for rocprofv3 --pmc runs (no timing output)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(the MoE layer would shard by expert, one process per GPU, with an "
              f"all-reduce of the partial outputs in decode)", file=sys.stderr)
        sys.exit(2)
    steps = max(CHUNK, (args.steps + CHUNK - 1) // CHUNK * CHUNK)
    warm = max(CHUNK, (args.warmup + CHUNK - 1) // CHUNK * CHUNK)

    gpu = Gpu(0)
    if args.traffic_probe:
        traffic_probe(gpu, args.traffic_probe)
        gpu.close()
        return
    log(f"[bench] device {gpu.name}; building {LAYERS} config-2 layers")
    layers, host0 = [], None
    for l in range(LAYERS):
        t = make_layer_tensors(500 + l)
        layers.append(upload_layer(gpu, t))
        if l == 0:
            host0 = t
        log(f"[bench] layer {l} resident ({gpu.allocated_bytes() / 1e9:.2f} GB)")
    xs = gpu.upload(synth.normal(4242, CHUNK * H))
    outs = gpu.zeros(CHUNK * H)
    ws = gpu.zeros(layers[0].workspace_elems(1))

    def issue(b, j):
        x = xs.view(j * H, H)
        o = outs.view(j * H, H)
        b.moe_block(layers[j % LAYERS], x, o, 1, ws)

    # per-kernel durations: hipEvents around each launch on the library's
    # stream, with the stream held until all CHUNK steps are enqueued so that
    # the events bracket GPU execution and not host enqueue gaps
    gpu.profile_reset()
    gpu.profile(True)
    with gpu.batch() as b:
        b.hold(HOLD_US)
        t_enq = time.perf_counter()
        for j in range(CHUNK):
            issue(b, j)
        t_enq = time.perf_counter() - t_enq
    prof = gpu.profile_read()
    if t_enq * 1e6 > HOLD_US:
        log(f"[bench] warning: enqueue took {t_enq * 1e3:.1f} ms, longer than the hold")
    gpu.profile(False)
    kernels = {k: v[1] / v[0] for k, v in prof.items()}
    log("[bench] kernel averages (us): " + ", ".join(f"{k} {v * 1e6:.2f}" for k, v in kernels.items()))

    # eager throughput (no graph) for reference
    with gpu.batch() as b:
        for j in range(CHUNK):
            issue(b, j)
    eager_s = b.seconds / CHUNK

    cap = gpu.capture()
    with cap as b:
        for j in range(CHUNK):
            issue(b, j)
    graph = cap.graph
    with gpu.batch() as b:
        for _ in range(warm // CHUNK):
            b.graph(graph)
    log(f"[bench] warmup {warm} steps done")
    t0 = time.perf_counter()
    with gpu.batch() as b:
        for _ in range(steps // CHUNK):
            b.graph(graph)
    wall = time.perf_counter() - t0
    gpu_s = b.seconds
    log(f"[bench] timed {steps} steps: {gpu_s * 1e3:.2f} ms (events), {wall * 1e3:.2f} ms (wall)")
    elapsed = max(gpu_s, 1e-12)
    per_step = elapsed / steps

    dom = "decode_gateup"
    dom_s = kernels.get(dom)
    roof = None
    if dom_s:
        achieved = GATEUP_BYTES / dom_s / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK / 1e9,
                "unit": "GB/s", "frac": round(achieved * 1e9 / HBM_PEAK, 4), "traffic": None,
                "kernel": dom, "algorithmic_bytes_per_launch": GATEUP_BYTES,
                "avg_launch_us": round(dom_s * 1e6, 3)}
        traffic = committed_traffic("decode_gateup_kernel")
        if traffic:
            roof["traffic"] = traffic
            roof["traffic_source"] = "profiles/traffic.json (rocprofv3 --pmc, calibrated)"

    layer_gbps = EXPERT_BYTES_PER_TOKEN / per_step / 1e9
    result = {
        "metric": METRIC,
        "value": round(steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(per_step * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "config2: Qwen3-Next MoE layer decode b=1 (h2048 E512 top10 "
                               "ff512 + shared ff512, 4-bit g64 bf16, F32 router)",
                   "layers_rotated": LAYERS, "graph_steps": CHUNK, "path": "fused decode"},
        "layer_hbm": {"expert_bytes_per_token": EXPERT_BYTES_PER_TOKEN,
                      "all_bytes_per_token": EXPERT_BYTES_PER_TOKEN + ROUTER_BYTES,
                      "achieved_GBps": round(layer_gbps, 1),
                      "frac": round(layer_gbps * 1e9 / HBM_PEAK, 4)},
        "eager_ms_per_step": round(eager_s * 1e3, 6),
        "kernels_us": {k: round(v * 1e6, 3) for k, v in kernels.items()},
        "roofline": roof,
        "cpu_baseline": None,
    }
    if not args.no_prefill:
        log("[bench] config-4 prefill (bf16 MFMA)")
        result["prefill"] = bench_prefill(gpu)
        log(f"[bench] prefill: {result['prefill']['ms_per_layer']} ms/layer, "
            f"{result['prefill']['achieved_TFLOPs']} TFLOP/s")
    if not args.no_batched:
        c3 = c3_layers(gpu, layers)
        result["batched"] = []
        for T in C3_BATCHES:
            r = bench_batched(gpu, c3, T)
            log(f"[bench] config-3 T={T}: {r['us_per_step']} us/step, {r['tokens_per_s']} tokens/s, "
                f"{r['achieved_GBps']} GB/s over {r['distinct_experts_per_step']} experts")
            result["batched"].append(r)
        del c3
    if not args.no_stack:
        result["stack"] = []
        for v in STACK_VARIANTS:
            r = bench_stack(gpu, v)
            log(f"[bench] config-5 {v}: {r['us_per_token']} us/token over {STACK_LAYERS} layers, "
                f"{r['achieved_GBps']} GB/s")
            result["stack"].append(r)
    if not args.no_cpu:
        log("[bench] timing the CPU oracle")
        result["cpu_baseline"] = cpu_baseline(host0, args.cpu_seconds)
        result["cpu_baseline"]["host_cpus"] = os.cpu_count()
    print(json.dumps(result), flush=True)
    gpu.close()


if __name__ == "__main__":
    main()
