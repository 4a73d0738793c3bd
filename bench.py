#!/usr/bin/env python3
"""MoE-layer benchmark on one MI355X.

Workload ("config 2"): Qwen3-Next-shaped MoE layer
decode at batch 1 -- hidden 2048, 512 experts, top-10 renormalised softmax
routing, expert ff 512 with SwiGLU, shared expert ff 512 with a sigmoid gate;
routed and shared expert weights MLX-affine 4-bit g64 with bf16 scales and
biases quantized from seeded N(0, 0.02), F32 router N(0, 0.02), N(0, 1)
activations.  A step is one MoE layer applied to one token; `value` is the
steps per second over exactly --steps steps.

Cold-HBM protocol: 8 distinct layers (each with all 512 experts resident,
~7.3 GB in total, far beyond the 256 MB Infinity Cache) are rotated step by
step, every step on a fresh N(0,1) token.  Steps are captured into HIP graphs
(64 steps, plus one graph of the remainder) and replayed; the timed region is
bracketed by stream synchronisation (hipEvents on the library's stream).
Weights are generated on the GPU (hip_backend.probe: the reference fixture
LCG, Box-Muller, the documented affine quantizer).

Further legs: config 4 prefill (4096 tokens on the bf16 MFMA path, eager and
as a graph replay; skip with --no-prefill); config 3, the same layers with
8-bit g64 routers and shared experts and hot-set routing, at 1, 8, 32 and 64
concurrent tokens (--no-batched); config 5, the 48-layer MoE-only stack
(RMSNorm, MoE block, residual) at the config-2 shapes with 2-bit g32 and 8-bit
g128 experts, distinct weights per layer, 256 decode steps each (--no-stack).
The measured peaks (an MFMA-only loop, a streaming HBM read) are reported
beside the published ones (--no-peaks).

Output: one JSON line (see the driver contract) with the dominant kernel's
roofline (algorithmic bytes / its hipEvent-measured average duration) and the
CPU oracle timed on this host's cores: single thread and all cores on
config-2 decode, all cores on a config-4 prefill sample.
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

from hip_backend import BF16, BlockWeights, Gpu, Tensor, probe, synth  # noqa: E402

METRIC = ("MoE-layer tokens/s + achieved HBM GB/s (decode b=1) and MFMA util (prefill)")
H, E, K, FF, FFS, BITS, GROUP = 2048, 512, 10, 512, 512, 4, 64
# affine matrix bytes = out*in*bits/8 + 2*(out*in/group)*2 (bf16 scales + biases)
MAT_BYTES = FF * H * BITS // 8 + 2 * (FF * H // GROUP) * 2          # 589,824
EXPERT_BYTES_PER_TOKEN = K * 3 * MAT_BYTES + 3 * MAT_BYTES          # 19,464,192
ROUTER_BYTES = H * E * 4 + H * 4                                    # F32 router + gate row
GATEUP_BYTES = K * 2 * MAT_BYTES + 2 * MAT_BYTES                    # decode_gateup per launch (routed + shared gate/up)
HBM_PEAK = 8.0e12
MFMA_PEAK = 2.5e15   # dense bf16
F32_MFMA_PEAK = 157.3e12
CHUNK = 64       # steps per captured graph
HOLD_US = 40000  # stream hold before a profiled batch (covers its host enqueue)
LAYERS = 8       # distinct weight sets rotated
LONG_RUN = 6400  # steps of the steady-state run reported beside `value`


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_layer(gpu, seed):
    """One config-2 layer on the GPU: F32 router N(0, 0.02); routed and shared
    experts quantized (4-bit g64 bf16) from N(0, 0.02); F32 shared-expert gate
    row.  Returns (BlockWeights, [router, gate, up, down, sg, su, sd, gate_row])."""
    s = seed * 100
    router = probe.synth_dense_weight(gpu, [H, E], s + 1)
    experts = [probe.synth_affine_weight(gpu, d, BITS, GROUP, BF16, s + 2 + i)
               for i, d in enumerate(([H, FF, E], [H, FF, E], [FF, H, E]))]
    shared = [probe.synth_affine_weight(gpu, d, BITS, GROUP, BF16, s + 5 + i)
              for i, d in enumerate(([H, FFS], [H, FFS], [FFS, H]))]
    sgate = gpu.weight_tensor(Tensor.dense([H], synth.normal(s + 8, H, 0.0, 0.02)))
    bw = BlockWeights(router, experts[0], experts[1], experts[2], K, True, tuple(shared), sgate)
    return bw, [router, *experts, *shared, sgate]


# Captured graphs, one per (issue function, steps per graph): made once, replayed
# by every later call with the same pair, and destroyed only at the end of
# main() after the final synchronisation, so no executable is torn down while
# a profiler may still be recording the dispatches of earlier replays.
_GRAPHS = {}


def graph_of(gpu, issue, n):
    """The graph of steps issue(b, 0 .. n-1), captured on first use."""
    g = _GRAPHS.get((issue, n))
    if g is None:
        cap = gpu.capture()
        with cap as b:
            for j in range(n):
                issue(b, j)
        g = _GRAPHS[(issue, n)] = cap.graph
    return g


def release_graphs():
    for g in _GRAPHS.values():
        g.destroy()
    _GRAPHS.clear()


def run_graphs(gpu, issue, steps, chunk):
    """`steps` steps as replays of a captured graph of `chunk` steps plus one
    graph of the remainder, in one batch; returns the batch's GPU seconds.
    issue(b, j) issues step j (0 <= j < chunk)."""
    graphs = []
    for n in (chunk, steps % chunk):
        if n == 0 or (n == chunk and steps < chunk):
            graphs.append(None)
            continue
        graphs.append(graph_of(gpu, issue, n))
    full, rest = graphs
    with gpu.batch() as b:
        for _ in range(steps // chunk):
            b.graph(full)
        if rest is not None:
            b.graph(rest)
    return b.seconds


# ---- config 4: Qwen3-30B-A3B-shaped prefill (bf16 MFMA grouped GEMM) ----
P_T, P_H, P_E, P_K, P_FF = 4096, 2048, 128, 8, 768
PREFILL_FLOPS = 2 * P_T * P_K * 3 * P_H * P_FF          # 309,237,645,312 expert FLOPs
ROUTER_FLOPS = 2 * P_T * P_H * P_E


def zipf_bias(tokens, experts, seed, s=1.1):
    rng = np.random.Generator(np.random.PCG64(seed))
    rank = np.empty(experts, np.float64)
    rank[rng.permutation(experts)] = np.arange(1, experts + 1)
    return np.broadcast_to((-s * np.log(rank)).astype(np.float32), (tokens, experts)).copy()


def prefill_layer(gpu, packed=True):
    """Config-4 weights on the GPU (4-bit g64 bf16 quantized from N(0, 0.02),
    router too); with `packed`, also the experts' MFMA tile-order copies
    (moe_pack_weight), which the MFMA path reads."""
    s = 600 * 100
    router = probe.synth_affine_weight(gpu, [P_H, P_E], 4, 64, BF16, s + 1)
    ex = [probe.synth_affine_weight(gpu, d, 4, 64, BF16, s + 2 + i)
          for i, d in enumerate(([P_H, P_FF, P_E], [P_H, P_FF, P_E], [P_FF, P_H, P_E]))]
    pk = [gpu.pack_weight(t) for t in ex] if packed else None
    return BlockWeights(router, ex[0], ex[1], ex[2], P_K, True, packed=pk), [router, *ex]


def bench_prefill(gpu, bw, iters=10, T=P_T, flops=PREFILL_FLOPS, bias_np=None, workload=None):
    """One MoE layer over T tokens (default: config 4, Zipf(1.1)-skewed
    routing), timed eagerly (one moe_block call per layer) and as replays of
    a captured graph of one layer; per-kernel times from a held batch."""
    h, E, K = bw.hidden, bw.experts, bw.k
    if bias_np is None:
        bias_np = zipf_bias(T, E, 4)
    x = probe.synth_normal(gpu, T * h, 6060)
    out = gpu.zeros(T * h)
    ws = gpu.zeros(bw.workspace_elems(T))
    bias = gpu.upload(bias_np)
    ids = gpu.zeros(T * K)
    for _ in range(2):
        with gpu.batch() as b:
            b.moe_block(bw, x, out, T, ws, logit_bias=bias, ids_out=ids)
    gpu.profile_reset()
    gpu.profile(True)
    with gpu.batch() as b:
        b.hold(HOLD_US)  # every launch queued before the GPU starts: events time GPU work only
        b.moe_block(bw, x, out, T, ws, logit_bias=bias, ids_out=ids)
    prof = gpu.profile_read()
    gpu.profile(False)
    with gpu.batch() as b:
        for _ in range(iters):
            b.moe_block(bw, x, out, T, ws, logit_bias=bias, ids_out=ids)
    t_eager = b.seconds / iters
    graph = graph_of(gpu, lambda b, j: b.moe_block(bw, x, out, T, ws, logit_bias=bias, ids_out=ids), 1)
    with gpu.batch() as b:
        b.graph(graph)
    with gpu.batch() as b:
        for _ in range(iters):
            b.graph(graph)
    t = b.seconds / iters
    counts = np.bincount(gpu.read_u32(ids), minlength=E)
    k_us = {k: round(v[1] / v[0] * 1e6, 2) for k, v in prof.items()}
    expert_s = sum(v[1] / v[0] for k, v in prof.items() if k in ("gemm_gateup", "gemm_down"))
    routed_flops = 2 * T * K * 3 * h * bw.keep[1].dims[1]
    for buf in (x, out, ws, bias, ids):
        gpu.release(buf)
    return {
        "workload": workload or ("config4: Qwen3-30B-A3B MoE layer prefill, 4096 tokens (h2048 E128 top8 "
                                 "ff768, 4-bit g64 bf16 quantized from N(0,0.02), Zipf(1.1) router skew), "
                                 "F32 router product, bf16 MFMA expert products"),
        "expert_weights": "MFMA tile-order copies (moe_pack_weight)" if bw.packed else "row-major",
        "tokens_per_s": round(T / t, 1),
        "ms_per_layer": round(t * 1e3, 4),
        "timing": "graph replay of one layer (hipEvents over 10 replays)",
        "eager_ms_per_layer": round(t_eager * 1e3, 4),
        "expert_flops": flops,
        "achieved_TFLOPs": round(flops / t / 1e12, 2),
        "mfma_frac": round(flops / t / MFMA_PEAK, 4),
        "routed_expert_kernels_TFLOPs": round(routed_flops / expert_s / 1e12, 2) if expert_s else None,
        "routed_expert_kernels_mfma_frac": round(routed_flops / expert_s / MFMA_PEAK, 4) if expert_s else None,
        "kernels_sum_us": round(sum(k_us.values()), 2),
        "segment_max": int(counts.max()), "segment_min": int(counts.min()),
        "kernels_us": k_us,
    }


QN_T = 4096
QN_FLOPS = 2 * QN_T * K * 3 * H * FF + 2 * QN_T * 3 * H * FFS  # routed + shared expert FLOPs


def bench_prefill_qwen3next(gpu, layer):
    """A Qwen3-Next-shaped prefill (config-2 shapes: E 512, top 10, ff 512,
    shared ff 512, F32 router, 4-bit g64 experts and shared expert) of 4096
    tokens over layer 0 of the decode leg, with the MFMA tile-order copies of
    the routed and the shared experts: the shared expert runs as one more
    segment of the routed experts' bf16 GEMMs, its gate input from the
    router's pass over x."""
    bw0, ws0 = layer
    router, g, u, d = ws0[:4]
    pk = [gpu.pack_weight(t) for t in (g, u, d)]
    _, _, _, _, shared, sgate = bw0.keep
    spk = [gpu.pack_weight(t) for t in shared]
    bw = BlockWeights(router, g, u, d, K, True, shared, sgate, packed=pk, shared_packed=spk)
    r = bench_prefill(gpu, bw, T=QN_T, flops=QN_FLOPS, bias_np=np.zeros((QN_T, E), np.float32),
                      workload="Qwen3-Next-shaped MoE layer prefill, 4096 tokens (config-2 shapes: h2048 "
                               "E512 top10 ff512 + shared ff512, 4-bit g64 bf16 quantized from N(0,0.02), "
                               "F32 router, no skew), shared expert as one more segment of the bf16 GEMMs")
    for p_ in pk + spk:
        for b_ in p_.buffers:
            gpu.release(b_)
    return r


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
    routers and shared experts quantized from N(0, 0.02), one per layer."""
    out = []
    for l, (bw, _) in enumerate(layers):
        s = 800 * 100 + 10 * l
        router = probe.synth_affine_weight(gpu, [H, E], 8, GROUP, BF16, s)
        shared = tuple(probe.synth_affine_weight(gpu, d, 8, GROUP, BF16, s + 1 + i)
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
    xs = probe.synth_normal(gpu, C3_CHUNK * T * H, 8000 + T)
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
    run_graphs(gpu, issue, C3_CHUNK, C3_CHUNK)  # warm
    per_step = run_graphs(gpu, issue, C3_REPS * C3_CHUNK, C3_CHUNK) / (C3_REPS * C3_CHUNK)
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
    Every layer has its own weights, generated on the GPU: experts and shared
    expert quantized from N(0, 0.02) at the variant's bits and group (bf16
    scales and biases), F32 router N(0, 0.02), norm weights 1 + 0.1 N(0, 1)."""
    bits, group = STACK_VARIANTS[variant]
    s0 = 700 * 100 + bits
    layers, norms, keep = [], [], []
    for l in range(STACK_LAYERS):
        s = s0 + 1000 * l
        router = probe.synth_dense_weight(gpu, [H, E], s)
        ex = [probe.synth_affine_weight(gpu, d, bits, group, BF16, s + 1 + i)
              for i, d in enumerate(([H, FF, E], [H, FF, E], [FF, H, E]))]
        sh = [probe.synth_affine_weight(gpu, d, bits, group, BF16, s + 4 + i)
              for i, d in enumerate(([H, FFS], [H, FFS], [FFS, H]))]
        sgate = gpu.weight_tensor(Tensor.dense([H], synth.normal(s + 7, H, 0.0, 0.02)))
        layers.append(BlockWeights(router, ex[0], ex[1], ex[2], K, True, tuple(sh), sgate))
        keep += [router, *ex, *sh]
        norms.append(gpu.upload((1.0 + 0.1 * synth.normal(s + 8, H)).astype(np.float32)))
    resident = gpu.allocated_bytes()
    log(f"[bench] config-5 {variant}: {STACK_LAYERS} distinct layers resident "
        f"({resident / 1e9:.1f} GB on the GPU)")
    xs = probe.synth_normal(gpu, STACK_CHUNK * H, s0 + 200)
    hs = gpu.zeros(STACK_CHUNK * H)
    ws = gpu.zeros(layers[0].workspace_elems(1))

    def step(b, j):
        h = hs.view(j * H, H)
        b.copy(xs.view(j * H, H), h)
        for l in range(STACK_LAYERS):
            b.moe_block(layers[l], h, h, 1, ws, norm_weight=norms[l], norm_eps=1e-6, residual=True)

    run_graphs(gpu, step, STACK_CHUNK, STACK_CHUNK)  # warm
    per_token = run_graphs(gpu, step, STACK_STEPS, STACK_CHUNK) / STACK_STEPS
    mat = lambda i, o: o * i * bits // 8 + 2 * (o * i // group) * 2
    expert_bytes = STACK_LAYERS * (K + 1) * (2 * mat(H, FF) + mat(FF, H))
    token_bytes = expert_bytes + STACK_LAYERS * (H * E * 4 + H * 4)
    for w in keep:
        probe.release(gpu, w)
    for buf in (*norms, xs, hs, ws):
        gpu.release(buf)
    return {"variant": variant, "layers": STACK_LAYERS, "steps": STACK_STEPS,
            "expert_bytes_per_token": expert_bytes,
            "us_per_token": round(per_token * 1e6, 2), "tokens_per_s": round(1.0 / per_token, 1),
            "us_per_layer": round(per_token * 1e6 / STACK_LAYERS, 3),
            "bytes_per_token": token_bytes,
            "achieved_GBps": round(token_bytes / per_token / 1e9, 1),
            "hbm_frac": round(token_bytes / per_token / HBM_PEAK, 4),
            "resident_GB": round(resident / 1e9, 1),
            "weights": "48 distinct layers generated on the GPU (N(0,0.02) quantized experts and "
                       "shared experts, F32 routers)"}


# ---- CPU baseline: the C oracle on this host's cores ----
def host_cores():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))  # the box's CPU share for one GPU is 16


def time_oracle(spec, h, tokens_per_call, budget_s, seed0):
    import oracle
    n, t0 = 0, time.perf_counter()
    while True:
        x = synth.normal(seed0 + n, tokens_per_call * h).reshape(tokens_per_call, h)
        oracle.moe_block(spec, x, tokens_per_call)
        n += tokens_per_call
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 100000:
            return n, el


def cpu_baseline(gpu, layer0, pre, budget_s):
    """The C oracle (oracle/moe_oracle.c) on host copies of the benchmark's own
    weights: config-2 decode on one thread and on all cores, and a bounded
    config-4 prefill sample on all cores (token by token, as the reference's
    per-token loop runs, crates/model-runtime/src/execute.rs:208)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()
    bw, ws2 = layer0
    router, g, u, d, sg, su, sd, sgate = ws2
    host = [probe.to_host(gpu, w) for w in (router, g, u, d, sg, su, sd)]
    gate_row = Tensor.dense([H], synth.normal(500 * 100 + 8, H, 0.0, 0.02))
    spec2 = oracle.MoeSpec(host[0], host[1], host[2], host[3], K, True, tuple(host[4:7]), gate_row)
    cores = host_cores()
    oracle.set_threads(1)
    n1, e1 = time_oracle(spec2, H, 1, budget_s, 900000)
    oracle.set_threads(cores)
    nc, ec = time_oracle(spec2, H, 1, budget_s, 910000)
    res = {"value": round(nc / ec, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
           "sample": f"{nc} config-2 decode tokens (layer 0 of the benchmark's weights, seeds 910000+) "
                     f"through oracle/moe_oracle.c orc_moe_block, OpenMP rows over {cores} threads, "
                     f"{ec:.1f} s",
           "single_thread": {"value": round(n1 / e1, 3), "unit": "tokens/s", "cores": 1,
                             "sample": f"{n1} config-2 decode tokens, one thread, {e1:.1f} s"}}
    if pre is not None:
        pbw, pws = pre
        ph = [probe.to_host(gpu, w) for w in pws]
        spec4 = oracle.MoeSpec(ph[0], ph[1], ph[2], ph[3], P_K, True)
        np_, ep = time_oracle(spec4, P_H, 1, budget_s, 920000)
        res["prefill"] = {"value": round(np_ / ep, 3), "unit": "tokens/s", "cores": cores,
                          "sample": f"{np_} config-4 tokens (the benchmark's prefill weights, "
                                    f"token by token) on {cores} threads, {ep:.1f} s"}
    oracle.set_threads(cores)
    res["host_cpus"] = os.cpu_count()
    return res


COPY_BYTES = 256 << 20  # calibration copy: reads and writes 256 MiB


def traffic_probe(gpu, which):
    """Eager workload for HBM-traffic counters (rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE): a few launches of the named path, then a plain copy kernel of
    COPY_BYTES (reads COPY_BYTES, writes COPY_BYTES) whose counter readings
    calibrate the scale of the counters."""
    src = gpu.zeros(COPY_BYTES // 4)
    dst = gpu.zeros(COPY_BYTES // 4)
    if which == "decode":
        layers = [make_layer(gpu, 500 + l)[0] for l in range(LAYERS)]
        xs = probe.synth_normal(gpu, CHUNK * H, 4242)
        outs = gpu.zeros(CHUNK * H)
        ws = gpu.zeros(layers[0].workspace_elems(1))
        with gpu.batch() as b:
            for j in range(CHUNK):
                b.moe_block(layers[j % LAYERS], xs.view(j * H, H), outs.view(j * H, H), 1, ws)
        log(f"[probe] {CHUNK} eager config-2 decode steps done")
    elif which == "prefill":
        bench_prefill(gpu, prefill_layer(gpu)[0], iters=1)
        log("[probe] config-4 prefill done")
    else:  # the peak probes, short (MFMA counters calibrate against them)
        log(f"[probe] bf16 MFMA {probe.mfma_peak('bf16', iters=2000, reps=1):.1f} TFLOP/s, "
            f"F32 MFMA {probe.mfma_peak('f32', iters=200, reps=1):.1f} TFLOP/s, "
            f"read {probe.hbm_read(1 << 30, reps=1):.1f} GB/s")
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


def peaks():
    """This GPU's measured rates beside the published MI355X peaks."""
    return {"hbm_read_GBps": round(probe.hbm_read(4 << 30, reps=5), 1),
            "mfma_bf16_TFLOPs": round(probe.mfma_peak("bf16"), 1),
            "mfma_f32_TFLOPs": round(probe.mfma_peak("f32"), 1),
            "published": {"hbm_GBps": HBM_PEAK / 1e9, "mfma_bf16_TFLOPs": MFMA_PEAK / 1e12,
                          "mfma_f32_TFLOPs": F32_MFMA_PEAK / 1e12},
            "method": "hip_backend.probe: a streaming 16-byte-load read of 4 GiB, and MFMA-only loops "
                      "(4 independent 32x32 accumulators per wave, 8 four-wave blocks per CU); best of "
                      "5 / 3 timed launches"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=12800)
    ap.add_argument("--warmup", type=int, default=640)
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-stack", action="store_true")
    ap.add_argument("--no-batched", action="store_true")
    ap.add_argument("--no-peaks", action="store_true")
    ap.add_argument("--long-run", type=int, default=LONG_RUN,
                    help="steps of the steady-state run reported beside `value` (0: none)")
    ap.add_argument("--traffic-probe", choices=["decode", "prefill", "peaks"], default=None,
                    help="short workload for rocprofv3 --pmc runs (no timing output)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(the MoE layer would shard by expert, one process per GPU, with an "
              f"all-reduce of the partial outputs in decode)", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        sys.exit(2)
    steps, warm = args.steps, args.warmup

    gpu = Gpu(0)
    if args.traffic_probe:
        traffic_probe(gpu, args.traffic_probe)
        release_graphs()
        gpu.close()
        return
    log(f"[bench] device {gpu.name}; generating {LAYERS} config-2 layers on the GPU")
    layers = []
    for l in range(LAYERS):
        layers.append(make_layer(gpu, 500 + l))
        log(f"[bench] layer {l} resident ({gpu.allocated_bytes() / 1e9:.2f} GB)")
    xs = probe.synth_normal(gpu, CHUNK * H, 4242)
    outs = gpu.zeros(CHUNK * H)
    ws = gpu.zeros(layers[0][0].workspace_elems(1))

    def issue(b, j):
        b.moe_block(layers[j % LAYERS][0], xs.view(j * H, H), outs.view(j * H, H), 1, ws)

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

    if warm:
        run_graphs(gpu, issue, warm, CHUNK)
    log(f"[bench] warmup {warm} steps done")
    t0 = time.perf_counter()
    gpu_s = run_graphs(gpu, issue, steps, CHUNK)
    wall = time.perf_counter() - t0
    log(f"[bench] timed {steps} steps: {gpu_s * 1e3:.3f} ms (events), {wall * 1e3:.3f} ms (wall)")
    elapsed = max(gpu_s, 1e-12)
    per_step = elapsed / steps
    long_s = run_graphs(gpu, issue, args.long_run, CHUNK) / args.long_run if args.long_run > 0 else None

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
        "data": "synthetic (seeded N(0,0.02) weights quantized to 4-bit g64 on the GPU, N(0,1) tokens)",
        "config": {"workload": "config2: Qwen3-Next MoE layer decode b=1 (h2048 E512 top10 "
                               "ff512 + shared ff512, 4-bit g64 bf16, F32 router)",
                   "layers_rotated": LAYERS, "graph_steps": CHUNK, "path": "fused decode"},
        "layer_hbm": {"expert_bytes_per_token": EXPERT_BYTES_PER_TOKEN,
                      "all_bytes_per_token": EXPERT_BYTES_PER_TOKEN + ROUTER_BYTES,
                      "achieved_GBps": round(layer_gbps, 1),
                      "frac": round(layer_gbps * 1e9 / HBM_PEAK, 4)},
        "long_run": {"steps": args.long_run, "ms_per_step": round(long_s * 1e3, 6),
                     "tokens_per_s": round(1.0 / long_s, 1)} if long_s else None,
        "eager_ms_per_step": round(eager_s * 1e3, 6),
        "kernels_us": {k: round(v * 1e6, 3) for k, v in kernels.items()},
        "roofline": roof,
        "cpu_baseline": None,
    }
    pre = None
    if not args.no_prefill:
        log("[bench] config-4 prefill (F32 router, bf16 MFMA experts)")
        pre = prefill_layer(gpu)
        result["prefill"] = bench_prefill(gpu, pre[0])
        log(f"[bench] prefill: {result['prefill']['ms_per_layer']} ms/layer (graph), "
            f"{result['prefill']['eager_ms_per_layer']} ms eager, {result['prefill']['achieved_TFLOPs']} TFLOP/s")
        result["prefill_qwen3next"] = bench_prefill_qwen3next(gpu, layers[0])
        log(f"[bench] Qwen3-Next-shaped prefill: {result['prefill_qwen3next']['ms_per_layer']} ms/layer, "
            f"{result['prefill_qwen3next']['achieved_TFLOPs']} TFLOP/s, kernels "
            f"{result['prefill_qwen3next']['kernels_us']}")
    if not args.no_batched:
        c3 = c3_layers(gpu, layers)
        result["batched"] = []
        for T in C3_BATCHES:
            r = bench_batched(gpu, c3, T)
            log(f"[bench] config-3 T={T}: {r['us_per_step']} us/step, {r['tokens_per_s']} tokens/s, "
                f"{r['achieved_GBps']} GB/s over {r['distinct_experts_per_step']} experts")
            result["batched"].append(r)
        del c3
    if not args.no_peaks:
        result["peaks"] = peaks()
        log(f"[bench] peaks: {result['peaks']}")
        if "prefill" in result:
            p = result["prefill"]
            p["mfma_frac_of_measured_peak"] = round(p["achieved_TFLOPs"] / result["peaks"]["mfma_bf16_TFLOPs"], 4)
    if not args.no_cpu:
        log("[bench] timing the CPU oracle")
        result["cpu_baseline"] = cpu_baseline(gpu, layers[0], pre, args.cpu_seconds)
    if not args.no_stack:
        for bw, ws_ in layers[1:]:
            for w in ws_[:7]:
                probe.release(gpu, w)  # room for the stack
        result["stack"] = []
        for v in STACK_VARIANTS:
            r = bench_stack(gpu, v)
            log(f"[bench] config-5 {v}: {r['us_per_token']} us/token over {STACK_LAYERS} layers, "
                f"{r['achieved_GBps']} GB/s")
            result["stack"].append(r)
    release_graphs()  # every batch above has completed (each one ends synchronised)
    print(json.dumps(result), flush=True)
    gpu.close()


if __name__ == "__main__":
    main()
