"""GPU parity of the whole MoE block (moe_block behind the C ABI) against the
CPU oracle on the benchmark configurations.

Protocol: the GPU's router logits are read back
and routed by the oracle; expert ids and the dispatch order must then be
bit-exact, and the F32-path output within max-abs 1e-4 of the oracle's
output max-abs norm.  The router product itself is checked separately
against the oracle's logits."""
import numpy as np
import pytest

import oracle
from helpers import (DENSE, HostBlock, close, config1, config2, config3, config4, config5, hot_bias,
                     pack_reference, rel_max_err, zipf_bias)
from hip_backend import (BF16, F16, F32, PATH_AUTO, PATH_GROUPED, PATH_MFMA, PATH_OPS, BlockWeights,
                         ShapeError, Tensor, synth)
from hip_backend.api import MoePackedWeightC, MoeRegionC, PackedWeight

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
BF16_TOL = 2e-2  # bf16-MFMA prefill path


def run_block(gpu, bw, x, T, path=PATH_AUTO, bias=None, norm_w=None, residual=False, ws_out=None):
    """One moe_block call; with `ws_out` (a dict) the workspace's words after
    the call are stored under "ws" for the in-block dispatch checks."""
    E, K, h = bw.experts, bw.k, bw.hidden
    xb = gpu.upload(x)
    out = gpu.zeros(T * h)
    ws = gpu.zeros(bw.workspace_elems(T))
    lo, io_, wo = gpu.zeros(T * E), gpu.zeros(T * K), gpu.zeros(T * K)
    bb = gpu.upload(bias) if bias is not None else None
    nb = gpu.upload(norm_w) if norm_w is not None else None
    with gpu.batch() as b:
        b.moe_block(bw, xb, out, T, ws, logit_bias=bb, logits_out=lo, ids_out=io_, weights_out=wo,
                    norm_weight=nb, norm_eps=1e-6, residual=residual, path=path)
    res = (gpu.read(out).reshape(T, h), gpu.read(lo).reshape(T, E),
           gpu.read_u32(io_).reshape(T, K), gpu.read(wo).reshape(T, K))
    if ws_out is not None:
        ws_out["ws"] = gpu.read_u32(ws)
    for buf in (xb, out, ws, lo, io_, wo, bb, nb):
        if buf is not None:
            gpu.release(buf)
    return res


def tile_schedule(offsets, tm):
    """(expert, first position) of every run of tm pairs of the non-empty
    segments, experts ascending (the work list the dispatch writes)."""
    out = []
    for e in range(len(offsets) - 1):
        for q in range(int(offsets[e]), int(offsets[e + 1]), tm):
            out.append((e, q))
    return np.array(out, np.uint32).reshape(-1, 2)


def check_in_block_dispatch(bw, T, ids, ws, tm=None):
    """The dispatch moe_block built inside its workspace against the
    oracle's stable counting sort (orc_dispatch) of the same ids: counts,
    offsets, perm and pos bit-exact; with `tm`, the work list of tm-pair runs
    too."""
    lay = bw.workspace_layout(T)
    E, K = bw.experts, bw.k
    counts, offsets, perm, pos = oracle.dispatch(ids, E)
    got = {n: ws[lay[n]:lay[n] + m] for n, m in (("counts", E), ("offsets", E + 1), ("perm", T * K),
                                                  ("pos", T * K))}
    assert np.array_equal(got["counts"], counts)
    assert np.array_equal(got["offsets"], offsets)
    assert np.array_equal(got["perm"], perm)
    assert np.array_equal(got["pos"], pos)
    if tm is not None:
        ref = tile_schedule(offsets, tm)
        n = int(ws[lay["ntiles"]])
        assert n == len(ref), (n, len(ref))
        assert np.array_equal(ws[lay["tiles"]:lay["tiles"] + 2 * n].reshape(-1, 2), ref)


def check_all_ids(blk, got, normalize=True):
    """Every token's ids (bit-exact) and weights: the oracle routes the
    GPU's logits of all T tokens (sampling.metal:1-36)."""
    _, logits, ids, wts = got
    ref_ids, ref_w = oracle.route_tokens(logits, blk.K, normalize)
    assert np.array_equal(ids, ref_ids)
    np.testing.assert_allclose(wts, ref_w, rtol=2e-6, atol=1e-9)


def check_against_oracle(blk, x, got, tokens=None, bias=None, tol=F32_TOL, norm_w=None,
                         residual=False, logit_tol=1e-5):
    out, logits, ids, wts = got
    T = x.shape[0]
    rows = range(T) if tokens is None else tokens
    xin = x
    if norm_w is not None:
        xin = np.stack([oracle.rms_norm(r, norm_w, 1e-6) for r in x])
    sel = np.array(list(rows))
    # router product vs the oracle's (independent of routing)
    ref_logits = oracle.matmul(blk.router, xin[sel], len(sel)).reshape(len(sel), -1)
    if bias is not None:
        ref_logits = ref_logits + bias[sel]
    assert rel_max_err(logits[sel], ref_logits) < logit_tol
    # routing + experts on the GPU's logits (many tokens: the expert-major
    # oracle, equal to the per-token one bit for bit)
    ref_out, _, ref_ids, ref_w = oracle.moe_block(blk.spec(), xin[sel], len(sel),
                                                  logits_in=logits[sel],
                                                  expert_major=len(sel) >= 64)
    assert np.array_equal(ids[sel], ref_ids)
    np.testing.assert_allclose(wts[sel], ref_w, rtol=2e-6, atol=1e-9)
    if residual:
        ref_out = x[sel] + ref_out
    err = rel_max_err(out[sel], ref_out)
    assert err <= tol, err
    return err


# ------------------------------------------------------------------ config 1 --
@pytest.mark.parametrize("kind", ["f32", "affine"])
@pytest.mark.parametrize("path", [PATH_AUTO, PATH_OPS, PATH_GROUPED])
def test_config1_fixture_all_paths(gpu, kind, path):
    import os
    print(f"[case] config1 {kind} path={path}", flush=True)
    blk, x = config1(kind)
    g = np.load(os.path.join(os.path.dirname(__file__), "golden",
                             "config1.npz" if kind == "f32" else "config1_affine.npz"))
    assert np.array_equal(x, g["x"])
    bw = blk.upload(gpu)
    got = run_block(gpu, bw, x, 4, path)
    check_against_oracle(blk, x, got)
    # and against the committed golden vectors (identical ids; same logits up to rounding)
    assert np.array_equal(got[2], g["ids"])
    assert rel_max_err(got[0], g["out"]) <= F32_TOL


# ------------------------------------------------------------------ config 2 --
@pytest.fixture(scope="module")
def c2(gpu):
    blk = config2()
    return blk, blk.upload(gpu)


def test_config2_decode_fused(gpu, c2):
    blk, bw = c2
    for seed in range(3):
        x = synth.normal(1000 + seed, 2048).reshape(1, 2048)
        print(f"[case] config2 fused seed={seed}", flush=True)
        check_against_oracle(blk, x, run_block(gpu, bw, x, 1, PATH_AUTO))


@pytest.mark.parametrize("levels", [5, 64])
def test_config2_decode_tied_logits(gpu, c2, levels):
    """Zero router plus a bias drawn from `levels` values: the logits are the
    bias exactly, full of ties.  Each gate/up wave selects its expert on its
    own, so the output only matches the oracle if every selection breaks the
    ties toward the lower index (5 levels: ~100 experts share the top value,
    more candidates than one wave ranks; 64 levels: ~8 per value)."""
    import copy
    blk, bw = c2
    zero = Tensor.dense([2048, 512], np.zeros(2048 * 512, np.float32))
    blk0 = copy.copy(blk)
    blk0.router = zero
    _, gate, up, down, shared, sgi = bw.keep
    bw0 = BlockWeights(gpu.weight_tensor(zero), gate, up, down, bw.k, True, shared, sgi)
    rng = np.random.default_rng(49 + levels)
    vals = np.linspace(-2.0, 2.0, levels).astype(np.float32)
    for seed in range(2):
        bias = vals[rng.integers(0, levels, 512)].reshape(1, 512)
        x = synth.normal(1500 + seed, 2048).reshape(1, 2048)
        print(f"[case] config2 tied logits levels={levels} seed={seed}", flush=True)
        got = run_block(gpu, bw0, x, 1, PATH_AUTO, bias=bias)
        assert np.array_equal(got[1], bias)
        check_against_oracle(blk0, x, got, bias=bias)


def test_config2_paths_agree(gpu, c2):
    blk, bw = c2
    x = synth.normal(1100, 2048).reshape(1, 2048)
    a = run_block(gpu, bw, x, 1, PATH_AUTO)
    o = run_block(gpu, bw, x, 1, PATH_OPS)
    g = run_block(gpu, bw, x, 1, PATH_GROUPED)
    for r in (o, g):
        assert np.array_equal(a[2], r[2])
        assert rel_max_err(a[0], r[0]) <= F32_TOL


def test_config2_batched_tokens(gpu, c2):
    blk, bw = c2
    x = synth.normal(1200, 8 * 2048).reshape(8, 2048)
    check_against_oracle(blk, x, run_block(gpu, bw, x, 8, PATH_AUTO))


def test_config2_graph_replay(gpu, c2):
    blk, bw = c2
    x = synth.normal(1300, 2048)
    xb = gpu.upload(x)
    out = gpu.zeros(2048)
    ws = gpu.zeros(bw.workspace_elems(1))
    eager = run_block(gpu, bw, x.reshape(1, -1), 1, PATH_AUTO)[0].ravel()
    cap = gpu.capture()
    with cap as b:
        b.moe_block(bw, xb, out, 1, ws)
    for i in range(3):
        gpu.clear(out)
        with gpu.batch() as b:
            b.graph(cap.graph)
        got = gpu.read(out)
        assert np.array_equal(got, eager), i
        run_block(gpu, bw, synth.normal(1400 + i, 2048).reshape(1, -1), 1)  # eager work between


def profiled(gpu, fn):
    gpu.profile_reset()
    gpu.profile(True)
    res = fn()
    prof = gpu.profile_read()
    gpu.profile(False)
    return res, prof


def test_profiling_names_kernels(gpu, c2):
    blk, bw = c2
    x = synth.normal(1500, 2048).reshape(1, 2048)
    _, prof = profiled(gpu, lambda: run_block(gpu, bw, x, 1, PATH_AUTO))
    for k in ("decode_pre", "decode_gateup", "decode_down"):
        assert k in prof and prof[k][0] == 1 and prof[k][1] > 0


def test_config2_decode_replays_follow_their_inputs(gpu, c2):
    """40 graph replays of the fused decode over 8 inputs written between the
    replays (every replay's routing and activations differ from the previous
    one's): each output equals the eager call on its input and is finite."""
    blk, bw = c2
    xs = [synth.normal(1600 + i, 2048) for i in range(8)]
    eager = [run_block(gpu, bw, x.reshape(1, -1), 1, PATH_AUTO)[0].ravel() for x in xs]
    xb = gpu.zeros(2048)
    out = gpu.zeros(2048)
    ws = gpu.zeros(bw.workspace_elems(1))
    cap = gpu.capture()
    with cap as b:
        b.moe_block(bw, xb, out, 1, ws)
    for i in range(40):
        gpu.write(xb, xs[i % 8])
        with gpu.batch() as b:
            b.graph(cap.graph)
        got = gpu.read(out)
        assert np.all(np.isfinite(got)), i
        assert np.array_equal(got, eager[i % 8]), i
    for buf in (xb, out, ws):
        gpu.release(buf)


# ------------------------------------------------------------------ config 3 --
@pytest.fixture(scope="module")
def c3(gpu):
    blk = config3()
    return blk, blk.upload(gpu)


@pytest.mark.parametrize("T", [1, 8, 32, 50, 64])
def test_config3_mixed_precision_hot_set(gpu, c3, T):
    """Config 3 through AUTO (fused decode at 1 token, the batched decode with
    the fused route + dispatch launch above): every token's ids and output
    against the oracle, and the dispatch and 8-pair work list built inside
    the block against orc_dispatch.  From 48 tokens the all-token products
    run over entries of 4 input rows; at 50 the last entry holds 2."""
    blk, bw = c3
    print(f"[case] config3 T={T}", flush=True)
    x = synth.normal(2000 + T, T * 2048).reshape(T, 2048)
    bias = hot_bias(T, 512, seed=T)
    wsd = {}
    got = run_block(gpu, bw, x, T, PATH_AUTO, bias=bias, ws_out=wsd)
    check_all_ids(blk, got)
    check_against_oracle(blk, x, got, bias=bias)
    if T > 1:
        check_in_block_dispatch(bw, T, got[2], wsd["ws"], tm=bw.workspace_layout(T)["tile_pairs_batched"])


def test_config3_batched_wide_range_inputs(gpu, c3):
    """The batched gate/up's 4-bit limb products (inputs block-scaled per
    32-element chunk) on inputs whose magnitudes span 2^-40 .. 2^40 inside a
    chunk, a token of zeros and a token of subnormals: ids and outputs
    against the oracle at the F32-path tolerance."""
    blk, bw = c3
    T = 8
    rng = np.random.default_rng(77)
    x = synth.normal(2400, T * 2048).reshape(T, 2048)
    x = (x * np.exp2(rng.integers(-40, 41, size=x.shape))).astype(np.float32)
    x[3] = 0.0
    x[5] = (synth.normal(2401, 2048) * np.float32(1e-39)).astype(np.float32)
    bias = hot_bias(T, 512, seed=11)
    got = run_block(gpu, bw, x, T, PATH_AUTO, bias=bias)
    assert np.all(np.isfinite(got[0]))
    check_all_ids(blk, got)
    check_against_oracle(blk, x, got, bias=bias)


def test_batched_limb_products_tiny_chunks(gpu):
    """The batched gate/up's 4-bit limb products on input chunks whose maximum
    lies below 2^-106 (every input about 2^-110, some subnormal), with gate/up
    scales and biases raised by 2^100 so the products stay normal and reach
    the output: ids and outputs against the oracle at the F32-path
    tolerance.  (A chunk scale of 2^(22-e) overflowed to infinity there.)"""
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": (8, 32, BF16), "shared_gate": DENSE}
    blk = HostBlock(256, 24, 4, 128, 64, kinds, seed=81, random_experts=True)
    for t in (blk.gate, blk.up):
        for a in (t.scales, t.biases):
            nz = (a & 0x7fff) != 0
            a[nz] = a[nz] + np.uint16(100 << 7)  # bf16 exponent + 100
    bw = blk.upload(gpu)
    T = 5
    x = (synth.normal(4700, T * 256) * np.float32(2.0 ** -110)).astype(np.float32).reshape(T, 256)
    x[2, :32] = (synth.normal(4701, 32) * np.float32(2.0 ** -135)).astype(np.float32)  # subnormals
    bias = hot_bias(T, 24, seed=3, frac=1.0, hot=4, boost=8.0)
    got = run_block(gpu, bw, x, T, PATH_AUTO, bias=bias)
    assert np.all(np.isfinite(got[0])) and np.abs(got[0]).max() > 1e-12
    check_all_ids(blk, got)
    check_against_oracle(blk, x, got, bias=bias)


@pytest.mark.parametrize("experts", [DENSE, (2, 32, BF16), (2, 128, F32), (4, 32, F16),
                                     (8, 64, F16), (8, 128, BF16)])
@pytest.mark.parametrize("T", [2, 5, 9])
def test_batched_decode_layouts(gpu, experts, T):
    """The batched decode kernels (AUTO with T >= 2 and short expert
    segments) over every code width and scale type, on rows whose chunk counts
    take the run-time lanes-per-row form (h 256, ff 128, shared ff 64) and a
    router of 24 rows (not a multiple of a wave's rows).  Every token gets a
    boost on two experts, so at T = 9 their segments span two 8-pair entries;
    odd T leaves a one-row run over the all-token products."""
    print(f"[case] batched experts={experts} T={T}", flush=True)
    kinds = {"router": DENSE if experts == DENSE else (8, 64, BF16), "experts": experts,
             "shared": DENSE if experts == DENSE else (8, 32, BF16), "shared_gate": DENSE}
    blk = HostBlock(256, 24, 4, 128, 64, kinds, seed=70 + T, random_experts=experts != DENSE)
    bw = blk.upload(gpu)
    x = synth.normal(4600 + T, T * 256).reshape(T, 256)
    bias = hot_bias(T, 24, seed=T, frac=1.0, hot=2, boost=8.0)
    gpu.profile_reset()
    gpu.profile(True)
    got = run_block(gpu, bw, x, T, PATH_AUTO, bias=bias)
    prof = gpu.profile_read()
    gpu.profile(False)
    for k in ("seg_router", "route_dispatch", "seg_gateup", "seg_down", "seg_shared_gateup",
              "seg_shared_down"):
        assert k in prof and prof[k][0] == 1, k
    check_against_oracle(blk, x, got, bias=bias)
    ref = run_block(gpu, bw, x, T, PATH_GROUPED, bias=bias)
    assert np.array_equal(got[2], ref[2])
    assert rel_max_err(got[0], ref[0]) <= F32_TOL


def test_route_dispatch_grids_in_sequence(gpu):
    """The fused route + dispatch launch counts its finished blocks on a
    device word that its last block puts back to zero: launches of 1, 18, 2
    and 1 blocks (T 3, 70, 6, 2) in a row each route and place exactly."""
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": (8, 32, BF16), "shared_gate": DENSE}
    blk = HostBlock(256, 24, 4, 128, 64, kinds, seed=91, random_experts=True)
    bw = blk.upload(gpu)
    for T in (3, 70, 6, 2):
        print(f"[case] route_dispatch sequence T={T}", flush=True)
        x = synth.normal(4700 + T, T * 256).reshape(T, 256)
        gpu.profile_reset()
        gpu.profile(True)
        got = run_block(gpu, bw, x, T, PATH_AUTO)
        prof = gpu.profile_read()
        gpu.profile(False)
        assert "route_dispatch" in prof, T
        check_against_oracle(blk, x, got)
        ref = run_block(gpu, bw, x, T, PATH_GROUPED)
        assert np.array_equal(got[2], ref[2])
        assert rel_max_err(got[0], ref[0]) <= F32_TOL


@pytest.mark.parametrize("shared", [0, 2048])
def test_decode_long_down_rows(gpu, shared):
    """Fused decode with 2048-wide down rows (ff 2048, K 8): the activation
    slots of the down kernel's waves would exceed its LDS share, so each wave
    loads its activation row directly."""
    print(f"[case] decode ff 2048 shared={shared}", flush=True)
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": (4, 64, BF16), "shared_gate": DENSE}
    blk = HostBlock(256, 16, 8, 2048, shared, kinds, seed=90 + (shared > 0), random_experts=True)
    bw = blk.upload(gpu)
    for seed in range(2):
        x = synth.normal(5100 + seed, 256).reshape(1, 256)
        got = run_block(gpu, bw, x, 1, PATH_AUTO)
        check_against_oracle(blk, x, got)
        ref = run_block(gpu, bw, x, 1, PATH_GROUPED)
        assert np.array_equal(got[2], ref[2])
        assert rel_max_err(got[0], ref[0]) <= F32_TOL


@pytest.mark.parametrize("E,shared", [(1100, 0), (1100, 128)])
def test_decode_many_experts(gpu, E, shared):
    """The fused decode past 1024 experts, where every routing wave keeps the
    logits in its LDS: ids, weights and output against the oracle and the
    grouped path."""
    print(f"[case] decode E={E} shared={shared}", flush=True)
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": (4, 64, BF16), "shared_gate": DENSE}
    blk = HostBlock(256, E, 8, 128, shared, kinds, seed=96 + (shared > 0), random_experts=True)
    bw = blk.upload(gpu)
    x = synth.normal(5150 + shared, 256).reshape(1, 256)
    got, prof = profiled(gpu, lambda: run_block(gpu, bw, x, 1, PATH_AUTO))
    assert all(k in prof for k in ("decode_pre", "decode_gateup", "decode_down")), sorted(prof)
    check_against_oracle(blk, x, got)
    ref = run_block(gpu, bw, x, 1, PATH_GROUPED)
    assert np.array_equal(got[2], ref[2])
    assert rel_max_err(got[0], ref[0]) <= F32_TOL


@pytest.mark.parametrize("E,K,normalize,ffs", [(64, 1, True, 128), (32, 32, False, 0), (100, 7, False, 128)])
@pytest.mark.parametrize("T", [1, 5, 300])
def test_routing_edges_every_path(gpu, E, K, normalize, ffs, T):
    """Top-1, top-E (every expert selected), an expert count that is no power
    of two, and unnormalised routing weights, through the fused decode (T 1),
    the batched decode (T 5) and the bf16-MFMA path (T 300)."""
    print(f"[case] routing edges E={E} K={K} normalize={normalize} ffs={ffs} T={T}", flush=True)
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": (4, 64, BF16), "shared_gate": DENSE}
    blk = HostBlock(256, E, K, 128, ffs, kinds, seed=E + K, normalize=normalize, random_experts=True)
    bw = blk.upload(gpu)
    x = synth.normal(5200 + E + T, T * 256).reshape(T, 256)
    got = run_block(gpu, bw, x, T, PATH_AUTO)
    if T == 300:
        check_against_oracle(blk, x, got, tol=BF16_TOL)
    else:
        check_against_oracle(blk, x, got)
        ref = run_block(gpu, bw, x, T, PATH_GROUPED)
        assert np.array_equal(got[2], ref[2])
        assert rel_max_err(got[0], ref[0]) <= F32_TOL


def test_config3_batched_graph_replay(gpu, c3):
    """The batched decode with its shared expert forked onto the side stream,
    captured into a graph and replayed (eager work between replays): every
    replay equals the eager result bit for bit."""
    blk, bw = c3
    T = 8
    x = synth.normal(2100, T * 2048)
    bias = hot_bias(T, 512, seed=21)
    eager = run_block(gpu, bw, x.reshape(T, -1), T, PATH_AUTO, bias=bias)[0].ravel()
    xb, bb = gpu.upload(x), gpu.upload(bias)
    out = gpu.zeros(T * 2048)
    ws = gpu.zeros(bw.workspace_elems(T))
    cap = gpu.capture()
    with cap as b:
        b.moe_block(bw, xb, out, T, ws, logit_bias=bb)
    for i in range(3):
        gpu.clear(out)
        with gpu.batch() as b:
            b.graph(cap.graph)
        assert np.array_equal(gpu.read(out), eager), i
        run_block(gpu, bw, synth.normal(2200 + i, T * 2048).reshape(T, -1), T, PATH_AUTO,
                  bias=hot_bias(T, 512, seed=30 + i))
    for buf in (xb, bb, out, ws):
        gpu.release(buf)


# ------------------------------------------------------------------ config 5 --
@pytest.fixture(scope="module")
def c5(gpu):
    """Config-5 layers by variant, generated and uploaded once per module."""
    cache = {}

    def get(variant):
        if variant not in cache:
            blk = config5(variant)
            cache[variant] = (blk, blk.upload(gpu))
        return cache[variant]
    return get


@pytest.mark.parametrize("variant", ["2bit", "8bit"])
def test_config5_layer_norm_residual(gpu, c5, variant):
    print(f"[case] config5 {variant}", flush=True)
    blk, bw = c5(variant)
    nw = (1.0 + 0.1 * synth.normal(3000, 2048)).astype(np.float32)
    x = synth.normal(3001, 2048).reshape(1, 2048)
    got = run_block(gpu, bw, x, 1, PATH_AUTO, norm_w=nw, residual=True)
    check_against_oracle(blk, x, got, norm_w=nw, residual=True)
    got_g = run_block(gpu, bw, x, 1, PATH_GROUPED, norm_w=nw, residual=True)
    assert np.array_equal(got[2], got_g[2])
    assert rel_max_err(got_g[0], got[0]) <= F32_TOL


@pytest.mark.parametrize("variant", ["2bit", "8bit"])
def test_config5_stack_chain(gpu, c5, variant):
    """All 48 layers of the config-5 stack (RMSNorm -> MoE block -> residual,
    execute.rs:196-197,236), chained in place on the GPU in one batch, against
    the oracle's stack (orc_moe_stack) on the same input: the error after the
    full depth.  The layers share the expert weights and differ in their
    norm weights, so every layer routes differently."""
    print(f"[case] config5 stack {variant} 48 layers", flush=True)
    blk, bw = c5(variant)
    nws = [(1.0 + 0.3 * synth.normal(3100 + l, 2048)).astype(np.float32) for l in range(48)]
    x = synth.normal(3200, 2048).reshape(1, 2048)
    h = gpu.upload(x)
    ws = gpu.zeros(bw.workspace_elems(1))
    nbs = [gpu.upload(n) for n in nws]
    with gpu.batch() as b:
        for nb in nbs:
            b.moe_block(bw, h, h, 1, ws, norm_weight=nb, norm_eps=1e-6, residual=True)
    got = gpu.read(h).reshape(1, 2048)
    ref = oracle.moe_stack([blk.spec()] * 48, nws, 1e-6, x, 1)
    err = rel_max_err(got, ref)
    print(f"[case] config5 stack {variant} 48 layers rel err {err:.3e}", flush=True)
    assert err <= F32_TOL
    # the stack moved the hidden state: the check is not of the input alone
    assert rel_max_err(ref, x) > 0.1
    for buf in (h, ws, *nbs):
        gpu.release(buf)


def test_mlx_checkpoint_layer(gpu, tmp_path):
    """A synthetic MLX checkpoint (sharded SafeTensors, 8-bit router, 4-bit
    experts and shared expert, bf16 norm) loaded by hip_backend.mlx and run
    through moe_block with its norm and the residual, decode and batched."""
    import oracle as orc
    from hip_backend.mlx import MoeCheckpoint
    from mlx_fixture import make_checkpoint
    make_checkpoint(str(tmp_path), layers=1, shards=2)
    ck = MoeCheckpoint(str(tmp_path))
    bw, nb = ck.upload(gpu, 0)
    L = ck.layers[0]

    class Spec:
        router = L["router"]

        @staticmethod
        def spec():
            return orc.MoeSpec(L["router"], L["gate"], L["up"], L["down"], ck.experts_used,
                               ck.normalize, (L["shared_gate"], L["shared_up"], L["shared_down"]),
                               L["shared_gate_inp"])
    nw = gpu.read(nb)
    for T in (1, 3):
        print(f"[case] mlx checkpoint T={T}", flush=True)
        x = synth.normal(3300 + T, T * 256).reshape(T, 256)
        got = run_block(gpu, bw, x, T, PATH_AUTO, norm_w=nw, residual=True)
        check_against_oracle(Spec, x, got, norm_w=nw, residual=True)
    gpu.release(nb)


def test_in_place_residual_stream(gpu, c2):
    blk, bw = c2
    x = synth.normal(3100, 2048)
    hb = gpu.upload(x)
    ws = gpu.zeros(bw.workspace_elems(1))
    with gpu.batch() as b:
        b.moe_block(bw, hb, hb, 1, ws, residual=True)
    ref = run_block(gpu, bw, x.reshape(1, -1), 1, PATH_AUTO)[0].ravel()
    close(gpu.read(hb), x + ref, 1e-6)


# ------------------------------------------------------- config 4 (MFMA) --
@pytest.fixture(scope="module")
def c4(gpu):
    blk = config4()
    return blk, blk.upload(gpu)


@pytest.mark.parametrize("packed", [False, True])
def test_config4_prefill_mfma_zipf(gpu, c4, packed):
    """Config 4 at its real size (4096 tokens, E 128, top 8, ff 768, 4-bit g64
    bf16, Zipf(1.1) skew) through AUTO (the bf16 MFMA path), over the
    row-major tensors and over the MFMA tile-order copies the benchmark
    makes (moe_pack_weight): every token's ids and weights against the
    oracle's routing of the GPU logits, the dispatch and the 128-pair M-tile
    list built inside the block against orc_dispatch, every token's output
    against the oracle (bf16 tolerance), and the packed run equal to the
    row-major run bit for bit on every token."""
    blk, bw = c4
    T = 4096
    if packed:
        router, gate, up, down = bw.keep[:4]
        bw = BlockWeights(router, gate, up, down, bw.k, True,
                          packed=[gpu.pack_weight(w) for w in (gate, up, down)])
    print(f"[case] config4 prefill T=4096 packed={packed} (auto -> bf16 MFMA)", flush=True)
    x = synth.normal(4000, T * 2048).reshape(T, 2048)
    bias = zipf_bias(T, 128, seed=4)
    wsd = {}
    got = run_block(gpu, bw, x, T, PATH_AUTO, bias=bias, ws_out=wsd)
    check_all_ids(blk, got)
    check_in_block_dispatch(bw, T, got[2], wsd["ws"], tm=bw.workspace_layout(T)["tile_pairs_mfma"])
    err = check_against_oracle(blk, x, got, bias=bias, tol=BF16_TOL)
    print(f"[case] config4 packed={packed} rel err {err:.3e} (all {T} tokens)", flush=True)
    counts = np.bincount(got[2].ravel(), minlength=128)
    assert counts.max() > 8 * counts.mean()  # the Zipf skew is realised
    if packed:
        ref = run_block(gpu, c4[1], x, T, PATH_AUTO, bias=bias)
        assert np.array_equal(got[2], ref[2])
        assert np.array_equal(got[0], ref[0])
        for pw in bw.packed:
            for b in pw.buffers:
                gpu.release(b)


@pytest.mark.parametrize("T", [33, 32768])
def test_config4_prefill_sizes(gpu, c4, T):
    """Prefill at a ragged token count (partial M-tiles everywhere) and at
    32768 tokens, where the router GEMM runs unsplit (its tiles alone fill the
    grid), so it adds the bias itself and the routing reads plain logits; the
    dispatch places 262144 pairs.  Every token against the oracle."""
    blk, bw = c4
    print(f"[case] config4 prefill T={T}", flush=True)
    x = synth.normal(4300 + T, T * 2048).reshape(T, 2048)
    bias = zipf_bias(T, 128, seed=5)
    got = run_block(gpu, bw, x, T, PATH_MFMA, bias=bias)
    err = check_against_oracle(blk, x, got, bias=bias, tol=BF16_TOL)
    print(f"[case] config4 T={T} rel err {err:.3e}", flush=True)


@pytest.mark.parametrize("bits,group,st", [(2, 32, BF16), (2, 128, F32), (4, 32, F16), (4, 128, F32),
                                           (8, 32, F32), (8, 64, F16), (8, 128, BF16)])
def test_mfma_experts_all_affine_layouts(gpu, bits, group, st):
    """bf16-MFMA expert products over every code width and scale type (h 256,
    8 experts, top 2, ff 128, 300 tokens).  The skewed routing gives M-tiles
    (128 pairs) with one, two, three and four live 32-row slices."""
    print(f"[case] MFMA experts bits={bits} group={group} st={st}", flush=True)
    blk = HostBlock(256, 8, 2, 128, 0, {"router": DENSE, "experts": (bits, group, st)},
                    seed=60 + bits, random_experts=True)
    bw = blk.upload(gpu)
    T = 300
    x = synth.normal(4400 + bits, T * 256).reshape(T, 256)
    bias = zipf_bias(T, 8, seed=0, s=0.5)
    got = run_block(gpu, bw, x, T, PATH_MFMA, bias=bias)
    slices = {(min(c - m, 128) + 31) // 32 for c in np.bincount(got[2].ravel(), minlength=8)
              for m in range(0, int(c), 128)}
    assert slices >= {1, 2, 3, 4}
    check_against_oracle(blk, x, got, bias=bias, tol=BF16_TOL)


@pytest.mark.parametrize("dims,bits,group,st", [([256, 40, 3], 2, 128, F16), ([256, 64, 2], 4, 64, BF16),
                                                 ([128, 96, 2], 8, 32, BF16), ([384, 33, 1], 4, 32, F16)])
def test_pack_weight_layout(gpu, dims, bits, group, st):
    """moe_pack_weight writes the documented MFMA tile-order layout (compared
    word for word with its numpy restatement), rows past `out` zero."""
    print(f"[case] pack layout dims={dims} bits={bits} group={group}", flush=True)
    t = Tensor.affine(dims, *synth.random_affine(7700 + bits, int(np.prod(dims)), bits, group, st), bits,
                      group, st)
    pw = gpu.pack_weight(gpu.weight_tensor(t))
    codes, scales, biases = pack_reference(t)
    assert np.array_equal(gpu.read(pw.buffers[0]).view(np.uint32), codes)
    assert np.array_equal(gpu.read(pw.buffers[1]).view(np.uint16), scales)
    assert np.array_equal(gpu.read(pw.buffers[2]).view(np.uint16), biases)


def test_packed_weights_are_validated(gpu):
    """moe_pack_weight and moe_block refuse packed copies that do not fit:
    wrong region sizes, an output overlapping the weight, a gate copy without
    the up copy, and weights without a packed form (F32 scales)."""
    def tensor(dims, st, seed):
        return Tensor.affine(dims, *synth.random_affine(seed, int(np.prod(dims)), 4, 64, st), 4, 64, st)

    gate = gpu.weight_tensor(tensor([256, 128, 4], BF16, 1))
    up = gpu.weight_tensor(tensor([256, 128, 4], BF16, 2))
    down = gpu.weight_tensor(tensor([128, 256, 4], BF16, 3))
    router = gpu.weight_f32(synth.normal(4, 256 * 4), [256, 4])
    pg, pu = gpu.pack_weight(gate), gpu.pack_weight(up)
    # a region one element short
    c = MoePackedWeightC.from_buffer_copy(pg.c)
    c.data.bytes -= 4
    with pytest.raises(ShapeError):
        with gpu.batch() as b:
            b.pack_weight(gate, PackedWeight(c, pg.buffers))
    # the copy written over the weight itself
    c = MoePackedWeightC.from_buffer_copy(pg.c)
    c.data = MoeRegionC(gate.c.data.ptr, c.data.bytes)
    with pytest.raises(ShapeError):
        with gpu.batch() as b:
            b.pack_weight(gate, PackedWeight(c, pg.buffers))
    # gate copy without the up copy, and a down copy one element short in the block
    x = gpu.upload(synth.normal(5, 300 * 256))
    out = gpu.zeros(300 * 256)
    pd = gpu.pack_weight(down)
    c = MoePackedWeightC.from_buffer_copy(pd.c)
    c.scales.bytes -= 4
    for packed in ([pg, None, None], [pg, pu, PackedWeight(c, pd.buffers)]):
        bwp = BlockWeights(router, gate, up, down, 2, True, packed=packed)
        ws = gpu.zeros(bwp.workspace_elems(300))
        with pytest.raises(ShapeError):
            with gpu.batch() as b:
                b.moe_block(bwp, x, out, 300, ws, path=PATH_MFMA)
        gpu.release(ws)
    # F32 scales have no packed form
    f32s = gpu.weight_tensor(tensor([256, 128, 4], F32, 6))
    assert gpu.pack_weight(f32s) is None


@pytest.mark.parametrize("bits,group,st", [(2, 32, BF16), (4, 64, F16), (4, 128, BF16), (8, 64, BF16),
                                           (8, 128, F16)])
def test_mfma_packed_matches_unpacked(gpu, bits, group, st):
    """The MFMA path over packed copies of gate/up/down computes exactly what
    it computes over the row-major tensors (same products, same order), and
    both match the oracle to the bf16 tolerance."""
    print(f"[case] MFMA packed bits={bits} group={group} st={st}", flush=True)
    blk = HostBlock(256, 8, 2, 128, 0, {"router": DENSE, "experts": (bits, group, st)},
                    seed=80 + bits, random_experts=True)
    bw = blk.upload(gpu)
    router, gate, up, down = bw.keep[:4]
    packed = [gpu.pack_weight(w) for w in (gate, up, down)]
    assert all(p is not None for p in packed)
    bwp = BlockWeights(router, gate, up, down, bw.k, True, packed=packed)
    T = 300
    x = synth.normal(4500 + bits, T * 256).reshape(T, 256)
    bias = zipf_bias(T, 8, seed=1, s=0.5)
    got = run_block(gpu, bw, x, T, PATH_MFMA, bias=bias)
    gotp = run_block(gpu, bwp, x, T, PATH_MFMA, bias=bias)
    assert np.array_equal(got[2], gotp[2])
    assert np.array_equal(got[0], gotp[0])
    check_against_oracle(blk, x, gotp, bias=bias, tol=BF16_TOL)


def test_mfma_path_with_shared_expert(gpu, c2):
    blk, bw = c2
    T = 256
    print("[case] config2 shapes T=256 forced MFMA", flush=True)
    x = synth.normal(4100, T * 2048).reshape(T, 2048)
    got = run_block(gpu, bw, x, T, PATH_MFMA)
    check_against_oracle(blk, x, got, tol=BF16_TOL)


def test_mfma_path_8bit_router_norm_residual(gpu, c3):
    blk, bw = c3
    T = 64
    x = synth.normal(4200, T * 2048).reshape(T, 2048)
    nw = (1.0 + 0.1 * synth.normal(4201, 2048)).astype(np.float32)
    bias = hot_bias(T, 512, seed=7)
    got = run_block(gpu, bw, x, T, PATH_MFMA, bias=bias, norm_w=nw, residual=True)
    check_against_oracle(blk, x, got, bias=bias, tol=BF16_TOL,
                         norm_w=nw, residual=True)


@pytest.mark.parametrize("E,T,path", [(1024, 1024, PATH_MFMA), (1100, 5, PATH_AUTO), (1100, 40, PATH_GROUPED)])
def test_dispatch_fallbacks_in_block(gpu, E, T, path):
    """Expert counts whose dispatch histograms exceed the single-launch
    dispatch's LDS ((2 + 16) * E words > 48 KiB for E > 682): the MFMA path
    and the batched decode (which, past 1024 experts, also leaves the fused
    route + dispatch) take the three-launch dispatch plus the separate
    work-list kernel; the VALU grouped path the three launches alone.  Ids,
    dispatch and work list against the oracle, every token's output too."""
    print(f"[case] dispatch fallback E={E} T={T} path={path}", flush=True)
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": (4, 64, BF16), "shared_gate": DENSE}
    blk = HostBlock(256, E, 8, 128, 128, kinds, seed=95, random_experts=True)
    bw = blk.upload(gpu)
    x = synth.normal(5300 + T, T * 256).reshape(T, 256)
    # a hot set of 8 experts for half of the tokens: some segments span several tiles
    bias = hot_bias(T, E, seed=E + T, frac=0.5, hot=8, boost=6.0)
    wsd = {}
    gpu.profile_reset()
    gpu.profile(True)
    got = run_block(gpu, bw, x, T, path, bias=bias, ws_out=wsd)
    prof = gpu.profile_read()
    gpu.profile(False)
    assert "dispatch_place" in prof, sorted(prof)
    lay = bw.workspace_layout(T)
    tm = {PATH_MFMA: lay["tile_pairs_mfma"], PATH_AUTO: lay["tile_pairs_batched"], PATH_GROUPED: None}[path]
    if tm is not None:
        assert "tile_schedule" in prof, sorted(prof)
    check_all_ids(blk, got)
    check_in_block_dispatch(bw, T, got[2], wsd["ws"], tm=tm)
    tol = BF16_TOL if path == PATH_MFMA else F32_TOL
    check_against_oracle(blk, x, got, bias=bias, tol=tol,
                         logit_tol=1e-5)


@pytest.mark.parametrize("T", [300, 2048])
def test_grouped_and_mfma_dispatch_in_block(gpu, c4, T):
    """The single-launch dispatch inside the MFMA path and the VALU grouped
    path (config-4 shapes): dispatch bit-exact against orc_dispatch, the
    M-tile list against its numpy schedule."""
    blk, bw = c4
    x = synth.normal(4700 + T, T * 2048).reshape(T, 2048)
    bias = zipf_bias(T, 128, seed=6)
    for path in (PATH_MFMA, PATH_GROUPED):
        print(f"[case] in-block dispatch T={T} path={path}", flush=True)
        wsd = {}
        got = run_block(gpu, bw, x, T, path, bias=bias, ws_out=wsd)
        check_all_ids(blk, got)
        tm = bw.workspace_layout(T)["tile_pairs_mfma"] if path == PATH_MFMA else None
        check_in_block_dispatch(bw, T, got[2], wsd["ws"], tm=tm)


def bf16_rne_bits(v):
    """float32 -> bf16 bits, rounded to nearest even (no NaNs in the inputs)."""
    u = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("norm", [False, True])
def test_mfma_bf16_input_copy(gpu, c4, norm):
    """The bf16 copy of the block input the expert GEMMs multiply: without a
    norm weight the router product writes it while it stages x; with one, the
    norm kernel does.  Both bit-exact against round-to-nearest-even of x (of
    RMSNorm(x) as the oracle computes it, to one bf16 step, with the norm)."""
    blk, bw = c4
    T, h = 300, 2048
    x = synth.normal(6100 + norm, T * h).reshape(T, h)
    nw = (1.0 + 0.1 * synth.normal(6110, h)).astype(np.float32) if norm else None
    wsd = {}
    run_block(gpu, bw, x, T, PATH_MFMA, norm_w=nw, ws_out=wsd)
    lay = bw.workspace_layout(T)
    got = wsd["ws"][lay["xb16"]:lay["xb16"] + T * h // 2].view(np.uint16).reshape(T, h)
    if not norm:
        assert np.array_equal(got, bf16_rne_bits(x))
    else:
        ref = np.stack([oracle.rms_norm(r, nw, 1e-6) for r in x])
        diff = np.abs(got.astype(np.int32) - bf16_rne_bits(ref).astype(np.int32))
        assert diff.max() <= 1, diff.max()


def test_config4_routing_matches_oracle_f32_logits(gpu, c4):
    """The prefill path routes on F32 router products: its logits of all
    4096 tokens agree with the oracle's own F32 logits (orc_matmul, the
    decoded router times x) to F32 accuracy, and its ids equal the oracle's
    routing of the oracle's logits on every token whose top K+1 logits are
    separated by more than twice that token's logit difference (only those
    can have their order changed by summation order).  The near-tie tokens
    are counted: at most 0.1% of them.  (bf16 router products differ by
    ~1e-2 and change the expert set of 1-2% of the tokens.)"""
    blk, bw = c4
    T, K = 4096, blk.K
    x = synth.normal(4000, T * 2048).reshape(T, 2048)
    bias = zipf_bias(T, 128, seed=4)
    print("[case] config4 routing vs oracle F32 logits", flush=True)
    got = run_block(gpu, bw, x, T, PATH_AUTO, bias=bias)
    ref_logits = oracle.matmul(blk.router, x, T).reshape(T, 128) + bias
    diff = np.abs(got[1].astype(np.float64) - ref_logits)
    scale = np.abs(ref_logits).max()
    assert diff.max() <= 1e-5 * scale, diff.max() / scale
    ref_ids, ref_w = oracle.route_tokens(ref_logits, K, True)
    top = -np.sort(-ref_logits, axis=1)[:, :K + 1].astype(np.float64)
    gap = np.min(top[:, :-1] - top[:, 1:], axis=1)
    clear = gap > 2 * diff.max(axis=1)
    print(f"[case] config4 routing: {int((~clear).sum())} near-tie tokens, max logit diff "
          f"{diff.max():.3e}", flush=True)
    assert (~clear).sum() <= T // 1000
    assert np.array_equal(got[2][clear], ref_ids[clear])
    np.testing.assert_allclose(got[3][clear], ref_w[clear], rtol=1e-5, atol=1e-8)


@pytest.mark.parametrize("gate_kind,packed,norm,T", [(DENSE, "all", False, 300), (DENSE, "routed", True, 300),
                                                     (DENSE, "none", False, 2048), ((8, 64, BF16), "all", True, 130),
                                                     (DENSE, "shared", False, 64)])
def test_mfma_path_shared_expert_folded(gpu, gate_kind, packed, norm, T):
    """A shared expert of the routed experts' kind and width runs as one more
    segment of the routed experts' bf16 GEMMs (its rows after the T*K pairs,
    spread over the item order), with no side stream, identity schedule or
    separate shared GEMMs; a dense F32 gate row is multiplied inside the
    router's pass over x (partial sums per K range), other gate kinds keep
    their one-row product.  Every token against the oracle at the bf16
    tolerance, with and without packed copies (of the routed experts, of the
    shared expert, of both), the RMSNorm input path and the residual; the
    packed runs equal the row-major run bit for bit."""
    print(f"[case] MFMA shared folded gate={gate_kind} packed={packed} norm={norm} T={T}", flush=True)
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": (4, 64, BF16), "shared_gate": gate_kind}
    blk = HostBlock(256, 16, 4, 128, 128, kinds, seed=107, random_experts=True)
    bw = blk.upload(gpu)
    router, gate, up, down, shared, sg = bw.keep
    pk = [gpu.pack_weight(w) for w in (gate, up, down)] if packed in ("all", "routed") else None
    spk = [gpu.pack_weight(w) for w in shared] if packed in ("all", "shared") else None
    bwp = BlockWeights(router, gate, up, down, bw.k, True, shared, sg, packed=pk, shared_packed=spk)
    x = synth.normal(5500 + T, T * 256).reshape(T, 256)
    nw = (1.0 + 0.1 * synth.normal(5501, 256)).astype(np.float32) if norm else None
    bias = hot_bias(T, 16, seed=T, frac=0.5, hot=3, boost=4.0)
    gpu.profile_reset()
    gpu.profile(True)
    got = run_block(gpu, bwp, x, T, PATH_MFMA, bias=bias, norm_w=nw, residual=True)
    prof = gpu.profile_read()
    gpu.profile(False)
    for name in ("gemm_shared_gateup", "gemm_shared_down", "identity_schedule"):
        assert name not in prof, sorted(prof)
    assert ("gemv_row1" in prof) == (gate_kind != DENSE), sorted(prof)
    check_all_ids(blk, got)
    check_against_oracle(blk, x, got, bias=bias, tol=BF16_TOL, norm_w=nw, residual=True)
    if packed != "none":
        ref = run_block(gpu, bw, x, T, PATH_MFMA, bias=bias, norm_w=nw, residual=True)
        assert np.array_equal(got[2], ref[2])
        assert np.array_equal(got[0], ref[0])
    for pw in (pk or []) + (spk or []):
        for b in pw.buffers:
            gpu.release(b)


def test_packed_shared_copies_are_validated(gpu):
    """moe_block refuses packed shared-expert copies without a shared expert,
    or a shared gate copy without the shared up copy."""
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": (4, 64, BF16), "shared_gate": DENSE}
    blk = HostBlock(256, 8, 2, 128, 128, kinds, seed=108, random_experts=True)
    bw = blk.upload(gpu)
    router, gate, up, down, shared, sg = bw.keep
    spk = [gpu.pack_weight(w) for w in shared]
    x = gpu.upload(synth.normal(5600, 64 * 256))
    out = gpu.zeros(64 * 256)
    for bad in (BlockWeights(router, gate, up, down, 2, True, shared_packed=spk),
                BlockWeights(router, gate, up, down, 2, True, shared, sg, shared_packed=[spk[0], None, spk[2]])):
        ws = gpu.zeros(bad.workspace_elems(64))
        with pytest.raises(ShapeError):
            with gpu.batch() as b:
                b.moe_block(bad, x, out, 64, ws, path=PATH_MFMA)
        gpu.release(ws)
    for pw in spk:
        for b in pw.buffers:
            gpu.release(b)


@pytest.mark.parametrize("shared,ffs,on_gemm", [((8, 32, BF16), 256, True), ((4, 64, F16), 256, True),
                                                (DENSE, 256, True), ((4, 64, BF16), 192, False)])
def test_mfma_path_shared_expert_kinds(gpu, shared, ffs, on_gemm):
    """The MFMA path runs the shared expert as one all-token segment of the
    grouped bf16 GEMM when the GEMM takes its kinds (affine or dense, gate
    and up alike, K of both products a multiple of 128), and keeps the
    per-token products otherwise (a shared width of 192); both against the
    oracle at the bf16 tolerance, with the shared gate and the residual."""
    print(f"[case] MFMA shared kind={shared} ffs={ffs}", flush=True)
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": shared, "shared_gate": DENSE}
    blk = HostBlock(256, 16, 4, 128, ffs, kinds, seed=101, random_experts=True)
    bw = blk.upload(gpu)
    T = 300
    x = synth.normal(5400, T * 256).reshape(T, 256)
    gpu.profile_reset()
    gpu.profile(True)
    got = run_block(gpu, bw, x, T, PATH_MFMA, residual=True)
    prof = gpu.profile_read()
    gpu.profile(False)
    assert ("gemm_shared_gateup" in prof) == on_gemm and ("gemm_shared_down" in prof) == on_gemm, sorted(prof)
    check_all_ids(blk, got)
    check_against_oracle(blk, x, got, tol=BF16_TOL, residual=True)
