"""Pins the CPU oracle (oracle/moe_oracle.c) against the reference's own
known-answer tests and against independent closed forms, so a plausible
mistake (dropped term, wrong index, wrong tie order, transposed operand)
fails here.  CPU only."""
import itertools
import math

import numpy as np
import pytest

import oracle
from hip_backend import BF16, F16, F32, Tensor, synth
from helpers import DENSE, HostBlock, config1


# ------------------------------------------------------------------ dtypes --
def test_scale_bit_patterns_kat():
    # crates/metal-backend/tests/affine.rs:16-27 writes these exact patterns
    for bits, val in [(0x3000, 0.125), (0x3400, 0.25), (0xB800, -0.5), (0xB400, -0.25)]:
        assert oracle.f16_to_f32(bits) == val
    for bits, val in [(0x3E00, 0.125), (0x3E80, 0.25), (0xBF00, -0.5), (0xBE80, -0.25)]:
        assert oracle.bf16_to_f32(bits) == val


def test_f16_decode_exhaustive_vs_numpy():
    L = oracle.lib()
    allh = np.arange(65536, dtype=np.uint16)
    ref = allh.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(h)) for h in allh], np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f32_to_f16_and_bf16_rounding():
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-8, 5, 4000),
                           np.array([0.0, -0.0, 65504, 65520, 1e-8, 6e-8, 2.0 ** -24, np.inf, -np.inf],
                                    np.float32)]).astype(np.float32)
    for v in vals:
        with np.errstate(over="ignore"):
            ref16 = np.float32(v).astype(np.float16).view(np.uint16)
        assert oracle.f32_to_f16(v) == ref16
    # bf16: round-to-nearest-even on the upper 16 bits (independent integer form)
    for v in vals:
        b = int(np.float32(v).view(np.uint32))
        upper, rem = b >> 16, b & 0xFFFF
        exp = upper + (1 if rem > 0x8000 or (rem == 0x8000 and upper & 1) else 0)
        assert oracle.f32_to_bf16(v) == (exp & 0xFFFF)


# ------------------------------------------------------------------ decode --
def test_affine_decode_kat_mlx_loader():
    # crates/model-format/tests/mlx.rs:39-99: words 0x11111111 (every 4-bit code 1),
    # group 32, F32 scale 0.5 / bias -0.25, dims [64, 3] -> 192 x 0.25
    t = Tensor.affine([64, 3], np.full(24, 0x11111111, np.uint32), np.full(6, 0.5, np.float32),
                      np.full(6, -0.25, np.float32), 4, 32, F32)
    assert (oracle.decode(t) == 0.25).all()


def _numpy_decode(t):
    per = 32 // t.bits
    n = t.elements()
    i = np.arange(n)
    codes = (t.data[i // per] >> ((i % per) * t.bits).astype(np.uint32)) & ((1 << t.bits) - 1)
    if t.scale_type == F32:
        s, b = t.scales.astype(np.float64), t.biases.astype(np.float64)
    elif t.scale_type == F16:
        s, b = t.scales.view(np.float16).astype(np.float64), t.biases.view(np.float16).astype(np.float64)
    else:
        s = synth.bf16_bits_to_f32(t.scales).astype(np.float64)
        b = synth.bf16_bits_to_f32(t.biases).astype(np.float64)
    return codes * s[i // t.group_size] + b[i // t.group_size]


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("st", [F32, F16, BF16])
def test_affine_pattern_decode_all_layouts(bits, group, st):
    # the 27 layouts of crates/metal-backend/tests/affine.rs:53-89 on its pattern
    n = 256 * 19
    packed, s, b = oracle.affine_pattern(n, bits, group, st)
    t = Tensor.affine([256, 19], packed, s, b, bits, group, st)
    got = oracle.decode(t)
    ref = _numpy_decode(t)
    assert np.array_equal(got.astype(np.float64), ref)  # exact: code*s+b is exact here
    # the code sequence is the reference's (i*37 + i/13) & mask
    i = np.arange(n)
    codes = (t.data[i // (32 // bits)] >> ((i % (32 // bits)) * bits).astype(np.uint32)) & ((1 << bits) - 1)
    assert np.array_equal(codes, (i * 37 + i // 13) & ((1 << bits) - 1))


def test_decode_rows_slice_matches_full():
    packed, s, b = oracle.affine_pattern(64 * 3 * 4, 4, 32, F16)
    t = Tensor.affine([64, 3, 4], packed, s, b, 4, 32, F16)
    full = oracle.decode(t)
    assert np.array_equal(oracle.decode(t, 6, 3), full[6 * 64:9 * 64])


def test_validation_mirrors_tensor_new():
    # crates/model-format/src/checkpoint.rs:106-116
    good = Tensor.affine([64, 2], np.zeros(16, np.uint32), np.zeros(4, np.uint16),
                         np.zeros(4, np.uint16), 4, 32, BF16)
    assert oracle.validate(good) == 0
    for bits, group, st, dims in [(3, 32, BF16, [64, 2]), (4, 16, BF16, [64, 2]),
                                  (4, 32, 2, [64, 2]), (4, 128, BF16, [64, 2])]:
        t = Tensor.affine(dims, np.zeros(16, np.uint32), np.zeros(4, np.uint16),
                          np.zeros(4, np.uint16), bits, group, st)
        assert oracle.validate(t) != 0


# ------------------------------------------------------------- tensor-core --
def test_matvec_softmax_silu_rmsnorm_closed_forms():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((7, 65)).astype(np.float32)
    x = rng.standard_normal(65).astype(np.float32)
    np.testing.assert_allclose(oracle.matvec(w, x), w.astype(np.float64) @ x, rtol=1e-5, atol=1e-5)
    z = rng.standard_normal(19).astype(np.float32) * 4
    e = np.exp(z.astype(np.float64) - z.max())
    np.testing.assert_allclose(oracle.softmax(z), e / e.sum(), rtol=4e-6, atol=1e-9)
    for v in [-20.0, -1.5, 0.0, 0.3, 7.0]:
        assert math.isclose(oracle.silu(v), v / (1 + math.exp(-v)), rel_tol=1e-6, abs_tol=1e-12)
    nw = rng.standard_normal(65).astype(np.float32)
    ref = x.astype(np.float64) * nw / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
    np.testing.assert_allclose(oracle.rms_norm(x, nw, 1e-5), ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kind", [("dense", F32), ("dense", BF16), (4, 64, BF16), (8, 32, F16),
                                  (2, 128, F32)])
@pytest.mark.parametrize("tokens", [1, 3, 17])
def test_matmul_tokens_vs_independent_float64(kind, tokens):
    """orc_matmul over several tokens (matrix.rs:63-148: y[t*out + r] =
    W[r] . x[t*in..]) against a float64 product of the numpy-decoded weight.
    A wrong token stride (x or y), a transposed weight or a dropped token
    fails here: every token's row is compared, with distinct inputs."""
    from helpers import make_tensor
    inn, out = 256, 24
    t = make_tensor([inn, out], kind, seed=500 + tokens)
    x = synth.normal(600 + tokens, tokens * inn).reshape(tokens, inn)
    if t.bits:
        wd = _numpy_decode(t).reshape(out, inn)
    elif t.dtype == F32:
        wd = t.data.astype(np.float64).reshape(out, inn)
    else:
        wd = synth.bf16_bits_to_f32(t.data).astype(np.float64).reshape(out, inn)
    ref = x.astype(np.float64) @ wd.T
    got = oracle.matmul(t, x, tokens).reshape(tokens, out)
    np.testing.assert_allclose(got, ref, rtol=0, atol=2e-5 * np.abs(ref).max())
    # a shuffled token order is caught (distinct rows)
    if tokens > 1:
        assert not np.allclose(got[::-1], ref, rtol=0, atol=2e-5 * np.abs(ref).max())


def test_expert_matmul_per_expert_inputs_vs_float64():
    """orc_expert_matmul: y[k*out + r] = expert ids[k] row r . x (shared input)
    or . x[k*in..] (per-expert input, the down product), id >= E -> zeros
    (matrix.rs:149-205, affine.metal:90-91)."""
    from helpers import make_tensor
    inn, out, E = 128, 16, 5
    t = make_tensor([inn, out, E], (4, 32, BF16), seed=77)
    wd = _numpy_decode(t).reshape(E, out, inn)
    ids = np.array([3, 0, 7, 3], np.uint32)  # 7 >= E
    xs = synth.normal(78, 4 * inn).reshape(4, inn)
    got = oracle.expert_matmul(t, xs, ids, True).reshape(4, out)
    for k, e in enumerate(ids):
        ref = wd[e] @ xs[k].astype(np.float64) if e < E else np.zeros(out)
        np.testing.assert_allclose(got[k], ref, rtol=0, atol=2e-5 * max(1.0, np.abs(ref).max()))
    got1 = oracle.expert_matmul(t, xs[0], ids, False).reshape(4, out)
    for k, e in enumerate(ids):
        ref = wd[e] @ xs[0].astype(np.float64) if e < E else np.zeros(out)
        np.testing.assert_allclose(got1[k], ref, rtol=0, atol=2e-5 * max(1.0, np.abs(ref).max()))


def test_elementwise_closed_forms():
    rng = np.random.default_rng(2)
    a, b = rng.standard_normal(50).astype(np.float32), rng.standard_normal(50).astype(np.float32)
    np.testing.assert_allclose(oracle.swiglu(a, b), a / (1 + np.exp(-a.astype(np.float64))) * b,
                               rtol=1e-6, atol=1e-7)
    x = rng.standard_normal((3, 50)).astype(np.float32)
    w = np.array([0.5, -1.0, 2.0], np.float32)
    np.testing.assert_allclose(oracle.mix(x, w), (w[:, None].astype(np.float64) * x).sum(0),
                               rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.gate_scalar(a, 0.7), a / (1 + np.exp(-0.7)), rtol=1e-6)
    np.testing.assert_allclose(oracle.add(a, b), a + b)


# ------------------------------------------------------------------ routing --
def test_route_kat():
    # crates/metal-backend/tests/affine.rs:96-112: logits [1,4,3,2], K=2 -> ids [1, 2]
    ids, w = oracle.route([1.0, 4.0, 3.0, 2.0], 2, True)
    assert ids.tolist() == [1, 2]
    e4, e3 = math.exp(4), math.exp(3)
    np.testing.assert_allclose(w, [e4 / (e4 + e3), e3 / (e4 + e3)], rtol=1e-6)
    ids, w = oracle.route([1.0, 4.0, 3.0, 2.0], 2, False)
    den = sum(math.exp(v - 4) for v in [1, 4, 3, 2])
    np.testing.assert_allclose(w, [1 / den, math.exp(-1) / den], rtol=1e-6)


def _expected_ids(x, k):
    cand = [j for j in range(len(x)) if not math.isnan(x[j]) and x[j] > -math.inf]
    cand.sort(key=lambda j: (-x[j], j))  # stable: value desc, index asc
    ids = cand[:k]
    return ids + [0] * (k - len(ids))


def test_route_brute_force_ties():
    vals = [-math.inf, 0.0, 1.0, 1.0 + 2 ** -20, float("nan")]
    for x in itertools.product(vals, repeat=5):
        for k in range(1, 6):
            ids, w = oracle.route(np.array(x, np.float32), k, False)
            assert ids.tolist() == _expected_ids(np.array(x, np.float32).tolist(), k), (x, k)
            if not any(math.isnan(v) for v in x) and any(v > -math.inf for v in x):
                xs = np.array(x, np.float64)
                mx = xs.max()
                den = np.exp(xs - mx).sum()
                exp_w = [math.exp(float(np.float32(x[j])) - mx) / den if x[j] > -math.inf else 0.0
                         for j in ids.tolist()]
                # exhausted passes have score -inf -> weight 0
                sel = _expected_ids(list(x), k)
                n_valid = sum(1 for v in x if v > -math.inf)
                exp_w = [e if i < n_valid else 0.0 for i, e in enumerate(exp_w)]
                np.testing.assert_allclose(w, exp_w, rtol=1e-6, atol=1e-12)
                assert sel == ids.tolist()


def test_route_nan_poisons_weights_not_ids():
    ids, w = oracle.route(np.array([1.0, np.nan, 3.0], np.float32), 2, True)
    assert ids.tolist() == [2, 0]
    assert np.isnan(w).all()


def test_route_signed_zero_tie_goes_low():
    ids, _ = oracle.route(np.array([-0.0, 0.0, -1.0], np.float32), 2, True)
    assert ids.tolist() == [0, 1]


# ---------------------------------------------------------------- dispatch --
def test_dispatch_invariants_and_stable_sort():
    rng = np.random.default_rng(3)
    T, K, E = 300, 4, 37
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.uint32)
    counts, offsets, perm, pos = oracle.dispatch(ids, E)
    assert np.array_equal(counts, np.bincount(ids.ravel(), minlength=E))
    assert offsets[0] == 0 and offsets[-1] == T * K
    assert np.array_equal(np.diff(offsets.astype(np.int64)), counts)
    assert np.array_equal(perm, np.argsort(ids.ravel(), kind="stable"))
    assert np.array_equal(pos[perm], np.arange(T * K))
    for e in range(E):
        seg = perm[offsets[e]:offsets[e + 1]]
        assert (ids.ravel()[seg] == e).all()
        assert (np.diff(seg.astype(np.int64)) > 0).all()


# --------------------------------------------------------------- generator --
def test_generator_lcg_matches_reference_recurrence():
    # crates/llama-rs/tests/common/mod.rs:86-97
    s = 42
    states = []
    for _ in range(10):
        s = (s * 6364136223846793005 + 1) % (1 << 64)
        states.append(s)
    assert synth.lcg_states(42, 10).tolist() == states
    u1 = ((states[0] >> 32) + 0.5) / 2 ** 32
    u2 = ((states[1] >> 32) + 0.5) / 2 ** 32
    z0 = math.sqrt(-2 * math.log(u1)) * math.cos(2 * math.pi * u2)
    assert oracle.normal(42, 2)[0] == np.float32(z0)


def test_generator_oracle_and_product_agree():
    a = oracle.normal(123, 100001, 0.0, 0.02)
    b = synth.normal(123, 100001, 0.0, 0.02)
    diff = a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64)
    assert np.abs(diff).max() <= 1 and (diff == 0).mean() > 0.999
    big = synth.normal(7, 200000)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1) < 0.01


@pytest.mark.parametrize("bits,group,st", [(4, 64, BF16), (8, 128, F16), (2, 32, F32)])
def test_quantizer_oracle_and_product_agree(bits, group, st):
    w = synth.normal(9, 64 * 256, 0.0, 0.02)
    p1, s1, b1 = oracle.quantize_affine(w, bits, group, st)
    p2, s2, b2 = synth.quantize_affine(w, bits, group, st)
    assert np.array_equal(p1, p2) and np.array_equal(s1, s2) and np.array_equal(b1, b2)
    t = Tensor.affine([128, 128], p1, s1, b1, bits, group, st)
    dec = oracle.decode(t).reshape(-1, group)
    err = np.abs(dec - w.reshape(-1, group)).max(axis=1)
    ones = synth.pack_codes(np.ones(64 * 256, np.uint32), bits)
    zb = np.zeros_like(b1)
    sc = oracle.decode(Tensor.affine([128, 128], ones, s1, zb, bits, group, st)).reshape(-1, group)[:, 0]
    bi = oracle.decode(Tensor.affine([128, 128], np.zeros_like(p1), s1, b1, bits, group, st))
    bi = bi.reshape(-1, group)[:, 0]
    # round-to-nearest code: error <= scale/2, plus the scale/bias rounding to st
    qmax = (1 << bits) - 1
    rnd = 2.0 ** -8 if st == BF16 else (2.0 ** -11 if st == F16 else 2.0 ** -24)
    bound = 0.5 * sc + rnd * (qmax * sc + np.abs(bi)) + 1e-8
    assert (err <= bound).all()
    # and a code off by one would break it
    assert (err < sc).all()


# --------------------------------------------------------------- MoE block --
def _np_block(blk, x, logits_in=None):
    """Independent float64 restatement of execute.rs:208-233 from the reference."""
    def rows(t):
        if t.bits == 0:
            return t.data.astype(np.float64).reshape(-1, t.dims[0])
        return _numpy_decode(t).reshape(-1, t.dims[0])
    R = rows(blk.router)
    G, U, D = rows(blk.gate), rows(blk.up), rows(blk.down)
    h, ff, E, K = blk.h, blk.ff, blk.E, blk.K
    out = []
    for t in range(x.shape[0]):
        xt = x[t].astype(np.float64)
        lg = R @ xt if logits_in is None else logits_in[t].astype(np.float64)
        ids = _expected_ids(np.float32(lg).tolist() if logits_in is None else logits_in[t].tolist(), K)
        p = np.exp(lg - lg.max())
        p /= p.sum()
        w = p[ids]
        if blk.normalize:
            w = w / w.sum()
        y = np.zeros(h)
        for k, e in enumerate(ids):
            g = G[e * ff:(e + 1) * ff] @ xt
            u = U[e * ff:(e + 1) * ff] @ xt
            a = g / (1 + np.exp(-g)) * u
            y += w[k] * (D[e * h:(e + 1) * h] @ a)
        if blk.shared is not None:
            sg, su, sd = (rows(s) for s in blk.shared)
            g, u = sg @ xt, su @ xt
            a = g / (1 + np.exp(-g)) * u
            gate = rows(blk.shared_gate).ravel() @ xt
            y += (sd @ a) / (1 + np.exp(-gate))
        out.append(y)
    return np.array(out)


@pytest.mark.parametrize("kind", ["f32", "affine"])
def test_moe_block_vs_independent_float64(kind):
    blk, x = config1(kind)
    out, logits, ids, w = oracle.moe_block(blk.spec(), x, 4)
    ref = _np_block(blk, x, logits_in=logits)
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.max(np.abs(ref))
    for t in range(4):
        assert ids[t].tolist() == _expected_ids(logits[t].tolist(), blk.K)


def test_moe_block_logits_in_skips_router():
    blk, x = config1("f32")
    out, logits, ids, _ = oracle.moe_block(blk.spec(), x, 4)
    forced = logits.copy()
    forced[:, 0] += 100.0  # force expert 0 first
    out2, _, ids2, _ = oracle.moe_block(blk.spec(), x, 4, logits_in=forced)
    assert (ids2[:, 0] == 0).all()
    assert not np.allclose(out, out2)


def test_moe_block_golden_fixture():
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "config1.npz")
    g = np.load(path)
    blk, x = config1("f32")
    assert np.array_equal(x, g["x"])
    out, logits, ids, w = oracle.moe_block(blk.spec(), x, 4)
    assert np.array_equal(ids, g["ids"])
    np.testing.assert_allclose(out, g["out"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(logits, g["logits"], rtol=0, atol=1e-6)
    np.testing.assert_allclose(w, g["weights"], rtol=0, atol=1e-7)


def test_moe_stack_residual():
    blk, x = config1("f32")
    nw = np.ones(64, np.float32)
    h = oracle.moe_stack([blk.spec()], [nw], 1e-6, x, 4)
    xn = np.stack([oracle.rms_norm(r, nw, 1e-6) for r in x])
    out, *_ = oracle.moe_block(blk.spec(), xn, 4)
    np.testing.assert_allclose(h, x + out, rtol=1e-6, atol=1e-6)


def test_threads_do_not_change_results():
    """The oracle's row-parallel loops (the all-core CPU baseline) give the
    single-thread results bit for bit: every row keeps its sequential sum."""
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": (8, 64, BF16), "shared_gate": DENSE}
    blk = HostBlock(512, 64, 4, 512, 256, kinds, seed=33)
    x = synth.normal(34, 3 * 512).reshape(3, 512)
    n = oracle.threads()
    try:
        oracle.set_threads(1)
        one = oracle.moe_block(blk.spec(), x, 3)
        oracle.set_threads(max(4, n))
        many = oracle.moe_block(blk.spec(), x, 3)
    finally:
        oracle.set_threads(n)
    for a, b in zip(one, many):
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


# ------------------------------------------------- expert-major evaluation --
def _bits(outs):
    return [np.asarray(a).view(np.uint32) if np.asarray(a).dtype == np.float32 else np.asarray(a)
            for a in outs]


def _same(a, b):
    for p, q in zip(_bits(a), _bits(b)):
        assert np.array_equal(p, q)


@pytest.mark.parametrize("kind", ["f32", "affine"])
def test_moe_block_expert_major_equals_per_token_config1(kind):
    """orc_moe_block_em (every expert decoded once for all its pairs) gives
    orc_moe_block's outputs, logits, ids and weights bit for bit on the
    config-1 fixture: each (pair, row) product is the same sequential sum."""
    blk, x = config1(kind)
    _same(oracle.moe_block(blk.spec(), x, 4), oracle.moe_block(blk.spec(), x, 4, expert_major=True))


@pytest.mark.parametrize("normalize", [True, False])
def test_moe_block_expert_major_chunks_shared_bias(normalize):
    """Mixed weight kinds (8-bit router and shared gate row, f16-scaled 4-bit
    experts, F32-scaled 2-bit shared expert), a logit bias and 4100 tokens,
    so the pairs are sorted in two chunks (4096 + 4): bit for bit equal."""
    kinds = {"router": (8, 64, BF16), "experts": (4, 32, F16), "shared": (2, 32, F32),
             "shared_gate": (8, 64, BF16)}
    blk = HostBlock(64, 8, 3, 32, 96, kinds, seed=5, normalize=normalize, random_experts=True)
    T = 4100
    x = synth.normal(7, T * 64).reshape(T, 64)
    rng = np.random.default_rng(3)
    bias = (rng.standard_normal((T, 8)) * 2).astype(np.float32)
    a = oracle.moe_block(blk.spec(), x, T, logit_bias=bias)
    b = oracle.moe_block(blk.spec(), x, T, logit_bias=bias, expert_major=True)
    _same(a, b)
    assert len(np.unique(a[2][:, 0])) == 8  # every expert receives pairs


def test_moe_block_expert_major_ties_and_logits_in():
    """Routing of given logits with heavy ties (ids to the lower index) and
    K = E, so every expert holds every token: expert-major equals per-token."""
    kinds = {"router": DENSE, "experts": (8, 32, BF16)}
    blk = HostBlock(96, 6, 6, 32, 0, kinds, seed=9, random_experts=True)
    T = 37
    x = synth.normal(11, T * 96).reshape(T, 96)
    lg = np.round(synth.normal(12, T * 6).reshape(T, 6)).astype(np.float32)  # integers: ties
    a = oracle.moe_block(blk.spec(), x, T, logits_in=lg)
    b = oracle.moe_block(blk.spec(), x, T, logits_in=lg, expert_major=True)
    _same(a, b)
    for t in range(T):
        assert a[2][t].tolist() == _expected_ids(lg[t].tolist(), 6)


def test_moe_block_expert_major_prefill_shape():
    """Config-4 shapes (h 2048, E 128, top 8, ff 768, 4-bit g64) at 48 tokens
    under the Zipf skew: expert-major equals per-token bit for bit."""
    from helpers import config4, zipf_bias
    blk = config4()
    T = 48
    x = synth.normal(4000, T * 2048).reshape(T, 2048)
    bias = zipf_bias(T, 128, seed=4)
    _same(oracle.moe_block(blk.spec(), x, T, logit_bias=bias),
          oracle.moe_block(blk.spec(), x, T, logit_bias=bias, expert_major=True))


def test_matmul_tokens_equal_per_token_matvec():
    """orc_matmul over many tokens (decoded once, eight tokens per pass) gives
    each token's orc_matvec of the decoded rows bit for bit."""
    from helpers import make_tensor
    t = make_tensor([320, 40], (4, 64, BF16), seed=21)
    T = 13
    x = synth.normal(22, T * 320).reshape(T, 320)
    got = oracle.matmul(t, x, T).reshape(T, 40)
    dec = oracle.decode(t)
    for i in range(T):
        assert np.array_equal(got[i].view(np.uint32), oracle.matvec(dec, x[i]).view(np.uint32))


def test_moe_stack_equals_chained_per_token_blocks():
    """orc_moe_stack (expert-major blocks) over 3 layers with distinct norm
    weights equals RMSNorm -> orc_moe_block -> add chained by hand."""
    kinds = {"router": DENSE, "experts": (2, 32, BF16), "shared": (2, 32, BF16), "shared_gate": DENSE}
    blk = HostBlock(128, 16, 4, 64, 64, kinds, seed=13, random_experts=True)
    nws = [(1.0 + 0.3 * synth.normal(50 + l, 128)).astype(np.float32) for l in range(3)]
    x = synth.normal(60, 2 * 128).reshape(2, 128)
    got = oracle.moe_stack([blk.spec()] * 3, nws, 1e-6, x, 2)
    h = x.copy()
    for nw in nws:
        xn = np.stack([oracle.rms_norm(r, nw, 1e-6) for r in h])
        out, *_ = oracle.moe_block(blk.spec(), xn, 2)
        h = oracle.add(h, out).reshape(h.shape)
    assert np.array_equal(got.view(np.uint32), h.view(np.uint32))
