"""GPU parity of the op surface (Batch ops behind the C ABI) against the CPU
oracle, mirroring the reference's own GPU op tests
(crates/metal-backend/tests/affine.rs, operations.rs).  Integer outputs
(expert ids, dispatch permutation) must be bit-exact; float outputs use the
reference tests' element tolerance |a-b| < tol*(1+|b|)."""
import numpy as np
import pytest

import oracle
from helpers import close, zipf_bias
from hip_backend import BF16, F16, F32, Gpu, ShapeError, Tensor, synth

pytestmark = pytest.mark.gpu


def _pattern_tensor(dims, bits, group, st):
    n = int(np.prod(dims))
    packed, s, b = oracle.affine_pattern(n, bits, group, st)
    return Tensor.affine(dims, packed, s, b, bits, group, st)


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("st", [F32, F16, BF16])
def test_affine_gemv_and_prefill_all_layouts(gpu, bits, group, st):
    # crates/metal-backend/tests/affine.rs:53-89
    print(f"[case] affine matmul bits={bits} group={group} st={st}", flush=True)
    t = _pattern_tensor([256, 19], bits, group, st)
    w = gpu.weight_tensor(t)
    for count in [1, 3, 4, 17]:
        x = (np.sin(np.arange(256 * count, dtype=np.float32) * np.float32(0.27)) * np.float32(0.1))
        x = x.astype(np.float32)
        xb = gpu.upload(x)
        y = gpu.zeros(19 * count)
        with gpu.batch() as b:
            b.matmul(w, xb, y, count)
        close(gpu.read(y), oracle.matmul(t, x, count))


@pytest.mark.parametrize("kind", [("dense", F32), ("dense", BF16), ("dense", F16), (4, 64, BF16),
                                  (8, 128, F16), (2, 32, F32)])
@pytest.mark.parametrize("tokens", [4, 17, 64, 4096])
def test_matmul_tiled_f32_tokens(gpu, kind, tokens):
    """Batch::matmul at 4 tokens or more runs the tiled F32 product (the
    reference's affine_mm / gemm_simd switch, matrix.rs:77-123) on the F32
    matrix cores: every token's row against orc_matmul (affine.rs:46-51
    tolerance), at the dense projection shape h 2048 -> 512 (the shared
    expert's gate), for every dtype; below 4 tokens the GEMV runs."""
    from helpers import make_tensor
    print(f"[case] tiled matmul kind={kind} tokens={tokens}", flush=True)
    t = make_tensor([2048, 512], kind, seed=tokens + len(kind))
    w = gpu.weight_tensor(t)
    x = synth.normal(7000 + tokens, tokens * 2048).reshape(tokens, 2048)
    xb, y = gpu.upload(x), gpu.zeros(tokens * 512)
    gpu.profile_reset()
    gpu.profile(True)
    with gpu.batch() as b:
        b.matmul(w, xb, y, tokens)
    prof = gpu.profile_read()
    gpu.profile(False)
    assert "matmul_f32" in prof, sorted(prof)
    rows = range(tokens) if tokens <= 64 else list(range(0, tokens, 97)) + [tokens - 1]
    rows = np.array(list(rows))
    got = gpu.read(y).reshape(tokens, 512)
    if tokens <= 64:
        ref = oracle.matmul(t, x, tokens).reshape(tokens, 512)
        close(got, ref)
    else:
        close(got[rows], oracle.matmul(t, x[rows], len(rows)).reshape(len(rows), 512))
    for b_ in (xb, y):
        gpu.release(b_)


def test_matmul_unaligned_input_uses_gemv(gpu):
    """An input view that is not 16-byte aligned keeps the per-token GEMV
    (the tiled product loads 16-byte vectors), with the same results."""
    t = _pattern_tensor([256, 40], 4, 64, BF16)
    w = gpu.weight_tensor(t)
    T = 8
    x = synth.normal(7100, T * 256 + 1)
    xb = gpu.upload(x)
    y = gpu.zeros(T * 40)
    gpu.profile_reset()
    gpu.profile(True)
    with gpu.batch() as b:
        b.matmul(w, xb.view(1, T * 256), y, T)
    prof = gpu.profile_read()
    gpu.profile(False)
    assert "matmul_f32" not in prof
    close(gpu.read(y), oracle.matmul(t, x[1:], T))


def test_affine_experts_use_gpu_selected_ids(gpu):
    # crates/metal-backend/tests/affine.rs:91-113
    t = _pattern_tensor([64, 3, 4], 4, 32, F16)
    values = oracle.decode(t)
    w = gpu.weight_tensor(t)
    logits = gpu.upload(np.array([1, 4, 3, 2], np.float32))
    ids = gpu.zeros(2)
    probs = gpu.zeros(2)
    x = np.arange(64, dtype=np.float32) * np.float32(0.01)
    xb = gpu.upload(x)
    out = gpu.zeros(6)
    with gpu.batch() as b:
        b.route(logits, ids, probs, True)
        b.expert_matmul(w, xb, ids, out, False)
    assert gpu.read_u32(ids).tolist() == [1, 2]
    expected = np.concatenate([oracle.matvec(values[e * 3 * 64:(e + 1) * 3 * 64], x) for e in [1, 2]])
    close(gpu.read(out), expected)
    e4, e3 = np.exp(4.0), np.exp(3.0)
    np.testing.assert_allclose(gpu.read(probs), [e4 / (e4 + e3), e3 / (e4 + e3)], rtol=1e-6)


def test_expert_matmul_per_expert_input_and_out_of_range_id(gpu):
    t = _pattern_tensor([64, 5, 6], 8, 64, BF16)
    w = gpu.weight_tensor(t)
    ids = np.array([5, 0, 9], np.uint32)  # 9 >= E: zeros (affine.metal:91)
    x = synth.normal(5, 3 * 64)
    out = gpu.zeros(15)
    xb, ib = gpu.upload(x), gpu.upload_u32(ids)
    with gpu.batch() as b:
        b.expert_matmul(w, xb, ib, out, True)
    ref = oracle.expert_matmul(t, x, ids, True)
    close(gpu.read(out), ref)
    assert (gpu.read(out)[10:] == 0).all()


def test_expert_matmul_single_row_weight_honours_ids(gpu):
    """A one-row, one-expert weight ([64, 1, 1]) under expert_matmul with a
    GPU id: id 0 gives the product, id 5 (>= E) gives 0 (affine.metal:91,
    matrix.metal:52-55) -- the one-row fast path applies only without ids."""
    t = _pattern_tensor([64, 1, 1], 4, 32, BF16)
    w = gpu.weight_tensor(t)
    x = synth.normal(8, 64)
    xb = gpu.upload(x)
    for e in (0, 5):
        ib, out = gpu.upload_u32(np.array([e], np.uint32)), gpu.zeros(1)
        with gpu.batch() as b:
            b.expert_matmul(w, xb, ib, out, False)
        ref = oracle.expert_matmul(t, x, np.array([e], np.uint32), False)
        close(gpu.read(out), ref)
        if e == 5:
            assert gpu.read(out)[0] == 0.0
        else:
            assert ref[0] != 0.0


def test_actual_gpu_ops(gpu):
    # crates/metal-backend/tests/operations.rs:8-28
    data = np.sin(np.arange(65 * 7, dtype=np.float32) * np.float32(0.13)).astype(np.float32)
    x = (np.arange(65, dtype=np.float32) / np.float32(65)).astype(np.float32)
    w = gpu.weight_f32(data, [65, 7])
    nw = gpu.weight_f32(np.ones(65, np.float32), [65])
    xb = gpu.upload(x)
    y = gpu.zeros(7)
    norm = gpu.zeros(65)
    with gpu.batch() as b:
        b.matmul(w, xb, y, 1)
        b.norm(xb, nw, norm, 1, 65, 1e-5)
    close(gpu.read(y), oracle.matvec(data, x), 2e-4)
    close(gpu.read(norm), oracle.rms_norm(x, np.ones(65, np.float32), 1e-5), 2e-4)


@pytest.mark.parametrize("dtype", [F32, F16, BF16])
def test_dense_matmul_dtypes(gpu, dtype):
    v = synth.normal(11, 96 * 33, 0.0, 0.5)
    if dtype == F32:
        t = Tensor.dense([96, 33], v)
    elif dtype == F16:
        t = Tensor.dense([96, 33], v.astype(np.float16).view(np.uint16), F16)
    else:
        t = Tensor.dense([96, 33], synth.f32_to_bf16_bits(v), BF16)
    x = synth.normal(12, 96 * 5)
    y = gpu.zeros(33 * 5)
    wt, xb = gpu.weight_tensor(t), gpu.upload(x)
    with gpu.batch() as b:
        b.matmul(wt, xb, y, 5)
    close(gpu.read(y), oracle.matmul(t, x, 5), 2e-4)


def test_rejects_aliases_and_foreign_buffers(gpu):
    # crates/metal-backend/tests/operations.rs:101-111
    other = Gpu()
    w = gpu.weight_f32(np.ones(64, np.float32), [8, 8])
    x = gpu.upload(np.ones(8, np.float32))
    foreign = other.upload(np.ones(8, np.float32))
    with gpu.batch() as b:
        with pytest.raises(ShapeError):
            b.matmul(w, x, x, 1)
        with pytest.raises(ShapeError):
            b.add(x, foreign, x)
        # exact in-place add is allowed (commands.rs:35,52)
        b.add(x, x, x)
    assert (gpu.read(x) == 2).all()
    other.close()


def test_shape_checks_mirror_the_reference(gpu):
    w = gpu.weight_f32(np.ones(64, np.float32), [8, 8])
    x = gpu.zeros(8)
    y = gpu.zeros(9)
    ids = gpu.zeros(3)
    z2, z3, z2b, z2c, z8 = gpu.zeros(2), gpu.zeros(3), gpu.zeros(2), gpu.zeros(2), gpu.zeros(8)
    with gpu.batch() as b:
        with pytest.raises(ShapeError):
            b.matmul(w, x, y, 1)            # matrix.rs:64-75
        with pytest.raises(ShapeError):
            b.route(x, ids, z2, True)       # sampling.rs:28
        with pytest.raises(ShapeError):
            b.mix(x, z3, z2b)               # elementwise.rs:93
        with pytest.raises(ShapeError):
            b.gate_scalar(x, z2c, z8)       # elementwise.rs:80
    with pytest.raises(ShapeError):         # memory access while a batch is open
        with gpu.batch() as b:
            gpu.zeros(4)
    from hip_backend.api import Batch
    with pytest.raises(ShapeError):   # ops need an open batch (the Batch borrow)
        Batch(gpu, begin=False).add(x, x, x)


# ----------------------------------------------------------------- routing --
def _route_case(gpu, logits, k, normalize):
    T, E = logits.shape
    lb = gpu.upload(logits)
    ids = gpu.zeros(T * k)
    w = gpu.zeros(T * k)
    with gpu.batch() as b:
        b.route_tokens(lb, ids, w, T, normalize)
    got_ids = gpu.read_u32(ids).reshape(T, k)
    got_w = gpu.read(w).reshape(T, k)
    ref_ids, ref_w = oracle.route_tokens(logits, k, normalize)
    assert np.array_equal(got_ids, ref_ids)
    both_nan = np.isnan(got_w) & np.isnan(ref_w)
    assert (np.isnan(got_w) == np.isnan(ref_w)).all()
    np.testing.assert_allclose(got_w[~both_nan], ref_w[~both_nan], rtol=2e-6, atol=1e-9)


@pytest.mark.parametrize("normalize", [True, False])
def test_route_bit_exact_random(gpu, normalize):
    logits = synth.normal(21, 257 * 512, 0.0, 1.0).reshape(257, 512)
    _route_case(gpu, logits, 10, normalize)


def test_route_bit_exact_heavy_ties(gpu):
    # logits drawn from 5 values -> many exact ties; order must be lowest index first
    rng = np.random.default_rng(22)
    vals = np.array([-1.0, 0.0, 0.5, 0.5 + 2 ** -20, 2.0], np.float32)
    logits = vals[rng.integers(0, 5, (300, 128))]
    _route_case(gpu, logits, 8, True)
    _route_case(gpu, logits[:, :64], 64, False)  # K = E


def test_route_nonfinite(gpu):
    logits = np.array([[1.0, np.nan, 3.0, -np.inf],
                       [-np.inf, -np.inf, -np.inf, 2.0],
                       [-0.0, 0.0, -1.0, -0.0]], np.float32)
    _route_case(gpu, logits, 3, True)


# ---------------------------------------------------------------- dispatch --
# (4096, 8, 128) runs the single-pass kernel with per-chunk count tables;
# (8192, 8, 512) the same kernel without them (16 chunks x 512 experts of
# tables exceed its 64 KiB of LDS); (4096, 10, 512) and (5600, 10, 512) the
# tables at 10 and 14 chunks over 512 experts (the Qwen3-Next prefill's
# dispatch), the latter filling the 64 KiB
@pytest.mark.parametrize("T,K,E", [(4096, 8, 128), (8192, 8, 512), (4096, 10, 512), (5600, 10, 512),
                                   (64, 10, 512), (1, 10, 512), (777, 3, 40)])
def test_dispatch_bit_exact(gpu, T, K, E):
    logits = synth.normal(23 + T, T * E).reshape(T, E) + zipf_bias(T, E, 5)
    ids, _ = oracle.route_tokens(logits, K, True)
    counts, offsets, perm, pos = (gpu.zeros(E), gpu.zeros(E + 1), gpu.zeros(T * K), gpu.zeros(T * K))
    ib = gpu.upload_u32(ids.ravel())
    with gpu.batch() as b:
        b.dispatch(ib, T, K, E, counts, offsets, perm, pos)
    rc, ro, rp, rpos = oracle.dispatch(ids, E)
    assert np.array_equal(gpu.read_u32(counts), rc)
    assert np.array_equal(gpu.read_u32(offsets), ro)
    assert np.array_equal(gpu.read_u32(perm), rp)
    assert np.array_equal(gpu.read_u32(pos), rpos)


# ------------------------------------------------------------- elementwise --
def test_elementwise_ops(gpu):
    a = synth.normal(31, 1000) * 4
    bb = synth.normal(32, 1000)
    ab, bbuf = gpu.upload(a), gpu.upload(bb)
    y1, y2, y3 = gpu.zeros(1000), gpu.zeros(1000), gpu.zeros(1000)
    g = gpu.upload(np.array([0.3], np.float32))
    xk = synth.normal(33, 4 * 250)
    wk = np.array([0.5, -0.25, 1.5, 0.0], np.float32)
    ym = gpu.zeros(250)
    xkb, wkb = gpu.upload(xk), gpu.upload(wk)
    with gpu.batch() as b:
        b.swiglu(ab, bbuf, y1)
        b.add(ab, bbuf, y2)
        b.gate_scalar(ab, g, y3)
        b.mix(xkb, wkb, ym)
        b.swiglu(ab, bbuf, ab)  # exact in-place (commands.rs:35)
    close(gpu.read(y1), oracle.swiglu(a, bb), 1e-5)
    close(gpu.read(y2), oracle.add(a, bb), 1e-6)
    close(gpu.read(y3), oracle.gate_scalar(a, 0.3), 1e-5)
    close(gpu.read(ym), oracle.mix(xk, wk), 1e-5)
    close(gpu.read(ab), oracle.swiglu(a, bb), 1e-5)


def test_allocation_error_carries_bytes(gpu):
    """Error::Allocation(usize) carries the requested size
    (crates/metal-backend/src/lib.rs:12-13, apple/memory.rs:9-26): zero-sized
    and over-limit requests report their byte counts; a later shape error
    clears it."""
    from hip_backend import AllocationError, ShapeError
    with pytest.raises(AllocationError) as e:
        gpu.zeros(1 << 33)  # more than u32::MAX elements (memory.rs:10)
    assert e.value.bytes == 4 << 33
    with pytest.raises(AllocationError) as e:
        gpu.zeros(0)
    assert e.value.bytes == 0
    with pytest.raises(AllocationError) as e:
        gpu.zeros(1 << 33)
    b = gpu.zeros(4)
    with pytest.raises(ShapeError):
        b.view(2, 8)
    with pytest.raises(ShapeError):
        with gpu.batch() as bt:
            bt.add(b, b.view(0, 2), b)
    from hip_backend.api import _lib
    assert _lib.moe_last_error_bytes(gpu._h) == 0
    gpu.release(b)
