"""moe_block_noalloc (the entry point that allocates nothing: its workspace
is the library's per-GPU scratch array) against moe_block with a fresh
caller workspace, through the C ABI: the same kernels on the same inputs, so
ids, logits, weights and outputs must agree bit for bit.  Two calls in a row
per path, the second with fewer tokens, so the second call finds the first
call's contents in the shared array."""
import numpy as np
import pytest

from helpers import DENSE, HostBlock, config3, hot_bias, zipf_bias
from hip_backend import BF16, PATH_AUTO, PATH_MFMA, ShapeError, synth

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # MOE_NOALLOC_SCRATCH_BYTES


def run(gpu, bw, x, T, bias, path, noalloc):
    E, K, h = bw.experts, bw.k, bw.hidden
    xb = gpu.upload(x)
    bb = gpu.upload(bias)
    out = gpu.zeros(T * h)
    lo, io_, wo = gpu.zeros(T * E), gpu.zeros(T * K), gpu.zeros(T * K)
    ws = None if noalloc else gpu.zeros(bw.workspace_elems(T))
    with gpu.batch() as b:
        if noalloc:
            b.moe_block_noalloc(bw, xb, out, T, logit_bias=bb, logits_out=lo, ids_out=io_,
                                weights_out=wo, path=path)
        else:
            b.moe_block(bw, xb, out, T, ws, logit_bias=bb, logits_out=lo, ids_out=io_,
                        weights_out=wo, path=path)
    res = [gpu.read(out), gpu.read(lo), gpu.read_u32(io_), gpu.read(wo)]
    for buf in (xb, bb, out, lo, io_, wo, ws):
        if buf is not None:
            gpu.release(buf)
    return res


def same(a, b):
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))


@pytest.fixture(scope="module")
def c3(gpu):
    blk = config3()
    return blk, blk.upload(gpu)


@pytest.mark.parametrize("sizes", [(64, 8), (8, 1)])
def test_noalloc_matches_moe_block_config3(gpu, c3, sizes):
    """Config 3 (8-bit router and shared expert, 4-bit experts): the batched
    decode at 64 then 8 tokens, and at 8 tokens then the fused single-token
    decode."""
    blk, bw = c3
    for i, T in enumerate(sizes):
        print(f"[case] noalloc config3 T={T} (call {i + 1})", flush=True)
        assert bw.workspace_elems(T) * 4 <= SCRATCH_BYTES
        x = synth.normal(9100 + T, T * 2048).reshape(T, 2048)
        bias = hot_bias(T, 512, seed=90 + T)
        got = run(gpu, bw, x, T, bias, PATH_AUTO, True)
        ref = run(gpu, bw, x, T, bias, PATH_AUTO, False)
        same(got, ref)


def test_noalloc_matches_moe_block_mfma(gpu):
    """The bf16 MFMA path (h 256, 8 experts, top 2, ff 128) at 600 then 90
    tokens."""
    blk = HostBlock(256, 8, 2, 128, 0, {"router": DENSE, "experts": (4, 64, BF16)}, seed=97,
                    random_experts=True)
    bw = blk.upload(gpu)
    for i, T in enumerate((600, 90)):
        print(f"[case] noalloc mfma T={T} (call {i + 1})", flush=True)
        x = synth.normal(9200 + T, T * 256).reshape(T, 256)
        bias = zipf_bias(T, 8, seed=T, s=0.5)
        got = run(gpu, bw, x, T, bias, PATH_MFMA, True)
        ref = run(gpu, bw, x, T, bias, PATH_MFMA, False)
        same(got, ref)


def test_noalloc_rejects_oversize_and_workspace(gpu, c3):
    """A shape whose workspace exceeds the scratch array fails with a shape
    error before anything runs; so does a call that passes a workspace."""
    blk, bw = c3
    T = 2048
    assert bw.workspace_elems(T) * 4 > SCRATCH_BYTES
    x = gpu.zeros(T * 2048)
    out = gpu.zeros(T * 2048)
    with pytest.raises(ShapeError, match="no-allocation scratch"):
        with gpu.batch() as b:
            b.moe_block_noalloc(bw, x, out, T)
    ws = gpu.zeros(bw.workspace_elems(1))
    from hip_backend.api import _lib, MoeBlockIOC
    io = MoeBlockIOC()
    io.workspace = ws.c
    import ctypes as C
    with gpu.batch():
        st = _lib.moe_block_noalloc(gpu._h, C.byref(bw.c), x.view(0, 2048).c, out.view(0, 2048).c, 1,
                                    C.byref(io))
    assert st == 3
    for buf in (x, out, ws):
        gpu.release(buf)
