"""The benchmark's GPU helpers (libmoe_probe.so): the seeded synthetic weights
follow the host generator (hip_backend.synth: the reference fixture LCG,
Box-Muller, the documented affine quantizer), and the peak probes run."""
import numpy as np
import pytest

from hip_backend import BF16, F16, F32, probe, synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,seed", [(4096, 7), (100_003, 12345)])
def test_synth_normal_follows_the_host_stream(gpu, n, seed):
    """The device stream is synth.normal's: the same LCG states and
    Box-Muller pairs (odd n ends on the cosine half of a pair); only the float
    (device) versus double (host) evaluation differs."""
    dev = gpu.read(probe.synth_normal(gpu, n, seed, std=1.0))
    host = synth.normal(seed, n)
    np.testing.assert_allclose(dev, host, rtol=0, atol=2e-5)
    # a shifted stream would not match
    assert not np.allclose(dev[1:], host[:-1], atol=1e-2)


@pytest.mark.parametrize("bits,group,st", [(2, 32, BF16), (4, 64, BF16), (4, 128, F16), (8, 64, F32),
                                           (8, 128, BF16)])
def test_synth_affine_is_the_host_quantizer(gpu, bits, group, st):
    """probe_synth_affine's codes, scales and biases are exactly
    synth.quantize_affine of the device's own normal values, and decode to
    values within half a step of them."""
    n = 64 * 1024
    dims = [256, n // 256]
    w = probe.synth_affine_weight(gpu, dims, bits, group, st, seed=900 + bits, std=0.02)
    t = probe.to_host(gpu, w)
    vals = gpu.read(probe.synth_normal(gpu, n, 900 + bits, std=0.02))
    codes, s, b = synth.quantize_affine(vals, bits, group, st)
    assert np.array_equal(t.data, codes)
    assert np.array_equal(np.asarray(t.scales).view(np.uint8), np.asarray(s).view(np.uint8))
    assert np.array_equal(np.asarray(t.biases).view(np.uint8), np.asarray(b).view(np.uint8))
    import oracle
    dec = oracle.decode(t)
    sc = oracle.decode(type(t).affine(dims, synth.pack_codes(np.ones(n, np.uint32), bits), t.scales,
                                      np.zeros_like(t.biases), bits, group, st))
    # round-to-nearest codes: half a step, plus the rounding of scale and bias
    # to the scale dtype (which the clamp to 2^bits - 1 can expose)
    qmax = (1 << bits) - 1
    rnd = 2.0 ** -8 if st == BF16 else (2.0 ** -11 if st == F16 else 2.0 ** -24)
    bi = oracle.decode(type(t).affine(dims, synth.pack_codes(np.zeros(n, np.uint32), bits), t.scales,
                                      t.biases, bits, group, st))
    assert (np.abs(dec - vals) <= 0.5 * sc + rnd * (qmax * sc + np.abs(bi)) + 1e-8).all()
    assert abs(float(np.std(dec)) - 0.02) < 2e-3
    probe.release(gpu, w)


def test_peak_probes_run(gpu):
    """The MFMA-only loops and the streaming read return rates (short runs)."""
    assert probe.mfma_peak("bf16", iters=200, reps=1) > 100.0
    assert probe.mfma_peak("f32", iters=50, reps=1) > 10.0
    assert probe.hbm_read(256 << 20, reps=1) > 500.0
