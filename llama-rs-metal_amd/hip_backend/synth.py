"""Seeded synthetic inputs for the benchmark configurations.

- `normal`: the reference fixture LCG (s = s*6364136223846793005 + 1,
  crates/llama-rs/tests/common/mod.rs:86-97) with u = ((s>>32)+0.5)/2^32
  feeding Box-Muller in float64, vectorised by LCG jump-ahead.
- `quantize_affine`: MLX-affine quantizer (per group: scale=(max-min)/(2^b-1),
  bias=min, both rounded to the scale dtype; codes rint((w-bias)/scale)
  clamped), packed low bits first into little-endian uint32 words.
- `random_affine`: uniformly random codes with per-group scale/bias of the
  size a quantised N(0, 0.02) group has -- the benchmark's stand-in for
  multi-GB expert tensors, whose values do not affect the kernels' work.
"""
import numpy as np

from .api import BF16, F16, F32

_A = 6364136223846793005
_M = (1 << 64) - 1


def lcg_states(seed, n):
    """The first n LCG states after `seed` (s1 .. sn)."""
    out = np.empty(n, np.uint64)
    if n == 0:
        return out
    out[0] = (seed * _A + 1) & _M
    filled, a_pow, c_acc = 1, _A, 1
    with np.errstate(over="ignore"):
        while filled < n:
            m = min(filled, n - filled)
            out[filled:filled + m] = out[:m] * np.uint64(a_pow) + np.uint64(c_acc)
            c_acc = (c_acc * (a_pow + 1)) & _M
            a_pow = (a_pow * a_pow) & _M
            filled += m
    return out


def normal(seed, n, mean=0.0, std=1.0):
    pairs = (n + 1) // 2
    s = lcg_states(seed, 2 * pairs)
    u = ((s >> np.uint64(32)).astype(np.float64) + 0.5) / 4294967296.0
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    t = 6.283185307179586476925286766559 * u2
    z = np.empty(2 * pairs, np.float64)
    z[0::2] = r * np.cos(t)
    z[1::2] = r * np.sin(t)
    # mean and std enter as float32 values widened to float64
    mean, std = float(np.float32(mean)), float(np.float32(std))
    return (mean + std * z[:n]).astype(np.float32)


def f32_to_bf16_bits(x):
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((b[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def _round_scale(v, scale_type):
    if scale_type == BF16:
        bits = f32_to_bf16_bits(v)
        return bits, bf16_bits_to_f32(bits)
    if scale_type == F16:
        h = v.astype(np.float16)
        return h.view(np.uint16), h.astype(np.float32)
    return v.astype(np.float32), v.astype(np.float32)


def pack_codes(codes, bits):
    codes = np.ascontiguousarray(codes, np.uint32).reshape(-1, 32 // bits)
    shifts = (np.arange(32 // bits, dtype=np.uint32) * bits)
    return np.bitwise_or.reduce(codes << shifts, axis=1).astype(np.uint32)


def quantize_affine(w, bits, group, scale_type):
    w = np.ascontiguousarray(w, np.float32).reshape(-1, group)
    qmax = np.float32((1 << bits) - 1)
    mn = w.min(axis=1)
    mx = w.max(axis=1)
    sbits, s = _round_scale((mx - mn) / qmax, scale_type)
    bbits, b = _round_scale(mn, scale_type)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.rint((w - b[:, None]) / s[:, None])
    q = np.where(s[:, None] > 0, q, 0.0)
    q = np.clip(q, 0, qmax).astype(np.uint32)
    return pack_codes(q.ravel(), bits), sbits, bbits


def random_affine(seed, n, bits, group, scale_type, std=0.02):
    """(packed, scales, biases) with uniform codes; see module docstring."""
    rng = np.random.Generator(np.random.PCG64(seed))
    packed = rng.integers(0, 1 << 32, size=n * bits // 32, dtype=np.uint32)
    ng = n // group
    qmax = (1 << bits) - 1
    span = std * 2 * 2.4  # max - min of a ~64-sample N(0, std) group
    scale = (span / qmax) * (1.0 + 0.1 * rng.standard_normal(ng))
    bias = -0.5 * span * (1.0 + 0.1 * rng.standard_normal(ng))
    sbits, _ = _round_scale(scale.astype(np.float32), scale_type)
    bbits, _ = _round_scale(bias.astype(np.float32), scale_type)
    return packed, sbits, bbits


SCALE_NP = {F32: np.float32, F16: np.uint16, BF16: np.uint16}
