"""bench.py's measurement and synthetic-weight helpers over libmoe_probe.so.

Not part of the MoE path or of include/moe_hip.h: the peaks the roofline
fractions are priced against, re-measured on the GPU (an MFMA-only loop and a
streaming HBM read), and the benchmark configurations' seeded weights
generated on the GPU -- the LCG stream of hip_backend.synth.normal through
Box-Muller (in float on the GPU: within ~1e-6 of the host's double
evaluation) and the documented affine quantizer of synth.quantize_affine --
without generating or uploading multi-GB tensors from the host.
"""
import ctypes as C
import os

import numpy as np

from .api import BF16, F16, F32, MoeRegionC, MoeWeightC, Tensor, Weight, _check

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBE_PATH = os.path.join(PKG_DIR, "libmoe_probe.so")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(PROBE_PATH):
            raise OSError(f"{PROBE_PATH} is missing: build it first (python llama-rs-metal_amd/build.py)")
        L = C.CDLL(PROBE_PATH)
        P, U32, U64, I32, F = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int, C.c_float
        for name, args in {
            "probe_mfma_peak": [I32, I32, I32, C.POINTER(C.c_double)],
            "probe_hbm_read": [U64, I32, C.POINTER(C.c_double)],
            "probe_synth_normal": [P, U64, U64, F, F],
            "probe_synth_affine": [P, P, P, U64, U32, U32, U32, U64, F, F],
        }.items():
            f = getattr(L, name)
            f.restype = I32
            f.argtypes = args
        _lib = L
    return _lib


def _ok(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed: hipError {rc}")


def mfma_peak(kind="bf16", iters=None, reps=3):
    """Dense matrix-core rate in TFLOP/s: kind "bf16" (v_mfma_f32_32x32x16_bf16)
    or "f32" (v_mfma_f32_32x32x2_f32), eight 4-wave blocks per CU."""
    k = 0 if kind == "bf16" else 1
    iters = iters or (8000 if k == 0 else 1000)
    out = C.c_double()
    _ok(lib().probe_mfma_peak(k, iters, reps, C.byref(out)), "probe_mfma_peak")
    return out.value


def hbm_read(nbytes=2 << 30, reps=5):
    """Streaming-read rate in GB/s over `nbytes` of fresh device memory."""
    out = C.c_double()
    _ok(lib().probe_hbm_read(nbytes, reps, C.byref(out)), "probe_hbm_read")
    return out.value


def _scalar_bytes(t):
    return 4 if t == F32 else 2


def alloc_regions(gpu, sizes):
    """Owned, zeroed device regions of the given byte sizes (each its own
    allocation; a region's length is exact even when the allocation rounds up
    to 4-byte elements)."""
    regs, bufs = [], []
    for n in sizes:
        b = gpu.zeros((n + 3) // 4)
        r = MoeRegionC()
        r.ptr, r.bytes = b.ptr, n
        regs.append(r)
        bufs.append(b)
    return regs, bufs


def synth_affine_weight(gpu, dims, bits, group, scale_type, seed, std=0.02, mean=0.0):
    """An affine Weight of `dims`: synth.quantize_affine of the seeded N(mean,
    std) stream (probe_synth_normal's values), generated on the GPU."""
    n = int(np.prod(dims))
    sb = (n // group) * _scalar_bytes(scale_type)
    (rd, rs, rb), bufs = alloc_regions(gpu, [n * bits // 8, sb, sb])
    _ok(lib().probe_synth_affine(rd.ptr, rs.ptr, rb.ptr, n, bits, group, scale_type, seed, mean, std),
        "probe_synth_affine")
    c = MoeWeightC()
    c.data, c.scales, c.biases = rd, rs, rb
    c.bits, c.group_size, c.scale_type = bits, group, scale_type
    c.ndims = len(dims)
    for i, d in enumerate(dims):
        c.dims[i] = d
    w = Weight(c, [rd, rs, rb], dims, bits)
    w.buffers = bufs
    return w


def synth_dense_weight(gpu, dims, seed, std=0.02, mean=0.0):
    """An F32 Weight of `dims` holding the seeded N(mean, std) stream of
    synth.normal(seed, n, mean, std) (Box-Muller in float), generated on the
    GPU."""
    n = int(np.prod(dims))
    (rd,), bufs = alloc_regions(gpu, [4 * n])
    _ok(lib().probe_synth_normal(rd.ptr, n, seed, mean, std), "probe_synth_normal")
    c = MoeWeightC()
    c.data = rd
    c.dtype = F32
    c.ndims = len(dims)
    for i, d in enumerate(dims):
        c.dims[i] = d
    w = Weight(c, [rd], dims, 0)
    w.buffers = bufs
    return w


def to_host(gpu, w):
    """The host Tensor of a Weight made by this module (read back)."""
    def raw(i, dtype):
        return gpu.read(w.buffers[i]).view(np.uint8)[:w.regions[i].bytes].view(dtype).copy()
    if w.bits == 0:
        return Tensor.dense(w.dims, raw(0, np.float32))
    st = w.c.scale_type
    sdt = np.float32 if st == F32 else np.uint16
    return Tensor.affine(w.dims, raw(0, np.uint32), raw(1, sdt), raw(2, sdt), w.bits, w.c.group_size, st)


def synth_normal(gpu, n, seed, std=1.0, mean=0.0):
    """A Buffer of n values of the seeded N(mean, std) stream."""
    b = gpu.zeros(n)
    _ok(lib().probe_synth_normal(b.ptr, n, seed, mean, std), "probe_synth_normal")
    return b


def release(gpu, w):
    """Free the device regions of a Weight made by this module."""
    for b in w.buffers:
        gpu.release(b)
    w.buffers = []
