"""Python mirror of metal_backend's Gpu / Batch / Buffer / Weight over the C ABI.

Names, argument meaning and error behaviour follow the reference's op
surface (crates/metal-backend/src/apple.rs, apple/commands.rs,
apple/memory.rs, apple/ops/*.rs) so code written against it reads the same:

    gpu = Gpu()
    weight = gpu.weight_tensor(tensor)
    with gpu.batch() as b:
        b.route(logits, ids, probabilities, True)
        b.expert_matmul(weight, x, ids, out, False)
    out_host = gpu.read(out)

Every call goes through libmoe_hip.so; there is no CPU fallback.  A missing
library raises at import of the first Gpu.
"""
import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libmoe_hip.so")

F32, F16, BF16 = 0, 1, 30  # crates/model-format/src/dtype.rs:5-15
PATH_AUTO, PATH_OPS, PATH_GROUPED, PATH_MFMA = 0, 1, 2, 3


# --------------------------------------------------------------- errors --
class MoeError(Exception):
    """metal_backend::Error (crates/metal-backend/src/lib.rs:5-14)."""


class UnavailableError(MoeError):
    pass


class GpuError(MoeError):
    pass


class ShapeError(MoeError):
    pass


class AllocationError(MoeError):
    """Error::Allocation(usize): `bytes` is the requested size."""

    def __init__(self, msg="", bytes=0):
        super().__init__(msg)
        self.bytes = bytes


_ERRORS = {1: UnavailableError, 2: GpuError, 3: ShapeError, 4: AllocationError}


# ------------------------------------------------------------- ctypes ABI --
class MoeBufferC(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("len", C.c_uint64)]


class MoeRegionC(C.Structure):
    _fields_ = [("ptr", C.c_void_p), ("bytes", C.c_uint64)]


class MoeWeightC(C.Structure):
    _fields_ = [
        ("data", MoeRegionC),
        ("scales", MoeRegionC),
        ("biases", MoeRegionC),
        ("dtype", C.c_uint32),
        ("bits", C.c_uint32),
        ("group_size", C.c_uint32),
        ("scale_type", C.c_uint32),
        ("ndims", C.c_uint32),
        ("reserved", C.c_uint32),
        ("dims", C.c_uint64 * 3),
    ]


class MoePackedWeightC(C.Structure):
    _fields_ = [("data", MoeRegionC), ("scales", MoeRegionC), ("biases", MoeRegionC)]


class MoeBlockWeightsC(C.Structure):
    _fields_ = [
        ("router", MoeWeightC),
        ("gate", MoeWeightC),
        ("up", MoeWeightC),
        ("down", MoeWeightC),
        ("shared_gate", MoeWeightC),
        ("shared_up", MoeWeightC),
        ("shared_down", MoeWeightC),
        ("shared_gate_inp", MoeWeightC),
        ("has_shared", C.c_uint32),
        ("experts_used", C.c_uint32),
        ("normalize", C.c_uint32),
        ("reserved", C.c_uint32),
        ("gate_packed", MoePackedWeightC),
        ("up_packed", MoePackedWeightC),
        ("down_packed", MoePackedWeightC),
        ("shared_gate_packed", MoePackedWeightC),
        ("shared_up_packed", MoePackedWeightC),
        ("shared_down_packed", MoePackedWeightC),
    ]


class MoeBlockLayoutC(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "logits", "ids", "weights", "counts", "offsets", "perm", "pos", "tiles", "ntiles", "xb16",
        "tile_pairs_mfma", "tile_pairs_batched", "total")]


class MoeBlockIOC(C.Structure):
    _fields_ = [
        ("workspace", MoeBufferC),
        ("logit_bias", MoeBufferC),
        ("logits_out", MoeBufferC),
        ("ids_out", MoeBufferC),
        ("weights_out", MoeBufferC),
        ("norm_weight", MoeBufferC),
        ("norm_eps", C.c_float),
        ("residual", C.c_uint32),
        ("path", C.c_uint32),
        ("reserved", C.c_uint32),
    ]


# Every symbol include/moe_hip.h declares, with its signature.
P, U32, U64, I32, F = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int, C.c_float
BUF = MoeBufferC
SIGNATURES = {
    "moe_gpu_create": (I32, [I32, C.POINTER(C.c_void_p)]),
    "moe_gpu_destroy": (None, [P]),
    "moe_gpu_name": (I32, [P, C.c_char_p, C.c_size_t]),
    "moe_allocated_bytes": (U64, [P]),
    "moe_last_error": (C.c_char_p, [P]),
    "moe_last_error_bytes": (U64, [P]),
    "moe_zeros": (I32, [P, U64, C.POINTER(BUF)]),
    "moe_upload": (I32, [P, P, U64, C.POINTER(BUF)]),
    "moe_upload_bytes": (I32, [P, P, U64, C.POINTER(MoeRegionC)]),
    "moe_read": (I32, [P, BUF, P]),
    "moe_write": (I32, [P, BUF, P]),
    "moe_clear": (I32, [P, BUF]),
    "moe_release": (I32, [P, P]),
    "moe_register": (I32, [P, P, U64]),
    "moe_unregister": (I32, [P, P]),
    "moe_view": (I32, [BUF, U64, U64, C.POINTER(BUF)]),
    "moe_batch_begin": (I32, [P]),
    "moe_batch_finish": (I32, [P, C.POINTER(C.c_double)]),
    "moe_matmul": (I32, [P, C.POINTER(MoeWeightC), BUF, BUF, U64]),
    "moe_expert_matmul": (I32, [P, C.POINTER(MoeWeightC), BUF, BUF, BUF, I32]),
    "moe_route": (I32, [P, BUF, BUF, BUF, I32]),
    "moe_swiglu": (I32, [P, BUF, BUF, BUF]),
    "moe_mix": (I32, [P, BUF, BUF, BUF]),
    "moe_gate_scalar": (I32, [P, BUF, BUF, BUF]),
    "moe_add": (I32, [P, BUF, BUF, BUF]),
    "moe_norm": (I32, [P, BUF, C.POINTER(MoeWeightC), BUF, U64, U64, F]),
    "moe_route_tokens": (I32, [P, BUF, BUF, BUF, U64, I32]),
    "moe_dispatch": (I32, [P, BUF, U64, U64, U64, BUF, BUF, BUF, BUF]),
    "moe_pack_size": (I32, [C.POINTER(MoeWeightC), C.POINTER(U64), C.POINTER(U64)]),
    "moe_pack_weight": (I32, [P, C.POINTER(MoeWeightC), MoePackedWeightC]),
    "moe_block_workspace": (I32, [C.POINTER(MoeBlockWeightsC), U64, C.POINTER(U64)]),
    "moe_block_workspace_layout": (I32, [C.POINTER(MoeBlockWeightsC), U64, C.POINTER(MoeBlockLayoutC)]),
    "moe_block": (I32, [P, C.POINTER(MoeBlockWeightsC), BUF, BUF, U64, C.POINTER(MoeBlockIOC)]),
    "moe_block_noalloc": (I32, [P, C.POINTER(MoeBlockWeightsC), BUF, BUF, U64, C.POINTER(MoeBlockIOC)]),
    "moe_profile_enable": (I32, [P, I32]),
    "moe_profile_count": (I32, [P, C.POINTER(U32)]),
    "moe_profile_get": (I32, [P, U32, C.c_char_p, C.c_size_t, C.POINTER(U64),
                              C.POINTER(C.c_double)]),
    "moe_profile_reset": (I32, [P]),
    "moe_profile_hold": (I32, [P, U32]),
    "moe_graph_begin": (I32, [P]),
    "moe_graph_end": (I32, [P, C.POINTER(C.c_void_p)]),
    "moe_graph_launch": (I32, [P, P]),
    "moe_graph_destroy": (None, [P]),
    "moe_copy": (I32, [P, BUF, BUF]),
    "moe_version": (C.c_char_p, []),
}

_lib = None


def load_library(path=LIB_PATH):
    """Load libmoe_hip.so and bind every declared symbol (raises if absent)."""
    global _lib
    if _lib is not None and path == LIB_PATH:
        return _lib
    if not os.path.exists(path):
        raise UnavailableError(
            f"{path} is missing: build it first (python llama-rs-metal_amd/build.py)")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    if path == LIB_PATH:
        _lib = lib
    return lib


# ------------------------------------------------------------ host tensor --
class Tensor:
    """model_format::Tensor (crates/model-format/src/checkpoint.rs:63-196):
    dims ``[in, out(, experts)]``; dense ``data`` of ``dtype`` or MLX affine
    packed uint32 codes with per-group ``scales``/``biases``."""

    def __init__(self, dims, data, dtype=F32, bits=0, group_size=0, scale_type=F32, scales=None,
                 biases=None):
        self.dims = [int(d) for d in dims]
        self.data = np.ascontiguousarray(data)
        self.dtype = dtype
        self.bits = bits
        self.group_size = group_size
        self.scale_type = scale_type
        self.scales = None if scales is None else np.ascontiguousarray(scales)
        self.biases = None if biases is None else np.ascontiguousarray(biases)

    @classmethod
    def dense(cls, dims, values, dtype=F32):
        if dtype == F32:
            data = np.ascontiguousarray(values, np.float32)
        else:
            data = np.ascontiguousarray(values, np.uint16)  # raw f16/bf16 bits
        return cls(dims, data, dtype=dtype)

    @classmethod
    def affine(cls, dims, packed, scales, biases, bits, group_size, scale_type):
        return cls(dims, np.ascontiguousarray(packed, np.uint32), bits=bits, group_size=group_size,
                   scale_type=scale_type, scales=scales, biases=biases)

    def elements(self):
        return int(np.prod(self.dims))


# ------------------------------------------------------------------ handles --
class Buffer:
    """Buffer (crates/metal-backend/src/apple.rs:38-64): view of 4-byte elements."""

    def __init__(self, gpu, c, base):
        self.gpu = gpu
        self.c = c
        self.base = base  # allocation base pointer (for release)

    def __len__(self):
        return int(self.c.len)

    @property
    def ptr(self):
        return int(self.c.ptr)

    def view(self, start, length):
        out = MoeBufferC()
        if _lib.moe_view(self.c, start, length, C.byref(out)) != 0:
            raise ShapeError("view bounds")
        return Buffer(self.gpu, out, self.base)


class Weight:
    """Weight + AffineWeight (apple.rs:65-115): device regions + metadata."""

    def __init__(self, c, regions, dims, bits):
        self.c = c
        self.regions = regions
        self.dims = list(dims)
        self.bits = bits

    def reshape(self, dims):
        """Weight::reshape (apple.rs:65-85)."""
        n = int(np.prod(dims))
        if n != int(np.prod(self.dims)) or 0 in dims:
            raise ShapeError("weight reshape")
        if self.bits and dims[0] != self.dims[0]:
            raise ShapeError("affine reshape must preserve row width")
        c = MoeWeightC.from_buffer_copy(self.c)
        c.ndims = len(dims)
        for i in range(3):
            c.dims[i] = dims[i] if i < len(dims) else 0
        return Weight(c, self.regions, dims, self.bits)


class PackedWeight:
    """MFMA tile-order copy of an affine expert weight (moe_pack_weight; no
    reference counterpart): its three device buffers and the C struct."""

    def __init__(self, c, buffers):
        self.c = c
        self.buffers = buffers


def pack_size(weight):
    """(code bytes, scale-or-bias bytes) of the packed copy of `weight`, or
    None when it has no packed form."""
    db, sb = C.c_uint64(), C.c_uint64()
    if _lib.moe_pack_size(C.byref(weight.c), C.byref(db), C.byref(sb)) != 0:
        return None
    return int(db.value), int(sb.value)


def _empty_weight():
    return MoeWeightC()


class BlockWeights:
    """FeedForward::Moe (crates/model-runtime/src/lib.rs:46-56)."""

    def __init__(self, router, gate, up, down, experts_used, normalize, shared=None,
                 shared_gate=None, packed=None, shared_packed=None):
        c = MoeBlockWeightsC()
        c.router, c.gate, c.up, c.down = router.c, gate.c, up.c, down.c
        if packed is not None:  # PackedWeight copies of (gate, up, down), any of them None
            for name, pw in zip(("gate_packed", "up_packed", "down_packed"), packed):
                if pw is not None:
                    setattr(c, name, pw.c)
        if shared_packed is not None:  # the same for the shared expert's (gate, up, down)
            for name, pw in zip(("shared_gate_packed", "shared_up_packed", "shared_down_packed"),
                                shared_packed):
                if pw is not None:
                    setattr(c, name, pw.c)
        if shared is not None:
            c.shared_gate, c.shared_up, c.shared_down = shared[0].c, shared[1].c, shared[2].c
            c.shared_gate_inp = shared_gate.c
            c.has_shared = 1
        c.experts_used = experts_used
        c.normalize = int(bool(normalize))
        self.c = c
        self.keep = (router, gate, up, down, shared, shared_gate)
        self.packed = packed
        self.shared_packed = shared_packed
        self.hidden = router.dims[0]
        self.experts = router.dims[1]
        self.k = experts_used

    def workspace_elems(self, tokens):
        n = C.c_uint64()
        _check(None, _lib.moe_block_workspace(C.byref(self.c), tokens, C.byref(n)))
        return int(n.value)

    def workspace_layout(self, tokens):
        """Element offsets of the routing and dispatch inside the workspace
        (moe_block_workspace_layout) as a dict."""
        lay = MoeBlockLayoutC()
        _check(None, _lib.moe_block_workspace_layout(C.byref(self.c), tokens, C.byref(lay)))
        return {name: int(getattr(lay, name)) for name, _ in MoeBlockLayoutC._fields_}


def _check(gpu, status):
    if status != 0:
        msg = _lib.moe_last_error(gpu._h).decode() if gpu is not None else ""
        if status == 4:
            raise AllocationError(msg, int(_lib.moe_last_error_bytes(gpu._h)) if gpu is not None else 0)
        raise _ERRORS.get(status, MoeError)(msg)


_NULLBUF = MoeBufferC()


def _c(b):
    return _NULLBUF if b is None else b.c


class Gpu:
    """Gpu (crates/metal-backend/src/apple.rs:125-211)."""

    def __init__(self, device=0):
        load_library()
        h = C.c_void_p()
        st = _lib.moe_gpu_create(device, C.byref(h))
        if st != 0:
            raise _ERRORS.get(st, MoeError)("no usable gfx950 device")
        self._h = h
        buf = C.create_string_buffer(256)
        _lib.moe_gpu_name(h, buf, 256)
        self.name = buf.value.decode()

    def close(self):
        if self._h:
            _lib.moe_gpu_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # memory (apple/memory.rs)
    def zeros(self, n):
        out = MoeBufferC()
        _check(self, _lib.moe_zeros(self._h, n, C.byref(out)))
        return Buffer(self, out, out.ptr)

    def upload(self, data):
        a = np.ascontiguousarray(data)
        if a.dtype != np.float32:
            a = a.view(np.float32) if a.dtype.itemsize == 4 else a.astype(np.float32)
        a = np.ascontiguousarray(a.ravel())
        out = MoeBufferC()
        _check(self, _lib.moe_upload(self._h, a.ctypes.data, a.size, C.byref(out)))
        return Buffer(self, out, out.ptr)

    def upload_u32(self, data):
        return self.upload(np.ascontiguousarray(data, np.uint32).view(np.float32))

    def read(self, b):
        out = np.empty(len(b), np.float32)
        _check(self, _lib.moe_read(self._h, b.c, out.ctypes.data))
        return out

    def read_u32(self, b):
        return self.read(b).view(np.uint32)

    def write(self, b, data):
        a = np.ascontiguousarray(data).ravel()
        if a.dtype != np.float32:
            a = a.view(np.float32) if a.dtype.itemsize == 4 else a.astype(np.float32)
        if a.size != len(b):
            raise ShapeError("write length")
        _check(self, _lib.moe_write(self._h, b.c, a.ctypes.data))

    def clear(self, b):
        _check(self, _lib.moe_clear(self._h, b.c))

    def release(self, b):
        _check(self, _lib.moe_release(self._h, b.base))

    def allocated_bytes(self):
        return int(_lib.moe_allocated_bytes(self._h))

    def _region(self, arr):
        a = np.ascontiguousarray(arr)
        out = MoeRegionC()
        _check(self, _lib.moe_upload_bytes(self._h, a.ctypes.data, a.nbytes, C.byref(out)))
        return out

    # weights (apple/weights.rs:101-141)
    def weight_tensor(self, t):
        c = MoeWeightC()
        c.data = self._region(t.data)
        regions = [c.data]
        if t.bits:
            c.scales = self._region(t.scales)
            c.biases = self._region(t.biases)
            regions += [c.scales, c.biases]
            c.scale_type = t.scale_type
            c.group_size = t.group_size
        else:
            c.dtype = t.dtype
        c.bits = t.bits
        c.ndims = len(t.dims)
        for i, d in enumerate(t.dims):
            c.dims[i] = d
        return Weight(c, regions, t.dims, t.bits)

    def pack_weight(self, weight):
        """Allocate and fill the packed copy of `weight` (one batch); None
        when it has no packed form."""
        sizes = pack_size(weight)
        if sizes is None:
            return None
        db, sb = sizes
        bufs = [self.zeros(db // 4), self.zeros(sb // 4), self.zeros(sb // 4)]
        c = MoePackedWeightC()
        for name, b, n in zip(("data", "scales", "biases"), bufs, (db, sb, sb)):
            r = MoeRegionC()
            r.ptr, r.bytes = b.c.ptr, n
            setattr(c, name, r)
        pw = PackedWeight(c, bufs)
        with self.batch() as b:
            b.pack_weight(weight, pw)
        return pw

    def weight_f32(self, data, dims):
        return self.weight_tensor(Tensor.dense(dims, np.asarray(data, np.float32)))

    # batches (apple/commands.rs:67-99)
    def batch(self):
        return Batch(self)

    def with_batch(self, f):
        with self.batch() as b:
            value = f(b)
        return value, b.seconds

    # profiling (the LLAMA_METAL_PROFILE analogue)
    def profile(self, enable=True):
        _check(self, _lib.moe_profile_enable(self._h, int(enable)))

    def profile_read(self):
        n = C.c_uint32()
        _check(self, _lib.moe_profile_count(self._h, C.byref(n)))
        out = {}
        name = C.create_string_buffer(128)
        for i in range(n.value):
            launches, secs = C.c_uint64(), C.c_double()
            _check(self, _lib.moe_profile_get(self._h, i, name, 128, C.byref(launches),
                                              C.byref(secs)))
            out[name.value.decode()] = (int(launches.value), float(secs.value))
        return out

    def profile_reset(self):
        _check(self, _lib.moe_profile_reset(self._h))

    # graphs
    def capture(self):
        return Capture(self)


class Graph:
    """A captured, instantiated graph.  destroy() frees it (call it after the
    replays have completed); otherwise it is freed on collection."""

    def __init__(self, gpu, h):
        self.gpu, self.h = gpu, h

    def destroy(self):
        if self.h:
            _lib.moe_graph_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Capture:
    """Context manager capturing the ops issued inside into a Graph."""

    def __init__(self, gpu):
        self.gpu = gpu
        self.graph = None
        self.batch = Batch(gpu, begin=False)

    def __enter__(self):
        _check(self.gpu, _lib.moe_graph_begin(self.gpu._h))
        return self.batch

    def __exit__(self, et, ev, tb):
        h = C.c_void_p()
        st = _lib.moe_graph_end(self.gpu._h, C.byref(h))
        if et is None:
            _check(self.gpu, st)
            self.graph = Graph(self.gpu, h)
        return False


class Batch:
    """Batch (crates/metal-backend/src/apple.rs:214-222, apple/ops/*.rs)."""

    def __init__(self, gpu, begin=True):
        self.gpu = gpu
        self.seconds = None
        self._open = False
        if begin:
            _check(gpu, _lib.moe_batch_begin(gpu._h))
            self._open = True

    def __enter__(self):
        return self

    def __exit__(self, et, ev, tb):
        if self._open:
            if et is None:
                self.finish()
            else:
                try:
                    self.finish()
                except MoeError:
                    pass
        return False

    def finish(self):
        """Batch::finish (commands.rs:215-224): waits, returns GPU seconds."""
        s = C.c_double()
        self._open = False
        _check(self.gpu, _lib.moe_batch_finish(self.gpu._h, C.byref(s)))
        self.seconds = s.value
        return s.value

    def _ck(self, st):
        _check(self.gpu, st)

    # matrix.rs
    def matmul(self, w, x, y, tokens):
        self._ck(_lib.moe_matmul(self.gpu._h, C.byref(w.c), x.c, y.c, tokens))

    def expert_matmul(self, w, x, ids, y, per_expert_input):
        self._ck(_lib.moe_expert_matmul(self.gpu._h, C.byref(w.c), x.c, ids.c, y.c,
                                        int(bool(per_expert_input))))

    # sampling.rs
    def route(self, logits, ids, weights, normalize):
        self._ck(_lib.moe_route(self.gpu._h, logits.c, ids.c, weights.c, int(bool(normalize))))

    # elementwise.rs
    def swiglu(self, a, b, y):
        self._ck(_lib.moe_swiglu(self.gpu._h, a.c, b.c, y.c))

    def mix(self, x, w, y):
        self._ck(_lib.moe_mix(self.gpu._h, x.c, w.c, y.c))

    def gate_scalar(self, x, g, y):
        self._ck(_lib.moe_gate_scalar(self.gpu._h, x.c, g.c, y.c))

    def add(self, a, b, y):
        self._ck(_lib.moe_add(self.gpu._h, a.c, b.c, y.c))

    # attention.rs:3-45
    def norm(self, x, w, y, heads, stride, eps):
        self._ck(_lib.moe_norm(self.gpu._h, x.c, C.byref(w.c), y.c, heads, stride, eps))

    # token-batched additions
    def route_tokens(self, logits, ids, weights, tokens, normalize):
        self._ck(_lib.moe_route_tokens(self.gpu._h, logits.c, ids.c, weights.c, tokens,
                                       int(bool(normalize))))

    def dispatch(self, ids, tokens, k, experts, counts, offsets, perm, pos):
        self._ck(_lib.moe_dispatch(self.gpu._h, ids.c, tokens, k, experts, counts.c, offsets.c,
                                   perm.c, pos.c))

    def copy(self, src, dst):
        self._ck(_lib.moe_copy(self.gpu._h, src.c, dst.c))

    def pack_weight(self, weight, packed):
        _check(self.gpu, _lib.moe_pack_weight(self.gpu._h, C.byref(weight.c), packed.c))

    def moe_block(self, bw, x, out, tokens, workspace, logit_bias=None, logits_out=None,
                  ids_out=None, weights_out=None, norm_weight=None, norm_eps=1e-6,
                  residual=False, path=PATH_AUTO):
        io = self._io(workspace, logit_bias, logits_out, ids_out, weights_out, norm_weight, norm_eps,
                      residual, path)
        self._ck(_lib.moe_block(self.gpu._h, C.byref(bw.c), x.c, out.c, tokens, C.byref(io)))

    def moe_block_noalloc(self, bw, x, out, tokens, logit_bias=None, logits_out=None, ids_out=None,
                          weights_out=None, norm_weight=None, norm_eps=1e-6, residual=False,
                          path=PATH_AUTO):
        """moe_block with the library's per-GPU scratch array as its workspace
        (moe_block_noalloc: nothing is allocated)."""
        io = self._io(None, logit_bias, logits_out, ids_out, weights_out, norm_weight, norm_eps,
                      residual, path)
        self._ck(_lib.moe_block_noalloc(self.gpu._h, C.byref(bw.c), x.c, out.c, tokens, C.byref(io)))

    @staticmethod
    def _io(workspace, logit_bias, logits_out, ids_out, weights_out, norm_weight, norm_eps, residual,
            path):
        io = MoeBlockIOC()
        io.workspace = _c(workspace)
        io.logit_bias = _c(logit_bias)
        io.logits_out = _c(logits_out)
        io.ids_out = _c(ids_out)
        io.weights_out = _c(weights_out)
        io.norm_weight = _c(norm_weight)
        io.norm_eps = norm_eps
        io.residual = int(bool(residual))
        io.path = path
        return io

    def graph(self, graph):
        self._ck(_lib.moe_graph_launch(self.gpu._h, graph.h))

    def hold(self, microseconds):
        """Occupy the stream for `microseconds` so the launches enqueued next
        are queued before the GPU reaches them (profiled durations then
        exclude host enqueue gaps)."""
        self._ck(_lib.moe_profile_hold(self.gpu._h, int(microseconds)))
