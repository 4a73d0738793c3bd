"""ctypes view of the CPU oracle (moe_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check and by the
cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never as the product path.  Each wrapper names the reference
file:line its C function restates (see moe_oracle.h for the pinning status).

Weights are passed as any object with the attributes of
model_format::Tensor (crates/model-format/src/checkpoint.rs:63-86):
``dims`` (list, ``[in, out(, experts)]``), ``bits`` (0 for dense),
``dtype`` (0/1/30 when dense), ``group_size``, ``scale_type`` and the numpy
arrays ``data`` (dense elements or packed uint32 codes), ``scales``,
``biases``.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")


def build():
    """Compile liboracle.so with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, "liboracle.so"], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    return C.CDLL(LIB_PATH)


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
        _declare(_lib)
    return _lib


class OrcWeight(C.Structure):
    _fields_ = [
        ("data", C.c_void_p),
        ("scales", C.c_void_p),
        ("biases", C.c_void_p),
        ("dtype", C.c_uint32),
        ("bits", C.c_uint32),
        ("group_size", C.c_uint32),
        ("scale_type", C.c_uint32),
        ("ndims", C.c_uint32),
        ("pad_", C.c_uint32),
        ("dims", C.c_uint64 * 3),
    ]


class OrcMoe(C.Structure):
    _fields_ = [
        ("router", OrcWeight),
        ("gate", OrcWeight),
        ("up", OrcWeight),
        ("down", OrcWeight),
        ("sh_gate", OrcWeight),
        ("sh_up", OrcWeight),
        ("sh_down", OrcWeight),
        ("sh_gate_inp", OrcWeight),
        ("has_shared", C.c_uint32),
        ("k", C.c_uint32),
        ("normalize", C.c_uint32),
        ("pad_", C.c_uint32),
    ]


P = C.c_void_p
U32, U64, F32, I32 = C.c_uint32, C.c_uint64, C.c_float, C.c_int


def _declare(L):
    sig = {
        "orc_f16_to_f32": (F32, [C.c_uint16]),
        "orc_bf16_to_f32": (F32, [C.c_uint16]),
        "orc_f32_to_bf16": (C.c_uint16, [F32]),
        "orc_f32_to_f16": (C.c_uint16, [F32]),
        "orc_weight_validate": (I32, [P]),
        "orc_weight_decode_rows": (I32, [P, U64, U64, P]),
        "orc_matvec": (None, [P, P, U64, U64, P]),
        "orc_softmax": (None, [P, U64, P]),
        "orc_silu": (F32, [F32]),
        "orc_rms_norm": (None, [P, P, U64, F32, P]),
        "orc_route": (None, [P, U32, U32, I32, P, P]),
        "orc_swiglu": (None, [P, P, P, U64]),
        "orc_mix": (None, [P, P, U32, U64, P]),
        "orc_gate_scalar": (None, [P, P, P, U64]),
        "orc_add": (None, [P, P, P, U64]),
        "orc_matmul": (I32, [P, P, P, U64]),
        "orc_expert_matmul": (I32, [P, P, P, U32, P, I32]),
        "orc_dispatch": (I32, [P, U32, U32, U32, P, P, P, P]),
        "orc_moe_block": (I32, [P, P, U32, P, P, P, P, P, P]),
        "orc_moe_block_em": (I32, [P, P, U32, P, P, P, P, P, P]),
        "orc_moe_stack": (I32, [P, P, U32, F32, P, U32]),
        "orc_normal": (None, [U64, U64, F32, F32, P]),
        "orc_quantize_affine": (I32, [P, U64, U32, U32, U32, P, P, P]),
        "orc_affine_pattern": (I32, [U64, U32, U32, U32, P, P, P]),
        "orc_set_threads": (None, [I32]),
        "orc_threads": (I32, []),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def scale_np_dtype(scale_type):
    return np.float32 if scale_type == 0 else np.uint16


def weight_struct(t):
    """OrcWeight for a Tensor-like object; keeps its arrays alive via the caller."""
    w = OrcWeight()
    w.data = t.data.ctypes.data
    w.scales = t.scales.ctypes.data if t.bits else None
    w.biases = t.biases.ctypes.data if t.bits else None
    w.dtype = t.dtype if not t.bits else 0
    w.bits = t.bits
    w.group_size = t.group_size if t.bits else 0
    w.scale_type = t.scale_type if t.bits else 0
    w.ndims = len(t.dims)
    for i, d in enumerate(t.dims):
        w.dims[i] = d
    return w


# ------------------------------------------------------------------ dtypes --
def f16_to_f32(h):
    return lib().orc_f16_to_f32(int(h))


def bf16_to_f32(h):
    return lib().orc_bf16_to_f32(int(h))


def f32_to_bf16(f):
    return lib().orc_f32_to_bf16(float(f))


def f32_to_f16(f):
    return lib().orc_f32_to_f16(float(f))


# ------------------------------------------------------------------ decode --
def decode(t, row0=0, nrows=None):
    """Tensor::decode (checkpoint.rs:164-196) over rows of dims[0] elements."""
    total_rows = int(np.prod(t.dims)) // t.dims[0]
    if nrows is None:
        nrows = total_rows - row0
    out = np.empty(nrows * t.dims[0], np.float32)
    rc = lib().orc_weight_decode_rows(C.byref(weight_struct(t)), row0, nrows, _p(out))
    if rc:
        raise ValueError("invalid affine/dense tensor")
    return out


def validate(t):
    return lib().orc_weight_validate(C.byref(weight_struct(t)))


# -------------------------------------------------------------- tensor-core --
def matvec(w, x):
    """tensor_core::matvec (crates/tensor-core/src/lib.rs:80-85)."""
    w, x = _f32(w), _f32(x)
    rows = w.size // x.size
    y = np.empty(rows, np.float32)
    lib().orc_matvec(_p(w), _p(x), rows, x.size, _p(y))
    return y


def softmax(x):
    """tensor_core::softmax (lib.rs:71-79)."""
    x = _f32(x)
    y = np.empty_like(x)
    lib().orc_softmax(_p(x), x.size, _p(y))
    return y


def silu(x):
    """tensor_core::silu (lib.rs:86-88)."""
    return lib().orc_silu(float(x))


def rms_norm(x, w, eps):
    """tensor_core::rms_norm (lib.rs:64-70)."""
    x, w = _f32(x), _f32(w)
    y = np.empty_like(x)
    lib().orc_rms_norm(_p(x), _p(w), x.size, eps, _p(y))
    return y


# ------------------------------------------------------------------ routing --
def route(logits, k, normalize):
    """route kernel (crates/metal-backend/src/shaders/sampling.metal:1-36)."""
    x = _f32(logits)
    ids = np.empty(k, np.uint32)
    w = np.empty(k, np.float32)
    lib().orc_route(_p(x), x.size, k, int(bool(normalize)), _p(ids), _p(w))
    return ids, w


def route_tokens(logits, k, normalize):
    """route applied to each row of logits[T, E]."""
    logits = _f32(logits)
    T, E = logits.shape
    ids = np.empty((T, k), np.uint32)
    w = np.empty((T, k), np.float32)
    for t in range(T):
        ids[t], w[t] = route(logits[t], k, normalize)
    return ids, w


# -------------------------------------------------------------- elementwise --
def swiglu(a, b):
    """activation (elementwise.metal:8-17)."""
    a, b = _f32(a), _f32(b)
    y = np.empty_like(a)
    lib().orc_swiglu(_p(a), _p(b), _p(y), a.size)
    return y


def mix(x, w):
    """mix (elementwise.metal:47-57)."""
    x, w = _f32(x), _f32(w)
    n = x.size // w.size
    y = np.empty(n, np.float32)
    lib().orc_mix(_p(x), _p(w), w.size, n, _p(y))
    return y


def gate_scalar(x, g):
    """gate_scalar (elementwise.metal:65-72)."""
    x, g = _f32(x), _f32(np.atleast_1d(g))
    y = np.empty_like(x)
    lib().orc_gate_scalar(_p(x), _p(g), _p(y), x.size)
    return y


def add(a, b):
    """add (elementwise.metal:1-7)."""
    a, b = _f32(a), _f32(b)
    y = np.empty_like(a)
    lib().orc_add(_p(a), _p(b), _p(y), a.size)
    return y


# ----------------------------------------------------------------- products --
def matmul(t, x, tokens):
    """Batch::matmul (crates/metal-backend/src/apple/ops/matrix.rs:63-148)."""
    x = _f32(x)
    y = np.empty(t.dims[1] * tokens, np.float32)
    rc = lib().orc_matmul(C.byref(weight_struct(t)), _p(x), _p(y), tokens)
    if rc:
        raise ValueError("matmul shape")
    return y


def expert_matmul(t, x, ids, per_expert_input):
    """Batch::expert_matmul (matrix.rs:149-205)."""
    x = _f32(x)
    ids = np.ascontiguousarray(ids, np.uint32)
    y = np.empty(t.dims[1] * ids.size, np.float32)
    rc = lib().orc_expert_matmul(C.byref(weight_struct(t)), _p(x), _p(ids), ids.size, _p(y),
                                 int(bool(per_expert_input)))
    if rc:
        raise ValueError("expert matmul shape")
    return y


def dispatch(ids, experts):
    """Stable counting sort of (token, k) pairs by expert (no reference counterpart)."""
    ids = np.ascontiguousarray(ids, np.uint32)
    T, K = ids.shape
    counts = np.empty(experts, np.uint32)
    offsets = np.empty(experts + 1, np.uint32)
    perm = np.empty(T * K, np.uint32)
    pos = np.empty(T * K, np.uint32)
    rc = lib().orc_dispatch(_p(ids), T, K, experts, _p(counts), _p(offsets), _p(perm), _p(pos))
    if rc:
        raise ValueError("expert id out of range")
    return counts, offsets, perm, pos


class MoeSpec:
    """Weights of one MoE block, Tensor-like objects keyed as the reference
    binds them (crates/model-runtime/src/loader.rs:172-203)."""

    def __init__(self, router, gate, up, down, k, normalize, shared=None, shared_gate=None):
        self.router, self.gate, self.up, self.down = router, gate, up, down
        self.shared = shared  # (gate, up, down) or None
        self.shared_gate = shared_gate
        self.k, self.normalize = k, normalize

    def struct(self):
        m = OrcMoe()
        m.router = weight_struct(self.router)
        m.gate = weight_struct(self.gate)
        m.up = weight_struct(self.up)
        m.down = weight_struct(self.down)
        if self.shared is not None:
            m.sh_gate = weight_struct(self.shared[0])
            m.sh_up = weight_struct(self.shared[1])
            m.sh_down = weight_struct(self.shared[2])
            m.sh_gate_inp = weight_struct(self.shared_gate)
            m.has_shared = 1
        m.k = self.k
        m.normalize = int(bool(self.normalize))
        return m


def moe_block(spec, x, tokens, logit_bias=None, logits_in=None, expert_major=False):
    """MoE block composition (crates/model-runtime/src/execute.rs:208-233).
    Returns (out[T,h], logits[T,E], ids[T,K], weights[T,K]).  With
    expert_major the same values come from orc_moe_block_em (each expert
    decoded once per 4096 tokens instead of once per pair)."""
    h = spec.gate.dims[0]
    E = spec.gate.dims[2]
    K = spec.k
    x = _f32(x)
    out = np.empty((tokens, h), np.float32)
    logits = np.empty((tokens, E), np.float32)
    ids = np.empty((tokens, K), np.uint32)
    w = np.empty((tokens, K), np.float32)
    lb = None if logit_bias is None else _f32(logit_bias)
    li = None if logits_in is None else _f32(logits_in)
    m = spec.struct()
    fn = lib().orc_moe_block_em if expert_major else lib().orc_moe_block
    rc = fn(C.byref(m), _p(x), tokens, _p(lb), _p(li), _p(out), _p(logits), _p(ids), _p(w))
    if rc:
        raise ValueError("moe block shape")
    return out, logits, ids, w


def moe_stack(specs, norm_ws, eps, hidden, tokens):
    """RMSNorm -> MoE -> residual per layer (execute.rs:197,236)."""
    hidden = _f32(hidden).copy()
    arr = (OrcMoe * len(specs))(*[s.struct() for s in specs])
    nws = [_f32(w) for w in norm_ws]
    ptrs = (C.c_void_p * len(nws))(*[w.ctypes.data for w in nws])
    rc = lib().orc_moe_stack(arr, ptrs, len(specs), eps, _p(hidden), tokens)
    if rc:
        raise ValueError("moe stack")
    return hidden


# ---------------------------------------------------------- synthetic data --
def normal(seed, n, mean=0.0, std=1.0):
    """Reference fixture LCG (crates/llama-rs/tests/common/mod.rs:86-97) + Box-Muller."""
    out = np.empty(n, np.float32)
    lib().orc_normal(seed, n, mean, std, _p(out))
    return out


def quantize_affine(w, bits, group, scale_type):
    """This build's affine quantizer; returns (packed u32, scales, biases)."""
    w = _f32(w).ravel()
    n = w.size
    packed = np.empty(n * bits // 32, np.uint32)
    sd = scale_np_dtype(scale_type)
    scales = np.empty(n // group, sd)
    biases = np.empty(n // group, sd)
    rc = lib().orc_quantize_affine(_p(w), n, bits, group, scale_type, _p(packed), _p(scales),
                                   _p(biases))
    if rc:
        raise ValueError("quantize")
    return packed, scales, biases


def affine_pattern(n, bits, group, scale_type):
    """Deterministic pattern of crates/metal-backend/tests/affine.rs:3-45."""
    packed = np.empty(n * bits // 32, np.uint32)
    sd = scale_np_dtype(scale_type)
    scales = np.empty(n // group, sd)
    biases = np.empty(n // group, sd)
    rc = lib().orc_affine_pattern(n, bits, group, scale_type, _p(packed), _p(scales), _p(biases))
    if rc:
        raise ValueError("pattern")
    return packed, scales, biases


def set_threads(n):
    """Threads of the oracle's parallel loops (1: the scalar baseline)."""
    lib().orc_set_threads(int(n))


def threads():
    return int(lib().orc_threads())
