"""Builders for the benchmark configurations' MoE blocks (host tensors, GPU
uploads and the matching oracle spec) and the parity measures the tests use."""
import numpy as np

import oracle
from hip_backend import BF16, F16, F32, BlockWeights, Tensor, synth

DENSE = ("dense", F32)


def prod(dims):
    n = 1
    for d in dims:
        n *= d
    return n


def make_tensor(dims, kind, seed, std=0.02, random_codes=False):
    """kind: ("dense", dtype) or (bits, group, scale_type)."""
    n = prod(dims)
    if kind[0] == "dense":
        v = synth.normal(seed, n, 0.0, std)
        if kind[1] == F32:
            return Tensor.dense(dims, v)
        if kind[1] == BF16:
            return Tensor.dense(dims, synth.f32_to_bf16_bits(v), BF16)
        return Tensor.dense(dims, v.astype(np.float16).view(np.uint16), F16)
    bits, group, st = kind
    if random_codes:
        packed, s, b = synth.random_affine(seed, n, bits, group, st, std)
    else:
        packed, s, b = synth.quantize_affine(synth.normal(seed, n, 0.0, std), bits, group, st)
    return Tensor.affine(dims, packed, s, b, bits, group, st)


class HostBlock:
    """Host tensors of one MoE block (roles as bound by
    crates/model-runtime/src/loader.rs:172-203)."""

    def __init__(self, h, E, K, ff, ffs, kinds, seed, normalize=True, random_experts=False):
        self.h, self.E, self.K, self.ff, self.ffs = h, E, K, ff, ffs
        self.normalize = normalize
        s = seed * 100
        self.router = make_tensor([h, E], kinds["router"], s + 1)
        self.gate = make_tensor([h, ff, E], kinds["experts"], s + 2, random_codes=random_experts)
        self.up = make_tensor([h, ff, E], kinds["experts"], s + 3, random_codes=random_experts)
        self.down = make_tensor([ff, h, E], kinds["experts"], s + 4, random_codes=random_experts)
        self.shared = None
        self.shared_gate = None
        if ffs:
            self.shared = (make_tensor([h, ffs], kinds["shared"], s + 5),
                           make_tensor([h, ffs], kinds["shared"], s + 6),
                           make_tensor([ffs, h], kinds["shared"], s + 7))
            self.shared_gate = make_tensor([h], kinds.get("shared_gate", DENSE), s + 8)

    def spec(self):
        return oracle.MoeSpec(self.router, self.gate, self.up, self.down, self.K, self.normalize,
                              self.shared, self.shared_gate)

    def upload(self, gpu):
        w = {name: gpu.weight_tensor(getattr(self, name)) for name in ("router", "gate", "up",
                                                                        "down")}
        shared = None
        sg = None
        if self.shared is not None:
            shared = tuple(gpu.weight_tensor(t) for t in self.shared)
            sg = gpu.weight_tensor(self.shared_gate)
        return BlockWeights(w["router"], w["gate"], w["up"], w["down"], self.K, self.normalize,
                            shared, sg)


# ------------------------------------------------------------ configurations --
def config1(kind="f32"):
    """Config 1: h 64, 8 experts, top-2, ff 32, shared ff 32, 4 tokens, seed 43."""
    if kind == "f32":
        kinds = {"router": DENSE, "experts": DENSE, "shared": DENSE}
    else:  # mixed affine variant of the same shapes
        kinds = {"router": (8, 64, BF16), "experts": (4, 32, BF16), "shared": (8, 32, BF16),
                 "shared_gate": DENSE}
    blk = HostBlock(64, 8, 2, 32, 32, kinds, seed=43)
    x = synth.normal(43 * 100 + 99, 4 * 64, 0.0, 1.0).reshape(4, 64)
    return blk, x


def config2(seed=44, random_experts=True):
    """Config 2: Qwen3-Next decode, 4-bit g64 bf16 experts/shared, F32 router."""
    kinds = {"router": DENSE, "experts": (4, 64, BF16), "shared": (4, 64, BF16),
             "shared_gate": DENSE}
    return HostBlock(2048, 512, 10, 512, 512, kinds, seed=seed, random_experts=random_experts)


def config3(seed=45):
    """Config 3: 8-bit g64 router and shared expert, 4-bit g64 routed experts."""
    kinds = {"router": (8, 64, BF16), "experts": (4, 64, BF16), "shared": (8, 64, BF16),
             "shared_gate": (8, 64, BF16)}
    return HostBlock(2048, 512, 10, 512, 512, kinds, seed=seed, random_experts=True)


def config4(seed=46):
    """Config 4: Qwen3-30B-A3B-shaped prefill layer, 4-bit g64 everywhere, no shared expert."""
    kinds = {"router": (4, 64, BF16), "experts": (4, 64, BF16)}
    return HostBlock(2048, 128, 8, 768, 0, kinds, seed=seed, random_experts=True)


def config5(variant, seed=47):
    """Config 5 layer: config-2 shapes with 2-bit g32 or 8-bit g128 experts."""
    q = (2, 32, BF16) if variant == "2bit" else (8, 128, BF16)
    kinds = {"router": DENSE, "experts": q, "shared": q, "shared_gate": DENSE}
    return HostBlock(2048, 512, 10, 512, 512, kinds, seed=seed, random_experts=True)


def hot_bias(tokens, experts, seed, frac=0.2, hot=16, boost=8.0):
    """Config-3 skew: a seeded `frac` of tokens gets +boost on `hot` experts."""
    rng = np.random.Generator(np.random.PCG64(seed))
    hot_ids = rng.choice(experts, hot, replace=False)
    sel = rng.random(tokens) < frac
    b = np.zeros((tokens, experts), np.float32)
    b[np.ix_(sel, hot_ids)] = boost
    return b


def zipf_bias(tokens, experts, seed, s=1.1):
    """Config-4 skew: bias_e = -s*ln(rank_e) over a seeded expert permutation."""
    rng = np.random.Generator(np.random.PCG64(seed))
    rank = np.empty(experts, np.float64)
    rank[rng.permutation(experts)] = np.arange(1, experts + 1)
    return np.broadcast_to((-s * np.log(rank)).astype(np.float32), (tokens, experts)).copy()


# --------------------------------------------------------------- measures --
def rel_max_err(a, b):
    """max|a-b| relative to the reference output's max-abs norm."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def close(a, b, tol=5e-4):
    """Element test of crates/metal-backend/tests/affine.rs:46-51: |a-b| < tol*(1+|b|)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    bad = np.abs(a - b) >= tol * (1 + np.abs(b))
    assert not bad.any(), f"{int(bad.sum())} mismatches, first {np.argwhere(bad)[:3].ravel()}: " \
                          f"{a[bad][:3]} != {b[bad][:3]}"


# ----------------------------------------------------------- packed layout --
def pack_reference(t):
    """The MFMA tile-order copy of affine tensor t (dims [in, out, E]) as
    (codes uint32, scales uint16, biases uint16) -- the layout documented at
    moe_packed_weight in include/moe_hip.h, restated with numpy: block
    (e, tile, kb) holds lanes l = 32h + r in order, lane l the `bits` words of
    row 32*tile + r covering codes 64*kb + 32h .. +32; block (e, tile, p) of
    the scales holds rows r = 0..31, each its 128/group values of the step
    pair p.  Rows past `out` are zero."""
    in_, out = t.dims[0], t.dims[1]
    E = t.dims[2] if len(t.dims) > 2 else 1
    bits, gs = t.bits, t.group_size
    ntile, nk = (out + 31) // 32, in_ // 64
    wpr = in_ * bits // 32
    words = np.zeros((E, ntile * 32, wpr), np.uint32)
    words[:, :out] = np.asarray(t.data, np.uint32).reshape(E, out, wpr)
    codes = words.reshape(E, ntile, 32, nk, 2, bits).transpose(0, 1, 3, 4, 2, 5).ravel()
    G, g2 = in_ // gs, 128 // gs

    def groups(a):
        v = np.zeros((E, ntile * 32, G), np.uint16)
        v[:, :out] = np.asarray(a).view(np.uint16).reshape(E, out, G)
        return v.reshape(E, ntile, 32, nk // 2, g2).transpose(0, 1, 3, 2, 4).ravel()

    return codes, groups(t.scales), groups(t.biases)
