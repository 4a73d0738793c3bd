"""The C ABI library on the CPU: it loads, exports every symbol the header
declares, the Python mirror binds exactly those, and the pure-host entry
points behave (no GPU compute here)."""
import ctypes as C
import os
import re

import pytest

from hip_backend import api

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "moe_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_op_surface():
    names = declared()
    for op in ["moe_matmul", "moe_expert_matmul", "moe_route", "moe_swiglu", "moe_mix",
               "moe_gate_scalar", "moe_add", "moe_norm", "moe_batch_begin", "moe_batch_finish",
               "moe_block", "moe_dispatch", "moe_route_tokens"]:
        assert op in names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(api.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_mirror_binds_exactly_the_header():
    assert sorted(api.SIGNATURES) == declared()
    api.load_library()


def test_version_and_view_are_host_only():
    lib = api.load_library()
    assert b"gfx950" in lib.moe_version()
    b = api.MoeBufferC(C.c_void_p(4096), 10)
    out = api.MoeBufferC()
    assert lib.moe_view(b, 2, 8, C.byref(out)) == 0
    assert out.ptr == 4096 + 8 and out.len == 8
    assert lib.moe_view(b, 3, 8, C.byref(out)) == 3          # view bounds (apple.rs:57-59)
    assert lib.moe_view(b, 0, 0, C.byref(out)) == 3          # empty view
    assert lib.moe_view(b, 2 ** 64 - 1, 2, C.byref(out)) == 3  # overflow


def test_workspace_size_is_host_only():
    lib = api.load_library()
    w = api.MoeBlockWeightsC()
    w.router.ndims, w.router.dims[0], w.router.dims[1] = 2, 2048, 512
    w.gate.ndims = 3
    w.gate.dims[0], w.gate.dims[1], w.gate.dims[2] = 2048, 512, 512
    w.has_shared = 1
    w.shared_gate.dims[1] = 512
    w.experts_used = 10
    n = C.c_uint64()
    assert lib.moe_block_workspace(C.byref(w), 1, C.byref(n)) == 0
    # logits + ids + weights + counts + offsets + perm + pos + act + yexp + shared ... > minimum
    assert n.value >= 512 + 10 * 512 + 10 * 2048
    assert lib.moe_block_workspace(C.byref(w), 0, C.byref(n)) == 3


def test_gpu_create_without_device_is_unavailable():
    # On a machine with no gfx950 device the library refuses with
    # Error::Unavailable; it never falls back to the CPU.
    lib = api.load_library()
    h = C.c_void_p()
    st = lib.moe_gpu_create(0, C.byref(h))
    if st == 0:
        lib.moe_gpu_destroy(h)
        pytest.skip("a gfx950 device is present")
    assert st == 1
    with pytest.raises(api.UnavailableError):
        api.Gpu()


def test_null_handles_are_rejected():
    lib = api.load_library()
    assert lib.moe_batch_begin(None) == 3
    assert lib.moe_profile_enable(None, 1) == 3
    assert lib.moe_allocated_bytes(None) == 0


def test_pack_size_is_host_only():
    """moe_pack_size: the MFMA tile-order copy's sizes from the weight's
    metadata alone (32-row tiles, rows padded; 64-value K steps of 256*bits
    bytes; per pair of steps 32 x 128/group 16-bit values), and no packed form
    for dense weights, F32 scales or rows not a multiple of 128."""
    lib = api.load_library()

    def w(dims, bits, group, st):
        c = api.MoeWeightC()
        c.ndims = len(dims)
        for i, d in enumerate(dims):
            c.dims[i] = d
        c.bits, c.group_size, c.scale_type = bits, group, st
        return c

    db, sb = C.c_uint64(), C.c_uint64()
    for dims, bits, group in [([2048, 768, 128], 4, 64), ([768, 2048, 128], 8, 32),
                              ([256, 40, 3], 2, 128)]:
        assert lib.moe_pack_size(C.byref(w(dims, bits, group, api.BF16)), C.byref(db), C.byref(sb)) == 0
        ntile, nk = (dims[1] + 31) // 32, dims[0] // 64
        assert db.value == dims[2] * ntile * nk * 256 * bits
        assert sb.value == dims[2] * ntile * (nk // 2) * 32 * (128 // group) * 2
    for c in [w([2048, 768, 128], 4, 64, api.F32), w([2048, 768, 128], 0, 0, 0),
              w([192, 64, 2], 4, 64, api.BF16)]:
        assert lib.moe_pack_size(C.byref(c), C.byref(db), C.byref(sb)) == 3


def test_workspace_layout_is_host_only():
    """moe_block_workspace_layout: the routing, dispatch and bf16-input
    regions lie inside the workspace, do not overlap, and are large enough for
    T tokens; the work-list region holds the largest list either tile size can
    produce."""
    lib = api.load_library()
    w = api.MoeBlockWeightsC()
    w.router.ndims, w.router.dims[0], w.router.dims[1] = 2, 2048, 128
    w.gate.ndims = 3
    w.gate.dims[0], w.gate.dims[1], w.gate.dims[2] = 2048, 768, 128
    w.experts_used = 8
    T, E, K = 4096, 128, 8
    lay = api.MoeBlockLayoutC()
    n = C.c_uint64()
    assert lib.moe_block_workspace_layout(C.byref(w), T, C.byref(lay)) == 0
    assert lib.moe_block_workspace(C.byref(w), T, C.byref(n)) == 0
    assert lay.total == n.value
    assert lay.tile_pairs_mfma == 128 and lay.tile_pairs_batched == 8
    worst_tiles = T * K // lay.tile_pairs_batched + E  # one partial run per expert
    spans = sorted([(lay.logits, T * E), (lay.ids, T * K), (lay.weights, T * K), (lay.counts, E),
                    (lay.offsets, E + 1), (lay.perm, T * K), (lay.pos, T * K),
                    (lay.tiles, 2 * worst_tiles), (lay.ntiles, 1), (lay.xb16, T * 2048 // 2)])
    for (a, na), (b, _) in zip(spans, spans[1:]):
        assert a + na <= b
    assert spans[-1][0] + spans[-1][1] <= lay.total
    assert lib.moe_block_workspace_layout(C.byref(w), 0, C.byref(lay)) == 3


def test_error_bytes_without_gpu():
    lib = api.load_library()
    assert lib.moe_last_error_bytes(None) == 0
