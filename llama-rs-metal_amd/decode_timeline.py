"""Phase timeline of the single-token decode (bench.py's config-2 leg).

Runs 3 x 640 graph-replayed decode steps over 8 resident config-2 layers
with libmoe_hip_timeline.so (build.py --timeline: the decode kernels store a
s_memrealtime stamp per wave and phase) and prints, for the last step, the
percentiles of every phase in microseconds from the first decode_pre wave's
start.  Run from the repository root:

    python3 llama-rs-metal_amd/build.py --timeline
    python3 llama-rs-metal_amd/decode_timeline.py
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))

from hip_backend import api, probe  # noqa: E402

import bench  # noqa: E402

SLOTS, PRE, GATE, DOWN = 16384, 0, 4096, 10240  # slot ranges of k_decode.hip's MOE_STAMP


def main():
    lib_path = os.path.join(HERE, "libmoe_hip_timeline.so")
    if not os.path.exists(lib_path):
        sys.exit("decode_timeline.py: build libmoe_hip_timeline.so first (build.py --timeline)")
    api._lib = api.load_library(lib_path)
    lib = C.CDLL(lib_path)
    gpu = api.Gpu(0)
    layers = [bench.make_layer(gpu, 500 + l) for l in range(bench.LAYERS)]
    H, CH = bench.H, bench.CHUNK
    xs = probe.synth_normal(gpu, CH * H, 4242)
    outs = gpu.zeros(CH * H)
    ws = gpu.zeros(layers[0][0].workspace_elems(1))

    def issue(b, j):
        b.moe_block(layers[j % bench.LAYERS][0], xs.view(j * H, H), outs.view(j * H, H), 1, ws)

    if lib.moe_timeline_clear() != 0:
        sys.exit("moe_timeline_clear failed")
    for rep in range(3):
        s = bench.run_graphs(gpu, issue, 10 * CH, CH)
        print(f"[timeline] {10 * CH} steps: {s / (10 * CH) * 1e6:.2f} us per step", flush=True)
    buf = np.zeros(SLOTS * 8, np.uint64)
    if lib.moe_timeline_read(buf.ctypes.data_as(C.c_void_p), C.c_size_t(buf.nbytes)) != 0:
        sys.exit("moe_timeline_read failed")
    T = buf.reshape(SLOTS, 8).astype(np.int64)
    E, K, FF = bench.E, bench.K, bench.FF
    n_pre = E // 2 + 1                      # two router rows per wave + the shared gate row
    n_routed = K * FF // 4                  # four gate/up rows per wave (one row per sub-wave)
    n_shared = bench.FFS // 4
    n_down = (bench.H // 8) * (K + 1)       # 8 rows per block, one wave per expert
    pre, gate, down = T[PRE:PRE + n_pre], T[GATE:GATE + n_routed + n_shared + 1], T[DOWN:DOWN + n_down]
    t0 = pre[:, 0].min()

    def row(name, v):
        v = (np.asarray(v, np.float64) - t0) / 100.0
        q = np.percentile(v, [0, 10, 50, 90, 100])
        print(f"| {name} | {len(v)} | " + " | ".join(f"{x:.2f}" for x in q) + " |")

    print("\n| phase | waves | min | p10 | median | p90 | max |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    row("decode_pre: wave start", pre[:, 0])
    row("decode_pre: logits stored", pre[:, 1])
    r = gate[:n_routed]
    row("decode_gateup routed: wave start", r[:, 0])
    row("decode_gateup routed: expert id derived", r[:, 1])
    row("decode_gateup routed: weight loads issued", r[:, 2])
    row("decode_gateup routed: dot products done", r[:, 3])
    row("decode_gateup routed: activations stored", r[:, 4])
    row("decode_gateup shared: activations stored", gate[n_routed:n_routed + n_shared, 4])
    row("decode_gateup routing wave: ids, weights stored", gate[n_routed + n_shared:, 4])
    row("decode_down: wave start", down[:, 0])
    routed_down = down[down[:, 1] > 0]
    row("decode_down: first weight loads issued", routed_down[:, 1])
    row("decode_down: dot products done", down[:, 3])
    row("decode_down: output rows stored", down[:, 4])
    gpu.close()


if __name__ == "__main__":
    main()
