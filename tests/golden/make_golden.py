"""Writes tests/golden/config1*.npz: the config-1 MoE block fixtures (inputs,
weights and the oracle's outputs).

Config 1: hidden 64, 8 experts, top-2 renormalised, expert ff
32 with SwiGLU, shared expert ff 32 gated by sigmoid(x.w_g); 4 tokens;
weights N(0, 0.02), activations N(0, 1), seeded LCG (seed 43).  The
"affine" fixture keeps the shapes with 4-bit g32 experts, 8-bit g64
router and 8-bit g32 shared weights (bf16 scales).  Outputs come from the C oracle, which
tests/test_oracle.py pins against the reference's known answers and an
independent float64 restatement.

Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "llama-rs-metal_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    sys.path.insert(0, p)

import oracle  # noqa: E402
from helpers import config1  # noqa: E402


def main():
    for kind, name in [("f32", "config1.npz"), ("affine", "config1_affine.npz")]:
        blk, x = config1(kind)
        out, logits, ids, w = oracle.moe_block(blk.spec(), x, 4)
        arrays = dict(x=x, out=out, logits=logits, ids=ids, weights=w)
        for role in ("router", "gate", "up", "down"):
            t = getattr(blk, role)
            arrays[f"{role}_data"] = t.data
            if t.bits:
                arrays[f"{role}_scales"], arrays[f"{role}_biases"] = t.scales, t.biases
        for role, t in zip(("sh_gate", "sh_up", "sh_down"), blk.shared):
            arrays[f"{role}_data"] = t.data
            if t.bits:
                arrays[f"{role}_scales"], arrays[f"{role}_biases"] = t.scales, t.biases
        arrays["sh_gate_inp_data"] = blk.shared_gate.data
        np.savez_compressed(os.path.join(HERE, name), **arrays)
        print(name, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
