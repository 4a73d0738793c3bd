"""Synthetic MLX checkpoints for the ingestion tests: SafeTensors files written
byte by byte (8-byte little-endian header length, JSON header, raw data) with
MLX's MoE tensor names and shapes ([E, out, in/codes-per-word] packed U32 with
[E, out, in/group] scales and biases)."""
import json
import os

import numpy as np

from hip_backend import BF16, synth


def write_safetensors(path, tensors):
    """tensors: name -> (dtype name, shape, array of the raw element bits)."""
    header, blobs, off = {}, [], 0
    for name, (dt, shape, arr) in tensors.items():
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


def _affine(seed, E, out, inn, bits, group):
    """Packed codes, bf16 scales and biases of a [E, out, inn] expert tensor."""
    n = E * out * inn
    packed, s, b = synth.random_affine(seed, n, bits, group, BF16)
    return {
        "weight": ("U32", [E, out, inn * bits // 32], packed),
        "scales": ("BF16", [E, out, inn // group], s),
        "biases": ("BF16", [E, out, inn // group], b),
    }


def make_checkpoint(directory, layers=2, h=256, E=8, K=2, ff=64, ffs=64, bits=4, group=64,
                    router_bits=8, shards=2, root="model."):
    """Writes config.json and the MoE tensors of `layers` layers named
    `{root}layers.{l}.…` (root "model.", "language_model.model." or
    "model.language_model."); returns the source tensors by name
    (name -> (dtype, shape, array))."""
    os.makedirs(directory, exist_ok=True)
    tensors = {}
    for l in range(layers):
        base = f"{root}layers.{l}."
        s = 9000 + 100 * l
        r = _affine(s + 1, 1, E, h, router_bits, group)  # router [E, h]
        for k, (dt, shape, arr) in r.items():
            tensors[f"{base}mlp.gate.{k}"] = (dt, shape[1:], arr)
        for i, (proj, o, inn) in enumerate((("gate_proj", ff, h), ("up_proj", ff, h), ("down_proj", h, ff))):
            for k, v in _affine(s + 2 + i, E, o, inn, bits, group).items():
                tensors[f"{base}mlp.switch_mlp.{proj}.{k}"] = v
            for k, (dt, shape, arr) in _affine(s + 5 + i, 1, ffs if proj != "down_proj" else h,
                                               h if proj != "down_proj" else ffs, bits, group).items():
                tensors[f"{base}mlp.shared_expert.{proj}.{k}"] = (dt, shape[1:], arr)
        tensors[f"{base}mlp.shared_expert_gate.weight"] = (
            "F32", [1, h], synth.normal(s + 8, h, 0.0, 0.02))
        tensors[f"{base}post_attention_layernorm.weight"] = (
            "BF16", [h], synth.f32_to_bf16_bits(1.0 + 0.1 * synth.normal(s + 9, h)))
    # a tensor outside the MoE roles, ignored by the loader
    tensors[f"{root}embed_tokens.weight"] = ("F32", [4, h], synth.normal(1, 4 * h))
    quant = {"group_size": group, "bits": bits}
    for l in range(layers):
        quant[f"{root}layers.{l}.mlp.gate"] = {"group_size": group, "bits": router_bits}
    config = {"model_type": "qwen3_next", "num_experts": E, "num_experts_per_tok": K,
              "norm_topk_prob": True, "moe_intermediate_size": ff,
              "shared_expert_intermediate_size": ffs, "hidden_size": h, "rms_norm_eps": 1e-6,
              "quantization": quant}
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(config, f)
    names = sorted(tensors)
    if shards == 1:
        write_safetensors(os.path.join(directory, "model.safetensors"), tensors)
    else:
        wm = {}
        for i in range(shards):
            part = {n: tensors[n] for n in names[i::shards]}
            fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            write_safetensors(os.path.join(directory, fname), part)
            wm.update({n: fname for n in part})
        with open(os.path.join(directory, "model.safetensors.index.json"), "w") as f:
            json.dump({"weight_map": wm}, f)
    return tensors
