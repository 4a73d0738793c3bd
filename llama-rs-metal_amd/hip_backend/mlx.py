"""MLX checkpoint ingestion for the MoE layers.

Follows the reference's native MLX reader (crates/model-format/src/mlx/):
- SafeTensors shards, either ``model.safetensors`` or ``model.safetensors.index.json``
  with a ``weight_map`` whose shard names must be plain ``*.safetensors`` file names
  and must assign every tensor to the shard that holds it (safetensors.rs:27-90);
- source names mapped to the MoE roles after stripping the ``language_model.`` and
  ``model.language_model.`` prefixes (names.rs:2-8, 36-43);
- dims reversed from the file's row-major shape, so ``[E, out, in]`` becomes
  ``[in, out, E]`` (mod.rs:50);
- packed ``U32`` weights read their ``bits`` / ``group_size`` from
  ``config.json["quantization"]`` (or ``quantization_config``), where a per-module
  entry overrides the global one (mod.rs:20-27).  Mode must be ``affine``, bits
  2/4/8, and scales and biases must match the packed tensor's leading dims with one
  column per group (mod.rs:51-95);
- the shared-expert gate ``[1, h]`` is reshaped to ``[h]`` (mod.rs:113-125);
- ``config.json`` (or its ``text_config``) gives the routing semantics as
  ``mlx/config.rs`` does: ``model_type`` selects the architecture and unknown
  types are rejected (config.rs:27-44), ``norm_topk_prob`` defaults to true
  except for Qwen3-Next (config.rs:230-233), ``rms_norm_eps`` to 1e-5
  (config.rs:93).

Tensors are memory-mapped and uploaded to the GPU as they are: MLX's layout is the
layout the kernels read, so nothing is repacked.  Only JSON and raw tensor bytes are
read from the files; nothing in them is executed.
"""
import json
import os
import re

import numpy as np

from .api import BF16, F16, F32, BlockWeights, Tensor


class CheckpointError(ValueError):
    """model_format::Error::{Invalid, Unsupported} for MLX checkpoints."""


# safetensors dtype -> (numpy view dtype, backend scalar type code or None)
_DTYPES = {"F32": (np.float32, F32), "F16": (np.uint16, F16), "BF16": (np.uint16, BF16),
           "U32": (np.uint32, None)}
_MAX_JSON = 128 * 1024 * 1024  # safetensors.rs:21-24

# MoE roles of one layer (names.rs:36-43; the MoE block's input norm is the
# layer's post-attention norm in the hybrid models, names.rs:20-26)
_ROLES = {
    "mlp.gate.weight": "router",
    "mlp.switch_mlp.gate_proj.weight": "gate",
    "mlp.switch_mlp.up_proj.weight": "up",
    "mlp.switch_mlp.down_proj.weight": "down",
    "mlp.shared_expert.gate_proj.weight": "shared_gate",
    "mlp.shared_expert.up_proj.weight": "shared_up",
    "mlp.shared_expert.down_proj.weight": "shared_down",
    "mlp.shared_expert_gate.weight": "shared_gate_inp",
    "post_attention_layernorm.weight": "norm",
}
_LAYER = re.compile(r"^model\.layers\.(\d+)\.(.+)$")


def _bad(msg):
    return CheckpointError(msg)


def _number(v, key, default=None):
    """config.rs:7-18: a non-negative integer, the default when absent, at
    most 1,000,000."""
    n = v.get(key)
    if not (isinstance(n, int) and not isinstance(n, bool) and n >= 0):
        n = default
    if n is None:
        raise _bad(f"missing config.{key}")
    if n > 1_000_000:
        raise _bad(f"config.{key} exceeds supported limit")
    return n


def _real(v, key, default):
    """config.rs:19-25: a finite number, the default when absent."""
    n = v.get(key)
    n = float(n) if isinstance(n, (int, float)) and not isinstance(n, bool) else float(default)
    with np.errstate(over="ignore"):
        n = float(np.float32(n))  # the reference reads the value as f32
    if not np.isfinite(n):
        raise _bad(f"nonfinite config.{key}")
    return n


def architecture(root):
    """config.rs:27-44: the architecture a ``model_type`` selects (the
    ``text_config`` object, when present, holds the text model's keys)."""
    text = root.get("text_config", root)
    kind = root.get("model_type")
    if not isinstance(kind, str):
        raise _bad("config.model_type")
    if kind == "llama":
        return "llama"
    if kind in ("qwen3_5", "qwen3_5_text"):
        return "qwen35moe" if _number(text, "num_experts", 0) > 0 else "qwen35"
    if kind in ("qwen3_5_moe", "qwen3_5_moe_text"):
        return "qwen35moe"
    if kind == "qwen3_next":
        return "qwen3next"
    raise CheckpointError(f"MLX model_type {kind}")


def _read_json(path):
    if os.path.getsize(path) > _MAX_JSON:
        raise _bad("JSON metadata exceeds 128 MiB")
    with open(path, "rb") as f:
        try:
            return json.loads(f.read())
        except ValueError as e:
            raise _bad(f"{path}: {e}") from None


class _Raw:
    __slots__ = ("dtype", "shape", "array")

    def __init__(self, dtype, shape, array):
        self.dtype, self.shape, self.array = dtype, shape, array


def read_safetensors(path):
    """name -> _Raw over a memory map of one SafeTensors file (8-byte
    little-endian header length, JSON header, raw little-endian data)."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise _bad(f"{path}: truncated header")
        n = int.from_bytes(head, "little")
        if n > _MAX_JSON or 8 + n > size:
            raise _bad(f"{path}: header length")
        try:
            header = json.loads(f.read(n))
        except ValueError as e:
            raise _bad(f"{path}: {e}") from None
    data = np.memmap(path, dtype=np.uint8, mode="r", offset=8 + n) if size > 8 + n else \
        np.zeros(0, np.uint8)
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        dt = info.get("dtype")
        if dt not in _DTYPES:
            raise CheckpointError(f"MLX tensor dtype {dt} ({name})")
        shape = [int(d) for d in info["shape"]]
        lo, hi = (int(v) for v in info["data_offsets"])
        npdt = _DTYPES[dt][0]
        if not 0 <= lo <= hi <= data.size or (hi - lo) != int(np.prod(shape)) * np.dtype(npdt).itemsize:
            raise _bad(f"{path}: {name}: data offsets")
        out[name] = _Raw(dt, shape, data[lo:hi].view(npdt).reshape(shape))
    return out


def load_raw(directory):
    """All tensors of a checkpoint directory (safetensors.rs:27-90)."""
    index_path = os.path.join(directory, "model.safetensors.index.json")
    index = None
    if os.path.exists(index_path):
        index = _read_json(index_path)
        wm = index.get("weight_map")
        if not isinstance(wm, dict):
            raise _bad("missing safetensors index weight_map")
        files = set()
        for shard in wm.values():
            if (not isinstance(shard, str) or not shard.endswith(".safetensors")
                    or os.path.basename(shard) != shard or shard in (".", "..")):
                raise _bad("unsafe safetensors shard name")
            files.add(shard)
    elif os.path.isfile(os.path.join(directory, "model.safetensors")):
        files = {"model.safetensors"}
    else:
        raise _bad("checkpoint needs model.safetensors or model.safetensors.index.json")
    tensors = {}
    for shard in sorted(files):
        for key, raw in read_safetensors(os.path.join(directory, shard)).items():
            if index is not None and index["weight_map"].get(key) != shard:
                raise _bad(f"index does not assign {key} to {shard}")
            if key in tensors:
                raise _bad(f"duplicate tensor {key}")
            tensors[key] = raw
    if index is not None:
        for key in index["weight_map"]:
            if key not in tensors:
                raise _bad(f"index tensor {key} is missing")
    return tensors, sorted(files)


def _strip(name):
    """names.rs:3-8."""
    if name.startswith("language_model."):
        name = name[len("language_model."):]
    if name.startswith("model.language_model."):
        name = "model." + name[len("model.language_model."):]
    return name


def _quantization(root, name):
    """mod.rs:20-27: the module's own entry if it is an object, else the global one."""
    q = root.get("quantization", root.get("quantization_config"))
    if not isinstance(q, dict):
        raise _bad("packed MLX weights require quantization metadata")
    module = name[:-len(".weight")] if name.endswith(".weight") else name
    own = q.get(module)
    return own if isinstance(own, dict) else q


def _tensor(raw, root, name):
    """One source tensor as a backend Tensor (mod.rs:49-127)."""
    r = raw[name]
    module = name[:-len(".weight")] if name.endswith(".weight") else name
    dims = list(reversed(r.shape))
    if r.dtype == "U32":
        q = _quantization(root, name)
        mode = q.get("mode", "affine")
        if mode != "affine":
            raise CheckpointError(f"MLX quantization mode {mode}")
        bits, group = q.get("bits"), q.get("group_size")
        if not isinstance(bits, int):
            raise _bad(f"{name}: missing quantization bits")
        if not isinstance(group, int):
            raise _bad(f"{name}: missing group size")
        if bits not in (2, 4, 8):
            raise CheckpointError(f"MLX affine {bits}-bit (supported: 2/4/8)")
        s, b = raw.get(module + ".scales"), raw.get(module + ".biases")
        if s is None:
            raise _bad(f"{name}: missing scales")
        if b is None:
            raise _bad(f"{name}: missing biases")
        if (len(dims) < 2 or s.dtype != b.dtype or s.shape != b.shape or len(s.shape) != len(r.shape)
                or s.shape[:-1] != r.shape[:-1] or s.dtype not in ("F32", "F16", "BF16")):
            raise _bad(f"{name}: affine metadata shape")
        dims[0] *= 32 // bits
        if group <= 0 or dims[0] // group != s.shape[-1] or dims[0] % group:
            raise _bad(f"{name}: affine group count")
        if name.endswith("mlp.shared_expert_gate.weight") and len(dims) == 2 and dims[1] == 1:
            dims = dims[:1]  # [h, 1] -> [h] (mod.rs:120-125)
        return Tensor.affine(dims, r.array.reshape(-1), s.array.reshape(-1), b.array.reshape(-1),
                             bits, group, _DTYPES[s.dtype][1])
    if r.dtype not in ("F32", "F16", "BF16"):
        raise CheckpointError(f"MLX tensor dtype {r.dtype} ({name})")
    if name.endswith("mlp.shared_expert_gate.weight") and len(dims) == 2 and dims[1] == 1:
        dims = dims[:1]  # [1, h] -> [h] (mod.rs:113-125)
    return Tensor.dense(dims, r.array.reshape(-1), _DTYPES[r.dtype][1])


class MoeCheckpoint:
    """The MoE layers of an MLX checkpoint: ``layers[i]`` maps a role
    (router, gate, up, down, shared_gate, shared_up, shared_down,
    shared_gate_inp, norm) to a host Tensor over the memory-mapped file."""

    def __init__(self, directory):
        self.directory = directory
        self.config = _read_json(os.path.join(directory, "config.json"))
        text = self.config.get("text_config", self.config)
        self.architecture = architecture(self.config)
        self.experts_used = _number(text, "num_experts_per_tok", 0)  # config.rs:221
        # config.rs:230-233: Qwen3-Next leaves the top-k weights unnormalised
        # unless the config asks for it; every other architecture normalises
        norm = text.get("norm_topk_prob")
        self.normalize = norm if isinstance(norm, bool) else self.architecture != "qwen3next"
        self.eps = _real(text, "rms_norm_eps", 1e-5)  # config.rs:93
        if self.eps <= 0.0:
            raise _bad("invalid model dimensions or normalization")  # config.rs:94-108
        raw, self.shards = load_raw(directory)
        layers = {}
        for name in raw:
            m = _LAYER.match(_strip(name))
            if not m or m.group(2) not in _ROLES:
                continue
            role = _ROLES[m.group(2)]
            layer = layers.setdefault(int(m.group(1)), {})
            if role in layer:
                raise _bad(f"multiple source tensors map to layer {m.group(1)} {role}")
            layer[role] = _tensor(raw, self.config, name)
        self.layers = {i: l for i, l in sorted(layers.items()) if "router" in l}
        if not self.layers:
            raise _bad("no MoE layers (mlp.gate / mlp.switch_mlp) in the checkpoint")
        for i, l in self.layers.items():
            for role in ("gate", "up", "down"):
                if role not in l:
                    raise _bad(f"layer {i}: missing mlp.switch_mlp.{role}_proj")
            if not 0 < self.experts_used <= l["router"].dims[1]:
                raise _bad("config.num_experts_per_tok")

    def upload(self, gpu, layer):
        """(BlockWeights, norm weight Buffer or None) of one layer, on `gpu`."""
        l = self.layers[layer]
        w = {r: gpu.weight_tensor(l[r]) for r in ("router", "gate", "up", "down")}
        shared = sg = None
        if "shared_gate" in l:
            shared = tuple(gpu.weight_tensor(l[r]) for r in ("shared_gate", "shared_up", "shared_down"))
            sg = gpu.weight_tensor(l["shared_gate_inp"])
        norm = None
        if "norm" in l:
            t = l["norm"]
            vals = t.data if t.dtype == F32 else _widen(t.data, t.dtype)
            norm = gpu.upload(np.asarray(vals, np.float32))
        bw = BlockWeights(w["router"], w["gate"], w["up"], w["down"], self.experts_used,
                          self.normalize, shared, sg)
        return bw, norm


def _widen(bits, dtype):
    """F16/BF16 bit patterns -> F32 (exact widening, quantization.rs:28-31)."""
    bits = np.asarray(bits, np.uint16)
    if dtype == BF16:
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)
