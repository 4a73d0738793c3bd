"""MLX checkpoint ingestion (hip_backend.mlx) on the CPU: roles, dims and bytes
of the MoE tensors, and the reference loader's rejections
(crates/model-format/tests/mlx.rs:61-130, src/mlx/mod.rs:20-127,
src/mlx/safetensors.rs:27-90)."""
import json
import os

import numpy as np
import pytest

import oracle
from hip_backend import BF16, F32
from hip_backend.mlx import CheckpointError, MoeCheckpoint, load_raw
from mlx_fixture import make_checkpoint, write_safetensors

H, E, K, FF, FFS = 256, 8, 2, 64, 64


def _same(t, src):
    dt, shape, arr = src
    return np.array_equal(np.asarray(t.data).view(np.uint8), np.ascontiguousarray(arr).view(np.uint8))


@pytest.mark.parametrize("shards,root", [(2, "model."), (1, "language_model.model."),
                                         (3, "model.language_model.")])
def test_loads_moe_layers(tmp_path, shards, root):
    src = make_checkpoint(str(tmp_path), shards=shards, root=root)
    ck = MoeCheckpoint(str(tmp_path))
    assert sorted(ck.layers) == [0, 1]
    assert ck.experts_used == K and ck.normalize
    for l, layer in ck.layers.items():
        def s(role):
            return src[f"{root}layers.{l}.{role}"]
        r = layer["router"]
        assert r.dims == [H, E] and r.bits == 8 and r.group_size == 64 and r.scale_type == BF16
        assert _same(r, s("mlp.gate.weight"))
        assert np.array_equal(r.scales, s("mlp.gate.scales")[2])
        for role, dims in (("gate", [H, FF, E]), ("up", [H, FF, E]), ("down", [FF, H, E])):
            t = layer[role]
            assert t.dims == dims and t.bits == 4
            assert _same(t, s(f"mlp.switch_mlp.{role}_proj.weight"))
            assert np.array_equal(t.biases, s(f"mlp.switch_mlp.{role}_proj.biases")[2])
        assert layer["shared_gate"].dims == [H, FFS] and layer["shared_down"].dims == [FFS, H]
        g = layer["shared_gate_inp"]
        assert g.dims == [H] and g.dtype == F32  # [1, h] -> [h]
        assert layer["norm"].dims == [H] and layer["norm"].dtype == BF16


def test_decoded_values_follow_the_reference_known_answer(tmp_path):
    # crates/model-format/tests/mlx.rs:99: 4-bit code 1, scale 0.5, bias -0.25 -> 0.25
    make_checkpoint(str(tmp_path), layers=1, shards=1)
    raw, _ = load_raw(str(tmp_path))
    tensors = {n: (r.dtype, r.shape, np.array(r.array)) for n, r in raw.items()}
    name = "model.layers.0.mlp.switch_mlp.gate_proj"
    shape = tensors[name + ".weight"][1]
    tensors[name + ".weight"] = ("U32", shape, np.full(shape, 0x11111111, np.uint32))
    gshape = tensors[name + ".scales"][1]
    tensors[name + ".scales"] = ("BF16", gshape, np.full(gshape, 0x3f00, np.uint16))
    tensors[name + ".biases"] = ("BF16", gshape, np.full(gshape, 0xbe80, np.uint16))
    write_safetensors(os.path.join(str(tmp_path), "model.safetensors"), tensors)
    t = MoeCheckpoint(str(tmp_path)).layers[0]["gate"]
    assert (oracle.decode(t, 0, 3) == 0.25).all()


def _rewrite(tmp_path, drop=None, edit=None):
    raw, _ = load_raw(str(tmp_path))
    tensors = {n: (r.dtype, r.shape, np.array(r.array)) for n, r in raw.items() if n != drop}
    for f in os.listdir(str(tmp_path)):
        if f.endswith(".safetensors") or f.endswith(".index.json"):
            os.remove(os.path.join(str(tmp_path), f))
    if edit:
        edit(tensors)
    write_safetensors(os.path.join(str(tmp_path), "model.safetensors"), tensors)


def _config(tmp_path, change):
    path = os.path.join(str(tmp_path), "config.json")
    with open(path) as f:
        c = json.load(f)
    change(c)
    with open(path, "w") as f:
        json.dump(c, f)


def test_rejects_missing_affine_metadata(tmp_path):
    make_checkpoint(str(tmp_path), layers=1)
    _rewrite(tmp_path, drop="model.layers.0.mlp.switch_mlp.up_proj.biases")
    with pytest.raises(CheckpointError, match="missing biases"):
        MoeCheckpoint(str(tmp_path))


def test_rejects_unsupported_quantization(tmp_path):
    make_checkpoint(str(tmp_path), layers=1)
    _config(tmp_path, lambda c: c["quantization"].update(bits=3))
    with pytest.raises(CheckpointError, match="3-bit"):
        MoeCheckpoint(str(tmp_path))
    _config(tmp_path, lambda c: c["quantization"].update(bits=4, mode="mxfp4"))
    with pytest.raises(CheckpointError, match="mode"):
        MoeCheckpoint(str(tmp_path))
    _config(tmp_path, lambda c: c.pop("quantization"))
    with pytest.raises(CheckpointError, match="quantization metadata"):
        MoeCheckpoint(str(tmp_path))


def test_rejects_wrong_group_count(tmp_path):
    make_checkpoint(str(tmp_path), layers=1)
    _config(tmp_path, lambda c: c["quantization"].update(group_size=32))
    with pytest.raises(CheckpointError, match="group count"):
        MoeCheckpoint(str(tmp_path))


def test_rejects_unsafe_or_inconsistent_shards(tmp_path):
    make_checkpoint(str(tmp_path), layers=1, shards=2)
    idx = os.path.join(str(tmp_path), "model.safetensors.index.json")
    with open(idx) as f:
        good = json.load(f)
    bad = {"weight_map": dict(good["weight_map"])}
    bad["weight_map"]["model.layers.0.mlp.gate.weight"] = "../outside.safetensors"
    with open(idx, "w") as f:
        json.dump(bad, f)
    with pytest.raises(CheckpointError, match="unsafe"):
        MoeCheckpoint(str(tmp_path))
    swapped = {"weight_map": dict(good["weight_map"])}
    names = sorted(swapped["weight_map"])
    a, b = names[0], names[1]
    swapped["weight_map"][a], swapped["weight_map"][b] = good["weight_map"][b], good["weight_map"][a]
    with open(idx, "w") as f:
        json.dump(swapped, f)
    with pytest.raises(CheckpointError, match="does not assign"):
        MoeCheckpoint(str(tmp_path))
    missing = {"weight_map": dict(good["weight_map"])}
    missing["weight_map"]["model.layers.0.mlp.extra.weight"] = good["weight_map"][a]
    with open(idx, "w") as f:
        json.dump(missing, f)
    with pytest.raises(CheckpointError, match="missing"):
        MoeCheckpoint(str(tmp_path))


def test_rejects_truncated_file(tmp_path):
    make_checkpoint(str(tmp_path), layers=1, shards=1)
    path = os.path.join(str(tmp_path), "model.safetensors")
    with open(path, "r+b") as f:
        f.truncate(os.path.getsize(path) - 64)
    with pytest.raises(CheckpointError, match="data offsets"):
        MoeCheckpoint(str(tmp_path))


@pytest.mark.parametrize("model_type,arch,normalize", [
    ("qwen3_next", "qwen3next", False), ("qwen3_5_moe", "qwen35moe", True),
    ("qwen3_5_moe_text", "qwen35moe", True), ("qwen3_5", "qwen35moe", True)])
def test_config_defaults_follow_the_reference(tmp_path, model_type, arch, normalize):
    """Without norm_topk_prob the top-k weights are normalised for every
    architecture except Qwen3-Next, and rms_norm_eps defaults to 1e-5
    (crates/model-format/src/mlx/config.rs:93,230-233); "qwen3_5" with
    num_experts > 0 is the MoE architecture (config.rs:33-39)."""
    make_checkpoint(str(tmp_path), layers=1, shards=1)

    def strip(c):
        c["model_type"] = model_type
        c.pop("norm_topk_prob")
        c.pop("rms_norm_eps")
    _config(tmp_path, strip)
    ck = MoeCheckpoint(str(tmp_path))
    assert ck.architecture == arch
    assert ck.normalize is normalize
    assert ck.eps == pytest.approx(1e-5, rel=1e-7)
    # an explicit flag wins over the architecture default
    _config(tmp_path, lambda c: c.update(norm_topk_prob=not normalize))
    assert MoeCheckpoint(str(tmp_path)).normalize is (not normalize)


def test_config_text_config_and_uploaded_block_flag(tmp_path):
    """A multimodal config keeps the text model's keys in text_config
    (config.rs:26); the block weights carry the resolved normalize flag."""
    make_checkpoint(str(tmp_path), layers=1, shards=1)

    def nest(c):
        text = {k: c.pop(k) for k in ("num_experts", "num_experts_per_tok", "moe_intermediate_size",
                                      "shared_expert_intermediate_size", "hidden_size",
                                      "rms_norm_eps", "norm_topk_prob")}
        text.pop("norm_topk_prob")
        text["rms_norm_eps"] = 2e-6
        c["text_config"] = text
        c["model_type"] = "qwen3_next"
    _config(tmp_path, nest)
    ck = MoeCheckpoint(str(tmp_path))
    assert ck.experts_used == K and ck.normalize is False
    assert ck.eps == pytest.approx(2e-6, rel=1e-7)


@pytest.mark.parametrize("change,match", [
    (lambda c: c.pop("model_type"), "model_type"),
    (lambda c: c.update(model_type="mixtral"), "MLX model_type mixtral"),
    (lambda c: c.update(model_type=7), "model_type"),
    (lambda c: c.update(rms_norm_eps=0.0), "normalization"),
    (lambda c: c.update(rms_norm_eps=1e300), "nonfinite"),
    (lambda c: c.update(num_experts_per_tok=2_000_000), "exceeds supported limit"),
    (lambda c: c.pop("num_experts_per_tok"), "num_experts_per_tok"),
])
def test_config_rejections(tmp_path, change, match):
    """config.rs:7-44,94-108: model_type is required and must be one the
    reader knows; eps must be finite and positive; counts are bounded."""
    make_checkpoint(str(tmp_path), layers=1, shards=1)
    _config(tmp_path, change)
    with pytest.raises(CheckpointError, match=match):
        MoeCheckpoint(str(tmp_path))
