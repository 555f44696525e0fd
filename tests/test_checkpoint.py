"""Checkpoint directory loading: the BF16 device path keeps weights in bf16
(no fp32 widening), packs the projection weights on the device exactly, and the
widening loader follows src/safetensors.jl:28-30 (bf16 bits << 16).

The checkpoints are written here from the native fixture's weights rounded to
bf16, in the Hugging Face layout the reference reads (``model.language_model.*``
names, optional sharded index)."""
import json
import os

import numpy as np
import pytest
import torch

from oracle import qdc_oracle as O
from qdc_amd import backbone
from qdc_amd.weights import read_checkpoint, read_checkpoint_tensors

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _fixture():
    d = np.load(os.path.join(GOLDEN, "native_fixture.npz"), allow_pickle=False)
    weights = {k[2:]: O.round_bf16(d[k]) for k in d.files if k.startswith("w/")}
    return json.loads(str(d["config_json"])), weights


def _write(directory, sharded=False):
    from safetensors.torch import save_file
    config, weights = _fixture()
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(config, f)
    tensors = {"model.language_model." + k: torch.from_numpy(v).to(torch.bfloat16)
               for k, v in weights.items()}
    tensors["model.visual.patch.weight"] = torch.zeros(3, dtype=torch.bfloat16)  # not loaded
    if not sharded:
        save_file(tensors, os.path.join(directory, "model.safetensors"))
    else:
        names = sorted(tensors)
        shards = {"model-00001-of-00002.safetensors": names[::2],
                  "model-00002-of-00002.safetensors": names[1::2]}
        for fname, keys in shards.items():
            save_file({k: tensors[k] for k in keys}, os.path.join(directory, fname))
        with open(os.path.join(directory, "model.safetensors.index.json"), "w") as f:
            json.dump({"weight_map": {k: fn for fn, keys in shards.items() for k in keys}}, f)
    return weights


@pytest.mark.parametrize("sharded", [False, True])
def test_bf16_tensors_stay_bf16(tmp_path, sharded):
    weights = _write(str(tmp_path), sharded)
    got = read_checkpoint_tensors(str(tmp_path))
    assert set(got) == set(weights)
    for name, value in got.items():
        assert value.dtype == torch.bfloat16, name
        bits = value.view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(bits, O.f32_to_bf16(weights[name])), name
    # the widening loader: bf16 bits << 16, exactly (src/safetensors.jl:28-30)
    wide = read_checkpoint(str(tmp_path))
    for name, value in wide.items():
        assert value.dtype == np.float32 and np.array_equal(value, weights[name]), name


def test_unsafe_shard_path(tmp_path):
    with open(os.path.join(tmp_path, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": {"a": "../outside.safetensors"}}, f)
    with pytest.raises(ValueError):
        read_checkpoint_tensors(str(tmp_path))


def test_from_directory_packs_bf16_without_widening(tmp_path):
    weights = _write(str(tmp_path))
    model = backbone.QwenBackbone.from_directory(str(tmp_path), device="cpu",
                                                 dtype=torch.bfloat16)
    t = lambda name: torch.from_numpy(weights[name]).to(torch.bfloat16)  # noqa: E731
    assert torch.equal(model.embedding, t("embed_tokens.weight"))
    assert model.final_norm.dtype == torch.float32
    assert torch.equal(model.final_norm, torch.from_numpy(weights["norm.weight"]))
    for i, layer in enumerate(model.layers):
        p = f"layers.{i}."
        for key in ("gate_up", "down", "input_norm", "post_norm", "out"):
            assert layer[key].dtype == torch.bfloat16, (i, key)
        assert torch.equal(layer["gate_up"], torch.cat([t(p + "mlp.gate_proj.weight"),
                                                        t(p + "mlp.up_proj.weight")]).t())
        if layer["kind"] == "linear_attention":
            a = p + "linear_attn."
            packed = torch.cat([t(a + n) for n in ("in_proj_qkv.weight", "in_proj_z.weight",
                                                   "in_proj_a.weight", "in_proj_b.weight")]).t()
            width = packed.shape[1]
            assert torch.equal(layer["proj"][:, :width], packed)
            assert layer["proj"].shape[1] % 256 == 0 and not layer["proj"][:, width:].any()
            assert layer["conv"].dtype == torch.float32
        else:
            a = p + "self_attn."
            # q_proj rows [q_h; gate_h] per head, regrouped as [q; k; v; gate]
            hd, H = model.cfg.head_dim, model.cfg.heads
            qg = t(a + "q_proj.weight").reshape(H, 2, hd, -1)
            packed = torch.cat([qg[:, 0].reshape(H * hd, -1), t(a + "k_proj.weight"),
                                t(a + "v_proj.weight"), qg[:, 1].reshape(H * hd, -1)]).t()
            assert torch.equal(layer["qkv"], packed)
    # fp32 storage of the same checkpoint widens exactly
    wide = backbone.QwenBackbone.from_directory(str(tmp_path), device="cpu", dtype=torch.float32)
    assert torch.equal(wide.layers[0]["gate_up"], model.layers[0]["gate_up"].float())
