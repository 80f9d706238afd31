"""MXFP4 checkpoint layout guard on tiny safetensors checkpoints, CPU only.

Mirrors the reference's guard cases (tests/test_mxfp4_guard.py:160-247): a well-formed packed
checkpoint passes with the reference's byte count, and expanded or malformed expert storage,
missing scales, a wrong layer range or layer count, and a dequantizing config all fail closed."""
import json
import os

import pytest
import torch

from flyai_amd.checkpoint import (CheckpointReader, MXFP4LayoutError, inspect_mxfp4_checkpoint,
                                  shape_from_config)
from tests.ckpt_fixtures import head_tail_tensors, hf_layer_tensors, random_layer, tiny_config, write_checkpoint


def _tensors(config, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = {}
    for i in range(config["num_hidden_layers"]):
        t.update(hf_layer_tensors(random_layer(config, g), i, config))
    t.update(head_tail_tensors(config, g))
    return t


def _inspect(tmp_path, tensors, config=None, shards=2, layer_range=None):
    config = config or tiny_config()
    path = write_checkpoint(str(tmp_path / "ckpt"), tensors, config, shards=shards)
    reader = CheckpointReader(path)
    shape, n, _ = shape_from_config(config)
    return inspect_mxfp4_checkpoint(reader, shape, n, layer_range)


@pytest.mark.parametrize("shards", [1, 3])
def test_packed_checkpoint_verified_with_reference_byte_count(tmp_path, shards):
    report = _inspect(tmp_path, _tensors(tiny_config()), shards=shards)
    assert report["packed_layout_verified"] is True and report["native_execution_verified"] is False
    assert len(report["experts"]) == 2
    # the reference's count for the same two-layer fixture (tests/test_mxfp4_guard.py:166)
    assert report["packed_weight_scale_bytes"] == 2 * (4096 + 256 + 2048 + 128)


def test_e8m0_typed_scales_accepted(tmp_path):
    t = _tensors(tiny_config())
    for name in list(t):
        if name.endswith("_scales"):
            t[name] = t[name].view(torch.float8_e8m0fnu)
    assert _inspect(tmp_path, t)["packed_layout_verified"]


@pytest.mark.parametrize("corruption", ["bf16", "scale_dtype", "scale_shape", "missing_scale", "extra_dense",
                                        "fake_bias", "blocks_shape", "bias_shape", "router_shape"])
def test_expanded_or_malformed_expert_storage_fails_closed(tmp_path, corruption):
    t = _tensors(tiny_config())
    p = "model.layers.0.mlp.experts."
    if corruption == "bf16":  # dequantized expert matrix in place of the packed blocks
        del t[p + "gate_up_proj_blocks"], t[p + "gate_up_proj_scales"]
        t[p + "gate_up_proj"] = torch.zeros(2, 128, 32, dtype=torch.bfloat16)
    elif corruption == "scale_dtype":
        t[p + "gate_up_proj_scales"] = t[p + "gate_up_proj_scales"].float()
    elif corruption == "scale_shape":
        t[p + "gate_up_proj_scales"] = torch.zeros(2, 127, 1, dtype=torch.uint8)
    elif corruption == "missing_scale":
        del t[p + "gate_up_proj_scales"]
    elif corruption == "extra_dense":
        t[p + "expanded_extra_weight"] = torch.zeros(2, 128, 32, dtype=torch.bfloat16)
    elif corruption == "fake_bias":
        t[p + "fake_bias_weight"] = torch.zeros(2, 128, 32)
    elif corruption == "blocks_shape":
        t[p + "down_proj_blocks"] = torch.zeros(2, 32, 4, 8, dtype=torch.uint8)
    elif corruption == "bias_shape":
        t[p + "down_proj_bias"] = torch.zeros(2, 64)
    else:
        t["model.layers.1.mlp.router.weight"] = torch.zeros(3, 32, dtype=torch.bfloat16)
    with pytest.raises(MXFP4LayoutError):
        _inspect(tmp_path, t)


def test_assigned_range_only_reads_assigned_layers(tmp_path):
    t = _tensors(tiny_config())
    t["model.layers.1.mlp.experts.gate_up_proj_scales"] = torch.zeros(1, dtype=torch.float32)
    report = _inspect(tmp_path, t, layer_range=(0, 1))
    assert report["layer_range"] == [0, 1] and report["packed_weight_scale_bytes"] == 4096 + 256 + 2048 + 128
    for bad in ((1, 3), (1, 1), (-1, 1), (0, 2.0)):
        with pytest.raises(MXFP4LayoutError, match="range"):
            _inspect(tmp_path, _tensors(tiny_config()), layer_range=bad)


def test_layer_count_and_missing_layers(tmp_path):
    t = _tensors(tiny_config())
    with pytest.raises(MXFP4LayoutError, match="layers"):
        _inspect(tmp_path, t, config=tiny_config(num_hidden_layers=3,
                                                 layer_types=["sliding_attention", "full_attention", "sliding_attention"]))
    missing = {n: x for n, x in t.items() if not n.startswith("model.layers.0.")}
    with pytest.raises(MXFP4LayoutError, match="layers"):
        _inspect(tmp_path, missing)


def test_malformed_layer_name_fails_closed(tmp_path):
    t = _tensors(tiny_config())
    t["model.layers.x.mlp.router.weight"] = torch.zeros(2, 32, dtype=torch.bfloat16)
    with pytest.raises(MXFP4LayoutError, match="layer tensor name"):
        _inspect(tmp_path, t)


def test_missing_packed_experts(tmp_path):
    t = {n: x for n, x in _tensors(tiny_config()).items() if not n.startswith("model.layers.0.mlp.experts.")}
    with pytest.raises(MXFP4LayoutError, match="missing packed"):
        _inspect(tmp_path, t)


@pytest.mark.parametrize("q", [None, {"quant_method": "bf16"}, {"quant_method": "mxfp4", "dequantize": True}])
def test_config_must_declare_native_mxfp4(tmp_path, q):
    with pytest.raises(MXFP4LayoutError, match="MXFP4|dequantized"):
        _inspect(tmp_path, _tensors(tiny_config()), config=tiny_config(quantization_config=q))


def test_dimensions_must_be_blocks_of_32(tmp_path):
    with pytest.raises(MXFP4LayoutError, match="blocks of 32"):
        _inspect(tmp_path, _tensors(tiny_config()), config=tiny_config(intermediate_size=48))


def test_shape_from_gpt_oss_120b_config():
    """GPT-OSS-120B's published config (36 layers alternating sliding/full, 128 experts top-4)."""
    c = tiny_config(hidden_size=2880, intermediate_size=2880, num_local_experts=128, num_experts_per_tok=4,
                    num_attention_heads=64, num_key_value_heads=8, head_dim=64, num_hidden_layers=36,
                    layer_types=["sliding_attention", "full_attention"] * 18)
    shape, n, sliding = shape_from_config(c)
    assert (shape.hidden, shape.intermediate, shape.n_experts, shape.top_k) == (2880, 2880, 128, 4)
    assert shape.qkv_width == 5120 and n == 36 and sliding[:3] == [True, False, True]


def test_index_weight_map_routes_names_to_shards(tmp_path):
    t = _tensors(tiny_config())
    path = write_checkpoint(str(tmp_path / "c"), t, tiny_config(), shards=3)
    reader = CheckpointReader(path)
    with open(os.path.join(path, "model.safetensors.index.json")) as f:
        assert set(json.load(f)["weight_map"]) == set(t)
    for name in ("model.layers.1.mlp.experts.down_proj_blocks", "lm_head.weight", "model.layers.0.self_attn.sinks"):
        assert torch.equal(reader.get(name), t[name])
        assert reader.meta(name)[1] == tuple(t[name].shape)
