"""The reference-shaped ``parts`` adapter on the CPU, against real transformers GPT-OSS modules.

``module_tensors`` must read a ``GptOssDecoderLayer`` by the attribute names transformers gives it
(``phase0/pipeline.py:166-179`` hands these modules to ``FastVerify``, ``phase0/fastverify.py:85-91``):
q/k/v stacked in that order, norms/sinks/biases in fp32, and the packed MXFP4 experts in either form
the reference's guard accepts (``phase0/mxfp4_guard.py:245-276``: ``<proj>_blocks`` + ``_scales``
before the load swizzle, or raw ``<proj>`` bytes + ``<proj>_scales``).  A dequantized expert (what
transformers builds without MXFP4 kernels) must be refused, not silently re-quantised.  The rope table
built from the module's own inv_freq must equal what the module's forward returns, bit for bit."""
from types import SimpleNamespace

import pytest
import torch

from flyai_amd import stage_parts
from flyai_amd.checkpoint import MXFP4LayoutError

transformers = pytest.importorskip("transformers")
from transformers import GptOssConfig  # noqa: E402
from transformers.models.gpt_oss.modeling_gpt_oss import GptOssDecoderLayer, GptOssRotaryEmbedding  # noqa: E402

E, H, I, NQ, NKV, HD = 4, 64, 96, 8, 1, 8


def _config():
    return GptOssConfig(hidden_size=H, intermediate_size=I, num_attention_heads=NQ, num_key_value_heads=NKV,
                        head_dim=HD, num_local_experts=E, num_experts_per_tok=2, num_hidden_layers=2,
                        sliding_window=128, vocab_size=256)


def _mxfp4_layer(cfg, seed, raw_form=False, e8m0_scales=False):
    """A GptOssDecoderLayer whose experts hold packed MXFP4 storage with known bytes."""
    torch.manual_seed(seed)
    layer = GptOssDecoderLayer(cfg, 0)
    for p in layer.parameters():
        p.data.normal_()
    g = torch.Generator().manual_seed(seed + 1)
    ex = torch.nn.Module()
    for proj, (rows, cols) in (("gate_up_proj", (2 * I, H)), ("down_proj", (H, I))):
        blocks = torch.randint(0, 256, (E, rows, cols // 32, 16), dtype=torch.uint8, generator=g)
        scales = torch.randint(119, 124, (E, rows, cols // 32), dtype=torch.uint8, generator=g)
        if e8m0_scales:
            scales = scales.view(torch.float8_e8m0fnu)
        if raw_form:
            setattr(ex, proj, torch.nn.Parameter(blocks.reshape(E, rows, cols // 2), requires_grad=False))
        else:
            setattr(ex, proj + "_blocks", torch.nn.Parameter(blocks, requires_grad=False))
        setattr(ex, proj + "_scales", torch.nn.Parameter(scales, requires_grad=False))
        setattr(ex, proj + "_bias", torch.nn.Parameter(torch.randn(E, rows, generator=g), requires_grad=False))
    layer.mlp.experts = ex
    return layer


def _shape(cfg):
    return stage_parts.stage_shape({"_model": SimpleNamespace(config=cfg)})


def test_shape_from_the_models_config():
    sh = _shape(_config())
    assert (sh.hidden, sh.intermediate, sh.n_experts, sh.top_k, sh.n_q_heads, sh.n_kv_heads, sh.head_dim) == \
        (H, I, E, 2, NQ, NKV, HD)


@pytest.mark.parametrize("raw_form,e8m0", [(False, False), (True, False), (False, True)])
def test_module_tensors_read_by_transformers_names(raw_form, e8m0):
    cfg = _config()
    layer = _mxfp4_layer(cfg, 3, raw_form, e8m0)
    t = stage_parts.module_tensors(layer, _shape(cfg), sliding=True)
    at = layer.self_attn
    want_wqkv = torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight]).to(torch.bfloat16)
    assert torch.equal(t["wqkv"], want_wqkv) and t["wqkv"].shape == ((NQ + 2 * NKV) * HD, H)
    assert torch.equal(t["bqkv"], torch.cat([at.q_proj.bias, at.k_proj.bias, at.v_proj.bias]).to(torch.bfloat16))
    assert torch.equal(t["wo"], at.o_proj.weight.to(torch.bfloat16))
    assert t["sinks"].dtype == torch.float32 and torch.equal(t["sinks"], at.sinks.float())
    assert torch.equal(t["ln1"], layer.input_layernorm.weight) and torch.equal(t["ln2"], layer.post_attention_layernorm.weight)
    assert torch.equal(t["router_w"], layer.mlp.router.weight.to(torch.bfloat16))
    ex = layer.mlp.experts
    for key, proj, rows, cols in (("w13", "gate_up_proj", 2 * I, H), ("w2", "down_proj", H, I)):
        src = getattr(ex, proj if raw_form else proj + "_blocks").reshape(E, rows, cols // 32, 16)
        assert t[key + "_blocks"].dtype == torch.uint8 and torch.equal(t[key + "_blocks"], src)
        assert t[key + "_scales"].dtype == torch.uint8
        assert torch.equal(t[key + "_scales"], getattr(ex, proj + "_scales").view(torch.uint8))
    assert torch.equal(t["b13"], ex.gate_up_proj_bias) and torch.equal(t["b2"], ex.down_proj_bias)
    assert t["sliding"] is True


def test_dequantized_or_swizzled_experts_refused():
    cfg = _config()
    dense = GptOssDecoderLayer(cfg, 0)       # transformers' bf16 GptOssExperts: no packed storage
    with pytest.raises(MXFP4LayoutError, match="load_stage"):
        stage_parts.module_tensors(dense, _shape(cfg), sliding=False)
    layer = _mxfp4_layer(cfg, 4)
    del layer.mlp.experts.down_proj_scales   # the load swizzle deletes the raw scales
    with pytest.raises(MXFP4LayoutError, match="down_proj"):
        stage_parts.module_tensors(layer, _shape(cfg), sliding=False)


def test_wrong_shapes_refused():
    cfg = _config()
    layer = _mxfp4_layer(cfg, 5)
    layer.self_attn.k_proj = torch.nn.Linear(H, 2 * HD)
    with pytest.raises(MXFP4LayoutError, match="k_proj"):
        stage_parts.module_tensors(layer, _shape(cfg), sliding=False)


def test_rope_table_from_the_module_matches_its_forward():
    cfg = _config()
    rot = GptOssRotaryEmbedding(cfg)
    n = 700
    ours = stage_parts.YarnRotary.from_inv_freq(rot.inv_freq, rot.attention_scaling, n, device="cpu")
    x = torch.zeros(1, n, HD, dtype=torch.bfloat16)
    cos, sin = rot(x, torch.arange(n)[None])
    # transformers returns cos/sin of the half-split frequencies concatenated twice
    assert torch.equal(ours.cos, cos[0, :, :HD // 2]) and torch.equal(ours.sin, sin[0, :, :HD // 2])


def test_as_stage_parts_passes_our_own_dict_through():
    parts = {"layers": [], "rotary": None}
    out = stage_parts.as_stage_parts(parts, "cpu")
    assert out["layers"] == [] and out["shape"] is not None


# ---- the wrapped form native MXFP4 loading leaves (phase0/pipeline.py:147-160) -------------------

def _wrapped_layer(cfg, seed, keep_padding=False, e8m0=False):
    from wrapped_mxfp4 import wrap_projection
    layer = _mxfp4_layer(cfg, seed, e8m0_scales=e8m0)
    ex = layer.mlp.experts
    raw = {p: (getattr(ex, p + "_blocks").detach().clone(), getattr(ex, p + "_scales").detach().view(torch.uint8).clone())
           for p in ("gate_up_proj", "down_proj")}
    for p, (b, s) in raw.items():
        wrap_projection(ex, p, b, getattr(ex, p + "_scales").detach() if e8m0 else s, keep_padding=keep_padding)
    return layer, raw


@pytest.mark.parametrize("keep_padding,e8m0", [(False, False), (True, False), (False, True)])
def test_wrapped_experts_repack_to_the_raw_bytes(keep_padding, e8m0):
    cfg = _config()
    layer, raw = _wrapped_layer(cfg, 11, keep_padding, e8m0)
    ex = layer.mlp.experts
    assert not hasattr(ex, "gate_up_proj_blocks") and not hasattr(ex, "down_proj_scales")
    # the stand-in swizzle really moves the bytes, so reading storage.data as it lies would fail
    codes = raw["gate_up_proj"][0].reshape(E, 2 * I, H // 2).transpose(1, 2).reshape(-1)
    assert not torch.equal(ex.gate_up_proj.storage.data.reshape(-1)[:codes.numel()], codes)
    t = stage_parts.module_tensors(layer, _shape(cfg), sliding=False)
    for key, proj in (("w13", "gate_up_proj"), ("w2", "down_proj")):
        b, s = raw[proj]
        assert t[key + "_blocks"].dtype == torch.uint8 and torch.equal(t[key + "_blocks"], b), proj
        assert t[key + "_scales"].dtype == torch.uint8 and torch.equal(t[key + "_scales"], s), proj


def test_wrapped_experts_checked_like_the_reference_guard():
    from wrapped_mxfp4 import WrappedTensor
    cfg = _config()
    sh = _shape(cfg)
    # logical shape not the transposed [E, K, N]
    layer, _ = _wrapped_layer(cfg, 12)
    layer.mlp.experts.down_proj.shape = torch.Size((E, H, I))
    with pytest.raises(MXFP4LayoutError, match="logical shape"):
        stage_parts.module_tensors(layer, sh, sliding=False)
    # physical storage smaller than the packed bytes
    layer, _ = _wrapped_layer(cfg, 13)
    w = layer.mlp.experts.gate_up_proj
    w.storage.data = w.storage.data.reshape(-1)[:100].clone()
    with pytest.raises(MXFP4LayoutError, match="bytes"):
        stage_parts.module_tensors(layer, sh, sliding=False)
    # an expanded (non-FP4) wrapper
    layer, _ = _wrapped_layer(cfg, 14)
    layer.mlp.experts.down_proj.dtype = torch.bfloat16
    with pytest.raises(MXFP4LayoutError, match="not FP4"):
        stage_parts.module_tensors(layer, sh, sliding=False)
    # scales missing from the precision config
    layer, _ = _wrapped_layer(cfg, 15)
    layer.mlp.experts.gate_up_proj_precision_config.weight_scale = None
    with pytest.raises(MXFP4LayoutError, match="weight_scale"):
        stage_parts.module_tensors(layer, sh, sliding=False)
    # a layout that cannot unswizzle
    layer, _ = _wrapped_layer(cfg, 16)
    layer.mlp.experts.down_proj.storage.layout = object()
    with pytest.raises(MXFP4LayoutError, match="unswizzle_data"):
        stage_parts.module_tensors(layer, sh, sliding=False)
    assert isinstance(_wrapped_layer(cfg, 17)[0].mlp.experts.down_proj, WrappedTensor)
