"""Tiny GPT-OSS-layout safetensors checkpoints for the loader and layout-guard tests.

Tensor names and storage follow the HF GPT-OSS MXFP4 checkpoint (per layer ``model.layers.{i}.``:
``mlp.experts.{gate_up,down}_proj_{blocks,scales,bias}``, ``mlp.router.*``,
``self_attn.{q,k,v,o}_proj.*``, ``self_attn.sinks``, the two layer norms; plus embed, final norm
and lm_head).  The reference's own guard fixture (tests/test_mxfp4_guard.py:14-37) uses 2 experts,
hidden 32, intermediate 64 and 2 layers; ``tiny_config`` is that configuration."""
import json
import os

import torch
from safetensors.torch import save_file


def tiny_config(**changes):
    c = dict(model_type="gpt_oss", hidden_size=32, intermediate_size=64, num_local_experts=2,
             num_experts_per_tok=2, num_attention_heads=2, num_key_value_heads=1, head_dim=16,
             num_hidden_layers=2, sliding_window=128, rms_norm_eps=1e-5, vocab_size=8,
             layer_types=["sliding_attention", "full_attention"], tie_word_embeddings=False,
             quantization_config={"quant_method": "mxfp4"})
    c.update(changes)
    return c


def random_layer(config, gen):
    """CPU tensors of one layer under the stage's names (q/k/v stacked as in LayerWeights)."""
    H, I, E = config["hidden_size"], config["intermediate_size"], config["num_local_experts"]
    D, nq, nkv = config["head_dim"], config["num_attention_heads"], config["num_key_value_heads"]
    qkv = (nq + 2 * nkv) * D

    def bf(*s):
        return (torch.randn(*s, generator=gen) * 0.02).to(torch.bfloat16)

    def u8(lo, hi, *s):
        return torch.randint(lo, hi, s, dtype=torch.uint8, generator=gen)

    return dict(ln1=1 + 0.05 * torch.randn(H, generator=gen), ln2=1 + 0.05 * torch.randn(H, generator=gen),
                wqkv=bf(qkv, H), bqkv=bf(qkv), wo=bf(H, nq * D), bo=bf(H),
                sinks=torch.randn(nq, generator=gen), router_w=bf(E, H), router_b=bf(E),
                w13_blocks=u8(0, 256, E, 2 * I, H // 32, 16), w13_scales=u8(119, 124, E, 2 * I, H // 32),
                b13=torch.randn(E, 2 * I, generator=gen) * 0.02,
                w2_blocks=u8(0, 256, E, H, I // 32, 16), w2_scales=u8(119, 124, E, H, I // 32),
                b2=torch.randn(E, H, generator=gen) * 0.02)


def hf_layer_tensors(layer, i, config, norm_dtype=torch.bfloat16):
    """The HF checkpoint tensors of one layer given under the stage's names."""
    D = config["head_dim"]
    nq, nkv = config["num_attention_heads"] * D, config["num_key_value_heads"] * D
    p = f"model.layers.{i}."
    q, k, v = layer["wqkv"].split([nq, nkv, nkv])
    bq, bk, bv = layer["bqkv"].split([nq, nkv, nkv])
    t = {p + "input_layernorm.weight": layer["ln1"].to(norm_dtype),
         p + "post_attention_layernorm.weight": layer["ln2"].to(norm_dtype),
         p + "self_attn.q_proj.weight": q, p + "self_attn.k_proj.weight": k, p + "self_attn.v_proj.weight": v,
         p + "self_attn.q_proj.bias": bq, p + "self_attn.k_proj.bias": bk, p + "self_attn.v_proj.bias": bv,
         p + "self_attn.o_proj.weight": layer["wo"], p + "self_attn.o_proj.bias": layer["bo"],
         p + "self_attn.sinks": layer["sinks"].to(norm_dtype),
         p + "mlp.router.weight": layer["router_w"], p + "mlp.router.bias": layer["router_b"],
         p + "mlp.experts.gate_up_proj_blocks": layer["w13_blocks"],
         p + "mlp.experts.gate_up_proj_scales": layer["w13_scales"],
         p + "mlp.experts.gate_up_proj_bias": layer["b13"].to(norm_dtype),
         p + "mlp.experts.down_proj_blocks": layer["w2_blocks"],
         p + "mlp.experts.down_proj_scales": layer["w2_scales"],
         p + "mlp.experts.down_proj_bias": layer["b2"].to(norm_dtype)}
    return {name: x.detach().cpu().contiguous().clone() for name, x in t.items()}


def head_tail_tensors(config, gen):
    V, H = config["vocab_size"], config["hidden_size"]
    return {"model.embed_tokens.weight": torch.randn(V, H, generator=gen).to(torch.bfloat16),
            "model.norm.weight": (1 + 0.05 * torch.randn(H, generator=gen)).to(torch.bfloat16),
            "lm_head.weight": (0.02 * torch.randn(V, H, generator=gen)).to(torch.bfloat16)}


def write_checkpoint(path, tensors, config=None, shards=2):
    """Write `tensors` as `shards` safetensors files plus a model.safetensors.index.json weight map
    (shards=1: a single model.safetensors), and config.json when given."""
    os.makedirs(path, exist_ok=True)
    names = sorted(tensors)
    if shards == 1:
        save_file(tensors, os.path.join(path, "model.safetensors"))
    else:
        weight_map = {}
        for s in range(shards):
            fn = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            part = {n: tensors[n] for n in names[s::shards]}
            save_file(part, os.path.join(path, fn))
            weight_map.update({n: fn for n in part})
        with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {}, "weight_map": weight_map}, f)
    if config is not None:
        with open(os.path.join(path, "config.json"), "w") as f:
            json.dump(config, f)
    return path
