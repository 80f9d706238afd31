"""The reference-shaped ``parts`` dict drives the stage on the GPU.

A dict like the reference's ``load_stage`` returns (``phase0/pipeline.py:166-179``: transformers
``GptOssDecoderLayer`` modules with packed MXFP4 experts, the model's rotary module, ``_model.config``,
``sliding``/``window``, and ``embed``/``norm``/``lm_head`` modules) goes straight into
``FastVerifyStage`` and ``BatchedFastVerifyStage`` (the call sites ``phase0/specpipe.py:544``, ``:666``).
Its steps must equal, bit for bit, the steps of the stage built from the same tensors as this build's
own ``LayerWeights`` -- which the oracle parity tests cover -- so the adapter reads every tensor from
the right attribute.  The head and tail callables (``specpipe.py:596``, ``:611-612``, ``:796``) are
checked against the embedding rows, the oracle's RMSNorm and an fp64 logit product."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
E, V = 8, 4096


def _reference_parts(layers, shape, vocab_weights):
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssDecoderLayer, GptOssRMSNorm, GptOssRotaryEmbedding
    cfg = GptOssConfig(hidden_size=shape.hidden, intermediate_size=shape.intermediate,
                       num_attention_heads=shape.n_q_heads, num_key_value_heads=shape.n_kv_heads,
                       head_dim=shape.head_dim, num_local_experts=E, num_experts_per_tok=shape.top_k,
                       num_hidden_layers=len(layers), sliding_window=shape.window, vocab_size=V)
    nq, nkv = shape.n_q_heads * shape.head_dim, shape.n_kv_heads * shape.head_dim
    P = lambda t: torch.nn.Parameter(t.detach().clone(), requires_grad=False)
    mods = []
    for i, lw in enumerate(layers):
        with torch.device("meta"):
            m = GptOssDecoderLayer(cfg, i)
        at = m.self_attn
        at.q_proj.weight, at.k_proj.weight, at.v_proj.weight = (P(w) for w in lw.wqkv.split([nq, nkv, nkv]))
        at.q_proj.bias, at.k_proj.bias, at.v_proj.bias = (P(b) for b in lw.bqkv.split([nq, nkv, nkv]))
        at.o_proj.weight, at.o_proj.bias = P(lw.wo), P(lw.bo)
        at.sinks = P(lw.sinks.to(torch.bfloat16))           # the checkpoint's sinks are bf16
        m.input_layernorm.weight, m.post_attention_layernorm.weight = P(lw.ln1), P(lw.ln2)
        m.mlp.router.weight, m.mlp.router.bias = P(lw.router_w), P(lw.router_b)
        ex = torch.nn.Module()
        ex.gate_up_proj_blocks, ex.gate_up_proj_scales = P(lw.w13_blocks), P(lw.w13_scales)
        ex.down_proj_blocks, ex.down_proj_scales = P(lw.w2_blocks), P(lw.w2_scales)
        ex.gate_up_proj_bias, ex.down_proj_bias = P(lw.b13), P(lw.b2)
        m.mlp.experts = ex
        mods.append(m)
    emb_w, norm_w, head_w = vocab_weights
    embed = torch.nn.Embedding(V, shape.hidden, device=DEV, dtype=torch.bfloat16)
    embed.weight = P(emb_w)
    norm = GptOssRMSNorm(shape.hidden, eps=shape.rms_eps).to(DEV)
    norm.weight = P(norm_w)
    head = torch.nn.Linear(shape.hidden, V, bias=False, device=DEV, dtype=torch.bfloat16)
    head.weight = P(head_w)
    return {"layers": torch.nn.ModuleList(mods), "rotary": GptOssRotaryEmbedding(cfg),
            "_model": SimpleNamespace(config=cfg), "sliding": [lw.sliding for lw in layers], "window": shape.window,
            "n_layers": len(layers), "lo": 0, "hi": len(layers), "embed": embed, "norm": norm, "lm_head": head}


def _setup():
    from flyai_amd.rope import YarnRotary
    from flyai_amd.weights import GptOssShape, synthetic_layer
    shape = GptOssShape(n_experts=E)
    layers = [synthetic_layer(shape, 500 + i, DEV, sliding=(i % 2 == 0), keep_hf=True) for i in range(2)]
    g = torch.Generator(device=DEV)
    g.manual_seed(77)
    vocab = (torch.randn(V, shape.hidden, device=DEV, generator=g).to(torch.bfloat16),
             (1 + 0.05 * torch.randn(shape.hidden, device=DEV, generator=g)).float(),
             (torch.randn(V, shape.hidden, device=DEV, generator=g) * 0.02).to(torch.bfloat16))
    ours = {"layers": layers, "rotary": YarnRotary(2048, device=DEV), "shape": shape}
    return shape, layers, ours, _reference_parts(layers, shape, vocab), vocab, g


def test_fast_verify_from_reference_parts_equals_own_parts():
    from flyai_amd.runtime import FastVerifyStage
    shape, _, ours, ref, _, g = _setup()
    fv_ref, fv_own = FastVerifyStage(ref, maxlen=2048), FastVerifyStage(ours, maxlen=2048)
    assert fv_ref.shape == shape
    h = torch.randn(1, 40, shape.hidden, device=DEV, generator=g).to(torch.bfloat16)
    a, b = fv_ref.prefill(h, 0).clone(), fv_own.prefill(h, 0).clone()
    torch.cuda.synchronize()
    assert torch.equal(a, b), "prefill differs between the reference-shaped and the own parts"
    for step in range(3):
        h = torch.randn(1, 4, shape.hidden, device=DEV, generator=g).to(torch.bfloat16)
        a, b = fv_ref.decode(h, 40 + 4 * step).clone(), fv_own.decode(h, 40 + 4 * step).clone()
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"decode step {step} differs"


def test_batched_fast_verify_from_reference_parts():
    from flyai_amd.runtime import BatchedFastVerifyStage
    shape, _, ours, ref, _, g = _setup()
    bref, bown = BatchedFastVerifyStage(ref, 3, maxlen=2048), BatchedFastVerifyStage(ours, 3, maxlen=2048)
    h = torch.randn(3, 5, shape.hidden, device=DEV, generator=g).to(torch.bfloat16)
    starts = torch.tensor([0, 17, 300])
    a, b = bref.decode(h, starts).clone(), bown.decode(h, starts).clone()
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_head_and_tail_callables():
    from gpu_harness import metrics
    from flyai_amd.stage_parts import parts_from_reference
    from oracle import layer as olayer
    shape, _, _, ref, (emb_w, norm_w, head_w), g = _setup()
    parts = parts_from_reference(ref)
    ids = torch.tensor([[5, 0, V - 1, 77, 5]], device=DEV)
    x = parts["embed"](ids)
    assert x.shape == (1, 5, shape.hidden) and torch.equal(x[0], emb_w[ids[0]])
    h = torch.randn(1, 70, shape.hidden, device=DEV, generator=g).to(torch.bfloat16)
    hn = parts["norm"](h)
    ref_n = olayer.rmsnorm(h[0].float().cpu(), norm_w.cpu(), shape.rms_eps)
    mar, c = metrics(hn[0].float().cpu().numpy(), ref_n.numpy())
    assert mar <= 1e-2 and c >= 0.9999
    logits = parts["lm_head"](hn)                           # 70 rows: two launches of <= 64 rows
    assert logits.shape == (1, 70, V) and logits.dtype == torch.bfloat16
    exact = hn[0].double().cpu() @ head_w.double().cpu().T
    err = (logits[0].double().cpu() - exact).abs()
    assert bool((err <= exact.abs() * 2.0 ** -8 + 1e-6).all()), "logits beyond one bf16 rounding step"
    ids_g = parts["lm_head"].argmax(hn)
    own = logits[0].float()
    assert torch.equal(ids_g[0], own.argmax(-1).to(ids_g.dtype))
