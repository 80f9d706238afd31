"""The reference-shaped ``parts`` dict drives the stage on the GPU.

A dict like the reference's ``load_stage`` returns (``phase0/pipeline.py:166-179``: decoder-layer
modules under transformers' ``GptOssDecoderLayer`` attribute names with packed MXFP4 experts, the
model's rotary module, ``_model.config``, ``sliding``/``window``, and ``embed``/``norm``/``lm_head``
modules) goes straight into ``FastVerifyStage`` and ``BatchedFastVerifyStage`` (the call sites
``phase0/specpipe.py:544``, ``:666``).  The experts come in both forms: packed blocks and scales, and
the wrapped codes with precision configs that native MXFP4 loading leaves (``pipeline.py:147-160``).
The modules are plain containers and the rotary values come from a committed fixture, so nothing of
transformers runs here.
Its steps must equal, bit for bit, the steps of the stage built from the same tensors as this build's
own ``LayerWeights`` -- which the oracle parity tests cover -- so the adapter reads every tensor from
the right attribute.  The head and tail callables (``specpipe.py:596``, ``:611-612``, ``:796``) are
checked against the embedding rows, the oracle's RMSNorm and an fp64 logit product."""
import os
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from conftest import GOLDEN

pytestmark = pytest.mark.gpu

DEV = "cuda"
E, V = 8, 4096


def _holder(**tensors):
    """A plain module carrying parameters under transformers' attribute names."""
    m = torch.nn.Module()
    for k, v in tensors.items():
        if torch.is_tensor(v):
            m.register_parameter(k, torch.nn.Parameter(v.detach().clone(), requires_grad=False))
        else:
            setattr(m, k, v)
    return m


def _rotary_module():
    """The model's rotary module as the stage reads it: ``inv_freq`` and ``attention_scaling``, the
    values transformers' ``GptOssRotaryEmbedding`` holds for the GPT-OSS config (committed fixture)."""
    f = np.load(os.path.join(GOLDEN, "rope_yarn.npz"))
    m = torch.nn.Module()
    m.register_buffer("inv_freq", torch.from_numpy(f["inv_freq"]))
    m.attention_scaling = float(f["attention_scaling"])
    return m


def _reference_parts(layers, shape, vocab_weights, wrapped=False):
    """What the reference's ``load_stage`` returns (``phase0/pipeline.py:166-179``), with each decoder
    layer a module tree under transformers' ``GptOssDecoderLayer`` attribute names.  ``wrapped`` gives
    the experts the form native MXFP4 loading leaves (wrapped codes + precision configs)."""
    from wrapped_mxfp4 import wrap_projection
    cfg = SimpleNamespace(hidden_size=shape.hidden, intermediate_size=shape.intermediate,
                          num_attention_heads=shape.n_q_heads, num_key_value_heads=shape.n_kv_heads,
                          head_dim=shape.head_dim, num_local_experts=E, num_experts_per_tok=shape.top_k,
                          num_hidden_layers=len(layers), sliding_window=shape.window, vocab_size=V,
                          rms_norm_eps=shape.rms_eps, max_position_embeddings=2048)
    nq, nkv = shape.n_q_heads * shape.head_dim, shape.n_kv_heads * shape.head_dim
    mods = []
    for lw in layers:
        (wq, wk, wv), (bq, bk, bv) = lw.wqkv.split([nq, nkv, nkv]), lw.bqkv.split([nq, nkv, nkv])
        at = _holder(q_proj=_holder(weight=wq, bias=bq), k_proj=_holder(weight=wk, bias=bk),
                     v_proj=_holder(weight=wv, bias=bv), o_proj=_holder(weight=lw.wo, bias=lw.bo),
                     sinks=lw.sinks.to(torch.bfloat16))          # the checkpoint's sinks are bf16
        ex = _holder(gate_up_proj_blocks=lw.w13_blocks, gate_up_proj_scales=lw.w13_scales,
                     down_proj_blocks=lw.w2_blocks, down_proj_scales=lw.w2_scales,
                     gate_up_proj_bias=lw.b13, down_proj_bias=lw.b2)
        if wrapped:
            wrap_projection(ex, "gate_up_proj", lw.w13_blocks, lw.w13_scales)
            wrap_projection(ex, "down_proj", lw.w2_blocks, lw.w2_scales)
        mlp = _holder(router=_holder(weight=lw.router_w, bias=lw.router_b), experts=ex)
        mods.append(_holder(input_layernorm=_holder(weight=lw.ln1), post_attention_layernorm=_holder(weight=lw.ln2),
                            self_attn=at, mlp=mlp))
    emb_w, norm_w, head_w = vocab_weights
    return {"layers": torch.nn.ModuleList(mods), "rotary": _rotary_module(),
            "_model": SimpleNamespace(config=cfg), "sliding": [lw.sliding for lw in layers], "window": shape.window,
            "n_layers": len(layers), "lo": 0, "hi": len(layers), "embed": _holder(weight=emb_w),
            "norm": _holder(weight=norm_w), "lm_head": _holder(weight=head_w)}


def _setup(wrapped=False):
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
    return shape, layers, ours, _reference_parts(layers, shape, vocab, wrapped), vocab, g


@pytest.mark.parametrize("wrapped", [False, True])
def test_fast_verify_from_reference_parts_equals_own_parts(wrapped):
    from flyai_amd.runtime import FastVerifyStage
    shape, _, ours, ref, _, g = _setup(wrapped)
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


@pytest.mark.parametrize("wrapped", [False, True])
def test_batched_fast_verify_from_reference_parts(wrapped):
    from flyai_amd.runtime import BatchedFastVerifyStage
    shape, _, ours, ref, _, g = _setup(wrapped)
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
