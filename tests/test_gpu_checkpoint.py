"""Loading a GPT-OSS MXFP4 safetensors checkpoint into the stage, on the GPU: the loaded layers hold
the same bytes as the layers the checkpoint was written from (experts re-packed identically), and
the stage step over loaded layers is bit-identical to the step over the originals."""
import pytest
import torch

from tests import gpu_harness as gh
from tests.ckpt_fixtures import hf_layer_tensors, tiny_config, write_checkpoint
from flyai_amd.checkpoint import (CheckpointReader, inspect_mxfp4_checkpoint, load_head_tail,
                                  load_stage_layers, shape_from_config)
from flyai_amd.runtime import RaggedStage

pytestmark = pytest.mark.gpu
DEV = "cuda"
FIELDS = ("ln1", "ln2", "wqkv", "bqkv", "wo", "bo", "sinks", "router_w", "router_b", "b13", "b2",
          "w13_packed", "w2_packed")


def _config(shape, n_layers):
    return tiny_config(hidden_size=shape.hidden, intermediate_size=shape.intermediate,
                       num_local_experts=shape.n_experts, num_experts_per_tok=shape.top_k,
                       num_attention_heads=shape.n_q_heads, num_key_value_heads=shape.n_kv_heads,
                       head_dim=shape.head_dim, num_hidden_layers=n_layers, vocab_size=512,
                       layer_types=["sliding_attention" if i % 2 == 0 else "full_attention" for i in range(n_layers)])


@pytest.mark.parametrize("e8m0", [False, True])
def test_loaded_stage_equals_written_layers(tmp_path, e8m0):
    print(f"checkpoint load e8m0={e8m0}", flush=True)
    case = gh.small_stage_case(n_layers=2, n_experts=8, seed=5)
    shape, layers = case["shape"], case["layers"]
    config = _config(shape, len(layers))
    tensors = {}
    for i, lw in enumerate(layers):
        tensors.update(hf_layer_tensors(vars(lw), i, config, norm_dtype=torch.float32))
    if e8m0:
        for name in list(tensors):
            if name.endswith("_scales"):
                tensors[name] = tensors[name].view(torch.float8_e8m0fnu)
    g = torch.Generator().manual_seed(3)
    tensors["model.embed_tokens.weight"] = torch.randn(512, shape.hidden, generator=g).to(torch.bfloat16)
    tensors["model.norm.weight"] = (1 + 0.05 * torch.randn(shape.hidden, generator=g)).to(torch.bfloat16)
    tensors["lm_head.weight"] = (0.02 * torch.randn(512, shape.hidden, generator=g)).to(torch.bfloat16)
    path = write_checkpoint(str(tmp_path / "ckpt"), tensors, config, shards=3)
    del tensors

    reader = CheckpointReader(path)
    cshape, n, sliding = shape_from_config(reader.config)
    assert cshape == shape and n == 2 and sliding == [True, False]
    report = inspect_mxfp4_checkpoint(reader, cshape, n)
    assert report["packed_layout_verified"]
    loaded = load_stage_layers(reader, cshape, (0, n), DEV)
    torch.cuda.synchronize()
    for a, b in zip(loaded, layers):
        assert a.sliding == b.sliding
        for f in FIELDS:
            x, y = getattr(a, f), getattr(b, f)
            assert x.dtype == y.dtype and x.shape == y.shape and torch.equal(x, y), f
    embed, norm_w, lm = load_head_tail(reader, DEV)
    assert embed.shape == (512, shape.hidden) and norm_w.dtype == torch.float32 and lm.dtype == torch.bfloat16

    kv = case["kv"]
    saved = [t.clone() for t in kv.k + kv.v]
    outs = []
    for ls in (layers, loaded):
        for t, s in zip(kv.k + kv.v, saved):
            t.copy_(s)
        st = RaggedStage(shape, ls, case["rot"], kv, max_tokens=64, max_seqs=len(case["slots"]))
        outs.append(st.forward(case["hidden"].clone(), case["q_lens"], case["starts"], case["slots"]))
        torch.cuda.synchronize()
        del st
    assert torch.equal(outs[0], outs[1])
