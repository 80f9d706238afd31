"""Write the golden fixtures that pin the CPU oracle to the GPT-OSS math the reference calls.

The reference's stage step runs GPT-OSS layers from the third-party ``transformers`` package
(``phase0/pipeline.py:160`` AutoModelForCausalLM; pinned 5.12.1 in
``phase0/requirements_vmoe.txt:178``; installed here: see ``transformers_version`` in each
fixture).  That package is pure Python over torch, so this script imports it IN THIS CONTAINER
ONLY and records input/output vectors for:

  mxfp4_table.npz   ``_convert_moe_packed_tensors`` (transformers/integrations/mxfp4.py:257-313)
                    over all 256 code bytes x a spread of E8M0 scale bytes
  rope_yarn.npz     ``GptOssRotaryEmbedding`` (modeling_gpt_oss.py:149-200) with the GPT-OSS
                    default yarn parameters, at selected positions up to 131071
  gptoss_layers.npz two tiny ``GptOssDecoderLayer``s (sliding + full) in fp32, run as a 5-token
                    prefill then a 3-token continuation through a ``DynamicCache``; the experts are
                    the eager ``GptOssExperts`` on weights dequantised from random MXFP4 blocks
                    with ``_convert_moe_packed_tensors``

Nothing here runs on the GPU box and nothing imports /root/reference.  Run:
    python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

OUT = os.path.dirname(os.path.abspath(__file__))


def mxfp4_table():
    from transformers.integrations.mxfp4 import _convert_moe_packed_tensors
    codes = np.arange(256, dtype=np.uint8).reshape(16, 16)           # every byte value once
    scales = np.array([0, 1, 64, 100, 119, 120, 121, 122, 123, 126, 127, 128, 130, 150, 200, 254],
                      dtype=np.uint8)
    blocks = np.broadcast_to(codes[None, :, :], (16, 16, 16)).copy()   # [N=16 rows, G=16, 16]
    sc = np.broadcast_to(scales[:, None], (16, 16)).copy()             # row n uses scales[n]
    out = _convert_moe_packed_tensors(torch.from_numpy(blocks[None]), torch.from_numpy(sc[None]),
                                      dtype=torch.float32)             # [1, K=512, N=16]
    deq = out[0].transpose(0, 1).contiguous().numpy()                  # [N, K]
    return dict(blocks=blocks, scales=sc, dequant=deq)


def rope_yarn():
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssRotaryEmbedding
    cfg = GptOssConfig()
    rot = GptOssRotaryEmbedding(cfg)
    pos = torch.tensor([[0, 1, 2, 3, 7, 100, 127, 128, 511, 4095, 4096, 8191, 8192, 32767, 65536,
                         131071]])
    x = torch.zeros(1, 1, 64, dtype=torch.bfloat16)
    cos, sin = rot(x, pos)
    return dict(positions=pos[0].numpy().astype(np.int64),
                cos_bits=cos[0].view(torch.int16).numpy(), sin_bits=sin[0].view(torch.int16).numpy(),
                inv_freq=rot.inv_freq.numpy(), attention_scaling=np.float64(rot.attention_scaling))


def _bf16v(t):
    return t.to(torch.bfloat16).float()


def gptoss_layers(seed=3):
    from transformers import DynamicCache
    from transformers.integrations.mxfp4 import _convert_moe_packed_tensors
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig
    from transformers.models.gpt_oss import modeling_gpt_oss as M

    H, I, E, K, NQ, NKV, D, W = 256, 128, 8, 2, 8, 2, 64, 4
    cfg = GptOssConfig(hidden_size=H, intermediate_size=I, num_local_experts=E, num_experts_per_tok=K,
                       num_attention_heads=NQ, num_key_value_heads=NKV, head_dim=D, sliding_window=W,
                       num_hidden_layers=2, layer_types=["sliding_attention", "full_attention"])
    cfg._attn_implementation = "eager"
    cfg._experts_implementation = "eager"
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    rot = M.GptOssRotaryEmbedding(cfg)
    rec = {"H": H, "I": I, "E": E, "K": K, "NQ": NQ, "NKV": NKV, "D": D, "W": W}
    x0 = _bf16v(torch.randn(1, 8, H, generator=g))
    rec["x"] = x0[0].numpy()
    cache = DynamicCache()          # full-length KV on both layers, masks do the windowing
    layers = []
    for li in range(2):
        layer = M.GptOssDecoderLayer(cfg, li).float().eval()
        p = {}
        with torch.no_grad():
            for name, shape, std in (("q", (NQ * D, H), 0.05), ("k", (NKV * D, H), 0.05),
                                     ("v", (NKV * D, H), 0.05), ("o", (H, NQ * D), 0.05)):
                wt = _bf16v(torch.randn(*shape, generator=g) * std)
                bs = _bf16v(torch.randn(shape[0], generator=g) * 0.05)
                getattr(layer.self_attn, f"{name}_proj").weight.copy_(wt)
                getattr(layer.self_attn, f"{name}_proj").bias.copy_(bs)
                p[f"w{name}"], p[f"b{name}"] = wt.numpy(), bs.numpy()
            sinks = _bf16v(torch.randn(NQ, generator=g))
            layer.self_attn.sinks.copy_(sinks)
            p["sinks"] = sinks.numpy()
            ln1 = 1.0 + 0.1 * torch.randn(H, generator=g)
            ln2 = 1.0 + 0.1 * torch.randn(H, generator=g)
            layer.input_layernorm.weight.copy_(ln1)
            layer.post_attention_layernorm.weight.copy_(ln2)
            p["ln1"], p["ln2"] = ln1.numpy(), ln2.numpy()
            # router with well-separated logits so bf16 rounding cannot flip a selection
            rw = _bf16v(torch.randn(E, H, generator=g) * 0.5)
            rb = _bf16v(torch.randn(E, generator=g) * 2.0)
            layer.mlp.router.weight.copy_(rw)
            layer.mlp.router.bias.copy_(rb)
            p["router_w"], p["router_b"] = rw.numpy(), rb.numpy()
            for proj, n_out, n_in in (("gate_up", 2 * I, H), ("down", H, I)):
                blocks = rng.integers(0, 256, size=(E, n_out, n_in // 32, 16), dtype=np.uint8)
                scales = rng.integers(119, 124, size=(E, n_out, n_in // 32), dtype=np.uint8)
                dense = _convert_moe_packed_tensors(torch.from_numpy(blocks), torch.from_numpy(scales),
                                                    dtype=torch.float32)          # [E, in, out]
                getattr(layer.mlp.experts, f"{proj}_proj").copy_(dense)
                bias = torch.randn(E, n_out, generator=g) * 0.1
                getattr(layer.mlp.experts, f"{proj}_proj_bias").copy_(bias)
                p[f"{proj}_blocks"], p[f"{proj}_scales"] = blocks, scales
                p[f"{proj}_bias"] = bias.numpy()
        layers.append((layer, p))
        for kk, vv in p.items():
            rec[f"L{li}_{kk}"] = vv
    # step 1: 5-token prefill from position 0; step 2: 3 new tokens at positions 5..7
    x1 = _bf16v(torch.randn(1, 3, H, generator=g))
    rec["x_step1"] = x1[0].numpy()
    for step, (start, n) in enumerate(((0, 5), (5, 3))):
        h = x0[:, :5].clone() if step == 0 else x1.clone()
        pos = torch.arange(start, start + n)[None]
        pe = rot(h, pos)
        for li, (layer, _) in enumerate(layers):
            win = W if li == 0 else 0
            rows = torch.arange(start, start + n)[:, None]
            cols = torch.arange(start + n)[None, :]
            allow = cols <= rows
            if win:
                allow &= (rows - cols) < win
            mask = torch.where(allow, 0.0, torch.finfo(torch.float32).min)[None, None]
            with torch.no_grad():
                h = layer(h, attention_mask=mask, position_ids=pos, past_key_values=cache,
                          use_cache=True, position_embeddings=pe)
            h = h[0] if isinstance(h, tuple) else h
            rec[f"out_step{step}_L{li}"] = h[0].numpy()
    return rec


def main():
    import transformers
    ver = np.array(transformers.__version__)
    np.savez_compressed(os.path.join(OUT, "mxfp4_table.npz"), transformers_version=ver, **mxfp4_table())
    np.savez_compressed(os.path.join(OUT, "rope_yarn.npz"), transformers_version=ver, **rope_yarn())
    np.savez_compressed(os.path.join(OUT, "gptoss_layers.npz"), transformers_version=ver, **gptoss_layers())
    print("wrote fixtures with transformers", transformers.__version__)


if __name__ == "__main__":
    main()
