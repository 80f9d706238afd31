"""GPT-OSS stage weights on the GPU: synthetic random-init layers and the MXFP4 re-pack.

Shapes follow the GPT-OSS decoder layer (transformers/models/gpt_oss/modeling_gpt_oss.py:338-346)
and the MXFP4 expert parameters (transformers/integrations/mxfp4.py:349-365).  q_proj, k_proj and
v_proj are stacked into one [Hq*D + 2*Hkv*D, H] weight (same outputs, one GEMM).  Synthetic values
follow the workload definitions: E2M1 codes uniform over all 16 codes, E8M0 scale bytes uniform in
119..123 (2^-8 .. 2^-4), dense weights N(0, 0.02) like HF's _init_weights
(modeling_gpt_oss.py:406-418)."""
from dataclasses import dataclass

import torch

from . import ops


@dataclass
class GptOssShape:
    hidden: int = 2880
    intermediate: int = 2880
    n_experts: int = 128
    top_k: int = 4
    n_q_heads: int = 64
    n_kv_heads: int = 8
    head_dim: int = 64
    window: int = 128
    rms_eps: float = 1e-5

    @property
    def qkv_width(self):
        return (self.n_q_heads + 2 * self.n_kv_heads) * self.head_dim


class LayerWeights:
    """Device tensors of one decoder layer.  ``w13_blocks``/``w2_blocks`` (HF layout) are kept only
    when ``keep_hf`` is set (tests read them back for the oracle)."""

    def __init__(self, **kw):
        self.__dict__.update(kw)

    def repack(self, keep_hf=False):
        self.w13_packed = ops.mxfp4_repack(self.w13_blocks, self.w13_scales)
        self.w2_packed = ops.mxfp4_repack(self.w2_blocks, self.w2_scales)
        if not keep_hf:
            del self.w13_blocks, self.w13_scales, self.w2_blocks, self.w2_scales
        return self


def synthetic_moe(shape: GptOssShape, gen, device, scale_lo=119, scale_hi=123):
    E, H, I = shape.n_experts, shape.hidden, shape.intermediate
    u8 = dict(dtype=torch.uint8, device=device, generator=gen)
    return dict(
        w13_blocks=torch.randint(0, 256, (E, 2 * I, H // 32, 16), **u8),
        w13_scales=torch.randint(scale_lo, scale_hi + 1, (E, 2 * I, H // 32), **u8),
        b13=(torch.randn(E, 2 * I, device=device, generator=gen) * 0.02).float(),
        w2_blocks=torch.randint(0, 256, (E, H, I // 32, 16), **u8),
        w2_scales=torch.randint(scale_lo, scale_hi + 1, (E, H, I // 32), **u8),
        b2=(torch.randn(E, H, device=device, generator=gen) * 0.02).float(),
    )


def synthetic_layer(shape: GptOssShape, seed, device="cuda", sliding=False, keep_hf=False,
                    router_std=0.02):
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    H, E = shape.hidden, shape.n_experts
    nq = shape.n_q_heads * shape.head_dim

    def bf(*s, std=0.02):
        return (torch.randn(*s, device=device, generator=gen) * std).to(torch.bfloat16)

    lw = LayerWeights(
        ln1=(1.0 + 0.05 * torch.randn(H, device=device, generator=gen)).float(),
        ln2=(1.0 + 0.05 * torch.randn(H, device=device, generator=gen)).float(),
        wqkv=bf(shape.qkv_width, H), bqkv=bf(shape.qkv_width),
        wo=bf(H, nq), bo=bf(H),
        sinks=bf(shape.n_q_heads, std=1.0).float(),
        router_w=bf(E, H, std=router_std), router_b=bf(E, std=router_std),
        sliding=bool(sliding),
        **synthetic_moe(shape, gen, device),
    )
    return lw.repack(keep_hf=keep_hf)
