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


# ---- DeepSeek-V3-shaped FP8 MoE stage ------------------------------------------------------------

@dataclass
class DsV3Shape:
    hidden: int = 7168
    intermediate: int = 2048
    n_experts: int = 256
    top_k: int = 8
    n_group: int = 8
    topk_group: int = 4
    route_scale: float = 2.5
    rms_eps: float = 1e-6
    zipf_s: float = 1.1


def fp8_block_quant(w):
    """fp32 [..., N, K] -> (e4m3 bytes u8 [..., N, K], E8M0 scale bytes u8 [..., N/128, K/128]):
    one power-of-two scale 2^ceil(log2(amax/448)) per 128x128 block, the weight layout of
    engines/deepseek_v4/v4_moe_grouped.py:769-783 (``_fp8_block_quant``)."""
    *lead, N, K = w.shape
    b = w.float().reshape(*lead, N // 128, 128, K // 128, 128)
    amax = b.abs().amax(dim=(-3, -1)).clamp_min(1e-4)
    e = torch.ceil(torch.log2(amax / 448.0))
    q = (b / torch.exp2(e)[..., :, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.reshape(*lead, N, K).view(torch.uint8), (e + 127).to(torch.uint8)


def synthetic_fp8_experts(n_experts, hidden, inter, gen, device, std=0.02, chunk=16):
    """Random N(0, std) expert weights quantised per 128x128 block: dict of w1/w3 [E, I, H],
    w2 [E, H, I] e4m3 bytes and s1/s3 [E, I/128, H/128], s2 [E, H/128, I/128] E8M0 bytes."""
    out = {n: [] for n in ("w1", "s1", "w3", "s3", "w2", "s2")}
    for e0 in range(0, n_experts, chunk):
        n = min(chunk, n_experts - e0)
        for wn, sn, shp in (("w1", "s1", (n, inter, hidden)), ("w3", "s3", (n, inter, hidden)),
                            ("w2", "s2", (n, hidden, inter))):
            q, s = fp8_block_quant(torch.randn(*shp, device=device, generator=gen) * std)
            out[wn].append(q)
            out[sn].append(s)
    return {k: torch.cat(v) for k, v in out.items()}


class Fp8MoeLayerWeights:
    """Device tensors of one FP8 MoE layer: ln (fp32), router_w (bf16 [E, H]), e_bias (fp32 [E]),
    w13_packed / w2_packed (E routed experts followed by the shared expert as expert E).
    ``raw`` / ``shared_raw`` keep the unpacked e4m3 + E8M0 tensors when asked (for the oracle)."""

    def __init__(self, **kw):
        self.__dict__.update(kw)


def zipf_bias(n_experts, s, gen, device, amplitude=1.6):
    """Selection-only bias (e_score_correction_bias) giving expert popularity a Zipf(s) shape over a
    random expert order: bias_e = amplitude * rank_e^-s.  With the synthetic router (std 0.02) and
    s = 1.1 at top-8 of 256 over ~163 tokens this touches ~212 experts, puts every token on the most
    popular one and ~60% of assignments on the top 10% of experts -- close to sampling 8 distinct
    experts per token with probabilities proportional to rank^-1.1 (204 touched, 63%)."""
    rank = torch.randperm(n_experts, generator=gen, device=device).float() + 1.0
    return (amplitude * rank.pow(-s)).float()


def synthetic_fp8_moe_layer(shape: DsV3Shape, seed, device="cuda", keep_raw=False):
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    H, I, E = shape.hidden, shape.intermediate, shape.n_experts
    routed = synthetic_fp8_experts(E, H, I, gen, device)
    shared = synthetic_fp8_experts(1, H, I, gen, device)
    lw = Fp8MoeLayerWeights(
        ln=(1.0 + 0.05 * torch.randn(H, device=device, generator=gen)).float(),
        router_w=(torch.randn(E, H, device=device, generator=gen) * 0.02).to(torch.bfloat16),
        e_bias=zipf_bias(E, shape.zipf_s, gen, device),
        # the shared expert is packed as expert E of the same buffers (one launch serves both)
        w13_packed=ops.fp8_repack(*(torch.cat([routed[n], shared[n]]) for n in ("w1", "s1", "w3", "s3"))),
        w2_packed=ops.fp8_repack(*(torch.cat([routed[n], shared[n]]) for n in ("w2", "s2"))),
    )
    if keep_raw:
        lw.raw, lw.shared_raw = routed, shared
    return lw
