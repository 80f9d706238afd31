"""Expert FFNs: GPT-OSS SwiGLU on MXFP4 weights (row a6) and DeepSeek FP8 block-scaled experts (a7).

GPT-OSS, per routed assignment (token t, expert e), following ``GptOssExperts.forward`` /
``_apply_gate`` (``transformers/models/gpt_oss/modeling_gpt_oss.py:82-88``, ``:108-111``) and the
fused triton path (``transformers/integrations/mxfp4.py:372-403``: matmul_ogs with fp32 bias and a
fused swiglu(alpha, limit), bf16 intermediate, second matmul with fp32 bias and ``gammas``):

    gu   = fp32(x_t . W13[e]^T) + b13[e]             (2I outputs; row 2j = gate_j, 2j+1 = up_j)
    g    = min(gate, 7);  u = clamp(up, -7, 7)
    h    = bf16((u + 1) * g * sigmoid(1.702 * g))     (bf16 intermediate, like matmul_ogs's cache1)
    y    = fp32(h . W2[e]^T) + b2[e]                  (kept fp32 until the combine)

W13/W2 are MXFP4 (oracle.mxfp4); their dequantised values are exact in bf16, so the only freedom
left to a kernel is fp32 accumulation order.  Parity: fp64 brute force on tiny shapes; closed-form
SwiGLU at the clamp boundaries (+-7, 0); transformers fixture (eager GptOssExperts on the
dequantised weights) in tests/golden.

DeepSeek FP8 (the 4-layer, 155-token DeepSeek-V3-shaped stage), following the vendored V4 model (``vendor/deepseek_v4_ref/inference/
model.py:592-611`` Expert, ``:634-650`` MoE) and its GEMM semantics (``vendor/deepseek_v4_ref/
inference/kernel.py:204-254`` fp8_gemm; CPU transcription ``engines/deepseek_v4/v4_kernels_cpu.py:
67-104`` act_quant with power-of-two scale, ``:158-164`` fp8_gemm):
    activations are quantised per row per 128-K block to e4m3 with scale 2**ceil(log2(amax/448)),
    weights are e4m3 with one power-of-two scale per 128x128 block, and
    C = sum_kb fp32(sum_{k in kb} a_q * w_q) * sa[m, kb] * sw[n//128, kb], returned as bf16.
    expert(x, w) = w2(bf16(w * silu(w1(x)) * w3(x)))  (weight applied before w2, model.py:606-610)
    MoE out = bf16(sum over selected experts in ascending id of expert outputs + shared(x)).
Parity: quantiser restated exactly (frexp form, v4_kernels_cpu.py:67-75); GEMM fp64 brute force.
"""
import numpy as np
import torch

from . import mxfp4
from .numerics import bf16

ALPHA = 1.702
LIMIT = 7.0
FP8_MAX = 448.0


def swiglu(gate, up, alpha=ALPHA, limit=LIMIT):
    """modeling_gpt_oss.py:82-88 in fp32."""
    g = torch.clamp(gate, max=limit)
    u = torch.clamp(up, min=-limit, max=limit)
    return (u + 1.0) * (g * torch.sigmoid(g * alpha))


class MxExpertWeights:
    """Host (numpy) copy of one layer's MXFP4 expert tensors in the HF layout (mxfp4.py:349-365)."""

    def __init__(self, w13_blocks, w13_scales, b13, w2_blocks, w2_scales, b2):
        self.w13_blocks = np.asarray(w13_blocks, dtype=np.uint8)
        self.w13_scales = np.asarray(w13_scales, dtype=np.uint8)
        self.b13 = np.asarray(b13, dtype=np.float32)
        self.w2_blocks = np.asarray(w2_blocks, dtype=np.uint8)
        self.w2_scales = np.asarray(w2_scales, dtype=np.uint8)
        self.b2 = np.asarray(b2, dtype=np.float32)
        self._cache = {}

    @property
    def n_experts(self):
        return self.w13_blocks.shape[0]

    def dense(self, e):
        """(W13 fp32 [2I, H], W2 fp32 [H, I]) for expert e, dequantised exactly."""
        if e not in self._cache:
            self._cache = {e: (torch.from_numpy(mxfp4.dequant(self.w13_blocks[e], self.w13_scales[e])),
                               torch.from_numpy(mxfp4.dequant(self.w2_blocks[e], self.w2_scales[e])))}
        return self._cache[e]


def experts_mxfp4(x, perm, offsets, k, wts: MxExpertWeights, return_h=False):
    """x bf16-valued fp32 [T, H]; perm/offsets from routing.permute.
    Returns y_perm fp32 [T*k, H] in permuted row order (and the bf16 intermediate if asked)."""
    x = torch.as_tensor(x).float()
    perm = np.asarray(perm, dtype=np.int64)
    offsets = np.asarray(offsets, dtype=np.int64)
    P = perm.size
    H = wts.b2.shape[1]
    inter = wts.b13.shape[1] // 2
    y = torch.zeros(P, H, dtype=torch.float32)
    hbuf = torch.zeros(P, inter, dtype=torch.float32)
    for e in range(wts.n_experts):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi == lo:
            continue
        tok = torch.from_numpy(perm[lo:hi] // k)
        w13, w2 = wts.dense(e)
        gu = x[tok] @ w13.T + torch.from_numpy(wts.b13[e])[None, :]
        h = bf16(swiglu(gu[:, 0::2], gu[:, 1::2]))
        hbuf[lo:hi] = h
        y[lo:hi] = h @ w2.T + torch.from_numpy(wts.b2[e])[None, :]
    return (y, hbuf) if return_h else y


# ------------------------------------------------------------------------------------------------
# FP8 e4m3 128x128 block-scaled experts (DeepSeek-V3-shaped config)

def round_scale_pow2(amax, max_inv):
    """2**ceil(log2(amax * max_inv)) exactly (v4_kernels_cpu.py:67-75 frexp form; kernel.py:22-37)."""
    x = (amax * np.float32(max_inv)).astype(np.float32)
    mant, exp = np.frexp(x)
    e = np.where(mant == 0.5, exp - 1, exp)
    return np.ldexp(np.float32(1.0), e).astype(np.float32)


def e4m3_round(v):
    """fp32 -> nearest e4m3fn value (RNE, saturating is the caller's clamp), as fp32."""
    return torch.as_tensor(np.asarray(v, dtype=np.float32)).to(torch.float8_e4m3fn).float().numpy()


def act_quant_blocks(x, block):
    """Per-row per-`block` e4m3 quantisation with power-of-two scales: the act_quant rule of
    v4_kernels_cpu.py:89-104 (s = 2**ceil(log2(max(amax, 1e-4) / 448)), q = e4m3(clamp(x / s))) at any
    block size dividing K.  x fp32 [M, K] -> (q fp32 [M, K] holding e4m3 values, s fp32 [M, K/block])."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    assert K % block == 0
    z = x.reshape(M, K // block, block)
    amax = np.maximum(np.abs(z).max(axis=2, keepdims=True), np.float32(1e-4)).astype(np.float32)
    s = round_scale_pow2(amax, 1.0 / FP8_MAX)
    q = np.clip((z / s).astype(np.float32), -FP8_MAX, FP8_MAX)
    return e4m3_round(q).reshape(M, K), s.reshape(M, K // block)


def act_quant_128(x):
    """Per-row per-128 e4m3 quantisation with power-of-two scales (v4_kernels_cpu.py:89-104).
    x fp32 [M, K] -> (q fp32 [M, K] holding e4m3 values, s fp32 [M, K/128])."""
    return act_quant_blocks(x, 128)


def _dequant_blocks(q, s, block=32):
    M, K = q.shape
    return (q.reshape(M, K // block, block) * s[:, :, None]).reshape(M, K).astype(np.float32)


def mx_act_quant_two_term(x):
    """x fp32 [M, K] (K % 32 == 0) -> the two-term e4m3 form of the dense groups' activation operand:
    (q1, s1, q2, s2), the high term act_quant_blocks(x, 32) and the low term the same rule on the
    residual x - q1 s1 (exact in fp32: q1 s1 is x rounded to 4 significant bits).  q* hold e4m3 values
    as fp32, s* the power-of-two scales per 32-block."""
    x = np.asarray(x, dtype=np.float32)
    q1, s1 = act_quant_blocks(x, 32)
    r = (x - _dequant_blocks(q1, s1)).astype(np.float32)
    q2, s2 = act_quant_blocks(r, 32)
    return q1, s1, q2, s2


def mx_fp8_roundtrip(x):
    """x fp32 [M, K] (K % 32 == 0) -> the fp32 values the two-term e4m3 activation operand (one E8M0 scale
    per 32 values per term) carries: q1 s1 + q2 s2 from mx_act_quant_two_term (exact in fp32)."""
    q1, s1, q2, s2 = mx_act_quant_two_term(x)
    return (_dequant_blocks(q1, s1) + _dequant_blocks(q2, s2)).astype(np.float32)


def experts_mxfp4_fp8act(x, perm, offsets, k, wts: MxExpertWeights, return_h=False):
    """experts_mxfp4 with both activation operands carried in the two-term e4m3 form with per-32 E8M0
    scales (the dense groups' scaled-MFMA path): the gathered x rows and the bf16 intermediate h each
    pass through mx_fp8_roundtrip before their product with the MXFP4 weights, the precedent being the
    reference's fp8-activation x fp4-weight GEMM (vendor/deepseek_v4_ref/inference/kernel.py:441-449,
    activations quantised per block on K with power-of-two scales).  Everything else as
    experts_mxfp4: fp32 bias, SwiGLU, bf16 h, fp32 y."""
    xq = torch.from_numpy(mx_fp8_roundtrip(np.asarray(torch.as_tensor(x).float())))
    perm = np.asarray(perm, dtype=np.int64)
    offsets = np.asarray(offsets, dtype=np.int64)
    H = wts.b2.shape[1]
    inter = wts.b13.shape[1] // 2
    y = torch.zeros(perm.size, H, dtype=torch.float32)
    hbuf = torch.zeros(perm.size, inter, dtype=torch.float32)
    for e in range(wts.n_experts):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi == lo:
            continue
        w13, w2 = wts.dense(e)
        gu = xq[torch.from_numpy(perm[lo:hi] // k)] @ w13.T + torch.from_numpy(wts.b13[e])[None, :]
        h = bf16(swiglu(gu[:, 0::2], gu[:, 1::2]))
        hbuf[lo:hi] = h
        hq = torch.from_numpy(mx_fp8_roundtrip(h.numpy()))
        y[lo:hi] = hq @ w2.T + torch.from_numpy(wts.b2[e])[None, :]
    return (y, hbuf) if return_h else y


def fp8_block_gemm(aq, sa, wq, sw):
    """C = sum_kb (aq . wq^T over block kb) * sa[:, kb] * sw[n // 128, kb] (kernel.py:241-254), fp64."""
    aq = np.asarray(aq, dtype=np.float64)
    wq = np.asarray(wq, dtype=np.float64)
    M, K = aq.shape
    N = wq.shape[0]
    out = np.zeros((M, N), dtype=np.float64)
    for kb in range(K // 128):
        part = aq[:, kb * 128:(kb + 1) * 128] @ wq[:, kb * 128:(kb + 1) * 128].T
        scale_n = np.repeat(np.asarray(sw, dtype=np.float64)[:, kb], 128)[:N]
        out += part * np.asarray(sa, dtype=np.float64)[:, kb:kb + 1] * scale_n[None, :]
    return out


def fp8_linear(x_bf16, wq, sw):
    """bf16 x -> act_quant -> fp8 block GEMM -> bf16 (model.py linear() for e4m3 weights)."""
    aq, sa = act_quant_128(x_bf16)
    return bf16(torch.from_numpy(fp8_block_gemm(aq, sa, wq, sw).astype(np.float32)))


def deepseek_expert(x_bf16, w1, s1, w3, s3, w2, s2, weight=None):
    """model.py:601-611: gate = w1(x), up = w3(x) (bf16 outputs, computed in fp32),
    h = silu(gate) * up [* routing weight], y = w2(bf16(h))."""
    gate = fp8_linear(x_bf16, w1, s1)
    up = fp8_linear(x_bf16, w3, s3)
    h = torch.nn.functional.silu(gate) * up
    if weight is not None:
        h = torch.as_tensor(weight).float()[:, None] * h
    return fp8_linear(bf16(h).numpy(), w2, s2)


def fp8_block_quant_weight(w):
    """Synthetic weight quantiser with one power-of-two scale per 128x128 tile
    (``engines/deepseek_v4/v4_moe_grouped.py:769-783``).  Returns (q fp32 e4m3 values, s fp32)."""
    w = np.asarray(w, dtype=np.float32)
    out, inn = w.shape
    b = w.reshape(out // 128, 128, inn // 128, 128)
    amax = np.maximum(np.abs(b).max(axis=(1, 3)), np.float32(1e-4))
    scale = np.exp2(np.ceil(np.log2(amax / np.float32(448.0)))).astype(np.float32)
    q = np.clip(b / scale[:, None, :, None], -448.0, 448.0)
    return e4m3_round(q).reshape(out, inn), scale


class Fp8ExpertWeights:
    """FP8 expert weights as numpy fp32 arrays holding e4m3 values, with fp32 power-of-two scales:
    w1, w3 [E, I, H], s1, s3 [E, I/128, H/128]; w2 [E, H, I], s2 [E, H/128, I/128]
    (``vendor/deepseek_v4_ref/inference/model.py:143-149`` layout, scale per 128x128 block)."""

    def __init__(self, w1, s1, w3, s3, w2, s2):
        self.w1, self.s1, self.w3, self.s3, self.w2, self.s2 = w1, s1, w3, s3, w2, s2

    def expert(self, e, x_bf16, weight=None):
        return deepseek_expert(x_bf16, self.w1[e], self.s1[e], self.w3[e], self.s3[e],
                               self.w2[e], self.s2[e], weight)


def deepseek_moe(x_bf16, ids, wts, experts: Fp8ExpertWeights, shared: Fp8ExpertWeights):
    """MoE.forward (model.py:634-650): fp32 y; for each expert in ascending id, y[tokens] += its
    bf16 output (routing weight applied before w2); y += shared expert (expert 0 of ``shared``);
    returned as bf16 values.  x_bf16 fp32 [T, H] holding bf16 values; ids/wts [T, k]."""
    x = np.asarray(x_bf16, dtype=np.float32)
    ids = np.asarray(ids)
    wts = np.asarray(wts, dtype=np.float32)
    y = torch.zeros(x.shape, dtype=torch.float32)
    for e in np.unique(ids):
        tok, slot = np.nonzero(ids == e)                 # token order, like torch.where
        ye = experts.expert(int(e), x[tok], wts[tok, slot])
        y[torch.from_numpy(tok)] += ye
    y += shared.expert(0, x)
    return bf16(y)
