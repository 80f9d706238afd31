"""Layer glue and the stage step (rows a9, a10).

* ``rmsnorm``  -- ``GptOssRMSNorm.forward`` (``modeling_gpt_oss.py:57-62``): fp32 compute, fp32
  weight, one cast to bf16 at the end.
* ``linear``   -- bf16 Linear with bias (q/k/v/o, ``modeling_gpt_oss.py:280-291``): fp32 accumulate,
  fp32 bias add, one rounding to bf16.
* ``yarn_inv_freq`` / ``rope_table`` -- ``_compute_yarn_parameters``
  (``transformers/modeling_rope_utils.py:345-483``) with the GPT-OSS defaults
  (``configuration_gpt_oss.py:29``, ``:80-88``: theta 150000, factor 32, beta_fast 32, beta_slow 1,
  original 4096, truncate False) and ``GptOssRotaryEmbedding.forward`` (``modeling_gpt_oss.py:
  189-200``): cos/sin of fp32 inv_freq * position times ``attention_scaling``, cast to bf16.  The
  same torch fp32 operation sequence as transformers, so the table is bit-identical to it
  (pinned by the transformers fixture in tests/golden).
* ``apply_rope`` -- ``_apply_rotary_emb`` (``modeling_gpt_oss.py:215-223``), half-split, computed as
  torch does it on bf16 tensors: every product and difference rounded to bf16.
* ``decoder_layer`` -- ``GptOssDecoderLayer.forward`` (``modeling_gpt_oss.py:347-376``) on a ragged
  token batch: RMSNorm -> q/k/v -> RoPE -> KV write at each token's position (``fastverify.py:
  71-77``, ``batchverify.py:42-48``) -> attention (oracle.attention) -> o_proj -> residual ->
  RMSNorm -> router -> experts -> combine + residual.
* ``decoder_layer(..., tree=(par, dep))`` -- the tree-verify step (``fastverify.py:233-299``).
* ``stage_step`` -- the per-layer loop of ``FastVerify._layers`` / ``BatchedFastVerify._layers``
  (``fastverify.py:116-122``, ``batchverify.py:132-138``); layer i is sliding iff ``sliding[i]``.
"""
import math

import numpy as np
import torch

from . import attention, experts, routing
from .numerics import bf16
from .packing import pack_ragged

HIDDEN = 2880
N_Q_HEADS = 64
N_KV_HEADS = 8
HEAD_DIM = 64
WINDOW = 128
EPS = 1e-5


def rmsnorm(x, w, eps=EPS):
    xf = torch.as_tensor(x).float()
    var = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    return bf16(torch.as_tensor(w).float() * xf)


def linear(x, w, b=None):
    y = torch.as_tensor(x).float() @ torch.as_tensor(w).float().T
    if b is not None:
        y = y + torch.as_tensor(b).float()[None, :]
    return bf16(y)


def yarn_inv_freq(head_dim=HEAD_DIM, base=150000.0, factor=32.0, beta_fast=32.0, beta_slow=1.0,
                  original_max=4096, truncate=False):
    """modeling_rope_utils.py:406-483 restated with the same torch fp32 operations."""
    dim = head_dim

    def get_mscale(scale, mscale=1):
        return 1.0 if scale <= 1 else 0.1 * mscale * math.log(scale) + 1.0

    attention_factor = get_mscale(factor)

    def find_correction_dim(num_rotations):
        return (dim * math.log(original_max / (num_rotations * 2 * math.pi))) / (2 * math.log(base))

    low, high = find_correction_dim(beta_fast), find_correction_dim(beta_slow)
    if truncate:
        low, high = math.floor(low), math.ceil(high)
    low, high = max(low, 0), min(high, dim - 1)
    if low == high:
        high += 0.001
    ramp = torch.clamp((torch.arange(dim // 2, dtype=torch.float32) - low) / (high - low), 0, 1)
    pos_freqs = base ** (torch.arange(0, dim, 2).to(dtype=torch.float) / dim)
    inv_extra = 1.0 / pos_freqs
    inv_inter = 1.0 / (factor * pos_freqs)
    extra_factor = 1 - ramp
    inv_freq = inv_inter * (1 - extra_factor) + inv_extra * extra_factor
    return inv_freq, attention_factor


def rope_table(n_pos, **kw):
    """bf16-valued fp32 (cos, sin), each [n_pos, head_dim/2], for positions 0..n_pos-1."""
    inv_freq, att = yarn_inv_freq(**kw)
    pos = torch.arange(n_pos, dtype=torch.float32)
    freqs = (inv_freq[None, :, None].float() @ pos[None, None, :].float()).transpose(1, 2)[0]
    return bf16(freqs.cos() * att), bf16(freqs.sin() * att)


def apply_rope(x, cos, sin):
    """x bf16-valued [T, nh, D]; cos/sin bf16-valued [T, D/2].  Each op rounded to bf16."""
    x = torch.as_tensor(x).float()
    d2 = x.shape[-1] // 2
    x1, x2 = x[..., :d2], x[..., d2:]
    c, s = cos[:, None, :], sin[:, None, :]
    first = bf16(bf16(x1 * c) - bf16(x2 * s))
    second = bf16(bf16(x2 * c) + bf16(x1 * s))
    return torch.cat([first, second], dim=-1)


class LayerParams:
    """Host copy of one GPT-OSS decoder layer.  Dense tensors are bf16-valued fp32 torch tensors.
    wqkv is q_proj, k_proj, v_proj stacked on the output axis ([4096+512+512, 2880])."""

    def __init__(self, ln1, ln2, wqkv, bqkv, wo, bo, sinks, router_w, router_b, moe, sliding):
        self.ln1, self.ln2 = ln1, ln2
        self.wqkv, self.bqkv, self.wo, self.bo = wqkv, bqkv, wo, bo
        self.sinks = sinks
        self.router_w, self.router_b = router_w, router_b
        self.moe = moe                      # experts.MxExpertWeights
        self.sliding = sliding


def moe_block(x_norm, p: LayerParams, k=4, trace=None, force_ids=None):
    """Router -> permute -> experts -> combine (no residual); x_norm is the RMSNorm output.
    force_ids (int [T, k], optional): teacher forcing for parity tests -- rows whose own selection
    differs from it are routed to its experts (routing.forced_route); the trace keeps the block's own
    ids under "ids" and the replaced rows under "forced_rows"."""
    ids, wts, logits = routing.gptoss_route(x_norm, p.router_w, p.router_b, k)
    own_ids, forced_rows = ids, np.zeros(0, dtype=np.int64)
    if force_ids is not None:
        ids, wts, forced_rows = routing.forced_route(logits, ids, wts, force_ids)
    hist, offsets, perm, inv = routing.permute(ids, p.router_w.shape[0])
    y = experts.experts_mxfp4(x_norm, perm, offsets, k, p.moe)
    out = routing.combine(y, inv, wts)
    if trace is not None:
        trace.update(ids=own_ids, used_ids=ids, forced_rows=forced_rows, weights=wts, logits=logits, hist=hist,
                     offsets=offsets, perm=perm, inv=inv, y_perm=y, moe_out=out)
    return out


def decoder_layer(h, p: LayerParams, kv, q_lens, starts, cos_tab, sin_tab, trace=None, tree=None, force_ids=None):
    """h bf16-valued fp32 [T, H]; kv = (k_seqs, v_seqs), per-sequence fp32 [Hkv, cap, D] tensors
    that are written in place.  Returns the new hidden state.  force_ids: moe_block's teacher forcing.

    tree = (par, dep) makes this the tree-verify step of one sequence (``FastVerify.tree_decode``,
    ``phase0/fastverify.py:233-299``): q_lens == [M], node i is rotated at position
    start + dep[i], its K/V go to slot start + i, and attention uses the ancestor mask."""
    h = torch.as_tensor(h).float()
    T = h.shape[0]
    pk = pack_ragged(q_lens, starts)
    if tree is not None:
        assert len(q_lens) == 1 and int(q_lens[0]) == T == len(tree[0]) == len(tree[1])
        pk["kv_pos"] = pk["positions"].copy()                    # slot start + i
        pk["positions"] = (int(starts[0]) + np.asarray(tree[1], dtype=np.int64)).astype(np.int32)
    else:
        pk["kv_pos"] = pk["positions"]
    pos = torch.from_numpy(pk["positions"].astype(np.int64))
    xn = rmsnorm(h, p.ln1)
    qkv = linear(xn, p.wqkv, p.bqkv)
    nq, nkv = N_Q_HEADS * HEAD_DIM, N_KV_HEADS * HEAD_DIM
    q = qkv[:, :nq].view(T, N_Q_HEADS, HEAD_DIM)
    k = qkv[:, nq:nq + nkv].view(T, N_KV_HEADS, HEAD_DIM)
    v = qkv[:, nq + nkv:].view(T, N_KV_HEADS, HEAD_DIM)
    c, s = cos_tab[pos], sin_tab[pos]
    qr, kr = apply_rope(q, c, s), apply_rope(k, c, s)
    k_seqs, v_seqs = kv
    for t in range(T):
        b, ps = int(pk["seq_id"][t]), int(pk["kv_pos"][t])
        k_seqs[b][:, ps, :] = kr[t]
        v_seqs[b][:, ps, :] = v[t]
    if tree is not None:
        o = attention.tree_attention(qr, k_seqs[0], v_seqs[0], int(starts[0]), list(tree[0]),
                                     list(tree[1]), p.sinks, WINDOW if p.sliding else 0)
    else:
        o = attention.ragged_attention(qr, k_seqs, v_seqs, q_lens, starts, p.sinks,
                                       WINDOW if p.sliding else 0)
    ao = linear(o.reshape(T, nq), p.wo, p.bo)
    h = bf16(h + ao)
    xn2 = rmsnorm(h, p.ln2)
    mo = moe_block(xn2, p, trace=trace, force_ids=force_ids)
    h_out = bf16(h + mo)
    if trace is not None:
        trace.update(xn=xn, qkv=qkv, q_rope=qr, k_rope=kr, attn=o, h_mid=h, xn2=xn2, h_out=h_out)
    return h_out


def stage_step(h, layers, kv_per_layer, q_lens, starts, cos_tab, sin_tab, traces=None, tree=None):
    for i, p in enumerate(layers):
        tr = {} if traces is not None else None
        h = decoder_layer(h, p, kv_per_layer[i], q_lens, starts, cos_tab, sin_tab, trace=tr, tree=tree)
        if traces is not None:
            traces.append(tr)
    return h


def deepseek_moe_layer(h, ln_w, eps, router_w, e_bias, n_group, topk_group, k, route_scale,
                       moe: "experts.Fp8ExpertWeights", shared: "experts.Fp8ExpertWeights"):
    """One FP8 MoE layer of the DeepSeek-V3-shaped stage: h + MoE(RMSNorm(h)) in bf16 (the FFN half
    of a pre-norm block; ``vendor/deepseek_v4_ref/inference/model.py:634-650`` MoE with the
    grouped sigmoid gate of ``vendor/kimi_k3_ref/modeling_kimi_linear.py:703-759``).
    Returns (new h, ids, weights)."""
    hf = torch.as_tensor(h).float()
    xn = rmsnorm(hf, ln_w, eps)
    ids, wts, _ = routing.grouped_sigmoid_route(xn.numpy(), router_w, e_bias, n_group, topk_group, k,
                                                route_scale)
    y = experts.deepseek_moe(xn.numpy(), ids, wts, moe, shared)
    return bf16(hf + y), ids, wts
