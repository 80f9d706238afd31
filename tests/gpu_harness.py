"""Helpers for the GPU parity tests and smoke(): build seeded stage cases on the GPU, mirror them
into the CPU oracle, and compare.  Imported by tests/ and __graft_entry__.smoke() only."""
import numpy as np
import torch

from flyai_amd.rope import YarnRotary
from flyai_amd.runtime import KVWorkspace, RaggedStage
from flyai_amd.weights import GptOssShape, synthetic_layer
from oracle import experts as oexperts
from oracle import layer as olayer

DEV = "cuda"


def metrics(a, b):
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    mar = float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))
    cos = float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-30))
    return mar, cos


def cpu_f32(t):
    return t.detach().float().cpu()


def oracle_layer_params(lw, sliding):
    moe = oexperts.MxExpertWeights(lw.w13_blocks.cpu().numpy(), lw.w13_scales.cpu().numpy(),
                                   lw.b13.cpu().numpy(), lw.w2_blocks.cpu().numpy(),
                                   lw.w2_scales.cpu().numpy(), lw.b2.cpu().numpy())
    return olayer.LayerParams(cpu_f32(lw.ln1), cpu_f32(lw.ln2), cpu_f32(lw.wqkv), cpu_f32(lw.bqkv),
                              cpu_f32(lw.wo), cpu_f32(lw.bo), cpu_f32(lw.sinks), cpu_f32(lw.router_w),
                              cpu_f32(lw.router_b), moe, sliding)


def fill_kv_random(kv: KVWorkspace, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    for t in kv.k + kv.v:
        t.copy_(torch.randn(t.shape, device=DEV, generator=g).to(torch.bfloat16))


def oracle_kv(kv: KVWorkspace, layer, slots):
    ks = [cpu_f32(kv.k_dense(layer, s)) for s in slots]
    vs = [cpu_f32(kv.v_dense(layer, s)) for s in slots]
    return ks, vs


def small_stage_case(n_layers=2, n_experts=8, seed=0, q_lens=(1, 1, 4, 7, 16), starts=(300, 5, 1000, 0, 130),
                     maxlen=2048):
    shape = GptOssShape(n_experts=n_experts)
    layers = [synthetic_layer(shape, seed * 100 + i, DEV, sliding=(i % 2 == 0), keep_hf=True)
              for i in range(n_layers)]
    rot = YarnRotary(maxlen, device=DEV)
    S = len(q_lens)
    kv = KVWorkspace(n_layers, S, maxlen, shape.n_kv_heads, shape.head_dim, DEV)
    fill_kv_random(kv, seed + 7)
    T = int(sum(q_lens))
    g = torch.Generator(device=DEV)
    g.manual_seed(seed + 11)
    hidden = torch.randn(T, shape.hidden, device=DEV, generator=g).to(torch.bfloat16)
    return dict(shape=shape, layers=layers, rot=rot, kv=kv, q_lens=list(q_lens), starts=list(starts),
                slots=list(range(S)), hidden=hidden, T=T, maxlen=maxlen)


def run_stage_vs_oracle(case, per_layer=False):
    """Run the GPU stage step and the oracle on the same inputs.  With per_layer, the oracle runs one
    layer at a time from the GPU's own per-layer input (the per-layer bar) and returns lists."""
    shape, layers, kv = case["shape"], case["layers"], case["kv"]
    slots = case["slots"]
    okv = [oracle_kv(kv, l, slots) for l in range(len(layers))]
    params = [oracle_layer_params(lw, lw.sliding) for lw in layers]
    cos, sin = olayer.rope_table(case["maxlen"])
    h0 = case["hidden"].clone()
    if not per_layer:
        st = RaggedStage(shape, layers, case["rot"], kv, max_tokens=max(64, case["T"]), max_seqs=len(slots))
        out = st.forward(h0.clone(), case["q_lens"], case["starts"], slots)
        torch.cuda.synchronize()
        ref = olayer.stage_step(cpu_f32(h0), params, okv, case["q_lens"], case["starts"], cos, sin)
        return cpu_f32(out).numpy(), ref.numpy()
    outs, refs = [], []
    h = h0.clone()
    for l, lw in enumerate(layers):
        st = RaggedStage(shape, [lw], case["rot"], _SingleLayerKV(kv, l), max_tokens=max(64, case["T"]),
                         max_seqs=len(slots))
        hin = cpu_f32(h)
        h = st.forward(h.clone(), case["q_lens"], case["starts"], slots)
        torch.cuda.synchronize()
        ref = olayer.decoder_layer(hin, params[l], okv[l], case["q_lens"], case["starts"], cos, sin)
        outs.append(cpu_f32(h).numpy())
        refs.append(ref.numpy())
        del st
    return outs, refs


class _SingleLayerKV:
    """View of one layer of a KVWorkspace as a one-layer workspace."""

    def __init__(self, kv, layer):
        self.k, self.v = [kv.k[layer]], [kv.v[layer]]
        self.cap, self.maxlen, self.n_slots = kv.cap, kv.maxlen, kv.n_slots
        self.caps, self.maxlens, self.bases = kv.caps, kv.maxlens, kv.bases
        self.slab, self.n_kv_heads, self.head_dim = kv.slab, kv.n_kv_heads, kv.head_dim

    def base(self, slot):
        return int(self.bases[slot])

    def slot_cap(self, slot):
        return self.caps[slot]


def tokens_with_same_routing(ids, ref_ids, ref_logits, k):
    """Tokens whose GPU router ids equal the oracle's own.  A differing token must sit on a near-tie of
    the oracle's logits (k-th and (k+1)-th within 2 bf16 ulps), and at most 2 may differ.  The layer
    tests then teacher-force the oracle's MoE with the GPU's ids (decoder_layer's force_ids) and hold
    every row to the bar."""
    ref_ids = np.asarray(ref_ids)
    bad = np.nonzero((ids != ref_ids).any(1))[0]
    assert len(bad) <= 2, f"{len(bad)} tokens routed differently"
    for t in bad:
        lg = np.sort(np.asarray(ref_logits, dtype=np.float64)[t])[::-1]
        ulp = 2.0 ** (np.floor(np.log2(max(abs(lg[k - 1]), abs(lg[k]), 1e-30))) - 7)
        assert lg[k - 1] - lg[k] <= 2 * ulp, f"token {t} routed differently without a near-tie"
    return np.setdiff1d(np.arange(ids.shape[0]), bad)
