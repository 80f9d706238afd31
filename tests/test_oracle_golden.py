"""Pin the CPU oracle against fixtures written by the transformers GPT-OSS code (tests/golden).

Tolerance bar (per layer, bf16 outputs): max-abs-rel <= 2e-2 and cosine >= 0.999.
"""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN, metrics
from oracle import attention, experts, layer, mxfp4, routing
from oracle.numerics import bf16

MAR, COS = 2e-2, 0.999


def _load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_mxfp4_dequant_matches_transformers_table():
    f = _load("mxfp4_table.npz")
    ours = mxfp4.dequant(f["blocks"], f["scales"])
    ref = f["dequant"]
    assert ours.shape == ref.shape
    same = (ours == ref) | (np.isnan(ours) & np.isnan(ref))
    assert same.all(), "MXFP4 dequant differs from transformers' _convert_moe_packed_tensors"
    # negative zero survives (code 8): sign bit set, value 0
    assert np.signbit(ours[0, 16]) and ours[0, 16] == 0.0


def test_mxfp4_nibble_order_and_scale_closed_form():
    blk = np.zeros((1, 16), dtype=np.uint8)
    blk[0, 0] = 0x71                          # low nibble 1 (0.5) is element 0, high 7 (6.0) element 1
    out = mxfp4.dequant(blk, np.array([128], dtype=np.uint8))
    assert out[0] == 1.0 and out[1] == 12.0   # x 2**(128-127)
    assert np.isnan(mxfp4.dequant(blk, np.array([255], dtype=np.uint8))[1])
    assert mxfp4.dequant(blk, np.array([0], dtype=np.uint8))[0] == np.float32(2.0 ** -128)


def test_rope_yarn_table_bit_exact():
    f = _load("rope_yarn.npz")
    inv_freq, att = layer.yarn_inv_freq()
    assert torch.equal(inv_freq, torch.from_numpy(f["inv_freq"]))
    assert att == float(f["attention_scaling"])
    cos, sin = layer.rope_table(131072)
    pos = torch.from_numpy(f["positions"])
    ref_cos = torch.from_numpy(f["cos_bits"]).view(torch.bfloat16).float()
    ref_sin = torch.from_numpy(f["sin_bits"]).view(torch.bfloat16).float()
    assert torch.equal(cos[pos], ref_cos) and torch.equal(sin[pos], ref_sin)


def _layer_params(f, li, sliding):
    g = lambda k: f[f"L{li}_{k}"]
    t = lambda a: torch.from_numpy(np.asarray(a, dtype=np.float32))
    wqkv = torch.cat([t(g("wq")), t(g("wk")), t(g("wv"))], 0)
    bqkv = torch.cat([t(g("bq")), t(g("bk")), t(g("bv"))], 0)
    moe = experts.MxExpertWeights(g("gate_up_blocks"), g("gate_up_scales"), g("gate_up_bias"),
                                  g("down_blocks"), g("down_scales"), g("down_bias"))
    return layer.LayerParams(t(g("ln1")), t(g("ln2")), wqkv, bqkv, t(g("wo")), t(g("bo")),
                             t(g("sinks")), t(g("router_w")), t(g("router_b")), moe, sliding)


def _run_small_stage(f, params, steps, teacher=True):
    """Drive the oracle's decoder layers through the fixture's two steps with the module constants
    patched to the fixture's tiny shapes; returns {(step, layer): output}.  With ``teacher`` each
    layer reads transformers' own input for that layer (the bar is per layer, not chained)."""
    H, NQ, NKV, D, W, K = (int(f[k]) for k in ("H", "NQ", "NKV", "D", "W", "K"))
    saved = (layer.N_Q_HEADS, layer.N_KV_HEADS, layer.HEAD_DIM, layer.WINDOW)
    layer.N_Q_HEADS, layer.N_KV_HEADS, layer.HEAD_DIM, layer.WINDOW = NQ, NKV, D, W
    orig_moe = layer.moe_block
    layer.moe_block = lambda x, p, k=K, trace=None, force_ids=None: orig_moe(x, p, k=K, trace=trace, force_ids=force_ids)
    try:
        cos, sin = layer.rope_table(64)
        kv = [([torch.zeros(NKV, 16, D)], [torch.zeros(NKV, 16, D)]) for _ in params]
        outs = {}
        for si, (start, h) in enumerate(steps):
            for li, p in enumerate(params):
                if teacher and li > 0:
                    h = torch.from_numpy(f[f"out_step{si}_L{li - 1}"])
                h = layer.decoder_layer(h, p, kv[li], [h.shape[0]], [start], cos, sin)
                outs[(si, li)] = h
        return outs
    finally:
        layer.N_Q_HEADS, layer.N_KV_HEADS, layer.HEAD_DIM, layer.WINDOW = saved
        layer.moe_block = orig_moe


def test_decoder_layers_match_transformers():
    f = _load("gptoss_layers.npz")
    params = [_layer_params(f, 0, True), _layer_params(f, 1, False)]
    x = torch.from_numpy(f["x"])[:5]
    x1 = torch.from_numpy(f["x_step1"])
    outs = _run_small_stage(f, params, [(0, x), (5, x1)])
    for si in range(2):
        for li in range(2):
            ref = f[f"out_step{si}_L{li}"]
            mar, cos = metrics(outs[(si, li)].numpy(), ref)
            assert mar <= MAR and cos >= COS, f"step {si} layer {li}: max-abs-rel {mar:.3g} cos {cos:.6f}"


def test_decoder_layer_catches_planted_mistakes():
    """Each plausible restatement mistake, planted in the oracle, must fail the fixture bar."""
    f = _load("gptoss_layers.npz")
    x = torch.from_numpy(f["x"])[:5]
    x1 = torch.from_numpy(f["x_step1"])
    ref = f["out_step1_L1"]

    def run():
        params = [_layer_params(f, 0, True), _layer_params(f, 1, False)]
        return _run_small_stage(f, params, [(0, x), (5, x1)])[(1, 1)].numpy()

    planted = []
    orig_swiglu = experts.swiglu
    experts.swiglu = lambda g, u, alpha=1.702, limit=7.0: orig_swiglu(u, g, alpha, limit)  # gate/up swapped
    planted.append(("gate/up interleave swapped", run()))
    experts.swiglu = orig_swiglu
    orig_deq = mxfp4.dequant
    mxfp4.dequant = lambda b, s: orig_deq(((b & 0x0F) << 4) | (b >> 4), s)                 # nibble order
    planted.append(("nibble order swapped", run()))
    mxfp4.dequant = orig_deq
    orig_rope = layer.apply_rope
    layer.apply_rope = lambda xx, c, s: orig_rope(xx, c, -s)                              # rotation sign
    planted.append(("rope sign flipped", run()))
    layer.apply_rope = orig_rope
    orig_attn = attention.ragged_attention
    attention.ragged_attention = lambda q, k, v, ql, st, sinks, w, scale=None: orig_attn(
        q, k, v, ql, st, sinks * 0 - 1e9, w, scale)                                      # sink dropped
    planted.append(("sink ignored", run()))
    attention.ragged_attention = orig_attn
    for name, out in planted:
        mar, cos = metrics(out, ref)
        assert not (mar <= MAR and cos >= COS), f"planted mistake not caught: {name}"
    mar, cos = metrics(run(), ref)
    assert mar <= MAR and cos >= COS
