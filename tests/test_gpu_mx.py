"""Dense MXFP4 expert groups on the CDNA4 scaled MFMA (two-term fp8 activations x E2M1 weights).

* flyai_mx_act_quant: bit-exact against the oracle's mx_act_quant_two_term -- every e4m3 byte and every
  E8M0 scale byte of both terms (rows 0..M-1 the high term, M..2M-1 the low term), in the MFMA-ordered
  scale layout, padding bytes 127.
* gate_up / down with the fp8 activation operand: against oracle.experts_mxfp4_fp8act, which carries
  the same two-term operands through an fp32 product (the bar: fp32 accumulation order and bf16
  rounding of h only), and against the bf16 model math (experts_mxfp4) at the path's accuracy bar
  (max-abs-rel 2e-2, cosine 0.999; the two terms hold the bf16 operand to 2^-6 of each block's largest
  value, so the measured agreement is far inside it).  Groups of 8 rows or fewer keep the bf16 row-pass
  kernel, so a decode-sized batch gives the bf16 path's exact bits."""
import numpy as np
import pytest
import torch

from oracle import experts as oexperts

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _gen(seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return g


def _metrics(a, b):
    from gpu_harness import metrics
    return metrics(a, b)


def _unpack_scales(s, K):
    """MFMA-ordered scale bytes [M, row bytes] -> [M, K/32] in block order."""
    G = K // 32
    s = s.cpu().numpy()
    out = np.zeros((s.shape[0], G), dtype=np.uint8)
    for blk in range(G):
        kg, g = blk // 4, blk % 4
        out[:, blk] = s[:, 4 * ((kg // 4) * 4 + g) + (kg % 4)]
    return out


@pytest.mark.parametrize("M,K", [(7, 2880), (33, 4096), (5, 96)])
def test_mx_act_quant_bit_exact(M, K):
    from flyai_amd import ops
    x = torch.randn(M, K, device=DEV, generator=_gen(M + K))
    x = x * torch.logspace(-3, 2, M, device=DEV)[:, None]           # rows of very different magnitude
    x[0, 32:64] = 0.0                                               # a zero block: the 1e-4 amax floor
    x = x.to(torch.bfloat16)
    q, s = ops.mx_act_quant(x)
    torch.cuda.synchronize()
    assert q.shape == (2 * M, K) and s.shape[0] == 2 * M
    rq1, rs1, rq2, rs2 = oexperts.mx_act_quant_two_term(x.float().cpu().numpy())
    got_q = q.cpu().view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(got_q[:M], rq1), "high-term fp8 bytes differ from the oracle"
    assert np.array_equal(got_q[M:], rq2), "low-term fp8 bytes differ from the oracle"
    got_s = _unpack_scales(s, K)
    for name, rs, part in (("high", rs1, got_s[:M]), ("low", rs2, got_s[M:])):
        want_s = (np.log2(rs).astype(np.int32) + 127).astype(np.uint8)
        assert np.array_equal(part, want_s), f"{name}-term E8M0 scale bytes differ from the oracle"
    # every byte past the row's last block reads 127 (2^0)
    G, rowb = K // 32, s.shape[1]
    used = {4 * ((blk // 16) * 4 + blk % 4) + (blk // 4) % 4 for blk in range(G)}
    pad = [b for b in range(rowb) if b not in used]
    assert (s.cpu().numpy()[:, pad] == 127).all()


def _moe_case(T, E, seed, hot=None):
    from flyai_amd import ops
    from flyai_amd.weights import GptOssShape, synthetic_moe
    shape = GptOssShape(n_experts=E)
    m = synthetic_moe(shape, _gen(seed), DEV)
    w13 = ops.mxfp4_repack(m["w13_blocks"], m["w13_scales"])
    w2 = ops.mxfp4_repack(m["w2_blocks"], m["w2_scales"])
    x = (torch.randn(T, shape.hidden, device=DEV, generator=_gen(seed + 1))).to(torch.bfloat16)
    rw = (torch.randn(E, shape.hidden, device=DEV, generator=_gen(seed + 2)) * 0.02).to(torch.bfloat16)
    rb = torch.zeros(E, dtype=torch.bfloat16, device=DEV)
    if hot is not None:
        rb[hot] = 4.0
    ids, wts = ops.router_topk_softmax(x, rw, rb, 4)
    hist, off, perm, inv = ops.moe_permute(ids, E)
    wo = oexperts.MxExpertWeights(*(m[n].cpu().numpy() for n in
                                    ("w13_blocks", "w13_scales", "b13", "w2_blocks", "w2_scales", "b2")))
    return shape, m, w13, w2, x, off, perm, wo


@pytest.mark.parametrize("T,E,hot", [(128, 8, None), (320, 4, None), (600, 32, None), (12, 128, None), (600, 16, 5)])
def test_moe_experts_fp8act_vs_oracle(T, E, hot):
    """(128, 8): 64 rows per expert, one 64-row pass; (320, 4): every token on every expert, passes of
    96 + 96 + 96 + 32 rows; (600, 32): a spread of group sizes, a few under 9 rows on the row-pass kernel;
    (12, 128): decode-sized, all groups on the bf16 row-pass kernel (bit-identical to the bf16 path);
    (600, 16, hot 5): one expert holds nearly every token (seven passes, each its own work unit)."""
    from flyai_amd import ops
    shape, m, w13, w2, x, off, perm, wo = _moe_case(T, E, 60 + E, hot)
    I, H = shape.intermediate, shape.hidden
    xq, xs = ops.mx_act_quant(x)
    h = ops.moe_gate_up_fp8act(x, xq, xs, perm, off, 4, w13, m["b13"], E, I)
    hq, hs = ops.mx_act_quant(h)
    y = ops.moe_down_fp8act(h, hq, hs, off, w2, m["b2"], E, H)
    torch.cuda.synchronize()
    perm_c, off_c = perm.cpu().numpy(), off.cpu().numpy()
    hist = np.diff(off_c)
    if T * 4 < 8 * E:
        h16 = ops.moe_gate_up(x, perm, off, 4, w13, m["b13"], E, I)
        y16 = ops.moe_down(h16, off, w2, m["b2"], E, H)
        torch.cuda.synchronize()
        assert torch.equal(h, h16) and torch.equal(y, y16), "decode-sized batch left the bf16 row-pass kernel"
        return
    dense = np.repeat(hist > 8, hist)        # rows of dense groups (the scaled-MFMA kernel)
    ry, rh = oexperts.experts_mxfp4_fp8act(x.float().cpu(), perm_c, off_c, 4, wo, return_h=True)
    ry16, rh16 = oexperts.experts_mxfp4(x.float().cpu(), perm_c, off_c, 4, wo, return_h=True)
    hd, yd = h.float().cpu().numpy()[dense], y.cpu().numpy()[dense]
    mar, cos = _metrics(hd, rh.numpy()[dense])
    assert mar <= 1e-2 and cos >= 0.99999, f"gate_up vs the fp8-activation oracle: {mar:.3g} {cos:.7f}"
    mar, cos = _metrics(yd, ry.numpy()[dense])
    assert mar <= 1e-2 and cos >= 0.99999, f"down vs the fp8-activation oracle: {mar:.3g} {cos:.7f}"
    # against the bf16 model math: the accuracy bar on the expert outputs themselves
    mar, cos = _metrics(hd, rh16.numpy()[dense])
    print(f"T={T} E={E}: gate_up vs bf16 math max-abs-rel {mar:.3g} cos {cos:.7f}")
    assert mar <= 2e-2 and cos >= 0.999, f"gate_up vs the bf16 model math: {mar:.3g} {cos:.6f}"
    mar, cos = _metrics(yd, ry16.numpy()[dense])
    print(f"T={T} E={E}: down vs bf16 math max-abs-rel {mar:.3g} cos {cos:.7f}")
    assert mar <= 2e-2 and cos >= 0.999, f"down vs the bf16 model math: {mar:.3g} {cos:.6f}"
    if (~dense).any():   # small groups stay on the bf16 row-pass kernel
        mar, cos = _metrics(h.float().cpu().numpy()[~dense], rh16.numpy()[~dense])
        assert mar <= 2e-2 and cos >= 0.999
