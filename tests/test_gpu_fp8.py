"""GPU parity tests of the DeepSeek-V3-shaped FP8 MoE path against the CPU oracle.

Bars: bit-exact for the activation quantiser (e4m3 bytes and E8M0 scale bytes) and for the grouped
router's ids and weights; bf16 outputs of the experts and the whole layer within max-abs-rel 2e-2 and
cosine >= 0.999 (fp32 MFMA accumulation vs the oracle's fp64, plus bf16 rounding of gate/up/h)."""
import numpy as np
import pytest
import torch

from oracle import experts as oexperts
from oracle import layer as olayer
from oracle import routing as oroute

pytestmark = pytest.mark.gpu

MAR, COS = 2e-2, 0.999
DEV = "cuda"


def _metrics(a, b):
    from gpu_harness import metrics
    return metrics(a, b)


def _gen(seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return g


def e4m3_vals(u8):
    return u8.cpu().view(torch.float8_e4m3fn).float().numpy()


def e8m0_vals(u8):
    return np.ldexp(np.float32(1.0), u8.cpu().numpy().astype(np.int32) - 127).astype(np.float32)


class GpuFp8Experts:
    """Oracle view of device expert weights: converts only the experts the oracle asks for."""

    def __init__(self, raw):
        self.raw = raw

    def arrays(self, e):
        r = self.raw
        return (e4m3_vals(r["w1"][e]), e8m0_vals(r["s1"][e]), e4m3_vals(r["w3"][e]), e8m0_vals(r["s3"][e]),
                e4m3_vals(r["w2"][e]), e8m0_vals(r["s2"][e]))

    def expert(self, e, x, weight=None):
        return oexperts.deepseek_expert(x, *self.arrays(e), weight)


# ---- activation quantiser -----------------------------------------------------------------------

@pytest.mark.parametrize("M,K", [(5, 1024), (37, 7168)])
def test_fp8_act_quant_bit_exact(M, K):
    from flyai_amd import ops
    scale = torch.logspace(-6, 3, M, device=DEV)[:, None]
    x = torch.randn(M, K, device=DEV, generator=_gen(1)) * scale
    x[0, :128] = 0.0            # amax clamps to 1e-4
    x[1, 5] = 3.0e4             # one outlier dominates its block
    x[2, 130] = -448.0 * 2.0 ** 3  # amax exactly 448 * 2^k: scale 2^k, value 448
    xb = x.to(torch.bfloat16)
    q, s = ops.fp8_act_quant(xb)
    rq, rs = oexperts.act_quant_128(xb.float().cpu().numpy())
    want_q = torch.from_numpy(rq).to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(q.cpu(), want_q)
    assert np.array_equal(s.cpu().numpy().astype(np.int32) - 127, np.log2(rs).astype(np.int32))


# ---- grouped sigmoid router ----------------------------------------------------------------------

@pytest.mark.parametrize("T,H,E,ng,tg,k", [(37, 7168, 256, 8, 4, 8), (19, 1024, 32, 8, 4, 4),
                                           (8, 512, 64, 1, 1, 6), (64, 2048, 128, 4, 2, 8)])
def test_grouped_router_bit_exact(T, H, E, ng, tg, k):
    from flyai_amd import ops
    from flyai_amd.weights import zipf_bias
    g = _gen(2)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, H, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    bias = zipf_bias(E, 1.1, g, DEV)
    ids, wts, logits = ops.router_grouped_sigmoid(x, w, bias, ng, tg, k, 2.5)
    rl = oroute.dot_fixed(x.float().cpu(), w.float().cpu()).numpy()
    assert np.array_equal(logits.cpu().numpy(), rl)
    rids, rwts, _ = oroute.grouped_sigmoid_route(x.float().cpu().numpy(), w.float().cpu().numpy(),
                                                 bias.cpu().numpy(), ng, tg, k, 2.5)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.array_equal(wts.cpu().numpy(), rwts)


def test_grouped_router_ties_go_to_lower_ids():
    """Zero router weights make every score sigmoid(0) = 0.5; a bias with repeated values then
    leaves ties in both the group scores and the expert choices."""
    from flyai_amd import ops
    T, H, E, ng, tg, k = 5, 512, 64, 8, 4, 8
    x = torch.randn(T, H, device=DEV, generator=_gen(3)).to(torch.bfloat16)
    w = torch.zeros(E, H, device=DEV, dtype=torch.bfloat16)
    bias = torch.tensor([(e % 3) * 0.25 for e in range(E)], device=DEV, dtype=torch.float32)
    ids, wts, _ = ops.router_grouped_sigmoid(x, w, bias, ng, tg, k, 2.5)
    rids, rwts, _ = oroute.grouped_sigmoid_route(x.float().cpu().numpy(), w.float().cpu().numpy(),
                                                 bias.cpu().numpy(), ng, tg, k, 2.5)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.array_equal(wts.cpu().numpy(), rwts)


# ---- FP8 experts ---------------------------------------------------------------------------------

def _assignments(T, k, E, hot, n_hot, gen):
    """ids [T, k] (distinct, ascending per row): the first n_hot tokens all pick expert `hot`;
    expert E-1 is never picked."""
    rows = []
    for t in range(T):
        pool = torch.randperm(E - 1, generator=gen).tolist()
        pick = ([hot] if t < n_hot else []) + [e for e in pool if e != hot]
        rows.append(sorted(pick[:k]))
    return torch.tensor(rows, dtype=torch.int32)


@pytest.mark.parametrize("T,n_hot", [(12, 0), (80, 0), (160, 150)])
def test_fp8_experts_vs_oracle(T, n_hot):
    """gate_up (+ silu * up * weight) and down per routed row.  T=12 keeps every group at most 16
    rows (one-row-tile kernel); T=80 puts ~23 rows on each expert (8-row-tile kernel, one pass);
    n_hot=150 puts 150 rows on one expert (8-row-tile kernel, two passes of up to 128 rows)."""
    from flyai_amd import ops
    from flyai_amd.weights import synthetic_fp8_experts
    E, H, I, k = 8, 2048, 1024, 2
    g = _gen(4)
    ex = synthetic_fp8_experts(E, H, I, g, DEV, std=0.05)
    w13 = ops.fp8_repack(ex["w1"], ex["s1"], ex["w3"], ex["s3"])
    w2 = ops.fp8_repack(ex["w2"], ex["s2"])
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    ids = _assignments(T, k, E, 3, n_hot, torch.Generator().manual_seed(5)).to(DEV)
    wts = torch.rand(T, k, device=DEV, generator=g) + 0.5
    hist, off, perm, inv = ops.moe_permute(ids, E)
    xq, xs = ops.fp8_act_quant(x)
    h = ops.moe_gate_up_fp8(xq, xs, perm, off, k, wts, w13, E, I)
    hq, hs = ops.fp8_act_quant(h)
    y = ops.moe_down_fp8(hq, hs, off, w2, E, H)
    torch.cuda.synchronize()
    assert int(hist.max()) >= max(n_hot, 1)
    view = GpuFp8Experts(ex)
    xc, hc, yc = x.float().cpu().numpy(), h.float().cpu().numpy(), y.float().cpu().numpy()
    perm_c, off_c = perm.cpu().numpy(), off.cpu().numpy()
    ids_f, wts_f = ids.cpu().numpy().reshape(-1), wts.cpu().numpy().reshape(-1)
    for e in range(E):
        lo, hi = off_c[e], off_c[e + 1]
        if lo == hi:
            continue
        w1, s1, w3, s3, w2a, s2 = view.arrays(e)
        f = perm_c[lo:hi]
        assert (ids_f[f] == e).all()
        xt = xc[f // k]
        gate = oexperts.fp8_linear(xt, w1, s1)
        up = oexperts.fp8_linear(xt, w3, s3)
        h_ref = (torch.nn.functional.silu(gate) * up * torch.from_numpy(wts_f[f])[:, None]).numpy()
        mar, cos = _metrics(hc[lo:hi], h_ref)
        assert mar <= MAR and cos >= COS, f"gate_up expert {e}: {mar:.3g} {cos:.6f}"
        y_ref = oexperts.fp8_linear(hc[lo:hi], w2a, s2).numpy()
        mar, cos = _metrics(yc[lo:hi], y_ref)
        assert mar <= MAR and cos >= COS, f"down expert {e}: {mar:.3g} {cos:.6f}"


def test_fp8_shared_expert_group():
    """The shared expert as group E of the same launch: 40 tokens (a dense-sized group) next to
    routed rows; its rows come after the routed ones and equal the oracle's expert on every token."""
    from flyai_amd import ops
    from flyai_amd.weights import synthetic_fp8_experts
    E, H, I, T, k = 4, 1024, 1024, 40, 1
    g = _gen(6)
    ex = synthetic_fp8_experts(E + 1, H, I, g, DEV, std=0.05)   # expert E is the shared one
    w13 = ops.fp8_repack(ex["w1"], ex["s1"], ex["w3"], ex["s3"])
    w2 = ops.fp8_repack(ex["w2"], ex["s2"])
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    ids = (torch.arange(T, device=DEV, dtype=torch.int32) % E).view(T, 1)
    wts = torch.ones(T, 1, device=DEV)
    hist, off, perm, inv = ops.moe_permute(ids, E)
    xq, xs = ops.fp8_act_quant(x)
    h = ops.moe_gate_up_fp8(xq, xs, perm, off, k, wts, w13, E, I, n_shared=T)
    hq, hs = ops.fp8_act_quant(h)
    y = ops.moe_down_fp8(hq, hs, off, w2, E, H, n_shared=T)
    torch.cuda.synchronize()
    ref = GpuFp8Experts(ex).expert(E, x.float().cpu().numpy()).numpy()
    mar, cos = _metrics(y[T * k:].float().cpu().numpy(), ref)
    assert mar <= MAR and cos >= COS, f"shared expert: {mar:.3g} {cos:.6f}"
    perm_c = perm.cpu().numpy()
    for e in range(E):
        rows = slice(int(off[e]), int(off[e + 1]))
        ref_e = GpuFp8Experts(ex).expert(e, x.float().cpu().numpy()[perm_c[rows] // k]).numpy()
        mar, cos = _metrics(y[rows].float().cpu().numpy(), ref_e)
        assert mar <= MAR and cos >= COS, f"routed expert {e}: {mar:.3g} {cos:.6f}"


def test_deepseek_moe_layer_vs_oracle():
    """One full DeepSeek-V3-shaped layer (H 7168, 256 experts, top-8 grouped sigmoid, shared
    expert).  The oracle routes the GPU's own RMSNorm output (checked against the oracle's RMSNorm
    first), so a 1-ulp bf16 difference cannot flip an expert choice near a tie."""
    from flyai_amd import ops
    from flyai_amd.runtime import Fp8MoeStage
    from flyai_amd.weights import DsV3Shape, synthetic_fp8_moe_layer
    sh = DsV3Shape()
    lw = synthetic_fp8_moe_layer(sh, 11, DEV, keep_raw=True)
    T = 6
    h0 = torch.randn(T, sh.hidden, device=DEV, generator=_gen(12)).to(torch.bfloat16)
    xn = ops.rmsnorm(h0, lw.ln, sh.rms_eps)
    h = Fp8MoeStage(sh, [lw]).forward(h0.clone())
    torch.cuda.synchronize()
    xn_ref = olayer.rmsnorm(h0.float().cpu(), lw.ln.cpu(), sh.rms_eps)
    mar, cos = _metrics(xn.float().cpu().numpy(), xn_ref.numpy())
    assert mar <= MAR and cos >= COS, f"rmsnorm: {mar:.3g} {cos:.6f}"
    xc = xn.float().cpu().numpy()
    rids, rwts, _ = oroute.grouped_sigmoid_route(xc, lw.router_w.float().cpu().numpy(), lw.e_bias.cpu().numpy(),
                                                 sh.n_group, sh.topk_group, sh.top_k, sh.route_scale)
    y = oexperts.deepseek_moe(xc, rids, rwts, GpuFp8Experts(lw.raw), GpuFp8Experts(lw.shared_raw))
    ref = (h0.float().cpu() + y).to(torch.bfloat16).float()
    mar, cos = _metrics(h.float().cpu().numpy(), ref.numpy())
    assert mar <= MAR and cos >= COS, f"layer: {mar:.3g} {cos:.6f}"
    # the MoE increment alone (the residual dominates the sum)
    mar, cos = _metrics((h.float() - h0.float()).cpu().numpy(), (ref - h0.float().cpu()).numpy())
    assert cos >= COS, f"moe delta cos {cos:.6f}"
