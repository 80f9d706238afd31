"""GPU parity tests: every kernel through the C ABI against the CPU oracle on the same seeded inputs.

Bars: bit-exact for packing, router indices, histogram / permutation (and for the RoPE / KV writes,
whose rounding is per element); bf16 outputs within max-abs-rel 2e-2 and cosine >= 0.999."""
import numpy as np
import pytest
import torch

from flyai_amd import kvlayout

from oracle import attention as oattn
from oracle import experts as oexperts
from oracle import layer as olayer
from oracle import packing as opack
from oracle import routing as oroute
from oracle.numerics import bf16

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


# ---- a1 ----------------------------------------------------------------------------------------

@pytest.mark.parametrize("q_lens,starts", [([1, 1, 3, 7], [0, 5, 9, 100]),
                                           ([1] * 24 + [4] * 8, list(range(512, 512 + 32 * 200, 200))),
                                           ([2048] + [1] * 48, [4096] + list(range(600, 648)))])
def test_pack_ragged_bit_exact(q_lens, starts):
    from flyai_amd import ops
    S = len(q_lens)
    base = [s * 1000 * 64 for s in range(S)]
    cap = [8192] * S
    t = lambda v, dt: torch.tensor(v, dtype=dt, device=DEV)
    out = ops.pack_ragged(t(q_lens, torch.int32), t(starts, torch.int32), t(base, torch.int64),
                          t(cap, torch.int32), 64, 4096)
    ref = opack.pack_ragged(q_lens, starts, kv_base=base, kv_cap=cap, head_dim=64)
    T = sum(q_lens)
    assert out["status"].item() == 0
    assert out["cu_seqlens"].cpu().numpy().tolist() == ref["cu_seqlens"].tolist()
    assert out["positions"][:T].cpu().numpy().tolist() == ref["positions"].tolist()
    assert out["seq_id"][:T].cpu().numpy().tolist() == ref["seq_id"].tolist()
    assert out["kv_slot"][:T].cpu().numpy().tolist() == ref["kv_slot"].tolist()
    assert out["kv_len"].cpu().numpy().tolist() == ref["kv_len"].tolist()


def test_pack_ragged_overflow_status():
    from flyai_amd import ops
    t = lambda v, dt: torch.tensor(v, dtype=dt, device=DEV)
    out = ops.pack_ragged(t([8, 8], torch.int32), t([92, 93], torch.int32), t([0, 0], torch.int64),
                          t([100, 100], torch.int32), 64, 64)
    assert out["status"].item() & 1
    slots = out["kv_slot"][:16].cpu().numpy()
    assert (slots[:8] >= 0).all() and slots[15] == -1      # only the out-of-capacity token is blanked


# ---- a2 / a3 / a4 ------------------------------------------------------------------------------

def _rms_input(T, H, seed):
    x = torch.randn(T, H, device=DEV, generator=_gen(seed))
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5)
    return x.to(torch.bfloat16)


# (300, *, *, *) and (2096, ...) take the prefill-sized logits kernel, whose 1-D grid runs a token group's
# expert groups back to back on one XCD and exits the token groups past T (300 = 37.5 groups of 8)
@pytest.mark.parametrize("T,E,k,H", [(56, 128, 4, 2880), (12, 128, 4, 2880), (300, 32, 4, 256), (5, 8, 2, 128),
                                     (300, 128, 4, 2880), (2096, 128, 4, 2880)])
def test_router_indices_bit_exact(T, E, k, H):
    from flyai_amd import ops
    x = _rms_input(T, H, 1)
    w = (torch.randn(E, H, device=DEV, generator=_gen(2)) * 0.02).to(torch.bfloat16)
    b = (torch.randn(E, device=DEV, generator=_gen(3)) * 0.02).to(torch.bfloat16)
    ids, wts, logits = ops.router_topk_softmax(x, w, b, k, want_logits=True)
    rids, rw, rlog = oroute.gptoss_route(x.float().cpu(), w.float().cpu(), b.float().cpu(), k)
    assert torch.equal(logits.cpu(), rlog), "router logits differ from the fixed-order oracle"
    assert np.array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)


def test_router_exact_ties_go_to_lower_id():
    from flyai_amd import ops
    T, E, H = 16, 64, 128
    x = _rms_input(T, H, 4)
    base = (torch.randn(8, H, device=DEV, generator=_gen(5)) * 0.05).to(torch.bfloat16)
    w = base.repeat(8, 1).contiguous()                      # experts e and e+8 are identical rows
    b = torch.zeros(E, dtype=torch.bfloat16, device=DEV)
    ids, _ = ops.router_topk_softmax(x, w, b, 4)
    rids, _, _ = oroute.gptoss_route(x.float().cpu(), w.float().cpu(), b.float().cpu(), 4)
    assert np.array_equal(ids.cpu().numpy(), rids)
    # the winning row has 8 identical copies (r, r+8, ..., r+56): top-4 must be its 4 lowest ids
    got = ids.cpu().numpy()
    r = got[:, :1] % 8
    assert (got == r + np.arange(4)[None, :] * 8).all()


@pytest.mark.parametrize("T,E,H", [(56, 128, 2880), (12, 128, 2880), (1024, 128, 2880), (1025, 128, 2880),
                                   (33, 256, 7168)])
def test_fused_route_permute_bit_exact(T, E, H):
    """The stage's fused path (one-workgroup top-k + permute for T*k <= 4096, split above)."""
    from flyai_amd import ops
    k = 4 if E == 128 else 8
    x = _rms_input(T, H, 12)
    w = (torch.randn(E, H, device=DEV, generator=_gen(13)) * 0.02).to(torch.bfloat16)
    b = (torch.randn(E, device=DEV, generator=_gen(14)) * 0.02).to(torch.bfloat16)
    ids, wts, hist, off, perm, inv = ops.moe_route_permute(x, w, b, k)
    rids, rw, _ = oroute.gptoss_route(x.float().cpu(), w.float().cpu(), b.float().cpu(), k)
    rh, ro, rp, ri = oroute.permute(rids, E)
    assert np.array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)
    for got, ref in ((hist, rh), (off, ro), (perm, rp), (inv, ri)):
        assert np.array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("T,E,k", [(20, 128, 4), (56, 128, 8), (7, 64, 2)])
def test_fused_route_permute_ties_go_to_lower_id(T, E, k):
    """Zero router weights leave logits = bias; a bias with many equal values makes ties inside a
    lane's quarter and across the four lanes that share a token.  Bit-exact ids and weights."""
    from flyai_amd import ops
    x = _rms_input(T, 2880, 15)
    w = torch.zeros(E, 2880, device=DEV, dtype=torch.bfloat16)
    b = torch.tensor([((e * 7) % 5) * 0.125 for e in range(E)], device=DEV).to(torch.bfloat16)
    ids, wts, hist, off, perm, inv = ops.moe_route_permute(x, w, b, k)
    rids, rw, _ = oroute.gptoss_route(x.float().cpu(), w.float().cpu(), b.float().cpu(), k)
    assert np.array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(wts.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)
    rh, ro, rp, ri = oroute.permute(rids, E)
    for got, ref in ((hist, rh), (off, ro), (perm, rp), (inv, ri)):
        assert np.array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("T,k,E,mode", [(1, 4, 128, "rand"), (56, 4, 128, "rand"), (2096, 4, 128, "rand"),
                                        (4096, 4, 256, "skew"), (64, 4, 8, "one"), (16384, 4, 128, "rand")])
def test_permute_bit_exact(T, k, E, mode):
    from flyai_amd import ops
    rng = np.random.default_rng(T + E)
    if mode == "one":
        ids = np.tile(np.arange(k), (T, 1))
    elif mode == "skew":
        hot = rng.choice(E, E // 10, replace=False)
        ids = np.stack([np.sort(rng.choice(hot, k, replace=False)) if rng.random() < 0.5
                        else np.sort(rng.choice(E, k, replace=False)) for _ in range(T)])
    else:
        ids = np.sort(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]), axis=1)
    ids_d = torch.tensor(ids, dtype=torch.int32, device=DEV)
    hist, off, perm, inv = ops.moe_permute(ids_d, E)
    rh, ro, rp, ri = oroute.permute(ids, E)
    assert np.array_equal(hist.cpu().numpy(), rh)
    assert np.array_equal(off.cpu().numpy(), ro)
    assert np.array_equal(perm.cpu().numpy(), rp)
    assert np.array_equal(inv.cpu().numpy(), ri)


def test_nan_router_rows_route_consistently():
    """A router row of NaN (a NaN hidden state) must not break the routing's index invariants: the
    expert and combine kernels index with perm, inv and offsets.  The top-k gives such a row
    in-range ids, and the permute counts any id outside [0, E) as expert 0, so the histogram sums to
    T*k and perm / inv stay a permutation and its inverse."""
    from flyai_amd import ops
    T, H, E, k = 40, 2880, 128, 4
    g = _gen(140)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    x[3] = float("nan")
    x[17, 5] = float("nan")
    rw = (0.02 * torch.randn(E, H, device=DEV, generator=g)).to(torch.bfloat16)
    rb = torch.zeros(E, device=DEV, dtype=torch.bfloat16)
    ids, wts = ops.router_topk_softmax(x, rw, rb, k)
    ids_h = ids.cpu().numpy()
    assert ((ids_h >= 0) & (ids_h < E)).all(), "router ids out of range on a NaN row"
    # ids outside [0, E) straight into the permute: counted as expert 0
    bad = ids_h.copy()
    bad[0] = [-1, E, 2**31 - 1, 7]
    hist, off, perm, inv = ops.moe_permute(torch.tensor(bad, dtype=torch.int32, device=DEV), E)
    want = np.where((bad >= 0) & (bad < E), bad, 0)
    rh, ro, rp, ri = oroute.permute(want, E)
    assert np.array_equal(hist.cpu().numpy(), rh) and np.array_equal(off.cpu().numpy(), ro)
    assert np.array_equal(perm.cpu().numpy(), rp) and np.array_equal(inv.cpu().numpy(), ri)


def test_combine_matches_oracle():
    from flyai_amd import ops
    T, k, H = 56, 4, 2880
    rng = np.random.default_rng(9)
    y = torch.randn(T * k, H, device=DEV, generator=_gen(9)) * 5
    inv = torch.tensor(rng.permutation(T * k), dtype=torch.int32, device=DEV)
    w = torch.softmax(torch.randn(T, k, device=DEV, generator=_gen(10)), -1)
    res = torch.randn(T, H, device=DEV, generator=_gen(11)).to(torch.bfloat16)
    out = ops.moe_combine(y, inv, w, residual=res.clone())
    ref = oroute.combine(y.cpu(), inv.cpu().numpy(), w.cpu(), residual=res.float().cpu())
    mar, cos = _metrics(out.float().cpu().numpy(), ref.numpy())
    assert mar < 1e-2 and cos > 0.99999


# ---- a5 / a6 -----------------------------------------------------------------------------------

@pytest.mark.parametrize("T,E,hot", [(12, 128, None), (128, 8, None), (3, 4, None), (320, 4, None), (600, 16, 5)])
def test_moe_experts_vs_oracle(T, E, hot):
    """gate_up (+SwiGLU) and down through the packed MXFP4 layout.  (12, 128) and (3, 4) are
    decode-sized (row-pass kernel); (128, 8) averages 64 rows per expert (dense kernel, one pass);
    (320, 4) puts all 320 tokens on every expert (dense kernel, four passes of up to 96 rows, each its
    own work unit); (600, 16, hot 5) biases the router to one expert, which then holds nearly every
    token (seven passes) beside groups of about 120 rows."""
    from flyai_amd import ops
    from flyai_amd.weights import GptOssShape, synthetic_moe
    shape = GptOssShape(n_experts=E)
    m = synthetic_moe(shape, _gen(20 + E), DEV)
    w13 = ops.mxfp4_repack(m["w13_blocks"], m["w13_scales"])
    w2 = ops.mxfp4_repack(m["w2_blocks"], m["w2_scales"])
    x = _rms_input(T, shape.hidden, 21)
    rw = (torch.randn(E, shape.hidden, device=DEV, generator=_gen(22)) * 0.02).to(torch.bfloat16)
    rb = torch.zeros(E, dtype=torch.bfloat16, device=DEV)
    if hot is not None:
        rb[hot] = 4.0
    ids, wts = ops.router_topk_softmax(x, rw, rb, 4)
    hist, off, perm, inv = ops.moe_permute(ids, E)
    if hot is not None:
        hc = hist.cpu().numpy()
        assert hc[hot] > 5 * 96, hc
    h = ops.moe_gate_up(x, perm, off, 4, w13, m["b13"], E, shape.intermediate)
    y = ops.moe_down(h, off, w2, m["b2"], E, shape.hidden)
    torch.cuda.synchronize()
    wts_o = oexperts.MxExpertWeights(*(m[n].cpu().numpy() for n in
                                       ("w13_blocks", "w13_scales", "b13", "w2_blocks", "w2_scales", "b2")))
    ry, rh = oexperts.experts_mxfp4(x.float().cpu(), perm.cpu().numpy(), off.cpu().numpy(), 4, wts_o,
                                    return_h=True)
    mar, cos = _metrics(h.float().cpu().numpy(), rh.numpy())
    assert mar <= MAR and cos >= COS, f"gate_up+swiglu: {mar:.3g} {cos:.6f}"
    mar, cos = _metrics(y.cpu().numpy(), ry.numpy())
    assert mar <= MAR and cos >= COS, f"down: {mar:.3g} {cos:.6f}"


# ---- a9 ----------------------------------------------------------------------------------------

def test_rmsnorm_and_linear_vs_oracle():
    from flyai_amd import ops
    T, H, N = 56, 2880, 5120
    x = torch.randn(T, H, device=DEV, generator=_gen(30)).to(torch.bfloat16) * 3
    w = (1 + 0.1 * torch.randn(H, device=DEV, generator=_gen(31))).float()
    y = ops.rmsnorm(x, w)
    ref = olayer.rmsnorm(x.float().cpu(), w.cpu())
    mar, cos = _metrics(y.float().cpu().numpy(), ref.numpy())
    assert mar < 1e-2 and cos > 0.9999
    W = (torch.randn(N, H, device=DEV, generator=_gen(32)) * 0.02).to(torch.bfloat16)
    b = (torch.randn(N, device=DEV, generator=_gen(33)) * 0.02).to(torch.bfloat16)
    out = ops.linear(y, W, b)
    ref = olayer.linear(y.float().cpu(), W.float().cpu(), b.float().cpu())
    mar, cos = _metrics(out.float().cpu().numpy(), ref.numpy())
    assert mar < 1e-2 and cos > 0.9999
    Wo = (torch.randn(H, 4096, device=DEV, generator=_gen(34)) * 0.02).to(torch.bfloat16)
    a = torch.randn(T, 4096, device=DEV, generator=_gen(35)).to(torch.bfloat16)
    res = x.clone()
    ops.linear(a, Wo, None, residual=res)
    ref = bf16(x.float().cpu() + olayer.linear(a.float().cpu(), Wo.float().cpu()))
    mar, cos = _metrics(res.float().cpu().numpy(), ref.numpy())
    assert mar < 1e-2 and cos > 0.9999


@pytest.mark.parametrize("N,K", [(5120, 2880), (2880, 4096), (2000, 2880), (1008, 2080), (512, 7168)])
def test_linear_tiled_equals_split_k_bit_exact(N, K):
    """Prefill-sized batches (>= 256 rows) take a tiled GEMM, decode-sized ones the split-K GEMM;
    a row's projection must come out the same bits either way (batch invariance), and within the bar
    of the oracle.  K % 64 == 0 takes the direct-to-LDS tiled kernel (2880: 5 slices and a partial
    one; 4096 and 7168: whole slices only), K = 2080 the register-staged one."""
    from flyai_amd import ops
    M = 300
    x = torch.randn(M, K, device=DEV, generator=_gen(110)).to(torch.bfloat16)
    w = (0.02 * torch.randn(N, K, device=DEV, generator=_gen(111))).to(torch.bfloat16)
    b = (0.1 * torch.randn(N, device=DEV, generator=_gen(112))).to(torch.bfloat16)
    big = ops.linear(x, w, b)                       # tiled path
    parts = [ops.linear(x[r0:r0 + 60].contiguous(), w, b) for r0 in range(0, M, 60)]  # split-K path
    torch.cuda.synchronize()
    assert torch.equal(big, torch.cat(parts)), "tiled and split-K projections differ"
    ref = olayer.linear(x.float().cpu(), w.float().cpu(), b.float().cpu())
    mar, cos = _metrics(big.float().cpu().numpy(), ref.numpy())
    assert mar < 1e-2 and cos > 0.99999


def test_rope_kv_append_bit_exact():
    from flyai_amd import ops
    from flyai_amd.rope import YarnRotary
    q_lens, starts = [1, 4, 3], [100, 7, 4090]
    T, Hq, Hkv, D, cap = sum(q_lens), 64, 8, 64, 4160
    rot = YarnRotary(cap, device=DEV)
    pk = opack.pack_ragged(q_lens, starts)
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, device=DEV, generator=_gen(40)).to(torch.bfloat16)
    slab = Hkv * cap * D
    kp = torch.zeros(3 * slab, dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros(3 * slab, dtype=torch.bfloat16, device=DEV)
    base = torch.tensor([0, slab, 2 * slab], dtype=torch.int64, device=DEV)
    capt = torch.tensor([cap] * 3, dtype=torch.int32, device=DEV)
    pos = torch.tensor(pk["positions"], device=DEV)
    sid = torch.tensor(pk["seq_id"], device=DEV)
    q = ops.rope_kv_append(qkv, pos, sid, rot.cos, rot.sin, Hq, Hkv, D, base, capt, kp, vp)
    cos, sin = olayer.rope_table(cap)
    p = torch.from_numpy(pk["positions"].astype(np.int64))
    qc = qkv.float().cpu()
    rq = olayer.apply_rope(qc[:, :Hq * D].view(T, Hq, D), cos[p], sin[p])
    rk = olayer.apply_rope(qc[:, Hq * D:(Hq + Hkv) * D].view(T, Hkv, D), cos[p], sin[p])
    assert torch.equal(q.float().cpu(), rq)
    kcpu = [kvlayout.gather(kp[b * slab:(b + 1) * slab], Hkv, cap, "k").float().cpu() for b in range(3)]
    vcpu = [kvlayout.gather(vp[b * slab:(b + 1) * slab], Hkv, cap, "v").float().cpu() for b in range(3)]
    written = set()
    for t in range(T):
        b, ps = int(pk["seq_id"][t]), int(pk["positions"][t])
        written.add((b, ps))
        assert torch.equal(kcpu[b][:, ps, :], rk[t])
        assert torch.equal(vcpu[b][:, ps, :], qc[t, (Hq + Hkv) * D:].view(Hkv, D))
    # nothing else in the slabs was touched (the tiled offsets of distinct positions never overlap)
    for b in range(3):
        others = [p_ for p_ in range(cap) if (b, p_) not in written]
        assert not kcpu[b][:, others].any() and not vcpu[b][:, others].any()


# ---- a8 ----------------------------------------------------------------------------------------

@pytest.mark.parametrize("window", [0, 128])
@pytest.mark.parametrize("q_lens,starts", [([1] * 6 + [4] * 2, [700, 5, 64, 129, 1000, 2047, 300, 0]),
                                           ([130, 1, 9], [0, 3000, 511]),
                                           ([1, 8, 3], [0, 1, 4093])])
def test_attention_vs_oracle(window, q_lens, starts):
    from flyai_amd import ops
    Hq, Hkv, D, cap = 64, 8, 64, 4160
    S, T = len(q_lens), sum(q_lens)
    slab = Hkv * cap * D
    kp = torch.randn(S * slab, device=DEV, generator=_gen(50)).to(torch.bfloat16)
    vp = torch.randn(S * slab, device=DEV, generator=_gen(51)).to(torch.bfloat16)
    q = torch.randn(T, Hq, D, device=DEV, generator=_gen(52)).to(torch.bfloat16)
    sinks = torch.randn(Hq, device=DEV, generator=_gen(53)).to(torch.bfloat16).float()
    base = torch.tensor([b * slab for b in range(S)], dtype=torch.int64, device=DEV)
    capt = torch.tensor([cap] * S, dtype=torch.int32, device=DEV)
    items, groups, n_small = ops.attn_plan(q_lens, starts, Hkv, window, 512)
    out = ops.attn_ragged(q, kp, vp, base, capt, sinks, window, items, groups, n_small, Hkv)
    ks = [kvlayout.gather(kp[b * slab:(b + 1) * slab], Hkv, cap, "k").float().cpu() for b in range(S)]
    vs = [kvlayout.gather(vp[b * slab:(b + 1) * slab], Hkv, cap, "v").float().cpu() for b in range(S)]
    ref = oattn.ragged_attention(q.float().cpu(), ks, vs, q_lens, starts, sinks.cpu(), window)
    mar, cos = _metrics(out.float().cpu().numpy(), ref.numpy())
    assert mar <= MAR and cos >= COS, f"attention: {mar:.3g} {cos:.6f}"


@pytest.mark.parametrize("window", [0, 128])
def test_attention_many_splits_vs_oracle(window):
    """128-key splits: up to 32 splits per (token, head), so the merge reads its split maxima and
    records over several batches, including a partial last batch."""
    from flyai_amd import ops
    Hq, Hkv, D, cap = 64, 8, 64, 4160
    q_lens, starts = [1, 4, 2], [4093, 2301, 17]
    S, T = len(q_lens), sum(q_lens)
    slab = Hkv * cap * D
    kp = torch.randn(S * slab, device=DEV, generator=_gen(60)).to(torch.bfloat16)
    vp = torch.randn(S * slab, device=DEV, generator=_gen(61)).to(torch.bfloat16)
    q = torch.randn(T, Hq, D, device=DEV, generator=_gen(62)).to(torch.bfloat16)
    sinks = torch.randn(Hq, device=DEV, generator=_gen(63)).to(torch.bfloat16).float()
    base = torch.tensor([b * slab for b in range(S)], dtype=torch.int64, device=DEV)
    capt = torch.tensor([cap] * S, dtype=torch.int32, device=DEV)
    items, groups, n_small = ops.attn_plan(q_lens, starts, Hkv, window, 128)
    if window == 0:
        assert max(int(g[1]) for g in groups.cpu().view(-1, 8).tolist()) >= 32
    out = ops.attn_ragged(q, kp, vp, base, capt, sinks, window, items, groups, n_small, Hkv)
    ks = [kvlayout.gather(kp[b * slab:(b + 1) * slab], Hkv, cap, "k").float().cpu() for b in range(S)]
    vs = [kvlayout.gather(vp[b * slab:(b + 1) * slab], Hkv, cap, "v").float().cpu() for b in range(S)]
    ref = oattn.ragged_attention(q.float().cpu(), ks, vs, q_lens, starts, sinks.cpu(), window)
    mar, cos = _metrics(out.float().cpu().numpy(), ref.numpy())
    assert mar <= MAR and cos >= COS, f"attention: {mar:.3g} {cos:.6f}"


@pytest.mark.parametrize("window", [0, 128])
def test_attention_prefill_items_vs_oracle(window):
    """Chunked-prefill rows (q_len >= 32) on the prefill kernel, mixed with decode and verify rows on
    the split kernel, into one output; against the oracle.  The unwritten slots past each sequence
    hold NaN, which neither kernel may read into a result."""
    from flyai_amd import ops
    Hq, Hkv, D, cap = 64, 8, 64, 1600
    q_lens, starts = [300, 1, 4, 45, 33], [700, 1000, 64, 0, 1200]
    S, T = len(q_lens), sum(q_lens)
    slab = Hkv * cap * D
    kp = torch.full((S * slab,), float("nan"), device=DEV).to(torch.bfloat16)
    vp = torch.full((S * slab,), float("nan"), device=DEV).to(torch.bfloat16)
    for b, (ql, st) in enumerate(zip(q_lens, starts)):
        pos = torch.arange(st + ql, device=DEV)
        kvlayout.scatter(kp[b * slab:(b + 1) * slab], Hkv, cap, "k",
                         torch.randn(Hkv, st + ql, D, device=DEV, generator=_gen(90 + b)), pos)
        kvlayout.scatter(vp[b * slab:(b + 1) * slab], Hkv, cap, "v",
                         torch.randn(Hkv, st + ql, D, device=DEV, generator=_gen(95 + b)), pos)
    q = torch.randn(T, Hq, D, device=DEV, generator=_gen(52)).to(torch.bfloat16)
    sinks = torch.randn(Hq, device=DEV, generator=_gen(53)).to(torch.bfloat16).float()
    base = torch.tensor([b * slab for b in range(S)], dtype=torch.int64, device=DEV)
    capt = torch.tensor([cap] * S, dtype=torch.int32, device=DEV)
    items, groups, n_small, pitems = ops.attn_plan_prefill(q_lens, starts, Hkv, window, 512, 32)
    assert pitems.shape[0] == (19 + 3 + 3) * Hkv
    out = ops.attn_ragged(q, kp, vp, base, capt, sinks, window, items, groups, n_small, Hkv)
    ops.attn_prefill(q, kp, vp, base, capt, sinks, window, pitems, Hkv, out)
    torch.cuda.synchronize()
    ks = [kvlayout.gather(kp[b * slab:(b + 1) * slab], Hkv, cap, "k").float().cpu() for b in range(S)]
    vs = [kvlayout.gather(vp[b * slab:(b + 1) * slab], Hkv, cap, "v").float().cpu() for b in range(S)]
    ref = oattn.ragged_attention(q.float().cpu(), ks, vs, q_lens, starts, sinks.cpu(), window)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    mar, cos = _metrics(got, ref.numpy())
    assert mar <= MAR and cos >= COS, f"prefill attention: {mar:.3g} {cos:.6f}"
    # the prefill path against the split path on the same rows: same math, different blocking
    items0, groups0, ns0 = ops.attn_plan(q_lens, starts, Hkv, window, 512)
    out0 = ops.attn_ragged(q, kp, vp, base, capt, sinks, window, items0, groups0, ns0, Hkv)
    torch.cuda.synchronize()
    mar0, cos0 = _metrics(got, out0.float().cpu().numpy())
    assert mar0 < 1e-2 and cos0 > 0.99999


def test_attention_ignores_unwritten_nan_slots():
    """Keys/values past each sequence's length (and before its window) are never read into the
    result even when they hold NaN: the kernel masks scores and zeroes out-of-range values."""
    from flyai_amd import ops
    Hq, Hkv, D, cap = 64, 8, 64, 1024
    q_lens, starts = [1, 3], [200, 517]
    S, T = 2, 4
    slab = Hkv * cap * D
    kp = torch.full((S * slab,), float("nan"), device=DEV).to(torch.bfloat16)
    vp = torch.full((S * slab,), float("nan"), device=DEV).to(torch.bfloat16)
    for b, (ql, st) in enumerate(zip(q_lens, starts)):
        pos = torch.arange(st + ql, device=DEV)
        kvlayout.scatter(kp[b * slab:(b + 1) * slab], Hkv, cap, "k",
                         torch.randn(Hkv, st + ql, D, device=DEV, generator=_gen(60 + b)), pos)
        kvlayout.scatter(vp[b * slab:(b + 1) * slab], Hkv, cap, "v",
                         torch.randn(Hkv, st + ql, D, device=DEV, generator=_gen(70 + b)), pos)
    q = torch.randn(T, Hq, D, device=DEV, generator=_gen(80)).to(torch.bfloat16)
    sinks = torch.zeros(Hq, device=DEV)
    base = torch.tensor([0, slab], dtype=torch.int64, device=DEV)
    capt = torch.tensor([cap, cap], dtype=torch.int32, device=DEV)
    for window in (0, 128):
        items, groups, n_small = ops.attn_plan(q_lens, starts, Hkv, window, 128)
        out = ops.attn_ragged(q, kp, vp, base, capt, sinks, window, items, groups, n_small, Hkv)
        assert torch.isfinite(out.float()).all()


# ---- a10: the stage step ------------------------------------------------------------------------

def test_stage_step_per_layer_vs_oracle():
    from gpu_harness import run_stage_vs_oracle, small_stage_case
    case = small_stage_case(n_layers=2, n_experts=8, seed=1)
    outs, refs = run_stage_vs_oracle(case, per_layer=True)
    for l, (o, r) in enumerate(zip(outs, refs)):
        mar, cos = _metrics(o, r)
        assert mar <= MAR and cos >= COS, f"layer {l}: max-abs-rel {mar:.3g} cos {cos:.6f}"


def test_stage_step_hidden_3584_per_layer_vs_oracle():
    """Hidden 3584 (> 3072): the router-logits finalizer's wide variant, which keeps one split-K
    slice in registers and adds the other 7 of the 4096-wide o-proj in its tail loop."""
    from gpu_harness import oracle_layer_params, oracle_kv, fill_kv_random, metrics
    from flyai_amd.rope import YarnRotary
    from flyai_amd.runtime import KVWorkspace, RaggedStage
    from flyai_amd.weights import GptOssShape, synthetic_layer
    shape = GptOssShape(hidden=3584, n_experts=8)
    lw = synthetic_layer(shape, 77, DEV, sliding=False, keep_hf=True)
    rot = YarnRotary(2048, device=DEV)
    q_lens, starts = [1, 4, 1], [300, 17, 1500]
    kv = KVWorkspace(1, 3, 2048, shape.n_kv_heads, shape.head_dim, DEV)
    fill_kv_random(kv, 78)
    T = sum(q_lens)
    h = torch.randn(T, shape.hidden, device=DEV, generator=_gen(79)).to(torch.bfloat16)
    okv = oracle_kv(kv, 0, [0, 1, 2])
    st = RaggedStage(shape, [lw], rot, kv, max_tokens=64, max_seqs=3)
    out = st.forward(h.clone(), q_lens, starts, [0, 1, 2])
    torch.cuda.synchronize()
    cos, sin = olayer.rope_table(2048)
    ref = olayer.decoder_layer(h.float().cpu(), oracle_layer_params(lw, False), okv, q_lens, starts, cos, sin)
    mar, cs = metrics(out.float().cpu().numpy(), ref.numpy())
    assert mar <= MAR and cs >= COS, f"hidden 3584 layer: {mar:.3g} {cs:.6f}"


def test_c0_moe_block_vs_oracle():
    """Workload C0: one GPT-OSS MoE block (H=I=2880, 128 experts, top-4) on 4 sequences of lengths
    {1,1,3,7}, E2M1 codes uniform, E8M0 scales 2^-8..2^-4, bf16 N(0,1) activations RMSNorm'd."""
    from flyai_amd import ops
    from flyai_amd.weights import GptOssShape, synthetic_moe
    shape = GptOssShape()
    m = synthetic_moe(shape, _gen(0), DEV)
    w13 = ops.mxfp4_repack(m["w13_blocks"], m["w13_scales"])
    w2 = ops.mxfp4_repack(m["w2_blocks"], m["w2_scales"])
    T = 12
    x = torch.randn(T, shape.hidden, device=DEV, generator=_gen(1)).to(torch.bfloat16)
    lnw = torch.ones(shape.hidden, device=DEV)
    rw = (torch.randn(128, shape.hidden, device=DEV, generator=_gen(2)) * 0.02).to(torch.bfloat16)
    rb = (torch.randn(128, device=DEV, generator=_gen(3)) * 0.02).to(torch.bfloat16)
    xn = ops.rmsnorm(x, lnw)
    ids, wts = ops.router_topk_softmax(xn, rw, rb, 4)
    hist, off, perm, inv = ops.moe_permute(ids, 128)
    h = ops.moe_gate_up(xn, perm, off, 4, w13, m["b13"], 128, shape.intermediate)
    y = ops.moe_down(h, off, w2, m["b2"], 128, shape.hidden)
    out = ops.moe_combine(y, inv, wts, residual=x.clone())
    torch.cuda.synchronize()
    xn_ref = olayer.rmsnorm(x.float().cpu(), lnw.cpu())
    rids, rwts, _ = oroute.gptoss_route(xn.float().cpu(), rw.float().cpu(), rb.float().cpu(), 4)
    assert np.array_equal(ids.cpu().numpy(), rids)
    _, roff, rperm, rinv = oroute.permute(rids, 128)
    assert np.array_equal(perm.cpu().numpy(), rperm)
    wo = oexperts.MxExpertWeights(*(m[n].cpu().numpy() for n in
                                    ("w13_blocks", "w13_scales", "b13", "w2_blocks", "w2_scales", "b2")))
    ry = oexperts.experts_mxfp4(xn.float().cpu(), rperm, roff, 4, wo)
    ref = oroute.combine(ry, rinv, rwts, residual=x.float().cpu())
    mar, cos = _metrics(out.float().cpu().numpy(), ref.numpy())
    assert mar <= MAR and cos >= COS, f"C0 MoE block: {mar:.3g} {cos:.6f}"
    mar, cos = _metrics(xn.float().cpu().numpy(), xn_ref.numpy())
    assert mar < 1e-2 and cos > 0.9999


def test_stage_step_with_prefill_chunk_per_layer_vs_oracle():
    """A chunked-prefill row (q_len 96, prefill attention items) packed with decode and verify rows,
    layer by layer from the GPU's own input: the attention output within a tight bar, and the layer
    output on every token routed alike (a token may route differently only on a near-tie of the
    oracle's logits, which the bf16 rounding of its input can flip)."""
    import gpu_harness as gh
    from flyai_amd.runtime import RaggedStage
    q_lens, starts = [96, 1, 4, 1], [300, 40, 1000, 0]
    case = gh.small_stage_case(n_layers=2, n_experts=32, seed=4, q_lens=q_lens, starts=starts)
    shape, kv, T = case["shape"], case["kv"], case["T"]
    cos, sin = olayer.rope_table(case["maxlen"])
    h = case["hidden"].clone()
    for l, lw in enumerate(case["layers"]):
        okv = gh.oracle_kv(kv, l, case["slots"])
        st = RaggedStage(shape, [lw], case["rot"], gh._SingleLayerKV(kv, l), max_tokens=128, max_seqs=4)
        hin = gh.cpu_f32(h)
        h = st.forward(h.clone(), q_lens, starts, case["slots"])
        torch.cuda.synchronize()
        tr = {}
        ids = st.debug_buffer(4, torch.int32, (T, shape.top_k)).cpu().numpy()
        ref = olayer.decoder_layer(hin, gh.oracle_layer_params(lw, lw.sliding), okv, q_lens, starts, cos, sin,
                                   trace=tr, force_ids=ids)
        attn = gh.cpu_f32(st.debug_buffer(3, torch.bfloat16, (T, shape.n_q_heads * shape.head_dim))).numpy()
        mar_a, cos_a = _metrics(attn, tr["attn"].reshape(T, -1).numpy())
        assert mar_a <= 1e-2 and cos_a >= 0.9999, (l, mar_a, cos_a)
        gh.tokens_with_same_routing(ids, tr["ids"], tr["logits"], shape.top_k)
        mar, cos_ = _metrics(gh.cpu_f32(h).numpy(), ref.numpy())
        assert mar <= MAR and cos_ >= COS, f"layer {l}: max-abs-rel {mar:.3g} cos {cos_:.6f}"
        del st


def test_batched_equals_solo_bit_exact():
    """Size-independent property on a C1-shaped batch: a stream's output inside a ragged batch equals
    running that stream alone (per-row fixed reduction orders everywhere), bit for bit."""
    from gpu_harness import small_stage_case
    from flyai_amd.runtime import KVWorkspace, RaggedStage
    q_lens = [1] * 6 + [4] * 2
    starts = [600, 513, 4000, 800, 1, 2500, 1500, 7000]
    case = small_stage_case(n_layers=2, n_experts=16, seed=3, q_lens=q_lens, starts=starts, maxlen=8192)
    kv0 = [(k.clone(), v.clone()) for k, v in zip(case["kv"].k, case["kv"].v)]
    st = RaggedStage(case["shape"], case["layers"], case["rot"], case["kv"], 64, 8)
    batched = st.forward(case["hidden"].clone(), q_lens, starts, list(range(8)))
    torch.cuda.synchronize()
    cu = np.concatenate([[0], np.cumsum(q_lens)])
    for b in (0, 6, 7):
        for l, (k, v) in enumerate(kv0):
            case["kv"].k[l].copy_(k)
            case["kv"].v[l].copy_(v)
        solo = st.forward(case["hidden"][cu[b]:cu[b + 1]].clone(), [q_lens[b]], [starts[b]], [b])
        torch.cuda.synchronize()
        assert torch.equal(solo, batched[cu[b]:cu[b + 1]]), f"stream {b} differs solo vs batched"


def test_prefill_batch_decode_rows_equal_solo_bit_exact():
    """A 300-token prefill chunk makes the batch prefill-sized: the qkv projection then runs the tiled
    GEMM with the finalize, RoPE and KV append in its epilogue, the o-projection the tiled GEMM and the
    router the unfused path.  The decode rows beside it must come out as they do alone (split-K
    projections, the separate qkv finalize kernel, the fused router finalizer), bit for bit."""
    from gpu_harness import small_stage_case
    from flyai_amd.runtime import RaggedStage
    q_lens = [300, 1, 1, 4]
    starts = [0, 700, 2100, 1500]
    case = small_stage_case(n_layers=2, n_experts=16, seed=5, q_lens=q_lens, starts=starts, maxlen=4096)
    kv0 = [(k.clone(), v.clone()) for k, v in zip(case["kv"].k, case["kv"].v)]
    st = RaggedStage(case["shape"], case["layers"], case["rot"], case["kv"], 320, 4)
    batched = st.forward(case["hidden"].clone(), q_lens, starts, list(range(4)))
    torch.cuda.synchronize()
    assert torch.isfinite(batched.float()).all()
    cu = np.concatenate([[0], np.cumsum(q_lens)])
    for b in (1, 2, 3):
        for l, (k, v) in enumerate(kv0):
            case["kv"].k[l].copy_(k)
            case["kv"].v[l].copy_(v)
        solo = st.forward(case["hidden"][cu[b]:cu[b + 1]].clone(), [q_lens[b]], [starts[b]], [b])
        torch.cuda.synchronize()
        assert torch.equal(solo, batched[cu[b]:cu[b + 1]]), f"stream {b} differs solo vs beside a prefill chunk"


def test_dense_and_row_pass_experts_bit_identical():
    """The same rows through the row-pass expert kernel (a batch below the dense cutoff of 8 rows per
    expert on average) and through the dense tiled GEMM (a batch above it) give bit-identical h and y:
    both feed the MFMA the same K-to-lane mapping, accumulate the 128-K groups in the same order from
    zero and share the epilogue arithmetic.  So a row's tokens do not depend on whether its batch
    mates push the batch across the cutoff (the reference's Triton path measured the opposite,
    docs/receipts/batched-verify-20260623.json:27-30).  Dense groups of 100 rows take a 96-row pass
    and a 32-row pass; H = I = 2880 leaves a partial last 128-K group."""
    from flyai_amd import ops
    from flyai_amd.weights import GptOssShape, synthetic_moe
    E, k = 4, 4
    shape = GptOssShape(n_experts=E)
    m = synthetic_moe(shape, _gen(31), DEV)
    w13 = ops.mxfp4_repack(m["w13_blocks"], m["w13_scales"])
    w2 = ops.mxfp4_repack(m["w2_blocks"], m["w2_scales"])
    T = 100
    x = _rms_input(T, shape.hidden, 32)
    ids = torch.arange(E, dtype=torch.int32, device=DEV).repeat(T, 1).contiguous()  # every token on every expert
    _, off_a, perm_a, _ = ops.moe_permute(ids, E)
    h_a = ops.moe_gate_up(x, perm_a, off_a, k, w13, m["b13"], E, shape.intermediate)   # 400 rows: dense
    y_a = ops.moe_down(h_a, off_a, w2, m["b2"], E, shape.hidden)
    for sel in ([0, 1, 2, 3, 4, 5, 6], [99, 17, 50], [64, 95, 96, 97]):   # 4 * len(sel) < 32: row-pass
        sel_t = torch.tensor(sel, device=DEV)
        ids_b = ids[:len(sel)].contiguous()
        _, off_b, perm_b, _ = ops.moe_permute(ids_b, E)
        xb = x[sel_t].contiguous()
        h_b = ops.moe_gate_up(xb, perm_b, off_b, k, w13, m["b13"], E, shape.intermediate)
        y_b = ops.moe_down(h_b, off_b, w2, m["b2"], E, shape.hidden)
        torch.cuda.synchronize()
        oa, ob = off_a.cpu().tolist(), off_b.cpu().tolist()
        for e in range(E):
            ra = torch.tensor([oa[e] + t for t in sel], device=DEV)   # expert e's rows are its tokens in order
            rb = torch.arange(ob[e], ob[e] + len(sel), device=DEV)
            assert torch.equal(h_a[ra], h_b[rb]), f"expert {e}, tokens {sel}: gate_up differs"
            assert torch.equal(y_a[ra], y_b[rb]), f"expert {e}, tokens {sel}: down differs"
