"""Pin the oracle's remaining functions against pure-Python brute force, closed forms and the
reference's own known-answer cases (no transformers needed)."""
import math

import numpy as np
import pytest
import torch

from conftest import metrics
from oracle import attention, experts, mxfp4, packing, routing
from oracle.numerics import bf16, bf16_bits_to_f32, f32_to_bf16_bits


# ---- a1 packing -------------------------------------------------------------------------------

def test_pack_ragged_brute_force():
    rng = np.random.default_rng(0)
    q = rng.integers(1, 9, size=13)
    st = rng.integers(0, 500, size=13)
    out = packing.pack_ragged(q, st, kv_base=np.arange(13) * 10_000, head_dim=64)
    pos, sid, slot, cu = [], [], [], [0]
    for b in range(13):
        for i in range(q[b]):
            pos.append(st[b] + i); sid.append(b); slot.append(b * 10_000 + (st[b] + i) * 64)
        cu.append(cu[-1] + q[b])
    assert out["positions"].tolist() == pos and out["seq_id"].tolist() == sid
    assert out["kv_slot"].tolist() == slot and out["cu_seqlens"].tolist() == cu
    assert out["kv_len"].tolist() == (st + q).tolist()


def test_context_overflow_boundary():
    """Boundary cases of the reference's KV bound (tests/test_kv_bound.py:17-24): writes
    positions [start, start+q-1]; in bounds iff start + q <= capacity."""
    packing.pack_ragged([8], [92], kv_cap=[100])                 # max index 99: exactly fits
    packing.pack_ragged([100], [0], kv_cap=[100])
    with pytest.raises(packing.ContextOverflow):
        packing.pack_ragged([8], [93], kv_cap=[100])
    with pytest.raises(packing.ContextOverflow):
        packing.pack_ragged([1], [100], kv_cap=[100])


@pytest.mark.parametrize("starts", [[0, 0, 0, 0], [17, 5, 900, 233], [2039, 1, 64, 2039]])
def test_batched_mask_per_stream(starts):
    """The per-stream mask cases of the reference's tests/test_graph_batch.py:38-55: row (b, qi)
    allows col j iff j <= starts[b]+qi (and inside the window on sliding layers)."""
    q = [9] * 4
    for window in (0, 128):
        m = packing.batched_mask(q, starts, 2048, window)
        r = 0
        for b in range(4):
            for qi in range(9):
                p = starts[b] + qi
                for j in (0, max(0, p - 127) - 1, max(0, p - 127), p, p + 1, 2047):
                    if 0 <= j < 2048:
                        want = j <= p and (not window or p - j < window)
                        assert m[r, j] == want
                r += 1


# ---- a2/a3/a4 routing --------------------------------------------------------------------------

def _bf16_rand(rng, shape, std=1.0):
    return bf16(torch.from_numpy(rng.standard_normal(shape).astype(np.float32) * std))


def test_dot_fixed_matches_sequential_restatement():
    """Lane l sums k = 512 j + 8 l + i (k < K) in order, then the xor butterfly; K = 600 leaves
    lanes 11..63 without a second chunk."""
    rng = np.random.default_rng(1)
    K = 600
    x = _bf16_rand(rng, (2, K))
    w = _bf16_rand(rng, (3, K))
    got = routing.dot_fixed(x, w)
    for t in range(2):
        for e in range(3):
            lanes = []
            for l in range(64):
                acc = np.float32(0.0)
                for j in range(2):
                    for i in range(8):
                        k = 512 * j + 8 * l + i
                        if k < K:
                            acc = np.float32(acc + np.float32(x[t, k]) * np.float32(w[e, k]))
                lanes.append(acc)
            for off in (32, 16, 8, 4, 2, 1):
                lanes = [np.float32(lanes[i] + lanes[i ^ off]) for i in range(64)]
            assert np.float32(got[t, e]) == lanes[0]


def test_gptoss_topk_ties_to_lower_id_and_softmax():
    x = torch.zeros(3, 64)
    x[:, 0] = 1.0
    w = torch.zeros(8, 64)
    b = torch.tensor([0.5, 2.0, 2.0, -1.0, 2.0, 0.5, 3.0, 0.5])      # ties at 2.0 and at 0.5
    ids, wts, _ = routing.gptoss_route(x, w, b, k=4)
    assert ids.tolist() == [[1, 2, 4, 6]] * 3                           # 6 first, then 1,2,4 (lowest ids)
    v = np.array([2.0, 2.0, 2.0, 3.0])
    e = np.exp(v - 3.0)
    np.testing.assert_allclose(wts[0], e / e.sum(), rtol=1e-6)
    b2 = torch.tensor([0.5, 2.0, 1.0, -1.0, 2.0, 0.5, 3.0, 0.5])
    ids2, _, _ = routing.gptoss_route(x, w, b2, k=4)
    assert ids2.tolist()[0] == [1, 2, 4, 6]
    b3 = torch.tensor([0.5, 2.0, 0.0, -1.0, 2.0, 0.5, 3.0, 0.5])        # 0.5 tie among 0, 5, 7 -> 0
    assert routing.gptoss_route(x, w, b3, k=4)[0].tolist()[0] == [0, 1, 4, 6]


def test_gptoss_route_brute_force():
    rng = np.random.default_rng(2)
    x = _bf16_rand(rng, (40, 128))
    w = _bf16_rand(rng, (16, 128), 0.1)
    b = _bf16_rand(rng, (16,), 0.1)
    ids, wts, logits = routing.gptoss_route(x, w, b, k=4)
    L = logits.numpy()
    for t in range(40):
        order = sorted(range(16), key=lambda e: (-float(L[t, e]), e))[:4]
        assert ids[t].tolist() == sorted(order)
        vals = [float(L[t, e]) for e in sorted(order)]
        m = max(vals)
        ex = [math.exp(v - m) for v in vals]
        np.testing.assert_allclose(wts[t], [v / sum(ex) for v in ex], rtol=1e-6)
    # logits are the bf16 rounding of the fixed-order fp32 dot (+ bias)
    ref = x.double() @ w.double().T + b.double()
    assert torch.allclose(logits.double(), ref, rtol=1e-2, atol=1e-2)


def test_permute_brute_force_and_invariants():
    rng = np.random.default_rng(3)
    T, k, E = 37, 4, 16
    ids = np.sort(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]), axis=1)
    hist, off, perm, inv = routing.permute(ids, E)
    flat = ids.reshape(-1)
    want = [a for e in range(E) for a in range(T * k) if flat[a] == e]
    assert perm.tolist() == want
    assert hist.sum() == T * k and (np.diff(off) == hist).all() and off[0] == 0
    assert (perm[inv] == np.arange(T * k)).all() and (inv[perm] == np.arange(T * k)).all()
    for e in range(E):
        assert (flat[perm[off[e]:off[e + 1]]] == e).all()


def test_combine_fp64_brute_force():
    rng = np.random.default_rng(4)
    T, k, H = 5, 4, 32
    y = rng.standard_normal((T * k, H)).astype(np.float32)
    inv = rng.permutation(T * k).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    res = bf16(torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)))
    out = routing.combine(y, inv, w, residual=res).numpy()
    ref = np.zeros((T, H))
    for t in range(T):
        for s in range(k):
            ref[t] += float(w[t, s]) * y[inv[t * k + s]].astype(np.float64)
    ref = bf16(res + bf16(torch.from_numpy(ref.astype(np.float32)))).numpy()
    mar, cos = metrics(out, ref)
    assert mar < 1e-2 and cos > 0.9999


def test_sigmoid_det_accuracy():
    x = np.linspace(-30, 30, 20001, dtype=np.float32)
    got = routing.sigmoid_det(x).astype(np.float64)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(got - ref) / ref) < 4e-7
    e = routing.exp_det(np.linspace(-80, 80, 1001, dtype=np.float32)).astype(np.float64)
    np.testing.assert_allclose(e, np.exp(np.linspace(-80, 80, 1001, dtype=np.float32).astype(np.float64)),
                               rtol=4e-7)


def test_grouped_sigmoid_brute_force():
    rng = np.random.default_rng(5)
    T, H, E, G, TG, K = 12, 64, 32, 8, 4, 8
    x = _bf16_rand(rng, (T, H))
    w = _bf16_rand(rng, (E, H), 0.2)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    ids, wts, scores = routing.grouped_sigmoid_route(x, w, bias, G, TG, K, 2.5)
    logits = routing.dot_fixed(x, w).numpy()
    for t in range(T):
        s = [float(routing.sigmoid_det(np.float32(logits[t, e]))) for e in range(E)]
        c = [np.float32(np.float32(s[e]) + bias[e]) for e in range(E)]
        gs = []
        for g in range(G):
            grp = sorted(c[g * 4:(g + 1) * 4], reverse=True)
            gs.append(np.float32(grp[0] + grp[1]))
        keep = sorted(range(G), key=lambda g: (-gs[g], g))[:TG]
        cand = [e for e in range(E) if e // 4 in keep]
        sel = sorted(sorted(cand, key=lambda e: (-c[e], e))[:K])
        assert ids[t].tolist() == sel
        ws = np.array([s[e] for e in sel])
        np.testing.assert_allclose(wts[t], ws / (ws.sum() + 1e-20) * 2.5, rtol=1e-6)


# ---- a5/a6 experts -----------------------------------------------------------------------------

def test_swiglu_closed_form_boundaries():
    g = torch.tensor([-10.0, 0.0, 7.0, 9.0, 2.0])
    u = torch.tensor([-9.0, 3.0, -7.0, 8.0, -1.0])
    out = experts.swiglu(g, u)
    sig = lambda v: 1.0 / (1.0 + math.exp(-1.702 * v))
    ref = [(-7 + 1) * (-10) * sig(-10), 0.0, (-7 + 1) * 7 * sig(7), (7 + 1) * 7 * sig(7), 0.0]
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-6, atol=1e-7)


def test_experts_mxfp4_fp64_brute_force():
    rng = np.random.default_rng(6)
    E, H, I, T, k = 3, 64, 64, 4, 2
    mk = lambda n, kk: (rng.integers(0, 256, (E, n, kk // 32, 16), dtype=np.uint8),
                        rng.integers(119, 124, (E, n, kk // 32), dtype=np.uint8))
    b13, s13 = mk(2 * I, H)
    b2, s2 = mk(H, I)
    bias13 = rng.standard_normal((E, 2 * I)).astype(np.float32) * 0.1
    bias2 = rng.standard_normal((E, H)).astype(np.float32) * 0.1
    wts = experts.MxExpertWeights(b13, s13, bias13, b2, s2, bias2)
    x = _bf16_rand(rng, (T, H))
    ids = np.array([[0, 2], [1, 2], [0, 1], [2, 0]])
    ids.sort(axis=1)
    _, off, perm, inv = routing.permute(ids, E)
    y = experts.experts_mxfp4(x, perm, off, k, wts).numpy()
    for p in range(T * k):
        t, e = perm[p] // k, ids.reshape(-1)[perm[p]]
        W13 = mxfp4.dequant(b13[e], s13[e]).astype(np.float64)
        W2 = mxfp4.dequant(b2[e], s2[e]).astype(np.float64)
        gu = W13 @ x[t].double().numpy() + bias13[e]
        gte, up = np.minimum(gu[0::2], 7.0), np.clip(gu[1::2], -7.0, 7.0)
        h = (up + 1) * gte / (1 + np.exp(-1.702 * gte))
        h = bf16(torch.from_numpy(h.astype(np.float32))).double().numpy()
        ref = W2 @ h + bias2[e]
        mar, cos = metrics(y[p], ref)
        assert mar < 1e-5 and cos > 0.999999


# ---- a7 fp8 ------------------------------------------------------------------------------------

def test_round_scale_pow2_exact_at_powers_of_two():
    """v4_kernels_cpu.py:34-39: scale = 2**ceil(log2(amax/448)), exact when amax = 448 * 2**k."""
    for kk in range(-10, 10):
        amax = np.float32(448.0 * 2.0 ** kk)
        assert experts.round_scale_pow2(np.array([amax]), 1.0 / 448.0)[0] == np.float32(2.0 ** kk)
        just_over = np.nextafter(amax, np.float32(np.inf))
        assert experts.round_scale_pow2(np.array([just_over]), 1.0 / 448.0)[0] == np.float32(2.0 ** (kk + 1))


def test_fp8_block_gemm_fp64():
    rng = np.random.default_rng(7)
    x = bf16(torch.from_numpy(rng.standard_normal((3, 256)).astype(np.float32))).numpy()
    wq, ws = experts.fp8_block_quant_weight(rng.standard_normal((256, 256)).astype(np.float32) * 0.05)
    aq, sa = experts.act_quant_128(x)
    out = experts.fp8_block_gemm(aq, sa, wq, ws)
    deq_a = aq * np.repeat(sa, 128, axis=1)
    deq_w = wq * np.repeat(np.repeat(ws, 128, axis=0), 128, axis=1)
    np.testing.assert_allclose(out, deq_a.astype(np.float64) @ deq_w.astype(np.float64).T, rtol=1e-9, atol=1e-9)
    assert np.abs(aq).max() <= 448.0
    mar, cos = metrics(out, x.astype(np.float64) @ deq_w.astype(np.float64).T)
    assert cos > 0.999


# ---- a8 attention ------------------------------------------------------------------------------

@pytest.mark.parametrize("window", [0, 4])
def test_ragged_attention_brute_force(window):
    rng = np.random.default_rng(8)
    Hq, Hkv, D = 4, 2, 8
    q_lens, starts = [1, 3, 2], [5, 0, 9]
    T = sum(q_lens)
    q = bf16(torch.from_numpy(rng.standard_normal((T, Hq, D)).astype(np.float32)))
    ks = [torch.from_numpy(rng.standard_normal((Hkv, 16, D)).astype(np.float32)) for _ in q_lens]
    vs = [torch.from_numpy(rng.standard_normal((Hkv, 16, D)).astype(np.float32)) for _ in q_lens]
    sinks = rng.standard_normal(Hq).astype(np.float32)
    got = attention.ragged_attention(q, ks, vs, q_lens, starts, sinks, window).numpy()
    ref = attention.brute_force_attention(q.numpy(), ks, vs, q_lens, starts, sinks, window)
    mar, cos = metrics(got, ref)
    assert mar < 1e-2 and cos > 0.99999


def test_bf16_bit_helpers_roundtrip():
    x = np.array([1.0, -2.5, 3.14159, 1e-20, 65504.0], dtype=np.float32)
    bits = f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (bits == ref).all()
    assert (bf16_bits_to_f32(bits) == torch.from_numpy(x).to(torch.bfloat16).float().numpy()).all()


# ---- a7 composition: the DeepSeek expert and MoE block ----------------------------------------

def _fp8_experts(rng, n, H, I):
    """n experts with synthetic 128x128-block e4m3 weights (std 0.05) and their dequantised fp64
    matrices."""
    qs, deq = {"w1": [], "s1": [], "w3": [], "s3": [], "w2": [], "s2": []}, {"w1": [], "w3": [], "w2": []}
    for _ in range(n):
        for name, shape in (("w1", (I, H)), ("w3", (I, H)), ("w2", (H, I))):
            q, s = experts.fp8_block_quant_weight(rng.standard_normal(shape).astype(np.float32) * 0.05)
            qs[name].append(q)
            qs["s" + name[1]].append(s)
            deq[name].append(q.astype(np.float64) * np.repeat(np.repeat(s, 128, 0), 128, 1))
    w = experts.Fp8ExpertWeights(*(np.stack(qs[k]) for k in ("w1", "s1", "w3", "s3", "w2", "s2")))
    return w, {k: np.stack(v) for k, v in deq.items()}


def _silu(v):
    return v / (1.0 + np.exp(-v))


def _textbook_expert(x, d, e, weight=None):
    """Unquantised fp64 SwiGLU expert on the dequantised weights: w2 . (weight * silu(w1 x) * w3 x)."""
    h = _silu(x @ d["w1"][e].T) * (x @ d["w3"][e].T)
    if weight is not None:
        h = np.asarray(weight, np.float64)[:, None] * h
    return h @ d["w2"][e].T


def test_deepseek_expert_matches_textbook_swiglu_within_fp8_error():
    """model.py:601-611 against an unquantised fp64 SwiGLU: the only differences are the e4m3
    activation quantisation and bf16 roundings (a few percent per element, averaged down by the
    dot products).  Swapping gate and up, dropping the routing weight or the silu fails it."""
    rng = np.random.default_rng(21)
    H, I = 256, 256
    w, d = _fp8_experts(rng, 1, H, I)
    x = bf16(torch.from_numpy(rng.standard_normal((6, H)).astype(np.float32))).numpy()
    wt = np.array([0.9, 0.5, 0.25, 1.0, 0.1, 0.7], np.float32)
    got = w.expert(0, x, wt).numpy()
    ref = _textbook_expert(x.astype(np.float64), d, 0, wt)
    mar, cos = metrics(got, ref)
    assert mar < 6e-2 and cos > 0.997
    # planted mistakes in the reference side of the comparison must not pass the same bar
    swapped = (_silu(x @ d["w3"][0].T) * (x @ d["w1"][0].T) * wt[:, None]) @ d["w2"][0].T
    no_weight = _textbook_expert(x.astype(np.float64), d, 0)
    no_silu = (((x @ d["w1"][0].T) * (x @ d["w3"][0].T)) * wt[:, None]) @ d["w2"][0].T
    for bad in (swapped, no_weight, no_silu):
        mar_b, cos_b = metrics(got, bad)
        assert not (mar_b < 6e-2 and cos_b > 0.997)


def test_deepseek_moe_equals_token_major_restatement():
    """MoE.forward (model.py:634-650) sums per expert in ascending id with torch.where rows; the same
    block restated token by token (each token's k selected experts, then the shared expert) must give
    the same fp32 sum to rounding of the summation order, and the unquantised textbook block must
    agree within the fp8 error.  Catches a wrong slot/weight pairing, a dropped shared expert or a
    scatter to the wrong token."""
    rng = np.random.default_rng(22)
    H, I, E, k, T = 128, 128, 6, 2, 5
    routed, d = _fp8_experts(rng, E, H, I)
    shared, ds = _fp8_experts(rng, 1, H, I)
    x = bf16(torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32))).numpy()
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)])
    wts = rng.uniform(0.1, 1.0, size=(T, k)).astype(np.float32)
    got = experts.deepseek_moe(x, ids, wts, routed, shared).float().numpy()

    ref = np.zeros((T, H), np.float32)
    text = np.zeros((T, H), np.float64)
    for t in range(T):
        acc = np.zeros(H, np.float32)
        for s in range(k):
            acc += routed.expert(int(ids[t, s]), x[t:t + 1], wts[t, s:s + 1]).numpy()[0]
            text[t] += _textbook_expert(x[t:t + 1].astype(np.float64), d, int(ids[t, s]), wts[t, s:s + 1])[0]
        acc += shared.expert(0, x[t:t + 1]).numpy()[0]
        text[t] += _textbook_expert(x[t:t + 1].astype(np.float64), ds, 0)[0]
        ref[t] = acc
    mar, cos = metrics(got, bf16(torch.from_numpy(ref)).numpy())
    assert mar < 1e-2 and cos > 0.99999
    mar_t, cos_t = metrics(got, text)
    assert mar_t < 6e-2 and cos_t > 0.997
    # a dropped shared expert or routing weights paired with the wrong slot fail the token-major bar
    no_shared = experts.deepseek_moe(x, ids, wts, routed, experts.Fp8ExpertWeights(
        *(np.zeros_like(a) for a in (shared.w1, shared.s1, shared.w3, shared.s3, shared.w2, shared.s2))))
    swapped = experts.deepseek_moe(x, ids, wts[:, ::-1].copy(), routed, shared)
    for bad in (no_shared, swapped):
        mar_b, cos_b = metrics(bad.float().numpy(), ref)
        assert not (mar_b < 1e-2 and cos_b > 0.99999)


# ---- a10 tree verify ---------------------------------------------------------------------------

TREE_PAR = [-1, 0, 1, 2, 0, 4, 1, 6]        # tree.py's example plus a second branch off node 1
TREE_DEP = [0, 1, 2, 3, 1, 2, 2, 3]


def _tree_case(rng, M, start, Hq=4, Hkv=2, D=8):
    q = bf16(torch.from_numpy(rng.standard_normal((M, Hq, D)).astype(np.float32)))
    K = torch.from_numpy(rng.standard_normal((Hkv, start + M + 3, D)).astype(np.float32))
    V = torch.from_numpy(rng.standard_normal((Hkv, start + M + 3, D)).astype(np.float32))
    sinks = rng.standard_normal(Hq).astype(np.float32)
    return q, K, V, sinks


@pytest.mark.parametrize("window", [0, 3, 6])
def test_tree_attention_brute_force(window):
    """FastVerify tree masks (fastverify.py:250-272, tree.py:26-46) against fp64 loops over the
    reference's dense additive mask."""
    rng = np.random.default_rng(9)
    start = 7
    q, K, V, sinks = _tree_case(rng, len(TREE_PAR), start)
    got = attention.tree_attention(q, K, V, start, TREE_PAR, TREE_DEP, sinks, window).numpy()
    ref = attention.brute_force_tree_attention(q.numpy(), K.numpy(), V.numpy(), start, TREE_PAR, TREE_DEP,
                                               sinks, window)
    mar, cos = metrics(got, ref)
    assert mar < 1e-2 and cos > 0.99999


@pytest.mark.parametrize("window", [0, 4])
def test_chain_tree_equals_causal_verify(window):
    """A chain (par[i] = i-1, dep[i] = i) is an ordinary verify row: tree attention must equal
    causal ragged attention of q_len M at the same start; a branching tree must not."""
    rng = np.random.default_rng(10)
    M, start = 6, 11
    q, K, V, sinks = _tree_case(rng, M, start)
    chain_par, chain_dep = list(range(-1, M - 1)), list(range(M))
    got = attention.tree_attention(q, K, V, start, chain_par, chain_dep, sinks, window).numpy()
    ref = attention.ragged_attention(q, [K], [V], [M], [start], sinks, window).numpy()
    mar, cos = metrics(got, ref)
    assert mar < 1e-6 and cos > 0.9999999
    q8, K8, V8, s8 = _tree_case(rng, len(TREE_PAR), start)
    tree = attention.tree_attention(q8, K8, V8, start, TREE_PAR, TREE_DEP, s8, window).numpy()
    causal = attention.ragged_attention(q8, [K8], [V8], [len(TREE_PAR)], [start], s8, window).numpy()
    assert metrics(tree, causal)[0] > 1e-2      # siblings must stay invisible


def test_tree_attention_planted_sibling_leak_fails():
    """Planting the classic mistake (a node also sees a sibling's slot) in the brute force must
    break agreement: the check is sensitive to the ancestor mask."""
    rng = np.random.default_rng(11)
    start = 5
    q, K, V, sinks = _tree_case(rng, len(TREE_PAR), start)
    got = attention.tree_attention(q, K, V, start, TREE_PAR, TREE_DEP, sinks, 0).numpy()
    leaky = list(TREE_PAR)
    leaky[4] = 3            # node 4 re-parented under node 3: now sees nodes 1..3 of the other branch
    ref = attention.brute_force_tree_attention(q.numpy(), K.numpy(), V.numpy(), start, leaky,
                                               [0, 1, 2, 3, 4, 5, 2, 3], sinks, 0)
    assert metrics(got, ref)[0] > 1e-2


# ---- tail: lm_head + greedy pick ----------------------------------------------------------------

def test_greedy_pick_is_first_max():
    """torch.argmax semantics (the reference's greedy pick): the first index of the maximum."""
    from oracle import tail
    rng = np.random.default_rng(30)
    lg = bf16(torch.from_numpy(rng.integers(-3, 4, size=(40, 17)).astype(np.float32))).numpy()
    got = tail.greedy_pick(lg)
    for r in range(lg.shape[0]):
        best = 0
        for v in range(1, lg.shape[1]):
            if lg[r, v] > lg[r, best]:
                best = v
        assert got[r] == best
    assert (got == torch.from_numpy(lg).argmax(-1).numpy()).all()


def test_lm_head_logits_exact_on_small_integers():
    """Integer weights and unit-RMS integer rows: the logits are exact integers (no rounding), so
    the tail's composition (norm weight applied, weight not transposed) is fixed by the closed form."""
    from oracle import tail
    rng = np.random.default_rng(31)
    H, V = 32, 48
    h = np.where(rng.random((3, H)) < 0.5, -1.0, 1.0).astype(np.float32)       # RMS exactly 1
    norm_w = rng.integers(1, 3, size=H).astype(np.float32)
    lm_w = rng.integers(-2, 3, size=(V, H)).astype(np.float32)
    got = tail.lm_head_logits(torch.from_numpy(h), torch.from_numpy(norm_w), torch.from_numpy(lm_w), eps=0.0)
    want = (h * norm_w) @ lm_w.T
    assert np.array_equal(got.numpy(), want)
    assert not np.array_equal(got.numpy(), (h * norm_w) @ lm_w[::-1].T)


# ---- fp8 activation operands of the dense MXFP4 groups (per-32 E8M0 scales) -----------------------

def _e4m3_grid():
    """Every finite e4m3fn value with its code (sign, 4 exponent bits, 3 mantissa bits; bias 7;
    exponent 0 subnormal; code 0x7f/0xff NaN), enumerated from the format's definition."""
    vals = []
    for code in range(256):
        s, e, m = code >> 7, (code >> 3) & 15, code & 7
        if e == 15 and m == 7:
            continue
        mag = (m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
        vals.append(((-1) ** s * mag, code))
    return vals


def _e4m3_rne_brute(v, grid):
    """Nearest grid value; a tie goes to the code with an even mantissa."""
    best = min(abs(v - g) for g, _ in grid)
    cands = [(g, c) for g, c in grid if abs(v - g) == best]
    even = [g for g, c in cands if (c & 1) == 0]
    return (even or [cands[0][0]])[0]


def test_act_quant_blocks_brute_force():
    import math
    rng = np.random.default_rng(41)
    x = rng.standard_normal((3, 96)).astype(np.float32) * np.array([1.0, 300.0, 1e-3], dtype=np.float32)[:, None]
    x[1, 32:64] = 0.0                                     # an all-zero block: amax floor 1e-4
    q, s = experts.act_quant_blocks(x, 32)
    grid = _e4m3_grid()
    for r in range(3):
        for b in range(3):
            blk = x[r, 32 * b:32 * (b + 1)].astype(np.float64)
            amax = max(float(np.float32(np.abs(blk).max())), 1e-4)
            a = float(np.float32(np.float32(amax) * np.float32(1.0 / 448.0)))
            want_s = 2.0 ** math.ceil(math.log2(a))
            assert s[r, b] == want_s, (r, b)
            for i in range(32):
                y = float(np.float32(np.float32(blk[i]) / np.float32(want_s)))
                y = min(max(y, -448.0), 448.0)
                assert q[r, 32 * b + i] == _e4m3_rne_brute(y, grid), (r, b, i)
    assert np.abs(q).max() <= 448.0


def test_mx_fp8_roundtrip_is_identity_on_the_grid_with_unit_scales():
    grid = np.array(sorted({g for g, _ in _e4m3_grid()}), dtype=np.float32)
    rng = np.random.default_rng(42)
    x = rng.choice(grid, size=(4, 64)).astype(np.float32)
    x[:, ::32] = 448.0 * np.where(rng.random((4, 2)) < 0.5, -1, 1)   # amax 448 in every block: s = 1
    assert np.array_equal(experts.mx_fp8_roundtrip(x), x)
    y = x * np.float32(2.0 ** -5)                                   # s = 2^-5, still exact
    assert np.array_equal(experts.mx_fp8_roundtrip(y), y)


def test_two_term_quantiser_brute_force_and_error_bound():
    """The low term is act_quant_blocks of the residual, computed exactly (fp64 agrees with the fp32
    difference).  Bounds from the format: a block's largest magnitude maps into (224, 448], where e4m3
    steps are at most 32, so one term's rounding error is at most 2^-3 of the block's largest value;
    the low term rounds a residual of at most 2^-3 of it, so the two terms leave at most 2^-6.  The high
    term alone exceeds 2^-6 on these inputs (a dropped low term fails the two-term bound)."""
    rng = np.random.default_rng(44)
    x = rng.standard_normal((6, 128)).astype(np.float32)
    x *= np.array([1.0, 300.0, 1e-3, 7.0, 0.05, 2.0], dtype=np.float32)[:, None]
    x = torch.from_numpy(x).to(torch.bfloat16).float().numpy()     # bf16 inputs, as the kernels see
    x[2, 32:64] = 0.0
    q1, s1, q2, s2 = experts.mx_act_quant_two_term(x)
    rq1, rs1 = experts.act_quant_blocks(x, 32)
    assert np.array_equal(q1, rq1) and np.array_equal(s1, rs1)
    x1 = (q1.reshape(6, 4, 32).astype(np.float64) * s1[:, :, None]).reshape(6, 128)
    r64 = x.astype(np.float64) - x1
    assert np.array_equal(r64.astype(np.float32).astype(np.float64), r64), "residual not exact in fp32"
    rq2, rs2 = experts.act_quant_blocks(r64.astype(np.float32), 32)
    assert np.array_equal(q2, rq2) and np.array_equal(s2, rs2)
    xhat = experts.mx_fp8_roundtrip(x).astype(np.float64)
    blk_max = np.abs(x).reshape(6, 4, 32).max(axis=2, keepdims=True).repeat(32, axis=2).reshape(6, 128)
    err2 = np.abs(xhat - x)
    assert (err2 <= blk_max * 2.0 ** -6 + 1e-30).all()
    err1 = np.abs(x1 - x)
    assert (err1 > blk_max * 2.0 ** -6).any(), "the high term alone must not meet the two-term bound"
    assert (err1 <= blk_max * 2.0 ** -3 + 1e-30).all()


def test_experts_fp8act_gate_up_exact_on_grid_inputs_and_down_recomputed():
    """gate_up: inputs already on the fp8 grid with unit scales give exactly experts_mxfp4's h.
    down: y is recomputed in fp64 from that h carried by mx_fp8_roundtrip and the down weights
    dequantised directly -- a bias on the wrong side fails."""
    E, H, I, k, T = 3, 64, 64, 2, 5
    rng = np.random.default_rng(43)
    grid = np.array(sorted({g for g, _ in _e4m3_grid()}), dtype=np.float32)
    x = rng.choice(grid[np.abs(grid) <= 8], size=(T, H)).astype(np.float32)
    x[:, ::32] = 448.0
    w = experts.MxExpertWeights(rng.integers(0, 256, (E, 2 * I, H // 32, 16), dtype=np.uint8),
                                rng.integers(118, 122, (E, 2 * I, H // 32), dtype=np.uint8),
                                rng.standard_normal((E, 2 * I)).astype(np.float32),
                                rng.integers(0, 256, (E, H, I // 32, 16), dtype=np.uint8),
                                rng.integers(118, 122, (E, H, I // 32), dtype=np.uint8),
                                rng.standard_normal((E, H)).astype(np.float32))
    ids = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    ids.sort(axis=1)
    _, offsets, perm, _ = routing.permute(ids, E)
    y8, h8 = experts.experts_mxfp4_fp8act(torch.from_numpy(x), perm, offsets, k, w, return_h=True)
    y16, h16 = experts.experts_mxfp4(torch.from_numpy(x), perm, offsets, k, w, return_h=True)
    assert torch.equal(h8, h16)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi == lo:
            continue
        w2 = mxfp4.dequant(w.w2_blocks[e], w.w2_scales[e]).astype(np.float64)
        hq = experts.mx_fp8_roundtrip(h16[lo:hi].numpy()).astype(np.float64)
        want = hq @ w2.T + w.b2[e][None, :].astype(np.float64)
        np.testing.assert_allclose(y8[lo:hi].numpy(), want, rtol=1e-5, atol=1e-4)


def test_forced_route_pinned():
    """routing.forced_route (teacher forcing for the GPU parity tests): forcing the router's own
    selection changes nothing, bit for bit (ties included); forcing another expert set gives exactly
    the sorted set and the fp64 softmax over its logits, and leaves every other row's bits alone.
    Weights taken over the router's own experts (the mistake forcing exists to avoid) must fail."""
    import torch
    from oracle import routing
    g = torch.Generator().manual_seed(21)
    T, E, H, k = 40, 32, 256, 4
    x = torch.randn(T, H, generator=g).bfloat16().float()
    w = (0.05 * torch.randn(E, H, generator=g)).bfloat16().float()
    b = torch.zeros(E).bfloat16().float()
    ids, wts, logits = routing.gptoss_route(x, w, b, k)
    lg = logits.numpy()
    lg[3, :] = lg[3, 0]                                   # a row of exact ties: lower ids first
    ids3, wts3 = routing._selection_weights(lg, routing._topk_desc(lg, k))
    i2, w2, rows = routing.forced_route(lg, ids3, wts3, ids3)
    assert len(rows) == 0 and np.array_equal(i2, ids3) and np.array_equal(w2.view(np.uint32), wts3.view(np.uint32))
    rng = np.random.default_rng(5)
    force = ids3.copy()
    picked = [1, 3, 17, 39]
    for t in picked:
        force[t] = rng.choice(E, size=k, replace=False)   # any order; forced_route sorts
    i2, w2, rows = routing.forced_route(lg, ids3, wts3, force)
    changed = [t for t in picked if set(force[t]) != set(ids3[t])]
    assert sorted(rows.tolist()) == sorted(changed)
    keep = np.setdiff1d(np.arange(T), rows)
    assert np.array_equal(i2[keep], ids3[keep]) and np.array_equal(w2[keep].view(np.uint32), wts3[keep].view(np.uint32))
    caught = 0
    for t in rows:
        s = np.sort(force[t])
        assert np.array_equal(i2[t], s)
        v = lg[t, s].astype(np.float64)
        ref = np.exp(v - v.max()) / np.exp(v - v.max()).sum()
        assert np.allclose(w2[t], ref, rtol=2e-6, atol=0), (t, w2[t], ref)
        own = lg[t, ids3[t]].astype(np.float64)
        wrong = np.exp(own - own.max()) / np.exp(own - own.max()).sum()
        caught += not np.allclose(wrong, ref, rtol=2e-6, atol=0)
    assert caught >= len(rows) - 1, "weights over the router's own experts must fail (all but the all-tie row)"
