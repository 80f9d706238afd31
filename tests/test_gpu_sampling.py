"""flyai_sample_rows / flyai_sample_probs and the kernel-backed Sampler against the sampler oracle,
bit for bit: integer weights make the kernel's sums independent of its reduction order, so the fp32
probabilities, the drafted-token probabilities and every draw for given uniforms must be identical.
Vocabulary of GPT-OSS (201088) and small odd sizes; rows with heavy bf16 ties so that the top-k and
top-p boundaries fall inside runs of equal logits."""
import numpy as np
import pytest
import torch

from oracle import sampling as S

pytestmark = pytest.mark.gpu

DEV = "cuda"
V_GPTOSS = 201088


def _logits(R, V, seed, ties=False, scale=3.0):
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    x = torch.randn(R, V, generator=g) * scale
    if ties:
        x = torch.round(x * 2) / 2
    return x.to(torch.bfloat16)


CASES = [  # (V, temp, top_k, top_p, ties)
    (V_GPTOSS, 0.7, 0, 0.9, False),
    (V_GPTOSS, 1.0, 50, 1.0, False),
    (V_GPTOSS, 1.3, 1000, 0.95, True),
    (V_GPTOSS, 1e-3, 0, 0.9, False),
    (V_GPTOSS, 0.8, 0, 1e-6, False),
    (V_GPTOSS, 2.0, 0, 0.5, True),
    (1, 1.0, 0, 0.9, False),
    (1000, 0.9, 999, 0.99, True),
    (3001, 1.0, 0, 1.0, True),
]


@pytest.mark.parametrize("V,temp,top_k,top_p,ties", CASES)
def test_sample_rows_bit_exact(V, temp, top_k, top_p, ties):
    from flyai_amd import ops
    R = 4
    x = _logits(R, V, seed=V + top_k, ties=ties)
    xf = x.float().numpy()
    rng = np.random.default_rng(V)
    w = [S.weights(xf[r], temp, top_k, top_p) for r in range(R)]
    # drafts: the most likely token, a kept mid token, a dropped token (if any), none
    draft = []
    for r in range(R):
        kept = np.flatnonzero(w[r])
        dead = np.flatnonzero(w[r] == 0)
        choice = [int(np.argmax(w[r])), int(kept[len(kept) // 2]), int(dead[0]) if dead.size else 0, -1][r]
        draft.append(choice)
    u = rng.random(R)
    u[0] = 0.0
    xd = x.to(DEV)
    out = ops.sample_rows(xd, temp, top_k, top_p, draft=torch.tensor(draft, dtype=torch.int32, device=DEV),
                          u=torch.tensor(u, dtype=torch.float64, device=DEV),
                          want_p_draft=True, want_draw=True, want_probs=True)
    torch.cuda.synchronize()
    probs = out["probs"].cpu().numpy()
    for r in range(R):
        assert np.array_equal(probs[r], S.probs(w[r])), f"row {r}: probabilities differ"
        want_p = float(S.p_of(w[r], draft[r])) if draft[r] >= 0 else 0.0
        assert out["p_draft"][r].item() == want_p, f"row {r}: p_draft"
        assert out["draw"][r].item() == S.draw(w[r], u[r], exclude=draft[r]), f"row {r}: draw"


def test_sample_rows_greedy():
    from flyai_amd import ops
    x = _logits(6, V_GPTOSS, seed=3, ties=True)
    x[2, 7] = x[2].max() + 1
    x[2, 9] = x[2, 7]                       # a tie for the maximum: the first id
    xd = x.to(DEV)
    d = torch.tensor([0, 1, 7, 9, -1, 5], dtype=torch.int32, device=DEV)
    out = ops.sample_rows(xd, 0.0, draft=d, want_p_draft=True, want_draw=True, want_probs=True)
    torch.cuda.synchronize()
    want = [S.greedy(r) for r in x.float().numpy()]
    assert out["draw"].tolist() == want and want[2] == 7
    assert out["p_draft"].tolist() == [1.0 if a == b else 0.0 for a, b in zip(d.tolist(), want)]
    p = out["probs"].cpu()
    assert torch.equal(p.argmax(-1), torch.tensor(want)) and (p.sum(-1) == 1).all()


def test_sample_probs_bit_exact():
    from flyai_amd import ops
    x = _logits(1, V_GPTOSS, seed=9)[0].float().numpy()
    p = S.probs(S.weights(x, 0.9, 0, 0.97))
    pd = torch.from_numpy(p).to(DEV)
    for u in (0.0, 0.123456789, 0.5, 0.999999):
        assert ops.sample_probs(pd, u).item() == S.draw_probs(p, u)
    assert ops.sample_probs(torch.zeros(17, device=DEV), 0.4).item() == 0


@pytest.mark.parametrize("temp,top_k,top_p", [(0.8, 0, 0.95), (1.0, 20, 1.0), (0.0, 0, 1.0)])
def test_sampler_accept_matches_oracle(temp, top_k, top_p):
    """The kernel-backed Sampler and the oracle's accept, fed the same uniforms, return the same doctored
    list; drafts mix likely, unlikely and filtered-out tokens so both accept and reject paths run."""
    from flyai_amd.sampling import Sampler
    K = 4
    for trial in range(6):
        x = _logits(K + 1, V_GPTOSS, seed=100 + trial, ties=trial % 2 == 1)
        xf = x.float().numpy()
        w = [S.weights(xf[j], max(temp, 1e-6), top_k, top_p) for j in range(K)]
        draft = [int(np.argmax(w[j])) if (trial + j) % 3 else int(np.argsort(xf[j])[trial]) for j in range(K)]
        seed = 1000 + trial
        sm = Sampler(temp=temp, top_p=top_p, top_k=top_k, seed=seed, device=DEV)
        got = sm.accept(x.to(DEV), draft)
        uni = np.random.Generator(np.random.PCG64(seed))
        want = S.accept(list(xf), draft, temp, top_k, top_p, iter(lambda: float(uni.random()), None))
        assert got == want, f"trial {trial}: {got} vs {want}"


def test_sampler_api():
    from flyai_amd.sampling import Sampler
    x = _logits(1, 5000, seed=4)[0]
    sm = Sampler(temp=0.0, device=DEV)
    assert sm.greedy and sm.sample_logits(x.to(DEV)) == S.greedy(x.float().numpy())
    sm = Sampler(temp=0.9, top_p=0.9, seed=5, device=DEV)
    p = sm.dist(x.to(DEV))
    assert p.dtype == torch.float32 and p.shape == (5000,)
    assert np.array_equal(p.cpu().numpy(), S.probs(S.weights(x.float().numpy(), 0.9, 0, 0.9)))
    u = np.random.Generator(np.random.PCG64(5))
    assert sm.sample_logits(x.to(DEV)) == S.draw(S.weights(x.float().numpy(), 0.9, 0, 0.9), float(u.random()))
    assert sm.sample(p) == S.draw_probs(p.cpu().numpy(), float(u.random()))
    with pytest.raises(ValueError):
        sm.accept(_logits(2, 5000, seed=1).to(DEV), [1, 2])           # K=2 needs 3 rows
    with pytest.raises(TypeError):
        sm.dist(x.float().to(DEV))


def test_tail_tokens_over_the_lm_head():
    """tail_tokens on the stage parts (final norm + lm_head over the 201088-token vocabulary): greedy
    replies are bit-identical to the fused lm_head argmax; sampled replies (prefill, per-row, accept over
    K+1 rows) equal the oracle's for the same uniforms over the same bf16 logits."""
    from flyai_amd.sampling import Sampler, tail_tokens
    from flyai_amd.stage_parts import FinalNorm, LmHead
    H = 2880
    g = torch.Generator(device="cpu")
    g.manual_seed(21)
    parts = {"norm": FinalNorm((1 + 0.1 * torch.randn(H, generator=g)).to(DEV)),
             "lm_head": LmHead((torch.randn(V_GPTOSS, H, generator=g) * 0.03).to(torch.bfloat16).to(DEV))}
    h = (torch.randn(1, 5, H, generator=g) * 2).to(torch.bfloat16).to(DEV)
    logits = parts["lm_head"](parts["norm"](h))[0].float().cpu().numpy()
    greedy = Sampler(device=DEV)
    want = [S.greedy(r) for r in logits]
    assert tail_tokens(parts, h, greedy) == want
    assert tail_tokens(parts, h, greedy, draft=[want[0], 3, want[2], 4]) == want
    assert tail_tokens(parts, h, greedy, prefill=True) == [want[-1]]
    temp, top_k, top_p, seed = 0.9, 0, 0.95, 77
    ws = [S.weights(r, temp, top_k, top_p) for r in logits]

    def uni():
        u = np.random.Generator(np.random.PCG64(seed))
        return iter(lambda: float(u.random()), None)
    sm = lambda: Sampler(temp=temp, top_p=top_p, top_k=top_k, seed=seed, device=DEV)  # noqa: E731
    u = uni()
    assert tail_tokens(parts, h, sm(), prefill=True) == [S.draw(ws[-1], next(u))]
    u = uni()
    assert tail_tokens(parts, h, sm()) == [S.draw(w, next(u)) for w in ws]
    draft = [int(np.argmax(ws[0])), int(np.argmax(ws[1])), 5, 6]
    assert tail_tokens(parts, h, sm(), draft=draft) == S.accept(list(logits), draft, temp, top_k, top_p, uni())


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf")])
def test_sample_rows_non_finite_logits_and_out_of_range_uniforms(bad):
    """A row with a NaN or infinite logit: the kernel's weights and draw equal the oracle's (every weight
    0 for NaN/+inf, so the draw is id 0, inside the vocabulary); uniforms outside [0, 1) are held to its
    ends, so they draw what 0 and the largest double below 1 draw."""
    from flyai_amd import ops
    V = 3001
    x = _logits(4, V, seed=5)
    x[0, 17] = bad
    x[1, 0] = bad
    x[1, V - 1] = bad
    xf = x.float().numpy()
    u = np.array([0.3, 0.6, -0.25, 1.5])
    u_eff = np.array([0.3, 0.6, 0.0, np.nextafter(1.0, 0.0)])
    out = ops.sample_rows(x.to(DEV), 0.9, 0, 1.0, draft=torch.tensor([17, -1, 5, 9], dtype=torch.int32, device=DEV),
                          u=torch.tensor(u, dtype=torch.float64, device=DEV), want_draw=True, want_probs=True)
    draw = out["draw"].cpu().numpy()
    probs = out["probs"].cpu().numpy()
    for r, d in enumerate([17, -1, 5, 9]):
        w = S.weights(xf[r], 0.9)
        want = S.draw(w, float(u_eff[r]), exclude=d)
        assert 0 <= draw[r] < V and draw[r] == want, (r, draw[r], want)
        if w.sum(dtype=np.uint64) > 0:
            assert np.array_equal(probs[r], S.probs(w)), r
        else:
            assert not probs[r].any(), r
