"""The served model's head and tail on the GPU, and the continuous-batch backend end to end:
lm_head + greedy pick against the oracle, the embedding gather, and a ring-style worker loop whose
tokens must not depend on batch mates and must follow the oracle's greedy choice."""
import numpy as np
import pytest
import torch

from tests import gpu_harness as gh
from tests.test_serving_host import Job, run_worker
from flyai_amd import ops
from flyai_amd.rope import YarnRotary
from flyai_amd.serving import GptOssBatchBackend, GptOssModel
from flyai_amd.weights import GptOssShape, synthetic_layer
from oracle import layer as olayer
from oracle import tail as otail

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _gen(seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    return g


def _bf16_ulp(x):
    return 2.0 ** (np.floor(np.log2(np.maximum(np.abs(x), 1e-30))) - 7)


@pytest.mark.parametrize("V,R,n_rows", [(4096, 80, 64), (4096, 5, 1), (201088, 40, 17)])
def test_lm_head_argmax_vs_oracle(V, R, n_rows):
    print(f"lm_head V={V} R={R} n_rows={n_rows}", flush=True)
    H = 2880
    h = torch.randn(R, H, device=DEV, generator=_gen(1)).to(torch.bfloat16)
    norm_w = (1.0 + 0.1 * torch.randn(H, device=DEV, generator=_gen(2))).float()
    w = (0.02 * torch.randn(V, H, device=DEV, generator=_gen(3))).to(torch.bfloat16)
    rows = torch.randperm(R, device=DEV, generator=_gen(4))[:n_rows].to(torch.int32)
    xn = ops.rmsnorm(h, norm_w)
    packed = ops.bf16_tile_repack(w)
    ids, logits = ops.lm_head_argmax(xn, packed, V, rows=rows, want_logits=True)
    torch.cuda.synchronize()
    ids, logits = ids.cpu().numpy(), logits.float().cpu().numpy()
    sel = rows.cpu().long()
    # the final norm against the oracle's (its own rounding, within the bar)
    mar, cos = gh.metrics(gh.cpu_f32(xn)[sel].numpy(),
                          olayer.rmsnorm(gh.cpu_f32(h)[sel], gh.cpu_f32(norm_w)).numpy())
    assert mar < 1e-2 and cos > 0.99999
    # the lm_head on the same normed rows: fp32 MFMA accumulation vs fp64, each rounded once to
    # bf16, so at most one rounding step apart (plus a hair for the fp32 sum)
    ref = otail.logits_from_normed(gh.cpu_f32(xn)[sel], gh.cpu_f32(w)).numpy()
    tol = np.maximum(_bf16_ulp(ref), _bf16_ulp(logits)) * 1.01 + 1e-5
    dev = np.abs(logits - ref)
    worst = np.unravel_index(np.argmax(dev - tol), dev.shape)
    print(f"  max |gpu - oracle| {dev.max():.3e}; worst vs tolerance at {worst}: gpu {logits[worst]} "
          f"oracle {ref[worst]}; over tolerance {(dev > tol).sum()}", flush=True)
    assert (dev <= tol).all()
    # the pick is exactly the first maximum of the kernel's own logits ...
    assert (ids == logits.argmax(-1)).all()
    # ... and the oracle's pick unless the oracle's top two are within one rounding step
    want = otail.greedy_pick(ref)
    for r in np.nonzero(ids != want)[0]:
        assert ref[r, want[r]] - ref[r, ids[r]] <= tol[r, want[r]] + tol[r, ids[r]], r


def test_embed_gather_rows_and_out_of_range():
    V, H = 300, 2880
    table = torch.randn(V, H, device=DEV, generator=_gen(5)).to(torch.bfloat16)
    ids = torch.tensor([0, 299, 17, -1, 300, 17], dtype=torch.int32, device=DEV)
    out = ops.embed_gather(table, ids)
    torch.cuda.synchronize()
    for i, t in enumerate([0, 299, 17, None, None, 17]):
        assert torch.equal(out[i], table[t] if t is not None else torch.zeros_like(out[i]))


def _model(vocab=1024, max_jobs=4, max_context=256, chunk=8, seed=11):
    shape = GptOssShape(n_experts=32)
    layers = [synthetic_layer(shape, seed * 10 + i, DEV, sliding=(i % 2 == 0), keep_hf=True) for i in range(2)]
    embed = torch.randn(vocab, shape.hidden, device=DEV, generator=_gen(seed)).to(torch.bfloat16)
    norm_w = (1.0 + 0.1 * torch.randn(shape.hidden, device=DEV, generator=_gen(seed + 1))).float()
    lm = (0.02 * torch.randn(vocab, shape.hidden, device=DEV, generator=_gen(seed + 2))).to(torch.bfloat16)
    rot = YarnRotary(max_context, device=DEV)
    m = GptOssModel(shape, layers, embed, norm_w, lm, rot, max_jobs, max_context, max_jobs * chunk, DEV)
    return m, dict(shape=shape, layers=layers, embed=embed, norm_w=norm_w, lm=lm)


def _backend(model, chunk=8):
    return GptOssBatchBackend(model, model_id="gpt-oss-synthetic", cohort_id="c", tokenize=lambda p: p["ids"],
                              max_prompt_tokens=64, max_new_tokens=16, prefill_chunk_tokens=chunk)


def test_backend_tokens_batch_invariant_and_follow_oracle():
    """Three jobs with 1-3 prefill chunks each, run together through a ring-style worker loop, commit
    exactly the tokens each job commits alone (per-row reductions everywhere); every committed token
    is the oracle's greedy choice on that job's own sequence, or a near-tie of it."""
    rng = np.random.default_rng(0)
    prompts = [rng.integers(0, 1024, size=n).tolist() for n in (5, 13, 20)]
    max_new = [6, 4, 5]
    model, w = _model()
    be = _backend(model)
    w0 = be.warmup()
    assert w0["proof_verified"] is True
    jobs = [Job(f"j{i}", p, n) for i, (p, n) in enumerate(zip(prompts, max_new))]
    done, _ = run_worker(be, jobs)
    torch.cuda.synchronize()
    for j in jobs:
        assert len(j.tokens) == j.max_new and be.verify_result_proof(j, done[j.id])
        solo = Job(j.id, j.payload["ids"], j.max_new)
        run_worker(be, [solo])
        assert solo.tokens == j.tokens, f"{j.id}: batched {j.tokens} solo {solo.tokens}"
    # oracle, teacher-forced on each job's committed sequence
    params = [gh.oracle_layer_params(lw, lw.sliding) for lw in w["layers"]]
    cos, sin = olayer.rope_table(model.max_context)
    exact = total = 0
    for j in jobs:
        p = j.payload["ids"]
        seq = p + j.tokens[:-1]
        lg = otail.greedy_continue(seq, gh.cpu_f32(w["embed"]), params, gh.cpu_f32(w["norm_w"]),
                                   gh.cpu_f32(w["lm"]), cos, sin).numpy()
        for i, tok in enumerate(j.tokens):
            row = lg[len(p) - 1 + i]
            best = int(otail.greedy_pick(row[None])[0])
            total += 1
            exact += tok == best
            assert row[best] - row[tok] <= 2e-2 * np.abs(row).max(), (j.id, i, tok, best)
    print(f"oracle greedy agreement {exact}/{total}", flush=True)
    assert exact >= 0.8 * total
