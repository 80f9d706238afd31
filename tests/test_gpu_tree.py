"""Tree verify on the GPU (FastVerify.tree_decode, phase0/fastverify.py:233-299) against the oracle's
tree-verify layer, plus the chain tree, which must reproduce a linear verify row bit for bit."""
import numpy as np
import pytest
import torch

from tests import gpu_harness as gh
from flyai_amd.runtime import FastVerifyStage, RaggedStage
from oracle import layer as olayer

pytestmark = pytest.mark.gpu


def _random_tree(rng, M):
    """Parents precede children (as propose_tree emits them); node 0 is the root."""
    par = [-1] + [int(rng.integers(0, i)) for i in range(1, M)]
    dep = [0] * M
    for i in range(1, M):
        dep[i] = dep[par[i]] + 1
    return par, dep


def _deep_tree(rng, M, chain):
    """A chain of `chain` nodes (depths past the 128-key sliding window), then random branches."""
    par = [-1] + list(range(chain - 1)) + [int(rng.integers(0, i)) for i in range(chain, M)]
    dep = [0] * M
    for i in range(1, M):
        dep[i] = dep[par[i]] + 1
    return par, dep


TREES = {
    "tree8": ([-1, 0, 1, 2, 0, 4, 1, 6], [0, 1, 2, 3, 1, 2, 2, 3]),
    "root_not_first": ([1, -1, 1, 0, 3], [1, 0, 1, 2, 3]),
}


@pytest.mark.parametrize("name,start,M", [("tree8", 300, 8), ("root_not_first", 64, 5), ("random40", 1000, 40),
                                          ("random64", 130, 64), ("random150", 64, 150), ("deep200", 1000, 200)])
def test_tree_decode_per_layer_vs_oracle(name, start, M):
    """Two layers (sliding, then full) from the GPU's own per-layer input: attention output and the
    K/V at slots start..start+M-1 against the oracle, and the layer output within the bar.  Trees
    past 64 nodes take several mask words per node (starts 64 and 1000: word-aligned and shifted
    key blocks); deep200's chain of 160 reaches past the sliding window inside the tree."""
    print(f"tree case {name} start={start} M={M}", flush=True)
    rng = np.random.default_rng(M)
    if name in TREES:
        par, dep = TREES[name]
    elif name.startswith("deep"):
        par, dep = _deep_tree(rng, M, 160)
    else:
        par, dep = _random_tree(rng, M)
    case = gh.small_stage_case(n_layers=2, n_experts=8, seed=3, q_lens=(M,), starts=(start,))
    shape, layers, kv = case["shape"], case["layers"], case["kv"]
    cos, sin = olayer.rope_table(case["maxlen"])
    h = case["hidden"].clone()
    for l, lw in enumerate(layers):
        okv = gh.oracle_kv(kv, l, [0])
        st = RaggedStage(shape, [lw], case["rot"], gh._SingleLayerKV(kv, l), max_tokens=max(64, M), max_seqs=1)
        hin = gh.cpu_f32(h)
        h = st.forward_tree(h.clone(), start, par, dep, 0)
        torch.cuda.synchronize()
        tr = {}
        ids = st.debug_buffer(4, torch.int32, (M, shape.top_k)).cpu().numpy()
        ref = olayer.decoder_layer(hin, gh.oracle_layer_params(lw, lw.sliding), okv, [M], [start], cos, sin,
                                   trace=tr, tree=(par, dep), force_ids=ids)
        # the tree-specific part: attention output under the ancestor masks
        attn = gh.cpu_f32(st.debug_buffer(3, torch.bfloat16, (M, shape.n_q_heads * shape.head_dim))).numpy()
        mar_a, cos_a = gh.metrics(attn, tr["attn"].reshape(M, -1).numpy())
        print(f"  layer {l} sliding={lw.sliding}: attention max-abs-rel {mar_a:.3e} cos {cos_a:.7f}", flush=True)
        assert mar_a <= 1e-2 and cos_a >= 0.9999, (l, mar_a, cos_a)
        # the layer output on every token; a token may route differently only where the oracle's k-th
        # and (k+1)-th logits are a near-tie the bf16 input rounding can flip, and the oracle then
        # takes the GPU's experts for it (teacher forcing)
        gh.tokens_with_same_routing(ids, tr["ids"], tr["logits"], shape.top_k)
        mar, cos_ = gh.metrics(gh.cpu_f32(h).numpy(), ref.numpy())
        print(f"  layer {l}: {len(tr['forced_rows'])}/{M} tokens teacher-forced, max-abs-rel {mar:.3e} cos {cos_:.6f}",
              flush=True)
        assert mar <= 2e-2 and cos_ >= 0.999, (l, mar, cos_)
        # each node's K/V sits at its own slot (the QKV GEMM's summation order differs from the
        # oracle's, so values agree to bf16 rounding, not bit for bit; a misplaced slot is off by O(1))
        k_gpu = gh.cpu_f32(kv.k_dense(l, 0))[:, start:start + M]
        v_gpu = gh.cpu_f32(kv.v_dense(l, 0))[:, start:start + M]
        for i in range(M):
            for got, want in ((k_gpu[:, i], okv[0][0][:, start + i]), (v_gpu[:, i], okv[1][0][:, start + i])):
                mar_kv, cos_kv = gh.metrics(got.numpy(), want.numpy())
                assert mar_kv < 1e-2 and cos_kv > 0.9999, (l, i, mar_kv, cos_kv)
        del st


@pytest.mark.parametrize("M", [6, 150])
def test_chain_tree_equals_linear_verify_bit_exact(M):
    """A chain (par[i] = i-1, dep[i] = i) is a plain verify row: same hidden and KV bytes as the
    ragged step with q_len M at the same start (decode-sized attention items on both paths; at 150
    nodes the chain runs past the sliding window and over three mask words per node)."""
    start = 517
    print(f"chain tree M={M} start={start}", flush=True)
    par, dep = [-1] + list(range(M - 1)), list(range(M))
    case = gh.small_stage_case(n_layers=2, n_experts=8, seed=5, q_lens=(M,), starts=(start,))
    shape, layers, kv = case["shape"], case["layers"], case["kv"]
    st = RaggedStage(shape, layers, case["rot"], kv, max_tokens=max(64, M), max_seqs=1, prefill_min=0)
    k0 = [t.clone() for t in kv.k]
    v0 = [t.clone() for t in kv.v]
    lin = st.forward(case["hidden"].clone(), [M], [start], [0])
    torch.cuda.synchronize()
    k_lin = [t.clone() for t in kv.k]
    v_lin = [t.clone() for t in kv.v]
    for t, s in zip(kv.k + kv.v, k0 + v0):
        t.copy_(s)
    tr = st.forward_tree(case["hidden"].clone(), start, par, dep, 0)
    torch.cuda.synchronize()
    assert torch.equal(lin, tr)
    for a, b in zip(kv.k + kv.v, k_lin + v_lin):
        assert torch.equal(a, b)


def test_fast_verify_tree_decode_then_gather():
    """The drop-in surface: tree_decode returns [1, M, H] and tree_gather compacts the accepted
    path's KV to contiguous positions (fastverify.py:301-309)."""
    par, dep = TREES["tree8"]
    M, start = len(par), 200
    case = gh.small_stage_case(n_layers=2, n_experts=8, seed=6, q_lens=(M,), starts=(start,))
    parts = {"layers": case["layers"], "rotary": case["rot"], "shape": case["shape"]}
    fv = FastVerifyStage(parts, maxlen=case["maxlen"], dev="cuda", max_tokens=64)
    gh.fill_kv_random(fv.cache, 13)
    h = case["hidden"].view(1, M, -1)
    out = fv.tree_decode(h, start, par, dep)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (1, M, case["shape"].hidden) and torch.isfinite(out.float()).all()
    keep = [0, 1, 6, 7]
    k_before = [fv.cache.k_dense(l, 0)[:, [start + i for i in keep]] for l in range(2)]
    v_before = [fv.cache.v_dense(l, 0)[:, [start + i for i in keep]] for l in range(2)]
    fv.tree_gather(start, keep)
    torch.cuda.synchronize()
    for l in range(2):
        assert torch.equal(fv.cache.k_dense(l, 0)[:, start:start + len(keep)], k_before[l])
        assert torch.equal(fv.cache.v_dense(l, 0)[:, start:start + len(keep)], v_before[l])
