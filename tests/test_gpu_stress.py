"""Stress shape: 256 sequences with Zipf query lengths (mostly single-token decode, verify chunks up to
8 tokens, two 1024-token prefill chunks), KV lengths log-uniform in [128, 32768], and a router bias
that sends ~50% of the assignments to 10% of the experts.  Two layers (sliding, then full) keep the
KV pools at ~34 GB.

The GPU runs the full batch one layer at a time.  Checked on the full batch: finite outputs and the
routing invariants (histogram sums to T*k, perm a permutation, inv its inverse, the designed skew).
Checked against the oracle: the last rows of a handful of sequences (the longest KV, both prefill
chunks, verify rows, short decode rows) as their own ragged batch, from the GPU's own layer input
and the GPU-written KV: the attention output within a tight bar, and the layer output on every
token routed alike (a token may route differently only on a near-tie of the oracle's router logits,
which a last-bit difference of its attention output can flip).  That subset comparison is valid because a row's result does not depend on
its batch mates (test_batched_equals_solo_bit_exact checks this bit for bit)."""
import numpy as np
import pytest
import torch

from oracle import layer as olayer

pytestmark = pytest.mark.gpu

MAR, COS = 2e-2, 0.999
DEV = "cuda"
MAXLEN = 32768


def _batch(seed=4, S=256):
    rng = np.random.default_rng(seed)
    q = np.minimum(rng.zipf(2.2, size=S), 8)
    prefill = rng.choice(S, size=2, replace=False)
    q[prefill] = 1024
    kv = np.exp(rng.uniform(np.log(128), np.log(MAXLEN), size=S)).astype(np.int64)
    starts = np.maximum(kv - q, 0)
    return [int(v) for v in q], [int(v) for v in starts], [int(v) for v in prefill]


@pytest.mark.parametrize("dense_fp8", [False, True], ids=["bf16-dense", "fp8-dense"])
def test_stress_batch_layers_vs_oracle(dense_fp8):
    from flyai_amd import ops
    from flyai_amd.rope import YarnRotary
    from flyai_amd.runtime import KVWorkspace, RaggedStage
    from flyai_amd.weights import GptOssShape, synthetic_layer
    from gpu_harness import _SingleLayerKV, cpu_f32, metrics, oracle_layer_params, tokens_with_same_routing

    shape = GptOssShape()
    q_lens, starts, prefill = _batch()
    S, T = len(q_lens), sum(q_lens)
    E, k = shape.n_experts, shape.top_k
    hot = torch.randperm(E, generator=torch.Generator().manual_seed(9))[:E // 10]
    layers = []
    for i in range(2):
        lw = synthetic_layer(shape, 4000 + i, DEV, sliding=(i % 2 == 0), keep_hf=True)
        rb = lw.router_b.float()
        rb[hot.to(DEV)] += 1.2   # skew: ~50% of the assignments go to 10% of the experts
        lw.router_b = rb.to(torch.bfloat16)
        layers.append(lw)
    rot = YarnRotary(MAXLEN + 64, device=DEV)
    kv = KVWorkspace(2, S, MAXLEN + 64, shape.n_kv_heads, shape.head_dim, DEV)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    for t in kv.k + kv.v:
        t.normal_(generator=g)
    h = torch.randn(T, shape.hidden, device=DEV, generator=g).to(torch.bfloat16)

    # the subset checked against the oracle: (sequence, rows from its end)
    order = np.argsort([s + q for s, q in zip(starts, q_lens)])
    verify = [b for b in range(S) if 2 <= q_lens[b] <= 8]
    decode = [b for b in range(S) if q_lens[b] == 1]
    picks = [(int(order[-1]), 1), (prefill[0], 4), (prefill[1], 4), (verify[0], q_lens[verify[0]]),
             (decode[0], 1), (int(order[0]), 1)]
    cu = np.concatenate([[0], np.cumsum(q_lens)])
    rows = np.concatenate([np.arange(cu[b + 1] - n, cu[b + 1]) for b, n in picks])
    sub_q = [n for _, n in picks]
    sub_starts = [starts[b] + q_lens[b] - n for b, n in picks]
    cos, sin = olayer.rope_table(MAXLEN + 64)

    for l, lw in enumerate(layers):
        st = RaggedStage(shape, [lw], rot, _SingleLayerKV(kv, l), max_tokens=T, max_seqs=S, dense_fp8=dense_fp8)
        hin = h
        h = st.forward(hin.clone(), q_lens, starts, list(range(S)))
        torch.cuda.synchronize()
        assert torch.isfinite(h.float()).all(), f"layer {l}: non-finite output"
        # routing invariants on the full batch (the stage's own buffers of this step)
        ids = st.debug_buffer(4, torch.int32, (T, k)).cpu().numpy()
        perm = st.debug_buffer(7, torch.int32, (T * k,)).cpu().numpy()
        inv = st.debug_buffer(8, torch.int32, (T * k,)).cpu().numpy()
        off = st.debug_buffer(6, torch.int32, (E + 1,)).cpu().numpy()
        hist = np.bincount(ids.reshape(-1), minlength=E)
        assert off[-1] == T * k and np.array_equal(np.diff(off), hist)
        assert np.array_equal(np.sort(perm), np.arange(T * k))
        assert np.array_equal(inv[perm], np.arange(T * k))
        assert (ids.reshape(-1)[perm] == np.repeat(np.arange(E), hist)).all()
        share = hist[hot.numpy()].sum() / hist.sum()
        assert 0.35 < share < 0.7, f"hot-expert share {share:.2f}"
        # oracle on the subset, from the GPU's layer input and the GPU-written KV of this layer
        ks = [cpu_f32(kv.k_dense(l, b)) for b, _ in picks]
        vs = [cpu_f32(kv.v_dense(l, b)) for b, _ in picks]
        tr = {}
        ref = olayer.decoder_layer(cpu_f32(hin)[rows], oracle_layer_params(lw, lw.sliding), (ks, vs),
                                   sub_q, sub_starts, cos, sin, trace=tr, force_ids=ids[rows])
        attn = cpu_f32(st.debug_buffer(3, torch.bfloat16, (T, shape.n_q_heads * shape.head_dim)))[rows].numpy()
        mar_a, cos_a = metrics(attn, np.asarray(tr["attn"]).reshape(len(rows), -1))
        tokens_with_same_routing(ids[rows], tr["ids"], tr["logits"], k)
        mar, cos_ = metrics(cpu_f32(h)[rows].numpy(), ref.numpy())
        print(f"C4 {'fp8' if dense_fp8 else 'bf16'} dense, layer {l}: attention max-abs-rel {mar_a:.4g} cos "
              f"{cos_a:.6f}; layer max-abs-rel {mar:.4g} cos {cos_:.6f} on all {len(rows)} rows, "
              f"{len(tr['forced_rows'])} teacher-forced")
        assert mar_a <= 1e-2 and cos_a >= 0.9999, f"layer {l} attention: {mar_a:.3g} {cos_a:.6f}"
        assert mar <= MAR and cos_ >= COS, f"layer {l}: {mar:.3g} {cos_:.6f}"
        del st
