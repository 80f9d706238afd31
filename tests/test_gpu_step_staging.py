"""Consecutive stage steps each carry their own batch description.

Every decode step of the reference builds its batch (row lengths, positions, KV geometry) afresh
(phase0/batchverify.py:166-190).  Here the host writes it as one blob into one of two pinned
staging halves, alternating step by step, and a kernel reads it from there before the step's first
launch.  Three different batches on disjoint KV slots run back to back on one stage, so the third
reuses the first one's half.  Each step's output must equal, bit for bit, a fresh stage's single
run of the same batch on a copy of the initial KV: a step that read a stale or mixed blob would
attend with the wrong rows, positions or slabs."""
import pytest
import torch

pytestmark = pytest.mark.gpu

MAXLEN = 4096
SLOTS = 12


def test_consecutive_steps_read_their_own_batch():
    from gpu_harness import small_stage_case
    from flyai_amd.runtime import KVWorkspace, RaggedStage
    case = small_stage_case(n_layers=2, n_experts=16, seed=9, q_lens=[1] * SLOTS, starts=[100] * SLOTS,
                            maxlen=MAXLEN)
    shape, layers, rot, kv = case["shape"], case["layers"], case["rot"], case["kv"]
    kv0 = KVWorkspace(len(layers), SLOTS, MAXLEN, shape.n_kv_heads, shape.head_dim)
    for l in range(len(layers)):
        kv0.k[l].copy_(kv.k[l])
        kv0.v[l].copy_(kv.v[l])
    # (q_lens, starts, slots): different token counts, sequence counts, positions and slots
    batches = [
        ([1, 4, 1, 2], [700, 1200, 33, 2500], [0, 1, 2, 3]),
        ([4, 4, 1], [3000, 90, 1800], [4, 5, 6]),
        ([2, 1, 1, 4, 1], [512, 2047, 64, 1000, 3100], [8, 9, 10, 11, 7]),
    ]
    stage = RaggedStage(shape, layers, rot, kv, 64, SLOTS)
    g = torch.Generator(device="cuda")
    g.manual_seed(23)
    runs = []
    for ql, st, sl in batches:
        h = torch.randn(sum(ql), shape.hidden, device="cuda", generator=g).to(torch.bfloat16)
        out = stage.forward(h.clone(), ql, st, sl).clone()
        runs.append((h, out))
    torch.cuda.synchronize()
    for i, ((ql, st, sl), (h, out)) in enumerate(zip(batches, runs)):
        kv_i = KVWorkspace(len(layers), SLOTS, MAXLEN, shape.n_kv_heads, shape.head_dim)
        for l in range(len(layers)):
            kv_i.k[l].copy_(kv0.k[l])
            kv_i.v[l].copy_(kv0.v[l])
        fresh = RaggedStage(shape, layers, rot, kv_i, 64, SLOTS)
        ref = fresh.forward(h.clone(), ql, st, sl)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"step {i} (staging half {i % 2}) differs from a fresh stage's run"
