"""HIP-graph replay of the stage step (the CUDA-graph capture of FastVerify.decode /
BatchedFastVerify.decode, phase0/fastverify.py:221-231, phase0/batchverify.py:180-190).

The replayed step must equal the eager step bit for bit (same kernels, same launch order), on
every replay, with the program's own eager work and synchronisations between replays; a graph is
captured only when the key (tokens, sequences, attention-plan capacity) changes."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _eager_noise(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    a = torch.randn(512, 512, device="cuda", generator=g)
    (a @ a).sum().item()  # eager work and a synchronisation between replays
    torch.cuda.synchronize()


def test_graph_replay_bit_exact_and_captured_per_key():
    from gpu_harness import small_stage_case
    from flyai_amd.runtime import KVWorkspace, RaggedStage
    q_lens = [1] * 6 + [4] * 2
    starts = [600, 513, 4000, 800, 1, 2500, 1500, 3000]
    case = small_stage_case(n_layers=2, n_experts=16, seed=5, q_lens=q_lens, starts=starts, maxlen=8192)
    shape, layers, rot = case["shape"], case["layers"], case["rot"]
    kv_e = case["kv"]
    kv_g = KVWorkspace(len(layers), 8, 8192, shape.n_kv_heads, shape.head_dim)
    for l in range(len(layers)):
        kv_g.k[l].copy_(kv_e.k[l])
        kv_g.v[l].copy_(kv_e.v[l])
    eager = RaggedStage(shape, layers, rot, kv_e, 64, 8)
    graph = RaggedStage(shape, layers, rot, kv_g, 64, 8, use_graphs=True)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(17)

    def step(ql, st, tag):
        T = sum(ql)
        h = torch.randn(T, shape.hidden, device="cuda", generator=gen).to(torch.bfloat16)
        out_e = eager.forward(h.clone(), ql, st, list(range(len(ql))))
        out_g = graph.forward(h.clone(), ql, st, list(range(len(ql))))
        torch.cuda.synchronize()
        assert torch.equal(out_e, out_g), f"{tag}: replayed step differs from eager"
        for l in range(len(layers)):
            assert torch.equal(kv_e.k[l], kv_g.k[l]) and torch.equal(kv_e.v[l], kv_g.v[l]), f"{tag}: KV differs"
        _eager_noise(len(tag))

    # decode steps whose KV grows inside one plan bucket: one capture, then replays
    st = list(starts)
    for i in range(4):
        step(q_lens, st, f"decode {i}")
        st = [s + q for s, q in zip(st, q_lens)]
    assert graph.graphs_captured == 1
    # 2048 more keys per sequence: more attention items, a new plan bucket
    far = [s + 2048 for s in st]
    step(q_lens, far, "longer KV")
    assert graph.graphs_captured == 2
    # another batch shape (tokens and groups differ)
    step([2] * 8, st, "verify-2 rows")
    assert graph.graphs_captured == 3
    # back to the first key: replayed, not captured again
    step(q_lens, st, "first key again")
    step(q_lens, [s + 1 for s in st], "first key, next position")
    assert graph.graphs_captured == 3


def test_batched_fast_verify_graph_and_eager_agree():
    """BatchedFastVerifyStage.decode(use_graph=True/False) on the same inputs and KV."""
    from gpu_harness import small_stage_case
    from flyai_amd.runtime import BatchedFastVerifyStage
    case = small_stage_case(n_layers=2, n_experts=16, seed=9, q_lens=[4] * 4, starts=[10, 200, 1000, 50],
                            maxlen=2048)
    parts = {"layers": case["layers"], "rotary": case["rot"], "shape": case["shape"]}
    g = BatchedFastVerifyStage(parts, 4, maxlen=2048)
    e = BatchedFastVerifyStage(parts, 4, maxlen=2048)
    for l in range(2):
        for kv in (g.cache, e.cache):
            kv.k[l].copy_(case["kv"].k[l])
            kv.v[l].copy_(case["kv"].v[l])
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    starts = torch.tensor([10, 200, 1000, 50])
    for i in range(3):
        h = torch.randn(4, 4, case["shape"].hidden, device="cuda", generator=gen).to(torch.bfloat16)
        a = g.decode(h, starts + 4 * i, use_graph=True).clone()
        b = e.decode(h, starts + 4 * i, use_graph=False).clone()
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"step {i}"
        _eager_noise(i)
    assert g.stage.graphs_captured == 1 and e.stage.graphs_captured == 0


def test_rebinding_drops_captured_graphs():
    """A captured step graph holds the pointers bound at capture.  Rebinding a layer's weights and the
    workspace must drop the cache: the next step captures again and follows the new bindings, bit for
    bit equal to an eager stage bound the same way (a stale replay would still use the old layer-1
    weights, which stay alive here, so it would show as a mismatch, not as a fault)."""
    from gpu_harness import small_stage_case
    from flyai_amd.runtime import KVWorkspace, RaggedStage
    from flyai_amd.weights import synthetic_layer
    q_lens = [1] * 6 + [4] * 2
    starts = [600, 513, 4000, 800, 1, 2500, 1500, 3000]
    case = small_stage_case(n_layers=2, n_experts=16, seed=6, q_lens=q_lens, starts=starts, maxlen=8192)
    shape, layers, rot = case["shape"], case["layers"], case["rot"]
    other = synthetic_layer(shape, 991, "cuda", sliding=layers[1].sliding)
    kv0 = [(k.clone(), v.clone()) for k, v in zip(case["kv"].k, case["kv"].v)]
    kv_g = case["kv"]
    kv_e = KVWorkspace(2, 8, 8192, shape.n_kv_heads, shape.head_dim)

    def reset_kv():
        for l, (k, v) in enumerate(kv0):
            for kv in (kv_g, kv_e):
                kv.k[l].copy_(k)
                kv.v[l].copy_(v)

    graph = RaggedStage(shape, layers, rot, kv_g, 64, 8, use_graphs=True)
    eager = RaggedStage(shape, [layers[0], other], rot, kv_e, 64, 8)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(23)
    h = torch.randn(sum(q_lens), shape.hidden, device="cuda", generator=gen).to(torch.bfloat16)
    slots = list(range(8))
    reset_kv()
    graph.forward(h.clone(), q_lens, starts, slots)
    graph.forward(h.clone(), q_lens, starts, slots)
    torch.cuda.synchronize()
    assert graph.graphs_captured == 1
    old_workspace = graph.workspace            # kept alive: a stale graph must not touch freed memory
    graph.set_layer(1, other)
    graph.set_workspace()
    assert graph.workspace.data_ptr() != old_workspace.data_ptr()
    reset_kv()
    out_g = graph.forward(h.clone(), q_lens, starts, slots)
    out_e = eager.forward(h.clone(), q_lens, starts, slots)
    torch.cuda.synchronize()
    assert graph.graphs_captured == 2, "rebinding did not drop the captured graph"
    assert torch.equal(out_g, out_e), "replay after rebinding differs from the eager step"
    for l in range(2):
        assert torch.equal(kv_g.k[l], kv_e.k[l]) and torch.equal(kv_g.v[l], kv_e.v[l]), f"KV layer {l}"
    # the step's positions went to the new workspace
    pos = graph.debug_buffer(11, torch.int32, (sum(q_lens),)).cpu().tolist()
    want = [s + i for s, q in zip(starts, q_lens) for i in range(q)]
    assert pos == want
    _eager_noise(5)
    reset_kv()
    out_g2 = graph.forward(h.clone(), q_lens, starts, slots)   # replays the new capture
    torch.cuda.synchronize()
    assert graph.graphs_captured == 2
    assert torch.equal(out_g2, out_e), "second replay after rebinding differs"
    del old_workspace
