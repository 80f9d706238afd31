"""Host-side validation of the stage step's KV slabs through the C ABI (no GPU, no kernel launch).

A slab that runs past its layer's pools must fail with FLYAI_ERANGE and two sequences of one step
whose slabs overlap with FLYAI_EINVAL, both before anything is launched -- the reference raises
ContextOverflow before any out-of-bounds write (phase0/fastverify.py:23-26).  A well-formed batch
passes every check and stops at the first one that needs the device ("workspace not set"), which
shows that the validation above it accepted the batch.  Fake weight addresses are never
dereferenced: validation reads host memory only."""
import ctypes as C

import numpy as np
import pytest

from flyai_amd import _lib

HKV, D = 8, 64
CAP = 256
SLAB = HKV * CAP * D


@pytest.fixture
def stage():
    lib = _lib.lib()
    cfg = _lib.StageConfig(n_layers=2, hidden=2880, n_q_heads=64, n_kv_heads=HKV, head_dim=D, n_experts=128,
                           top_k=4, intermediate=2880, window=128, max_tokens=64, max_seqs=8, max_attn_items=512,
                           rope_positions=4096, attn_split_keys=1024, rms_eps=1e-5, attn_prefill_min=32)
    h = C.c_void_p()
    assert lib.flyai_stage_create(C.byref(cfg), C.byref(h)) == 0
    fake = 0x100000
    pools = (4 * SLAB, 3 * SLAB)          # layer 1's pools are the smaller ones: 3 slabs
    for l, n in enumerate(pools):
        d = _lib.LayerDesc(**{f: fake for f in ("ln1", "ln2", "wqkv", "bqkv", "wo", "bo", "sinks", "router_w",
                                                "router_b", "w13_packed", "b13", "w2_packed", "b2", "k_pool",
                                                "v_pool")}, sliding=l % 2, pad=0, kv_pool_elems=n)
        assert lib.flyai_stage_set_layer(h, l, C.byref(d)) == 0, lib.flyai_last_error()
    yield lib, h
    lib.flyai_stage_destroy(h)


def _forward(lib, h, q_lens, starts, bases, caps):
    S = len(q_lens)
    arr = lambda v, dt: np.ascontiguousarray(v, dtype=dt)
    q, s, b, c = arr(q_lens, np.int32), arr(starts, np.int32), arr(bases, np.int64), arr(caps, np.int32)
    rc = lib.flyai_stage_forward(h, q.ctypes.data_as(C.c_void_p), s.ctypes.data_as(C.c_void_p),
                                 b.ctypes.data_as(C.c_void_p), c.ctypes.data_as(C.c_void_p), S,
                                 C.c_void_p(0x200000), None)
    return rc, lib.flyai_last_error().decode()


def test_valid_batch_passes_validation(stage):
    lib, h = stage
    rc, msg = _forward(lib, h, [1, 4, 2], [10, 100, 0], [0, SLAB, 2 * SLAB], [CAP] * 3)
    assert rc == _lib.FLYAI_EINVAL and "workspace not set" in msg, msg


@pytest.mark.parametrize("bases,caps,what", [
    ([0, SLAB, 3 * SLAB], [CAP] * 3, "third slab starts at the smaller pool's end"),
    ([0, SLAB, 2 * SLAB + 8], [CAP] * 3, "third slab ends 8 elements past it"),
    ([0, SLAB, 2 * SLAB - 64], [CAP, CAP, CAP + 64], "a larger capacity runs past it"),
])
def test_slab_past_pool_is_erange(stage, bases, caps, what):
    lib, h = stage
    rc, msg = _forward(lib, h, [1, 1, 1], [5, 5, 5], bases, caps)
    assert rc == _lib.FLYAI_ERANGE and "ends past the pools" in msg, (what, msg)


@pytest.mark.parametrize("bases", [[0, 0, 2 * SLAB], [2 * SLAB, SLAB, SLAB + 8], [SLAB - 8, 0, 2 * SLAB]])
def test_overlapping_slabs_are_rejected(stage, bases):
    lib, h = stage
    rc, msg = _forward(lib, h, [1, 1, 1], [5, 5, 5], bases, [CAP] * 3)
    assert rc == _lib.FLYAI_EINVAL and "overlapping KV slabs" in msg, msg


def test_context_overflow_still_checked_first(stage):
    lib, h = stage
    rc, msg = _forward(lib, h, [4], [CAP - 2], [0], [CAP])
    assert rc == _lib.FLYAI_ERANGE and "KV capacity" in msg, msg


def test_tree_slab_past_pool_is_erange(stage):
    lib, h = stage
    par = np.array([-1, 0, 0], dtype=np.int32)
    dep = np.array([0, 1, 1], dtype=np.int32)
    rc = lib.flyai_stage_forward_tree(h, 10, 3, par.ctypes.data_as(C.c_void_p), dep.ctypes.data_as(C.c_void_p),
                                      2 * SLAB + 64, CAP, C.c_void_p(0x200000), None)
    assert rc == _lib.FLYAI_ERANGE and "ends past the pools" in lib.flyai_last_error().decode()
    rc = lib.flyai_stage_forward_tree(h, 10, 3, par.ctypes.data_as(C.c_void_p), dep.ctypes.data_as(C.c_void_p),
                                      2 * SLAB, CAP, C.c_void_p(0x200000), None)
    assert rc == _lib.FLYAI_EINVAL and "workspace not set" in lib.flyai_last_error().decode()


def _make_stage(max_tokens, cap):
    lib = _lib.lib()
    cfg = _lib.StageConfig(n_layers=2, hidden=2880, n_q_heads=64, n_kv_heads=HKV, head_dim=D, n_experts=128,
                           top_k=4, intermediate=2880, window=128, max_tokens=max_tokens, max_seqs=1,
                           max_attn_items=8192, rope_positions=8192, attn_split_keys=1024, rms_eps=1e-5,
                           attn_prefill_min=32)
    h = C.c_void_p()
    assert lib.flyai_stage_create(C.byref(cfg), C.byref(h)) == 0, lib.flyai_last_error()
    for l in range(2):
        d = _lib.LayerDesc(**{f: 0x100000 for f in ("ln1", "ln2", "wqkv", "bqkv", "wo", "bo", "sinks", "router_w",
                                                   "router_b", "w13_packed", "b13", "w2_packed", "b2", "k_pool",
                                                   "v_pool")}, sliding=l % 2, pad=0, kv_pool_elems=HKV * cap * D)
        assert lib.flyai_stage_set_layer(h, l, C.byref(d)) == 0, lib.flyai_last_error()
    return lib, h


def _tree(lib, h, start, par, cap):
    par = np.ascontiguousarray(par, dtype=np.int32)
    dep = np.zeros(len(par), dtype=np.int32)
    for i, p in enumerate(par):  # parents precede children in these trees
        dep[i] = 0 if p < 0 else dep[p] + 1
    rc = lib.flyai_stage_forward_tree(h, start, len(par), par.ctypes.data_as(C.c_void_p),
                                      dep.ctypes.data_as(C.c_void_p), 0, cap, C.c_void_p(0x200000), None)
    return rc, lib.flyai_last_error().decode()


@pytest.mark.parametrize("max_tokens,limit", [(64, 64), (300, 300), (4096, 2048)])
def test_tree_size_limit_is_min_of_max_tokens_and_2048(max_tokens, limit):
    """Trees of up to min(max_tokens, FLYAI_TREE_MAX_NODES = 2048) nodes pass validation (and stop at
    the first check that needs the device); one node more is FLYAI_EINVAL before any launch."""
    cap = 4096
    lib, h = _make_stage(max_tokens, cap)
    try:
        rng = np.random.default_rng(limit)
        wide = [-1] + [int(rng.integers(0, i)) for i in range(1, limit)]
        chain = [-1] + list(range(limit - 1))  # depth limit - 1, past the 128-key window
        for par in (wide, chain):
            rc, msg = _tree(lib, h, 100, par, cap)
            assert rc == _lib.FLYAI_EINVAL and "workspace not set" in msg, msg
        rc, msg = _tree(lib, h, 100, chain + [limit - 1], cap)
        assert rc == _lib.FLYAI_EINVAL and f"outside [1, {limit}]" in msg, msg
    finally:
        lib.flyai_stage_destroy(h)


def test_pool_size_is_required(stage):
    lib, h = stage
    d = _lib.LayerDesc(**{f: 0x100000 for f in ("ln1", "ln2", "wqkv", "bqkv", "wo", "bo", "sinks", "router_w",
                                               "router_b", "w13_packed", "b13", "w2_packed", "b2", "k_pool",
                                               "v_pool")}, sliding=0, pad=0, kv_pool_elems=0)
    assert lib.flyai_stage_set_layer(h, 0, C.byref(d)) == _lib.FLYAI_EINVAL
    assert "kv_pool_elems" in lib.flyai_last_error().decode()


def test_ragged_stage_rejects_shared_slots():
    """RaggedStage.forward refuses two sequences on one KV slot before calling the library."""
    import torch
    from flyai_amd.runtime import RaggedStage
    from flyai_amd.weights import GptOssShape

    class _KV:
        n_slots, maxlen, cap = 4, 2048, 2048

    st = object.__new__(RaggedStage)
    st.shape, st.kv, st._h = GptOssShape(), _KV(), None
    h = torch.zeros(3, 2880, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="share a KV slot"):
        st.forward(h, [1, 1, 1], [0, 4, 8], [0, 2, 2])
    with pytest.raises(ValueError, match="out of range"):
        st.forward(h, [1, 1, 1], [0, 4, 8], [0, 2, 4])
