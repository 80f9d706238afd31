"""Tree-verify input validation on the host (no GPU, no launch).

One table of trees -- well-formed ones and every malformation the reference's validate_tree guards
against (phase0/fastverify.py:29-49; its cases in tests/test_tree_validate.py) -- is run through both
validators this build has: ``runtime.validate_tree`` (what ``FastVerifyStage.tree_decode`` calls before
any parent walk) and the C ABI's own check in ``flyai_stage_forward_tree``.  A malformed tree must be
refused by both, a well-formed one accepted by both (the C call then stops at its first device-side
requirement, the unset workspace).  Overflow and the 64-node limit are checked through tree_decode."""
import ctypes as C
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from flyai_amd import _lib
from flyai_amd._lib import ContextOverflow
from flyai_amd.runtime import FastVerifyStage, validate_tree

# name, n_nodes, parents, depths, fragment the Python error must contain (None: valid tree)
TREES = [
    ("single root", 1, [-1], [0], None),
    ("chain with a side branch", 6, [-1, 0, 1, 2, 0, 4], [0, 1, 2, 3, 1, 2], None),
    ("root in the middle", 3, [1, -1, 1], [1, 0, 1], None),
    ("two-cycle", 3, [-1, 2, 1], [0, 1, 1], "depth"),
    ("self parent", 2, [-1, 1], [0, 1], "range"),
    ("parent past the tree", 3, [-1, 5, 0], [0, 1, 1], "range"),
    ("parent below -1", 3, [-1, -2, 0], [0, 1, 1], "range"),
    ("parent not an int", 2, [-1, "0"], [0, 1], "range"),
    ("too few parents", 3, [-1, 0], [0, 1, 1], "length"),
    ("too few depths", 3, [-1, 0, 0], [0, 1], "length"),
    ("empty tree", 0, [], [], "invalid"),
    ("depth skips a level", 2, [-1, 0], [0, 5], "depth"),
    ("negative depth", 2, [-1, 0], [0, -1], "invalid"),
    ("depth not an int", 2, [-1, 0], [0, "1"], "invalid"),
    ("root with depth 1", 2, [-1, 0], [1, 2], "depth"),
]


@pytest.mark.parametrize("name,n,par,dep,err", TREES, ids=[t[0] for t in TREES])
def test_python_validator(name, n, par, dep, err):
    if err is None:
        validate_tree(n, par, dep)
    else:
        with pytest.raises(ValueError, match=err):
            validate_tree(n, par, dep)


@pytest.fixture(scope="module")
def stage():
    lib = _lib.lib()
    cfg = _lib.StageConfig(n_layers=1, hidden=2880, n_q_heads=64, n_kv_heads=8, head_dim=64, n_experts=128,
                           top_k=4, intermediate=2880, window=128, max_tokens=64, max_seqs=4, max_attn_items=256,
                           rope_positions=4096, attn_split_keys=1024, rms_eps=1e-5, attn_prefill_min=0)
    h = C.c_void_p()
    assert lib.flyai_stage_create(C.byref(cfg), C.byref(h)) == 0
    names = ("ln1", "ln2", "wqkv", "bqkv", "wo", "bo", "sinks", "router_w", "router_b", "w13_packed", "b13",
             "w2_packed", "b2", "k_pool", "v_pool")
    d = _lib.LayerDesc(**{f: 0x100000 for f in names}, sliding=0, pad=0, kv_pool_elems=8 * 4096 * 64)
    assert lib.flyai_stage_set_layer(h, 0, C.byref(d)) == 0
    yield lib, h
    lib.flyai_stage_destroy(h)


@pytest.mark.parametrize("name,n,par,dep,err", [t for t in TREES if all(type(v) is int for v in t[2] + t[3])
                                                 and len(t[2]) == len(t[3]) == t[1]],
                         ids=lambda v: v if isinstance(v, str) else None)
def test_c_abi_validator_agrees(stage, name, n, par, dep, err):
    lib, h = stage
    pa = np.asarray(par if par else [0], dtype=np.int32)
    de = np.asarray(dep if dep else [0], dtype=np.int32)
    rc = lib.flyai_stage_forward_tree(h, 100, n, pa.ctypes.data_as(C.c_void_p), de.ctypes.data_as(C.c_void_p),
                                      0, 4096, C.c_void_p(0x200000), None)
    msg = lib.flyai_last_error().decode()
    assert rc == _lib.FLYAI_EINVAL, (name, rc, msg)
    if err is None:
        assert "workspace not set" in msg, (name, msg)
    else:
        assert "workspace" not in msg and "tree" in msg, (name, msg)


def _guards_only(maxlen):
    """tree_decode reads only maxlen before its guards fire."""
    return SimpleNamespace(maxlen=maxlen)


@pytest.mark.parametrize("name,n,par,dep,err", [t for t in TREES if t[4] is not None and t[1] > 0],
                         ids=lambda v: v if isinstance(v, str) else None)
def test_tree_decode_refuses_before_any_walk(name, n, par, dep, err):
    h = torch.zeros(1, n, 8)
    with pytest.raises(ValueError, match=err):
        FastVerifyStage.tree_decode(_guards_only(64), h, 0, par, dep)


@pytest.mark.parametrize("start,maxlen,overflows", [(61, 64, False), (62, 64, True), (0, 2, True)])
def test_tree_decode_context_overflow(start, maxlen, overflows):
    """A 3-node chain needs start + 3 positions; past maxlen it is ContextOverflow before any write."""
    h = torch.zeros(1, 3, 8)
    stub = _guards_only(maxlen)
    if overflows:
        with pytest.raises(ContextOverflow):
            FastVerifyStage.tree_decode(stub, h, start, [-1, 0, 1], [0, 1, 2])
    else:
        with pytest.raises(AttributeError):     # got past every guard to the (absent) stage
            FastVerifyStage.tree_decode(stub, h, start, [-1, 0, 1], [0, 1, 2])


@pytest.mark.parametrize("max_tokens,limit", [(100, 100), (4096, 2048)])
def test_tree_decode_node_limit(max_tokens, limit):
    """Trees are limited to min(max_tokens, 2048) nodes: one more is ValueError before any write."""
    stub = SimpleNamespace(maxlen=8192, stage=SimpleNamespace(max_tokens=max_tokens))
    n = limit + 1
    chain_par, chain_dep = [-1] + list(range(n - 1)), list(range(n))
    with pytest.raises(ValueError, match=f"{limit}-node"):
        FastVerifyStage.tree_decode(stub, torch.zeros(1, n, 8), 0, chain_par, chain_dep)
