"""CPU checks of the C ABI: the built library loads, exports every function include/flyai_stage.h
declares, and the host-only entry points (planner, sizes, validation) behave -- no GPU needed."""
import ctypes as C
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "flyai_stage.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(flyai_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from flyai_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from flyai_amd import build
        build.build(verbose=False)
    return _lib.lib()


def test_library_exports_every_declared_symbol(lib):
    names = _declared()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"missing exports: {missing}"
    from flyai_amd import _lib
    assert sorted(_lib.exported_names()) == names, "ctypes prototypes out of sync with the header"


def test_abi_version_and_error_string(lib):
    assert lib.flyai_abi_version() == 2
    from flyai_amd import _lib
    rc = lib.flyai_moe_permute(None, 4, 4, 300, None, None, None, None, None)
    assert rc == _lib.FLYAI_EINVAL
    assert b"E must be" in lib.flyai_last_error()


def test_packed_bytes_and_partials_bytes(lib):
    # gate_up of GPT-OSS: 360 tiles x (90 blocks x 256 B data + 6 x 256 B scales) per expert
    assert lib.flyai_mxfp4_packed_bytes(1, 5760, 2880) == 360 * (90 * 256 + 6 * 256)
    assert lib.flyai_mxfp4_packed_bytes(1, 5760, 2880 + 1) == 0
    assert lib.flyai_attn_partials_bytes(10) == 10 * 32 * 66 * 4


def test_attn_plan_host(lib):
    from flyai_amd import ops
    items, groups, n_small = ops.attn_plan([1, 4, 6], [700, 0, 130], n_kv_heads=2, window=0, split_keys=512)
    g = groups.numpy()
    it = items.numpy()
    # seq0: 1 group/kv head, keys [0, 701) -> 2 splits; seq1: [0,4) -> 1; seq2: tokens 0-3, 4-5
    assert g.shape[0] == 2 * (1 + 1 + 2)
    assert [int(x) for x in g[:, 1]] == [2, 2, 1, 1, 1, 1, 1, 1]
    assert it[0].tolist()[:8] == [0, 0, 0, 1, 700, 0, 512, 0]
    assert it[1].tolist()[5:7] == [512, 701]
    # sliding window 128: keys of tokens 130..133 start at 3 (aligned block 0)
    items_w, groups_w, _ = ops.attn_plan([4], [130], n_kv_heads=1, window=128, split_keys=512)
    assert items_w.numpy()[0, 5] == 130 - 127 and items_w.numpy()[0, 6] == 134


def test_stage_create_validation(lib):
    from flyai_amd import _lib
    cfg = _lib.StageConfig(n_layers=1, hidden=2880, n_q_heads=64, n_kv_heads=8, head_dim=128,
                           n_experts=128, top_k=4, intermediate=2880, window=128, max_tokens=64,
                           max_seqs=8, max_attn_items=100, rope_positions=4096, attn_split_keys=512,
                           rms_eps=1e-5, attn_prefill_min=32)
    h = C.c_void_p()
    assert lib.flyai_stage_create(C.byref(cfg), C.byref(h)) == _lib.FLYAI_EINVAL
    cfg.head_dim = 64
    assert lib.flyai_stage_create(C.byref(cfg), C.byref(h)) == 0
    assert lib.flyai_stage_workspace_bytes(h) > 0
    lib.flyai_stage_destroy(h)


def test_attn_plan_prefill_host(lib):
    """Sequences of q_len >= prefill_min become 16-token prefill items (last tile first); the rest
    keep the <= 4-token decode items."""
    from flyai_amd import ops
    items, groups, n_small, pitems = ops.attn_plan_prefill([1, 40, 3], [10, 100, 0], n_kv_heads=2, window=0,
                                                           split_keys=512, prefill_min=32)
    p = pitems.numpy()
    assert p.shape[0] == 3 * 2
    # (seq, kv_head, tok, ntok, pos0, key_lo, key_hi, group)
    assert p[0].tolist() == [1, 0, 1 + 32, 8, 132, 0, 140, -1] and p[1].tolist() == [1, 1, 33, 8, 132, 0, 140, -1]
    assert p[2].tolist() == [1, 0, 17, 16, 116, 0, 132, -1] and p[4].tolist() == [1, 0, 1, 16, 100, 0, 116, -1]
    assert sorted(set(items.numpy()[:, 0].tolist())) == [0, 2]
    _, _, _, pw = ops.attn_plan_prefill([40], [200], n_kv_heads=1, window=128, split_keys=512, prefill_min=32)
    assert pw.numpy()[0, 5] == 232 - 127 and pw.numpy()[-1, 5] == 200 - 127
    _, _, _, none = ops.attn_plan_prefill([40], [200], n_kv_heads=1, window=0, split_keys=512, prefill_min=0)
    assert none.shape[0] == 0
