"""Host-side tree-verify checks (no GPU): validate_tree and FastVerifyStage.tree_decode reject a
malformed or overflowing tree before any parent walk or launch.  The cases are the reference's own
(tests/test_tree_validate.py:24-88)."""
from types import SimpleNamespace

import pytest
import torch

from flyai_amd._lib import ContextOverflow
from flyai_amd.runtime import FastVerifyStage, validate_tree


def test_valid_trees_pass():
    validate_tree(1, [-1], [0])
    validate_tree(6, [-1, 0, 1, 2, 0, 4], [0, 1, 2, 3, 1, 2])
    validate_tree(3, [1, -1, 1], [1, 0, 1])          # any node order (root not node 0)


def test_cycle_rejected():
    with pytest.raises(ValueError, match="cycle|depth"):
        validate_tree(3, [-1, 2, 1], [0, 1, 1])
    with pytest.raises(ValueError, match="range"):
        validate_tree(2, [-1, 1], [0, 1])            # self-parent


def test_parent_out_of_range_rejected():
    with pytest.raises(ValueError, match="range"):
        validate_tree(3, [-1, 5, 0], [0, 1, 1])
    with pytest.raises(ValueError, match="range"):
        validate_tree(3, [-1, -2, 0], [0, 1, 1])
    with pytest.raises(ValueError, match="range"):
        validate_tree(2, [-1, "0"], [0, 1])


def test_length_mismatch_and_bad_depth_rejected():
    with pytest.raises(ValueError, match="length"):
        validate_tree(3, [-1, 0], [0, 1, 1])
    with pytest.raises(ValueError, match="length"):
        validate_tree(3, [-1, 0, 0], [0, 1])
    with pytest.raises(ValueError, match="invalid"):
        validate_tree(0, [], [])
    with pytest.raises(ValueError, match="depth"):
        validate_tree(2, [-1, 0], [0, 5])
    with pytest.raises(ValueError, match="invalid"):
        validate_tree(2, [-1, 0], [0, -1])
    with pytest.raises(ValueError, match="invalid"):
        validate_tree(2, [-1, 0], [0, "1"])


def _fake_fv(maxlen=64):
    """Just enough of a FastVerifyStage for tree_decode to reach (and stop at) its guards."""
    return SimpleNamespace(maxlen=maxlen)


def test_tree_decode_rejects_before_any_walk():
    h = torch.zeros(1, 3, 8)
    with pytest.raises(ValueError, match="range"):
        FastVerifyStage.tree_decode(_fake_fv(), h, 0, [-1, 5, 0], [0, 1, 1])
    with pytest.raises(ValueError, match="cycle|depth"):
        FastVerifyStage.tree_decode(_fake_fv(), h, 0, [-1, 2, 1], [0, 1, 1])


def test_tree_decode_overflow_fails_clean():
    h = torch.zeros(1, 3, 8)
    with pytest.raises(ContextOverflow):
        FastVerifyStage.tree_decode(_fake_fv(maxlen=64), h, 62, [-1, 0, 1], [0, 1, 2])


def test_tree_over_the_node_limit_rejected():
    M = 65
    h = torch.zeros(1, M, 8)
    with pytest.raises(ValueError, match="64-node"):
        FastVerifyStage.tree_decode(_fake_fv(maxlen=4096), h, 0, [-1] + list(range(M - 1)), list(range(M)))
