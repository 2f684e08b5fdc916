"""The reference modules' own self-tests (``check_equal``), as this package's replacements provide them:
tree_build_ext.check_equal (inference/hf/tree_build_ext.py:237-270, run by the reference's
tests/test_mixture_tree.py:122), tree_logits.check_equal (inference/hf/tree_logits.py:49-60) and
mode_attention.check_equal (inference/hf/mode_attention.py:167-181).

tree_build_ext.check_equal compares against the HF decode-loop module ``ddtree``'s Python builders; the
reference's module is not imported here, so a stand-in ``ddtree`` built on the C oracle (whose heaps are
pinned to golden trees of the reference's own compiled builders) takes its place in sys.modules."""

import sys
import types

import numpy as np
import pytest
import torch

from oracle import builder as B

pytestmark = pytest.mark.gpu


def _as_reference_tuple(t, d, p, n):
    vis = torch.from_numpy(B.visibility(p, n).astype(bool))
    child_maps = [dict() for _ in range(n + 1)]
    for i in range(1, n + 1):
        child_maps[int(p[i])][int(t[i])] = i
    return (torch.from_numpy(t[1 : n + 1].copy()), torch.from_numpy(d[1 : n + 1].copy()), [int(x) for x in p[: n + 1]],
            child_maps, vis, {})


def _candidates(logits, budget):
    lp = logits.float()
    top, ids = torch.topk(lp, k=min(budget, lp.shape[-1]), dim=-1)
    return (top - torch.logsumexp(lp, -1, keepdim=True)).float().numpy(), ids.numpy()


@pytest.fixture
def oracle_ddtree(monkeypatch):
    import ddtree_hf_ops

    mod = types.ModuleType("ddtree")

    def build_ddtree_tree(logits, budget):
        lp, ids = _candidates(logits, budget)
        t, d, p, n = B.build_single(lp, ids, budget)
        return _as_reference_tuple(t, d, p, n)

    def build_mixture_tree(logits, prior, budget):
        lp, ids = _candidates(logits, budget)
        t, d, p, n, _ = B.build_mixture(lp, ids, prior.float().numpy(), budget)
        return _as_reference_tuple(t, d, p, n)

    mod.build_ddtree_tree = build_ddtree_tree
    mod.build_mixture_tree = build_mixture_tree
    mod.follow_verified_tree = ddtree_hf_ops.follow_verified_tree
    monkeypatch.setitem(sys.modules, "ddtree", mod)
    return mod


def test_tree_build_ext_check_equal(oracle_ddtree):
    import tree_build_ext

    tree_build_ext.check_equal(trials=60)


def test_tree_build_ext_check_equal_catches_a_wrong_builder(oracle_ddtree):
    """A stand-in whose mixture builder drops the last node makes check_equal fail."""
    import tree_build_ext

    good = oracle_ddtree.build_mixture_tree

    def short(logits, prior, budget):
        t, d, p, cm, vis, st = good(logits, prior, budget)
        return t[:-1], d[:-1], p[:-1], cm, vis, st

    oracle_ddtree.build_mixture_tree = short
    with pytest.raises(AssertionError):
        tree_build_ext.check_equal(trials=3)


def test_tree_logits_check_equal():
    import tree_logits

    tree_logits.check_equal()


def test_mode_attention_check_equal():
    import mode_attention

    mode_attention.check_equal()
