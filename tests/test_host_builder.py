"""The host tree builder (mfd_build_trees_host, through ddtree_sglang_ops.build_trees_cpu): CPU only, no GPU.

Bar: bit-exact trees (tokens, depths, parents, counts and the tail) against the golden trees written by the
reference's own compiled C++ builders (tests/golden/builder_golden.npz), against the C oracle on tie-heavy inputs,
and against the reference's compiled SGLang build_trees when oracle/_ref holds it.
"""

import os

import numpy as np
import pytest
import torch

from oracle import builder as B

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "builder_golden.npz")


def _host(lp, ids, prior, budget):
    import ddtree_sglang_ops

    bs = lp.shape[0]
    tree = torch.full((bs, 3, budget + 1), 7, dtype=torch.int64)
    counts = torch.full((bs,), -1, dtype=torch.int64)
    ddtree_sglang_ops.build_trees_cpu(top_log_probs=lp, top_ids=ids, log_prior=prior, bs=bs, budget=budget,
                                      tree=tree, counts=counts)
    return tree, counts


def test_golden_trees():
    z = np.load(GOLDEN, allow_pickle=False)
    kinds = set()
    for i in range(int(z["n"])):
        kind = str(z[f"c{i}_kind"])
        lp, ids, budget = z[f"c{i}_lp"], z[f"c{i}_ids"], int(z[f"c{i}_budget"])
        prior = z[f"c{i}_prior"] if kind == "mixture" else np.zeros(1, np.float32)  # single: [1, L, k] already
        tree, counts = _host(torch.from_numpy(lp)[None].float(), torch.from_numpy(ids)[None].to(torch.int32),
                             torch.from_numpy(prior)[None].float(), budget)
        assert int(counts[0]) == int(z[f"c{i}_count"]), f"case {i}"
        np.testing.assert_array_equal(tree[0].numpy(), z[f"c{i}_tree"], err_msg=f"case {i} ({kind})")
        kinds.add(kind)
    assert kinds == {"mixture", "single"}


def _inputs(seed, bs, K, L, V, k, coarse):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(bs, K, L, V, generator=g) * 3
    if coarse:  # many exact ties between candidates, modes and siblings
        logits = (logits * 2).round() / 2
    top, ids = torch.topk(logits, k=k, dim=-1)
    lp = (top - torch.logsumexp(logits, -1, keepdim=True)).float()
    prior = torch.log_softmax(torch.randn(bs, K, generator=g), -1)
    if coarse:
        prior = (prior * 4).round() / 4
    return lp, ids.to(torch.int32), prior


@pytest.mark.parametrize("K,L,V,k,budget,coarse", [
    (8, 15, 64, 16, 63, True), (8, 16, 200, 8, 64, False), (3, 7, 40, 40, 255, True), (16, 4, 12, 12, 300, True),
    (1, 15, 64, 16, 63, True), (1, 40, 30, 5, 200, True), (2, 1, 9, 9, 20, False), (4, 6, 30, 3, 0, False),
])
def test_against_the_oracle(K, L, V, k, budget, coarse):
    bs = 3
    lp, ids, prior = _inputs(K * 1000 + budget, bs, K, L, V, k, coarse)
    tree, counts = _host(lp, ids, prior, budget)
    for b in range(bs):
        if K == 1:
            t, d, p, n = B.build_single(lp[b, 0].numpy(), ids[b, 0].numpy(), budget)
        else:
            t, d, p, n, _ = B.build_mixture(lp[b].numpy(), ids[b].numpy(), prior[b].numpy(), budget)
        assert int(counts[b]) == n
        np.testing.assert_array_equal(tree[b].numpy(), np.stack([t, d, p]))
    ref = B.ref_sglang_builder()
    if ref is not None:  # the reference's own compiled build_trees (oracle/_ref), when it was built here
        rt = torch.empty(bs, 3, budget + 1, dtype=torch.long)
        rc = torch.empty(bs, dtype=torch.long)
        ref.build_trees(lp.contiguous(), ids.contiguous(), prior.contiguous(), bs, budget, rt, rc)
        assert torch.equal(rt, tree) and torch.equal(rc, counts)


def test_uniform_prior_and_partial_batch():
    """log_prior None = uniform (prior 0 for every mode); only the first bs rows are built, the rest untouched."""
    lp, ids, _ = _inputs(5, 4, 3, 5, 20, 6, True)
    import ddtree_sglang_ops

    tree = torch.full((4, 3, 33), 9, dtype=torch.int64)
    counts = torch.full((4,), 9, dtype=torch.int64)
    ddtree_sglang_ops.build_trees_cpu(top_log_probs=lp, top_ids=ids, log_prior=None, bs=2, budget=32, tree=tree,
                                      counts=counts)
    for b in range(2):
        t, d, p, n, _ = B.build_mixture(lp[b].numpy(), ids[b].numpy(), np.zeros(3, np.float32), 32)
        np.testing.assert_array_equal(tree[b].numpy(), np.stack([t, d, p]))
        assert int(counts[b]) == n
    assert (tree[2:] == 9).all() and (counts[2:] == 9).all()


def test_rejects_device_or_wrong_dtype_tensors():
    import ddtree_sglang_ops

    lp, ids, prior = _inputs(1, 1, 2, 3, 10, 4, False)
    tree = torch.empty(1, 3, 9, dtype=torch.int64)
    counts = torch.empty(1, dtype=torch.int64)
    with pytest.raises(TypeError):
        ddtree_sglang_ops.build_trees_cpu(top_log_probs=lp.double(), top_ids=ids, log_prior=prior, bs=1, budget=8,
                                          tree=tree, counts=counts)
    with pytest.raises(ValueError):
        ddtree_sglang_ops.build_trees_cpu(top_log_probs=lp, top_ids=ids, log_prior=prior, bs=1, budget=9, tree=tree,
                                          counts=counts)


def test_hf_host_builders_match_golden_and_oracle():
    """The HF host-tensor builders (build_mixture / build_single, inference/hf/tree_build_ext.py:118-234) on host
    inputs: the host heap, the golden trees' tokens / depths / parents / visibility, and the mixture heap for one
    mode (the HF mixture builder does not switch heaps)."""
    import tree_build_ext

    z = np.load(GOLDEN, allow_pickle=False)
    for i in range(int(z["n"])):
        kind = str(z[f"c{i}_kind"])
        lp, ids, budget, n = z[f"c{i}_lp"], z[f"c{i}_ids"], int(z[f"c{i}_budget"]), int(z[f"c{i}_count"])
        if kind == "mixture":
            tok, dep, par, tree, vis = tree_build_ext.build_mixture(torch.from_numpy(lp), torch.from_numpy(ids),
                                                                    torch.from_numpy(z[f"c{i}_prior"]), budget)
        else:
            tok, dep, par, tree, vis = tree_build_ext.build_single(torch.from_numpy(lp[0]), torch.from_numpy(ids[0]),
                                                                   budget)
        gt = z[f"c{i}_tree"]
        np.testing.assert_array_equal(tok.numpy(), gt[0, 1 : n + 1], err_msg=f"case {i}")
        np.testing.assert_array_equal(dep.numpy(), gt[1, 1 : n + 1], err_msg=f"case {i}")
        assert par == gt[2, : n + 1].tolist()
        gv = np.unpackbits(z[f"c{i}_vis"])[: (n + 1) ** 2].reshape(n + 1, n + 1)
        np.testing.assert_array_equal(vis.numpy().astype(np.uint8), gv, err_msg=f"case {i}")
    # one mode through the mixture builder: the mixture heap (prior added, float key), as the oracle's
    lp, ids, prior = _inputs(9, 1, 1, 12, 30, 6, True)
    tok, dep, par, _, _ = tree_build_ext.build_mixture(lp[0], ids[0].long(), prior[0], 40)
    t, d, p, n, _ = B.build_mixture(lp[0].numpy(), ids[0].numpy(), prior[0].numpy(), 40)
    np.testing.assert_array_equal(tok.numpy(), t[1 : n + 1])
    assert par == p[: n + 1].tolist()
