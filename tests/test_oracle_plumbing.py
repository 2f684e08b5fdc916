"""Pins of the verify-plumbing oracle (CPU).

verify_inputs' tree part equals the builder's ancestor-or-self visibility (inference/hf/tree_build_ext.py:101-110),
its prefix part is all ones, ids / positions follow their definitions; follow equals the HF Tree.follow walk over
the tree's child maps (inference/hf/tree_build_ext.py:70-83) on posteriors that plant a random path; kv_move
equals torch index_select compaction of the appended window (inference/hf/ddtree.py:398-404). Planted mistakes
(walk one step short, the lowest instead of the highest match, stores before loads) fail.
"""

import numpy as np
import pytest
import torch

from oracle import builder as B
from oracle import plumbing as P


def random_trees(seed, bs, K=4, L=6, k=4, budget=30):
    rng = np.random.default_rng(seed)
    trees = []
    for _ in range(bs):
        lp = np.sort(np.log(rng.dirichlet(np.ones(16), size=(K, L)))[..., :k], axis=-1)[..., ::-1].astype(np.float32)
        ids = np.stack([[rng.permutation(16)[:k] for _ in range(L)] for _ in range(K)]).astype(np.int64) + 100
        t, d, p, n, _ = B.build_mixture(lp, ids, np.zeros(K, np.float32), budget)
        trees.append((t, d, p, n))
    return trees


def test_verify_inputs_tree_part_is_the_builder_visibility():
    trees = random_trees(0, 3)
    W = 31
    tok = np.stack([t for t, _, _, _ in trees])
    dep = np.stack([d for _, d, _, _ in trees])
    par = np.stack([p for _, _, p, _ in trees])
    prefix = np.array([5, 0, 17])
    root = np.array([7, 8, 9])
    ids, pos, masks = P.verify_inputs(root, prefix, tok, dep, par, max_depth=6)
    for b, (t, d, p, n) in enumerate(trees):
        m = masks[b]
        assert m[:, : prefix[b]].all()
        vis = B.visibility(p, n)
        np.testing.assert_array_equal(m[: n + 1, prefix[b] : prefix[b] + n + 1], vis)
        assert ids[b, 0] == root[b] and np.array_equal(ids[b, 1:], t[1:])
        np.testing.assert_array_equal(pos[b], prefix[b] + d)
    # planted: a walk one step short misses the root for the deepest nodes
    _, _, short = P.verify_inputs(root, prefix, tok, dep, par, max_depth=int(dep.max()) - 1)
    assert any(not np.array_equal(a, b) for a, b in zip(short, masks))


def child_maps_of(tokens, parents, n):
    maps = [dict() for _ in range(n + 1)]
    for i in range(1, n + 1):
        maps[int(parents[i])][int(tokens[i])] = i
    return maps


def hf_follow(maps, post):
    accepted, cur = [0], 0
    nxt = int(post[0])
    while nxt in maps[cur]:
        cur = maps[cur][nxt]
        accepted.append(cur)
        nxt = int(post[cur])
    return accepted, nxt


@pytest.mark.parametrize("seed", range(4))
def test_follow_equals_hf_tree_walk(seed):
    rng = np.random.default_rng(seed)
    trees = random_trees(seed + 10, 4)
    W, L = 31, 8
    bs = len(trees)
    verify_ids = np.zeros((bs, W), np.int64)
    parents = np.full((bs, W), -1, np.int64)
    post = rng.integers(100, 116, size=(bs, W))
    window = rng.permutation(10_000)[: bs * W].reshape(bs, W)
    prefix = rng.integers(0, 100, size=bs)
    for b, (t, d, p, n) in enumerate(trees):
        verify_ids[b] = t
        verify_ids[b, 0] = 1
        parents[b] = p
        # plant a path: follow random children for a random number of steps
        maps = child_maps_of(t, p, n)
        cur = 0
        for _ in range(int(rng.integers(0, 7))):
            if not maps[cur]:
                break
            tok = int(rng.choice(list(maps[cur])))
            post[b, cur] = tok
            cur = maps[cur][tok]
    out = P.follow(post, verify_ids, parents, window, prefix, L)
    for b, (t, d, p, n) in enumerate(trees):
        acc, bonus = hf_follow(child_maps_of(t, p, n), post[b])
        acc = acc[:L]
        nacc = len(acc) - 1
        assert out["accept_len"][b] == nacc and out["commit_lens"][b] == nacc + 1
        assert out["bonus"][b] == int(post[b, acc[-1]])
        if len(acc) < L:
            assert out["bonus"][b] == bonus
        np.testing.assert_array_equal(out["hidden_index"][b, : nacc + 1], b * W + np.array(acc))
        np.testing.assert_array_equal(out["move_src"][b, : nacc + 1], window[b, acc])
        np.testing.assert_array_equal(out["move_tgt"][b, : nacc + 1], window[b, : nacc + 1])
        np.testing.assert_array_equal(out["out_tokens"][b, :nacc], [post[b, a] for a in acc[:-1]])
        assert out["new_seq_lens"][b] == prefix[b] + nacc + 1


def test_kv_move_equals_index_select_compaction():
    rng = np.random.default_rng(3)
    past, cur, H, D = 10, 12, 3, 8
    keep = np.array([0, 2, 3, 7, 11])
    cache = rng.standard_normal((H, past + cur, D))
    ref = torch.from_numpy(cache.copy())
    kept = ref.narrow(-2, past, cur).index_select(-2, torch.from_numpy(keep))
    ref.narrow(-2, past, len(keep)).copy_(kept)
    # the oracle works on [slots, ...] rows: positions are the rows of each head plane
    planes = [cache[h] for h in range(H)]
    src = (keep + past)[None]
    tgt = (np.arange(len(keep)) + past)[None]
    P.kv_move(planes, src, tgt)
    np.testing.assert_array_equal(np.stack(planes), ref.numpy())
    # planted: storing each move before reading the next source breaks when a target is a later source
    bad = [cache[h].copy() for h in range(H)]
    for s, t in zip(src[0], tgt[0]):
        for pl in bad:
            pl[t] = pl[s]
    chain_src = np.array([[12, 13]]); chain_tgt = np.array([[13, 14]])
    x = [np.arange(20.0)[:, None].repeat(2, 1)]
    y = [a.copy() for a in x]
    P.kv_move(x, chain_src, chain_tgt)
    for s, t in zip(chain_src[0], chain_tgt[0]):
        y[0][t] = y[0][s]
    assert not np.array_equal(x[0], y[0])


def test_hf_verify_inputs_rounds_leave_only_the_live_tree_masked():
    """Two decode rounds in the same persistent buffers: after round 2 the rows of its tree see every prefix
    column (round 1's block was cleared) and, in their own block, exactly the builder's visibility. A planted
    mistake (the previous block not cleared) leaves blocked entries inside the prefix."""
    trees = random_trees(3, 2)
    mmin = -3.0e38
    rows, cols = 40, 120
    mask = np.zeros((rows, cols))
    ids = np.zeros(64, np.int64)
    pos = np.zeros(64, np.int64)
    vbuf = np.zeros((64, 64), bool)
    past, prev = 10, (0, 0)
    for t, d, p, n in trees:
        vis = B.visibility(p, n)
        n1 = P.hf_verify_inputs(mask, ids, pos, vbuf, 5, past, t[1:n + 1], d[1:n + 1], vis, past, *prev, mmin)
        assert n1 == n + 1
        np.testing.assert_array_equal(mask[:n1, :past], 0)
        np.testing.assert_array_equal(mask[:n1, past:past + n1] == 0, vis)
        np.testing.assert_array_equal(pos[:n1], past + d[:n + 1])
        assert ids[0] == 5 and np.array_equal(ids[1:n1], t[1:n + 1])
        prev = (past, n1)
        past += 3  # three nodes accepted
    # planted: skipping the clear keeps round 1's blocked entries inside round 2's prefix
    t, d, p, n = trees[0]
    stale = np.zeros((rows, cols))
    P.hf_verify_inputs(stale, ids, pos, vbuf, 5, 10, t[1:n + 1], d[1:n + 1], B.visibility(p, n), 10, 0, 0, mmin)
    t2, d2, p2, n2 = trees[1]
    P.hf_verify_inputs(stale, ids, pos, vbuf, 5, 13, t2[1:n2 + 1], d2[1:n2 + 1], B.visibility(p2, n2), 13, 0, 0, mmin)
    assert (stale[:n2 + 1, :13] != 0).any()


def test_draft_prepare_matches_torch_gathers():
    """Window slots = torch gather of req_to_token rows at [prefix, prefix + W); ids = bonus then the mask token;
    positions = prefix + arange (P:1572-1588)."""
    g = torch.Generator().manual_seed(5)
    r2t = torch.randint(0, 10 ** 6, (9, 300), generator=g)
    bs, L, W = 4, 16, 40
    prefix = torch.tensor([0, 17, 250, 3])
    pool = torch.tensor([8, 0, 3, 3])
    bonus = torch.randint(0, 1000, (bs,), generator=g)
    ids, pos, win = P.draft_prepare(bonus.numpy(), prefix.numpy(), pool.numpy(), r2t.numpy(), 99, L, W)
    cols = prefix[:, None] + torch.arange(W)[None, :]
    want_win = torch.gather(r2t.index_select(0, pool), 1, cols)
    assert np.array_equal(win, want_win.numpy())
    want_ids = torch.full((bs, L), 99)
    want_ids[:, 0] = bonus
    assert np.array_equal(ids, want_ids.numpy())
    assert np.array_equal(pos, (prefix[:, None] + torch.arange(L)).numpy())


def test_mode_mask_is_the_attention_block_mask():
    """Each request's rows reshape to the visibility of the attention oracle's block mask (context visible, own
    mode block only), the semantics definition of inference/hf/mode_attention.py:158-160."""
    from oracle import attention as A

    K, L = 3, 5
    prefix = np.array([7, 0, 33])
    sizes = [K * L * (p + K * L) for p in prefix]
    offsets = np.concatenate([[0], np.cumsum(sizes)[:-1]]) + np.array([0, 4, 9])  # gaps between requests
    total = int(offsets[-1] + sizes[-1] + 3)
    m = P.mode_mask(prefix, offsets, total, K, L)
    covered = np.zeros(total, bool)
    for b, p in enumerate(prefix):
        rows = m[offsets[b] : offsets[b] + sizes[b]].reshape(K * L, p + K * L)
        assert np.array_equal(rows.astype(bool), np.isfinite(A.block_mask(K, L, int(p))))
        covered[offsets[b] : offsets[b] + sizes[b]] = True
    assert not m[~covered].any()


def test_mode_mask_planted_mistake_fails():
    """A mask that lets a row see the next mode's block differs from the attention oracle's."""
    from oracle import attention as A

    K, L, p = 2, 4, 3
    m = P.mode_mask([p], [0], K * L * (p + K * L), K, L).reshape(K * L, p + K * L)
    bad = m.copy()
    bad[0, p + L] = 1
    assert np.array_equal(m.astype(bool), np.isfinite(A.block_mask(K, L, p)))
    assert not np.array_equal(bad.astype(bool), np.isfinite(A.block_mask(K, L, p)))
