"""GPU parity of the verify-side plumbing (through the C ABI): verify inputs, the accept walk and the KV moves
bit-exact against the oracle (tests/test_oracle_plumbing.py pins it); the HF compaction of a transformers
DynamicCache equals the reference's index_select compaction."""

import numpy as np
import pytest
import torch

from oracle import builder as B
from oracle import plumbing as P

pytestmark = pytest.mark.gpu


def batch_of_trees(seed, bs, K=8, L=15, k=8, budget=63, V=64):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(bs, K, L, V, generator=g) * 3
    lp = torch.log_softmax(logits, -1)
    top, ids = torch.topk(lp, k, dim=-1)
    tree = np.zeros((bs, 3, budget + 1), np.int64)
    counts = []
    for b in range(bs):
        t, d, p, n, _ = B.build_mixture(top[b].numpy(), ids[b].numpy(), np.zeros(K, np.float32), budget)
        tree[b] = np.stack([t, d, p])
        counts.append(n)
    return tree, counts


def test_verify_inputs_match_oracle():
    import ddtree_sglang_ops

    bs, W, L = 5, 64, 15
    tree, _ = batch_of_trees(1, bs, L=L, budget=W - 1)
    rng = np.random.default_rng(1)
    prefix = np.array([0, 1, 17, 250, 4099])
    root = rng.integers(0, 1000, size=bs)
    offs = np.concatenate([[0], np.cumsum([W * (p + W) for p in prefix])[:-1]]) + 3  # odd offsets: unaligned rows
    total = int(sum(W * (p + W) for p in prefix)) + 3
    print(f"case: verify inputs bs={bs} W={W} prefixes={prefix.tolist()}", flush=True)
    tt = torch.from_numpy(tree).cuda()
    ids = torch.empty(bs, W, dtype=torch.long, device="cuda")
    pos = torch.empty(bs, W, dtype=torch.long, device="cuda")
    mask = torch.full((total,), True, dtype=torch.bool, device="cuda")
    ddtree_sglang_ops.ddtree_verify_inputs(root_tokens=torch.from_numpy(root).cuda(), prefix_lens=torch.from_numpy(prefix).cuda(),
                                      tokens=tt[:, 0], depths=tt[:, 1], parents=tt[:, 2],
                                      mask_offsets=torch.from_numpy(offs).cuda(), ids_out=ids, positions_out=pos,
                                      mask_out=mask, max_depth=L)
    torch.cuda.synchronize()
    rid, rpos, rmasks = P.verify_inputs(root, prefix, tree[:, 0], tree[:, 1], tree[:, 2], L)
    np.testing.assert_array_equal(ids.cpu().numpy(), rid)
    np.testing.assert_array_equal(pos.cpu().numpy(), rpos)
    m = mask.cpu().numpy().astype(np.uint8)
    for b in range(bs):
        np.testing.assert_array_equal(m[offs[b]: offs[b] + rmasks[b].size].reshape(rmasks[b].shape), rmasks[b],
                                      err_msg=f"request {b}")
    assert m[:3].all()  # bytes before the first row untouched


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_follow_matches_oracle(seed):
    import ddtree_sglang_ops

    bs, W, L = 6, 64, 16
    tree, counts = batch_of_trees(seed + 5, bs, L=15, budget=W - 1)
    rng = np.random.default_rng(seed)
    verify_ids = tree[:, 0].copy()
    verify_ids[:, 0] = rng.integers(0, 64, size=bs)
    post = rng.integers(0, 64, size=(bs, W))
    for b in range(bs):  # plant a path of random length
        maps = [dict() for _ in range(W)]
        for i in range(1, counts[b] + 1):
            maps[int(tree[b, 2, i])][int(tree[b, 0, i])] = i
        cur = 0
        for _ in range(int(rng.integers(0, 16))):
            if not maps[cur]:
                break
            tok = int(rng.choice(list(maps[cur])))
            post[b, cur] = tok
            cur = maps[cur][tok]
    window = rng.permutation(100_000)[: bs * W].reshape(bs, W)
    prefix = rng.integers(0, 5000, size=bs)
    print(f"case: follow seed={seed}", flush=True)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    tt = d(tree)
    out = dict(accept_len=torch.empty(bs, dtype=torch.int32, device="cuda"),
               commit_lens=torch.empty(bs, dtype=torch.int32, device="cuda"),
               bonus=torch.empty(bs, dtype=torch.long, device="cuda"),
               out_tokens=torch.empty(bs, L, dtype=torch.long, device="cuda"),
               new_seq_lens=torch.empty(bs, dtype=torch.long, device="cuda"),
               move_src=torch.empty(bs, L, dtype=torch.long, device="cuda"),
               move_tgt=torch.empty(bs, L, dtype=torch.long, device="cuda"),
               hidden_index=torch.empty(bs, L, dtype=torch.long, device="cuda"))
    ddtree_sglang_ops.ddtree_follow(posterior=d(post), verify_ids=d(verify_ids), parents=tt[:, 2], window=d(window),
                               prefix_lens=d(prefix), accept_len_out=out["accept_len"],
                               commit_lens_out=out["commit_lens"], bonus_out=out["bonus"],
                               out_tokens_out=out["out_tokens"], new_seq_lens_out=out["new_seq_lens"],
                               move_src_out=out["move_src"], move_tgt_out=out["move_tgt"],
                               hidden_index_out=out["hidden_index"])
    torch.cuda.synchronize()
    ref = P.follow(post, verify_ids, tree[:, 2], window, prefix, L)
    for key, val in out.items():
        np.testing.assert_array_equal(val.cpu().numpy().astype(np.int64), ref[key], err_msg=key)


def test_kv_compactor_matches_oracle():
    import ddtree_sglang_ops

    g = torch.Generator().manual_seed(4)
    slots, Hkv, D, nlayers, bs, L = 4096, 8, 128, 3, 4, 16
    bufs = [torch.randn(slots, Hkv, D, generator=g).to(torch.bfloat16) for _ in range(2 * nlayers)]
    rng = np.random.default_rng(4)
    src = np.zeros((bs, L), np.int64)
    tgt = np.zeros((bs, L), np.int64)
    for b in range(bs):
        win = rng.permutation(slots)[:L]
        n = int(rng.integers(0, L))
        path = np.sort(rng.choice(np.arange(1, L), size=n, replace=False)) if n else np.zeros(0, np.int64)
        path = np.concatenate([[0], path])
        src[b, : n + 1] = win[path]
        tgt[b, : n + 1] = win[: n + 1]
    dev = [t.cuda() for t in bufs]
    ptrs = torch.tensor([t.data_ptr() for t in dev], dtype=torch.int64).cuda()
    comp = ddtree_sglang_ops.DDTreeKVCompactor(data_ptrs=ptrs, slot_bytes=Hkv * D * 2, num_slots=slots)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    comp(move_src=torch.from_numpy(src).cuda(), move_tgt=torch.from_numpy(tgt).cuda(), err_flag=err)
    torch.cuda.synchronize()
    assert int(err) == 0
    ref = P.kv_move([t.view(torch.int16).numpy().copy() for t in bufs], src, tgt)
    for got, want in zip(dev, ref):
        np.testing.assert_array_equal(got.cpu().view(torch.int16).numpy(), want)


def test_compact_dynamic_cache_matches_index_select():
    """inference/hf/ddtree.py:389-436 on a transformers DynamicCache: keep rows past + keep[m] at past + m."""
    import ddtree_hf_ops
    from transformers import DynamicCache

    g = torch.Generator().manual_seed(8)
    past, cur, H, D, nl = 37, 20, 4, 128, 3
    keep = [0, 1, 4, 5, 9, 13, 19]
    cache = DynamicCache()
    ref = []
    for l in range(nl):
        k = torch.randn(1, H, past + cur, D, generator=g).to(torch.bfloat16)
        v = torch.randn(1, H, past + cur, D, generator=g).to(torch.bfloat16)
        cache.update(k.cuda(), v.cuda(), l)
        kk, vv = k.clone(), v.clone()
        for t in (kk, vv):
            kept = t.narrow(-2, past, cur).index_select(-2, torch.tensor(keep))
            t.narrow(-2, past, len(keep)).copy_(kept)
        ref.append((kk[:, :, : past + len(keep)], vv[:, :, : past + len(keep)]))
    ddtree_hf_ops.compact_dynamic_cache(cache, past, keep)
    torch.cuda.synchronize()
    for l in range(nl):
        layer = cache.layers[l]
        assert layer.keys.shape[-2] == past + len(keep)
        assert torch.equal(layer.keys.cpu(), ref[l][0]) and torch.equal(layer.values.cpu(), ref[l][1])


@pytest.mark.parametrize("mask_dtype", [torch.bfloat16, torch.float32])
def test_hf_compile_ddtree_tree_rounds_match_oracle(mask_dtype):
    """compile_ddtree_tree (inference/hf/ddtree.py:317-357) over three decode rounds in the same persistent
    buffers, host-tensor inputs as the HF builder returns them, bit-exact against the oracle: ids, positions,
    the visibility copy and the whole mask buffer (the previous round's block cleared, nothing else touched)."""
    import ddtree_hf_ops

    tree, counts = batch_of_trees(7, 3, budget=40)
    rows, cols = 48, 200
    dev = torch.device("cuda")
    mask = torch.zeros(1, 1, rows, cols, dtype=mask_dtype, device=dev)
    ids = torch.zeros(1, 64, dtype=torch.int64, device=dev)
    pos = torch.zeros(1, 64, dtype=torch.int64, device=dev)
    vbuf = torch.zeros(64, 64, dtype=torch.bool, device=dev)
    m_ref = np.zeros((rows, cols), np.float64)
    ids_ref = np.zeros(64, np.int64)
    pos_ref = np.zeros(64, np.int64)
    vb_ref = np.zeros((64, 64), bool)
    mmin = float(torch.finfo(mask_dtype).min)
    past, prev = 20, (0, 0)
    for r in range(3):
        n = counts[r]
        tok = torch.from_numpy(tree[r, 0, 1:n + 1].copy())
        dep = torch.from_numpy(tree[r, 1, 1:n + 1].copy())
        vis = torch.from_numpy(B.visibility(tree[r, 2], n))
        root = torch.tensor(1000 + r, device=dev)
        print(f"case: hf compile round {r} n={n} past={past} {mask_dtype}", flush=True)
        out = ddtree_hf_ops.compile_ddtree_tree(root, past, tok, dep, vis, past, mask_dtype, dev, ids, pos, mask, vbuf, *prev)
        P.hf_verify_inputs(m_ref, ids_ref, pos_ref, vb_ref, 1000 + r, past, tok.numpy(), dep.numpy(), vis.numpy(),
                           past, *prev, mmin)
        torch.cuda.synchronize()
        v_ids, v_pos, v_mask, pl, n1 = out
        assert pl == past and n1 == n + 1 and v_mask.shape == (1, 1, n + 1, past + n + 1)
        np.testing.assert_array_equal(ids[0].cpu().numpy(), ids_ref)
        np.testing.assert_array_equal(pos[0].cpu().numpy(), pos_ref)
        np.testing.assert_array_equal(vbuf.cpu().numpy(), vb_ref)
        np.testing.assert_array_equal(mask[0, 0].float().cpu().numpy(), m_ref.astype(np.float32))
        prev = (past, n + 1)
        past += 1 + r  # accepted nodes of this round


def test_hf_compile_rejects_a_block_outside_the_buffer():
    import ddtree_hf_ops
    import mfd_hip

    dev = torch.device("cuda")
    mask = torch.zeros(1, 1, 8, 30, dtype=torch.bfloat16, device=dev)
    ids = torch.zeros(1, 64, dtype=torch.int64, device=dev)
    vbuf = torch.zeros(64, 64, dtype=torch.bool, device=dev)
    tok = torch.arange(5)
    vis = torch.from_numpy(B.visibility(np.array([-1, 0, 1, 1, 0, 4]), 5))
    with pytest.raises(mfd_hip.MFDError):
        ddtree_hf_ops.compile_ddtree_tree(1, 0, tok, tok, vis, 26, torch.bfloat16, dev, ids, ids.clone(), mask, vbuf, 0, 0)


def test_hf_follow_verified_tree_matches_oracle():
    """follow_verified_tree over a Tree and over plain child-map dicts (inference/hf/ddtree.py:367-382) against the
    oracle walk, on posteriors that plant random accepted paths."""
    import ddtree_hf_ops
    import tree_build_ext

    tree, counts = batch_of_trees(11, 4, budget=50)
    rng = np.random.default_rng(11)
    for b in range(4):
        n = counts[b]
        tok, par = tree[b, 0, :n + 1], tree[b, 2, :n + 1]
        maps = [dict() for _ in range(n + 1)]
        for i in range(1, n + 1):
            maps[int(par[i])][int(tok[i])] = i
        for _ in range(5):
            post = rng.integers(0, 64, size=n + 1)
            cur = 0  # plant a path: follow random children for a few steps
            for _ in range(rng.integers(0, 6)):
                if not maps[cur]:
                    break
                t, c = list(maps[cur].items())[rng.integers(0, len(maps[cur]))]
                post[cur] = t
                cur = c
            ref = P.follow(post[None], np.concatenate([[0], tok[1:]])[None], par[None], np.arange(n + 1)[None],
                           np.zeros(1, np.int64), 64)
            path_ref = [int(x) for x in ref["hidden_index"][0, :int(ref["accept_len"][0]) + 1]]
            post_t = torch.from_numpy(post)[None].cuda()
            for cm in (maps, tree_build_ext.Tree(tok[1:].tolist(), par.tolist())):
                path, nxt = ddtree_hf_ops.follow_verified_tree(cm, post_t)
                assert path == path_ref and nxt == int(ref["bonus"][0])


@pytest.mark.parametrize("wide", [0, 15, 5])
def test_draft_prepare_matches_oracle(wide):
    """ddtree_prepare (P:1590-1623) bit-exact against the oracle, int32 / int64 index inputs mixed by ``wide``."""
    import ddtree_sglang_ops

    g = torch.Generator().manual_seed(40 + wide)
    bs, L, W, cols = 5, 16, 64, 5000
    r2t = torch.randint(0, 2 ** 31 - 1, (11, cols), generator=g)
    prefix = torch.tensor([0, 1, 4000, 4936, 77])
    pool = torch.tensor([10, 0, 3, 3, 7])
    bonus = torch.randint(0, 151936, (bs,), generator=g)
    ins = [bonus, prefix, pool, r2t]
    dev = [(t.to(torch.int64) if wide >> i & 1 else t.to(torch.int32)).cuda() for i, t in enumerate(ins)]
    ids = torch.full((bs, L), -5, dtype=torch.int64, device="cuda")
    pos, win = torch.full_like(ids, -5), torch.full((bs, W), -5, dtype=torch.int64, device="cuda")
    ddtree_sglang_ops.ddtree_prepare(bonus_tokens=dev[0], prefix_lens=dev[1], req_pool_indices=dev[2],
                                     req_to_token=dev[3], block_ids_out=ids, positions_out=pos, window_out=win,
                                     mask_token_id=151669)
    want = P.draft_prepare(bonus.numpy(), prefix.numpy(), pool.numpy(), r2t.numpy(), 151669, L, W)
    for got, ref in zip((ids, pos, win), want):
        assert np.array_equal(got.cpu().numpy(), ref)


def test_mode_mask_matches_oracle():
    """ddtree_mode_mask (P:1914-1935) bit-exact against the oracle, with gaps between requests left untouched."""
    import ddtree_sglang_ops

    K, L = 8, 16
    prefix = np.array([1, 0, 4099, 17, 2048])
    sizes = [K * L * (int(p) + K * L) for p in prefix]
    offsets = np.concatenate([[0], np.cumsum(sizes)[:-1]]) + np.arange(len(prefix)) * 3
    total = int(offsets[-1] + sizes[-1] + 5)
    mask = torch.zeros(total, dtype=torch.bool, device="cuda")
    ddtree_sglang_ops.ddtree_mode_mask(prefix_lens=torch.from_numpy(prefix).cuda(),
                                       mask_offsets=torch.from_numpy(offsets).cuda(), mask_out=mask, num_modes=K,
                                       block_size=L)
    want = P.mode_mask(prefix, offsets, total, K, L)
    assert np.array_equal(mask.cpu().numpy().astype(np.uint8), want)
