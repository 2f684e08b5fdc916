"""CPU oracle of the verify-side plumbing of a tree round. TEST INFRASTRUCTURE ONLY.

Plain-loop restatements of the reference's device kernels in the SGLang patch
(inference/sglang/patches/sglang-v0.5.22-mfd.patch, "P" below):
  * ``verify_inputs`` — _ddtree_verify_inputs_kernel (P:1625-1667): flat mask rows [prefix ones | ancestor
    bits], verify ids and positions;
  * ``follow`` — _ddtree_follow_kernel (P:1706-1766): the accept walk, bonus, commit moves, hidden rows;
  * ``kv_move`` — _ddtree_compact_kv_kernel (P:1769-1793): every move's source read before any target written;
  * ``hf_verify_inputs`` — the HF compile_ddtree_tree (inference/hf/ddtree.py:317-357): one tree's ids,
    positions and additive mask block in persistent buffers, the previous round's block cleared first;
  * ``draft_prepare`` — _ddtree_prepare_kernel (P:1557-1588): draft block ids / positions and the verify
    window's cache slots read from req_to_token;
  * ``mode_mask`` — _ddtree_mode_mask_kernel (P:1889-1912): the multi-mode draft mask rows.
They are pinned (tests/test_oracle_plumbing.py) against the builder's visibility matrix, the HF Tree.follow
walk over child maps, torch index_select compaction, torch gathers of req_to_token, and the attention
oracle's block mask (the semantics definition of inference/hf/mode_attention.py:158-160).
"""

from __future__ import annotations

import numpy as np


def verify_inputs(root, prefix, tokens, depths, parents, max_depth):
    """root [bs], prefix [bs], tokens/depths/parents [bs, W] -> ids [bs, W], positions [bs, W], and the mask
    rows of each request as a list of [W, prefix + W] uint8 arrays."""
    bs, W = tokens.shape
    ids = np.zeros((bs, W), np.int64)
    pos = np.zeros((bs, W), np.int64)
    masks = []
    for b in range(bs):
        P = int(prefix[b])
        m = np.zeros((W, P + W), np.uint8)
        m[:, :P] = 1
        for i in range(W):
            anc = i
            for _ in range(max_depth + 1):
                if anc >= 0:
                    m[i, P + anc] = 1
                nxt = int(parents[b, max(anc, 0)])
                anc = nxt if anc > 0 else -1
            ids[b, i] = root[b] if i == 0 else tokens[b, i]
            pos[b, i] = P + depths[b, i]
        masks.append(m)
    return ids, pos, masks


def follow(posterior, verify_ids, parents, window, prefix, L):
    """posterior / verify_ids / window [bs, W], parents [bs, W], prefix [bs] -> dict of the commit outputs."""
    bs, W = verify_ids.shape
    out = {k: np.zeros((bs, L), np.int64) for k in ("out_tokens", "move_src", "move_tgt", "hidden_index")}
    out.update(accept_len=np.zeros(bs, np.int64), commit_lens=np.zeros(bs, np.int64), bonus=np.zeros(bs, np.int64),
               new_seq_lens=np.zeros(bs, np.int64))
    for b in range(bs):
        path, emitted = [0], []
        cur = 0
        for _ in range(L - 1):
            t = int(posterior[b, cur])
            kids = [c for c in range(W) if parents[b, c] == cur and verify_ids[b, c] == t]
            if not kids:
                break
            emitted.append(t)
            cur = max(kids)
            path.append(cur)
        n = len(path) - 1
        bonus = int(posterior[b, cur])
        emitted.append(bonus)
        for j in range(L):
            live = j <= n
            out["out_tokens"][b, j] = emitted[j] if live else 0
            p = path[j] if live else 0
            out["hidden_index"][b, j] = b * W + p
            out["move_src"][b, j] = window[b, p] if live else 0
            out["move_tgt"][b, j] = window[b, j] if live else 0
        out["accept_len"][b], out["commit_lens"][b], out["bonus"][b] = n, n + 1, bonus
        out["new_seq_lens"][b] = int(prefix[b]) + n + 1
    return out


def kv_move(buffers, move_src, move_tgt):
    """buffers: list of [slots, ...] arrays, modified in place: per request, every source row is read first,
    then the rows whose source differs from their target are written."""
    for buf in buffers:
        for b in range(move_src.shape[0]):
            rows = {int(t): buf[int(s)].copy() for s, t in zip(move_src[b], move_tgt[b]) if s != t}
            for t, v in rows.items():
                buf[t] = v
    return buffers


def hf_verify_inputs(mask, ids, pos, vis_buf, root, start, tokens, depths, vis, past, prev_start, prev_len, mask_min):
    """In place on numpy buffers (mask [rows, cols] float, ids / pos [max] int64, vis_buf [max, max] bool), as
    inference/hf/ddtree.py:317-357: clear the previous tree block, then write the n + 1 ids and positions, the
    visibility and the tree block (0 where visible, mask_min elsewhere) at columns past .. past + n."""
    n1 = 1 + len(tokens)
    if prev_len > 0:
        mask[:prev_len, prev_start:prev_start + prev_len] = 0
    ids[0] = root
    ids[1:n1] = tokens
    pos[0] = start
    pos[1:n1] = start + np.asarray(depths)
    vis_buf[:n1, :n1] = vis
    mask[:n1, past:past + n1] = np.where(vis, 0.0, mask_min)
    return n1


def draft_prepare(bonus, prefix, req_pool, req_to_token, mask_token, L, W):
    """bonus, prefix, req_pool [bs]; req_to_token [rows, cols] -> block ids [bs, L], positions [bs, L],
    window [bs, W] (int64), as P:1572-1588 writes them."""
    bs = len(bonus)
    ids = np.zeros((bs, L), np.int64)
    pos = np.zeros((bs, L), np.int64)
    win = np.zeros((bs, W), np.int64)
    for b in range(bs):
        for l in range(L):
            ids[b, l] = int(bonus[b]) if l == 0 else int(mask_token)
            pos[b, l] = int(prefix[b]) + l
        for w in range(W):
            win[b, w] = int(req_to_token[int(req_pool[b]), int(prefix[b]) + w])
    return ids, pos, win


def mode_mask(prefix, mask_offsets, total, num_modes, block_size):
    """Flat bool mask of ``total`` bytes with the rows of P:1900-1912: request b, row r < K L at
    mask_offsets[b] + r (prefix + K L) = [prefix ones | columns of r's own mode block]. Bytes outside the rows
    stay 0."""
    KL = num_modes * block_size
    out = np.zeros(total, np.uint8)
    for b in range(len(prefix)):
        P = int(prefix[b])
        for r in range(KL):
            row = int(mask_offsets[b]) + r * (P + KL)
            out[row : row + P] = 1
            for c in range(KL):
                out[row + P + c] = 1 if c // block_size == r // block_size else 0
    return out
