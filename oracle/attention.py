"""CPU oracle of K-mode drafter attention ("mode attention"). TEST INFRASTRUCTURE ONLY.

Restates the reference's semantics definitions, inference/hf/mode_attention.py:153-164
(``reference``) and the SGLang patch's ``paged_mode_block_attention_reference``
(inference/sglang/patches/sglang-v0.5.22-mfd.patch:965-988), as an explicit masked softmax in
float64 numpy:

  * each query row of mode m sees every context key, plus the ``block_size`` keys of its own
    mode block and none of the other modes' blocks (mask -inf on the block columns where
    mode(row) != mode(col); inference/hf/mode_attention.py:158-160);
  * GQA: query head h reads KV head h // (H / Hkv) (``repeat_interleave``, :161-162);
  * ``causal_in_block=True`` additionally masks block key t' > t within the own block. The
    reference is bidirectional inside the block; this switch only serves the causal variant
    named by the benchmark configuration and is never the default.
"""

from __future__ import annotations

import numpy as np

F64 = np.float64


def _softmax_attend(qh, kh, vh, mask_add, scaling):
    """qh [M, D], kh/vh [N, D], mask_add [M, N] (0 or -inf) -> [M, D] float64."""
    s = (qh @ kh.T) * scaling + mask_add
    m = np.max(s, axis=1, keepdims=True)
    p = np.exp(s - m)
    return (p @ vh) / np.sum(p, axis=1, keepdims=True)


def block_mask(num_modes, block_size, ctx, causal_in_block=False):
    KL = num_modes * block_size
    mask = np.zeros((KL, ctx + KL), dtype=F64)
    mode = np.arange(KL) // block_size
    blk = np.where(mode[:, None] != mode[None, :], -np.inf, 0.0)
    if causal_in_block:
        t = np.arange(KL) % block_size
        blk = np.where(t[None, :] > t[:, None], -np.inf, blk)
    mask[:, ctx:] = blk
    return mask


def mode_attention(q, k, v, num_modes, block_size, scaling, causal_in_block=False):
    """Flat layout of inference/hf/mode_attention.py:123-124: q [1, H, K*bs, D];
    k, v [1, Hkv, ctx + K*bs, D] (block keys last). Returns [1, K*bs, H, D] float64."""
    q, k, v = (np.asarray(x, dtype=F64) for x in (q, k, v))
    _, H, KL, D = q.shape
    Hkv = k.shape[1]
    ctx = k.shape[2] - KL
    G = H // Hkv
    mask = block_mask(num_modes, block_size, ctx, causal_in_block)
    out = np.zeros((1, KL, H, D), dtype=F64)
    for h in range(H):
        out[0, :, h] = _softmax_attend(q[0, h], k[0, h // G], v[0, h // G], mask, scaling)
    return out


def paged_mode_attention(q, k_new, v_new, k_cache, v_cache, token_slots, num_modes, block_size, scaling,
                         causal_in_block=False):
    """Paged layout of the SGLang patch (P:917-919): q [T, H, D], k_new/v_new [T, Hkv, D] mode-major
    per request; caches [slots, Hkv, D]; ``token_slots[b]`` = the context's slot ids of request b
    (already resolved from a per-token table or from pages). Returns [T, H, D] float64."""
    q, k_new, v_new = (np.asarray(x, dtype=F64) for x in (q, k_new, v_new))
    k_cache = np.asarray(k_cache, dtype=F64)
    v_cache = np.asarray(v_cache, dtype=F64)
    T, H, D = q.shape
    Hkv = k_new.shape[1]
    G = H // Hkv
    KL = num_modes * block_size
    out = np.zeros((T, H, D), dtype=F64)
    for b in range(T // KL):
        slots = np.asarray(token_slots[b], dtype=np.int64)
        ctx = len(slots)
        rows = slice(b * KL, (b + 1) * KL)
        kk = np.concatenate([k_cache[slots], k_new[rows]], 0)
        vv = np.concatenate([v_cache[slots], v_new[rows]], 0)
        mask = block_mask(num_modes, block_size, ctx, causal_in_block)
        for h in range(H):
            out[rows, h] = _softmax_attend(q[rows, h], kk[:, h // G], vv[:, h // G], mask, scaling)
    return out


def slots_from_req_to_token(req_to_token, req_pool_indices, ctx_lens):
    """Per-token table (page size 1, P:2410-2414): slots of request b = req_to_token[rpi[b], :ctx[b]]."""
    r2t = np.asarray(req_to_token)
    return [r2t[int(req_pool_indices[b]), :int(ctx_lens[b])] for b in range(len(ctx_lens))]


def slots_from_pages(page_table, ctx_lens, page_size):
    """Paged table: token t of request b lives at page_table[b, t // P] * P + t % P."""
    pt = np.asarray(page_table, dtype=np.int64)
    out = []
    for b in range(len(ctx_lens)):
        t = np.arange(int(ctx_lens[b]))
        out.append(pt[b, t // page_size] * page_size + t % page_size)
    return out
