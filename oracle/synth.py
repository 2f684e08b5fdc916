"""Seeded synthetic inputs of the benchmark/parity configurations. TEST INFRASTRUCTURE ONLY.

Draw order and distributions follow the configuration text: torch.Generator seeded per config,
trees with uniform parents over earlier nodes whose root path is shorter than the depth cap,
q/k L2-normalised per head, beta = sigmoid(randn), g = -softplus(randn) * 0.1, G accumulated
along parent pointers, s0 = randn * 0.02; attention tensors randn * 0.5; builder logits randn * 3
with one +6 spike per position.
"""

from __future__ import annotations

import numpy as np
import torch


def random_tree(n: int, max_depth: int, gen: torch.Generator) -> np.ndarray:
    """Node 0 is the root (parent -1, depth 1); node i's parent is uniform over earlier nodes
    whose depth is below ``max_depth`` (so no root path exceeds max_depth nodes)."""
    parents = np.full(n, -1, dtype=np.int32)
    depth = np.zeros(n, dtype=np.int64)
    depth[0] = 1
    for i in range(1, n):
        ok = np.nonzero(depth[:i] < max_depth)[0]
        j = int(torch.randint(0, len(ok), (1,), generator=gen))
        parents[i] = ok[j]
        depth[i] = depth[ok[j]] + 1
    return parents


def gdn_inputs(n_nodes, HK, H, D, seed, max_depth=16, parents=None):
    """One or several trees. ``n_nodes``: int (one tree) or a list of per-request sizes.
    Returns dict of float32 numpy arrays (q, k, v rounded through bf16 as the GPU receives them),
    request-local parents, cu_nodes, g (per node), g_cum, beta, s0 [R, H, D, D].
    ``parents``: reuse these trees (another layer of the same verify round) instead of drawing new ones."""
    sizes = [n_nodes] if isinstance(n_nodes, int) else list(n_nodes)
    gen = torch.Generator().manual_seed(seed)
    if parents is None:
        parents = np.concatenate([random_tree(n, max_depth, gen) for n in sizes]).astype(np.int32)
    else:
        parents = np.asarray(parents, dtype=np.int32).copy()
        assert parents.shape == (int(sum(sizes)),)
    N = int(sum(sizes))
    R = len(sizes)
    q = torch.nn.functional.normalize(torch.randn(N, HK, D, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(N, HK, D, generator=gen), dim=-1)
    v = torch.randn(N, H, D, generator=gen)
    beta = torch.sigmoid(torch.randn(N, H, generator=gen))
    g = -torch.nn.functional.softplus(torch.randn(N, H, generator=gen)) * 0.1
    s0 = torch.randn(R, H, D, D, generator=gen) * 0.02
    cu = np.zeros(R + 1, dtype=np.int32)
    cu[1:] = np.cumsum(sizes)
    g_np = g.numpy().astype(np.float64)
    g_cum = np.zeros_like(g_np)
    for r in range(R):
        a, b = cu[r], cu[r + 1]
        for i in range(a, b):
            p = parents[i]
            g_cum[i] = g_np[i] + (g_cum[a + p] if p >= 0 else 0.0)
    bf = lambda t: t.to(torch.bfloat16).float().numpy()
    return dict(q=bf(q), k=bf(k), v=bf(v), beta=beta.numpy(), g=g.numpy(), g_cum=g_cum.astype(np.float32),
                s0=s0.numpy(), parents=parents, cu_nodes=cu, sizes=sizes)


def attention_inputs(seed, K=8, bs=16, H=32, Hkv=8, D=128, ctx=4096, scale=0.5):
    """Config-2 style flat inputs, reference layout: q [1,H,K*bs,D], k/v [1,Hkv,ctx+K*bs,D] (bf16)."""
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(1, H, K * bs, D, generator=gen) * scale).to(torch.bfloat16)
    k = (torch.randn(1, Hkv, ctx + K * bs, D, generator=gen) * scale).to(torch.bfloat16)
    v = (torch.randn(1, Hkv, ctx + K * bs, D, generator=gen) * scale).to(torch.bfloat16)
    return q, k, v


def paged_attention_inputs(seed, ctx_lens, K=8, bs=16, H=40, Hkv=8, D=128, page_size=64, scale=0.5,
                           extra_pages=3):
    """Config-4 style paged inputs. KV cache [slots, Hkv, D] bf16 with 64-token pages drawn as a
    random permutation of a page pool. Returns dict with q/k_new/v_new [T, *, D], caches, the
    page table [R, max_pages] int32 (page ids), the equivalent per-token table req_to_token
    [R + 2, max_ctx] int32, req_pool_indices, ctx_lens."""
    gen = torch.Generator().manual_seed(seed)
    R = len(ctx_lens)
    T = R * K * bs
    pages_per = [(c + page_size - 1) // page_size for c in ctx_lens]
    num_pages = sum(pages_per) + extra_pages
    perm = torch.randperm(num_pages, generator=gen)
    max_pages = max(pages_per) if R else 1
    page_table = torch.zeros(R, max(max_pages, 1), dtype=torch.int32)
    off = 0
    for r, np_ in enumerate(pages_per):
        page_table[r, :np_] = perm[off:off + np_].to(torch.int32)
        off += np_
    slots = num_pages * page_size
    k_cache = (torch.randn(slots, Hkv, D, generator=gen) * scale).to(torch.bfloat16)
    v_cache = (torch.randn(slots, Hkv, D, generator=gen) * scale).to(torch.bfloat16)
    q = (torch.randn(T, H, D, generator=gen) * scale).to(torch.bfloat16)
    k_new = (torch.randn(T, Hkv, D, generator=gen) * scale).to(torch.bfloat16)
    v_new = (torch.randn(T, Hkv, D, generator=gen) * scale).to(torch.bfloat16)
    max_ctx = max(max(ctx_lens) if R else 1, 1)
    req_to_token = torch.zeros(R + 2, max_ctx, dtype=torch.int32)
    for r, c in enumerate(ctx_lens):
        t = torch.arange(c)
        req_to_token[r + 2, :c] = (page_table[r, t // page_size].long() * page_size + t % page_size).to(torch.int32)
    req_pool_indices = torch.arange(R, dtype=torch.int64) + 2
    return dict(q=q, k_new=k_new, v_new=v_new, k_cache=k_cache, v_cache=v_cache, page_table=page_table,
                req_to_token=req_to_token, req_pool_indices=req_pool_indices,
                ctx_lens=torch.tensor(ctx_lens, dtype=torch.int64), num_modes=K, block_size=bs,
                scaling=D ** -0.5, page_size=page_size)


def builder_logits(seed, K=8, L=16, V=151936, scale=3.0, spike=6.0):
    """Config-1 logits: randn * 3 (fp32), then for each position one (mode, token) gets +6; bf16."""
    gen = torch.Generator().manual_seed(seed)
    logits = torch.randn(K, L, V, generator=gen) * scale
    for pos in range(L):
        m = int(torch.randint(0, K, (1,), generator=gen))
        t = int(torch.randint(0, V, (1,), generator=gen))
        logits[m, pos, t] += spike
    return logits.to(torch.bfloat16)
