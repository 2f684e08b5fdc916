"""CPU oracle of tree gated-delta-rule (Gated-DeltaNet) verification. TEST INFRASTRUCTURE ONLY.

Two independent restatements of the same quantity, both in float64:

  * ``tree_gdn_chunk`` — the chunk form the reference kernel computes
    (inference/hf/tree_gdn_kernel.py:3-6, inference/hf/qwen35_tree.py:9-20): one dense
    ancestor-masked unit-lower-triangular solve per value head,

        u_i + sum_{j strict anc i} beta_i e^{G_i-G_j} (k_i.k_j) u_j = beta_i (v_i - e^{G_i} S0^T k_i)
        o_i = e^{G_i} S0^T q_i + sum_{j anc-or-self i} e^{G_i-G_j} (q_i.k_j) u_j

    with S0 in the [d_k, d_v] layout and value head h reading key head h // (H / HK)
    (inference/hf/tree_gdn_kernel.py:153-156, :71, :102).
  * ``tree_gdn_recurrence`` — node-by-node gated delta rule from the parent's state
    (tests/test_gdn_tree_math.py:34-39), S_i = e^{g_i} (I - beta_i k_i k_i^T) S_{p(i)} + beta_i k_i v_i^T
    in the [d_k, d_v] layout, o_i = S_i^T q_i, u_i = beta_i (v_i - e^{g_i} S_{p(i)}^T k_i).

They are pinned against each other (tests/test_oracle_gdn.py), against the closed-form special
cases (chain = sequential delta rule, beta = 0, S0 = 0 with g = 0) and against the commit state
(inference/hf/qwen35_tree.py:19, tests/test_gdn_tree_math.py:57-60).
"""

from __future__ import annotations

import numpy as np

F64 = np.float64


def depths_from_parents(parents: np.ndarray) -> np.ndarray:
    """Depth of every node counted in nodes on its root path (root = 1), parents first."""
    n = len(parents)
    d = np.zeros(n, dtype=np.int64)
    for i in range(n):
        p = int(parents[i])
        assert p < i, "nodes must be in topological order (parents first)"
        d[i] = 1 if p < 0 else d[p] + 1
    return d


def ancestor_matrix(parents: np.ndarray) -> np.ndarray:
    """[n, n] bool, row i = ancestors of i and i itself (inference/hf/qwen35_tree.py:36)."""
    n = len(parents)
    anc = np.zeros((n, n), dtype=bool)
    for i in range(n):
        p = int(parents[i])
        if p >= 0:
            anc[i] = anc[p]
        anc[i, i] = True
    return anc


def parents_from_anc(anc: np.ndarray) -> np.ndarray:
    """Parent = the largest-index strict ancestor (ancestors precede their descendants)."""
    n = anc.shape[0]
    out = np.full(n, -1, dtype=np.int32)
    for i in range(n):
        js = np.nonzero(anc[i, :i])[0]
        if len(js):
            out[i] = js[-1]
    return out


def g_cum_from_g(g: np.ndarray, parents: np.ndarray) -> np.ndarray:
    """G_i = G_{p(i)} + g_i (log decay summed along the root path; inference/hf/qwen35_tree.py:79)."""
    G = np.zeros_like(g, dtype=F64)
    for i in range(len(parents)):
        p = int(parents[i])
        G[i] = g[i] + (G[p] if p >= 0 else 0.0)
    return G


def gates(a, b, A_log, dt_bias, parents):
    """Gates of one tree (inference/hf/qwen35_tree.py:77-79), float64: beta = sigmoid(b),
    g = -exp(A_log) * softplus(a + dt_bias) with torch's softplus (x above 20 returned as is), and
    G = g summed along the root path (node included). a, b: [n, H]; A_log, dt_bias: [H]."""
    a = np.asarray(a, dtype=F64)
    b = np.asarray(b, dtype=F64)
    x = a + np.asarray(dt_bias, dtype=F64)[None, :]
    sp = np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))
    g = -np.exp(np.asarray(A_log, dtype=F64))[None, :] * sp
    beta = 1.0 / (1.0 + np.exp(-b))
    return g_cum_from_g(g, parents), beta


def tree_gdn_chunk(q, k, v, g_cum, beta, s0, parents):
    """Dense chunk form, one tree. q, k: [n, HK, D]; v: [n, H, V]; g_cum, beta: [n, H];
    s0: [H, D, V] ([d_k, d_v]); parents: [n]. Returns u, o: [n, H, V] float64."""
    q, k, v = (np.asarray(x, dtype=F64) for x in (q, k, v))
    g_cum, beta, s0 = (np.asarray(x, dtype=F64) for x in (g_cum, beta, s0))
    n, HK, _ = k.shape
    H, V = v.shape[1], v.shape[2]
    rep = H // HK
    anc = ancestor_matrix(np.asarray(parents))
    strict = anc & ~np.eye(n, dtype=bool)
    u = np.zeros((n, H, V), dtype=F64)
    o = np.zeros((n, H, V), dtype=F64)
    for h in range(H):
        hk = h // rep
        kh, qh, G, b = k[:, hk], q[:, hk], g_cum[:, h], beta[:, h]
        with np.errstate(under="ignore"):
            gamma = np.where(anc, np.exp(np.where(anc, G[:, None] - G[None, :], 0.0)), 0.0)
        lower = b[:, None] * gamma * (kh @ kh.T) * strict
        rhs = b[:, None] * (v[:, h] - np.exp(G)[:, None] * (kh @ s0[h]))
        # unit lower triangular solve by forward substitution (parents first)
        uh = np.zeros((n, V), dtype=F64)
        for i in range(n):
            uh[i] = rhs[i] - lower[i, :i] @ uh[:i]
        u[:, h] = uh
        o[:, h] = np.exp(G)[:, None] * (qh @ s0[h]) + (gamma * (qh @ kh.T) * anc) @ uh
    return u, o


def tree_gdn_recurrence(q, k, v, g, beta, s0, parents):
    """Node-by-node recurrence, one tree. g: [n, H] per-node log decay (NOT accumulated).
    Returns u, o: [n, H, V] and the per-node states [n, H, D, V] (float64)."""
    q, k, v = (np.asarray(x, dtype=F64) for x in (q, k, v))
    g, beta, s0 = (np.asarray(x, dtype=F64) for x in (g, beta, s0))
    n, HK, D = k.shape
    H, V = v.shape[1], v.shape[2]
    rep = H // HK
    states = np.zeros((n, H, D, V), dtype=F64)
    u = np.zeros((n, H, V), dtype=F64)
    o = np.zeros((n, H, V), dtype=F64)
    for i in range(n):
        p = int(parents[i])
        for h in range(H):
            kk, qq = k[i, h // rep], q[i, h // rep]
            sp = s0[h] if p < 0 else states[p, h]
            decayed = np.exp(g[i, h]) * sp
            ui = beta[i, h] * (v[i, h] - decayed.T @ kk)
            si = decayed + np.outer(kk, ui)
            states[i, h] = si
            u[i, h] = ui
            o[i, h] = si.T @ qq
    return u, o, states


def commit_state(k, u, g_cum, s0, parents, node):
    """State after accepting the root path ending at ``node``
    (inference/hf/qwen35_tree.py:19, :135-137): S = e^{G_a} S0 + sum_j e^{G_a - G_j} k_j u_j^T."""
    k, u, g_cum, s0 = (np.asarray(x, dtype=F64) for x in (k, u, g_cum, s0))
    H = u.shape[1]
    rep = H // k.shape[1]
    path = []
    i = node
    while i >= 0:
        path.append(i)
        i = int(parents[i])
    out = np.exp(g_cum[node])[:, None, None] * s0
    for j in path:
        for h in range(H):
            out[h] += np.exp(g_cum[node, h] - g_cum[j, h]) * np.outer(k[j, h // rep], u[j, h])
    return out


def tree_gdn_varlen(q, k, v, g_cum, beta, s0, parents, cu_nodes):
    """Ragged batch of trees packed along the node axis; s0: [R, H, D, V]; parents request-local."""
    N = k.shape[0]
    H, V = v.shape[1], v.shape[2]
    u = np.zeros((N, H, V), dtype=F64)
    o = np.zeros((N, H, V), dtype=F64)
    for r in range(len(cu_nodes) - 1):
        a, b = int(cu_nodes[r]), int(cu_nodes[r + 1])
        if b > a:
            u[a:b], o[a:b] = tree_gdn_chunk(q[a:b], k[a:b], v[a:b], g_cum[a:b], beta[a:b], s0[r], parents[a:b])
    return u, o


def tree_gdn_dense_torch(q, k, v, g_cum, beta, s0, parents):
    """CPU baseline in float32 torch, heads batched: the dense ancestor-masked triangular solve
    (tests/test_gdn_tree_math.py:41-56 semantics; inference/hf/qwen35_tree.py:9-20). One tree.
    q, k [n, HK, D]; v [n, H, V]; g_cum, beta [n, H]; s0 [H, D, V] (torch float32 tensors)."""
    import torch

    n, HK, _ = k.shape
    H = v.shape[1]
    rep = H // HK
    anc = torch.from_numpy(ancestor_matrix(np.asarray(parents)))
    strict = anc & ~torch.eye(n, dtype=torch.bool)
    kh = k.transpose(0, 1).repeat_interleave(rep, 0)  # [H, n, D]
    qh = q.transpose(0, 1).repeat_interleave(rep, 0)
    G = g_cum.transpose(0, 1)  # [H, n]
    b = beta.transpose(0, 1)
    diff = torch.where(anc, G[:, :, None] - G[:, None, :], torch.full((), float("-inf")))
    gamma = diff.exp()  # [H, n, n]
    lower = b[:, :, None] * gamma * (kh @ kh.transpose(1, 2)) * strict
    rhs = b[:, :, None] * (v.transpose(0, 1) - G.exp()[:, :, None] * (kh @ s0))
    eye = torch.eye(n).expand(H, n, n)
    u = torch.linalg.solve_triangular(eye + lower, rhs, upper=False, unitriangular=True)
    o = G.exp()[:, :, None] * (qh @ s0) + (gamma * (qh @ kh.transpose(1, 2)) * anc) @ u
    return u.transpose(0, 1), o.transpose(0, 1)


# ---------------------------------------------------------------------------- conv windows, tree_prep, commit


def conv_index(parents, kernel: int) -> np.ndarray:
    """Conv window of every node, oldest first, as indices into [conv state (kernel columns) ; nodes]
    (inference/hf/qwen35_tree.py:39-52): the node, its parent, grandparent, ..., then the cached columns
    from the most recent one (kernel - 1) backwards."""
    parents = np.asarray(parents)
    n = len(parents)
    out = np.zeros((n, kernel), dtype=np.int32)
    for i in range(n):
        chain, p = [kernel + i], int(parents[i])
        while len(chain) < kernel and p >= 0:
            chain.append(kernel + p)
            p = int(parents[p])
        last = kernel - 1
        while len(chain) < kernel:
            chain.append(last)
            last -= 1
        out[i] = chain[::-1]
    return out


def round_bf16(a) -> np.ndarray:
    """Round to the nearest bfloat16 (ties to even), returned as float64."""
    f = np.asarray(a, dtype=np.float32)
    b = f.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    r = np.where(np.isnan(f), b | 0x400000, r)
    return r.astype(np.uint32).view(np.float32).astype(F64)


def tree_prep(x, conv_state, cidx, conv_w, HK: int, H: int, D: int, scale: float):
    """q, k, v of the tree nodes (inference/hf/tree_gdn_kernel.py:29-56 _tree_prep, :135-150), float64:
    acc = sum_t w[c, t] * [conv_state ; x][cidx[i, t], c] (conv_state as columns), y = bf16(silu(acc)),
    q / k heads normalised as y / sqrt(sum y^2 + 1e-6) (q times scale), v = y. x [n, CD]; conv_state and
    conv_w [CD, KC]; cidx [n, KC]. Returns q, k [n, HK, D] and v [n, H, D] (not rounded)."""
    x = np.asarray(x, dtype=F64)
    cs = np.asarray(conv_state, dtype=F64)
    w = np.asarray(conv_w, dtype=F64)
    cidx = np.asarray(cidx)
    n, CD = x.shape
    KC = w.shape[1]
    assert CD == (2 * HK + H) * D
    src = np.concatenate([cs.T, x], axis=0)  # [KC + n, CD]
    acc = np.zeros((n, CD), dtype=F64)
    for t in range(KC):
        acc += w[:, t][None, :] * src[cidx[:, t]]
    y = round_bf16(acc / (1.0 + np.exp(-acc)))
    q = y[:, : HK * D].reshape(n, HK, D)
    k = y[:, HK * D : 2 * HK * D].reshape(n, HK, D)
    v = y[:, 2 * HK * D :].reshape(n, H, D)
    q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) * scale
    k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    return q, k, v


def commit_conv(conv, x, cidx, node) -> np.ndarray:
    """Conv state after accepting ``node`` (inference/hf/qwen35_tree.py:141-146): column t = old column
    cidx[node, t] if that index is below the kernel size, else the node input x[cidx[node, t] - KC].
    conv [CD, KC]; x [n, CD]."""
    conv = np.asarray(conv, dtype=F64)
    x = np.asarray(x, dtype=F64)
    KC = conv.shape[1]
    cols = [conv[:, i] if i < KC else x[i - KC] for i in np.asarray(cidx)[node]]
    return np.stack(cols, axis=1)
