"""Pins of the tree-GDN oracle (CPU, float64).

The chunk form (the reference kernel's equations, inference/hf/tree_gdn_kernel.py:3-6) is checked
against an independent node-by-node recurrence (tests/test_gdn_tree_math.py:34-39 of the reference),
against closed forms (a chain is the sequential delta rule; beta = 0 leaves only the S0 term; S0 = 0
and g = 0 on a chain is the plain delta rule), against the commit state, and the checks are shown to
catch planted mistakes (a dropped decay, a flipped sign, a transposed state, a wrong GQA map).
"""

import numpy as np
import pytest

from oracle import gdn
from oracle.synth import random_tree


def make_case(seed, n=40, HK=2, H=4, dk=16, dv=12, forest=False):
    rng = np.random.default_rng(seed)
    if forest:
        parents = np.array([-1] + [int(rng.integers(-1, i)) for i in range(1, n)], dtype=np.int32)
    else:
        parents = np.array([-1] + [int(rng.integers(0, i)) for i in range(1, n)], dtype=np.int32)
    k = rng.standard_normal((n, HK, dk))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    q = rng.standard_normal((n, HK, dk))
    v = rng.standard_normal((n, H, dv))
    beta = rng.random((n, H))
    g = -rng.random((n, H))
    s0 = rng.standard_normal((H, dk, dv))
    return parents, q, k, v, beta, g, s0


def g_cum_of(g, parents):
    G = np.zeros_like(g)
    for i in range(len(parents)):
        p = parents[i]
        G[i] = g[i] + (G[p] if p >= 0 else 0.0)
    return G


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("forest", [False, True])
def test_chunk_form_matches_recurrence(seed, forest):
    parents, q, k, v, beta, g, s0 = make_case(seed, forest=forest)
    u_c, o_c = gdn.tree_gdn_chunk(q, k, v, g_cum_of(g, parents), beta, s0, parents)
    u_r, o_r, _ = gdn.tree_gdn_recurrence(q, k, v, g, beta, s0, parents)
    np.testing.assert_allclose(u_c, u_r, rtol=0, atol=1e-10)
    np.testing.assert_allclose(o_c, o_r, rtol=0, atol=1e-10)


def test_commit_state_matches_recurrence():
    parents, q, k, v, beta, g, s0 = make_case(7)
    G = g_cum_of(g, parents)
    u, _ = gdn.tree_gdn_chunk(q, k, v, G, beta, s0, parents)
    _, _, states = gdn.tree_gdn_recurrence(q, k, v, g, beta, s0, parents)
    depth = gdn.depths_from_parents(parents)
    deepest = int(np.argmax(depth))
    np.testing.assert_allclose(gdn.commit_state(k, u, G, s0, parents, deepest), states[deepest], rtol=0, atol=1e-10)


def sequential_delta_rule(q, k, v, g, beta, s0):
    """Textbook gated delta rule over a sequence (one head), S in [d_k, d_v]."""
    S = s0.copy()
    outs = []
    for t in range(len(k)):
        S = np.exp(g[t]) * S
        S = S + np.outer(k[t], beta[t] * (v[t] - S.T @ k[t]))
        outs.append(S.T @ q[t])
    return np.array(outs)


def test_chain_is_sequential_delta_rule():
    n = 30
    parents, q, k, v, beta, g, s0 = make_case(3, n=n, HK=1, H=1)
    chain = np.arange(-1, n - 1, dtype=np.int32)
    _, o = gdn.tree_gdn_chunk(q, k, v, g_cum_of(g, chain), beta, s0, chain)
    ref = sequential_delta_rule(q[:, 0], k[:, 0], v[:, 0], g[:, 0], beta[:, 0], s0[0])
    np.testing.assert_allclose(o[:, 0], ref, rtol=0, atol=1e-10)


def test_beta_zero_leaves_state_term():
    parents, q, k, v, beta, g, s0 = make_case(4)
    G = g_cum_of(g, parents)
    u, o = gdn.tree_gdn_chunk(q, k, v, G, np.zeros_like(beta), s0, parents)
    assert np.abs(u).max() == 0.0
    rep = o.shape[1] // q.shape[1]
    for h in range(o.shape[1]):
        np.testing.assert_allclose(o[:, h], np.exp(G[:, h])[:, None] * (q[:, h // rep] @ s0[h]), atol=1e-12)


def test_zero_state_zero_decay_chain_is_plain_delta_rule():
    n = 20
    _, q, k, v, beta, g, s0 = make_case(5, n=n, HK=1, H=1)
    chain = np.arange(-1, n - 1, dtype=np.int32)
    zg = np.zeros_like(g)
    _, o = gdn.tree_gdn_chunk(q, k, v, zg, beta, np.zeros_like(s0), chain)
    # plain delta rule: S_t = S_{t-1} + beta k (v - S^T k)^T
    S = np.zeros((k.shape[2], v.shape[2]))
    for t in range(n):
        S = S + np.outer(k[t, 0], beta[t, 0] * (v[t, 0] - S.T @ k[t, 0]))
        np.testing.assert_allclose(o[t, 0], S.T @ q[t, 0], atol=1e-10)


def test_linear_in_v_and_state_pair():
    parents, q, k, v, beta, g, s0 = make_case(6)
    G = g_cum_of(g, parents)
    u1, o1 = gdn.tree_gdn_chunk(q, k, v, G, beta, s0, parents)
    u2, o2 = gdn.tree_gdn_chunk(q, k, 2 * v, G, beta, 2 * s0, parents)
    np.testing.assert_allclose(u2, 2 * u1, atol=1e-10)
    np.testing.assert_allclose(o2, 2 * o1, atol=1e-10)


def test_parents_round_trip_through_anc():
    import torch

    gen = torch.Generator().manual_seed(0)
    parents = random_tree(64, 16, gen)
    anc = gdn.ancestor_matrix(parents)
    assert (gdn.parents_from_anc(anc) == parents).all()
    assert gdn.depths_from_parents(parents).max() <= 16


# ---- planted mistakes: each variant must be caught by the recurrence check


def _chunk_variant(q, k, v, G, beta, s0, parents, mistake):
    n, HK, _ = k.shape
    H = v.shape[1]
    rep = H // HK
    anc = gdn.ancestor_matrix(parents)
    strict = anc & ~np.eye(n, dtype=bool)
    u = np.zeros((n, H, v.shape[2]))
    o = np.zeros_like(u)
    for h in range(H):
        hk = (h % HK) if mistake == "gqa" else h // rep
        kh, qh, Gh, b = k[:, hk], q[:, hk], G[:, h], beta[:, h]
        gamma = np.where(anc, np.exp(np.where(anc, Gh[:, None] - Gh[None, :], 0.0)), 0.0)
        if mistake == "decay":
            gamma = anc.astype(float)
        sign = -1.0 if mistake == "sign" else 1.0
        lower = sign * b[:, None] * gamma * (kh @ kh.T) * strict
        st = s0[h].T if mistake == "transpose" else s0[h]
        rhs = b[:, None] * (v[:, h] - np.exp(Gh)[:, None] * (kh @ st))
        uh = np.zeros_like(rhs)
        for i in range(n):
            uh[i] = rhs[i] - lower[i, :i] @ uh[:i]
        u[:, h] = uh
        o[:, h] = np.exp(Gh)[:, None] * (qh @ st) + (gamma * (qh @ kh.T) * anc) @ uh
    return u, o


@pytest.mark.parametrize("mistake", ["decay", "sign", "transpose", "gqa"])
def test_planted_mistakes_are_caught(mistake):
    parents, q, k, v, beta, g, s0 = make_case(11, HK=2, H=4, dk=8, dv=8)
    _, o_r, _ = gdn.tree_gdn_recurrence(q, k, v, g, beta, s0, parents)
    _, o_bad = _chunk_variant(q, k, v, g_cum_of(g, parents), beta, s0, parents, mistake)
    assert np.abs(o_bad - o_r).max() > 1e-3


# ---------------------------------------------------------------- gates (inference/hf/qwen35_tree.py:77-79)

def _gate_inputs(n, H, seed):
    import torch

    from oracle.synth import random_tree

    gen = torch.Generator().manual_seed(seed)
    parents = random_tree(n, 16, gen)
    a = torch.randn(n, H, generator=gen) * 4
    a[0, 0] = 30.0   # softplus above its threshold
    b = torch.randn(n, H, generator=gen) * 3
    A_log = torch.randn(H, generator=gen) * 0.5
    dt = torch.randn(H, generator=gen)
    return a, b, A_log, dt, parents


def test_gates_match_the_reference_expression():
    """The reference's own torch lines (softplus, sigmoid, and G as the dense ancestor product anc_f @ g)
    against the oracle's parent-pointer sums."""
    import torch
    import torch.nn.functional as F

    a, b, A_log, dt, parents = _gate_inputs(97, 12, 5)
    anc = torch.from_numpy(gdn.ancestor_matrix(parents).astype(np.float64))
    beta_ref = b.double().sigmoid()
    g_ref = -A_log.double().exp() * F.softplus(a.double() + dt.double())
    G_ref = anc @ g_ref
    G, beta = gdn.gates(a.numpy(), b.numpy(), A_log.numpy(), dt.numpy(), parents)
    np.testing.assert_allclose(beta, beta_ref.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(G, G_ref.numpy(), rtol=1e-12, atol=1e-12)


def test_gates_planted_mistakes_fail():
    import torch
    import torch.nn.functional as F

    a, b, A_log, dt, parents = _gate_inputs(40, 4, 6)
    anc = torch.from_numpy(gdn.ancestor_matrix(parents).astype(np.float64))
    G_ref = (anc @ (-A_log.double().exp() * F.softplus(a.double() + dt.double()))).numpy()
    G_nodt, _ = gdn.gates(a.numpy(), b.numpy(), A_log.numpy(), np.zeros_like(dt.numpy()), parents)
    assert not np.allclose(G_nodt, G_ref, rtol=1e-6)
    G_parent_only, _ = gdn.gates(a.numpy(), b.numpy(), A_log.numpy(), dt.numpy(), np.full_like(parents, -1))
    assert not np.allclose(G_parent_only, G_ref, rtol=1e-6)
