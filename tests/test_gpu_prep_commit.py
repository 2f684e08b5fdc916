"""GPU parity of the conv windows, tree_prep and the GDN commit (through the C ABI).

Bars: windows and conv commits bit-exact (index and copy work). tree_prep outputs are bf16: every element
within 2 bf16 ulps of the float64 oracle (2^-7 relative; the GPU accumulates in fp32, so a value next to a
rounding boundary of the SiLU output can round the other way) and 2e-3 norm-wise. Commit states: fp32, max
abs error <= 1e-5 x max |ref| against the float64 oracle, and the end-to-end chain prep -> gates -> verify
-> commit equals the node-by-node recurrence's state at the accepted node within 2e-3 x max |ref|.
"""

import numpy as np
import pytest
import torch

from oracle import gdn
from oracle.synth import random_tree

pytestmark = pytest.mark.gpu


def bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("KC", [2, 4, 8])
def test_conv_index_matches_oracle_ragged(KC):
    import tree_gdn_kernel

    g = torch.Generator().manual_seed(KC)
    sizes = [1, 17, 64, 5]
    trees = [random_tree(n, 16, g) for n in sizes]
    parents = np.concatenate(trees).astype(np.int32)
    cu = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    print(f"case: conv_index KC={KC} sizes={sizes}", flush=True)
    idx = tree_gdn_kernel.conv_index(torch.from_numpy(parents).cuda(), KC, torch.from_numpy(cu).cuda())
    ref = np.concatenate([gdn.conv_index(t, KC) for t in trees])
    np.testing.assert_array_equal(idx.cpu().numpy(), ref)


def prep_inputs(seed, n, HK, H, D, KC, R=1):
    rng = np.random.default_rng(seed)
    CD = (2 * HK + H) * D
    x = gdn.round_bf16(rng.standard_normal((n, CD)))
    cs = gdn.round_bf16(rng.standard_normal((R, CD, KC)))
    w = gdn.round_bf16(rng.standard_normal((CD, KC)) * 0.5)
    return x, cs, w


def check_bf16_close(got, ref, name):
    got = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    assert np.all(err <= 2.0 ** -7 * np.abs(ref) + 1e-6), f"{name}: max rel {np.max(err / (np.abs(ref) + 1e-30))}"
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= 2e-3, f"{name}: norm rel {rel}"


@pytest.mark.parametrize("n,HK,H,KC", [(64, 16, 32, 4), (128, 16, 48, 4), (7, 2, 6, 3), (33, 4, 4, 1), (256, 2, 4, 4),
                                       (300, 2, 4, 4)])
def test_tree_prep_matches_oracle(n, HK, H, KC):
    import tree_gdn_kernel

    D = 128
    g = torch.Generator().manual_seed(n + H)
    parents = random_tree(n, 16, g)
    x, cs, w = prep_inputs(n, n, HK, H, D, KC)
    idx = gdn.conv_index(parents, KC)
    print(f"case: tree_prep n={n} HK={HK} H={H} KC={KC}", flush=True)
    q, k, v = tree_gdn_kernel.tree_prep(bf(x).cuda(), bf(cs[0]).cuda(), torch.from_numpy(idx).cuda(), bf(w).cuda(),
                                        HK, H, D)
    torch.cuda.synchronize()
    qr, kr, vr = gdn.tree_prep(x, cs[0], idx, w, HK, H, D, D ** -0.5)
    check_bf16_close(q, qr, "q")
    check_bf16_close(k, kr, "k")
    check_bf16_close(v, vr, "v")


def test_tree_prep_ragged_requests_use_their_own_state_and_nodes():
    import tree_gdn_kernel

    HK, H, D, KC = 2, 4, 128, 4
    sizes = [5, 16, 3]
    g = torch.Generator().manual_seed(3)
    trees = [random_tree(s, 16, g) for s in sizes]
    N = sum(sizes)
    x, cs, w = prep_inputs(9, N, HK, H, D, KC, R=len(sizes))
    cu = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    idx = np.concatenate([gdn.conv_index(t, KC) for t in trees])
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    q, k, v = tree_gdn_kernel.tree_prep(bf(x).cuda(), bf(cs).cuda(), torch.from_numpy(idx).cuda(), bf(w).cuda(), HK, H,
                                        D, cu_nodes=torch.from_numpy(cu).cuda(), err_flag=err)
    torch.cuda.synchronize()
    assert int(err) == 0
    for r in range(len(sizes)):
        a, b = cu[r], cu[r + 1]
        qr, kr, vr = gdn.tree_prep(x[a:b], cs[r], idx[a:b], w, HK, H, D, D ** -0.5)
        check_bf16_close(q[a:b], qr, f"q req {r}")
        check_bf16_close(v[a:b], vr, f"v req {r}")


def test_tree_prep_out_of_range_window_is_flagged_not_read():
    import tree_gdn_kernel

    HK, H, D, KC, n = 2, 2, 128, 4, 6
    x, cs, w = prep_inputs(1, n, HK, H, D, KC)
    idx = gdn.conv_index(np.arange(-1, n - 1, dtype=np.int32), KC)
    idx[2, 1] = KC + n + 1000  # past the last node
    idx[3, 0] = -5
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    tree_gdn_kernel.tree_prep(bf(x).cuda(), bf(cs[0]).cuda(), torch.from_numpy(idx).cuda(), bf(w).cuda(), HK, H, D,
                              err_flag=err)
    torch.cuda.synchronize()
    assert int(err) & 16


def commit_case(seed, L=3, n=48, HK=4, H=8, D=128, KC=4, chain=False):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    parents = np.arange(-1, n - 1, dtype=np.int32) if chain else random_tree(n, 16, g)
    u = rng.standard_normal((L, n, H, D)).astype(np.float32)
    k = gdn.round_bf16(rng.standard_normal((L, n, HK, D)) / np.sqrt(D))
    G = np.stack([gdn.g_cum_from_g(-0.1 * rng.random((n, H)), parents) for _ in range(L)]).astype(np.float32)
    S = (rng.standard_normal((L, H, D, D)) * 0.02).astype(np.float32)
    CD = (2 * HK + H) * D
    conv = gdn.round_bf16(rng.standard_normal((L, CD, KC)))
    x = gdn.round_bf16(rng.standard_normal((L, n, CD)))
    return parents, u, k, G, S, conv, x


@pytest.mark.parametrize("seed,chain", [(0, False), (1, False), (2, True)])
def test_gdn_commit_matches_oracle(seed, chain):
    """Random trees (paths of at most 16 nodes: rows staged once, the state in two halves) and a 48-node chain
    (a 48-node path: rows staged 32 at a time)."""
    import tree_gdn_kernel

    L, n, HK, H, D, KC = 3, 48, 4, 8, 128, 4
    parents, u, k, G, S, conv, x = commit_case(seed, L, n, HK, H, D, KC, chain=chain)
    node = int(np.argmax(gdn.depths_from_parents(parents)))
    path = []
    i = node
    while i >= 0:
        path.append(i)
        i = int(parents[i])
    path = path[::-1]
    idx = gdn.conv_index(parents, KC)
    print(f"case: gdn_commit seed={seed} path={path}", flush=True)
    St = torch.from_numpy(S).cuda()
    ct = bf(conv).cuda()
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    tree_gdn_kernel.gdn_commit(St, torch.from_numpy(u).cuda(), bf(k).cuda(), torch.from_numpy(G).cuda(), path,
                               conv=ct, x=bf(x).cuda(), conv_index=torch.from_numpy(idx).cuda(), err_flag=err)
    torch.cuda.synchronize()
    assert int(err) == 0
    for l in range(L):
        ref = gdn.commit_state(k[l], u[l].astype(np.float64), G[l].astype(np.float64), S[l].astype(np.float64),
                               parents, node)
        got = St[l].cpu().numpy()
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max(), f"layer {l}"
        cref = gdn.commit_conv(conv[l], x[l], idx, node)
        np.testing.assert_array_equal(ct[l].float().cpu().numpy(), cref)


def test_gdn_commit_bad_path_end_writes_nothing():
    import tree_gdn_kernel

    L, n, HK, H, D, KC = 2, 8, 2, 2, 128, 4
    parents, u, k, G, S, conv, x = commit_case(4, L, n, HK, H, D, KC)
    St = torch.from_numpy(S).cuda()
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    tree_gdn_kernel.gdn_commit(St, torch.from_numpy(u).cuda(), bf(k).cuda(), torch.from_numpy(G).cuda(),
                               torch.tensor([0, 99], dtype=torch.int32), err_flag=err)
    torch.cuda.synchronize()
    assert int(err) & 16
    np.testing.assert_array_equal(St.cpu().numpy(), S)


def test_chain_prep_verify_commit_equals_recurrence():
    """A chain verified as a tree and committed at its last node leaves the state the sequential gated
    delta rule reaches (inference/hf/qwen35_tree.py:19-22): prep -> gates -> tree_gdn -> commit on the GPU
    against the float64 node-by-node recurrence on the same bf16 q / k / v."""
    import tree_gdn_kernel

    n, HK, H, D, KC = 12, 2, 4, 128, 4
    rng = np.random.default_rng(11)
    parents = np.arange(-1, n - 1, dtype=np.int32)
    x, cs, w = prep_inputs(11, n, HK, H, D, KC)
    idx = gdn.conv_index(parents, KC)
    a = rng.standard_normal((n, H)).astype(np.float32)
    b = rng.standard_normal((n, H)).astype(np.float32)
    A_log = np.log(rng.random(H) * 4 + 1).astype(np.float32)
    dt_bias = rng.standard_normal(H).astype(np.float32)
    S0 = (rng.standard_normal((H, D, D)) * 0.02).astype(np.float32)
    q, k, v = tree_gdn_kernel.tree_prep(bf(x).cuda(), bf(cs[0]).cuda(), torch.from_numpy(idx).cuda(), bf(w).cuda(), HK,
                                        H, D)
    pt = torch.from_numpy(parents).cuda()
    g_cum, beta = tree_gdn_kernel.tree_gates(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(),
                                             torch.from_numpy(A_log).cuda(), torch.from_numpy(dt_bias).cuda(),
                                             parents=pt)
    cu = torch.tensor([0, n], dtype=torch.int32, device="cuda")
    u, o = tree_gdn_kernel.tree_gdn_varlen(q, k, v, g_cum, beta, torch.from_numpy(S0)[None].cuda(), pt, cu)
    St = torch.from_numpy(S0)[None].cuda().contiguous()
    tree_gdn_kernel.gdn_commit(St, u[None], k[None], g_cum[None], list(range(n)))
    torch.cuda.synchronize()
    qf, kf, vf = (t.float().cpu().numpy().astype(np.float64) for t in (q, k, v))
    G, bt = gdn.gates(a, b, A_log, dt_bias, parents)
    gstep = np.diff(np.concatenate([np.zeros((1, H)), G]), axis=0)
    _, o_ref, states = gdn.tree_gdn_recurrence(qf, kf, vf, gstep, bt, S0.astype(np.float64), parents)
    ref = states[n - 1]
    assert np.abs(St[0].cpu().numpy() - ref).max() <= 2e-3 * np.abs(ref).max()
    assert np.abs(o.cpu().numpy() - o_ref).max() <= 2e-3 * np.abs(o_ref).max()
