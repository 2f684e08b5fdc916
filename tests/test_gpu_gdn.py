"""GPU parity of the tree-GDN HIP kernel (through the C ABI) against the float64 oracle.

Tolerance (north star: GDN outputs within 2e-3 relative, bf16 inputs, fp32 state):
max |got - ref| <= 2e-3 * max |ref| per output tensor, on the same bf16-rounded inputs.
"""

import numpy as np
import pytest
import torch

from oracle import gdn
from oracle.synth import gdn_inputs

pytestmark = pytest.mark.gpu
RTOL = 2e-3


def _dev(d):
    dev = torch.device("cuda")
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(torch.bfloat16)
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
    return dict(q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), g_cum=f32(d["g_cum"]), beta=f32(d["beta"]),
                s0=f32(d["s0"]), parents=torch.from_numpy(d["parents"]).to(dev),
                cu_nodes=torch.from_numpy(d["cu_nodes"]).to(dev))


def _rel(got, ref):
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def _oracle(d):
    return gdn.tree_gdn_varlen(d["q"], d["k"], d["v"], d["g_cum"], d["beta"], d["s0"], d["parents"], d["cu_nodes"])


def test_tree_gdn_config0_anc8_api():
    """Config 0: one 64-node tree, HK 16, H 32, D 128, through the reference's tree_gdn signature (32 units:
    each (request, value head) split over four value-column blocks)."""
    import tree_gdn_kernel

    d = gdn_inputs(64, 16, 32, 128, seed=0)
    t = _dev(d)
    anc8 = torch.from_numpy(gdn.ancestor_matrix(d["parents"]).astype(np.int8)).cuda()
    print("case: config0 n=64 HK=16 H=32", flush=True)
    u, o = tree_gdn_kernel.tree_gdn(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"][0], anc8)
    torch.cuda.synchronize()
    u_ref, o_ref = _oracle(d)
    eu, eo = _rel(u.cpu().numpy(), u_ref), _rel(o.cpu().numpy(), o_ref)
    print(f"config0 rel err u {eu:.2e} o {eo:.2e}")
    assert eu <= RTOL and eo <= RTOL


@pytest.mark.parametrize("sizes,HK,H", [
    ([128] * 8, 16, 32),                       # config 3 shape (one layer)
    ([16, 37, 64, 1, 128, 5, 64, 33], 16, 48),  # ragged, GQA 3 (config 4 heads)
    ([1], 2, 4),                               # root only
    ([32, 64, 96], 4, 4),                      # no GQA
    ([40, 128, 77], 16, 32),                   # 96 (request, value head) units: two value-column blocks each
    ([50, 64, 17, 33], 8, 24),                 # the same with trees of at most 64 nodes
])
def test_tree_gdn_varlen(sizes, HK, H):
    import tree_gdn_kernel

    d = gdn_inputs(sizes, HK, H, 128, seed=3000 + len(sizes))
    t = _dev(d)
    print(f"case: varlen sizes={sizes} HK={HK} H={H}", flush=True)
    u, o = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], t["parents"],
                                           t["cu_nodes"], max_nodes=max(sizes))
    torch.cuda.synchronize()
    u_ref, o_ref = _oracle(d)
    eu, eo = _rel(u.cpu().numpy(), u_ref), _rel(o.cpu().numpy(), o_ref)
    print(f"rel err u {eu:.2e} o {eo:.2e}")
    assert eu <= RTOL and eo <= RTOL


def _ragged(lo, hi, R, seed):
    return [int(x) for x in np.random.default_rng(seed).integers(lo, hi + 1, R)]


@pytest.mark.parametrize("sizes,HK,H", [
    (_ragged(16, 64, 16, 4000), 16, 48),  # config 4 shape: trees of 16 - 64 nodes (2 tile pairs, 2 waves each)
    ([64] * 8, 8, 24),                    # full 64-node trees
    (_ragged(1, 32, 12, 41), 8, 16),      # trees of at most 32 nodes (one tile pair, 4 waves)
    ([32] * 10, 8, 16),
    (_ragged(65, 128, 6, 42), 8, 32),     # trees of 65 - 128 nodes (4 tile pairs, one wave each)
])
@pytest.mark.parametrize("with_ctx", [False, True])
def test_tree_gdn_full_grid(sizes, HK, H, with_ctx):
    """Grids of more than half a (request, value head) unit per CU take the kernel whose tree waves split the
    Gram blocks and coefficient rows of a tile pair over 4 / NT waves: every split, partial and full last tiles,
    with and without a tree context; three launches agree bit for bit (the hand-overs between the waves
    leave nothing to timing) and match the oracle."""
    import tree_gdn_kernel

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert len(sizes) * H * 2 > cus, "the case must fill the chip to reach the one-block-per-unit kernel"
    d = gdn_inputs(sizes, HK, H, 128, seed=4100 + len(sizes))
    t = _dev(d)
    print(f"case: full grid sizes={sizes} HK={HK} H={H} ctx={with_ctx}", flush=True)
    ctx = tree_gdn_kernel.tree_context(t["parents"], t["cu_nodes"], max_nodes=max(sizes)) if with_ctx else None
    outs = []
    for _ in range(3):
        outs.append(tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"],
                                                    None if with_ctx else t["parents"], t["cu_nodes"],
                                                    max_nodes=max(sizes), ctx=ctx))
    torch.cuda.synchronize()
    for u, o in outs[1:]:
        assert torch.equal(u, outs[0][0]) and torch.equal(o, outs[0][1])
    u_ref, o_ref = _oracle(d)
    eu, eo = _rel(outs[0][0].cpu().numpy(), u_ref), _rel(outs[0][1].cpu().numpy(), o_ref)
    print(f"rel err u {eu:.2e} o {eo:.2e}")
    assert eu <= RTOL and eo <= RTOL


def test_tree_gdn_chain_max_depth():
    """A 16-node chain (deepest allowed path) and a bushy tree of depth 2 in one launch."""
    import tree_gdn_kernel

    d = gdn_inputs([16, 100], 2, 4, 128, seed=5)
    d["parents"][:16] = np.arange(-1, 15, dtype=np.int32)
    d["parents"][16:] = np.array([-1] + [0] * 99, dtype=np.int32)
    # recompute G along the new parents
    g = d["g"].astype(np.float64)
    for a, b in ((0, 16), (16, 116)):
        d["g_cum"][a:b] = gdn.g_cum_from_g(g[a:b], d["parents"][a:b]).astype(np.float32)
    t = _dev(d)
    u, o = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], t["parents"],
                                           t["cu_nodes"], max_nodes=100)
    torch.cuda.synchronize()
    u_ref, o_ref = _oracle(d)
    assert _rel(u.cpu().numpy(), u_ref) <= RTOL and _rel(o.cpu().numpy(), o_ref) <= RTOL


def test_tree_gdn_rejects_too_deep_tree():
    """A 17-node chain exceeds the depth limit: the request is rejected through err_flag and its outputs are NaN
    (never left as stale memory); the other request is computed."""
    import tree_gdn_kernel

    d = gdn_inputs([17, 8], 2, 4, 128, seed=6)
    d["parents"][:17] = np.arange(-1, 16, dtype=np.int32)
    t = _dev(d)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    u = torch.full((25, 4, 128), 7.0, device="cuda")
    o = torch.full((25, 4, 128), 7.0, device="cuda")
    tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], t["parents"],
                                    t["cu_nodes"], max_nodes=17, out=(u, o), err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 2
    assert bool(torch.isnan(u[:17]).all()) and bool(torch.isnan(o[:17]).all())
    u_ref, o_ref = _oracle(dict(d, parents=d["parents"][17:], cu_nodes=np.array([0, 8], dtype=np.int32),
                                q=d["q"][17:], k=d["k"][17:], v=d["v"][17:], g_cum=d["g_cum"][17:],
                                beta=d["beta"][17:], s0=d["s0"][1:]))
    assert _rel(u[17:].cpu().numpy(), u_ref) <= RTOL and _rel(o[17:].cpu().numpy(), o_ref) <= RTOL


def test_tree_gdn_graph_replay():
    """Captured in a HIP graph and replayed with new inputs copied into the same buffers."""
    import tree_gdn_kernel

    d1 = gdn_inputs([64, 128], 4, 8, 128, seed=10)
    d2 = gdn_inputs([64, 128], 4, 8, 128, seed=11)
    t = _dev(d1)
    u = torch.empty(192, 8, 128, device="cuda")
    o = torch.empty_like(u)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], t["parents"],
                                        t["cu_nodes"], max_nodes=128, out=(u, o))
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], t["parents"],
                                        t["cu_nodes"], max_nodes=128, out=(u, o))
    for d in (d2, d1, d2):
        t2 = _dev(d)
        for key in t:
            t[key].copy_(t2[key])
        graph.replay()
        torch.cuda.synchronize()
        u_ref, o_ref = _oracle(d)
        assert _rel(u.cpu().numpy(), u_ref) <= RTOL and _rel(o.cpu().numpy(), o_ref) <= RTOL


# ---------------------------------------------------------------- tree context


def _parse_ctx(buf, R, nmax):
    """Tree context blocks as (anc [R, nmax/32, nmax] u32, path [R, nmax, 16] u8, depth [R, nmax], header)."""
    raw = buf.cpu().numpy()
    blk = nmax * nmax // 8 + 16 * nmax + 4 * nmax + 16
    assert raw.size == R * blk
    out = []
    for r in range(R):
        b = raw[r * blk:(r + 1) * blk]
        o = 0
        anc = b[o:o + nmax * nmax // 8].view(np.uint32).reshape(nmax // 32, nmax)
        o += nmax * nmax // 8
        path = b[o:o + 16 * nmax].reshape(nmax, 16)
        o += 16 * nmax
        depth = b[o:o + 4 * nmax].view(np.int32)
        o += 4 * nmax
        hdr = b[o:o + 16].view(np.int32)
        out.append((anc, path, depth, hdr))
    return out


@pytest.mark.parametrize("sizes,max_nodes", [([128] * 8, 128), ([16, 37, 64, 1, 5, 64, 33], 64), ([3, 30], 32)])
def test_tree_context_contents(sizes, max_nodes):
    """Context blocks against the oracle's depths and ancestor matrix; path[i][depth(j) - 1] = j."""
    import tree_gdn_kernel

    d = gdn_inputs(sizes, 2, 4, 128, seed=40 + len(sizes))
    t = _dev(d)
    ctx = tree_gdn_kernel.tree_context(t["parents"], t["cu_nodes"], max_nodes=max_nodes)
    torch.cuda.synchronize()
    nmax = 32 * ((max_nodes + 31) // 32)
    assert ctx.buf.numel() == len(sizes) * (nmax * nmax // 8 + 20 * nmax + 16)
    for r, (anc, path, depth, hdr) in enumerate(_parse_ctx(ctx.buf, len(sizes), nmax)):
        a, b = d["cu_nodes"][r], d["cu_nodes"][r + 1]
        n = b - a
        par = d["parents"][a:b]
        assert hdr[0] == 0 and hdr[1] == n and hdr[2] == nmax
        dep = gdn.depths_from_parents(par)
        assert (depth[:n] == dep).all() and (depth[n:] == 0).all()
        am = gdn.ancestor_matrix(par)
        bits = ((anc[:, :n, None] >> np.arange(32, dtype=np.uint32)) & 1).astype(bool)  # [w, i, b]
        got = bits.transpose(1, 0, 2).reshape(n, nmax)
        assert (got[:, :n] == am).all() and not got[:, n:].any()
        for i in range(n):
            js = np.nonzero(am[i])[0]
            assert (path[i, dep[js] - 1] == js).all()


@pytest.mark.parametrize("sizes,HK,H", [([128] * 8, 16, 32), ([16, 37, 64, 1, 128, 5, 64, 33], 16, 48),
                                        ([20, 9], 2, 4)])
def test_tree_gdn_ctx_two_layers(sizes, HK, H):
    """One context, two layers with different data on the same trees: identical to the parent-pointer path
    (bit for bit) and within tolerance of the oracle."""
    import tree_gdn_kernel

    d1 = gdn_inputs(sizes, HK, H, 128, seed=70)
    d2 = gdn_inputs(sizes, HK, H, 128, seed=71, parents=d1["parents"])
    t1, t2 = _dev(d1), _dev(d2)
    print(f"case: ctx sizes={sizes} HK={HK} H={H}", flush=True)
    ctx = tree_gdn_kernel.tree_context(t1["parents"], t1["cu_nodes"], max_nodes=max(sizes))
    for d, t in ((d1, t1), (d2, t2)):
        u, o = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], None,
                                               t["cu_nodes"], ctx=ctx)
        u2, o2 = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"],
                                                 t["parents"], t["cu_nodes"], max_nodes=max(sizes))
        torch.cuda.synchronize()
        assert torch.equal(u, u2) and torch.equal(o, o2)
        u_ref, o_ref = _oracle(d)
        eu, eo = _rel(u.cpu().numpy(), u_ref), _rel(o.cpu().numpy(), o_ref)
        print(f"rel err u {eu:.2e} o {eo:.2e}")
        assert eu <= RTOL and eo <= RTOL


def test_tree_gdn_ctx_from_anc8():
    """A context built from the reference's anc8 input of one tree."""
    import tree_gdn_kernel

    d = gdn_inputs(64, 16, 32, 128, seed=1)
    t = _dev(d)
    anc8 = torch.from_numpy(gdn.ancestor_matrix(d["parents"]).astype(np.int8)).cuda()
    ctx = tree_gdn_kernel.tree_context(anc8=anc8)
    u, o = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], None,
                                           t["cu_nodes"], ctx=ctx)
    torch.cuda.synchronize()
    u_ref, o_ref = _oracle(d)
    assert _rel(u.cpu().numpy(), u_ref) <= RTOL and _rel(o.cpu().numpy(), o_ref) <= RTOL


def test_tree_gdn_ctx_rejects_bad_trees():
    """Too deep and non-topological trees are flagged when the context is built and rejected by the GDN call
    (NaN outputs); a context used with other request sizes is rejected with MFD_DEVERR_BAD_CONTEXT."""
    import tree_gdn_kernel

    d = gdn_inputs([17, 8, 12], 2, 4, 128, seed=8)
    d["parents"][:17] = np.arange(-1, 16, dtype=np.int32)  # 17-node chain: too deep
    d["parents"][17 + 3] = 5                                # node 3 of the second tree: parent after it
    t = _dev(d)
    err_ctx = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx = tree_gdn_kernel.tree_context(t["parents"], t["cu_nodes"], max_nodes=32, err_flag=err_ctx)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    u = torch.full((37, 4, 128), 7.0, device="cuda")
    o = torch.full((37, 4, 128), 7.0, device="cuda")
    tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], None, t["cu_nodes"],
                                    out=(u, o), err_flag=err, ctx=ctx)
    torch.cuda.synchronize()
    assert int(err_ctx.item()) == 2 | 4 and int(err.item()) == 2 | 4
    assert bool(torch.isnan(u[:25]).all()) and bool(torch.isnan(o[:25]).all())
    sub = slice(25, 37)
    u_ref, o_ref = _oracle(dict(d, parents=d["parents"][sub], cu_nodes=np.array([0, 12], dtype=np.int32),
                                q=d["q"][sub], k=d["k"][sub], v=d["v"][sub], g_cum=d["g_cum"][sub],
                                beta=d["beta"][sub], s0=d["s0"][2:]))
    assert _rel(u[sub].cpu().numpy(), u_ref) <= RTOL and _rel(o[sub].cpu().numpy(), o_ref) <= RTOL
    # same R and N, other request sizes: every request of the other sizes is rejected
    cu2 = torch.tensor([0, 10, 25, 37], dtype=torch.int32, device="cuda")
    err.zero_()
    u.fill_(7.0)
    tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], None, cu2,
                                    out=(u, o), err_flag=err, ctx=ctx)
    torch.cuda.synchronize()
    assert int(err.item()) & 8
    assert bool(torch.isnan(u[:25]).all())


# ---------------------------------------------------------------- gates


def _gates_case(sizes, H, seed, dtype):
    from oracle.synth import random_tree

    gen = torch.Generator().manual_seed(seed)
    parents = np.concatenate([random_tree(n, 16, gen) for n in sizes]).astype(np.int32)
    N = int(sum(sizes))
    wide = torch.randn(N, 2 * H + 3, generator=gen) * 4  # a and b are strided column slices of one tensor
    a, b = wide[:, :H], wide[:, H + 3:]
    A_log = torch.randn(H, generator=gen) * 0.5
    dt = torch.randn(H, generator=gen)
    cu = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    return wide.to(dtype), a, b, A_log, dt, parents, cu


def _gates_ref(a, b, A_log, dt, parents, cu, dtype):
    a = a.to(dtype).float().numpy()
    b = b.to(dtype).float().numpy()
    G = np.zeros_like(a, dtype=np.float64)
    beta = np.zeros_like(a, dtype=np.float64)
    for r in range(len(cu) - 1):
        s, e = cu[r], cu[r + 1]
        G[s:e], beta[s:e] = gdn.gates(a[s:e], b[s:e], A_log.numpy(), dt.numpy(), parents[s:e])
    return G, beta


@pytest.mark.parametrize("sizes,H,dtype", [([64], 32, torch.bfloat16), ([128] * 8, 32, torch.float32),
                                           ([17, 64, 3, 40, 1], 48, torch.bfloat16)])
def test_tree_gates(sizes, H, dtype):
    import tree_gdn_kernel

    wide, a, b, A_log, dt, parents, cu = _gates_case(sizes, H, 77 + len(sizes), dtype)
    print(f"case: gates sizes={sizes} H={H} {dtype}", flush=True)
    wd = wide.cuda()
    G, beta = tree_gdn_kernel.tree_gates(wd[:, :H], wd[:, H + 3:], A_log.cuda(), dt.cuda(),
                                         parents=torch.from_numpy(parents).cuda(), cu_nodes=torch.from_numpy(cu).cuda())
    torch.cuda.synchronize()
    G_ref, beta_ref = _gates_ref(a, b, A_log, dt, parents, cu, dtype)
    np.testing.assert_allclose(beta.cpu().numpy(), beta_ref, rtol=0, atol=1e-6)
    np.testing.assert_allclose(G.cpu().numpy(), G_ref, rtol=0, atol=1e-5 * np.abs(G_ref).max())


def test_tree_gates_anc8_and_into_tree_gdn():
    """Single tree given by its ancestor matrix (the HF TreeContext form); the gates then feed tree_gdn,
    which must match the oracle fed with the oracle's gates."""
    import tree_gdn_kernel

    d = gdn_inputs(64, 16, 32, 128, seed=21)
    wide, a, b, A_log, dt, _, _ = _gates_case([64], 32, 9, torch.bfloat16)
    parents = d["parents"]
    anc8 = torch.from_numpy(gdn.ancestor_matrix(parents).astype(np.int8)).cuda()
    G, beta = tree_gdn_kernel.tree_gates(wide[:, :32].cuda(), wide[:, 35:].cuda(), A_log.cuda(), dt.cuda(), anc8=anc8)
    G_ref, beta_ref = gdn.gates(a.to(torch.bfloat16).float().numpy(), b.to(torch.bfloat16).float().numpy(),
                                A_log.numpy(), dt.numpy(), parents)
    np.testing.assert_allclose(G.cpu().numpy(), G_ref, rtol=0, atol=1e-5 * np.abs(G_ref).max())
    dev = torch.device("cuda")
    bf = lambda x: torch.from_numpy(x).to(dev).to(torch.bfloat16)
    u, o = tree_gdn_kernel.tree_gdn(bf(d["q"]), bf(d["k"]), bf(d["v"]), G, beta,
                                    torch.from_numpy(d["s0"][0]).to(dev), anc8)
    torch.cuda.synchronize()
    u_ref, o_ref = gdn.tree_gdn_chunk(d["q"], d["k"], d["v"], G_ref, beta_ref, d["s0"][0], parents)
    assert np.abs(u.cpu().numpy() - u_ref).max() <= RTOL * np.abs(u_ref).max()
    assert np.abs(o.cpu().numpy() - o_ref).max() <= RTOL * np.abs(o_ref).max()


def test_tree_gates_rejects_non_topological_parents():
    import mfd_hip  # noqa: F401
    import tree_gdn_kernel

    H = 4
    a = torch.zeros(5, H, device="cuda")
    par = torch.tensor([-1, 0, 3, 1, 2], dtype=torch.int32, device="cuda")  # node 2's parent comes after it
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    G, _ = tree_gdn_kernel.tree_gates(a, a, torch.zeros(H, device="cuda"), torch.zeros(H, device="cuda"),
                                      parents=par, err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 4
    assert torch.isnan(G[2]).all() and torch.isfinite(G[:2]).all()
