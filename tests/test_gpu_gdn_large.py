"""GPU parity of the large-tree tree-GDN path (trees of 129..512 nodes: Gram kernel + path-local solve) through
the C ABI, against the float64 oracle.

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


def _check(u, o, d, tag):
    torch.cuda.synchronize()
    u_ref, o_ref = _oracle(d)
    eu, eo = _rel(u.cpu().numpy(), u_ref), _rel(o.cpu().numpy(), o_ref)
    print(f"{tag}: rel err u {eu:.2e} o {eo:.2e}", flush=True)
    assert eu <= RTOL and eo <= RTOL


def _reparent(d, spans):
    """Replace the trees of some requests: ``spans`` = [(request, parents array)]; G recomputed along them."""
    g = d["g"].astype(np.float64)
    for r, par in spans:
        a, b = d["cu_nodes"][r], d["cu_nodes"][r + 1]
        assert len(par) == b - a
        d["parents"][a:b] = par
        d["g_cum"][a:b] = gdn.g_cum_from_g(g[a:b], d["parents"][a:b]).astype(np.float32)
    return d


def test_tree_gdn_257_nodes_anc8_api():
    """The HF default budget of 256 drafts gives a 257-node tree: the reference's tree_gdn(..., anc8) signature,
    HK 16, H 32."""
    import tree_gdn_kernel

    d = gdn_inputs(257, 16, 32, 128, seed=257)
    t = _dev(d)
    anc8 = torch.from_numpy(gdn.ancestor_matrix(d["parents"]).astype(np.int8)).cuda()
    print("case: anc8 n=257 HK=16 H=32", flush=True)
    u, o = tree_gdn_kernel.tree_gdn(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"][0], anc8)
    _check(u, o, d, "n=257")


@pytest.mark.parametrize("sizes,HK,H", [
    ([257] * 4, 16, 32),                 # 4 x 257 ragged, config shapes
    ([300, 129, 512, 1, 64, 200], 4, 12),  # mixed sizes around the path switch, GQA 3, root only
    ([512], 2, 2),                       # largest tree, no GQA
    ([129, 257, 140], 4, 8),             # 256 workgroups: the one-launch form (Gram chunks inside the main kernel)
])
def test_tree_gdn_large_varlen(sizes, HK, H):
    import tree_gdn_kernel

    d = gdn_inputs(sizes, HK, H, 128, seed=500 + len(sizes))
    t = _dev(d)
    print(f"case: large varlen sizes={sizes} HK={HK} H={H}", flush=True)
    u, o = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], t["parents"],
                                           t["cu_nodes"], max_nodes=max(sizes))
    _check(u, o, d, f"sizes={sizes}")


def test_tree_gdn_large_one_launch_two_streams():
    """Two streams running the one-launch form at once (one 257-node tree each, HK 16 / H 32: 256 workgroups per
    call, so the second call's workgroups start as the first's end): each stream has hand-over words of its own."""
    import tree_gdn_kernel

    ds = [gdn_inputs(257, 16, 32, 128, seed=31 + i) for i in range(2)]
    ts = [_dev(d) for d in ds]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    print("case: one-launch form on two streams, n=257 HK=16 H=32", flush=True)
    outs = []
    for rep in range(3):
        for i in range(2):
            streams[i].wait_stream(torch.cuda.current_stream())
            t = ts[i]
            with torch.cuda.stream(streams[i]):
                uo = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"],
                                                     t["parents"], t["cu_nodes"], max_nodes=257)
            outs.append((i, uo))
    torch.cuda.synchronize()
    for i, (u, o) in outs:
        _check(u, o, ds[i], f"stream {i}")


def test_tree_gdn_large_one_launch_many_calls():
    """The one-launch form's hand-over words carry a call count from call to call: 40 calls in a row (no host
    synchronisation between them), interleaved with two-kernel calls of another shape, all bit-identical to the
    first and within tolerance of the oracle."""
    import tree_gdn_kernel

    d1 = gdn_inputs(257, 16, 32, 128, seed=71)        # 256 workgroups: the one-launch form
    d4 = gdn_inputs([257] * 4, 16, 32, 128, seed=72)  # 512 workgroups: Gram kernel + main kernel
    t1, t4 = _dev(d1), _dev(d4)
    call = lambda t, mx: tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"],
                                                         t["parents"], t["cu_nodes"], max_nodes=mx)
    print("case: one-launch form, 40 calls interleaved with 4 x 257", flush=True)
    first1, first4 = call(t1, 257), call(t4, 257)
    outs = []
    for i in range(40):
        outs.append(call(t1, 257))
        if i % 8 == 0:
            outs.append(call(t4, 257))
    torch.cuda.synchronize()
    for u, o in outs:
        ref = first1 if u.shape[0] == 257 else first4
        assert torch.equal(u, ref[0]) and torch.equal(o, ref[1])
    _check(*first1, d1, "one launch")
    _check(*first4, d4, "two kernels")


def test_tree_gdn_large_chain_and_star():
    """A 300-node tree holding a 16-node chain (the deepest allowed path) and a 512-node star (depth 2), and
    a 200-node two-level broom, in one launch."""
    import tree_gdn_kernel

    d = gdn_inputs([300, 512, 200], 2, 4, 128, seed=9)
    from oracle.synth import random_tree

    gen = torch.Generator().manual_seed(99)
    p0 = random_tree(300, 16, gen)
    p0[:16] = np.arange(-1, 15, dtype=np.int32)  # nodes 0..15: a chain of 16
    # keep the later nodes within depth 16: hang any node under the chain's tail on node 0
    dep = np.zeros(300, dtype=np.int64)
    for i in range(300):
        dep[i] = 1 if p0[i] < 0 else dep[p0[i]] + 1
        if dep[i] > 16:
            p0[i] = 0
            dep[i] = 2
    star = np.array([-1] + [0] * 511, dtype=np.int32)
    broom = np.empty(200, dtype=np.int32)
    broom[:16] = np.arange(-1, 15)        # a 16-node chain
    broom[16:] = np.arange(16, 200) % 15  # every other node hangs on one of the chain's first 15 nodes
    d = _reparent(d, [(0, p0), (1, star), (2, broom)])
    assert gdn.depths_from_parents(d["parents"][:300]).max() == 16
    t = _dev(d)
    u, o = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], t["parents"],
                                           t["cu_nodes"], max_nodes=512)
    _check(u, o, d, "chain/star/broom")


def _parse_large_ctx(buf, R, nmax):
    """Large-tree context blocks as (path [R, nmax, 16] u16, depth [R, nmax] u8, header)."""
    raw = buf.cpu().numpy()
    blk = 32 * nmax + nmax + 16
    assert raw.size == R * blk
    out = []
    for r in range(R):
        b = raw[r * blk:(r + 1) * blk]
        path = b[:32 * nmax].view(np.uint16).reshape(nmax, 16)
        depth = b[32 * nmax:33 * nmax]
        hdr = b[33 * nmax:33 * nmax + 16].view(np.int32)
        out.append((path, depth, hdr))
    return out


@pytest.mark.parametrize("sizes,max_nodes,nmax", [([257, 3, 130], 257, 512), ([200, 129], 256, 256)])
def test_large_tree_context_contents(sizes, max_nodes, nmax):
    """Large-layout context against the oracle: depth, path[i][depth(j) - 1] = j for every ancestor j, the
    slots past the depth hold i itself."""
    import tree_gdn_kernel

    d = gdn_inputs(sizes, 2, 4, 128, seed=60 + len(sizes))
    t = _dev(d)
    ctx = tree_gdn_kernel.tree_context(t["parents"], t["cu_nodes"], max_nodes=max_nodes)
    torch.cuda.synchronize()
    for r, (path, depth, hdr) in enumerate(_parse_large_ctx(ctx.buf, len(sizes), nmax)):
        a, b = d["cu_nodes"][r], d["cu_nodes"][r + 1]
        n = b - a
        par = d["parents"][a:b]
        assert hdr[0] == 0 and hdr[1] == n and hdr[2] == nmax
        dep = gdn.depths_from_parents(par)
        assert (depth[:n] == dep).all() and (depth[n:] == 0).all()
        am = gdn.ancestor_matrix(par)
        for i in range(n):
            js = np.nonzero(am[i])[0]
            assert (path[i, dep[js] - 1] == js).all()
            assert (path[i, dep[i]:] == i).all()


def test_tree_gdn_large_ctx_two_layers_and_graph():
    """One large-tree context for two layers: bit-identical to the parent-pointer call, within tolerance of the
    oracle; then the same call captured in a HIP graph and replayed with new inputs."""
    import tree_gdn_kernel

    sizes = [257, 140, 300]
    d1 = gdn_inputs(sizes, 4, 8, 128, seed=80)
    d2 = gdn_inputs(sizes, 4, 8, 128, seed=81, parents=d1["parents"])
    t1, t2 = _dev(d1), _dev(d2)
    ctx = tree_gdn_kernel.tree_context(t1["parents"], t1["cu_nodes"], max_nodes=300)
    for d, t in ((d1, t1), (d2, t2)):
        u, o = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], None,
                                               t["cu_nodes"], ctx=ctx)
        u2, o2 = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"],
                                                 t["parents"], t["cu_nodes"], max_nodes=300)
        torch.cuda.synchronize()
        assert torch.equal(u, u2) and torch.equal(o, o2)
        _check(u, o, d, "ctx layer")
    # graph capture: the workspace is allocated inside the captured call (graph-private pool)
    N = sum(sizes)
    u = torch.empty(N, 8, 128, device="cuda")
    o = torch.empty_like(u)
    t = _dev(d1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], None,
                                        t["cu_nodes"], out=(u, o), ctx=ctx)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], None,
                                        t["cu_nodes"], out=(u, o), ctx=ctx)
    for d in (d2, d1, d2):
        t2 = _dev(d)
        for key in t:
            t[key].copy_(t2[key])
        graph.replay()
        _check(u, o, d, "graph replay")


def test_tree_gdn_large_rejects_too_deep_tree():
    """A 300-node tree with a 17-node root path is rejected (NaN outputs, MFD_DEVERR_TOO_DEEP); the other
    request of the launch is computed."""
    import tree_gdn_kernel

    d = gdn_inputs([300, 150], 2, 4, 128, seed=12)
    par = d["parents"][:300].copy()
    par[:17] = np.arange(-1, 16, dtype=np.int32)
    d["parents"][:300] = par
    t = _dev(d)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    u, o = tree_gdn_kernel.tree_gdn_varlen(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"], t["parents"],
                                           t["cu_nodes"], max_nodes=300, err_flag=err)
    torch.cuda.synchronize()
    assert int(err.item()) & 2
    assert bool(torch.isnan(u[:300]).all()) and bool(torch.isnan(o[:300]).all())
    sub = slice(300, 450)
    u_ref, o_ref = _oracle(dict(d, parents=d["parents"][sub], cu_nodes=np.array([0, 150], dtype=np.int32),
                                q=d["q"][sub], k=d["k"][sub], v=d["v"][sub], g_cum=d["g_cum"][sub],
                                beta=d["beta"][sub], s0=d["s0"][1:]))
    assert _rel(u[sub].cpu().numpy(), u_ref) <= RTOL and _rel(o[sub].cpu().numpy(), o_ref) <= RTOL


def test_tree_gdn_hf_api_rejection_is_visible():
    """The HF signature has no error flag: a 17-node chain passed through tree_gdn(..., anc8) must come back as
    NaN, not as stale memory (fused and large-tree paths)."""
    import tree_gdn_kernel

    for n in (40, 200):
        d = gdn_inputs(n, 2, 4, 128, seed=13)
        d["parents"][:17] = np.arange(-1, 16, dtype=np.int32)
        t = _dev(d)
        anc8 = torch.from_numpy(gdn.ancestor_matrix(d["parents"]).astype(np.int8)).cuda()
        u, o = tree_gdn_kernel.tree_gdn(t["q"], t["k"], t["v"], t["g_cum"], t["beta"], t["s0"][0], anc8)
        torch.cuda.synchronize()
        assert bool(torch.isnan(u).all()) and bool(torch.isnan(o).all()), n
