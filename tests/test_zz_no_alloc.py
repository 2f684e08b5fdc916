"""The allocation-free tree-GDN entry point (mfd_tree_gdn_noalloc, static device scratch) through the C ABI:
its outputs equal mfd_tree_gdn's (the workspace form) bit for bit, and the oracle's within the 2e-3 bound, on two
calls in a row, the second smaller; oversized requests are refused before any launch."""

import numpy as np
import pytest
import torch

from oracle import gdn
from oracle.synth import gdn_inputs

pytestmark = pytest.mark.gpu


def _dev(d):
    dev = torch.device("cuda")
    bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(torch.bfloat16)
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
    return dict(q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), g_cum=f32(d["g_cum"]), beta=f32(d["beta"]),
                s0=f32(d["s0"]), parents=torch.from_numpy(d["parents"]).to(dev),
                cu_nodes=torch.from_numpy(d["cu_nodes"]).to(dev))


def _run(name, t, R, N, HK, H, max_nodes, ws=None):
    import mfd_hip

    u = torch.full((N, H, 128), 7.0, device="cuda")
    o = torch.full((N, H, 128), 7.0, device="cuda")
    args = [t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(), t["g_cum"].data_ptr(), t["beta"].data_ptr(),
            t["s0"].data_ptr(), t["parents"].data_ptr(), None, t["cu_nodes"].data_ptr(), R, N, HK, H, 128, max_nodes,
            u.data_ptr(), o.data_ptr(), None]
    if name == "mfd_tree_gdn":
        args += [mfd_hip.ptr(ws), 0 if ws is None else ws.numel()]
    mfd_hip.call(name, *args, mfd_hip.stream_of(u))
    return u, o


@pytest.mark.parametrize("sizes_first,sizes_second,HK,H", [
    ([300, 257, 129], [140], 4, 8),   # large-tree path: the static scratch holds contexts and Gram rows
    ([128, 64], [20], 2, 4),          # fused path: no scratch in use
])
def test_noalloc_matches_workspace_entry_on_two_calls(sizes_first, sizes_second, HK, H):
    import mfd_hip

    for call, sizes in enumerate((sizes_first, sizes_second)):
        d = gdn_inputs(sizes, HK, H, 128, seed=900 + call)
        t = _dev(d)
        R, N, mx = len(sizes), sum(sizes), max(sizes)
        print(f"case: noalloc call {call} sizes={sizes} HK={HK} H={H}", flush=True)
        nbytes = mfd_hip.lib().mfd_tree_gdn_workspace_bytes(R, N, HK, mx, 0)
        ws = mfd_hip.workspace(nbytes, torch.device("cuda"))
        u_ws, o_ws = _run("mfd_tree_gdn", t, R, N, HK, H, mx, ws)
        u_na, o_na = _run("mfd_tree_gdn_noalloc", t, R, N, HK, H, mx)
        torch.cuda.synchronize()
        assert torch.equal(u_na, u_ws) and torch.equal(o_na, o_ws)
        u_ref, o_ref = gdn.tree_gdn_varlen(d["q"], d["k"], d["v"], d["g_cum"], d["beta"], d["s0"], d["parents"],
                                           d["cu_nodes"])
        for got, ref in ((u_na, u_ref), (o_na, o_ref)):
            assert np.abs(got.cpu().numpy() - ref).max() <= 2e-3 * np.abs(ref).max()


def test_noalloc_refuses_more_than_its_scratch():
    import mfd_hip

    lib = mfd_hip.lib()
    # 40000 nodes of 16 key heads: 80 MB of Gram rows, above the 16 MiB scratch; refused on the host
    assert lib.mfd_tree_gdn_workspace_bytes(100, 40000, 16, 512, 0) > 16 << 20
    rc = lib.mfd_tree_gdn_noalloc(16, 16, 16, 16, 16, 16, 16, None, 16, 100, 40000, 16, 32, 128, 512, 16, 16, None,
                                  None)
    assert rc == -2 and b"scratch" in lib.mfd_last_error()
