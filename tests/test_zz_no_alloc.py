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


_CAPTURE_CHILD = r"""
import sys
import numpy as np
import torch
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import mfd_hip
from oracle import gdn
from oracle.synth import gdn_inputs

sizes, HK, H = [200, 140], 2, 4
R, N, mx = len(sizes), sum(sizes), max(sizes)
dev = torch.device("cuda")
ins = {n: torch.zeros(N, HK if n in ("q", "k") else H, 128, dtype=torch.bfloat16, device=dev) for n in ("q", "k", "v")}
ins["g_cum"] = torch.zeros(N, H, device=dev)
ins["beta"] = torch.zeros(N, H, device=dev)
ins["s0"] = torch.zeros(R, H, 128, 128, device=dev)
ins["parents"] = torch.zeros(N, dtype=torch.int32, device=dev)
ins["cu_nodes"] = torch.zeros(R + 1, dtype=torch.int32, device=dev)
u = torch.zeros(N, H, 128, device=dev)
o = torch.zeros(N, H, 128, device=dev)
args = [ins[n].data_ptr() for n in ("q", "k", "v", "g_cum", "beta", "s0", "parents")] + [None, ins["cu_nodes"].data_ptr(),
        R, N, HK, H, 128, mx, u.data_ptr(), o.data_ptr(), None]
graph = torch.cuda.CUDAGraph()
stream = torch.cuda.Stream()
torch.cuda.synchronize()
with torch.cuda.stream(stream):
    with torch.cuda.graph(graph, stream=stream):
        # the first mfd_tree_gdn_noalloc call of this process, under capture (max_nodes > 128: the large-tree
        # path, whose workspace is the static scratch)
        mfd_hip.call("mfd_tree_gdn_noalloc", *args, stream.cuda_stream)
for seed in (11, 12):
    d = gdn_inputs(sizes, HK, H, 128, seed=seed)
    for n in ("q", "k", "v"):
        ins[n].copy_(torch.from_numpy(d[n]).to(torch.bfloat16))
    for n in ("g_cum", "beta", "s0"):
        ins[n].copy_(torch.from_numpy(np.ascontiguousarray(d[n], dtype=np.float32)))
    ins["parents"].copy_(torch.from_numpy(d["parents"]))
    ins["cu_nodes"].copy_(torch.from_numpy(d["cu_nodes"]))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    u_ref, o_ref = gdn.tree_gdn_varlen(d["q"], d["k"], d["v"], d["g_cum"], d["beta"], d["s0"], d["parents"],
                                       d["cu_nodes"])
    for got, ref in ((u, u_ref), (o, o_ref)):
        err = float(np.abs(got.cpu().numpy() - ref).max() / np.abs(ref).max())
        assert err <= 2e-3, (seed, err)
print("capture child ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture(tmp_path):
    """In a fresh process, the first mfd_tree_gdn_noalloc call on the device is made under HIP graph capture (the
    scratch address is resolved then); the graph replays correctly with new inputs, twice."""
    import os
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = tmp_path / "capture_child.py"
    script.write_text(_CAPTURE_CHILD)
    print("case: noalloc first call under capture (child process)", flush=True)
    res = subprocess.run([sys.executable, str(script), os.path.join(repo, "multi-future-drafting_amd"), repo],
                         capture_output=True, text=True, timeout=110)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "capture child ok" in res.stdout
