"""Benchmark of the MFD hot path on one MI355X.

Headline (BASELINE.json metric "tree-verify nodes/sec per GDN layer + mode-attn us/step, % of HBM
roofline"): configuration 3 — tree-GDN verify of 8 requests x 128-node random trees (depth <= 16),
16 q/k heads, 32 v heads, head dim 128, bf16 q/k/v, fp32 state and gates, 24 layers with independent
seeds. One step = the 24 layer calls (one verify forward's GDN layers), captured in a HIP graph and
replayed; inputs are resident in HBM before the timed region. ``value`` = nodes verified per second
per GDN layer = 1024 nodes / (step time / 24).

The JSON line also carries the roofline of the dominant kernel (algorithmic bytes per launch over the
kernel's average duration, HIP events on the launch stream) and the CPU baseline (the float32 torch
dense triangular-solve restatement of the reference's CPU path, timed on this host's cores).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(REPO, "multi-future-drafting_amd"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0

# config 3 shape
R3, N3, HK3, H3, D = 8, 128, 16, 32, 128
LAYERS = 24


def gdn_alg_bytes(N, R, HK, H, D=128):
    """Algorithmic bytes of one tree-GDN launch: s0 fp32 + q,k,v bf16 + g,beta fp32 + parents int32 + u,o fp32."""
    return R * H * D * D * 4 + N * HK * D * 2 * 2 + N * H * D * 2 + N * H * 4 * 2 + N * 4 + N * H * D * 4 * 2


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_gdn_layers(torch, n_layers):
    import numpy as np

    from oracle.synth import gdn_inputs

    dev = torch.device("cuda")
    layers = []
    for layer in range(n_layers):
        d = gdn_inputs([N3] * R3, HK3, H3, D, seed=3000 + layer)
        bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(torch.bfloat16)
        f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
        layers.append(dict(q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), g_cum=f32(d["g_cum"]), beta=f32(d["beta"]),
                           s0=f32(d["s0"]), parents=torch.from_numpy(d["parents"]).to(dev),
                           cu_nodes=torch.from_numpy(d["cu_nodes"]).to(dev),
                           u=torch.empty(R3 * N3, H3, D, device=dev), o=torch.empty(R3 * N3, H3, D, device=dev),
                           host=d))
    return layers


def bench_gdn(torch, steps, warmup):
    import tree_gdn_kernel

    log("building config-3 inputs (24 layers)")
    layers = make_gdn_layers(torch, LAYERS)

    def step():
        for L in layers:
            tree_gdn_kernel.tree_gdn_varlen(L["q"], L["k"], L["v"], L["g_cum"], L["beta"], L["s0"], L["parents"],
                                            L["cu_nodes"], max_nodes=N3, out=(L["u"], L["o"]))

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        step()  # eager run (also the parity spot check below)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # graph.replay() launches on the current stream: the events go on that same stream
    replay_stream = torch.cuda.current_stream()
    t0 = time.perf_counter()
    start.record(replay_stream)
    for _ in range(steps):
        graph.replay()
    end.record(replay_stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = start.elapsed_time(end)
    ms_step = ms_total / steps
    us_launch = ms_total * 1000.0 / (steps * LAYERS)
    log(f"tree_gdn: {us_launch:.2f} us per layer launch, {ms_step:.3f} ms per 24-layer step (wall {wall:.3f} s)")
    # spot parity of the last layer against the float64 oracle
    import numpy as np

    from oracle import gdn

    L = layers[-1]
    hd = L["host"]
    u_ref, o_ref = gdn.tree_gdn_varlen(hd["q"], hd["k"], hd["v"], hd["g_cum"], hd["beta"], hd["s0"], hd["parents"],
                                       hd["cu_nodes"])
    rel = max(float(np.abs(L["u"].cpu().numpy() - u_ref).max() / np.abs(u_ref).max()),
              float(np.abs(L["o"].cpu().numpy() - o_ref).max() / np.abs(o_ref).max()))
    log(f"tree_gdn parity (last layer) rel err {rel:.2e}")
    return dict(ms_step=ms_step, us_launch=us_launch, parity_rel=rel, layers=layers)


def cpu_baseline_gdn(torch, layers, budget_s=12.0):
    """float32 torch dense triangular solve per head (the reference's CPU path semantics), one layer of
    config 3 (8 trees), repeated within a bounded time budget; median per layer."""
    import numpy as np

    from oracle import gdn

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    hd = layers[0]["host"]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    per_tree = []
    cu = hd["cu_nodes"]
    for r in range(R3):
        a, b = int(cu[r]), int(cu[r + 1])
        per_tree.append((t(hd["q"][a:b]), t(hd["k"][a:b]), t(hd["v"][a:b]), t(hd["g_cum"][a:b]),
                         t(hd["beta"][a:b]), t(hd["s0"][r]), hd["parents"][a:b]))

    def one_layer():
        for args in per_tree:
            gdn.tree_gdn_dense_torch(*args)

    for _ in range(3):
        one_layer()
    times = []
    t_start = time.perf_counter()
    while len(times) < 20 or (time.perf_counter() - t_start < budget_s and len(times) < 200):
        t0 = time.perf_counter()
        one_layer()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 3 * budget_s:
            break
    med = statistics.median(times)
    return dict(value=R3 * N3 / med, unit="nodes/s per GDN layer", cores=cores, kind="port",
                sample=f"config-3 layer 0 (8 x 128-node trees, H32/HK16/D128), float32 torch dense solve, "
                       f"median of {len(times)} reps after 3 warm-ups ({med * 1e3:.2f} ms per layer)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: every part of the hot path is a "
                                   "single-GPU kernel (see DESIGN.md for how it would shard); run --gpus 1"}))
        sys.exit(2)
    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    gdn_res = bench_gdn(torch, args.steps, args.warmup)
    nodes_per_s = R3 * N3 / (gdn_res["us_launch"] * 1e-6)
    alg = gdn_alg_bytes(R3 * N3, R3, HK3, H3)
    achieved = alg / (gdn_res["us_launch"] * 1e-6) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline (float32 torch)")
        cpu = cpu_baseline_gdn(torch, gdn_res["layers"])
    out = {
        "metric": "tree-verify nodes/sec per GDN layer + mode-attn us/step, % of HBM roofline",
        "value": nodes_per_s,
        "unit": "nodes/s per GDN layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": gdn_res["ms_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 inputs, f32 state/outputs (bf16 hi+lo MFMA)",
        "data": "synthetic (seeded, BASELINE.json config 3)",
        "config": {"workload": "config 3: tree-GDN verify, 8 requests x 128-node trees (depth<=16), "
                               "HK16/H32/D128, 24 layers per step", "requests": R3, "nodes_per_tree": N3,
                   "layers_per_step": LAYERS, "parallelism": "single GPU"},
        "gdn_us_per_layer": gdn_res["us_launch"],
        "gdn_parity_rel_err": gdn_res["parity_rel"],
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None, "kernel": "tree_gdn_kernel<4>",
                     "alg_bytes_per_launch": alg},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
