"""Benchmark of the MFD hot path on one MI355X.

Headline (BASELINE.json metric "tree-verify nodes/sec per GDN layer + mode-attn us/step, % of HBM roofline"):
configuration 3 — tree-GDN verify of 8 requests x 128-node random trees (depth <= 16), 16 q/k heads, 32 v heads,
head dim 128, bf16 q/k/v, fp32 state and gates, 24 layers with independent seeds. One step = the 24 layer calls
(one verify forward's GDN layers), captured in a HIP graph and replayed; inputs are resident in HBM before the
timed region. ``value`` = nodes verified per second per GDN layer = 1024 nodes / (step time / 24).

The same JSON line carries the other parts of the path at their configurations (mode attention config 2 and
the paged config 4, GDN config 0 and the ragged config 4, the config-1 logits step and tree builder), the
roofline of the dominant kernel (algorithmic bytes per launch over its average duration, HIP events on the
launch stream) and the CPU baseline (the float32 torch dense triangular-solve restatement of the reference's
CPU path, timed on this host's cores).
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
BF16_PEAK_TFLOPS = 2500.0

# config 3 shape
R3, N3, HK3, H3, D = 8, 128, 16, 32, 128
LAYERS = 24
# single-call workloads are captured INNER times per graph, so that the graph launch (about 10 us per
# replay here) is amortised as it is inside a serving step's graph; their inputs stay the same across calls
INNER = 8
# kernels of a few microseconds: a graph of 8 of them is shorter than the host's submission of the next replay,
# so they are captured 64 per graph
SMALL_INNER = 64


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gdn_alg_bytes(N, R, HK, H, D=128):
    """Algorithmic bytes of one tree-GDN launch: s0 fp32 + q,k,v bf16 + g,beta fp32 + parents int32 + u,o fp32."""
    return R * H * D * D * 4 + N * HK * D * 2 * 2 + N * H * D * 2 + N * H * 4 * 2 + N * 4 + N * H * D * 4 * 2


def attn_alg(ctx_lens, K, L, H, Hkv, D=128, table_bytes=0):
    """Algorithmic bytes / flops of one mode-attention step: Q + context K/V + block K/V + O (bf16) + table."""
    KL = K * L
    nbytes = sum(KL * H * D * 2 * 2 + c * Hkv * D * 2 * 2 + KL * Hkv * D * 2 * 2 for c in ctx_lens) + table_bytes
    flops = sum(4 * H * D * KL * (c + L) for c in ctx_lens)
    return nbytes, flops


def time_graph(torch, fn, steps, warmup, inner=1):
    """Capture ``inner`` calls of fn in a HIP graph; replay; HIP events on the replay stream. Returns us per call."""
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(inner):
            fn()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    replay_stream = torch.cuda.current_stream()  # graph.replay() launches on the current stream
    start.record(replay_stream)
    for _ in range(steps):
        graph.replay()
    end.record(replay_stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / (steps * inner)


def cpu_median(fn, min_reps=5, budget_s=6.0, max_reps=200):
    for _ in range(2):
        fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_reps or (time.perf_counter() - t_start < budget_s and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


# ------------------------------------------------------------------------------------------------ GDN


def make_gdn_layers(torch, n_layers, sizes=None, HK=HK3, H=H3, seed0=3000):
    import numpy as np

    from oracle.synth import gdn_inputs

    sizes = sizes or [N3] * R3
    dev = torch.device("cuda")
    layers = []
    trees = None  # every layer of a verify round works on the same trees
    for layer in range(n_layers):
        d = gdn_inputs(sizes, HK, H, D, seed=seed0 + layer, parents=trees)
        trees = d["parents"]
        bf = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(torch.bfloat16)
        f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
        N = sum(sizes)
        layers.append(dict(q=bf(d["q"]), k=bf(d["k"]), v=bf(d["v"]), g_cum=f32(d["g_cum"]), beta=f32(d["beta"]),
                           s0=f32(d["s0"]), parents=torch.from_numpy(d["parents"]).to(dev),
                           cu_nodes=torch.from_numpy(d["cu_nodes"]).to(dev), max_nodes=max(sizes),
                           u=torch.empty(N, H, D, device=dev), o=torch.empty(N, H, D, device=dev), host=d))
    return layers


def gdn_call(tree_gdn_kernel, L, ctx=None):
    tree_gdn_kernel.tree_gdn_varlen(L["q"], L["k"], L["v"], L["g_cum"], L["beta"], L["s0"], L["parents"], L["cu_nodes"],
                                    max_nodes=L["max_nodes"], out=(L["u"], L["o"]), ctx=ctx)


def gdn_round(tree_gdn_kernel, layers, ctx):
    """One verify round of config 3: the tree context of the round's trees, then every layer."""
    L0 = layers[0]
    tree_gdn_kernel.tree_context(L0["parents"], L0["cu_nodes"], max_nodes=L0["max_nodes"], out=ctx)
    for L in layers:
        gdn_call(tree_gdn_kernel, L, ctx)


def gdn_parity(L):
    import numpy as np

    from oracle import gdn

    hd = L["host"]
    u_ref, o_ref = gdn.tree_gdn_varlen(hd["q"], hd["k"], hd["v"], hd["g_cum"], hd["beta"], hd["s0"], hd["parents"],
                                       hd["cu_nodes"])
    return max(float(np.abs(L["u"].cpu().numpy() - u_ref).max() / np.abs(u_ref).max()),
               float(np.abs(L["o"].cpu().numpy() - o_ref).max() / np.abs(o_ref).max()))


def bench_gdn(torch, steps, warmup):
    import tree_gdn_kernel

    log("config 3: building inputs (24 layers)")
    layers = make_gdn_layers(torch, LAYERS)
    L0 = layers[0]
    ctx = tree_gdn_kernel.tree_context(L0["parents"], L0["cu_nodes"], max_nodes=L0["max_nodes"])

    def step():
        gdn_round(tree_gdn_kernel, layers, ctx)

    us_launch = time_graph(torch, step, steps, warmup) / LAYERS
    log(f"config 3 tree_gdn: {us_launch:.2f} us per layer (tree context once per round + 24 layers, / 24)")
    # every layer of the timed round against the fp64 oracle (about a second of CPU time per layer)
    rel = max(gdn_parity(L) for L in layers)
    log(f"config 3 parity (all {len(layers)} layers) max rel err {rel:.2e}")
    return dict(us_launch=us_launch, ms_step=us_launch * LAYERS / 1000.0, parity_rel=rel, layers=layers)


def bench_gdn_small(torch, steps, warmup):
    """Config 0 (one 64-node tree, latency; the kernel walks the parents itself) and config 4 (16 ragged trees of
    U[16, 64] nodes, 48 v heads; per layer of a 24-layer round with the round's tree context, as config 3)."""
    import torch as _t

    import tree_gdn_kernel

    out = {}
    L0 = make_gdn_layers(torch, 1, sizes=[64], seed0=0)[0]
    us0 = time_graph(torch, lambda: gdn_call(tree_gdn_kernel, L0), steps, warmup, inner=INNER)
    out["config0_us_per_layer"] = us0
    out["config0_parity_rel_err"] = gdn_parity(L0)
    g = _t.Generator().manual_seed(4000)
    sizes = [int(x) for x in _t.randint(16, 65, (16,), generator=g)]
    L4 = make_gdn_layers(torch, 1, sizes=sizes, H=48, seed0=4000)[0]
    # a verify round as in config 3: the round's tree context once, then the layers (the same layer inputs
    # stand for each of the 24), per layer
    ctx4 = tree_gdn_kernel.tree_context(L4["parents"], L4["cu_nodes"], max_nodes=L4["max_nodes"])
    us4 = time_graph(torch, lambda: gdn_round(tree_gdn_kernel, [L4] * LAYERS, ctx4), steps, warmup) / LAYERS
    N4 = sum(sizes)
    b4 = gdn_alg_bytes(N4, 16, 16, 48)
    out["config4_nodes"] = N4
    out["config4_us_per_layer"] = us4
    out["config4_nodes_per_s"] = N4 / (us4 * 1e-6)
    out["config4_hbm_frac"] = b4 / (us4 * 1e-6) / (HBM_PEAK_GBS * 1e9)
    out["config4_parity_rel_err"] = gdn_parity(L4)
    log(f"GDN config 0: {us0:.2f} us; config 4 ({N4} nodes, H48): {us4:.2f} us")
    # the HF path's default tree budget of 256 (257-node trees, inference/hf/ddtree.py; guides/INFERENCE_HF.md:100
    # quotes 86 us per GDN layer for one such tree on its GPU): trees of more than 128 nodes take the large-tree
    # path. One tree and four trees, HK16 / H32, per layer of a 24-layer round with the round's tree context.
    for name, R in (("large1", 1), ("large4", 4)):
        Lb = make_gdn_layers(torch, 1, sizes=[257] * R, seed0=257 + R)[0]
        ctxb = tree_gdn_kernel.tree_context(Lb["parents"], Lb["cu_nodes"], max_nodes=Lb["max_nodes"])
        usb = time_graph(torch, lambda: gdn_round(tree_gdn_kernel, [Lb] * LAYERS, ctxb), steps, warmup) / LAYERS
        bb = gdn_alg_bytes(257 * R, R, 16, 32)
        out[f"{name}_nodes"] = 257 * R
        out[f"{name}_us_per_layer"] = usb
        out[f"{name}_hbm_frac"] = bb / (usb * 1e-6) / (HBM_PEAK_GBS * 1e9)
        out[f"{name}_parity_rel_err"] = gdn_parity(Lb)
        log(f"GDN {R} x 257 nodes: {usb:.2f} us per layer")
    out["large1_reference_us"] = 86.0  # guides/INFERENCE_HF.md:100 (RTX PRO 6000), for scale only
    return out


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

    med, n = cpu_median(one_layer, min_reps=20, budget_s=budget_s)
    return dict(value=R3 * N3 / med, unit="nodes/s per GDN layer", cores=cores, kind="port",
                sample=f"config-3 layer 0 (8 x 128-node trees, H32/HK16/D128), float32 torch dense solve, "
                       f"median of {n} reps after 2 warm-ups ({med * 1e3:.2f} ms per layer)")


# ------------------------------------------------------------------------------------------------ attention


def bench_attention(torch, steps, warmup, with_cpu):
    import mode_attention
    import paged_mode_attention as dm
    from oracle.synth import attention_inputs, paged_attention_inputs

    out = {}
    q, k, v = (t.cuda() for t in attention_inputs(2))
    scale = 128 ** -0.5
    fn = lambda: mode_attention.mode_block_attention(q, k, v, 8, 16, scale)
    us2 = time_graph(torch, fn, steps, warmup, inner=INNER)
    nb, fl = attn_alg([4096], 8, 16, 32, 8)
    t_b = max(nb / (HBM_PEAK_GBS * 1e9), fl / (BF16_PEAK_TFLOPS * 1e12))
    out["config2_us_per_step"] = us2
    out["config2_hbm_frac"] = nb / (us2 * 1e-6) / (HBM_PEAK_GBS * 1e9)
    out["config2_mfma_frac"] = fl / (us2 * 1e-6) / (BF16_PEAK_TFLOPS * 1e12)
    out["config2_roofline_frac"] = t_b / (us2 * 1e-6)
    log(f"mode attention config 2: {us2:.2f} us/step (MFMA {out['config2_mfma_frac']:.2%}, HBM {out['config2_hbm_frac']:.2%})")
    # the causal-in-block variant named by the configuration (the reference's default is bidirectional)
    fnc = lambda: mode_attention.mode_block_attention(q, k, v, 8, 16, scale, causal_in_block=True)
    us2c = time_graph(torch, fnc, steps, warmup, inner=INNER)
    out["config2_causal_us_per_step"] = us2c
    out["config2_causal_mfma_frac"] = fl / (us2c * 1e-6) / (BF16_PEAK_TFLOPS * 1e12)
    log(f"mode attention config 2, causal in block: {us2c:.2f} us/step")

    g = torch.Generator().manual_seed(4000)
    lens = [int(x) for x in torch.randint(1024, 8193, (16,), generator=g)]
    d = paged_attention_inputs(4000, lens, H=40, Hkv=8, page_size=64)
    pt = torch.zeros(18, d["page_table"].shape[1], dtype=torch.int32)
    pt[2:] = d["page_table"]
    dev = {kk: (vv.cuda() if torch.is_tensor(vv) else vv) for kk, vv in d.items()}
    ptc = pt.cuda()
    outbuf = torch.empty_like(dev["q"])
    fn4 = lambda: dm.paged_mode_block_attention(
        q=dev["q"], k_new=dev["k_new"], v_new=dev["v_new"], k_cache=dev["k_cache"], v_cache=dev["v_cache"],
        req_to_token=ptc, req_pool_indices=dev["req_pool_indices"], ctx_lens=dev["ctx_lens"], num_modes=8,
        block_size=16, scaling=scale, num_ctx_splits=-1, out=outbuf, page_size=64)
    us4 = time_graph(torch, fn4, steps, warmup)
    nb4, fl4 = attn_alg(lens, 8, 16, 40, 8, table_bytes=pt.numel() * 4)
    out["config4_us_per_step"] = us4
    out["config4_ctx_lens_mean"] = sum(lens) / len(lens)
    out["config4_hbm_frac"] = nb4 / (us4 * 1e-6) / (HBM_PEAK_GBS * 1e9)
    out["config4_mfma_frac"] = fl4 / (us4 * 1e-6) / (BF16_PEAK_TFLOPS * 1e12)
    out["config4_roofline_frac"] = max(nb4 / (HBM_PEAK_GBS * 1e9), fl4 / (BF16_PEAK_TFLOPS * 1e12)) / (us4 * 1e-6)
    log(f"mode attention config 4 (paged 64): {us4:.2f} us/step (MFMA {out['config4_mfma_frac']:.2%})")
    if with_cpu:
        from oracle import attention as oracle_attention

        qc, kc, vc = (t.float().numpy() for t in attention_inputs(2))
        med, n = cpu_median(lambda: oracle_attention.mode_attention(qc, kc, vc, 8, 16, scale), budget_s=8.0)
        out["config2_cpu_baseline"] = dict(value_us=med * 1e6, cores=len(os.sched_getaffinity(0)), kind="port",
                                           sample=f"config 2, the oracle's float64 numpy masked softmax per head "
                                                  f"(oracle/attention.py mode_attention, BLAS threads up to the core "
                                                  f"count), median of {n}")
    return out


# ------------------------------------------------------------------------------------------------ builder


def bench_builder(torch, steps, warmup, with_cpu):
    import numpy as np

    import tree_build_ext
    import tree_logits
    from oracle import builder as B
    from oracle.synth import builder_logits

    out = {}
    logits = builder_logits(1).cuda()
    us_lp = time_graph(torch, lambda: tree_logits.topk_logz(logits, 8, ids_dtype=torch.int32), steps, warmup,
                       inner=INNER)
    nb = logits.numel() * 2 + 128 * 8 * 8
    out["config1_logits_us"] = us_lp
    out["config1_logits_hbm_frac"] = nb / (us_lp * 1e-6) / (HBM_PEAK_GBS * 1e9)
    logp, ids = tree_logits.topk_logz(logits, 8, ids_dtype=torch.int32)
    lp4, id4, pr = logp[None], ids[None], torch.zeros(1, 8, device="cuda")
    us_heap = time_graph(torch, lambda: tree_build_ext.build_trees_device(lp4, id4, pr, 64, with_visibility=True),
                         steps, warmup, inner=INNER)
    out["config1_heap_us"] = us_heap
    out["config1_round_us"] = us_lp + us_heap
    log(f"builder config 1: logits {us_lp:.2f} us (HBM {out['config1_logits_hbm_frac']:.2%}), heap {us_heap:.2f} us")
    if with_cpu:
        lpc, idc = logp.cpu().numpy(), ids.cpu().numpy().astype(np.int64)
        ref = B.ref_sglang_builder()
        if ref is not None:
            lpt = torch.from_numpy(lpc).reshape(1, 8, 16, 8).contiguous()
            idt = torch.from_numpy(idc).reshape(1, 8, 16, 8).to(torch.int32).contiguous()
            prt = torch.zeros(1, 8)
            tr = torch.empty(1, 3, 65, dtype=torch.long)
            cn = torch.empty(1, dtype=torch.long)
            med, n = cpu_median(lambda: ref.build_trees(lpt, idt, prt, 1, 64, tr, cn), min_reps=50, budget_s=3.0,
                                max_reps=20000)
            out["config1_heap_cpu_baseline"] = dict(value_us=med * 1e6, cores=1, kind="reference",
                                                    sample=f"the reference's C++ build_trees (compiled from its "
                                                           f"sources), config 1, median of {n}")
        xl = builder_logits(1).reshape(128, -1)
        med, n = cpu_median(lambda: B.top_candidates(xl, 8), min_reps=3, budget_s=4.0)
        out["config1_logits_cpu_baseline"] = dict(value_us=med * 1e6, cores=1, kind="port",
                                                  sample=f"oracle C logits step (top-8 + log Z), config 1, median of {n}")
    return out


# ------------------------------------------------------------------------------------------------ prep + commit


def prep_inputs(torch, KC=4):
    """tree_prep inputs at the config-3 shape (8 x 128-node trees of depth <= 16, CD 8192, conv kernel KC), on
    the device: x, conv states, conv weights, windows, request offsets, then the trees' parents (host) and the
    generator, whose stream later inputs continue."""
    import numpy as np

    import tree_gdn_kernel
    from oracle.synth import random_tree

    CD = (2 * HK3 + H3) * D
    g = torch.Generator().manual_seed(3100)
    trees = [random_tree(N3, 16, g) for _ in range(R3)]
    parents = torch.from_numpy(np.concatenate(trees)).cuda()
    cu = torch.arange(0, R3 * N3 + 1, N3, dtype=torch.int32).cuda()
    x = (torch.randn(R3 * N3, CD, generator=g) * 0.5).to(torch.bfloat16).cuda()
    cs = (torch.randn(R3, CD, KC, generator=g) * 0.5).to(torch.bfloat16).cuda()
    w = (torch.randn(CD, KC, generator=g) * 0.5).to(torch.bfloat16).cuda()
    idx = tree_gdn_kernel.conv_index(parents, KC, cu)
    return x, cs, w, idx, cu, trees, g


def bench_prep_commit(torch, steps, warmup, with_cpu):
    """The steps either side of tree-GDN verification at the config-3 shape: tree_prep of 8 x 128 nodes
    (HK 16, H 32, D 128, conv kernel 4: conv over each node's window, SiLU, q / k normalisation) and the
    commit of one request's accepted 16-node path into 24 GDN layers' states and conv states."""
    import numpy as np

    import tree_gdn_kernel
    from oracle import gdn

    out = {}
    KC = 4
    CD = (2 * HK3 + H3) * D
    x, cs, w, idx, cu, trees, g = prep_inputs(torch)
    fn = lambda: tree_gdn_kernel.tree_prep(x, cs, idx, w, HK3, H3, D, cu_nodes=cu)
    us_prep = time_graph(torch, fn, steps, warmup, inner=INNER)
    nb_prep = x.numel() * 2 * 2 + cs.numel() * 2 + w.numel() * 2 + idx.numel() * 4
    out["prep_config3_us"] = us_prep
    out["prep_config3_hbm_frac"] = nb_prep / (us_prep * 1e-6) / (HBM_PEAK_GBS * 1e9)
    out["prep_alg_bytes"] = nb_prep
    log(f"tree_prep config 3 (1024 nodes, CD {CD}): {us_prep:.2f} us (HBM {out['prep_config3_hbm_frac']:.2%})")
    if with_cpu:
        # the reference's tree_prep semantics (inference/hf/tree_gdn_kernel.py:29-56) in float32 torch on the host:
        # gather each node's window from [conv state ; nodes], weighted sum, SiLU, bf16 rounding, q / k l2 norm
        xc, csc, wc, idc = x.cpu().float(), cs.cpu().float(), w.cpu().float(), idx.cpu().long()
        cuc = cu.cpu().long()

        def cpu_prep():
            outs = []
            for r in range(R3):
                a, b = int(cuc[r]), int(cuc[r + 1])
                src = torch.cat([csc[r].T, xc[a:b]])  # [KC + n, CD]
                acc = (src[idc[a:b]] * wc.T[None]).sum(1)  # [n, CD]
                y = torch.nn.functional.silu(acc).to(torch.bfloat16).float()
                qk = y[:, : 2 * HK3 * D].reshape(b - a, 2 * HK3, D)
                qk = qk * torch.rsqrt((qk * qk).sum(-1, keepdim=True) + 1e-6)
                outs.append((qk.to(torch.bfloat16), y[:, 2 * HK3 * D:].to(torch.bfloat16)))
            return outs

        med, reps = cpu_median(cpu_prep, budget_s=4.0)
        out["prep_cpu_baseline"] = dict(value_us=med * 1e6, cores=torch.get_num_threads(), kind="port",
                                        sample=f"the reference's tree_prep semantics in float32 torch, config 3 "
                                               f"(1024 nodes), median of {reps}")

    Lc, n = LAYERS, N3
    par0 = trees[0]
    node = int(np.argmax(gdn.depths_from_parents(par0)))
    path = []
    i = node
    while i >= 0:
        path.append(i)
        i = int(par0[i])
    path = torch.tensor(path[::-1], dtype=torch.int32).cuda()
    state = torch.randn(Lc, H3, D, D, generator=g).mul_(0.02).cuda()
    u = torch.randn(Lc, n, H3, D, generator=g).cuda()
    kk = torch.nn.functional.normalize(torch.randn(Lc, n, HK3, D, generator=g), dim=-1).to(torch.bfloat16).cuda()
    G = torch.randn(Lc, n, H3, generator=g).abs().mul(-0.05).cumsum(1).cuda()
    conv = (torch.randn(Lc, CD, KC, generator=g) * 0.5).to(torch.bfloat16).cuda()
    xs = (torch.randn(Lc, n, CD, generator=g) * 0.5).to(torch.bfloat16).cuda()
    idx0 = tree_gdn_kernel.conv_index(torch.from_numpy(par0).cuda(), KC)
    fn = lambda: tree_gdn_kernel.gdn_commit(state, u, kk, G, path, conv=conv, x=xs, conv_index=idx0)
    us_c = time_graph(torch, fn, steps, warmup, inner=INNER)
    p = path.numel()
    nb_c = state.numel() * 4 * 2 + Lc * p * (H3 * D * 4 + HK3 * D * 2 + H3 * 4) + conv.numel() * 2 * 2
    out["commit_layers"] = Lc
    out["commit_path_nodes"] = p
    out["commit_us"] = us_c
    out["commit_hbm_frac"] = nb_c / (us_c * 1e-6) / (HBM_PEAK_GBS * 1e9)
    out["commit_alg_bytes"] = nb_c
    log(f"gdn commit ({Lc} layers, {p}-node path): {us_c:.2f} us (HBM {out['commit_hbm_frac']:.2%})")
    if with_cpu:
        # the reference's commit expression (inference/hf/qwen35_tree.py:131-138) in float32 torch on the host
        sc, uc, kc, Gc, pc = state.cpu(), u.cpu(), kk.cpu().float(), G.cpu(), path.cpu().long()
        rep = H3 // HK3

        def cpu_commit():
            uu = uc[:, pc].transpose(1, 2)
            kp = kc[:, pc].transpose(1, 2).repeat_interleave(rep, dim=1)
            GG = Gc.transpose(1, 2)
            wt = (GG[..., pc[-1]:pc[-1] + 1] - GG[..., pc]).exp()
            new = GG[..., pc[-1]].exp()[..., None, None] * sc
            return new + (kp * wt[..., None]).transpose(-1, -2) @ uu

        med, reps = cpu_median(cpu_commit, budget_s=4.0)
        out["commit_cpu_baseline"] = dict(value_us=med * 1e6, cores=torch.get_num_threads(), kind="port",
                                          sample=f"the reference's commit state update in float32 torch, {Lc} layers, "
                                                 f"median of {reps}")
    return out


# ------------------------------------------------------------------------------------------------ draft top-k head


def bench_draft_head(torch, steps, warmup, with_cpu=False):
    """The draft top-k head (DDTreeDraftTopK) at the config-1 round: 8 modes x 15 drafted positions, draft hidden
    2560 (a Qwen3-4B-sized drafter), the full 151936-token vocabulary and a reduced 32768-token draft vocabulary,
    top-8. One mfd_draft_topk_head call: the hand-written LM-head GEMM (csrc/draft_head.hip), then the logits
    kernel (top-k, log Z and the id map)."""
    import ddtree_sglang_ops

    out = {}
    g = torch.Generator().manual_seed(1100)
    K, L, Hd = 8, 16, 2560
    hidden = torch.randn(K * L, Hd, generator=g).to(torch.bfloat16).cuda()
    for name, V in (("full", 151936), ("reduced", 32768)):
        weight = (torch.randn(V, Hd, generator=g) * 0.02).to(torch.bfloat16).cuda()
        vids = torch.sort(torch.randperm(151936, generator=g)[:V]).values.to(torch.int32).cuda() if V < 151936 else None
        head = ddtree_sglang_ops.DDTreeDraftTopK(weight=weight, block_size=L, num_modes=K, budget=8, max_bs=1,
                                            vocab_ids=vids)
        us = time_graph(torch, lambda: head(hidden), steps, warmup, inner=INNER)
        rows = K * (L - 1)
        nb = V * Hd * 2 + rows * Hd * 2 + rows * 8 * 8
        out[f"{name}_vocab"] = V
        out[f"{name}_us"] = us
        out[f"{name}_hbm_frac"] = nb / (us * 1e-6) / (HBM_PEAK_GBS * 1e9)
        log(f"draft head ({name} vocab {V}): {us:.2f} us (HBM {out[f'{name}_hbm_frac']:.2%} of the weight stream)")
        if with_cpu and name == "reduced":
            # the reference's DDTreeDraftTopK.__call__ (P:1523-1538) with float32 torch on the host
            hc = hidden.cpu().float().view(K, L, Hd)[:, 1:].reshape(-1, Hd)
            wc = weight.cpu().float()
            vc = vids.cpu().long()

            def cpu_head():
                lg = hc @ wc.T
                tv, ti = torch.topk(lg, 8, dim=-1)
                lz = torch.logsumexp(lg, -1, keepdim=True)
                return tv - lz, vc[ti]

            med, reps = cpu_median(cpu_head, budget_s=4.0)
            out["reduced_cpu_baseline"] = dict(value_us=med * 1e6, cores=torch.get_num_threads(), kind="port",
                                               sample=f"DDTreeDraftTopK's GEMM + topk + logsumexp + id map in float32 "
                                                      f"torch, 32768-token vocabulary, median of {reps}")
        del weight, head
    return out


# ------------------------------------------------------------------------------------------------ verify plumbing


def bench_plumbing(torch, steps, warmup, with_cpu=False):
    """Verify-side plumbing at the config-4 batch (16 requests, contexts U[1024, 8192], 64-node trees of the
    config-1 builder shape): verify inputs (flat mask rows prefix + 64), the accept walk, and the KV moves of
    the accepted paths in a 36-layer token-major pool (8 KV heads x 128, bf16: 2 KiB slots)."""
    import numpy as np

    import ddtree_sglang_ops
    from oracle import builder as B

    out = {}
    g = torch.Generator().manual_seed(4000)
    lens = [int(x) for x in torch.randint(1024, 8193, (16,), generator=g)]
    bs, W, L = 16, 64, 16
    trees = []
    for b in range(bs):
        logits = torch.randn(8, L - 1, 256, generator=g) * 3
        top, ids = torch.topk(torch.log_softmax(logits, -1), 8, dim=-1)
        t, d, p, n, _ = B.build_mixture(top.numpy(), ids.numpy(), np.zeros(8, np.float32), W - 1)
        trees.append(np.stack([t, d, p]))
    tree = torch.from_numpy(np.stack(trees)).cuda()
    prefix = torch.tensor(lens, dtype=torch.long).cuda()
    offs = torch.tensor(np.concatenate([[0], np.cumsum([W * (c + W) for c in lens])[:-1]]), dtype=torch.long).cuda()
    mask = torch.empty(int(sum(W * (c + W) for c in lens)), dtype=torch.bool, device="cuda")
    ids_o = torch.empty(bs, W, dtype=torch.long, device="cuda")
    pos_o = torch.empty(bs, W, dtype=torch.long, device="cuda")
    root = torch.arange(bs, dtype=torch.long).cuda()
    fn = lambda: ddtree_sglang_ops.ddtree_verify_inputs(root_tokens=root, prefix_lens=prefix, tokens=tree[:, 0],
                                                   depths=tree[:, 1], parents=tree[:, 2], mask_offsets=offs,
                                                   ids_out=ids_o, positions_out=pos_o, mask_out=mask, max_depth=L)
    us = time_graph(torch, fn, steps, warmup, inner=SMALL_INNER)
    nb = mask.numel() + bs * W * 8 * 5
    out["verify_inputs_us"] = us
    out["verify_inputs_hbm_frac"] = nb / (us * 1e-6) / (HBM_PEAK_GBS * 1e9)
    # the accept walk: posteriors that follow each tree for a few steps
    post = torch.randint(0, 256, (bs, W), generator=g)
    tr = tree.cpu().numpy()
    for b in range(bs):
        cur = 0
        for _ in range(5):
            kids = [i for i in range(1, W) if tr[b, 2, i] == cur]
            if not kids:
                break
            post[b, cur] = int(tr[b, 0, kids[0]])
            cur = kids[0]
    post = post.cuda()
    vids = tree[:, 0].contiguous()
    window = torch.randperm(200_000, generator=g)[: bs * W].reshape(bs, W).cuda()
    o = dict(a=torch.empty(bs, dtype=torch.int32, device="cuda"), c=torch.empty(bs, dtype=torch.int32, device="cuda"),
             b=torch.empty(bs, dtype=torch.long, device="cuda"), t=torch.empty(bs, L, dtype=torch.long, device="cuda"),
             n=torch.empty(bs, dtype=torch.long, device="cuda"), s=torch.empty(bs, L, dtype=torch.long, device="cuda"),
             g=torch.empty(bs, L, dtype=torch.long, device="cuda"), h=torch.empty(bs, L, dtype=torch.long, device="cuda"))
    fn = lambda: ddtree_sglang_ops.ddtree_follow(posterior=post, verify_ids=vids, parents=tree[:, 2], window=window,
                                            prefix_lens=prefix, accept_len_out=o["a"], commit_lens_out=o["c"],
                                            bonus_out=o["b"], out_tokens_out=o["t"], new_seq_lens_out=o["n"],
                                            move_src_out=o["s"], move_tgt_out=o["g"], hidden_index_out=o["h"])
    out["follow_us"] = time_graph(torch, fn, steps, warmup, inner=SMALL_INNER)
    fn()
    # KV moves of the accepted paths in a 36-layer pool
    nlayers, Hkv = 36, 8
    pool = [torch.empty(200_000, Hkv, D, dtype=torch.bfloat16, device="cuda") for _ in range(2 * nlayers)]
    ptrs = torch.tensor([t.data_ptr() for t in pool], dtype=torch.int64).cuda()
    comp = ddtree_sglang_ops.DDTreeKVCompactor(data_ptrs=ptrs, slot_bytes=Hkv * D * 2, num_slots=200_000)
    fn = lambda: comp(move_src=o["s"], move_tgt=o["g"])
    us_mv = time_graph(torch, fn, steps, warmup, inner=SMALL_INNER)
    moves = int((o["s"] != o["g"]).sum())
    out["kv_move_us"] = us_mv
    out["kv_move_slots"] = moves
    out["kv_move_hbm_frac"] = moves * 2 * nlayers * Hkv * D * 2 * 2 / (us_mv * 1e-6) / (HBM_PEAK_GBS * 1e9)
    log(f"plumbing: verify inputs {us:.2f} us, follow {out['follow_us']:.2f} us, kv moves {us_mv:.2f} us "
        f"({moves} slots x {2 * nlayers} buffers)")
    if with_cpu:
        # the host forms of the reference: compile_ddtree_tree's mask / ids / positions per request and the
        # Tree.follow walk over child maps (inference/hf/ddtree.py:317-382), torch on the CPU
        import tree_build_ext

        trc, postc, pref = tree.cpu(), post.cpu(), lens
        vis = []
        for b in range(bs):
            p = trc[b, 2].tolist()
            v = torch.zeros(W, W, dtype=torch.bool)
            v[0, 0] = True
            for i in range(1, W):
                if p[i] >= 0:
                    v[i] = v[p[i]]
                v[i, i] = True
            vis.append(v)
        trees_h = [tree_build_ext.Tree(trc[b, 0, 1:].tolist(), trc[b, 2].tolist()) for b in range(bs)]

        def cpu_verify():
            for b in range(bs):
                m = torch.full((W, pref[b] + W), torch.finfo(torch.bfloat16).min, dtype=torch.bfloat16)
                m[:, : pref[b]] = 0
                m[:, pref[b]:].masked_fill_(vis[b], 0)
                ids = trc[b, 0].clone()
                ids[0] = b
                pos = trc[b, 1] + pref[b]
                trees_h[b].follow(postc[b])

        med, reps = cpu_median(cpu_verify, budget_s=3.0)
        out["verify_follow_cpu_baseline"] = dict(value_us=med * 1e6, cores=torch.get_num_threads(), kind="port",
                                                 sample=f"the HF host forms (compile_ddtree_tree mask / ids / positions "
                                                        f"+ Tree.follow) for the 16 requests, median of {reps}")
    return out


def profile_pass(torch):
    """Eager launches for rocprofv3 counter runs (no graph): a plain 256 MiB float32 copy kernel (torch.neg reads
    and writes 256 MiB) that scales FETCH_SIZE / WRITE_SIZE to bytes, then two passes over the 24 config-3 layers,
    then mode attention: four steps of config 2 (the automatic split: 15 context splits on 256 CUs, and the merge) and one of config 4 (paged),
    then four calls of the draft top-k head at the config-1 round with the reduced 32768-token vocabulary and
    four with the full 151936-token one (bench_draft_head's shapes), then four tree_prep launches at the config-3
    shape (prep_inputs)."""
    import ddtree_sglang_ops
    import paged_mode_attention as dm
    import mode_attention
    import tree_gdn_kernel
    from oracle.synth import attention_inputs, paged_attention_inputs

    x = torch.randn(64 << 20, device="cuda")
    y = torch.empty_like(x)
    torch.neg(x, out=y)
    layers = make_gdn_layers(torch, LAYERS)
    L0 = layers[0]
    ctx = tree_gdn_kernel.tree_context(L0["parents"], L0["cu_nodes"], max_nodes=L0["max_nodes"])
    for _ in range(2):
        gdn_round(tree_gdn_kernel, layers, ctx)
    torch.cuda.synchronize()
    del layers
    q, k, v = (t.cuda() for t in attention_inputs(2))
    for _ in range(4):
        mode_attention.mode_block_attention(q, k, v, 8, 16, 128 ** -0.5)
    g = torch.Generator().manual_seed(4000)
    lens = [int(t) for t in torch.randint(1024, 8193, (16,), generator=g)]
    d = paged_attention_inputs(4000, lens, H=40, Hkv=8, page_size=64)
    pt = torch.zeros(18, d["page_table"].shape[1], dtype=torch.int32)
    pt[2:] = d["page_table"]
    dev = {kk: (vv.cuda() if torch.is_tensor(vv) else vv) for kk, vv in d.items()}
    dm.paged_mode_block_attention(q=dev["q"], k_new=dev["k_new"], v_new=dev["v_new"], k_cache=dev["k_cache"],
                                  v_cache=dev["v_cache"], req_to_token=pt.cuda(),
                                  req_pool_indices=dev["req_pool_indices"], ctx_lens=dev["ctx_lens"], num_modes=8,
                                  block_size=16, scaling=128 ** -0.5, num_ctx_splits=-1, page_size=64)
    torch.cuda.synchronize()
    gh = torch.Generator().manual_seed(1100)
    hidden = torch.randn(8 * 16, 2560, generator=gh).to(torch.bfloat16).cuda()
    for V in (32768, 151936):
        weight = (torch.randn(V, 2560, generator=gh) * 0.02).to(torch.bfloat16).cuda()
        head = ddtree_sglang_ops.DDTreeDraftTopK(weight=weight, block_size=16, num_modes=8, budget=8, max_bs=1)
        for _ in range(4):
            head(hidden)
        torch.cuda.synchronize()
        del weight, head
    x3, cs3, w3, idx3, cu3 = prep_inputs(torch)[:5]
    for _ in range(4):
        tree_gdn_kernel.tree_prep(x3, cs3, idx3, w3, HK3, H3, D, cu_nodes=cu3)
    torch.cuda.synchronize()
    print(json.dumps({"copy_kernel": "torch.neg float32", "copy_read_bytes": x.numel() * 4,
                      "copy_write_bytes": y.numel() * 4, "gdn_alg_bytes": gdn_alg_bytes(R3 * N3, R3, HK3, H3)}))


def measured_traffic():
    """HBM bytes per config-3 tree-GDN launch from the committed counter summary, or None."""
    path = os.path.join(REPO, "profiles", "tree_gdn_config3_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch"):
                    return float(line.split("=", 1)[1])
    except OSError:
        pass
    return None


def device_info(torch):
    p = torch.cuda.get_device_properties(0)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"gpu": p.name, "cus": p.multi_processor_count, "host_cpu": cpu_model,
            "host_cores": len(os.sched_getaffinity(0))}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-gdn", action="store_true")
    ap.add_argument("--profile-pass", action="store_true", help="eager launches for rocprofv3 --pmc runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: every part of the hot path is a single-GPU "
                                   "kernel (DESIGN.md describes how it would shard); run with --gpus 1"}))
        sys.exit(2)
    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.profile_pass:
        profile_pass(torch)
        return
    gdn_res = bench_gdn(torch, args.steps, args.warmup)
    nodes_per_s = R3 * N3 / (gdn_res["us_launch"] * 1e-6)
    alg = gdn_alg_bytes(R3 * N3, R3, HK3, H3)
    achieved = alg / (gdn_res["us_launch"] * 1e-6) / 1e9
    extra = {}
    if not args.only_gdn:
        extra["gdn"] = bench_gdn_small(torch, args.steps, args.warmup)
        extra["mode_attention"] = bench_attention(torch, args.steps, args.warmup, not args.no_cpu_baseline)
        extra["builder"] = bench_builder(torch, args.steps, args.warmup, not args.no_cpu_baseline)
        extra["prep_commit"] = bench_prep_commit(torch, args.steps, args.warmup, not args.no_cpu_baseline)
        extra["plumbing"] = bench_plumbing(torch, args.steps, args.warmup, not args.no_cpu_baseline)
        extra["draft_head"] = bench_draft_head(torch, args.steps, args.warmup, not args.no_cpu_baseline)
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
        "dtype": "bf16 q/k/v, f32 state, gates and u/o (bf16 MFMA for the S0 products, fp16 for u = T R, o = E + W R)",
        "data": "synthetic (seeded, BASELINE.json configs; random weights-free inputs of the configured shapes)",
        "config": {"workload": "config 3: tree-GDN verify, 8 requests x 128-node trees (depth<=16), HK16/H32/D128, "
                               "24 layers per step", "requests": R3, "nodes_per_tree": N3, "layers_per_step": LAYERS,
                   "parallelism": "single GPU"},
        "gdn_us_per_layer": gdn_res["us_launch"],
        "gdn_parity_rel_err": gdn_res["parity_rel"],
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": measured_traffic(), "kernel": "tree_gdn_pipe_kernel<4, true>",
                     "alg_bytes_per_launch": alg,
                     "note": "launch duration = (tree context + 24 layers) / 24 per round, so it includes the "
                             "round's share of tree_ctx_kernel and the launch gaps"},
        "cpu_baseline": cpu,
        "device": device_info(torch),
        **extra,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
