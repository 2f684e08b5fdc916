"""GPU parity of the logits step and the mixture-tree builder (through the C ABI).

Bar: bit-exact. Log-probs, ids and log Z equal the CPU oracle's bits; trees (tokens, depths, parents, counts,
visibility) equal the golden vectors written by the reference's own C++ builders, and the end-to-end device
pipeline from config-1 logits equals the oracle pipeline.
"""

import os

import numpy as np
import pytest
import torch

from oracle import builder as B
from oracle.synth import builder_logits

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "builder_golden.npz")


def _logits_case(kind, rows, V, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "randn3":
        x = torch.randn(rows, V, generator=g) * 3
    elif kind == "coarse":  # many exact ties
        x = (torch.randn(rows, V, generator=g) * 2).round() / 2
    elif kind == "inf":
        x = torch.full((rows, V), float("-inf"))
        x[1::2, V // 3] = 5.0
    else:
        x = torch.randn(rows, V, generator=g) * 16
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("kind,rows,V,k", [
    ("randn3", 128, 151936, 8), ("coarse", 16, 151936, 64), ("wide", 8, 248320, 256), ("randn3", 5, 8192, 32),
    ("coarse", 7, 8200, 16), ("inf", 4, 20000, 3), ("randn3", 3, 8193, 8), ("randn3", 2, 24, 24),
    # rows of at most 16 pieces with k <= 8: one workgroup per row merges its own pieces
    ("randn3", 120, 32768, 8), ("coarse", 9, 30000, 1), ("coarse", 5, 2048, 8),
    # k <= 8 and 17..128 pieces per row, ties, -inf rows, a single row: the piece kernel, then the row merge
    ("coarse", 33, 100000, 4), ("inf", 6, 60000, 8), ("randn3", 3, 262144, 1), ("wide", 1, 34817, 8),
])
def test_topk_logz_bit_exact(kind, rows, V, k):
    import tree_logits

    x = _logits_case(kind, rows, V, seed=V + k)
    print(f"case: topk_logz {kind} rows={rows} V={V} k={k}", flush=True)
    logp, ids, logz = tree_logits.topk_logz(x.cuda(), k, with_logz=True)
    torch.cuda.synchronize()
    lp_ref, ids_ref, lz_ref = B.top_candidates(x, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(logz.cpu().numpy().view(np.uint32), lz_ref.view(np.uint32))
    np.testing.assert_array_equal(logp.cpu().numpy().view(np.uint32), lp_ref.view(np.uint32))


def test_row_logsumexp_and_top_candidates_api():
    import tree_logits

    x = _logits_case("randn3", 6, 151936, 3)
    lz = tree_logits.row_logsumexp(x.cuda())
    assert lz.shape == (6, 1)
    _, _, lz_ref = B.top_candidates(x, 1)
    np.testing.assert_array_equal(lz.cpu().numpy()[:, 0], lz_ref)
    lp, ids = tree_logits.top_candidates(x.cuda().view(2, 3, -1), 8)
    assert lp.device.type == "cpu" and ids.dtype == torch.int64 and lp.shape == (2, 3, 8)
    lp_ref, ids_ref, _ = B.top_candidates(x, 8)
    np.testing.assert_array_equal(ids.reshape(6, 8).numpy(), ids_ref)


def golden_cases():
    z = np.load(GOLDEN, allow_pickle=False)
    for i in range(int(z["n"])):
        c = {k: z[f"c{i}_{k}"] for k in ("kind", "lp", "ids", "prior", "budget", "tree", "count", "vis")}
        if str(c["kind"]) == "mixture":
            yield i, c


def test_builder_matches_reference_golden_trees():
    import tree_build_ext

    n_cases = 0
    for i, c in golden_cases():
        budget = int(c["budget"])
        lp = torch.from_numpy(c["lp"])[None].cuda()
        ids = torch.from_numpy(c["ids"]).to(torch.int32)[None].cuda()
        prior = torch.from_numpy(c["prior"])[None].cuda()
        tree, counts, anc8 = tree_build_ext.build_trees_device(lp, ids, prior, budget, with_visibility=True)
        torch.cuda.synchronize()
        n = int(c["count"])
        assert int(counts[0]) == n, f"case {i}"
        np.testing.assert_array_equal(tree[0].cpu().numpy(), c["tree"], err_msg=f"case {i}")
        vis = np.unpackbits(c["vis"])[: (n + 1) ** 2].reshape(n + 1, n + 1)
        np.testing.assert_array_equal(anc8[0, : n + 1, : n + 1].cpu().numpy(), vis, err_msg=f"case {i}")
        assert not anc8[0, n + 1 :].any()
        n_cases += 1
    assert n_cases >= 60


def test_build_trees_batched_sglang_contract():
    """A batch of requests sharing (K, L, k) in one launch, int32 ids, random priors (build_trees, P:1377-1407)."""
    import ddtree_sglang_ops

    g = torch.Generator().manual_seed(11)
    bs, K, L, V, budget = 6, 8, 15, 64, 63
    logits = (torch.randn(bs, K, L, V, generator=g) * 3)
    logits[::2] = (logits[::2] * 2).round() / 2
    logits = logits.to(torch.bfloat16)
    lp = logits.float()
    top, ids = torch.topk(lp, k=min(budget, V), dim=-1)
    logp = (top - torch.logsumexp(lp, -1, keepdim=True)).float()
    prior = torch.log_softmax(torch.randn(bs, K, generator=g), -1)
    tree = torch.empty(bs, 3, budget + 1, dtype=torch.long, device="cuda")
    counts = torch.empty(bs, dtype=torch.long, device="cuda")
    ddtree_sglang_ops.build_trees(top_log_probs=logp.cuda(), top_ids=ids.to(torch.int32).cuda(), log_prior=prior.cuda(),
                             bs=bs, budget=budget, tree=tree, counts=counts)
    torch.cuda.synchronize()
    for b in range(bs):
        t, d, p, n, _ = B.build_mixture(logp[b].numpy(), ids[b].numpy(), prior[b].numpy(), budget)
        assert int(counts[b]) == n
        np.testing.assert_array_equal(tree[b].cpu().numpy(), np.stack([t, d, p]))
    ref = B.ref_sglang_builder()
    if ref is not None:  # the compiled reference travels with the tree when it was built
        rt = torch.empty(bs, 3, budget + 1, dtype=torch.long)
        rc = torch.empty(bs, dtype=torch.long)
        ref.build_trees(logp.contiguous(), ids.to(torch.int32).contiguous(), prior.contiguous(), bs, budget, rt, rc)
        assert torch.equal(rt, tree.cpu()) and torch.equal(rc, counts.cpu())


def test_end_to_end_config1_from_logits():
    """Config 1: K 8 x L 16 x V 151936 bf16 logits, top-8, B 64: device pipeline == oracle pipeline."""
    import ddtree_sglang_ops

    logits = builder_logits(1)
    print("case: config1 end to end", flush=True)
    tree, counts, anc8, logp, ids = ddtree_sglang_ops.build_mixture_trees_from_logits(logits.cuda(), torch.zeros(8).cuda(),
                                                                                 64, topk=8)
    torch.cuda.synchronize()
    lp_ref, ids_ref, _ = B.top_candidates(logits.reshape(128, -1), 8)
    np.testing.assert_array_equal(logp[0].cpu().numpy().reshape(128, 8).view(np.uint32), lp_ref.view(np.uint32))
    np.testing.assert_array_equal(ids[0].cpu().numpy().reshape(128, 8), ids_ref)
    t, d, p, n, _ = B.build_mixture(lp_ref.reshape(8, 16, 8), ids_ref.reshape(8, 16, 8), np.zeros(8, np.float32), 64)
    assert int(counts[0]) == n == 64
    np.testing.assert_array_equal(tree[0].cpu().numpy(), np.stack([t, d, p]))
    np.testing.assert_array_equal(anc8[0].cpu().numpy(), B.visibility(p, n))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_batch_steps_with_ties_and_merges(seed):
    """Top lists whose log-probs sit on a 0.25 grid (many equal keys across paths and modes) and whose ids come
    from 12 tokens (modes share prefixes: about two pops per node). The first step pops ~50 entries at once
    (every frontier entry below the smallest child key), the rest one by one; the tree must equal the
    sequential heap's, tie order and merged prefixes included."""
    import tree_build_ext

    g = torch.Generator().manual_seed(100 + seed)
    K, L, k, budget = 8, 16, 8, 64
    lp = torch.sort(-(2.0 + 0.25 * torch.randint(0, 12, (K, L, k), generator=g).float()), -1, descending=True).values
    ids = torch.stack([torch.randperm(12, generator=g)[:k] for _ in range(K * L)]).reshape(K, L, k)
    prior = torch.zeros(K)
    print(f"case: ties and merges seed {seed}", flush=True)
    tree, counts, anc8 = tree_build_ext.build_trees_device(lp[None].cuda(), ids[None].to(torch.int32).cuda(),
                                                           prior[None].cuda(), budget, with_visibility=True)
    torch.cuda.synchronize()
    t, d, p, n, pops = B.build_mixture(lp.numpy(), ids.numpy(), prior.numpy(), budget)
    assert pops > n  # prefixes were merged
    assert int(counts[0]) == n
    np.testing.assert_array_equal(tree[0].cpu().numpy(), np.stack([t, d, p]))
    np.testing.assert_array_equal(anc8[0, : n + 1, : n + 1].cpu().numpy(), B.visibility(p, n))


def test_hf_build_mixture_contract_and_follow():
    import tree_build_ext

    i, c = next(iter(golden_cases()))
    toks, deps, parents, tree, vis = tree_build_ext.build_mixture(torch.from_numpy(c["lp"]), torch.from_numpy(c["ids"]),
                                                                  torch.from_numpy(c["prior"]), int(c["budget"]))
    n = int(c["count"])
    assert toks.device.type == "cpu" and toks.dtype == torch.int64 and len(parents) == n + 1 and parents[0] == -1
    np.testing.assert_array_equal(toks.numpy(), c["tree"][0, 1 : n + 1])
    assert vis.dtype == torch.bool and vis.shape == (n + 1, n + 1)
    # a posterior agreeing along the deepest path accepts exactly that path (tests/test_mixture_tree.py:103-114)
    leaf = int(np.argmax(c["tree"][1, : n + 1]))
    path = [leaf]
    while parents[path[-1]] > 0:
        path.append(parents[path[-1]])
    path = [0] + path[::-1]
    post = torch.zeros(n + 1, dtype=torch.long)
    for node, child in zip(path, path[1:]):
        post[node] = int(toks[child - 1])
    post[leaf] = 7
    accepted, bonus = tree.follow(post)
    assert accepted == path and bonus == 7


def test_budget_zero_and_exhausted_heap():
    import tree_build_ext

    lp = torch.log_softmax(torch.randn(1, 2, 1, 2), -1).float().cuda()
    ids = torch.tensor([[[[5, 6]], [[6, 5]]]], dtype=torch.int32).cuda()
    tree, counts, _ = tree_build_ext.build_trees_device(lp, ids, None, 0)
    assert int(counts[0]) == 0 and tree.shape == (1, 3, 1) and int(tree[0, 2, 0]) == -1
    # K L k = 2 distinct candidates < budget: the heap empties, count = 2, tail (0, 0, -1)
    tree, counts, _ = tree_build_ext.build_trees_device(lp, ids, None, 10)
    torch.cuda.synchronize()
    t, d, p, n, _ = B.build_mixture(lp[0].cpu().numpy(), ids[0].cpu().numpy().astype(np.int64), np.zeros(2, np.float32), 10)
    assert int(counts[0]) == n == 2
    np.testing.assert_array_equal(tree[0].cpu().numpy(), np.stack([t, d, p]))


def golden_single_cases():
    z = np.load(GOLDEN, allow_pickle=False)
    for i in range(int(z["n"])):
        c = {k: z[f"c{i}_{k}"] for k in ("kind", "lp", "ids", "prior", "budget", "tree", "count", "vis")}
        if str(c["kind"]) == "single":
            yield i, c


def test_single_builder_matches_reference_golden_trees():
    """The DDTree heap (K = 1 through build_trees, HF build_single) against the trees the reference's own
    build_single wrote (tests/golden/builder_golden.npz, single cases)."""
    import tree_build_ext

    n_cases = 0
    for i, c in golden_single_cases():
        budget = int(c["budget"])
        print(f"case: golden single {i} L={c['lp'].shape[1]} k={c['lp'].shape[2]} budget={budget}", flush=True)
        lp = torch.from_numpy(c["lp"])[None].cuda()
        ids = torch.from_numpy(c["ids"]).to(torch.int32)[None].cuda()
        tree, counts, anc8 = tree_build_ext.build_trees_device(lp, ids, None, budget, with_visibility=True,
                                                               single_mode_heap=True)
        torch.cuda.synchronize()
        n = int(c["count"])
        assert int(counts[0]) == n, f"case {i}"
        np.testing.assert_array_equal(tree[0].cpu().numpy(), c["tree"], err_msg=f"case {i}")
        vis = np.unpackbits(c["vis"])[: (n + 1) ** 2].reshape(n + 1, n + 1)
        np.testing.assert_array_equal(anc8[0, : n + 1, : n + 1].cpu().numpy(), vis, err_msg=f"case {i}")
        n_cases += 1
    assert n_cases >= 20


@pytest.mark.parametrize("seed,coarse,L,k,budget", [(0, False, 16, 8, 64), (1, True, 15, 16, 63), (2, True, 8, 32, 255),
                                                    (3, True, 4, 64, 500), (4, False, 63, 2, 100), (5, True, 1, 7, 7)])
def test_single_builder_matches_oracle_ties(seed, coarse, L, k, budget):
    """Random and tie-heavy (coarse) log-probs: equal fp64 keys are ordered by the rank tuple."""
    import tree_build_ext

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(L, 64, generator=g) * 2
    if coarse:
        x = (x * 2).round() / 2
    top, ids = torch.topk(x, k, dim=-1)
    lp = (top - torch.logsumexp(x, -1, keepdim=True)).float()
    if coarse:  # exact ties between the sums: log-probs on a coarse grid
        lp = (lp * 4).round() / 4
    print(f"case: single oracle seed={seed} coarse={coarse} L={L} k={k} budget={budget}", flush=True)
    t, d, p, n = B.build_single(lp.numpy(), ids.numpy(), budget)
    tree, counts, anc8 = tree_build_ext.build_trees_device(lp[None, None].cuda(), ids.to(torch.int32)[None, None].cuda(),
                                                           None, budget, with_visibility=True, single_mode_heap=True)
    torch.cuda.synchronize()
    assert int(counts[0]) == n
    np.testing.assert_array_equal(tree[0].cpu().numpy(), np.stack([t, d, p]))
    np.testing.assert_array_equal(anc8[0, : n + 1, : n + 1].cpu().numpy(), B.visibility(p, n))


def test_build_trees_k1_is_the_single_heap_and_hf_build_mixture_k1_the_mixture_heap():
    """SGLang's build_trees builds one-mode requests with build_single_one (P:1397-1398); the HF build_mixture
    keeps the mixture heap for K = 1 (inference/hf/ddtree.py:247-254). Tie-heavy inputs tell them apart."""
    import ddtree_sglang_ops
    import tree_build_ext

    g = torch.Generator().manual_seed(21)
    bs, L, k, budget = 3, 12, 8, 40
    x = (torch.randn(bs, 1, L, 32, generator=g) * 2).round()
    top, ids = torch.topk(x, k, dim=-1)
    lp = ((top - torch.logsumexp(x, -1, keepdim=True)) * 2).round().float() / 2
    tree = torch.empty(bs, 3, budget + 1, dtype=torch.long, device="cuda")
    counts = torch.empty(bs, dtype=torch.long, device="cuda")
    ddtree_sglang_ops.build_trees(top_log_probs=lp.cuda(), top_ids=ids.to(torch.int32).cuda(),
                             log_prior=torch.zeros(bs, 1).cuda(), bs=bs, budget=budget, tree=tree, counts=counts)
    torch.cuda.synchronize()
    differ = False
    for b in range(bs):
        t, d, p, n = B.build_single(lp[b, 0].numpy(), ids[b, 0].numpy(), budget)
        assert int(counts[b]) == n
        np.testing.assert_array_equal(tree[b].cpu().numpy(), np.stack([t, d, p]))
        tm, dm, pm, nm, _ = B.build_mixture(lp[b].numpy(), ids[b].numpy(), np.zeros(1, np.float32), budget)
        toks, deps, parents, _, _ = tree_build_ext.build_mixture(lp[b], ids[b], torch.zeros(1), budget)
        assert len(parents) == nm + 1 and np.array_equal(np.asarray(parents), pm[: nm + 1])
        np.testing.assert_array_equal(toks.numpy(), tm[1 : nm + 1])
        differ |= not np.array_equal(np.stack([tm, dm, pm]), np.stack([t, d, p]))
    assert differ, "the tie-heavy inputs should separate the two heaps"
    ref = B.ref_sglang_builder()
    if ref is not None:
        rt = torch.empty(bs, 3, budget + 1, dtype=torch.long)
        rc = torch.empty(bs, dtype=torch.long)
        ref.build_trees(lp.contiguous(), ids.to(torch.int32).contiguous(), torch.zeros(bs, 1), bs, budget, rt, rc)
        assert torch.equal(rt, tree.cpu()) and torch.equal(rc, counts.cpu())


def test_hf_build_single_contract():
    import tree_build_ext

    i, c = next(iter(golden_single_cases()))
    toks, deps, parents, tree, vis = tree_build_ext.build_single(torch.from_numpy(c["lp"][0]),
                                                                 torch.from_numpy(c["ids"][0]), int(c["budget"]))
    n = int(c["count"])
    assert toks.device.type == "cpu" and toks.dtype == torch.int64 and len(parents) == n + 1 and parents[0] == -1
    np.testing.assert_array_equal(toks.numpy(), c["tree"][0, 1 : n + 1])
    np.testing.assert_array_equal(deps.numpy(), c["tree"][1, 1 : n + 1])
    assert vis.dtype == torch.bool and vis.shape == (n + 1, n + 1)


def _gemm_reference_check(got, hs, weight):
    """The draft LM-head product against the exact (fp64) product of the bf16 inputs. Tolerance, per element:
    one bf16 ulp of the exact value (the final rounding) plus K * 2^-24 * sum_k |h_k w_k| (fp32 accumulation
    of K terms); also the share of elements equal to the correctly rounded value must be near 1."""
    K = hs.shape[1]
    exact = hs.double().cpu() @ weight.double().cpu().T
    mag = hs.double().abs().cpu() @ weight.double().abs().cpu().T
    rounded = exact.to(torch.bfloat16).double()
    ulp = torch.exp2(torch.floor(torch.log2(rounded.abs().clamp_min(2.0 ** -120))) - 7)
    err = (got.double().cpu() - exact).abs()
    tol = ulp + K * 2.0 ** -24 * mag
    assert bool((err <= tol).all()), f"max err/tol {(err / tol).max().item():.3f}"
    assert (got.double().cpu() == rounded).double().mean().item() > 0.99


@pytest.mark.parametrize("M,N,K,L,gap", [(1, 1000, 256, 16, 0), (37, 4100, 512, 16, 0), (120, 131, 64, 16, 1),
                                         (128, 20000, 256, 17, 3), (200, 5000, 128, 9, 0), (15, 33333, 2560, 16, 0),
                                         (37, 90000, 512, 16, 0), (200, 100000, 128, 9, 2), (1, 150001, 64, 16, 0)])
def test_draft_head_gemm_shapes(M, N, K, L, gap):
    """mfd_draft_head_gemm (the LM-head product of DDTreeDraftTopK, P:1523-1532) on ragged shapes: drafted rows
    read in place from [blocks, L, K + gap] hidden states (the anchor row of each block skipped), vocabularies
    that are not multiples of the 128-row pass, more than 128 drafted rows (two launches), and K down to one
    64-wide stage; the columns past N and the rows past M stay untouched. Vocabularies above 256 rows per
    workgroup (90000 and up) take the wide form (every workgroup's whole range against k streamed once)."""
    import mfd_hip

    print(f"case: draft head gemm M={M} N={N} K={K} L={L} gap={gap}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    blocks = (M + L - 2) // (L - 1)
    ld = K + 8 * gap
    hid = torch.randn(blocks * L, ld, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).cuda()
    ostride = (N + 3) // 4 * 4 + 4
    out = torch.full((M + 1, ostride), -7.0, dtype=torch.bfloat16, device="cuda")
    mfd_hip.call("mfd_draft_head_gemm", hid.data_ptr() + ld * 2, ld, L - 1, L * ld, w.data_ptr(), M, N, K,
                 out.data_ptr(), ostride, mfd_hip.stream_of(out))
    torch.cuda.synchronize()
    hs = hid.view(blocks, L, ld)[:, 1:, :K].reshape(-1, K)[:M]
    _gemm_reference_check(out[:M, :N], hs, w)
    assert bool((out[:M, N:] == -7.0).all()) and bool((out[M] == -7.0).all())


def test_draft_head_gemm_full_vocabulary_sampled():
    """The config-1 draft head shape: 8 modes x 15 drafted rows, hidden 2560, the full 151936-token vocabulary
    (every workgroup takes several 128-row passes; the last pass of each is partial). 4096 sampled columns
    against the exact product, every logit finite, the row padding untouched."""
    import mfd_hip

    print("case: draft head gemm M=120 N=151936 K=2560 (sampled)", flush=True)
    g = torch.Generator(device="cuda").manual_seed(77)
    K, L, M, N = 2560, 16, 120, 151936
    hid = torch.randn(8 * L, K, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    out = torch.full((M, N + 8), -7.0, dtype=torch.bfloat16, device="cuda")
    mfd_hip.call("mfd_draft_head_gemm", hid.data_ptr() + K * 2, K, L - 1, L * K, w.data_ptr(), M, N, K,
                 out.data_ptr(), N + 8, mfd_hip.stream_of(out))
    torch.cuda.synchronize()
    cols = torch.randperm(N, generator=torch.Generator().manual_seed(5))[:4096]
    cols = torch.cat([cols, torch.tensor([0, N - 1])])
    hs = hid.view(8, L, K)[:, 1:].reshape(-1, K)
    _gemm_reference_check(out[:, cols.cuda()], hs, w[cols.cuda()])
    assert bool(torch.isfinite(out[:, :N].float()).all())
    assert bool((out[:, N:] == -7.0).all())


def test_draft_head_gemm_rejects_bad_shapes():
    """K not a multiple of 64 and misaligned rows are refused with an error, not computed."""
    import mfd_hip

    w = torch.zeros(64, 96, dtype=torch.bfloat16, device="cuda")
    hid = torch.zeros(16, 96, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(15, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(mfd_hip.MFDError, match="K %"):
        mfd_hip.call("mfd_draft_head_gemm", hid.data_ptr(), 96, 15, 16 * 96, w.data_ptr(), 15, 64, 96,
                     out.data_ptr(), 64, mfd_hip.stream_of(out))
    w2 = torch.zeros(64, 128, dtype=torch.bfloat16, device="cuda")
    hid2 = torch.zeros(16, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(mfd_hip.MFDError, match="alignment"):
        mfd_hip.call("mfd_draft_head_gemm", hid2.data_ptr() + 2, 128, 15, 16 * 128, w2.data_ptr(), 15, 64, 128,
                     out.data_ptr(), 64, mfd_hip.stream_of(out))


@pytest.mark.parametrize("reduced", [False, True])
def test_draft_topk_head_matches_oracle(reduced):
    """DDTreeDraftTopK (P:1485-1544) through mfd_draft_topk_head: the drafted rows' logits (the hand-written LM-head
    GEMM, against the exact product within the accumulation bound), then their top-k log-probs and ids, and with a
    reduced vocabulary the map back to full-vocabulary ids, bit-exact against the oracle logits step on the same
    bf16 logits."""
    import ddtree_sglang_ops

    g = torch.Generator().manual_seed(31 + reduced)
    bs, K, L, Hd, Vfull, budget = 2, 4, 16, 256, 20000, 24
    if reduced:
        vocab_ids = torch.sort(torch.randperm(Vfull, generator=g)[:4100]).values.to(torch.int32)
    else:
        vocab_ids = None
    V = 4100 if reduced else Vfull
    weight = (torch.randn(V, Hd, generator=g) * 0.05).to(torch.bfloat16).cuda()
    hidden = torch.randn(bs * K * L, Hd, generator=g).to(torch.bfloat16).cuda()
    head = ddtree_sglang_ops.DDTreeDraftTopK(weight=weight, block_size=L, num_modes=K, budget=budget, max_bs=4,
                                        vocab_ids=None if vocab_ids is None else vocab_ids.cuda())
    head(hidden)
    lp, ids = head.outputs(bs)
    torch.cuda.synchronize()
    assert lp.shape == (bs, K, L - 1, budget) and ids.dtype == torch.int32
    logits = head.logits[: bs * K * (L - 1)].cpu()
    # the drafted rows feed the GEMM: rows 1..L-1 of every block
    hs = hidden.view(bs * K, L, Hd)[:, 1:].reshape(-1, Hd)
    _gemm_reference_check(logits, hs, weight)
    lp_ref, ids_ref, lz_ref = B.top_candidates(logits, budget)
    if reduced:
        ids_ref = vocab_ids.numpy()[ids_ref]
    np.testing.assert_array_equal(lp.reshape(-1, budget).cpu().numpy().view(np.uint32), lp_ref.view(np.uint32))
    np.testing.assert_array_equal(ids.reshape(-1, budget).cpu().numpy(), ids_ref)
    np.testing.assert_array_equal(head.log_z[: bs * K * (L - 1)].cpu().numpy().view(np.uint32), lz_ref.view(np.uint32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("kind,rows,V,k", [
    ("randn3", 120, 248320, 256), ("coarse", 16, 151936, 64), ("inf", 4, 20000, 3), ("randn3", 3, 8193, 8),
    ("randn3", 2, 27, 27), ("coarse", 9, 30001, 1), ("wide", 5, 4099, 0),
])
def test_topk_logz_wide_dtypes(dtype, kind, rows, V, k):
    """float32 / float16 logits (the reference takes any float dtype): ids exactly as torch.topk orders the values
    (ties by column ascending), log Z within 2e-6 relative of a float64 logsumexp, log-probs value - log Z."""
    import tree_logits

    x = _logits_case(kind, rows, V, seed=V + k + 1).float().to(dtype)
    if kind == "randn3":
        x = x + torch.rand(x.shape, generator=torch.Generator().manual_seed(V)).to(dtype) * 1e-3  # off the bf16 grid
    print(f"case: topk_logz wide {dtype} {kind} rows={rows} V={V} k={k}", flush=True)
    logp, ids, logz = tree_logits.topk_logz(x.cuda(), k, with_logz=True)
    torch.cuda.synchronize()
    lp_ref, ids_ref, lz_ref = B.top_candidates_wide(x, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    lz = logz.cpu().numpy().astype(np.float64)
    fin = np.isfinite(lz_ref)
    assert (np.isfinite(lz) == fin).all() and (lz[~fin] == lz_ref[~fin]).all()
    assert np.abs(lz[fin] - lz_ref[fin]).max(initial=0) <= 2e-6 * max(1.0, np.abs(lz_ref[fin]).max(initial=0))
    if k:
        got = logp.cpu().numpy().astype(np.float64)
        ok = np.isfinite(lp_ref)
        assert np.abs(got[ok] - lp_ref[ok]).max(initial=0) <= 4e-6 * max(1.0, np.abs(lp_ref[ok]).max(initial=0))


def test_topk_logz_wide_vocab_map_and_api():
    """A reduced vocabulary's id map and the reference's entry points on float32 logits."""
    import tree_logits

    x = _logits_case("randn3", 6, 5000, 11).float()
    vocab = torch.randperm(150000, generator=torch.Generator().manual_seed(3))[:5000].to(torch.int32)
    logp, ids = tree_logits.topk_logz(x.cuda(), 16, vocab_ids=vocab.cuda())
    _, ids_ref, _ = B.top_candidates_wide(x, 16)
    np.testing.assert_array_equal(ids.cpu().numpy(), vocab.numpy()[ids_ref])
    lz = tree_logits.row_logsumexp(x.cuda().half())
    assert lz.shape == (6, 1) and lz.dtype == torch.float32
    lp, ids2 = tree_logits.top_candidates(x.cuda().view(2, 3, -1), 8)
    assert lp.device.type == "cpu" and ids2.dtype == torch.int64
    np.testing.assert_array_equal(ids2.reshape(6, 8).numpy(), ids_ref[:, :8])
