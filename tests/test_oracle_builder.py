"""Pins of the builder and logits-step oracle (CPU).

Heap: against the golden vectors written by the reference's own C++ builders (tests/golden/), against
the compiled reference directly when oracle/_ref is present (random and tie-heavy trials as in the
reference's tests/test_sglang_tree_builder.py and tree_build_ext.check_equal), against brute force
(tests/test_mixture_tree.py:39-74 of the reference), the K = 1 reduction to DDTree, and the structure
invariants; planted mistakes (a dropped term, a wrong index, no node reuse) are caught.
Logits step: log Z against torch.logsumexp in float64, the deterministic exp / log against math,
top-k values against torch.topk, the id tie rule (value descending, id ascending) on crafted rows.
"""

import itertools
import math
import os

import numpy as np
import pytest
import torch

from oracle import builder as B

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "builder_golden.npz")


def golden_cases():
    z = np.load(GOLDEN, allow_pickle=False)
    for i in range(int(z["n"])):
        yield i, {k: z[f"c{i}_{k}"] for k in ("kind", "lp", "ids", "prior", "budget", "tree", "count", "vis")}


def test_heap_matches_reference_golden_vectors():
    seen = 0
    for i, c in golden_cases():
        budget = int(c["budget"])
        n = int(c["count"])
        if str(c["kind"]) == "mixture":
            t, d, p, cnt, _ = B.build_mixture(c["lp"], c["ids"], c["prior"], budget)
        else:
            t, d, p, cnt = B.build_single(c["lp"][0], c["ids"][0], budget)
        assert cnt == n, f"case {i}"
        np.testing.assert_array_equal(np.stack([t, d, p]), c["tree"], err_msg=f"case {i}")
        vis = np.unpackbits(c["vis"])[: (n + 1) ** 2].reshape(n + 1, n + 1)
        np.testing.assert_array_equal(B.visibility(p, n), vis, err_msg=f"case {i}")
        seen += 1
    assert seen >= 80


@pytest.mark.skipif(B.ref_sglang_builder() is None, reason="oracle/_ref not built (needs /root/reference)")
def test_heap_matches_compiled_reference_random_trials():
    sg = B.ref_sglang_builder()
    gen = torch.Generator().manual_seed(7)
    for trial in range(150):
        modes = (2, 8, 3)[trial % 3]
        depth = int(torch.randint(1, 16, (1,), generator=gen))
        vocab = 64 if trial % 5 else 512
        budget = (16, 31, 63, 128, 255)[(trial // 3) % 5]
        logits = torch.randn(modes, depth, vocab, generator=gen) * 3
        if trial % 4 == 0:
            logits = (logits * 2).round() / 2
        lp = logits.to(torch.bfloat16).float()
        top, ids = torch.topk(lp, k=min(budget, vocab), dim=-1)
        logp = (top - torch.logsumexp(lp, -1, keepdim=True)).float()
        prior = torch.log_softmax(torch.randn(modes, generator=gen), -1) if trial % 2 else torch.zeros(modes)
        tree = torch.empty((1, 3, budget + 1), dtype=torch.long)
        counts = torch.empty(1, dtype=torch.long)
        sg.build_trees(logp[None].contiguous(), ids[None].to(torch.int32).contiguous(), prior[None].contiguous(), 1,
                       budget, tree, counts)
        t, d, p, n, _ = B.build_mixture(logp.numpy(), ids.numpy(), prior.numpy(), budget)
        assert n == int(counts[0]), trial
        np.testing.assert_array_equal(np.stack([t, d, p]), tree[0].numpy(), err_msg=f"trial {trial}")


def prefixes(tokens, parents, n):
    out = [()]
    for i in range(1, n + 1):
        out.append(out[parents[i]] + (int(tokens[i]),))
    return out[1:]


def test_top_budget_prefixes_by_max_over_modes():
    gen = torch.Generator().manual_seed(0)
    compared = 0
    for trial in range(40):
        K, L, V = (1, 2, 3, 4)[trial % 4], 3, 4
        budget = (5, 12, 30)[trial % 3]
        logits = torch.randn(K, L, V, generator=gen) * 2
        prior = torch.log_softmax(torch.randn(K, generator=gen), -1) if trial % 2 else torch.zeros(K)
        logp = torch.log_softmax(logits.double(), -1)
        scored = []
        for length in range(1, L + 1):
            for prefix in itertools.product(range(V), repeat=length):
                s = max(float(prior[k]) + sum(float(logp[k, i, t]) for i, t in enumerate(prefix)) for k in range(K))
                scored.append((s, prefix))
        scored.sort(reverse=True)
        if len(scored) > budget and abs(scored[budget - 1][0] - scored[budget][0]) < 1e-6:
            continue
        top, ids = torch.topk(logp.float(), k=min(budget, V), dim=-1)
        t, d, p, n, _ = B.build_mixture(top.numpy(), ids.numpy(), prior.float().numpy(), budget)
        got = prefixes(t, p, n)
        assert len(got) == min(budget, len(scored)) and len(set(got)) == len(got)
        assert set(got) == {q for _, q in scored[:budget]}, trial
        assert [len(q) for q in got] == d[1 : n + 1].tolist()
        compared += 1
    assert compared >= 35


def test_one_mode_mixture_is_ddtree_on_continuous_values():
    gen = torch.Generator().manual_seed(1)
    for _ in range(30):
        logp = torch.log_softmax(torch.randn(1, 6, 10, generator=gen) * 2, -1)
        top, ids = torch.topk(logp, k=10, dim=-1)
        a = B.build_mixture(top.numpy(), ids.numpy(), np.zeros(1, np.float32), 40)
        s = B.build_single(top[0].numpy(), ids[0].numpy(), 40)
        for x, y in zip(a[:3], s[:3]):
            np.testing.assert_array_equal(x, y)


def test_structure_invariants_config1_shape():
    from oracle.synth import builder_logits

    lp, ids, _ = B.top_candidates(builder_logits(1)[:, :, :4096].contiguous().reshape(128, -1), 8)
    t, d, p, n, _ = B.build_mixture(lp.reshape(8, 16, 8), ids.reshape(8, 16, 8), np.zeros(8, np.float32), 64)
    assert n == 64 and p[0] == -1
    vis = B.visibility(p, n)
    for i in range(1, n + 1):
        assert p[i] < i and d[i] == d[p[i]] + 1
        anc = {i}
        j = p[i]
        while j >= 0:
            anc.add(int(j))
            j = p[j]
        assert set(np.nonzero(vis[i])[0].tolist()) == anc


def _py_mixture(lp, ids, prior, budget, mistake=None):
    """Small heapq restatement of the heap, used only to plant mistakes (the C oracle is the pinned one)."""
    import heapq

    K, L, k = lp.shape
    key = lambda lw, m: float(-(np.float32(lw) + prior[m]))
    heap = [(key(float(lp[m, 0, 0]), m), m, 0, 1, 0, float(lp[m, 0, 0])) for m in range(K)]
    heapq.heapify(heap)
    tokens, depths, parents, child = [0], [0], [-1], [dict()]
    while heap and len(tokens) - 1 < budget:
        _, m, par, d, r, lw = heapq.heappop(heap)
        tok = int(ids[m, d - 1, r])
        cur = None if mistake == "no_reuse" else child[par].get(tok)
        if cur is None:
            cur = len(tokens)
            tokens.append(tok); depths.append(d); parents.append(par); child.append(dict())
            child[par][tok] = cur
        if r + 1 < k:
            drop = 0.0 if mistake == "dropped_term" else float(lp[m, d - 1, r])
            lw2 = lw - drop + float(lp[m, d - 1, r + 1])
            heapq.heappush(heap, (key(lw2, m), m, par, d, r + 1, lw2))
        if d < L:
            lw2 = lw + float(lp[m, d, r if mistake == "wrong_index" else 0])
            heapq.heappush(heap, (key(lw2, m), m, cur, d + 1, 0, lw2))
    return tokens, depths, parents


@pytest.mark.parametrize("mistake", ["dropped_term", "wrong_index", "no_reuse"])
def test_planted_mistakes_are_caught(mistake):
    """The restatement reproduces every golden tree; each planted mistake changes some of them."""
    changed = 0
    for i, c in golden_cases():
        if str(c["kind"]) != "mixture":
            continue
        n = int(c["count"])
        ok = _py_mixture(c["lp"], c["ids"], c["prior"], int(c["budget"]))
        assert ok[2] == c["tree"][2, : n + 1].tolist() and ok[0] == c["tree"][0, : n + 1].tolist(), i
        bad = _py_mixture(c["lp"], c["ids"], c["prior"], int(c["budget"]), mistake)
        if bad[2] != c["tree"][2, : n + 1].tolist() or bad[0] != c["tree"][0, : n + 1].tolist():
            changed += 1
    assert changed > 0, mistake


# ---------------------------------------------------------------- logits step


def test_exp_det_and_log_det_accuracy():
    for d in np.linspace(-80, 0, 2001):
        x = B.exp_det(float(np.float32(d)))
        assert abs(x - math.exp(float(np.float32(d)))) <= 3e-7 * math.exp(float(np.float32(d)))
    for z in (1.0, 1.5, 2.0, 3.7, 1e3, 123456.789, 2.0 ** 40 + 3):
        assert abs(B.log_det(z) - math.log(z)) <= 4e-16 * max(1.0, math.log(z))


def _bf16_value(bits: int) -> float:
    return float(np.array([bits << 16], dtype=np.uint32).view(np.float32)[0])


def test_exp_table_entries_and_index():
    """The e^x table over bf16 x: the kernel's header (exp_bf16_table.h) equals the oracle's entry by entry;
    every bf16 bit pattern with 2^-25 <= |x| < 88 reaches, through the index function, the float nearest to
    e^x (so a wrong sign position, base or shift in the index fails); magnitudes below 2^-25 read 1.0, magnitudes
    of 128 and above and -inf read 0.0."""
    import re

    hdr = open(os.path.join(os.path.dirname(__file__), "..", "multi-future-drafting_amd", "csrc", "exp_bf16_table.h")).read()
    vals = np.array([int(v, 16) for v in re.findall(r"0x([0-9a-f]{8})u", hdr)], dtype=np.uint32).view(np.float32)
    assert vals.size == 8192
    ora = np.array([B.exp_table(i) for i in range(8192)], dtype=np.float32)
    np.testing.assert_array_equal(vals.view(np.uint32), ora.view(np.uint32))
    for bits in range(65536):
        x = _bf16_value(bits)
        if not np.isfinite(x):
            continue
        e = ora[B.exp_table_index(bits)]
        if 2.0 ** -25 <= abs(x) < 88.0:
            ref = math.exp(x)
            assert abs(float(e) - ref) <= 2.0 ** -24 * ref, (hex(bits), x, e, ref)
        elif abs(x) < 2.0 ** -25:
            assert e == 1.0
        elif abs(x) >= 128.0:
            assert e == 0.0
    assert ora[B.exp_table_index(0xFF80)] == 0.0  # -inf
    # a planted mistake: the sign taken from bit 14 instead of bit 15 sends -1.0 to e^+1
    bad = ((0xBF80 << 1) | ((0xBF80 >> 14) & 1)) & 0xFFFF
    assert abs(float(ora[min(max(bad - 0x6600, 0), 8191)]) - math.exp(-1.0)) > 1e-3


@pytest.mark.parametrize("scale,shift", [(3.0, 0.0), (3.0, 55.0), (1.0, -55.0), (0.01, 0.0), (3.0, 70.0),
                                         (3.0, -70.0), (30.0, 0.0)])
def test_chunk_sum_accuracy(scale, shift):
    """S_c against sum e^(x - m) in float64 for chunks whose maximum lies inside the table range (-60 <= m < 64)
    and outside it (the polynomial path), full and partial (the row's last chunk); relative error <= 2e-6.
    A planted mistake (the table's C taken as E(m) instead of E(-m)) is far outside that bound."""
    rng = np.random.default_rng(int(scale * 100 + shift))
    for n in (1, 1500, 2048):
        x = torch.from_numpy(rng.standard_normal(n) * scale + shift).to(torch.bfloat16)
        bits = x.view(torch.int16).numpy().view(np.uint16)
        xf = x.double().numpy()
        m = float(xf.max())
        s = B.chunk_sum(bits, np.float32(m))
        ref = float(np.exp(xf - m).sum())
        assert abs(s - ref) <= 2e-6 * ref, (n, s, ref)
    if -60 <= m < 64 and abs(m) > 1:
        mb = int(np.array([np.float32(m)], dtype=np.float32).view(np.uint32)[0] >> 16)
        C_bad = np.float64(B.exp_table(B.exp_table_index(mb)))
        s_bad = float(sum(np.float64(B.exp_table(B.exp_table_index(int(b)))) * C_bad for b in bits))
        assert abs(s_bad - ref) > 1e-3 * ref


def test_chunk_sum_all_minus_inf():
    bits = np.full(2048, 0xFF80, dtype=np.uint16)
    assert B.chunk_sum(bits, -np.inf) == 0.0


@pytest.mark.parametrize("V,scale", [(151936, 3.0), (5000, 16.0), (8192, 1.0), (8193, 4.0), (2049, 2.0), (1, 1.0)])
def test_logz_and_topk_against_torch(V, scale):
    g = torch.Generator().manual_seed(V)
    x = (torch.randn(6, V, generator=g) * scale).to(torch.bfloat16)
    k = min(8, V)
    lp, ids, lz = B.top_candidates(x, k)
    ref = torch.logsumexp(x.double(), -1).numpy()
    assert np.abs(lz - ref).max() <= 2e-6 * max(1.0, np.abs(ref).max())
    tv, _ = torch.topk(x.float(), k, dim=-1)
    np.testing.assert_array_equal(np.take_along_axis(x.float().numpy(), ids, -1), tv.numpy())
    np.testing.assert_allclose(lp, tv.numpy() - lz[:, None], rtol=0, atol=0)


def test_topk_tie_rule_value_desc_id_asc():
    x = torch.full((2, 50), -5.0)
    x[0, [3, 7, 11, 40]] = 2.0
    x[0, 20] = 3.0
    x[1, :] = 1.0
    lp, ids, _ = B.top_candidates(x.to(torch.bfloat16), 4)
    assert ids[0].tolist() == [20, 3, 7, 11]
    assert ids[1].tolist() == [0, 1, 2, 3]


def test_all_minus_inf_row_and_spike():
    x = torch.full((2, 20000), float("-inf"))
    x[1, 12345] = 7.0
    lp, ids, lz = B.top_candidates(x.to(torch.bfloat16), 2)
    assert lz[0] == -np.inf and lz[1] == np.float32(7.0)
    assert ids[1, 0] == 12345 and lp[1, 0] == 0.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_wide_oracle_against_torch(dtype):
    """The float32 / float16 restatement against torch's own topk and logsumexp (in float64), ties by column."""
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(5, 30011, generator=g) * 4).to(dtype)
    x[2, :] = (x[2, :].float() * 2).round().to(dtype) / 2  # many exact ties
    k = 40
    lp, ids, lz = B.top_candidates_wide(x, k)
    ref = torch.logsumexp(x.double(), -1).numpy()
    assert np.abs(lz - ref).max() <= 1e-12 * max(1.0, np.abs(ref).max())
    tv, _ = torch.topk(x.double(), k, dim=-1)
    np.testing.assert_array_equal(np.take_along_axis(x.double().numpy(), ids, -1), tv.numpy())
    # among equal values the lower column comes first
    vals = np.take_along_axis(x.double().numpy(), ids, -1)
    same = vals[:, 1:] == vals[:, :-1]
    assert (ids[:, 1:][same] > ids[:, :-1][same]).all()
    np.testing.assert_allclose(lp, tv.numpy() - lz[:, None], rtol=0, atol=1e-12)


def test_wide_oracle_planted_mistake_is_caught():
    """A restatement that keeps the largest values but breaks ties by column descending fails the tie check."""
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0]])
    _, ids, _ = B.top_candidates_wide(x, 3)
    assert ids[0].tolist() == [1, 2, 4]
    bad = np.lexsort((-np.arange(5), -x[0].double().numpy()))[:3]
    assert bad.tolist() != ids[0].tolist()
