"""Best-first construction of the multi-mode mixture tree on MI355X — drop-in for the reference's
inference/hf/tree_build_ext.py (build_mixture, Tree, load_module) and the SGLang build_trees entry.

The heaps run on the device (csrc/tree_build.hip): one wave per request reproduces the reference C++ heaps'
pop order node for node — the mixture heap (fp32 key -(float(logw) + log prior), fp64 logw, ties by mode,
parent, depth, rank; a prefix popped again by another mode reuses its node) and the single-mode DDTree heap
(fp64 key, ties by the rank tuple) — and also emits the ancestor-or-self visibility matrix, so a device
pipeline (logits -> top-k / log Z -> tree) never round-trips to the host.
The HF-facing functions keep the reference's host-tensor contract: they move their inputs to the GPU,
build there, and return host tensors plus a Tree whose follow() walks the verified path.
"""

from __future__ import annotations

import torch

import mfd_hip


class Tree:
    """Child maps (token -> node per node) of a built tree; follow(posterior) walks the verified path
    (inference/hf/tree_build_ext.py:68-86)."""

    def __init__(self, tokens, parents):
        n = len(parents)
        self.child_maps = [dict() for _ in range(n)]
        for i in range(1, n):
            self.child_maps[int(parents[i])][int(tokens[i - 1])] = i

    def follow(self, posterior: torch.Tensor):
        post = posterior.to(device="cpu", dtype=torch.long).tolist()
        accepted, current = [0], 0
        nxt = post[0]
        while nxt in self.child_maps[current]:
            current = self.child_maps[current][nxt]
            accepted.append(current)
            nxt = post[current]
        return accepted, nxt

    def children(self, i: int) -> dict:
        return dict(self.child_maps[i])

    def __len__(self) -> int:
        return len(self.child_maps)


def load_module():
    """The device builder needs no runtime compilation; kept for interface compatibility."""
    return mfd_hip.lib()


def build_trees_device(top_log_probs: torch.Tensor, top_ids: torch.Tensor, log_prior, budget: int,
                       with_visibility: bool = False, tree: torch.Tensor | None = None,
                       counts: torch.Tensor | None = None, single_mode_heap: bool = False):
    """Device form. top_log_probs [bs, K, L, k] f32, top_ids [bs, K, L, k] int32 / int64, log_prior [bs, K] f32
    or None, all CUDA. Returns (tree [bs, 3, budget + 1] int64, counts [bs] int64, anc8 [bs, budget + 1,
    budget + 1] int8 or None); no host synchronisation. ``single_mode_heap``: one-mode requests (K == 1) use the
    DDTree heap (fp64 key, rank-tuple ties), as the SGLang build_trees does (P:1397-1398); otherwise every K uses
    the mixture heap, as the HF build_mixture does (inference/hf/ddtree.py:247-254)."""
    mfd_hip.require_cuda(top_log_probs, top_ids, log_prior)
    bs, K, L, k = top_log_probs.shape
    if top_ids.shape != top_log_probs.shape:
        raise ValueError("top_ids must match top_log_probs")
    lp = top_log_probs.contiguous().float()
    ids = top_ids.contiguous()
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.to(torch.int64)
    prior = None if log_prior is None else log_prior.reshape(bs, K).contiguous().float()
    dev = lp.device
    W = budget + 1
    if tree is None:
        tree = torch.empty(bs, 3, W, dtype=torch.int64, device=dev)
    if counts is None:
        counts = torch.empty(bs, dtype=torch.int64, device=dev)
    anc8 = torch.empty(bs, W, W, dtype=torch.int8, device=dev) if with_visibility else None
    i64 = 1 if ids.dtype == torch.int64 else 0
    if K == 1 and single_mode_heap:
        mfd_hip.call("mfd_build_single", lp.data_ptr(), ids.data_ptr(), i64, bs, L, k, budget, tree.data_ptr(),
                     counts.data_ptr(), mfd_hip.ptr(anc8), None, mfd_hip.stream_of(lp))
    else:
        mfd_hip.call("mfd_build_mixture", lp.data_ptr(), ids.data_ptr(), i64, mfd_hip.ptr(prior), bs, K, L, k, budget,
                     tree.data_ptr(), counts.data_ptr(), mfd_hip.ptr(anc8), None, mfd_hip.stream_of(lp))
    return tree, counts, anc8


def _host_result(tree, counts, anc8):
    tree, n, anc8 = tree.cpu(), int(counts.cpu()[0]), anc8.cpu()
    tokens = tree[0, 0, 1 : n + 1].clone()
    depths = tree[0, 1, 1 : n + 1].clone()
    parents = tree[0, 2, : n + 1].tolist()
    vis = anc8[0, : n + 1, : n + 1].to(torch.bool)
    return tokens, depths, parents, Tree(tokens.tolist(), parents), vis


def _build_host(lp, ids, prior, budget: int, single_mode_heap: bool):
    """One request on the host (mfd_build_trees_host): lp / ids [1, K, L, k] CPU tensors, prior [1, K] or None."""
    lp = lp.contiguous().float()
    ids = ids.contiguous()
    if ids.dtype not in (torch.int32, torch.int64):
        ids = ids.to(torch.int64)
    prior = None if prior is None else prior.contiguous().float()
    _, K, L, k = lp.shape
    W = budget + 1
    tree = torch.empty(1, 3, W, dtype=torch.int64)
    counts = torch.empty(1, dtype=torch.int64)
    anc8 = torch.empty(1, W, W, dtype=torch.int8)
    mfd_hip.call("mfd_build_trees_host", lp.data_ptr(), ids.data_ptr(), 1 if ids.dtype == torch.int64 else 0,
                 mfd_hip.ptr(prior), 1, K, L, k, budget, 1 if single_mode_heap else 0, tree.data_ptr(),
                 counts.data_ptr(), anc8.data_ptr())
    return tree, counts, anc8


def build_mixture(top_log_probs: torch.Tensor, top_token_ids: torch.Tensor, log_prior: torch.Tensor, budget: int):
    """[K, L, k] float32 / int64 and [K] float32 tensors (host or device) -> (node_token_ids [n] int64,
    node_depths [n] int64, parents list of n + 1 (parents[0] = -1), Tree, visibility [n + 1, n + 1] bool),
    as inference/hf/tree_build_ext.py:231-234 returns them (host tensors). Host inputs (what the HF decode loop
    passes: top_candidates returns host tensors) are built on the host, device inputs by the device heap."""
    if not top_log_probs.is_cuda:
        return _host_result(*_build_host(top_log_probs[None], top_token_ids.cpu()[None], log_prior.cpu()[None],
                                         budget, single_mode_heap=False))
    dev = top_log_probs.device
    lp = top_log_probs.to(dev, torch.float32)[None]
    ids = top_token_ids.to(dev)[None]
    prior = log_prior.to(dev, torch.float32)[None]
    return _host_result(*build_trees_device(lp, ids, prior, budget, with_visibility=True))


def build_single(top_log_probs: torch.Tensor, top_token_ids: torch.Tensor, budget: int):
    """Single-mode DDTree (inference/hf/tree_build_ext.py:118-156, :229-230): [L, k] float32 / int64 tensors (host
    or device) -> the same tuple as build_mixture, built by the DDTree heap (fp64 key, ties by the rank tuple): on
    the host for host inputs, on the device otherwise."""
    if not top_log_probs.is_cuda:
        return _host_result(*_build_host(top_log_probs[None, None], top_token_ids.cpu()[None, None], None, budget,
                                         single_mode_heap=True))
    dev = top_log_probs.device
    lp = top_log_probs.to(dev, torch.float32)[None, None]
    ids = top_token_ids.to(dev)[None, None]
    return _host_result(*build_trees_device(lp, ids, None, budget, with_visibility=True, single_mode_heap=True))


def check_equal(trials: int = 200, seed: int = 0) -> None:
    """Self-test of inference/hf/tree_build_ext.py:237-270: the device builders against the reference's Python
    definitions ``ddtree.build_ddtree_tree`` (one mode) and ``ddtree.build_mixture_tree`` (the HF decode-loop
    module, which must be importable) on random bf16 logits, every fourth trial with coarse values that tie
    exactly; tokens, depths, parents, child maps, the verified walk and the visibility must be identical."""
    import ddtree

    gen = torch.Generator().manual_seed(seed)
    vocab = 64
    for trial in range(trials):
        modes = (1, 2, 8)[trial % 3]
        depth = int(torch.randint(1, 16, (1,), generator=gen))
        budget = (16, 64, 256)[(trial // 3) % 3]
        logits = torch.randn(modes, depth, vocab, generator=gen) * 3
        if trial % 4 == 0:
            logits = torch.round(logits * 2) / 2
        logits = logits.to(torch.bfloat16)
        prior = torch.log_softmax(torch.randn(modes, generator=gen), -1) if trial % 2 else torch.zeros(modes)
        lp = logits.float()
        top, ids = torch.topk(lp, k=min(budget, vocab), dim=-1)
        logp = (top - torch.logsumexp(lp, -1, keepdim=True)).float()
        if modes == 1:
            want = ddtree.build_ddtree_tree(logits[0], budget)
            got = build_single(logp[0], ids[0], budget)
        else:
            want = ddtree.build_mixture_tree(logits, prior, budget)
            got = build_mixture(logp, ids, prior, budget)
        where = f"trial {trial} (modes {modes}, depth {depth}, budget {budget})"
        if not (torch.equal(want[0], got[0]) and torch.equal(want[1], got[1])):
            raise AssertionError(f"{where}: node tokens or depths differ")
        if list(want[2]) != list(got[2]):
            raise AssertionError(f"{where}: parents differ")
        if [dict(c) for c in want[3]] != [got[3].children(i) for i in range(len(got[3]))]:
            raise AssertionError(f"{where}: child maps differ")
        posterior = torch.randint(0, vocab, (1, len(want[3])), generator=gen)
        first_child = torch.tensor([min(c) if c else 0 for c in want[3]])
        posterior[0, ::2] = first_child[::2]  # follow some edges
        if ddtree.follow_verified_tree(want[3], posterior) != ddtree.follow_verified_tree(got[3], posterior):
            raise AssertionError(f"{where}: verified walk differs")
        if not torch.equal(want[4], got[4]):
            raise AssertionError(f"{where}: visibility differs")
    print(f"tree_build_ext: {trials} trials identical to the Python builders")


if __name__ == "__main__":
    check_equal()
