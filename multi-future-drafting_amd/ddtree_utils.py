"""SGLang-facing tree utilities on MI355X — the hot-path subset of the SGLang patch's ``ddtree_utils`` module
(inference/sglang/patches/sglang-v0.5.22-mfd.patch:1027-1550): ``build_trees`` / ``build_trees_cpu`` (the
batched mixture builder) and ``row_logsumexp``, plus ``build_mixture_trees_from_logits``, the device pipeline
from draft logits to trees that replaces the patch's D2H -> host heap -> H2D round trip.
"""

from __future__ import annotations

from typing import Optional

import torch

import mfd_hip
import tree_build_ext
import tree_logits


def build_trees(*, top_log_probs: torch.Tensor, top_ids: torch.Tensor, log_prior: torch.Tensor, bs: int, budget: int,
                tree: torch.Tensor, counts: torch.Tensor) -> None:
    """Device tree build for ``bs`` requests into ``tree[bs, 3, B + 1]`` (tokens, depths, parents; index 0 = root,
    tail (0, 0, -1)) and ``counts[bs]`` (P:1377-1407). All tensors on the GPU; no host synchronisation."""
    tree_build_ext.build_trees_device(top_log_probs[:bs], top_ids[:bs], log_prior[:bs], budget, tree=tree[:bs],
                                      counts=counts[:bs], single_mode_heap=True)


def build_trees_cpu(*, top_log_probs, top_ids, log_prior, bs: int, budget: int, tree, counts) -> None:
    """The patch's host-tensor contract (P:1431-1445): inputs and outputs on the CPU. The build runs on the GPU;
    the tensors are copied there and back."""
    dev = torch.device("cuda")
    t, c, _ = tree_build_ext.build_trees_device(top_log_probs[:bs].to(dev), top_ids[:bs].to(dev),
                                                log_prior[:bs].to(dev), budget, single_mode_heap=True)
    tree[:bs].copy_(t.cpu())
    counts[:bs].copy_(c.cpu())


def row_logsumexp(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """log-sum-exp over the last dim of a 2D row-major bf16 CUDA tensor, float32 [rows] (P:1472-1482)."""
    assert x.ndim == 2 and x.stride(1) == 1
    _, _, logz = tree_logits.topk_logz(x, 0, with_logz=True)
    if out is not None:
        out.copy_(logz)
        return out
    return logz


def build_mixture_trees_from_logits(draft_logits: torch.Tensor, mode_log_prior: Optional[torch.Tensor], budget: int,
                                    topk: Optional[int] = None, with_visibility: bool = True):
    """draft_logits [bs, K, L, V] (or [K, L, V]) bf16 on the GPU -> (tree [bs, 3, B + 1], counts [bs],
    anc8 [bs, B + 1, B + 1] or None, top log-probs, top ids), all on the device. ``topk`` defaults to
    min(budget, V) as the reference (inference/hf/ddtree.py:232)."""
    if draft_logits.dim() == 3:
        draft_logits = draft_logits[None]
        if mode_log_prior is not None and mode_log_prior.dim() == 1:
            mode_log_prior = mode_log_prior[None]
    bs, K, L, V = draft_logits.shape
    k = min(budget, V) if topk is None else topk
    logp, ids = tree_logits.topk_logz(draft_logits, k, ids_dtype=torch.int32)
    tree, counts, anc8 = tree_build_ext.build_trees_device(logp, ids, mode_log_prior, budget,
                                                           with_visibility=with_visibility)
    return tree, counts, anc8, logp, ids
