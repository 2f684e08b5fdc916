"""SGLang-facing tree utilities on MI355X — the hot-path subset of the SGLang patch's ``ddtree_utils`` module
(inference/sglang/patches/sglang-v0.5.22-mfd.patch:1027-1550): ``build_trees`` / ``build_trees_cpu`` (the
batched mixture builder) and ``row_logsumexp``, plus ``build_mixture_trees_from_logits``, the device pipeline
from draft logits to trees that replaces the patch's D2H -> host heap -> H2D round trip.

The patch's ``ddtree_utils`` module also holds the engine configuration (``DDTreeProfile``, ``ddtree_budget``,
``ddtree_enabled``, ...) that the worker and the CUDA-graph runner import, so this module does not take its
name: ``install()`` rebinds the hot-path names on the patch's modules (``ddtree_utils`` and
``ddtree_mode_attention``) instead and leaves everything else of them as it is.
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
    """The patch's host-tensor contract (P:1431-1445): inputs and outputs on the CPU, the build on the calling
    thread (mfd_build_trees_host: the mixture heap for K > 1, the DDTree heap for K == 1; no GPU work)."""
    if bs <= 0:
        return
    # rows [0, bs) of row-major tensors start at their data pointers: no slicing needed (called every round)
    lp, ids, prior = top_log_probs, top_ids, log_prior
    if (lp.is_cuda or ids.is_cuda or tree.is_cuda or counts.is_cuda or lp.dtype != torch.float32
            or ids.dtype != torch.int32 or tree.dtype != torch.int64 or counts.dtype != torch.int64):
        raise TypeError("build_trees_cpu takes CPU tensors: float32 log-probs, int32 ids, int64 tree / counts")
    if prior is not None and (prior.is_cuda or prior.dtype != torch.float32):
        raise TypeError("log_prior must be a float32 CPU tensor")
    if not lp.is_contiguous():
        lp = lp[:bs].contiguous()
    if not ids.is_contiguous():
        ids = ids[:bs].contiguous()
    if prior is not None and not prior.is_contiguous():
        prior = prior[:bs].contiguous()
    _, K, L, k = lp.shape
    if not (tree.is_contiguous() and counts.is_contiguous()) or tree.shape[1:] != (3, budget + 1):
        raise ValueError(f"tree must be a contiguous [bs, 3, {budget + 1}] tensor")
    if lp.shape[0] < bs or ids.shape != lp.shape or tree.shape[0] < bs or counts.shape[0] < bs:
        raise ValueError("fewer rows than bs")
    mfd_hip.call("mfd_build_trees_host", lp.data_ptr(), ids.data_ptr(), 0, None if prior is None else prior.data_ptr(),
                 bs, K, L, k, budget, 1, tree.data_ptr(), counts.data_ptr(), None)


def row_logsumexp(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """log-sum-exp over the last dim of a 2D row-major bf16, fp16 or fp32 CUDA tensor, float32 [rows]
    (P:1472-1482)."""
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


def ddtree_verify_inputs(*, root_tokens: torch.Tensor, prefix_lens: torch.Tensor, tokens: torch.Tensor,
                         depths: torch.Tensor, parents: torch.Tensor, mask_offsets: torch.Tensor, ids_out: torch.Tensor,
                         positions_out: torch.Tensor, mask_out: torch.Tensor, max_depth: int, err_flag=None) -> None:
    """Verify ids, positions and the flat tree mask of a batch (P:1670-1700): for request b and node i,
    ids_out[b, i] = root token or token, positions_out[b, i] = prefix + depth, and mask row i at
    mask_offsets[b] of length prefix + W = [prefix ones | ancestor-or-self bits]. tokens / depths / parents:
    [bs, W] int64 views with one row stride (the rows of the [bs, 3, W] tree); mask_out bool."""
    bs, W = tokens.shape
    if bs == 0:
        return
    assert tokens.stride() == depths.stride() == parents.stride() and tokens.stride(1) == 1
    mfd_hip.require_cuda(root_tokens, prefix_lens, tokens, mask_offsets, ids_out, positions_out, mask_out)
    for t in (root_tokens, prefix_lens, tokens, mask_offsets, ids_out, positions_out):
        if t.dtype != torch.int64:
            raise TypeError("verify inputs take int64 tensors (mask_out bool)")
    assert ids_out.is_contiguous() and positions_out.is_contiguous() and mask_out.is_contiguous()
    mfd_hip.call("mfd_verify_inputs", root_tokens.data_ptr(), prefix_lens.data_ptr(), tokens.data_ptr(),
                 depths.data_ptr(), parents.data_ptr(), tokens.stride(0), mask_offsets.data_ptr(), ids_out.data_ptr(),
                 positions_out.data_ptr(), mask_out.data_ptr(), bs, W, int(max_depth), mfd_hip.ptr(err_flag),
                 mfd_hip.stream_of(tokens))


def ddtree_follow(*, posterior: torch.Tensor, verify_ids: torch.Tensor, parents: torch.Tensor, window: torch.Tensor,
                  prefix_lens: torch.Tensor, accept_len_out: torch.Tensor, commit_lens_out: torch.Tensor,
                  bonus_out: torch.Tensor, out_tokens_out: torch.Tensor, new_seq_lens_out: torch.Tensor,
                  move_src_out: torch.Tensor, move_tgt_out: torch.Tensor, hidden_index_out: torch.Tensor) -> None:
    """Accept walk of a verified batch and its commit (P:1844-1885): accepted path, tokens + bonus, KV moves
    window[path[j]] -> window[j], hidden rows of the path. L = out_tokens_out.shape[1] <= 64."""
    bs, W = verify_ids.shape
    if bs == 0:
        return
    L = int(out_tokens_out.shape[1])
    assert parents.stride(1) == 1 and posterior.is_contiguous() and window.is_contiguous()
    assert verify_ids.is_contiguous()
    mfd_hip.require_cuda(posterior, verify_ids, parents, window, prefix_lens)
    mfd_hip.call("mfd_tree_follow", posterior.data_ptr(), verify_ids.data_ptr(), parents.data_ptr(),
                 parents.stride(0), window.data_ptr(), prefix_lens.data_ptr(), accept_len_out.data_ptr(),
                 commit_lens_out.data_ptr(), bonus_out.data_ptr(), out_tokens_out.data_ptr(),
                 new_seq_lens_out.data_ptr(), move_src_out.data_ptr(), move_tgt_out.data_ptr(),
                 hidden_index_out.data_ptr(), bs, W, L, mfd_hip.stream_of(verify_ids))


def ddtree_prepare(*, bonus_tokens: torch.Tensor, prefix_lens: torch.Tensor, req_pool_indices: torch.Tensor,
                   req_to_token: torch.Tensor, block_ids_out: torch.Tensor, positions_out: torch.Tensor,
                   window_out: torch.Tensor, mask_token_id: int) -> None:
    """Draft-block ids / positions and the verify window's cache slots of a round (P:1590-1623): for request b,
    block_ids_out[b] = [bonus, mask, ..., mask], positions_out[b, l] = prefix + l, and window_out[b, w] =
    req_to_token[req_pool_indices[b], prefix + w]. Index inputs int32 or int64; outputs int64."""
    bs = int(bonus_tokens.numel())
    if bs == 0:
        return
    L, W = int(block_ids_out.shape[1]), int(window_out.shape[1])
    assert req_to_token.stride(1) == 1
    mfd_hip.require_cuda(bonus_tokens, prefix_lens, req_pool_indices, req_to_token, block_ids_out, positions_out,
                         window_out)
    flags = 0
    for bit, t in enumerate((bonus_tokens, prefix_lens, req_pool_indices, req_to_token)):
        if t.dtype == torch.int64:
            flags |= 1 << bit
        elif t.dtype != torch.int32:
            raise TypeError(f"index tensors must be int32 or int64, got {t.dtype}")
    for t in (block_ids_out, positions_out, window_out):
        if t.dtype != torch.int64 or not t.is_contiguous():
            raise TypeError("ddtree_prepare writes contiguous int64 outputs")
    bonus, prefix, pool = (t.contiguous() for t in (bonus_tokens, prefix_lens, req_pool_indices))
    mfd_hip.call("mfd_draft_prepare", bonus.data_ptr(), prefix.data_ptr(), pool.data_ptr(), req_to_token.data_ptr(),
                 req_to_token.stride(0), flags, int(mask_token_id), block_ids_out.data_ptr(), positions_out.data_ptr(),
                 window_out.data_ptr(), bs, L, W, mfd_hip.stream_of(block_ids_out))


def ddtree_mode_mask(*, prefix_lens: torch.Tensor, mask_offsets: torch.Tensor, mask_out: torch.Tensor, num_modes: int,
                     block_size: int) -> None:
    """Multi-mode draft mask rows (P:1914-1935): row r of request b, at mask_offsets[b] + r (prefix + K L), is
    prefix ones then the L columns of row r's own mode block. prefix_lens / mask_offsets int64; mask_out bool."""
    bs = int(prefix_lens.numel())
    if bs == 0:
        return
    mfd_hip.require_cuda(prefix_lens, mask_offsets, mask_out)
    if prefix_lens.dtype != torch.int64 or mask_offsets.dtype != torch.int64:
        raise TypeError("prefix_lens and mask_offsets must be int64")
    if mask_out.element_size() != 1 or not mask_out.is_contiguous():
        raise TypeError("mask_out must be a contiguous one-byte (bool) tensor")
    mfd_hip.call("mfd_mode_mask", prefix_lens.contiguous().data_ptr(), mask_offsets.contiguous().data_ptr(),
                 mask_out.data_ptr(), bs, int(num_modes), int(block_size), mfd_hip.stream_of(mask_out))


class DDTreeKVCompactor:
    """Commit-time KV moves on a token-major pool (P:1805-1841): one device array of buffer addresses (the
    pool's per-layer K and V buffers), one slot stride; only the moves that change a slot are copied, every
    source of a request before any target."""

    def __init__(self, kv_pool=None, *, data_ptrs: torch.Tensor | None = None, slot_bytes: int | None = None,
                 num_slots: int | None = None):
        if kv_pool is not None:
            strides = {int(s) for s in kv_pool.data_strides.tolist()}
            if len(strides) != 1 or next(iter(strides)) % 16:
                raise ValueError(f"DDTree KV compaction needs one slot stride (multiple of 16 bytes), got {strides}")
            data_ptrs, slot_bytes = kv_pool.data_ptrs, next(iter(strides))
            num_slots = num_slots or int(getattr(kv_pool, "size", 0) + getattr(kv_pool, "page_size", 1))
        if data_ptrs is None or slot_bytes is None:
            raise ValueError("a kv_pool or data_ptrs + slot_bytes is required")
        self.data_ptrs = data_ptrs
        self.slot_bytes = int(slot_bytes)
        self.num_slots = int(num_slots) if num_slots else 2 ** 62

    @staticmethod
    def supports(kv_pool) -> bool:
        strides = {int(s) for s in kv_pool.data_strides.tolist()}
        return len(strides) == 1 and next(iter(strides)) % 16 == 0

    def __call__(self, *, move_src: torch.Tensor, move_tgt: torch.Tensor, err_flag=None) -> None:
        bs, L = move_src.shape
        if bs == 0:
            return
        mfd_hip.call("mfd_kv_move", self.data_ptrs.data_ptr(), self.data_ptrs.numel(), self.slot_bytes, 1, 0,
                     self.slot_bytes, self.num_slots, move_src.contiguous().data_ptr(),
                     move_tgt.contiguous().data_ptr(), bs, L, mfd_hip.ptr(err_flag), mfd_hip.stream_of(move_src))


class DDTreeDraftTopK:
    """Top-k candidates of every drafted position, inside the draft step (the patch's DDTreeDraftTopK,
    P:1485-1544; same constructor keywords, call and outputs()).

    A draft step yields ``hidden_states [bs * num_modes * block_size, hidden]``: per (request, mode) block the
    anchor row, then the block_size - 1 drafted positions. One call of mfd_draft_topk_head runs the draft LM head
    over the drafted rows, read in place (csrc/draft_head.hip: a hand-written weight-stream GEMM into a static
    bf16 logits buffer), then the logits step (csrc/logits_topk.hip): their top-k log-probabilities (bf16 value
    minus an fp32 log Z), token ids and log Z. With a reduced draft vocabulary, ``weight`` holds the LM head's
    rows of ``vocab_ids`` (int32 [N]) and the winning columns are mapped back to full-vocabulary ids. Every buffer
    is sized at construction for ``max_bs`` requests: a call allocates nothing (for bf16 hidden states with
    16-byte aligned rows), so it can be captured in a graph."""

    def __init__(self, *, weight: torch.Tensor, block_size: int, num_modes: int, budget: int, max_bs: int,
                 vocab_ids: Optional[torch.Tensor] = None):
        mfd_hip.require_cuda(weight, vocab_ids)
        vocab, hidden = weight.shape
        if weight.dtype != torch.bfloat16 or not weight.is_contiguous() or weight.data_ptr() % 16 or hidden % 64:
            raise ValueError(f"weight must be a contiguous bf16 [vocab, hidden] matrix with hidden % 64 == 0, got "
                             f"{weight.dtype} {tuple(weight.shape)}")
        if vocab_ids is not None and (vocab_ids.dtype != torch.int32 or tuple(vocab_ids.shape) != (vocab,)):
            raise ValueError(f"vocab_ids must be int32 [{vocab}] (one id per LM-head row), got "
                             f"{vocab_ids.dtype} {tuple(vocab_ids.shape)}")
        self.weight = weight
        self.vocab_ids = None if vocab_ids is None else vocab_ids.contiguous()
        self.block_size, self.num_modes, self.max_bs = int(block_size), int(num_modes), int(max_bs)
        self.vocab = int(vocab)
        self.topk = min(int(budget), self.vocab)  # every rank a best-first tree of `budget` nodes can reach
        cap = self._rows(self.max_bs)
        dev = weight.device
        # logits rows padded to a multiple of 8 elements (16-byte aligned rows for both kernels)
        self._logits = torch.empty((cap, (self.vocab + 7) // 8 * 8), dtype=torch.bfloat16, device=dev)
        self.logits = self._logits[:, : self.vocab]
        self.top_logp = torch.empty((cap, self.topk), dtype=torch.float32, device=dev)
        self.top_ids = torch.empty((cap, self.topk), dtype=torch.int32, device=dev)
        self.log_z = torch.empty((cap,), dtype=torch.float32, device=dev)
        self.workspace = torch.empty(mfd_hip.lib().mfd_topk_logz_workspace_bytes(cap, self.vocab, self.topk),
                                     dtype=torch.uint8, device=dev)

    def _rows(self, bs: int) -> int:
        """Drafted rows of bs requests (the anchors excluded)."""
        return bs * self.num_modes * (self.block_size - 1)

    def __call__(self, hidden_states: torch.Tensor, input_ids=None) -> None:
        del input_ids  # the candidates depend on the hidden states only
        L, H = self.block_size, hidden_states.shape[-1]
        if H != self.weight.shape[1] or hidden_states.shape[0] % L:
            raise ValueError(f"hidden_states must be [blocks * {L}, {self.weight.shape[1]}], got "
                             f"{tuple(hidden_states.shape)}")
        x = hidden_states
        if x.dtype != torch.bfloat16 or x.stride(-1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
            x = x.to(torch.bfloat16).contiguous()
        n = (x.shape[0] // L) * (L - 1)
        if n > self.logits.shape[0]:
            raise ValueError(f"{n} drafted rows exceed the {self.logits.shape[0]} of max_bs={self.max_bs}")
        rs = x.stride(0)
        mfd_hip.call("mfd_draft_topk_head", x.data_ptr() + rs * 2, rs, L - 1, L * rs, self.weight.data_ptr(), n,
                     self.vocab, H, self._logits.data_ptr(), self._logits.stride(0), self.topk,
                     self.top_logp.data_ptr(), self.top_ids.data_ptr(), 0, self.log_z.data_ptr(),
                     mfd_hip.ptr(self.vocab_ids), self.workspace.data_ptr(), self.workspace.numel(),
                     mfd_hip.stream_of(x))

    def outputs(self, bs: int):
        """(top_logp [bs, K, L - 1, k] float32, top_ids [bs, K, L - 1, k] int32), views of the static buffers."""
        n = self._rows(bs)
        dims = (bs, self.num_modes, self.block_size - 1, self.topk)
        return self.top_logp[:n].view(dims), self.top_ids[:n].view(dims)


# names of the patch's ddtree_utils this module replaces (P:1431-1885), plus the device builder it adds
SGLANG_UTILS_NAMES = ("build_trees_cpu", "row_logsumexp", "DDTreeDraftTopK", "ddtree_prepare", "ddtree_verify_inputs",
                      "DDTreeKVCompactor", "ddtree_follow", "ddtree_mode_mask", "build_trees")
# names of the patch's ddtree_mode_attention this package replaces (P:886-1026)
SGLANG_ATTENTION_NAMES = ("resolve_ctx_splits", "paged_mode_block_attention", "paged_mode_block_attention_reference",
                          "PagedModeAttention")


def install(utils_module=None, attention_module=None) -> dict:
    """Rebind the hot-path names of the SGLang patch's ``sglang.srt.speculative.ddtree_utils`` and
    ``ddtree_mode_attention`` modules (defaults: those modules, imported) to this package's, together with any
    imported module that bound them by name (the worker's ``from ...ddtree_utils import build_trees_cpu, ...``,
    P:2003-2030). Call it before the worker module is imported, or after: both work. Returns
    {name: the patch's object (None for the added ``build_trees``)}."""
    import paged_mode_attention

    if utils_module is None:
        from sglang.srt.speculative import ddtree_utils as utils_module
    if attention_module is None:
        from sglang.srt.speculative import ddtree_mode_attention as attention_module
    old = mfd_hip.rebind(utils_module, {name: globals()[name] for name in SGLANG_UTILS_NAMES})
    old.update(mfd_hip.rebind(attention_module,
                              {name: getattr(paged_mode_attention, name) for name in SGLANG_ATTENTION_NAMES}))
    return old
