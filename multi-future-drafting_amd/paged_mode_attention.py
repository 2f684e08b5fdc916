"""Paged attention of a multi-mode (MFD) DFlash draft step on MI355X — drop-in for the SGLang patch's
``ddtree_mode_attention`` module (inference/sglang/patches/sglang-v0.5.22-mfd.patch:593-1026).

The K mode blocks of a request sit side by side (K x block_size queries, mode-major); every query attends
to the request's context (the draft KV cache, read through ``req_to_token``) and to the block_size keys
of its own mode block (this step's projected k/v, never written to the cache). The kernel is the same as
mode_attention.py's (csrc/mode_attn.hip) with the context gathered through the slot table on the device:
  * page_size == 1: ``req_to_token[req_pool_indices[b], t]`` is the slot of context token t (the
    reference's only supported layout, P:2410-2414);
  * page_size  > 1: ``req_to_token`` is a page table, token t of request b lives at slot
    ``req_to_token[req_pool_indices[b], t // page_size] * page_size + t % page_size``.
Context lengths are read on the device and the grid depends only on the batch size and the split
count, so a captured graph replays correctly with new lengths.
"""

from __future__ import annotations

from typing import Optional

import torch

import mfd_hip
import mode_attention


def resolve_ctx_splits(num_ctx_splits: int, *, programs: int, device) -> int:
    """num_ctx_splits > 0: that many context splits (merged by log-sum-exp); 0: one fused pass; < 0: auto —
    fused once the (request, KV head, unit group) programs cover the CUs, else enough splits to cover them
    (at most 16). (P:886-894.)"""
    if num_ctx_splits >= 0:
        return num_ctx_splits
    want = mfd_hip.cu_count(device)
    if programs >= want:
        return 0
    return min(16, max(1, -(-want // programs)))


def paged_mode_block_attention(
    *,
    q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    req_to_token: torch.Tensor,
    req_pool_indices: torch.Tensor,
    ctx_lens: torch.Tensor,
    num_modes: int,
    block_size: int,
    scaling: float,
    num_ctx_splits: int,
    out: Optional[torch.Tensor] = None,
    modes_per_program: int = 2,
    block_n: int = 64,
    min_chunk: int = 64,
    num_warps: Optional[int] = None,
    page_size: int = 1,
    causal_in_block: bool = False,
) -> torch.Tensor:
    """q [T, H, D], k_new/v_new [T, Hkv, D] with T = bs * K * block_size (mode-major per request);
    k_cache/v_cache [slots, Hkv, D]; the context of request b is given by req_to_token[req_pool_indices[b]]
    and ctx_lens[b] (see the module docstring for page_size). Returns [T, H, D] (``out`` if given).
    ``modes_per_program``, ``block_n``, ``min_chunk`` and ``num_warps`` are accepted for signature
    compatibility."""
    del modes_per_program, block_n, min_chunk, num_warps
    T, H, D = q.shape
    Hkv = k_new.shape[1]
    KL = num_modes * block_size
    bs = T // KL
    assert T == bs * KL and H % Hkv == 0
    assert q.stride(-1) == 1 and k_new.stride(-1) == 1 and v_new.stride(-1) == 1
    assert k_cache.stride(-1) == 1 and v_cache.stride(-1) == 1 and req_to_token.stride(1) == 1
    assert req_to_token.dtype == torch.int32
    mfd_hip.require_cuda(q, k_new, v_new, k_cache, v_cache, req_to_token, req_pool_indices, ctx_lens)
    if out is None:
        out = torch.empty((T, H, D), device=q.device, dtype=q.dtype)
    if bs == 0:
        return out
    G = H // Hkv
    programs = bs * Hkv * -(-(G * KL // 32) // 4)
    splits = resolve_ctx_splits(num_ctx_splits, programs=programs, device=q.device)
    rpi = req_pool_indices[:bs]
    if rpi.dtype != torch.int64:
        rpi = rpi.to(torch.int64)
    cl = ctx_lens[:bs]
    if cl.dtype != torch.int64:
        cl = cl.to(torch.int64)
    return mode_attention.launch(
        q=q, q_st=q.stride(0), q_sh=q.stride(1), k_new=k_new, v_new=v_new, kn_st=k_new.stride(0),
        kn_sh=k_new.stride(1), vn_st=v_new.stride(0), vn_sh=v_new.stride(1), k_cache=k_cache, v_cache=v_cache,
        kc_ss=k_cache.stride(0), kc_sh=k_cache.stride(1), vc_ss=v_cache.stride(0), vc_sh=v_cache.stride(1),
        table=req_to_token, table_stride=req_to_token.stride(0), page_size=page_size, req_idx=rpi, ctx_lens=cl,
        ctx_const=0, bs=bs, num_modes=num_modes, block_size=block_size, H=H, Hkv=Hkv, D=D, scaling=scaling,
        causal=causal_in_block, splits=max(1, splits), out=out, o_st=out.stride(0), o_sh=out.stride(1),
        stream=mfd_hip.stream_of(q))


def _context_slots(row: torch.Tensor, ctx: int, page_size: int) -> torch.Tensor:
    """Cache slots of a request's ctx context tokens from its table row (per-token table or page table)."""
    if page_size == 1:
        return row[:ctx].long()
    t = torch.arange(ctx, device=row.device)
    return row[t // page_size].long() * page_size + t % page_size


def paged_mode_block_attention_reference(
    *, q, k_new, v_new, k_cache, v_cache, req_to_token, req_pool_indices, ctx_lens, num_modes, block_size, scaling,
    page_size: int = 1, causal_in_block: bool = False,
) -> torch.Tensor:
    """The float32 checking path of the patch (P:965-988): each request's context gathered from the cache through
    its table row, then mode_attention.modes_fp32 on it. Returns [T, H, D] float32 (runs where the tensors are)."""
    T, H, D = q.shape
    KL = num_modes * block_size
    out = torch.empty((T, H, D), device=q.device, dtype=torch.float32)
    for b in range(T // KL):
        slots = _context_slots(req_to_token[int(req_pool_indices[b])], int(ctx_lens[b]), page_size)
        rows = slice(b * KL, (b + 1) * KL)
        head_major = lambda t: t.transpose(0, 1)
        o = mode_attention.modes_fp32(head_major(q[rows]), head_major(k_cache[slots]), head_major(v_cache[slots]),
                                      head_major(k_new[rows]), head_major(v_new[rows]), num_modes, block_size,
                                      scaling, causal_in_block)
        out[rows] = o.transpose(0, 1)
    return out


class PagedModeAttention:
    """The DFlashAttention hook (``mode_attention``, P:222-225; the reference class P:991-1026): q / k / v of
    the multi-mode draft forward arrive as [T, heads * D] slices of the fused qkv and leave as [T, H * D].
    ``impl``: "hip" (this library's kernel; "triton", the reference's name for its kernel, selects it too) or
    "reference" (the float32 checking path)."""

    _KERNELS = ("hip", "triton")

    def __init__(self, *, kv_pool, req_to_token, num_modes: int, block_size: int, num_heads: int, num_kv_heads: int,
                 head_dim: int, scaling: float, num_ctx_splits: int, impl: str, page_size: int = 1):
        if impl not in self._KERNELS + ("reference",):
            raise ValueError(f"impl {impl!r}: one of hip, triton, reference")
        self.kv_pool, self.req_to_token = kv_pool, req_to_token
        self.shape = (int(num_heads), int(num_kv_heads), int(head_dim))
        self.blocks = (int(num_modes), int(block_size))
        self.scaling, self.num_ctx_splits, self.page_size = float(scaling), int(num_ctx_splits), int(page_size)
        self.exact = impl == "reference"

    def __call__(self, q, k, v, forward_batch, layer_id: int) -> torch.Tensor:
        H, Hkv, D = self.shape
        K, L = self.blocks
        T = q.shape[0]
        bs = T // (K * L)
        k_cache, v_cache = self.kv_pool.get_kv_buffer(layer_id)
        common = dict(q=q.view(T, H, D), k_new=k.view(T, Hkv, D), v_new=v.view(T, Hkv, D), k_cache=k_cache,
                      v_cache=v_cache, req_to_token=self.req_to_token,
                      req_pool_indices=forward_batch.req_pool_indices[:bs], ctx_lens=forward_batch.seq_lens[:bs],
                      num_modes=K, block_size=L, scaling=self.scaling, page_size=self.page_size)
        if self.exact:
            o = paged_mode_block_attention_reference(**common).to(q.dtype)
        else:
            o = paged_mode_block_attention(**common, num_ctx_splits=self.num_ctx_splits)
        return o.reshape(T, H * D)
