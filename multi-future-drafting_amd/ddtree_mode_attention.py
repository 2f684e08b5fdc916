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


def paged_mode_block_attention_reference(
    *, q, k_new, v_new, k_cache, v_cache, req_to_token, req_pool_indices, ctx_lens, num_modes, block_size, scaling,
    page_size: int = 1,
) -> torch.Tensor:
    """Float32 masked attention (mode_attention.reference on the gathered context); returns [T, H, D] float32.
    The checking path of the reference (P:965-988); runs where the tensors are."""
    T, H, D = q.shape
    Hkv = k_new.shape[1]
    KL = num_modes * block_size
    out = torch.empty((T, H, D), device=q.device, dtype=torch.float32)
    for b in range(T // KL):
        ctx = int(ctx_lens[b])
        row = req_to_token[int(req_pool_indices[b])]
        t = torch.arange(ctx, device=q.device)
        slots = row[:ctx].long() if page_size == 1 else row[t // page_size].long() * page_size + t % page_size
        rows = slice(b * KL, (b + 1) * KL)
        kk = torch.cat([k_cache[slots], k_new[rows]], 0).float()
        vv = torch.cat([v_cache[slots], v_new[rows]], 0).float()
        qb = q[rows].float().transpose(0, 1)
        kk = kk.transpose(0, 1).repeat_interleave(H // Hkv, dim=0)
        vv = vv.transpose(0, 1).repeat_interleave(H // Hkv, dim=0)
        mode = torch.arange(KL, device=q.device) // block_size
        mask = torch.zeros((KL, ctx + KL), device=q.device)
        mask[:, ctx:].masked_fill_(mode[:, None] != mode[None, :], float("-inf"))
        o = torch.nn.functional.scaled_dot_product_attention(qb, kk, vv, attn_mask=mask, scale=scaling)
        out[rows] = o.transpose(0, 1)
    return out


class PagedModeAttention:
    """Called by DFlashAttention (``mode_attention`` hook, P:222-225) in place of its RadixAttention for the
    multi-mode draft forward: q/k/v as [T, heads * D] slices of the fused qkv; returns [T, heads * D]."""

    def __init__(self, *, kv_pool, req_to_token, num_modes: int, block_size: int, num_heads: int, num_kv_heads: int,
                 head_dim: int, scaling: float, num_ctx_splits: int, impl: str, page_size: int = 1):
        self.kv_pool = kv_pool
        self.req_to_token = req_to_token
        self.num_modes = int(num_modes)
        self.block_size = int(block_size)
        self.num_heads = int(num_heads)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.scaling = float(scaling)
        self.num_ctx_splits = int(num_ctx_splits)
        self.page_size = int(page_size)
        assert impl in ("hip", "triton", "reference"), impl
        self.impl = impl

    def __call__(self, q, k, v, forward_batch, layer_id: int) -> torch.Tensor:
        T = q.shape[0]
        qh = q.view(T, self.num_heads, self.head_dim)
        kh = k.view(T, self.num_kv_heads, self.head_dim)
        vh = v.view(T, self.num_kv_heads, self.head_dim)
        k_cache, v_cache = self.kv_pool.get_kv_buffer(layer_id)
        bs = T // (self.num_modes * self.block_size)
        args = dict(
            q=qh, k_new=kh, v_new=vh, k_cache=k_cache, v_cache=v_cache, req_to_token=self.req_to_token,
            req_pool_indices=forward_batch.req_pool_indices[:bs], ctx_lens=forward_batch.seq_lens[:bs],
            num_modes=self.num_modes, block_size=self.block_size, scaling=self.scaling, page_size=self.page_size,
        )
        if self.impl == "reference":
            out = paged_mode_block_attention_reference(**args).to(q.dtype)
        else:
            out = paged_mode_block_attention(**args, num_ctx_splits=self.num_ctx_splits)
        return out.view(T, self.num_heads * self.head_dim)
