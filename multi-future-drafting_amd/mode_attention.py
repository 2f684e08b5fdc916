"""The attention of a multi-mode (MFD) draft step on MI355X, without a dense mask — drop-in for the reference's
inference/hf/mode_attention.py (ModeBlocks, mode_block_attention, reference).

Every query of mode m attends to the whole context plus the block_size keys of its own mode block. One
hand-written HIP kernel (csrc/mode_attn.hip) splits the context across workgroups, shares each 64-key
K / V tile among the queries of a KV head's GQA group through LDS, runs QK^T and PV on MFMA with an
fp32 online softmax, and handles the own-block keys as masked extra tiles; context splits are merged
by their log-sum-exp in a second small kernel.
"""

from __future__ import annotations

import math

import torch

import mfd_hip

LOG2E = 1.4426950408889634


class ModeBlocks:
    """Passed as the attention mask of forward_modes in place of the dense mask: the layers then call
    mode_block_attention for (num_modes, block_size) (inference/hf/mode_attention.py:24-30)."""

    def __init__(self, num_modes: int, block_size: int, exact: bool = False):
        self.mode_blocks = (num_modes, block_size)
        self.exact = exact  # checks only: float32 reference() instead of the kernel


def _auto_splits(programs: int, ctx: int, device) -> int:
    """Context splits for num_ctx_splits < 0: the most for which the whole grid (per program the context splits
    plus the block partial) fits one round of workgroup slots, two per CU, keeping >= 256 keys per split; one
    pass when no second split fits. (A grid one slot round larger runs a second round: config 2 measures 29.4-29.8
    us with 13-15 splits, 31 us with 12, 37 us with 16.)"""
    if ctx <= 256:
        return 1
    slots = 2 * mfd_hip.cu_count(device)
    return max(1, min(slots // programs - 1, -(-ctx // 256), 64))


def launch(*, q, q_st, q_sh, k_new, v_new, kn_st, kn_sh, vn_st, vn_sh, k_cache, v_cache, kc_ss, kc_sh, vc_ss, vc_sh,
           table, table_stride, page_size, req_idx, ctx_lens, ctx_const, bs, num_modes, block_size, H, Hkv, D, scaling,
           causal, splits, out, o_st, o_sh, stream):
    """Raw launch through the C ABI (pointers are tensors or None); allocates the split workspace."""
    ws_bytes = mfd_hip.lib().mfd_mode_attn_workspace_bytes(bs, num_modes, block_size, H, splits)
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=q.device) if ws_bytes > 0 else None
    mfd_hip.call("mfd_mode_attn", q.data_ptr(), q_st, q_sh, k_new.data_ptr(), v_new.data_ptr(), kn_st, kn_sh, vn_st,
                 vn_sh, mfd_hip.ptr(k_cache), mfd_hip.ptr(v_cache), kc_ss, kc_sh, vc_ss, vc_sh, mfd_hip.ptr(table),
                 table_stride, page_size, mfd_hip.ptr(req_idx), mfd_hip.ptr(ctx_lens), ctx_const, bs, num_modes,
                 block_size, H, Hkv, D, float(scaling), 1 if causal else 0, splits, out.data_ptr(), o_st, o_sh,
                 mfd_hip.ptr(ws), ws_bytes, stream)
    return out


def mode_block_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_modes: int, block_size: int,
                         scaling: float, modes_per_program: int = 2, target_programs: int = 384,
                         block_n: int = 64, causal_in_block: bool = False, num_ctx_splits: int = -1) -> torch.Tensor:
    """Attention of the K mode blocks. q: [1, heads, K * bs, D]; k, v: [1, KV heads, context + K * bs, D] (the
    draft cache after the update, the blocks last). Returns [1, K * bs, heads, D] in q.dtype.
    ``modes_per_program`` / ``target_programs`` / ``block_n`` are accepted for signature compatibility (grid
    tuning of the reference for its GPU; here the automatic context split, num_ctx_splits < 0, fills the MI355X's
    workgroup slots); num_ctx_splits 0 or 1 = one pass."""
    del modes_per_program, target_programs, block_n
    _, num_heads, num_queries, head_dim = q.shape
    num_kv_heads, total = k.shape[1], k.shape[2]
    assert num_queries == num_modes * block_size and num_heads % num_kv_heads == 0
    assert q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride(-1) == 1
    assert q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16
    mfd_hip.require_cuda(q, k, v)
    ctx = total - num_queries
    G = num_heads // num_kv_heads
    programs = num_kv_heads * -(-(G * num_queries // 32) // 4)
    if num_ctx_splits < 0:
        splits = _auto_splits(programs, ctx, q.device)
    else:
        splits = max(1, num_ctx_splits)
    out = torch.empty((1, num_queries, num_heads, head_dim), device=q.device, dtype=q.dtype)
    k_new = k[:, :, ctx:]
    v_new = v[:, :, ctx:]
    return launch(q=q, q_st=q.stride(2), q_sh=q.stride(1), k_new=k_new, v_new=v_new, kn_st=k.stride(2),
                  kn_sh=k.stride(1), vn_st=v.stride(2), vn_sh=v.stride(1), k_cache=k, v_cache=v, kc_ss=k.stride(2),
                  kc_sh=k.stride(1), vc_ss=v.stride(2), vc_sh=v.stride(1), table=None, table_stride=0, page_size=1,
                  req_idx=None, ctx_lens=None, ctx_const=ctx, bs=1, num_modes=num_modes, block_size=block_size,
                  H=num_heads, Hkv=num_kv_heads, D=head_dim, scaling=scaling, causal=causal_in_block, splits=splits,
                  out=out, o_st=out.stride(1), o_sh=out.stride(2), stream=mfd_hip.stream_of(q))


def modes_fp32(q, k_ctx, v_ctx, k_blk, v_blk, num_modes: int, block_size: int, scaling: float,
               causal_in_block: bool = False) -> torch.Tensor:
    """Float32 mode attention of one request, computed per mode block (no dense mask): the queries of mode m
    see the context keys and the block_size keys of block m. q [H, K * bs, D]; k_ctx, v_ctx [Hkv, ctx, D];
    k_blk, v_blk [Hkv, K * bs, D]; query head h reads KV head h // (H / Hkv) (heads grouped, not repeated).
    Returns [H, K * bs, D] float32 on the tensors' device."""
    H, KL, D = q.shape
    Hkv, ctx = k_ctx.shape[0], k_ctx.shape[1]
    G, K, L = H // Hkv, num_modes, block_size
    qg = q.float().reshape(Hkv, G, K, L, D)
    kb = k_blk.float().reshape(Hkv, 1, K, L, D)
    vb = v_blk.float().reshape(Hkv, 1, K, L, D)
    kc = k_ctx.float().reshape(Hkv, 1, 1, ctx, D)
    vc = v_ctx.float().reshape(Hkv, 1, 1, ctx, D)
    s_ctx = torch.matmul(qg, kc.transpose(-1, -2).contiguous())   # [Hkv, G, K, L, ctx]
    s_blk = torch.matmul(qg, kb.transpose(-1, -2).contiguous())   # [Hkv, G, K, L, L]: own block only
    if causal_in_block:
        later = torch.ones(L, L, dtype=torch.bool, device=q.device).triu(1)
        s_blk = s_blk.masked_fill(later, float("-inf"))
    p = torch.softmax(torch.cat([s_ctx, s_blk], dim=-1) * scaling, dim=-1)
    out = torch.matmul(p[..., :ctx], vc) + torch.matmul(p[..., ctx:], vb)
    return out.reshape(H, KL, D)


def reference(q, k, v, num_modes, block_size, scaling):
    """The exact=True checking path of ModeBlocks (inference/hf/mode_attention.py:153-164): the same attention
    in float32 torch, wherever the tensors are. q [1, H, K * bs, D]; k, v [1, Hkv, ctx + K * bs, D] (blocks
    last). Returns [1, K * bs, H, D] float32."""
    ctx = k.shape[2] - num_modes * block_size
    o = modes_fp32(q[0], k[0, :, :ctx], v[0, :, :ctx], k[0, :, ctx:], v[0, :, ctx:], num_modes, block_size, scaling)
    return o.transpose(0, 1).unsqueeze(0)


def check_equal(seed: int = 0) -> None:
    """Self-test of inference/hf/mode_attention.py:167-181: the kernel against the float32 ``reference`` for
    context lengths 1 .. 5000 (8 modes x 16 tokens, 32 heads over 8 KV heads, D 128), max |error| < 2e-2.
    ``modes_per_program`` is the reference's tuning knob; every value gives the same kernel here."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    K, bs, H, Hkv, D = 8, 16, 32, 8, 128
    for ctx in (1, 37, 500, 2048, 5000):
        for mpg in (1, 2, 4):
            q = torch.randn(1, H, K * bs, D, device="cuda", generator=gen).to(torch.bfloat16)
            k = (torch.randn(1, Hkv, ctx + K * bs, D, device="cuda", generator=gen) * 2).to(torch.bfloat16)
            v = torch.randn(1, Hkv, ctx + K * bs, D, device="cuda", generator=gen).to(torch.bfloat16)
            got = mode_block_attention(q, k, v, K, bs, D ** -0.5, modes_per_program=mpg)
            err = (got.float() - reference(q, k, v, K, bs, D ** -0.5)).abs().max().item()
            if not err < 2e-2:
                raise AssertionError(f"ctx {ctx} modes/program {mpg}: max |err| {err:.2e}")
            print(f"ctx {ctx} modes/program {mpg}: max |err| {err:.2e}")


if __name__ == "__main__":
    check_equal()
