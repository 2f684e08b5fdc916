"""Tree verification of a gated delta rule (Gated-DeltaNet) layer on MI355X — drop-in for the reference's
``tree_gdn`` (inference/hf/tree_gdn_kernel.py:153-171), plus the ragged batch ``tree_gdn_varlen``.

For every node i of a draft tree in topological order (parents first):

  u_i + sum_{j strict ancestor of i} beta_i exp(G_i - G_j) (k_i . k_j) u_j = beta_i (v_i - exp(G_i) S0^T k_i)
  o_i = exp(G_i) S0^T q_i + sum_{j ancestor or i} exp(G_i - G_j) (q_i . k_j) u_j

computed by one hand-written HIP kernel (csrc/tree_gdn.hip): one workgroup per (request, value head)
works along the tree's root paths for the triangular part and runs the dense S0 products on MFMA with the
fp32 state split into bf16 hi + lo (about 2^-17 relative), so u and o stay fp32-accurate. The root paths
come from the parent pointers, or from a TreeContext built once per round and shared by all layers.
"""

from __future__ import annotations

import torch

import mfd_hip

MAX_NODES = 128  # MFD_GDN_MAX_NODES
MAX_DEPTH = 16   # MFD_GDN_MAX_DEPTH


def _check_inputs(q, k, v, g_cum, beta):
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("q, k, v must be bfloat16")
    if q.shape != k.shape or q.dim() != 3 or v.dim() != 3 or v.shape[0] != k.shape[0]:
        raise ValueError(f"bad shapes q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    N, HK, D = k.shape
    H = v.shape[1]
    if v.shape[2] != D or H % HK != 0:
        raise ValueError(f"value heads {H} must be a multiple of key heads {HK}, head dims equal")
    if g_cum.shape != (N, H) or beta.shape != (N, H):
        raise ValueError("g_cum and beta must be [n, H]")
    return N, HK, H, D


def tree_gdn(q, k, v, g_cum, beta, s0, anc8, block_t: int = 64, block_v: int = 32):
    """q, k: [n, H_k, K] bf16 (l2-normalized, q scaled; value head h uses key head h // (H // H_k));
    v: [n, H, V] bf16; g_cum, beta: [n, H] fp32 (g_cum = log decay summed along the root path);
    s0: [H, K, V]; anc8: [n, n] int8, ancestors or self. Returns u and o, [n, H, V] fp32.
    ``block_t`` / ``block_v`` are accepted for signature compatibility and ignored."""
    del block_t, block_v
    mfd_hip.require_cuda(q, k, v, g_cum, beta, s0, anc8)
    N, HK, H, D = _check_inputs(q, k, v, g_cum, beta)
    if anc8.shape != (N, N):
        raise ValueError("anc8 must be [n, n]")
    if N > MAX_NODES:
        raise ValueError(f"tree of {N} nodes exceeds {MAX_NODES}")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    g_cum, beta = g_cum.contiguous().float(), beta.contiguous().float()
    s0 = s0.contiguous().float()
    anc8 = anc8.contiguous().to(torch.int8)
    u = torch.empty(N, H, D, dtype=torch.float32, device=k.device)
    o = torch.empty(N, H, D, dtype=torch.float32, device=k.device)
    mfd_hip.call("mfd_tree_gdn", q.data_ptr(), k.data_ptr(), v.data_ptr(), g_cum.data_ptr(), beta.data_ptr(),
                 s0.data_ptr(), None, anc8.data_ptr(), None, 1, N, HK, H, D, N, u.data_ptr(), o.data_ptr(), None,
                 mfd_hip.stream_of(k))
    return u, o


class TreeContext:
    """Root paths, depths and ancestor masks of a batch of trees, on the device, built once per verify round
    (``tree_context``) and passed to the tree-GDN call of every layer — the counterpart of the reference's
    TreeContext (inference/hf/qwen35_tree.py:33-53), whose ancestor matrix every layer reuses.
    ``buf``: the uint8 device buffer; ``cu_nodes``: the node offsets it was built for; ``max_nodes``: the
    bound it was built with (the GDN call must use the same)."""

    def __init__(self, buf: torch.Tensor, cu_nodes: torch.Tensor | None, R: int, N: int, max_nodes: int):
        self.buf, self.cu_nodes, self.R, self.N, self.max_nodes = buf, cu_nodes, R, N, max_nodes


def tree_context(parents=None, cu_nodes=None, max_nodes: int | None = None, anc8=None, err_flag=None,
                 out: TreeContext | None = None) -> TreeContext:
    """Build the tree context of a ragged batch (``parents`` [N] int32 request-local, ``cu_nodes`` [R + 1]
    int32) or of one tree given as its [n, n] int8 ancestor-or-self matrix ``anc8``. ``max_nodes`` as for
    ``tree_gdn_varlen``. Trees that are too large, too deep or not topologically ordered set MFD_DEVERR_* bits
    in ``err_flag`` (optional int32 device tensor) and are rejected by every GDN call that uses the context.
    ``out``: an existing context of the same R, N and max_nodes to rebuild in place (no allocation, so the
    call can be captured in a graph)."""
    if parents is None and anc8 is None:
        raise ValueError("tree_context needs parents (+ cu_nodes) or anc8")
    if parents is not None:
        mfd_hip.require_cuda(parents, cu_nodes)
        if parents.dtype != torch.int32 or (cu_nodes is not None and cu_nodes.dtype != torch.int32):
            raise TypeError("parents and cu_nodes must be int32")
        N = parents.numel()
        R = cu_nodes.numel() - 1 if cu_nodes is not None else 1
        dev = parents.device
        if max_nodes is None:
            max_nodes = int((cu_nodes[1:] - cu_nodes[:-1]).max()) if cu_nodes is not None else N
        parents = parents.contiguous()
    else:
        mfd_hip.require_cuda(anc8)
        N = anc8.shape[0]
        if anc8.shape != (N, N):
            raise ValueError("anc8 must be [n, n]")
        R, dev, cu_nodes = 1, anc8.device, None
        max_nodes = N if max_nodes is None else max_nodes
        anc8 = anc8.contiguous().to(torch.int8)
    if not 1 <= max_nodes <= MAX_NODES:
        raise ValueError(f"max_nodes {max_nodes} not in [1, {MAX_NODES}]")
    nbytes = mfd_hip.lib().mfd_tree_ctx_bytes(R, max_nodes)
    if out is not None:
        if (out.R, out.N, out.max_nodes) != (R, N, max_nodes) or out.buf.numel() != nbytes:
            raise ValueError("out context was built for other sizes")
        buf = out.buf
    else:
        buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    cu = cu_nodes.contiguous() if cu_nodes is not None else None
    mfd_hip.call("mfd_tree_context", mfd_hip.ptr(parents), mfd_hip.ptr(anc8), mfd_hip.ptr(cu), R, N, max_nodes,
                 buf.data_ptr(), mfd_hip.ptr(err_flag), mfd_hip.stream_of(buf))
    if out is not None:
        out.cu_nodes = cu
        return out
    return TreeContext(buf, cu, R, N, max_nodes)


def tree_gdn_varlen(q, k, v, g_cum, beta, s0, parents, cu_nodes, max_nodes: int | None = None, out=None,
                    err_flag=None, ctx: TreeContext | None = None):
    """Ragged batch of trees packed along the node axis, one launch.

    q, k: [N, H_k, D] bf16; v: [N, H, D] bf16; g_cum, beta: [N, H] fp32; s0: [R, H, D, D] fp32;
    parents: [N] int32 request-local parent (-1 = root); cu_nodes: [R + 1] int32 node offsets (device).
    ``max_nodes``: upper bound of the per-request node count (computed from cu_nodes with a host sync
    when omitted; pass it to stay graph-capturable). ``out``: optional (u, o) to write into.
    ``err_flag``: optional int32 device tensor receiving MFD_DEVERR_* bits for rejected requests.
    ``ctx``: a TreeContext of these trees (then ``parents`` may be None and ``max_nodes`` is the context's):
    the kernel loads the root paths instead of walking the parent pointers."""
    mfd_hip.require_cuda(q, k, v, g_cum, beta, s0, parents, cu_nodes)
    N, HK, H, D = _check_inputs(q, k, v, g_cum, beta)
    R = cu_nodes.numel() - 1
    if R < 1 or s0.shape != (R, H, D, D) or (parents is not None and parents.shape != (N,)):
        raise ValueError("s0 must be [R, H, D, D] and parents [N]")
    if cu_nodes.dtype != torch.int32 or (parents is not None and parents.dtype != torch.int32):
        raise TypeError("parents and cu_nodes must be int32")
    if ctx is not None:
        if ctx.R != R or ctx.N != N:
            raise ValueError(f"tree context of R={ctx.R}, N={ctx.N} used for R={R}, N={N}")
        if max_nodes is not None and max_nodes != ctx.max_nodes:
            raise ValueError(f"max_nodes {max_nodes} differs from the context's {ctx.max_nodes}")
        max_nodes = ctx.max_nodes
    elif parents is None:
        raise ValueError("parents or ctx required")
    if max_nodes is None:
        max_nodes = int((cu_nodes[1:] - cu_nodes[:-1]).max()) if R else 0
    if max_nodes > MAX_NODES:
        raise ValueError(f"tree of {max_nodes} nodes exceeds {MAX_NODES}")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    g_cum, beta, s0 = g_cum.contiguous().float(), beta.contiguous().float(), s0.contiguous().float()
    if out is None:
        u = torch.empty(N, H, D, dtype=torch.float32, device=k.device)
        o = torch.empty(N, H, D, dtype=torch.float32, device=k.device)
    else:
        u, o = out
    if ctx is not None:
        mfd_hip.call("mfd_tree_gdn_ctx", q.data_ptr(), k.data_ptr(), v.data_ptr(), g_cum.data_ptr(),
                     beta.data_ptr(), s0.data_ptr(), ctx.buf.data_ptr(), cu_nodes.contiguous().data_ptr(), R, N, HK,
                     H, D, max_nodes, u.data_ptr(), o.data_ptr(), mfd_hip.ptr(err_flag), mfd_hip.stream_of(k))
    else:
        mfd_hip.call("mfd_tree_gdn", q.data_ptr(), k.data_ptr(), v.data_ptr(), g_cum.data_ptr(), beta.data_ptr(),
                     s0.data_ptr(), parents.contiguous().data_ptr(), None, cu_nodes.contiguous().data_ptr(), R, N,
                     HK, H, D, max_nodes, u.data_ptr(), o.data_ptr(), mfd_hip.ptr(err_flag), mfd_hip.stream_of(k))
    return u, o


def tree_gates(a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor, parents=None,
               cu_nodes=None, anc8=None, err_flag=None):
    """The gates tree_gdn consumes (inference/hf/qwen35_tree.py:77-79): a = in_proj_a(h), b = in_proj_b(h),
    [N, H] bf16 or fp32 (rows may be strided); A_log, dt_bias [H]. Returns (g_cum, beta) [N, H] fp32 with
    beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias), g_cum_i = sum of g over the ancestors-or-self
    of node i. The tree is given by request-local ``parents`` [N] int32 with ``cu_nodes`` [R + 1] int32
    (ragged batch), or by the ancestor-or-self matrix ``anc8`` [n, n] of a single tree."""
    mfd_hip.require_cuda(a, b, A_log, dt_bias, parents, cu_nodes, anc8)
    if a.shape != b.shape or a.dim() != 2 or a.dtype != b.dtype or a.stride() != b.stride():
        raise ValueError("a and b must be [N, H] with the same dtype and strides")
    if a.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("a, b must be bfloat16 or float32")
    if a.stride(1) != 1:
        a, b = a.contiguous(), b.contiguous()
    N, H = a.shape
    A_log = A_log.reshape(H).float().contiguous()
    dt_bias = dt_bias.reshape(H).float().contiguous()
    if parents is None and anc8 is None:
        raise ValueError("parents or anc8 required")
    if parents is not None:
        parents = parents.to(torch.int32).contiguous()
    if anc8 is not None and parents is None:
        anc8 = anc8.to(torch.int8).contiguous()
    R = 1 if cu_nodes is None else cu_nodes.numel() - 1
    cu = None if cu_nodes is None else cu_nodes.to(torch.int32).contiguous()
    g_cum = torch.empty(N, H, dtype=torch.float32, device=a.device)
    beta = torch.empty(N, H, dtype=torch.float32, device=a.device)
    mfd_hip.call("mfd_tree_gates", a.data_ptr(), b.data_ptr(), 1 if a.dtype == torch.bfloat16 else 0, a.stride(0),
                 A_log.data_ptr(), dt_bias.data_ptr(), mfd_hip.ptr(parents), mfd_hip.ptr(anc8), mfd_hip.ptr(cu), R, N,
                 H, g_cum.data_ptr(), beta.data_ptr(), mfd_hip.ptr(err_flag), mfd_hip.stream_of(a))
    return g_cum, beta

