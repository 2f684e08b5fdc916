"""Tree verification of a gated delta rule (Gated-DeltaNet) layer on MI355X — drop-in for the reference's
``tree_gdn`` (inference/hf/tree_gdn_kernel.py:153-171), plus the ragged batch ``tree_gdn_varlen``.

For every node i of a draft tree in topological order (parents first):

  u_i + sum_{j strict ancestor of i} beta_i exp(G_i - G_j) (k_i . k_j) u_j = beta_i (v_i - exp(G_i) S0^T k_i)
  o_i = exp(G_i) S0^T q_i + sum_{j ancestor or i} exp(G_i - G_j) (q_i . k_j) u_j

Trees of up to 128 nodes run in one hand-written HIP kernel (csrc/tree_gdn.hip): one workgroup per
(request, value head) works along the tree's root paths for the triangular part (path-local back
substitution instead of a dense triangular inverse) and runs the dense products on MFMA: S0^T k and S0^T q
with S0 rounded to bf16 (as the reference's s_blk), and u = T R, o = E + W R with T, W and R in fp16 scaled
by powers of two per row / column (about 2^-11 relative per operand, fp32 accumulation); small grids use a
variant that splits a head's value columns over 2 or 4 workgroups and keeps R, T and W as bf16 hi + lo
pairs. Trees of up to 512 nodes (the HF path's default budget of 256 drafts 257 nodes) take the
large-tree path (csrc/tree_gdn_large.hip): a Gram kernel writes each node's k.k / q.k entries against its
root path, then one workgroup per (request, value head, 16 or 32 value columns) solves along the root paths
with fp32 gathers. Root paths come from the parent pointers, or from a TreeContext built once per round and
shared by all layers. Depth is limited to 16 nodes on a root path; a request over a limit gets NaN outputs
(and MFD_DEVERR_* bits in ``err_flag`` where one is passed).
"""

from __future__ import annotations

import torch

import mfd_hip

MAX_NODES = 512        # MFD_GDN_MAX_NODES
FUSED_MAX_NODES = 128  # one-kernel path up to here, large-tree path above
MAX_DEPTH = 16         # MFD_GDN_MAX_DEPTH


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


def _workspace(R, N, HK, max_nodes, has_ctx, device):
    nbytes = mfd_hip.lib().mfd_tree_gdn_workspace_bytes(R, N, HK, max_nodes, 1 if has_ctx else 0)
    if nbytes < 0:
        raise ValueError(f"bad tree-GDN sizes R={R} N={N} HK={HK} max_nodes={max_nodes}")
    return mfd_hip.workspace(nbytes, device)


def _check_out(out, N, H, D):
    u, o = out
    for t in (u, o):
        if t.shape != (N, H, D) or t.dtype != torch.float32 or not t.is_contiguous() or not t.is_cuda:
            raise ValueError(f"out tensors must be contiguous float32 [{N}, {H}, {D}] on the GPU")
    return u, o


def tree_gdn(q, k, v, g_cum, beta, s0, anc8, block_t: int = 64, block_v: int = 32):
    """q, k: [n, H_k, K] bf16 (l2-normalized, q scaled; value head h uses key head h // (H // H_k));
    v: [n, H, V] bf16; g_cum, beta: [n, H] fp32 (g_cum = log decay summed along the root path);
    s0: [H, K, V]; anc8: [n, n] int8, ancestors or self. Returns u and o, [n, H, V] fp32.
    ``block_t`` / ``block_v`` are accepted for signature compatibility and ignored. Trees of up to
    MAX_NODES nodes and MAX_DEPTH nodes per root path; a tree beyond them gets NaN outputs."""
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
    ws = _workspace(1, N, HK, N, False, k.device)
    mfd_hip.call("mfd_tree_gdn", q.data_ptr(), k.data_ptr(), v.data_ptr(), g_cum.data_ptr(), beta.data_ptr(),
                 s0.data_ptr(), None, anc8.data_ptr(), None, 1, N, HK, H, D, N, u.data_ptr(), o.data_ptr(), None,
                 mfd_hip.ptr(ws), 0 if ws is None else ws.numel(), mfd_hip.stream_of(k))
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
    nbytes = int(mfd_hip.lib().mfd_tree_ctx_bytes(R, max_nodes))
    if out is not None:
        if (out.R, out.N, out.max_nodes) != (R, N, max_nodes) or out.buf.numel() != nbytes:
            raise ValueError("out context was built for other sizes")
        buf = out.buf
    else:
        buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    cu = cu_nodes.contiguous() if cu_nodes is not None else None
    mfd_hip.call("mfd_tree_context", mfd_hip.ptr(parents), mfd_hip.ptr(anc8), mfd_hip.ptr(cu), R, N, max_nodes,
                 buf.data_ptr(), buf.numel(), mfd_hip.ptr(err_flag), mfd_hip.stream_of(buf))
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
        u, o = _check_out(out, N, H, D)
    ws = _workspace(R, N, HK, max_nodes, ctx is not None, k.device)
    ws_args = (mfd_hip.ptr(ws), 0 if ws is None else ws.numel())
    if ctx is not None:
        mfd_hip.call("mfd_tree_gdn_ctx", q.data_ptr(), k.data_ptr(), v.data_ptr(), g_cum.data_ptr(),
                     beta.data_ptr(), s0.data_ptr(), ctx.buf.data_ptr(), ctx.buf.numel(),
                     cu_nodes.contiguous().data_ptr(), R, N, HK, H, D, max_nodes, u.data_ptr(), o.data_ptr(),
                     mfd_hip.ptr(err_flag), *ws_args, mfd_hip.stream_of(k))
    else:
        mfd_hip.call("mfd_tree_gdn", q.data_ptr(), k.data_ptr(), v.data_ptr(), g_cum.data_ptr(), beta.data_ptr(),
                     s0.data_ptr(), parents.contiguous().data_ptr(), None, cu_nodes.contiguous().data_ptr(), R, N,
                     HK, H, D, max_nodes, u.data_ptr(), o.data_ptr(), mfd_hip.ptr(err_flag), *ws_args,
                     mfd_hip.stream_of(k))
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



def conv_index(parents: torch.Tensor, kernel: int, cu_nodes: torch.Tensor | None = None, err_flag=None) -> torch.Tensor:
    """Conv windows of the tree nodes on the device (the reference builds them with host loops in
    TreeContext, inference/hf/qwen35_tree.py:39-52): row i = node i's ``kernel`` inputs, oldest first, as
    request-local indices into [cached conv state ; the request's nodes]. ``parents`` [N] int32 request-local
    (-1 = root), ``cu_nodes`` [R + 1] int32 for a ragged batch. Returns [N, kernel] int32."""
    mfd_hip.require_cuda(parents, cu_nodes)
    if parents.dtype != torch.int32 or (cu_nodes is not None and cu_nodes.dtype != torch.int32):
        raise TypeError("parents and cu_nodes must be int32")
    N = parents.numel()
    R = 1 if cu_nodes is None else cu_nodes.numel() - 1
    out = torch.empty(N, kernel, dtype=torch.int32, device=parents.device)
    mfd_hip.call("mfd_conv_index", parents.contiguous().data_ptr(), mfd_hip.ptr(cu_nodes), R, N, kernel,
                 out.data_ptr(), mfd_hip.ptr(err_flag), mfd_hip.stream_of(parents))
    return out


def tree_prep(x, conv_state, conv_index, conv_w, num_k_heads: int, num_v_heads: int, head_dim: int,
              block_n: int = 16, cu_nodes=None, err_flag=None):
    """x: [n, conv_dim] pre-conv projections of the nodes; conv_state: [conv_dim, KC] cached inputs
    (oldest first), or [R, conv_dim, KC] with ``cu_nodes``; conv_index: [n, KC] int32, each node's window
    (oldest first) as indices into [conv_state ; nodes]; conv_w: [conv_dim, KC]. Returns q (l2-normalized,
    scaled by head_dim^-0.5), k (l2-normalized) [n, H_k, D] and v [n, H, D], bf16
    (inference/hf/tree_gdn_kernel.py:135-150). ``block_n`` is accepted for signature compatibility."""
    del block_n
    mfd_hip.require_cuda(x, conv_state, conv_index, conv_w, cu_nodes)
    n, cd = x.shape
    KC = conv_w.shape[-1]
    HK, H, D = num_k_heads, num_v_heads, head_dim
    if cd != (2 * HK + H) * D or conv_w.shape != (cd, KC) or conv_state.shape[-2:] != (cd, KC):
        raise ValueError(f"conv_dim {cd} must be (2 HK + H) D = {(2 * HK + H) * D}; conv_w / conv_state [conv_dim, KC]")
    if conv_index.shape != (n, KC) or conv_index.dtype != torch.int32:
        raise ValueError("conv_index must be [n, KC] int32")
    R = 1 if cu_nodes is None else cu_nodes.numel() - 1
    if conv_state.dim() == 3 and conv_state.shape[0] != R:
        raise ValueError("conv_state [R, conv_dim, KC] must match cu_nodes")
    x = x.to(torch.bfloat16)
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    conv_state = conv_state.to(torch.bfloat16).contiguous()
    conv_w = conv_w.to(torch.bfloat16).contiguous()
    q = torch.empty(n, HK, D, dtype=torch.bfloat16, device=x.device)
    k = torch.empty_like(q)
    v = torch.empty(n, H, D, dtype=torch.bfloat16, device=x.device)
    mfd_hip.call("mfd_tree_prep", x.data_ptr(), x.stride(0), conv_state.data_ptr(), cd * KC,
                 conv_index.contiguous().data_ptr(), conv_w.data_ptr(), mfd_hip.ptr(cu_nodes), R, n, HK, H, D, KC,
                 float(D) ** -0.5, q.data_ptr(), k.data_ptr(), v.data_ptr(), mfd_hip.ptr(err_flag),
                 mfd_hip.stream_of(x))
    return q, k, v


def _stack(t):
    return torch.stack(list(t)) if isinstance(t, (list, tuple)) else t


def gdn_commit(recurrent, u, k, g_cum, path, conv=None, x=None, conv_index=None, err_flag=None):
    """Advance every GDN layer of one request to the deepest accepted node (the state and conv updates of
    commit(), inference/hf/qwen35_tree.py:122-148), all layers in one launch, in place.

    recurrent: [L, H, D, D] (or [L, 1, H, D, D]) fp32 states in the [d_k, d_v] layout; u [L, n, H, D] fp32,
    k [L, n, HK, D] bf16, g_cum [L, n, H] fp32 (or lists of L per-layer tensors): the verify pass's values;
    path: the accepted node ids, root first (list or int32 device tensor). conv: [L, CD, KC]
    (or [L, 1, CD, KC]) bf16 conv states with x [L, n, CD] bf16 pre-conv inputs and conv_index [n, KC] int32,
    or None to leave the conv states alone."""
    u, k, g_cum = _stack(u), _stack(k), _stack(g_cum)
    dev = u.device
    if not torch.is_tensor(path):
        path = torch.tensor(list(path), dtype=torch.int32)
    path = path.to(device=dev, dtype=torch.int32).contiguous()
    mfd_hip.require_cuda(recurrent, u, k, g_cum, conv, x, conv_index)
    L, n, H, D = u.shape
    HK = k.shape[2]
    if recurrent.dtype != torch.float32 or not recurrent.is_contiguous() or recurrent.numel() != L * H * D * D:
        raise ValueError("recurrent must be contiguous float32 [L, H, D, D] (or [L, 1, H, D, D])")
    state = recurrent.reshape(L, H, D, D) if recurrent.dim() == 5 else recurrent
    if state.shape != (L, H, D, D):
        raise ValueError("recurrent must be contiguous float32 [L, H, D, D] (or [L, 1, H, D, D])")
    if k.shape != (L, n, HK, D) or g_cum.shape != (L, n, H):
        raise ValueError("k must be [L, n, HK, D] and g_cum [L, n, H]")
    u = u.float().contiguous()
    k = k.to(torch.bfloat16).contiguous()
    g_cum = g_cum.float().contiguous()
    p = path.numel()
    cptr, xptr, ciptr, CD, KC, c_lst, x_lst, x_rst = None, None, None, 0, 0, 0, 0, 0
    if conv is not None:
        if conv.dtype != torch.bfloat16 or not conv.is_contiguous():
            raise ValueError("conv must be contiguous bfloat16 [L, CD, KC] (or [L, 1, CD, KC])")
        cv = conv.reshape(L, conv.shape[-2], conv.shape[-1]) if conv.dim() == 4 else conv
        if cv.shape[0] != L:
            raise ValueError("conv must be contiguous bfloat16 [L, CD, KC] (or [L, 1, CD, KC])")
        CD, KC = cv.shape[1], cv.shape[2]
        x = _stack(x).to(torch.bfloat16)
        if x.shape != (L, n, CD) or x.stride(2) != 1:
            x = x.contiguous()
        if conv_index is None or conv_index.shape != (n, KC):
            raise ValueError("conv_index [n, KC] is required with conv")
        cptr, xptr, ciptr = cv.data_ptr(), x.data_ptr(), conv_index.to(torch.int32).contiguous().data_ptr()
        c_lst, x_lst, x_rst = CD * KC, x.stride(0), x.stride(1)
    mfd_hip.call("mfd_gdn_commit", state.data_ptr(), H * D * D, u.data_ptr(), n * H * D, k.data_ptr(), n * HK * D,
                 g_cum.data_ptr(), n * H, path.data_ptr(), p, L, n, HK, H, D, cptr, c_lst, xptr, x_lst, x_rst,
                 ciptr, CD, KC, mfd_hip.ptr(err_flag), mfd_hip.stream_of(u))
    return recurrent, conv
