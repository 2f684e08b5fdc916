"""HF tree-round plumbing on MI355X — the hot-path subset of the reference's inference/hf/ddtree.py:
``compile_ddtree_tree`` (verify ids, positions and the additive tree mask in the caller's buffers,
:317-357), ``follow_verified_tree`` (the accept walk, :367-382) and ``compact_dynamic_cache`` (the accepted
nodes' KV moved to the front of the appended window, :385-436).

The verify inputs (one launch of ``tree_mask_kernel``) and the KV moves run as HIP kernels
(csrc/verify_plumbing.hip); the walk over a built Tree stays on the host, as the HF decode loop needs its
result there (the device walk for a batch is ``ddtree_sglang_ops.ddtree_follow``).

The reference's ``ddtree`` module also holds the decode loop (``ddtree_generate``) and the switches
``benchmark.py`` imports, so this module does not take its name: ``install()`` rebinds the three functions on
the reference's module instead, and ``ddtree_generate`` (which calls them by module-level name, :576-618) and
``dflash.py``'s lazy ``from ddtree import compact_dynamic_cache`` (:54) then reach this module's versions.
"""

from __future__ import annotations

import torch

import mfd_hip

_BITS_VIEW = {2: torch.int16, 4: torch.int32}


def _min_bits(dtype: torch.dtype, buffer_dtype: torch.dtype) -> int:
    """Bit pattern of finfo(dtype).min stored in a buffer of buffer_dtype (the value the mask blocks keys with)."""
    v = torch.tensor(torch.finfo(dtype).min, dtype=torch.float64).to(buffer_dtype)
    size = v.element_size()
    return int(v.reshape(1).view(_BITS_VIEW[size]).item()) & ((1 << (8 * size)) - 1)


def _on(t, device, dtype) -> torch.Tensor:
    return torch.as_tensor(t).to(device=device, dtype=dtype).contiguous()


def compile_ddtree_tree(root_token_id, start: int, node_token_ids, node_depths, visibility_cpu, past_length: int,
                        dtype, device, verify_input_ids_buffer, verify_position_ids_buffer, attention_mask_buffer,
                        tree_visibility_buffer, previous_tree_start: int, previous_tree_length: int):
    """Contract of inference/hf/ddtree.py:317-357. Writes, in one kernel launch into the persistent buffers:
    the verify ids [1, n + 1] (the root, then the node tokens), the positions (start + depth), the tree's
    visibility, and row i < n + 1 of the [1, 1, rows, cols] additive mask at columns past_length + j: 0 where
    node j is visible from node i, finfo(dtype).min elsewhere — after clearing the previous round's tree block
    (rows and columns [previous_tree_start, + previous_tree_length)), which joins the visible prefix. Inputs may
    be host tensors (the HF builder's) or device tensors (the device builder's). Returns (ids, positions, mask,
    past_length, n + 1), views of the buffers."""
    del device
    n1 = 1 + int(node_token_ids.numel())
    dev = attention_mask_buffer.device
    mask2d = attention_mask_buffer[0, 0]
    ids_row = verify_input_ids_buffer[0]
    pos_row = verify_position_ids_buffer[0]
    for t in (mask2d, ids_row, pos_row, tree_visibility_buffer):
        if t.stride(-1) != 1:
            raise ValueError("the verify buffers need a contiguous last dimension")
    if ids_row.dtype != torch.int64 or pos_row.dtype != torch.int64 or tree_visibility_buffer.dtype != torch.bool:
        raise TypeError("verify id / position buffers must be int64 and the visibility buffer bool")
    if ids_row.numel() < n1 or pos_row.numel() < n1 or min(tree_visibility_buffer.shape) < n1:
        raise ValueError(f"buffers too small for a tree of {n1} nodes")
    esize = mask2d.element_size()
    if esize not in (2, 4):
        raise TypeError("the attention mask buffer must be a 16- or 32-bit float tensor")
    root = _on(root_token_id, dev, torch.int64).reshape(1)
    tok = _on(node_token_ids, dev, torch.int64).reshape(-1)
    dep = _on(node_depths, dev, torch.int64).reshape(-1)
    vis = _on(visibility_cpu, dev, torch.bool).reshape(n1, n1)
    mfd_hip.call("mfd_tree_mask", root.data_ptr(), int(start), tok.data_ptr(), dep.data_ptr(), vis.data_ptr(), n1,
                 int(past_length), mask2d.data_ptr(), esize, _min_bits(dtype, mask2d.dtype), mask2d.stride(0),
                 mask2d.shape[1], mask2d.shape[0], ids_row.data_ptr(), pos_row.data_ptr(),
                 tree_visibility_buffer.data_ptr(), tree_visibility_buffer.stride(0), int(previous_tree_start),
                 int(previous_tree_length), mfd_hip.stream_of(mask2d))
    return (verify_input_ids_buffer[:, :n1], verify_position_ids_buffer[:, :n1],
            attention_mask_buffer[:, :, :n1, : past_length + n1], past_length, n1)


def follow_verified_tree(child_maps, posterior: torch.Tensor) -> tuple[list[int], int]:
    """Accept walk of inference/hf/ddtree.py:367-382: from the root, move to the child whose token is the
    target's choice at the current node until there is none; returns (accepted node indices, the next token).
    ``child_maps`` is a built Tree (its own follow) or a list of token -> node dicts, one per node."""
    if not isinstance(child_maps, list):
        accepted, next_token = child_maps.follow(posterior[0])
        return list(accepted), int(next_token)
    choice = posterior[0].to(device="cpu", dtype=torch.long).tolist()  # the target's token after each node
    path = [0]
    for _ in range(len(child_maps)):  # a path visits each node at most once
        token = int(choice[path[-1]])
        child = child_maps[path[-1]].get(token)
        if child is None:
            return path, token
        path.append(child)
    raise ValueError("child maps hold a cycle")


def compact_window_(tensors: list[torch.Tensor], past_length: int, keep_current_indices) -> None:
    """Move rows past_length + keep[m] to past_length + m (m = 0..len(keep) - 1) along dim -2 of every tensor,
    in place, with one kernel launch per group of equally shaped tensors (inference/hf/ddtree.py:389-404).
    Tensors [B, H, S, D] with a contiguous last dim; rows whose source equals their target are skipped."""
    if not tensors:
        return
    dev = tensors[0].device
    keep = torch.as_tensor(list(keep_current_indices), dtype=torch.int64)
    L = keep.numel()
    if L == 0:
        return
    src = (keep + past_length).to(dev)
    tgt = (torch.arange(L, dtype=torch.int64) + past_length).to(dev)
    groups: dict[tuple, list[torch.Tensor]] = {}
    for t in tensors:
        if t is None or t.numel() == 0:
            continue
        if t.stride(-1) != 1 or t.dim() != 4:
            raise ValueError("cache tensors must be [B, H, S, D] with a contiguous last dim")
        groups.setdefault((tuple(t.shape), tuple(t.stride()), t.element_size()), []).append(t)
    for (shape, stride, esize), ts in groups.items():
        B, H, S, D = shape
        if (D * esize) % 16 or (stride[2] * esize) % 16 or (stride[1] * esize) % 16 or (stride[0] * esize) % 16:
            raise ValueError("rows and head strides must be multiples of 16 bytes")
        # every (batch, head) plane is a segment; a plane's rows are the positions
        ptrs = torch.tensor([t.data_ptr() + b * stride[0] * esize for t in ts for b in range(B)], dtype=torch.int64)
        ptrs = ptrs.to(dev)
        for m0 in range(0, L, 64):
            m1 = min(L, m0 + 64)
            # chunks of at most 64 moves, in order: keep is increasing, so keep[m] >= m and no later chunk's
            # source (>= its own m) is an earlier chunk's target (< m0); inside a chunk the kernel reads every
            # source before it writes a target
            mfd_hip.call("mfd_kv_move", ptrs.data_ptr(), ptrs.numel(), stride[2] * esize, H, stride[1] * esize,
                         D * esize, S, src[m0:m1].contiguous().data_ptr(), tgt[m0:m1].contiguous().data_ptr(), 1,
                         m1 - m0, None, mfd_hip.stream_of(ts[0]))


def compact_dynamic_cache(past_key_values, past_length: int, keep_current_indices: list[int]) -> None:
    """inference/hf/ddtree.py:407-436: keep only the accepted nodes of the appended window in every attention
    layer of a DynamicCache, then crop."""
    if len(keep_current_indices) == 0:
        past_key_values.crop(past_length)
        return
    tensors = []
    if hasattr(past_key_values, "key_cache") and hasattr(past_key_values, "value_cache"):
        tensors = list(past_key_values.key_cache) + list(past_key_values.value_cache)
    elif hasattr(past_key_values, "layers"):
        for layer in past_key_values.layers:
            if getattr(layer, "keys", None) is None or layer.keys.numel() == 0:
                continue
            tensors += [layer.keys, layer.values]
    else:
        raise RuntimeError("Unsupported DynamicCache layout for DDTree cache compaction.")
    keep = list(keep_current_indices)
    current = [t.shape[-2] - past_length for t in tensors]
    if tensors and not (len(keep) == 0 or all(len(keep) == c for c in current)):
        compact_window_(tensors, past_length, keep)
    past_key_values.crop(past_length + len(keep))


HF_DDTREE_NAMES = ("compile_ddtree_tree", "follow_verified_tree", "compact_dynamic_cache")


def install(ddtree_module=None) -> dict:
    """Rebind ``compile_ddtree_tree``, ``follow_verified_tree`` and ``compact_dynamic_cache`` of the reference's
    HF ``ddtree`` module (inference/hf/ddtree.py:317-436) to this module's, together with any imported module
    that bound them by name. ``ddtree_module`` defaults to ``import ddtree`` (the reference's module, on the
    caller's path). Returns {name: the reference's function}."""
    if ddtree_module is None:
        import ddtree as ddtree_module  # the reference's decode-loop module; this package ships none of that name
    return mfd_hip.rebind(ddtree_module, {name: globals()[name] for name in HF_DDTREE_NAMES})
