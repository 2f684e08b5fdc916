"""HF tree-round plumbing on MI355X — the hot-path subset of the reference's inference/hf/ddtree.py:
``compile_ddtree_tree`` (verify ids, positions and the additive tree mask in the caller's buffers,
:317-357), ``follow_verified_tree`` (the accept walk, :367-382) and ``compact_dynamic_cache`` (the accepted
nodes' KV moved to the front of the appended window, :385-436).

The mask rows and the KV moves run as HIP kernels (csrc/verify_plumbing.hip); the walk over a built Tree stays
on the host as in the reference (the device walk for a batch is ``ddtree_utils.ddtree_follow``).
"""

from __future__ import annotations

import torch

import mfd_hip


def compile_ddtree_tree(root_token_id, start: int, node_token_ids, node_depths, visibility_cpu, past_length: int,
                        dtype, device, verify_input_ids_buffer, verify_position_ids_buffer, attention_mask_buffer,
                        tree_visibility_buffer, previous_tree_start: int, previous_tree_length: int):
    """Same contract as inference/hf/ddtree.py:317-357: fills the verify ids [1, n + 1], positions and the
    [1, 1, n + 1, past + n + 1] additive mask (0 where visible, finfo.min elsewhere) in the given buffers and
    returns (ids, positions, mask, past_length, n + 1)."""
    current_length = 1 + int(node_token_ids.numel())
    if previous_tree_length > 0:
        attention_mask_buffer[0, 0, :previous_tree_length,
                              previous_tree_start: previous_tree_start + previous_tree_length] = 0
    verify_input_ids = verify_input_ids_buffer[:, :current_length]
    verify_input_ids[0, 0] = root_token_id
    if current_length > 1:
        verify_input_ids[0, 1:current_length].copy_(node_token_ids, non_blocking=False)
    verify_position_ids = verify_position_ids_buffer[:, :current_length]
    verify_position_ids[0, 0] = start
    if current_length > 1:
        verify_position_ids[0, 1:current_length].copy_(node_depths, non_blocking=False)
        verify_position_ids[0, 1:current_length].add_(start)
    visibility = tree_visibility_buffer[:current_length, :current_length]
    visibility.copy_(visibility_cpu, non_blocking=False)
    tree_block = attention_mask_buffer[0, 0, :current_length, past_length: past_length + current_length]
    tree_block.fill_(torch.finfo(dtype).min)
    tree_block.masked_fill_(visibility, 0)
    attention_mask = attention_mask_buffer[:, :, :current_length, : past_length + current_length]
    return verify_input_ids, verify_position_ids, attention_mask, past_length, current_length


def follow_verified_tree(child_maps, posterior: torch.Tensor) -> tuple[list[int], int]:
    """inference/hf/ddtree.py:367-382: walk the built tree along the target's tokens; ``child_maps`` is a
    Tree (tree_build_ext) or a list of token -> node dicts."""
    if not isinstance(child_maps, list):
        accepted, next_token = child_maps.follow(posterior[0].to(device="cpu", dtype=torch.long))
        return list(accepted), int(next_token)
    post = posterior[0].tolist()
    accepted, current = [0], 0
    nxt = int(post[0])
    while nxt in child_maps[current]:
        current = child_maps[current][nxt]
        accepted.append(current)
        nxt = int(post[current])
    return accepted, nxt


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
