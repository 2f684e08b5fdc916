"""The float32 checking paths of the attention mirrors, on CPU tensors, against the float64 oracle:
mode_attention.reference (ModeBlocks(exact=True), inference/hf/mode_attention.py:153-164),
paged_mode_block_attention_reference (P:965-988) and PagedModeAttention(impl="reference") (P:991-1026) with a
stub KV pool. Runs without a GPU (no kernel is launched)."""

import numpy as np
import pytest
import torch

from oracle import attention as att
from oracle.synth import attention_inputs, paged_attention_inputs


def _rel(got, ref):
    return float(np.abs(np.asarray(got, dtype=np.float64) - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("K,bs,H,Hkv,ctx", [(8, 16, 32, 8, 300), (3, 16, 8, 2, 100), (1, 16, 4, 4, 0), (5, 7, 6, 3, 65)])
def test_flat_reference(K, bs, H, Hkv, ctx):
    import mode_attention

    q, k, v = attention_inputs(K + ctx, K=K, bs=bs, H=H, Hkv=Hkv, ctx=ctx)
    got = mode_attention.reference(q, k, v, K, bs, 128 ** -0.5)
    assert got.shape == (1, K * bs, H, 128) and got.dtype == torch.float32
    ref = att.mode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), K, bs, 128 ** -0.5)
    assert _rel(got.numpy(), ref) <= 1e-5


def test_modes_fp32_causal_in_block():
    import mode_attention

    q, k, v = attention_inputs(3, K=4, bs=8, H=8, Hkv=2, ctx=50)
    o = mode_attention.modes_fp32(q[0], k[0, :, :50], v[0, :, :50], k[0, :, 50:], v[0, :, 50:], 4, 8, 0.1,
                                  causal_in_block=True)
    ref = att.mode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 4, 8, 0.1, causal_in_block=True)
    assert _rel(o.transpose(0, 1).numpy(), ref[0]) <= 1e-5
    # planted: the bidirectional form differs from the causal one
    o2 = mode_attention.modes_fp32(q[0], k[0, :, :50], v[0, :, :50], k[0, :, 50:], v[0, :, 50:], 4, 8, 0.1)
    assert _rel(o2.transpose(0, 1).numpy(), ref[0]) > 1e-3


@pytest.mark.parametrize("page_size", [1, 64])
def test_paged_reference_and_hook(page_size):
    import paged_mode_attention as dm

    lens = [130, 1, 700]
    d = paged_attention_inputs(40 + page_size, lens, H=16, Hkv=4, page_size=64)
    if page_size == 1:
        table = d["req_to_token"]
    else:
        table = torch.zeros(len(lens) + 2, d["page_table"].shape[1], dtype=torch.int32)
        table[2:] = d["page_table"]
    slots = att.slots_from_pages(d["page_table"], d["ctx_lens"], 64)
    f = lambda t: t.float().numpy()
    ref = att.paged_mode_attention(f(d["q"]), f(d["k_new"]), f(d["v_new"]), f(d["k_cache"]), f(d["v_cache"]), slots,
                                   8, 16, d["scaling"])
    got = dm.paged_mode_block_attention_reference(
        q=d["q"], k_new=d["k_new"], v_new=d["v_new"], k_cache=d["k_cache"], v_cache=d["v_cache"],
        req_to_token=table, req_pool_indices=d["req_pool_indices"], ctx_lens=d["ctx_lens"], num_modes=8,
        block_size=16, scaling=d["scaling"], page_size=page_size)
    assert _rel(got.numpy(), ref) <= 1e-5

    class Pool:
        def get_kv_buffer(self, layer_id):
            assert layer_id == 3
            return d["k_cache"], d["v_cache"]

    class Batch:
        req_pool_indices = d["req_pool_indices"]
        seq_lens = d["ctx_lens"]

    hook = dm.PagedModeAttention(kv_pool=Pool(), req_to_token=table, num_modes=8, block_size=16, num_heads=16,
                                 num_kv_heads=4, head_dim=128, scaling=d["scaling"], num_ctx_splits=-1,
                                 impl="reference", page_size=page_size)
    T = d["q"].shape[0]
    out = hook(d["q"].reshape(T, -1), d["k_new"].reshape(T, -1), d["v_new"].reshape(T, -1), Batch(), 3)
    assert out.shape == (T, 16 * 128) and out.dtype == torch.bfloat16
    assert _rel(out.view(T, 16, 128).float().numpy(), ref) <= 1e-2
    with pytest.raises(ValueError):
        dm.PagedModeAttention(kv_pool=Pool(), req_to_token=table, num_modes=8, block_size=16, num_heads=16,
                              num_kv_heads=4, head_dim=128, scaling=1.0, num_ctx_splits=0, impl="cuda")
