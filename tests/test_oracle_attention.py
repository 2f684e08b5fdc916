"""Pins of the mode-attention oracle (CPU, float64).

The oracle restates the reference's masked-SDPA definition (inference/hf/mode_attention.py:153-164,
P:965-988). It is pinned by torch's SDPA (a library routine) with the reference's own mask, by an
independent per-mode formulation (each mode block is plain unmasked attention over the context plus its
own block), by K = 1 reducing to plain attention, by GQA equivalence to repeated K/V, by mode-permutation
equivariance, by paged == flat gathering, and the checks catch planted mistakes (cross-mode leakage,
wrong GQA map, dropped scale).
"""

import numpy as np
import pytest
import torch

from oracle import attention as att
from oracle.synth import paged_attention_inputs


def flat_case(seed, K=4, bs=8, H=8, Hkv=2, D=32, ctx=40):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, H, K * bs, D, generator=g)
    k = torch.randn(1, Hkv, ctx + K * bs, D, generator=g)
    v = torch.randn(1, Hkv, ctx + K * bs, D, generator=g)
    return q, k, v


def sdpa_reference(q, k, v, K, bs, scaling):
    H, Hkv = q.shape[1], k.shape[1]
    ctx = k.shape[2] - K * bs
    qb = torch.arange(K * bs) // bs
    mask = torch.zeros((K * bs, k.shape[2]), dtype=torch.float64)
    mask[:, ctx:].masked_fill_(qb[:, None] != qb[None, :], float("-inf"))
    kk = k.double().repeat_interleave(H // Hkv, dim=1)
    vv = v.double().repeat_interleave(H // Hkv, dim=1)
    return torch.nn.functional.scaled_dot_product_attention(q.double(), kk, vv, attn_mask=mask, scale=scaling).transpose(1, 2)


@pytest.mark.parametrize("seed,ctx", [(0, 40), (1, 0), (2, 1), (3, 97)])
def test_matches_torch_sdpa_with_reference_mask(seed, ctx):
    q, k, v = flat_case(seed, ctx=ctx)
    got = att.mode_attention(q.numpy(), k.numpy(), v.numpy(), 4, 8, 0.25)
    ref = sdpa_reference(q, k, v, 4, 8, 0.25).numpy()
    np.testing.assert_allclose(got, ref, atol=1e-12)


def per_mode_attention(q, k, v, K, bs, scaling):
    """Independent formulation: mode m's queries against [context ; block m], no mask at all."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    _, H, KL, D = q.shape
    Hkv = k.shape[1]
    ctx = k.shape[2] - KL
    out = np.zeros((1, KL, H, D))
    for m in range(K):
        rows = slice(m * bs, (m + 1) * bs)
        keys = np.r_[0:ctx, ctx + m * bs:ctx + (m + 1) * bs]
        for h in range(H):
            kh, vh = k[0, h // (H // Hkv)][keys], v[0, h // (H // Hkv)][keys]
            s = q[0, h, rows] @ kh.T * scaling
            p = np.exp(s - s.max(1, keepdims=True))
            out[0, rows, h] = (p / p.sum(1, keepdims=True)) @ vh
    return out


def test_matches_per_mode_formulation():
    q, k, v = flat_case(5, K=3, bs=6, H=6, Hkv=3, ctx=17)
    np.testing.assert_allclose(att.mode_attention(q.numpy(), k.numpy(), v.numpy(), 3, 6, 0.3),
                               per_mode_attention(q, k, v, 3, 6, 0.3), atol=1e-12)


def test_one_mode_is_plain_attention():
    q, k, v = flat_case(6, K=1, bs=16, H=4, Hkv=4, ctx=33)
    ref = torch.nn.functional.scaled_dot_product_attention(q.double(), k.double(), v.double(), scale=0.2)
    np.testing.assert_allclose(att.mode_attention(q.numpy(), k.numpy(), v.numpy(), 1, 16, 0.2),
                               ref.transpose(1, 2).numpy(), atol=1e-12)


def test_mode_permutation_equivariance():
    K, bs = 4, 8
    q, k, v = flat_case(7, K=K, bs=bs, ctx=20)
    perm = [2, 0, 3, 1]
    idx = np.concatenate([np.arange(p * bs, (p + 1) * bs) for p in perm])
    ctx = k.shape[2] - K * bs
    kidx = np.concatenate([np.arange(ctx), ctx + idx])
    base = att.mode_attention(q.numpy(), k.numpy(), v.numpy(), K, bs, 0.3)
    permuted = att.mode_attention(q.numpy()[:, :, idx], k.numpy()[:, :, kidx], v.numpy()[:, :, kidx], K, bs, 0.3)
    np.testing.assert_allclose(permuted, base[:, idx], atol=1e-12)


def test_paged_equals_flat_gather():
    d = paged_attention_inputs(1, [70, 5, 130], K=2, bs=16, H=4, Hkv=2, D=32, page_size=16)
    slots_pages = att.slots_from_pages(d["page_table"], d["ctx_lens"], 16)
    slots_tok = att.slots_from_req_to_token(d["req_to_token"], d["req_pool_indices"], d["ctx_lens"])
    for a, b in zip(slots_pages, slots_tok):
        assert (a == b).all()
    f = lambda t: t.float().numpy()
    got = att.paged_mode_attention(f(d["q"]), f(d["k_new"]), f(d["v_new"]), f(d["k_cache"]), f(d["v_cache"]),
                                   slots_pages, 2, 16, 0.2)
    # request by request through the flat form
    KL = 32
    for b, slots in enumerate(slots_pages):
        rows = slice(b * KL, (b + 1) * KL)
        kk = np.concatenate([f(d["k_cache"])[slots], f(d["k_new"])[rows]], 0).transpose(1, 0, 2)[None]
        vv = np.concatenate([f(d["v_cache"])[slots], f(d["v_new"])[rows]], 0).transpose(1, 0, 2)[None]
        qq = f(d["q"])[rows].transpose(1, 0, 2)[None]
        np.testing.assert_allclose(got[rows], att.mode_attention(qq, kk, vv, 2, 16, 0.2)[0], atol=1e-12)


def test_causal_variant_masks_later_block_keys():
    q, k, v = flat_case(8, K=2, bs=4, H=2, Hkv=1, D=8, ctx=0)
    out = att.mode_attention(q.numpy(), k.numpy(), v.numpy(), 2, 4, 0.5, causal_in_block=True)
    # with no context, the first query of each block sees only its own key
    for m in range(2):
        np.testing.assert_allclose(out[0, m * 4, 0], v.numpy()[0, 0, m * 4], atol=1e-12)


@pytest.mark.parametrize("mistake", ["leak", "gqa", "scale"])
def test_planted_mistakes_are_caught(mistake):
    q, k, v = flat_case(9, K=3, bs=6, H=6, Hkv=3, ctx=17)
    ref = per_mode_attention(q, k, v, 3, 6, 0.3)
    qn, kn, vn = q.numpy(), k.numpy(), v.numpy()
    if mistake == "leak":  # no block mask
        H, Hkv = 6, 3
        bad = np.zeros_like(ref)
        for h in range(H):
            s = qn[0, h] @ kn[0, h // 2].T * 0.3
            p = np.exp(s - s.max(1, keepdims=True))
            bad[0, :, h] = (p / p.sum(1, keepdims=True)) @ vn[0, h // 2]
    elif mistake == "gqa":  # head h reads KV head h % Hkv
        bad = att.mode_attention(qn[:, [0, 3, 1, 4, 2, 5]], kn, vn, 3, 6, 0.3)[:, :, [0, 2, 4, 1, 3, 5]]
    else:
        bad = att.mode_attention(qn, kn, vn, 3, 6, 1.0)
    assert np.abs(bad - ref).max() > 1e-3
