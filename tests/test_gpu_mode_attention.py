"""GPU parity of the mode-attention HIP kernel (through the C ABI) against the float64 oracle.

Tolerance (north star: attention outputs within 2e-3 relative, bf16 inputs): the outputs are bf16, and a
single bf16 rounding alone costs up to 2^-9 = 1.95e-3 of an element, so the 2e-3 bound is applied to the
norm-wise relative error ||got - ref||_2 / ||ref||_2; the largest element error must also stay below
1e-2 * max |ref|.
"""

import numpy as np
import pytest
import torch

from oracle import attention as att
from oracle.synth import attention_inputs, paged_attention_inputs

pytestmark = pytest.mark.gpu


def _check(got, ref, tag=""):
    got = got.float().cpu().numpy().astype(np.float64)
    rms = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    mx = float(np.abs(got - ref).max() / np.abs(ref).max())
    print(f"{tag} rms-rel {rms:.2e} max-rel {mx:.2e}")
    assert rms <= 2e-3 and mx <= 1e-2, (tag, rms, mx)


@pytest.mark.parametrize("splits", [-1, 0, 3])
def test_config2_flat(splits):
    import mode_attention

    q, k, v = attention_inputs(2)
    print(f"case: config2 flat splits={splits}", flush=True)
    got = mode_attention.mode_block_attention(q.cuda(), k.cuda(), v.cuda(), 8, 16, 128 ** -0.5,
                                              num_ctx_splits=splits)
    torch.cuda.synchronize()
    ref = att.mode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 8, 16, 128 ** -0.5)
    _check(got, ref, f"config2 splits={splits}")


@pytest.mark.parametrize("ctx,K,bs,H,Hkv,splits", [
    (0, 8, 16, 32, 8, -1), (1, 8, 16, 32, 8, 2), (37, 4, 8, 8, 8, 1), (500, 2, 16, 16, 4, 5), (2048, 8, 16, 40, 8, -1),
])
def test_flat_shapes(ctx, K, bs, H, Hkv, splits):
    import mode_attention

    q, k, v = attention_inputs(10 + ctx, K=K, bs=bs, H=H, Hkv=Hkv, ctx=ctx)
    print(f"case: flat ctx={ctx} K={K} bs={bs} H={H} Hkv={Hkv} splits={splits}", flush=True)
    got = mode_attention.mode_block_attention(q.cuda(), k.cuda(), v.cuda(), K, bs, 128 ** -0.5, num_ctx_splits=splits)
    torch.cuda.synchronize()
    ref = att.mode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), K, bs, 128 ** -0.5)
    _check(got, ref, f"flat ctx={ctx}")


def test_causal_in_block_variant():
    import mode_attention

    q, k, v = attention_inputs(21, ctx=300)
    got = mode_attention.mode_block_attention(q.cuda(), k.cuda(), v.cuda(), 8, 16, 128 ** -0.5, causal_in_block=True)
    torch.cuda.synchronize()
    ref = att.mode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 8, 16, 128 ** -0.5,
                             causal_in_block=True)
    _check(got, ref, "causal")


def _paged(d, page_size, splits, table):
    import paged_mode_attention as dm

    cuda = lambda t: t.cuda()
    return dm.paged_mode_block_attention(
        q=cuda(d["q"]), k_new=cuda(d["k_new"]), v_new=cuda(d["v_new"]), k_cache=cuda(d["k_cache"]),
        v_cache=cuda(d["v_cache"]), req_to_token=cuda(table), req_pool_indices=cuda(d["req_pool_indices"]),
        ctx_lens=cuda(d["ctx_lens"]), num_modes=d["num_modes"], block_size=d["block_size"], scaling=d["scaling"],
        num_ctx_splits=splits, page_size=page_size)


def _paged_ref(d):
    f = lambda t: t.float().numpy()
    slots = att.slots_from_pages(d["page_table"], d["ctx_lens"], d["page_size"])
    return att.paged_mode_attention(f(d["q"]), f(d["k_new"]), f(d["v_new"]), f(d["k_cache"]), f(d["v_cache"]), slots,
                                    d["num_modes"], d["block_size"], d["scaling"])


@pytest.mark.parametrize("lens,splits", [([5, 900, 129], -1), ([1, 40, 700, 1500], 0), ([2048], 4), ([64, 3000], 11)])
def test_paged_per_token_table(lens, splits):
    d = paged_attention_inputs(30 + len(lens), lens, H=32, Hkv=8)
    print(f"case: paged page_size=1 lens={lens} splits={splits}", flush=True)
    # page_size 1: req_to_token holds the slot of every token; rows 0 and 1 unused as in SGLang's pool
    got = _paged(d, 1, splits, d["req_to_token"])
    torch.cuda.synchronize()
    _check(got, _paged_ref(d), f"paged1 {lens}")


def test_paged_64_token_pages_config4_heads():
    """Config 4 attention shapes (40 q heads over 8 KV heads, K=8 x 16), 64-token pages, U[1024, 8192] contexts."""
    g = torch.Generator().manual_seed(4000)
    lens = [int(x) for x in torch.randint(1024, 8193, (6,), generator=g)]
    d = paged_attention_inputs(4000, lens, H=40, Hkv=8, page_size=64)
    # page table rows addressed through req_pool_indices = b + 2
    pt = torch.zeros(len(lens) + 2, d["page_table"].shape[1], dtype=torch.int32)
    pt[2:] = d["page_table"]
    print(f"case: paged page_size=64 lens={lens}", flush=True)
    for splits in (-1, 0):
        got = _paged(d, 64, splits, pt)
        torch.cuda.synchronize()
        _check(got, _paged_ref(d), f"paged64 splits={splits}")


def test_paged_graph_replay_new_lengths():
    """Captured once, replayed with other context lengths (graph safety, P:607-609)."""
    import paged_mode_attention as dm

    d = paged_attention_inputs(50, [300], H=32, Hkv=8, extra_pages=100)
    r2t = torch.zeros(3, 4096, dtype=torch.int32)
    r2t[2, :300] = d["req_to_token"][2, :300]
    d["req_to_token"] = r2t
    dev = {k: (v.cuda() if torch.is_tensor(v) else v) for k, v in d.items()}
    out = torch.empty_like(dev["q"])
    args = dict(q=dev["q"], k_new=dev["k_new"], v_new=dev["v_new"], k_cache=dev["k_cache"], v_cache=dev["v_cache"],
                req_to_token=dev["req_to_token"], req_pool_indices=dev["req_pool_indices"], ctx_lens=dev["ctx_lens"],
                num_modes=8, block_size=16, scaling=128 ** -0.5, out=out)
    for splits in (8, 0):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            dm.paged_mode_block_attention(**args, num_ctx_splits=splits)
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            dm.paged_mode_block_attention(**args, num_ctx_splits=splits)
        slots_total = dev["k_cache"].shape[0]
        for c in (1, 17, 300, 1234, 4000):
            if c > slots_total:
                continue
            perm = torch.randperm(slots_total, generator=torch.Generator().manual_seed(c))[:c].to(torch.int32)
            row = torch.zeros(dev["req_to_token"].shape[1], dtype=torch.int32)
            row[:c] = perm
            dev["req_to_token"][2].copy_(row.cuda())
            dev["ctx_lens"].fill_(c)
            graph.replay()
            torch.cuda.synchronize()
            f = lambda t: t.float().cpu().numpy()
            ref = att.paged_mode_attention(f(dev["q"]), f(dev["k_new"]), f(dev["v_new"]), f(dev["k_cache"]),
                                           f(dev["v_cache"]), [perm.numpy()], 8, 16, 128 ** -0.5)
            _check(out, ref, f"graph splits={splits} ctx={c}")


@pytest.mark.parametrize("K", [1, 3])
def test_any_num_modes_flat_ctx4096(K):
    """num_modes * block_size not a multiple of 32 (K = 1, 3 at block 16): the last unit of every head is padded
    (the reference falls back to one mode per program for odd counts, inference/hf/mode_attention.py:129-132)."""
    import mode_attention

    q, k, v = attention_inputs(60 + K, K=K, ctx=4096)
    for splits in (-1, 0):
        print(f"case: flat K={K} ctx=4096 splits={splits}", flush=True)
        got = mode_attention.mode_block_attention(q.cuda(), k.cuda(), v.cuda(), K, 16, 128 ** -0.5,
                                                  num_ctx_splits=splits)
        torch.cuda.synchronize()
        ref = att.mode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), K, 16, 128 ** -0.5)
        _check(got, ref, f"flat K={K} splits={splits}")


@pytest.mark.parametrize("K,bs", [(1, 16), (3, 16), (5, 7)])
def test_any_num_modes_paged(K, bs):
    lens = [4096, 777, 1500]
    d = paged_attention_inputs(70 + K, lens, K=K, bs=bs, H=40, Hkv=8, page_size=64)
    pt = torch.zeros(len(lens) + 2, d["page_table"].shape[1], dtype=torch.int32)
    pt[2:] = d["page_table"]
    for splits in (-1, 0, 3):
        print(f"case: paged K={K} bs={bs} splits={splits}", flush=True)
        got = _paged(d, 64, splits, pt)
        torch.cuda.synchronize()
        _check(got, _paged_ref(d), f"paged K={K} bs={bs} splits={splits}")


def test_causal_in_block_config2_full_size():
    """The causal-in-block variant at config 2's size (ctx 4096, K 8 x 16, H 32 / Hkv 8), split and one pass."""
    import mode_attention

    q, k, v = attention_inputs(2)
    ref = att.mode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 8, 16, 128 ** -0.5,
                             causal_in_block=True)
    for splits in (-1, 0):
        print(f"case: causal config2 splits={splits}", flush=True)
        got = mode_attention.mode_block_attention(q.cuda(), k.cuda(), v.cuda(), 8, 16, 128 ** -0.5,
                                                  causal_in_block=True, num_ctx_splits=splits)
        torch.cuda.synchronize()
        _check(got, ref, f"causal config2 splits={splits}")


def test_fp32_checking_paths_on_gpu_match_oracle():
    """mode_attention.reference (ModeBlocks(exact=True)) and paged_mode_block_attention_reference on GPU tensors:
    float32 results within 1e-5 of the float64 oracle."""
    import paged_mode_attention as dm
    import mode_attention

    q, k, v = attention_inputs(80, K=3, ctx=1000)
    got = mode_attention.reference(q.cuda(), k.cuda(), v.cuda(), 3, 16, 128 ** -0.5)
    ref = att.mode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 3, 16, 128 ** -0.5)
    assert got.dtype == torch.float32 and got.shape == (1, 48, 32, 128)
    assert np.abs(got.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
    d = paged_attention_inputs(81, [300, 64], H=16, Hkv=4, page_size=64)
    pt = torch.zeros(4, d["page_table"].shape[1], dtype=torch.int32)
    pt[2:] = d["page_table"]
    cuda = lambda t: t.cuda()
    got = dm.paged_mode_block_attention_reference(
        q=cuda(d["q"]), k_new=cuda(d["k_new"]), v_new=cuda(d["v_new"]), k_cache=cuda(d["k_cache"]),
        v_cache=cuda(d["v_cache"]), req_to_token=cuda(pt), req_pool_indices=cuda(d["req_pool_indices"]),
        ctx_lens=cuda(d["ctx_lens"]), num_modes=8, block_size=16, scaling=d["scaling"], page_size=64)
    ref = _paged_ref(d)
    assert np.abs(got.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()


class _StubPool:
    """The two calls PagedModeAttention makes on SGLang's KV pool."""

    def __init__(self, k, v):
        self.k, self.v = k, v

    def get_kv_buffer(self, layer_id):
        return self.k[layer_id], self.v[layer_id]


class _StubBatch:
    def __init__(self, rpi, seq_lens):
        self.req_pool_indices, self.seq_lens = rpi, seq_lens


@pytest.mark.parametrize("impl", ["hip", "reference"])
def test_paged_mode_attention_hook(impl):
    """PagedModeAttention as DFlashAttention calls it (P:1010-1026): [T, heads * D] slices in, [T, H * D] out,
    layer-indexed KV pool, per-token req_to_token table; against the oracle."""
    import paged_mode_attention as dm

    lens = [900, 37]
    d = paged_attention_inputs(90, lens, H=32, Hkv=8)
    dev = torch.device("cuda")
    T = d["q"].shape[0]
    pool = _StubPool([None, d["k_cache"].to(dev)], [None, d["v_cache"].to(dev)])
    hook = dm.PagedModeAttention(kv_pool=pool, req_to_token=d["req_to_token"].to(dev), num_modes=8, block_size=16,
                                 num_heads=32, num_kv_heads=8, head_dim=128, scaling=d["scaling"], num_ctx_splits=-1,
                                 impl=impl)
    batch = _StubBatch(d["req_pool_indices"].to(dev), d["ctx_lens"].to(dev))
    out = hook(d["q"].reshape(T, -1).to(dev), d["k_new"].reshape(T, -1).to(dev), d["v_new"].reshape(T, -1).to(dev),
               batch, 1)
    torch.cuda.synchronize()
    assert out.shape == (T, 32 * 128) and out.dtype == torch.bfloat16
    slots = att.slots_from_req_to_token(d["req_to_token"], d["req_pool_indices"], d["ctx_lens"])
    f = lambda t: t.float().numpy()
    ref = att.paged_mode_attention(f(d["q"]), f(d["k_new"]), f(d["v_new"]), f(d["k_cache"]), f(d["v_cache"]), slots,
                                   8, 16, d["scaling"])
    _check(out.view(T, 32, 128), ref, f"hook impl={impl}")


def test_misaligned_rows_are_refused():
    """Rows are moved in 16-byte pieces: an output (or input) base or stride that is not a multiple of 8 elements
    is refused with an error instead of being read or written unaligned."""
    import mfd_hip
    import mode_attention

    q, k, v = (t.cuda() for t in attention_inputs(0, ctx=64, K=2, bs=16, H=4, Hkv=2))
    ctx = k.shape[2] - 32
    buf = torch.empty(1 * 32 * 4 * 128 + 4, dtype=torch.bfloat16, device="cuda")
    out = buf[4:].view(1, 32, 4, 128)  # base 8 bytes past a 16-byte boundary
    with pytest.raises(mfd_hip.MFDError, match="16-byte aligned"):
        mode_attention.launch(q=q, q_st=q.stride(2), q_sh=q.stride(1), k_new=k[:, :, ctx:], v_new=v[:, :, ctx:],
                              kn_st=k.stride(2), kn_sh=k.stride(1), vn_st=v.stride(2), vn_sh=v.stride(1), k_cache=k,
                              v_cache=v, kc_ss=k.stride(2), kc_sh=k.stride(1), vc_ss=v.stride(2), vc_sh=v.stride(1),
                              table=None, table_stride=0, page_size=1, req_idx=None, ctx_lens=None, ctx_const=ctx,
                              bs=1, num_modes=2, block_size=16, H=4, Hkv=2, D=128, scaling=128 ** -0.5, causal=False,
                              splits=1, out=out, o_st=out.stride(1), o_sh=out.stride(2), stream=mfd_hip.stream_of(q))


def _big(v, lo, hi, factor):
    """v with keys [lo, hi) of every KV head scaled by ``factor`` (bf16): magnitudes up to about 2e5, beyond fp16."""
    v = v.clone()
    v[..., lo:hi, :] = (v[..., lo:hi, :].float() * factor).to(torch.bfloat16)
    return v


@pytest.mark.parametrize("lo,hi,splits", [(0, 428, -1), (0, 428, 0), (0, 428, 3), (200, 203, 0), (310, 320, 2)])
def test_large_v_flat(lo, hi, splits):
    """|v| beyond fp16's range (65504), in every key, in a few context keys, or in the block keys (300 context keys,
    128 block keys): the workgroups that meet such a value compute their tiles again with the P V product in bf16,
    the reference's own arithmetic, and match the oracle like any other input."""
    import mode_attention

    q, k, v = attention_inputs(60, ctx=300)
    v = _big(v, lo, hi, 1e5)
    assert v.float().abs().max() > 65536
    print(f"case: large v flat keys [{lo}, {hi}) splits={splits}", flush=True)
    got = mode_attention.mode_block_attention(q.cuda(), k.cuda(), v.cuda(), 8, 16, 128 ** -0.5, num_ctx_splits=splits)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    ref = att.mode_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 8, 16, 128 ** -0.5)
    _check(got, ref, f"large v flat [{lo}, {hi}) splits={splits}")


@pytest.mark.parametrize("page_size,splits", [(1, -1), (64, 0), (64, 3)])
def test_large_v_paged(page_size, splits):
    """The same through the paged layouts (per-token table and 64-token pages): large values in part of the cache
    and in the new block values."""
    d = paged_attention_inputs(61, [100, 700], H=32, Hkv=8, page_size=64)
    d["v_cache"] = _big(d["v_cache"].transpose(0, 1), 0, d["v_cache"].shape[0] // 3, 2e5).transpose(0, 1).contiguous()
    d["v_new"] = _big(d["v_new"].transpose(0, 1), 0, 16, 2e5).transpose(0, 1).contiguous()
    print(f"case: large v paged page_size={page_size} splits={splits}", flush=True)
    if page_size == 1:
        got = _paged(d, 1, splits, d["req_to_token"])
    else:
        pt = torch.zeros(4, d["page_table"].shape[1], dtype=torch.int32)
        pt[2:] = d["page_table"]
        got = _paged(d, 64, splits, pt)
    torch.cuda.synchronize()
    assert torch.isfinite(got).all()
    _check(got, _paged_ref(d), f"large v paged{page_size} splits={splits}")
