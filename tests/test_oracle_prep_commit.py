"""Pins of the oracle's conv windows, tree_prep and conv commit (CPU, float64).

The windows (inference/hf/qwen35_tree.py:39-52) are checked against their definition read forwards: the
last KC entries of [cached columns ; the root path from the root down to the node]. tree_prep
(inference/hf/tree_gdn_kernel.py:29-56) is checked on chains against torch's causal depthwise conv1d over
[conv state ; inputs] — the native layer's own convolution — followed by SiLU, the bf16 rounding and the
l2 normalisation written out independently. The conv commit (inference/hf/qwen35_tree.py:141-146) on a
chain is the last KC columns of [conv state ; inputs up to the accepted node]. Planted mistakes (reversed
windows, a dropped SiLU, the q / k head blocks swapped, the conv commit reading the wrong node) fail.
"""

import numpy as np
import pytest
import torch

from oracle import gdn


def random_parents(rng, n, forest=False):
    lo = -1 if forest else 0
    return np.array([-1] + [int(rng.integers(lo, i)) for i in range(1, n)], dtype=np.int32)


def root_path(parents, i):
    path = []
    while i >= 0:
        path.append(i)
        i = int(parents[i])
    return path[::-1]


@pytest.mark.parametrize("KC", [1, 2, 4, 6])
def test_conv_index_is_suffix_of_root_path(KC):
    rng = np.random.default_rng(KC)
    parents = random_parents(rng, 50, forest=True)
    idx = gdn.conv_index(parents, KC)
    for i in range(len(parents)):
        seq = list(range(KC)) + [KC + j for j in root_path(parents, i)]
        assert list(idx[i]) == seq[-KC:]


def chain_reference(x, conv_state, conv_w, HK, H, D, scale):
    """Causal depthwise conv1d over [state ; x] (torch, float64), SiLU, bf16 rounding, l2 normalisation."""
    CD, KC = conv_w.shape
    seq = torch.cat([torch.from_numpy(conv_state), torch.from_numpy(x).T], dim=1)[None]  # [1, CD, KC + n]
    w = torch.from_numpy(conv_w)[:, None, :]  # [CD, 1, KC]
    acc = torch.nn.functional.conv1d(seq, w, groups=CD)[0, :, 1:].T.numpy()  # outputs at the n node positions
    y = gdn.round_bf16(acc * (1.0 / (1.0 + np.exp(-acc))))
    n = x.shape[0]
    q = y[:, : HK * D].reshape(n, HK, D)
    k = y[:, HK * D : 2 * HK * D].reshape(n, HK, D)
    v = y[:, 2 * HK * D :].reshape(n, H, D)
    q = q * scale / np.sqrt(np.einsum("nhd,nhd->nh", q, q)[..., None] + 1e-6)
    k = k / np.sqrt(np.einsum("nhd,nhd->nh", k, k)[..., None] + 1e-6)
    return q, k, v


def prep_case(seed, n=12, HK=2, H=4, D=16, KC=4):
    rng = np.random.default_rng(seed)
    CD = (2 * HK + H) * D
    x = gdn.round_bf16(rng.standard_normal((n, CD)))
    conv_state = gdn.round_bf16(rng.standard_normal((CD, KC)))
    conv_w = gdn.round_bf16(rng.standard_normal((CD, KC)) * 0.5)
    return x, conv_state, conv_w


@pytest.mark.parametrize("seed", range(3))
def test_tree_prep_on_a_chain_is_the_causal_conv(seed):
    HK, H, D, KC, n = 2, 4, 16, 4, 12
    x, cs, w = prep_case(seed, n, HK, H, D, KC)
    parents = np.arange(-1, n - 1, dtype=np.int32)
    q, k, v = gdn.tree_prep(x, cs, gdn.conv_index(parents, KC), w, HK, H, D, D ** -0.5)
    qr, kr, vr = chain_reference(x, cs, w, HK, H, D, D ** -0.5)
    for a, b in ((q, qr), (k, kr), (v, vr)):
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


def test_tree_prep_branches_read_their_own_root_path():
    """Two siblings of one parent get the same window except for the last entry."""
    HK, H, D, KC = 2, 4, 16, 4
    x, cs, w = prep_case(7, 6, HK, H, D, KC)
    parents = np.array([-1, 0, 1, 1, 2, 3], dtype=np.int32)
    idx = gdn.conv_index(parents, KC)
    assert list(idx[2][:-1]) == list(idx[3][:-1]) and idx[2][-1] != idx[3][-1]
    q, k, v = gdn.tree_prep(x, cs, idx, w, HK, H, D, 0.25)
    # node 4 (path 0-1-2-4) equals the chain 0-1-2-4 computed as a sequence
    xs = x[[0, 1, 2, 4]]
    qr, kr, vr = chain_reference(xs, cs, w, HK, H, D, 0.25)
    np.testing.assert_allclose(q[4], qr[3], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(v[4], vr[3], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("mistake", ["reversed_window", "no_silu", "swapped_heads"])
def test_tree_prep_planted_mistakes_fail(mistake):
    HK, H, D, KC, n = 2, 4, 16, 4, 10
    x, cs, w = prep_case(3, n, HK, H, D, KC)
    parents = np.arange(-1, n - 1, dtype=np.int32)
    idx = gdn.conv_index(parents, KC)
    qr, kr, vr = chain_reference(x, cs, w, HK, H, D, D ** -0.5)
    if mistake == "reversed_window":
        q, k, v = gdn.tree_prep(x, cs, idx[:, ::-1].copy(), w, HK, H, D, D ** -0.5)
    elif mistake == "no_silu":
        acc = np.zeros((n, x.shape[1]))
        src = np.concatenate([cs.T, x])
        for t in range(KC):
            acc += w[:, t][None] * src[idx[:, t]]
        y = gdn.round_bf16(acc)
        v = y[:, 2 * HK * D :].reshape(n, H, D)
        q, k = qr, kr
    else:
        xs = x.copy()
        xs[:, : HK * D], xs[:, HK * D : 2 * HK * D] = x[:, HK * D : 2 * HK * D], x[:, : HK * D]
        q, k, v = gdn.tree_prep(xs, cs, idx, w, HK, H, D, D ** -0.5)
    diff = max(np.abs(q - qr).max(), np.abs(k - kr).max(), np.abs(v - vr).max())
    assert diff > 1e-3


def test_commit_conv_on_a_chain_is_the_input_suffix():
    KC, n, CD = 4, 9, 24
    rng = np.random.default_rng(5)
    conv = rng.standard_normal((CD, KC))
    x = rng.standard_normal((n, CD))
    parents = np.arange(-1, n - 1, dtype=np.int32)
    idx = gdn.conv_index(parents, KC)
    seq = np.concatenate([conv, x.T], axis=1)  # [CD, KC + n]
    for a in range(n):
        np.testing.assert_array_equal(gdn.commit_conv(conv, x, idx, a), seq[:, a + 1 : a + 1 + KC])
    # planted: reading the window of the wrong node fails
    assert not np.array_equal(gdn.commit_conv(conv, x, idx, 3), seq[:, 5 : 5 + KC])


def test_round_bf16_ties_to_even():
    vals = np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 3.0e38])
    out = gdn.round_bf16(vals)
    ref = torch.tensor(vals, dtype=torch.float32).to(torch.bfloat16).double().numpy()
    np.testing.assert_array_equal(out, ref)
