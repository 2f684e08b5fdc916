"""Writes tests/golden/builder_golden.npz: (top_log_probs, top_ids, log_prior, budget) -> tree from the
reference's own C++ builders, compiled from /root/reference by oracle/build_oracle.py into oracle/_ref/.

  python tests/golden/make_builder_golden.py

Cases: the config-1 shape (K 8, L 16, k 8, B 64) on the logits-pass output of the synthetic config-1
logits; random trials in the style of the reference's own tests (tests/test_sglang_tree_builder.py:51-95,
inference/hf/tree_build_ext.py:237-269): modes 2/8, vocab 64/512, budgets 16..255, every fourth trial
with coarse (round(2x)/2) logits so that scores tie exactly; and single-mode DDTree cases through the
HF build_single. The vectors are data; no reference source is stored.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import builder  # noqa: E402
from oracle.synth import builder_logits  # noqa: E402


def _logp_ids(logits, k):
    lp = logits.float()
    top, ids = torch.topk(lp, k=k, dim=-1)
    return (top - torch.logsumexp(lp, -1, keepdim=True)).float(), ids


def main():
    sg = builder.ref_sglang_builder()
    hf = builder.ref_hf_builder()
    assert sg is not None and hf is not None, "build oracle/_ref first (oracle/build_oracle.py, needs /root/reference)"
    cases = []

    # config 1: logits-pass output of the synthetic logits (the product's deterministic logits step)
    lp, ids, _ = builder.top_candidates(builder_logits(1).reshape(128, -1), 8)
    cases.append(("mixture", lp.reshape(8, 16, 8), ids.reshape(8, 16, 8), np.zeros(8, np.float32), 64))

    gen = torch.Generator().manual_seed(0)
    for trial in range(60):
        modes = (2, 8)[trial % 2]
        depth = int(torch.randint(1, 16, (1,), generator=gen))
        vocab = 64 if trial % 5 else 512
        budget = (16, 31, 63, 128, 255)[(trial // 2) % 5]
        logits = torch.randn(modes, depth, vocab, generator=gen) * 3
        if trial % 4 == 0:
            logits = (logits * 2).round() / 2
        logits = logits.to(torch.bfloat16)
        prior = torch.log_softmax(torch.randn(modes, generator=gen), -1) if trial % 3 == 0 else torch.zeros(modes)
        lpt, idt = _logp_ids(logits, min(budget, vocab))
        cases.append(("mixture", lpt.numpy(), idt.numpy(), prior.float().numpy(), budget))
    for trial in range(20):
        depth = int(torch.randint(1, 16, (1,), generator=gen))
        budget = (16, 63, 255)[trial % 3]
        logits = torch.randn(1, depth, 64, generator=gen) * 3
        if trial % 2 == 0:
            logits = (logits * 2).round() / 2
        lpt, idt = _logp_ids(logits.to(torch.bfloat16), min(budget, 64))
        cases.append(("single", lpt.numpy(), idt.numpy(), np.zeros(1, np.float32), budget))

    out = {"n": np.array(len(cases))}
    for i, (kind, lp, ids, prior, budget) in enumerate(cases):
        if kind == "mixture":
            K = lp.shape[0]
            width = budget + 1
            tree = torch.empty((1, 3, width), dtype=torch.long)
            counts = torch.empty(1, dtype=torch.long)
            sg.build_trees(torch.from_numpy(lp)[None].contiguous(), torch.from_numpy(ids)[None].to(torch.int32).contiguous(),
                           torch.from_numpy(prior)[None].contiguous(), 1, budget, tree, counts)
            n = int(counts[0])
            hf_res = hf.build_mixture(torch.from_numpy(lp).contiguous(), torch.from_numpy(ids).long().contiguous(),
                                      torch.from_numpy(prior).contiguous(), budget)
            assert list(hf_res[2]) == tree[0, 2, : n + 1].tolist(), "HF and SGLang reference builders disagree"
            vis = hf_res[4].numpy().astype(np.uint8)
            tr = tree[0].numpy()
        else:
            res = hf.build_single(torch.from_numpy(lp[0]).contiguous(), torch.from_numpy(ids[0]).long().contiguous(), budget)
            n = len(res[0])
            tr = np.zeros((3, budget + 1), dtype=np.int64)
            tr[2, :] = -1
            tr[0, 1 : n + 1] = res[0].numpy()
            tr[1, 1 : n + 1] = res[1].numpy()
            tr[2, : n + 1] = np.asarray(res[2])
            vis = res[4].numpy().astype(np.uint8)
        out[f"c{i}_kind"] = np.array(kind)
        out[f"c{i}_lp"] = lp.astype(np.float32)
        out[f"c{i}_ids"] = ids.astype(np.int64)
        out[f"c{i}_prior"] = prior.astype(np.float32)
        out[f"c{i}_budget"] = np.array(budget)
        out[f"c{i}_tree"] = tr.astype(np.int64)
        out[f"c{i}_count"] = np.array(n)
        out[f"c{i}_vis"] = np.packbits(vis, axis=None)
    np.savez_compressed(os.path.join(HERE, "builder_golden.npz"), **out)
    print(f"wrote {len(cases)} cases")


if __name__ == "__main__":
    main()
