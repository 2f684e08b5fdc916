"""The logits step of tree construction on MI355X (top-k candidates, their log-probabilities, log Z) — drop-in for
the reference's inference/hf/tree_logits.py (row_logsumexp, top_candidates).

One HIP kernel pass over the bf16 logits (csrc/logits_topk.hip): per 2048-element piece the piece max, a sum
of exp(x - max) in a fixed order from a table of e^x over bf16 values, and the piece's top-k; a second small
kernel merges the pieces of a row. The top-k order is value descending, token id ascending (torch.topk leaves
ties unspecified), and log Z is reproducible bit for bit on the CPU while agreeing with torch.logsumexp to
about one fp32 ulp. float32 / float16 logits, which the reference also takes, go through csrc/logits_wide.hip:
one workgroup per row, an exact radix select on 32-bit order keys and an fp32 log Z.
"""

from __future__ import annotations

import torch

import mfd_hip


def topk_logz(logits: torch.Tensor, k: int, ids_dtype=torch.int64, with_logz: bool = False, vocab_ids=None,
              out=None, workspace: torch.Tensor | None = None):
    """Device form: logits [..., V] bf16, fp16 or fp32 (CUDA) -> (log-probs [..., k] f32, ids [..., k], [log Z [...] f32]),
    all on the device; no host synchronisation. ``vocab_ids`` [V] int32: logit column c is token vocab_ids[c]
    (a reduced draft vocabulary; the ids returned are mapped through it). ``out``: (log-probs [R, k], ids [R, k],
    log Z [R] or None) buffers to write into; ``workspace``: a uint8 buffer of at least
    mfd_topk_logz_workspace_bytes(R, V, k) bytes (both optional, for graph capture without allocation).
    Limits: k <= 256; for bf16 ceil(V / 2048) * max(k, 1) <= 8192 for k <= 32 and ceil(V / 8192) * k <= 8192
    above (the row merge holds 8192 candidates); larger requests raise MFDError. fp16 / fp32 logits (the reference
    takes any float dtype) go through a radix-select kernel with an fp32 log Z (no workspace, no V limit)."""
    mfd_hip.require_cuda(logits, vocab_ids)
    wide = {torch.float32: 0, torch.float16: 1}.get(logits.dtype)  # MFD_DTYPE_F32 / MFD_DTYPE_F16
    if logits.dtype != torch.bfloat16 and wide is None:
        raise TypeError("logits must be bfloat16, float16 or float32")
    V = logits.shape[-1]
    lead = logits.shape[:-1]
    rows = logits.reshape(-1, V)
    vec = 16 // logits.element_size()  # elements per 16-byte unit: rows start 16-byte aligned
    if rows.stride(-1) != 1 or rows.stride(0) % vec != 0 or rows.data_ptr() % 16 != 0:
        rows = rows.contiguous()
        if V % vec != 0:
            padded = torch.empty(rows.shape[0], (V + vec - 1) // vec * vec, dtype=rows.dtype, device=rows.device)
            padded[:, :V] = rows
            rows = padded
    R = rows.shape[0]
    if out is not None:
        logp, ids, logz = out
        ids_dtype = ids.dtype
        if logp.shape != (R, k) or ids.shape != (R, k) or (logz is not None and logz.shape != (R,)):
            raise ValueError("out buffers must be [R, k], [R, k] and [R]")
    else:
        logp = torch.empty(R, k, dtype=torch.float32, device=logits.device)
        ids = torch.empty(R, k, dtype=ids_dtype, device=logits.device)
        logz = torch.empty(R, dtype=torch.float32, device=logits.device) if (with_logz or k == 0) else None
    if vocab_ids is not None and (vocab_ids.dtype != torch.int32 or vocab_ids.numel() != V):
        raise ValueError("vocab_ids must be int32 [V]")
    args = (rows.data_ptr(), R, V, rows.stride(0), k, logp.data_ptr() if k else None, ids.data_ptr() if k else None,
            1 if ids_dtype == torch.int64 else 0, mfd_hip.ptr(logz))
    if wide is not None:  # float32 / float16 logits: one kernel, no workspace
        mfd_hip.call("mfd_topk_logz_wide", rows.data_ptr(), wide, *args[1:],
                     None if vocab_ids is None else vocab_ids.contiguous().data_ptr(), mfd_hip.stream_of(logits))
    else:
        nbytes = mfd_hip.lib().mfd_topk_logz_workspace_bytes(R, V, k)
        ws = workspace if workspace is not None else torch.empty(nbytes, dtype=torch.uint8, device=logits.device)
        if ws.numel() < nbytes:
            raise ValueError(f"workspace of {nbytes} bytes needed")
        if vocab_ids is not None:
            mfd_hip.call("mfd_topk_logz_vocab", *args, vocab_ids.contiguous().data_ptr(), ws.data_ptr(), ws.numel(),
                         mfd_hip.stream_of(logits))
        else:
            mfd_hip.call("mfd_topk_logz", *args, ws.data_ptr(), ws.numel(), mfd_hip.stream_of(logits))
    res = (logp.view(*lead, k), ids.view(*lead, k))
    if with_logz:
        res = res + (logz.view(lead),)
    return res


def row_logsumexp(x: torch.Tensor) -> torch.Tensor:
    """logsumexp over the last dim of a bf16, fp16 or fp32 CUDA tensor, as float32 with keepdim
    (inference/hf/tree_logits.py:34-39)."""
    _, _, logz = topk_logz(x, 0, with_logz=True)
    return logz.view(*x.shape[:-1], 1)


def top_candidates(logits: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(top-k log-probabilities as float32 on CPU, their token ids as int64 on CPU) of [..., V] draft logits
    (inference/hf/tree_logits.py:42-46: the HF builder consumes them on the host)."""
    logp, ids = topk_logz(logits, k, ids_dtype=torch.int64)
    return logp.to(device="cpu"), ids.to(device="cpu")


def check_equal(seed: int = 0) -> None:
    """Self-test of inference/hf/tree_logits.py:49-60: top_candidates on [8, 15, 248320] bf16 logits at three
    scales against torch.topk / torch.logsumexp in float32 — ids identical (ties, which bf16 rows at this size
    have, follow the id-ascending rule, so the comparison is on the tie-broken torch order), log-probs within
    1e-4."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    for scale in (1.0, 4.0, 16.0):
        x = (torch.randn(8, 15, 248320, device="cuda", generator=gen) * scale).to(torch.bfloat16)
        xf = x.float()
        # torch order with ties broken by id: sort by (value desc, id asc) over the top 512 candidates
        vals, idx = torch.topk(xf, 512, dim=-1)
        order = torch.argsort(idx, dim=-1, stable=True)
        vals, idx = vals.gather(-1, order), idx.gather(-1, order)
        order = torch.argsort(vals, dim=-1, descending=True, stable=True)
        ref_top, ref_ids = vals.gather(-1, order)[..., :256], idx.gather(-1, order)[..., :256]
        ref = ref_top - torch.logsumexp(xf, dim=-1, keepdim=True)
        got, ids = top_candidates(x, 256)
        if not torch.equal(ids, ref_ids.cpu()):
            raise AssertionError(f"scale {scale}: top-k ids differ")
        err = (got - ref.cpu()).abs().max().item()
        if not err < 1e-4:
            raise AssertionError(f"scale {scale}: max |dlogp| {err:.2e}")
        print(f"scale {scale}: ids identical, max |dlogp| {err:.2e}")


if __name__ == "__main__":
    check_equal()
