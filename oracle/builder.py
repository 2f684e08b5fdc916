"""CPU oracle of the logits step and the mixture-tree builder. TEST INFRASTRUCTURE ONLY.

Thin ctypes wrappers over oracle/csrc/oracle.c (the C restatement; see its header for the exact
semantics and the reference lines it follows) plus loaders for the reference's own C++ builders
compiled into oracle/_ref/ by oracle/build_oracle.py (present only where /root/reference was
available at build time; the GPU box receives the compiled modules, never the reference sources).
"""

from __future__ import annotations

import ctypes
import glob
import importlib.util
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "lib", "liboracle.so")
LZ_CHUNK = 2048

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            from oracle import build_oracle

            build_oracle.build_oracle()
        _lib = ctypes.CDLL(LIB)
        P, I, I64, F, D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_double
        _lib.oracle_exp_det.restype = F
        _lib.oracle_exp_det.argtypes = [F]
        _lib.oracle_exp_table.restype = F
        _lib.oracle_exp_table.argtypes = [ctypes.c_int]
        _lib.oracle_chunk_sum.restype = F
        _lib.oracle_chunk_sum.argtypes = [P, I, F]
        _lib.oracle_log_det.restype = D
        _lib.oracle_log_det.argtypes = [D]
        _lib.oracle_logz_row.restype = F
        _lib.oracle_logz_row.argtypes = [P, I64]
        _lib.oracle_top_candidates.restype = None
        _lib.oracle_top_candidates.argtypes = [P, I64, I64, I, P, P, P]
        _lib.oracle_build_mixture.restype = I64
        _lib.oracle_build_mixture.argtypes = [P, P, P, I, I, I, I64, P, P, P, P]
        _lib.oracle_build_single.restype = I64
        _lib.oracle_build_single.argtypes = [P, P, I, I, I64, P, P, P]
        _lib.oracle_visibility.restype = None
        _lib.oracle_visibility.argtypes = [P, I64, P]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def exp_det(d: float) -> float:
    return float(lib().oracle_exp_det(float(d)))


def exp_table(i: int) -> float:
    """Entry i of the e^x table over bf16 x (index min(max(rotl16(bits, 1) - 0x6600, 0), 8191))."""
    return float(lib().oracle_exp_table(int(i)))


def exp_table_index(bits: int) -> int:
    r = (((bits << 1) | (bits >> 15)) & 0xFFFF) - 0x6600
    return min(max(r, 0), 8191)


def chunk_sum(bits: np.ndarray, m: float) -> float:
    """S_c of one chunk (uint16 bf16 bit patterns, at most LZ_CHUNK of them) against its maximum m."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    assert b.size <= LZ_CHUNK
    return float(lib().oracle_chunk_sum(_p(b), int(b.size), float(m)))


def log_det(z: float) -> float:
    return float(lib().oracle_log_det(float(z)))


def as_bf16_bits(x) -> np.ndarray:
    """uint16 bit patterns of a bf16 torch tensor (or of an existing uint16 array)."""
    import torch

    if isinstance(x, np.ndarray):
        assert x.dtype == np.uint16
        return np.ascontiguousarray(x)
    assert x.dtype == torch.bfloat16
    return np.ascontiguousarray(x.contiguous().view(torch.int16).numpy().view(np.uint16))


def top_candidates(logits, k: int):
    """logits [..., V] bf16 -> (log-probs [..., k] f32, ids [..., k] int64, log Z [...] f32)."""
    bits = as_bf16_bits(logits)
    shape = bits.shape[:-1]
    V = bits.shape[-1]
    rows = int(np.prod(shape)) if shape else 1
    flat = bits.reshape(rows, V)
    lp = np.zeros((rows, k), dtype=np.float32)
    ids = np.zeros((rows, k), dtype=np.int64)
    lz = np.zeros(rows, dtype=np.float32)
    lib().oracle_top_candidates(_p(flat), rows, V, k, _p(lp), _p(ids), _p(lz))
    return lp.reshape(*shape, k), ids.reshape(*shape, k), lz.reshape(shape)


def top_candidates_wide(logits, k: int):
    """logits [..., V] float32 / float16 (numpy or torch, CPU) -> (log-probs [..., k] f64, ids [..., k] int64,
    log Z [...] f64): the reference's top_candidates / row_logsumexp on logits of any float dtype
    (inference/hf/tree_logits.py:34-46: torch.topk in the logits' dtype, a logsumexp of the same values), restated
    in float64: the k largest values (ties by column ascending, -0 as +0), log Z = M + log(sum e^(x - M))."""
    x = logits.float().numpy() if hasattr(logits, "numpy") else np.asarray(logits, dtype=np.float32)
    x = x.astype(np.float64)
    shape = x.shape[:-1]
    V = x.shape[-1]
    flat = x.reshape(-1, V)
    lp = np.zeros((flat.shape[0], k))
    ids = np.zeros((flat.shape[0], k), dtype=np.int64)
    lz = np.zeros(flat.shape[0])
    for r, row in enumerate(flat):
        m = row.max()
        if np.isfinite(m):
            lz[r] = m + np.log(np.exp(row - m).sum())
        else:
            lz[r] = m
        order = np.lexsort((np.arange(V), -row))[:k]  # value descending, then column ascending
        ids[r] = order
        lp[r] = row[order] - lz[r]
    return lp.reshape(*shape, k), ids.reshape(*shape, k), lz.reshape(shape)


def build_mixture(lp, ids, prior, budget: int):
    """lp [K, L, k] f32, ids [K, L, k] int, prior [K] f32 -> (tokens, depths, parents) each [budget + 1]
    int64 (index 0 = root; tail (0, 0, -1)), node count, pop count."""
    lp = np.ascontiguousarray(lp, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    prior = np.ascontiguousarray(prior, dtype=np.float32)
    K, L, k = lp.shape
    width = max(budget, 0) + 1
    t = np.zeros(width, dtype=np.int64)
    d = np.zeros(width, dtype=np.int64)
    p = np.zeros(width, dtype=np.int64)
    pops = np.zeros(1, dtype=np.int64)
    n = lib().oracle_build_mixture(_p(lp), _p(ids), _p(prior), K, L, k, max(budget, 0), _p(t), _p(d), _p(p), _p(pops))
    return t, d, p, int(n), int(pops[0])


def build_single(lp, ids, budget: int):
    lp = np.ascontiguousarray(lp, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    L, k = lp.shape
    width = max(budget, 0) + 1
    t = np.zeros(width, dtype=np.int64)
    d = np.zeros(width, dtype=np.int64)
    p = np.zeros(width, dtype=np.int64)
    n = lib().oracle_build_single(_p(lp), _p(ids), L, k, max(budget, 0), _p(t), _p(d), _p(p))
    assert n >= 0, "path deeper than the oracle's limit"
    return t, d, p, int(n)


def visibility(parents, n: int) -> np.ndarray:
    """[n + 1, n + 1] ancestor-or-self matrix (uint8) of parents[0..n]."""
    par = np.ascontiguousarray(parents[: n + 1], dtype=np.int64)
    vis = np.zeros((n + 1, n + 1), dtype=np.uint8)
    lib().oracle_visibility(_p(par), n, _p(vis))
    return vis


# ---------------------------------------------------------------- the reference's own compiled builders


def _load_ref(name: str):
    hits = glob.glob(os.path.join(HERE, "_ref", name + "*.so"))
    if not hits:
        return None
    spec = importlib.util.spec_from_file_location(name, hits[0])
    mod = importlib.util.module_from_spec(spec)
    import torch  # noqa: F401  (the modules link against torch)

    spec.loader.exec_module(mod)
    return mod


def ref_hf_builder():
    """inference/hf/tree_build_ext.py's C++ (build_single, build_mixture, Tree), or None."""
    return _load_ref("ref_hf_builder")


def ref_sglang_builder():
    """The SGLang patch's C++ build_trees (P:1377-1407), or None."""
    return _load_ref("ref_sglang_builder")
