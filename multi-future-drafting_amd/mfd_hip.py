"""ctypes binding of libmfd_hip.so (the C ABI declared in include/mfd_hip.h).

The library must be built (``__graft_entry__.build()`` or ``python build_lib.py``); importing this
module without it raises immediately — there is no fallback implementation. Tensors cross the
boundary as raw device pointers; kernels run on the caller's current HIP stream.
"""

from __future__ import annotations

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmfd_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() (hipcc, gfx950)")

_lib = ctypes.CDLL(LIB_PATH)

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float

_lib.mfd_last_error.restype = ctypes.c_char_p
_lib.mfd_mode_attn_workspace_bytes.restype = _I64
_lib.mfd_mode_attn_workspace_bytes.argtypes = [_I, _I, _I, _I, _I]
_lib.mfd_version.restype = _I
_lib.mfd_topk_logz_workspace_bytes.restype = _I64
_lib.mfd_topk_logz_workspace_bytes.argtypes = [_I, _I, _I]
_lib.mfd_build_mixture_smem_bytes.restype = _I
_lib.mfd_build_mixture_smem_bytes.argtypes = [_I, _I, _I, _I, _P]
_lib.mfd_build_single_smem_bytes.restype = _I
_lib.mfd_build_single_smem_bytes.argtypes = [_I, _I, _I, _P]
_lib.mfd_tree_ctx_bytes.restype = ctypes.c_size_t
_lib.mfd_tree_ctx_bytes.argtypes = [_I, _I]
_lib.mfd_tree_gdn_workspace_bytes.restype = _I64
_lib.mfd_tree_gdn_workspace_bytes.argtypes = [_I, _I, _I, _I, _I]

_SIGNATURES = {
    # name: argtypes (all return int status)
    "mfd_tree_gdn": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I64, _P],
    "mfd_tree_gdn_noalloc": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P],
    "mfd_tree_gates": [_P, _P, _I, _I64, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _P],
    "mfd_tree_context": [_P, _P, _P, _I, _I, _I, _P, _I64, _P, _P],
    "mfd_tree_gdn_ctx": [_P, _P, _P, _P, _P, _P, _P, _I64, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I64, _P],
    "mfd_mode_attn": [_P, _I64, _I64,                      # q, token / head strides
                      _P, _P, _I64, _I64, _I64, _I64,      # k_new, v_new, strides
                      _P, _P, _I64, _I64, _I64, _I64,      # k_cache, v_cache, strides
                      _P, _I64, _I,                        # slot table, its row stride, page size
                      _P, _P, _I,                          # req_idx, ctx_lens, ctx_len_const
                      _I, _I, _I, _I, _I, _I, _F, _I,      # bs, K, L, H, Hkv, D, scale, causal
                      _I, _P, _I64, _I64,                  # splits, out, out strides
                      _P, _I64, _P],                       # workspace, bytes, stream
    "mfd_topk_logz": [_P, _I, _I, _I64, _I, _P, _P, _I, _P, _P, _I64, _P],
    "mfd_topk_logz_vocab": [_P, _I, _I, _I64, _I, _P, _P, _I, _P, _P, _P, _I64, _P],
    "mfd_topk_logz_wide": [_P, _I, _I, _I, _I64, _I, _P, _P, _I, _P, _P, _P],
    "mfd_draft_head_gemm": [_P, _I64, _I, _I64, _P, _I, _I, _I, _P, _I64, _P],
    "mfd_draft_topk_head": [_P, _I64, _I, _I64, _P, _I, _I, _I, _P, _I64, _I, _P, _P, _I, _P, _P, _P, _I64, _P],
    "mfd_build_mixture": [_P, _P, _I, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P],
    "mfd_build_trees_host": [_P, _P, _I, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P],
    "mfd_build_single": [_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P],
    "mfd_conv_index": [_P, _P, _I, _I, _I, _P, _P, _P],
    "mfd_verify_inputs": [_P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _I, _I, _I, _P, _P],
    "mfd_tree_mask": [_P, _I64, _P, _P, _P, _I, _I64, _P, _I, ctypes.c_uint32, _I64, _I64, _I, _P, _P, _P, _I64,
                      _I64, _I, _P],
    "mfd_tree_follow": [_P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "mfd_kv_move": [_P, _I, _I64, _I, _I64, _I, _I64, _P, _P, _I, _I, _P, _P],
    "mfd_draft_prepare": [_P, _P, _P, _P, _I64, _I, _I64, _P, _P, _P, _I, _I, _I, _P],
    "mfd_mode_mask": [_P, _P, _P, _I, _I, _I, _P],
    "mfd_tree_prep": [_P, _I64, _P, _I64, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P],
    "mfd_gdn_commit": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I, _I, _I, _I, _I, _I, _P, _I64, _P, _I64,
                       _I64, _P, _I, _I, _P, _P],
}
for _name, _args in _SIGNATURES.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = _I


class MFDError(RuntimeError):
    pass


def lib():
    return _lib


def check(status: int, name: str) -> None:
    if status != 0:
        raise MFDError(f"{name} failed ({status}): {_lib.mfd_last_error().decode(errors='replace')}")


def call(name: str, *args) -> None:
    check(getattr(_lib, name)(*args), name)


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    if t is None:
        return None
    return t.data_ptr()


def workspace(nbytes: int, device) -> torch.Tensor | None:
    """A 256-byte aligned device scratch buffer of ``nbytes`` bytes (None for 0)."""
    if nbytes <= 0:
        return None
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_cuda(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("MFD kernels take GPU tensors (got a tensor on %s)" % t.device)


def exported_symbols() -> list[str]:
    return ["mfd_last_error", "mfd_version", "mfd_mode_attn_workspace_bytes", "mfd_topk_logz_workspace_bytes",
            "mfd_build_mixture_smem_bytes", "mfd_build_single_smem_bytes", "mfd_tree_ctx_bytes",
            "mfd_tree_gdn_workspace_bytes", *_SIGNATURES]


_CU_COUNT = {}


def cu_count(device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _CU_COUNT:
        _CU_COUNT[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CU_COUNT[idx]


def rebind(target, replacements: dict) -> dict:
    """Point the module-level names of ``target`` (a module object) at ``replacements`` ({name: object}), and
    also every name of an already-imported module that is bound to one of the objects being replaced (a caller
    that ran ``from target import name`` before the switch). Returns {name: the object it replaced, or None}.
    Names ``target`` does not define are added; nothing else of ``target`` changes."""
    import sys

    old = {name: getattr(target, name, None) for name in replacements}
    for name, new in replacements.items():
        setattr(target, name, new)
    originals = {id(obj): name for name, obj in old.items() if obj is not None}
    if originals:
        for mod in list(sys.modules.values()):
            if mod is None or mod is target:
                continue
            attrs = getattr(mod, "__dict__", None)
            if not isinstance(attrs, dict):
                continue
            for attr, value in list(attrs.items()):
                name = originals.get(id(value))
                if name is not None and value is old[name]:
                    setattr(mod, attr, replacements[name])
    return old
