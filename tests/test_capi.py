"""The C ABI library loads, exports every function include/mfd_hip.h declares, and rejects bad arguments
before touching the GPU (host-side validation only: no kernel is launched here)."""

import ctypes
import os
import re

import pytest

import mfd_hip

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "mfd_hip.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\s*\*?\s*(mfd_[a-z0-9_]+)\s*\(", text, re.M)))


def test_header_declares_the_hot_path():
    names = declared_functions()
    for n in ("mfd_tree_gdn", "mfd_mode_attn", "mfd_topk_logz", "mfd_build_mixture", "mfd_last_error"):
        assert n in names


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(mfd_hip.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) <= set(mfd_hip.exported_symbols())


def test_tree_context_sizes_and_validation_without_gpu():
    lib = mfd_hip.lib()
    # fused layout (max_nodes <= 128), one block per request: anc [nmax/32][nmax] u32 + path [nmax][16] u8 +
    # depth [nmax] i32 + 16-byte header
    for max_nodes, nmax in ((1, 32), (32, 32), (33, 64), (64, 64), (100, 128), (128, 128)):
        blk = nmax * nmax // 8 + 16 * nmax + 4 * nmax + 16
        assert lib.mfd_tree_ctx_bytes(3, max_nodes) == 3 * blk
    # large-tree layout: path [nmax][16] u16 + depth [nmax] u8 + 16-byte header
    for max_nodes, nmax in ((129, 256), (256, 256), (257, 512), (512, 512)):
        assert lib.mfd_tree_ctx_bytes(3, max_nodes) == 3 * (32 * nmax + nmax + 16)
    assert lib.mfd_tree_ctx_bytes(0, 64) == 0 and lib.mfd_tree_ctx_bytes(2, 513) == 0
    # context: buffer required, 16-byte aligned and large enough, max_nodes in range, parents or anc8
    big = 1 << 20
    assert lib.mfd_tree_context(1, None, 1, 2, 10, 16, None, big, None, None) == -1
    assert lib.mfd_tree_context(1, None, 1, 2, 10, 16, 8, big, None, None) == -1
    assert lib.mfd_tree_context(1, None, 1, 2, 10, 0, 16, big, None, None) == -2
    assert lib.mfd_tree_context(1, None, 1, 2, 10, 600, 16, big, None, None) == -2
    assert lib.mfd_tree_context(None, None, 1, 2, 10, 16, 16, big, None, None) == -1
    assert lib.mfd_tree_context(1, None, 1, 2, 10, 16, 16, 100, None, None) == -1
    assert b"needed" in lib.mfd_last_error()
    # GDN with a context: the context is required and must cover R blocks, sizes are checked as for mfd_tree_gdn
    assert lib.mfd_tree_gdn_ctx(1, 1, 1, 1, 1, 1, None, big, 1, 2, 10, 2, 4, 128, 16, 1, 1, None, None, 0,
                                None) == -1
    assert lib.mfd_tree_gdn_ctx(1, 1, 1, 1, 1, 1, 16, big, 1, 2, 10, 2, 4, 64, 16, 1, 1, None, None, 0, None) == -2
    assert lib.mfd_tree_gdn_ctx(1, 1, 1, 1, 1, 1, 16, big, 1, 2, 10, 2, 4, 128, 600, 1, 1, None, None, 0,
                                None) == -2
    need = lib.mfd_tree_ctx_bytes(2, 16)
    assert lib.mfd_tree_gdn_ctx(1, 1, 1, 1, 1, 1, 16, need - 16, 1, 2, 10, 2, 4, 128, 16, 1, 1, None, None, 0,
                                None) == -1
    assert b"ctx of" in lib.mfd_last_error()
    # large trees need the workspace (Gram rows, plus the contexts when the call builds them)
    assert lib.mfd_tree_gdn_workspace_bytes(2, 300, 4, 128, 0) == 0
    ws = lib.mfd_tree_gdn_workspace_bytes(2, 300, 4, 200, 0)
    gram = 300 * 4 * 32 * 4
    ctxb = ((2 * (32 * 256 + 256 + 16) + 255) // 256) * 256
    assert ws == ctxb + ((gram + 255) // 256) * 256
    assert lib.mfd_tree_gdn_workspace_bytes(2, 300, 4, 200, 1) == ((gram + 255) // 256) * 256
    assert lib.mfd_tree_gdn_workspace_bytes(2, 300, 4, 600, 0) == -1
    assert lib.mfd_tree_gdn_ctx(16, 16, 16, 16, 16, 16, 16, big, 16, 2, 300, 4, 8, 128, 200, 16, 16, None, None, 0,
                                None) == -1
    assert b"workspace" in lib.mfd_last_error()


def test_argument_validation_without_gpu():
    lib = mfd_hip.lib()
    nul = (None, None, None, None, None, None)
    # unsupported head dim
    rc = lib.mfd_tree_gdn(*nul, None, None, None, 1, 4, 2, 4, 64, 4, None, None, None, None, 0, None)
    assert rc == -2 and b"head dim" in lib.mfd_last_error()
    # H not a multiple of HK
    rc = lib.mfd_tree_gdn(*nul, None, None, None, 1, 4, 3, 4, 128, 4, None, None, None, None, 0, None)
    assert rc == -1
    # too many nodes for any kernel
    rc = lib.mfd_tree_gdn(*nul, 1, None, None, 1, 600, 2, 4, 128, 600, None, None, None, None, 0, None)
    assert rc == -2 and b"max_nodes" in lib.mfd_last_error()
    # parents or anc8 required
    rc = lib.mfd_tree_gdn(*nul, None, None, None, 1, 30, 2, 4, 128, 30, None, None, None, None, 0, None)
    assert rc == -1
    # a large tree without its workspace
    rc = lib.mfd_tree_gdn(16, 16, 16, 16, 16, 16, 16, None, None, 1, 300, 2, 4, 128, 300, 16, 16, None, None, 0,
                          None)
    assert rc == -1 and b"workspace" in lib.mfd_last_error()
    # attention: any K * L up to 65536 (an odd count is padded, not refused), head dim 128 only
    rc = lib.mfd_mode_attn(None, 0, 0, None, None, 0, 0, 0, 0, None, None, 0, 0, 0, 0, None, 0, 1, None, None, 0, 1, 3, 5,
                           8, 8, 128, 1.0, 0, 1, None, 0, 0, None, 0, None)
    assert rc == -1 and b"null" in lib.mfd_last_error()
    rc = lib.mfd_mode_attn(None, 0, 0, None, None, 0, 0, 0, 0, None, None, 0, 0, 0, 0, None, 0, 1, None, None, 0, 1,
                           4097, 17, 8, 8, 128, 1.0, 0, 1, None, 0, 0, None, 0, None)
    assert rc == -2 and b"65536" in lib.mfd_last_error()
    rc = lib.mfd_mode_attn(None, 0, 0, None, None, 0, 0, 0, 0, None, None, 0, 0, 0, 0, None, 0, 1, None, None, 0, 1, 3, 5,
                           8, 8, 64, 1.0, 0, 1, None, 0, 0, None, 0, None)
    assert rc == -2
    # attention: rows must be 16-byte aligned
    rc = lib.mfd_mode_attn(1, 0, 0, 16, 16, 0, 0, 0, 0, 16, 16, 0, 0, 0, 0, None, 0, 1, None, None, 10, 1, 8, 16, 32, 8,
                           128, 1.0, 0, 4, 16, 0, 0, None, 0, None)
    assert rc == -2 and b"16-byte" in lib.mfd_last_error()
    rc = lib.mfd_mode_attn(16, 12, 0, 16, 16, 0, 0, 0, 0, 16, 16, 0, 0, 0, 0, None, 0, 1, None, None, 10, 1, 8, 16, 32,
                           8, 128, 1.0, 0, 4, 16, 0, 0, None, 0, None)
    assert rc == -2 and b"16-byte" in lib.mfd_last_error()
    # attention: split workspace required
    rc = lib.mfd_mode_attn(16, 0, 0, 16, 16, 0, 0, 0, 0, 16, 16, 0, 0, 0, 0, None, 0, 1, None, None, 10, 1, 8, 16, 32, 8,
                           128, 1.0, 0, 4, 16, 0, 0, None, 0, None)
    assert rc == -1 and b"workspace" in lib.mfd_last_error()
    # logits step: k too large, misaligned rows
    assert lib.mfd_topk_logz(None, 4, 100, 104, 300, None, None, 0, None, None, 0, None) == -1
    assert lib.mfd_topk_logz(16, 4, 100, 100, 8, None, None, 0, None, None, 0, None) == -2
    assert lib.mfd_topk_logz_vocab(16, 4, 104, 104, 8, None, None, 0, None, None, None, 0, None) == -1
    # builder limits
    assert lib.mfd_build_mixture(None, None, 0, None, 1, 17, 4, 4, 8, None, None, None, None, None) == -2
    assert lib.mfd_build_mixture(None, None, 0, None, 1, 8, 4, 4, 5000, None, None, None, None, None) == -2


def test_prep_and_commit_validation_without_gpu():
    lib = mfd_hip.lib()
    # conv windows: kernel size 1..8, parents required
    assert lib.mfd_conv_index(None, None, 1, 4, 9, None, None, None) == -1
    assert lib.mfd_conv_index(None, None, 1, 4, 4, None, None, None) == -1
    # tree_prep: head dim 128 only, x row stride >= conv_dim, pointers required
    assert lib.mfd_tree_prep(1, 512, 1, 0, 1, 1, None, 1, 4, 1, 2, 64, 4, 1.0, 1, 1, 1, None, None) == -2
    assert lib.mfd_tree_prep(1, 500, 1, 0, 1, 1, None, 1, 4, 1, 2, 128, 4, 1.0, 1, 1, 1, None, None) == -2
    assert lib.mfd_tree_prep(16, 516, 16, 0, 1, 16, None, 1, 4, 1, 2, 128, 4, 1.0, 16, 16, 16, None, None) == -2
    assert lib.mfd_tree_prep(8, 512, 16, 0, 1, 16, None, 1, 4, 1, 2, 128, 4, 1.0, 16, 16, 16, None, None) == -2
    assert lib.mfd_tree_prep(None, 512, 1, 0, 1, 1, None, 1, 4, 1, 2, 128, 4, 1.0, 1, 1, 1, None, None) == -1
    # commit: path length in [1, n], GQA map, conv kernel size
    assert lib.mfd_gdn_commit(16, 0, 16, 0, 1, 0, 1, 0, 1, 0, 2, 8, 2, 4, 128, None, 0, None, 0, 0, None, 0, 0,
                              None, None) == -1
    assert lib.mfd_gdn_commit(16, 0, 16, 0, 1, 0, 1, 0, 1, 9, 2, 8, 2, 4, 128, None, 0, None, 0, 0, None, 0, 0,
                              None, None) == -1
    assert lib.mfd_gdn_commit(16, 0, 16, 0, 1, 0, 1, 0, 1, 2, 2, 8, 3, 4, 128, None, 0, None, 0, 0, None, 0, 0,
                              None, None) == -1
    assert lib.mfd_gdn_commit(16, 0, 16, 0, 1, 0, 1, 0, 1, 2, 2, 8, 2, 4, 128, 1, 0, 1, 0, 0, 1, 1024, 9,
                              None, None) == -1


def test_plumbing_validation_without_gpu():
    lib = mfd_hip.lib()
    # verify inputs: W in 1..4096, tree rows at least W long
    assert lib.mfd_verify_inputs(1, 1, 1, 1, 1, 8, 1, 1, 1, 1, 2, 0, 4, None, None) == -1
    assert lib.mfd_verify_inputs(1, 1, 1, 1, 1, 8, 1, 1, 1, 1, 2, 16, 4, None, None) == -1
    # follow: L in 1..64
    assert lib.mfd_tree_follow(1, 1, 1, 8, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 2, 8, 65, None) == -1
    # kv moves: 16-byte granularity, L in 1..64
    assert lib.mfd_kv_move(1, 2, 256, 1, 0, 200, 10, 1, 1, 1, 4, None, None) == -1
    assert lib.mfd_kv_move(1, 2, 256, 1, 0, 256, 10, 1, 1, 1, 65, None, None) == -1


def test_workspace_size_helpers():
    lib = mfd_hip.lib()
    assert lib.mfd_mode_attn_workspace_bytes(1, 8, 16, 32, 1) == 0
    # 9 partials of 32 x 128 rows: fp16 rows of 128, lse, scale exponent
    assert lib.mfd_mode_attn_workspace_bytes(1, 8, 16, 32, 8) == 9 * 32 * 128 * (128 * 2 + 4 + 4)
    assert lib.mfd_topk_logz_workspace_bytes(128, 151936, 8) >= 128 * 19 * (4 + 8 + 64)
    cap = ctypes.c_int(0)
    n = lib.mfd_build_mixture_smem_bytes(8, 16, 8, 64, ctypes.byref(cap))
    # frontier slots (logw, key, fields, child key, last rank: 24 B), 512 hash slots (16 B), 64 batch
    # candidates (20 B), records (8 B), prior, nodes, counter
    assert cap.value == 8 + 2 * 8 * 64 + 2
    assert n == cap.value * 24 + 512 * 16 + 64 * 20 + 8 * 16 * 8 * 8 + 64 + 65 * 12 + 16


def test_logits_step_limits_at_the_boundary():
    """The merge limit: ceil(V / 2048) * max(k, 1) <= 8192 for k <= 32, ceil(V / 8192) * k <= 8192 above; the
    workspace is rows * ceil(V / 2048) * (12 + 8 max(k, 1)) + 64 bytes. Checked without a launch: an accepted size
    gets past the limit checks to the null-pointer check (-1), a refused one stops at -2."""
    lib = mfd_hip.lib()
    for rows, V, k in ((3, 151936, 8), (1, 600000, 1), (2, 33333, 0), (5, 248320, 256)):
        assert lib.mfd_topk_logz_workspace_bytes(rows, V, k) == rows * (-(-V // 2048)) * (12 + 8 * max(k, 1)) + 64
    # k <= 32: one list per 2048-element piece
    v_max_32 = 8192 // 32 * 2048          # 256 pieces of 2048
    assert lib.mfd_topk_logz(16, 1, v_max_32, v_max_32, 32, None, None, 0, None, None, 0, None) == -1
    assert lib.mfd_topk_logz(16, 1, v_max_32 + 8, v_max_32 + 8, 32, None, None, 0, None, None, 0, None) == -2
    assert b"merge capacity" in lib.mfd_last_error()
    v_max_1 = 8192 * 2048                 # k = 1 (and k = 0: log Z only) take one entry per piece
    assert lib.mfd_topk_logz(16, 1, v_max_1, v_max_1, 1, None, None, 0, None, None, 0, None) == -1
    assert lib.mfd_topk_logz(16, 1, v_max_1 + 8, v_max_1 + 8, 0, None, None, 0, None, None, 0, None) == -2
    # k > 32: one list per 8192 elements
    v_max_64 = 8192 // 64 * 8192
    assert lib.mfd_topk_logz(16, 1, v_max_64, v_max_64, 64, None, None, 0, None, None, 0, None) == -1
    assert lib.mfd_topk_logz(16, 1, v_max_64 + 8, v_max_64 + 8, 64, None, None, 0, None, None, 0, None) == -2
