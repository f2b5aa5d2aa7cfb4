"""C-ABI library checks that need no GPU: it loads, exports every function
declared in include/mi355_dsa.h, and rejects bad arguments before any launch
(the reference's TORCH_CHECK conditions, e.g. csrc/attention/
sm70_attn_fp8.cu:158-162, sm70_mla_decode.cu:2644-2653)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mi355_dsa.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mi355_dsa_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_op_surface():
    names = declared_functions()
    for op in ["indexer_k_store", "indexer_logits", "indexer_logits_packed", "decode_topk",
               "persistent_topk", "sparse_mla_decode", "attn_fp8_gemv", "attn_fp8_dequant",
               "selfcheck", "last_error", "concat_and_cache_mla", "head_proj", "mla_decode", "varlen_attention",
               "indexer_shard_merge"]:
        assert f"mi355_dsa_{op}" in names


def test_library_exports_every_declared_symbol(pkg, lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported"
    assert lib.mi355_dsa_abi_version() == 1


def _err(pkg):
    return pkg._lib.last_error()


def test_gemv_rejects_bad_m(pkg, lib):
    rc = lib.mi355_dsa_attn_fp8_gemv(None, None, None, None, 9, 128, 128, None)
    assert rc == 1 and "M must be 1..8, got 9" in _err(pkg)


def test_gemv_rejects_bad_alignment(pkg, lib):
    rc = lib.mi355_dsa_attn_fp8_gemv(None, None, None, None, 1, 12, 128, None)
    assert rc == 1 and "bad N/K alignment" in _err(pkg)


def test_dequant_rejects_bad_k(pkg, lib):
    rc = lib.mi355_dsa_attn_fp8_dequant(None, None, None, 8, 24, None)
    assert rc == 1 and "multiple of 16" in _err(pkg)


def test_indexer_rejects_non_pow2_page(pkg, lib):
    rc = lib.mi355_dsa_indexer_logits(None, 1, 64, None, 32, 128, None, 0, 64, 48,
                                      None, None, 1, None, None, None)
    assert rc == 1
    rc = lib.mi355_dsa_indexer_logits(1, 1, 64, 1, 32, 128, 1, 0, 64, 48, 1, 1, 1, 1, None, None)
    assert rc == 1 and "power of two" in _err(pkg)


def test_indexer_rejects_head_shape(pkg, lib):
    rc = lib.mi355_dsa_indexer_logits(1, 1, 64, 1, 16, 128, 1, 0, 64, 64, 1, 1, 1, 1, None, None)
    assert rc == 1 and "32 indexer heads" in _err(pkg)


def test_k_store_fp8_needs_128(pkg, lib):
    rc = lib.mi355_dsa_indexer_k_store(1, 1, 10, 16, 4, 64, 1, None)
    assert rc == 1 and "head_dim == 128" in _err(pkg)


def test_topk_rejects_k0(pkg, lib):
    rc = lib.mi355_dsa_decode_topk(None, None, None, None, 1, 10, 0, None, 0, None)
    assert rc == 1 and "k must be >= 1" in _err(pkg)


def test_empty_inputs_are_noops(pkg, lib):
    assert lib.mi355_dsa_indexer_k_store(None, 0, 0, None, 0, 128, None, None) == 0
    assert lib.mi355_dsa_persistent_topk(None, 0, 0, None, None, 4, 0, None, 0, None) == 0
    assert lib.mi355_dsa_sparse_mla_decode(None, None, None, 0, 64, None, 0, 0, 64, None, 0,
                                           None, 0, None, 1.0, None, 0, None) == 0


def test_sparse_workspace_size(lib):
    # decode config at B=4, H=64, topk=2048: 16 splits of fp16 partials + (m, l)
    n = lib.mi355_dsa_sparse_mla_workspace_size(4, 64, 2048)
    assert n == 4 * 64 * 16 * (512 * 2 + 2 * 4)
    # prefill config (>= 256 workgroups) needs none
    assert lib.mi355_dsa_sparse_mla_workspace_size(4096, 64, 2048) == 0


def test_sparse_rejects_small_workspace(pkg, lib):
    rc = lib.mi355_dsa_sparse_mla_decode(16, 16, 16, 4, 64, 16, 0, 100, 64, 16, 2048,
                                         16, 4, 16, 0.1, 16, 10, None)
    assert rc == 1 and "workspace too small" in _err(pkg)


def test_cache_writer_rejects_misaligned_rows(pkg, lib):
    rc = lib.mi355_dsa_concat_and_cache_mla(16, 1, 64, 16, 500, 16, 64, 0, 1, 16, 1, None)
    assert rc == 1 and "row strides" in _err(pkg)
    rc = lib.mi355_dsa_concat_and_cache_mla(16, 0, 64, 16, 512, 16, 64, 1, 1, 16, 1, None)
    assert rc == 1 and "fp16 inputs" in _err(pkg)


def test_head_proj_rejects_bad_shapes(pkg, lib):
    # K not a multiple of 32
    rc = lib.mi355_dsa_head_proj(16, 576 * 4, 576, 16, 4 * 192, 192, 16, 4, 4, 512, 100, 64, None)
    assert rc == 1 and "multiple of 32" in _err(pkg)
    # N not a multiple of 64 at K = 128
    rc = lib.mi355_dsa_head_proj(16, 576 * 4, 576, 16, 4 * 192, 192, 16, 4, 4, 480, 128, 64, None)
    assert rc == 1 and "multiple of 64" in _err(pkg)
    # x head stride too small for K + tail
    rc = lib.mi355_dsa_head_proj(16, 576 * 4, 576, 16, 4 * 128, 128, 16, 4, 4, 512, 128, 64, None)
    assert rc == 1 and "strides too small" in _err(pkg)
    # T = 0 is a no-op
    assert lib.mi355_dsa_head_proj(None, 0, 0, None, 0, 0, None, 0, 4, 512, 128, 64, None) == 0
