"""The drop-in boundary: libkmoe.so loads and exports every entry point that
include/kmoe.h declares (no GPU needed: nothing is called)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "kmoe.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(kmoe_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_path():
    names = declared()
    for must in ["kmoe_matmul", "kmoe_quantize_q8k", "kmoe_quantize_q8", "kmoe_route", "kmoe_dispatch",
                 "kmoe_moe_ffn", "kmoe_layer_create", "kmoe_expert_upload", "kmoe_expert_part",
                 "kmoe_expert_is_ready", "kmoe_q4k_block_sums", "kmoe_q6k_block_sums", "kmoe_last_error"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    path = os.path.join(ROOT, "kestrel_amd", "libkmoe.so")
    if not os.path.exists(path):
        pytest.skip("libkmoe.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.kmoe_abi_version() == 1


def test_binding_covers_the_header():
    from kestrel_amd.kmoe import SIGNATURES

    assert sorted(SIGNATURES) == declared()
