"""CPU checks of the C ABI: the library loads, exports every symbol the header
declares, the Python binding covers exactly those symbols, and argument
validation rejects bad calls before anything touches a GPU."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT

from engine import _hip

HEADER = os.path.join(ROOT, "include", "specverify.h")


def _declared():
    src = open(HEADER).read()
    return re.findall(r"^(?:const\s+)?\w+\*?\s+\*?(spv_\w+)\s*\(", src, re.M)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_hip.LIB_PATH):
        pytest.fail("libspecverify.so is not built; run __graft_entry__.build()")
    return _hip.lib()


def test_header_declares_the_path_entry_points():
    names = set(_declared())
    for need in ("spv_kv_append", "spv_kv_rewind", "spv_verify_attn", "spv_verify_sample",
                 "spv_pool_alloc_one", "spv_pool_free_one", "spv_kv_gather", "spv_kv_append_fp8"):
        assert need in names


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(_hip.LIB_PATH)
    for name in _declared():
        assert hasattr(raw, name), name


def test_binding_matches_header():
    assert set(_hip.SIGNATURES) == set(_declared())


def test_version(lib):
    assert b"gfx950" in lib.spv_version()


def test_argument_validation_needs_no_gpu(lib):
    ARG = _hip.SPV_ERR_ARG
    assert lib.spv_pool_init(None, None, None, 8, None) == ARG
    assert lib.spv_kv_rewind(None, 1, None, None, None, None, None, None, None, None, 1, 8, 16, 0, None) == ARG
    assert lib.spv_kv_rewind_append(None, None, 1, None, None, None, 4, None, None, None, None, None, None, None,
                                    None, None, 1, 1, 0, 8, 16, 2, 8, None, None) == ARG
    # an fp8 pool is refused before anything is launched (no device memory is touched)
    fake = ctypes.c_void_p(16)
    assert lib.spv_kv_rewind_append(fake, fake, _hip.SPV_FP8E4M3, fake, fake, fake, 4, fake, fake, fake, fake,
                                    fake, fake, None, None, fake, 1, 1, 0, 8, 16, 2, 64, None, None) == ARG
    assert lib.spv_kv_append(None, None, 1, None, None, None, 4, None, None, None, None, None, None,
                             None, 1, 1, 0, 8, 16, 2, 8, 1, 1, None) == ARG
    assert lib.spv_verify_sample(None, None, 0, 1.0, None, None, None, None, None, None, -1, 1, 5, 8,
                                 None, None, None, None, None, None, None, 0, None, 0, None) == ARG
    assert lib.spv_draft_sample(None, 8, 1.0, None, 1, 8, None, 1, None, None, None, 0, None) == ARG
    assert lib.spv_filter_logits(None, 8, None, 8, 1, 8, 1.0, 2, 1.0, None, None) == ARG
    assert lib.spv_race_argmax(None, None, 8, None, None) == ARG
    # fp8 append: no scales, then an input dtype the quantiser does not take
    assert lib.spv_kv_append_fp8(None, None, None, 0, None, None, None, 4, None, None, None, None, None,
                                 None, None, 1, 1, 0, 1, 8, 16, 2, 8, 1, 1, None) == ARG
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    assert lib.spv_kv_append_fp8(p, p, p, 3, p, p, p, 4, p, p, p, p, p, p, p, 1, 1, 0, 1, 8, 16, 2, 8, 1,
                                 1, None) == ARG
    assert lib.spv_kv_append_fp8(p, p, p, 0, p, p, p, 4, p, p, p, p, p, p, p, 1, 1, 2, 2, 8, 16, 2, 8, 1,
                                 1, None) == ARG  # layer beyond num_layers


def test_workspace_queries(lib):
    # Qwen2.5-1.5B-shaped verify attention: B=32, C=6, 12/2 heads, d=128, ctx <= 4102.
    ws = lib.spv_verify_attn_workspace_bytes(32, 6, 12, 2, 128, 16, 4102)
    assert ws > 0
    assert lib.spv_verify_attn_workspace_bytes(32, 6, 12, 5, 128, 16, 4102) == 0  # Hq % Hkv != 0
    assert lib.spv_verify_sample_workspace_bytes(64, 5, 151936) > 64 * 11 * 19 * 8
    assert lib.spv_verify_sample_workspace_bytes(64, 0, 151936) == 0
