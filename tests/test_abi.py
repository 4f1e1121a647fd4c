"""CPU checks of the C ABI: the library loads without a GPU, exports every
function include/it_kv.h declares, and validates arguments before touching
the device (no compute is launched here)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "it_kv.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(it_[a-z0-9_]+)\s*\(", src)))


def test_every_declared_symbol_is_exported():
    from infer_train_amd._lib import LIB_PATH, SIGNATURES

    raw = C.CDLL(LIB_PATH)
    names = _declared()
    assert len(names) >= 35
    missing = [n for n in names if not hasattr(raw, n)]
    assert not missing, missing
    assert set(names) == set(SIGNATURES), set(names) ^ set(SIGNATURES)


def test_product_does_not_reference_oracle():
    pkg = os.path.join(ROOT, "infer_train_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".hpp", ".h", "Makefile")):
                text = open(os.path.join(dirpath, f), errors="replace").read()
                assert "import oracle" not in text and "liboracle" not in text and "it_oracle" not in text, f


def test_status_codes_and_pure_queries():
    from infer_train_amd import _lib as L

    lib = L.lib
    assert lib.it_abi_version() == 1
    assert lib.it_supports(L.OP_PAGED_DECODE, L.BF16) == 1
    assert lib.it_supports(L.OP_PAGED_DECODE, L.Q4_0) == 1
    assert lib.it_supports(L.OP_PAGED_DECODE, L.Q4_1) == 1
    assert lib.it_supports(L.OP_PAGED_DECODE, 6) == 0  # Q5_0 caches are not implemented
    assert lib.it_kv_page_bytes(32, 256, L.Q4_1) == 32 * 128 + 32 * 8 * 4  # 5120
    assert lib.it_supports(L.OP_PAGED_PREFILL, L.Q4_0) == 0
    assert lib.it_kv_page_bytes(32, 256, L.Q4_0) == 32 * 128 + 32 * 8 * 2  # 4608
    assert lib.it_kv_page_bytes(16, 128, L.BF16) == 4096
    assert lib.it_kv_page_bytes(32, 256, L.Q8_0) == 32 * 256 + 32 * 8 * 2  # 8704
    assert lib.it_kv_page_bytes(16, 128, L.F32) == 8192
    ws = lib.it_paged_decode_workspace(32, 28, 128, 4097, 512)
    assert ws >= 32 * 28 * 9 * (128 + 2) * 4


def test_invalid_input_before_device():
    from infer_train_amd import _lib as L

    lib = L.lib
    assert lib.it_kv_append(None, None, None, L.BF16, None, 1, None) == L.INVALID_INPUT
    assert b"NULL" in lib.it_last_error()
    assert lib.it_kv_gather(None, None, 1, None, None, None, 1, 1, None, None, None) == L.INVALID_INPUT
    assert lib.it_paged_decode(None, None, L.BF16, 28, None, 1, None, None, 1, 1, C.c_float(0.1), 512, None, 0,
                               None, L.BF16, None) == L.INVALID_INPUT
    assert lib.it_flash_attention(None, None, None, None, None, 1, 128, 1, None, 0, None) == L.INVALID_INPUT
    h = C.c_void_p()
    assert lib.it_kv_cache_new(0, 16, 12, 2, 128, L.BF16, C.byref(h)) == L.NOT_IMPLEMENTED  # bs not 2^k
    assert lib.it_kv_cache_new(0, 16, 16, 2, 100, L.Q8_0, C.byref(h)) == L.INVALID_INPUT  # D % 32
    assert lib.it_kv_cache_new(0, 16, 16, 2, 128, 6, C.byref(h)) == L.NOT_IMPLEMENTED  # Q5_0
    assert lib.it_kv_cache_new(0, 16, 16, 2, 96 + 8, L.Q4_0, C.byref(h)) == L.INVALID_INPUT  # D % 32


def test_python_error_mapping():
    from infer_train_amd import BlockPool, InvalidInput

    p = BlockPool(2)
    with pytest.raises(InvalidInput):
        p.free(1)
