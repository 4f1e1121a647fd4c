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
    for dt in (L.Q5_0, L.Q5_1):
        for op in (L.OP_KV_APPEND, L.OP_KV_GATHER, L.OP_KV_EVICT, L.OP_KV_COPY_BLOCKS, L.OP_PAGED_DECODE):
            assert lib.it_supports(op, dt) == 1
        assert lib.it_supports(L.OP_PAGED_PREFILL, dt) == 0
    assert lib.it_supports(L.OP_PAGED_DECODE, 9) == 0  # Q8_1 caches are not implemented
    assert lib.it_kv_page_bytes(32, 256, L.Q4_1) == 32 * 128 + 32 * 8 * 4  # 5120
    # nibble plane + per token 8 groups of (qh u32, d fp16) / (qh u32, d and m fp16)
    assert lib.it_kv_page_bytes(16, 128, L.Q5_0) == 16 * 64 + 16 * 4 * 6  # 1408 = 16 x 4 x 22 bytes
    assert lib.it_kv_page_bytes(32, 256, L.Q5_1) == 32 * 128 + 32 * 8 * 8  # 6144 = 32 x 8 x 24 bytes
    assert lib.it_supports(L.OP_PAGED_PREFILL, L.Q4_0) == 0
    assert lib.it_supports(L.OP_PAGED_PREFILL, L.BF16) == 1
    assert lib.it_supports(L.OP_PAGED_PREFILL, L.F16) == 1  # F16 caches run the same MFMA kernel
    assert lib.it_kv_page_bytes(32, 256, L.Q4_0) == 32 * 128 + 32 * 8 * 2  # 4608
    assert lib.it_kv_page_bytes(16, 128, L.BF16) == 4096
    assert lib.it_kv_page_bytes(32, 256, L.Q8_0) == 32 * 256 + 32 * 8 * 2  # 8704
    assert lib.it_kv_page_bytes(16, 128, L.F32) == 8192
    ws = lib.it_paged_decode_workspace(32, 28, 128, 4097, 512)
    assert ws >= 32 * 28 * 9 * (128 + 2) * 4


def test_decode_partition_planner():
    """it_paged_decode_partition: the smallest multiple of 64 whose
    non-empty units run in the fewest rounds of four resident workgroups per
    compute unit (host arithmetic, no device with n_cu given)."""
    import numpy as np

    from infer_train_amd import _lib as L
    from infer_train_amd.kv import decode_partition

    def plan(ctx, start=None, hq=28, hkv=4, dt=L.BF16, D=128, bs=16, n_cu=256):
        return decode_partition(dt, D, bs, hq, hkv, ctx, start, n_cu)

    # Config 2 at 4k: 32 x 4 heads x 8 partitions of 512 = 1024 = 4 x 256.
    assert plan(np.full(32, 4096)) == 512
    # Config 2 as specified (ragged): 256-token partitions give 1024 units.
    ctx = np.random.default_rng(22).integers(256, 4097, 32) + 1
    assert plan(ctx) == 256
    units = lambda p: int(sum((c + p - 1) // p for c in ctx)) * 4
    assert units(256) <= 1024 < units(192)
    # One 1024-token sequence (config 1 heads): the shortest partition.
    assert plan([1024], hq=12, hkv=2, dt=L.F32) == 64
    # Windows count only [start, ctx); empty batches take the shortest.
    assert plan(np.full(32, 8192), np.full(32, 8192 - 4096)) == 512
    assert plan([0, 5], [0, 5]) == 64
    # Half the compute units: 512-token partitions take 2 rounds of 512
    # slots; 1024-token ones also 2 (their LDS leaves 2 per CU); shorter
    # ones 3 or more.
    assert plan(np.full(32, 4096), n_cu=128) == 512
    # Config 5 (Q8_0, D 256, block 32, 16 x U[32k, 128k]) needs many rounds
    # at any size: the longest partition with two workgroups per CU (at
    # 1792 tokens a 4-wave workgroup takes just under 80 KiB of LDS; at
    # 1856 it would not fit twice).
    c5 = np.random.default_rng(5).integers(32768, 131073, 16)
    assert plan(c5, hq=24, hkv=4, dt=L.Q8_0, D=256, bs=32) == 1792
    assert plan(c5, hq=24, hkv=4, dt=L.Q4_0, D=256, bs=32) == 1920
    with pytest.raises(L.InvalidInput):
        plan([5], hq=7, hkv=2)
    with pytest.raises(L.NotImplementedOp):
        plan([5], D=96)
    with pytest.raises(ValueError):
        plan([5, 6], [1])


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
    assert lib.it_kv_cache_new(0, 16, 16, 2, 128, 9, C.byref(h)) == L.NOT_IMPLEMENTED  # Q8_1
    assert lib.it_kv_cache_new(0, 16, 16, 2, 100, L.Q5_1, C.byref(h)) == L.INVALID_INPUT  # D % 32
    assert lib.it_kv_cache_new(0, 16, 16, 2, 96 + 8, L.Q4_0, C.byref(h)) == L.INVALID_INPUT  # D % 32


def test_python_error_mapping():
    from infer_train_amd import BlockPool, InvalidInput

    p = BlockPool(2)
    with pytest.raises(InvalidInput):
        p.free(1)
