"""ctypes binding of libit_kv.so (the C ABI declared in include/it_kv.h).

The library is the product: every device entry point runs hand-written
gfx950 kernels.  There is no fallback; if the library is missing this module
raises at import time.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libit_kv.so")

# Status codes and dtype ids (include/it_kv.h; OpError src/types.rs:227-231,
# QuantType src/types.rs:106-144).
OK, NOT_IMPLEMENTED, INVALID_INPUT, DEVICE_ERROR = 0, 1, 2, 3
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, BF16 = 0, 1, 2, 3, 6, 7, 8, 30
BLOCK_SIZE = 16
QK8_0 = 32
BLOCK_Q8_0_BYTES = 34
QK4_0 = 32
BLOCK_Q4_0_BYTES = 18
QK4_1 = 32
BLOCK_Q4_1_BYTES = 20
QK5_0 = QK5_1 = 32
BLOCK_Q5_0_BYTES = 22  # ggml block_q5_0 (types.rs:116 has only the id)
BLOCK_Q5_1_BYTES = 24  # ggml block_q5_1 (types.rs:117)
QUANT_TYPES = (Q8_0, Q4_0, Q4_1, Q5_0, Q5_1)
OP_KV_APPEND, OP_KV_GATHER, OP_KV_EVICT, OP_PAGED_DECODE, OP_PAGED_PREFILL, OP_FLASH_ATTENTION, OP_KV_COPY_BLOCKS = range(1, 8)


class OpError(RuntimeError):
    """Mirror of the reference's OpError enum (src/types.rs:227-231)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{_NAMES.get(code, code)}: {msg}")
        self.code = code
        self.msg = msg


class NotImplementedOp(OpError):
    pass


class InvalidInput(OpError):
    pass


class DeviceError(OpError):
    pass


_NAMES = {NOT_IMPLEMENTED: "NotImplemented", INVALID_INPUT: "InvalidInput", DEVICE_ERROR: "DeviceError"}
_CLASSES = {NOT_IMPLEMENTED: NotImplementedOp, INVALID_INPUT: InvalidInput, DEVICE_ERROR: DeviceError}


class CacheDesc(C.Structure):
    _fields_ = [
        ("k_pool", C.c_void_p),
        ("v_pool", C.c_void_p),
        ("num_blocks", C.c_int64),
        ("page_bytes", C.c_int64),
        ("block_size", C.c_int32),
        ("n_kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("dtype", C.c_int32),
        ("device", C.c_int32),
        ("owns_memory", C.c_int32),
        ("n_layers", C.c_int32),
    ]


class StepPlanC(C.Structure):
    """it_kv_step_plan (include/it_kv.h)."""
    _fields_ = [
        ("slots", C.c_void_p),
        ("token_seq", C.c_void_p),
        ("token_pos", C.c_void_p),
        ("tokens_cap", C.c_int32),
        ("n_tokens", C.c_int32),
        ("evicted", C.c_void_p),
        ("evicted_cap", C.c_int32),
        ("n_evicted", C.c_int32),
        ("cow_src", C.c_void_p),
        ("cow_dst", C.c_void_p),
        ("cow_cap", C.c_int32),
        ("n_cow", C.c_int32),
        ("ctx_lens", C.c_void_p),
        ("start_pos", C.c_void_p),
    ]


P = C.c_void_p
i32, i64, f32, sz = C.c_int32, C.c_int64, C.c_float, C.c_size_t
PP = C.POINTER(C.c_void_p)

# name -> (restype, argtypes)
SIGNATURES = {
    "it_last_error": (C.c_char_p, []),
    "it_abi_version": (i32, []),
    "it_supports": (i32, [i32, i32]),
    "it_block_pool_new": (i32, [i64, i32, PP]),
    "it_block_pool_new_ordered": (i32, [P, i64, i32, PP]),
    "it_block_pool_destroy": (None, [P]),
    "it_block_pool_allocate": (i64, [P]),
    "it_block_pool_share": (i32, [P, i64]),
    "it_block_pool_free": (i32, [P, i64]),
    "it_block_pool_quant_type": (i32, [P]),
    "it_block_pool_num_free": (i64, [P]),
    "it_block_pool_capacity": (i64, [P]),
    "it_block_pool_ref_count": (i64, [P, i64]),
    "it_kv_manager_new": (i32, [P, i32, i32, i32, i32, PP]),
    "it_kv_manager_destroy": (None, [P]),
    "it_kv_manager_seed_seq": (i32, [P, i32, i64, i64, P, i32]),
    "it_kv_manager_step": (i32, [P, P, P, i32, C.POINTER(StepPlanC)]),
    "it_kv_manager_append": (i32, [P, P, P, i32, P, P, i32, P]),
    "it_kv_manager_release_seq": (i32, [P, i32, P, i32, P]),
    "it_kv_manager_fork": (i32, [P, i32, i32]),
    "it_kv_manager_append_cow": (i32, [P, P, P, i32, P, P, i32, P, P, P, i32, P]),
    "it_kv_manager_tables": (i32, [P, P, i32, P, P]),
    "it_kv_page_bytes": (i64, [i32, i32, i32]),
    "it_kv_cache_new": (i32, [i32, i64, i32, i32, i32, i32, PP]),
    "it_kv_cache_wrap": (i32, [i32, P, P, i64, i32, i32, i32, i32, PP]),
    "it_kv_cache_new_layers": (i32, [i32, i32, i64, i32, i32, i32, i32, PP]),
    "it_kv_cache_wrap_layers": (i32, [i32, i32, P, P, i64, i32, i32, i32, i32, PP]),
    "it_kv_cache_layer": (i32, [P, i32, PP]),
    "it_kv_cache_destroy": (i32, [P]),
    "it_kv_cache_describe": (i32, [P, C.POINTER(CacheDesc)]),
    "it_kv_cache_check": (i32, [P, P]),
    "it_kv_append": (i32, [P, P, P, i32, P, i32, P]),
    "it_kv_gather": (i32, [P, P, i32, P, P, P, i32, i32, P, P, P]),
    "it_kv_evict": (i32, [P, P, i32, P]),
    "it_kv_copy_blocks": (i32, [P, P, P, i32, P]),
    "it_rope_table_new": (i32, [i32, i32, f32, i32, PP]),
    "it_rope_table_destroy": (i32, [P]),
    "it_kv_append_rope": (i32, [P, P, P, i32, P, P, P, P, i32, P, i32, P]),
    "it_kv_sync_tables": (i32, [P, P, i32, i32, P, P, P, i32, P]),
    "it_paged_decode_workspace": (sz, [i32, i32, i32, i32, i32]),
    "it_paged_decode_partition": (i32, [i32, i32, i32, i32, i32, P, P, i32, i32, P]),
    "it_paged_decode": (i32, [P, P, i32, i32, P, i32, P, P, i32, i32, f32, i32, P, sz, P, i32, P]),
    "it_paged_decode_split": (i32, [P, P, i32, i32, P, i32, P, P, i32, i32, f32, i32, P, sz, P, i32, P]),
    "it_paged_decode_combine": (i32, [P, P, i32, i32, P, i32, P, P, i32, i32, f32, i32, P, sz, P, i32, P]),
    "it_paged_decode_noalloc": (i32, [P, P, i32, i32, P, i32, P, P, i32, i32, f32, i32, P, i32, P]),
    "it_paged_prefill": (i32, [P, P, i32, i32, P, i32, P, i32, P, i32, f32, i32, P, i32, P]),
    "it_flash_attention_workspace": (sz, [i32, i32, i32]),
    "it_flash_attention": (i32, [P, P, P, P, P, i32, i32, i32, P, sz, P]),
}


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(there is no CPU fallback for the KV-cache kernels)")
    # One HIP runtime per process.  torch ships its own libamdhip64 and asks
    # for it as "libamdhip64.so"; this library asks for "libamdhip64.so.7".
    # If this library loaded first, torch would map a second runtime next to
    # /opt/rocm's, and whichever came second sees no device.  Loading torch
    # first makes the dynamic loader satisfy "libamdhip64.so.7" with torch's
    # copy (same SONAME), so device pointers and streams are shared.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(rc: int) -> None:
    """Raise the OpError subclass for a non-OK status."""
    if rc != OK:
        msg = lib.it_last_error().decode(errors="replace")
        raise _CLASSES.get(rc, OpError)(rc, msg)
