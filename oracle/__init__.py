"""CPU oracle for the KV-cache hot path -- TEST INFRASTRUCTURE ONLY.

numpy-level ctypes binding of oracle/liboracle.so, the plain-C restatement of
the reference crate's CPU arithmetic (see it_oracle.h for the file:line each
function follows).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this package; the product (infer_train_amd)
never does.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, BF16 = 0, 1, 2, 3, 6, 7, 8, 30
QK8_0 = 32
BLOCK_Q8_0_BYTES = 34
QK4_0 = 32
BLOCK_Q4_0_BYTES = 18
QK4_1 = 32
BLOCK_Q4_1_BYTES = 20
QK5_0 = QK5_1 = 32
BLOCK_Q5_0_BYTES = 22
BLOCK_Q5_1_BYTES = 24
QUANT_TYPES = (Q8_0, Q4_0, Q4_1, Q5_0, Q5_1)


class CacheDesc(C.Structure):
    _fields_ = [("num_blocks", C.c_int64), ("block_size", C.c_int32), ("n_kv_heads", C.c_int32),
                ("head_dim", C.c_int32), ("dtype", C.c_int32)]


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} missing: run `make -C oracle`")
    lib = C.CDLL(LIB_PATH)
    P, i32, i64, f32, sz, u64 = C.c_void_p, C.c_int32, C.c_int64, C.c_float, C.c_size_t, C.c_uint64
    sig = {
        "orc_fill_normal_f32": (None, [u64, P, sz]),
        "orc_fill_uniform_i32": (None, [u64, i32, i32, P, sz]),
        "orc_permutation_i64": (None, [u64, P, sz]),
        "orc_f32_to_f16": (C.c_uint16, [f32]),
        "orc_f16_to_f32": (f32, [C.c_uint16]),
        "orc_f32_to_bf16": (C.c_uint16, [f32]),
        "orc_bf16_to_f32": (f32, [C.c_uint16]),
        "orc_f32_to_bf16_array": (None, [P, P, sz]),
        "orc_bf16_to_f32_array": (None, [P, P, sz]),
        "orc_f32_to_f16_array": (None, [P, P, sz]),
        "orc_f16_to_f32_array": (None, [P, P, sz]),
        "orc_pool_new": (P, [i64, i32]),
        "orc_pool_new_ordered": (P, [P, i64, i32]),
        "orc_pool_destroy": (None, [P]),
        "orc_pool_allocate": (i64, [P]),
        "orc_pool_share": (i32, [P, i64]),
        "orc_pool_free": (i32, [P, i64]),
        "orc_pool_quant_type": (i32, [P]),
        "orc_pool_num_free": (i64, [P]),
        "orc_pool_ref_count": (i64, [P, i64]),
        "orc_pool_free_list": (None, [P, P]),
        "orc_quantize_row_q8_0": (i32, [P, sz, P]),
        "orc_dequantize_row_q8_0": (None, [P, sz, P]),
        "orc_quantize_row_q4_0": (i32, [P, sz, P]),
        "orc_dequantize_row_q4_0": (None, [P, sz, P]),
        "orc_quantize_row_q4_1": (i32, [P, sz, P]),
        "orc_dequantize_row_q4_1": (None, [P, sz, P]),
        "orc_quantize_row_q5_0": (i32, [P, sz, P]),
        "orc_dequantize_row_q5_0": (None, [P, sz, P]),
        "orc_quantize_row_q5_1": (i32, [P, sz, P]),
        "orc_dequantize_row_q5_1": (None, [P, sz, P]),
        "orc_rope_f32": (i32, [P, P, sz, i64, i32, i32, f32]),
        "orc_flash_attn_f32": (None, [P, P, P, P, P, i32, i32, f32]),
        "orc_backend_flash_attention": (i32, [P, P, P, P, P, i32, i32, i32]),
        "orc_page_bytes": (sz, [P]),
        "orc_kv_append": (i32, [P, P, P, P, P, P, i32]),
        "orc_kv_gather": (i32, [P, P, P, P, i32, P, P, P, i32, P, P]),
        "orc_kv_evict": (i32, [P, P, P, P, i32]),
        "orc_paged_decode": (i32, [P, P, P, P, i32, P, i32, P, P, i32, f32, P]),
        "orc_paged_decode_mt": (i32, [P, P, P, P, i32, P, i32, P, P, i32, f32, P, i32]),
        "orc_paged_prefill_rows_mt": (i32, [P, P, P, P, i32, P, P, i32, P, i32, i32, i32, f32, i32, P, i32]),
        "orc_paged_prefill": (i32, [P, P, P, P, i32, P, P, i32, P, i32, f32, i32, P]),
        "orc_paged_prefill_rows": (i32, [P, P, P, P, i32, P, P, i32, P, i32, i32, i32, f32, i32, P]),
        "orc_mgr_new": (P, [P, i32, i32, i32, i32]),
        "orc_mgr_destroy": (None, [P]),
        "orc_mgr_seed_seq": (i32, [P, i32, i64, i64, P, i32]),
        "orc_mgr_append": (i32, [P, P, P, i32, P, P, i32, P]),
        "orc_mgr_append_cow": (i32, [P, P, P, i32, i32, P, P, i32, P, P, P, i32, P]),
        "orc_mgr_fork": (i32, [P, i32, i32]),
        "orc_mgr_release": (i32, [P, i32, P, i32, P]),
        "orc_mgr_tables": (i32, [P, P, i32, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=dtype))


# ---- seeded inputs ---------------------------------------------------------
def normal(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib.orc_fill_normal_f32(seed, out.ctypes.data, n)
    return out


def uniform_i32(seed: int, lo: int, hi: int, n: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    lib.orc_fill_uniform_i32(seed, lo, hi, out.ctypes.data, n)
    return out


def permutation(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.int64)
    lib.orc_permutation_i64(seed, out.ctypes.data, n)
    return out


# ---- conversions -------------------------------------------------------------
def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib.orc_f32_to_bf16_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib.orc_bf16_to_f32_array(h.ctypes.data, out.ctypes.data, h.size)
    return out


def f32_to_f16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib.orc_f32_to_f16_array(x.ctypes.data, out.ctypes.data, x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib.orc_f16_to_f32_array(h.ctypes.data, out.ctypes.data, h.size)
    return out


# ---- BlockPool (paged.rs:21-58) ---------------------------------------------
class Pool:
    def __init__(self, capacity: int, quant_type: int = F32, order: Optional[Sequence[int]] = None):
        if order is None:
            self.h = lib.orc_pool_new(capacity, quant_type)
        else:
            o = _c(order, np.int64)
            self.h = lib.orc_pool_new_ordered(o.ctypes.data, capacity, quant_type)

    def allocate(self) -> Optional[int]:
        r = lib.orc_pool_allocate(self.h)
        return None if r < 0 else int(r)

    def share(self, i: int) -> int:
        return lib.orc_pool_share(self.h, i)

    def free(self, i: int) -> int:
        return lib.orc_pool_free(self.h, i)

    def quant_type(self) -> int:
        return lib.orc_pool_quant_type(self.h)

    def num_free(self) -> int:
        return int(lib.orc_pool_num_free(self.h))

    def ref_count(self, i: int) -> int:
        return int(lib.orc_pool_ref_count(self.h, i))

    def free_list(self) -> np.ndarray:
        out = np.empty(max(self.num_free(), 1), np.int64)
        lib.orc_pool_free_list(self.h, out.ctypes.data)
        return out[: self.num_free()]

    def __del__(self):
        if getattr(self, "h", None):
            lib.orc_pool_destroy(self.h)
            self.h = None


# ---- Q8_0 (quant.rs:149-183) -------------------------------------------------
def quantize_row_q8_0(x) -> np.ndarray:
    """x: f32[n], n % 32 == 0 -> uint8[n/32, 34] packed BlockQ8_0 records."""
    x = _c(x, np.float32).ravel()
    out = np.empty((x.size // QK8_0, BLOCK_Q8_0_BYTES), np.uint8)
    rc = lib.orc_quantize_row_q8_0(x.ctypes.data, x.size, out.ctypes.data)
    if rc:
        raise ValueError("length not a multiple of 32")
    return out


def rope(x, pos: int, n_dims: int, head_dim: int, freq_base: float = 10000.0) -> np.ndarray:
    """rope_f32 (rope.rs:6-44) of f32 x (any shape whose size is a multiple
    of head_dim) at one position."""
    x = _c(x, np.float32)
    out = np.empty_like(x)
    rc = lib.orc_rope_f32(x.ctypes.data, out.ctypes.data, x.size, int(pos), n_dims, head_dim, C.c_float(freq_base))
    if rc:
        raise ValueError("orc_rope_f32: invalid shape")
    return out


def rope_rows(x, positions, n_dims: int, head_dim: int, freq_base: float = 10000.0) -> np.ndarray:
    """rope_f32 of x[t] at positions[t] for every leading index t."""
    x = _c(x, np.float32)
    out = np.empty_like(x)
    for t, p in enumerate(np.asarray(positions).ravel()):
        out[t] = rope(x[t], int(p), n_dims, head_dim, freq_base)
    return out


def dequantize_row_q8_0(y) -> np.ndarray:
    y = _c(y, np.uint8)
    n = y.size // BLOCK_Q8_0_BYTES * QK8_0
    out = np.empty(n, np.float32)
    lib.orc_dequantize_row_q8_0(y.ctypes.data, n, out.ctypes.data)
    return out


# ---- Q4_0 (block types.rs:15-22, dequant vec_dot.rs:425-440; quantiser = ----
# ---- ggml's quantize_row_q4_0_ref, which the reference does not carry) -------
def quantize_row_q4_0(x) -> np.ndarray:
    """x: f32[n], n % 32 == 0 -> uint8[n/32, 18] packed BlockQ4_0 records."""
    x = _c(x, np.float32).ravel()
    out = np.empty((x.size // QK4_0, BLOCK_Q4_0_BYTES), np.uint8)
    if lib.orc_quantize_row_q4_0(x.ctypes.data, x.size, out.ctypes.data):
        raise ValueError("length not a multiple of 32")
    return out


def dequantize_row_q4_0(y) -> np.ndarray:
    y = _c(y, np.uint8)
    n = y.size // BLOCK_Q4_0_BYTES * QK4_0
    out = np.empty(n, np.float32)
    lib.orc_dequantize_row_q4_0(y.ctypes.data, n, out.ctypes.data)
    return out


# ---- Q4_1 (block types.rs:24-32; quantiser and dequantiser = ggml's, which ---
# ---- the reference does not carry) ---------------------------------------------
def quantize_row_q4_1(x) -> np.ndarray:
    """x: f32[n], n % 32 == 0 -> uint8[n/32, 20] packed BlockQ4_1 records."""
    x = _c(x, np.float32).ravel()
    out = np.empty((x.size // QK4_1, BLOCK_Q4_1_BYTES), np.uint8)
    if lib.orc_quantize_row_q4_1(x.ctypes.data, x.size, out.ctypes.data):
        raise ValueError("length not a multiple of 32")
    return out


def dequantize_row_q4_1(y) -> np.ndarray:
    y = _c(y, np.uint8)
    n = y.size // BLOCK_Q4_1_BYTES * QK4_1
    out = np.empty(n, np.float32)
    lib.orc_dequantize_row_q4_1(y.ctypes.data, n, out.ctypes.data)
    return out


# ---- Q5_0 / Q5_1 (type ids types.rs:116-117; blocks, quantisers and ------------
# ---- dequantisers = ggml's, which the reference does not carry) ----------------
def quantize_row_q5_0(x) -> np.ndarray:
    """x: f32[n], n % 32 == 0 -> uint8[n/32, 22] packed block_q5_0 records."""
    x = _c(x, np.float32).ravel()
    out = np.empty((x.size // QK5_0, BLOCK_Q5_0_BYTES), np.uint8)
    if lib.orc_quantize_row_q5_0(x.ctypes.data, x.size, out.ctypes.data):
        raise ValueError("length not a multiple of 32")
    return out


def dequantize_row_q5_0(y) -> np.ndarray:
    y = _c(y, np.uint8)
    n = y.size // BLOCK_Q5_0_BYTES * QK5_0
    out = np.empty(n, np.float32)
    lib.orc_dequantize_row_q5_0(y.ctypes.data, n, out.ctypes.data)
    return out


def quantize_row_q5_1(x) -> np.ndarray:
    """x: f32[n], n % 32 == 0 -> uint8[n/32, 24] packed block_q5_1 records."""
    x = _c(x, np.float32).ravel()
    out = np.empty((x.size // QK5_1, BLOCK_Q5_1_BYTES), np.uint8)
    if lib.orc_quantize_row_q5_1(x.ctypes.data, x.size, out.ctypes.data):
        raise ValueError("length not a multiple of 32")
    return out


def dequantize_row_q5_1(y) -> np.ndarray:
    y = _c(y, np.uint8)
    n = y.size // BLOCK_Q5_1_BYTES * QK5_1
    out = np.empty(n, np.float32)
    lib.orc_dequantize_row_q5_1(y.ctypes.data, n, out.ctypes.data)
    return out


RECORD_BYTES = {Q8_0: BLOCK_Q8_0_BYTES, Q4_0: BLOCK_Q4_0_BYTES, Q4_1: BLOCK_Q4_1_BYTES, Q5_0: BLOCK_Q5_0_BYTES,
                Q5_1: BLOCK_Q5_1_BYTES}


def dequantize_records(y, dtype: int) -> np.ndarray:
    """Packed records of any quantised dtype -> f32 values."""
    return {Q8_0: dequantize_row_q8_0, Q4_0: dequantize_row_q4_0, Q4_1: dequantize_row_q4_1,
            Q5_0: dequantize_row_q5_0, Q5_1: dequantize_row_q5_1}[dtype](y)


# ---- attention (flash_attn.rs:6-72, arm.rs:304-370) ----------------------------
def flash_attn_f32(q, k, v, scale: float, mask=None) -> np.ndarray:
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    D = q.size
    n_kv = k.size // D
    m = None if mask is None else _c(mask, np.float32)
    out = np.empty(D, np.float32)
    lib.orc_flash_attn_f32(q.ctypes.data, k.ctypes.data, v.ctypes.data, _p(m), out.ctypes.data, D, n_kv,
                           C.c_float(scale))
    return out


def backend_flash_attention(q, k, v, mask=None) -> np.ndarray:
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    n_heads, D = q.shape
    n_kv = k.shape[0]
    m = None if mask is None else _c(mask, np.float32)
    out = np.empty_like(q)
    rc = lib.orc_backend_flash_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data, _p(m), out.ctypes.data,
                                         n_heads, D, n_kv)
    if rc:
        raise ValueError("invalid input")
    return out


# ---- paged cache ----------------------------------------------------------------
class Cache:
    """Host restatement of the paged pools (same byte layout as the device)."""

    def __init__(self, num_blocks: int, block_size: int, n_kv_heads: int, head_dim: int, dtype: int):
        self.desc = CacheDesc(num_blocks, block_size, n_kv_heads, head_dim, dtype)
        self.page_bytes = int(lib.orc_page_bytes(C.byref(self.desc)))
        n = num_blocks * n_kv_heads * self.page_bytes
        self.k = np.zeros(n, np.uint8)
        self.v = np.zeros(n, np.uint8)

    def _d(self):
        return C.byref(self.desc)

    def append(self, k, v, slots) -> None:
        src_dt = np.float32 if self.desc.dtype in (F32,) + QUANT_TYPES else np.uint16
        k, v, s = _c(k, src_dt), _c(v, src_dt), _c(slots, np.int64)
        rc = lib.orc_kv_append(self._d(), self.k.ctypes.data, self.v.ctypes.data, k.ctypes.data, v.ctypes.data,
                               s.ctypes.data, s.size)
        if rc:
            raise ValueError("orc_kv_append: invalid input")

    def row_out_bytes(self) -> int:
        D = self.desc.head_dim
        if self.desc.dtype == Q8_0:
            return D // QK8_0 * BLOCK_Q8_0_BYTES
        if self.desc.dtype == Q4_0:
            return D // QK4_0 * BLOCK_Q4_0_BYTES
        if self.desc.dtype in RECORD_BYTES:
            return D // 32 * RECORD_BYTES[self.desc.dtype]
        return D * (4 if self.desc.dtype == F32 else 2)

    def gather(self, tables, ctx_lens, start_pos, cu_out, n_out_tokens) -> Tuple[np.ndarray, np.ndarray]:
        t, cl = _c(tables, np.int32), _c(ctx_lens, np.int32)
        sp = None if start_pos is None else _c(start_pos, np.int32)
        cu = _c(cu_out, np.int64)
        nb = n_out_tokens * self.desc.n_kv_heads * self.row_out_bytes()
        ko, vo = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
        rc = lib.orc_kv_gather(self._d(), self.k.ctypes.data, self.v.ctypes.data, t.ctypes.data, t.shape[1],
                               cl.ctypes.data, _p(sp), cu.ctypes.data, cl.size, ko.ctypes.data, vo.ctypes.data)
        if rc:
            raise ValueError("orc_kv_gather: invalid input")
        return ko, vo

    def evict(self, blocks) -> None:
        b = _c(blocks, np.int32)
        if lib.orc_kv_evict(self._d(), self.k.ctypes.data, self.v.ctypes.data, b.ctypes.data, b.size):
            raise ValueError("orc_kv_evict: invalid input")

    def decode(self, q, n_heads, tables, ctx_lens, start_pos, scale, threads: int = 1) -> np.ndarray:
        """threads > 1: the same results on that many host threads (the
        all-cores CPU baseline)."""
        q = _c(q, np.float32)
        t, cl = _c(tables, np.int32), _c(ctx_lens, np.int32)
        sp = None if start_pos is None else _c(start_pos, np.int32)
        out = np.zeros_like(q)
        if threads > 1:
            rc = lib.orc_paged_decode_mt(self._d(), self.k.ctypes.data, self.v.ctypes.data, q.ctypes.data, n_heads,
                                         t.ctypes.data, t.shape[1], cl.ctypes.data, _p(sp), cl.size,
                                         C.c_float(scale), out.ctypes.data, threads)
        else:
            rc = lib.orc_paged_decode(self._d(), self.k.ctypes.data, self.v.ctypes.data, q.ctypes.data, n_heads,
                                      t.ctypes.data, t.shape[1], cl.ctypes.data, _p(sp), cl.size, C.c_float(scale),
                                      out.ctypes.data)
        if rc:
            raise ValueError("orc_paged_decode: invalid input")
        return out

    def prefill(self, q, n_heads, cu_q, tables, ctx_lens, scale, causal=True, rows=None, threads: int = 1) -> np.ndarray:
        """rows=(seq, begin, end) restricts the work to one sequence's rows
        (threads > 1: on that many host threads, same results)."""
        q = _c(q, np.float32)
        cq, t, cl = _c(cu_q, np.int32), _c(tables, np.int32), _c(ctx_lens, np.int32)
        out = np.zeros_like(q)
        if rows is None:
            rc = lib.orc_paged_prefill(self._d(), self.k.ctypes.data, self.v.ctypes.data, q.ctypes.data, n_heads,
                                       cq.ctypes.data, t.ctypes.data, t.shape[1], cl.ctypes.data, cl.size,
                                       C.c_float(scale), int(causal), out.ctypes.data)
        else:
            s, b, e = rows
            if threads > 1:
                rc = lib.orc_paged_prefill_rows_mt(self._d(), self.k.ctypes.data, self.v.ctypes.data, q.ctypes.data,
                                                   n_heads, cq.ctypes.data, t.ctypes.data, t.shape[1],
                                                   cl.ctypes.data, s, b, e, C.c_float(scale), int(causal),
                                                   out.ctypes.data, threads)
            else:
                rc = lib.orc_paged_prefill_rows(self._d(), self.k.ctypes.data, self.v.ctypes.data, q.ctypes.data,
                                                n_heads, cq.ctypes.data, t.ctypes.data, t.shape[1], cl.ctypes.data,
                                                s, b, e, C.c_float(scale), int(causal), out.ctypes.data)
        if rc:
            raise ValueError("orc_paged_prefill: invalid input")
        return out


class Manager:
    def __init__(self, pool: Pool, block_size: int, max_seqs: int, max_blocks: int, window: int = 0):
        self.pool = pool
        self.max_seqs, self.max_blocks = max_seqs, max_blocks
        self.h = lib.orc_mgr_new(pool.h, block_size, max_seqs, max_blocks, window)

    def seed_seq(self, s, pos, first_block, blocks) -> None:
        b = _c(blocks, np.int32)
        if lib.orc_mgr_seed_seq(self.h, s, pos, first_block, b.ctypes.data, b.size):
            raise ValueError("seed_seq")

    def append(self, seqs, n_tokens=1, cow: bool = False):
        """Slots and the blocks returned to the pool (refcount 0) of one step;
        cow=True also returns the copy-on-write (shared, fresh) pairs."""
        s = _c(seqs, np.int32)
        nt = np.full(s.size, n_tokens, np.int32) if np.isscalar(n_tokens) else _c(n_tokens, np.int32)
        slots = np.empty(max(int(nt.sum()), 1), np.int64)
        cap = s.size * self.max_blocks + 1
        ev = np.empty(cap, np.int32)
        ne = C.c_int32(0)
        cs, cd, nc = np.empty(cap, np.int32), np.empty(cap, np.int32), C.c_int32(0)
        rc = lib.orc_mgr_append_cow(self.h, s.ctypes.data, nt.ctypes.data, s.size, int(cow), slots.ctypes.data,
                                    ev.ctypes.data, cap, C.byref(ne), cs.ctypes.data, cd.ctypes.data, cap,
                                    C.byref(nc))
        if rc:
            raise ValueError("orc_mgr_append failed")
        if cow:
            return slots[: int(nt.sum())], ev[: ne.value].copy(), cs[: nc.value].copy(), cd[: nc.value].copy()
        return slots[: int(nt.sum())], ev[: ne.value].copy()

    def fork(self, src: int, dst: int) -> None:
        if lib.orc_mgr_fork(self.h, src, dst):
            raise ValueError("orc_mgr_fork failed")

    def release(self, s: int) -> np.ndarray:
        ev = np.empty(self.max_blocks, np.int32)
        ne = C.c_int32(0)
        if lib.orc_mgr_release(self.h, s, ev.ctypes.data, self.max_blocks, C.byref(ne)):
            raise ValueError("orc_mgr_release failed")
        return ev[: ne.value].copy()

    def tables(self):
        t = np.empty((self.max_seqs, self.max_blocks), np.int32)
        cl = np.empty(self.max_seqs, np.int32)
        sp = np.empty(self.max_seqs, np.int32)
        lib.orc_mgr_tables(self.h, t.ctypes.data, self.max_blocks, cl.ctypes.data, sp.ctypes.data)
        return t, cl, sp

    def __del__(self):
        if getattr(self, "h", None):
            lib.orc_mgr_destroy(self.h)
            self.h = None
