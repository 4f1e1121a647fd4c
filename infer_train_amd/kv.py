"""Device-side KV cache and attention entry points.

Thin wrappers that pass torch tensors' device pointers and the current HIP
stream to libit_kv.so.  torch only provides device memory and streams; all
work runs in the library's gfx950 kernels.  Shapes follow include/it_kv.h.
"""
from __future__ import annotations

import ctypes as C
import math
from typing import Optional, Tuple

import torch

from ._lib import BF16, CacheDesc, F16, F32, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, check, lib

__all__ = ["PagedKvCache", "RopeTable", "flash_attention", "torch_dtype_id", "stream_handle"]

_TORCH_IDS = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
_ID_TORCH = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}


def torch_dtype_id(t: torch.dtype) -> int:
    try:
        return _TORCH_IDS[t]
    except KeyError:
        raise TypeError(f"unsupported dtype {t}") from None


def stream_handle(device: Optional[torch.device] = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("device tensor expected")
    if not t.is_contiguous():
        raise ValueError("contiguous tensor expected")
    return t.data_ptr()


class RopeTable:
    """cos/sin of rope_f32's angles (src/backend/arm/rope.rs:30-34) for
    positions [0, max_pos), built on the host in float32 and held on the
    device (it_rope_table_new)."""

    def __init__(self, n_dims: int, max_pos: int, freq_base: float = 10000.0, device: int = 0):
        h = C.c_void_p()
        check(lib.it_rope_table_new(device, n_dims, C.c_float(freq_base), max_pos, C.byref(h)))
        self._h = h
        self.n_dims, self.max_pos, self.freq_base, self.device = n_dims, max_pos, freq_base, device
        self._destroy = lib.it_rope_table_destroy

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._destroy(h)
            self._h = None


class PagedKvCache:
    """Paged K/V pools in HBM, [num_blocks][n_kv_heads] pages of block_size
    token rows (Q8_0 pages: int8 rows then fp16 group scales; Q4_0 pages:
    rows of BlockQ4_0 nibble bytes then fp16 group scales; Q4_1 the same
    with (d, m) pairs; Q5_0 / Q5_1 the nibble rows then per token the
    groups' u32 qh words and their d or (d, m)).

    n_layers > 1 holds every layer of a model (the reference's per-layer
    kv_cache_k/v, forward.rs:17-18): each pool is n_layers such layers one
    after another, so one block id names the same pages in every layer.
    evict / copy_blocks / sync_tables act on the whole cache (every layer in
    one launch); append, gather, decode and prefill go through `layer(l)`."""

    def __init__(self, num_blocks: int, block_size: int, n_kv_heads: int, head_dim: int, dtype: int = BF16,
                 device: int = 0, n_layers: int = 1):
        page = lib.it_kv_page_bytes(block_size, head_dim, dtype)
        if page <= 0:
            raise ValueError("unsupported cache shape")
        nbytes = n_layers * num_blocks * n_kv_heads * page
        dev = torch.device("cuda", device)
        self.k_pool = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        self.v_pool = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        h = C.c_void_p()
        check(lib.it_kv_cache_wrap_layers(device, n_layers, self.k_pool.data_ptr(), self.v_pool.data_ptr(),
                                          num_blocks, block_size, n_kv_heads, head_dim, dtype, C.byref(h)))
        self._h = h
        # Bound now: at interpreter exit the module global may already be gone.
        self._destroy = lib.it_kv_cache_destroy
        self.num_blocks, self.block_size, self.n_kv_heads, self.head_dim = num_blocks, block_size, n_kv_heads, head_dim
        self.dtype = dtype
        self.page_bytes = page
        self.device = dev
        self.n_layers = n_layers
        self._parent = None

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def layer(self, index: int) -> "PagedKvCache":
        """One layer of a multi-layer cache (it_kv_cache_layer): a cache
        object whose pools are that layer's bytes of this cache's pools."""
        h = C.c_void_p()
        check(lib.it_kv_cache_layer(self._h, int(index), C.byref(h)))
        view = object.__new__(PagedKvCache)
        lb = self.num_blocks * self.n_kv_heads * self.page_bytes
        view.k_pool = self.k_pool[index * lb:(index + 1) * lb]
        view.v_pool = self.v_pool[index * lb:(index + 1) * lb]
        view._h = h
        view._destroy = lib.it_kv_cache_destroy
        for name in ("num_blocks", "block_size", "n_kv_heads", "head_dim", "dtype", "page_bytes", "device"):
            setattr(view, name, getattr(self, name))
        view.n_layers = 1
        view._parent = self  # destroyed before the parent
        return view

    def _one_layer(self) -> None:
        if self.n_layers != 1:
            raise TypeError("a multi-layer cache: take one layer's view with layer(l)")

    def describe(self) -> CacheDesc:
        d = CacheDesc()
        check(lib.it_kv_cache_describe(self._h, C.byref(d)))
        return d

    def view(self, which: str = "k") -> torch.Tensor:
        """Typed view [num_blocks, n_kv_heads, block_size, head_dim] (F32/F16/BF16)."""
        self._one_layer()
        pool = self.k_pool if which == "k" else self.v_pool
        if self.dtype == Q8_0:
            raise TypeError("use q8_planes() for a Q8_0 cache")
        if self.dtype in (Q4_0, Q4_1, Q5_0, Q5_1):
            raise TypeError("use q4_planes() for a Q4_0 / Q4_1 cache, q5_planes() for Q5_0 / Q5_1")
        return pool.view(_ID_TORCH[self.dtype]).view(self.num_blocks, self.n_kv_heads, self.block_size, self.head_dim)

    def q8_planes(self, which: str = "k") -> Tuple[torch.Tensor, torch.Tensor]:
        """(qs int8 [nb, H, bs, D], d fp16 bits int16 [nb, H, bs, D/32]) of a Q8_0 cache."""
        self._one_layer()
        pool = (self.k_pool if which == "k" else self.v_pool).view(self.num_blocks, self.n_kv_heads, self.page_bytes)
        bs, D = self.block_size, self.head_dim
        qs = pool[:, :, : bs * D].view(torch.int8).reshape(self.num_blocks, self.n_kv_heads, bs, D)
        d = pool[:, :, bs * D:].contiguous().view(torch.int16).reshape(self.num_blocks, self.n_kv_heads, bs, D // 32)
        return qs, d

    def q4_planes(self, which: str = "k") -> Tuple[torch.Tensor, torch.Tensor]:
        """(qs uint8 [nb, H, bs, D/2], scales fp16 bits int16 [nb, H, bs, D/32] (Q4_0: d) or
        [nb, H, bs, D/32, 2] (Q4_1: d, m)) of a Q4_0 / Q4_1 cache."""
        self._one_layer()
        pool = (self.k_pool if which == "k" else self.v_pool).view(self.num_blocks, self.n_kv_heads, self.page_bytes)
        bs, D = self.block_size, self.head_dim
        qs = pool[:, :, : bs * D // 2].reshape(self.num_blocks, self.n_kv_heads, bs, D // 2)
        shape = (self.num_blocks, self.n_kv_heads, bs, D // 32) + ((2,) if self.dtype == Q4_1 else ())
        d = pool[:, :, bs * D // 2:].contiguous().view(torch.int16).reshape(shape)
        return qs, d

    def q5_planes(self, which: str = "k") -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(qs uint8 [nb, H, bs, D/2] (low four bits of each value), qh int32
        [nb, H, bs, D/32], scales fp16 bits int16 [nb, H, bs, D/32] (Q5_0: d) or
        [nb, H, bs, D/32, 2] (Q5_1: d, m)) of a Q5_0 / Q5_1 cache."""
        self._one_layer()
        if self.dtype not in (Q5_0, Q5_1):
            raise TypeError("q5_planes() needs a Q5_0 / Q5_1 cache")
        pool = (self.k_pool if which == "k" else self.v_pool).view(self.num_blocks, self.n_kv_heads, self.page_bytes)
        bs, D = self.block_size, self.head_dim
        ng, mb = D // 32, 4 if self.dtype == Q5_1 else 2
        nb, H = self.num_blocks, self.n_kv_heads
        qs = pool[:, :, : bs * D // 2].reshape(nb, H, bs, D // 2)
        side = pool[:, :, bs * D // 2:].reshape(nb, H, bs, ng * (4 + mb))
        qh = side[..., : 4 * ng].contiguous().view(torch.int32)
        shape = (nb, H, bs, ng) + ((2,) if self.dtype == Q5_1 else ())
        d = side[..., 4 * ng:].contiguous().view(torch.int16).reshape(shape)
        return qs, qh, d

    def check(self) -> None:
        """Raise if a kernel latched a device-side range error (syncs the stream)."""
        check(lib.it_kv_cache_check(self._h, stream_handle(self.device)))

    # ---- data movement ----------------------------------------------------
    def append(self, k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """k, v: [n_tokens, n_kv_heads, head_dim]; slot_mapping int64 [n_tokens]."""
        if slot_mapping.dtype != torch.int64:
            raise TypeError("slot_mapping must be int64")
        n = slot_mapping.numel()
        check(lib.it_kv_append(self._h, _ptr(k), _ptr(v), torch_dtype_id(k.dtype), _ptr(slot_mapping), n,
                               stream_handle(self.device)))

    def append_rope(self, rope: RopeTable, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    slot_mapping: torch.Tensor, positions: torch.Tensor, q_out: Optional[torch.Tensor] = None,
                    q_out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """RoPE then append (forward.rs:195-229): q [n_tokens, n_heads, D],
        k, v [n_tokens, n_kv_heads, D] float32; positions int32 [n_tokens].
        Returns the rotated q (float32, or the cache's 16-bit dtype)."""
        if slot_mapping.dtype != torch.int64 or positions.dtype != torch.int32:
            raise TypeError("slot_mapping must be int64 and positions int32")
        if q.dtype != torch.float32 or k.dtype != torch.float32 or v.dtype != torch.float32:
            raise TypeError("q, k, v must be float32")
        if q_out is None:
            q_out = torch.empty(q.shape, dtype=q_out_dtype or torch.float32, device=q.device)
        check(lib.it_kv_append_rope(self._h, rope._h, _ptr(q), q.shape[1], _ptr(k), _ptr(v), _ptr(slot_mapping),
                                    _ptr(positions), slot_mapping.numel(), _ptr(q_out),
                                    torch_dtype_id(q_out.dtype), stream_handle(self.device)))
        return q_out

    def gather(self, block_tables: torch.Tensor, ctx_lens: torch.Tensor, start_pos: Optional[torch.Tensor],
               cu_out: torch.Tensor, max_tokens: int, k_out: torch.Tensor, v_out: torch.Tensor) -> None:
        check(lib.it_kv_gather(self._h, _ptr(block_tables), block_tables.shape[1], _ptr(ctx_lens), _ptr(start_pos),
                               _ptr(cu_out), ctx_lens.numel(), max_tokens, _ptr(k_out), _ptr(v_out),
                               stream_handle(self.device)))

    def evict(self, blocks: torch.Tensor) -> None:
        check(lib.it_kv_evict(self._h, _ptr(blocks), blocks.numel(), stream_handle(self.device)))

    def sync_tables(self, tables: torch.Tensor, seq: torch.Tensor, pos: torch.Tensor, slots: torch.Tensor) -> None:
        """tables[seq[i], pos[i] // bs] = slots[i] // bs (device int32 table [n_seqs, max_blocks])."""
        check(lib.it_kv_sync_tables(self._h, _ptr(tables), tables.shape[1], tables.shape[0], _ptr(seq), _ptr(pos),
                                    _ptr(slots), slots.numel(), stream_handle(self.device)))

    def copy_blocks(self, src: torch.Tensor, dst: torch.Tensor) -> None:
        check(lib.it_kv_copy_blocks(self._h, _ptr(src), _ptr(dst), src.numel(), stream_handle(self.device)))

    # ---- attention --------------------------------------------------------
    def decode_workspace(self, n_seqs: int, n_heads: int, max_tokens: int, partition: int = 512) -> torch.Tensor:
        nbytes = lib.it_paged_decode_workspace(n_seqs, n_heads, self.head_dim, max_tokens, partition)
        return torch.empty(nbytes, dtype=torch.uint8, device=self.device)

    def decode_partition(self, n_heads: int, ctx_lens, start_pos=None, n_cu: int = 0) -> int:
        """Partition for a decode over these host-side contexts
        (it_paged_decode_partition)."""
        return decode_partition(self.dtype, self.head_dim, self.block_size, n_heads, self.n_kv_heads, ctx_lens,
                                start_pos, n_cu)

    def decode(self, q: torch.Tensor, block_tables: torch.Tensor, ctx_lens: torch.Tensor,
               start_pos: Optional[torch.Tensor], max_tokens: int, scale: Optional[float] = None,
               partition: int = 512, out: Optional[torch.Tensor] = None, ws: Optional[torch.Tensor] = None,
               out_dtype: Optional[torch.dtype] = None, phase: str = "both") -> torch.Tensor:
        """q: [n_seqs, n_heads, head_dim] -> out [n_seqs, n_heads, head_dim].
        phase "split" / "combine" launches one pass (same arguments)."""
        n_seqs, n_heads, D = q.shape
        if scale is None:
            scale = 1.0 / math.sqrt(D)
        if out is None:
            out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=q.device)
        if ws is None:
            ws = self.decode_workspace(n_seqs, n_heads, max_tokens, partition)
        fn = {"both": lib.it_paged_decode, "split": lib.it_paged_decode_split,
              "combine": lib.it_paged_decode_combine}[phase]
        check(fn(self._h, _ptr(q), torch_dtype_id(q.dtype), n_heads, _ptr(block_tables),
                                  block_tables.shape[1], _ptr(ctx_lens), _ptr(start_pos), n_seqs, max_tokens,
                                  C.c_float(scale), partition, _ptr(ws), ws.numel(), _ptr(out),
                                  torch_dtype_id(out.dtype), stream_handle(self.device)))
        return out

    def prefill(self, q: torch.Tensor, cu_q: torch.Tensor, max_q_len: int, block_tables: torch.Tensor,
                ctx_lens: torch.Tensor, scale: Optional[float] = None, causal: bool = True,
                out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """q: [total_q, n_heads, head_dim] bf16 -> out [total_q, n_heads, head_dim]."""
        total, n_heads, D = q.shape
        if scale is None:
            scale = 1.0 / math.sqrt(D)
        if out is None:
            out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=q.device)
        check(lib.it_paged_prefill(self._h, _ptr(q), torch_dtype_id(q.dtype), n_heads, _ptr(cu_q), max_q_len,
                                   _ptr(block_tables), block_tables.shape[1], _ptr(ctx_lens), ctx_lens.numel(),
                                   C.c_float(scale), int(bool(causal)), _ptr(out), torch_dtype_id(out.dtype),
                                   stream_handle(self.device)))
        return out

    def __del__(self):
        h = getattr(self, "_h", None)
        destroy = getattr(self, "_destroy", None)
        if h is not None and h.value and destroy is not None:
            destroy(h)
            self._h = None


def decode_partition(dtype: int, head_dim: int, block_size: int, n_heads: int, n_kv_heads: int, ctx_lens,
                     start_pos=None, n_cu: int = 0) -> int:
    """Tokens per split for a paged decode over contexts known on the host
    (it_paged_decode_partition): the smallest multiple of 64 whose non-empty
    units run in the fewest rounds of resident workgroups.  n_cu 0 asks the
    current device."""
    import numpy as np

    ctx = np.ascontiguousarray(np.asarray(ctx_lens, dtype=np.int32))
    st = None if start_pos is None else np.ascontiguousarray(np.asarray(start_pos, dtype=np.int32))
    if st is not None and st.shape != ctx.shape:
        raise ValueError("start_pos must match ctx_lens")
    out = C.c_int32()
    check(lib.it_paged_decode_partition(dtype, head_dim, block_size, n_heads, n_kv_heads, ctx.ctypes.data,
                                        None if st is None else st.ctypes.data, ctx.size, n_cu, C.byref(out)))
    return out.value


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """CoreOperator::FlashAttention as ArmCpuBackend runs it (arm.rs:304-370):
    q [n_heads, D] f32, k/v [n_kv, D] f32 shared by all heads, mask [n_kv]."""
    n_heads, D = q.shape
    n_kv = k.shape[0]
    if out is None:
        out = torch.empty_like(q)
    ws = torch.empty(lib.it_flash_attention_workspace(n_heads, D, n_kv), dtype=torch.uint8, device=q.device)
    check(lib.it_flash_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(mask), _ptr(out), n_heads, D, n_kv, _ptr(ws),
                                 ws.numel(), stream_handle(q.device)))
    return out
