"""Host-side block allocator: mirror of the reference's `memory::paged`
(src/memory/paged.rs:9-58), backed by the native implementation in
libit_kv.so (it_block_pool_*)."""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import numpy as np

from ._lib import BLOCK_SIZE, F32, check, lib

__all__ = ["BLOCK_SIZE", "BlockPool"]


class BlockPool:
    """Refcounted LIFO free-list of KV blocks (paged.rs:21-58).

    `BlockPool(capacity, quant_type)` starts with free list 0..capacity-1, so
    the first `allocate()` returns capacity-1 (Vec::pop takes the last
    element).  `order=` installs a permutation as the free list instead
    (bottom to top).  `free` of a block whose refcount is already 0 raises
    InvalidInput where the reference would underflow a u32.
    """

    def __init__(self, capacity: int, quant_type: int = F32, order: Optional[Sequence[int]] = None):
        h = C.c_void_p()
        if order is None:
            check(lib.it_block_pool_new(int(capacity), int(quant_type), C.byref(h)))
        else:
            arr = np.ascontiguousarray(np.asarray(order, dtype=np.int64))
            if arr.size != capacity:
                raise ValueError("order must have `capacity` entries")
            check(lib.it_block_pool_new_ordered(arr.ctypes.data, int(capacity), int(quant_type), C.byref(h)))
        self._h = h
        self._destroy = lib.it_block_pool_destroy  # bound now: module globals may be gone at exit

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def allocate(self) -> Optional[int]:  # paged.rs:36-42
        r = lib.it_block_pool_allocate(self._h)
        return None if r < 0 else int(r)

    def share(self, block_id: int) -> None:  # paged.rs:44-46
        check(lib.it_block_pool_share(self._h, int(block_id)))

    def free(self, block_id: int) -> None:  # paged.rs:48-53
        check(lib.it_block_pool_free(self._h, int(block_id)))

    def quant_type(self) -> int:  # paged.rs:55-57
        return int(lib.it_block_pool_quant_type(self._h))

    def num_free(self) -> int:
        return int(lib.it_block_pool_num_free(self._h))

    def capacity(self) -> int:
        return int(lib.it_block_pool_capacity(self._h))

    def ref_count(self, block_id: int) -> int:
        return int(lib.it_block_pool_ref_count(self._h, int(block_id)))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._destroy(h)
            self._h = None
