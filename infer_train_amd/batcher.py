"""Host-side batch state: the reference's FIFO `ContinuousBatcher`
(src/batcher/continuous.rs:8-74) plus the per-step slot mapping, block
tables and sliding-window eviction it lacks (native: it_kv_manager_*)."""
from __future__ import annotations

import ctypes as C
from collections import deque
from dataclasses import dataclass, field
from enum import Enum
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from ._lib import check, lib
from .memory import BlockPool

__all__ = ["KvManager", "ContinuousBatcher", "RequestState", "RequestContext", "StepPlan"]


@dataclass
class StepPlan:
    """What one append step hands to the device: the slot of every new token,
    the blocks freed by the window (to clear with kv_evict) and the
    copy-on-write page pairs (to copy with kv_copy_blocks before the append)."""

    slots: np.ndarray
    evicted: np.ndarray
    cow_src: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    cow_dst: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    # Sequence and position of every new token (for it_kv_sync_tables).
    token_seq: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    token_pos: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))


class KvManager:
    """Slot mapping and block tables over a BlockPool.

    slot(pos) = table[pos // bs] * bs + pos % bs; a block is allocated when
    pos % bs == 0.  With `window` W > 0, before the token at position p every
    held block whose last position is < p - W + 1 is released (oldest first).
    Sequences of one step are processed in the order listed.
    """

    def __init__(self, pool: BlockPool, block_size: int, max_seqs: int, max_blocks_per_seq: int, window: int = 0):
        self.pool = pool  # keep the borrowed pool alive
        self.block_size = block_size
        self.max_seqs = max_seqs
        self.max_blocks = max_blocks_per_seq
        self.window = window
        h = C.c_void_p()
        check(lib.it_kv_manager_new(pool.handle, block_size, max_seqs, max_blocks_per_seq, window, C.byref(h)))
        self._h = h

    def seed_seq(self, seq: int, pos: int, first_block: int, blocks: Sequence[int]) -> None:
        arr = np.ascontiguousarray(np.asarray(blocks, dtype=np.int32))
        check(lib.it_kv_manager_seed_seq(self._h, seq, int(pos), int(first_block), arr.ctypes.data, arr.size))

    def append(self, seqs: Sequence[int], n_tokens: Sequence[int] | int = 1, cow: bool = False) -> StepPlan:
        seqs_a = np.ascontiguousarray(np.asarray(seqs, dtype=np.int32))
        if np.isscalar(n_tokens):
            nt = np.full(seqs_a.size, int(n_tokens), dtype=np.int32)
        else:
            nt = np.ascontiguousarray(np.asarray(n_tokens, dtype=np.int32))
        total = int(nt.sum())
        before = self.positions()
        token_seq = np.repeat(seqs_a, nt).astype(np.int32)
        # Each token's position: its sequence's position before the call plus
        # the tokens of that sequence listed before it (a sequence may be
        # listed more than once, as the native manager allows).
        token_pos = np.empty(total, dtype=np.int32)
        run = before.astype(np.int64)
        off = 0
        for sq, k in zip(seqs_a.tolist(), nt.tolist()):
            token_pos[off:off + k] = run[sq] + np.arange(k)
            run[sq] += k
            off += k
        slots = np.empty(max(total, 1), dtype=np.int64)
        # Upper bound of frees: every block of every listed sequence.
        cap = int(seqs_a.size * self.max_blocks + 1)
        ev = np.empty(cap, dtype=np.int32)
        nev = C.c_int32(0)
        if cow:
            cs = np.empty(cap, dtype=np.int32)
            cd = np.empty(cap, dtype=np.int32)
            nc = C.c_int32(0)
            check(lib.it_kv_manager_append_cow(self._h, seqs_a.ctypes.data, nt.ctypes.data, seqs_a.size,
                                               slots.ctypes.data, ev.ctypes.data, cap, C.byref(nev),
                                               cs.ctypes.data, cd.ctypes.data, cap, C.byref(nc)))
            return StepPlan(slots[:total], ev[:nev.value].copy(), cs[:nc.value].copy(), cd[:nc.value].copy(),
                            token_seq, token_pos)
        check(lib.it_kv_manager_append(self._h, seqs_a.ctypes.data, nt.ctypes.data, seqs_a.size,
                                       slots.ctypes.data, ev.ctypes.data, cap, C.byref(nev)))
        return StepPlan(slots[:total], ev[:nev.value].copy(), token_seq=token_seq, token_pos=token_pos)

    def positions(self) -> np.ndarray:
        """Next position (= context length) of every sequence slot."""
        cl = np.empty(self.max_seqs, dtype=np.int32)
        check(lib.it_kv_manager_tables(self._h, None, 0, cl.ctypes.data, None))
        return cl

    def release(self, seq: int) -> np.ndarray:
        cap = self.max_blocks
        ev = np.empty(cap, dtype=np.int32)
        nev = C.c_int32(0)
        check(lib.it_kv_manager_release_seq(self._h, seq, ev.ctypes.data, cap, C.byref(nev)))
        return ev[:nev.value].copy()

    def fork(self, src: int, dst: int) -> None:
        check(lib.it_kv_manager_fork(self._h, src, dst))

    def tables(self, max_blocks: Optional[int] = None) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
        mb = self.max_blocks if max_blocks is None else max_blocks
        t = np.empty((self.max_seqs, mb), dtype=np.int32)
        cl = np.empty(self.max_seqs, dtype=np.int32)
        sp = np.empty(self.max_seqs, dtype=np.int32)
        check(lib.it_kv_manager_tables(self._h, t.ctypes.data, mb, cl.ctypes.data, sp.ctypes.data))
        return t, cl, sp

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib.it_kv_manager_destroy(h)
            self._h = C.c_void_p()


class RequestState(Enum):  # continuous.rs:8-15
    Running = "Running"
    Waiting = "Waiting"
    Preempted = "Preempted"
    Finished = "Finished"


@dataclass
class RequestContext:  # continuous.rs:17-25
    request_id: int
    state: RequestState
    prompt_tokens: List[int]
    generated_tokens: List[int]
    max_tokens: int


class ContinuousBatcher:
    """FIFO admission (continuous.rs:28-74) wired to a KvManager.

    `schedule()` moves waiting requests to running up to max_batch_size, in
    arrival order (continuous.rs:62-73).  Each running request is bound to a
    manager sequence slot; `plan_prefill` / `plan_decode` produce the step's
    slot mapping through the manager, and `finish` releases the blocks.
    """

    def __init__(self, max_batch_size: int, manager: Optional[KvManager] = None):
        self.requests: Dict[int, RequestContext] = {}
        self.running: List[int] = []
        self.waiting: deque = deque()
        self.max_batch_size = max_batch_size
        self.manager = manager
        self.seq_of: Dict[int, int] = {}
        self._free_seqs: List[int] = list(range(manager.max_seqs - 1, -1, -1)) if manager else []

    def add_request(self, request_id: int, prompt: Sequence[int], max_tokens: int) -> None:  # :45-60
        self.requests[request_id] = RequestContext(request_id, RequestState.Waiting, list(prompt), [], max_tokens)
        self.waiting.append(request_id)

    def schedule(self) -> List[int]:  # :62-73
        while len(self.running) < self.max_batch_size:
            if not self.waiting:
                break
            rid = self.waiting.popleft()
            ctx = self.requests.get(rid)
            if ctx is not None:
                ctx.state = RequestState.Running
                self.running.append(rid)
                if self.manager is not None:
                    if not self._free_seqs:
                        raise RuntimeError("no free sequence slot in the KV manager")
                    self.seq_of[rid] = self._free_seqs.pop()
        return list(self.running)

    def plan_prefill(self, request_ids: Sequence[int]) -> StepPlan:
        seqs = [self.seq_of[r] for r in request_ids]
        lens = [len(self.requests[r].prompt_tokens) for r in request_ids]
        return self.manager.append(seqs, lens)

    def plan_decode(self) -> StepPlan:
        return self.manager.append([self.seq_of[r] for r in self.running], 1)

    def finish(self, request_id: int) -> np.ndarray:
        ctx = self.requests[request_id]
        ctx.state = RequestState.Finished
        self.running.remove(request_id)
        freed = np.zeros(0, np.int32)
        if self.manager is not None and request_id in self.seq_of:
            seq = self.seq_of.pop(request_id)
            freed = self.manager.release(seq)
            self._free_seqs.append(seq)
        return freed
