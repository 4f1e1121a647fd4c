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

from ._lib import StepPlanC, check, lib
from .memory import BlockPool

__all__ = ["KvManager", "ContinuousBatcher", "RequestState", "RequestContext", "StepPlan"]


_EMPTY = np.zeros(0, np.int32)
_EMPTY.flags.writeable = False


@dataclass
class StepPlan:
    """What one append step hands to the device: the slot of every new token
    with its sequence and position (it_kv_sync_tables' inputs), the blocks
    the step returned to the pool (refcount 0: the pages to clear with
    kv_evict), the copy-on-write page pairs (to copy with kv_copy_blocks
    before the append), and every sequence slot's context length and window
    start after the step."""

    slots: np.ndarray
    evicted: np.ndarray
    cow_src: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    cow_dst: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    token_seq: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    token_pos: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int32))
    ctx_lens: Optional[np.ndarray] = None
    start_pos: Optional[np.ndarray] = None


class KvManager:
    """Slot mapping and block tables over a BlockPool (native:
    it_kv_manager_step).

    slot(pos) = table[pos // bs] * bs + pos % bs; a block is allocated when
    pos % bs == 0.  With `window` W > 0, before the token at position p every
    held block whose last position is < p - W + 1 drops this sequence's
    reference (oldest first); the blocks whose refcount reaches 0 are the
    step's `evicted` list.  Sequences of one step are processed in the order
    listed.
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
        self._destroy = lib.it_kv_manager_destroy  # bound now: module globals may be gone at exit
        # Reused buffers of it_kv_manager_step (grown on demand), with their
        # addresses cached (ndarray.ctypes.data costs about a microsecond);
        # the plan returned to the caller holds copies.
        self._plan = StepPlanC()
        self._plan_ref = C.byref(self._plan)
        self._step_fn = lib.it_kv_manager_step
        self._tok_cap = 0
        self._seq_cap = 0
        # Blocks returned to the pool in one step: at most the pool's capacity.
        self._ev = np.empty(pool.capacity() + 1, np.int32)
        self._plan.evicted = self._ev.ctypes.data
        self._plan.evicted_cap = self._ev.size
        self._lens = np.empty((2, max_seqs), np.int32)  # ctx_lens, start_pos
        self._plan.ctx_lens, self._plan.start_pos = self._lens[0].ctypes.data, self._lens[1].ctypes.data
        self._grow_tokens(64)
        self._grow_seqs(64)

    def _grow_tokens(self, total: int) -> None:
        cap = max(total, 2 * self._tok_cap)
        self._slots = np.empty(cap, np.int64)
        self._tsp = np.empty((2, cap), np.int32)  # token_seq, token_pos
        self._cs = np.empty(cap, np.int32)
        self._cd = np.empty(cap, np.int32)
        pl = self._plan
        pl.slots, pl.token_seq, pl.token_pos = self._slots.ctypes.data, self._tsp[0].ctypes.data, self._tsp[1].ctypes.data
        pl.tokens_cap = cap
        pl.cow_cap = cap  # at most one copy per token
        self._cs_addr, self._cd_addr = self._cs.ctypes.data, self._cd.ctypes.data
        self._tok_cap = cap

    def _grow_seqs(self, n: int) -> None:
        cap = max(n, 2 * self._seq_cap)
        self._seqbuf = np.empty(cap, np.int32)
        self._ntbuf = np.empty(cap, np.int32)
        self._seq_addr, self._nt_addr = self._seqbuf.ctypes.data, self._ntbuf.ctypes.data
        self._seq_cap = cap

    def seed_seq(self, seq: int, pos: int, first_block: int, blocks: Sequence[int]) -> None:
        arr = np.ascontiguousarray(np.asarray(blocks, dtype=np.int32))
        check(lib.it_kv_manager_seed_seq(self._h, seq, int(pos), int(first_block), arr.ctypes.data, arr.size))

    def append(self, seqs: Sequence[int], n_tokens: Sequence[int] | int = 1, cow: bool = False) -> StepPlan:
        """One step: n_tokens[i] tokens to seqs[i] (in list order)."""
        n = len(seqs)
        if n > self._seq_cap:
            self._grow_seqs(n)
        self._seqbuf[:n] = seqs
        nt = self._ntbuf[:n]
        if np.isscalar(n_tokens):
            nt.fill(n_tokens)
            total = int(n_tokens) * n
        else:
            nt[:] = n_tokens
            total = int(nt.sum())
        if total > self._tok_cap:
            self._grow_tokens(total)
        pl = self._plan
        pl.cow_src = self._cs_addr if cow else None
        pl.cow_dst = self._cd_addr if cow else None
        rc = self._step_fn(self._h, self._seq_addr, self._nt_addr, n, self._plan_ref)
        if rc:
            check(rc)
        k, ne, nc = pl.n_tokens, pl.n_evicted, pl.n_cow
        tsp, lens = self._tsp[:, :k].copy(), self._lens.copy()
        return StepPlan(self._slots[:k].copy(), self._ev[:ne].copy() if ne else _EMPTY,
                        self._cs[:nc].copy() if nc else _EMPTY, self._cd[:nc].copy() if nc else _EMPTY,
                        tsp[0], tsp[1], lens[0], lens[1])

    def positions(self) -> np.ndarray:
        """Next position (= context length) of every sequence slot."""
        cl = np.empty(self.max_seqs, dtype=np.int32)
        check(lib.it_kv_manager_tables(self._h, None, 0, cl.ctypes.data, None))
        return cl

    def release(self, seq: int) -> np.ndarray:
        """Drop every block of `seq`; returns the blocks that went back to
        the pool (refcount 0), the pages to clear."""
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
            self._destroy(h)
            self._h = None


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

    Preemption (the reference declares RequestState::Preempted,
    continuous.rs:13, but never enters it): `preempt` moves a running
    request to Preempted, either releasing its blocks and sequence slot (the
    request is prefilled again, prompt and generated tokens, when it resumes)
    or keeping them (it resumes where it stopped).  `preempt_for(n)` frees
    pool blocks by preempting, releasing, the most recently admitted running
    requests first until n blocks are free.  `schedule()` resumes preempted
    requests, in the order they were preempted, before it admits waiting
    ones.  Every choice depends only on the call sequence, so block ids stay
    deterministic.
    """

    def __init__(self, max_batch_size: int, manager: Optional[KvManager] = None):
        self.requests: Dict[int, RequestContext] = {}
        self.running: List[int] = []
        self.waiting: deque = deque()
        self.max_batch_size = max_batch_size
        self.manager = manager
        self.seq_of: Dict[int, int] = {}
        self._free_seqs: List[int] = list(range(manager.max_seqs - 1, -1, -1)) if manager else []
        self.preempted: deque = deque()  # preemption order
        self.needs_prefill: set = set()  # released by preemption: prefill again on resume

    def add_request(self, request_id: int, prompt: Sequence[int], max_tokens: int) -> None:  # :45-60
        self.requests[request_id] = RequestContext(request_id, RequestState.Waiting, list(prompt), [], max_tokens)
        self.waiting.append(request_id)

    def schedule(self) -> List[int]:  # :62-73
        while len(self.running) < self.max_batch_size:
            if self.preempted:  # resumed first, in preemption order
                rid = self.preempted.popleft()
            elif self.waiting:
                rid = self.waiting.popleft()
            else:
                break
            ctx = self.requests.get(rid)
            if ctx is not None:
                ctx.state = RequestState.Running
                self.running.append(rid)
                if self.manager is not None and rid not in self.seq_of:
                    if not self._free_seqs:
                        raise RuntimeError("no free sequence slot in the KV manager")
                    self.seq_of[rid] = self._free_seqs.pop()
        return list(self.running)

    def preempt(self, request_id: int, keep_blocks: bool = False) -> np.ndarray:
        """Running -> Preempted.  keep_blocks False: the request's blocks are
        released (BlockPool::free, lowest logical block first) with its
        sequence slot, and it is prefilled again on resume; True: blocks and
        slot stay held.  Returns the blocks that went back to the pool
        (refcount 0: the pages to clear; a block a forked request still
        holds is not among them), empty when kept."""
        ctx = self.requests[request_id]
        if ctx.state != RequestState.Running:
            raise ValueError(f"request {request_id} is {ctx.state.value}, not Running")
        ctx.state = RequestState.Preempted
        self.running.remove(request_id)
        self.preempted.append(request_id)
        freed = np.zeros(0, np.int32)
        if not keep_blocks and self.manager is not None and request_id in self.seq_of:
            seq = self.seq_of.pop(request_id)
            freed = self.manager.release(seq)
            self._free_seqs.append(seq)
            self.needs_prefill.add(request_id)
        return freed

    def preempt_for(self, n_blocks: int) -> List[int]:
        """Preempt (releasing) the most recently admitted running requests
        until the pool holds n_blocks free blocks; returns them in the order
        they were preempted.  Raises if even preempting every running request
        does not free enough."""
        pool = self.manager.pool
        out: List[int] = []
        while pool.num_free() < n_blocks:
            if not self.running:
                raise RuntimeError(f"cannot free {n_blocks} blocks: {pool.num_free()} free with nothing running")
            rid = self.running[-1]
            self.preempt(rid, keep_blocks=False)
            out.append(rid)
        return out

    def plan_resume(self, request_ids: Sequence[int]) -> StepPlan:
        """Prefill again the requests a releasing preemption emptied: their
        prompt plus the tokens generated before the preemption."""
        seqs = [self.seq_of[r] for r in request_ids]
        lens = [len(self.requests[r].prompt_tokens) + len(self.requests[r].generated_tokens) for r in request_ids]
        for r in request_ids:
            self.needs_prefill.discard(r)
        return self.manager.append(seqs, lens)

    def plan_prefill(self, request_ids: Sequence[int]) -> StepPlan:
        seqs = [self.seq_of[r] for r in request_ids]
        lens = [len(self.requests[r].prompt_tokens) for r in request_ids]
        return self.manager.append(seqs, lens)

    def plan_decode(self) -> StepPlan:
        return self.manager.append([self.seq_of[r] for r in self.running], 1)

    def finish(self, request_id: int) -> np.ndarray:
        """Running or Preempted -> Finished; the request's blocks (if it
        still holds them) and sequence slot are released.  Returns the
        blocks that went back to the pool (refcount 0)."""
        ctx = self.requests[request_id]
        if ctx.state == RequestState.Running:
            self.running.remove(request_id)
        elif ctx.state == RequestState.Preempted:
            self.preempted.remove(request_id)
        else:
            raise ValueError(f"request {request_id} is {ctx.state.value}")
        ctx.state = RequestState.Finished
        self.needs_prefill.discard(request_id)
        freed = np.zeros(0, np.int32)
        if self.manager is not None and request_id in self.seq_of:
            seq = self.seq_of.pop(request_id)
            freed = self.manager.release(seq)
            self._free_seqs.append(seq)
        return freed
