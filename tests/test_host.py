"""The product's host-side allocator and slot manager (native, in
libit_kv.so) against the oracle's restatement: bit-exact block ids, slots,
eviction order and tables."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as orc
from infer_train_amd import BlockPool, ContinuousBatcher, InvalidInput, KvManager

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_block_pool_mirrors_reference():
    p = BlockPool(5)
    assert [p.allocate() for _ in range(5)] == [4, 3, 2, 1, 0]  # paged.rs:36-42
    assert p.allocate() is None
    p.free(3)
    p.share(1)
    p.free(1)
    assert p.ref_count(1) == 1 and p.num_free() == 1
    assert p.allocate() == 3
    with pytest.raises(InvalidInput):
        p.free(3) or p.free(3)
    assert BlockPool(3, quant_type=8).quant_type() == 8


def test_block_pool_random_ops_equal_oracle():
    rng = np.random.default_rng(5)
    cap = 64
    order = orc.permutation(9, cap)
    a, b = BlockPool(cap, order=order), orc.Pool(cap, order=order)
    for _ in range(20000):
        op, i = int(rng.integers(3)), int(rng.integers(cap))
        if op == 0:
            assert a.allocate() == b.allocate()
        elif op == 1:
            rb = b.share(i)
            if rb:
                with pytest.raises(InvalidInput):
                    a.share(i)
            else:
                a.share(i)
        else:
            rb = b.free(i)
            if rb:
                with pytest.raises(InvalidInput):
                    a.free(i)
            else:
                a.free(i)
        assert a.num_free() == b.num_free()


def _sha(x):
    return hashlib.sha256(np.ascontiguousarray(x).tobytes()).hexdigest()


def test_window_manager_config4_equals_oracle_and_golden():
    cap, bs, W, start = 16512, 16, 4096, 30000
    order = orc.permutation(4, cap)
    pa, pb = BlockPool(cap, order=order), orc.Pool(cap, order=order)
    mb = 32768 // bs + 1
    ma, mo = KvManager(pa, bs, 64, mb, W), orc.Manager(pb, bs, 64, mb, W)
    first, last = (start - W) // bs, (start - 1) // bs
    for s in range(64):
        blocks = [pa.allocate() for _ in range(last - first + 1)]
        assert blocks == [pb.allocate() for _ in range(last - first + 1)]
        ma.seed_seq(s, start, first, blocks)
        mo.seed_seq(s, start, first, blocks)
    slots, evs = [], []
    for _ in range(2768):
        plan = ma.append(list(range(64)))
        so, eo = mo.append(list(range(64)))
        np.testing.assert_array_equal(plan.slots, so)
        np.testing.assert_array_equal(plan.evicted, eo)
        slots.append(plan.slots)
        evs.append(plan.evicted)
    ta, ca, sa = ma.tables()
    to, co, so_ = mo.tables()
    np.testing.assert_array_equal(ta, to)
    np.testing.assert_array_equal(ca, co)
    np.testing.assert_array_equal(sa, so_)
    man = json.load(open(os.path.join(GOLDEN, "manifest.json")))["config4_schedule"]
    assert _sha(np.concatenate(slots)) == man["slots_sha256"]
    assert _sha(np.concatenate(evs)) == man["evicted_sha256"]
    assert _sha(ta) == man["tables_sha256"]


def test_manager_random_ragged_equals_oracle():
    rng = np.random.default_rng(7)
    cap, bs = 4096, 16
    order = orc.permutation(12, cap)
    pa, pb = BlockPool(cap, order=order), orc.Pool(cap, order=order)
    for W in (0, 100, 257):
        ma, mo = KvManager(pa, bs, 8, 400, W), orc.Manager(pb, bs, 8, 400, W)
        for _ in range(40):
            seqs = rng.permutation(8)[: int(rng.integers(1, 8))]
            nt = rng.integers(0, 40, seqs.size)
            plan = ma.append(seqs, nt)
            so, eo = mo.append(seqs, nt)
            np.testing.assert_array_equal(plan.slots, so)
            np.testing.assert_array_equal(plan.evicted, eo)
        for x, y in zip(ma.tables(), mo.tables()):
            np.testing.assert_array_equal(x, y)
        for s in range(8):
            ma.release(s)
            t, _, _ = mo.tables()
            for blk in t[s][t[s] >= 0]:
                assert pb.free(int(blk)) == 0
        assert pa.num_free() == pb.num_free() == cap


def test_slots_unique_and_exhaustion():
    pool = BlockPool(4)
    m = KvManager(pool, 16, 2, 8)
    with pytest.raises(InvalidInput, match="exhausted"):
        m.append([0, 1], [40, 20])  # 3 + 2 blocks > 4
    m2 = KvManager(BlockPool(64), 16, 2, 8)
    plan = m2.append([0, 1, 0], [33, 7, 2])
    assert len(set(plan.slots.tolist())) == 42


def test_fork_copy_on_write():
    pool = BlockPool(16)
    m = KvManager(pool, 16, 3, 8)
    a = m.append([0], [20])  # blocks 15 (full) and 14 (partial)
    m.fork(0, 1)
    assert pool.ref_count(15) == 2 and pool.ref_count(14) == 2
    plan = m.append([1], [1], cow=True)  # writing into shared partial block 14
    assert list(plan.cow_src) == [14] and pool.ref_count(14) == 1
    new = int(plan.cow_dst[0])
    assert plan.slots[0] == new * 16 + 4
    t, cl, _ = m.tables()
    assert t[1, 0] == 15 and t[1, 1] == new and t[0, 1] == 14 and cl[1] == 21
    plan0 = m.append([0], [1], cow=True)  # seq 0 now owns 14 alone: no copy
    assert plan0.cow_src.size == 0 and plan0.slots[0] == 14 * 16 + 4


def test_repeated_sequence_positions_match_slots():
    """A sequence listed twice in one append gets consecutive positions, in
    the order the native manager assigns its slots: the plan's positions
    and slots agree (slot = table[pos / bs] * bs + pos % bs), also across a
    block boundary."""
    from infer_train_amd import BF16, BlockPool, KvManager

    bs = 16
    pool = BlockPool(32, BF16)
    mgr = KvManager(pool, bs, 4, 8)
    mgr.append([0], [15])
    plan = mgr.append([0, 1, 0, 0], [1, 3, 1, 2])
    tables, ctx, _ = mgr.tables()
    assert list(plan.token_pos[plan.token_seq == 0]) == [15, 16, 17, 18]
    assert list(plan.token_pos[plan.token_seq == 1]) == [0, 1, 2]
    want = tables[plan.token_seq, plan.token_pos // bs].astype(np.int64) * bs + plan.token_pos % bs
    np.testing.assert_array_equal(plan.slots, want)
    assert ctx[0] == 19 and ctx[1] == 3


def test_batcher_fifo_admission_and_plans():
    pool = BlockPool(64)
    m = KvManager(pool, 16, 4, 16)
    b = ContinuousBatcher(2, m)
    for rid, n in ((10, 5), (11, 17), (12, 3)):
        b.add_request(rid, list(range(n)), 4)
    assert b.schedule() == [10, 11]  # continuous.rs:62-73, FIFO up to max_batch_size
    assert b.requests[12].state.value == "Waiting"
    plan = b.plan_prefill([10, 11])
    assert plan.slots.size == 22
    assert plan.slots[0] == 63 * 16 and plan.slots[5] == 62 * 16  # LIFO blocks: 63 for seq 0, 62 for seq 1
    d = b.plan_decode()
    assert d.slots.size == 2
    freed = b.finish(10)
    assert list(freed) == [63]
    assert b.schedule() == [11, 12]


def _oracle_release(mo, pool, s):
    """The oracle's release of sequence slot s (BlockPool::free of every held
    block, lowest logical block first, then an empty table row); returns the
    blocks that went back to the pool."""
    return [int(b) for b in mo.release(s)]


def test_batcher_preemption_releases_or_keeps_blocks_like_the_oracle():
    """Preempted requests: releasing ones give their blocks back (the LIFO
    pool hands them out again, last freed first) and are prefilled again,
    prompt plus generated tokens, on resume; kept ones resume at their
    position with their blocks.  Every slot, freed block and table equals
    the oracle manager driven through the same steps."""
    cap, bs = 12, 16
    order = orc.permutation(3, cap)
    pa, pb = BlockPool(cap, order=order), orc.Pool(cap, order=order)
    m, mo = KvManager(pa, bs, 4, 8), orc.Manager(pb, bs, 4, 8)
    b = ContinuousBatcher(3, m)
    for rid, n in ((1, 20), (2, 33), (3, 10), (4, 5)):
        b.add_request(rid, list(range(n)), 8)
    assert b.schedule() == [1, 2, 3]
    seq = dict(b.seq_of)
    assert seq == {1: 0, 2: 1, 3: 2}
    plan = b.plan_prefill([1, 2, 3])
    so, _ = mo.append([0, 1, 2], [20, 33, 10])
    np.testing.assert_array_equal(plan.slots, so)
    for step in range(2):
        plan = b.plan_decode()
        so, _ = mo.append([0, 1, 2], 1)
        np.testing.assert_array_equal(plan.slots, so)
        for r in (1, 2, 3):
            b.requests[r].generated_tokens.append(100 + step)
    assert pa.num_free() == pb.num_free() == 6

    # 8 free blocks wanted: request 3 (1 block) then 2 (3 blocks) preempted.
    assert b.preempt_for(8) == [3, 2]
    assert pa.num_free() == 10
    f3, f2 = _oracle_release(mo, pb, 2), _oracle_release(mo, pb, 1)
    assert [b.requests[r].state.value for r in (1, 2, 3)] == ["Running", "Preempted", "Preempted"]
    assert b.needs_prefill == {2, 3} and 2 not in b.seq_of and 3 not in b.seq_of

    # Keeping: blocks and slot stay, nothing freed.
    assert b.preempt(1, keep_blocks=True).size == 0 and b.seq_of[1] == 0
    assert pa.num_free() == 10 and 1 not in b.needs_prefill
    with pytest.raises(ValueError):
        b.preempt(1)  # already preempted

    # Resumed in preemption order before the waiting request 4.
    assert b.schedule() == [3, 2, 1]
    assert b.requests[4].state.value == "Waiting"
    # Slots are handed out again LIFO: request 3 takes slot 1 (freed last).
    assert b.seq_of == {1: 0, 3: 1, 2: 2}
    plan = b.plan_resume([3, 2])
    assert b.needs_prefill == set()
    so, _ = mo.append([1, 2], [12, 35])
    np.testing.assert_array_equal(plan.slots, so)
    # Request 3 (listed first) starts in the last block freed, request 2's
    # last logical block: the LIFO pool.
    assert plan.slots[0] // bs == f2[-1]
    plan = b.plan_decode()
    so, _ = mo.append([1, 2, 0], 1)
    np.testing.assert_array_equal(plan.slots, so)
    t, cl, _ = m.tables()
    to, clo, _ = mo.tables()
    np.testing.assert_array_equal(t, to)
    np.testing.assert_array_equal(cl, clo)
    assert list(cl[:3]) == [23, 13, 36]
    for r in (1, 2, 3):
        b.finish(r)
    assert pa.num_free() == cap and b.schedule() == [4]


def test_finish_a_preempted_request():
    pool = BlockPool(8)
    b = ContinuousBatcher(2, KvManager(pool, 16, 2, 8))
    b.add_request(0, list(range(20)), 1)
    b.add_request(1, list(range(5)), 1)
    b.schedule()
    b.plan_prefill([0, 1])
    b.preempt(0, keep_blocks=True)
    assert pool.num_free() == 5
    assert list(b.finish(0)) != [] and pool.num_free() == 7  # its kept blocks go back
    assert 0 not in b.preempted and b.requests[0].state.value == "Finished"
    with pytest.raises(ValueError):
        b.finish(0)
    assert b.schedule() == [1]


def test_preempt_for_raises_when_nothing_is_left():
    pool = BlockPool(4)
    b = ContinuousBatcher(2, KvManager(pool, 16, 2, 8))
    b.add_request(0, list(range(40)), 1)
    b.schedule()
    b.plan_prefill([0])
    assert pool.num_free() == 1
    with pytest.raises(RuntimeError, match="cannot free"):
        b.preempt_for(5)
    assert pool.num_free() == 4 and b.requests[0].state.value == "Preempted"


def test_host_code_under_sanitizers(tmp_path):
    """The host allocator and slot manager (csrc/it_host.cpp, plain C++)
    built with AddressSanitizer and UndefinedBehaviorSanitizer and driven by
    tests/host_sanitize_driver.cpp: 24,000 random steps of appends (plain and
    copy-on-write), releases and forks with and without a window, the error
    paths of a full table and an exhausted pool, and the pool's counters
    checked after every operation."""
    import shutil
    import subprocess

    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = str(tmp_path / "host_sanitize_driver")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", "-I", os.path.join(root, "include"), "-I",
           os.path.join(root, "infer_train_amd", "csrc"), os.path.join(root, "infer_train_amd", "csrc", "it_host.cpp"),
           os.path.join(root, "tests", "host_sanitize_driver.cpp"), "-o", exe]
    b = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    if b.returncode != 0 and "asan" in b.stderr.lower():
        pytest.skip("the sanitizer runtime is not installed: " + b.stderr[-200:])
    assert b.returncode == 0, b.stderr[-2000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    if r.returncode != 0 and "does not come first" in r.stderr:
        pytest.skip("another preloaded library precedes the sanitizer runtime in this environment")
    assert r.returncode == 0, (r.stdout + r.stderr)[-3000:]
    assert "host sanitize driver: ok" in r.stdout


def test_window_does_not_evict_blocks_a_fork_holds():
    """Pool 16, block size 4, window 8: seq 0 takes 10 tokens, seq 1 forks
    it, seq 0 appends 4 more with copy-on-write.  The window drops seq 0's
    reference to block 15 at p = 11, but seq 1 still holds it: it is not
    listed for clearing, keeps refcount 1 and stays in seq 1's table.  Plans
    equal the oracle manager's; seq 1's own window later lists it."""
    pool, opool = BlockPool(16), orc.Pool(16)
    m, mo = KvManager(pool, 4, 2, 8, 8), orc.Manager(opool, 4, 2, 8, 8)
    p = m.append([0], [10])
    np.testing.assert_array_equal(p.slots, mo.append([0], [10])[0])
    m.fork(0, 1)
    mo.fork(0, 1)
    p = m.append([0], [4], cow=True)
    so, eo, cs, cd = mo.append([0], [4], cow=True)
    np.testing.assert_array_equal(p.slots, so)
    np.testing.assert_array_equal(p.evicted, eo)
    np.testing.assert_array_equal(p.cow_src, cs)
    np.testing.assert_array_equal(p.cow_dst, cd)
    assert p.evicted.size == 0 and pool.ref_count(15) == 1
    t, _, _ = m.tables()
    assert t[1, 0] == 15 and t[0, 0] == -1
    p = m.append([1], [2], cow=True)
    assert list(p.evicted) == [15] and pool.ref_count(15) == 0
    assert list(p.evicted) == list(mo.append([1], [2], cow=True)[1])
    # Release returns only what no other sequence holds.
    freed = m.release(0)
    assert sorted(freed.tolist()) == sorted(mo.release(0).tolist()) == [11, 12]
    assert pool.ref_count(14) == 1


def test_manager_fork_cow_window_release_equal_oracle():
    """Random appends (plain and copy-on-write), forks and releases, with
    and without a window: every plan (slots, per-token sequence and
    position, evicted list, copy pairs, context lengths, window starts) and
    every table equals the oracle manager's."""
    rng = np.random.default_rng(23)
    for W in (0, 12, 40):
        cap, bs, S, mb = 48, 4, 5, 40
        order = orc.permutation(W + 3, cap)
        pa, pb = BlockPool(cap, order=order), orc.Pool(cap, order=order)
        ma, mo = KvManager(pa, bs, S, mb, W), orc.Manager(pb, bs, S, mb, W)
        n_dead = 0
        for _ in range(600):
            _, ctx0, _ = mo.tables()
            op = rng.integers(10)
            if op < 7:
                seqs = rng.permutation(S)[: int(rng.integers(1, S + 1))]
                # Now and then more tokens than the window holds in one step.
                nt = rng.integers(0, W + 20 if op == 0 else 6, seqs.size)
                if (ctx0[seqs] + nt).max() >= mb * bs or pb.num_free() < seqs.size * (nt.max() // bs + 3) + 2:
                    for s in range(S):
                        np.testing.assert_array_equal(ma.release(s), mo.release(s))
                    continue
                cow = bool(op % 2)
                plan = ma.append(seqs, nt, cow=cow)
                want = mo.append(seqs, nt, cow=cow)
                if cow:  # (without copy-on-write, forks writing one shared page collide by design)
                    live = plan.slots[plan.slots >= 0]
                    assert np.unique(live).size == live.size, "two live tokens of one step share a slot"
                n_dead += int((plan.slots < 0).sum())
                np.testing.assert_array_equal(plan.slots, want[0])
                np.testing.assert_array_equal(plan.evicted, want[1])
                if cow:
                    np.testing.assert_array_equal(plan.cow_src, want[2])
                    np.testing.assert_array_equal(plan.cow_dst, want[3])
                np.testing.assert_array_equal(plan.token_seq, np.repeat(seqs, nt))
                np.testing.assert_array_equal(plan.token_pos, np.concatenate(
                    [ctx0[s] + np.arange(n) for s, n in zip(seqs, nt)]).astype(np.int32))
                _, ctx1, st1 = mo.tables()
                np.testing.assert_array_equal(plan.ctx_lens, ctx1)
                np.testing.assert_array_equal(plan.start_pos, st1)
            elif op < 9:
                s = int(rng.integers(S))
                np.testing.assert_array_equal(ma.release(s), mo.release(s))
            else:
                empty = [s for s in range(S) if ctx0[s] == 0]
                src = int(rng.integers(S))
                if empty and empty[0] != src:
                    ma.fork(src, empty[0])
                    mo.fork(src, empty[0])
            for x, y in zip(ma.tables(), mo.tables()):
                np.testing.assert_array_equal(x, y)
            assert pa.num_free() == pb.num_free()
        assert n_dead > 0 or W == 0


def test_release_with_too_small_capacity_changes_nothing():
    from infer_train_amd._lib import lib
    import ctypes as C

    pool = BlockPool(16)
    m = KvManager(pool, 4, 2, 8)
    m.append([0], [10])
    before = m.tables()[0].copy()
    ev = np.empty(2, np.int32)
    n = C.c_int32(0)
    rc = lib.it_kv_manager_release_seq(m._h, 0, ev.ctypes.data, 2, C.byref(n))
    assert rc == 2 and "capacity" in lib.it_last_error().decode()
    np.testing.assert_array_equal(m.tables()[0], before)
    assert pool.num_free() == 13
    assert sorted(m.release(0).tolist()) == [13, 14, 15]


def test_step_longer_than_window_marks_dead_tokens():
    """Pool 16, block size 4, window 8: one step appends 14 tokens.  At
    p = 11 the window returns block 15 (positions 0-3) to the pool: those
    four tokens are dead (slot -1, never written), block 15 is listed for
    clearing, and it goes back on the free list only when the step ends, so
    p = 12 opens block 12, not 15, and no two tokens share a slot.  The next
    step releases block 14 and the one after opens it again (LIFO: the last
    block pushed back).  Equal to the oracle manager."""
    pool, opool = BlockPool(16), orc.Pool(16)
    m, mo = KvManager(pool, 4, 1, 8, 8), orc.Manager(opool, 4, 1, 8, 8)
    p = m.append([0], [14])
    so, eo = mo.append([0], [14])
    np.testing.assert_array_equal(p.slots, so)
    np.testing.assert_array_equal(p.evicted, eo)
    assert list(p.slots[:4]) == [-1] * 4
    assert list(p.slots[4:] // 4) == [14] * 4 + [13] * 4 + [12] * 2
    assert list(p.evicted) == [15] and pool.ref_count(15) == 0
    assert list(p.token_pos) == list(range(14)) and p.ctx_lens[0] == 14 and p.start_pos[0] == 6
    p = m.append([0], [2])
    np.testing.assert_array_equal(p.slots, mo.append([0], [2])[0])
    # p = 15 releases block 14 (positions 4-7, written by the first step).
    assert list(p.slots // 4) == [12, 12] and list(p.evicted) == [14]
    p = m.append([0], [2])  # p = 16 opens a block: 14, the last one pushed back
    np.testing.assert_array_equal(p.slots, mo.append([0], [2])[0])
    assert list(p.slots // 4) == [14, 14] and p.evicted.size == 0
