"""Prefix sharing end to end on the GPU: a prefilled sequence is forked
(blocks shared, refcounts raised), both branches append with copy-on-write
(the shared partial block is copied to a fresh page by it_kv_copy_blocks
before the append writes into it), a branch is forked again mid-block, and
every sequence is decoded.  Pools are compared byte for byte with the
oracle cache after every step, block ids and copy lists with a restatement
of the copy-on-write rule over the oracle's BlockPool, and decode outputs
with the oracle's flash-decode (bf16 tolerance, rtol 2e-3 / atol 1e-2)."""
import numpy as np
import pytest

import oracle as orc
from kvutil import assert_close_or_closer, exact_decode, from_dev, kv_values, lazy, to_dev, widen

pytestmark = pytest.mark.gpu

SENTINEL = 0x5C


class _CowMirror:
    """Block tables under fork / append-with-copy-on-write over the oracle's
    BlockPool: a token at pos % bs == 0 allocates a block; a token written
    into a partial block whose refcount is > 1 allocates a new block, lists
    (old, new) as a copy and drops one reference to the old block."""

    def __init__(self, pool, bs, max_seqs, max_blocks):
        self.pool, self.bs = pool, bs
        self.table = np.full((max_seqs, max_blocks), -1, np.int32)
        self.pos = np.zeros(max_seqs, np.int64)

    def fork(self, src, dst):
        for j, b in enumerate(self.table[src]):
            if b >= 0:
                assert self.pool.share(int(b)) == 0
                self.table[dst, j] = b
        self.pos[dst] = self.pos[src]

    def append(self, seqs, n_tokens):
        slots, cs, cd = [], [], []
        for s, n in zip(seqs, n_tokens):
            for _ in range(n):
                p = int(self.pos[s])
                lb = p // self.bs
                if p % self.bs == 0:
                    self.table[s, lb] = self.pool.allocate()
                elif self.pool.ref_count(int(self.table[s, lb])) > 1:
                    new = self.pool.allocate()
                    cs.append(int(self.table[s, lb]))
                    cd.append(new)
                    assert self.pool.free(int(self.table[s, lb])) == 0
                    self.table[s, lb] = new
                slots.append(int(self.table[s, lb]) * self.bs + p % self.bs)
                self.pos[s] = p + 1
        return np.array(slots, np.int64), np.array(cs, np.int32), np.array(cd, np.int32)

    def release(self, s):
        for b in self.table[s]:
            if b >= 0:
                assert self.pool.free(int(b)) == 0
        self.table[s] = -1
        self.pos[s] = 0


def test_fork_cow_copy_append_decode_matches_oracle():
    import torch
    from infer_train_amd import BF16, BlockPool, KvManager
    from infer_train_amd.kv import PagedKvCache

    cap, bs, hkv, hq, D, max_seqs, mb = 40, 16, 2, 8, 128, 4, 8
    order = orc.permutation(21, cap)
    pool, opool = BlockPool(cap, BF16, order=order), orc.Pool(cap, order=order)
    mgr, mirror = KvManager(pool, bs, max_seqs, mb), _CowMirror(opool, bs, max_seqs, mb)
    dev = PagedKvCache(cap, bs, hkv, D, BF16)
    dev.k_pool.fill_(SENTINEL)
    dev.v_pool.fill_(SENTINEL)
    ref = orc.Cache(cap, bs, hkv, D, orc.BF16)
    ref.k[:] = SENTINEL
    ref.v[:] = SENTINEL
    page = dev.page_bytes * hkv  # bytes of one block in one pool
    seed = [100]

    def write(plan_slots, cs, cd):
        """Copy the listed pages, then append fresh K/V at the slots, on both sides."""
        if cs.size:
            dev.copy_blocks(to_dev(cs), to_dev(cd))
            for s_, d_ in zip(cs, cd):
                ref.k[d_ * page:(d_ + 1) * page] = ref.k[s_ * page:(s_ + 1) * page]
                ref.v[d_ * page:(d_ + 1) * page] = ref.v[s_ * page:(s_ + 1) * page]
        n = plan_slots.size
        k = kv_values(seed[0], n * hkv * D, orc.BF16).reshape(n, hkv, D)
        v = kv_values(seed[0] + 1, n * hkv * D, orc.BF16).reshape(n, hkv, D)
        seed[0] += 2
        ref.append(k, v, plan_slots)
        dev.append(to_dev(k.view(np.int16), torch.bfloat16), to_dev(v.view(np.int16), torch.bfloat16),
                   to_dev(plan_slots))
        dev.check()
        for name, d, r in (("K", dev.k_pool, ref.k), ("V", dev.v_pool, ref.v)):
            got = from_dev(d)
            if not np.array_equal(got, r):
                i = np.flatnonzero(got != r)[0]
                raise AssertionError(f"{name} pool differs first at byte {i} (block {i // page})")

    def step(seqs, n_tokens):
        plan = mgr.append(seqs, n_tokens, cow=True)
        slots, cs, cd = mirror.append(seqs, n_tokens)
        np.testing.assert_array_equal(plan.slots, slots)
        np.testing.assert_array_equal(plan.cow_src, cs)
        np.testing.assert_array_equal(plan.cow_dst, cd)
        write(plan.slots, plan.cow_src, plan.cow_dst)
        return plan

    def decode(seqs):
        tables, ctx, _ = mgr.tables()
        np.testing.assert_array_equal(tables, mirror.table)
        t, c = tables[seqs], ctx[seqs]
        q = kv_values(seed[0], len(seqs) * hq * D, orc.BF16).reshape(len(seqs), hq, D)
        seed[0] += 1
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
        want = ref.decode(widen(q, orc.BF16), hq, t, c, None, scale)
        out = dev.decode(to_dev(q.view(np.int16), torch.bfloat16), to_dev(t), to_dev(c), None, int(c.max()),
                         scale=scale, partition=64, out_dtype=torch.float32)
        dev.check()
        got = from_dev(out).reshape(want.shape)
        assert_close_or_closer(got, want, lazy(lambda: exact_decode(ref, widen(q, orc.BF16), hq, t, c, None, scale,
                                                                    with_mag=True)),
                               2e-3, 1e-2, f"decode seqs {seqs} ctx {list(c)}")
        return got

    step([0], [45])  # blocks 0..2 of seq 0, the last one partial (13 of 16)
    mgr.fork(0, 1)
    mirror.fork(0, 1)
    b = mgr.tables()[0][0]
    assert [pool.ref_count(int(x)) for x in b[:3]] == [2, 2, 2]
    # Seq 1 writes first into the shared partial block: it gets the copy.
    p = step([1, 0], [1, 1])
    assert list(p.cow_src) == [b[2]] and pool.ref_count(int(b[2])) == 1
    t = mgr.tables()[0]
    assert t[1, 2] == p.cow_dst[0] and t[0, 2] == b[2] and (t[1, :2] == b[:2]).all()
    out = decode([0, 1])
    # Same prefix, different 46th token: the outputs differ.
    assert not np.array_equal(out[0], out[1])
    for _ in range(5):  # to position 51: a new block at 48 for both, no copies
        p = step([0, 1], [1, 1])
        assert p.cow_src.size == 0
    decode([0, 1])
    # Fork the fork mid-block (pos 51 of 64): three sequences share blocks.
    mgr.fork(1, 2)
    mirror.fork(1, 2)
    shared = int(mgr.tables()[0][1, 3])
    assert pool.ref_count(shared) == 2 and pool.ref_count(int(b[0])) == 3
    # Several tokens of seq 2 in one step: one copy, then writes to its own page.
    p = step([2, 1, 0], [3, 2, 1])
    assert list(p.cow_src) == [shared] and pool.ref_count(shared) == 1
    decode([0, 1, 2])
    for _ in range(14):  # seq 2 crosses 64 into a fifth block
        step([2, 0, 1], [1, 1, 1])
    decode([2, 1, 0])
    # Positions 0..44 hold the same bytes in all three sequences (shared
    # pages, or copies of them): one query over those 45 positions gives
    # bit-identical outputs through each sequence's own block table.
    tables, ctx, _ = mgr.tables()
    assert list(ctx[:3]) == [66, 67, 68]
    assert tables[1, 2] != tables[0, 2]
    q = kv_values(7, hq * D, orc.BF16).reshape(1, hq, D)
    qd = to_dev(np.repeat(q, 3, axis=0).view(np.int16), torch.bfloat16)
    c45 = np.full(3, 45, np.int32)
    out = from_dev(dev.decode(qd, to_dev(tables[:3]), to_dev(c45), None, 45,
                              scale=float(np.float32(1.0) / np.sqrt(np.float32(D))), partition=64,
                              out_dtype=torch.float32))
    dev.check()
    out = out.reshape(3, hq, D)
    np.testing.assert_array_equal(out[1], out[0])
    np.testing.assert_array_equal(out[2], out[0])
    for s in (2, 1, 0):
        mgr.release(s)
        mirror.release(s)
    assert pool.num_free() == opool.num_free() == cap
