"""Every layer of a model in one multi-layer cache, behind one manager (the
reference keeps one K and one V cache per layer, forward.rs:17-18, 36-37,
indexed by layer_idx at :224-228).  One step of the per-layer flow: the
manager plans the step once (slots, per-token sequence and
position, copy-on-write pairs, blocks returned to the pool); copy_blocks and
evict act on every layer in one launch; each layer appends its own K/V
through its view; sync_tables updates the one device block table; each layer
decodes through its view.

A forked sequence shares blocks with its parent under a sliding window: the
window and a release drop the parent's references, but only blocks whose
refcount reached 0 are cleared, so the sibling keeps reading intact pages.
Pools are compared byte for byte with per-layer oracle caches, plans with
the oracle manager, decode outputs with the oracle's flash-decode (bf16
tolerance, rtol 2e-3 / atol 1e-2)."""
import numpy as np
import pytest

import oracle as orc
from kvutil import assert_close_or_closer, exact_decode, from_dev, kv_values, lazy, to_dev, widen

pytestmark = pytest.mark.gpu

SENTINEL = 0x3C


def test_two_layers_fork_under_window_one_manager():
    import torch
    from infer_train_amd import BF16, BlockPool, KvManager
    from infer_train_amd.kv import PagedKvCache

    L, cap, bs, hkv, hq, D, W, S, mb = 2, 96, 16, 2, 8, 128, 128, 4, 24
    order = orc.permutation(77, cap)
    pool, opool = BlockPool(cap, BF16, order=order), orc.Pool(cap, orc.BF16, order=order)
    mgr, omgr = KvManager(pool, bs, S, mb, W), orc.Manager(opool, bs, S, mb, W)
    dev = PagedKvCache(cap, bs, hkv, D, BF16, n_layers=L)
    assert dev.describe().n_layers == L
    dev.k_pool.fill_(SENTINEL)
    dev.v_pool.fill_(SENTINEL)
    layers = [dev.layer(i) for i in range(L)]
    lb = cap * hkv * dev.page_bytes
    assert layers[1].describe().k_pool == dev.describe().k_pool + lb
    refs = [orc.Cache(cap, bs, hkv, D, orc.BF16) for _ in range(L)]
    for r in refs:
        r.k[:] = SENTINEL
        r.v[:] = SENTINEL
    page = hkv * dev.page_bytes  # bytes of one block in one layer of one pool
    tables_d = torch.full((S, mb), -1, dtype=torch.int32, device="cuda:0")
    seed = [500]
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))

    def check_pools(what):
        dev.check()
        for name, d, rs in (("K", dev.k_pool, [r.k for r in refs]), ("V", dev.v_pool, [r.v for r in refs])):
            got, want = from_dev(d), np.concatenate(rs)
            if not np.array_equal(got, want):
                i = np.flatnonzero(got != want)[0]
                raise AssertionError(f"{what}: {name} pool differs first at byte {i} (layer {i // lb}, "
                                     f"block {(i % lb) // page})")

    def clear(blocks):
        if blocks.size:
            dev.evict(to_dev(blocks))  # every layer, one launch
            for r in refs:
                r.evict(blocks)

    def step(seqs, nt):
        plan = mgr.append(seqs, nt, cow=True)
        so, eo, cs, cd = omgr.append(seqs, nt, cow=True)
        np.testing.assert_array_equal(plan.slots, so)
        np.testing.assert_array_equal(plan.evicted, eo)
        np.testing.assert_array_equal(plan.cow_src, cs)
        np.testing.assert_array_equal(plan.cow_dst, cd)
        # Copies before clears before the append: a block freed and
        # allocated again in the same step is cleared, then written.
        if plan.cow_src.size:
            dev.copy_blocks(to_dev(plan.cow_src), to_dev(plan.cow_dst))
            for r in refs:
                for s_, d_ in zip(plan.cow_src, plan.cow_dst):
                    r.k[d_ * page:(d_ + 1) * page] = r.k[s_ * page:(s_ + 1) * page]
                    r.v[d_ * page:(d_ + 1) * page] = r.v[s_ * page:(s_ + 1) * page]
        clear(plan.evicted)
        n = plan.slots.size
        for li in range(L):
            k = kv_values(seed[0], n * hkv * D, orc.BF16).reshape(n, hkv, D)
            v = kv_values(seed[0] + 1, n * hkv * D, orc.BF16).reshape(n, hkv, D)
            seed[0] += 2
            refs[li].append(k, v, plan.slots)
            layers[li].append(to_dev(k.view(np.int16), torch.bfloat16), to_dev(v.view(np.int16), torch.bfloat16),
                              to_dev(plan.slots))
        dev.sync_tables(tables_d, to_dev(plan.token_seq), to_dev(plan.token_pos), to_dev(plan.slots))
        return plan

    def decode(seqs, what):
        t, ctx, st = omgr.tables()
        np.testing.assert_array_equal(mgr.tables()[0], t)
        td = from_dev(tables_d)
        for s in seqs:  # the device table agrees inside each window
            lo, hi = int(st[s]) // bs, (int(ctx[s]) - 1) // bs
            np.testing.assert_array_equal(td[s, lo:hi + 1], t[s, lo:hi + 1])
        sel = np.asarray(seqs)
        for li in range(L):
            q = kv_values(seed[0], len(seqs) * hq * D, orc.BF16).reshape(len(seqs), hq, D)
            seed[0] += 1
            want = refs[li].decode(widen(q, orc.BF16), hq, t[sel], ctx[sel], st[sel], scale)
            out = layers[li].decode(to_dev(q.view(np.int16), torch.bfloat16), tables_d[to_dev(sel).long()].contiguous(),
                                    to_dev(ctx[sel]), to_dev(st[sel]), W, scale=scale, partition=64,
                                    out_dtype=torch.float32)
            dev.check()
            assert_close_or_closer(from_dev(out).reshape(want.shape), want,
                                   lazy(lambda: exact_decode(refs[li], widen(q, orc.BF16), hq, t[sel], ctx[sel],
                                                             st[sel], scale, with_mag=True)),
                                   2e-3, 1e-2, f"{what}: layer {li} seqs {seqs}")

    step([0, 2], [150, 40])  # seq 0 spans its window; seq 2 is unrelated
    check_pools("prefill")
    mgr.fork(0, 1)
    omgr.fork(0, 1)
    # The fork's table row on the device: copy row 0 (sync_tables covers
    # only appended tokens).
    tables_d[1].copy_(tables_d[0])
    shared = set(int(b) for b in mgr.tables()[0][0] if b >= 0)
    assert all(pool.ref_count(b) == 2 for b in shared)
    n_kept = 0
    for i in range(48):  # three block boundaries: both windows release shared blocks
        plan = step([0, 1, 2], [1, 1, 1])
        n_kept += sum(1 for b in shared if pool.ref_count(b) == 1)
        for b in plan.evicted:
            assert pool.ref_count(int(b)) in (0, 1)  # returned (maybe reused in the step)
        if i % 16 == 15:
            check_pools(f"step {i}")
            decode([0, 1, 2], f"step {i}")
    assert n_kept > 0, "the run must pass a state where the window dropped one of two references"
    # Seq 0 finishes: only blocks nobody else holds return to the pool, and
    # seq 1 still reads its shared pages.
    freed = mgr.release(0)
    np.testing.assert_array_equal(freed, omgr.release(0))
    t1 = mgr.tables()[0][1]
    assert not set(freed.tolist()) & set(int(b) for b in t1 if b >= 0)
    clear(freed)
    check_pools("after release")
    decode([1, 2], "after release")
    for i in range(20):
        step([1, 2], [1, 1])
    check_pools("end")
    decode([1, 2], "end")
    for s in (1, 2):
        clear(mgr.release(s))
        omgr.release(s)
    assert pool.num_free() == opool.num_free() == cap
    check_pools("all released")


def test_multi_layer_handle_rejects_per_layer_calls():
    import torch
    from infer_train_amd import BF16, InvalidInput
    from infer_train_amd.kv import PagedKvCache

    dev = PagedKvCache(8, 16, 2, 128, BF16, n_layers=3)
    k = torch.zeros((1, 2, 128), dtype=torch.bfloat16, device="cuda:0")
    slots = torch.zeros(1, dtype=torch.int64, device="cuda:0")
    with pytest.raises(InvalidInput, match="layers"):
        dev.append(k, k, slots)
    with pytest.raises(InvalidInput):
        dev.layer(3)
    dev.layer(2).append(k, k, slots)  # the last layer's view works
    dev.check()
    assert dev.describe().n_layers == 3 and dev.layer(0).describe().n_layers == 1
