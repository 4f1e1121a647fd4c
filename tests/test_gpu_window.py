"""Config-4 path end to end on the GPU: sliding-window ring cache with
eviction and block recycling.  Each step the host manager (slot mapping,
window release, LIFO reuse) plans the append; the device clears the freed
pages (evict) before appending, syncs its block tables from the slot
mapping, and runs split-K decode over the last W positions.  Pools must equal
the oracle's byte for byte; outputs must be within bf16 tolerance of the
oracle's flash_attn_f32 over the same window."""
import os

import numpy as np
import pytest

import oracle as orc
from kvutil import assert_close, from_dev, kv_values, to_dev, widen

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-2
THREADS = max(1, min(16, len(os.sched_getaffinity(0))))  # host threads for the oracle's decode


def _window_run(n_seqs, hq, hkv, W, start, steps, cap, seed, check_every, D=128, bs=16):
    import torch
    from infer_train_amd import BF16, BlockPool, KvManager
    from infer_train_amd.kv import PagedKvCache

    order = orc.permutation(seed, cap)
    pool, opool = BlockPool(cap, BF16, order=order), orc.Pool(cap, orc.BF16, order=order)
    mb = (start + steps) // bs + 2
    mgr, omgr = KvManager(pool, bs, n_seqs, mb, W), orc.Manager(opool, bs, n_seqs, mb, W)
    first, last = (start - W) // bs, (start - 1) // bs
    dev = PagedKvCache(cap, bs, hkv, D, BF16)
    ref = orc.Cache(cap, bs, hkv, D, orc.BF16)
    tables_d = torch.full((n_seqs, mb), -1, dtype=torch.int32, device="cuda:0")
    # Seed every sequence with the blocks of positions [first*bs, start) and fill them.
    seqs, pos, slots = [], [], []
    for s in range(n_seqs):
        blocks = [pool.allocate() for _ in range(last - first + 1)]
        assert blocks == [opool.allocate() for _ in range(last - first + 1)]
        mgr.seed_seq(s, start, first, blocks)
        omgr.seed_seq(s, start, first, blocks)
        for p in range(first * bs, start):
            seqs.append(s)
            pos.append(p)
            slots.append(blocks[p // bs - first] * bs + p % bs)
    slots = np.asarray(slots, np.int64)
    n = slots.size
    k = kv_values(seed + 1, n * hkv * D, orc.BF16).reshape(n, hkv, D)
    v = kv_values(seed + 2, n * hkv * D, orc.BF16).reshape(n, hkv, D)
    ref.append(k, v, slots)
    dev.append(to_dev(k.view(np.int16), torch.bfloat16), to_dev(v.view(np.int16), torch.bfloat16), to_dev(slots))
    dev.sync_tables(tables_d, to_dev(np.asarray(seqs, np.int32)), to_dev(np.asarray(pos, np.int32)), to_dev(slots))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    n_evicted = 0
    for step in range(steps):
        plan = mgr.append(list(range(n_seqs)))
        oslots, oev = omgr.append(list(range(n_seqs)))
        np.testing.assert_array_equal(plan.slots, oslots)
        np.testing.assert_array_equal(plan.evicted, oev)
        n_evicted += plan.evicted.size
        # Freed pages are cleared before the append: LIFO reuse can hand a
        # block freed by one sequence to a later sequence of the same step.
        if plan.evicted.size:
            ref.evict(plan.evicted)
            dev.evict(to_dev(plan.evicted))
        kn = kv_values(seed + 100 + step, n_seqs * hkv * D, orc.BF16).reshape(n_seqs, hkv, D)
        vn = kv_values(seed + 200 + step, n_seqs * hkv * D, orc.BF16).reshape(n_seqs, hkv, D)
        ref.append(kn, vn, plan.slots)
        dev.append(to_dev(kn.view(np.int16), torch.bfloat16), to_dev(vn.view(np.int16), torch.bfloat16),
                   to_dev(plan.slots))
        dev.sync_tables(tables_d, to_dev(plan.token_seq), to_dev(plan.token_pos), to_dev(plan.slots))
        if (step + 1) % check_every == 0 or step == steps - 1:
            t, ctx, st = omgr.tables()
            np.testing.assert_array_equal(st, np.maximum(ctx - W, 0))
            q = kv_values(seed + 300 + step, n_seqs * hq * D, orc.BF16).reshape(n_seqs, hq, D)
            out = dev.decode(to_dev(q.view(np.int16), torch.bfloat16), tables_d, to_dev(ctx), to_dev(st), W,
                             scale=scale, out_dtype=torch.float32)
            dev.check()
            want = ref.decode(widen(q, orc.BF16), hq, t, ctx, st, scale, threads=THREADS)
            assert_close(from_dev(out), want, RTOL, ATOL, what=f"window decode step {step}")
            np.testing.assert_array_equal(from_dev(dev.k_pool), ref.k)
            np.testing.assert_array_equal(from_dev(dev.v_pool), ref.v)
    assert n_evicted > 0, "the run must cross at least one eviction"
    return n_evicted


def test_window_small_unaligned():
    """8 sequences, W 256, starting at position 1000 (not block aligned), 48
    steps: allocations, releases and same-step reuse of freed blocks."""
    _window_run(n_seqs=8, hq=16, hkv=2, W=256, start=1000, steps=48, cap=160, seed=41, check_every=6)


def test_window_config4_full_size():
    """Config 4 at full size: 64 sequences, Hq 16 / Hkv 2, W 4096, from
    position 30000, pool of 16512 blocks in seeded order; 256 steps cross 16
    allocate / free cycles (allocations at p = 30000, 30016, ..., releases
    at p = 30015, 30031, ..., LIFO hand-offs between sequences), with slots
    and frees equal to the oracle's at every step, and the pools compared
    byte for byte and a decode checked once per cycle."""
    n_ev = _window_run(n_seqs=64, hq=16, hkv=2, W=4096, start=30000, steps=256, cap=16512, seed=4, check_every=16)
    assert n_ev == 64 * 16  # one block per sequence per cycle
