"""GPU parity of paged split-K flash-decode (+ combine) and of the Backend
FlashAttention operator against the oracle's flash_attn_f32 restatement.
Tolerances (|got - ref| <= atol + rtol |ref|): fp32 rtol 1e-5 / atol 1e-6;
bf16 rtol 2e-3 / atol 1e-2; softmax accumulates in fp32 throughout."""
import math
import os

import numpy as np
import pytest

import oracle as orc
from kvutil import (assert_close, assert_close_or_closer, exact_decode, from_dev, kv_values, lazy, random_tables,
                    slots_for, to_dev, widen)

pytestmark = pytest.mark.gpu

TOL = {orc.F32: (1e-5, 1e-6), orc.Q8_0: (1e-5, 1e-6), orc.Q4_0: (1e-5, 1e-6), orc.Q4_1: (1e-5, 1e-6),
       orc.Q5_0: (1e-5, 1e-6), orc.Q5_1: (1e-5, 1e-6), orc.BF16: (2e-3, 1e-2), orc.F16: (2e-3, 1e-2)}
QUANT = orc.QUANT_TYPES
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _build(dt, hq, hkv, D, bs, ctx, start=None, nb=None, seed=1, mb=None, vmul=None):
    """Fill oracle + device caches with every position of every sequence
    (V of token i of the append scaled by vmul[i] when given)."""
    import torch
    from infer_train_amd.kv import PagedKvCache

    ctx = np.asarray(ctx, np.int32)
    mb = mb or int(max(1, (ctx.max() + bs - 1) // bs))
    need = int(sum((int(c) + bs - 1) // bs for c in ctx))
    nb = nb or max(need, 1)
    tables = random_tables(seed, ctx, bs, nb, mb)
    seqs, pos = [], []
    for b, c in enumerate(ctx):
        seqs += [b] * int(c)
        pos += list(range(int(c)))
    slots = slots_for(tables, seqs, pos, bs)
    n = len(slots)
    src_dt = orc.F32 if dt in QUANT else dt
    k = kv_values(seed + 10, n * hkv * D, src_dt, outliers=dt in QUANT).reshape(n, hkv, D)
    v = kv_values(seed + 11, n * hkv * D, src_dt, outliers=dt in QUANT).reshape(n, hkv, D)
    if vmul is not None:
        v = (v * np.asarray(vmul, np.float32)[:n, None, None]).astype(np.float32)
    ref = orc.Cache(nb, bs, hkv, D, dt)
    ref.append(k, v, slots)
    dev = PagedKvCache(nb, bs, hkv, D, dt)
    if n:
        if src_dt == orc.F32:
            dk, dv = to_dev(k), to_dev(v)
        else:
            td = torch.bfloat16 if dt == orc.BF16 else torch.float16
            dk, dv = to_dev(k.view(np.int16), td), to_dev(v.view(np.int16), td)
        dev.append(dk, dv, to_dev(slots))
    qdt = orc.F32 if dt in (orc.F32,) + QUANT else dt
    q = kv_values(seed + 12, len(ctx) * hq * D, qdt).reshape(len(ctx), hq, D)
    return dev, ref, tables, ctx, q, qdt


def _run(dev, ref, tables, ctx, q, qdt, hq, start=None, partition=512, out_f32=True):
    import torch

    D = q.shape[2]
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))  # forward.rs:252
    n = ctx - (start if start is not None else 0)
    want = ref.decode(widen(q, qdt), hq, tables, ctx, start, scale)
    if qdt == orc.F32:
        dq = to_dev(q)
    else:
        dq = to_dev(q.view(np.int16), torch.bfloat16 if qdt == orc.BF16 else torch.float16)
    out = dev.decode(dq, to_dev(tables), to_dev(ctx), None if start is None else to_dev(start),
                     max(int(n.max()), 0), scale=scale, partition=partition,
                     out_dtype=torch.float32 if out_f32 else dq.dtype)
    dev.check()
    got = from_dev(out)
    if not out_f32 and qdt != orc.F32:
        got = widen(got, qdt)
    return got.reshape(want.shape), want


def test_config1_fp32_decode():
    """Config 1: Hq 12, Hkv 2, D 128, bs 16, one sequence of 1024 tokens over
    a 64-block pool with the identity table."""
    import torch
    from infer_train_amd.kv import PagedKvCache

    hq, hkv, D, bs = 12, 2, 128, 16
    k = kv_values(101, 1024 * hkv * D, orc.F32).reshape(1024, hkv, D)
    v = kv_values(102, 1024 * hkv * D, orc.F32).reshape(1024, hkv, D)
    q = kv_values(103, hq * D, orc.F32).reshape(1, hq, D)
    tables = np.arange(64, dtype=np.int32)[None, :]
    slots = np.arange(1024, dtype=np.int64)
    ref = orc.Cache(64, bs, hkv, D, orc.F32)
    ref.append(k, v, slots)
    dev = PagedKvCache(64, bs, hkv, D, orc.F32)
    dev.append(to_dev(k[:1023]), to_dev(v[:1023]), to_dev(slots[:1023]))
    dev.append(to_dev(k[1023:]), to_dev(v[1023:]), to_dev(slots[1023:]))
    ctx = np.array([1024], np.int32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    want = ref.decode(q, hq, tables, ctx, None, scale)
    out = dev.decode(to_dev(q), to_dev(tables), to_dev(ctx), None, 1024, scale=scale)
    dev.check()
    got = from_dev(out)
    assert_close(got, want, *TOL[orc.F32], what="config1")
    golden = np.load(os.path.join(GOLDEN, "config1_decode_out.npy"))
    assert_close(got.reshape(golden.shape), golden, *TOL[orc.F32], what="config1 golden")


@pytest.mark.parametrize("partition", [512, 256, 1024])
def test_config2_shape_bf16_ragged(partition):
    """Config-2 heads (Hq 28, Hkv 4, D 128, bs 16) with ragged contexts that
    exercise partial pages and partitions."""
    hq, hkv, D, bs = 28, 4, 128, 16
    ctx = [1, 15, 16, 17, 511, 512, 513, 1500, 2049, 0]
    dev, ref, tables, ctx, q, qdt = _build(orc.BF16, hq, hkv, D, bs, ctx, seed=3, nb=400)
    for out_f32 in (True, False):
        got, want = _run(dev, ref, tables, ctx, q, qdt, hq, partition=partition, out_f32=out_f32)
        assert_close(got, want, *TOL[orc.BF16], what=f"config2 ragged P={partition} f32out={out_f32}")
    assert np.all(got[-1] == 0)  # empty sequence -> zeros (flash_attn.rs:66-71)


def test_config2_full_size_bf16():
    """Config 2 at full size: B 32, ctx U[256, 4096] (+1 appended), pool of
    16384 blocks in seeded random order."""
    hq, hkv, D, bs = 28, 4, 128, 16
    ctx = orc.uniform_i32(2, 256, 4096, 32) + 1
    dev, ref, tables, ctx, q, qdt = _build(orc.BF16, hq, hkv, D, bs, ctx, seed=2, nb=16384, mb=257)
    got, want = _run(dev, ref, tables, ctx, q, qdt, hq, partition=512, out_f32=False)
    assert_close(got, want, *TOL[orc.BF16], what="config2 full")


def test_headline_config2_4k_full_size():
    """The headline workload itself: 32 sequences x 4096 tokens (Hq 28, Hkv
    4, D 128, bs 16) over a 16384-block pool in seeded random order,
    512-token partitions, bf16 q.  The 16-bit decode rounds the softmax
    weights to bf16 before P.V; the printed margin (max over elements of
    |got - ref| / (atol + rtol |ref|), 1.0 = at the tolerance) records what
    that leaves of the bf16 tolerance."""
    hq, hkv, D, bs = 28, 4, 128, 16
    ctx = np.full(32, 4096, np.int32)
    dev, ref, tables, ctx, q, qdt = _build(orc.BF16, hq, hkv, D, bs, ctx, seed=44, nb=16384, mb=256)
    rtol, atol = TOL[orc.BF16]
    margins = []
    for out_f32 in (False, True):
        got, want = _run(dev, ref, tables, ctx, q, qdt, hq, partition=512, out_f32=out_f32)
        assert_close(got, want, rtol, atol, what=f"headline f32out={out_f32}")
        err = np.abs(got.astype(np.float64) - want)
        margins.append(float((err / (atol + rtol * np.abs(want))).max()))
        print(f"headline 32x4096 out {'f32' if out_f32 else 'bf16'}: max |err| {err.max():.3g}, "
              f"{margins[-1]:.3f} of the bf16 tolerance")
    assert max(margins) < 1.0


def test_many_sequences_unit_mapping():
    """Workgroups run the non-empty (sequence, head, partition) units in
    order, found by a prefix sum over the context lengths 64 sequences at a
    time: 130 sequences (three scan steps) with empty ones (ctx 0, and a
    window start equal to ctx), windows, and 64-token partitions; the
    partition the host planner picks for the batch; and 600 sequences, past
    the 512 the scan takes, where workgroups map to units by grid index."""
    hq, hkv, D, bs = 8, 2, 128, 16
    rng = np.random.default_rng(41)
    ctx = rng.integers(0, 300, 130).astype(np.int32)
    ctx[[0, 63, 64, 127, 129]] = 0
    start = np.minimum(rng.integers(0, 100, 130), ctx).astype(np.int32)
    start[[5, 70, 128]] = ctx[[5, 70, 128]]
    dev, ref, tables, ctx, q, qdt = _build(orc.BF16, hq, hkv, D, bs, ctx, seed=41)
    p_host = dev.decode_partition(hq, ctx, start)
    assert 64 <= p_host <= 2048 and p_host % 64 == 0
    for partition in (64, 128, p_host):
        got, want = _run(dev, ref, tables, ctx, q, qdt, hq, start=start, partition=partition)
        assert_close(got, want, *TOL[orc.BF16], what=f"130 seqs P={partition}")
        n = ctx - start
        assert np.all(got[n <= 0] == 0)
    ctx2 = rng.integers(0, 40, 600).astype(np.int32)
    dev, ref, tables, ctx2, q, qdt = _build(orc.BF16, hq, hkv, D, bs, ctx2, seed=42)
    got, want = _run(dev, ref, tables, ctx2, q, qdt, hq, partition=64)
    assert_close(got, want, *TOL[orc.BF16], what="600 seqs")


@pytest.mark.parametrize("D", [128, 256])
def test_many_partitions_per_row(D):
    """Rows with 1, 33, 100 and 141 partitions of 64 tokens: the combine
    prefetches 32 partials per lane, weighs partitions 0-63 and 64-127 from
    the lanes holding their (m, l) pairs, and reads the pairs of partitions
    128 and up directly; every range is crossed.  fp32 and bf16 output, a
    128- and a 256-dim head (one and two combine slices per row)."""
    hq, hkv, bs = 8, 2, 16
    ctx = [3, 2100, 6400, 9000]  # 1, 33, 100, 141 partitions
    dev, ref, tables, c, q, qdt = _build(orc.BF16, hq, hkv, D, bs, ctx, seed=31)
    for out_f32 in (True, False):
        got, want = _run(dev, ref, tables, c, q, qdt, hq, partition=64, out_f32=out_f32)
        assert_close(got, want, *TOL[orc.BF16], what=f"many partitions D={D} f32out={out_f32}")


def test_uniform_lengths():
    """Equal lengths without start positions (the headline's shape at a
    smaller batch): full and partial last partitions, 64- and 512-token
    partitions, and one sequence shorter than the rest, which shifts the
    unit order of every workgroup after it."""
    hq, hkv, D, bs = 28, 4, 128, 16
    for ctx in ([2048] * 12, [1000] * 9, [1536] * 5 + [700] + [1536] * 4):
        dev, ref, tables, c, q, qdt = _build(orc.BF16, hq, hkv, D, bs, ctx, seed=12)
        for partition in (512, 64):
            got, want = _run(dev, ref, tables, c, q, qdt, hq, partition=partition)
            assert_close(got, want, *TOL[orc.BF16], what=f"uniform {ctx[0]} x {len(ctx)} P={partition}")


@pytest.mark.parametrize("n_seqs", [3, 600])
def test_negative_start_is_skipped_and_latched(n_seqs):
    """A negative start position is skipped, as the gather skips it: that
    sequence's output is zeros, the others are unaffected, and
    it_kv_cache_check reports the condition.  3 sequences take the compact
    unit scan, 600 the grid mapping."""
    import torch
    from infer_train_amd import InvalidInput

    hq, hkv, D, bs = 8, 2, 128, 16
    rng = np.random.default_rng(7)
    ctx = np.array([300, 200, 500], np.int32) if n_seqs == 3 else rng.integers(1, 40, n_seqs).astype(np.int32)
    dev, ref, tables, ctx, q, qdt = _build(orc.BF16, hq, hkv, D, bs, ctx, seed=8)
    start = np.zeros(n_seqs, np.int32)
    start[-1] = min(5, int(ctx[-1]) - 1)
    bad = 1
    start[bad] = -3
    ok_start = start.copy()
    ok_start[bad] = 0
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    want = ref.decode(widen(q, qdt), hq, tables, ctx, ok_start, scale)
    out = dev.decode(to_dev(q.view(np.int16), torch.bfloat16), to_dev(tables), to_dev(ctx), to_dev(start),
                     int(ctx.max()), scale=scale, partition=64, out_dtype=torch.float32)
    with pytest.raises(InvalidInput, match="negative-start"):
        dev.check()
    got = from_dev(out).reshape(want.shape)
    assert np.all(got[bad] == 0)
    keep = np.arange(n_seqs) != bad
    assert_close(got[keep], want[keep], *TOL[orc.BF16], what=f"negative start, {n_seqs} seqs")
    dev.check()  # the flag was cleared


def test_misaligned_out_is_rejected():
    """The combine stores two adjacent output elements at once, so out must
    be 8-byte aligned for F32 and 4-byte aligned for 16-bit types:
    InvalidInput before any launch, nothing written."""
    import torch
    from infer_train_amd import InvalidInput

    hq, hkv, D, bs = 8, 2, 128, 16
    dev, ref, tables, ctx, q, qdt = _build(orc.BF16, hq, hkv, D, bs, [100, 50], seed=3)
    qd = to_dev(q.view(np.int16), torch.bfloat16)
    for dt in (torch.float32, torch.bfloat16):
        buf = torch.zeros(2 * hq * D + 1, dtype=dt, device="cuda:0")
        with pytest.raises(InvalidInput, match="aligned"):
            dev.decode(qd, to_dev(tables), to_dev(ctx), None, int(ctx.max()), out=buf[1:].view(2, hq, D))
        assert not bool(buf.any())


def test_config5_full_size_q8_0():
    """Config 5 at full size: Q8_0, Hq 24 / Hkv 4 / D 256, block 32, 16
    sequences of U[32768, 131072] tokens over a seeded permutation of the
    pool, fp32 N(0,1) sources with 1% of elements x8 (the config's
    outliers), the planner's partition (1792 tokens: up to 74 partials
    merged per row).
      - Quantised bytes: 4096 sampled (token, head) rows of each append
        chunk, their device records equal the oracle's quantize_row_q8_0 of
        the same fp32 source rows, bit for bit.
      - Attention: the oracle decodes all 16 sequences (all 24 heads; the
        longest merges 74 partials) over the same pages (the device pools
        copied into an oracle cache).
      - A second decode at 1024-token partitions agrees with the first."""
    import os as _os

    import torch
    from infer_train_amd.kv import PagedKvCache

    hq, hkv, D, bs = 24, 4, 256, 32
    G = D // 32
    ctx = np.random.default_rng(5).integers(32768, 131073, 16).astype(np.int32)
    nblk = (ctx + bs - 1) // bs
    nb, mb = int(nblk.sum()), int(nblk.max())
    tables = random_tables(55, ctx, bs, nb, mb)
    dev = PagedKvCache(nb, bs, hkv, D, orc.Q8_0)
    seqs = np.repeat(np.arange(16), ctx)
    pos = np.concatenate([np.arange(c) for c in ctx])
    slots = tables[seqs, pos // bs].astype(np.int64) * bs + pos % bs
    g = torch.Generator(device="cuda:0")
    g.manual_seed(55)
    rng = np.random.default_rng(57)
    step = 1 << 16
    page_bytes = dev.page_bytes
    kpool = dev.k_pool.view(torch.uint8).view(nb, hkv, page_bytes)
    checked = 0
    for s0 in range(0, slots.size, step):
        n = min(step, slots.size - s0)
        k = torch.randn((n, hkv, D), generator=g, device="cuda:0")
        v = torch.randn((n, hkv, D), generator=g, device="cuda:0")
        k[torch.rand((n, hkv, D), generator=g, device="cuda:0") < 0.01] *= 8
        v[torch.rand((n, hkv, D), generator=g, device="cuda:0") < 0.01] *= 8
        dev.append(k, v, to_dev(slots[s0:s0 + n]))
        # Sampled rows of this chunk: device records = the oracle's quantiser.
        rows = rng.integers(0, n, 4096)
        heads = rng.integers(0, hkv, 4096)
        src = k[torch.from_numpy(rows).cuda(), torch.from_numpy(heads).cuda()].cpu().numpy()
        sl = slots[s0 + rows]
        blk, tok = sl // bs, sl % bs
        pages = kpool[torch.from_numpy(blk).cuda(), torch.from_numpy(heads).cuda()].cpu().numpy()
        qs = pages[np.arange(4096)[:, None], tok[:, None] * D + np.arange(D)[None, :]]
        dbytes = pages[np.arange(4096)[:, None], bs * D + tok[:, None] * (2 * G) + np.arange(2 * G)[None, :]]
        rec = np.concatenate([dbytes.reshape(4096, G, 2), qs.reshape(4096, G, 32)], axis=2)
        want_rec = np.stack([orc.quantize_row_q8_0(src[i]) for i in range(4096)])
        np.testing.assert_array_equal(rec.reshape(want_rec.shape), want_rec,
                                      err_msg=f"Q8_0 records of chunk at {s0}")
        checked += 4096
        del k, v
    dev.check()
    assert checked >= 16 * 4096
    q = kv_values(56, 16 * hq * D, orc.F32).reshape(16, hq, D)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    p_plan = dev.decode_partition(hq, ctx)
    assert p_plan == 1792
    outs = {}
    for partition in (p_plan, 1024):
        out = dev.decode(to_dev(q), to_dev(tables), to_dev(ctx), None, int(ctx.max()), scale=scale,
                         partition=partition)
        dev.check()
        outs[partition] = from_dev(out)
    assert_close(outs[1024], outs[p_plan], *TOL[orc.Q8_0], what="config5 1024 vs planner partition")

    # The oracle over every sequence, on the device's pages.
    assert -(-int(ctx.max()) // p_plan) >= 60  # the longest merges many partials
    ref = orc.Cache(nb, bs, hkv, D, orc.Q8_0)
    ref.k[:] = from_dev(dev.k_pool).reshape(-1)
    ref.v[:] = from_dev(dev.v_pool).reshape(-1)
    threads = max(1, min(16, len(_os.sched_getaffinity(0))))
    want = ref.decode(q, hq, tables, ctx, None, scale, threads=threads)
    exact = lazy(lambda: exact_decode(ref, q, hq, tables, ctx, None, scale, with_mag=True))
    got = outs[p_plan].reshape(want.shape)
    assert_close_or_closer(got, want, exact, *TOL[orc.Q8_0], what="config5 full, all 16 sequences")


@pytest.mark.parametrize("dt", [orc.F16, orc.F32])
def test_other_dtypes(dt):
    hq, hkv, D, bs = 8, 2, 128, 16
    dev, ref, tables, ctx, q, qdt = _build(dt, hq, hkv, D, bs, [700, 64, 1], seed=5)
    got, want = _run(dev, ref, tables, ctx, q, qdt, hq)
    assert_close(got, want, *TOL[dt], what=f"dtype {dt}")


def test_window_start_positions_bf16():
    """Config-4 heads (Hq 16, Hkv 2, G 8) reading only [start, ctx)."""
    hq, hkv, D, bs = 16, 2, 128, 16
    ctx = np.array([900, 1200, 300, 4097], np.int32)
    start = np.array([0, 1200 - 777, 299, 4097 - 4096], np.int32)
    dev, ref, tables, ctx, q, qdt = _build(orc.BF16, hq, hkv, D, bs, ctx, seed=6)
    got, want = _run(dev, ref, tables, ctx, q, qdt, hq, start=start)
    assert_close(got, want, *TOL[orc.BF16], what="window")


def test_q8_0_decode_d256():
    """Config-5 heads (Hq 24, Hkv 4, D 256, bs 32) on a Q8_0 cache; fp32 q and
    fp32 tolerance against the oracle on the same quantised cache."""
    hq, hkv, D, bs = 24, 4, 256, 32
    dev, ref, tables, ctx, q, qdt = _build(orc.Q8_0, hq, hkv, D, bs, [3000, 1025, 33], seed=7)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    exact = lazy(lambda: exact_decode(ref, q, hq, tables, ctx, None, scale, with_mag=True))
    for partition in (512, 1024, 2048):
        got, want = _run(dev, ref, tables, ctx, q, qdt, hq, partition=partition)
        assert_close_or_closer(got, want, exact, *TOL[orc.Q8_0], what=f"q8_0 P={partition}")


@pytest.mark.parametrize("dt", [orc.BF16, orc.F16, orc.F32] + list(QUANT))
def test_window_starts_inside_a_page(dt):
    """Windows that start inside a 16-token page: every 16-token group of the
    window straddles two pages (rows [0, 16 - start % 16) in one, the rest in
    the next; each lane looks up its own row's page).  The
    positions of the first page before the window start are overwritten
    with +inf K and V (16-bit caches hold inf, quantised blocks inf / NaN
    scales): a read of any of them turns the output into inf / NaN.  Starts
    5, 21, 15, 47 (in-page offsets 5, 5, 15, 15) and 32 (page-aligned);
    windows of 1 token, of whole partitions and with a short last one."""
    hq, hkv, D, bs, P = 8, 2, 128, 16, 64
    start = np.array([5, 21, 15, 32, 47, 5], np.int32)
    n = np.array([128, 64, 1, 100, 64, 193], np.int32)
    ctx = start + n
    dev, ref, tables, ctx_a, q, qdt = _build(dt, hq, hkv, D, bs, ctx, seed=77)
    seqs, pos = [], []
    for b, s in enumerate(start):
        lo = int(s) - int(s) % 16
        seqs += [b] * (int(s) - lo)
        pos += list(range(lo, int(s)))
    slots = slots_for(tables, seqs, pos, bs)
    m = len(slots)
    import torch
    if dt in (orc.BF16, orc.F16):
        bits = np.full((m, hkv, D), 0x7F80 if dt == orc.BF16 else 0x7C00, np.uint16).view(np.int16)
        td = torch.bfloat16 if dt == orc.BF16 else torch.float16
        pk = to_dev(bits, td)
        dev.append(pk, pk, to_dev(slots))
    else:
        inf = to_dev(np.full((m, hkv, D), np.inf, np.float32))
        dev.append(inf, inf, to_dev(slots))
    got, want = _run(dev, ref, tables, ctx_a, q, qdt, hq, start=start, partition=P)
    assert np.all(np.isfinite(got)), "a position before the window leaked into the output"
    if dt in QUANT:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
        assert_close_or_closer(got, want, lambda: exact_decode(ref, q, hq, tables, ctx_a, start, scale, with_mag=True),
                               *TOL[dt], what=f"dt={dt} aligned window partitions")
    else:
        assert_close(got, want, *TOL[dt], what=f"dt={dt} aligned window partitions")


@pytest.mark.parametrize("dt", QUANT)
@pytest.mark.parametrize("D", [128, 256])
def test_quant_group_sizes_and_windows(dt, D):
    """Q8_0, Q4_0, Q4_1, Q5_0 and Q5_1 (products on MFMA) at every heads-per-workgroup count
    1..8 (the tiles' padding rows and the second row of four heads), contexts
    that end inside a 16-token group and inside a page, window start
    positions, and two partition sizes; fp32 tolerance against the oracle."""
    bs = 32 if D == 256 else 16
    ctx = [1, 17, 100, 333, 0]
    start = np.array([0, 5, 37, 300, 0], np.int32)
    for hq, hkv in ((1, 1), (2, 1), (6, 2), (4, 1), (10, 2), (18, 3), (21, 3), (8, 1)):
        dev, ref, tables, ctx_a, q, qdt = _build(dt, hq, hkv, D, bs, ctx, seed=40 + hq)
        for partition in (64, 256):
            got, want = _run(dev, ref, tables, ctx_a, q, qdt, hq, start=start, partition=partition)
            scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
            assert_close_or_closer(got, want, lambda: exact_decode(ref, q, hq, tables, ctx_a, start, scale, with_mag=True),
                                   *TOL[dt],
                                   what=f"dt={dt} D={D} hq={hq} hkv={hkv} P={partition}")
        assert np.all(got[-1] == 0)


@pytest.mark.parametrize("dt", QUANT)
def test_quant_block_size_8(dt):
    """8-token pages: every 16-token group straddles two pages, so each lane
    looks up its own page for the main rows and the scale rows."""
    hq, hkv, D, bs = 12, 2, 128, 8
    ctx = [9, 300, 1037]
    start = np.array([0, 3, 500], np.int32)
    dev, ref, tables, ctx_a, q, qdt = _build(dt, hq, hkv, D, bs, ctx, seed=71)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    exact = lazy(lambda: exact_decode(ref, q, hq, tables, ctx_a, start, scale, with_mag=True))
    for partition in (64, 512):
        got, want = _run(dev, ref, tables, ctx_a, q, qdt, hq, start=start, partition=partition)
        assert_close_or_closer(got, want, exact, *TOL[dt], what=f"dt={dt} bs=8 P={partition}")


@pytest.mark.parametrize("dt", [orc.Q4_0, orc.Q4_1, orc.Q5_0, orc.Q5_1])
def test_nibble_decode_config5_heads(dt):
    """Config-5 heads (Hq 24, Hkv 4, D 256, bs 32) on a Q4_0 / Q4_1 / Q5_0 /
    Q5_1 cache."""
    hq, hkv, D, bs = 24, 4, 256, 32
    dev, ref, tables, ctx, q, qdt = _build(dt, hq, hkv, D, bs, [3000, 1025, 33], seed=9)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    exact = lazy(lambda: exact_decode(ref, q, hq, tables, ctx, None, scale, with_mag=True))
    for partition in (512, 1024):
        got, want = _run(dev, ref, tables, ctx, q, qdt, hq, partition=partition)
        assert_close_or_closer(got, want, exact, *TOL[dt], what=f"dt={dt} P={partition}")


@pytest.mark.parametrize("dt", QUANT)
@pytest.mark.parametrize("D", [128, 256])
def test_quant_v_scale_ranges(dt, D):
    """V scales of every range the decode distinguishes: runs of 37 tokens
    whose V is scaled by 2^17 (Q8_0 scales above 512, nibble scales above
    4096: those 16-token items take the three-part bf16 products), by 2^-12
    (subnormal fp16 scales) or left at N(0, 1), so items of one wave mix
    the ranges and an item's tokens may straddle two; fp32 tolerance against
    the oracle."""
    bs = 32 if D == 256 else 16
    ctx = [700, 333, 1029]
    n = sum(ctx)
    run = (np.arange(n) // 37) % 3
    vmul = np.where(run == 0, np.float32(2.0**17), np.where(run == 1, np.float32(2.0**-12), np.float32(1)))
    hq, hkv = (24, 4) if D == 256 else (8, 2)
    dev, ref, tables, ctx_a, q, qdt = _build(dt, hq, hkv, D, bs, ctx, seed=77, vmul=vmul)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    exact = lazy(lambda: exact_decode(ref, q, hq, tables, ctx_a, None, scale, with_mag=True))
    for partition in (64, 512):
        got, want = _run(dev, ref, tables, ctx_a, q, qdt, hq, partition=partition)
        assert_close_or_closer(got, want, exact, *TOL[dt], what=f"dt={dt} D={D} P={partition}")


def test_bf16_d256_and_group_sizes():
    for hq, hkv in ((3, 1), (10, 2), (12, 12)):
        dev, ref, tables, ctx, q, qdt = _build(orc.BF16, hq, hkv, 256, 16, [333, 1029], seed=8)
        got, want = _run(dev, ref, tables, ctx, q, qdt, hq)
        assert_close(got, want, *TOL[orc.BF16], what=f"bf16 d256 hq={hq} hkv={hkv}")


def test_backend_flash_attention_op():
    """CoreOperator::FlashAttention contract (arm.rs:304-370): K/V shared by
    all heads, optional additive mask with -inf keys skipped."""
    import torch
    from infer_train_amd.kv import flash_attention

    for n_heads, D, n_kv in ((12, 128, 1024), (7, 256, 77), (4, 128, 1)):
        q = kv_values(30, n_heads * D, orc.F32).reshape(n_heads, D)
        k = kv_values(31, n_kv * D, orc.F32).reshape(n_kv, D)
        v = kv_values(32, n_kv * D, orc.F32).reshape(n_kv, D)
        mask = (orc.normal(33, n_kv) * np.float32(2)).astype(np.float32)
        mask[::5] = -np.inf
        if n_kv == 1:
            mask[:] = 0
        for m in (None, mask):
            want = orc.backend_flash_attention(q, k, v, m)
            got = flash_attention(to_dev(q), to_dev(k), to_dev(v), None if m is None else to_dev(m))
            torch.cuda.synchronize()
            assert_close(from_dev(got), want, *TOL[orc.F32], what=f"backend op H={n_heads} D={D} n={n_kv}")
    # all keys masked -> zeros, as flash_attn_f32 leaves them
    q = kv_values(34, 4 * 128, orc.F32).reshape(4, 128)
    k = kv_values(35, 10 * 128, orc.F32).reshape(10, 128)
    got = flash_attention(to_dev(q), to_dev(k), to_dev(k), to_dev(np.full(10, -np.inf, np.float32)))
    torch.cuda.synchronize()
    assert np.all(from_dev(got) == 0)


def test_decode_graph_replay():
    """append + split + combine captured in a HIP graph: every replay, with
    eager decodes and synchronisations between replays, equals the eager
    result bit for bit (the kernels sum in a fixed order)."""
    import torch

    hq, hkv, D, bs = 28, 4, 128, 16
    dev, ref, tables, ctx, q, qdt = _build(orc.BF16, hq, hkv, D, bs, [300, 17, 1023, 512], seed=9)
    dq = to_dev(q.view(np.int16), torch.bfloat16)
    t_d, c_d = to_dev(tables), to_dev(ctx)
    max_t = int(ctx.max())
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    ws = dev.decode_workspace(len(ctx), hq, max_t, 512)
    out_g = torch.empty(dq.shape, dtype=torch.float32, device=dq.device)
    out_e = torch.empty_like(out_g)
    dev.decode(dq, t_d, c_d, None, max_t, scale=scale, out=out_e, ws=ws)
    torch.cuda.synchronize()
    eager = out_e.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dev.decode(dq, t_d, c_d, None, max_t, scale=scale, out=out_g, ws=ws)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dev.decode(dq, t_d, c_d, None, max_t, scale=scale, out=out_g, ws=ws)
    for _ in range(3):
        out_g.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager), "graph replay differs from the eager decode"
        dev.decode(dq, t_d, c_d, None, max_t, scale=scale, out=out_e, ws=ws)
        torch.cuda.synchronize()
        assert torch.equal(out_e, eager)
    dev.check()
    want = ref.decode(widen(q, qdt), hq, tables, ctx, None, scale)
    assert_close(from_dev(out_g).reshape(want.shape), want, *TOL[orc.BF16], what="graph replay vs oracle")
