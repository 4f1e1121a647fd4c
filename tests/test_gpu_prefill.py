"""GPU parity of chunked-prefill attention (MFMA) against the oracle's
flash_attn_f32 restatement driven per query row (causal: keys 0..position).
bf16 tolerance |got - ref| <= 1e-2 + 2e-3 |ref|; softmax accumulates in fp32.
The chunk's own K/V are appended through the cache's append kernel first,
exactly as a caller of the chunked-prefill path does."""
import numpy as np
import pytest

import oracle as orc
from kvutil import assert_close, from_dev, kv_values, random_tables, slots_for, to_dev, widen

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-2


def _setup(dt, hq, hkv, ctx, q_lens, seed, nb=None, bs=16, D=128, k_gain=None, mb=None):
    """Paged cache holding every position of every sequence (cached prefix
    and chunk), the chunk's queries, and the tables.  k_gain(pos) scales the
    K row at position pos (then rounded to the cache dtype)."""
    import torch
    from infer_train_amd.kv import PagedKvCache

    ctx = np.asarray(ctx, np.int32)
    q_lens = np.asarray(q_lens, np.int32)
    mb = max(int((ctx.max() + bs - 1) // bs), mb or 0)
    need = int(sum((int(c) + bs - 1) // bs for c in ctx))
    nb = nb or need + 3
    tables = random_tables(seed, ctx, bs, nb, mb)
    seqs, pos = [], []
    for b, c in enumerate(ctx):
        seqs += [b] * int(c)
        pos += list(range(int(c)))
    slots = slots_for(tables, seqs, pos, bs)
    n = len(slots)
    k = kv_values(seed + 1, n * hkv * D, dt).reshape(n, hkv, D)
    if k_gain is not None:
        g = np.array([k_gain(p) for p in pos], np.float32)[:, None, None]
        kf = widen(k, dt) * g
        k = orc.f32_to_bf16(kf) if dt == orc.BF16 else orc.f32_to_f16(kf)
    v = kv_values(seed + 2, n * hkv * D, dt).reshape(n, hkv, D)
    ref = orc.Cache(nb, bs, hkv, D, dt)
    ref.append(k, v, slots)
    dev = PagedKvCache(nb, bs, hkv, D, dt)
    td = torch.bfloat16 if dt == orc.BF16 else torch.float16
    dev.append(to_dev(k.view(np.int16), td), to_dev(v.view(np.int16), td), to_dev(slots))
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    q = kv_values(seed + 3, int(cu[-1]) * hq * D, dt).reshape(int(cu[-1]), hq, D)
    return dev, ref, tables, ctx, cu, q, td


def _run(dev, tables, ctx, cu, q, td, hq, causal=True, out_f32=True, scale=None):
    import torch

    D = q.shape[2]
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    dq = to_dev(q.view(np.int16), td)
    max_q = int(np.max(np.diff(cu)))
    out = dev.prefill(dq, to_dev(cu), max_q, to_dev(tables), to_dev(ctx), scale=scale, causal=causal,
                      out_dtype=torch.float32 if out_f32 else td)
    dev.check()
    return out, scale


@pytest.mark.parametrize("dt", [orc.BF16, orc.F16])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (4, 4), (6, 3), (16, 2), (6, 2), (5, 1), (7, 1)])
def test_prefill_small_causal(dt, hq, hkv):
    """Ragged chunks: partial 32-row query blocks and 64-key blocks, chunk
    lengths 1 and whole-context, GQA groups 4, 1, 2, 8, 3, 5, 7 (workgroups
    of 8, 8, 8, 8, 6, 5, 7 waves)."""
    ctx = [100, 37, 64, 1, 200]
    q_lens = [45, 37, 1, 1, 70]
    dev, ref, tables, ctx, cu, q, td = _setup(dt, hq, hkv, ctx, q_lens, seed=11 + hq)
    out, scale = _run(dev, tables, ctx, cu, q, td, hq)
    want = ref.prefill(widen(q, dt), hq, cu, tables, ctx, scale, causal=True)
    assert_close(from_dev(out), want, RTOL, ATOL, what=f"prefill dt={dt} hq={hq} hkv={hkv}")


def test_prefill_longest_first_order_with_tail_workgroups():
    """Workgroup ids are dealt to XCDs as 8 ranges; an XCD holding whole
    (sequence, KV head) pairs takes its query blocks longest first.  Here 9
    sequences x 2 KV heads x 2 query blocks of 64 rows = 36 workgroups:
    ranges of 4 (2 pairs each, so the remap is not the identity), and 4 tail
    workgroups past the last full set of 8 keep their ids.  Every row of
    every sequence against the oracle."""
    ctx = [128 + 16 * i for i in range(9)]
    q_lens = [128] * 9
    dev, ref, tables, ctx, cu, q, td = _setup(orc.BF16, 8, 2, ctx, q_lens, seed=71)
    out, scale = _run(dev, tables, ctx, cu, q, td, 8)
    want = ref.prefill(widen(q, orc.BF16), 8, cu, tables, ctx, scale, causal=True)
    assert_close(from_dev(out), want, RTOL, ATOL, what="prefill, 36 workgroups")


def test_prefill_non_causal_and_bf16_out():
    hq, hkv = 8, 2
    dev, ref, tables, ctx, cu, q, td = _setup(orc.BF16, hq, hkv, [130, 77], [33, 77], seed=5)
    out, scale = _run(dev, tables, ctx, cu, q, td, hq, causal=False, out_f32=False)
    want = ref.prefill(widen(q, orc.BF16), hq, cu, tables, ctx, scale, causal=False)
    assert_close(widen(from_dev(out), orc.BF16), want, RTOL, ATOL, what="prefill non-causal bf16 out")


@pytest.mark.parametrize("scale", [-0.0883883, 0.0, 0.25])
def test_prefill_scale_values(scale):
    """A negative scale (the max is taken over scaled scores), a zero scale
    (uniform weights over the visible keys) and a large one."""
    hq, hkv = 8, 2
    dev, ref, tables, ctx, cu, q, td = _setup(orc.BF16, hq, hkv, [150, 70], [90, 70], seed=21)
    out, scale = _run(dev, tables, ctx, cu, q, td, hq, scale=scale)
    want = ref.prefill(widen(q, orc.BF16), hq, cu, tables, ctx, scale, causal=True)
    assert_close(from_dev(out), want, RTOL, ATOL, what=f"prefill scale={scale}")


@pytest.mark.parametrize("dt", [orc.BF16, orc.F16])
def test_prefill_rising_scores(dt):
    """K rows grow with position, so each 64-key block raises the running
    max by several times the lazy-rescale threshold (2^8) and the
    accumulators are rescaled mid-context; also a falling ramp (the max is
    set by the first block and never rescaled)."""
    hq, hkv = 8, 2
    for gain in (lambda p: 1.0 + p / 24.0, lambda p: 8.0 / (1.0 + p / 24.0)):
        dev, ref, tables, ctx, cu, q, td = _setup(dt, hq, hkv, [600, 333], [200, 333], seed=31, k_gain=gain)
        out, scale = _run(dev, tables, ctx, cu, q, td, hq)
        want = ref.prefill(widen(q, dt), hq, cu, tables, ctx, scale, causal=True)
        assert_close(from_dev(out), want, RTOL, ATOL, what=f"prefill rising/falling dt={dt}")


@pytest.mark.parametrize("bs", [8, 32, 64])
def test_prefill_block_sizes(bs):
    """Pages of 8, 32 and 64 tokens: a 64-key block spans 8, 2 or 1 pages
    (each 4-row load stays inside one page)."""
    hq, hkv = 8, 2
    ctx, q_lens = [333, 200], [150, 200]
    dev, ref, tables, ctx, cu, q, td = _setup(orc.BF16, hq, hkv, ctx, q_lens, seed=71 + bs, bs=bs)
    out, scale = _run(dev, tables, ctx, cu, q, td, hq)
    want = ref.prefill(widen(q, orc.BF16), hq, cu, tables, ctx, scale, causal=True)
    assert_close(from_dev(out), want, RTOL, ATOL, what=f"prefill bs={bs}")


def test_prefill_wide_table_scalar_page_ids():
    """A block table wider than fits beside the K/V rings in LDS (13,000
    entries per row): page ids come from scalar loads of the table instead
    of the workgroup's LDS copy."""
    hq, hkv = 8, 2
    ctx, q_lens = [400, 150], [130, 150]
    dev, ref, tables, ctx, cu, q, td = _setup(orc.BF16, hq, hkv, ctx, q_lens, seed=81, mb=13000)
    assert tables.shape[1] == 13000
    out, scale = _run(dev, tables, ctx, cu, q, td, hq)
    want = ref.prefill(widen(q, orc.BF16), hq, cu, tables, ctx, scale, causal=True)
    assert_close(from_dev(out), want, RTOL, ATOL, what="prefill wide table")


def test_prefill_config3_rows():
    """Config 3: Hq 32, Hkv 8, D 128, bs 16; 8 sequences with 2048 cached
    tokens append a 512-token chunk; table = a permutation of a 4096-block
    pool.  Against the oracle (on the host's threads): every row of every
    sequence (4096 rows x 32 heads).  Every row: finite, and each output
    element inside the range of the V rows it attends (keys 0 .. its
    position of its KV head), as a convex combination must be."""
    import os

    hq, hkv, D = 32, 8, 128
    ctx = [2560] * 8
    q_lens = [512] * 8
    dev, ref, tables, ctx, cu, q, td = _setup(orc.BF16, hq, hkv, ctx, q_lens, seed=3, nb=4096)
    out, scale = _run(dev, tables, ctx, cu, q, td, hq)
    got = from_dev(out)
    assert np.isfinite(got).all()
    qf = widen(q, orc.BF16)
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    for s in range(8):
        want = ref.prefill(qf, hq, cu, tables, ctx, scale, causal=True, rows=(s, 0, 512), threads=threads)
        rows = slice(int(cu[s]), int(cu[s]) + 512)
        assert_close(got[rows], want[rows], RTOL, ATOL, what=f"config3 seq {s}, all 512 rows")
    # Convex hull: running min / max of V over positions, per KV head and dim.
    n = ctx.astype(np.int64)
    cu_tok = np.concatenate([[0], np.cumsum(n)[:-1]]).astype(np.int64)
    _, gv = ref.gather(tables, ctx, None, cu_tok, int(n.sum()))
    vrows = widen(gv.view(np.uint16), orc.BF16).reshape(-1, D)
    G = hq // hkv
    for s in range(8):
        V = vrows[int(cu_tok[s]) * hkv:(int(cu_tok[s]) + int(n[s])) * hkv].reshape(hkv, int(n[s]), D)
        hi = np.maximum.accumulate(V, axis=1)
        lo = np.minimum.accumulate(V, axis=1)
        pos = int(ctx[s]) - 512 + np.arange(512)
        o = got[int(cu[s]):int(cu[s + 1])].reshape(512, hkv, G, D)
        up = hi[:, pos, :].transpose(1, 0, 2)[:, :, None, :]
        dn = lo[:, pos, :].transpose(1, 0, 2)[:, :, None, :]
        assert np.all(o <= up + 1e-4) and np.all(o >= dn - 1e-4), f"config3 seq {s}: outside the V hull"
