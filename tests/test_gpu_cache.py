"""GPU parity of the data-movement kernels: slot-mapped append (bit copy,
Q8_0 / Q4_0 / Q4_1 / Q5_0 / Q5_1 quantise), block-table gather, evict and
copy-on-write page copy.  Every
result is compared byte for byte with the oracle on the same seeded inputs;
pools start filled with a sentinel so stray writes show up."""
import numpy as np
import pytest

import oracle as orc
from kvutil import from_dev, kv_values, random_tables, slots_for, to_dev

pytestmark = pytest.mark.gpu

SENTINEL = 0xA5


def _pair(num_blocks, bs, hkv, D, dt):
    import torch
    from infer_train_amd.kv import PagedKvCache

    dev = PagedKvCache(num_blocks, bs, hkv, D, dt)
    dev.k_pool.fill_(SENTINEL)
    dev.v_pool.fill_(SENTINEL)
    ref = orc.Cache(num_blocks, bs, hkv, D, dt)
    ref.k[:] = SENTINEL
    ref.v[:] = SENTINEL
    torch.cuda.synchronize()
    return dev, ref


def _src(seed, n_tokens, hkv, D, dt):
    if dt in orc.QUANT_TYPES:
        k = kv_values(seed, n_tokens * hkv * D, orc.F32, outliers=True)
        v = kv_values(seed + 1, n_tokens * hkv * D, orc.F32, outliers=True)
    else:
        k = kv_values(seed, n_tokens * hkv * D, dt)
        v = kv_values(seed + 1, n_tokens * hkv * D, dt)
    return k.reshape(n_tokens, hkv, D), v.reshape(n_tokens, hkv, D)


def _dev_src(a, dt):
    import torch

    if dt in (orc.F32,) + orc.QUANT_TYPES:
        return to_dev(a)
    return to_dev(a.view(np.int16), torch.bfloat16 if dt == orc.BF16 else torch.float16)


def _assert_pools(dev, ref, what):
    dev.check()
    for name, d, r in (("K", dev.k_pool, ref.k), ("V", dev.v_pool, ref.v)):
        got = from_dev(d)
        if not np.array_equal(got, r):
            i = np.flatnonzero(got != r)
            raise AssertionError(f"{what}: {name} pool differs at {i.size} bytes, first {i[0]} "
                                 f"(page {i[0] // dev.page_bytes}) got {got[i[0]]} want {r[i[0]]}")


@pytest.mark.parametrize("dt,D,bs", [(orc.BF16, 128, 16), (orc.F32, 128, 16), (orc.F16, 128, 16),
                                     (orc.BF16, 256, 32), (orc.Q8_0, 256, 32), (orc.Q8_0, 128, 16),
                                     (orc.Q4_0, 256, 32), (orc.Q4_0, 128, 16), (orc.Q4_0, 64, 8),
                                     (orc.Q4_1, 256, 32), (orc.Q4_1, 128, 16), (orc.Q4_1, 64, 8),
                                     (orc.Q5_0, 256, 32), (orc.Q5_0, 128, 16), (orc.Q5_0, 64, 8), (orc.Q5_0, 32, 16),
                                     (orc.Q5_1, 256, 32), (orc.Q5_1, 128, 16), (orc.Q5_1, 64, 8), (orc.Q5_1, 32, 8),
                                     # rows that are not a power-of-two number of 16-byte vectors
                                     (orc.BF16, 96, 16), (orc.F16, 80, 16), (orc.F32, 48, 16), (orc.F32, 12, 8),
                                     (orc.Q8_0, 64, 8), (orc.Q8_0, 96, 16), (orc.Q8_0, 128, 8)])
def test_append_bit_exact(dt, D, bs):
    hkv, nb, n = 4, 64, 300
    dev, ref = _pair(nb, bs, hkv, D, dt)
    perm = orc.permutation(7, nb * bs)
    slots = perm[:n].copy()
    slots[::37] = -1  # padding tokens are skipped
    k, v = _src(11, n, hkv, D, dt)
    ref.append(k, v, slots)
    dev.append(_dev_src(k, dt), _dev_src(v, dt), to_dev(slots))
    _assert_pools(dev, ref, f"append dt={dt}")


def test_append_q8_special_groups():
    """Ties, all-zero, constant, subnormal-scale, NaN and inf groups."""
    hkv, D, bs, nb = 1, 256, 32, 4
    dev, ref = _pair(nb, bs, hkv, D, orc.Q8_0)
    rows = []
    g = np.zeros((8, 32), np.float32)
    g[0, 0] = 127.0
    g[0, 1:7] = [2.5, -2.5, 0.5, -0.5, 3.5, -126.5]  # exact .5 ties, scale exactly 1
    g[1] = 0.0
    g[2] = 0.75
    g[3] = orc.normal(3, 32) * np.float32(1e-30)  # fp16-subnormal scale
    g[4] = orc.normal(4, 32) * np.float32(1e-40)  # fp32-subnormal inputs
    g[5] = orc.normal(5, 32)
    g[5, 9] = np.nan
    g[6] = orc.normal(6, 32)
    g[6, 2] = np.inf
    g[7] = orc.normal(7, 32) * np.float32(6e4)  # scale near the fp16 max
    rows.append(g.reshape(-1))
    for s in range(1, 8):
        rows.append(np.roll(g.reshape(-1), 32 * s))
    k = np.stack(rows).reshape(8, hkv, D)
    v = -k
    slots = np.array([0, 5, 31, 32, 63, 64, 100, 127], np.int64)
    ref.append(k, v, slots)
    dev.append(to_dev(k), to_dev(v), to_dev(slots))
    _assert_pools(dev, ref, "append q8 special")


@pytest.mark.parametrize("D", [256, 128, 64, 96])
def test_append_q8_near_ties(D):
    """Elements whose quotient x / scale lies within a few ulps of a
    half-integer, where round(fl(x / scale)) depends on the IEEE quotient's
    last bit: the append's fast reciprocal path must hand them to the exact
    division.  Scales from 1e-38 to 1e37 (the tiny and huge ones take the
    division for every element).  D 64 / 128 / 256 run the 16-element-per-
    lane kernel, D 96 the 4-element one."""
    hkv, bs, nb = 2, 16, 8
    n = 40
    rng = np.random.default_rng(D)
    x = np.empty((n * hkv * D // 32, 32), np.float32)
    for i in range(x.shape[0]):
        amax = np.float32(10.0 ** rng.uniform(-38, 37) if i % 7 == 0 else rng.uniform(0.05, 20.0))
        sc = np.float32(amax) / np.float32(127)
        kk = rng.integers(-126, 126, 31).astype(np.float64)
        y = ((kk + 0.5) * np.float64(sc)).astype(np.float32)
        for _ in range(3):  # nudge by up to three ulps either way
            step = rng.integers(-1, 2, 31)
            y = np.where(step > 0, np.nextafter(y, np.float32(np.inf)), np.where(step < 0, np.nextafter(y, np.float32(-np.inf)), y))
        y = np.clip(y, -amax, amax).astype(np.float32)
        x[i, 0] = amax if i % 2 else -amax
        x[i, 1:] = y
    k = x.reshape(n, hkv, D)
    v = (-x[:, ::-1]).reshape(n, hkv, D).copy()
    dev, ref = _pair(nb, bs, hkv, D, orc.Q8_0)
    slots = orc.permutation(D, nb * bs)[:n].copy()
    ref.append(k, v, slots)
    dev.append(to_dev(k), to_dev(v), to_dev(slots))
    _assert_pools(dev, ref, f"append q8 near ties D={D}")


@pytest.mark.parametrize("dt", [orc.Q4_0, orc.Q4_1, orc.Q5_0, orc.Q5_1])
def test_append_nibble_special_groups(dt):
    """Q4_0 / Q4_1 / Q5_0 / Q5_1 (ggml's quantisers; the reference has
    none): equal magnitudes of both signs, all-zero, -0, constant,
    subnormal, NaN, inf and a group whose 1/d overflows."""
    hkv, D, bs, nb = 1, 256, 32, 4
    dev, ref = _pair(nb, bs, hkv, D, dt)
    g = np.zeros((8, 32), np.float32)
    g[0, [2, 7, 20]] = [-4.0, 4.0, 4.0]  # first of equal magnitudes: max = -4
    g[0, [3, 4, 5]] = [1.25, -1.75, 3.0]  # x * id + 8.5 on .5 boundaries
    g[1] = -0.0
    g[2] = 0.75
    g[3] = orc.normal(3, 32) * np.float32(1e-30)
    g[4] = orc.normal(4, 32) * np.float32(1e-40)  # d underflows to 0 (or 1/d overflows)
    g[5] = orc.normal(5, 32)
    g[5, 9] = np.nan
    g[6] = orc.normal(6, 32)
    g[6, 2] = -np.inf
    g[7] = orc.normal(7, 32) * np.float32(6e4)
    if dt in (orc.Q4_1, orc.Q5_1):  # min over +0 and -0: the first stays
        g[1, :16] = 1.0
        g[1, [3, 9]] = [0.0, -0.0]
    rows = [np.roll(g.reshape(-1), 32 * s) for s in range(8)]
    k = np.stack(rows).reshape(8, hkv, D)
    v = -k
    slots = np.array([0, 5, 31, 32, 63, 64, 100, 127], np.int64)
    ref.append(k, v, slots)
    dev.append(to_dev(k), to_dev(v), to_dev(slots))
    _assert_pools(dev, ref, f"append nibble special dt={dt}")


@pytest.mark.parametrize("dt", [orc.Q8_0, orc.Q4_0, orc.Q4_1, orc.Q5_0, orc.Q5_1])
def test_append_golden_cases(dt):
    """The committed quantiser fixtures (tests/golden/q8_cases.json,
    q4_cases.json, q5_cases.json): each case is one 32-element token row of a
    D = 32 cache; append, then gather the records and compare them with the
    fixture bytes."""
    import json
    import os

    import torch

    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    name = {orc.Q8_0: "q8_cases.json", orc.Q5_0: "q5_cases.json", orc.Q5_1: "q5_cases.json"}.get(dt, "q4_cases.json")
    key = {orc.Q8_0: "record", orc.Q4_0: "q4_0", orc.Q4_1: "q4_1", orc.Q5_0: "q5_0", orc.Q5_1: "q5_1"}[dt]
    cases = json.load(open(os.path.join(golden, name)))
    x = np.stack([np.array(c["x_bits"], np.uint32).view(np.float32) for c in cases]).reshape(-1, 1, 32)
    n = len(cases)
    dev, _ = _pair(4, 8, 1, 32, dt)
    slots = np.arange(n, dtype=np.int64)
    dev.append(to_dev(x), to_dev(-x), to_dev(slots))
    rb = orc.RECORD_BYTES[dt]
    ko = torch.zeros(n * rb, dtype=torch.uint8, device="cuda:0")
    vo = torch.zeros(n * rb, dtype=torch.uint8, device="cuda:0")
    tables = np.arange(4, dtype=np.int32)[None, :]
    dev.gather(to_dev(tables), to_dev(np.array([n], np.int32)), None, to_dev(np.array([0], np.int64)), n, ko, vo)
    dev.check()
    got = from_dev(ko).reshape(n, rb)
    for i, c in enumerate(cases):
        assert list(got[i]) == c[key], c["name"]


def test_append_config1_full_step():
    # Config 1: fp32, Hkv 2, D 128, bs 16, 64 blocks, identity table; 1023
    # cached tokens then the token at position 1023.
    hkv, D, bs, nb = 2, 128, 16, 64
    dev, ref = _pair(nb, bs, hkv, D, orc.F32)
    k, v = _src(1, 1024, hkv, D, orc.F32)
    slots = np.arange(1024, dtype=np.int64)  # identity block table
    ref.append(k[:1023], v[:1023], slots[:1023])
    dev.append(to_dev(k[:1023]), to_dev(v[:1023]), to_dev(slots[:1023]))
    ref.append(k[1023:], v[1023:], slots[1023:])
    dev.append(to_dev(k[1023:]), to_dev(v[1023:]), to_dev(slots[1023:]))
    _assert_pools(dev, ref, "config1 append")


def test_append_bad_slot_is_latched_not_written():
    from infer_train_amd import InvalidInput

    hkv, D, bs, nb = 2, 128, 16, 8
    dev, ref = _pair(nb, bs, hkv, D, orc.BF16)
    k, v = _src(2, 3, hkv, D, orc.BF16)
    slots = np.array([3, nb * bs + 5, 9], np.int64)  # middle slot is out of range
    dev.append(_dev_src(k, orc.BF16), _dev_src(v, orc.BF16), to_dev(slots))
    with pytest.raises(InvalidInput):
        dev.check()
    ref.append(k[[0, 2]], v[[0, 2]], slots[[0, 2]])
    _assert_pools(dev, ref, "bad slot")  # nothing else written; flag cleared


@pytest.mark.parametrize("dt,D,bs", [(orc.BF16, 128, 16), (orc.F32, 128, 16), (orc.Q8_0, 256, 32),
                                     (orc.Q4_0, 128, 16), (orc.Q4_1, 256, 32), (orc.Q5_0, 128, 16),
                                     (orc.Q5_0, 256, 32), (orc.Q5_1, 128, 16), (orc.Q5_1, 256, 32)])
def test_gather_bit_exact(dt, D, bs):
    import torch

    hkv, nb = 2, 128
    ctx = np.array([0, 1, 17, 300, 511], np.int32)
    start = np.array([0, 0, 5, 33, 100], np.int32)  # windowed starts, not block aligned
    mb = 40
    tables = random_tables(5, ctx, bs, nb, mb)
    dev, ref = _pair(nb, bs, hkv, D, dt)
    seqs, pos = [], []
    for b, c in enumerate(ctx):
        seqs += [b] * int(c)
        pos += list(range(int(c)))
    slots = slots_for(tables, seqs, pos, bs)
    k, v = _src(3, len(slots), hkv, D, dt)
    ref.append(k, v, slots)
    dev.append(_dev_src(k, dt), _dev_src(v, dt), to_dev(slots))
    n = ctx - start
    cu = np.concatenate([[0], np.cumsum(n)[:-1]]).astype(np.int64)
    total = int(n.sum())
    rk, rv = ref.gather(tables, ctx, start, cu, total)
    ko = torch.zeros(rk.size, dtype=torch.uint8, device="cuda:0")
    vo = torch.zeros(rv.size, dtype=torch.uint8, device="cuda:0")
    dev.gather(to_dev(tables), to_dev(ctx), to_dev(start), to_dev(cu), int(n.max()), ko, vo)
    dev.check()
    np.testing.assert_array_equal(from_dev(ko), rk)
    np.testing.assert_array_equal(from_dev(vo), rv)
    if dt == orc.Q8_0:  # AoS records equal quantize_row_q8_0 of the source rows
        b = 3
        rows = []
        for h in range(hkv):
            for i in range(n[b]):
                t = int(sum(ctx[:b])) + int(start[b]) + i
                rows.append(orc.quantize_row_q8_0(k[t, h]))
        want = np.concatenate(rows).ravel()
        off = int(cu[b]) * hkv * (D // 32) * 34
        np.testing.assert_array_equal(from_dev(ko)[off:off + want.size], want)
    quant_row = {orc.Q4_0: orc.quantize_row_q4_0, orc.Q5_0: orc.quantize_row_q5_0,
                 orc.Q5_1: orc.quantize_row_q5_1}.get(dt)
    if quant_row is not None:  # AoS records equal the ggml quantiser of the source rows
        b = 3
        rows = []
        for h in range(hkv):
            for i in range(n[b]):
                t = int(sum(ctx[:b])) + int(start[b]) + i
                rows.append(quant_row(v[t, h]))
        want = np.concatenate(rows).ravel()
        off = int(cu[b]) * hkv * (D // 32) * orc.RECORD_BYTES[dt]
        np.testing.assert_array_equal(from_dev(vo)[off:off + want.size], want)


def test_gather_negative_start_is_latched():
    """A negative start position: the gather writes nothing for that
    sequence, the others are exact, and it_kv_cache_check reports it."""
    import torch
    from infer_train_amd import InvalidInput

    dt, D, bs, hkv, nb = orc.BF16, 128, 16, 2, 64
    ctx = np.array([40, 70], np.int32)
    tables = random_tables(9, ctx, bs, nb, 8)
    dev, ref = _pair(nb, bs, hkv, D, dt)
    seqs = [0] * 40 + [1] * 70
    pos = list(range(40)) + list(range(70))
    slots = slots_for(tables, seqs, pos, bs)
    k, v = _src(4, len(slots), hkv, D, dt)
    ref.append(k, v, slots)
    dev.append(_dev_src(k, dt), _dev_src(v, dt), to_dev(slots))
    start = np.array([-2, 3], np.int32)
    n = np.array([40, 67], np.int64)
    cu = np.array([0, 40], np.int64)
    rk, rv = ref.gather(tables, ctx, np.array([0, 3], np.int32), cu, int(n.sum()))
    ko = torch.zeros(rk.size, dtype=torch.uint8, device="cuda:0")
    vo = torch.zeros(rv.size, dtype=torch.uint8, device="cuda:0")
    dev.gather(to_dev(tables), to_dev(ctx), to_dev(start), to_dev(cu), 70, ko, vo)
    with pytest.raises(InvalidInput, match="negative-start"):
        dev.check()
    row = hkv * D * 2  # bytes per token (both heads), bf16
    np.testing.assert_array_equal(from_dev(ko)[:40 * row], 0)
    np.testing.assert_array_equal(from_dev(ko)[40 * row:], rk[40 * row:])
    np.testing.assert_array_equal(from_dev(vo)[40 * row:], rv[40 * row:])


def test_evict_and_copy_blocks():
    hkv, D, bs, nb = 2, 128, 16, 32
    dev, ref = _pair(nb, bs, hkv, D, orc.BF16)
    slots = np.arange(nb * bs, dtype=np.int64)
    k, v = _src(9, nb * bs, hkv, D, orc.BF16)
    ref.append(k, v, slots)
    dev.append(_dev_src(k, orc.BF16), _dev_src(v, orc.BF16), to_dev(slots))
    ev = np.array([3, 17, 31, 0], np.int32)
    ref.evict(ev)
    dev.evict(to_dev(ev))
    _assert_pools(dev, ref, "evict")
    src, dst = np.array([5, 6], np.int32), np.array([3, 0], np.int32)
    dev.copy_blocks(to_dev(src), to_dev(dst))
    pb = dev.page_bytes * hkv
    for s, d in zip(src, dst):
        ref.k[d * pb:(d + 1) * pb] = ref.k[s * pb:(s + 1) * pb]
        ref.v[d * pb:(d + 1) * pb] = ref.v[s * pb:(s + 1) * pb]
    _assert_pools(dev, ref, "copy_blocks")


def _to_cache_src(x, dt):
    """float32 rows -> the source the oracle's append takes for a cache of dt
    (16-bit caches: round to nearest even bits)."""
    if dt == orc.BF16:
        return orc.f32_to_bf16(x)
    if dt == orc.F16:
        return orc.f32_to_f16(x)
    return np.ascontiguousarray(x, np.float32)


@pytest.mark.parametrize("dt,D,bs", [(orc.BF16, 128, 16), (orc.F32, 128, 16), (orc.F16, 128, 16),
                                     (orc.Q8_0, 256, 32), (orc.Q4_0, 128, 16), (orc.Q4_1, 256, 32),
                                     (orc.Q5_0, 128, 16), (orc.Q5_1, 256, 32)])
def test_append_rope_bit_exact(dt, D, bs):
    """RoPE then append (forward.rs:195-229): the cache pools and the rotated
    q equal the oracle's rope_f32 (rope.rs:6-44) followed by its append,
    byte for byte.  Positions span 0 (the identity angle), small values and
    the table's last entry; one token is padding (q rotated, nothing
    written); the first token carries special values (NaN, inf, subnormals,
    rounding ties of the 16-bit formats)."""
    import torch
    from infer_train_amd.kv import RopeTable

    hq, hkv, nb, n = (8, 2, 64, 40) if D == 128 else (12, 2, 48, 24)
    max_pos = 5000
    dev, ref = _pair(nb, bs, hkv, D, dt)
    rope = RopeTable(D, max_pos)
    rng = np.random.default_rng(5 + D)
    slots = rng.permutation(nb * bs)[:n].astype(np.int64)
    slots[7] = -1
    pos = rng.integers(0, max_pos, n).astype(np.int32)
    pos[:3] = [0, 1, max_pos - 1]
    q = orc.normal(51, n * hq * D).reshape(n, hq, D)
    k = orc.normal(52, n * hkv * D).reshape(n, hkv, D)
    v = orc.normal(53, n * hkv * D).reshape(n, hkv, D)
    special = np.array([np.nan, np.inf, -np.inf, 1e-41, -3e-40, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8,
                        65519.0, 65520.0, 2 ** -25, 5.96e-8, -0.0], np.float32)
    k[0, 0, :special.size] = special
    v[0, 1, :special.size] = special
    q[0, 0, :special.size] = special
    q_rot = orc.rope_rows(q, pos, D, D)
    k_rot = orc.rope_rows(k, pos, D, D)
    ref.append(_to_cache_src(k_rot, dt), _to_cache_src(v, dt), slots)
    td = {orc.BF16: torch.bfloat16, orc.F16: torch.float16}.get(dt, torch.float32)
    q_out = dev.append_rope(rope, to_dev(q), to_dev(k), to_dev(v), to_dev(slots), to_dev(pos), q_out_dtype=td)
    dev.check()
    _assert_pools(dev, ref, f"append_rope dt={dt}")
    got = from_dev(q_out)
    want = q_rot if td == torch.float32 else _to_cache_src(q_rot, dt)
    assert np.array_equal(got.reshape(-1).view(np.uint8), np.ascontiguousarray(want).reshape(-1).view(np.uint8)), \
        "rotated q differs from rope_f32"
    if td != torch.float32:  # the F32 output path as well
        q32 = dev.append_rope(rope, to_dev(q), to_dev(k), to_dev(v), to_dev(slots), to_dev(pos))
        assert np.array_equal(from_dev(q32).view(np.uint32), q_rot.view(np.uint32))


def test_append_rope_bad_position_is_latched():
    """A position outside the table is latched (reported by check) and its
    token writes nothing; the other token is stored."""
    import torch
    from infer_train_amd import InvalidInput
    from infer_train_amd.kv import RopeTable

    dev, ref = _pair(8, 16, 1, 128, orc.F32)
    rope = RopeTable(128, 100)
    k = orc.normal(61, 2 * 128).reshape(2, 1, 128)
    q = orc.normal(62, 2 * 128).reshape(2, 1, 128)
    dev.append_rope(rope, to_dev(q), to_dev(k), to_dev(k), to_dev(np.array([3, 4], np.int64)),
                    to_dev(np.array([5, 100], np.int32)))
    with pytest.raises(InvalidInput):
        dev.check()
    torch.cuda.synchronize()
    for pool in (dev.k_pool, dev.v_pool):
        rows = from_dev(pool).reshape(8, 16, 128 * 4)
        assert np.all(rows[0, 4] == SENTINEL), "a row with an out-of-table position must not be written"
        assert not np.all(rows[0, 3] == SENTINEL)
