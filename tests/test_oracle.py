"""Pins the CPU oracle (oracle/it_oracle.c) before it is trusted as the
checker: the reference's own known-answer test, closed forms, special cases,
float64 brute force, and an exhaustive conversion check."""
import math
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ---------------- flash_attn_f32 (src/backend/arm/flash_attn.rs:6-72) ------
def test_flash_attn_reference_kat(orc):
    # flash_attn.rs:78-97: q=e0, keys e0,e1,e2, V = 1..12, scale 1.
    q = np.array([1, 0, 0, 0], np.float32)
    k = np.array([1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 1, 0], np.float32)
    v = np.arange(1, 13, dtype=np.float32)
    out = orc.flash_attn_f32(q, k, v, 1.0)
    assert np.all(out > 0) and abs(out[0] - 3.54) < 0.1  # the reference's own assertion
    e = math.e
    # Closed form: softmax weights (e, 1, 1)/(e+2) over rows (1..4, 5..8, 9..12).
    want = [(e * (1 + d) + (5 + d) + (9 + d)) / (e + 2) for d in range(4)]
    np.testing.assert_allclose(out, want, rtol=2e-7)
    assert abs(out[0] - (e + 14) / (e + 2)) < 1e-6


def test_flash_attn_single_key_is_value(orc):
    q, k, v = orc.normal(1, 64), orc.normal(2, 64), orc.normal(3, 64)
    np.testing.assert_array_equal(orc.flash_attn_f32(q, k, v, 0.125), v)


def test_flash_attn_equal_scores_is_mean(orc):
    D, n = 32, 50
    q = orc.normal(4, D)
    k = np.tile(orc.normal(5, D), n)
    v = orc.normal(6, n * D).reshape(n, D)
    np.testing.assert_allclose(orc.flash_attn_f32(q, k, v, 0.3), v.astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("n,D,scale", [(1, 8, 1.0), (7, 16, 0.25), (300, 128, 1 / math.sqrt(128)), (1000, 64, 0.9)])
def test_flash_attn_matches_float64_softmax(orc, n, D, scale):
    q, k, v = orc.normal(7, D), orc.normal(8, n * D).reshape(n, D), orc.normal(9, n * D).reshape(n, D)
    s = (k.astype(np.float64) @ q.astype(np.float64)) * scale
    p = np.exp(s - s.max())
    want = (p @ v.astype(np.float64)) / p.sum()
    np.testing.assert_allclose(orc.flash_attn_f32(q, k, v, scale), want, rtol=1e-5, atol=1e-6)


def test_flash_attn_mask_skips_and_shifts(orc):
    D, n = 16, 9
    q, k, v = orc.normal(10, D), orc.normal(11, n * D).reshape(n, D), orc.normal(12, n * D).reshape(n, D)
    mask = np.zeros(n, np.float32)
    mask[[1, 4, 8]] = -np.inf
    keep = mask == 0
    a = orc.flash_attn_f32(q, k, v, 0.5, mask)
    b = orc.flash_attn_f32(q, k[keep], v[keep], 0.5)
    np.testing.assert_array_equal(a, b)  # -inf keys are skipped (flash_attn.rs:35-40)
    shift = np.linspace(-1, 1, n).astype(np.float32)
    s = (k.astype(np.float64) @ q) * 0.5 + shift
    p = np.exp(s - s.max())
    np.testing.assert_allclose(orc.flash_attn_f32(q, k, v, 0.5, shift), p @ v / p.sum(), rtol=1e-5, atol=1e-6)
    assert np.all(orc.flash_attn_f32(q, k, v, 0.5, np.full(n, -np.inf, np.float32)) == 0)  # s == 0 -> zeros


def test_backend_op_gqa_shares_kv(orc):
    # arm.rs:304-370: every head reads the same K/V; scale 1/sqrtf(D).
    H, D, n = 5, 32, 40
    q = orc.normal(13, H * D).reshape(H, D)
    k, v = orc.normal(14, n * D).reshape(n, D), orc.normal(15, n * D).reshape(n, D)
    out = orc.backend_flash_attention(q, k, v)
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    for h in range(H):
        np.testing.assert_array_equal(out[h], orc.flash_attn_f32(q[h], k, v, float(scale)))


# ---------------- Q8_0 (src/backend/arm/quant.rs:149-183) ------------------
def _q8_numpy(x):
    """Independent numpy formulation of the x86 scalar Q8_0 semantics."""
    x = x.astype(np.float32).reshape(-1, 32)
    ax = np.where(np.isnan(x), np.float32(0), np.abs(x))
    amax = ax.max(1)
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = (amax / np.float32(127)).astype(np.float32)
        y = (x / scale[:, None]).astype(np.float32).astype(np.float64)
    r = np.sign(y) * np.floor(np.abs(y) + 0.5)  # half away from zero, exact in f64
    r = np.where(np.isnan(r), 0, np.clip(r, -128, 127)).astype(np.int8)
    r[amax == 0] = 0
    d = scale.astype(np.float16).view(np.uint16)
    d = np.where(amax == 0, 0, d).astype(np.uint16)
    rec = np.zeros((x.shape[0], 34), np.uint8)
    rec[:, 0] = d & 0xFF
    rec[:, 1] = d >> 8
    rec[:, 2:] = r.view(np.uint8)
    return rec


def test_q8_zero_group(orc):
    assert np.all(orc.quantize_row_q8_0(np.zeros(32, np.float32)) == 0)
    assert np.all(orc.quantize_row_q8_0(-np.zeros(32, np.float32)) == 0)


def test_q8_constant_and_spike(orc):
    rec = orc.quantize_row_q8_0(np.full(32, 0.75, np.float32))
    assert np.all(rec[0, 2:].view(np.int8) == 127)
    assert int(rec[0, 0]) | (int(rec[0, 1]) << 8) == np.float16(np.float32(0.75) / np.float32(127)).view(np.uint16)
    x = np.zeros(32, np.float32)
    x[5] = -8.0
    q = orc.quantize_row_q8_0(x)[0, 2:].view(np.int8)
    assert q[5] == -127 and np.count_nonzero(q) == 1


def test_q8_ties_round_half_away_from_zero(orc):
    # amax = 127 makes scale exactly 1, so x/scale = x: 2.5 -> 3 (RNE would
    # give 2), -2.5 -> -3, 0.5 -> 1, -0.5 -> -1, 3.5 -> 4.
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:6] = [2.5, -2.5, 0.5, -0.5, 3.5]
    q = orc.quantize_row_q8_0(x)[0, 2:].view(np.int8)
    assert list(q[:6]) == [127, 3, -3, 1, -1, 4]


def test_q8_nan_inf(orc):
    x = np.linspace(-1, 1, 32).astype(np.float32)
    x[3] = np.nan
    rec = orc.quantize_row_q8_0(x)
    q = rec[0, 2:].view(np.int8)
    assert q[3] == 0 and q[0] == -127 and q[31] == 127  # NaN ignored by the `>` amax
    x[7] = np.inf
    rec = orc.quantize_row_q8_0(x)
    assert int(rec[0, 0]) | (int(rec[0, 1]) << 8) == 0x7C00
    assert np.all(rec[0, 2:] == 0)  # finite/inf = 0, inf/inf = NaN -> 0 (Rust `as`)


def test_q8_matches_numpy_formulation(orc):
    x = orc.normal(20, 32 * 4096)
    rng = np.random.default_rng(0)
    x[rng.random(x.size) < 0.01] *= 8  # the C5 outlier model
    x[:32] *= 1e-30  # fp16-subnormal and fp32-subnormal scales
    x[32:64] *= 1e-40
    x[64:96] *= 3e4
    np.testing.assert_array_equal(orc.quantize_row_q8_0(x), _q8_numpy(x))


def test_q8_dequant_is_d_times_q(orc):
    x = orc.normal(21, 32 * 64)
    rec = orc.quantize_row_q8_0(x)
    deq = orc.dequantize_row_q8_0(rec).reshape(-1, 32)
    d = (rec[:, 0].astype(np.uint16) | (rec[:, 1].astype(np.uint16) << 8)).view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(deq, d[:, None] * rec[:, 2:].view(np.int8).astype(np.float32))
    assert np.max(np.abs(deq - x.reshape(-1, 32))) <= np.max(d) * 0.5 * (1 + 1e-3) + 1e-7


# ---------------- Q4_0 ------------------------------------------------------
# The reference fixes the block (types.rs:15-22) and its dequantisation
# (vec_dot.rs:425-440, and the NEON path :97-137 agrees); it has no Q4_0
# quantiser, so the quantiser is pinned to ggml's quantize_row_q4_0_ref by
# hand-worked cases below, not to reference output.
def _f16_bits(x) -> int:
    return int(np.float16(x).view(np.uint16))


def _q4_d(rec) -> np.ndarray:
    return (rec[:, 0].astype(np.uint16) | (rec[:, 1].astype(np.uint16) << 8)).view(np.float16)


def test_q4_dequant_layout(orc):
    rec = np.zeros((1, 18), np.uint8)
    rec[0, :2] = np.frombuffer(np.float16(0.1).tobytes(), np.uint8)
    rec[0, 2:] = 0x88  # the reference's own KAT input (gemv.rs:186-204): all zero
    assert np.all(orc.dequantize_row_q4_0(rec) == 0)
    rec[0, 2:] = [j | ((15 - j) << 4) for j in range(16)]  # low nibble j, high nibble 15 - j
    out = orc.dequantize_row_q4_0(rec)
    d = np.float32(np.float16(0.1))
    np.testing.assert_array_equal(out[:16], d * np.arange(-8, 8, dtype=np.float32))
    np.testing.assert_array_equal(out[16:], d * np.arange(7, -9, -1, dtype=np.float32))


def test_q4_zero_group(orc):
    for z in (np.zeros(32, np.float32), -np.zeros(32, np.float32)):
        rec = orc.quantize_row_q4_0(z)
        assert _q4_d(rec)[0] == 0 and np.all(rec[0, 2:] == 0x88)


def test_q4_hand_worked_group(orc):
    # max = 8.0 (index 5; the -8.0 at index 20 has the same magnitude and
    # comes later), so d = -1 and id = -1: nibble = min(15, trunc(8.5 - x)).
    x = np.zeros(32, np.float32)
    vals = {0: 3.0, 1: -3.0, 2: 2.5, 3: -2.5, 4: 0.49, 5: 8.0, 6: 0.51, 7: 7.9, 8: -7.9, 20: -8.0, 21: 1.0}
    for i, v in vals.items():
        x[i] = v
    rec = orc.quantize_row_q4_0(x)
    assert int(rec[0, 0]) | (int(rec[0, 1]) << 8) == _f16_bits(-1.0)
    want = np.full(32, 8)
    for i, q in {0: 5, 1: 11, 2: 6, 3: 11, 4: 8, 5: 0, 6: 7, 7: 0, 8: 15, 20: 15, 21: 7}.items():
        want[i] = q
    got = np.concatenate([rec[0, 2:] & 0xF, rec[0, 2:] >> 4])
    np.testing.assert_array_equal(got, want)


def test_q4_first_of_equal_magnitudes(orc):
    x = np.zeros(32, np.float32)
    x[2], x[7] = -4.0, 4.0  # max = -4: d = 0.5, id = 2
    rec = orc.quantize_row_q4_0(x)
    assert int(rec[0, 0]) | (int(rec[0, 1]) << 8) == _f16_bits(0.5)
    assert rec[0, 2 + 2] & 0xF == 0 and rec[0, 2 + 7] & 0xF == 15  # -8 + 8.5 -> 0; 8 + 8.5 -> 16 -> 15
    x[2], x[7] = 4.0, -4.0  # max = 4: d = -0.5
    rec = orc.quantize_row_q4_0(x)
    assert int(rec[0, 0]) | (int(rec[0, 1]) << 8) == _f16_bits(-0.5)


def test_q4_nan_inf(orc):
    x = np.linspace(-1, 1, 32).astype(np.float32)
    x[3] = np.nan  # never the max; its nibble is trunc(NaN) -> 0
    rec = orc.quantize_row_q4_0(x)
    assert _q4_d(rec)[0] == np.float16(0.125)  # max = x[0] = -1, the first of |-1| = |1|
    assert rec[0, 2 + 3] & 0xF == 0
    x[3] = -np.inf  # d = inf, id = 0: finite x -> 8; the inf element -> NaN -> 0
    rec = orc.quantize_row_q4_0(x)
    assert int(rec[0, 0]) | (int(rec[0, 1]) << 8) == 0x7C00
    nib = np.concatenate([rec[0, 2:] & 0xF, rec[0, 2:] >> 4])
    assert nib[3] == 0 and np.all(np.delete(nib, 3) == 8)


def test_q4_round_trip_bound(orc):
    x = orc.normal(22, 32 * 2048)
    rng = np.random.default_rng(1)
    x[rng.random(x.size) < 0.01] *= 8
    x[:32] *= 1e-3
    x[32:64] *= 3e3
    rec = orc.quantize_row_q4_0(x)
    deq = orc.dequantize_row_q4_0(rec).reshape(-1, 32)
    xg = x.reshape(-1, 32)
    d = np.abs(_q4_d(rec).astype(np.float32))[:, None]
    err = np.abs(deq - xg)
    # round half up onto the grid d * (-8..7): at most d / 2, except the +8
    # end (the opposite sign of max, clamped to nibble 15) at most d; slack for
    # the fp16 rounding of d (2^-11 relative, times 8 steps)
    assert np.all(err <= d * (1 + 8 * 2 ** -10) + 1e-30)
    inner = np.abs(xg) < 7.5 * d
    assert np.all(err[inner] <= (d * 0.5 * (1 + 16 * 2 ** -10))[np.nonzero(inner)[0]].ravel() + 1e-30)
    # the element of largest magnitude comes back as -8 d
    imax = np.argmax(np.abs(xg), axis=1)
    np.testing.assert_array_equal(deq[np.arange(len(xg)), imax], -8 * _q4_d(rec).astype(np.float32))


def test_oracle_q4_gather_records_equal_quantize_row(orc):
    nb, bs, hkv, D = 4, 16, 2, 64
    c = orc.Cache(nb, bs, hkv, D, orc.Q4_0)
    n = nb * bs
    x = (orc.normal(14, n * hkv * D) * np.float32(3)).reshape(n, hkv, D)
    c.append(x, -x, np.arange(n, dtype=np.int64))
    tables = np.arange(nb, dtype=np.int32)[None, :]
    gk, gv = c.gather(tables, np.array([n], np.int32), None, np.array([0], np.int64), n)
    rk, rv = gk.reshape(hkv, n, D // 32 * 18), gv.reshape(hkv, n, D // 32 * 18)
    for h in range(hkv):
        for t in (0, 1, 37, n - 1):
            assert bytes(rk[h, t]) == bytes(orc.quantize_row_q4_0(x[t, h]))
            assert bytes(rv[h, t]) == bytes(orc.quantize_row_q4_0(-x[t, h]))


# ---------------- Q4_1 ------------------------------------------------------
# The reference fixes only the block (types.rs:24-32, 20 bytes asserted at
# :249); quantiser and dequantiser follow ggml and are pinned here by
# hand-worked cases, not by reference output.
def test_q4_1_layout_and_hand_worked_group(orc):
    x = np.zeros(32, np.float32)
    x[:16] = np.arange(16)  # min 0, max 15: d = 1, id = 1, nibble = trunc(x + 0.5)
    x[16:24] = [7.4, 7.5, 7.6, 0.49, 0.5, 14.5, 14.51, 3.0]
    rec = orc.quantize_row_q4_1(x)
    assert rec.shape == (1, 20)
    assert int(rec[0, 0]) | (int(rec[0, 1]) << 8) == _f16_bits(1.0)  # d
    assert int(rec[0, 2]) | (int(rec[0, 3]) << 8) == _f16_bits(0.0)  # m = min
    lo, hi = rec[0, 4:] & 0xF, rec[0, 4:] >> 4
    np.testing.assert_array_equal(lo, np.arange(16))
    np.testing.assert_array_equal(hi, [7, 8, 8, 0, 1, 15, 15, 3] + [0] * 8)
    deq = orc.dequantize_row_q4_1(rec)
    np.testing.assert_array_equal(deq[:16], np.arange(16, dtype=np.float32))
    np.testing.assert_array_equal(deq[16:24], np.array([7, 8, 8, 0, 1, 15, 15, 3], np.float32))


def test_q4_1_offset_and_nan(orc):
    x = np.linspace(-1, 2, 32).astype(np.float32)  # d = 3/15, m = -1
    x[5] = np.nan  # never the min or the max; its nibble is trunc(NaN) -> 0
    rec = orc.quantize_row_q4_1(x)
    assert int(rec[0, 0]) | (int(rec[0, 1]) << 8) == _f16_bits(np.float32(3.0) / np.float32(15.0))
    assert int(rec[0, 2]) | (int(rec[0, 3]) << 8) == _f16_bits(-1.0)
    assert rec[0, 4 + 5] & 0xF == 0
    deq = orc.dequantize_row_q4_1(rec)
    d = np.float32(np.float16(np.float32(3.0) / np.float32(15.0)))
    nib = np.concatenate([rec[0, 4:] & 0xF, rec[0, 4:] >> 4]).astype(np.float32)
    np.testing.assert_array_equal(deq, d * nib + np.float32(-1.0))


def test_q4_1_round_trip_bound(orc):
    x = orc.normal(23, 32 * 2048)
    rng = np.random.default_rng(2)
    x[rng.random(x.size) < 0.01] *= 8
    x[:32] += 5.0  # all-positive group: m far from 0
    rec = orc.quantize_row_q4_1(x)
    deq = orc.dequantize_row_q4_1(rec).reshape(-1, 32)
    xg = x.reshape(-1, 32)
    d = (rec[:, 0].astype(np.uint16) | (rec[:, 1].astype(np.uint16) << 8)).view(np.float16).astype(np.float32)
    m = (rec[:, 2].astype(np.uint16) | (rec[:, 3].astype(np.uint16) << 8)).view(np.float16).astype(np.float32)
    # round half up onto min + d * (0..15), then fp16 rounding of d (15 steps)
    # and of m move the grid by at most 15 |d| 2^-11 + |m| 2^-11
    bound = d * 0.5 + (15 * d + np.abs(m)) * 2.0 ** -11 * 1.01 + 1e-30
    assert np.all(np.abs(deq - xg) <= bound[:, None])


def test_oracle_q4_1_gather_records_equal_quantize_row(orc):
    nb, bs, hkv, D = 4, 16, 2, 64
    c = orc.Cache(nb, bs, hkv, D, orc.Q4_1)
    n = nb * bs
    x = (orc.normal(15, n * hkv * D) * np.float32(3)).reshape(n, hkv, D)
    c.append(x, -x, np.arange(n, dtype=np.int64))
    tables = np.arange(nb, dtype=np.int32)[None, :]
    gk, gv = c.gather(tables, np.array([n], np.int32), None, np.array([0], np.int64), n)
    rk, rv = gk.reshape(hkv, n, D // 32 * 20), gv.reshape(hkv, n, D // 32 * 20)
    for h in range(hkv):
        for t in (0, 1, 37, n - 1):
            assert bytes(rk[h, t]) == bytes(orc.quantize_row_q4_1(x[t, h]))
            assert bytes(rv[h, t]) == bytes(orc.quantize_row_q4_1(-x[t, h]))


# ---------------- Q5_0 / Q5_1 ----------------------------------------------
# The reference names the types (types.rs:116-117) and their group size
# (types.rs:9-10) and has no code for them; blocks, quantisers and
# dequantisers follow ggml and are pinned by hand-worked cases, special
# values and round-trip bounds.
def _u16(rec, i):
    return int(rec[0, i]) | (int(rec[0, i + 1]) << 8)


def _q5_values(rec, off):
    """5-bit values of one record from its bytes: qh at off, qs at off + 4;
    element e < 16 in the low nibble of qs[e], e >= 16 in the high nibble of
    qs[e - 16], bit 4 from bit e of the little-endian qh."""
    qh = int.from_bytes(bytes(rec[0, off:off + 4]), "little")
    qs = rec[0, off + 4:off + 20]
    nib = np.concatenate([qs & 0xF, qs >> 4]).astype(np.int64)
    return nib | (((qh >> np.arange(32)) & 1) << 4)


def test_q5_0_dequant_layout(orc):
    rec = np.zeros((1, 22), np.uint8)
    rec[0, :2] = np.frombuffer(np.float16(0.1).tobytes(), np.uint8)
    rec[0, 2:6] = [0xFF, 0xFF, 0xFF, 0xFF]  # every bit 4 set, nibbles 0: value 16 - 16 = 0
    assert np.all(orc.dequantize_row_q5_0(rec) == 0)
    rec[0, 2:6] = [0x55, 0x55, 0x0F, 0xF0]  # qh = 0xF00F5555: bits 0, 2, .., 14, 16-19, 28-31
    rec[0, 6:] = [j | ((15 - j) << 4) for j in range(16)]
    d = np.float32(np.float16(0.1))
    want = np.empty(32, np.float32)
    for j in range(16):
        want[j] = d * np.float32(j + (16 if j % 2 == 0 else 0) - 16)
        hb = 16 if (j < 4 or j >= 12) else 0  # bit 16 + j of 0xF00F5555
        want[16 + j] = d * np.float32((15 - j) + hb - 16)
    np.testing.assert_array_equal(orc.dequantize_row_q5_0(rec), want)


def test_q5_0_hand_worked_group(orc):
    # max = 16.0 (index 5; the -16.0 at index 20 has the same magnitude and
    # comes later): d = -1, id = -1, q = min(31, trunc(16.5 - x)).
    x = np.zeros(32, np.float32)
    vals = {0: 3.0, 1: -3.0, 2: 2.5, 3: -2.5, 4: 0.49, 5: 16.0, 6: 0.51, 7: 15.9, 8: -15.9, 20: -16.0, 21: 1.0}
    for i, v in vals.items():
        x[i] = v
    rec = orc.quantize_row_q5_0(x)
    assert rec.shape == (1, 22) and _u16(rec, 0) == _f16_bits(-1.0)
    want = np.full(32, 16)
    for i, q in {0: 13, 1: 19, 2: 14, 3: 19, 4: 16, 5: 0, 6: 15, 7: 0, 8: 31, 20: 31, 21: 15}.items():
        want[i] = q  # 16.5 + 15.9 = 32.4 and 16.5 + 16 = 32.5 clamp to 31
    np.testing.assert_array_equal(_q5_values(rec, 2), want)
    # qh bit e is set exactly where q >= 16; with these q: everything except 0, 2, 5, 6, 7, 21
    qh = int.from_bytes(bytes(rec[0, 2:6]), "little")
    assert qh == 0xFFFFFFFF & ~((1 << 0) | (1 << 2) | (1 << 5) | (1 << 6) | (1 << 7) | (1 << 21))
    np.testing.assert_array_equal(orc.dequantize_row_q5_0(rec), (want - 16).astype(np.float32) * np.float32(-1.0))


def test_q5_0_first_of_equal_magnitudes_zero_nan_inf(orc):
    x = np.zeros(32, np.float32)
    x[2], x[7] = -4.0, 4.0  # max = -4: d = 0.25, id = 4: -4 -> 0, 4 -> 32 -> 31
    rec = orc.quantize_row_q5_0(x)
    assert _u16(rec, 0) == _f16_bits(0.25)
    q = _q5_values(rec, 2)
    assert q[2] == 0 and q[7] == 31 and np.all(np.delete(q, [2, 7]) == 16)
    for z in (np.zeros(32, np.float32), -np.zeros(32, np.float32)):  # d = 0, id = 0: q = 16
        rec = orc.quantize_row_q5_0(z)
        assert _u16(rec, 0) & 0x7FFF == 0 and np.all(_q5_values(rec, 2) == 16)
    y = np.linspace(-1, 1, 32).astype(np.float32)
    y[3] = np.nan  # never the max; trunc(NaN) -> 0
    rec = orc.quantize_row_q5_0(y)
    assert _u16(rec, 0) == _f16_bits(0.0625) and _q5_values(rec, 2)[3] == 0
    y[3] = -np.inf  # d = inf, id = 0: finite x -> 16; the inf element -> NaN -> 0
    rec = orc.quantize_row_q5_0(y)
    q = _q5_values(rec, 2)
    assert _u16(rec, 0) == 0x7C00 and q[3] == 0 and np.all(np.delete(q, 3) == 16)


def test_q5_0_round_trip_bound(orc):
    x = orc.normal(24, 32 * 2048)
    rng = np.random.default_rng(3)
    x[rng.random(x.size) < 0.01] *= 8
    x[:32] *= 1e-3
    x[32:64] *= 3e3
    rec = orc.quantize_row_q5_0(x)
    deq = orc.dequantize_row_q5_0(rec).reshape(-1, 32)
    xg = x.reshape(-1, 32)
    d = np.abs(_q4_d(rec).astype(np.float32))[:, None]
    err = np.abs(deq - xg)
    # round half up onto d * (-16..15): at most d / 2, except the +16 end
    # (clamped to 15) at most d; slack for the fp16 rounding of d (2^-11
    # relative, times 16 steps)
    assert np.all(err <= d * (1 + 16 * 2 ** -10) + 1e-30)
    inner = np.abs(xg) < 15.5 * d
    assert np.all(err[inner] <= (d * 0.5 * (1 + 32 * 2 ** -10))[np.nonzero(inner)[0]].ravel() + 1e-30)
    imax = np.argmax(np.abs(xg), axis=1)  # comes back as -16 d
    np.testing.assert_array_equal(deq[np.arange(len(xg)), imax], -16 * _q4_d(rec).astype(np.float32))
    # every value is d times an integer in [-16, 15]
    dd = _q4_d(rec).astype(np.float32)[:, None]
    k = deq / np.where(dd == 0, 1, dd)
    assert np.all(k == np.round(k)) and k.min() >= -16 and k.max() <= 15


def test_q5_1_hand_worked_groups(orc):
    r = np.arange(32, dtype=np.float32)  # min 0, max 31: d = 1, id = 1, q = trunc(x + 0.5) = x
    rec = orc.quantize_row_q5_1(r)
    assert rec.shape == (1, 24) and _u16(rec, 0) == _f16_bits(1.0) and _u16(rec, 2) == _f16_bits(0.0)
    assert bytes(rec[0, 4:8]) == b"\x00\x00\xff\xff"  # elements 16..31 have bit 4
    assert np.all(rec[0, 8:] == [j | (j << 4) for j in range(16)])
    np.testing.assert_array_equal(orc.dequantize_row_q5_1(rec), r)
    m = r.copy()
    m[16:24] = [7.4, 7.5, 7.6, 0.49, 0.5, 30.5, 30.51, 3.0]
    rec = orc.quantize_row_q5_1(m)
    want = np.arange(32)
    want[16:24] = [7, 8, 8, 0, 1, 31, 31, 3]  # round half up
    np.testing.assert_array_equal(_q5_values(rec, 4), want)
    np.testing.assert_array_equal(orc.dequantize_row_q5_1(rec), want.astype(np.float32))


def test_q5_1_offset_nan_zero(orc):
    x = np.linspace(-1, 2, 32).astype(np.float32)  # d = 3/31, m = -1
    x[5] = np.nan  # never the min or the max; trunc(NaN) -> 0
    rec = orc.quantize_row_q5_1(x)
    d32 = np.float32(3.0) / np.float32(31.0)
    assert _u16(rec, 0) == _f16_bits(d32) and _u16(rec, 2) == _f16_bits(-1.0)
    q = _q5_values(rec, 4)
    assert q[5] == 0 and q[0] == 0 and q[31] == 31
    d = np.float32(np.float16(d32))
    np.testing.assert_array_equal(orc.dequantize_row_q5_1(rec), d * q.astype(np.float32) + np.float32(-1.0))
    rec = orc.quantize_row_q5_1(np.full(32, 2.5, np.float32))  # constant: d = 0, every q 0, value m
    assert _u16(rec, 0) == 0 and np.all(_q5_values(rec, 4) == 0)
    assert np.all(orc.dequantize_row_q5_1(rec) == 2.5)


def test_q5_1_round_trip_bound(orc):
    x = orc.normal(25, 32 * 2048)
    rng = np.random.default_rng(4)
    x[rng.random(x.size) < 0.01] *= 8
    x[:32] += 5.0  # all-positive group: m far from 0
    rec = orc.quantize_row_q5_1(x)
    deq = orc.dequantize_row_q5_1(rec).reshape(-1, 32)
    xg = x.reshape(-1, 32)
    d = (rec[:, 0].astype(np.uint16) | (rec[:, 1].astype(np.uint16) << 8)).view(np.float16).astype(np.float32)
    m = (rec[:, 2].astype(np.uint16) | (rec[:, 3].astype(np.uint16) << 8)).view(np.float16).astype(np.float32)
    # round half up onto min + d * (0..31), then the fp16 rounding of d (31
    # steps) and of m move the grid by at most 31 |d| 2^-11 + |m| 2^-11
    bound = d * 0.5 + (31 * d + np.abs(m)) * 2.0 ** -11 * 1.01 + 1e-30
    assert np.all(np.abs(deq - xg) <= bound[:, None])


@pytest.mark.parametrize("dt", ["Q5_0", "Q5_1"])
def test_oracle_q5_gather_records_equal_quantize_row(orc, dt):
    dtype = getattr(orc, dt)
    quant = orc.quantize_row_q5_0 if dt == "Q5_0" else orc.quantize_row_q5_1
    nb, bs, hkv, D = 4, 16, 2, 128
    c = orc.Cache(nb, bs, hkv, D, dtype)
    assert c.page_bytes == bs * (D // 2 + D // 32 * (6 if dt == "Q5_0" else 8))
    n = nb * bs
    x = (orc.normal(16, n * hkv * D) * np.float32(3)).reshape(n, hkv, D)
    c.append(x, -x, np.arange(n, dtype=np.int64))
    tables = np.arange(nb, dtype=np.int32)[None, :]
    gk, gv = c.gather(tables, np.array([n], np.int32), None, np.array([0], np.int64), n)
    rb = orc.RECORD_BYTES[dtype]
    rk, rv = gk.reshape(hkv, n, D // 32 * rb), gv.reshape(hkv, n, D // 32 * rb)
    for h in range(hkv):
        for t in (0, 1, 37, n - 1):
            assert bytes(rk[h, t]) == bytes(quant(x[t, h]))
            assert bytes(rv[h, t]) == bytes(quant(-x[t, h]))


def test_exact_decode_helper_and_closer_check(orc):
    """The float64 tie-break the GPU decode tests use for fp32 tolerance:
    exact_decode agrees with the oracle's decode, and a result perturbed by
    1e-4 is rejected even though the tie-break is consulted."""
    from kvutil import assert_close_or_closer, exact_decode, random_tables, slots_for

    hq, hkv, D, bs = 6, 2, 128, 16
    ctx = np.array([40, 77], np.int32)
    start = np.array([0, 9], np.int32)
    nb = 8
    tables = random_tables(3, ctx, bs, nb, 5)
    seqs = [0] * 40 + [1] * 77
    pos = list(range(40)) + list(range(77))
    slots = slots_for(tables, seqs, pos, bs)
    c = orc.Cache(nb, bs, hkv, D, orc.Q4_0)
    c.append(orc.normal(5, len(slots) * hkv * D).reshape(-1, hkv, D),
             orc.normal(6, len(slots) * hkv * D).reshape(-1, hkv, D), slots)
    q = orc.normal(7, 2 * hq * D).reshape(2, hq, D)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    want = c.decode(q, hq, tables, ctx, start, scale)
    exact, mag = exact_decode(c, q, hq, tables, ctx, start, scale, with_mag=True)
    assert np.max(np.abs(want - exact)) < 1e-5
    # The oracle itself is within the per-element bound the helper applies.
    assert np.all(np.abs(want - exact) <= 1e-6 + 1e-5 * mag)
    # mag bounds |exact| (a convex combination of the v_i) and is positive.
    assert np.all(np.abs(exact) <= mag + 1e-12) and np.all(mag > 0)
    fn = lambda: (exact, mag)  # noqa: E731
    assert_close_or_closer(want, want, fn, 1e-5, 1e-6)
    bad = want.copy()
    bad[1, 3, 17] += 1e-4
    with pytest.raises(AssertionError):
        assert_close_or_closer(bad, want, fn, 1e-5, 1e-6)
    # A perturbation within the oracle's tolerance but outside the
    # per-element bound of one cancelling element is still rejected: the
    # bound is per element, not the output's worst error.
    i = np.unravel_index(np.argmin(mag), mag.shape)
    bad = want.copy()
    bad[i] = exact[i] + 3e-5 * mag[i] + 1e-6
    off = np.abs(bad - want) > 1e-6 + 1e-5 * np.abs(want)
    if off[i]:
        with pytest.raises(AssertionError):
            assert_close_or_closer(bad, want, fn, 1e-5, 1e-6)


# ---------------- committed fixtures (tests/golden, written by make_golden.py) --
GOLDEN = os.path.join(ROOT, "tests", "golden")


def _golden_x(case) -> np.ndarray:
    return np.array(case["x_bits"], np.uint32).view(np.float32)


def test_golden_quant_cases(orc):
    import json

    for case in json.load(open(os.path.join(GOLDEN, "q8_cases.json"))):
        assert list(orc.quantize_row_q8_0(_golden_x(case))[0]) == case["record"], case["name"]
    for case in json.load(open(os.path.join(GOLDEN, "q4_cases.json"))):
        assert list(orc.quantize_row_q4_0(_golden_x(case))[0]) == case["q4_0"], case["name"]
        assert list(orc.quantize_row_q4_1(_golden_x(case))[0]) == case["q4_1"], case["name"]
    for case in json.load(open(os.path.join(GOLDEN, "q5_cases.json"))):
        assert list(orc.quantize_row_q5_0(_golden_x(case))[0]) == case["q5_0"], case["name"]
        assert list(orc.quantize_row_q5_1(_golden_x(case))[0]) == case["q5_1"], case["name"]


def test_golden_digests(orc):
    import hashlib
    import json

    man = json.load(open(os.path.join(GOLDEN, "manifest.json")))

    def sha(a):
        return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()

    x = orc.normal(20, 32 * 4096)
    u = orc.uniform_i32(20 ^ 0x5A5A, 0, 99, x.size)
    x = np.where(u == 0, x * np.float32(8), x).astype(np.float32)
    assert sha(orc.quantize_row_q8_0(x)) == man["q8_0_outliers"]["records_sha256"]
    assert sha(orc.quantize_row_q4_0(x)) == man["q4_0_outliers"]["records_sha256"]
    assert sha(orc.quantize_row_q4_1(x)) == man["q4_1_outliers"]["records_sha256"]
    assert sha(orc.quantize_row_q5_0(x)) == man["q5_0_outliers"]["records_sha256"]
    assert sha(orc.quantize_row_q5_1(x)) == man["q5_1_outliers"]["records_sha256"]
    c1 = man["config1"]
    k = orc.normal(c1["seeds"]["k"], 1024 * 2 * 128).reshape(1024, 2, 128)
    v = orc.normal(c1["seeds"]["v"], 1024 * 2 * 128).reshape(1024, 2, 128)
    c = orc.Cache(64, 16, 2, 128, orc.F32)
    c.append(k, v, np.arange(1024, dtype=np.int64))
    assert sha(c.k) == c1["k_pool_sha256"] and sha(c.v) == c1["v_pool_sha256"]
    out = np.load(os.path.join(GOLDEN, "config1_decode_out.npy"))
    assert sha(out) == c1["out_sha256"]


# ---------------- conversions --------------------------------------------
def test_f16_bf16_converters_exhaustive():
    exe = os.path.join(ROOT, "oracle", "check_f16")
    if not os.path.exists(exe):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    r = subprocess.run([exe, "1"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr


def test_q8_fast_quotient_identities(tmp_path):
    """The arithmetic the Q8_0 quantise-append kernels use instead of IEEE
    divisions (tests/check_q8_fast.c): amax / 127 from a faithful quotient
    plus one exact-remainder correction equals the IEEE quotient for every
    positive normal float, and the reciprocal-based rounding equals
    round(fl(x / scale)) whenever its residual test passes, for reciprocals
    within one ulp, on inputs placed at ties."""
    import shutil

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    exe = str(tmp_path / "check_q8_fast")
    b = subprocess.run([gcc, "-O3", "-fopenmp", "-ffp-contract=off", "-o", exe,
                        os.path.join(ROOT, "tests", "check_q8_fast.c"), "-lm"], capture_output=True, text=True)
    assert b.returncode == 0, b.stderr
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 mismatches over all" in r.stdout


def test_converters_match_numpy(orc):
    x = orc.normal(22, 100000) * np.float32(300)
    np.testing.assert_array_equal(orc.f32_to_f16(x), x.astype(np.float16).view(np.uint16))
    np.testing.assert_array_equal(orc.f16_to_f32(orc.f32_to_f16(x)), x.astype(np.float16).astype(np.float32))


# ---------------- BlockPool (src/memory/paged.rs:21-58) ------------------
def test_pool_lifo_closed_form(orc):
    p = orc.Pool(6)
    assert [p.allocate() for _ in range(6)] == [5, 4, 3, 2, 1, 0]
    assert p.allocate() is None
    assert p.free(2) == 0 and p.free(4) == 0
    assert p.allocate() == 4 and p.allocate() == 2  # most recently freed first


def test_pool_refcounts(orc):
    p = orc.Pool(3)
    b = p.allocate()
    assert p.share(b) == 0 and p.ref_count(b) == 2
    assert p.free(b) == 0 and p.num_free() == 2  # still referenced
    assert p.free(b) == 0 and p.num_free() == 3
    assert p.free(b) != 0  # would underflow the reference's u32
    assert p.share(0) != 0 and p.free(99) != 0


def test_pool_ordered(orc):
    order = orc.permutation(3, 10)
    p = orc.Pool(10, order=order)
    assert [p.allocate() for _ in range(10)] == list(order[::-1])


def test_pool_random_ops_against_list_model(orc):
    rng = np.random.default_rng(1)
    cap = 32
    p = orc.Pool(cap)
    free_list, refs = list(range(cap)), [0] * cap
    for _ in range(5000):
        op = rng.integers(3)
        if op == 0:
            got = p.allocate()
            want = free_list.pop() if free_list else None
            if want is not None:
                refs[want] = 1
            assert got == want
        else:
            i = int(rng.integers(cap))
            rc = p.share(i) if op == 1 else p.free(i)
            if refs[i] == 0:
                assert rc != 0
                continue
            assert rc == 0
            if op == 1:
                refs[i] += 1
            else:
                refs[i] -= 1
                if refs[i] == 0:
                    free_list.append(i)
        assert p.num_free() == len(free_list)
    assert list(p.free_list()) == free_list


# ---------------- window manager: config-4 closed forms --------------------
def _c4_manager(orc, n_seqs=64, start=30000, W=4096, bs=16, cap=16512, seed=4):
    pool = orc.Pool(cap, order=orc.permutation(seed, cap))
    first = (start - W) // bs
    last = (start - 1) // bs
    max_blocks = 32768 // bs + 1
    m = orc.Manager(pool, bs, n_seqs, max_blocks, W)
    for s in range(n_seqs):
        blocks = [pool.allocate() for _ in range(last - first + 1)]
        m.seed_seq(s, start, first, blocks)
    return pool, m, first, last


def test_window_c4_schedule(orc):
    pool, m, first, last = _c4_manager(orc)
    assert (first, last, last - first + 1) == (1619, 1874, 256)
    seqs = list(range(64))
    frees = allocs = 0
    prev_free_top = None
    for p in range(30000, 32768):
        n_free_before = pool.num_free()
        slots, ev = m.append(seqs)
        if p % 16 == 15:
            assert len(ev) == 64
            prev_free_top = ev[-1]  # seq 63 frees last
        else:
            assert len(ev) == 0
        if p % 16 == 0:
            allocs += 1
            if prev_free_top is not None and p == 30016:
                # LIFO: seq 0 is handed the block seq 63 freed at p = 30015.
                assert slots[0] // 16 == prev_free_top
        frees += len(ev) // 64
        assert pool.num_free() == n_free_before + len(ev) - (64 if p % 16 == 0 else 0)
        assert np.all(slots % 16 == p % 16)
    assert frees == 173 and allocs == 173
    t, cl, sp = m.tables()
    assert np.all(cl == 32768) and np.all(sp == 32768 - 4096)
    held = (t >= 0).sum(1)
    assert np.all(held == 256)
    live = t[t >= 0]
    assert len(np.unique(live)) == live.size  # no block owned twice


# ---------------- paged cache restatement (append / gather / evict) --------
def _page_row(pool, page_bytes, hkv, D, e, slot, h, bs):
    """The documented pool layout: page (block, head) holds bs rows of D
    elements; row slot % bs of page (slot // bs) * Hkv + h."""
    off = ((slot // bs) * hkv + h) * page_bytes + (slot % bs) * D * e
    return pool[off:off + D * e]


@pytest.mark.parametrize("dt,e", [(0, 4), (30, 2), (1, 2)])
def test_oracle_append_layout_and_gather_round_trip(orc, dt, e):
    nb, bs, hkv, D = 12, 16, 3, 32
    c = orc.Cache(nb, bs, hkv, D, dt)
    c.k[:] = 0xA5
    c.v[:] = 0xA5
    slots = orc.permutation(5, nb * bs)[:40].copy()
    slots[7] = -1  # padding token: skipped
    n = slots.size
    if dt == orc.F32:
        k, v = orc.normal(6, n * hkv * D), orc.normal(7, n * hkv * D)
    else:
        conv = orc.f32_to_bf16 if dt == orc.BF16 else orc.f32_to_f16
        k, v = conv(orc.normal(6, n * hkv * D)), conv(orc.normal(7, n * hkv * D))
    k, v = k.reshape(n, hkv, D), v.reshape(n, hkv, D)
    c.append(k, v, slots)
    page_bytes = bs * D * e
    touched = np.zeros(c.k.size, bool)
    for t, s in enumerate(slots):
        if s < 0:
            continue
        for h in range(hkv):
            got = _page_row(c.k, page_bytes, hkv, D, e, int(s), h, bs)
            assert bytes(got) == k[t, h].tobytes()
            assert bytes(_page_row(c.v, page_bytes, hkv, D, e, int(s), h, bs)) == v[t, h].tobytes()
            off = ((s // bs) * hkv + h) * page_bytes + (s % bs) * D * e
            touched[off:off + D * e] = True
    assert np.all(c.k[~touched] == 0xA5) and np.all(c.v[~touched] == 0xA5)  # no stray writes
    # Gather through a block table reproduces the rows in logical order.
    seq_slots = np.array([s for s in slots if s >= 0][:20], np.int64)
    blocks = np.unique(seq_slots // bs)
    # one sequence holding those blocks in this order, positions = rows of those pages
    tables = blocks.astype(np.int32)[None, :]
    ctx = np.array([blocks.size * bs], np.int32)
    start = np.array([5], np.int32)
    cu = np.array([0], np.int64)
    gk, gv = c.gather(tables, ctx, start, cu, int(ctx[0] - start[0]))
    gk = gk.view(k.dtype).reshape(hkv, -1, D)
    for i in range(int(ctx[0] - start[0])):
        p = int(start[0]) + i
        s = int(blocks[p // bs]) * bs + p % bs
        for h in range(hkv):
            assert bytes(gk[h, i]) == bytes(_page_row(c.k, page_bytes, hkv, D, e, s, h, bs))


def test_oracle_evict_zeroes_exactly_the_listed_blocks(orc):
    nb, bs, hkv, D = 10, 16, 2, 32
    c = orc.Cache(nb, bs, hkv, D, orc.BF16)
    c.k[:] = 7
    c.v[:] = 9
    c.evict(np.array([2, 7], np.int32))
    pb = bs * D * 2 * hkv
    for b in range(nb):
        want_k, want_v = (0, 0) if b in (2, 7) else (7, 9)
        assert np.all(c.k[b * pb:(b + 1) * pb] == want_k) and np.all(c.v[b * pb:(b + 1) * pb] == want_v)


def test_oracle_q8_gather_records_equal_quantize_row(orc):
    nb, bs, hkv, D = 4, 32, 2, 64
    c = orc.Cache(nb, bs, hkv, D, orc.Q8_0)
    n = nb * bs
    x = (orc.normal(13, n * hkv * D) * np.float32(3)).reshape(n, hkv, D)
    c.append(x, -x, np.arange(n, dtype=np.int64))
    tables = np.arange(nb, dtype=np.int32)[None, :]
    gk, gv = c.gather(tables, np.array([n], np.int32), None, np.array([0], np.int64), n)
    rec = gk.reshape(hkv, n, D // 32 * 34)
    for h in range(hkv):
        for t in (0, 1, 77, n - 1):
            assert bytes(rec[h, t]) == bytes(orc.quantize_row_q8_0(x[t, h]))


# ---------------- paged attention restatement vs float64 brute force --------
def _softmax_av(q, K, V, scale):
    s = (K.astype(np.float64) @ q.astype(np.float64)) * scale
    p = np.exp(s - s.max())
    return (p @ V.astype(np.float64)) / p.sum()


def _fill(orc, nb, bs, hkv, D, seed):
    c = orc.Cache(nb, bs, hkv, D, orc.F32)
    c.k[:] = np.frombuffer(orc.normal(seed, c.k.size // 4).tobytes(), np.uint8)
    c.v[:] = np.frombuffer(orc.normal(seed + 1, c.v.size // 4).tobytes(), np.uint8)
    kf = c.k.view(np.float32).reshape(nb, hkv, bs, D)
    vf = c.v.view(np.float32).reshape(nb, hkv, bs, D)
    return c, kf, vf


def test_oracle_paged_decode_gqa_window_vs_float64(orc):
    """Paging (scrambled table), the GQA map h -> h * Hkv / Hq
    (forward.rs:234) and window starts, against float64 softmax over rows
    collected with numpy."""
    nb, bs, hkv, hq, D = 24, 16, 2, 6, 32
    c, kf, vf = _fill(orc, nb, bs, hkv, D, 21)
    perm = orc.permutation(22, nb).astype(np.int32)
    tables = np.stack([perm[:10], perm[10:20]])
    ctx = np.array([150, 97], np.int32)
    start = np.array([0, 40], np.int32)
    q = orc.normal(23, 2 * hq * D).reshape(2, hq, D)
    scale = 0.17
    got = c.decode(q, hq, tables, ctx, start, scale)
    for b in range(2):
        for h in range(hq):
            kvh = h * hkv // hq
            rows = range(int(start[b]), int(ctx[b]))
            K = np.stack([kf[tables[b, p // bs], kvh, p % bs] for p in rows])
            V = np.stack([vf[tables[b, p // bs], kvh, p % bs] for p in rows])
            np.testing.assert_allclose(got[b, h], _softmax_av(q[b, h], K, V, scale), rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("dt", ["Q5_0", "Q5_1", "Q4_1"])
def test_oracle_quant_decode_reads_the_dequantised_rows(orc, dt):
    """The oracle's decode over a quantised cache attends over exactly the
    dequantised records its gather returns (float64 softmax of those rows)."""
    dtype = getattr(orc, dt)
    nb, bs, hkv, hq, D = 8, 16, 2, 4, 64
    c = orc.Cache(nb, bs, hkv, D, dtype)
    n = nb * bs
    c.append(orc.normal(40, n * hkv * D).reshape(n, hkv, D), orc.normal(41, n * hkv * D).reshape(n, hkv, D),
             np.arange(n, dtype=np.int64))
    tables = orc.permutation(42, nb).astype(np.int32)[None, :]
    ctx = np.array([101], np.int32)
    q = orc.normal(43, hq * D).reshape(1, hq, D)
    got = c.decode(q, hq, tables, ctx, None, 0.125)
    gk, gv = c.gather(tables, ctx, None, np.array([0], np.int64), 101)
    K = orc.dequantize_records(gk, dtype).reshape(hkv, 101, D)
    V = orc.dequantize_records(gv, dtype).reshape(hkv, 101, D)
    for h in range(hq):
        np.testing.assert_allclose(got[0, h], _softmax_av(q[0, h], K[h * hkv // hq], V[h * hkv // hq], 0.125),
                                   rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("causal", [True, False])
def test_oracle_paged_prefill_vs_float64(orc, causal):
    nb, bs, hkv, hq, D = 20, 16, 2, 4, 32
    c, kf, vf = _fill(orc, nb, bs, hkv, D, 31)
    perm = orc.permutation(32, nb).astype(np.int32)
    tables = np.stack([perm[:10], perm[10:20]])
    ctx = np.array([120, 41], np.int32)
    ql = np.array([30, 41], np.int32)
    cu = np.array([0, 30, 71], np.int32)
    q = orc.normal(33, 71 * hq * D).reshape(71, hq, D)
    scale = 0.2
    got = c.prefill(q, hq, cu, tables, ctx, scale, causal=causal)
    for b in range(2):
        for i in range(int(ql[b])):
            last = int(ctx[b] - ql[b] + i) if causal else int(ctx[b]) - 1  # row i sits at ctx - q_len + i
            for h in range(hq):
                kvh = h * hkv // hq
                K = np.stack([kf[tables[b, p // bs], kvh, p % bs] for p in range(last + 1)])
                V = np.stack([vf[tables[b, p // bs], kvh, p % bs] for p in range(last + 1)])
                np.testing.assert_allclose(got[cu[b] + i, h], _softmax_av(q[cu[b] + i, h], K, V, scale),
                                           rtol=2e-5, atol=2e-6)


# ---- RoPE (rope.rs:6-44) ----------------------------------------------------
def test_rope_reference_kat(orc):
    """rope.rs:50-68: ones over 2 heads of 64, n_dims 64: position 0 keeps
    every element within 0.1 of 1; position 100 moves element 0 by > 0.1."""
    x = np.ones(128, np.float32)
    out0 = orc.rope(x, 0, 64, 64)
    assert np.all(np.abs(out0 - 1.0) < 0.1)
    assert abs(orc.rope(x, 100, 64, 64)[0] - 1.0) > 0.1


def test_rope_position_zero_is_identity(orc):
    x = orc.normal(41, 4 * 128).reshape(4, 128)
    assert np.array_equal(orc.rope(x, 0, 128, 128).view(np.uint32), x.view(np.uint32))


@pytest.mark.parametrize("pos", [1, 7, 100, 2047, 4095, 130000])
def test_rope_first_pair_angle_is_position(orc, pos):
    """Pair 0 has exponent -0/n, so theta = (float)pos exactly: (1, 0) maps to
    (cos pos, sin pos) of the float32 position."""
    x = np.zeros(128, np.float32)
    x[0] = 1.0
    out = orc.rope(x, pos, 128, 128)
    t = float(np.float32(pos))
    assert abs(out[0] - math.cos(t)) < 2e-7 and abs(out[1] - math.sin(t)) < 2e-7


@pytest.mark.parametrize("pos,n_dims,head_dim", [(5, 128, 128), (333, 64, 128), (4000, 256, 256)])
def test_rope_matches_float64_rotation(orc, pos, n_dims, head_dim):
    """Against a float64 rotation by the float32 angle of each pair (the
    angle computed as rope.rs:31 does, in numpy float32): agreement to a few
    float32 ulps; a swapped sign, a wrong pair or a wrong exponent would be
    off by O(1).  Elements past n_dims are copied bit for bit."""
    x = orc.normal(43 + pos, 3 * head_dim).reshape(3, head_dim)
    out = orc.rope(x, pos, n_dims, head_dim)
    i = np.arange(0, n_dims, 2)
    e = (-i.astype(np.float32)) / np.float32(n_dims)
    theta = (np.float32(pos) * np.power(np.float32(10000.0), e, dtype=np.float32)).astype(np.float64)
    c, s = np.cos(theta), np.sin(theta)
    x0, x1 = x[:, 0:n_dims:2].astype(np.float64), x[:, 1:n_dims:2].astype(np.float64)
    want0, want1 = x0 * c - x1 * s, x0 * s + x1 * c
    # numpy's float32 power may differ from powf by an ulp; that moves theta
    # by up to pos * 6e-8 rad.
    tol = 4e-6 + 2e-7 * pos * np.maximum(np.abs(x0), np.abs(x1))
    assert np.all(np.abs(out[:, 0:n_dims:2] - want0) <= tol)
    assert np.all(np.abs(out[:, 1:n_dims:2] - want1) <= tol)
    assert np.array_equal(out[:, n_dims:].view(np.uint32), x[:, n_dims:].view(np.uint32))


def test_rope_preserves_pair_norm_and_composes(orc):
    x = orc.normal(47, 2 * 128).reshape(2, 128)
    a = orc.rope(x, 300, 128, 128)
    n_in = np.hypot(x[:, 0::2].astype(np.float64), x[:, 1::2].astype(np.float64))
    n_out = np.hypot(a[:, 0::2].astype(np.float64), a[:, 1::2].astype(np.float64))
    assert np.allclose(n_out, n_in, rtol=1e-6, atol=1e-7)
    # theta is linear in the position: rotating by 300 then 200 = rotating by
    # 500, up to the float32 rounding of each angle (an ulp of 500 is 3e-5).
    b = orc.rope(a, 200, 128, 128)
    assert np.allclose(b, orc.rope(x, 500, 128, 128), atol=1.5e-4)


def test_rope_rejects_bad_shapes(orc):
    with pytest.raises(ValueError):
        orc.rope(np.ones(100, np.float32), 1, 64, 64)  # not a multiple of head_dim
    with pytest.raises(ValueError):
        orc.rope(np.ones(64, np.float32), 1, 63, 64)  # odd n_dims


# ---------------- manager: prefix sharing under a window --------------------
def test_window_release_keeps_blocks_a_fork_holds(orc):
    """Pool 16, block size 4, window 8.  Seq 0 takes 10 tokens (blocks 15,
    14, 13), seq 1 forks it, seq 0 appends 4 more with copy-on-write.  At
    p = 11 the window drops seq 0's reference to block 15, which seq 1 still
    holds: BlockPool::free (paged.rs:48-53) leaves it at refcount 1, off the
    free list, so it is not an evicted page.  When seq 1's own window passes
    it, the refcount reaches 0 and it is listed."""
    pool = orc.Pool(16)
    m = orc.Manager(pool, 4, 2, 8, 8)
    slots, ev = m.append([0], [10])
    assert list(slots // 4) == [15] * 4 + [14] * 4 + [13] * 2 and ev.size == 0
    m.fork(0, 1)
    assert [pool.ref_count(b) for b in (15, 14, 13)] == [2, 2, 2]
    slots, ev, cs, cd = m.append([0], [4], cow=True)
    # p=10 writes into shared partial block 13: copied to 12 (LIFO top).
    assert list(cs) == [13] and list(cd) == [12]
    # p=12 opens a new block: 11.
    assert list(slots // 4) == [12, 12, 11, 11]
    assert ev.size == 0
    assert pool.ref_count(15) == 1 and pool.ref_count(13) == 1 and pool.num_free() == 11
    t, cl, _ = m.tables()
    assert list(t[1, :3]) == [15, 14, 13] and t[0, 0] == -1 and list(t[0, 1:4]) == [14, 12, 11]
    # Seq 1 advances to p = 11: its window drops block 15, the last reference.
    slots, ev, cs, cd = m.append([1], [2], cow=True)
    assert list(cs) == [13] or cs.size == 0
    assert list(ev) == [15] and pool.ref_count(15) == 0
    # Releasing seq 0 returns only the blocks nobody else holds (12 and 11);
    # block 14 stays with seq 1.
    freed = m.release(0)
    assert sorted(freed.tolist()) == [11, 12] and pool.ref_count(14) == 1


def _held(t):
    return set(int(b) for b in t.ravel() if b >= 0)


def _check_manager_invariants(pool, t, cap):
    """Refcount of every block = the number of table entries naming it; a
    block no table names is on the free list (refcount 0)."""
    refs = {}
    for b in t.ravel():
        if b >= 0:
            refs[int(b)] = refs.get(int(b), 0) + 1
    for b in range(cap):
        assert pool.ref_count(b) == refs.get(b, 0), (b, pool.ref_count(b), refs.get(b, 0))
    assert pool.num_free() == cap - len(refs)


def test_manager_fork_cow_window_random_invariants(orc):
    """Random appends (plain and copy-on-write), forks and releases, with and
    without a window, on tiny pools: after every operation the refcounts equal
    the table entries naming each block, every slot lies in the block its
    table names, and the evicted list is exactly the blocks no table names
    any more (those BlockPool::free pushed: paged.rs:48-53)."""
    rng = np.random.default_rng(17)
    for W in (0, 12, 40):
        cap, bs, S, mb = 48, 4, 5, 40
        pool = orc.Pool(cap, order=orc.permutation(W + 1, cap))
        m = orc.Manager(pool, bs, S, mb, W)
        n_shared_release = n_ev = 0
        for _ in range(600):
            t0, ctx0, _ = m.tables()
            held0 = _held(t0)
            op = rng.integers(10)
            if op < 7:
                seqs = rng.permutation(S)[: int(rng.integers(1, S + 1))]
                nt = rng.integers(0, 6, seqs.size)
                if (ctx0[seqs] + nt).max() >= mb * bs or pool.num_free() < 3 * seqs.size + 2:
                    for s in range(S):
                        m.release(s)
                    continue
                slots, ev = m.append(seqs, nt, cow=bool(op % 2))[:2]
                t1, ctx1, _ = m.tables()
                k = 0
                for s, n in zip(seqs, nt):
                    for j in range(int(n)):
                        p = int(ctx0[s]) + j
                        assert slots[k] == int(t1[s, p // bs]) * bs + p % bs
                        k += 1
                held1 = _held(t1)
                # Listed = dropped from every table (a block reused by a later
                # token of the same step is listed and held again).
                assert held0 - held1 <= set(ev.tolist())
                for b in ev:
                    assert int(b) in held0
                    assert int(b) in held1 or pool.ref_count(int(b)) == 0
                n_shared_release += len([b for b in held0 & held1 if b not in ev])
                n_ev += ev.size
            elif op < 9:
                s = int(rng.integers(S))
                freed = m.release(s)
                t1, _, _ = m.tables()
                assert set(freed.tolist()) == held0 - _held(t1)
            else:
                empty = [s for s in range(S) if ctx0[s] == 0]
                src = int(rng.integers(S))
                if empty and empty[0] != src:
                    m.fork(src, empty[0])
            t, _, _ = m.tables()
            _check_manager_invariants(pool, t, cap)
        assert n_ev > 0 or W == 0


# ---------------- OpenMP entry points equal the single-threaded ones --------
def _ragged_cache(orc, dt, nb=96, bs=16, hkv=2, D=64, seed=50):
    c = orc.Cache(nb, bs, hkv, D, dt)
    n = nb * bs
    src_dt = orc.BF16 if dt == orc.BF16 else orc.F32
    k, v = orc.normal(seed, n * hkv * D), orc.normal(seed + 1, n * hkv * D)
    if src_dt == orc.BF16:
        k, v = orc.f32_to_bf16(k), orc.f32_to_bf16(v)
    c.append(k.reshape(n, hkv, D), v.reshape(n, hkv, D), np.arange(n, dtype=np.int64))
    return c


@pytest.mark.parametrize("dt", ["BF16", "F32", "Q8_0"])
def test_oracle_decode_mt_equals_single_thread(orc, dt):
    """orc_paged_decode_mt (the checker of the full-size GPU tests and the
    all-cores CPU baseline) equals orc_paged_decode bit for bit: ragged
    contexts, empty and one-token sequences, window starts, thread counts
    2..16 (fewer and more threads than sequences x heads)."""
    dtype = getattr(orc, dt)
    nb, bs, hkv, hq, D = 96, 16, 2, 6, 64
    c = _ragged_cache(orc, dtype, nb, bs, hkv, D)
    perm = orc.permutation(51, nb).astype(np.int32)
    ctx = np.array([300, 1, 0, 517, 64, 1000, 129], np.int32)
    tables = np.full((ctx.size, 64), -1, np.int32)
    k = 0
    for b, n in enumerate(ctx):
        nbk = (int(n) + bs - 1) // bs
        tables[b, :nbk] = perm[k % nb:k % nb + nbk] if k % nb + nbk <= nb else perm[:nbk]
        k += nbk
    q = orc.normal(52, ctx.size * hq * D).reshape(ctx.size, hq, D)
    for start in (None, np.array([0, 0, 0, 200, 63, 744, 1], np.int32)):
        want = c.decode(q, hq, tables, ctx, start, 0.125)
        for threads in (2, 3, 8, 16):
            got = c.decode(q, hq, tables, ctx, start, 0.125, threads=threads)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (threads, start is None)


@pytest.mark.parametrize("causal", [True, False])
def test_oracle_prefill_rows_mt_equals_single_thread(orc, causal):
    """orc_paged_prefill_rows_mt (the checker of the full-size prefill test)
    equals orc_paged_prefill_rows bit for bit, causal and not, for row
    ranges at the chunk's start, middle and end, thread counts 2..16."""
    nb, bs, hkv, hq, D = 96, 16, 2, 8, 64
    c = _ragged_cache(orc, orc.BF16, nb, bs, hkv, D, seed=60)
    perm = orc.permutation(61, nb).astype(np.int32)
    ctx = np.array([700, 333], np.int32)
    ql = np.array([90, 333], np.int32)
    cu = np.array([0, 90, 423], np.int32)
    tables = np.stack([perm[:48], perm[48:96]])
    q = orc.normal(62, int(cu[-1]) * hq * D).reshape(int(cu[-1]), hq, D)
    for s, b, e in ((0, 0, 90), (0, 37, 41), (1, 0, 5), (1, 300, 333)):
        want = c.prefill(q, hq, cu, tables, ctx, 0.1, causal=causal, rows=(s, b, e))
        for threads in (2, 5, 16):
            got = c.prefill(q, hq, cu, tables, ctx, 0.1, causal=causal, rows=(s, b, e), threads=threads)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (s, b, e, threads)
