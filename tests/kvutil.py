"""Shared helpers of the parity tests: seeded inputs (from the oracle's RNG),
block tables and slot mappings, and host<->device plumbing."""
from __future__ import annotations

import numpy as np

import oracle as orc

DT_NP = {orc.F32: np.float32, orc.BF16: np.uint16, orc.F16: np.uint16}


def kv_values(seed: int, n: int, dtype: int, outliers: bool = False) -> np.ndarray:
    """N(0,1) in the storage representation of `dtype` (bf16/f16 as bits)."""
    x = orc.normal(seed, n)
    if outliers:  # config 5: 1% of elements scaled by 8
        u = orc.uniform_i32(seed ^ 0x5A5A, 0, 99, n)
        x = np.where(u == 0, x * np.float32(8), x).astype(np.float32)
    if dtype == orc.BF16:
        return orc.f32_to_bf16(x)
    if dtype == orc.F16:
        return orc.f32_to_f16(x)
    return x


def widen(x: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == orc.BF16:
        return orc.bf16_to_f32(x)
    if dtype == orc.F16:
        return orc.f16_to_f32(x)
    return x.astype(np.float32)


def random_tables(seed: int, ctx_lens, bs: int, pool_blocks: int, max_blocks: int) -> np.ndarray:
    """Block tables over a seeded permutation of the pool (non-contiguous pages)."""
    perm = orc.permutation(seed, pool_blocks)
    t = np.full((len(ctx_lens), max_blocks), -1, np.int32)
    k = 0
    for b, c in enumerate(ctx_lens):
        nb = (int(c) + bs - 1) // bs
        t[b, :nb] = perm[k:k + nb]
        k += nb
    assert k <= pool_blocks
    return t


def slots_for(tables: np.ndarray, seqs, positions, bs: int) -> np.ndarray:
    return np.array([int(tables[s, p // bs]) * bs + p % bs for s, p in zip(seqs, positions)], np.int64)


def to_dev(a: np.ndarray, torch_dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if torch_dtype is not None:
        t = t.view(torch_dtype)
    return t.to("cuda:0")


def from_dev(t) -> np.ndarray:
    import torch

    t = t.detach().to("cpu").contiguous()
    if t.dtype == torch.bfloat16 or t.dtype == torch.float16:
        t = t.view(torch.int16)
    a = t.numpy()
    return a.view(np.uint16) if a.dtype == np.int16 else a


def assert_close(got: np.ndarray, want: np.ndarray, rtol: float, atol: float, what: str = "") -> None:
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    if bad.any():
        i = np.flatnonzero(bad.ravel())[0]
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside |d| <= {atol} + {rtol}|ref|; first at {i}: "
                             f"got {got.ravel()[i]!r} want {want.ravel()[i]!r}; max err {err.max():.3g}")


def exact_decode(ref, q, hq: int, tables, ctx, start, scale: float, with_mag: bool = False):
    """float64 softmax(q K^T * scale) V over the rows the oracle cache `ref`
    holds (its stored values widened exactly: bf16/f16, Q8_0 f32(d)*q, Q4_0
    f32(d)*(n-8)), keys start_b..ctx_b-1 of KV head h*Hkv/Hq.  The rounding-
    free answer both fp32 implementations approximate.  with_mag: also the
    magnitude of each output's terms, sum_i p_i |v_i| / sum_i p_i, which
    bounds what fp32 summation error can do to that element."""
    ctx = np.asarray(ctx, np.int32)
    st = np.zeros_like(ctx) if start is None else np.asarray(start, np.int32)
    n = ctx - st
    cu = np.concatenate([[0], np.cumsum(n)[:-1]]).astype(np.int64)
    hkv, D, dt = ref.desc.n_kv_heads, ref.desc.head_dim, ref.desc.dtype
    gk, gv = ref.gather(tables, ctx, st, cu, int(n.sum()))
    rb = ref.row_out_bytes()

    def rows(g, b):
        raw = g[int(cu[b]) * hkv * rb:(int(cu[b]) + int(n[b])) * hkv * rb].reshape(hkv, int(n[b]), rb)
        if dt in orc.QUANT_TYPES:
            return orc.dequantize_records(raw, dt).reshape(hkv, int(n[b]), D)
        if dt == orc.F32:
            return raw.view(np.float32).reshape(hkv, int(n[b]), D)
        return widen(raw.view(np.uint16), dt).reshape(hkv, int(n[b]), D)

    out = np.zeros((len(ctx), hq, D), np.float64)
    mag = np.zeros((len(ctx), hq, D), np.float64)
    for b in range(len(ctx)):
        if n[b] <= 0:
            continue
        K, V = rows(gk, b).astype(np.float64), rows(gv, b).astype(np.float64)
        for h in range(hq):
            kv = h * hkv // hq
            s = K[kv] @ q[b, h].astype(np.float64) * scale
            p = np.exp(s - s.max())
            out[b, h] = p @ V[kv] / p.sum()
            if with_mag:
                mag[b, h] = p @ np.abs(V[kv]) / p.sum()
    return (out, mag) if with_mag else out


def lazy(fn):
    """fn() computed on the first call only."""
    box = []

    def get():
        if not box:
            box.append(fn())
        return box[0]

    return get


def assert_close_or_closer(got, want, exact_fn, rtol: float, atol: float, what: str = "") -> None:
    """assert_close, except that an element outside the tolerance of the fp32
    oracle `want` passes when it is within atol + rtol * mag of the float64
    answer, where exact_fn() returns (exact, mag) as exact_decode(...,
    with_mag=True) does: mag = sum_i p_i |v_i| / sum_i p_i, the size of the
    terms that element sums.  Two fp32 summation orders cannot agree to
    rtol |ref| on an element whose terms cancel (an output of 0.009 from
    terms of total magnitude ~2), and there either one can be the closer;
    both stay within a relative error of the terms' magnitude, which is the
    bound fp32 summation gives, element by element."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bad = np.abs(got - want) > atol + rtol * np.abs(want)
    if not bad.any():
        return
    exact, mag = exact_fn()
    exact = np.asarray(exact, np.float64).reshape(got.shape)
    mag = np.asarray(mag, np.float64).reshape(got.shape)
    worse = bad & (np.abs(got - exact) > atol + rtol * mag)
    if worse.any():
        i = np.flatnonzero(worse.ravel())[0]
        raise AssertionError(f"{what}: {worse.sum()} of {worse.size} outside |d| <= {atol} + {rtol}|ref| and farther "
                             f"from the float64 answer than {atol} + {rtol} x the magnitude of its terms; first at "
                             f"{i}: got {got.ravel()[i]!r} want {want.ravel()[i]!r} exact {exact.ravel()[i]!r} "
                             f"terms {mag.ravel()[i]!r}")
