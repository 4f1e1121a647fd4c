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
