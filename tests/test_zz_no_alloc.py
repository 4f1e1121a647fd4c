"""it_paged_decode_noalloc (the decode entry point that allocates nothing:
its partials live in the library's per-GPU device array) against
it_paged_decode with a caller workspace, called through the C ABI.  Both run
the same kernels in a fixed reduction order, so outputs must be equal bit for
bit.  Two calls in a row, the second with a smaller batch, so the array still
holds the first call's partials; a request larger than the array is
rejected before any launch."""
import ctypes as C
import math

import numpy as np
import pytest

import oracle as orc
from kvutil import from_dev, kv_values, random_tables, slots_for, to_dev

pytestmark = pytest.mark.gpu


def _cache(hq, hkv, D, bs, ctx, seed):
    import torch
    from infer_train_amd.kv import PagedKvCache

    ctx = np.asarray(ctx, np.int32)
    mb = int((ctx.max() + bs - 1) // bs)
    nb = int(sum((int(c) + bs - 1) // bs for c in ctx))
    tables = random_tables(seed, ctx, bs, nb, mb)
    seqs, pos = [], []
    for b, c in enumerate(ctx):
        seqs += [b] * int(c)
        pos += list(range(int(c)))
    slots = slots_for(tables, seqs, pos, bs)
    n = len(slots)
    k = kv_values(seed + 1, n * hkv * D, orc.BF16).reshape(n, hkv, D)
    v = kv_values(seed + 2, n * hkv * D, orc.BF16).reshape(n, hkv, D)
    dev = PagedKvCache(nb, bs, hkv, D, orc.BF16)
    dev.append(to_dev(k.view(np.int16), torch.bfloat16), to_dev(v.view(np.int16), torch.bfloat16), to_dev(slots))
    q = kv_values(seed + 3, len(ctx) * hq * D, orc.BF16).reshape(len(ctx), hq, D)
    return dev, tables, ctx, q


def _noalloc(dev, q, tables, ctx, start, max_tokens, partition, out):
    from infer_train_amd._lib import BF16, F32, lib
    from infer_train_amd.kv import stream_handle

    n_seqs, n_heads, _ = q.shape
    return lib.it_paged_decode_noalloc(dev._h, q.data_ptr(), BF16, n_heads, tables.data_ptr(), tables.shape[1],
                                       ctx.data_ptr(), None if start is None else start.data_ptr(), n_seqs,
                                       max_tokens, C.c_float(1.0 / math.sqrt(q.shape[2])), partition,
                                       out.data_ptr(), F32, stream_handle())


def test_noalloc_equals_paged_decode_twice():
    import torch
    from infer_train_amd._lib import OK

    hq, hkv, D, bs = 28, 4, 128, 16
    cases = [  # (contexts, partition): the second call is smaller
        (orc.uniform_i32(5, 256, 4096, 32) + 1, 512),
        (np.array([900, 37, 1500], np.int32), 256),
    ]
    for i, (ctx, partition) in enumerate(cases):
        dev, tables, ctx, q = _cache(hq, hkv, D, bs, ctx, seed=60 + i)
        dq = to_dev(q.view(np.int16), torch.bfloat16)
        dt, dc = to_dev(tables), to_dev(ctx)
        max_tokens = int(ctx.max())
        want = dev.decode(dq, dt, dc, None, max_tokens, partition=partition, out_dtype=torch.float32)
        got = torch.full_like(want, float("nan"))
        assert _noalloc(dev, dq, dt, dc, None, max_tokens, partition, got) == OK
        dev.check()
        np.testing.assert_array_equal(from_dev(got), from_dev(want), err_msg=f"call {i}: {len(ctx)} sequences")
    # Windowed starts go through the same array.
    ctx = np.array([700, 1200, 64], np.int32)
    dev, tables, ctx, q = _cache(16, 2, D, bs, ctx, seed=70)
    start = np.array([100, 0, 63], np.int32)
    dq = to_dev(q.view(np.int16), torch.bfloat16)
    want = dev.decode(dq, to_dev(tables), to_dev(ctx), to_dev(start), 1200, partition=128, out_dtype=torch.float32)
    got = torch.full_like(want, float("nan"))
    assert _noalloc(dev, dq, to_dev(tables), to_dev(ctx), to_dev(start), 1200, 128, got) == OK
    np.testing.assert_array_equal(from_dev(got), from_dev(want))


def test_noalloc_rejects_more_than_its_array():
    import torch
    from infer_train_amd import InvalidInput
    from infer_train_amd._lib import INVALID_INPUT, check, lib

    hq, hkv, D, bs = 28, 4, 128, 16
    dev, tables, ctx, q = _cache(hq, hkv, D, bs, [64, 64], seed=80)
    dq = to_dev(q.view(np.int16), torch.bfloat16)
    out = torch.zeros(q.shape, dtype=torch.float32, device="cuda:0")
    # max_tokens 262144 at 64-token partitions: 4096 partials per row of
    # 2 sequences x 28 heads, 59 MB of partials > 32 MiB.
    rc = _noalloc(dev, dq, to_dev(tables), to_dev(ctx), None, 262144, 64, out)
    assert rc == INVALID_INPUT
    assert "scratch" in lib.it_last_error().decode()
    torch.cuda.synchronize()
    assert float(out.abs().sum()) == 0.0  # nothing ran
    with pytest.raises(InvalidInput):
        check(rc)


def test_noalloc_under_graph_capture():
    """A no-allocation decode captured in a HIP graph (the callers it is
    for): the array's address was looked up when the cache was made, so the
    captured call makes no runtime call that capture forbids.  Every replay,
    with eager no-allocation decodes of another batch between replays
    (which overwrite the shared array), equals the eager it_paged_decode
    bit for bit."""
    import torch
    from infer_train_amd._lib import OK

    hq, hkv, D, bs = 28, 4, 128, 16
    dev, tables, ctx, q = _cache(hq, hkv, D, bs, [300, 17, 1023, 512], seed=90)
    other, t2, c2, q2 = _cache(hq, hkv, D, bs, [2000, 64], seed=91)
    dq, dt, dc = to_dev(q.view(np.int16), torch.bfloat16), to_dev(tables), to_dev(ctx)
    dq2, dt2, dc2 = to_dev(q2.view(np.int16), torch.bfloat16), to_dev(t2), to_dev(c2)
    max_t = int(ctx.max())
    want = dev.decode(dq, dt, dc, None, max_t, partition=256, out_dtype=torch.float32)
    want2 = other.decode(dq2, dt2, dc2, None, 2000, partition=256, out_dtype=torch.float32)
    torch.cuda.synchronize()
    out_g = torch.empty_like(want)
    out2 = torch.empty_like(want2)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the capture, as torch asks
        assert _noalloc(dev, dq, dt, dc, None, max_t, 256, out_g) == OK
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert _noalloc(dev, dq, dt, dc, None, max_t, 256, out_g) == OK
    for i in range(3):
        out_g.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(from_dev(out_g), from_dev(want), err_msg=f"replay {i}")
        assert _noalloc(other, dq2, dt2, dc2, None, 2000, 256, out2) == OK
        torch.cuda.synchronize()
        np.testing.assert_array_equal(from_dev(out2), from_dev(want2), err_msg=f"eager call after replay {i}")
    dev.check()
