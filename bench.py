"""Benchmark of the MI355X KV-cache hot path.

Headline workload (BASELINE.json metric, config 2 at its 4k target): batched
paged decode, bf16, Hq 28 / Hkv 4 / D 128, block size 16, batch 32 with every
sequence at 4096 tokens after the step's append, pages scattered by a seeded
permutation of a 16384-block pool, split-K over 512-token partitions.  One
step = slot-mapped append of 1 token per sequence + split-K decode + combine.

value = KV bytes read per step / median(split + combine time), the
algorithmic bytes sum_b ctx_b * Hkv * 2 * D * 2.  Three pool replicas are
rotated so the 256 MB last-level cache does not hold the previous step's
pages (cold); warm numbers (one replica) are reported beside it.  Timing uses
HIP events on the stream the kernels run on.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--all]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, AMD-published
MFMA_BF16_PEAK_TFS = 2500.0  # dense bf16


def _events(n):
    import torch

    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


class DecodeWorkload:
    """A paged decode batch with `replicas` copies of the pools."""

    def __init__(self, dtype, hq, hkv, D, bs, ctx, pool_blocks, partition, seed, replicas=3, q_dtype=None):
        import torch

        import infer_train_amd as it
        from infer_train_amd.kv import PagedKvCache

        self.torch = torch
        self.hq, self.hkv, self.D, self.bs, self.partition = hq, hkv, D, bs, partition
        self.dtype = dtype
        self.ctx = np.asarray(ctx, np.int32)
        B = self.ctx.size
        self.B = B
        rng = np.random.default_rng(seed)
        perm = rng.permutation(pool_blocks).astype(np.int32)
        self.max_blocks = int((self.ctx.max() + bs - 1) // bs)
        t = np.full((B, self.max_blocks), -1, np.int32)
        k = 0
        for b, c in enumerate(self.ctx):
            nb = (int(c) + bs - 1) // bs
            t[b, :nb] = perm[k:k + nb]
            k += nb
        assert k <= pool_blocks, "pool too small"
        dev = torch.device("cuda", 0)
        self.tables = torch.from_numpy(t).to(dev)
        self.ctx_d = torch.from_numpy(self.ctx).to(dev)
        # The step appends the token at position ctx-1 of each sequence.
        slots = np.array([int(t[b, (c - 1) // bs]) * bs + (c - 1) % bs for b, c in enumerate(self.ctx)], np.int64)
        self.slots = torch.from_numpy(slots).to(dev)
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.caches = []
        for _ in range(replicas):
            c = PagedKvCache(pool_blocks, bs, hkv, D, dtype)
            if dtype == it.Q8_0:
                # Fill through the quantising append so pages hold valid Q8_0.
                n_rows = pool_blocks * bs
                step = 1 << 16
                for s0 in range(0, n_rows, step):
                    n = min(step, n_rows - s0)
                    kk = torch.randn((n, hkv, D), generator=g, device=dev)
                    kk[torch.rand((n, hkv, D), generator=g, device=dev) < 0.01] *= 8
                    vv = torch.randn((n, hkv, D), generator=g, device=dev)
                    c.append(kk, vv, torch.arange(s0, s0 + n, device=dev, dtype=torch.int64))
            else:
                td = {it.BF16: torch.bfloat16, it.F16: torch.float16, it.F32: torch.float32}[dtype]
                c.view("k").copy_(torch.randn(c.view("k").shape, generator=g, device=dev).to(td))
                c.view("v").copy_(torch.randn(c.view("v").shape, generator=g, device=dev).to(td))
            self.caches.append(c)
        qd = q_dtype if q_dtype is not None else ({it.Q8_0: torch.float32, it.F32: torch.float32,
                                                   it.BF16: torch.bfloat16, it.F16: torch.float16}[dtype])
        self.q = torch.randn((B, hq, D), generator=g, device=dev).to(qd)
        src_t = torch.float32 if dtype in (it.Q8_0, it.F32) else qd
        self.k_new = torch.randn((B, hkv, D), generator=g, device=dev).to(src_t)
        self.v_new = torch.randn((B, hkv, D), generator=g, device=dev).to(src_t)
        self.out = torch.empty((B, hq, D), dtype=qd, device=dev)
        self.max_tokens = int(self.ctx.max())
        self.ws = self.caches[0].decode_workspace(B, hq, self.max_tokens, partition)
        self.scale = 1.0 / math.sqrt(D)
        elem = {it.BF16: 2.0, it.F16: 2.0, it.F32: 4.0, it.Q8_0: 34.0 / 32.0}[dtype]
        self.kv_bytes = float(self.ctx.astype(np.int64).sum()) * hkv * 2 * D * elem
        src_elem = 4.0 if dtype in (it.Q8_0, it.F32) else 2.0
        self.append_bytes = B * hkv * 2 * D * (src_elem + elem)

    def step(self, i, ev=None):
        """append -> split -> combine; events (if given) bracket each kernel."""
        c = self.caches[i % len(self.caches)]
        if ev is not None:
            ev[0].record()
        c.append(self.k_new, self.v_new, self.slots)
        if ev is not None:
            ev[1].record()
        for j, phase in enumerate(("split", "combine")):
            c.decode(self.q, self.tables, self.ctx_d, None, self.max_tokens, scale=self.scale,
                     partition=self.partition, out=self.out, ws=self.ws, phase=phase)
            if ev is not None:
                ev[2 + j].record()

    def time(self, steps, warmup, rotate=True):
        """Per-kernel times (ms) over `steps` event-bracketed steps: medians of
        append and split+combine, mean of split alone, and wall ms per step."""
        torch = self.torch
        n_rep = len(self.caches) if rotate else 1
        for i in range(warmup):
            self.step(i % n_rep)
        torch.cuda.synchronize()
        evs = [_events(4) for _ in range(steps)]
        t0 = time.perf_counter()
        for i in range(steps):
            self.step(i % n_rep, evs[i])
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        app = np.array([e[0].elapsed_time(e[1]) for e in evs])
        split = np.array([e[1].elapsed_time(e[2]) for e in evs])
        dec = np.array([e[1].elapsed_time(e[3]) for e in evs])
        for c in self.caches:
            c.check()
        return {"append": float(np.median(app)), "decode": float(np.median(dec)), "split_mean": float(split.mean()),
                "split_median": float(np.median(split)), "step_wall": wall * 1e3 / steps}


def cpu_baseline_c2(n_seqs_total, ctx, hq=28, hkv=4, D=128, bs=16, budget_s=10.0):
    """The oracle (scalar C restatement of flash_attn_f32 + the GQA driver) on
    a bounded sample of the headline workload, on this host, 1 thread."""
    import oracle as orc

    B = 4
    nb = B * ((ctx + bs - 1) // bs)
    c = orc.Cache(nb, bs, hkv, D, orc.BF16)
    bits = orc.f32_to_bf16(orc.normal(1, c.k.size // 2))
    c.k[:] = np.frombuffer(bits.tobytes(), np.uint8)
    c.v[:] = np.frombuffer(orc.f32_to_bf16(orc.normal(2, c.v.size // 2)).tobytes(), np.uint8)
    t = np.arange(nb, dtype=np.int32).reshape(B, -1)
    cl = np.full(B, ctx, np.int32)
    q = orc.bf16_to_f32(orc.f32_to_bf16(orc.normal(3, B * hq * D)))
    done, t0 = 0, time.perf_counter()
    while True:
        c.decode(q, hq, t, cl, None, 1.0 / math.sqrt(D))
        done += B
        el = time.perf_counter() - t0
        if el >= budget_s or done >= 8 * n_seqs_total:
            break
    gbs = done * ctx * hkv * 2 * D * 2 / el / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle decode of {done} sequences x ctx {ctx} (Hq {hq}/Hkv {hkv}/D {D} bf16 widened to f32) "
                      f"in {el:.1f} s; full step = {n_seqs_total} sequences"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--all", action="store_true", help="also measure configs 1, 3, 4 and 5")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-probe", action="store_true",
                    help="first run 4 device copies of 256 MiB (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus > 1 is not supported (each GPU would own "
                                   "its sequences' pages and run the same kernels with no exchange)"}))
        sys.exit(2)
    import torch

    import infer_train_amd as it

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_probe:
        # A plain copy of known size: 256 MiB read + 256 MiB written per
        # dispatch.  Its counter readings give the KiB-per-byte factor used to
        # turn the decode kernel's FETCH_SIZE/WRITE_SIZE into HBM bytes.
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    # Headline: config 2 at the 4k target.
    w = DecodeWorkload(it.BF16, 28, 4, 128, 16, np.full(32, 4096), 16384, 512, seed=2)
    cold = w.time(args.steps, args.warmup, rotate=True)
    warm = w.time(args.steps, args.warmup, rotate=False)
    app_ms, dec_ms, step_ms = cold["append"], cold["decode"], cold["step_wall"]
    gbs = w.kv_bytes / (dec_ms * 1e-3) / 1e9
    gbs_warm = w.kv_bytes / (warm["decode"] * 1e-3) / 1e9
    split_gbs = w.kv_bytes / (cold["split_mean"] * 1e-3) / 1e9
    append_mtok = w.B / (app_ms * 1e-3) / 1e6
    kv_bytes = w.kv_bytes
    del w
    torch.cuda.empty_cache()
    # Config 2 as specified: ragged contexts U[256, 4096] (+1 appended).
    rng = np.random.default_rng(22)
    ctx2 = rng.integers(256, 4097, 32) + 1
    w2 = DecodeWorkload(it.BF16, 28, 4, 128, 16, ctx2, 16384, 512, seed=3)
    r2 = w2.time(args.steps, args.warmup, rotate=True)
    ragged = {"kv_gbs": round(w2.kv_bytes / (r2["decode"] * 1e-3) / 1e9, 1), "decode_us": round(r2["decode"] * 1e3, 2),
              "kv_bytes": int(w2.kv_bytes), "append_us": round(r2["append"] * 1e3, 2),
              "pct_hbm_peak": round(100 * w2.kv_bytes / (r2["decode"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)}
    del w2
    torch.cuda.empty_cache()
    line = {
        "metric": "paged flash-decode KV-read GB/s (% of HBM peak) + KV append Mtok/s",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) bf16 K/V/Q, seeded; pages a seeded permutation of the pool",
        "config": {"workload": "config 2 at its 4k target: batched paged decode, Hq 28 / Hkv 4 / D 128, block 16, "
                               "batch 32, ctx 4096 each (4095 cached + 1 appended), 16384-block pool, "
                               "split-K 512-token partitions + combine",
                   "global_batch": 32, "seq_len": 4096, "parallelism": "none (1 GPU)"},
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "decode_us": round(dec_ms * 1e3, 2),
        "split_us_mean": round(cold["split_mean"] * 1e3, 2),
        "kv_bytes_per_step": int(kv_bytes),
        "warm_kv_gbs": round(gbs_warm, 1),
        "append_mtok_s": round(append_mtok, 3),
        "append_us": round(app_ms * 1e3, 2),
        "config2_ragged": ragged,
        "roofline": {"bound": "hbm", "achieved": round(split_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(split_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "paged_decode_split<bf16,128,7> (mean of its HIP-event durations)",
                     "algorithmic_bytes_per_launch": int(kv_bytes)},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_c2(32, 4096)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
