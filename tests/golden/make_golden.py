"""Writes the committed golden fixtures from the CPU oracle (never from
reference code: the reference is a Rust crate that cannot be built here and
ships no fixtures of its own).  Run from the repo root:
    python tests/golden/make_golden.py
Fixtures:
  config1_decode_out.npy  oracle flash_attn_f32 output of config 1 (12x128 f32)
  q8_cases.json           explicit Q8_0 inputs/records incl. .5 ties, NaN, inf
  q4_cases.json           explicit Q4_0 / Q4_1 inputs/records (ggml's quantisers,
                          which the reference does not carry): hand-worked
                          groups, equal magnitudes, -0, NaN, inf
  q5_cases.json           the same for Q5_0 / Q5_1, plus groups that use every
                          5-bit value and the clamp of Q5_0's +16 end
  manifest.json           seeds, shapes and SHA-256 digests of larger results
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as orc  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def config1():
    hq, hkv, D, bs = 12, 2, 128, 16
    k = orc.normal(101, 1024 * hkv * D).reshape(1024, hkv, D)
    v = orc.normal(102, 1024 * hkv * D).reshape(1024, hkv, D)
    q = orc.normal(103, hq * D).reshape(1, hq, D)
    c = orc.Cache(64, bs, hkv, D, orc.F32)
    c.append(k, v, np.arange(1024, dtype=np.int64))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    out = c.decode(q, hq, np.arange(64, dtype=np.int32)[None, :], np.array([1024], np.int32), None, scale)
    return out.reshape(hq, D), c


def q8_cases():
    cases = []
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:6] = [2.5, -2.5, 0.5, -0.5, 3.5]
    cases.append(("ties_scale_1", x))
    cases.append(("zeros", np.zeros(32, np.float32)))
    cases.append(("constant", np.full(32, 0.75, np.float32)))
    y = np.linspace(-1, 1, 32).astype(np.float32)
    y[3] = np.nan
    cases.append(("nan_ignored", y))
    z = y.copy()
    z[7] = np.inf
    cases.append(("inf", z))
    cases.append(("normal", orc.normal(44, 32)))
    cases.append(("tiny", orc.normal(45, 32) * np.float32(1e-30)))
    out = []
    for name, a in cases:
        rec = orc.quantize_row_q8_0(a)[0]
        out.append({"name": name, "x_bits": [int(u) for u in a.view(np.uint32)], "record": [int(b) for b in rec]})
    return out


def q4_cases():
    cases = []
    x = np.zeros(32, np.float32)
    vals = {0: 3.0, 1: -3.0, 2: 2.5, 3: -2.5, 4: 0.49, 5: 8.0, 6: 0.51, 7: 7.9, 8: -7.9, 20: -8.0, 21: 1.0}
    for i, v in vals.items():
        x[i] = v
    cases.append(("hand_d_minus_1", x))
    e = np.zeros(32, np.float32)
    e[[2, 7]] = [-4.0, 4.0]
    cases.append(("equal_magnitudes", e))
    cases.append(("zeros", np.zeros(32, np.float32)))
    cases.append(("neg_zeros", -np.zeros(32, np.float32)))
    m = np.zeros(32, np.float32)
    m[:16] = np.arange(16)
    m[16:24] = [7.4, 7.5, 7.6, 0.49, 0.5, 14.5, 14.51, 3.0]
    cases.append(("ramp", m))
    y = np.linspace(-1, 2, 32).astype(np.float32)
    y[5] = np.nan
    cases.append(("nan_ignored", y))
    z = y.copy()
    z[9] = -np.inf
    cases.append(("inf", z))
    cases.append(("normal", orc.normal(46, 32)))
    cases.append(("tiny", orc.normal(47, 32) * np.float32(1e-30)))
    out = []
    for name, a in cases:
        out.append({"name": name, "x_bits": [int(u) for u in a.view(np.uint32)],
                    "q4_0": [int(b) for b in orc.quantize_row_q4_0(a)[0]],
                    "q4_1": [int(b) for b in orc.quantize_row_q4_1(a)[0]]})
    return out


def q5_cases():
    cases = []
    x = np.zeros(32, np.float32)
    vals = {0: 3.0, 1: -3.0, 2: 2.5, 3: -2.5, 4: 0.49, 5: 16.0, 6: 0.51, 7: 15.9, 8: -15.9, 20: -16.0, 21: 1.0}
    for i, v in vals.items():
        x[i] = v
    cases.append(("hand_d_minus_1", x))
    e = np.zeros(32, np.float32)
    e[[2, 7]] = [-4.0, 4.0]
    cases.append(("equal_magnitudes", e))
    cases.append(("zeros", np.zeros(32, np.float32)))
    cases.append(("neg_zeros", -np.zeros(32, np.float32)))
    r = np.arange(32, dtype=np.float32)
    cases.append(("ramp_0_31", r))
    m = r.copy()
    m[16:24] = [7.4, 7.5, 7.6, 0.49, 0.5, 30.5, 30.51, 3.0]
    cases.append(("ramp_ties", m))
    y = np.linspace(-1, 2, 32).astype(np.float32)
    y[5] = np.nan
    cases.append(("nan_ignored", y))
    z = y.copy()
    z[9] = -np.inf
    cases.append(("inf", z))
    cases.append(("normal", orc.normal(48, 32)))
    cases.append(("tiny", orc.normal(49, 32) * np.float32(1e-30)))
    out = []
    for name, a in cases:
        out.append({"name": name, "x_bits": [int(u) for u in a.view(np.uint32)],
                    "q5_0": [int(b) for b in orc.quantize_row_q5_0(a)[0]],
                    "q5_1": [int(b) for b in orc.quantize_row_q5_1(a)[0]]})
    return out


def c4_log(n_steps=2768):
    cap, bs, W, start = 16512, 16, 4096, 30000
    pool = orc.Pool(cap, order=orc.permutation(4, cap))
    m = orc.Manager(pool, bs, 64, 32768 // bs + 1, W)
    first, last = (start - W) // bs, (start - 1) // bs
    for s in range(64):
        m.seed_seq(s, start, first, [pool.allocate() for _ in range(last - first + 1)])
    slots, evs = [], []
    for _ in range(n_steps):
        sl, ev = m.append(list(range(64)))
        slots.append(sl)
        evs.append(ev)
    return np.concatenate(slots), np.concatenate(evs), m.tables()[0]


def main():
    out, c = config1()
    np.save(os.path.join(HERE, "config1_decode_out.npy"), out)
    with open(os.path.join(HERE, "q8_cases.json"), "w") as f:
        json.dump(q8_cases(), f, indent=0)
    with open(os.path.join(HERE, "q4_cases.json"), "w") as f:
        json.dump(q4_cases(), f, indent=0)
    with open(os.path.join(HERE, "q5_cases.json"), "w") as f:
        json.dump(q5_cases(), f, indent=0)
    slots, evs, tables = c4_log()
    x = orc.normal(20, 32 * 4096)
    u = orc.uniform_i32(20 ^ 0x5A5A, 0, 99, x.size)
    x = np.where(u == 0, x * np.float32(8), x).astype(np.float32)
    manifest = {
        "config1": {"seeds": {"k": 101, "v": 102, "q": 103}, "k_pool_sha256": sha(c.k), "v_pool_sha256": sha(c.v),
                    "out_sha256": sha(out)},
        "config4_schedule": {"seed": 4, "capacity": 16512, "steps": 2768, "slots_sha256": sha(slots),
                             "evicted_sha256": sha(evs), "tables_sha256": sha(tables),
                             "first_evicted": [int(e) for e in evs[:64]], "first_slots": [int(s) for s in slots[:64]]},
        "q8_0_outliers": {"seed": 20, "n": int(x.size), "records_sha256": sha(orc.quantize_row_q8_0(x))},
        "q4_0_outliers": {"seed": 20, "n": int(x.size), "records_sha256": sha(orc.quantize_row_q4_0(x))},
        "q4_1_outliers": {"seed": 20, "n": int(x.size), "records_sha256": sha(orc.quantize_row_q4_1(x))},
        "q5_0_outliers": {"seed": 20, "n": int(x.size), "records_sha256": sha(orc.quantize_row_q5_0(x))},
        "q5_1_outliers": {"seed": 20, "n": int(x.size), "records_sha256": sha(orc.quantize_row_q5_1(x))},
    }
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)


if __name__ == "__main__":
    main()
