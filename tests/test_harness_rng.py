"""Pins of the reference-harness input generator (oracle/harness.py, C in
oracle.c) and of the prototxt case fixtures, on the CPU.

* minstd_rand0 (libstdc++ std::default_random_engine): the C++ standard's
  check value, the 10000th output of a default-seeded engine is 1043618065
  ([rand.predef]), and agreement with a pure-Python integer LCG.
* generate_canonical<double, 53>: the C result equals the libstdc++
  expression evaluated from those integers, and lies in [0, 1).
* Distributions: uniform moments; the polar normal's moments and symmetry.
* Chunking of large tensors (pb_tools.h:283-305) and the half conversion
  (7e-5 flush, round to nearest even).
"""
import json
import os

import numpy as np

from oracle import harness
from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
M = 2147483647


def py_minstd(seed, n):
    x = seed % M or 1
    out = []
    for _ in range(n):
        x = x * 16807 % M
        out.append(x)
    return out


def test_minstd_standard_check_value():
    assert harness.minstd_nth(1, 10000) == 1043618065


def test_minstd_matches_integer_lcg():
    for seed in (1, 42, 12345, M, 0, -3):
        ref = py_minstd(seed if seed >= 0 else (seed % (1 << 64)), 50)
        for n in (1, 2, 17, 50):
            assert harness.minstd_nth(seed, n) == ref[n - 1], (seed, n)


def test_canonical_is_the_libstdcxx_expression():
    R = 2147483646.0
    for seed in (42, 43, 100, 7):
        u = py_minstd(seed, 40)
        got = harness.uniform(seed, 20, 0.0, 1.0)
        for i in range(20):
            s = float(u[2 * i] - 1) * 1.0
            s += float(u[2 * i + 1] - 1) * R
            c = s / (R * R)
            assert 0.0 <= c < 1.0
            assert got[i] == c * (1.0 - 0.0) + 0.0, (seed, i)
        lo, hi = -1.0, 1.0
        g2 = harness.uniform(seed, 20, lo, hi)
        assert np.array_equal(g2, got * (hi - lo) + lo)


def test_distribution_moments():
    u = harness.uniform(5, 200000, -1.0, 1.0)
    assert u.min() >= -1.0 and u.max() < 1.0
    assert abs(u.mean()) < 0.01 and abs(u.var() - 1 / 3) < 0.01
    g = harness.normal(6, 200000, 0.0, 1.0)
    assert abs(g.mean()) < 0.01 and abs(g.var() - 1.0) < 0.02
    assert abs((g > 0).mean() - 0.5) < 0.01
    g2 = harness.normal(6, 1000, 3.0, 2.0)
    assert np.allclose(g2, harness.normal(6, 1000, 0.0, 1.0) * 2.0 + 3.0)
    f = harness.uniform_f32(7, 100000, np.float32(-1), np.float32(1))
    assert f.dtype == np.float32 and f.min() >= -1 and f.max() < 1 and abs(f.mean()) < 0.01


def test_half_conversion_and_chunking():
    v = np.array([6.9e-5, -6.9e-5, 7.0e-5, 1 / 3, 65504.0, 1.0 + 2 ** -11])
    h = harness.half_from_double(v)
    assert list(h[:2]) == [0, 0]
    assert h[2] != 0
    assert h[3] == np.float16(np.float32(1 / 3)).view(np.uint16)
    assert h[5] == np.float16(1.0).view(np.uint16)  # tie rounds to even
    # >= 32768 elements: 32 chunks of ceil(n/32), chunk i seeded with seed + i
    spec = {"distribution": "UNIFORM", "seed": 9, "lower_bound": -1.0, "upper_bound": 1.0}
    t = harness.random_tensor(spec, (40000,), "DTYPE_HALF")
    per = -(-40000 // 32)
    for i in (0, 1, 31):
        ref = harness.half_from_double(harness.uniform(9 + i, min(per, 40000 - i * per), -1.0, 1.0))
        assert np.array_equal(t[i * per:(i + 1) * per], ref)
    small = harness.random_tensor(spec, (100,), "DTYPE_HALF")
    assert np.array_equal(small, harness.half_from_double(harness.uniform(9, 100, -1.0, 1.0)))
    ints = harness.random_tensor({"distribution": "UNIFORM", "seed": 44, "lower_bound": -1.0,
                                  "upper_bound": 1024.0}, (512,), "DTYPE_INT64")
    assert ints.dtype == np.int64 and ints.min() >= 0 and ints.max() <= 1023
    const = harness.random_tensor({"distribution": "UNIFORM", "seed": 1, "lower_bound": 256,
                                   "upper_bound": 256}, (3,), "DTYPE_INT32")
    assert list(const) == [256, 256, 256]
    bf = harness.random_tensor(spec, (64,), "DTYPE_BFLOAT16")
    assert np.array_equal(bf, orc.from_float(harness.uniform_f32(9, 64, np.float32(-1),
                                                                 np.float32(1)), orc.BF16))


def test_prototxt_fixture_cases():
    with open(os.path.join(GOLDEN, "prototxt_cases.json")) as f:
        cases = json.load(f)
    assert {k: len(v) for k, v in cases.items()} == {
        "rms_norm": 8, "reshape_and_cache": 3, "flash_attention": 6, "causal_conv1d": 2,
        "memset": 2}
    for op, cs in cases.items():
        for c in cs:
            assert c["op_name"] == op
            for t in c["input"]:
                assert "prev_value" in t or "random_data" in t, (c["file"], t["id"])
    # a small input regenerates with the expected shape, dtype and range
    rms = cases["rms_norm"][0]
    w = harness.tensor(rms["input"][1])
    assert w.shape == (4096,) and w.dtype == np.uint16
    wf = orc.to_float(w)
    assert wf.min() >= -1.0 and wf.max() <= 1.0
