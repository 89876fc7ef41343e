"""Inputs of the reference's C++ op tests, regenerated bit for bit.

TEST INFRASTRUCTURE ONLY (like the rest of oracle/): used by
tests/test_prototxt_replay.py to rebuild the tensors a reference test case
(tests/golden/prototxt_cases.json) describes, as the reference harness does:

  * random_data, float types: generateRandomData (test/src/case/pb_tools.h:
    283-305) splits tensors of >= 32 * 1024 elements into 32 chunks of
    ceil(count / 32), chunk i seeded with seed + i, each drawn serially by
    generateRandomDataSerial (pb_tools.h:123-200): UNIFORM values
    a + (b - a) * canonical, GAUSSIAN values from normal_distribution; for
    half tensors |v| < 7e-5 becomes 0 and the double is stored through
    half_float::half::operator=(float) (double -> float -> half, both round to
    nearest even; half.hpp 2.2.0 with HALF_ROUND_STYLE 1); lower >= upper
    gives every element `upper`.
  * bf16 tensors: generateRandomDataSerialBf16 (pb_tools.cpp:854-900) draws
    uniform_real_distribution<float> and rounds float -> bf16 to nearest even.
  * integer tensors: the same double draws converted by C++ truncation.
  * prev_value: the fixed value_i / value_f / value_l list.

The draws themselves come from the C oracle (orc_harness_*).
"""
import ctypes

import numpy as np

from . import oracle as orc

CHUNKS = 32
SERIAL_LIMIT = 1024 * CHUNKS

_NP = {"DTYPE_HALF": np.uint16, "DTYPE_BFLOAT16": np.uint16, "DTYPE_FLOAT": np.float32,
       "DTYPE_DOUBLE": np.float64, "DTYPE_INT8": np.int8, "DTYPE_INT16": np.int16,
       "DTYPE_INT32": np.int32, "DTYPE_INT64": np.int64, "DTYPE_UINT8": np.uint8}


def _declare():
    L = orc.lib()
    if getattr(L, "_harness_declared", False):
        return L
    P, ll, sz = ctypes.c_void_p, ctypes.c_longlong, ctypes.c_size_t
    L.orc_minstd_nth.argtypes = [ll, sz]
    L.orc_minstd_nth.restype = ctypes.c_uint32
    L.orc_harness_uniform.argtypes = [ll, sz, ctypes.c_double, ctypes.c_double, P]
    L.orc_harness_normal.argtypes = [ll, sz, ctypes.c_double, ctypes.c_double, P]
    L.orc_harness_uniform_f32.argtypes = [ll, sz, ctypes.c_float, ctypes.c_float, P]
    L._harness_declared = True
    return L


def minstd_nth(seed, n):
    return _declare().orc_minstd_nth(seed, n)


def uniform(seed, n, lo, hi):
    out = np.empty(n, np.float64)
    _declare().orc_harness_uniform(seed, n, lo, hi, out.ctypes.data_as(ctypes.c_void_p))
    return out


def normal(seed, n, mu, sigma):
    out = np.empty(n, np.float64)
    _declare().orc_harness_normal(seed, n, mu, sigma, out.ctypes.data_as(ctypes.c_void_p))
    return out


def uniform_f32(seed, n, lo, hi):
    out = np.empty(n, np.float32)
    _declare().orc_harness_uniform_f32(seed, n, lo, hi, out.ctypes.data_as(ctypes.c_void_p))
    return out


def half_from_double(v):
    """half_float::half = double: flush |v| < 7e-5, then double -> float -> half."""
    v = np.where(np.abs(v) < 7e-5, 0.0, v)
    return v.astype(np.float32).astype(np.float16).view(np.uint16)


def _chunks(count):
    if count < SERIAL_LIMIT:
        return [(0, count, 0)]
    per = -(-count // CHUNKS)
    return [(i * per, min(count, (i + 1) * per), i) for i in range(CHUNKS) if i * per < count]


def _convert(v, dtype):
    if dtype == "DTYPE_HALF":
        return half_from_double(v)
    if dtype in ("DTYPE_FLOAT", "DTYPE_DOUBLE"):
        return v.astype(_NP[dtype])
    return np.trunc(v).astype(_NP[dtype])


def random_tensor(spec, shape, dtype):
    """Tensor of `shape` from a random_data spec, as the reference harness fills it."""
    count = int(np.prod(shape)) if len(shape) else 1
    dist = spec.get("distribution", "UNIFORM")
    seed = int(spec.get("seed", 0))
    lo, hi = float(spec.get("lower_bound", 0.0)), float(spec.get("upper_bound", 0.0))
    out = np.empty(count, _NP[dtype])
    for start, end, i in _chunks(count):
        n = end - start
        if dtype == "DTYPE_BFLOAT16":
            if dist != "UNIFORM":
                raise NotImplementedError("bf16 harness inputs: only UNIFORM is used by the cases")
            vals = (np.full(n, hi, np.float32) if lo >= hi else
                    uniform_f32(seed + i, n, np.float32(lo), np.float32(hi)))
            out[start:end] = orc.from_float(vals, orc.BF16)
            continue
        if dist == "UNIFORM":
            v = np.full(n, hi) if lo >= hi else uniform(seed + i, n, lo, hi)
        elif dist == "GAUSSIAN":
            v = normal(seed + i, n, float(spec.get("mu", 0.0)), float(spec.get("sigma", 1.0)))
        else:
            raise NotImplementedError(f"distribution {dist}")
        if spec.get("positive"):
            v = np.abs(v)
        if spec.get("negative"):
            v = -np.abs(v)
        out[start:end] = _convert(v, dtype)
    return out.reshape(shape)


def tensor(t):
    """numpy array for one input / output entry of a parsed case."""
    shape = tuple(t["shape"]["dims"]) if "shape" in t else ()
    dtype = t["dtype"]
    if "prev_value" in t:
        pv = t["prev_value"]
        vals = pv.get("value_i", pv.get("value_l", pv.get("value_f")))
        return np.asarray(vals, _NP[dtype] if dtype not in ("DTYPE_HALF", "DTYPE_BFLOAT16")
                          else np.float32).reshape(shape)
    if "random_data" in t:
        return random_tensor(t["random_data"], shape, dtype)
    raise ValueError(f"tensor {t.get('id')} has no data recipe")
