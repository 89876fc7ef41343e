"""Shared helpers for the GPU parity tests: numpy <-> torch transfers of
16-bit bit patterns and the tolerance checks of the north star
(fp16/bf16 ops within 1e-2 abs/rel of the fp32 oracle)."""
import json
import os

import numpy as np
import torch

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

TORCH_DT = {orc.HALF: torch.float16, orc.BF16: torch.bfloat16}


def reference_cases():
    with open(os.path.join(GOLDEN, "reference_cases.json")) as f:
        return json.load(f)


def bits(rng_values, dtype=orc.HALF):
    """float array -> uint16 bit patterns of the 16-bit type (RNE)."""
    return orc.from_float(np.asarray(rng_values, np.float32), dtype)


def dev(a, dtype=None):
    """numpy -> cuda tensor; uint16 arrays become float16/bfloat16 views."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).cuda()
        return t.view(TORCH_DT[dtype or orc.HALF])
    return torch.from_numpy(a).cuda()


def host_bits(t):
    """16-bit cuda tensor -> numpy uint16 bit patterns."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def as_f32(t, dtype=orc.HALF):
    return orc.to_float(host_bits(t), dtype)


def assert_close(got, ref, atol=1e-2, rtol=1e-2, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {err.size} elements out of tolerance; "
                             f"worst at {i}: got {got[i]} ref {ref[i]} (max abs err {err.max():.3e})")
    return err.max()


def diff3_max(got, ref):
    """Reference harness criterion DIFF3_MAX (evaluator.h:62-63): max |d|/(|b|)
    where |b| >= 1e-4, else |d|.  Reported, not asserted."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    d = np.abs(got - ref)
    rel = np.where(np.abs(ref) < 1e-4, d, d / np.maximum(np.abs(ref), 1e-30))
    return float(rel.max()) if rel.size else 0.0


def record(line):
    """Prints a parity figure now and lists it again in the run's summary."""
    import conftest
    print(line, flush=True)
    conftest.FIGURES.append(line)
