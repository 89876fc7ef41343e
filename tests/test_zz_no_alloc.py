"""tecoopsFlashAttentionNoAlloc, the allocation-free flash-attention entry
point for callers that cannot allocate device memory (its split-KV partials
live in a static device array), against tecoopsFlashAttentionEx on the same
inputs, through the C ABI.  Both launch the same kernels with the same plan,
so the outputs must be bit-identical.  Two calls in a row, the second with a
smaller batch, then a prefill call and a decode whose plan needs more than
the static array (rejected), and a decode captured into a graph and
replayed."""
import ctypes
import math

import numpy as np
import pytest
import torch

import tecoops
from tecoops import _lib

pytestmark = pytest.mark.gpu


def make(B, H, Hkv, D, BS, q_lens, kv_lens, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    nblk = [-(-s // BS) for s in kv_lens]
    tot = max(1, sum(nblk))
    perm = np.random.default_rng(seed).permutation(tot)
    bt = np.zeros((B, max(1, max(nblk))), np.int32)
    i = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[i:i + nblk[b]]
        i += nblk[b]
    q = torch.randn((sum(q_lens), H, D), generator=g, device="cuda").to(torch.bfloat16)
    kc = torch.randn((tot, Hkv, BS, D), generator=g, device="cuda").to(torch.bfloat16)
    vc = torch.randn((tot, Hkv, BS, D), generator=g, device="cuda").to(torch.bfloat16)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32, device="cuda")
    kl = torch.tensor(kv_lens, dtype=torch.int32, device="cuda")
    return q, kc, vc, torch.from_numpy(bt).cuda(), cu, kl


def call(entry, q, kc, vc, bt, cu, kl, max_q, max_k):
    out = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device="cuda")
    code = _lib.DATA_BFLOAT16
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    scale = ctypes.c_float(1.0 / math.sqrt(q.shape[2]))
    with tecoops._Desc(bt, _lib.DATA_INT32) as btd, tecoops._Desc(q, code) as qd, \
            tecoops._Desc(kc, code) as kd, tecoops._Desc(vc, code) as vd, \
            tecoops._Desc(out, code) as od:
        args = [tecoops._handle(q.device), max_q, max_k, None, p(cu), p(kl), btd, p(bt), qd, p(q),
                kd, p(kc), vd, p(vc), od, p(out), scale, 1]
        if entry == "tecoopsFlashAttentionEx":
            args.append(None)
        status = getattr(_lib.lib(), entry)(*args)
    torch.cuda.synchronize()
    return status, out


def same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_no_alloc_matches_ex_twice_then_smaller():
    rng = np.random.default_rng(5)
    big = make(64, 32, 8, 128, 16, [1] * 64, rng.integers(512, 8193, 64).tolist(), 1)
    small = make(8, 32, 8, 128, 16, [1, 2, 1, 1, 4, 1, 1, 1], rng.integers(1, 3000, 8).tolist(), 2)
    for name, (q, kc, vc, bt, cu, kl) in (("B=64", big), ("B=8", small)):
        mq, mk = int((cu[1:] - cu[:-1]).max()), int(kl.max())
        st_ex, ref = call("tecoopsFlashAttentionEx", q, kc, vc, bt, cu, kl, mq, mk)
        st_na, got = call("tecoopsFlashAttentionNoAlloc", q, kc, vc, bt, cu, kl, mq, mk)
        assert st_ex == _lib.SUCCESS and st_na == _lib.SUCCESS, (st_ex, st_na)
        assert not torch.isnan(got.float()).any(), name
        assert same(got, ref), f"{name}: NoAlloc differs from Ex"


def test_no_alloc_prefill_and_limit():
    q, kc, vc, bt, cu, kl = make(2, 16, 4, 128, 16, [300, 77], [300, 500], 3)
    st_ex, ref = call("tecoopsFlashAttentionEx", q, kc, vc, bt, cu, kl, 300, 500)
    st_na, got = call("tecoopsFlashAttentionNoAlloc", q, kc, vc, bt, cu, kl, 300, 500)
    assert st_ex == st_na == _lib.SUCCESS
    assert same(got, ref)
    # a decode plan past the static array (64 MiB): B = 512 sequences, 128 kv
    # heads, one query head each, kv_len bound 1M -> rejected before any launch
    B, H, D = 512, 128, 128
    q = torch.zeros((B, H, D), dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((1, H, 16, D), dtype=torch.bfloat16, device="cuda")
    bt = torch.zeros((B, 65536), dtype=torch.int32, device="cuda")
    cu = torch.arange(0, B + 1, dtype=torch.int32, device="cuda")
    kl = torch.ones((B,), dtype=torch.int32, device="cuda")
    st, _ = call("tecoopsFlashAttentionNoAlloc", q, kc, kc, bt, cu, kl, 1, 1 << 20)
    assert st == _lib.BAD_PARAM


def test_no_alloc_graph_capture_replays():
    """The entry point's use case: a split-KV decode captured into a graph on
    a torch stream after one eager call (the first call looks up the static
    array's device address and raises the kernels' LDS limit), then replayed
    twice with new q written in between; each replay is bit-identical to the
    Ex entry point run eagerly on the same inputs."""
    rng = np.random.default_rng(9)
    q, kc, vc, bt, cu, kl = make(16, 32, 8, 128, 16, [1] * 16, rng.integers(600, 6000, 16).tolist(), 4)
    mk = int(kl.max())
    out = torch.zeros(q.shape, dtype=torch.bfloat16, device="cuda")
    code = _lib.DATA_BFLOAT16
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    scale = ctypes.c_float(1.0 / math.sqrt(q.shape[2]))
    with tecoops._Desc(bt, _lib.DATA_INT32) as btd, tecoops._Desc(q, code) as qd, \
            tecoops._Desc(kc, code) as kd, tecoops._Desc(vc, code) as vd, \
            tecoops._Desc(out, code) as od:
        def enqueue():
            return _lib.lib().tecoopsFlashAttentionNoAlloc(
                tecoops._handle(q.device), 1, mk, None, p(cu), p(kl), btd, p(bt), qd, p(q), kd, p(kc),
                vd, p(vc), od, p(out), scale, 1)

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            assert enqueue() == _lib.SUCCESS
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        status = []
        with torch.cuda.graph(graph):
            status.append(enqueue())
        assert status == [_lib.SUCCESS]
        g = torch.Generator(device="cuda").manual_seed(17)
        prev = None
        for rep in range(2):
            q.copy_(torch.randn(q.shape, generator=g, device="cuda").to(torch.bfloat16))
            out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            st, ref = call("tecoopsFlashAttentionEx", q, kc, vc, bt, cu, kl, 1, mk)
            assert st == _lib.SUCCESS
            assert same(out, ref), f"replay {rep} differs from the Ex entry point"
            if prev is not None:
                assert not same(out, prev), "the second replay saw the new q"
            prev = out.clone()
