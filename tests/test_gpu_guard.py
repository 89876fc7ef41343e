"""Out-of-bounds writes and run-to-run stability of every op, the MI355X
counterparts of the reference harness's checks: its stability hash (the same
output over repeated runs, test/src/suite/executor.cpp:313-366) and its
whole-memory out-of-bounds check after each case (executor.cpp:590-603).

Every output (and in-place operand) lives in a buffer with GUARD bytes of
sentinel on each side; after each run the bands must be untouched.  Each op
runs twice from identical inputs and the two outputs must be bit-identical.
Shapes: the BASELINE.json configs and ragged edge shapes.
"""
import math

import numpy as np
import pytest
import torch

import tecoops

pytestmark = pytest.mark.gpu

GUARD = 4096
SENTINEL = 0xA5


class Guarded:
    """A tensor of `shape` / `dtype` in the middle of a byte buffer with GUARD
    sentinel bytes on each side (the data stays 16-byte aligned)."""

    def __init__(self, shape, dtype, init=None):
        n = int(np.prod(shape)) * torch.empty((), dtype=dtype).element_size()
        self.n = n
        self.buf = torch.full((n + 2 * GUARD,), SENTINEL, dtype=torch.uint8, device="cuda")
        self.t = self.buf[GUARD:GUARD + n].view(dtype).view(shape)
        if init is not None:
            self.t.copy_(init)

    def check_bands(self, what):
        torch.cuda.synchronize()
        lo = self.buf[:GUARD]
        hi = self.buf[GUARD + self.n:]
        assert bool((lo == SENTINEL).all()), f"{what}: write before the buffer"
        assert bool((hi == SENTINEL).all()), f"{what}: write past the buffer"


def bitwise(t):
    return t.contiguous().view(torch.uint8).clone()


def randn(shape, dtype=torch.float16, scale=1.0, seed=0):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda") * scale).to(dtype)


def twice(make_outputs, run, what):
    """Runs `run(outputs)` on two fresh sets of guarded outputs; checks the
    guard bands after each run and that both runs wrote the same bits."""
    results = []
    for rep in range(2):
        outs = make_outputs()
        run([o.t for o in outs])
        for i, o in enumerate(outs):
            o.check_bands(f"{what} output {i} run {rep}")
        results.append([bitwise(o.t) for o in outs])
    for i, (a, b) in enumerate(zip(*results)):
        assert torch.equal(a, b), f"{what}: output {i} differs between two runs"


@pytest.mark.parametrize("shape", [(4096, 4096), (37, 5000), (3, 8)])
@pytest.mark.parametrize("fused", [False, True])
def test_rms_norm(shape, fused):
    x = randn(shape, seed=1)
    w = randn((shape[1],), scale=0.5, seed=2) + 1
    r = randn(shape, seed=3) if fused else None

    def outs():
        o = [Guarded(shape, torch.float16)]
        if fused:
            o.append(Guarded(shape, torch.float16))
        return o

    twice(outs, lambda o: tecoops.rms_norm(x, w, r, o[0], o[1] if fused else None, 1e-6),
          f"rms_norm {shape} fused={fused}")


@pytest.mark.parametrize("T,NB,BS", [(8192, 1024, 16), (77, 13, 7)])
def test_reshape_and_cache(T, NB, BS):
    Hkv, D = 8, 128
    key, val = randn((T, Hkv, D), seed=4), randn((T, Hkv, D), seed=5)
    # distinct slots (a seeded permutation) plus a skipped negative slot
    slots = torch.randperm(NB * BS, generator=torch.Generator().manual_seed(6))[:T]
    slots[T // 2] = -1
    slots = slots.to(torch.int64).cuda()
    outs = lambda: [Guarded((NB, Hkv, BS, D), torch.float16, torch.zeros((NB, Hkv, BS, D),
                                                                       dtype=torch.float16)),
                    Guarded((NB, Hkv, BS, D), torch.float16, torch.zeros((NB, Hkv, BS, D),
                                                                       dtype=torch.float16))]
    twice(outs, lambda o: tecoops.reshape_and_cache(key, val, slots, o[0], o[1]),
          f"reshape_and_cache T={T}")


@pytest.mark.parametrize("B,C,L", [(8, 4096, 2048), (3, 40, 37)])
def test_causal_conv1d(B, C, L):
    x = randn((B, C, L), seed=7)
    w = randn((C, 4), scale=0.5, seed=8)
    bias = randn((C,), seed=9)
    outs = lambda: [Guarded((B, C, L), torch.float16),
                    Guarded((B, 3, C), torch.float16, torch.zeros((B, 3, C), dtype=torch.float16))]
    twice(outs, lambda o: tecoops.causal_conv1d(x, w, bias, o[0], conv_states=o[1]),
          f"causal_conv1d {B}x{C}x{L}")


@pytest.mark.parametrize("T,H,Hkv", [(8192, 32, 8), (19, 5, 3)])
def test_causal_conv1d_token_major(T, H, Hkv):
    """The reference layout [totalSeqLen, dim] through causal_conv1d_fn_torch."""
    dim = H * 64
    qsl = torch.tensor([0, T // 3, T], dtype=torch.int32, device="cuda")
    x = randn((dim, T), seed=10)     # [dim, tokens] view of token-major storage
    w = randn((4, dim), scale=0.5, seed=11)
    cache_idx = torch.tensor([1, 0], dtype=torch.int32, device="cuda")
    has_init = torch.tensor([1, 0], dtype=torch.int8, device="cuda")
    init_state = randn((2, 3, dim), seed=12)
    outs = lambda: [Guarded((T, dim), torch.float16), Guarded((2, 3, dim), torch.float16,
                                                              init_state)]
    twice(outs, lambda o: tecoops.causal_conv1d_fn_torch(o[0].t(), o[1], x.t().contiguous().t(),
                                                         w, qsl, cache_idx, has_init, -1),
          f"causal_conv1d token-major T={T}")


@pytest.mark.parametrize("T,H,Hkv", [(8192, 32, 8), (13, 3, 1)])
def test_rotary(T, H, Hkv):
    D = 128
    q0, k0 = randn((T, H, D), seed=13), randn((T, Hkv, D), seed=14)
    pos = (torch.arange(T, device="cuda") % 2048).to(torch.int64)
    outs = lambda: [Guarded((T, H, D), torch.float16, q0), Guarded((T, Hkv, D), torch.float16, k0)]
    twice(outs, lambda o: tecoops.rotary_embedding(pos, o[0], o[1], D), f"rotary T={T}")


@pytest.mark.parametrize("T,NB", [(8192, 1024), (21, 4)])
def test_rotary_reshape_and_cache(T, NB):
    H, Hkv, D, BS = 32, 8, 128, 16
    q0, k0, v = randn((T, H, D), seed=15), randn((T, Hkv, D), seed=16), randn((T, Hkv, D), seed=17)
    pos = (torch.arange(T, device="cuda") % 2048).to(torch.int64)
    slots = torch.randperm(NB * BS, generator=torch.Generator().manual_seed(18))[:T]
    slots = slots.to(torch.int64).cuda()
    z = torch.zeros((NB, Hkv, BS, D), dtype=torch.float16)
    outs = lambda: [Guarded((T, H, D), torch.float16, q0), Guarded((T, Hkv, D), torch.float16, k0),
                    Guarded((NB, Hkv, BS, D), torch.float16, z),
                    Guarded((NB, Hkv, BS, D), torch.float16, z)]
    twice(outs, lambda o: tecoops.rotary_reshape_and_cache(pos, o[0], o[1], v, slots, o[2], o[3],
                                                           D, write_key=True),
          f"rotary_reshape_and_cache T={T}")


@pytest.mark.parametrize("N,K", [(14336, 4096), (77, 1000), (5, 256)])
@pytest.mark.parametrize("B", [1, 8, 3])
def test_gemv(N, K, B):
    W = randn((N, K), scale=0.02, seed=19)
    x = randn((B, K), seed=20)
    twice(lambda: [Guarded((B, N), torch.float16)], lambda o: tecoops.gemv(W, x, o[0]),
          f"gemv {N}x{K} B={B}")


@pytest.mark.parametrize("N,K", [(14336, 4096), (77, 1000), (5, 256)])
@pytest.mark.parametrize("B", [1, 8, 3])
def test_gemv_int8(N, K, B):
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    Wq = torch.randint(-127, 128, (N, K), generator=g, device="cuda", dtype=torch.int8)
    sc = (torch.rand((N,), generator=g, device="cuda") * 0.009 + 0.001).half()
    x = randn((B, K), seed=22)
    twice(lambda: [Guarded((B, N), torch.float16)], lambda o: tecoops.gemv_int8(Wq, sc, x, o[0]),
          f"gemv_int8 {N}x{K} B={B}")


def fa_inputs(B, H, Hkv, D, BS, q_lens, kv_lens, seed):
    nblk = [-(-s // BS) for s in kv_lens]
    tot = sum(nblk)
    perm = torch.randperm(tot, generator=torch.Generator().manual_seed(seed))
    bt = torch.zeros((B, max(nblk)), dtype=torch.int32)
    i = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[i:i + nblk[b]]
        i += nblk[b]
    q = randn((sum(q_lens), H, D), torch.bfloat16, seed=seed + 1)
    kc = randn((tot, Hkv, BS, D), torch.bfloat16, seed=seed + 2)
    vc = randn((tot, Hkv, BS, D), torch.bfloat16, seed=seed + 3)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32, device="cuda")
    kl = torch.tensor(kv_lens, dtype=torch.int32, device="cuda")
    return q, kc, vc, bt.cuda(), cu, kl


@pytest.mark.parametrize("kind", ["prefill_baseline", "decode_baseline", "mixed_edge"])
def test_flash_attention(kind):
    if kind == "prefill_baseline":
        B, H, Hkv, D, BS = 4, 32, 8, 128, 16
        q_lens, kv_lens = [4096] * 4, [4096] * 4
    elif kind == "decode_baseline":
        B, H, Hkv, D, BS = 64, 32, 8, 128, 16
        q_lens = [1] * 64
        kv_lens = np.random.default_rng(1008).integers(512, 8193, 64).tolist()
    else:
        B, H, Hkv, D, BS = 3, 12, 4, 96, 5
        q_lens, kv_lens = [1, 77, 5], [300, 77, 9]
    q, kc, vc, bt, cu, kl = fa_inputs(B, H, Hkv, D, BS, q_lens, kv_lens, seed=23)
    twice(lambda: [Guarded(q.shape, torch.bfloat16)],
          lambda o: tecoops.flash_attn_varlen_func(q, kc, vc, max(q_lens), cu, max(kv_lens), None,
                                                   kl, 1.0 / math.sqrt(D), True, None, bt, False,
                                                   o[0]),
          f"flash_attention {kind}")


@pytest.mark.parametrize("n", [1, 15, 4096 + 3, 1 << 24])
def test_memset(n):
    twice(lambda: [Guarded((n,), torch.uint8)], lambda o: tecoops.memset(o[0], 0x3C),
          f"memset {n}")
