"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Every oracle function is compared with an independent formulation, a golden
vector, a closed form or an invariant, chosen so that a plausible mistake (a
dropped term, a wrong index, a transposed operand, an off-by-one mask) fails.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def bf16_bits(a):
    t = torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ conversions

def test_half_to_float_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    got = orc.to_float(bits, orc.HALF)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_rne():
    rng = np.random.default_rng(0)
    special = np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 1e-8, 2.0 ** -25,
                        2.0 ** -25 * 1.0000001, 2.0 ** -24, 3 * 2.0 ** -26, 6.0975552e-05,
                        np.inf, -np.inf, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 1e-40],
                       np.float32)
    # ties: every exact midpoint between adjacent halves must round to even
    h = np.arange(0, 0x7bff, dtype=np.uint16)
    mids = (h.view(np.float16).astype(np.float64) +
            (h + 1).view(np.float16).astype(np.float64)) / 2
    x = np.concatenate([special, rng.standard_normal(200000).astype(np.float32) * 300,
                        rng.standard_normal(20000).astype(np.float32) * 1e-5,
                        mids.astype(np.float32)])
    got = orc.from_float(x, orc.HALF)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_bfloat16_rne():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 1e3,
                        np.array([0, -0.0, 1.00390625, 1.01171875, 3.4e38, -np.inf], np.float32)])
    assert np.array_equal(orc.from_float(x, orc.BF16), bf16_bits(x))
    bits = np.arange(0, 65536, 7, dtype=np.uint16)
    back = orc.to_float(bits, orc.BF16)
    exp = (bits.astype(np.uint32) << 16).view(np.float32)
    same = np.isnan(exp) | (back.view(np.uint32) == exp.view(np.uint32))
    assert same.all()


# ------------------------------------------------------------ reshape_and_cache

def test_reshape_and_cache_doc_example():
    with open(os.path.join(GOLDEN, "reshape_and_cache_doc_example.json")) as f:
        ex = json.load(f)
    T, H, D = ex["num_tokens"], ex["num_kv_heads"], ex["head_size"]
    NB, BS = ex["num_blocks"], ex["block_size"]
    key = np.arange(T * H * D, dtype=np.uint16).reshape(T, H, D) + 1
    value = key + 1000
    kc = np.zeros((NB, H, BS, D), np.uint16)
    vc = np.zeros_like(kc)
    orc.reshape_and_cache(key, value, np.array(ex["slot_mapping"]), kc, vc)
    written = np.zeros((NB, BS), bool)
    for t, (blk, off) in enumerate(ex["expected_placement"]):
        for h in range(H):
            assert np.array_equal(kc[blk, h, off], key[t, h])
            assert np.array_equal(vc[blk, h, off], value[t, h])
        written[blk, off] = True
    assert not kc[~written.repeat(1, 0)[:, None, :].repeat(H, 1)].any()


def test_reshape_and_cache_vs_flash_layout_reference():
    """python_api_test/test_reshape_and_cache.py:36-47 writes the cache in the
    [blocks, block_size, heads, D] layout by slot index; the oracle's
    [blocks, heads, block_size, D] layout must agree after a permute."""
    rng = np.random.default_rng(2)
    T, H, D, NB, BS = 37, 3, 16, 8, 8
    key = rng.integers(0, 65535, (T, H, D), dtype=np.uint16)
    value = rng.integers(0, 65535, (T, H, D), dtype=np.uint16)
    slots = rng.permutation(NB * BS)[:T].astype(np.int64)
    slots[[3, 10]] = -1
    sentinel = np.uint16(0x7e00)
    kc = np.full((NB, H, BS, D), sentinel, np.uint16)
    vc = kc.copy()
    orc.reshape_and_cache(key, value, slots, kc, vc)
    flat_k = np.full((NB * BS, H, D), sentinel, np.uint16)
    flat_v = flat_k.copy()
    for i, s in enumerate(slots):
        if s == -1:
            continue
        flat_k[s] = key[i]
        flat_v[s] = value[i]
    assert np.array_equal(kc.transpose(0, 2, 1, 3).reshape(NB * BS, H, D), flat_k)
    assert np.array_equal(vc.transpose(0, 2, 1, 3).reshape(NB * BS, H, D), flat_v)


def test_reshape_and_cache_out_of_range_slot_skipped():
    key = np.ones((2, 1, 8), np.uint16)
    kc = np.zeros((1, 1, 2, 8), np.uint16)
    vc = kc.copy()
    orc.reshape_and_cache(key, key, np.array([2, 1]), kc, vc)
    assert kc[0, 0, 1].all() and not kc[0, 0, 0].any()


# --------------------------------------------------------------------- rms_norm

def test_rms_norm_constant_row_closed_form():
    eps = 1e-6
    c = np.float32(0.75)
    x = f16(np.full((3, 64), c))
    w = f16(np.ones(64))
    out, _ = orc.rms_norm(x, w, eps=eps)
    expect = np.float16(c / math.sqrt(c * c + eps))
    assert (out.view(np.float16) == expect).all()
    zero, _ = orc.rms_norm(f16(np.zeros((2, 32))), f16(np.ones(32)), eps=eps)
    assert not zero.any()


def test_rms_norm_matches_reference_python_formula():
    """python_api_test/test_rms_norm.py:31-43 in float64; fp16 output within 1 ulp."""
    rng = np.random.default_rng(3)
    for D, eps in [(128, 1e-6), (1536, 1e-5), (4096, 1e-6)]:
        x = f16(rng.standard_normal((16, D)))
        r = f16(rng.standard_normal((16, D)))
        w = f16(rng.uniform(0.5, 1.5, D))
        xf, rf, wf = (a.view(np.float16).astype(np.float64) for a in (x, r, w))
        out, _ = orc.rms_norm(x, w, eps=eps)
        ref = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + eps) * wf
        assert np.abs(out.view(np.float16).astype(np.float64) - ref).max() <= \
            np.abs(ref).max() * 2 ** -10
        out2, res_out = orc.rms_norm(x, w, residual=r, eps=eps)
        s = (xf.astype(np.float32) + rf.astype(np.float32))
        assert np.array_equal(res_out, f16(s))
        s64 = s.astype(np.float64)
        ref2 = res_out.view(np.float16).astype(np.float64) / np.sqrt(
            (s64 ** 2).mean(-1, keepdims=True) + eps) * wf
        assert np.abs(out2.view(np.float16).astype(np.float64) - ref2).max() <= \
            np.abs(ref2).max() * 2 ** -10


def test_rms_norm_power_of_two_scale_invariance():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 256)).astype(np.float16)
    w = f16(rng.uniform(0.5, 1.5, 256))
    a, _ = orc.rms_norm(x.view(np.uint16), w, eps=0.0)
    b, _ = orc.rms_norm((x * np.float16(4)).view(np.uint16), w, eps=0.0)
    assert np.array_equal(a, b)


def test_rms_norm_bf16():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    xb = bf16_bits(x)
    w = bf16_bits(np.ones(512))
    out, _ = orc.rms_norm(xb, w, eps=1e-6, dtype=orc.BF16)
    xf = orc.to_float(xb, orc.BF16).astype(np.float64)
    ref = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-6)
    assert np.abs(orc.to_float(out, orc.BF16) - ref).max() < 2 ** -7 * np.abs(ref).max()


# --------------------------------------------------------------- flash attention

def _paged(rng, kv_lens, H, Hkv, D, BS, dtype_bits, extra_blocks=3):
    nb_needed = sum(-(-s // BS) for s in kv_lens)
    NB = nb_needed + extra_blocks
    kc = dtype_bits(rng.standard_normal((NB, Hkv, BS, D)))
    vc = dtype_bits(rng.standard_normal((NB, Hkv, BS, D)))
    perm = rng.permutation(NB)
    cols = max(-(-s // BS) for s in kv_lens) + 1
    bt = np.full((len(kv_lens), cols), -7, np.int32)
    i = 0
    for b, s in enumerate(kv_lens):
        for j in range(-(-s // BS)):
            bt[b, j] = perm[i]
            i += 1
    return kc, vc, bt


def dense_attention_f64(q, kc, vc, bt, q_lens, kv_lens, scale, causal, dtype=orc.HALF):
    """Independent float64 formulation: gather the dense K/V per sequence,
    build the mask with the reference's `ones(S,S).tril().logical_not()[-L:]`
    (flash_attention.py:116-119) and apply softmax with GQA repeat_interleave."""
    to = lambda a: orc.to_float(a, dtype).astype(np.float64)
    qf, kf, vf = to(q), to(kc), to(vc)
    _, H, D = q.shape
    _, Hkv, BS, _ = kc.shape
    out = np.zeros(q.shape)
    off = 0
    for b, (L, S) in enumerate(zip(q_lens, kv_lens)):
        idx = np.arange(S)
        K = kf[bt[b, idx // BS], :, idx % BS]  # [S, Hkv, D]
        V = vf[bt[b, idx // BS], :, idx % BS]
        K = np.repeat(K, H // Hkv, axis=1)
        V = np.repeat(V, H // Hkv, axis=1)
        Q = qf[off:off + L]
        s = np.einsum("lhd,shd->hls", Q, K) * scale
        if causal:
            mask = ~np.tril(np.ones((S, S), bool))[-L:] if L <= S else \
                ~np.tril(np.ones((L, S), bool))
            s = np.where(mask[None], -np.inf, s)
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        out[off:off + L] = np.einsum("hls,shd->lhd", p, V)
        off += L
    return out


@pytest.mark.parametrize("case", [
    dict(H=4, Hkv=2, D=64, BS=16, q=[5, 1, 33], kv=[5, 40, 70], causal=True),
    dict(H=8, Hkv=8, D=32, BS=4, q=[9], kv=[9], causal=False),
    dict(H=6, Hkv=2, D=16, BS=7, q=[3, 12], kv=[20, 12], causal=True),
])
def test_flash_attention_vs_dense_f64(case):
    rng = np.random.default_rng(6)
    H, Hkv, D, BS = case["H"], case["Hkv"], case["D"], case["BS"]
    kc, vc, bt = _paged(rng, case["kv"], H, Hkv, D, BS, f16)
    q = f16(rng.standard_normal((sum(case["q"]), H, D)))
    scale = 1 / math.sqrt(D)
    got = orc.flash_attention(q, kc, vc, bt, case["q"], case["kv"], scale, case["causal"])
    ref = dense_attention_f64(q, kc, vc, bt, case["q"], case["kv"], scale, case["causal"])
    assert np.abs(got - ref).max() < 1e-5


def test_flash_attention_single_key_returns_v0():
    rng = np.random.default_rng(7)
    kc, vc, bt = _paged(rng, [1], 2, 1, 32, 4, f16)
    q = f16(rng.standard_normal((1, 2, 32)))
    got = orc.flash_attention(q, kc, vc, bt, [1], [1])
    v0 = orc.to_float(vc[bt[0, 0], 0, 0])
    assert np.allclose(got[0], v0[None], atol=0)


def test_flash_attention_constant_keys_average_values():
    rng = np.random.default_rng(8)
    S, BS, D = 24, 8, 16
    kc, vc, bt = _paged(rng, [S], 1, 1, D, BS, f16)
    kc[:] = f16(np.full(D, 0.5))
    q = f16(rng.standard_normal((S, 1, D)))
    got = orc.flash_attention(q, kc, vc, bt, [S], [S])
    idx = np.arange(S)
    V = orc.to_float(vc[bt[0, idx // BS], 0, idx % BS])
    expect = np.cumsum(V, 0) / np.arange(1, S + 1)[:, None]
    assert np.abs(got[:, 0] - expect).max() < 1e-5


def test_flash_attention_decode_is_last_prefill_row():
    rng = np.random.default_rng(9)
    S, H, Hkv, D, BS = 50, 4, 2, 32, 16
    kc, vc, bt = _paged(rng, [S], H, Hkv, D, BS, f16)
    q = f16(rng.standard_normal((S, H, D)))
    full = orc.flash_attention(q, kc, vc, bt, [S], [S])
    dec = orc.flash_attention(q[-1:], kc, vc, bt, [1], [S])
    assert np.abs(full[-1] - dec[0]).max() < 1e-6


def test_flash_attention_bf16_matches_dense():
    rng = np.random.default_rng(10)
    kc, vc, bt = _paged(rng, [40], 4, 1, 64, 16, bf16_bits)
    q = bf16_bits(rng.standard_normal((40, 4, 64)))
    got = orc.flash_attention(q, kc, vc, bt, [40], [40], dtype=orc.BF16)
    ref = dense_attention_f64(q, kc, vc, bt, [40], [40], 1 / 8, True, orc.BF16)
    assert np.abs(got - ref).max() < 1e-5


# ----------------------------------------------------------------- causal_conv1d

def silu(v):
    return v / (1 + np.exp(-v))


def test_conv1d_vs_numpy_convolve_bdl_with_bias():
    rng = np.random.default_rng(11)
    B, dim, L, W = 2, 5, 19, 4
    x = f16(rng.standard_normal((B, dim, L)))
    w = f16(rng.standard_normal((dim, W)) * 0.5)
    bias = f16(rng.standard_normal(dim))
    got = orc.causal_conv1d(x, w, bias=bias, layout="bdl")
    xf = x.view(np.float16).astype(np.float64)
    wf = w.view(np.float16).astype(np.float64)
    bf = bias.view(np.float16).astype(np.float64)
    for b in range(B):
        for d in range(dim):
            ref = np.convolve(xf[b, d], wf[d, ::-1])[:L] + bf[d]
            assert np.abs(got[b, d] - silu(ref)).max() < 1e-5


def test_conv1d_identity_tap_is_silu():
    rng = np.random.default_rng(12)
    x = f16(rng.standard_normal((32, 10)))  # [dim, total] reference torch layout
    w = np.zeros((4, 32), np.float32)
    w[3] = 1.0
    got = orc.causal_conv1d(x, f16(w), query_start_loc=np.array([0, 4, 10]), layout="dl")
    xf = x.view(np.float16).astype(np.float64)
    assert np.abs(got - silu(xf)).max() < 1e-6


def test_conv1d_state_carry_composes():
    """Running a sequence in two chunks with the state carried (has_init=1 on
    the second) equals running it whole; zero initial state == has_init 0."""
    rng = np.random.default_rng(13)
    dim, L, W = 8, 23, 4
    x = f16(rng.standard_normal((L, dim)))  # reference C API layout [tokens, dim]
    w = f16(rng.standard_normal((W, dim)))
    st_full = f16(rng.standard_normal((1, W - 1, dim)))
    st_zero = np.zeros_like(st_full)
    whole = orc.causal_conv1d(x, w, conv_state=st_full, query_start_loc=np.array([0, L]),
                              cache_indices=np.array([0]), has_initial_state=np.array([0]),
                              layout="ld")
    whole_z = orc.causal_conv1d(x, w, conv_state=st_zero, query_start_loc=np.array([0, L]),
                                cache_indices=np.array([0]), has_initial_state=np.array([1]),
                                layout="ld")
    assert np.array_equal(whole, whole_z)
    assert np.array_equal(st_full, st_zero) and np.array_equal(st_full[0], x[-3:])
    st = np.zeros((1, W - 1, dim), np.uint16)
    a = orc.causal_conv1d(x[:9], w, conv_state=st, query_start_loc=np.array([0, 9]),
                          has_initial_state=np.array([0]), layout="ld")
    b = orc.causal_conv1d(x[9:], w, conv_state=st, query_start_loc=np.array([0, L - 9]),
                          has_initial_state=np.array([1]), layout="ld")
    assert np.abs(np.concatenate([a, b]) - whole).max() == 0
    # short sequence: state shifts (len 1 < W-1)
    st2 = f16(np.arange(3 * dim).reshape(1, 3, dim))
    orc.causal_conv1d(x[:1], w, conv_state=st2, query_start_loc=np.array([0, 1]),
                      has_initial_state=np.array([1]), layout="ld")
    expect = np.concatenate([f16(np.arange(3 * dim).reshape(3, dim))[1:], x[:1]])
    assert np.array_equal(st2[0], expect)


def test_conv1d_pad_slot_skipped():
    rng = np.random.default_rng(14)
    x = f16(rng.standard_normal((4, 12)))
    w = f16(rng.standard_normal((4, 4)))
    st = f16(rng.standard_normal((3, 3, 4)))
    st0 = st.copy()
    out = orc.causal_conv1d(x, w, conv_state=st, query_start_loc=np.array([0, 6, 12]),
                            cache_indices=np.array([-1, 2]), has_initial_state=np.array([0, 1]),
                            pad_slot_id=-1, layout="dl")
    assert not out[:, :6].any()
    assert np.array_equal(st[:2], st0[:2]) and not np.array_equal(st[2], st0[2])


# ------------------------------------------------------------------------ rotary

def test_rotary_position_zero_identity_and_norm():
    rng = np.random.default_rng(15)
    T, H, D = 6, 3, 64
    q = f16(rng.standard_normal((T, H, D)))
    pos = np.array([0, 1, 7, 100, 2047, 5000])
    qo, _ = orc.rotary_embedding(pos, q, None)
    qf = q.view(np.float16).astype(np.float32)
    assert np.array_equal(qo[0], qf[0])
    n_in = qf[..., :32] ** 2 + qf[..., 32:] ** 2
    n_out = qo[..., :32] ** 2 + qo[..., 32:] ** 2
    assert np.abs(n_in - n_out).max() < 1e-4 * max(1.0, n_in.max())


def test_rotary_matches_complex_multiplication():
    rng = np.random.default_rng(16)
    T, H, Hk, D = 5, 2, 1, 32
    q = f16(rng.standard_normal((T, H, D)))
    k = f16(rng.standard_normal((T, Hk, D)))
    pos = rng.integers(0, 2048, T)
    qo, ko = orc.rotary_embedding(pos, q, k, base=10000.0)
    for src, got in ((q, qo), (k, ko)):
        xf = src.view(np.float16).astype(np.float64)
        i = np.arange(D // 2)
        theta = pos[:, None] * 10000.0 ** (-2 * i / D)
        z = (xf[..., :D // 2] + 1j * xf[..., D // 2:]) * np.exp(1j * theta)[:, None, :]
        assert np.abs(got[..., :D // 2] - z.real).max() < 1e-5
        assert np.abs(got[..., D // 2:] - z.imag).max() < 1e-5
    # GPT-J pairing equals NeoX on the de-interleaved vector
    qg, _ = orc.rotary_embedding(pos, q, None, is_neox=False)
    perm = np.concatenate([np.arange(0, D, 2), np.arange(1, D, 2)])
    qn, _ = orc.rotary_embedding(pos, q[..., perm], None, is_neox=True)
    assert np.abs(qg[..., perm] - qn).max() < 1e-6


def test_rotary_inverse_and_cache_equivalence():
    rng = np.random.default_rng(17)
    T, H, D = 4, 2, 16
    x = rng.standard_normal((T, H, D)).astype(np.float32)
    pos = np.array([3, 10, 77, 1999])
    maxpos = 2048
    i = np.arange(D // 2)
    th = np.arange(maxpos)[:, None] * 10000.0 ** (-2 * i / D)
    cache = np.concatenate([np.cos(th), np.sin(th)], 1).astype(np.float32)
    a, _ = orc.rotary_embedding(pos, f16(x), None)
    b, _ = orc.rotary_embedding(pos, f16(x), None, cos_sin_cache=cache)
    assert np.abs(a - b).max() < 1e-5
    neg = np.concatenate([np.cos(-th), np.sin(-th)], 1).astype(np.float32)
    back, _ = orc.rotary_embedding(pos, f16(a), None, cos_sin_cache=neg)
    assert np.abs(back - f16(x).view(np.float16)).max() < 3e-3


# -------------------------------------------------------------------------- GEMV

def test_gemv_vs_numpy_f64():
    rng = np.random.default_rng(18)
    W = f16(rng.standard_normal((70, 96)) * 0.02)
    x = f16(rng.standard_normal((3, 96)))
    got = orc.gemv(W, x)
    ref = x.view(np.float16).astype(np.float64) @ W.view(np.float16).astype(np.float64).T
    assert np.abs(got - ref).max() < 1e-6


def test_gemv_int8_exact_integers():
    rng = np.random.default_rng(19)
    W = rng.integers(-127, 128, (33, 64), dtype=np.int8)
    x = rng.integers(-4, 5, (2, 64)).astype(np.float16)
    s = f16(np.full(33, 0.5))
    got = orc.gemv_int8(W, s, x.view(np.uint16))
    ref = 0.5 * (x.astype(np.int64) @ W.astype(np.int64).T)
    assert np.array_equal(got, ref.astype(np.float32))
    s2 = f16(rng.uniform(0.001, 0.01, 33))
    got2 = orc.gemv_int8(W, s2, x.view(np.uint16))
    ref2 = s2.view(np.float16).astype(np.float64) * (x.astype(np.float64) @ W.astype(np.float64).T)
    assert np.abs(got2 - ref2).max() < 1e-6


def test_memset_truncates_to_byte():
    buf = np.zeros(37, np.uint8)
    orc.memset(buf, 0x1ab)
    assert (buf == 0xab).all()
