"""GPU parity of the bandwidth-bound ops against the CPU oracle.

Each test calls libtecoops.so through the C ABI (tecoops package) on cuda:0
with seeded inputs and compares with oracle/oracle.c on the same inputs:
bit-exact for reshape_and_cache and memset, within 1e-2 abs/rel for the
fp16/bf16 ops, 1e-2 relative for the int8 GEMV.  Shapes: the reference's own
test cases (tests/golden/reference_cases.json), edge cases, and the full
BASELINE.json configs.
"""
import numpy as np
import pytest
import torch

import tecoops
from oracle import oracle as orc

from helpers import as_f32, assert_close, bits, dev, host_bits, reference_cases

pytestmark = pytest.mark.gpu

CASES = reference_cases()


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------- reshape_and_cache

def _run_reshape(T, H, D, NB, BS, seed, dtype=orc.HALF, neg=0, collisions_free=True,
                 out_of_range=0):
    r = rng(seed)
    key = bits(r.standard_normal((T, H, D)), dtype)
    value = bits(r.standard_normal((T, H, D)), dtype)
    slots = r.permutation(NB * BS)[:T].astype(np.int64)
    if neg:
        slots[r.choice(T, neg, replace=False)] = -1
    if out_of_range:
        slots[r.choice(T, out_of_range, replace=False)] = NB * BS + 5
    sentinel = bits(np.full((NB, H, BS, D), 3.5), dtype)
    kc_ref, vc_ref = sentinel.copy(), sentinel.copy()
    orc.reshape_and_cache(key, value, slots, kc_ref, vc_ref)
    kc, vc = dev(sentinel, dtype), dev(sentinel, dtype)
    tecoops.reshape_and_cache(dev(key, dtype), dev(value, dtype), dev(slots), kc, vc)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(kc), kc_ref)
    assert np.array_equal(host_bits(vc), vc_ref)


@pytest.mark.parametrize("case", CASES["reshape_and_cache"], ids=lambda c: f"kv{c['kv_heads']}")
def test_reshape_and_cache_reference_cases(case):
    _run_reshape(case["tokens"], case["kv_heads"], case["head"], case["num_blocks"],
                 case["block_size"], seed=42, neg=7)


@pytest.mark.parametrize("D", [6, 7, 64])
def test_reshape_and_cache_narrow_heads_and_bf16(D):
    _run_reshape(100, 3, D, 20, 8, seed=D, dtype=orc.BF16, neg=3, out_of_range=2)


def test_reshape_and_cache_baseline_config():
    """BASELINE config: 8192 tokens x 8 kv heads x 128, 1024 blocks x 16,
    slot_mapping a seeded permutation of distinct slots in [0, 16384)."""
    _run_reshape(8192, 8, 128, 1024, 16, seed=1234)


# ---------------------------------------------------------------------- rms_norm

def _run_rms(N, D, eps, residual, seed, dtype=orc.HALF):
    r = rng(seed)
    x = bits(r.uniform(-1, 1, (N, D)), dtype)
    w = bits(r.uniform(0.5, 1.5, D), dtype)
    res = bits(r.uniform(-1, 1, (N, D)), dtype) if residual else None
    ref, ref_res = orc.rms_norm(x, w, residual=res, eps=eps, dtype=dtype)
    tdt = torch.float16 if dtype == orc.HALF else torch.bfloat16
    out = torch.empty((N, D), dtype=tdt, device="cuda")
    res_out = torch.empty((N, D), dtype=tdt, device="cuda") if residual else None
    tecoops.rms_norm(dev(x, dtype), dev(w, dtype), dev(res, dtype) if residual else None, out,
                     res_out, eps)
    torch.cuda.synchronize()
    assert_close(as_f32(out, dtype), orc.to_float(ref, dtype), what="rms_norm out")
    if residual:
        assert np.array_equal(host_bits(res_out), ref_res)


@pytest.mark.parametrize("case", CASES["rms_norm"],
                         ids=lambda c: f"{c['hidden']}-{'add' if c['residual'] else 'pure'}")
def test_rms_norm_reference_cases(case):
    _run_rms(case["tokens"], case["hidden"], case["eps"], case["residual"], seed=42)


@pytest.mark.parametrize("D", [100, 8, 24576, 20000])
def test_rms_norm_odd_and_wide_rows(D):
    _run_rms(5, D, 1e-5, residual=True, seed=D)
    _run_rms(5, D, 1e-5, residual=False, seed=D + 1)


def test_rms_norm_bf16():
    _run_rms(33, 2048, 1e-6, residual=True, seed=7, dtype=orc.BF16)


def test_rms_norm_baseline_config():
    """BASELINE config: x fp16 [4096, 4096] ~N(0,1), w ~U(0.5,1.5), eps 1e-6."""
    r = rng(2024)
    x = bits(r.standard_normal((4096, 4096)))
    w = bits(r.uniform(0.5, 1.5, 4096))
    ref, _ = orc.rms_norm(x, w, eps=1e-6)
    out = torch.empty((4096, 4096), dtype=torch.float16, device="cuda")
    tecoops.rms_norm(dev(x), dev(w), None, out, None, 1e-6)
    torch.cuda.synchronize()
    got = host_bits(out)
    assert_close(orc.to_float(got), orc.to_float(ref), what="rms_norm 4096^2")
    # fp32 sums in a different order: at most 1 ulp of fp16 from the oracle
    ulp = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert ulp.max() <= 1


# ------------------------------------------------------------------------ rotary

def _run_rotary(T, H, Hkv, D, seed, is_neox=True, use_cache=False, dtype=orc.HALF,
                rot_dim=None, maxpos=2048):
    r = rng(seed)
    q = bits(r.standard_normal((T, H, D)), dtype)
    k = bits(r.standard_normal((T, Hkv, D)), dtype)
    pos = (np.arange(T) % maxpos).astype(np.int64)
    r.shuffle(pos)
    rd = rot_dim or D
    cache = None
    if use_cache:
        i = np.arange(rd // 2)
        th = np.arange(maxpos)[:, None] * 10000.0 ** (-2 * i / rd)
        cache = np.concatenate([np.cos(th), np.sin(th)], 1).astype(np.float32)
    qo, ko = orc.rotary_embedding(pos, q, k, rot_dim=rd, is_neox=is_neox, cos_sin_cache=cache,
                                  dtype=dtype)
    qt, kt = dev(q, dtype), dev(k, dtype)
    tecoops.rotary_embedding(dev(pos), qt, kt, D, dev(cache) if use_cache else None,
                             is_neox=is_neox, rot_dim=rd)
    torch.cuda.synchronize()
    assert_close(as_f32(qt, dtype), qo, what="rotary q")
    assert_close(as_f32(kt, dtype), ko, what="rotary k")


@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("use_cache", [False, True])
def test_rotary_variants(is_neox, use_cache):
    _run_rotary(300, 4, 2, 128, seed=5, is_neox=is_neox, use_cache=use_cache)


def test_rotary_wide_heads_tails_and_skips():
    """NeoX 16-byte path: 72 heads x 16 tasks per token (rot_dim 256) make
    several task rounds per thread (1152 tasks over the 256 threads of a
    token's workgroup, 2 in flight at a time); an odd token count (303);
    with the cos/sin cache, positions past it are left unrotated; without a
    key only q rotates; rot_dim < head_size leaves the tail untouched."""
    r = rng(31)
    T, H, Hkv, D = 303, 64, 8, 256
    q = bits(r.standard_normal((T, H, D)))
    k = bits(r.standard_normal((T, Hkv, D)))
    pos = r.integers(0, 1100, T).astype(np.int64)
    i = np.arange(D // 2)
    th = np.arange(1000)[:, None] * 10000.0 ** (-2 * i / D)
    cache = np.concatenate([np.cos(th), np.sin(th)], 1).astype(np.float32)
    qo, ko = orc.rotary_embedding(pos, q, k, cos_sin_cache=cache)
    qt, kt = dev(q), dev(k)
    tecoops.rotary_embedding(dev(pos), qt, kt, D, dev(cache))
    torch.cuda.synchronize()
    assert_close(as_f32(qt), qo, what="rotary q, cache")
    assert_close(as_f32(kt), ko, what="rotary k, cache")
    skipped = pos >= 1000
    assert skipped.any() and np.array_equal(host_bits(qt)[skipped], q[skipped])
    # no key, rot_dim 64 of head_size 128
    q2 = bits(r.standard_normal((T, 8, 128)))
    pos2 = (np.arange(T) % 2048).astype(np.int64)
    qo2, _ = orc.rotary_embedding(pos2, q2, None, rot_dim=64)
    qt2 = dev(q2)
    tecoops.rotary_embedding(dev(pos2), qt2, None, 128, rot_dim=64)
    torch.cuda.synchronize()
    assert_close(as_f32(qt2), qo2, what="rotary q only, rot_dim 64")
    assert np.array_equal(host_bits(qt2)[:, :, 64:], q2[:, :, 64:])


def test_rotary_partial_rot_dim_bf16_and_scalar_path():
    _run_rotary(64, 3, 1, 64, seed=6, rot_dim=32, dtype=orc.BF16)
    _run_rotary(64, 3, 1, 20, seed=7, rot_dim=10)   # rot/2 = 5: scalar path


def _run_rotary_cache(T, H, Hkv, D, NB, BS, seed, is_neox=True, use_cache=False,
                      dtype=orc.HALF, rot_dim=None, write_key=False, maxpos=2048,
                      oob_positions=False):
    """Fused decode step against (a) rotary_embedding then reshape_and_cache on
    the GPU (bit-exact: same arithmetic) and (b) the oracle (q and cached k
    within tolerance, cached v bit-exact)."""
    r = rng(seed)
    q = bits(r.standard_normal((T, H, D)), dtype)
    k = bits(r.standard_normal((T, Hkv, D)), dtype)
    v = bits(r.standard_normal((T, Hkv, D)), dtype)
    pos = (np.arange(T) % maxpos).astype(np.int64)
    r.shuffle(pos)
    if oob_positions:
        pos[::5] = maxpos + 3        # past the cos/sin cache: cached unrotated
    slots = r.permutation(NB * BS)[:T].astype(np.int64)
    slots[::7] = -1                  # skipped
    slots[3::11] = NB * BS + 5       # past the cache: skipped
    rd = rot_dim or D
    cache = None
    if use_cache:
        i = np.arange(rd // 2)
        th = np.arange(maxpos)[:, None] * 10000.0 ** (-2 * i / rd)
        cache = np.concatenate([np.cos(th), np.sin(th)], 1).astype(np.float32)
    sentinel = bits(np.full((NB, Hkv, BS, D), 7.0), dtype)
    # (a) two-kernel path on the GPU
    q2, k2 = dev(q, dtype), dev(k, dtype)
    kc2, vc2 = dev(sentinel, dtype), dev(sentinel, dtype)
    tecoops.rotary_embedding(dev(pos), q2, k2, D, dev(cache) if use_cache else None,
                             is_neox=is_neox, rot_dim=rd)
    tecoops.reshape_and_cache(k2, dev(v, dtype), dev(slots), kc2, vc2)
    # fused
    q1, k1 = dev(q, dtype), dev(k, dtype)
    kc1, vc1 = dev(sentinel, dtype), dev(sentinel, dtype)
    tecoops.rotary_reshape_and_cache(dev(pos), q1, k1, dev(v, dtype), dev(slots), kc1, vc1, D,
                                     dev(cache) if use_cache else None, is_neox=is_neox,
                                     rot_dim=rd, write_key=write_key)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(q1), host_bits(q2)), "query differs from the two-kernel path"
    assert np.array_equal(host_bits(kc1), host_bits(kc2)), "key cache differs"
    assert np.array_equal(host_bits(vc1), host_bits(vc2)), "value cache differs"
    if write_key:
        assert np.array_equal(host_bits(k1), host_bits(k2)), "key differs"
    else:
        assert np.array_equal(host_bits(k1), k), "key changed without write_key"
    # (b) oracle
    qo, ko = orc.rotary_embedding(pos, q, k, rot_dim=rd, is_neox=is_neox, cos_sin_cache=cache,
                                  dtype=dtype)
    assert_close(as_f32(q1, dtype), qo, what="fused q")
    kc_ref, vc_ref = sentinel.copy(), sentinel.copy()
    orc.reshape_and_cache(np.zeros_like(k), v, slots, kc_ref, vc_ref)
    assert np.array_equal(host_bits(vc1), vc_ref), "value cache vs oracle"
    got_k = as_f32(kc1, dtype)
    ok = (slots >= 0) & (slots < NB * BS)
    for t in np.nonzero(ok)[0]:
        blk, off = divmod(int(slots[t]), BS)
        assert_close(got_k[blk, :, off, :], ko[t], what=f"cached k token {t}")
    free = np.ones(NB * BS, bool)
    free[slots[ok]] = False
    untouched = got_k.transpose(0, 2, 1, 3).reshape(NB * BS, Hkv, D)[free]
    assert (untouched == 7.0).all(), "slots outside slot_mapping were written"


@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("use_cache", [False, True])
def test_rotary_reshape_and_cache_variants(is_neox, use_cache):
    _run_rotary_cache(300, 4, 2, 128, 40, 16, seed=21, is_neox=is_neox, use_cache=use_cache)


def test_rotary_reshape_and_cache_partial_bf16_scalar_write_key():
    _run_rotary_cache(64, 3, 1, 64, 12, 8, seed=22, rot_dim=32, dtype=orc.BF16, write_key=True)
    _run_rotary_cache(50, 3, 2, 20, 10, 5, seed=23, rot_dim=10, write_key=True)  # scalar path


@pytest.mark.parametrize("write_key", [True, False])
def test_rotary_reshape_and_cache_batched_edges(write_key):
    """NeoX 16-byte fused path with rot_dim = head_size (each thread loads a
    batch of tasks before storing): 301 tokens leave a partial last
    workgroup, every fifth position lies past the cos/sin cache, and skipped
    slots mix with cached ones in every batch."""
    _run_rotary_cache(301, 8, 2, 128, 60, 16, seed=26 + write_key, use_cache=True,
                      write_key=write_key, oob_positions=True)


def test_rotary_reshape_and_cache_baseline_shape():
    """q [8192, 32, 128], k/v [8192, 8, 128] into 1024 blocks x 16 (the BASELINE
    rotary and reshape_and_cache configs, as one decode-step op)."""
    _run_rotary_cache(8192, 32, 8, 128, 1024, 16, seed=24)


def test_rotary_baseline_config():
    """BASELINE config: q [8192, 32, 128], k [8192, 8, 128], positions 0..2047
    per sequence, base 10000, neox."""
    r = rng(99)
    T = 8192
    q = bits(r.standard_normal((T, 32, 128)))
    k = bits(r.standard_normal((T, 8, 128)))
    pos = (np.arange(T) % 2048).astype(np.int64)
    qo, ko = orc.rotary_embedding(pos, q, k)
    qt, kt = dev(q), dev(k)
    tecoops.rotary_embedding(dev(pos), qt, kt, 128)
    torch.cuda.synchronize()
    assert_close(as_f32(qt), qo, what="rotary q")
    assert_close(as_f32(kt), ko, what="rotary k")


# ------------------------------------------------------------------ causal_conv1d

@pytest.mark.parametrize("ci", range(len(CASES["causal_conv1d"])))
def test_causal_conv1d_reference_cases(ci):
    """Reference torch layout: x/out [dim, tokens], weight [width, dim]
    (python_api_test/test_causal_conv1d.py:108-147)."""
    c = CASES["causal_conv1d"][ci]
    r = rng(100 + ci)
    dim, lens = c["dim"], c["seq_lens"]
    total = sum(lens)
    x = bits(r.standard_normal((dim, total)))
    w = bits(r.standard_normal((4, dim)))
    st = bits(r.standard_normal((c["num_entries"], 3, dim)))
    qsl = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cidx = np.array(c["cache_indices"], np.int32)
    hinit = np.array(c["has_init"], np.int8)
    st_ref = st.copy()
    ref = orc.causal_conv1d(x, w, conv_state=st_ref, query_start_loc=qsl, cache_indices=cidx,
                            has_initial_state=hinit, pad_slot_id=c["pad_slot_id"], layout="dl")
    out = torch.zeros((dim, total), dtype=torch.float16, device="cuda")
    st_dev = dev(st)
    tecoops.causal_conv1d_fn_torch(out, st_dev, dev(x), dev(w), dev(qsl), dev(cidx), dev(hinit),
                                   c["pad_slot_id"])
    torch.cuda.synchronize()
    assert_close(as_f32(out), ref, what="conv out")
    assert np.array_equal(host_bits(st_dev), st_ref)


def test_causal_conv1d_c_api_token_major():
    """tecoopsCausalConv1d with the reference C layout [tokens, dim], api_mode 1
    and width 3 / 2 (state of width-1 rows)."""
    import ctypes
    from tecoops import _lib
    for W in (4, 3, 2):
        r = rng(200 + W)
        dim, lens = 96, [5, 1, 2, 40]
        total = sum(lens)
        x = bits(r.standard_normal((total, dim)))
        w = bits(r.standard_normal((W, dim)))
        st = bits(r.standard_normal((len(lens), W - 1, dim)))
        qsl = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        st_ref = st.copy()
        ref = orc.causal_conv1d(x, w, conv_state=st_ref, query_start_loc=qsl, api_mode=1,
                                layout="ld")
        xd, wd, sd, qd = dev(x), dev(w), dev(st), dev(qsl)
        out = torch.zeros((total, dim), dtype=torch.float16, device="cuda")
        h = ctypes.c_void_p()
        _lib.call("tecoopsCreate", ctypes.byref(h))
        _lib.call("tecoopsSetStream", h, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        _lib.call("tecoopsCausalConv1d", h, len(lens), total, dim, W, (W - 1) * dim, dim, dim,
                  -1, 1, 0, ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(sd.data_ptr()),
                  ctypes.c_void_p(wd.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                  ctypes.c_void_p(qd.data_ptr()), None, None)
        torch.cuda.synchronize()
        _lib.call("tecoopsDestroy", h)
        assert_close(as_f32(out), ref, what=f"conv width {W}")
        assert np.array_equal(host_bits(sd), st_ref)


@pytest.mark.parametrize("W", [4, 3, 2])
@pytest.mark.parametrize("L", [5000, 4999, 2051, 513])
def test_causal_conv1d_long_rows(W, L):
    """Token-contiguous rows longer than one group of loads (4 x 512 tokens),
    so the last inputs of a group carry into the next; partial segments at
    the end; L = 4999 / 2051 / 513 leave most rows misaligned for 16-byte
    access; sequences 0 and 2 start from their conv state."""
    r = rng(800 + 10 * W + L % 97)
    B, dim = 3, 40
    x = bits(r.standard_normal((B, dim, L)))
    w = bits(r.normal(0, 0.5, (dim, W)))
    bias = bits(r.standard_normal(dim))
    st = bits(r.standard_normal((B, W - 1, dim)))
    hinit = np.array([1, 0, 1], np.int8)
    st_ref = st.copy()
    ref = orc.causal_conv1d(x, w, bias=bias, conv_state=st_ref, has_initial_state=hinit,
                            layout="bdl")
    out = torch.empty((B, dim, L), dtype=torch.float16, device="cuda")
    st_dev = dev(st)
    tecoops.causal_conv1d(dev(x), dev(w), dev(bias), out, conv_states=st_dev,
                          has_initial_state=dev(hinit))
    torch.cuda.synchronize()
    assert_close(as_f32(out), ref, what=f"conv W={W} L={L}")
    assert np.array_equal(host_bits(st_dev), st_ref)


def test_causal_conv1d_reference_layout_long_varlen():
    """Reference torch layout [dim, tokens] with sequences of 3000, 7 and 2100
    tokens (cache slots 2, 0, 1; slot 0 starts from zeros)."""
    r = rng(900)
    dim, lens = 24, [3000, 7, 2100]
    total = sum(lens)
    x = bits(r.standard_normal((dim, total)))
    w = bits(r.standard_normal((4, dim)))
    st = bits(r.standard_normal((3, 3, dim)))
    qsl = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cidx = np.array([2, 0, 1], np.int32)
    hinit = np.array([1, 0, 1], np.int8)
    st_ref = st.copy()
    ref = orc.causal_conv1d(x, w, conv_state=st_ref, query_start_loc=qsl, cache_indices=cidx,
                            has_initial_state=hinit, layout="dl")
    out = torch.zeros((dim, total), dtype=torch.float16, device="cuda")
    st_dev = dev(st)
    tecoops.causal_conv1d_fn_torch(out, st_dev, dev(x), dev(w), dev(qsl), dev(cidx), dev(hinit),
                                   -1)
    torch.cuda.synchronize()
    assert_close(as_f32(out), ref, what="conv [dim, tokens] long varlen")
    assert np.array_equal(host_bits(st_dev), st_ref)


@pytest.mark.parametrize("W", [2, 3, 4])
@pytest.mark.parametrize("case", ["decode", "short_varlen"])
def test_causal_conv1d_short_sequences(W, case):
    """Reference torch layout [dim, tokens] with short sequences (mean <= 32
    tokens: the per-(sequence, channel) kernel): a decode step of 70
    sequences of one token, and a chunked mix of 1..40 tokens; shuffled cache
    slots, sequences without initial state and one pad slot (its output and
    state untouched).  Output and state against the oracle; the state is
    bit-exact."""
    r = rng(950 + W + (0 if case == "decode" else 10))
    dim = 200
    lens = [1] * 70 if case == "decode" else r.integers(1, 41, 37).tolist()
    B, total = len(lens), sum(lens)
    x = bits(r.standard_normal((dim, total)))
    w = bits(r.standard_normal((W, dim)))
    st = bits(r.standard_normal((B + 3, W - 1, dim)))
    qsl = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cidx = r.permutation(B + 3)[:B].astype(np.int32)
    cidx[5] = -7  # pad slot
    hinit = (r.random(B) < 0.7).astype(np.int8)
    st_ref = st.copy()
    ref = orc.causal_conv1d(x, w, conv_state=st_ref, query_start_loc=qsl, cache_indices=cidx,
                            has_initial_state=hinit, pad_slot_id=-7, layout="dl")
    out = torch.zeros((dim, total), dtype=torch.float16, device="cuda")
    st_dev = dev(st)
    tecoops.causal_conv1d_fn_torch(out, st_dev, dev(x), dev(w), dev(qsl), dev(cidx), dev(hinit),
                                   -7)
    torch.cuda.synchronize()
    assert_close(as_f32(out), ref, what=f"conv short {case} W={W}")
    assert np.array_equal(host_bits(st_dev), st_ref)


@pytest.mark.parametrize("W", [2, 3, 4])
@pytest.mark.parametrize("lo,hi", [(8, 40), (20, 110), (60, 200), (100, 420)])
def test_causal_conv1d_grouped_rows_varlen(W, lo, hi):
    """Reference torch layout [dim, tokens] with sequences of lo..hi tokens
    (mean 13..256: several rows per wave, 4 to 32 lanes each, rows of one
    wave of different lengths and mostly misaligned), shuffled cache slots,
    sequences without initial state and one pad slot."""
    r = rng(980 + W + lo)
    dim = 72
    lens = r.integers(lo, hi + 1, 23).tolist()
    B, total = len(lens), sum(lens)
    x = bits(r.standard_normal((dim, total)))
    w = bits(r.standard_normal((W, dim)))
    st = bits(r.standard_normal((B + 2, W - 1, dim)))
    qsl = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cidx = r.permutation(B + 2)[:B].astype(np.int32)
    cidx[3] = -7
    hinit = (r.random(B) < 0.7).astype(np.int8)
    st_ref = st.copy()
    ref = orc.causal_conv1d(x, w, conv_state=st_ref, query_start_loc=qsl, cache_indices=cidx,
                            has_initial_state=hinit, pad_slot_id=-7, layout="dl")
    out = torch.zeros((dim, total), dtype=torch.float16, device="cuda")
    st_dev = dev(st)
    tecoops.causal_conv1d_fn_torch(out, st_dev, dev(x), dev(w), dev(qsl), dev(cidx), dev(hinit),
                                   -7)
    torch.cuda.synchronize()
    assert_close(as_f32(out), ref, what=f"conv grouped rows {lo}..{hi} W={W}")
    assert np.array_equal(host_bits(st_dev), st_ref)


@pytest.mark.parametrize("L", [13, 24, 40, 64, 100, 200, 256])
def test_causal_conv1d_grouped_rows_bdl(L):
    """[B, dim, L] with 13..256 tokens per row, bias and SiLU, no state."""
    r = rng(990 + L)
    xb = bits(r.standard_normal((9, 50, L)))
    wb = bits(r.standard_normal((50, 4)))
    bb = bits(r.standard_normal(50))
    ob = torch.empty((9, 50, L), dtype=torch.float16, device="cuda")
    tecoops.causal_conv1d(dev(xb), dev(wb), dev(bb), ob)
    torch.cuda.synchronize()
    assert_close(as_f32(ob), orc.causal_conv1d(xb, wb, bias=bb, layout="bdl"), what=f"conv bdl L={L}")


def test_causal_conv1d_short_rows_bdl():
    """[B, dim, L] with L = 16 (the per-(sequence, channel) kernel), bias and
    SiLU, no state."""
    r = rng(970)
    xb = bits(r.standard_normal((40, 96, 16)))
    wb = bits(r.standard_normal((96, 4)))
    bb = bits(r.standard_normal(96))
    ob = torch.empty((40, 96, 16), dtype=torch.float16, device="cuda")
    tecoops.causal_conv1d(dev(xb), dev(wb), dev(bb), ob)
    torch.cuda.synchronize()
    assert_close(as_f32(ob), orc.causal_conv1d(xb, wb, bias=bb, layout="bdl"), what="conv bdl L=16")


def _conv_c_api(x, w, st, qsl, cidx, hinit, pad, api_mode, W):
    """tecoopsCausalConv1d on token-major x [tokens, dim] (the reference C
    layout); returns out and the updated state as numpy bits."""
    import ctypes
    from tecoops import _lib
    total, dim = x.shape
    xd, wd, sd, qd = dev(x), dev(w), dev(st), dev(qsl)
    cd = dev(cidx) if cidx is not None else None
    hd = dev(hinit) if hinit is not None else None
    out = torch.full((total, dim), float("nan"), dtype=torch.float16, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None
    _lib.call("tecoopsCausalConv1d", tecoops._handle(xd.device), len(qsl) - 1, total, dim, W,
              (W - 1) * dim, dim, dim, pad, api_mode, 0, p(xd), p(sd), p(wd), p(out), p(qd),
              p(cd), p(hd))
    torch.cuda.synchronize()
    return host_bits(out), host_bits(sd)


def test_causal_conv1d_token_major_baseline_shape():
    """The BASELINE conv shape in the reference C layout: x [8 x 2048 tokens,
    4096] token-major through tecoopsCausalConv1d, weight [4, 4096], no
    initial state, final state written (16-byte channel vectors)."""
    r = rng(78)
    dim, lens = 4096, [2048] * 8
    total = sum(lens)
    x = bits(r.standard_normal((total, dim), dtype=np.float32))
    w = bits(r.normal(0, 0.5, (4, dim)).astype(np.float32))
    st = bits(r.standard_normal((8, 3, dim), dtype=np.float32))
    qsl = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    hinit = np.zeros(8, np.int8)
    st_ref = st.copy()
    ref = orc.causal_conv1d(x, w, conv_state=st_ref, query_start_loc=qsl,
                            has_initial_state=hinit, layout="ld")
    out, st_got = _conv_c_api(x, w, st, qsl, None, hinit, -1, 0, 4)
    assert_close(orc.to_float(out), ref, what="conv token-major 16384x4096")
    assert np.array_equal(st_got, st_ref)


@pytest.mark.parametrize("W", [4, 3, 2])
@pytest.mark.parametrize("dim", [2056, 104, 100])
def test_causal_conv1d_token_major_boundaries(W, dim):
    """Token-major sequences whose starts fall on every position of a 16-token
    chunk (among them the last two, whose first tokens belong to the chunk
    before), empty and one-token sequences, a padded slot, mixed initial
    states, api_mode 0; dim 2056 spans a partial 2048-channel slab and 100 is
    not a multiple of 8 (the 2-byte path)."""
    r = rng(300 + W + dim)
    lens = [14, 1, 0, 17, 15, 2, 33, 16, 1, 0, 47, 3]
    total = sum(lens)
    n = len(lens)
    x = bits(r.standard_normal((total, dim), dtype=np.float32))
    w = bits(r.normal(0, 0.5, (W, dim)).astype(np.float32))
    st = bits(r.standard_normal((n + 1, W - 1, dim), dtype=np.float32))
    qsl = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cidx = np.array([3, 0, 1, 2, 12, 5, 4, 7, 6, 9, 8, 11], np.int32)
    cidx[5] = 99        # padded slot: skipped
    hinit = (r.integers(0, 2, n)).astype(np.int8)
    st_ref = st.copy()
    ref = orc.causal_conv1d(x, w, conv_state=st_ref, query_start_loc=qsl, cache_indices=cidx,
                            has_initial_state=hinit, pad_slot_id=99, layout="ld")
    out, st_got = _conv_c_api(x, w, st, qsl, cidx, hinit, 99, 0, W)
    got = orc.to_float(out)
    pad_rows = slice(qsl[5], qsl[6])
    assert np.isnan(got[pad_rows]).all(), "padded sequence was written"
    keep = np.ones(total, bool)
    keep[pad_rows] = False
    assert_close(got[keep], ref[keep], what=f"conv token-major W={W} dim={dim}")
    assert np.array_equal(st_got, st_ref)


def test_causal_conv1d_token_major_ex_batch_strides():
    """tecoopsCausalConv1dEx on [B, L, D] storage (no query_start_loc: batch
    strides) with bias and state, through tecoops.causal_conv1d on a
    [B, D, L] view."""
    r = rng(310)
    B, L, dim = 3, 530, 1032
    xs = bits(r.standard_normal((B, L, dim), dtype=np.float32))
    w = bits(r.normal(0, 0.5, (dim, 4)).astype(np.float32))
    bias = bits(r.standard_normal(dim, dtype=np.float32))
    st = bits(r.standard_normal((B, 3, dim), dtype=np.float32))
    hinit = np.array([1, 0, 1], np.int8)
    st_ref = st.copy()
    x_bdl = np.ascontiguousarray(xs.transpose(0, 2, 1))
    ref = orc.causal_conv1d(x_bdl, w, bias=bias, conv_state=st_ref, has_initial_state=hinit,
                            layout="bdl")
    xt = dev(xs).permute(0, 2, 1)
    out = torch.empty((B, L, dim), dtype=torch.float16, device="cuda").permute(0, 2, 1)
    st_dev = dev(st)
    tecoops.causal_conv1d(xt, dev(w), dev(bias), out, conv_states=st_dev,
                          has_initial_state=dev(hinit))
    torch.cuda.synchronize()
    assert_close(as_f32(out.permute(0, 2, 1)).transpose(0, 2, 1), ref, what="conv [B, L, D]")
    assert np.array_equal(host_bits(st_dev), st_ref)


def test_causal_conv1d_baseline_config():
    """BASELINE config: x fp16 [8, 4096, 2048] ~N(0,1), weight [4096, 4]
    ~N(0,0.5), bias [4096] ~N(0,1), SiLU, final state written."""
    r = rng(77)
    B, dim, L = 8, 4096, 2048
    x = bits(r.standard_normal((B, dim, L)))
    w = bits(r.normal(0, 0.5, (dim, 4)))
    bias = bits(r.standard_normal(dim))
    st = np.zeros((B, 3, dim), np.uint16)
    ref = orc.causal_conv1d(x, w, bias=bias, conv_state=st, layout="bdl")
    out = torch.empty((B, dim, L), dtype=torch.float16, device="cuda")
    st_dev = torch.zeros((B, 3, dim), dtype=torch.float16, device="cuda")
    tecoops.causal_conv1d(dev(x), dev(w), dev(bias), out, conv_states=st_dev)
    torch.cuda.synchronize()
    assert_close(as_f32(out), ref, what="conv 8x4096x2048")
    assert np.array_equal(host_bits(st_dev), st)


# -------------------------------------------------------------------------- GEMV

@pytest.mark.parametrize("B", [1, 8, 3, 11, 20])
def test_gemv_fp16(B):
    r = rng(300 + B)
    N, K = (14336, 4096) if B in (1, 8) else (1000, 512)
    W = bits(r.normal(0, 0.02, (N, K)))
    x = bits(r.standard_normal((B, K)))
    ref = orc.gemv(W, x)
    y = torch.empty((B, N), dtype=torch.float16, device="cuda")
    tecoops.gemv(dev(W), dev(x), y)
    torch.cuda.synchronize()
    assert_close(as_f32(y), ref, what=f"gemv B={B}")


@pytest.mark.parametrize("B", [1, 8, 5, 17])
def test_gemv_int8(B):
    r = rng(400 + B)
    N, K = (14336, 4096) if B in (1, 8) else (777, 1024)
    W = r.integers(-127, 128, (N, K), dtype=np.int8)
    s = bits(r.uniform(0.001, 0.01, N))
    x = bits(r.standard_normal((B, K)))
    ref = orc.gemv_int8(W, s, x)
    y = torch.empty((B, N), dtype=torch.float16, device="cuda")
    tecoops.gemv_int8(dev(W), dev(s), dev(x), y)
    torch.cuda.synchronize()
    got = as_f32(y)
    # 1e-2 relative, with an absolute floor of 1e-3 of the output scale for
    # outputs that cancel to near zero
    assert_close(got, ref, atol=1e-3 * np.abs(ref).max(), rtol=1e-2, what=f"gemv_int8 B={B}")


@pytest.mark.parametrize("N,K", [(10243, 2000), (10240, 4096), (10239, 4096), (10240, 4112)])
def test_gemv_int8_batch1_row_split(N, K):
    """Batch-1 int8 rows of at most 4096 values over at least 10240 rows take
    one row per wave (workgroups of 4 rows, the last one ragged at N = 10243);
    one row fewer, or 16 values more per row, takes two rows per wave."""
    r = rng(450 + N % 7 + K // 16)
    W = r.integers(-127, 128, (N, K), dtype=np.int8)
    s = bits(r.uniform(0.001, 0.01, N))
    x = bits(r.standard_normal((1, K)))
    ref = orc.gemv_int8(W, s, x)
    y = torch.empty((1, N), dtype=torch.float16, device="cuda")
    tecoops.gemv_int8(dev(W), dev(s), dev(x), y)
    torch.cuda.synchronize()
    assert_close(as_f32(y), ref, atol=1e-3 * np.abs(ref).max(), rtol=1e-2,
                 what=f"gemv_int8 1x{N}x{K}")


@pytest.mark.parametrize("B,K", [(1, 14336), (2, 14336), (4, 14336), (5, 14336), (8, 14336),
                                 (4, 20480), (3, 24576), (1, 40960)])
@pytest.mark.parametrize("i8", [False, True], ids=["fp16", "int8"])
def test_gemv_long_rows(B, K, i8):
    """Rows longer than 64 KiB of staged x: the 4x4x4 path stages up to the
    workgroup's whole LDS (4 x 20480 x 2 bytes is exactly 160 KiB) and sweeps
    K in phases, x staged one phase at a time, when the batch's rows do not
    fit (8 x 14336, 4 x 20480 with the split-K sums, 3 x 24576); the VALU
    path (batch 1) stages up to 160 KiB of x per launch."""
    r = rng(700 + B + K // 1024 + (50 if i8 else 0))
    N = 1000
    x = bits(r.standard_normal((B, K)))
    y = torch.empty((B, N), dtype=torch.float16, device="cuda")
    if i8:
        W = r.integers(-127, 128, (N, K), dtype=np.int8)
        s = bits(r.uniform(0.001, 0.01, N))
        ref = orc.gemv_int8(W, s, x)
        tecoops.gemv_int8(dev(W), dev(s), dev(x), y)
        torch.cuda.synchronize()
        assert_close(as_f32(y), ref, atol=1e-3 * np.abs(ref).max(), rtol=1e-2,
                     what=f"gemv_int8 {B}x{N}x{K}")
    else:
        W = bits(r.normal(0, 0.02, (N, K)))
        ref = orc.gemv(W, x)
        tecoops.gemv(dev(W), dev(x), y)
        torch.cuda.synchronize()
        assert_close(as_f32(y), ref, what=f"gemv {B}x{N}x{K}")


@pytest.mark.parametrize("K", [32, 224, 1248, 2080])
@pytest.mark.parametrize("dt", [orc.HALF, orc.BF16])
def test_gemv_matrix_core_ragged_k(K, dt):
    """Batch 4 runs on the matrix-core path, whose 4 waves take the 32-k
    steps w, w+4, ... of K: 1, 7, 39 and 65 steps give waves 0, 1, 2 and
    several steps each, unequal step counts, and counts below, between and
    above the multiples of the load-ahead depth."""
    r = rng(600 + K)
    N = 300
    W = bits(r.normal(0, 0.05, (N, K)), dt)
    x = bits(r.standard_normal((4, K)), dt)
    ref = orc.gemv(W, x, dtype=dt)
    y = torch.empty((4, N), dtype=torch.float16 if dt == orc.HALF else torch.bfloat16,
                    device="cuda")
    tecoops.gemv(dev(W, dt), dev(x, dt), y)
    torch.cuda.synchronize()
    assert_close(as_f32(y, dt), ref, what=f"gemv 4x{N}x{K}")


@pytest.mark.parametrize("K", [64, 448, 1472, 4160])
def test_gemv_int8_matrix_core_ragged_k(K):
    """int8 steps are 64 k: 1, 7, 23 and 65 steps over 4 waves."""
    r = rng(700 + K)
    N = 200
    W = r.integers(-127, 128, (N, K), dtype=np.int8)
    s = bits(r.uniform(0.001, 0.01, N))
    x = bits(r.standard_normal((3, K)))
    ref = orc.gemv_int8(W, s, x)
    y = torch.empty((3, N), dtype=torch.float16, device="cuda")
    tecoops.gemv_int8(dev(W), dev(s), dev(x), y)
    torch.cuda.synchronize()
    assert_close(as_f32(y), ref, atol=1e-3 * np.abs(ref).max(), rtol=1e-2,
                 what=f"gemv_int8 3x{N}x{K}")


@pytest.mark.parametrize("B,K,dt", [(4, 128, orc.HALF), (6, 1152, orc.BF16),
                                    (8, 2944, orc.HALF), (3, 4096, orc.BF16)])
def test_gemv_small_batch_matrix_core(B, K, dt):
    """Batches 3-8 with K % 128 == 0 run the 4x4x4 path: each wave streams 4
    rows with 8 loads in flight.  K = 128 is one load per row (fewer than the
    ring depth), 1152 and 2944 are 9 and 23 loads (not multiples of it); N =
    301 leaves a partial row group and waves past the last row."""
    r = rng(800 + K + B)
    N = 301
    W = bits(r.normal(0, 0.05, (N, K)), dt)
    x = bits(r.standard_normal((B, K)), dt)
    ref = orc.gemv(W, x, dtype=dt)
    y = torch.empty((B, N), dtype=torch.float16 if dt == orc.HALF else torch.bfloat16,
                    device="cuda")
    tecoops.gemv(dev(W, dt), dev(x, dt), y)
    torch.cuda.synchronize()
    assert_close(as_f32(y, dt), ref, what=f"gemv {B}x{N}x{K}")


@pytest.mark.parametrize("B,K", [(2, 256), (7, 2304), (4, 4096), (8, 768)])
def test_gemv_int8_small_batch_matrix_core(B, K):
    """int8 batches 2-8 with K % 256 == 0 take the 4x4x4 path: 1, 9, 16 and 3
    loads per row."""
    r = rng(900 + K + B)
    N = 203
    W = r.integers(-127, 128, (N, K), dtype=np.int8)
    s = bits(r.uniform(0.001, 0.01, N))
    x = bits(r.standard_normal((B, K)))
    ref = orc.gemv_int8(W, s, x)
    y = torch.empty((B, N), dtype=torch.float16, device="cuda")
    tecoops.gemv_int8(dev(W), dev(s), dev(x), y)
    torch.cuda.synchronize()
    assert_close(as_f32(y), ref, atol=1e-3 * np.abs(ref).max(), rtol=1e-2,
                 what=f"gemv_int8 {B}x{N}x{K}")


@pytest.mark.parametrize("B,N,K", [(3, 301, 256), (8, 4099, 2304), (5, 8191, 4096),
                                   (2, 1000, 14336), (4, 6144, 512)])
@pytest.mark.parametrize("i8", [False, True], ids=["fp16", "int8"])
def test_gemv_split_k(B, N, K, i8):
    """Below 8192 rows the 4x4x4 path gives each row group two waves, each
    sweeping half of K, and adds their sums through LDS: halves of 1 load
    step (K = 256 fp16 / 512 int8), 9 and 5 steps (not multiples of the
    ring depth), a partial row group and waves past the last row; an int8 K
    that is an odd number of 256-k steps (2304) takes the unsplit kernel;
    fp16 batch 2 takes this path only for K above 10240."""
    r = rng(960 + N + K + B + i8)
    x = bits(r.standard_normal((B, K)))
    y = torch.empty((B, N), dtype=torch.float16, device="cuda")
    if i8:
        W = r.integers(-127, 128, (N, K), dtype=np.int8)
        s = bits(r.uniform(0.001, 0.01, N))
        ref = orc.gemv_int8(W, s, x)
        tecoops.gemv_int8(dev(W), dev(s), dev(x), y)
        torch.cuda.synchronize()
        assert_close(as_f32(y), ref, atol=1e-3 * np.abs(ref).max(), rtol=1e-2,
                     what=f"gemv_int8 {B}x{N}x{K}")
    else:
        W = bits(r.normal(0, 0.05, (N, K)))
        ref = orc.gemv(W, x)
        tecoops.gemv(dev(W), dev(x), y)
        torch.cuda.synchronize()
        assert_close(as_f32(y), ref, what=f"gemv {B}x{N}x{K}")


@pytest.mark.parametrize("B,N,K,i8", [(8, 1000, 14336, False), (6, 8200, 10496, False),
                                      (8, 1000, 30720, True), (7, 8192, 21504, True),
                                      (5, 1000, 10624, False)])
def test_gemv_phased_x(B, N, K, i8):
    """x that does not fit in LDS whole is staged in K phases, W still read
    once: 2 phases with K split over four waves (8 x 14336 fp16), 2 unsplit
    (8200 rows), 5 with K split over four waves (int8 8 x 30720: 5 x 6144)
    and 3 unsplit (int8 8192 x 21504: 3 x 7168).  K = 10624 = 83 x 128 has no
    phase count that divides it into whole load steps: batch 5 runs as
    slices of 4 and 1."""
    r = rng(990 + B + N + K // 128 + i8)
    x = bits(r.standard_normal((B, K)))
    y = torch.empty((B, N), dtype=torch.float16, device="cuda")
    if i8:
        W = r.integers(-127, 128, (N, K), dtype=np.int8)
        s = bits(r.uniform(0.001, 0.01, N))
        ref = orc.gemv_int8(W, s, x)
        tecoops.gemv_int8(dev(W), dev(s), dev(x), y)
        torch.cuda.synchronize()
        assert_close(as_f32(y), ref, atol=1e-3 * np.abs(ref).max(), rtol=1e-2,
                     what=f"gemv_int8 {B}x{N}x{K}")
    else:
        W = bits(r.normal(0, 0.02, (N, K)))
        ref = orc.gemv(W, x)
        tecoops.gemv(dev(W), dev(x), y)
        torch.cuda.synchronize()
        assert_close(as_f32(y), ref, what=f"gemv {B}x{N}x{K}")


@pytest.mark.parametrize("N", [16384, 14336, 12288, 301])
@pytest.mark.parametrize("i8", [False, True])
def test_gemv_small_batch_workgroup_sizes(N, i8):
    """The 4x4x4 path sizes its workgroups from N and the CU count: on 256
    CUs these N take 16, 14, 12 and 8 waves per workgroup (the grid stages x
    once per workgroup; waves past the last row still stage their share)."""
    r = rng(950 + N + i8)
    B, K = 5, 256
    x = bits(r.standard_normal((B, K)))
    y = torch.empty((B, N), dtype=torch.float16, device="cuda")
    if i8:
        W = r.integers(-127, 128, (N, K), dtype=np.int8)
        s = bits(r.uniform(0.001, 0.01, N))
        ref = orc.gemv_int8(W, s, x)
        tecoops.gemv_int8(dev(W), dev(s), dev(x), y)
        torch.cuda.synchronize()
        assert_close(as_f32(y), ref, atol=1e-3 * np.abs(ref).max(), rtol=1e-2,
                     what=f"gemv_int8 {B}x{N}x{K}")
    else:
        W = bits(r.normal(0, 0.05, (N, K)))
        ref = orc.gemv(W, x)
        tecoops.gemv(dev(W), dev(x), y)
        torch.cuda.synchronize()
        assert_close(as_f32(y), ref, what=f"gemv {B}x{N}x{K}")


def test_gemv_odd_shapes_and_bf16():
    r = rng(500)
    for N, K, dt in ((33, 100, orc.HALF), (64, 4096, orc.BF16)):
        W = bits(r.normal(0, 0.05, (N, K)), dt)
        x = bits(r.standard_normal((2, K)), dt)
        ref = orc.gemv(W, x, dtype=dt)
        y = torch.empty((2, N), dtype=torch.float16 if dt == orc.HALF else torch.bfloat16,
                        device="cuda")
        tecoops.gemv(dev(W, dt), dev(x, dt), y)
        torch.cuda.synchronize()
        assert_close(as_f32(y, dt), ref, what=f"gemv {N}x{K}")
    W = r.integers(-127, 128, (50, 40), dtype=np.int8)  # K % 16 != 0: scalar path
    s = bits(r.uniform(0.001, 0.01, 50))
    x = bits(r.standard_normal((1, 40)))
    y = torch.empty((1, 50), dtype=torch.float16, device="cuda")
    tecoops.gemv_int8(dev(W), dev(s), dev(x), y)
    torch.cuda.synchronize()
    assert_close(as_f32(y), orc.gemv_int8(W, s, x), what="gemv_int8 scalar")


# ------------------------------------------------------------------------ memset

@pytest.mark.parametrize("offset,size", [(0, 4096), (3, 1000), (1, 15), (5, 1 << 20)])
def test_memset_bit_exact(offset, size):
    buf = torch.full((size + 64,), 0x11, dtype=torch.uint8, device="cuda")
    view = buf[offset:offset + size]
    tecoops.memset(view, 0x3a7)
    torch.cuda.synchronize()
    h = buf.cpu().numpy()
    ref = np.full(size + 64, 0x11, np.uint8)
    orc.memset(ref[offset:offset + size], 0x3a7)
    assert np.array_equal(h, ref)
