"""numpy front end of the C oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY.  The parity checker and the CPU baseline: only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module.  The product path (libtecoops.so and the tecoops package) never does.

16-bit tensors are passed as numpy uint16 bit patterns; ``dtype`` is 1 for fp16
and 9 for bfloat16 (the tecoopsDataType_t values).
"""
import ctypes
import os
import subprocess

import numpy as np

HALF = 1
BF16 = 9

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        _LIB = ctypes.CDLL(path)
        _declare(_LIB)
    return _LIB


def _declare(L):
    P = ctypes.c_void_p
    i, f, ll = ctypes.c_int, ctypes.c_float, ctypes.c_longlong
    L.orc_set_threads.argtypes = [i]
    L.orc_get_threads.restype = i
    L.orc_h2f.argtypes = [ctypes.c_uint16]
    L.orc_h2f.restype = f
    L.orc_f2h.argtypes = [f]
    L.orc_f2h.restype = ctypes.c_uint16
    L.orc_b2f.argtypes = [ctypes.c_uint16]
    L.orc_b2f.restype = f
    L.orc_f2b.argtypes = [f]
    L.orc_f2b.restype = ctypes.c_uint16
    L.orc_to_f_array.argtypes = [P, P, ctypes.c_size_t, i]
    L.orc_from_f_array.argtypes = [P, P, ctypes.c_size_t, i]
    L.orc_memset.argtypes = [P, i, ctypes.c_size_t]
    L.orc_reshape_and_cache.argtypes = [P, P, P, P, P, i, i, i, i, i]
    L.orc_rms_norm.argtypes = [P, P, P, P, P, i, i, f, i]
    L.orc_flash_attention.argtypes = [P, P, P, P, i, P, P, i, i, i, i, i, f, i, i, P]
    L.orc_flash_attention_heads.argtypes = [P, P, P, P, i, P, P, i, i, i, i, i, f, i, i,
                                            i, i, i, P]
    L.orc_causal_conv1d.argtypes = [i, i, i, i, P, ll, ll, ll, P, ll, ll, ll, P, i, i, P,
                                    P, i, P, P, P, i, i, i]
    L.orc_rotary_embedding.argtypes = [P, P, P, P, P, i, i, i, i, i, ll, ll, P, i, f, i, i]
    L.orc_gemv.argtypes = [P, P, P, i, i, i, i]
    L.orc_gemv_int8.argtypes = [P, P, P, P, i, i, i]


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return None if a is None else np.ascontiguousarray(a, dtype=dt)


def set_threads(n):
    lib().orc_set_threads(int(n))


def get_threads():
    return lib().orc_get_threads()


# ---------------------------------------------------------------- conversions

def to_float(bits, dtype=HALF):
    bits = _c(bits, np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_to_f_array(_p(bits), _p(out), bits.size, dtype)
    return out


def from_float(x, dtype=HALF):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_from_f_array(_p(x), _p(out), x.size, dtype)
    return out


# ---------------------------------------------------------------------- ops

def memset(buf, value):
    """In place byte fill of a numpy array (value truncated to uint8)."""
    assert buf.flags.c_contiguous
    lib().orc_memset(_p(buf), int(value), buf.nbytes)


def reshape_and_cache(key, value, slot_mapping, key_cache, value_cache):
    """In place on key_cache / value_cache (uint16 [NB, H, BS, D])."""
    key, value = _c(key, np.uint16), _c(value, np.uint16)
    slot_mapping = _c(slot_mapping, np.int64)
    assert key_cache.flags.c_contiguous and value_cache.flags.c_contiguous
    T, H, D = key.shape
    NB, _, BS, _ = key_cache.shape
    lib().orc_reshape_and_cache(_p(key), _p(value), _p(slot_mapping), _p(key_cache),
                                _p(value_cache), T, H, D, NB, BS)


def rms_norm(x, w, residual=None, eps=1e-6, dtype=HALF):
    """Returns (out, residual_out or None) as uint16 bit patterns."""
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    residual = _c(residual, np.uint16)
    N, D = x.shape
    out = np.empty_like(x)
    res_out = np.empty_like(x) if residual is not None else None
    lib().orc_rms_norm(_p(x), _p(w), _p(residual), _p(out), _p(res_out), N, D,
                       float(eps), dtype)
    return out, res_out


def flash_attention(q, k_cache, v_cache, block_table, q_seq_lens, kv_seq_lens,
                    softmax_scale=None, causal=True, dtype=HALF, b_only=-1,
                    h_begin=-1, h_end=-1):
    """q uint16 [sum(L), H, D]; caches uint16 [NB, Hkv, BS, D]; returns fp32 like q."""
    q = _c(q, np.uint16)
    k_cache, v_cache = _c(k_cache, np.uint16), _c(v_cache, np.uint16)
    block_table = _c(block_table, np.int32)
    q_seq_lens, kv_seq_lens = _c(q_seq_lens, np.int32), _c(kv_seq_lens, np.int32)
    _, H, D = q.shape
    _, Hkv, BS, _ = k_cache.shape
    if softmax_scale is None:
        softmax_scale = 1.0 / np.sqrt(D)
    out = np.zeros(q.shape, np.float32)
    lib().orc_flash_attention_heads(
        _p(q), _p(k_cache), _p(v_cache), _p(block_table), block_table.shape[1],
        _p(q_seq_lens), _p(kv_seq_lens), len(q_seq_lens), H, Hkv, D, BS,
        float(softmax_scale), int(bool(causal)), dtype, b_only, h_begin, h_end, _p(out))
    return out


def causal_conv1d(x, weight, bias=None, conv_state=None, query_start_loc=None,
                  cache_indices=None, has_initial_state=None, pad_slot_id=-1,
                  api_mode=0, silu=True, layout="bdl", seq_len=None):
    """Depthwise causal conv.  Returns fp32 output of x's shape; conv_state
    (uint16 [entries, W-1, dim]) is updated in place.

    layout "bdl": x [batch, dim, seqlen] (query_start_loc must be None).
    layout "dl":  x [dim, total] channel-major varlen (reference torch layout).
    layout "ld":  x [total, dim] token-major varlen (reference C API layout).
    weight is [dim, width] for "bdl" and [width, dim] otherwise.
    """
    x = _c(x, np.uint16)
    weight = _c(weight, np.uint16)
    bias = _c(bias, np.uint16)
    qsl = _c(query_start_loc, np.int32)
    cidx = _c(cache_indices, np.int32)
    hinit = _c(has_initial_state, np.int8)
    if layout == "bdl":
        B, dim, L = x.shape
        xs = (dim * L, 1, L)
        width = weight.shape[1]
        ws = (width, 1)
        batch, sl = B, L
    elif layout == "dl":
        dim, total = x.shape
        xs = (0, 1, total)
        width = weight.shape[0]
        ws = (1, dim)
        batch, sl = len(qsl) - 1 if qsl is not None else total, 1
    else:
        total, dim = x.shape
        xs = (dim, dim, 1)
        width = weight.shape[0]
        ws = (1, dim)
        batch, sl = len(qsl) - 1 if qsl is not None else total, 1
    if seq_len is not None:
        sl = seq_len
    out = np.zeros(x.shape, np.float32)
    st_stride = 0
    if conv_state is not None:
        assert conv_state.dtype == np.uint16 and conv_state.flags.c_contiguous
        st_stride = conv_state.shape[1] * conv_state.shape[2]
    lib().orc_causal_conv1d(batch, sl, dim, width, _p(x), xs[0], xs[1], xs[2],
                            _p(out), xs[0], xs[1], xs[2], _p(weight), ws[0], ws[1],
                            _p(bias), _p(conv_state), st_stride, _p(qsl), _p(cidx),
                            _p(hinit), int(pad_slot_id), int(api_mode), int(bool(silu)))
    return out


def rotary_embedding(positions, query, key, rot_dim=None, base=10000.0, is_neox=True,
                     cos_sin_cache=None, dtype=HALF):
    """query uint16 [T, H, D], key uint16 [T, Hkv, D] or None; returns fp32 copies."""
    positions = _c(positions, np.int64)
    query = _c(query, np.uint16)
    key = _c(key, np.uint16)
    T, H, D = query.shape
    Hkv = key.shape[1] if key is not None else 0
    rot = D if rot_dim is None else rot_dim
    qo = np.empty(query.shape, np.float32)
    ko = np.empty(key.shape, np.float32) if key is not None else None
    cache = _c(cos_sin_cache, np.float32)
    maxpos = cache.shape[0] if cache is not None else 0
    lib().orc_rotary_embedding(_p(positions), _p(query), _p(key), _p(qo), _p(ko), T, H, Hkv,
                               D, rot, H * D, Hkv * D, _p(cache), maxpos, float(base),
                               int(bool(is_neox)), dtype)
    return qo, ko


def gemv(weight, x, dtype=HALF):
    weight, x = _c(weight, np.uint16), _c(x, np.uint16)
    N, K = weight.shape
    B = x.shape[0]
    y = np.empty((B, N), np.float32)
    lib().orc_gemv(_p(weight), _p(x), _p(y), B, N, K, dtype)
    return y


def gemv_int8(weight, scales, x):
    weight = _c(weight, np.int8)
    scales, x = _c(scales, np.uint16), _c(x, np.uint16)
    N, K = weight.shape
    B = x.shape[0]
    y = np.empty((B, N), np.float32)
    lib().orc_gemv_int8(_p(weight), _p(scales), _p(x), _p(y), B, N, K)
    return y
