"""The TORCH_LIBRARY(tecoops) registration (libtecoops_torch.so): schemas on
the CPU; on the GPU every torch.ops.tecoops op against the oracle."""
import math

import numpy as np
import pytest
import torch

import tecoops
from oracle import oracle as orc

from helpers import as_f32, assert_close, bits, dev, host_bits

# Reference names and argument order (api/torch_ext.cpp:61-206) plus extensions.
EXPECTED = {
    "reshape_and_cache": "reshape_and_cache(Tensor key, Tensor value, Tensor slot_mapping, "
                         "Tensor(a!) key_cache, Tensor(b!) value_cache) -> ()",
    "rms_norm": "rms_norm(Tensor input, Tensor weight, Tensor? residual, Tensor(a!) output, "
                "Tensor(b!)? residual_out, float eps) -> ()",
    "flash_attn_varlen_func": "flash_attn_varlen_func(Tensor q, Tensor k, Tensor v, "
                              "int max_seqlen_q, Tensor cu_seqlens_q, int max_seqlen_k, "
                              "Tensor? cu_seqlens_k, Tensor seqused_k, float softmax_scale, "
                              "bool causal, Tensor? window_size, Tensor block_table, "
                              "bool return_softmax_lse, Tensor(a!) out) -> ()",
    "causal_conv1d_fn_torch": "causal_conv1d_fn_torch(Tensor(a!) out, Tensor(b!) conv_states, "
                              "Tensor x, Tensor weight, Tensor query_start_loc, "
                              "Tensor cache_indices, Tensor has_initial_state, "
                              "int pad_slot_id) -> ()",
}


def test_library_loaded_with_schemas():
    assert tecoops.ops is not None, "libtecoops_torch.so not built"
    for name, schema in EXPECTED.items():
        op = getattr(torch.ops.tecoops, name).default
        assert str(op._schema) == "tecoops::" + schema
    for name in ("causal_conv1d", "rotary_embedding", "rotary_reshape_and_cache", "gemv",
                 "gemv_int8", "memset"):
        assert hasattr(torch.ops.tecoops, name)


@pytest.mark.gpu
def test_torch_ops_parity():
    r = np.random.default_rng(3)
    ops = torch.ops.tecoops
    # reshape_and_cache (bit-exact)
    key, val = bits(r.standard_normal((40, 2, 64))), bits(r.standard_normal((40, 2, 64)))
    slots = r.permutation(80)[:40].astype(np.int64)
    kc_ref = np.zeros((10, 2, 8, 64), np.uint16)
    vc_ref = kc_ref.copy()
    orc.reshape_and_cache(key, val, slots, kc_ref, vc_ref)
    kc, vc = dev(np.zeros_like(kc_ref)), dev(np.zeros_like(vc_ref))
    ops.reshape_and_cache(dev(key), dev(val), dev(slots), kc, vc)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(kc), kc_ref) and np.array_equal(host_bits(vc), vc_ref)
    # rms_norm with residual
    x, res = bits(r.uniform(-1, 1, (8, 256))), bits(r.uniform(-1, 1, (8, 256)))
    w = bits(r.uniform(0.5, 1.5, 256))
    ref, ref_res = orc.rms_norm(x, w, residual=res, eps=1e-6)
    out = torch.empty((8, 256), dtype=torch.float16, device="cuda")
    ro = torch.empty_like(out)
    ops.rms_norm(dev(x), dev(w), dev(res), out, ro, 1e-6)
    torch.cuda.synchronize()
    assert_close(as_f32(out), orc.to_float(ref), what="rms_norm")
    assert np.array_equal(host_bits(ro), ref_res)
    # flash attention (bf16, paged, chunked prefill + decode row)
    H, Hkv, D, BS = 4, 2, 128, 16
    q_lens, kv_lens = [1, 20], [50, 20]
    kcache = bits(r.uniform(-1, 1, (8, Hkv, BS, D)), orc.BF16)
    vcache = bits(r.uniform(-1, 1, (8, Hkv, BS, D)), orc.BF16)
    q = bits(r.uniform(-1, 1, (21, H, D)), orc.BF16)
    bt = np.array([[3, 1, 6, 0], [5, 2, 0, 0]], np.int32)
    cu = np.array([0, 1, 21], np.int32)
    o = torch.empty((21, H, D), dtype=torch.bfloat16, device="cuda")
    ops.flash_attn_varlen_func(dev(q, orc.BF16), dev(kcache, orc.BF16), dev(vcache, orc.BF16),
                               20, dev(cu), 50, None, dev(np.array(kv_lens, np.int32)),
                               1 / math.sqrt(D), True, None, dev(bt), False, o)
    torch.cuda.synchronize()
    ref = orc.flash_attention(q, kcache, vcache, bt, q_lens, kv_lens, dtype=orc.BF16)
    assert_close(as_f32(o, orc.BF16), ref, what="flash_attn_varlen_func")
    # causal_conv1d_fn_torch ([dim, tokens] layout)
    xc = bits(r.standard_normal((64, 12)))
    wc = bits(r.standard_normal((4, 64)))
    st = bits(r.standard_normal((2, 3, 64)))
    st_ref = st.copy()
    qsl = np.array([0, 5, 12], np.int32)
    cidx = np.array([1, 0], np.int32)
    hin = np.array([1, 0], np.int8)
    ref = orc.causal_conv1d(xc, wc, conv_state=st_ref, query_start_loc=qsl, cache_indices=cidx,
                            has_initial_state=hin, layout="dl")
    outc = torch.zeros((64, 12), dtype=torch.float16, device="cuda")
    st_d = dev(st)
    ops.causal_conv1d_fn_torch(outc, st_d, dev(xc), dev(wc), dev(qsl), dev(cidx), dev(hin), -1)
    torch.cuda.synchronize()
    assert_close(as_f32(outc), ref, what="causal_conv1d_fn_torch")
    assert np.array_equal(host_bits(st_d), st_ref)
    # extensions
    pos = np.arange(6, dtype=np.int64) * 100
    qr, kr = bits(r.standard_normal((6, 4, 64))), bits(r.standard_normal((6, 2, 64)))
    qo, ko = orc.rotary_embedding(pos, qr, kr)
    qt, kt = dev(qr), dev(kr)
    ops.rotary_embedding(dev(pos), qt, kt, 64, None, True, 10000.0, 64)
    Wg = bits(r.normal(0, 0.02, (96, 128)))
    xg = bits(r.standard_normal((3, 128)))
    yg = torch.empty((3, 96), dtype=torch.float16, device="cuda")
    ops.gemv(dev(Wg), dev(xg), yg)
    Wq = r.integers(-127, 128, (96, 128), dtype=np.int8)
    sq = bits(r.uniform(0.001, 0.01, 96))
    yq = torch.empty((3, 96), dtype=torch.float16, device="cuda")
    ops.gemv_int8(dev(Wq), dev(sq), dev(xg), yq)
    xb = bits(r.standard_normal((2, 16, 40)))
    wb = bits(r.standard_normal((16, 4)))
    bb = bits(r.standard_normal(16))
    ob = torch.empty((2, 16, 40), dtype=torch.float16, device="cuda")
    ops.causal_conv1d(dev(xb), dev(wb), dev(bb), ob, None, True)
    buf = torch.zeros(100, dtype=torch.uint8, device="cuda")
    ops.memset(buf, 7)
    torch.cuda.synchronize()
    assert_close(as_f32(qt), qo, what="rotary q")
    assert_close(as_f32(kt), ko, what="rotary k")
    assert_close(as_f32(yg), orc.gemv(Wg, xg), what="gemv")
    assert_close(as_f32(yq), orc.gemv_int8(Wq, sq, xg), atol=1e-3, what="gemv_int8")
    assert_close(as_f32(ob), orc.causal_conv1d(xb, wb, bias=bb, layout="bdl"), what="conv bdl")
    assert (buf.cpu().numpy() == 7).all()
