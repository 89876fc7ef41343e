"""The engine plugin contract (include/tecoops_plugin.h, libtecoops_plugin.so).

CPU: registration (names, inputs, output counts as in the reference plugins
teco/plugin/*/plugin_*.cc), InferOutputShape of every plugin, attribute
handling and error statuses, and that the library exports what the header
declares.  GPU: every plugin's Enqueue against the oracle, including the
reference's zero-then-compute semantics (the packed reshape_and_cache output,
conv1d's zeroed outputs and copied state)."""
import math
import os
import re
import subprocess

import numpy as np
import pytest

from tecoops import _lib, plugin
from oracle import oracle as orc

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "tecoops_plugin.h")

# Registration order of inputs and number of outputs, as in the reference
# (plugin_rms_norm.cc:80-84, :136-149; plugin_reshape_and_cache.cc:117-130;
#  plugin_causal_conv1d.cc:162-186; plugin_flash_attention.cc:136-160).
SPECS = {
    "plugin_rms_norm": (["input", "weight"], 1),
    "plugin_rms_norm_add": (["input", "weight", "residual"], 2),
    "plugin_reshape_and_cache": (["key", "value", "slot_mapping"], 1),
    "plugin_causal_conv1d_fn": (["x", "weight", "queryStartLoc", "convStateIndices",
                                 "hasInitialState", "convState"], 2),
    "plugin_flash_attention": (["q", "k_cache", "v_cache", "block_table", "cu_seqlens_q",
                                "seqused_k"], 1),
}


def test_header_functions_exported():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(tecoopsPlugin[A-Z]\w*)\s*\(", text)))
    assert len(declared) == 9
    out = subprocess.run(["nm", "-D", "--defined-only", plugin._PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (tecoopsPlugin\w+)", out))
    assert set(declared) <= exported, set(declared) - exported


def test_registry():
    assert plugin.names() == sorted(SPECS)
    for name, (inputs, n_out) in SPECS.items():
        assert plugin.spec(name) == (inputs, n_out)
    with pytest.raises(KeyError):
        plugin.spec("plugin_nope")
    with pytest.raises(_lib.TecoopsError) as e:
        plugin.Plugin("plugin_nope")
    assert e.value.status == _lib.NOT_SUPPORTED


def test_infer_output_shapes():
    p = plugin.Plugin("plugin_rms_norm")
    assert p.infer_output_shape([(7, 256), (256,)]) == [(7, 256)]
    p = plugin.Plugin("plugin_rms_norm_add")
    assert p.infer_output_shape([(7, 256), (256,), (7, 256)], eps=1e-6) == [(7, 256), (7, 256)]
    p = plugin.Plugin("plugin_reshape_and_cache")
    # K and V packed in one [2 * num_blocks, Hkv, block_size, D] output.
    assert p.infer_output_shape([(40, 2, 64), (40, 2, 64), (40,)], num_blocks=10,
                                block_size=8) == [(20, 2, 8, 64)]
    p = plugin.Plugin("plugin_causal_conv1d_fn")
    assert p.infer_output_shape([(12, 64), (4, 64), (3,), (2,), (2,), (5, 3, 64)]) == \
        [(12, 64), (5, 3, 64)]
    p = plugin.Plugin("plugin_flash_attention")
    assert p.infer_output_shape([(21, 4, 128), (8, 2, 16, 128), (8, 2, 16, 128), (2, 4), (3,),
                                 (2,)], max_seqlen_q=20, max_seqlen_k=50) == [(21, 4, 128)]


def test_attribute_and_shape_errors():
    p = plugin.Plugin("plugin_reshape_and_cache")
    shapes = [(40, 2, 64), (40, 2, 64), (40,)]
    for attrs in ({}, {"num_blocks": 0, "block_size": 8}):  # default num_blocks is 0
        with pytest.raises(_lib.TecoopsError) as e:
            p.infer_output_shape(shapes, **attrs)
        assert e.value.status == _lib.BAD_PARAM
    with pytest.raises(_lib.TecoopsError) as e:
        p.infer_output_shape(shapes, num_blocks=4, block_size=8, bogus=1)
    assert e.value.status == _lib.BAD_PARAM
    with pytest.raises(_lib.TecoopsError) as e:   # wrong number of inputs
        p.infer_output_shape(shapes[:2], num_blocks=4, block_size=8)
    assert e.value.status == _lib.BAD_PARAM
    with pytest.raises(_lib.TecoopsError) as e:   # key must be rank 3
        p.infer_output_shape([(40, 128), (40, 128), (40,)], num_blocks=4, block_size=8)
    assert e.value.status == _lib.BAD_PARAM
    # Reals, integers and lists parse; a real where an integer is expected truncates.
    assert plugin.format_attrs({"a": 1, "b": 0.5, "c": [1, 2], "d": True}) == b"a=1;b=0.5;c=[1,2];d=1"
    assert p.infer_output_shape(shapes, num_blocks=4.0, block_size=8) == [(8, 2, 8, 64)]


# ------------------------------------------------------------------------ GPU

@pytest.mark.gpu
@pytest.mark.parametrize("dt", [orc.HALF, orc.BF16])
def test_rms_norm_plugins(dt):
    import torch
    from helpers import as_f32, assert_close, bits, dev, host_bits
    r = np.random.default_rng(11)
    x = bits(r.standard_normal((64, 512)), dt)
    w = bits(r.uniform(0.5, 1.5, 512), dt)
    res = bits(r.standard_normal((64, 512)), dt)
    tdt = torch.float16 if dt == orc.HALF else torch.bfloat16
    p = plugin.Plugin("plugin_rms_norm")
    out = torch.empty((64, 512), dtype=tdt, device="cuda")
    p.enqueue([dev(x, dt), dev(w, dt)], [out], eps=1e-6)
    ref, _ = orc.rms_norm(x, w, eps=1e-6, dtype=dt)
    pa = plugin.Plugin("plugin_rms_norm_add")
    out2, rout = torch.empty_like(out), torch.empty_like(out)
    pa.enqueue([dev(x, dt), dev(w, dt), dev(res, dt)], [out2, rout], eps=1e-6)
    ref2, rref = orc.rms_norm(x, w, residual=res, eps=1e-6, dtype=dt)
    torch.cuda.synchronize()
    assert_close(as_f32(out, dt), orc.to_float(ref, dt), what="plugin_rms_norm")
    assert_close(as_f32(out2, dt), orc.to_float(ref2, dt), what="plugin_rms_norm_add")
    assert np.array_equal(host_bits(rout), rref)


@pytest.mark.gpu
def test_reshape_and_cache_plugin():
    import torch
    from helpers import bits, dev, host_bits
    r = np.random.default_rng(12)
    T, H, D, NB, BS = 40, 2, 64, 10, 8
    key, val = bits(r.standard_normal((T, H, D))), bits(r.standard_normal((T, H, D)))
    slots = r.permutation(NB * BS)[:T].astype(np.int64)
    slots[5] = -1  # skipped
    p = plugin.Plugin("plugin_reshape_and_cache")
    (shape,) = p.infer_output_shape([key.shape, val.shape, slots.shape], num_blocks=NB,
                                    block_size=BS)
    out = torch.full(shape, float("nan"), dtype=torch.float16, device="cuda")  # must be zeroed
    p.enqueue([dev(key), dev(val), dev(slots)], [out], num_blocks=NB, block_size=BS)
    kc = np.zeros((NB, H, BS, D), np.uint16)
    vc = np.zeros_like(kc)
    orc.reshape_and_cache(key, val, slots, kc, vc)
    torch.cuda.synchronize()
    got = host_bits(out)
    assert np.array_equal(got[:NB], kc) and np.array_equal(got[NB:], vc)


@pytest.mark.gpu
def test_causal_conv1d_plugin():
    import torch
    from helpers import as_f32, assert_close, bits, dev, host_bits
    r = np.random.default_rng(13)
    dim, W = 64, 4
    qsl = np.array([0, 5, 12, 14], np.int32)
    x = bits(r.standard_normal((14, dim)))
    w = bits(r.standard_normal((W, dim)))
    st = bits(r.standard_normal((4, W - 1, dim)))
    cidx = np.array([2, -1, 0], np.int32)    # sequence 1 is padding: skipped, out stays 0
    hin = np.array([1, 0, 0], np.int8)
    st_ref = st.copy()
    ref = orc.causal_conv1d(x, w, conv_state=st_ref, query_start_loc=qsl, cache_indices=cidx,
                            has_initial_state=hin, pad_slot_id=-1, layout="ld")
    p = plugin.Plugin("plugin_causal_conv1d_fn")
    ins = [dev(x), dev(w), dev(qsl), dev(cidx), dev(hin), dev(st)]
    shapes = p.infer_output_shape([t.shape for t in ins])
    out = torch.full(shapes[0], 3.0, dtype=torch.float16, device="cuda")
    st_out = torch.full(shapes[1], 3.0, dtype=torch.float16, device="cuda")
    p.enqueue(ins, [out, st_out], pad_slot_id=-1)
    torch.cuda.synchronize()
    assert_close(as_f32(out), ref, what="plugin_causal_conv1d_fn")
    assert not as_f32(out)[5:12].any()
    assert np.array_equal(host_bits(st_out), st_ref)
    assert np.array_equal(host_bits(ins[5]), st_ref)  # the input state is updated in place too


@pytest.mark.gpu
@pytest.mark.parametrize("dt,set_bounds", [(orc.HALF, True), (orc.BF16, False)])
def test_flash_attention_plugin(dt, set_bounds):
    import torch
    from helpers import as_f32, assert_close, bits, dev
    r = np.random.default_rng(14)
    H, Hkv, D, BS = 4, 2, 128, 16
    q_lens, kv_lens = [1, 20], [50, 20]
    kc = bits(r.uniform(-1, 1, (8, Hkv, BS, D)), dt)
    vc = bits(r.uniform(-1, 1, (8, Hkv, BS, D)), dt)
    q = bits(r.uniform(-1, 1, (21, H, D)), dt)
    bt = np.array([[3, 1, 6, 0], [5, 2, 0, 0]], np.int32)
    cu = np.array([0, 1, 21], np.int32)
    p = plugin.Plugin("plugin_flash_attention")
    ins = [dev(q, dt), dev(kc, dt), dev(vc, dt), dev(bt), dev(cu),
           dev(np.array(kv_lens, np.int32))]
    (shape,) = p.infer_output_shape([t.shape for t in ins])
    out = torch.empty(shape, dtype=ins[0].dtype, device="cuda")
    attrs = dict(max_seqlen_q=20, max_seqlen_k=50, max_block_num=4) if set_bounds else {}
    p.enqueue(ins, [out], **attrs)
    torch.cuda.synchronize()
    ref = orc.flash_attention(q, kc, vc, bt, q_lens, kv_lens, dtype=dt)
    assert_close(as_f32(out, dt), ref, what="plugin_flash_attention")
    # Extension attributes: explicit scale, no mask.
    p.enqueue(ins, [out], softmax_scale=0.05, causal=0, **attrs)
    torch.cuda.synchronize()
    ref = orc.flash_attention(q, kc, vc, bt, q_lens, kv_lens, softmax_scale=0.05, causal=False,
                              dtype=dt)
    assert_close(as_f32(out, dt), ref, what="plugin_flash_attention scale/no mask")
    assert math.isfinite(float(out.float().abs().max()))
