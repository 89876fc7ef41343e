"""Host-only checks of the C ABI: every symbol of include/tecoops.h is exported,
and the argument-validation branches of the reference interface layer return
the reference's status codes before any device work
(teco/interface/ops/*.cpp check functions; tecoops.cpp:38-258)."""
import ctypes
import os
import re
import subprocess

import pytest

from tecoops import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "tecoops.h")

BAD, NOT_INIT, NOT_SUP, OK = _lib.BAD_PARAM, _lib.NOT_INITIALIZED, _lib.NOT_SUPPORTED, _lib.SUCCESS


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tecoops[A-Z]\w*)\s*\(", text)))


def test_header_and_binding_agree():
    assert header_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_header_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (tecoops\w+)", out))
    missing = [f for f in header_functions() if f not in exported]
    assert not missing, missing
    L = _lib.lib()
    for f in header_functions():
        assert getattr(L, f) is not None


@pytest.fixture
def handle():
    h = ctypes.c_void_p()
    assert _lib.lib().tecoopsCreate(ctypes.byref(h)) == OK
    yield h
    assert _lib.lib().tecoopsDestroy(h) == OK


def test_error_strings():
    L = _lib.lib()
    names = ["SUCCESS", "NOT_INITIALIZED", "ALLOC_FAILED", "BAD_PARAM", "INTERNAL_ERROR",
             "INVALID_VALUE", "NOT_SUPPORTED"]
    for i, n in enumerate(names):
        assert L.tecoopsGetErrorString(i).decode() == "TECOOPS_STATUS_" + n
    assert L.tecoopsGetErrorString(77).decode() == "UNKNOWN_ERROR"


def test_handle_and_stream(handle):
    L = _lib.lib()
    assert L.tecoopsCreate(None) == BAD
    assert L.tecoopsDestroy(None) == BAD
    assert L.tecoopsSetStream(None, None) == BAD
    s = ctypes.c_void_p(1234)
    assert L.tecoopsSetStream(handle, ctypes.c_void_p(0x5000)) == OK
    assert L.tecoopsGetStream(handle, ctypes.byref(s)) == OK and s.value == 0x5000
    assert L.tecoopsGetStream(handle, None) == BAD
    assert L.tecoopsSetStream(handle, None) == OK


def test_descriptors():
    L = _lib.lib()
    d = ctypes.c_void_p()
    assert L.tecoopsCreateTensorDescriptor(ctypes.byref(d)) == OK
    dims = (ctypes.c_int * 3)(4, 5, 6)
    assert L.tecoopsSetTensorNdDescriptor(d, 1, 0, dims, None) == BAD  # tecoops.cpp:168-170
    assert L.tecoopsSetTensorNdDescriptor(d, 9, 3, dims, None) == OK
    dt, nb = ctypes.c_int(), ctypes.c_int()
    gd, gs = (ctypes.c_int * 3)(), (ctypes.c_int * 3)()
    assert L.tecoopsGetTensorNdDescriptor(d, 3, ctypes.byref(dt), ctypes.byref(nb), gd, gs) == OK
    assert (dt.value, nb.value, list(gd), list(gs)) == (9, 3, [4, 5, 6], [30, 6, 1])
    # more than TECOOPS_DIM_MAX dims
    big = (ctypes.c_int * 10)(*([2] * 10))
    assert L.tecoopsSetTensorNdDescriptor(d, 1, 10, big, None) == OK
    gd10 = (ctypes.c_int * 10)()
    assert L.tecoopsGetTensorNdDescriptor(d, 10, None, ctypes.byref(nb), gd10, None) == OK
    assert nb.value == 10 and list(gd10) == [2] * 10
    # 4d NHWC strides (tecoops.cpp:91-95)
    assert L.tecoopsSetTensor4dDescriptor(d, 1, 1, 2, 3, 4, 5) == OK
    v = [ctypes.c_int() for _ in range(9)]
    assert L.tecoopsGetTensor4dDescriptor(d, *[ctypes.byref(x) for x in v]) == OK
    assert [x.value for x in v] == [1, 2, 3, 4, 5, 60, 1, 15, 3]
    assert L.tecoopsSetTensor4dDescriptor(d, 5, 1, 2, 3, 4, 5) == BAD
    assert L.tecoopsDestroyTensorDescriptor(d) == OK
    assert L.tecoopsDestroyTensorDescriptor(None) == OK


P = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first


def test_reshape_and_cache_validation(handle):
    L = _lib.lib()
    f = L.tecoopsReshapeAndCache
    assert f(None, P, P, P, P, P, 1, 1, 8, 1, 1) == NOT_INIT
    assert f(handle, None, P, P, P, P, 1, 1, 8, 1, 1) == BAD
    assert f(handle, P, P, None, P, P, 1, 1, 8, 1, 1) == BAD
    assert f(handle, P, P, P, None, P, 1, 1, 8, 1, 1) == BAD
    for bad in [(0, 1, 8, 1, 1), (1, 0, 8, 1, 1), (1, 1, 0, 1, 1), (1, 1, 8, 0, 1),
                (1, 1, 8, 1, 0)]:
        assert f(handle, P, P, P, P, P, *bad) == BAD
    assert L.tecoopsReshapeAndCacheEx(handle, P, P, P, P, P, 1, 1, 8, 1, 1, 0) == BAD


def test_rms_norm_validation(handle):
    f = _lib.lib().tecoopsRmsNorm
    assert f(None, P, P, None, P, None, 1, 8, 1e-6) == NOT_INIT
    assert f(handle, None, P, None, P, None, 1, 8, 1e-6) == BAD
    assert f(handle, P, None, None, P, None, 1, 8, 1e-6) == BAD
    assert f(handle, P, P, None, None, None, 1, 8, 1e-6) == BAD
    assert f(handle, P, P, P, P, None, 1, 8, 1e-6) == BAD  # residual without residual_out
    assert f(handle, P, P, None, P, None, 0, 8, 1e-6) == BAD
    assert f(handle, P, P, None, P, None, 1, 0, 1e-6) == BAD
    assert _lib.lib().tecoopsRmsNormEx(handle, P, P, None, P, None, 1, 8, 1e-6, 0) == BAD


def test_causal_conv1d_validation(handle):
    f = _lib.lib().tecoopsCausalConv1d
    args = [1, 4, 8, 4, 24, 8, 8, -1, 0, 0]
    assert f(None, *args, P, P, P, P, None, None, None) == NOT_INIT
    assert f(handle, *args, None, P, P, P, None, None, None) == BAD
    assert f(handle, *args, P, P, None, P, None, None, None) == BAD
    assert f(handle, *args, P, P, P, None, None, None, None) == BAD
    for i in range(4):
        a = list(args)
        a[i] = 0
        assert f(handle, *a, P, P, P, P, None, None, None) == BAD
    a = list(args)
    a[3] = 5  # width beyond the supported range
    assert f(handle, *a, P, P, P, P, None, None, None) == NOT_SUP


def test_memset_validation(handle):
    f = _lib.lib().tecoopsMemset
    assert f(None, P, 0, 16) == BAD  # reference memset.cpp:37-45
    assert f(handle, None, 0, 16) == BAD
    assert f(handle, P, 0, 0) == OK  # nothing to do, no launch


def test_out_of_path_ops_not_supported(handle):
    L = _lib.lib()
    assert L.tecoopsFlattenRays(None, P, 1, 1, P, 0) == NOT_INIT
    assert L.tecoopsFlattenRays(handle, P, 1, 1, P, 0) == NOT_SUP
    assert L.tecoopsMorton3DInvert(handle, P, 1, P) == NOT_SUP
    assert L.tecoopsReduceVariance(handle, 0, 0, P, P, P, P) == NOT_SUP


def _desc(dtype, dims):
    d = ctypes.c_void_p()
    _lib.lib().tecoopsCreateTensorDescriptor(ctypes.byref(d))
    arr = (ctypes.c_int * len(dims))(*dims)
    _lib.lib().tecoopsSetTensorNdDescriptor(d, dtype, len(dims), arr, None)
    return d


def test_flash_attention_validation(handle):
    L = _lib.lib()
    bt = _desc(_lib.DATA_INT32, [2, 4])
    q = _desc(_lib.DATA_HALF, [8, 4, 128])
    k = _desc(_lib.DATA_HALF, [16, 2, 16, 128])
    v = _desc(_lib.DATA_HALF, [16, 2, 16, 128])
    o = _desc(_lib.DATA_HALF, [8, 4, 128])
    vf = _desc(_lib.DATA_FLOAT, [16, 2, 16, 128])
    vbf = _desc(_lib.DATA_BFLOAT16, [16, 2, 16, 128])
    kbf = _desc(_lib.DATA_BFLOAT16, [16, 2, 16, 128])
    vshape = _desc(_lib.DATA_HALF, [16, 2, 32, 128])
    q80 = _desc(_lib.DATA_HALF, [8, 4, 80])
    k80 = _desc(_lib.DATA_HALF, [16, 2, 16, 80])
    f = L.tecoopsFlashAttention

    def call(h=handle, kd=k, vd=v, qd=q, od=o):
        return f(h, 4, 16, 16, P, P, bt, P, qd, P, kd, P, vd, P, od, P, None)

    assert call(h=None) == NOT_INIT
    assert call(vd=vbf) == BAD            # k/v dtype mismatch (flash_attention.cpp:52-55)
    assert call(kd=vf, vd=vf) == BAD      # neither half nor bf16
    assert call(kd=kbf, vd=vbf) == BAD    # q/o stay half: types must agree
    assert call(vd=vshape) == BAD         # k/v shape mismatch (:62-67)
    # head sizes: multiples of 32 up to 192 (flash_attention.scpp:188, :347-348)
    assert call(qd=q80, od=q80, kd=k80, vd=k80) == NOT_SUP
    # max_seqlen_q / max_seqlen_k are launch hints (the reference never reads
    # them), but a caller workspace is sized by max_seqlen_k, so the Ex entry
    # point needs it positive when one is passed
    ex = L.tecoopsFlashAttentionEx
    assert ex(handle, 1, 0, P, None, P, bt, P, q, P, k, P, v, P, o, P, -1.0, 1, P) == BAD
    assert ex(handle, 1, 16, None, None, P, bt, P, q, P, k, P, v, P, o, P, -1.0, 1, P) == BAD
    for d in (bt, q, k, v, o, vf, vbf, kbf, vshape, q80, k80):
        L.tecoopsDestroyTensorDescriptor(d)


def test_rotary_and_gemv_validation(handle):
    L = _lib.lib()
    r = L.tecoopsRotaryEmbedding
    assert r(None, P, P, P, 1, 1, 1, 64, 64, 64, 64, None, 0, 1e4, 1, 1) == NOT_INIT
    assert r(handle, P, P, P, 1, 1, 1, 64, 63, 64, 64, None, 0, 1e4, 1, 1) == BAD  # odd rot
    assert r(handle, P, P, P, 1, 1, 1, 64, 128, 64, 64, None, 0, 1e4, 1, 1) == BAD  # rot > head
    assert r(handle, P, P, P, 1, 1, 1, 64, 64, 32, 64, None, 0, 1e4, 1, 1) == BAD  # stride
    assert r(handle, P, P, P, 1, 1, 1, 64, 64, 64, 64, P, 0, 1e4, 1, 1) == BAD  # cache w/o size
    assert L.tecoopsGemv(None, P, P, P, 1, 8, 8, 1) == NOT_INIT
    assert L.tecoopsGemv(handle, P, P, P, 0, 8, 8, 1) == BAD
    assert L.tecoopsGemv(handle, P, P, P, 1, 8, 8, 2) == BAD
    assert L.tecoopsGemvInt8(handle, P, None, P, P, 1, 8, 8) == BAD
    ws = ctypes.c_size_t()
    assert L.tecoopsGetFlashAttentionWorkspaceSize(64, 32, 128, 1, 8192, ctypes.byref(ws)) == OK
    assert ws.value > 0
    # max_seqlen_q <= 0 sizes for the longest q the decode route takes
    big = ctypes.c_size_t()
    assert L.tecoopsGetFlashAttentionWorkspaceSize(64, 32, 128, 0, 8192, ctypes.byref(big)) == OK
    assert big.value >= ws.value
    assert L.tecoopsGetFlashAttentionWorkspaceSize(64, 32, 128, 1, 0, ctypes.byref(ws)) == BAD


def test_reference_artefact_names():
    """The reference's library names (teco/CMakeLists.txt:99-129) load this
    build's libraries and export the tecoops.h / plugin entry points."""
    d = os.path.dirname(_lib.LIB_PATH)
    for name in ("libteco_ops.so", "libteco_ops_plugin.so"):
        L = ctypes.CDLL(os.path.join(d, name))
        for f in header_functions():
            assert getattr(L, f) is not None, (name, f)
    P_ = ctypes.CDLL(os.path.join(d, "libTecoInferPlugin.so"))
    assert P_.tecoopsPluginCreate is not None


def test_torch_ext_module_names():
    """The reference package's extension module (api/tecoops/__init__.py:3)."""
    from tecoops import _torch_ext
    for name in ("flatten_rays", "morton3D_invert", "reshape_and_cache", "rms_norm",
                 "flash_attn_varlen_func", "causal_conv1d_fn_torch"):
        assert callable(getattr(_torch_ext, name))
    from tecoops._torch_ext import rms_norm  # noqa: F401
