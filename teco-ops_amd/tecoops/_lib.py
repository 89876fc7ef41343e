"""ctypes binding of libtecoops.so (declarations mirror include/tecoops.h).

Loading fails loudly when the library has not been built: there is no
fallback implementation.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtecoops.so")

# tecoopsStatus_t (reference teco/interface/include/tecoops.h:39-47)
SUCCESS = 0
NOT_INITIALIZED = 1
ALLOC_FAILED = 2
BAD_PARAM = 3
INTERNAL_ERROR = 4
INVALID_VALUE = 5
NOT_SUPPORTED = 6

# tecoopsDataType_t (reference tecoops.h:73-85)
DATA_FLOAT = 0
DATA_HALF = 1
DATA_INT8 = 2
DATA_INT32 = 4
DATA_INT64 = 5
DATA_BFLOAT16 = 9


class TecoopsError(RuntimeError):
    def __init__(self, status, what=""):
        self.status = status
        name = lib().tecoopsGetErrorString(status).decode()
        super().__init__(f"{what}: {name}" if what else name)


P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float
LL = ctypes.c_longlong
SZ = ctypes.c_size_t

# name -> (restype, argtypes); one entry per function declared in tecoops.h
SIGNATURES = {
    "tecoopsCreate": (I, [P]),
    "tecoopsDestroy": (I, [P]),
    "tecoopsSetStream": (I, [P, P]),
    "tecoopsGetStream": (I, [P, P]),
    "tecoopsGetErrorString": (ctypes.c_char_p, [I]),
    "tecoopsCreateTensorDescriptor": (I, [P]),
    "tecoopsSetTensor4dDescriptor": (I, [P, I, I, I, I, I, I]),
    "tecoopsGetTensor4dDescriptor": (I, [P, P, P, P, P, P, P, P, P, P]),
    "tecoopsSetTensorNdDescriptor": (I, [P, I, I, P, P]),
    "tecoopsGetTensorNdDescriptor": (I, [P, I, P, P, P, P]),
    "tecoopsDestroyTensorDescriptor": (I, [P]),
    "tecoopsFlattenRays": (I, [P, P, ctypes.c_uint32, ctypes.c_uint32, P, I]),
    "tecoopsReduceVariance": (I, [P, I, I, P, P, P, P]),
    "tecoopsMorton3DInvert": (I, [P, P, ctypes.c_uint32, P]),
    "tecoopsMemset": (I, [P, P, I, SZ]),
    "tecoopsReshapeAndCache": (I, [P, P, P, P, P, P, I, I, I, I, I]),
    "tecoopsRmsNorm": (I, [P, P, P, P, P, P, I, I, F]),
    "tecoopsFlashAttention": (I, [P, I, I, I, P, P, P, P, P, P, P, P, P, P, P, P, P]),
    "tecoopsCausalConv1d": (I, [P, I, I, I, I, I, I, I, I, I, I, P, P, P, P, P, P, P]),
    "tecoopsRmsNormEx": (I, [P, P, P, P, P, P, I, I, F, I]),
    "tecoopsReshapeAndCacheEx": (I, [P, P, P, P, P, P, I, I, I, I, I, I]),
    "tecoopsFlashAttentionEx": (I, [P, I, I, P, P, P, P, P, P, P, P, P, P, P, P, P, F, I, P]),
    "tecoopsFlashAttentionNoAlloc": (I, [P, I, I, P, P, P, P, P, P, P, P, P, P, P, P, P, F, I]),
    "tecoopsGetFlashAttentionWorkspaceSize": (I, [I, I, I, I, I, P]),
    "tecoopsCausalConv1dEx": (I, [P, I, I, I, I, P, LL, LL, LL, P, LL, LL, LL, P, I, I, P, P, I,
                                  P, P, P, I, I, I]),
    "tecoopsRotaryEmbedding": (I, [P, P, P, P, I, I, I, I, I, LL, LL, P, I, F, I, I]),
    "tecoopsRotaryReshapeAndCache": (I, [P, P, P, P, P, P, P, P, I, I, I, I, I, LL, LL, LL, P, I,
                                         F, I, I, I, I, I]),
    "tecoopsGemv": (I, [P, P, P, P, I, I, I, I]),
    "tecoopsGemvInt8": (I, [P, P, P, P, P, I, I, I]),
}

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python teco-ops_amd/build.py` "
                "(tecoops has no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(status, what=""):
    if status != SUCCESS:
        raise TecoopsError(status, what)


def call(name, *args):
    check(getattr(lib(), name)(*args), name)
