"""Engine-side driver of the tecoops plugins (libtecoops_plugin.so).

Plays the part of the inference engine of the reference plugin contract
(doc/README_PLUGIN.md:56-141): one `Plugin` per graph node, `infer_output_shape`
before allocation, `enqueue` with device tensors on the current torch stream.
Shapes, element types and attributes travel through the C entry points
declared in include/tecoops_plugin.h.

    p = Plugin("plugin_reshape_and_cache")
    (shape,) = p.infer_output_shape([key.shape, value.shape, slots.shape],
                                    num_blocks=64, block_size=16)
    out = torch.empty(shape, dtype=key.dtype, device="cuda")
    p.enqueue([key, value, slots], [out], num_blocks=64, block_size=16)
"""
import ctypes
import os

from . import _lib

_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtecoops_plugin.so")
_L = None
DIM_MAX = 8


def lib():
    global _L
    if _L is None:
        if not os.path.exists(_PATH):
            raise RuntimeError(f"{_PATH} not built: run teco-ops_amd/build.py")
        _lib.lib()  # libtecoops.so first (the plugin library links it by rpath)
        L = ctypes.CDLL(_PATH)
        c_int_p = ctypes.POINTER(ctypes.c_int)
        vp = ctypes.c_void_p
        for name, res, args in [
            ("tecoopsPluginCount", ctypes.c_int, []),
            ("tecoopsPluginName", ctypes.c_char_p, [ctypes.c_int]),
            ("tecoopsPluginNumInputs", ctypes.c_int, [ctypes.c_char_p]),
            ("tecoopsPluginInputName", ctypes.c_char_p, [ctypes.c_char_p, ctypes.c_int]),
            ("tecoopsPluginNumOutputs", ctypes.c_int, [ctypes.c_char_p]),
            ("tecoopsPluginCreate", ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(vp)]),
            ("tecoopsPluginDestroy", ctypes.c_int, [vp]),
            ("tecoopsPluginInferOutputShape", ctypes.c_int,
             [vp, ctypes.c_int, c_int_p, c_int_p, ctypes.c_char_p, ctypes.c_int, c_int_p, c_int_p]),
            ("tecoopsPluginEnqueue", ctypes.c_int,
             [vp, ctypes.c_int, ctypes.POINTER(vp), c_int_p, c_int_p, c_int_p, ctypes.c_int,
              ctypes.POINTER(vp), c_int_p, c_int_p, c_int_p, ctypes.c_char_p, vp]),
        ]:
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _L = L
    return _L


def names():
    L = lib()
    return [L.tecoopsPluginName(i).decode() for i in range(L.tecoopsPluginCount())]


def spec(op):
    """(input names, number of outputs) as registered."""
    L = lib()
    b = op.encode()
    n = L.tecoopsPluginNumInputs(b)
    if n < 0:
        raise KeyError(op)
    return [L.tecoopsPluginInputName(b, i).decode() for i in range(n)], L.tecoopsPluginNumOutputs(b)


def format_attrs(attrs):
    parts = []
    for k, v in attrs.items():
        if isinstance(v, (list, tuple)):
            v = "[" + ",".join(str(int(x)) for x in v) + "]"
        elif isinstance(v, bool):
            v = int(v)
        elif isinstance(v, float):
            v = repr(v)
        parts.append(f"{k}={v}")
    return ";".join(parts).encode()


def _shapes(shapes):
    shapes = [tuple(int(d) for d in s) for s in shapes]
    nd = (ctypes.c_int * max(1, len(shapes)))(*[len(s) for s in shapes])
    flat = [d for s in shapes for d in s]
    dims = (ctypes.c_int * max(1, len(flat)))(*flat)
    return nd, dims


def _dtype_code(t):
    import torch
    return {torch.float16: _lib.DATA_HALF, torch.bfloat16: _lib.DATA_BFLOAT16,
            torch.float32: 0, torch.int8: 2, torch.int16: 3, torch.int32: 4, torch.int64: 5,
            torch.uint8: 6, torch.bool: 7, torch.float64: 8}[t.dtype]


class Plugin:
    """One plugin instance (the engine keeps one per graph node)."""

    def __init__(self, op):
        self.op = op
        self._h = ctypes.c_void_p()
        _lib.check(lib().tecoopsPluginCreate(op.encode(), ctypes.byref(self._h)),
                   "tecoopsPluginCreate")
        self.inputs, self.num_outputs = spec(op)

    def close(self):
        if self._h:
            lib().tecoopsPluginDestroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def infer_output_shape(self, input_shapes, **attrs):
        nd, dims = _shapes(input_shapes)
        n_out = self.num_outputs
        ond = (ctypes.c_int * n_out)()
        odims = (ctypes.c_int * (n_out * DIM_MAX))()
        _lib.check(lib().tecoopsPluginInferOutputShape(self._h, len(input_shapes), nd, dims,
                                                       format_attrs(attrs), n_out, ond, odims),
                   f"{self.op}.InferOutputShape")
        return [tuple(odims[i * DIM_MAX:i * DIM_MAX + ond[i]]) for i in range(n_out)]

    def enqueue(self, inputs, outputs, stream=None, **attrs):
        """inputs / outputs: device tensors in registration order."""
        import torch
        n_in, n_out = len(inputs), len(outputs)
        ptrs = (ctypes.c_void_p * max(1, n_in))(*[t.data_ptr() for t in inputs])
        optrs = (ctypes.c_void_p * max(1, n_out))(*[t.data_ptr() for t in outputs])
        idt = (ctypes.c_int * max(1, n_in))(*[_dtype_code(t) for t in inputs])
        odt = (ctypes.c_int * max(1, n_out))(*[_dtype_code(t) for t in outputs])
        ind, idims = _shapes([t.shape for t in inputs])
        ond, odims = _shapes([t.shape for t in outputs])
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        _lib.check(lib().tecoopsPluginEnqueue(self._h, n_in, ptrs, idt, ind, idims, n_out, optrs,
                                              odt, ond, odims, format_attrs(attrs),
                                              ctypes.c_void_p(stream)),
                   f"{self.op}.Enqueue")
