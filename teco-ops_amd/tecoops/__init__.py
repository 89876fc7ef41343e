"""tecoops — PyTorch-ROCm front end of the MI355X operator library.

Mirrors the reference package api/tecoops/__init__.py:3-5 and the wrappers of
api/tecoops/../torch_ext.cpp:61-206: the same function names, positional
arguments and in-place semantics (outputs are caller-allocated tensors; the
functions return None), with device='cuda' in place of 'sdaa'.  Every call
goes through the C ABI of libtecoops.so on the current torch stream; there is
no CPU fallback.

Differences from the reference wrappers, all toward its documented intent:
  * each call binds torch.cuda.current_stream() (the reference never calls
    tecoopsSetStream and runs on the null stream, torch_ext.cpp:35-42);
  * flash_attn_varlen_func passes cu_seqlens_q to the device instead of copying
    it to the host (torch_ext.cpp:119-126), honours softmax_scale and causal,
    and takes the element type (fp16 or bf16) from q;
  * causal_conv1d_fn_torch reads the [dim, tokens] layout in place instead of
    transposing x and out (torch_ext.cpp:186-205).
"""
import ctypes
import os
import sys
import threading

import torch

from . import _lib
from ._lib import TecoopsError  # noqa: F401

# TORCH_LIBRARY(tecoops) registrations (libtecoops_torch.so): the same ops as
# torch.ops.tecoops.*, with torch schemas and the current-stream binding done
# in C++.  Loaded when built; the Python functions below call the C ABI
# directly and do not depend on it.
_TORCH_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtecoops_torch.so")
ops = None
if os.path.exists(_TORCH_LIB):
    torch.ops.load_library(_TORCH_LIB)
    ops = torch.ops.tecoops

__all__ = [
    "flatten_rays", "morton3D_invert", "reshape_and_cache", "rms_norm",
    "flash_attn_varlen_func", "causal_conv1d_fn_torch",
    # extensions
    "rotary_embedding", "rotary_reshape_and_cache", "gemv", "gemv_int8", "causal_conv1d",
    "memset", "ops",
]

_tls = threading.local()   # per thread: {device index: _Handle}
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


class _Handle:
    """One tecoops handle of one (thread, device), bound to that thread's
    current torch stream of the device.  Threads never share a handle, so a
    thread cannot enqueue on another thread's stream, and the handle orders
    its split-KV scratch across the streams it is used on."""

    def __init__(self):
        self.h = ctypes.c_void_p()
        _lib.call("tecoopsCreate", ctypes.byref(self.h))
        self.stream = None

    def __del__(self):
        # the thread ended: its handle (and scratch) go with it
        try:
            if self.h and not sys.is_finalizing():
                _lib.lib().tecoopsDestroy(self.h)
        except Exception:
            pass


def _handle(device):
    """The calling thread's handle for `device`, bound to the thread's current
    torch stream there (rebound only when that stream changes)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    handles = getattr(_tls, "handles", None)
    if handles is None:
        handles = _tls.handles = {}
    entry = handles.get(idx)
    if entry is None:
        entry = handles[idx] = _Handle()
    stream = _raw_stream(idx) if _raw_stream else torch.cuda.current_stream(idx).cuda_stream
    if stream != entry.stream:
        _lib.call("tecoopsSetStream", entry.h, ctypes.c_void_p(stream))
        entry.stream = stream
    return entry.h


def _dtype_code(t):
    if t.dtype == torch.float16:
        return _lib.DATA_HALF
    if t.dtype == torch.bfloat16:
        return _lib.DATA_BFLOAT16
    raise TypeError(f"tecoops: unsupported dtype {t.dtype} (float16 or bfloat16)")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _check_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("tecoops: tensors must live on a cuda (ROCm) device")


def _check_contiguous(**ts):
    """The C ABI takes plain pointers with packed row-major extents."""
    for name, t in ts.items():
        if t is not None and not t.is_contiguous():
            raise ValueError(f"tecoops: {name} must be contiguous")


def _check_dtype(t, name, *dtypes):
    if t is not None and t.dtype not in dtypes:
        raise TypeError(f"tecoops: {name} must be {' or '.join(str(d) for d in dtypes)}, "
                        f"got {t.dtype}")


class _Desc:
    """tecoopsTensorDescriptor_t for a row-major tensor, freed on exit."""

    def __init__(self, t, dtype_code):
        self.d = ctypes.c_void_p()
        _lib.call("tecoopsCreateTensorDescriptor", ctypes.byref(self.d))
        dims = (ctypes.c_int * t.dim())(*t.shape)
        strides = (ctypes.c_int * t.dim())(*t.stride())
        _lib.call("tecoopsSetTensorNdDescriptor", self.d, dtype_code, t.dim(), dims, strides)

    def __enter__(self):
        return self.d

    def __exit__(self, *exc):
        _lib.lib().tecoopsDestroyTensorDescriptor(self.d)


# ------------------------------------------------------------------ reference API

def flatten_rays(rays, N, M, res):
    """Reference NeRF op (outside the LLM path): not supported."""
    _lib.call("tecoopsFlattenRays", _handle(rays.device), _ptr(rays), N, M, _ptr(res), 0)


def morton3D_invert(indices, N, coords):
    """Reference NeRF op (outside the LLM path): not supported."""
    _lib.call("tecoopsMorton3DInvert", _handle(indices.device), _ptr(indices), N, _ptr(coords))


def reshape_and_cache(key, value, slot_mapping, key_cache, value_cache):
    """key/value [T, Hkv, D]; caches [num_blocks, Hkv, block_size, D];
    slot_mapping int64 [T] (reference torch_ext.cpp:61-79)."""
    _check_cuda(key, value, slot_mapping, key_cache, value_cache)
    _check_contiguous(key=key, value=value, slot_mapping=slot_mapping, key_cache=key_cache,
                      value_cache=value_cache)
    if slot_mapping.dtype != torch.int64:
        raise TypeError("slot_mapping must be int64")
    T, H, D = key.shape
    _lib.call("tecoopsReshapeAndCacheEx", _handle(key.device), _ptr(key), _ptr(value),
              _ptr(slot_mapping), _ptr(key_cache), _ptr(value_cache), T, H, D,
              key_cache.shape[0], key_cache.shape[2], _dtype_code(key))


def rms_norm(input, weight, residual, output, residual_out, eps):
    """(reference torch_ext.cpp:81-97)."""
    _check_cuda(input, weight, residual, output, residual_out)
    _check_contiguous(input=input, weight=weight, residual=residual, output=output,
                      residual_out=residual_out)
    D = input.shape[-1]
    N = input.numel() // D if D else 0      # leading dims are rows, as in the plugin
    for name, t in (("weight", weight), ("residual", residual), ("output", output),
                    ("residual_out", residual_out)):
        _check_dtype(t, name, input.dtype)
    if weight.numel() != D or output.numel() != input.numel():
        raise ValueError("tecoops.rms_norm: weight must hold hidden_size elements and output "
                         "match input")
    for name, t in (("residual", residual), ("residual_out", residual_out)):
        if t is not None and t.numel() != input.numel():
            raise ValueError(f"tecoops.rms_norm: {name} must match input")
    _lib.call("tecoopsRmsNormEx", _handle(input.device), _ptr(input), _ptr(weight),
              _ptr(residual), _ptr(output), _ptr(residual_out), N, D, float(eps),
              _dtype_code(input))


def flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q, max_seqlen_k, cu_seqlens_k,
                           seqused_k, softmax_scale, causal, window_size, block_table,
                           return_softmax_lse, out):
    """Paged varlen attention (reference torch_ext.cpp:99-165).

    q [sum(L), H, D]; k/v caches [num_blocks, Hkv, block_size, D];
    cu_seqlens_q int32 [B+1]; seqused_k int32 [B]; block_table int32 [B, nb].
    cu_seqlens_k, window_size and return_softmax_lse are accepted and ignored,
    as in the reference."""
    _check_cuda(q, k, v, cu_seqlens_q, seqused_k, block_table, out)
    code = _dtype_code(q)
    scale = float(softmax_scale) if softmax_scale is not None and softmax_scale > 0 else -1.0
    with _Desc(block_table, _lib.DATA_INT32) as btd, _Desc(q, code) as qd, \
            _Desc(k, code) as kd, _Desc(v, code) as vd, _Desc(out, code) as od:
        _lib.call("tecoopsFlashAttentionEx", _handle(q.device), int(max_seqlen_q),
                  int(max_seqlen_k), None, _ptr(cu_seqlens_q), _ptr(seqused_k), btd,
                  _ptr(block_table), qd, _ptr(q), kd, _ptr(k), vd, _ptr(v), od, _ptr(out),
                  scale, int(bool(causal)), None)


def causal_conv1d_fn_torch(out, conv_states, x, weight, query_start_loc, cache_indices,
                           has_initial_state, pad_slot_id):
    """x, out [dim, total_tokens]; weight [width, dim]; conv_states
    [entries, width-1, dim]; query_start_loc int32 [B+1] (reference
    torch_ext.cpp:167-206).  SiLU is applied, as in the reference."""
    _check_cuda(out, conv_states, x, weight, query_start_loc, cache_indices, has_initial_state)
    dim, total = x.shape
    width = weight.shape[0]
    batch = query_start_loc.shape[0] - 1
    _lib.call("tecoopsCausalConv1dEx", _handle(x.device), batch, total, dim, width,
              _ptr(x), 0, x.stride(1), x.stride(0), _ptr(out), 0, out.stride(1), out.stride(0),
              _ptr(weight), weight.stride(1), weight.stride(0), None, _ptr(conv_states),
              conv_states.stride(0) if conv_states is not None else 0, _ptr(query_start_loc),
              _ptr(cache_indices), _ptr(has_initial_state), int(pad_slot_id), 0, 1)


# ---------------------------------------------------------------------- extensions

def causal_conv1d(x, weight, bias, out, conv_states=None, cache_indices=None,
                  has_initial_state=None, pad_slot_id=-1, activation="silu"):
    """Batched causal conv on x [B, dim, L] with weight [dim, width] and optional
    bias [dim]; writes out [B, dim, L]."""
    _check_cuda(x, weight, bias, out, conv_states, cache_indices, has_initial_state)
    B, dim, L = x.shape
    width = weight.shape[1]
    _lib.call("tecoopsCausalConv1dEx", _handle(x.device), B, L, dim, width,
              _ptr(x), x.stride(0), x.stride(2), x.stride(1),
              _ptr(out), out.stride(0), out.stride(2), out.stride(1),
              _ptr(weight), weight.stride(0), weight.stride(1), _ptr(bias), _ptr(conv_states),
              conv_states.stride(0) if conv_states is not None else 0, None,
              _ptr(cache_indices), _ptr(has_initial_state), int(pad_slot_id), 0,
              int(activation in ("silu", "swish", True)))


def rotary_embedding(positions, query, key, head_size, cos_sin_cache=None, is_neox=True,
                     base=10000.0, rot_dim=None):
    """In place on query [T, H*D or H, D] and key [T, Hkv*D or Hkv, D]."""
    _check_cuda(positions, query, key, cos_sin_cache)
    T = positions.numel()
    H = query.numel() // (T * head_size)
    Hkv = key.numel() // (T * head_size) if key is not None else 0
    rd = rot_dim if rot_dim is not None else (
        cos_sin_cache.shape[1] if cos_sin_cache is not None else head_size)
    if cos_sin_cache is not None and cos_sin_cache.dtype != torch.float32:
        raise TypeError("cos_sin_cache must be float32")
    _lib.call("tecoopsRotaryEmbedding", _handle(query.device), _ptr(positions), _ptr(query),
              _ptr(key), T, H, Hkv, head_size, rd, query.stride(0),
              key.stride(0) if key is not None else 0, _ptr(cos_sin_cache),
              cos_sin_cache.shape[0] if cos_sin_cache is not None else 0, float(base),
              int(bool(is_neox)), _dtype_code(query))


def rotary_reshape_and_cache(positions, query, key, value, slot_mapping, key_cache, value_cache,
                             head_size, cos_sin_cache=None, is_neox=True, base=10000.0,
                             rot_dim=None, write_key=False):
    """Decode step: rotary on query (in place) and key, then the rotated key and
    value stored into the paged caches [num_blocks, Hkv, block_size, head_size]
    at slot_mapping (int64); key is updated in place only when write_key."""
    _check_cuda(positions, query, key, value, slot_mapping, key_cache, value_cache, cos_sin_cache)
    if slot_mapping.dtype != torch.int64 or positions.dtype != torch.int64:
        raise TypeError("positions and slot_mapping must be int64")
    if cos_sin_cache is not None and cos_sin_cache.dtype != torch.float32:
        raise TypeError("cos_sin_cache must be float32")
    T = positions.numel()
    H = query.numel() // (T * head_size)
    Hkv = key.numel() // (T * head_size)
    rd = rot_dim if rot_dim is not None else (
        cos_sin_cache.shape[1] if cos_sin_cache is not None else head_size)
    _lib.call("tecoopsRotaryReshapeAndCache", _handle(query.device), _ptr(positions), _ptr(query),
              _ptr(key), _ptr(value), _ptr(slot_mapping), _ptr(key_cache), _ptr(value_cache),
              T, H, Hkv, head_size, rd, query.stride(0), key.stride(0), value.stride(0),
              _ptr(cos_sin_cache), cos_sin_cache.shape[0] if cos_sin_cache is not None else 0,
              float(base), int(bool(is_neox)), key_cache.shape[0], key_cache.shape[2],
              int(bool(write_key)), _dtype_code(query))


def gemv(weight, x, out):
    """out[b, n] = sum_k weight[n, k] x[b, k]; weight [N, K], x [B, K], out [B, N]."""
    _check_cuda(weight, x, out)
    _check_contiguous(weight=weight, x=x, out=out)
    _check_dtype(weight, "weight", x.dtype)
    _check_dtype(out, "out", x.dtype)
    N, K = weight.shape
    B = x.shape[0] if x.dim() == 2 else 1
    if x.shape[-1] != K or out.numel() != B * N:
        raise ValueError(f"tecoops.gemv: x must be [B, {K}] and out [B, {N}]")
    _lib.call("tecoopsGemv", _handle(x.device), _ptr(weight), _ptr(x), _ptr(out), B, N, K,
              _dtype_code(x))


def gemv_int8(weight, scales, x, out):
    """out[b, n] = scales[n] * sum_k weight[n, k] x[b, k]; weight int8 [N, K]."""
    _check_cuda(weight, scales, x, out)
    _check_contiguous(weight=weight, scales=scales, x=x, out=out)
    _check_dtype(weight, "weight", torch.int8)
    _check_dtype(scales, "scales", torch.float16)
    _check_dtype(x, "x", torch.float16)
    _check_dtype(out, "out", torch.float16)
    N, K = weight.shape
    B = x.shape[0] if x.dim() == 2 else 1
    if x.shape[-1] != K or out.numel() != B * N or scales.numel() != N:
        raise ValueError(f"tecoops.gemv_int8: x must be [B, {K}], out [B, {N}], scales [{N}]")
    _lib.call("tecoopsGemvInt8", _handle(x.device), _ptr(weight), _ptr(scales), _ptr(x),
              _ptr(out), B, N, K)


def memset(t, value):
    """Byte fill of a tensor's storage (value truncated to uint8)."""
    _check_cuda(t)
    _lib.call("tecoopsMemset", _handle(t.device), _ptr(t), int(value),
              t.numel() * t.element_size())
