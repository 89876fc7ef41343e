"""tecoops._torch_ext — the reference's extension-module name.

The reference package imports its six ops from a compiled module of this name
(api/tecoops/__init__.py:3; built from api/torch_ext.cpp:208-215).  Here the
same names are the TORCH_LIBRARY(tecoops) ops of libtecoops_torch.so
(torch.ops.tecoops.*), which bind the current HIP stream in C++, with the
reference's positional arguments and in-place outputs.  flatten_rays and
morton3D_invert are outside the LLM-inference path and have no torch op; they
are the package's C-ABI wrappers, which report NOT_SUPPORTED.

Importing fails loudly when libtecoops_torch.so has not been built.
"""
import os

import torch

_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtecoops_torch.so")
if not os.path.exists(_LIB):
    raise ImportError(f"{_LIB} is missing: build it with `python teco-ops_amd/build.py`")
if not hasattr(torch.ops.tecoops, "rms_norm"):
    torch.ops.load_library(_LIB)

from . import flatten_rays, morton3D_invert  # noqa: E402  (C-ABI wrappers)

reshape_and_cache = torch.ops.tecoops.reshape_and_cache
rms_norm = torch.ops.tecoops.rms_norm
flash_attn_varlen_func = torch.ops.tecoops.flash_attn_varlen_func
causal_conv1d_fn_torch = torch.ops.tecoops.causal_conv1d_fn_torch

__all__ = ["flatten_rays", "morton3D_invert", "reshape_and_cache", "rms_norm",
           "flash_attn_varlen_func", "causal_conv1d_fn_torch"]
