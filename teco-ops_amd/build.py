"""Builds libtecoops.so (the C-ABI operator library) for gfx950.

    python teco-ops_amd/build.py          # or __graft_entry__.build()

Each source under csrc/ is compiled by hipcc into _build/ (in parallel), then
linked into tecoops/libtecoops.so next to the Python package that loads it.
All HIP code is built with packed FP32 instructions disabled.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "tecoops", "libtecoops.so")
TORCH_OUT = os.path.join(HERE, "tecoops", "libtecoops_torch.so")
PLUGIN_OUT = os.path.join(HERE, "tecoops", "libtecoops_plugin.so")
PLUGIN_SOURCES = ["plugin/registry.cpp", "plugin/plugins.cpp"]
# The reference's artefact names (teco/CMakeLists.txt:99-129): libteco_ops.so
# (the operator library of the torch build), libteco_ops_plugin.so (the same
# library in the plugin build) and libTecoInferPlugin.so (the plugins, linked
# against it).  Each is a link to the library built here that holds the same
# interface, so a caller linked against a reference name loads this build.
REFERENCE_NAMES = {
    "libteco_ops.so": "libtecoops.so",
    "libteco_ops_plugin.so": "libtecoops.so",
    "libTecoInferPlugin.so": "libtecoops_plugin.so",
}
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

SOURCES = [
    "handle.cpp",
    "memset.hip",
    "reshape_and_cache.hip",
    "rms_norm.hip",
    "rotary.hip",
    "causal_conv1d.hip",
    "gemv.hip",
    "flash_attention.hip",
    "fa_noalloc.hip",
]

ARCH = os.environ.get("TECOOPS_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    "-I", os.path.join(REPO, "include"), "-I", CSRC,
]


# Per-source flags.  Attention scores are never NaN for finite inputs (masked
# scores are -inf), so the softmax max tree needs no NaN canonicalisation.
EXTRA_FLAGS = {
    "flash_attention.hip": ["-fno-honor-nans"],
}


# Sources whose kernels copy global memory straight into LDS
# (global_load_lds_dwordx4, inline assembly) and then wait for the copies
# with a fixed vmcnt that leaves the compiler's own younger loads in flight.
# The count is right only if those loads stay between the copies and the
# wait, which the compiler does not promise for loads of read-only memory,
# so the device assembly of these sources is checked on every build.
# flash_attention.hip waits for its copies by counting only younger copies
# (inline assembly, which the compiler keeps in order), so only its use of M0
# is checked there.
COPY_WAIT_CHECKED = {"gemv.hip": True, "flash_attention.hip": False}


def check_copy_waits(asm_text, src="", waits=True):
    """Checks, in each kernel of `asm_text` that copies into LDS, the first
    vmcnt wait after each run of copies: its count N must not exceed the
    vector-memory operations issued between the last copy and the wait (so
    that the copies are among the completed ones, vector-memory loads
    completing in issue order), no barrier may come between the copies and
    that wait, and M0 may be written only right before a copy (with waits
    False, only the last).  Returns the number of waits checked (of copies
    seen, with waits False); raises RuntimeError on a violation."""
    import re
    checked = 0
    kernels = list(re.finditer(r"^(_Z\S*):", asm_text, re.M))
    for m in kernels:
        end = asm_text.find(".Lfunc_end", m.end())
        lines = [l.split(";")[0].strip() for l in asm_text[m.end():end].split("\n")]
        lines = [l for l in lines if l and not l.startswith(".")]
        if not any(l.startswith("global_load_lds") for l in lines):
            continue
        pending, since = False, 0
        for i, l in enumerate(lines):
            if re.search(r"\bm0\b", l) and not (l.startswith("s_mov_b32 m0,") and i + 1 < len(lines)
                                                and lines[i + 1].startswith("global_load_lds")):
                raise RuntimeError(f"{src}: {m.group(1)}: M0 used outside a copy: {l}")
            if l.startswith("global_load_lds"):
                pending, since = True, 0
                if not waits:
                    checked += 1
                continue
            if not pending or not waits:
                continue
            if re.match(r"(global|buffer|flat)_(load|store|atomic)", l):
                since += 1
            w = re.match(r"s_waitcnt\b.*\bvmcnt\((\d+)\)", l)
            if w:
                if int(w.group(1)) > since:
                    raise RuntimeError(f"{src}: {m.group(1)}: {l} after copies with only {since} "
                                       "younger vector-memory operations: the copies may be in flight")
                pending = False
                checked += 1
            elif l.startswith("s_barrier"):
                raise RuntimeError(f"{src}: {m.group(1)}: barrier before the copies are waited for")
    return checked


def _check_copies(src, waits):
    out = os.path.join(BUILD, os.path.splitext(src)[0] + ".s")
    cmd = [HIPCC, *CFLAGS, *EXTRA_FLAGS.get(src, []), "--cuda-device-only", "-S",
           os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"assembly failed: {src}\n{' '.join(cmd)}\n{r.stderr[-4000:]}")
    with open(out) as f:
        n = check_copy_waits(f.read(), src, waits)
    os.remove(out)
    if n == 0:
        raise RuntimeError(f"{src}: no LDS copies found to check")
    return out, ""


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd.insert(1, "-x")
        cmd.insert(2, "hip")
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{err}")
    return obj, err


def build_torch_ext(verbose=False):
    """TORCH_LIBRARY(tecoops) registration (host C++) linked against
    libtecoops.so; loaded with torch.ops.load_library."""
    import torch
    from torch.utils import cpp_extension as ce
    inc = ce.include_paths(device_type="cuda") if "device_type" in \
        ce.include_paths.__code__.co_varnames else ce.include_paths(cuda=True)
    libdirs = [os.path.join(os.path.dirname(torch.__file__), "lib")]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1",
           "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=tecoops",
           "-Wno-deprecated-declarations",
           "-I", os.path.join(REPO, "include"), *sum((["-I", d] for d in inc), []),
           os.path.join(CSRC, "torch_ext.cpp"), "-o", TORCH_OUT + ".tmp",
           *sum((["-L", d] for d in libdirs), []),
           "-L", os.path.dirname(OUT), "-ltecoops", "-lc10", "-lc10_hip", "-ltorch_cpu",
           "-ltorch_hip", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdirs[0]}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch extension build failed:\n{' '.join(cmd)}\n{r.stderr[-4000:]}")
    os.replace(TORCH_OUT + ".tmp", TORCH_OUT)
    return TORCH_OUT


def build_plugins(verbose=False):
    """Engine plugins (host C++, include/tecoops_plugin.h) linked against
    libtecoops.so and the HIP runtime."""
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-D__HIP_PLATFORM_AMD__=1",
           "-I", os.path.join(REPO, "include"), "-I", os.path.join(ROCM, "include"),
           *[os.path.join(CSRC, s) for s in PLUGIN_SOURCES], "-o", PLUGIN_OUT + ".tmp",
           "-L", os.path.dirname(OUT), "-ltecoops", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"plugin build failed:\n{' '.join(cmd)}\n{r.stderr[-4000:]}")
    if verbose and r.stderr.strip():
        print(r.stderr, file=sys.stderr)
    os.replace(PLUGIN_OUT + ".tmp", PLUGIN_OUT)
    return PLUGIN_OUT


def link_reference_names():
    """(Re)creates the reference-named links next to the built libraries."""
    d = os.path.dirname(OUT)
    for name, target in REFERENCE_NAMES.items():
        path = os.path.join(d, name)
        if os.path.lexists(path):
            os.remove(path)
        os.symlink(target, path)


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    jobs = min(len(SOURCES), os.cpu_count() or 4, 16)
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        checks = [ex.submit(_check_copies, src, w) for src, w in COPY_WAIT_CHECKED.items()]
        results = list(ex.map(_compile, SOURCES))
        for c in checks:
            c.result()
    for _, err in results:
        if err.strip() and verbose:
            print(err, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, OUT)
    build_plugins(verbose)
    build_torch_ext(verbose)
    link_reference_names()
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
