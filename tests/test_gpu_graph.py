"""A decode step captured in a CUDA graph through torch.ops.tecoops and
replayed: rms_norm -> three GEMVs (q, k, v) -> reshape_and_cache -> paged
flash-attention decode -> int8 GEMV.  Every replay, with new inputs written
and eager work run between replays, must equal an eager run of the same ops
on the same inputs bit for bit; the attention output of the first replay is
also checked against the oracle."""
import math

import numpy as np
import pytest
import torch

import tecoops  # noqa: F401  (loads libtecoops_torch.so)
from oracle import oracle as orc

from helpers import as_f32, assert_close, host_bits

pytestmark = pytest.mark.gpu

T, HID, H, HKV, D, BS = 8, 512, 8, 2, 128, 16


def _bufs(seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    kv_lens = [37, 100, 250, 513, 16, 1, 64, 300]  # each includes the new token
    nblk = [(L + BS - 1) // BS for L in kv_lens]
    perm = torch.randperm(sum(nblk) + 7, generator=torch.Generator().manual_seed(seed)).numpy()
    bt = np.zeros((T, max(nblk)), np.int32)
    o = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[o:o + n]
        o += n
    slots = [int(bt[i, (L - 1) // BS]) * BS + (L - 1) % BS for i, L in enumerate(kv_lens)]
    num_blocks = int(perm.max()) + 1
    rn = lambda *s, sc=1.0: (torch.randn(*s, device="cuda", generator=g) * sc).half()
    return {
        "x": rn(T, HID),
        "w_norm": (torch.rand(HID, device="cuda", generator=g) + 0.5).half(),
        "wq": rn(H * D, HID, sc=0.05), "wk": rn(HKV * D, HID, sc=0.05), "wv": rn(HKV * D, HID, sc=0.05),
        "wo": torch.randint(-127, 128, (HID, H * D), device="cuda", generator=g, dtype=torch.int8),
        "so": (torch.rand(HID, device="cuda", generator=g) * 0.01 + 0.001).half(),
        "kc": rn(num_blocks, HKV, BS, D), "vc": rn(num_blocks, HKV, BS, D),
        "bt": torch.from_numpy(bt).cuda(),
        "slots": torch.tensor(slots, dtype=torch.int64, device="cuda"),
        "cu": torch.arange(0, T + 1, dtype=torch.int32, device="cuda"),
        "kv": torch.tensor(kv_lens, dtype=torch.int32, device="cuda"),
        "max_k": max(kv_lens),
        "xn": torch.empty(T, HID, dtype=torch.half, device="cuda"),
        "q": torch.empty(T, H * D, dtype=torch.half, device="cuda"),
        "k": torch.empty(T, HKV * D, dtype=torch.half, device="cuda"),
        "v": torch.empty(T, HKV * D, dtype=torch.half, device="cuda"),
        "o": torch.empty(T, H, D, dtype=torch.half, device="cuda"),
        "y": torch.empty(T, HID, dtype=torch.half, device="cuda"),
    }


def _step(b):
    ops = torch.ops.tecoops
    ops.rms_norm(b["x"], b["w_norm"], None, b["xn"], None, 1e-6)
    ops.gemv(b["wq"], b["xn"], b["q"])
    ops.gemv(b["wk"], b["xn"], b["k"])
    ops.gemv(b["wv"], b["xn"], b["v"])
    ops.reshape_and_cache(b["k"].view(T, HKV, D), b["v"].view(T, HKV, D), b["slots"], b["kc"], b["vc"])
    ops.flash_attn_varlen_func(b["q"].view(T, H, D), b["kc"], b["vc"], 1, b["cu"], b["max_k"], None,
                               b["kv"], 1.0 / math.sqrt(D), True, None, b["bt"], False, b["o"])
    ops.gemv_int8(b["wo"], b["so"], b["o"].view(T, H * D), b["y"])


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_decode_step_graph_replays():
    b = _bufs(7)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up: handles, LDS attributes, allocator pools
        for _ in range(2):
            _step(b)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _step(b)
    g = torch.Generator(device="cuda").manual_seed(11)
    prev_y = None
    for rep in range(3):
        b["x"].copy_(torch.randn(T, HID, device="cuda", generator=g).half())
        # eager reference on copies of the state the replay starts from
        e = {k: (v.clone() if torch.is_tensor(v) else v) for k, v in b.items()}
        _step(e)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name in ("xn", "q", "k", "v", "o", "y", "kc", "vc"):
            assert _same(b[name], e[name]), f"replay {rep}: {name} differs from the eager run"
        if prev_y is not None:
            assert not _same(b["y"], prev_y), f"replay {rep} left y unchanged"
        prev_y = b["y"].clone()
        if rep == 0:
            kv_lens = b["kv"].cpu().tolist()
            ref = orc.flash_attention(host_bits(b["q"].view(T, H, D)), host_bits(b["kc"]),
                                      host_bits(b["vc"]), b["bt"].cpu().numpy(), [1] * T, kv_lens,
                                      dtype=orc.HALF)
            assert_close(as_f32(b["o"]), ref, what="graph replay attention vs oracle")
