"""Benchmark of the LLM-inference operator path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--ops a,b]

A step runs every op of the path once at its BASELINE.json config, with all
inputs already resident in HBM (synthetic seeded data):
  rms_norm        x fp16 [4096, 4096], eps 1e-6
  reshape_cache   key/value fp16 [8192, 8, 128] -> 1024 blocks x 16 slots
  causal_conv1d   x fp16 [8, 4096, 2048], width 4, bias, SiLU, final state
  causal_conv1d_tm  the same shape in the reference C layout: x [8 x 2048
                  tokens, 4096] token-major through causal_conv1d_fn_torch
                  (query_start_loc, weight [4, 4096], no bias), final state
  rotary          q [8192, 32, 128], k [8192, 8, 128], neox, base 1e4
  rotary_cache    the fused decode step: rotary on q, k [8192, 8, 128] and
                  k, v into 1024 blocks x 16 (rotary + reshape_and_cache)
  gemv_f16_b{1,8} W fp16 [14336, 4096]
  gemv_i8_b{1,8}  W int8 [14336, 4096] + fp16 scales
  fa_prefill      bf16 q [4, 32, 4096, 128], k/v [4, 8, 4096, 128], causal
  fa_decode       bf16 B=64, 1 token, paged block 16, kv_len ~ U{512..8192}
Each op cycles through enough copies of its inputs/outputs (>= 1 GiB in
total, 4x the 256 MiB MALL) that no launch finds its data in L2 / MALL; in
this steady state an op's HBM traffic per launch equals its algorithmic bytes
(its own dirty outputs are written back during later launches).  Per-op kernel
time: K back-to-back launches of the op between one pair of torch.cuda events
on the stream the ops are enqueued on (tecoops binds the current torch
stream), divided by K, right after a warm-up of at least W launches and 200 ms
of the same op.  Beside it, `us_median20` is the median of 20 more launches
of the op, each between its own pair of events (the extra event markers
between launches can add a little to each).

Prints ONE JSON line.  `value` is flash-attention prefill TFLOP/s (causal
FLOP count / average kernel time), the throughput figure of BASELINE.json's
metric; `ops` lists every op's microseconds, algorithmic GB/s or TFLOP/s and
fraction of the MI355X peak.  `roofline` is the dominant kernel's (by time).
`cpu_baseline` times the CPU oracle (the reference algorithms restated in C)
on the host cores on a bounded sample of the FA prefill config, with a
single-thread figure beside it; `cpu_ops` times the oracle on every other op
at its full config, on all host cores and on one thread (the reference
harness's own CPU loops are single-threaded).  Both are reported baselines,
not targets.
"""
import argparse
import json
import math
import os
import platform
import subprocess
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
for p in (REPO, os.path.join(REPO, "teco-ops_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2516.6

# FA prefill causal FLOPs: 4 * B * H * D * S(S+1)/2
FA_B, FA_H, FA_HKV, FA_S, FA_D = 4, 32, 8, 4096, 128
FA_PREFILL_FLOP = 4 * FA_B * FA_H * FA_D * FA_S * (FA_S + 1) // 2


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ops", default="")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--cases", action="store_true",
                    help="time the reference's own prototxt cases (harness statistic) instead")
    return ap.parse_args()


def seeded_bits(rng, shape, kind="normal", scale=1.0, lo=0.0, hi=1.0, dtype="f16"):
    """Seeded synthetic tensor generated on the GPU (fp32, rounded to 16 bit);
    the torch generator is seeded from `rng`, so each op's data depends only
    on its own seed."""
    import torch
    gen = torch.Generator(device="cuda")
    gen.manual_seed(int(rng.integers(1 << 30)))
    if kind == "normal":
        t = torch.randn(shape, generator=gen, device="cuda") * scale
    else:
        t = torch.rand(shape, generator=gen, device="cuda") * (hi - lo) + lo
    return t.to(torch.float16 if dtype == "f16" else torch.bfloat16)


ROTATE_BYTES = 1 << 30   # rotating working set per op: 4x the 256 MiB MALL
# Minimum warm-up per op, seconds of its own launches.  FA prefill after 30 ms
# still ran its first timed launches slow (mean 579 us, median of the later
# launches 567 us); after 200 ms the mean and the median agree (569 us).
WARM_S = 0.2


def copies_for(ws_bytes, limit=16):
    return max(1, min(limit, -(-ROTATE_BYTES // max(ws_bytes, 1))))


def build_ops(names=None):
    """Allocates every op's inputs on the GPU.  Returns {name: (launches, work)}
    where launches is a list of closures, one per rotating copy of the op's
    inputs and outputs (enough copies that consecutive launches never find
    their data in L2 / MALL)."""
    import torch
    import tecoops

    ops = {}

    scale = 1.0 / math.sqrt(FA_D)

    def want(*ns):
        return names is None or any(n in names for n in ns)

    if names is not None and "copy_calibration" in names:
        # Plain device copy of known size (opt-in): the reference point that
        # scales rocprofv3's FETCH_SIZE / WRITE_SIZE into HBM bytes.
        n = 256 << 20
        fns = []
        for _ in range(copies_for(2 * n)):
            src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
            dst = torch.empty_like(src)
            fns.append(lambda src=src, dst=dst: dst.copy_(src))
        ops["copy_calibration"] = (fns, dict(bytes=2 * n))

    if want("rms_norm"):
        rng = np.random.default_rng(1001)  # each op has its own seed
        # rms_norm [4096, 4096]
        ws = 2 * 4096 * 4096 * 2
        w = seeded_bits(rng, (4096,), "uniform", lo=0.5, hi=1.5)
        fns = []
        for _ in range(copies_for(ws)):
            x = seeded_bits(rng, (4096, 4096))
            y = torch.empty_like(x)
            fns.append(lambda x=x, y=y, w=w: tecoops.rms_norm(x, w, None, y, None, 1e-6))
        ops["rms_norm"] = (fns, dict(bytes=2 * 4096 * 4096 * 2 + 4096 * 2))

    if want("reshape_and_cache"):
        rng = np.random.default_rng(1002)  # each op has its own seed
        # reshape_and_cache: 8192 tokens into 1024 blocks x 16 slots
        T, Hkv, D, NB, BS = 8192, 8, 128, 1024, 16
        ws = 4 * T * Hkv * D * 2
        slots = torch.from_numpy(rng.permutation(NB * BS)[:T].astype(np.int64)).cuda()
        fns = []
        for _ in range(copies_for(ws)):
            key = seeded_bits(rng, (T, Hkv, D))
            val = seeded_bits(rng, (T, Hkv, D))
            kc = torch.zeros((NB, Hkv, BS, D), dtype=torch.float16, device="cuda")
            vc = torch.zeros_like(kc)
            fns.append(lambda key=key, val=val, kc=kc, vc=vc, slots=slots:
                       tecoops.reshape_and_cache(key, val, slots, kc, vc))
        ops["reshape_and_cache"] = (fns, dict(bytes=4 * T * Hkv * D * 2 + T * 8))

    if want("causal_conv1d"):
        rng = np.random.default_rng(1003)  # each op has its own seed
        # causal_conv1d [8, 4096, 2048]
        B, C, L = 8, 4096, 2048
        ws = 2 * B * C * L * 2
        cw = seeded_bits(rng, (C, 4), scale=0.5)
        cb = seeded_bits(rng, (C,))
        fns = []
        for _ in range(copies_for(ws)):
            cx = seeded_bits(rng, (B, C, L))
            co = torch.empty_like(cx)
            cst = torch.zeros((B, 3, C), dtype=torch.float16, device="cuda")
            fns.append(lambda cx=cx, co=co, cst=cst, cw=cw, cb=cb: tecoops.causal_conv1d(
                cx, cw, cb, co, conv_states=cst))
        ops["causal_conv1d"] = (fns, dict(bytes=2 * B * C * L * 2 + C * 4 * 2 + C * 2 + B * 3 * C * 2))

    if want("causal_conv1d_tm"):
        rng = np.random.default_rng(1009)  # each op has its own seed
        # the BASELINE conv shape in the reference C layout [tokens, dim]
        B, C, L = 8, 4096, 2048
        T = B * L
        ws = 2 * T * C * 2
        cw = seeded_bits(rng, (4, C), scale=0.5)             # [width, dim]
        qsl = torch.arange(0, T + 1, L, dtype=torch.int32, device="cuda")
        cidx = torch.arange(B, dtype=torch.int32, device="cuda")
        hinit = torch.zeros(B, dtype=torch.int8, device="cuda")
        fns = []
        for _ in range(copies_for(ws)):
            cx = seeded_bits(rng, (T, C))                    # token-major storage
            co = torch.empty_like(cx)
            cst = torch.zeros((B, 3, C), dtype=torch.float16, device="cuda")
            fns.append(lambda cx=cx, co=co, cst=cst, cw=cw, qsl=qsl, cidx=cidx, hinit=hinit:
                       tecoops.causal_conv1d_fn_torch(co.t(), cst, cx.t(), cw, qsl, cidx, hinit,
                                                      -1))
        ops["causal_conv1d_tm"] = (fns, dict(bytes=2 * T * C * 2 + 4 * C * 2 + B * 3 * C * 2))

    if want("rotary"):
        rng = np.random.default_rng(1004)  # each op has its own seed
        # rotary (in place)
        ws = 2 * (8192 * 40 * 128) * 2
        pos = torch.from_numpy((np.arange(8192) % 2048).astype(np.int64)).cuda()
        fns = []
        for _ in range(copies_for(ws)):
            q = seeded_bits(rng, (8192, 32, 128))
            k = seeded_bits(rng, (8192, 8, 128))
            fns.append(lambda q=q, k=k, pos=pos: tecoops.rotary_embedding(pos, q, k, 128))
        ops["rotary"] = (fns, dict(bytes=2 * (8192 * 40 * 128) * 2 + 8192 * 8))

    if want("rotary_cache"):
        rng = np.random.default_rng(1005)  # each op has its own seed
        # fused decode step: rotary on q (in place) and k, k and v into the
        # paged cache (rotary + reshape_and_cache configs as one pass)
        T, H, Hkv, D, NB, BS = 8192, 32, 8, 128, 1024, 16
        ws = 2 * T * H * D * 2 + 4 * T * Hkv * D * 2
        pos = torch.from_numpy((np.arange(T) % 2048).astype(np.int64)).cuda()
        slots = torch.from_numpy(rng.permutation(NB * BS)[:T].astype(np.int64)).cuda()
        fns = []
        for _ in range(copies_for(ws)):
            q = seeded_bits(rng, (T, H, D))
            k = seeded_bits(rng, (T, Hkv, D))
            v = seeded_bits(rng, (T, Hkv, D))
            kc = torch.zeros((NB, Hkv, BS, D), dtype=torch.float16, device="cuda")
            vc = torch.zeros_like(kc)
            fns.append(lambda q=q, k=k, v=v, kc=kc, vc=vc, pos=pos, slots=slots:
                       tecoops.rotary_reshape_and_cache(pos, q, k, v, slots, kc, vc, D))
        ops["rotary_cache"] = (fns, dict(bytes=ws + 2 * T * 8))

    if want("gemv_f16_b1", "gemv_f16_b8", "gemv_i8_b1", "gemv_i8_b8"):
        rng = np.random.default_rng(1006)  # each op has its own seed
        # GEMV: W fp16 / int8 [14336, 4096]
        N, K = 14336, 4096
        Ws = [seeded_bits(rng, (N, K), scale=0.02) for _ in range(copies_for(N * K * 2))]
        Wqs = [torch.from_numpy(rng.integers(-127, 128, (N, K), dtype=np.int8)).cuda()
               for _ in range(copies_for(N * K))]
        sc = seeded_bits(rng, (N,), "uniform", lo=0.001, hi=0.01)
        for b in (1, 8):
            xv = seeded_bits(rng, (b, K))
            yv = torch.empty((b, N), dtype=torch.float16, device="cuda")
            ops[f"gemv_f16_b{b}"] = ([lambda W=W, xv=xv, yv=yv: tecoops.gemv(W, xv, yv) for W in Ws],
                                     dict(bytes=N * K * 2 + b * K * 2 + b * N * 2))
            ops[f"gemv_i8_b{b}"] = ([lambda Wq=Wq, xv=xv, yv=yv: tecoops.gemv_int8(Wq, sc, xv, yv)
                                     for Wq in Wqs],
                                    dict(bytes=N * K + N * 2 + b * K * 2 + b * N * 2))

    if want("fa_prefill"):
        rng = np.random.default_rng(1007)  # each op has its own seed
        # flash attention prefill: identity block tables over 4 x 256 blocks
        nbp = FA_S // 16
        bt = torch.arange(FA_B * nbp, dtype=torch.int32, device="cuda").view(FA_B, nbp)
        cu = torch.arange(0, FA_B + 1, dtype=torch.int32, device="cuda") * FA_S
        sk = torch.full((FA_B,), FA_S, dtype=torch.int32, device="cuda")
        q_bytes = FA_B * FA_S * FA_H * FA_D * 2
        kv_bytes = 2 * FA_B * FA_S * FA_HKV * FA_D * 2
        fns = []
        for _ in range(copies_for(2 * q_bytes + kv_bytes)):
            fq = seeded_bits(rng, (FA_B * FA_S, FA_H, FA_D), dtype="bf16")
            fk = seeded_bits(rng, (FA_B * nbp, FA_HKV, 16, FA_D), dtype="bf16")
            fv = seeded_bits(rng, (FA_B * nbp, FA_HKV, 16, FA_D), dtype="bf16")
            fo = torch.empty_like(fq)
            fns.append(lambda fq=fq, fk=fk, fv=fv, fo=fo, cu=cu, sk=sk, bt=bt:
                       tecoops.flash_attn_varlen_func(fq, fk, fv, FA_S, cu, FA_S, None, sk, scale,
                                                      True, None, bt, False, fo))
        ops["fa_prefill"] = (fns, dict(flops=FA_PREFILL_FLOP, bytes=2 * q_bytes + kv_bytes))

    if want("fa_decode"):
        rng = np.random.default_rng(1008)  # each op has its own seed
        # flash attention decode: B=64, seeded lengths U{512..8192}, shuffled blocks
        DB = 64
        lens = rng.integers(512, 8193, DB)
        nblk = (lens + 15) // 16
        tot = int(nblk.sum())
        perm = rng.permutation(tot)
        btd = np.zeros((DB, 512), np.int32)
        i = 0
        for b in range(DB):
            btd[b, :nblk[b]] = perm[i:i + nblk[b]]
            i += nblk[b]
        dq = seeded_bits(rng, (DB, FA_H, FA_D), dtype="bf16")
        dk = seeded_bits(rng, (tot, FA_HKV, 16, FA_D), dtype="bf16")
        dv = seeded_bits(rng, (tot, FA_HKV, 16, FA_D), dtype="bf16")
        do = torch.empty_like(dq)
        dbt = torch.from_numpy(btd).cuda()
        dcu = torch.arange(0, DB + 1, dtype=torch.int32, device="cuda")
        dsk = torch.from_numpy(lens.astype(np.int32)).cuda()
        sum_l = int(lens.sum())
        ops["fa_decode"] = (
            [lambda: tecoops.flash_attn_varlen_func(dq, dk, dv, 1, dcu, int(lens.max()), None, dsk,
                                                    scale, True, None, dbt, False, do)],
            dict(bytes=4096 * sum_l + 2 * dq.numel() * 2 + DB * 512 * 4,
                 flops=4 * FA_H * FA_D * sum_l, sum_kv=sum_l))
    return ops


def cpu_baseline(threads, budget_s=20.0):
    """Times the CPU oracle (C restatement of the reference's CPU paths) on the
    FA prefill config, one (batch, kv-group) slice at a time (4 query heads x
    4096 rows, causal): all 32 slices of the config when they fit in about
    `budget_s` seconds, else as many as do.  Reported as TFLOP/s."""
    from oracle import oracle as orc
    if threads > 0:
        orc.set_threads(threads)
    used = orc.get_threads()
    rng = np.random.default_rng(7)
    S, D, Hkv, H = FA_S, FA_D, FA_HKV, FA_H
    nbp = S // 16
    G = H // Hkv
    q = orc.from_float(rng.standard_normal((S, H, D), dtype=np.float32), orc.BF16)
    kc = orc.from_float(rng.standard_normal((nbp, Hkv, 16, D), dtype=np.float32), orc.BF16)
    vc = orc.from_float(rng.standard_normal((nbp, Hkv, 16, D), dtype=np.float32), orc.BF16)
    bt = np.arange(nbp, dtype=np.int32)[None]
    slice_flop = 4 * G * D * S * (S + 1) // 2
    done, t_total = 0, 0.0
    for _ in range(FA_B):           # each batch of the config has the same shape
        for g in range(Hkv):
            t0 = time.perf_counter()
            orc.flash_attention(q, kc, vc, bt, [S], [S], dtype=orc.BF16, b_only=0,
                                h_begin=g * G, h_end=(g + 1) * G)
            t_total += time.perf_counter() - t0
            done += 1
            if t_total >= budget_s:
                break
        if t_total >= budget_s:
            break
    total = FA_B * Hkv
    return {"value": done * slice_flop / t_total / 1e12, "unit": "TFLOP/s", "cores": used,
            "kind": "port",
            "sample": f"oracle flash_attention over {done} of the {total} (batch, kv-group) slices "
                      f"of the prefill config ({G} heads x {S} rows each, causal, bf16 in / fp32 "
                      f"math) in {t_total:.2f} s"
                      + ("" if done == total else
                         f"; the full config is {total / done:.1f}x this work"),
            "cpu_model": cpu_model()}


def cpu_single_thread(budget_s=5.0):
    """The FA prefill slice timing of cpu_baseline on one host thread (the
    reference harness's cpuCompute is single-threaded): as many (batch,
    kv-group) slices as fit in about `budget_s` seconds, at least one."""
    from oracle import oracle as orc
    prev = orc.get_threads()
    orc.set_threads(1)
    try:
        rng = np.random.default_rng(7)
        S, D, Hkv, H = FA_S, FA_D, FA_HKV, FA_H
        nbp = S // 16
        G = H // Hkv
        q = orc.from_float(rng.standard_normal((S, H, D), dtype=np.float32), orc.BF16)
        kc = orc.from_float(rng.standard_normal((nbp, Hkv, 16, D), dtype=np.float32), orc.BF16)
        vc = orc.from_float(rng.standard_normal((nbp, Hkv, 16, D), dtype=np.float32), orc.BF16)
        bt = np.arange(nbp, dtype=np.int32)[None]
        slice_flop = 4 * G * D * S * (S + 1) // 2
        done, t_total = 0, 0.0
        while done < FA_B * Hkv:
            g = done % Hkv
            t0 = time.perf_counter()
            orc.flash_attention(q, kc, vc, bt, [S], [S], dtype=orc.BF16, b_only=0,
                                h_begin=g * G, h_end=(g + 1) * G)
            t_total += time.perf_counter() - t0
            done += 1
            if t_total >= budget_s:
                break
    finally:
        orc.set_threads(prev)
    return {"value": done * slice_flop / t_total / 1e12, "unit": "TFLOP/s", "cores": 1,
            "sample": f"{done} (batch, kv-group) slice(s) of the prefill config in {t_total:.2f} s"}


def cpu_ops(threads):
    """Times the CPU oracle on every other op at its full BASELINE config, on
    all `threads` host threads (median of 3 runs; FA decode once) and on one
    thread (one run each), the way the reference harness's cpuCompute loops
    run (single-threaded: test/zoo/teco/rms_norm/rms_norm.cpp:195-234,
    reshape_and_cache/reshape_and_cache.cpp:116-148).  A reported baseline
    beside the GPU figures, not a target."""
    from oracle import oracle as orc
    if threads > 0:
        orc.set_threads(threads)
    used = orc.get_threads()
    all_cores = _cpu_ops_once(orc, runs=3)
    orc.set_threads(1)
    try:
        one = _cpu_ops_once(orc, runs=1)
    finally:
        orc.set_threads(used)
    return {"cores": used, "unit": "ms", "kind": "port",
            "sample": "full BASELINE config of each op; all cores: median of 3 runs (fa_decode 1 "
                      "run); one thread: 1 run",
            "ms": {k: round(v, 3) for k, v in all_cores.items()},
            "ms_1thread": {k: round(v, 3) for k, v in one.items()}}


def _cpu_ops_once(orc, runs):
    """{op: ms} of the oracle on every op but FA prefill at its full config,
    on the oracle's current thread count; median of `runs` runs (FA decode
    always one)."""
    rng = np.random.default_rng(11)

    # Inputs repeat a 1 Mi-element pool of seeded values, uniform on (-1, 1)
    # (the oracle's time does not depend on the values); this keeps the
    # set-up of the 270 M-element decode caches to a copy.
    pool = rng.random(1 << 20, dtype=np.float32) * 2.0 - 1.0
    pools = {orc.HALF: orc.from_float(pool, orc.HALF), orc.BF16: orc.from_float(pool, orc.BF16)}

    def bits(shape, scale=1.0, dt=None):
        dt = dt if dt is not None else orc.HALF
        if scale == 1.0:
            return np.resize(pools[dt], shape)
        return orc.from_float(np.resize(pool, shape) * np.float32(scale), dt)

    def timed(fn, runs=runs):
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return 1e3 * sorted(ts)[len(ts) // 2]

    res = {}
    x = bits((4096, 4096))
    w = orc.from_float(rng.uniform(0.5, 1.5, 4096).astype(np.float32))
    res["rms_norm"] = timed(lambda: orc.rms_norm(x, w, eps=1e-6))
    T, Hkv, D, NB, BS = 8192, 8, 128, 1024, 16
    key, val = bits((T, Hkv, D)), bits((T, Hkv, D))
    slots = rng.permutation(NB * BS)[:T].astype(np.int64)
    kc = np.zeros((NB, Hkv, BS, D), np.uint16)
    vc = np.zeros_like(kc)
    res["reshape_and_cache"] = timed(lambda: orc.reshape_and_cache(key, val, slots, kc, vc))
    cx = bits((8, 4096, 2048))
    cw, cb = bits((4096, 4), 0.5), bits((4096,))
    cst = np.zeros((8, 3, 4096), np.uint16)
    res["causal_conv1d"] = timed(lambda: orc.causal_conv1d(cx, cw, bias=cb, conv_state=cst))
    q, k = bits((8192, 32, 128)), bits((8192, 8, 128))
    pos = (np.arange(8192) % 2048).astype(np.int64)
    res["rotary"] = timed(lambda: orc.rotary_embedding(pos, q, k))
    N, K = 14336, 4096
    W = bits((N, K), 0.02)
    Wq = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sc = orc.from_float(rng.uniform(0.001, 0.01, N).astype(np.float32))
    for b in (1, 8):
        xv = bits((b, K))
        res[f"gemv_f16_b{b}"] = timed(lambda: orc.gemv(W, xv))
        res[f"gemv_i8_b{b}"] = timed(lambda: orc.gemv_int8(Wq, sc, xv))
    # decode: the bench's lengths (seed 1008), contiguous blocks
    lens = np.random.default_rng(1008).integers(512, 8193, 64)
    nblk = (lens + 15) // 16
    bt = np.zeros((64, 512), np.int32)
    off = np.concatenate([[0], np.cumsum(nblk)])
    for b in range(64):
        bt[b, :nblk[b]] = np.arange(off[b], off[b + 1])
    dk = bits((int(off[-1]), FA_HKV, 16, FA_D), dt=orc.BF16)
    dv = bits((int(off[-1]), FA_HKV, 16, FA_D), dt=orc.BF16)
    dq = bits((64, FA_H, FA_D), dt=orc.BF16)
    res["fa_decode"] = timed(lambda: orc.flash_attention(dq, dk, dv, bt, np.ones(64, np.int32),
                                                         lens.astype(np.int32), dtype=orc.BF16),
                             runs=1)
    return res


# ----------------------------------------------------------- reference cases

def _case_tensor(t, gen):
    """A device tensor for one input of a prototxt case: the case's own values
    where it gives them (lengths, offsets, indices), else seeded data of its
    shape, dtype and range (timing does not depend on the values; integer
    ranges, e.g. slot ids in [-1, 1024), are kept)."""
    import torch
    dt = {"DTYPE_HALF": torch.float16, "DTYPE_FLOAT": torch.float32,
          "DTYPE_INT32": torch.int32, "DTYPE_INT64": torch.int64}[t["dtype"]]
    shape = t["shape"]["dims"]
    if "prev_value" in t:
        vals = t["prev_value"].get("value_i", t["prev_value"].get("value_f"))
        return torch.tensor(vals, dtype=dt, device="cuda").reshape(shape)
    r = t.get("random_data", {})
    lo, hi = float(r.get("lower_bound", -1.0)), float(r.get("upper_bound", 1.0))
    u = torch.rand(shape, generator=gen, device="cuda") * (hi - lo) + lo
    return u.floor().to(dt) if not dt.is_floating_point else u.to(dt)


def time_cases(repeat=100, warm=10):
    """The reference's own op test cases (test/zoo/teco/<op>/test_case/
    *.prototxt, stored as data in tests/golden/prototxt_cases.json), each run
    through the C entry point the reference harness calls and timed the way
    the harness reports them (test/src/suite/executor.cpp:228-277): `warm`
    launches, then `repeat` launches each between its own pair of HIP events,
    sorted, the fastest and slowest tenth dropped, the rest averaged.  GB/s
    and TFLOP/s divide the harness's theory_io / theory_ops of each op
    (executor.cpp:893-913 and the ops' getTheoryIoSize / getTheoryOps:
    rms_norm.cpp:88-115, reshape_and_cache.cpp:103-114, causal_conv1d.cpp:
    119-135, flash_attention.cpp:106-114, memset.cpp:62-67).  The harness
    times kernels with its profiler; events also count each launch's own
    overhead (~2-5 us), so these small cases read slower than their kernels."""
    import ctypes
    import torch
    import tecoops
    from tecoops import _lib
    with open(os.path.join(REPO, "tests", "golden", "prototxt_cases.json")) as f:
        cases = json.load(f)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2024)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    out = []
    for op in ("rms_norm", "reshape_and_cache", "flash_attention", "causal_conv1d", "memset"):
        for c in cases[op]:
            ins = {t["id"]: _case_tensor(t, gen) for t in c["input"]}
            prm = next(iter(c.get("tecokernel_param", {}).values()), {})
            nbytes = lambda t: t.numel() * t.element_size()
            if op == "rms_norm":
                x, w, res = ins["input"], ins["weight"], ins.get("residual")
                N, D = x.shape
                y, ro = torch.empty_like(x), (torch.empty_like(x) if res is not None else None)
                eps = float(prm.get("eps", 1e-6))
                fn = lambda: tecoops.rms_norm(x, w, res, y, ro, eps)
                io = N * D * 2 + D * 2 + N * D * 2 + (2 * N * D * 2 if res is not None else 0)
                ops = N * D * 4 + (N * D if res is not None else 0)
            elif op == "reshape_and_cache":
                k, v, sl = ins["key"], ins["value"], ins["slot_mapping"]
                oc = {t["id"]: t["shape"]["dims"] for t in c["output"]}
                kc = torch.zeros(oc["key_cache"], dtype=torch.float16, device="cuda")
                vc = torch.zeros_like(kc)
                fn = lambda: tecoops.reshape_and_cache(k, v, sl, kc, vc)
                kv = k.numel() * 2
                io, ops = kv * 2 + sl.numel() * 8 + kv * 2, 0
            elif op == "flash_attention":
                bt = (ins["blockTable"] % ins["kCache"].shape[0]).to(torch.int32)
                q, kc, vc = ins["qData"], ins["kCache"], ins["vCache"]
                ql, kl = ins["q_seq_lens"].to(torch.int32), ins["kv_seq_lens"].to(torch.int32)
                o = torch.zeros_like(q)
                mq, mk = int(prm.get("max_seqlen_q", 0)), int(prm.get("max_seqlen_k", 0))
                d = lambda t, code: tecoops._Desc(t, code)
                with d(bt, _lib.DATA_INT32) as btd, d(q, _lib.DATA_HALF) as qd, \
                        d(kc, _lib.DATA_HALF) as kd, d(vc, _lib.DATA_HALF) as vd, \
                        d(o, _lib.DATA_HALF) as od:
                    args = (mq, mk, bt.shape[1], P(ql), P(kl), btd, P(bt), qd, P(q), kd, P(kc), vd,
                            P(vc), od, P(o), None)
                    fn = lambda args=args: _lib.call("tecoopsFlashAttention",
                                                     tecoops._handle(o.device), *args)
                    out.append(_time_case(c, op, fn, repeat, warm,
                                          sum(nbytes(t) for t in (bt, q, kc, vc, ql, kl, o)),
                                          4 * q.shape[0] * int(kl.sum()) * q.shape[2] * q.shape[1]))
                continue
            elif op == "causal_conv1d":
                x, w, st = ins["x"], ins["weight"], ins["convState"]
                qsl, cidx = ins["query_start_loc"], ins["cache_indices"]
                hin = ins["has_initial_state"].to(torch.int8)
                total, dim = x.shape
                width = w.shape[0]
                y = torch.empty_like(x)
                fn = lambda: _lib.call(
                    "tecoopsCausalConv1d", tecoops._handle(x.device), qsl.numel() - 1, total, dim,
                    width, int(prm["conv_state_stride"]), int(prm["x_seq_stride"]),
                    int(prm["out_seq_stride"]), int(prm["pad_slot_id"]), int(prm["api_mode"]),
                    int(prm["act_mode"]), P(x), P(st), P(w), P(y), P(qsl), P(cidx), P(hin))
                batch = qsl.numel() - 1
                io = total * dim * 2 + width * dim * 2 + batch * (width - 1) * dim * 2 * 2 + total * dim * 2
                ops = total * dim * 20
            else:  # memset
                x = ins["x"]
                size, value = int(prm["size"]), int(prm["value"])
                fn = lambda: _lib.call("tecoopsMemset", tecoops._handle(x.device), P(x), value, size)
                io, ops = size, x.numel()
            out.append(_time_case(c, op, fn, repeat, warm, io, ops))
    return out


def _time_case(c, op, fn, repeat, warm, io, ops):
    import torch
    for _ in range(warm):
        fn()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(2 * repeat)]
    for i in range(repeat):
        marks[2 * i].record()
        fn()
        marks[2 * i + 1].record()
    torch.cuda.synchronize()
    t = sorted(marks[2 * i].elapsed_time(marks[2 * i + 1]) * 1e3 for i in range(repeat))
    cut = repeat // 10
    us = sum(t[cut:repeat - cut]) / (repeat - 2 * cut)
    r = {"case": c["file"].split("test/zoo/teco/")[-1], "op": op, "us": round(us, 3),
         "theory_io": int(io), "gbs": round(io / us / 1e3, 2)}
    if ops:
        r.update(theory_ops=int(ops), tflops=round(ops / us / 1e6, 4))
    return r


def cpu_model():
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor()


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only (no multi-GPU path); "
                                   "run with --gpus 1"}))
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)
    if args.cases:
        print(json.dumps({"metric": "reference prototxt cases: trimmed-mean us of 100 launches "
                                    "(the harness statistic), GB/s and TFLOP/s of its theory_io / "
                                    "theory_ops", "n_gpus": 1, "cases": time_cases()}), flush=True)
        return
    keep = set(args.ops.split(",")) if args.ops else None
    ops = build_ops(keep)
    if keep:
        ops = {k: v for k, v in ops.items() if k in keep}
    # Per op: warm-up, then the timed region of K launches.  The warm-up runs
    # at least W launches and at least WARM_S seconds of the op's own work
    # right before its timed region, so the GPU clock has settled under that
    # load (a cold start measured FA prefill 13 % slow).  Launches of one op
    # run back to back (rotating over its input copies) between one pair of
    # events on the stream they are enqueued on, so the average per launch
    # excludes host overhead.
    ev = {}
    med = {}
    wall = 0.0
    for n, (fns, _) in ops.items():
        i, t_w = 0, time.perf_counter()
        while i < args.warmup or time.perf_counter() - t_w < WARM_S:
            for _ in range(10):
                fns[i % len(fns)]()
                i += 1
            torch.cuda.synchronize()
        # ten more warm-up launches left in flight: the timed launches queue
        # behind them, so the GPU never waits for the host between the two
        for _ in range(10):
            fns[i % len(fns)]()
            i += 1
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        a.record()
        for j in range(args.steps):  # the rotation continues where the warm-up left it
            fns[(i + j) % len(fns)]()
        b.record()
        torch.cuda.synchronize()
        wall += time.perf_counter() - t0
        ev[n] = (a, b)
        # 20 more launches, each between its own pair of events: the median
        i += args.steps
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(21)]
        marks[0].record()
        for j in range(20):
            fns[(i + j) % len(fns)]()
            marks[j + 1].record()
        torch.cuda.synchronize()
        med[n] = float(np.median([marks[j].elapsed_time(marks[j + 1]) for j in range(20)])) * 1e3

    report = {}
    for n, (fns, work) in ops.items():
        us = 1e3 * ev[n][0].elapsed_time(ev[n][1]) / args.steps
        r = {"us": round(us, 3), "us_median20": round(med[n], 3), "rotating_copies": len(fns)}
        if "flops" in work and n == "fa_prefill":
            tf = work["flops"] / (us * 1e-6) / 1e12
            r.update(tflops=round(tf, 2), frac=round(tf / MFMA_BF16_PEAK_TFLOPS, 4), bound="mfma")
        else:
            gbs = work["bytes"] / (us * 1e-6) / 1e9
            r.update(gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4), bound="hbm")
        r["algorithmic_bytes"] = work["bytes"]
        if "flops" in work:
            r["algorithmic_flops"] = work["flops"]
        if "sum_kv" in work:
            r["sum_kv_len"] = work["sum_kv"]
        report[n] = r

    dom = max(report, key=lambda n: report[n]["us"])
    d = report[dom]
    if d["bound"] == "mfma":
        roof = {"bound": "mfma", "achieved": d["tflops"], "peak": MFMA_BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": d["frac"]}
    else:
        roof = {"bound": "hbm", "achieved": d["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": d["frac"]}
    roof["kernel"] = dom
    roof["traffic"] = traffic_for(dom)

    value = report["fa_prefill"]["tflops"] if "fa_prefill" in report else None
    line = {
        "metric": "per-op µs + HBM GB/s vs peak; flash-attn prefill TFLOP/s vs MFMA peak",
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 (flash attention); fp16 / int8-weight (other ops)",
        "data": "synthetic seeded inputs of the BASELINE.json shapes, resident in HBM",
        "config": {
            "workload": "teco-ops LLM-inference operator path, one pass of every BASELINE.json "
                        "config per step (value: flash-attention prefill bf16 B4 H32 Hkv8 "
                        "S4096 D128 causal)",
            "fa_prefill": "q [4,32,4096,128], kv [4,8,4096,128], causal, scale 1/sqrt(128)",
            "fa_decode": "B=64, H=32, Hkv=8, D=128, block 16, kv_len seeded U{512..8192}",
            "rotating_input_copies": "each op cycles through copies of its inputs totalling "
                                     ">= 1 GiB (4x the MALL) so no launch reads cached data",
        },
        "ops": report,
        "roofline": roof,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_threads)
        line["cpu_baseline"]["single_thread"] = cpu_single_thread()
        line["cpu_ops"] = cpu_ops(args.cpu_threads)
    print(json.dumps(line), flush=True)


def traffic_for(kernel):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (profiles/traffic.json: FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the
    copy-kernel calibration), or None when not measured."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(kernel, {}).get("hbm_bytes")
    except (OSError, ValueError):
        return None


if __name__ == "__main__":
    main()
