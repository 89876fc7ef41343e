// bench_probes.hip — measurements of the box itself, beside bench.py: what
// plain kernels reach at the BASELINE byte counts, how the int8 GEMV's
// weight-stream shape behaves, and the issue rates of the gfx950 SIMD that
// bound the flash-attention prefill kernel.  No tecoops code is involved;
// these are the ceilings the per-op figures are compared with.
//
//   ./bench_probes ceilings   best plain read-only / copy kernel (no math) at
//                             each BASELINE byte count, over a sweep of launch
//                             shapes; back-to-back launches between one event
//                             pair, inputs rotated over >= 2 GiB (bench.py's
//                             timing)
//   ./bench_probes wstream    read-only streams with the int8 batch-8 GEMV's
//                             layout ([14336, 4096] int8, 4 rows per wave),
//                             CPL 16-byte loads in flight per lane
//   ./bench_probes convtm     the token-major causal_conv1d's loads and stores
//                             (window rows included) without its math
//   ./bench_probes issue      v_exp_f32 / v_fma_f32 issue cost per SIMD with
//                             1-4 waves per SIMD, and MFMA with exp in one wave
//   ./bench_probes lds        LDS read bandwidth per CU (ds_read_b128 / b64)
//                             and a 32x32x16 MFMA stream fed from LDS
//
// Cycle counts come from s_memtime (the shader clock) of wave 0..15 of
// workgroup 0; times from HIP events.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <vector>

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

#define CHECK(x)                                                                   \
    do {                                                                           \
        hipError_t e_ = (x);                                                       \
        if (e_ != hipSuccess) {                                                    \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x,              \
                    hipGetErrorString(e_));                                        \
            exit(1);                                                               \
        }                                                                          \
    } while (0)

// ------------------------------------------------------------ ceilings

// Thread t of workgroup g loads U chunks g*blockDim*U + u*blockDim + t (the
// last chunk for indices past n), all before using any.
template <int U, bool NT>
__global__ void read_kernel(const u32x4 *__restrict__ a, unsigned *out, long n) {
    const long base = static_cast<long>(blockIdx.x) * blockDim.x * U + threadIdx.x;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        long i = base + static_cast<long>(u) * blockDim.x;
        i = i < n ? i : n - 1;
        v[u] = NT ? __builtin_nontemporal_load(a + i) : a[i];
    }
    unsigned s = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) s ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (s == 0x9e3779b9u) out[0] = s;  // keeps the loads; never true for the fill
}

template <int U, bool NT>
__global__ void copy_kernel(const u32x4 *__restrict__ a, u32x4 *__restrict__ b, long n) {
    const long base = static_cast<long>(blockIdx.x) * blockDim.x * U + threadIdx.x;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        long i = base + static_cast<long>(u) * blockDim.x;
        i = i < n ? i : n - 1;
        v[u] = NT ? __builtin_nontemporal_load(a + i) : a[i];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const long i = base + static_cast<long>(u) * blockDim.x;
        if (i < n) {
            if (NT)
                __builtin_nontemporal_store(v[u], b + i);
            else
                b[i] = v[u];
        }
    }
}

template <int U, bool NT>
void launch_plain(bool copy, long grid, int threads, const u32x4 *a, u32x4 *b, unsigned *out,
                  long n) {
    if (copy)
        hipLaunchKernelGGL((copy_kernel<U, NT>), dim3(grid), dim3(threads), 0, 0, a, b, n);
    else
        hipLaunchKernelGGL((read_kernel<U, NT>), dim3(grid), dim3(threads), 0, 0, a, out, n);
}

template <bool NT>
void launch_u(int U, bool copy, long grid, int threads, const u32x4 *a, u32x4 *b, unsigned *out,
              long n) {
    switch (U) {
        case 1: launch_plain<1, NT>(copy, grid, threads, a, b, out, n); break;
        case 2: launch_plain<2, NT>(copy, grid, threads, a, b, out, n); break;
        case 4: launch_plain<4, NT>(copy, grid, threads, a, b, out, n); break;
        case 8: launch_plain<8, NT>(copy, grid, threads, a, b, out, n); break;
        default: launch_plain<16, NT>(copy, grid, threads, a, b, out, n); break;
    }
}

// Mean microseconds of `iters` back-to-back launches after `warm` more.
template <typename F>
double time_launches(F launch, int rotate, int warm = 60, int iters = 50) {
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    for (int i = 0; i < warm; ++i) launch(i % rotate);
    CHECK(hipEventRecord(e0));
    for (int i = 0; i < iters; ++i) launch((warm + i) % rotate);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    CHECK(hipGetLastError());
    CHECK(hipEventDestroy(e0));
    CHECK(hipEventDestroy(e1));
    return ms * 1000.0 / iters;
}

void ceilings() {
    const size_t pool_bytes = size_t(3) << 30;
    char *pool;
    CHECK(hipMalloc(&pool, pool_bytes));
    CHECK(hipMemset(pool, 1, pool_bytes));
    unsigned *out;
    CHECK(hipMalloc(&out, 4));
    struct Op {
        const char *name;
        long bytes;  // bytes read (copies also write as many)
        bool copy;
    };
    const Op ops[] = {
        {"gemv_i8_b8: read 59,043,840 B", 59043840, false},
        {"gemv_i8_b1: read 58,785,792 B", 58785792, false},
        {"gemv_f16_b8: read 117,735,424 B", 117735424, false},
        {"gemv_f16_b1: read 117,477,376 B", 117477376, false},
        {"rms_norm / reshape_and_cache: copy 2 x 33,554,432 B", 33554432, true},
        {"rotary: copy 2 x 83,886,080 B", 83886080, true},
        {"rotary_cache: copy 2 x 100,663,296 B", 100663296, true},
        {"causal_conv1d: copy 2 x 134,217,728 B", 134217728, true},
    };
    printf("%-52s %9s %8s %6s  %s\n", "byte count", "best us", "TB/s", "frac", "launch shape");
    for (const Op &op : ops) {
        const long n = op.bytes / 16;
        const size_t span = op.copy ? 2 * op.bytes : op.bytes;
        const int rotate = static_cast<int>((size_t(2) << 30) / span) + 1;
        double best = 1e30;
        char cfg[64] = "";
        for (int threads : {256, 512, 1024})
            for (int U : {1, 2, 4, 8, 16})
                for (int nt = 0; nt < 2; ++nt) {
                    const long grid = (n + static_cast<long>(threads) * U - 1) / (static_cast<long>(threads) * U);
                    auto launch = [&](int c) {
                        // copy c at offset c * span within the pool, 4 KiB aligned
                        size_t off = (size_t(c) * span) % (pool_bytes - span);
                        off &= ~size_t(4095);
                        const u32x4 *a = reinterpret_cast<const u32x4 *>(pool + off);
                        u32x4 *b = reinterpret_cast<u32x4 *>(pool + off + op.bytes);
                        if (nt)
                            launch_u<true>(U, op.copy, grid, threads, a, b, out, n);
                        else
                            launch_u<false>(U, op.copy, grid, threads, a, b, out, n);
                    };
                    const double us = time_launches(launch, rotate);
                    if (us < best) {
                        best = us;
                        snprintf(cfg, sizeof cfg, "%d threads, %d x 16 B per thread, %s", threads, U,
                                 nt ? "non-temporal" : "plain");
                    }
                }
        const double total = op.copy ? 2.0 * op.bytes : static_cast<double>(op.bytes);
        printf("%-52s %9.2f %8.2f %6.3f  %s\n", op.name, best, total / best / 1e6,
               total / best / 1e6 / 8.0, cfg);
        fflush(stdout);
    }
    CHECK(hipFree(pool));
    CHECK(hipFree(out));
}

// ------------------------------------------------------------- wstream

// Wave w of workgroup g reads rows [4*(g*NW + w), +4) of an int8 [N, 256 x
// 16 B] matrix.  PAT 0: lane 4*blk + r reads chunk blk of each 16-chunk run
// of row r (the GEMV's 4x4x4 layout: an instruction covers four 256-byte row
// segments); PAT 1: an instruction reads 1 KiB of one row.  ROT: each wave
// starts at a different step.  CPL steps (16 bytes per lane) in flight.
template <int NW, int CPL, int PAT, bool ROT>
__global__ void __launch_bounds__(NW * 64) wstream_kernel(const u32x4 *__restrict__ W,
                                                          unsigned *out, int N, int kw) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * NW + wave) * 4;
    if (n0 >= N) return;
    const int nsteps = kw * 4 / 64;
    const u32x4 *base = PAT == 0 ? W + static_cast<long>(n0 + (lane & 3)) * kw + (lane >> 2)
                                 : W + static_cast<long>(n0) * kw + lane;
    const int rot = ROT ? (blockIdx.x * NW + wave) % nsteps : 0;
    auto addr = [&](int i) {
        int s = i + rot;
        s = s < nsteps ? s : s - nsteps;
        return PAT == 0 ? base + 16 * s : base + 64 * s;
    };
    u32x4 q[CPL];
    unsigned acc = 0;
#pragma unroll
    for (int u = 0; u < CPL; ++u) q[u] = __builtin_nontemporal_load(addr(u));
    for (int i = 0; i < nsteps; i += CPL) {
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            acc ^= q[u].x ^ q[u].y ^ q[u].z ^ q[u].w;
            if (i + CPL + u < nsteps) q[u] = __builtin_nontemporal_load(addr(i + CPL + u));
        }
    }
    if (acc == 0x9e3779b9u) out[0] = acc;
}

void wstream() {
    const int N = 14336, K = 4096, rotate = 20;
    const int kw = K / 16;
    const size_t wb = size_t(N) * K;
    char *W;
    CHECK(hipMalloc(&W, wb * rotate));
    CHECK(hipMemset(W, 3, wb * rotate));
    unsigned *out;
    CHECK(hipMalloc(&out, 4));
    printf("int8 [14336, 4096] (58.7 MB) read in the GEMV's per-wave row layout\n");
#define WS(NW, CPL, PAT, ROT)                                                                     \
    {                                                                                             \
        const int grid = (N / 4 + NW - 1) / NW;                                                   \
        const double us = time_launches(                                                          \
            [&](int c) {                                                                          \
                hipLaunchKernelGGL((wstream_kernel<NW, CPL, PAT, ROT>), dim3(grid), dim3(NW * 64), \
                                   0, 0, reinterpret_cast<const u32x4 *>(W + c * wb), out, N, kw); \
            },                                                                                    \
            rotate);                                                                              \
        printf("  %2d waves/workgroup, %2d loads in flight per lane, %-26s %-16s %6.2f us\n", NW, \
               CPL, PAT ? "1 KiB of one row / instr," : "4 rows x 256 B / instr,",              \
               ROT ? "staggered starts" : "same start", us);                                      \
        fflush(stdout);                                                                           \
    }
    WS(14, 1, 0, true) WS(14, 2, 0, true) WS(14, 4, 0, true) WS(14, 8, 0, true) WS(14, 16, 0, true)
    WS(14, 2, 0, false) WS(14, 2, 1, true) WS(14, 8, 1, true) WS(16, 2, 0, true) WS(8, 2, 0, true)
    WS(8, 16, 1, true) WS(4, 16, 1, false)
#undef WS
    CHECK(hipFree(W));
    CHECK(hipFree(out));
}

// ------------------------------------------------------------- convtm

// The token-major causal_conv1d's memory pattern (conv1d_tokens_kernel at the
// BASELINE shape: x and out [16384 tokens, 4096] fp16) without its math.
// Work item (chunk, slab) = 8 tokens x 2048 channels, dealt to the XCDs in
// contiguous ranges; lane: 8 channels (16 bytes) of each row.  WIN: the lane
// loads the W-1 = 3 rows before its chunk too (plain, as the chunk's last 3
// rows, which the next chunk re-reads; the other 5 non-temporal) and stores
// row j as the XOR of rows j .. j+3; else it loads its 8 rows (non-temporal)
// and stores them.
template <bool WIN>
__global__ void __launch_bounds__(256) convtm_kernel(const u32x4 *__restrict__ x,
                                                     u32x4 *__restrict__ out, long nitems,
                                                     long per_xcd) {
    constexpr int CH = 8, WM1 = 3, ROWV = 512;  // 16-byte vectors per row
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (item >= nitems) return;
    const long t0 = (item / 2) * CH;
    const int dv = static_cast<int>(item % 2) * 256 + wave * 64 + lane;
    if (WIN) {
        u32x4 raw[WM1 + CH];
#pragma unroll
        for (int j = 0; j < WM1 + CH; ++j) {
            long row = t0 - WM1 + j;
            row = row < 0 ? 0 : row;
            const u32x4 *p = x + row * ROWV + dv;
            raw[j] = (j >= WM1 && j < CH) ? __builtin_nontemporal_load(p) : *p;
        }
#pragma unroll
        for (int j = 0; j < CH; ++j)
            __builtin_nontemporal_store(raw[j] ^ raw[j + 1] ^ raw[j + 2] ^ raw[j + 3],
                                        out + (t0 + j) * ROWV + dv);
    } else {
        u32x4 raw[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) raw[j] = __builtin_nontemporal_load(x + (t0 + j) * ROWV + dv);
#pragma unroll
        for (int j = 0; j < CH; ++j) __builtin_nontemporal_store(raw[j], out + (t0 + j) * ROWV + dv);
    }
}

void convtm() {
    const long tokens = 16384, bytes = tokens * 4096 * 2;  // x, and out alike
    const size_t pool_bytes = size_t(3) << 30, span = 2 * bytes;
    const int rotate = static_cast<int>((size_t(2) << 30) / span) + 1;
    char *pool;
    CHECK(hipMalloc(&pool, pool_bytes));
    CHECK(hipMemset(pool, 1, pool_bytes));
    const long nitems = tokens / 8 * 2, per_xcd = (nitems + 7) / 8;
    printf("token-major causal_conv1d pattern, x and out [16384, 4096] fp16 (2 x 134,217,728 B)\n");
    for (int win = 1; win >= 0; --win) {
        auto launch = [&](int c) {
            size_t off = (size_t(c) * span) % (pool_bytes - span);
            off &= ~size_t(4095);
            const u32x4 *a = reinterpret_cast<const u32x4 *>(pool + off);
            u32x4 *b = reinterpret_cast<u32x4 *>(pool + off + bytes);
            if (win)
                hipLaunchKernelGGL((convtm_kernel<true>), dim3(8 * per_xcd), dim3(256), 0, 0, a, b,
                                   nitems, per_xcd);
            else
                hipLaunchKernelGGL((convtm_kernel<false>), dim3(8 * per_xcd), dim3(256), 0, 0, a, b,
                                   nitems, per_xcd);
        };
        const double us = time_launches(launch, rotate);
        printf("  %-58s %7.2f us  %5.3f of 8 TB/s\n",
               win ? "11 rows loaded (3 re-read from L2), 8 stored per lane" :
                     "8 rows loaded, 8 stored per lane (same grid, no window)",
               us, 2.0 * bytes / us / 1e6 / 8.0);
        fflush(stdout);
    }
    CHECK(hipFree(pool));
}

// --------------------------------------------------------------- issue

// MODE 0: 16 independent exp per iteration, 1: 16 fma, 2: the first half of
// the waves exp and the second half fma (so with 2 or 4 waves per SIMD,
// every SIMD has both), 3: 16 exp + 16 fma in every wave.
template <int MODE>
__global__ void issue_kernel(float *out, long long *cyc, int iters, float seed) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    float x[16], y[16];
    for (int i = 0; i < 16; ++i) {
        x[i] = seed * (lane + i) - 4.0f;
        y[i] = seed * (lane - i);
    }
    const bool do_exp = MODE == 0 || MODE == 3 || (MODE == 2 && wave < nw / 2);
    const bool do_fma = MODE == 1 || MODE == 3 || (MODE == 2 && wave >= nw / 2);
    const long long t0 = __builtin_amdgcn_s_memtime();
    if (do_exp && !do_fma) {
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = __builtin_amdgcn_exp2f(-x[i]);
    } else if (do_fma && !do_exp) {
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int i = 0; i < 16; ++i) y[i] = fmaf(y[i], 0.999f, 0.001f);
    } else {
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                x[i] = __builtin_amdgcn_exp2f(-x[i]);
                y[i] = fmaf(y[i], 0.999f, 0.001f);
            }
    }
    const long long t1 = __builtin_amdgcn_s_memtime();
    float s = 0;
    for (int i = 0; i < 16; ++i) s += x[i] + y[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
    if (blockIdx.x == 0 && lane == 0) cyc[wave] = t1 - t0;
}

// One wave: 8 independent 32x32x16 bf16 MFMAs (4 accumulators) per
// iteration, with EXP independent exps interleaved (1 MFMA : 2 TRANS).
template <bool EXP>
__global__ void mfma_exp_kernel(float *out, long long *cyc, int iters, float seed) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    bf16x8_t a, b0, b1, b2, b3;
    for (int i = 0; i < 8; ++i) {
        a[i] = static_cast<__bf16>(seed * (lane + i));
        b0[i] = static_cast<__bf16>(seed * (lane - i));
        b1[i] = static_cast<__bf16>(seed * (lane - 2 * i));
        b2[i] = static_cast<__bf16>(seed * (lane - 3 * i));
        b3[i] = static_cast<__bf16>(seed * (lane + 3 * i));
    }
    f32x16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
    float x[16];
    for (int i = 0; i < 16; ++i) x[i] = seed * (lane + i) - 4.0f;
    const long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b0, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b1, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b2, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b3, c3, 0, 0, 0);
        }
        if (EXP) {
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = __builtin_amdgcn_exp2f(-x[i]);
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);  // TRANS
            }
        }
    }
    const long long t1 = __builtin_amdgcn_s_memtime();
    float s = 0;
    for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i] + x[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
    if (blockIdx.x == 0 && lane == 0) cyc[wave] = t1 - t0;
}

long long slowest_wave(const long long *dcyc, int waves) {
    long long h[16];
    CHECK(hipMemcpy(h, dcyc, 8 * waves, hipMemcpyDeviceToHost));
    long long m = 0;
    for (int w = 0; w < waves; ++w) m = h[w] > m ? h[w] : m;
    return m;
}

void issue() {
    float *out;
    long long *cyc;
    CHECK(hipMalloc(&out, 256 * 1024 * sizeof(float)));
    CHECK(hipMalloc(&cyc, 16 * 8));
    const int iters = 2000, blocks = 256;  // one workgroup per CU
    const char *names[4] = {"exp only", "fma only", "exp waves | fma waves", "exp + fma in each wave"};
    printf("cycles per instruction per SIMD (s_memtime), 16 independent chains per wave\n");
    for (int wps = 1; wps <= 4; ++wps) {
        const int threads = 256 * wps;
        for (int mode = 0; mode < 4; ++mode) {
            if (mode == 2 && wps == 1) continue;
            auto k = mode == 0 ? issue_kernel<0> : mode == 1 ? issue_kernel<1> : mode == 2 ? issue_kernel<2> : issue_kernel<3>;
            hipLaunchKernelGGL(k, dim3(blocks), dim3(threads), 0, 0, out, cyc, iters, 0.001f);
            CHECK(hipDeviceSynchronize());
            const double ops = double(iters) * 16 * wps * (mode == 3 ? 2 : 1);
            printf("  %d wave(s) per SIMD, %-24s %6.2f\n", wps, names[mode],
                   slowest_wave(cyc, threads / 64) / ops);
        }
    }
    for (int wps = 1; wps <= 2; ++wps) {
        const int threads = 256 * wps;
        for (int e = 0; e <= 1; ++e) {
            hipLaunchKernelGGL(e ? mfma_exp_kernel<true> : mfma_exp_kernel<false>, dim3(blocks),
                               dim3(threads), 0, 0, out, cyc, iters, 0.001f);
            CHECK(hipDeviceSynchronize());
            printf("  %d wave(s) per SIMD, 8 MFMA 32x32x16%s: %.1f cycles per iteration per wave\n",
                   wps, e ? " + 16 exp interleaved" : "", slowest_wave(cyc, threads / 64) / double(iters));
        }
    }
    CHECK(hipFree(out));
    CHECK(hipFree(cyc));
}

// ----------------------------------------------------------------- lds

template <typename V, int ELEMS>
__global__ void __launch_bounds__(1024) lds_read_kernel(unsigned *out, long long *cyc, int iters) {
    __shared__ V buf[ELEMS];  // 64 KiB
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    for (int i = t; i < ELEMS; i += blockDim.x) {
        V v;
        for (int c = 0; c < static_cast<int>(sizeof(V) / 4); ++c) v[c] = static_cast<unsigned>(i + c);
        buf[i] = v;
    }
    __syncthreads();
    unsigned acc = 0;
    const long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
        V r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = buf[((wave * 8 + j) * 64 + lane + it) & (ELEMS - 1)];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc ^= r[j][0] ^ r[j][1];
    }
    const long long t1 = __builtin_amdgcn_s_memtime();
    out[blockIdx.x * blockDim.x + t] = acc;
    if (blockIdx.x == 0 && lane == 0) cyc[wave] = t1 - t0;
}

// Each wave: 8 MFMAs per iteration, A (1 KiB per MFMA) read from LDS or held
// in registers.
__global__ void __launch_bounds__(1024) lds_mfma_kernel(float *out, long long *cyc, int iters,
                                                        int from_lds) {
    __shared__ u32x4 buf[4096];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    for (int i = t; i < 4096; i += blockDim.x)
        buf[i] = u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, static_cast<unsigned>(i)};
    __syncthreads();
    const u32x4 b = buf[lane];
    u32x4 areg[8];
    for (int j = 0; j < 8; ++j) areg[j] = buf[j * 64 + lane];
    f32x16_t c = {};
    const long long t0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const u32x4 a = from_lds ? buf[((wave * 8 + j) * 64 + lane + it) & 4095] : areg[j];
            c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                        __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
        }
    }
    const long long t1 = __builtin_amdgcn_s_memtime();
    float s = 0;
    for (int i = 0; i < 16; ++i) s += c[i];
    out[blockIdx.x * blockDim.x + t] = s;
    if (blockIdx.x == 0 && lane == 0) cyc[wave] = t1 - t0;
}

void lds() {
    unsigned *out;
    long long *cyc;
    CHECK(hipMalloc(&out, 256 * 1024 * sizeof(unsigned)));
    CHECK(hipMalloc(&cyc, 16 * 8));
    const int iters = 4000, blocks = 256;
    for (int threads : {256, 512, 1024}) {
        const int waves = threads / 64;
        hipLaunchKernelGGL((lds_read_kernel<u32x4, 4096>), dim3(blocks), dim3(threads), 0, 0, out, cyc, iters);
        CHECK(hipDeviceSynchronize());
        printf("  %2d waves per CU: ds_read_b128 %6.1f B/clk/CU", waves,
               double(iters) * 8 * 1024 * waves / slowest_wave(cyc, waves));
        hipLaunchKernelGGL((lds_read_kernel<u32x2, 8192>), dim3(blocks), dim3(threads), 0, 0, out, cyc, iters);
        CHECK(hipDeviceSynchronize());
        printf(", ds_read_b64 %6.1f B/clk/CU", double(iters) * 8 * 512 * waves / slowest_wave(cyc, waves));
        for (int fl = 0; fl <= 1; ++fl) {
            hipLaunchKernelGGL(lds_mfma_kernel, dim3(blocks), dim3(threads), 0, 0,
                               reinterpret_cast<float *>(out), cyc, iters, fl);
            CHECK(hipDeviceSynchronize());
            printf(", MFMA with A from %s %5.1f cycles", fl ? "LDS" : "registers",
                   slowest_wave(cyc, waves) / (double(iters) * 8 * (threads / 256)));
        }
        printf(" (per MFMA per SIMD)\n");
    }
    CHECK(hipFree(out));
    CHECK(hipFree(cyc));
}

int main(int argc, char **argv) {
    const char *what = argc > 1 ? argv[1] : "";
    if (!strcmp(what, "ceilings")) ceilings();
    else if (!strcmp(what, "wstream")) wstream();
    else if (!strcmp(what, "convtm")) convtm();
    else if (!strcmp(what, "issue")) issue();
    else if (!strcmp(what, "lds")) lds();
    else {
        fprintf(stderr, "usage: %s ceilings | wstream | convtm | issue | lds\n", argv[0]);
        return 2;
    }
    return 0;
}
