// gemv.hip — decode-time matrix-vector products that stream the weight
// matrix at HBM rate.
//
// No reference implementation: GEMV is absent from the reference library.
//   fp16 / bf16:  y[b, n] = T( sum_k W[n, k] * x[b, k] )            fp32 acc
//   int8:         y[b, n] = fp16( s[n] * sum_k float(Wq[n, k]) * x[b, k] )
//
// gfx950 design, by batch size (rows of x):
//   * 3-8 (fp16 / bf16) or 2-8 (int8) with K a multiple of 128 / 256: the
//     4x4x4 matrix-core path ("4x4x4 MFMA path" below).  Each wave streams 4
//     whole rows of W in 256-byte row segments, x sits in LDS (int8 W: copied
//     there straight from memory, no registers), and the waves start their
//     sweeps of K at staggered offsets.
//   * larger batches and other K (multiples of 32 / 64): the 16x16x32
//     matrix-core path ("MFMA path" below), in slices of 16 columns.
//   * 1-2 and all other shapes: the VALU path, which streams W fastest when
//     there is little math per byte.  A workgroup of 4 waves owns 4*R
//     consecutive output rows and stages x ([B, K], up to the workgroup's
//     160 KiB) in LDS; x (and the int8 scales) are loaded before W, so that waiting for
//     them leaves W in flight.  Each wave streams R rows of W with 16-byte
//     loads, lane-interleaved
//     along K so that every load instruction reads a contiguous 1 KiB run of
//     a row; a lane issues the loads of CPL chunks of each row before using
//     any (a whole fp16 row, or one or two int8 rows, in flight per wave at
//     K = 4096), and keeps R x B fp32 partial sums; the products use
//     v_dot2_f32_{f16,bf16} (two MACs per instruction, fp32 accumulation).  A
//     wave reduction through DPP and permlane swaps (wave_sum, no LDS)
//     finishes each (row, batch) sum.
// int8 weights are widened exactly to fp16 with one v_perm_b32 (bytes of
// w+128 under the exponent of 1024.0) and one packed fp16 subtract of 1152 per
// weight pair; the per-row int8 scale is applied to the fp32 sum.
// HBM-bound: algorithmic bytes = |W| + |x| + |y| (+|s|).
#include "common.h"
#include "device.h"


namespace {

using namespace tecoops::dev;

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

template <typename T> struct Dot2;
template <> struct Dot2<f16> {
    static __device__ __forceinline__ float run(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a),
                                      __builtin_bit_cast(half2_t, b), c, false);
    }
};
template <> struct Dot2<bf16> {
    static __device__ __forceinline__ float run(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162_t, a),
                                               __builtin_bit_cast(bf162_t, b), c, false);
    }
};

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

// Streaming 16-byte load of weight data that is read exactly once.
__device__ __forceinline__ uint4 load_stream(const uint4 *p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Copies x [B, K] (16-bit elements, K % 8 == 0, nvec 16-byte chunks) into
// LDS in two halves.  x_pre loads the first XP chunks of each thread into
// registers and is called before the W loads, so that waiting for x later
// leaves the younger W loads in flight (loads complete in order); x_post
// stores them, copies any remaining chunks and synchronises the workgroup.
template <int XP>
__device__ __forceinline__ void x_pre(uint4 (&xr)[XP], const uint4 *x, int nvec) {
    // Relaxed workgroup-scope atomic loads (plain global loads in the ISA):
    // the compiler neither sinks them to their use nor hoists the W loads
    // above them, as it does with ordinary loads of read-only memory.
#pragma unroll
    for (int j = 0; j < XP; ++j) {
        const uint64_t *p = reinterpret_cast<const uint64_t *>(
            x + min(static_cast<int>(threadIdx.x + j * blockDim.x), nvec - 1));
        const uint64_t lo = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const uint64_t hi = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        xr[j] = make_uint4(static_cast<uint32_t>(lo), static_cast<uint32_t>(lo >> 32),
                           static_cast<uint32_t>(hi), static_cast<uint32_t>(hi >> 32));
    }
}
template <int XP>
__device__ __forceinline__ void x_post(uint4 *xs, const uint4 (&xr)[XP], const uint4 *x, int nvec) {
    // unconditional (clamped) stores: a store under a branch lets the
    // compiler sink its load into that branch, behind the W loads; threads
    // past the end all write x's last chunk to its own place
#pragma unroll
    for (int j = 0; j < XP; ++j) xs[min(static_cast<int>(threadIdx.x + j * blockDim.x), nvec - 1)] = xr[j];
    for (int i = threadIdx.x + XP * blockDim.x; i < nvec; i += blockDim.x) xs[i] = x[i];
    __syncthreads();
}
// x chunks per thread loaded ahead of W: all of x for B = 1 and K <= 4096.
constexpr int x_pre_chunks(int B) { return B == 1 ? 2 : 4; }

// int8 weight dword (4 values) -> two packed fp16 pairs holding the exact values.
__device__ __forceinline__ void widen_i8(uint32_t w, uint32_t &p01, uint32_t &p23) {
    const uint32_t u = w ^ 0x80808080u;  // bytes now hold w + 128 in [0, 255]
    const half2_t bias = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    // 0x64XX as fp16 is 1024 + XX
    half2_t h01 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
    half2_t h23 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
    p01 = __builtin_bit_cast(uint32_t, h01 + bias);
    p23 = __builtin_bit_cast(uint32_t, h23 + bias);
}

// int8 weights, VALU path with the weight loads batched: each K step of a
// wave covers 64 * CPL 16-byte chunks of each of its R rows, and a lane issues
// all R * CPL of its loads before widening any of them, so every lane keeps
// R * CPL * 16 bytes in flight and a row needs K / (1024 * CPL) round trips.
template <int B, int R, int CPL, int NW>
__global__ void __launch_bounds__(NW * 64)
gemv_i8_kernel(const uint4 *__restrict__ W, const uint16_t *__restrict__ scales,
                       const uint4 *__restrict__ x, uint16_t *__restrict__ y, int N, int K) {
    extern __shared__ uint4 xs[];
    const int kx = K / 8;    // 16-byte chunks of an x row (8 fp16)
    const int kw = K / 16;   // 16-byte chunks of a W row (16 int8)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * NW + wave) * R;
    const uint4 *wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wrow[r] = W + static_cast<long long>(min(n0 + r, N - 1)) * kw;
    // the scales and x are loaded before W: they are waited for without
    // draining the W loads, and the scales are in registers by the end
    uint16_t sc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) sc[r] = scales[min(n0 + r, N - 1)];
    uint4 xr[x_pre_chunks(B)];
    x_pre(xr, x, B * kx);
    // W loads are unconditional (clamped to the row's last chunk) so that the
    // compiler waits for each one at its use rather than for all of them
    uint4 q[R][CPL];
#pragma unroll
    for (int u = 0; u < CPL; ++u)
#pragma unroll
        for (int r = 0; r < R; ++r) q[r][u] = load_stream(wrow[r] + min(lane + 64 * u, kw - 1));
    x_post(xs, xr, x, B * kx);
    if (n0 >= N) return;
    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[r][b] = 0.0f;
    for (int c0 = lane;; c0 += 64 * CPL) {
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            const int c = c0 + 64 * u;
            if (c < kw) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    uint32_t wh[8];  // 16 weights as 8 fp16 pairs
                    widen_i8(q[r][u].x, wh[0], wh[1]);
                    widen_i8(q[r][u].y, wh[2], wh[3]);
                    widen_i8(q[r][u].z, wh[4], wh[5]);
                    widen_i8(q[r][u].w, wh[6], wh[7]);
#pragma unroll
                    for (int b = 0; b < B; ++b) {
                        const uint4 x0 = xs[b * kx + 2 * c];
                        const uint4 x1 = xs[b * kx + 2 * c + 1];
                        const uint32_t xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                        float s = acc[r][b];
#pragma unroll
                        for (int j = 0; j < 8; ++j) s = Dot2<f16>::run(wh[j], xv[j], s);
                        acc[r][b] = s;
                    }
                }
            }
        }
        const int cn = c0 + 64 * CPL;
        if (cn - lane >= kw) break;
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
            for (int r = 0; r < R; ++r) q[r][u] = load_stream(wrow[r] + min(cn + 64 * u, kw - 1));
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float s = wave_sum(acc[r][b]);
            if (lane == 0 && n0 + r < N)
                y[static_cast<long long>(b) * N + n0 + r] = f2h(h2f(sc[r]) * s);
        }
    }
}

// fp16 / bf16 weights, VALU path with batched loads (as gemv_i8_kernel).
template <typename T, int B, int R, int CPL, int NW>
__global__ void __launch_bounds__(NW * 64)
gemv16_kernel(const uint4 *__restrict__ W, const uint4 *__restrict__ x,
                      uint16_t *__restrict__ y, int N, int K) {
    extern __shared__ uint4 xs[];
    const int kv = K / 8;  // 16-byte chunks per row
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * NW + wave) * R;
    const uint4 *wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wrow[r] = W + static_cast<long long>(min(n0 + r, N - 1)) * kv;
    uint4 xr[x_pre_chunks(B)];
    x_pre(xr, x, B * kv);
    uint4 q[R][CPL];
#pragma unroll
    for (int u = 0; u < CPL; ++u)
#pragma unroll
        for (int r = 0; r < R; ++r) q[r][u] = load_stream(wrow[r] + min(lane + 64 * u, kv - 1));
    x_post(xs, xr, x, B * kv);
    if (n0 >= N) return;
    float acc[R][B];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[r][b] = 0.0f;
    for (int c0 = lane;; c0 += 64 * CPL) {
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            const int c = c0 + 64 * u;
            if (c < kv) {
#pragma unroll
                for (int b = 0; b < B; ++b) {
                    const uint4 xv = xs[b * kv + c];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float s = acc[r][b];
                        s = Dot2<T>::run(q[r][u].x, xv.x, s);
                        s = Dot2<T>::run(q[r][u].y, xv.y, s);
                        s = Dot2<T>::run(q[r][u].z, xv.z, s);
                        s = Dot2<T>::run(q[r][u].w, xv.w, s);
                        acc[r][b] = s;
                    }
                }
            }
        }
        const int cn = c0 + 64 * CPL;
        if (cn - lane >= kv) break;
#pragma unroll
        for (int u = 0; u < CPL; ++u)
#pragma unroll
            for (int r = 0; r < R; ++r) q[r][u] = load_stream(wrow[r] + min(cn + 64 * u, kv - 1));
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float s = wave_sum(acc[r][b]);
            if (lane == 0 && n0 + r < N) y[static_cast<long long>(b) * N + n0 + r] = Cvt<T>::from(s);
        }
}

// ------------------------------------------------------------------ MFMA path
//
// Y^T = W X^T on v_mfma_f32_16x16x32_{f16,bf16}: A = 16 rows of W x 32 k,
// B = X^T (32 k x 16 batch columns, of which the first B are stored).  Lane l
// supplies A[row l%16][k 8*(l/16) .. +7] (one 16-byte load of W) and
// B[k 8*(l/16) .. +7][column l%16] (one 16-byte load of x, L2-resident); it
// receives C[row 4*(l/16) + v][column l%16], v < 4.  A workgroup owns RT*16
// rows; its 4 waves take interleaved 32-k steps (split-K), keep the W loads
// of their next steps in flight in a register ring, and add their partial C
// tiles through LDS.  For int8 weights a lane loads 16 weights (16 bytes),
// widens them exactly to fp16 and feeds two MFMAs whose k order is permuted
// consistently on A and B (k is a summation index).
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename T> struct Mma16;
template <> struct Mma16<f16> {
    static __device__ __forceinline__ f32x4_t run(u32x4_t a, u32x4_t b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
};
template <> struct Mma16<bf16> {
    static __device__ __forceinline__ f32x4_t run(u32x4_t a, u32x4_t b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    }
};

__device__ __forceinline__ u32x4_t ld16(const uint16_t *p) {
    return *reinterpret_cast<const u32x4_t *>(p);
}
__device__ __forceinline__ u32x4_t ld16_stream(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
}

// Adds the NW waves' partial tiles and writes y (scaled by s[n] when given).
template <typename T, int RT, int NW>
__device__ __forceinline__ void gemv_mfma_epilogue(f32x4_t (&c)[RT], float *red, int n0, int N,
                                                   int B, uint16_t *y, const uint16_t *scales) {
    static_assert(RT <= NW, "one wave finishes each row tile");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        *reinterpret_cast<f32x4_t *>(red + ((rt * NW + wave) * 64 + lane) * 4) = c[rt];
    __syncthreads();
    // wave w finishes row tile w
    if (wave < RT) {
        f32x4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < NW; ++w)
            sum += *reinterpret_cast<const f32x4_t *>(red + ((wave * NW + w) * 64 + lane) * 4);
        const int col = lane & 15;
        if (col < B) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = n0 + wave * 16 + 4 * (lane >> 4) + v;
                if (n < N) {
                    const float o = scales ? sum[v] * h2f(scales[n]) : sum[v];
                    y[static_cast<long long>(col) * N + n] = Cvt<T>::from(o);
                }
            }
        }
    }
}

// Runs one wave's n steps (n wave-uniform) with the loads of each step issued
// D steps ahead of its use: load(j, i) fetches step j into ring slot i and
// use(j, i) consumes step j from slot i; start() runs once, after the first
// loads are issued and before the first use.  Slot indices are compile-time
// constants after unrolling, so the ring stays in registers, and the loads of
// the main loop are unconditional, so the waits before each use leave the
// younger loads in flight.
template <int D, typename Load, typename Use, typename Start>
__device__ __forceinline__ void ring_steps(int n, Load &&load, Use &&use, Start &&start) {
    if (n < D) {
        for (int j = 0; j < n; ++j) {
            load(j, 0);
            if (j == 0) start();
            use(j, 0);
        }
        if (n <= 0) start();
        return;
    }
#pragma unroll
    for (int i = 0; i < D; ++i) load(i, i);
    start();
    int j = 0;
    for (; j + 2 * D <= n; j += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            use(j + i, i);
            load(j + D + i, i);
            // keep this order: the scheduler would otherwise batch the loads
            // at the end of the iteration and drain the ring at its top
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // steps j .. j+D-1 are in the ring; j+D .. n-1 (fewer than D) are not
#pragma unroll
    for (int i = 0; i < D; ++i) {
        use(j + i, i);
        if (j + D + i < n) load(j + D + i, i);
    }
#pragma unroll
    for (int i = 0; i < D; ++i)
        if (j + D + i < n) use(j + D + i, i);
}

template <int D, typename Load, typename Use>
__device__ __forceinline__ void ring_steps(int n, Load &&load, Use &&use) {
    ring_steps<D>(n, load, use, [] {});
}

// Depth of the 16x16x32 kernels' ring.  Measured on the [14336, 4096]
// batch-8 shapes, deeper rings do not pay: the fp16 kernel goes from 29 us at
// depth 1 to 33 us at depth 4 (each load instruction already touches 16 rows
// and the workgroups keep enough requests in flight), int8 with 4 row tiles
// is flat (17.0 / 17.2 / 17.3 us at depths 1 / 2 / 4).
constexpr int kRing = 1;

// Wave w takes the 32-k (16-bit W) or 64-k (int8 W) steps w, w+4, w+8, ...
// Columns >= B of the B operand read row B-1 of x: the C columns they produce
// are never stored, and every value read is an element of x.
template <typename T, int RT, int NW>
__global__ void __launch_bounds__(NW * 64)
gemv16_mfma_kernel(const uint16_t *__restrict__ W, const uint16_t *__restrict__ x,
                   uint16_t *__restrict__ y, int N, int K, int B) {
    __shared__ __attribute__((aligned(16))) float red[RT * NW * 64 * 4];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * (16 * RT);
    const int g = lane >> 4, col = lane & 15;
    const uint16_t *wr[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        wr[rt] = W + static_cast<long long>(min(n0 + rt * 16 + col, N - 1)) * K + 8 * g + 32 * wave;
    const uint16_t *xr = x + static_cast<long long>(min(col, B - 1)) * K + 8 * g + 32 * wave;
    f32x4_t c[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) c[rt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    u32x4_t a[kRing][RT], b[kRing];
    const int n = (K / 32 - wave + NW - 1) / NW;
    ring_steps<kRing>(
        n,
        [&](int j, int i) {
            const int k0 = j * (32 * NW);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) a[i][rt] = ld16_stream(wr[rt] + k0);
            b[i] = ld16(xr + k0);
        },
        [&](int, int i) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) c[rt] = Mma16<T>::run(a[i][rt], b[i], c[rt]);
        });
    gemv_mfma_epilogue<T, RT, NW>(c, red, n0, N, B, y, nullptr);
}

__device__ __forceinline__ void widen_i8x16(u32x4_t q, u32x4_t &lo8, u32x4_t &hi8) {
    uint32_t p[8];
    widen_i8(q.x, p[0], p[1]);
    widen_i8(q.y, p[2], p[3]);
    widen_i8(q.z, p[4], p[5]);
    widen_i8(q.w, p[6], p[7]);
    lo8 = u32x4_t{p[0], p[1], p[2], p[3]};
    hi8 = u32x4_t{p[4], p[5], p[6], p[7]};
}

template <int RT, int NW>
__global__ void __launch_bounds__(NW * 64)
gemv_i8_mfma_kernel(const int8_t *__restrict__ W, const uint16_t *__restrict__ scales,
                    const uint16_t *__restrict__ x, uint16_t *__restrict__ y, int N, int K,
                    int B) {
    __shared__ __attribute__((aligned(16))) float red[RT * NW * 64 * 4];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * (16 * RT);
    const int g = lane >> 4, col = lane & 15;
    const int8_t *wr[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        wr[rt] = W + static_cast<long long>(min(n0 + rt * 16 + col, N - 1)) * K + 16 * g + 64 * wave;
    const uint16_t *xr = x + static_cast<long long>(min(col, B - 1)) * K + 16 * g + 64 * wave;
    f32x4_t c[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) c[rt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    u32x4_t q[kRing][RT], b0[kRing], b1[kRing];
    const int n = (K / 64 - wave + NW - 1) / NW;
    ring_steps<kRing>(
        n,
        [&](int j, int i) {
            const int k0 = j * (64 * NW);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) q[i][rt] = ld16_stream(wr[rt] + k0);
            b0[i] = ld16(xr + k0);
            b1[i] = ld16(xr + k0 + 8);
        },
        [&](int, int i) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                u32x4_t a0, a1;
                widen_i8x16(q[i][rt], a0, a1);
                c[rt] = Mma16<f16>::run(a0, b0[i], c[rt]);
                c[rt] = Mma16<f16>::run(a1, b1[i], c[rt]);
            }
        });
    gemv_mfma_epilogue<f16, RT, NW>(c, red, n0, N, B, y, scales);
}

// ------------------------------------------------------ 4x4x4 MFMA path
//
// Batches of up to 8 rows of x: Y^T = W X^T on v_mfma_f32_4x4x4_16b_{f16,
// bf16}, which runs 16 independent 4x4x4 products (blocks) per instruction.
// Lane l = 4*blk + r supplies row r of block blk's A operand and column r of
// its B operand, and receives column r of its C block.  Each wave owns 4 whole
// rows of W: lane l loads the 16 bytes at chunk blk of every 16-chunk
// (256-byte) run of row n0 + r, so one load instruction reads four contiguous
// 256-byte row segments (the access pattern of the VALU path), and block blk
// accumulates those 4 rows against batch columns 4*cg + r over its own k
// values.  The 16 blocks hold partial sums over disjoint k; once the wave has
// covered K they are added across lanes l, l + 4, ..., l + 60 without LDS
// (DPP row rotations by 4 and 8, then the row-pair and half-wave permlane
// swaps).  Unless K is split over 2 or 4 waves (small N), no cross-wave
// reduction or barrier follows the staging of x.
//   x is staged in LDS as [4*NCG][K] 16-bit values with the 16-byte chunks of
//   row i XOR-swizzled by 4*(i % 4) inside each 256-byte run, so that the
//   128-bit B-operand reads of lanes 0-7 (rows 0-3, two chunks) hit distinct
//   banks.  int8 weights are widened exactly to fp16 (widen_i8) and feed 4
//   k-steps per 16-byte load; the per-row scale is applied to the fp32 sum.
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

template <typename T> struct Mma4;
template <> struct Mma4<f16> {
    static __device__ __forceinline__ f32x4_t run(uint32_t a0, uint32_t a1, uint32_t b0,
                                                  uint32_t b1, f32x4_t c) {
        const u32x2_t a = {a0, a1}, b = {b0, b1};
        return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4_t, a),
                                                  __builtin_bit_cast(f16x4_t, b), c, 0, 0, 0);
    }
};
template <> struct Mma4<bf16> {
    static __device__ __forceinline__ f32x4_t run(uint32_t a0, uint32_t a1, uint32_t b0,
                                                  uint32_t b1, f32x4_t c) {
        const u32x2_t a = {a0, a1}, b = {b0, b1};
        return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(i16x4_t, a),
                                                      __builtin_bit_cast(i16x4_t, b), c, 0, 0, 0);
    }
};

// 16 zero bytes: the source of staged x rows past the batch.
__device__ __attribute__((aligned(16))) const uint32_t kXZero16[4] = {0u, 0u, 0u, 0u};

// Global -> LDS with no register staging: 16 bytes per lane into
// dst + 16 * lane (dst wave-uniform, in M0).  Inline assembly so that the
// compiler does not count the copy among its own loads: through the builtin
// it would wait for every load in flight (the W ring included) before the
// first LDS read.  The copies are ordered by wait_vm() and the workgroup
// barrier after it.  No other code of these kernels uses M0 (build.py checks
// both in the assembly).
__device__ __forceinline__ void dma16(const void *src, void *dst) {
    const uint32_t lds = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)(dst)));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
                 : "memory");
}

// s_waitcnt vmcnt(N): all but the N youngest vector-memory operations of the
// wave are done (expcnt and lgkmcnt not waited for).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(((N >> 4) << 14) | 0x0F70 | (N & 15));
}

// x chunks (16 bytes) a workgroup of the 4x4x4 path loads into registers
// ahead of its first W loads (64 KiB, the whole x of batch 8 at K = 4096); a
// larger staged x copies the chunks past these straight to LDS.
constexpr int kMaxXChunks = 4096;

// LDS element offset of the 16-byte chunk c of staged x row `row`.
__device__ __forceinline__ int xs_chunk(int row, int c, int K) {
    return row * K + 8 * (c ^ (4 * (row & 3)));
}

// T: element type of x / y (and W unless I8).  NCG: batch column groups of 4
// (1 for B <= 4, else 2).  RG: groups of 4 rows per wave, which share each x
// read from LDS.  CPL: load steps a lane keeps in flight (RG loads each).
// KS: waves per row group, each sweeping 1/KS of K; their sums meet in LDS
// (KS = 2 or 4 when N is small, so that the grid still has enough waves).
// PHASED: K is swept in nph equal phases, x staged in LDS one phase at a
// time (rows whose whole x does not fit in LDS); W is still read once.
template <typename T, bool I8, int NCG, int RG, int NW, int CPL, int KS, bool PHASED>
__global__ void __launch_bounds__(NW * 64)
gemv_b8_kernel(const uint4 *__restrict__ W, const uint16_t *__restrict__ scales,
               const uint4 *__restrict__ x, uint16_t *__restrict__ y, int N, int K, int B,
               int nph_arg) {
    extern __shared__ uint4 xs_raw[];
    uint16_t *xs = reinterpret_cast<uint16_t *>(xs_raw);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr int GW = NW / KS;          // row groups per workgroup
    const int gw = wave % GW, part = wave / GW;
    const int r = lane & 3, blk = lane >> 2;
    const int n0 = (blockIdx.x * GW + gw) * 4 * RG;
    const int nph = PHASED ? nph_arg : 1;
    const int kp = K / nph;              // k values per phase
    const int kw = I8 ? K / 16 : K / 8;  // 16-byte chunks of a W row
    const int nl = kw / nph / 16 / KS;   // load steps per row, part and phase
    const uint4 *wr[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g)
        wr[g] = W + static_cast<long long>(min(n0 + 4 * g + r, N - 1)) * kw + blk;
    const int kx = K / 8;    // 16-byte chunks of an x row
    const int kxp = kp / 8;  // ... of one phase
    f32x4_t acc[RG][NCG];
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg) acc[g][cg] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    // The scales (int8) and x loads are issued first (unconditionally,
    // clamped to the last row / chunk), so that waiting for x leaves the
    // younger W loads in flight and the scales are in registers by the end.
    uint16_t sc[RG][4];
    if constexpr (I8) {
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int v = 0; v < 4; ++v) sc[g][v] = scales[min(n0 + 4 * g + v, N - 1)];
    }
    constexpr int XPT = (kMaxXChunks + NW * 64 - 1) / (NW * 64);  // x chunks per thread
    // int8 W with x staged in one phase: x goes straight into LDS (no
    // registers, no LDS stores).  [14336, 4096] batch 8, three alternating
    // runs, us register-staged / copied: int8 12.57-12.91 / 12.10-12.43;
    // fp16 20.92-21.02 / 21.77-21.86, so fp16 keeps the registers.
    constexpr bool XDMA = I8 && !PHASED;
    const int nxc = NCG * 4 * kxp;
    // This lane's x chunks in LDS: chunk 16i + blk (fp16 W) or 32i + 2blk and
    // the next (int8 W) of row 4cg + r.  The swizzle xor (4r < 16) stays below
    // the step's bits, so xs_chunk(4cg + r, c0 + 16i, kp) = xs_chunk(4cg + r,
    // c0, kp) + 128i (c0 = blk), likewise with 32i (c0 = 2blk), and rows 4
    // apart keep the same xor: one base address per lane.
    const uint16_t *xs_lane = xs + xs_chunk(r, I8 ? 2 * blk : blk, kp);
    uint4 q[CPL][RG];
    // Each wave starts its sweep of K at a different load step, so that the
    // requests in flight across the grid spread over all HBM channels instead
    // of every wave reading the same offset of its rows at the same time.
    const int rot = (blockIdx.x * GW + gw) % nl;
    const auto local = [&](int i) { return part * nl + (i + rot < nl ? i + rot : i + rot - nl); };
    for (int ph = 0; ph < nph; ++ph) {
        const int xc0 = ph * kxp;       // the phase's first chunk of an x row
        const int st0 = ph * nl * KS;   // ... and first load step of a W row
        uint4 xr[XDMA ? 1 : XPT];
        if constexpr (!XDMA) {
#pragma unroll
            for (int j = 0; j < XPT; ++j) {
                const int idx = min(static_cast<int>(threadIdx.x) + j * NW * 64, nxc - 1);
                const int row = min(idx / kxp, B - 1);
                xr[j] = x[static_cast<long long>(row) * kx + xc0 + idx % kxp];
            }
        } else {
            // the whole x straight into LDS: copy m fills LDS chunks [64m, 64m + 64), so lane
            // l loads the x chunk stored at 64m + l (the swizzle flips bits 2-3 of the chunk
            // index only, within the copy's 64); rows past the batch copy zeros
            for (int m = wave; m < nxc / 64; m += NW) {
                const int slot = 64 * m + lane;
                const int row = slot / kxp, cs = slot - row * kxp;
                const void *src = row < B ? static_cast<const void *>(
                                                x + static_cast<long long>(row) * kx +
                                                (cs ^ (4 * (row & 3))))
                                          : static_cast<const void *>(kXZero16);
                dma16(src, xs_raw + 64 * m);
            }
        }
        // int8 W on a full-GPU grid: every CU's x loads miss L2 together and,
        // at HBM, queue behind the first W loads of all waves, which start at
        // the same moment, while no wave can use its W before x is in LDS.
        // Pausing ~1000 cycles before the W loads lets the x misses reach HBM
        // first (batch 8 x [14336, 4096], A/B on two boxes: 13.4 -> 12.9 us
        // and 14.0 -> 13.8 us; waiting for x outright: 14.0 us; fp16 W, twice
        // the bytes per x byte, gains nothing).  With 2 W steps in flight per
        // lane, pauses of 0, 8, 16 and 32 (x 64 cycles) took 13.5-14.0, 13.4,
        // 12.9-13.1 and 13.3 us on one box.  The best pause is about one
        // vector L1 -> L2 read round trip of this stream (865 cycles with one
        // load in flight per lane, 1267 with two; rocprofv3
        // TCP_TCC_READ_REQ_LATENCY / TCP_TCC_READ_REQ), i.e. long enough for
        // x's requests to leave the L1 and L2 queues before the W requests
        // fill them, and shorter than waiting for x's data (the HBM round
        // trip, ~2000 cycles once the stream saturates).
        if constexpr (I8) {
            if (ph == 0 && gridDim.x >= 128) __builtin_amdgcn_s_sleep(16);
        }
        // Waves past the last row still stage x and reach the barriers; their
        // loads read row N - 1 and their sums are never stored.
        ring_steps<CPL>(
            nl,
            [&](int i, int u) {
                const int st = 16 * (st0 + local(i));
#pragma unroll
                for (int g = 0; g < RG; ++g) q[u][g] = load_stream(wr[g] + st);
            },
            [&](int i0, int u) {
                const int i = local(i0);
                if constexpr (I8) {
                    uint32_t p[RG][8];
#pragma unroll
                    for (int g = 0; g < RG; ++g) {
                        widen_i8(q[u][g].x, p[g][0], p[g][1]);
                        widen_i8(q[u][g].y, p[g][2], p[g][3]);
                        widen_i8(q[u][g].z, p[g][4], p[g][5]);
                        widen_i8(q[u][g].w, p[g][6], p[g][7]);
                    }
#pragma unroll
                    for (int cg = 0; cg < NCG; ++cg) {
                        // chunks 32i + 2blk and 32i + 2blk + 1 of row 4cg + r
                        const uint4 *xp =
                            reinterpret_cast<const uint4 *>(xs_lane + cg * 4 * kp) + 32 * i;
                        const uint4 xa = xp[0];
                        const uint4 xb = xp[1];
#pragma unroll
                        for (int g = 0; g < RG; ++g) {
                            f32x4_t c = acc[g][cg];
                            c = Mma4<f16>::run(p[g][0], p[g][1], xa.x, xa.y, c);
                            c = Mma4<f16>::run(p[g][2], p[g][3], xa.z, xa.w, c);
                            c = Mma4<f16>::run(p[g][4], p[g][5], xb.x, xb.y, c);
                            c = Mma4<f16>::run(p[g][6], p[g][7], xb.z, xb.w, c);
                            acc[g][cg] = c;
                        }
                    }
                } else {
#pragma unroll
                    for (int cg = 0; cg < NCG; ++cg) {
                        // chunk 16i + blk of row 4cg + r
                        const uint4 xv =
                            reinterpret_cast<const uint4 *>(xs_lane + cg * 4 * kp)[16 * i];
#pragma unroll
                        for (int g = 0; g < RG; ++g) {
                            acc[g][cg] =
                                Mma4<T>::run(q[u][g].x, q[u][g].y, xv.x, xv.y, acc[g][cg]);
                            acc[g][cg] =
                                Mma4<T>::run(q[u][g].z, q[u][g].w, xv.z, xv.w, acc[g][cg]);
                        }
                    }
                }
            },
            // the phase's x chunks reach LDS once its first W loads are in
            // flight (after every wave has finished the previous phase); an
            // x larger than the register-staged part (more than 4096 chunks)
            // copies the rest directly
            [&] {
                if constexpr (XDMA) {
                    // This wave's copies are older than the CPL steps of RG
                    // W loads ring_steps issues before start(), so waiting
                    // until at most those are outstanding leaves them in
                    // flight.  The compiler could legally sink a load of
                    // read-only memory below this wait, which would make the
                    // count too large: build.py checks the assembly of
                    // every such wait and fails the build if it ever does.
                    // A row with fewer steps (ring_steps' short path, K <
                    // 512) waits for everything.  The barrier then covers
                    // every wave's copies.
                    if (nl >= CPL) wait_vm<CPL * RG>();
                    else wait_vm<0>();
                    __syncthreads();
                    return;
                }
                if (ph > 0) __syncthreads();
#pragma unroll
                for (int j = 0; j < XPT; ++j) {
                    const int idx = threadIdx.x + j * NW * 64;
                    if (idx < nxc) {
                        const int row = idx / kxp, c = idx - row * kxp;
                        *reinterpret_cast<uint4 *>(xs + xs_chunk(row, c, kp)) =
                            row < B ? xr[j] : uint4{0u, 0u, 0u, 0u};
                    }
                }
                for (int idx = threadIdx.x + XPT * NW * 64; idx < nxc; idx += NW * 64) {
                    const int row = idx / kxp, c = idx - row * kxp;
                    *reinterpret_cast<uint4 *>(xs + xs_chunk(row, c, kp)) =
                        row < B ? x[static_cast<long long>(row) * kx + xc0 + c]
                                : uint4{0u, 0u, 0u, 0u};
                }
                __syncthreads();
            });
    }
    if constexpr (KS > 1) {
        // parts 1 .. KS-1 hand their sums to part 0 through LDS past the
        // staged x: value e of lane l of row group gw from part pt at
        // red[pt - 1][e][gw * 64 + l], so that the 64 lanes of a wave touch
        // 64 consecutive words per value
        constexpr int NV = RG * NCG * 4;
        const float *red = reinterpret_cast<const float *>(xs + 4 * NCG * kp) + gw * 64 + lane;
        if (part > 0) {
            float *mine = const_cast<float *>(red) + (part - 1) * NV * GW * 64;
#pragma unroll
            for (int g = 0; g < RG; ++g)
#pragma unroll
                for (int cg = 0; cg < NCG; ++cg)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        mine[((g * NCG + cg) * 4 + v) * GW * 64] = acc[g][cg][v];
        }
        __syncthreads();
        if (part > 0) return;
#pragma unroll
        for (int pt = 1; pt < KS; ++pt)
#pragma unroll
            for (int g = 0; g < RG; ++g)
#pragma unroll
                for (int cg = 0; cg < NCG; ++cg)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        acc[g][cg][v] += red[((pt - 1) * NV + (g * NCG + cg) * 4 + v) * GW * 64];
    }
    if (n0 >= N) return;
    // add the 16 blocks' partial sums (lanes r, r + 4, ..., r + 60: rotations
    // by 4 and 8 within each row of 16 lanes, then the row-pair and half-wave
    // swaps); lanes 0-3 then hold column r of rows n0 + 4g .. n0 + 4g + 3
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int cg = 0; cg < NCG; ++cg)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                float t = acc[g][cg][v];
                t += dpp<kDppRor4>(t);
                t += dpp<kDppRor8>(t);
                t = row_swap_sum(t);
                acc[g][cg][v] = half_swap_sum(t);
            }
    if (blk == 0) {
#pragma unroll
        for (int g = 0; g < RG; ++g)
#pragma unroll
            for (int cg = 0; cg < NCG; ++cg) {
                const int b = 4 * cg + r;
                if (b < B) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int n = n0 + 4 * g + v;
                        if (n < N) {
                            const float o = I8 ? acc[g][cg][v] * h2f(sc[g][v]) : acc[g][cg][v];
                            y[static_cast<long long>(b) * N + n] = Cvt<T>::from(o);
                        }
                    }
                }
            }
    }
}

// Fallback for shapes the vector kernels do not take (K not a multiple of 8 /
// 16, misaligned pointers): one wave per (row, batch), element-wise.
template <typename T, bool INT8>
__global__ void __launch_bounds__(kThreads)
gemv_scalar_kernel(const void *__restrict__ Wv, const uint16_t *__restrict__ scales,
                   const uint16_t *__restrict__ x, uint16_t *__restrict__ y, int N, int K,
                   int batch) {
    const int lane = threadIdx.x & 63;
    const long long task = static_cast<long long>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (task >= static_cast<long long>(N) * batch) return;
    const int n = static_cast<int>(task % N), b = static_cast<int>(task / N);
    float s = 0.0f;
    for (int k = lane; k < K; k += 64) {
        const float w = INT8 ? static_cast<float>(static_cast<const int8_t *>(Wv)[static_cast<long long>(n) * K + k])
                             : Cvt<T>::to(static_cast<const uint16_t *>(Wv)[static_cast<long long>(n) * K + k]);
        s += w * Cvt<T>::to(x[static_cast<long long>(b) * K + k]);
    }
    s = wave_sum(s);
    if (lane == 0) {
        if (INT8) s *= h2f(scales[n]);
        y[static_cast<long long>(b) * N + n] = Cvt<T>::from(s);
    }
}

// x staged in LDS may fill a workgroup's whole LDS (reserve_lds sets the
// kernels' attribute above the default 64 KiB when it does).
constexpr long long kMaxLdsBytes = static_cast<long long>(tecoops::kLdsMax);

// Matrix-core path: smallest batch that takes it, row tiles of 16 per
// workgroup and waves per workgroup.  int8 uses 4 row tiles per x fragment
// (x is loaded as 32 bytes per 16 bytes of weights, so sharing it over more
// rows pays: 19.9 -> 17.0 us at batch 8); for fp16 the extra tiles cost more
// in parallelism than they save (28.7 us at 1 tile, 30.9 at 2).
constexpr int kMfmaMinBatch16 = 3, kMfmaRT16 = 1, kMfmaWaves16 = 4;
constexpr int kMfmaMinBatchI8 = 2, kMfmaRTI8 = 4, kMfmaWavesI8 = 8;
// fp16 batch 2 takes the 4x4x4 path above this K: the VALU path's 2 staged
// rows of x then leave fewer than 4 workgroups per CU.  Batch 2, VALU against
// 4x4x4 (us): [4096, 8192] 14.1 / 16.8, [4096, 10240] 16.3-16.5 / 16.8-17.2,
// [14336, 10240] 48.3 / 46.9, [4096, 12288] 21.2 / 18.6, [4096, 14336]
// 23.1 / 21.7, [8192, 28672] 98.5 / 73.6.
constexpr int kB8Batch2MinK = 10240;

// VALU path shapes (rows per wave R, 16-byte W chunks per lane per K step
// CPL), measured on the [14336, 4096] batch-1 shapes: fp16 one row per wave
// with the whole 8 KiB row in flight (19.5 us; 4 rows with one chunk in
// flight: 22.6 us), int8 two 4 KiB rows per wave (12.9 us; 15.5 us before).
// Fewer rows per wave beat deeper per-wave queues: 4 rows x 4 chunks of int8
// took 16.2 us, and 8 or 16 waves per workgroup were slower for both types.
constexpr int kR16 = 1, kCpl16 = 8;
constexpr int kRI8 = 2, kCplI8 = 4;
// int8 at batch 1 with rows of at most kRI8OneMaxK values and at least
// kRI8OneMinN rows: one row per wave (the whole 4 KiB row in flight, twice
// the workgroups, half the bytes in flight per wave).  Standalone sweep, 16
// rotating weight copies, µs two rows / one row per wave: [14336, 4096]
// 10.57-10.69 / 10.46-10.57 on four boxes, [28672, 4096] 18.5-19.2 /
// 18.1-19.0, [11008, 4096] 9.0-9.2 / 8.7; at fewer rows or longer rows two
// stay: [8192, 4096] 7.1-7.2 / 7.3, [4096, 4096] 4.7-5.0 / 5.2-5.5,
// [14336, 14336] 33.5-36.0 / 35.0-37.2, [8192, 28672] 40-43 / 47-50 (some
// shapes outside the rule gain: [8192, 8192] 13.3-13.7 / 12.4-12.8,
// [4096, 14336] 12.4-13.0 / 12.1-12.5).
constexpr int kRI8OneMaxK = 4096, kRI8OneMinN = 10240;

// 4x4x4 path: groups of 4 rows per wave and load steps in flight per lane,
// for fp16 / int8 W.  x is staged in LDS once per workgroup, so workgroups
// are large (b8_waves picks their size).  Measured
// at batch 8 on [14336, 4096], same box: int8 with 1, 2, 3, 4, 8 and 16
// steps in flight took 16.5, 12.6, 13.1, 14.9, 15.9 and 16.3 us (2 row
// groups per wave: 15.0-15.6 us); fp16 with 2, 4, 6, 8, 10, 12 and 16 took
// 22.0, 22.5, 21.7, 20.8, 20.9, 21.2 and 20.8 us.  With x staged in one
// phase fp16 takes 16 (kB8CplF16Whole): three alternating runs on each of two
// boxes gave 8 / 10 / 12 / 14 / 16 / 20 / 24 in flight 21.07-21.17 / 21.00-
// 21.04 / 21.5-21.6 / 21.13-21.22 / 20.85-20.97 / 21.9-22.0 / 27.2-27.4 us
// (no spills at 16; at 24 and more the ring no longer fits the registers);
// on a third box 16 and 8 tied (21.18-21.25 / 21.22-21.38 us).
// Phased x keeps 8: its kernels spill 32-64 bytes at 16.
constexpr int kB8RgF16 = 1, kB8CplF16 = 8, kB8CplF16Whole = 16, kB8RgI8 = 1, kB8CplI8 = 2;
// Below kB8SmallN rows the grid holds too few waves (4 rows each) to keep HBM
// busy with 2 int8 steps in flight per lane; 8 then pay.  N = 4096, K = 14336
// at batch 2 / 4 / 8: 22.1 / 22.6 / 45.0 us with 2, 16.2 / 16.8 / 33.9 with 8;
// N = 6144, K = 4096 at batch 4: 9.0 against 7.2 us.  At N = 14336 and 28672,
// batch 8, 8 in flight was slower (12.7 -> 16.3 and 23.6 -> 30.3 us).
constexpr int kB8SmallN = 8192, kB8CplI8Small = 8;
// Below kB8SplitN rows two waves share each row group, each sweeping half of
// K, so that the grid holds twice the waves: N = 4096, K = 14336 at batch 4 /
// 8: fp16 27.5 / 54.7 -> 22.1 / 44.0 us, int8 16.9 / 34.2 -> 13.7 / 27.0 us;
// N = 4096, K = 4096, batch 8: fp16 11.0 -> 9.5 us.  Loads in flight per
// lane: 8 fp16 / 4 int8 (4 / 8 and 16 / 2 were slower at most shapes).
constexpr int kB8SplitN = 8192, kB8CplF16Split = 8, kB8CplI8Split = 4;
// Up to 4096 rows with rows of at least 8192 values, four waves share each
// row group (2 int8 / 4 fp16 steps in flight per lane): [4096, 14336] batch
// 5 / 8, int8 17.7 / 18.5 -> 16.5 / 17.3 us, fp16 25.0 / 25.7 -> 24.2 /
// 25.1 us.  At N = 6144 (batch 8: 11.5 -> 14.0 us) and K = 4096 it lost.
constexpr int kB8Split4N = 4096, kB8Split4MinK = 8192, kB8CplF16Split4 = 4, kB8CplI8Split4 = 2;
constexpr int kB8MaxBatch = 8;

// Rows of x per launch of the VALU path (x [rows, K] staged in LDS): up to 8.
int vec_slice(int batch, int k) {
    long long rows = kMaxLdsBytes / (2LL * k);
    if (rows > 8) rows = 8;
    if (rows > batch) rows = batch;
    return static_cast<int>(rows);
}

// Waves per workgroup of the 4x4x4 path: of 16, 14, 12, 8 and 7, the one that
// leaves the busiest CU the fewest waves (ceil(workgroups / CUs) * waves; the
// first listed on ties), so that a grid just short of the CU count does not
// idle CUs: N = 14336 takes 14 waves and 256 workgroups (16 waves: 224).
// With K split over ks waves a workgroup covers nw / ks row groups (nw even).
int b8_waves(int N, int rows_per_wave, int ks) {
    const long long cus = tecoops::device_cus();
    int best = 16;
    long long best_load = -1;
    for (int nw : {16, 14, 12, 8, 7}) {
        if (nw % ks != 0) continue;
        const long long wgs =
            tecoops::ceil_div(N, static_cast<long long>(rows_per_wave) * (nw / ks));
        const long long load = (wgs + cus - 1) / cus * nw;
        if (best_load < 0 || load < best_load) {
            best_load = load;
            best = nw;
        }
    }
    return best;
}

// LDS bytes of the 4x4x4 path: staged x (kp values of 4 * ncg rows), plus
// the partial sums the ks - 1 other parts of each row group hand to part 0.
size_t b8_lds(int ncg, int rg, int nw, int ks, int kp) {
    return 4 * ncg * static_cast<size_t>(kp) * 2 +
           static_cast<size_t>(rg) * ncg * 4 * (nw / ks) * 64 * 4 * (ks - 1);
}

// Phases the 4x4x4 path sweeps K in (x staged one phase at a time): the
// fewest equal phases, each a whole number of load steps for each of the ks
// waves of a row group, whose LDS fits; 0 if none up to kB8MaxPhases does.
constexpr int kB8MaxPhases = 8;
int b8_phases(int ncg, int rg, int ks, int k, bool i8) {
    const int step = (i8 ? 256 : 128) * ks;  // k values per load step of all ks waves
    for (int nph = 1; nph <= kB8MaxPhases; ++nph)
        if (k % (nph * step) == 0 &&
            b8_lds(ncg, rg, 16, ks, k / nph) <= static_cast<size_t>(kMaxLdsBytes))
            return nph;
    return 0;
}

// Rows of x the 4x4x4 path takes per launch for this batch and K (0: the
// path does not apply): the whole batch when its staged x (4 or 8 rows) fits
// in LDS in at most kB8MaxPhases phases, else slices of 4 rows, each launch
// streaming W once.
int b8_slice(int batch, int k, bool i8) {
    if (batch > kB8MaxBatch) return 0;
    const int rg = i8 ? kB8RgI8 : kB8RgF16;
    if (b8_phases(batch <= 4 ? 1 : 2, rg, 1, k, i8) > 0) return batch;
    return b8_phases(1, rg, 1, k, i8) > 0 ? 4 : 0;
}

template <typename T, bool I8, int NCG, int NW, int CPL, int KS, bool PHASED>
bool launch_b8_ph(const void *W, const void *sc, const void *x, void *y, int B, int N, int K,
                  int nph, hipStream_t s) {
    constexpr int RG = I8 ? kB8RgI8 : kB8RgF16;
    const size_t lds = b8_lds(NCG, RG, NW, KS, K / nph);
    auto *kern = &gemv_b8_kernel<T, I8, NCG, RG, NW, CPL, KS, PHASED>;
    if (!tecoops::reserve_lds(reinterpret_cast<const void *>(kern), lds)) return false;
    hipLaunchKernelGGL(kern, dim3(tecoops::ceil_div(N, 4 * RG * (NW / KS))), dim3(NW * 64), lds, s,
                       static_cast<const uint4 *>(W), static_cast<const uint16_t *>(sc),
                       static_cast<const uint4 *>(x), static_cast<uint16_t *>(y), N, K, B, nph);
    return true;
}

template <typename T, bool I8, int NCG, int NW, int CPL, int KS>
bool launch_b8_nw(const void *W, const void *sc, const void *x, void *y, int B, int N, int K,
                  int nph, hipStream_t s) {
    if (nph > 1) return launch_b8_ph<T, I8, NCG, NW, CPL, KS, true>(W, sc, x, y, B, N, K, nph, s);
    return launch_b8_ph<T, I8, NCG, NW, CPL, KS, false>(W, sc, x, y, B, N, K, 1, s);
}

template <typename T, bool I8, int NCG, int CPL, int KS>
bool launch_b8_cpl(const void *W, const void *sc, const void *x, void *y, int B, int N, int K,
                   int nph, hipStream_t s) {
    switch (b8_waves(N, 4 * (I8 ? kB8RgI8 : kB8RgF16), KS)) {
        case 14:
            if constexpr (14 % KS == 0)
                return launch_b8_nw<T, I8, NCG, 14, CPL, KS>(W, sc, x, y, B, N, K, nph, s);
            return false;
        case 12: return launch_b8_nw<T, I8, NCG, 12, CPL, KS>(W, sc, x, y, B, N, K, nph, s);
        case 8: return launch_b8_nw<T, I8, NCG, 8, CPL, KS>(W, sc, x, y, B, N, K, nph, s);
        case 7:
            if constexpr (KS == 1)
                return launch_b8_nw<T, I8, NCG, 7, CPL, KS>(W, sc, x, y, B, N, K, nph, s);
            return false;
        default: return launch_b8_nw<T, I8, NCG, 16, CPL, KS>(W, sc, x, y, B, N, K, nph, s);
    }
}

template <typename T, bool I8, int NCG>
bool launch_b8_ncg(const void *W, const void *sc, const void *x, void *y, int B, int N, int K,
                   hipStream_t s) {
    constexpr int RG = I8 ? kB8RgI8 : kB8RgF16;
    if (N <= kB8Split4N && K >= kB8Split4MinK) {  // K split over four waves
        const int nph = b8_phases(NCG, RG, 4, K, I8);
        if (nph > 0)
            return launch_b8_cpl<T, I8, NCG, I8 ? kB8CplI8Split4 : kB8CplF16Split4, 4>(
                W, sc, x, y, B, N, K, nph, s);
    }
    if (N < kB8SplitN) {  // K split over the two waves of each row group
        const int nph = b8_phases(NCG, RG, 2, K, I8);
        if (nph > 0)
            return launch_b8_cpl<T, I8, NCG, I8 ? kB8CplI8Split : kB8CplF16Split, 2>(
                W, sc, x, y, B, N, K, nph, s);
    }
    const int nph = b8_phases(NCG, RG, 1, K, I8);
    if (nph == 0) return false;
    if (I8 && N < kB8SmallN)
        return launch_b8_cpl<T, I8, NCG, kB8CplI8Small, 1>(W, sc, x, y, B, N, K, nph, s);
    if (!I8 && nph == 1)
        return launch_b8_cpl<T, I8, NCG, kB8CplF16Whole, 1>(W, sc, x, y, B, N, K, nph, s);
    return launch_b8_cpl<T, I8, NCG, I8 ? kB8CplI8 : kB8CplF16, 1>(W, sc, x, y, B, N, K, nph, s);
}

template <typename T, bool I8>
bool launch_b8(const void *W, const void *sc, const void *x, void *y, int B, int N, int K,
               hipStream_t s) {
    if (B <= 4) return launch_b8_ncg<T, I8, 1>(W, sc, x, y, B, N, K, s);
    return launch_b8_ncg<T, I8, 2>(W, sc, x, y, B, N, K, s);
}

template <typename T, int B>
bool launch16(const void *W, const void *x, void *y, int N, int K, hipStream_t s) {
    const unsigned grid = tecoops::ceil_div(N, kWaves * kR16);
    auto *kern = &gemv16_kernel<T, B, kR16, kCpl16, kWaves>;
    if (!tecoops::reserve_lds(reinterpret_cast<const void *>(kern), B * static_cast<size_t>(K) * 2))
        return false;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads),
                       B * K * 2, s, static_cast<const uint4 *>(W), static_cast<const uint4 *>(x),
                       static_cast<uint16_t *>(y), N, K);
    return true;
}

template <int B, int R>
bool launch_i8_r(const void *W, const void *sc, const void *x, void *y, int N, int K,
                 hipStream_t s) {
    const unsigned grid = tecoops::ceil_div(N, kWaves * R);
    auto *kern = &gemv_i8_kernel<B, R, kCplI8, kWaves>;
    if (!tecoops::reserve_lds(reinterpret_cast<const void *>(kern), B * static_cast<size_t>(K) * 2))
        return false;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads),
                       B * K * 2, s, static_cast<const uint4 *>(W),
                       static_cast<const uint16_t *>(sc), static_cast<const uint4 *>(x),
                       static_cast<uint16_t *>(y), N, K);
    return true;
}

template <int B>
bool launch_i8(const void *W, const void *sc, const void *x, void *y, int N, int K,
               hipStream_t s) {
    if constexpr (B == 1)
        if (K <= kRI8OneMaxK && N >= kRI8OneMinN) return launch_i8_r<B, 1>(W, sc, x, y, N, K, s);
    return launch_i8_r<B, kRI8>(W, sc, x, y, N, K, s);
}

template <typename T>
bool launch16_b(int B, const void *W, const void *x, void *y, int N, int K, hipStream_t s) {
    switch (B) {
        case 1: return launch16<T, 1>(W, x, y, N, K, s);
        case 2: return launch16<T, 2>(W, x, y, N, K, s);
        case 3: return launch16<T, 3>(W, x, y, N, K, s);
        case 4: return launch16<T, 4>(W, x, y, N, K, s);
        case 5: return launch16<T, 5>(W, x, y, N, K, s);
        case 6: return launch16<T, 6>(W, x, y, N, K, s);
        case 7: return launch16<T, 7>(W, x, y, N, K, s);
        default: return launch16<T, 8>(W, x, y, N, K, s);
    }
}

bool launch_i8_b(int B, const void *W, const void *sc, const void *x, void *y, int N, int K,
                 hipStream_t s) {
    switch (B) {
        case 1: return launch_i8<1>(W, sc, x, y, N, K, s);
        case 2: return launch_i8<2>(W, sc, x, y, N, K, s);
        case 3: return launch_i8<3>(W, sc, x, y, N, K, s);
        case 4: return launch_i8<4>(W, sc, x, y, N, K, s);
        case 5: return launch_i8<5>(W, sc, x, y, N, K, s);
        case 6: return launch_i8<6>(W, sc, x, y, N, K, s);
        case 7: return launch_i8<7>(W, sc, x, y, N, K, s);
        default: return launch_i8<8>(W, sc, x, y, N, K, s);
    }
}

}  // namespace

extern "C" tecoopsStatus_t tecoopsGemv(tecoopsHandle_t handle, const void *weight, const void *x,
                                       void *y, int batch, int n, int k,
                                       tecoopsDataType_t dataType) {
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (weight == nullptr || x == nullptr || y == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    if (batch <= 0 || n <= 0 || k <= 0) return TECOOPS_STATUS_BAD_PARAM;
    if (!tecoops::is_16bit_float(dataType)) return TECOOPS_STATUS_BAD_PARAM;
    using tecoops::dev::bf16;
    using tecoops::dev::f16;
    hipStream_t s = handle->stream;
    const bool al = tecoops::aligned(weight, 16) && tecoops::aligned(x, 16);
    const bool b8 = batch >= kMfmaMinBatch16 || (batch == 2 && k > kB8Batch2MinK);
    const int s8 = b8 && al ? b8_slice(batch, k, false) : 0;
    if (s8 > 0) {
        for (int b0 = 0; b0 < batch; b0 += s8) {
            const int nb = batch - b0 < s8 ? batch - b0 : s8;
            const void *xb = static_cast<const uint16_t *>(x) + static_cast<long long>(b0) * k;
            void *yb = static_cast<uint16_t *>(y) + static_cast<long long>(b0) * n;
            const bool ok = dataType == TECOOPS_DATA_HALF
                                ? launch_b8<f16, false>(weight, nullptr, xb, yb, nb, n, k, s)
                                : launch_b8<bf16, false>(weight, nullptr, xb, yb, nb, n, k, s);
            if (!ok) return TECOOPS_STATUS_INTERNAL_ERROR;
            TECO_CHECK_LAUNCH("gemv");
        }
        return TECOOPS_STATUS_SUCCESS;
    }
    if (batch >= kMfmaMinBatch16 && (k % 32) == 0 && tecoops::aligned(weight, 16) &&
        tecoops::aligned(x, 16)) {
        constexpr int RT = kMfmaRT16, NW = kMfmaWaves16;
        for (int b0 = 0; b0 < batch; b0 += 16) {
            const int nb = batch - b0 < 16 ? batch - b0 : 16;
            const uint16_t *xb = static_cast<const uint16_t *>(x) + static_cast<long long>(b0) * k;
            uint16_t *yb = static_cast<uint16_t *>(y) + static_cast<long long>(b0) * n;
            const unsigned grid = tecoops::ceil_div(n, 16 * RT);
            if (dataType == TECOOPS_DATA_HALF)
                hipLaunchKernelGGL((gemv16_mfma_kernel<f16, RT, NW>), dim3(grid), dim3(NW * 64), 0,
                                   s, static_cast<const uint16_t *>(weight), xb, yb, n, k, nb);
            else
                hipLaunchKernelGGL((gemv16_mfma_kernel<bf16, RT, NW>), dim3(grid), dim3(NW * 64),
                                   0, s, static_cast<const uint16_t *>(weight), xb, yb, n, k, nb);
            TECO_CHECK_LAUNCH("gemv");
        }
        return TECOOPS_STATUS_SUCCESS;
    }
    const int sv = (k % 8) == 0 && al ? vec_slice(batch, k) : 0;
    if (sv > 0) {
        // Batches beyond the slice (8 rows of x / y, fewer for long rows) run
        // in slices.
        for (int b0 = 0; b0 < batch; b0 += sv) {
            const int nb = batch - b0 < sv ? batch - b0 : sv;
            const void *xb = static_cast<const uint16_t *>(x) + static_cast<long long>(b0) * k;
            void *yb = static_cast<uint16_t *>(y) + static_cast<long long>(b0) * n;
            const bool ok = dataType == TECOOPS_DATA_HALF
                                ? launch16_b<f16>(nb, weight, xb, yb, n, k, s)
                                : launch16_b<bf16>(nb, weight, xb, yb, n, k, s);
            if (!ok) return TECOOPS_STATUS_INTERNAL_ERROR;
            TECO_CHECK_LAUNCH("gemv");
        }
        return TECOOPS_STATUS_SUCCESS;
    }
    const unsigned grid = tecoops::ceil_div(static_cast<long long>(n) * batch, kWaves);
    if (dataType == TECOOPS_DATA_HALF)
        hipLaunchKernelGGL((gemv_scalar_kernel<f16, false>), dim3(grid), dim3(kThreads), 0, s,
                           weight, nullptr, static_cast<const uint16_t *>(x),
                           static_cast<uint16_t *>(y), n, k, batch);
    else
        hipLaunchKernelGGL((gemv_scalar_kernel<bf16, false>), dim3(grid), dim3(kThreads), 0, s,
                           weight, nullptr, static_cast<const uint16_t *>(x),
                           static_cast<uint16_t *>(y), n, k, batch);
    TECO_CHECK_LAUNCH("gemv");
    return TECOOPS_STATUS_SUCCESS;
}

extern "C" tecoopsStatus_t tecoopsGemvInt8(tecoopsHandle_t handle, const int8_t *weight,
                                           const void *scales, const void *x, void *y,
                                           int batch, int n, int k) {
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (weight == nullptr || scales == nullptr || x == nullptr || y == nullptr)
        return TECOOPS_STATUS_BAD_PARAM;
    if (batch <= 0 || n <= 0 || k <= 0) return TECOOPS_STATUS_BAD_PARAM;
    using tecoops::dev::f16;
    hipStream_t s = handle->stream;
    const bool al = tecoops::aligned(weight, 16) && tecoops::aligned(x, 16);
    const int s8 = batch >= kMfmaMinBatchI8 && al ? b8_slice(batch, k, true) : 0;
    if (s8 > 0) {
        for (int b0 = 0; b0 < batch; b0 += s8) {
            const int nb = batch - b0 < s8 ? batch - b0 : s8;
            const void *xb = static_cast<const uint16_t *>(x) + static_cast<long long>(b0) * k;
            void *yb = static_cast<uint16_t *>(y) + static_cast<long long>(b0) * n;
            if (!launch_b8<f16, true>(weight, scales, xb, yb, nb, n, k, s))
                return TECOOPS_STATUS_INTERNAL_ERROR;
            TECO_CHECK_LAUNCH("gemv_int8");
        }
        return TECOOPS_STATUS_SUCCESS;
    }
    if (batch >= kMfmaMinBatchI8 && (k % 64) == 0 && tecoops::aligned(weight, 16) &&
        tecoops::aligned(x, 16)) {
        constexpr int RT = kMfmaRTI8, NW = kMfmaWavesI8;
        for (int b0 = 0; b0 < batch; b0 += 16) {
            const int nb = batch - b0 < 16 ? batch - b0 : 16;
            const uint16_t *xb = static_cast<const uint16_t *>(x) + static_cast<long long>(b0) * k;
            uint16_t *yb = static_cast<uint16_t *>(y) + static_cast<long long>(b0) * n;
            hipLaunchKernelGGL((gemv_i8_mfma_kernel<RT, NW>), dim3(tecoops::ceil_div(n, 16 * RT)),
                               dim3(NW * 64), 0, s, weight, static_cast<const uint16_t *>(scales),
                               xb, yb, n, k, nb);
            TECO_CHECK_LAUNCH("gemv_int8");
        }
        return TECOOPS_STATUS_SUCCESS;
    }
    const int sv = (k % 16) == 0 && al ? vec_slice(batch, k) : 0;
    if (sv > 0) {
        for (int b0 = 0; b0 < batch; b0 += sv) {
            const int nb = batch - b0 < sv ? batch - b0 : sv;
            const void *xb = static_cast<const uint16_t *>(x) + static_cast<long long>(b0) * k;
            void *yb = static_cast<uint16_t *>(y) + static_cast<long long>(b0) * n;
            if (!launch_i8_b(nb, weight, scales, xb, yb, n, k, s)) return TECOOPS_STATUS_INTERNAL_ERROR;
            TECO_CHECK_LAUNCH("gemv_int8");
        }
        return TECOOPS_STATUS_SUCCESS;
    }
    const unsigned grid = tecoops::ceil_div(static_cast<long long>(n) * batch, kWaves);
    hipLaunchKernelGGL((gemv_scalar_kernel<f16, true>), dim3(grid), dim3(kThreads), 0, s,
                       static_cast<const void *>(weight), static_cast<const uint16_t *>(scales),
                       static_cast<const uint16_t *>(x), static_cast<uint16_t *>(y), n, k, batch);
    TECO_CHECK_LAUNCH("gemv_int8");
    return TECOOPS_STATUS_SUCCESS;
}
