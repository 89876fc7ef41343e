// rotary.hip — in-place rotary position embedding on query and key.
//
// No reference implementation: rotary is absent from the reference library.
// The signature mirrors the vLLM-style rotary_embedding(positions, query, key,
// head_size, cos_sin_cache, is_neox) that the reference's other ops follow.
// theta_i = pos * base^(-2i/rot_dim); NeoX pairs (i, i + rot_dim/2), GPT-J
// pairs (2i, 2i+1):  o1 = x1 cos - x2 sin,  o2 = x2 cos + x1 sin  (fp32 math).
//
// gfx950 design: one workgroup per token.  The rot_dim/2 (cos, sin) pairs
// of each token are computed once (accurate sincosf, or read from the cache)
// into LDS and shared by all H + Hkv heads; each lane then rotates 8 NeoX
// pairs per task with two 16-byte loads and stores (4 pairs with 8-byte words
// when only 8-byte alignment holds; 4 GPT-J pairs per 16-byte word), streamed
// with the non-temporal policy.  On the 16-byte NeoX path a thread issues the
// loads of several tasks before any store (one memory round trip per batch
// instead of per task).  HBM-bound: every byte of q and k is read once and
// written once.
#include "common.h"
#include "device.h"

namespace {

using namespace tecoops::dev;

constexpr int kThreads = 256;
constexpr int kMaxHalf = 256;  // rot_dim <= 512

// One token per workgroup, each thread's (at most two) tasks loaded together
// before any store.  More tokens per workgroup put more of q and k in flight
// at once, which the memory system serves slower.  q [8192, 32, 128], k
// [8192, 8, 128], NeoX, µs rotary / fused rotary + cache (tokens per
// workgroup, tasks in flight per thread, 256 threads unless noted): 1, 2:
// 28.5 / 36.3-36.5; 2, 3: 29.4 / 36.6-36.8; 4, 6 (8 fused): 29.4 / 37.0-37.2;
// 8, 5: 31.8 / 41.7; 16, 10: 34.2 / 43.0; 1 token with 128 / 192 / 320 / 384
// threads: 29.6-29.7 / 28.9 / 29.1-29.3 / 29.6 (fused 37.5-37.7 / 36.4-36.5
// / 37.5-37.6 / 42.3).
constexpr int kTokensPerBlock = 1;
constexpr int kRotBatch = 2;  // rotation tasks per thread with loads in flight together
constexpr int kFusedBatch = 2;  // tasks per thread in flight together, fused kernel

// o1 = x1 cos - x2 sin, o2 = x2 cos + x1 sin with the roundings spelled out
// (one product, then one fused multiply-add), so every kernel that rotates
// gets bit-identical results whatever the compiler would contract.
__device__ __forceinline__ float rot1(float x1, float x2, float c, float s) {
    return fmaf(x1, c, -(x2 * s));
}
__device__ __forceinline__ float rot2(float x1, float x2, float c, float s) {
    return fmaf(x2, c, x1 * s);
}

// Rotation of 4 NeoX pairs (x1 = a, x2 = b, 4 elements each, as 8-byte words)
// with (cos, sin) c[0..3]: o1 = x1 cos - x2 sin, o2 = x2 cos + x1 sin.
template <typename T>
__device__ __forceinline__ void rot_neox4(const uint2 &a, const uint2 &b, const float2 *c,
                                          uint2 &oa, uint2 &ob) {
    const uint32_t pa[2] = {a.x, a.y}, pb[2] = {b.x, b.y};
    uint32_t qa[2], qb[2];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        const float2 c0 = c[2 * w], c1 = c[2 * w + 1];
        const float x10 = lo<T>(pa[w]), x11 = hi<T>(pa[w]);
        const float x20 = lo<T>(pb[w]), x21 = hi<T>(pb[w]);
        qa[w] = pack<T>(rot1(x10, x20, c0.x, c0.y), rot1(x11, x21, c1.x, c1.y));
        qb[w] = pack<T>(rot2(x10, x20, c0.x, c0.y), rot2(x11, x21, c1.x, c1.y));
    }
    oa = make_uint2(qa[0], qa[1]);
    ob = make_uint2(qb[0], qb[1]);
}

// Rotation of 8 NeoX pairs (x1 = a, x2 = b, 8 elements each, as 16-byte words).
template <typename T>
__device__ __forceinline__ void rot_neox8(const uint4 &a, const uint4 &b, const float2 *c,
                                          uint4 &oa, uint4 &ob) {
    uint2 lo_a, lo_b, hi_a, hi_b;
    rot_neox4<T>(make_uint2(a.x, a.y), make_uint2(b.x, b.y), c, lo_a, lo_b);
    rot_neox4<T>(make_uint2(a.z, a.w), make_uint2(b.z, b.w), c + 4, hi_a, hi_b);
    oa = make_uint4(lo_a.x, lo_a.y, hi_a.x, hi_a.y);
    ob = make_uint4(lo_b.x, lo_b.y, hi_b.x, hi_b.y);
}

// Rotation of 4 adjacent GPT-J pairs packed in 16 bytes.
template <typename T>
__device__ __forceinline__ uint4 rot_gptj4(const uint4 &a, const float2 *c) {
    uint32_t pa[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float2 cc = c[w];
        const float x1 = lo<T>(pa[w]), x2 = hi<T>(pa[w]);
        pa[w] = pack<T>(rot1(x1, x2, cc.x, cc.y), rot2(x1, x2, cc.x, cc.y));
    }
    return make_uint4(pa[0], pa[1], pa[2], pa[3]);
}

// One pair, scalar.
template <typename T>
__device__ __forceinline__ void rot_pair(uint16_t x1b, uint16_t x2b, float2 cc, uint16_t &o1,
                                         uint16_t &o2) {
    const float x1 = Cvt<T>::to(x1b), x2 = Cvt<T>::to(x2b);
    o1 = Cvt<T>::from(rot1(x1, x2, cc.x, cc.y));
    o2 = Cvt<T>::from(rot2(x1, x2, cc.x, cc.y));
}

// VW: 0 one pair per task; 1 four pairs (8-byte NeoX / 16-byte GPT-J words);
// 2 eight NeoX pairs (16-byte words).  q and k are streamed (non-temporal).
template <typename T, bool NEOX, int VW>
__global__ void __launch_bounds__(kThreads)
rotary_kernel(const int64_t *__restrict__ positions, uint16_t *__restrict__ query,
              uint16_t *__restrict__ key, int num_tokens, int num_heads, int num_kv_heads,
              int head_size, int rot_dim, long long q_stride, long long k_stride,
              const float *__restrict__ cos_sin_cache, int max_position, float log2_base) {
    __shared__ float2 cs[kTokensPerBlock][kMaxHalf];
    __shared__ int skip[kTokensPerBlock];
    const int half = rot_dim >> 1;
    const int tbase = blockIdx.x * kTokensPerBlock;
    for (int e = threadIdx.x; e < kTokensPerBlock * half; e += blockDim.x) {
        const int tt = e / half, i = e - tt * half;
        const int t = tbase + tt;
        if (t >= num_tokens) continue;
        const int64_t pos = positions[t];
        float c = 1.0f, s = 0.0f;
        if (cos_sin_cache != nullptr) {
            if (pos >= 0 && pos < max_position) {
                c = cos_sin_cache[pos * rot_dim + i];
                s = cos_sin_cache[pos * rot_dim + half + i];
            }
        } else {
            const float inv_freq = exp2f(-(2.0f * i / static_cast<float>(rot_dim)) * log2_base);
            sincosf(static_cast<float>(pos) * inv_freq, &s, &c);
        }
        cs[tt][i] = make_float2(c, s);
    }
    if (threadIdx.x < kTokensPerBlock) {
        const int t = tbase + threadIdx.x;
        int sk = t >= num_tokens;
        if (!sk && cos_sin_cache != nullptr) {
            const int64_t pos = positions[t];
            sk = pos < 0 || pos >= max_position;
        }
        skip[threadIdx.x] = sk;
    }
    __syncthreads();
    constexpr int P = VW == 2 ? 8 : VW == 1 ? 4 : 1;  // pairs per lane-task
    const int tasks_per_head = half / P;
    const int heads = num_heads + (key ? num_kv_heads : 0);
    const int per_token = heads * tasks_per_head;
    if constexpr (NEOX && VW == 2) {
        // A thread's tasks (threadIdx.x + kThreads * u) load their 16-byte
        // words kRotBatch at a time before any rotation or store, so each
        // pass costs one memory round trip instead of one per task.  The
        // loads are unconditional, at the last task / token when past the
        // end, so the compiler waits for each at its use.
        const int total = kTokensPerBlock * per_token;
        for (int base = threadIdx.x; base < total; base += kThreads * kRotBatch) {
            uint4 xa[kRotBatch], xb[kRotBatch];
            uint16_t *rp[kRotBatch];
            int ci[kRotBatch];  // cs offset of the task's first pair, or -1: no store
#pragma unroll
            for (int u = 0; u < kRotBatch; ++u) {
                const int task = min(base + kThreads * u, total - 1);
                const int tt = task / per_token;
                const int local0 = task - tt * per_token;
                const bool is_q = local0 < num_heads * tasks_per_head;
                const int local = is_q ? local0 : local0 - num_heads * tasks_per_head;
                const int h = local / tasks_per_head;
                const int i0 = (local - h * tasks_per_head) * P;
                const long long t = min(tbase + tt, num_tokens - 1);
                uint16_t *row = (is_q ? query + t * q_stride : key + t * k_stride) + h * head_size + i0;
                rp[u] = row;
                xa[u] = ld_stream(reinterpret_cast<const uint4 *>(row));
                xb[u] = ld_stream(reinterpret_cast<const uint4 *>(row + half));
                ci[u] = (base + kThreads * u < total && !skip[tt]) ? tt * kMaxHalf + i0 : -1;
            }
#pragma unroll
            for (int u = 0; u < kRotBatch; ++u) {
                if (ci[u] < 0) continue;
                uint4 oa, ob;
                rot_neox8<T>(xa[u], xb[u], &cs[0][0] + ci[u], oa, ob);
                st_stream(reinterpret_cast<uint4 *>(rp[u]), oa);
                st_stream(reinterpret_cast<uint4 *>(rp[u] + half), ob);
            }
        }
        return;
    }
    for (int task = threadIdx.x; task < kTokensPerBlock * per_token; task += blockDim.x) {
        const int tt = task / per_token;
        if (skip[tt]) continue;
        const int t = tbase + tt;
        const int local0 = task - tt * per_token;
        const bool is_q = local0 < num_heads * tasks_per_head;
        const int local = is_q ? local0 : local0 - num_heads * tasks_per_head;
        const int h = local / tasks_per_head;
        const int i0 = (local - h * tasks_per_head) * P;
        const float2 *c = cs[tt];
        uint16_t *row = (is_q ? query + t * q_stride : key + t * k_stride) + h * head_size;
        if (NEOX) {
            if (VW == 2) {
                uint4 *p1 = reinterpret_cast<uint4 *>(row + i0);
                uint4 *p2 = reinterpret_cast<uint4 *>(row + half + i0);
                uint4 oa, ob;
                rot_neox8<T>(ld_stream(p1), ld_stream(p2), c + i0, oa, ob);
                st_stream(p1, oa);
                st_stream(p2, ob);
            } else if (VW == 1) {
                uint2 *p1 = reinterpret_cast<uint2 *>(row + i0);
                uint2 *p2 = reinterpret_cast<uint2 *>(row + half + i0);
                uint2 oa, ob;
                rot_neox4<T>(*p1, *p2, c + i0, oa, ob);
                *p1 = oa;
                *p2 = ob;
            } else {
                rot_pair<T>(row[i0], row[half + i0], c[i0], row[i0], row[half + i0]);
            }
        } else {
            if (VW >= 1) {
                uint4 *pp = reinterpret_cast<uint4 *>(row + 2 * i0);
                st_stream(pp, rot_gptj4<T>(ld_stream(pp), c + i0));
            } else {
                rot_pair<T>(row[2 * i0], row[2 * i0 + 1], c[i0], row[2 * i0], row[2 * i0 + 1]);
            }
        }
    }
}

// Fused decode-step kernel: rotary on query (in place) and key, rotated key
// and value written straight into the paged caches [num_blocks, Hkv,
// block_size, D] at slot_mapping[t] (key also written back in place when
// write_key).  Same cos / sin and rotation arithmetic as rotary_kernel, so the
// cache holds exactly what rotary_embedding followed by reshape_and_cache
// would store.  A token whose position is outside the cos/sin cache is not
// rotated (identity), as in rotary_kernel, but is still cached; slots < 0 or
// >= num_blocks * block_size are not cached, as in reshape_and_cache.
struct FusedArgs {
    const int64_t *positions;
    uint16_t *query;
    uint16_t *key;
    const uint16_t *value;
    const int64_t *slots;
    uint16_t *kcache;
    uint16_t *vcache;
    int num_tokens, num_heads, num_kv_heads, head_size, rot_dim;
    long long q_stride, k_stride, v_stride;
    const float *cos_sin_cache;
    int max_position;
    float log2_base;
    int block_size, lbs;  // lbs = log2(block_size) or -1
    long long capacity;   // num_blocks * block_size
    int write_key;
};

template <typename T, bool NEOX, int VW>
__global__ void __launch_bounds__(kThreads) rotary_cache_kernel(FusedArgs a) {
    __shared__ float2 cs[kTokensPerBlock][kMaxHalf];
    __shared__ long long crow[kTokensPerBlock];  // first element of the token's cache row, or -1
    const int half = a.rot_dim >> 1;
    const int D = a.head_size;
    const int tbase = blockIdx.x * kTokensPerBlock;
    for (int e = threadIdx.x; e < kTokensPerBlock * half; e += blockDim.x) {
        const int tt = e / half, i = e - tt * half;
        const int t = tbase + tt;
        if (t >= a.num_tokens) continue;
        const int64_t pos = a.positions[t];
        float c = 1.0f, sn = 0.0f;
        if (a.cos_sin_cache != nullptr) {
            if (pos >= 0 && pos < a.max_position) {
                c = a.cos_sin_cache[pos * a.rot_dim + i];
                sn = a.cos_sin_cache[pos * a.rot_dim + half + i];
            }
        } else {
            const float inv_freq = exp2f(-(2.0f * i / static_cast<float>(a.rot_dim)) * a.log2_base);
            sincosf(static_cast<float>(pos) * inv_freq, &sn, &c);
        }
        cs[tt][i] = make_float2(c, sn);
    }
    if (threadIdx.x < kTokensPerBlock) {
        const int t = tbase + threadIdx.x;
        long long r = -1;
        if (t < a.num_tokens) {
            const int64_t slot = a.slots[t];
            if (slot >= 0 && slot < a.capacity) {
                const int s32 = static_cast<int>(slot);
                const int blk = a.lbs >= 0 ? s32 >> a.lbs : s32 / a.block_size;
                const int off = a.lbs >= 0 ? s32 & (a.block_size - 1) : s32 - blk * a.block_size;
                r = (static_cast<long long>(blk) * a.num_kv_heads * a.block_size + off) * D;
            }
        }
        crow[threadIdx.x] = r;
    }
    __syncthreads();
    constexpr bool VEC = VW >= 1;
    constexpr int P = VW == 2 ? 8 : VW == 1 ? 4 : 1;  // rotation pairs per task
    constexpr int CV = VEC ? 8 : 1;                   // elements per copy task
    const int rot_tasks = half / P;       // per head
    const int tail = D - a.rot_dim;       // key elements past rot_dim: copied unrotated
    const int tail_tasks = (tail + CV - 1) / CV;
    const int v_tasks = D / CV;
    const int nq = a.num_heads * rot_tasks;
    const int nk = a.num_kv_heads * (rot_tasks + tail_tasks);
    const int per_token = nq + nk + a.num_kv_heads * v_tasks;
    const long long head_stride = static_cast<long long>(a.block_size) * D;  // cache, per kv head
    if constexpr (NEOX && VW == 2) {
        if (tail_tasks == 0) {
            // As in rotary_kernel: each pass loads the 16-byte words of
            // kFusedBatch tasks of this thread before any rotation or store.
            // Every task issues two unconditional loads from selected
            // addresses (a value copy loads its word twice), clamped to the
            // last task / token past the end.
            const int total = kTokensPerBlock * per_token;
            for (int base = threadIdx.x; base < total; base += kThreads * kFusedBatch) {
                uint4 xa[kFusedBatch], xb[kFusedBatch];
                uint16_t *d0[kFusedBatch];  // in-place row (q, or k when write_key) or null
                uint16_t *d1[kFusedBatch];  // cache row or null
                int ci[kFusedBatch];        // cs offset of the first pair; -1: value copy
#pragma unroll
                for (int u = 0; u < kFusedBatch; ++u) {
                    const int task = min(base + kThreads * u, total - 1);
                    const int tt = task / per_token;
                    const int t = tbase + tt;
                    const long long tl = min(t, a.num_tokens - 1);
                    const bool live = base + kThreads * u < total && t < a.num_tokens;
                    const long long cr = crow[tt];
                    int local = task - tt * per_token;
                    const uint16_t *s0, *s1;
                    uint16_t *w0 = nullptr, *w1 = nullptr;
                    int c = -1;
                    if (local < nq) {  // query head: rotate in place
                        const int h = local / rot_tasks;
                        const int i0 = (local - h * rot_tasks) * P;
                        uint16_t *row = a.query + tl * a.q_stride + h * D + i0;
                        s0 = row;
                        s1 = row + half;
                        w0 = row;
                        c = tt * kMaxHalf + i0;
                    } else if ((local -= nq) < nk) {  // key head: rotate, cache (and write back)
                        const int h = local / rot_tasks;
                        const int i0 = (local - h * rot_tasks) * P;
                        uint16_t *row = a.key + tl * a.k_stride + h * D + i0;
                        s0 = row;
                        s1 = row + half;
                        if (a.write_key) w0 = row;
                        if (cr >= 0) w1 = a.kcache + cr + h * head_stride + i0;
                        c = tt * kMaxHalf + i0;
                    } else {  // value head: copy into the cache
                        local -= nk;
                        const int h = local / v_tasks;
                        const int e0 = (local - h * v_tasks) * CV;
                        s0 = s1 = a.value + tl * a.v_stride + h * D + e0;
                        if (cr >= 0) w1 = a.vcache + cr + h * head_stride + e0;
                    }
                    xa[u] = ld_stream(reinterpret_cast<const uint4 *>(s0));
                    xb[u] = ld_stream(reinterpret_cast<const uint4 *>(s1));
                    d0[u] = live ? w0 : nullptr;
                    d1[u] = live ? w1 : nullptr;
                    ci[u] = c;
                }
#pragma unroll
                for (int u = 0; u < kFusedBatch; ++u) {
                    if (ci[u] < 0) {
                        if (d1[u] != nullptr) st_stream(reinterpret_cast<uint4 *>(d1[u]), xa[u]);
                        continue;
                    }
                    uint4 oa, ob;
                    rot_neox8<T>(xa[u], xb[u], &cs[0][0] + ci[u], oa, ob);
                    if (d0[u] != nullptr) {
                        st_stream(reinterpret_cast<uint4 *>(d0[u]), oa);
                        st_stream(reinterpret_cast<uint4 *>(d0[u] + half), ob);
                    }
                    if (d1[u] != nullptr) {
                        st_stream(reinterpret_cast<uint4 *>(d1[u]), oa);
                        st_stream(reinterpret_cast<uint4 *>(d1[u] + half), ob);
                    }
                }
            }
            return;
        }
    }
    for (int task = threadIdx.x; task < kTokensPerBlock * per_token; task += blockDim.x) {
        const int tt = task / per_token;
        const int t = tbase + tt;
        if (t >= a.num_tokens) continue;
        int local = task - tt * per_token;
        const float2 *c = cs[tt];
        const long long cr = crow[tt];
        if (local < nq) {  // query head: rotate in place
            const int h = local / rot_tasks;
            const int i0 = (local - h * rot_tasks) * P;
            uint16_t *row = a.query + t * a.q_stride + h * D;
            if (NEOX) {
                if (VW == 2) {
                    uint4 *p1 = reinterpret_cast<uint4 *>(row + i0);
                    uint4 *p2 = reinterpret_cast<uint4 *>(row + half + i0);
                    uint4 oa, ob;
                    rot_neox8<T>(ld_stream(p1), ld_stream(p2), c + i0, oa, ob);
                    st_stream(p1, oa);
                    st_stream(p2, ob);
                } else if (VEC) {
                    uint2 *p1 = reinterpret_cast<uint2 *>(row + i0);
                    uint2 *p2 = reinterpret_cast<uint2 *>(row + half + i0);
                    uint2 oa, ob;
                    rot_neox4<T>(*p1, *p2, c + i0, oa, ob);
                    *p1 = oa;
                    *p2 = ob;
                } else {
                    rot_pair<T>(row[i0], row[half + i0], c[i0], row[i0], row[half + i0]);
                }
            } else {
                if (VEC) {
                    uint4 *pp = reinterpret_cast<uint4 *>(row + 2 * i0);
                    st_stream(pp, rot_gptj4<T>(ld_stream(pp), c + i0));
                } else {
                    rot_pair<T>(row[2 * i0], row[2 * i0 + 1], c[i0], row[2 * i0], row[2 * i0 + 1]);
                }
            }
            continue;
        }
        local -= nq;
        if (local < nk) {  // key head: rotate, then cache (and write back)
            const int per_head = rot_tasks + tail_tasks;
            const int h = local / per_head;
            const int r = local - h * per_head;
            uint16_t *row = a.key + t * a.k_stride + h * D;
            uint16_t *dst = cr >= 0 ? a.kcache + cr + h * head_stride : nullptr;
            if (r >= rot_tasks) {  // unrotated tail
                const int e0 = a.rot_dim + (r - rot_tasks) * CV;
                if (dst != nullptr)
                    for (int e = e0; e < e0 + CV && e < D; ++e) dst[e] = row[e];
                continue;
            }
            const int i0 = r * P;
            if (NEOX) {
                if (VW == 2) {
                    uint4 oa, ob;
                    rot_neox8<T>(ld_stream(reinterpret_cast<const uint4 *>(row + i0)),
                                 ld_stream(reinterpret_cast<const uint4 *>(row + half + i0)), c + i0,
                                 oa, ob);
                    if (a.write_key) {
                        st_stream(reinterpret_cast<uint4 *>(row + i0), oa);
                        st_stream(reinterpret_cast<uint4 *>(row + half + i0), ob);
                    }
                    if (dst != nullptr) {
                        st_stream(reinterpret_cast<uint4 *>(dst + i0), oa);
                        st_stream(reinterpret_cast<uint4 *>(dst + half + i0), ob);
                    }
                } else if (VEC) {
                    uint2 oa, ob;
                    rot_neox4<T>(*reinterpret_cast<const uint2 *>(row + i0),
                                 *reinterpret_cast<const uint2 *>(row + half + i0), c + i0, oa, ob);
                    if (a.write_key) {
                        *reinterpret_cast<uint2 *>(row + i0) = oa;
                        *reinterpret_cast<uint2 *>(row + half + i0) = ob;
                    }
                    if (dst != nullptr) {
                        *reinterpret_cast<uint2 *>(dst + i0) = oa;
                        *reinterpret_cast<uint2 *>(dst + half + i0) = ob;
                    }
                } else {
                    uint16_t o1, o2;
                    rot_pair<T>(row[i0], row[half + i0], c[i0], o1, o2);
                    if (a.write_key) {
                        row[i0] = o1;
                        row[half + i0] = o2;
                    }
                    if (dst != nullptr) {
                        dst[i0] = o1;
                        dst[half + i0] = o2;
                    }
                }
            } else {
                if (VEC) {
                    const uint4 o = rot_gptj4<T>(ld_stream(reinterpret_cast<const uint4 *>(row + 2 * i0)), c + i0);
                    if (a.write_key) st_stream(reinterpret_cast<uint4 *>(row + 2 * i0), o);
                    if (dst != nullptr) st_stream(reinterpret_cast<uint4 *>(dst + 2 * i0), o);
                } else {
                    uint16_t o1, o2;
                    rot_pair<T>(row[2 * i0], row[2 * i0 + 1], c[i0], o1, o2);
                    if (a.write_key) {
                        row[2 * i0] = o1;
                        row[2 * i0 + 1] = o2;
                    }
                    if (dst != nullptr) {
                        dst[2 * i0] = o1;
                        dst[2 * i0 + 1] = o2;
                    }
                }
            }
            continue;
        }
        local -= nk;
        if (cr < 0) continue;  // value head: copy into the cache
        const int h = local / v_tasks;
        const int e0 = (local - h * v_tasks) * CV;
        const uint16_t *src = a.value + t * a.v_stride + h * D + e0;
        uint16_t *dst = a.vcache + cr + h * head_stride + e0;
        if (VEC)
            st_stream(reinterpret_cast<uint4 *>(dst), ld_stream(reinterpret_cast<const uint4 *>(src)));
        else
            *dst = *src;
    }
}

template <typename T, bool NEOX, int VW>
void launch_vw(int T_, hipStream_t s, const int64_t *pos, void *q, void *k, int H, int Hkv, int D,
               int rot, long long qs, long long ks, const float *cache, int maxpos, float lb) {
    const unsigned grid = tecoops::ceil_div(T_, kTokensPerBlock);
    hipLaunchKernelGGL((rotary_kernel<T, NEOX, VW>), dim3(grid), dim3(kThreads), 0, s, pos,
                       static_cast<uint16_t *>(q), static_cast<uint16_t *>(k), T_, H, Hkv, D, rot,
                       qs, ks, cache, maxpos, lb);
}

template <typename T, bool NEOX>
void launch(int vw, int T_, hipStream_t s, const int64_t *pos, void *q, void *k, int H,
            int Hkv, int D, int rot, long long qs, long long ks, const float *cache, int maxpos,
            float lb) {
    if (vw == 2)
        launch_vw<T, NEOX, NEOX ? 2 : 1>(T_, s, pos, q, k, H, Hkv, D, rot, qs, ks, cache, maxpos, lb);
    else if (vw == 1)
        launch_vw<T, NEOX, 1>(T_, s, pos, q, k, H, Hkv, D, rot, qs, ks, cache, maxpos, lb);
    else
        launch_vw<T, NEOX, 0>(T_, s, pos, q, k, H, Hkv, D, rot, qs, ks, cache, maxpos, lb);
}

}  // namespace

extern "C" tecoopsStatus_t tecoopsRotaryEmbedding(tecoopsHandle_t handle,
                                                  const int64_t *positions, void *query,
                                                  void *key, int num_tokens, int num_heads,
                                                  int num_kv_heads, int head_size, int rot_dim,
                                                  long long query_stride, long long key_stride,
                                                  const float *cos_sin_cache, int max_position,
                                                  float base, int is_neox,
                                                  tecoopsDataType_t dataType) {
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (positions == nullptr || query == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    if (num_tokens <= 0 || num_heads <= 0 || head_size <= 0) return TECOOPS_STATUS_BAD_PARAM;
    if (key != nullptr && num_kv_heads <= 0) return TECOOPS_STATUS_BAD_PARAM;
    if (rot_dim <= 0 || (rot_dim & 1) || rot_dim > head_size || rot_dim / 2 > kMaxHalf)
        return TECOOPS_STATUS_BAD_PARAM;
    if (query_stride < static_cast<long long>(num_heads) * head_size) return TECOOPS_STATUS_BAD_PARAM;
    if (key != nullptr && key_stride < static_cast<long long>(num_kv_heads) * head_size)
        return TECOOPS_STATUS_BAD_PARAM;
    if (cos_sin_cache != nullptr && max_position <= 0) return TECOOPS_STATUS_BAD_PARAM;
    if (cos_sin_cache == nullptr && !(base > 0.0f)) return TECOOPS_STATUS_BAD_PARAM;
    if (!tecoops::is_16bit_float(dataType)) return TECOOPS_STATUS_BAD_PARAM;
    const int half = rot_dim / 2;
    // Vector paths: 4 pairs per lane with naturally aligned 8 / 16 byte
    // accesses, or 8 NeoX pairs per lane in 16-byte words.
    const size_t align = is_neox ? 8 : 16;
    bool vec = (half % 4) == 0 && (head_size % 4) == 0 && (query_stride % 4) == 0 &&
               tecoops::aligned(query, align);
    if (key != nullptr) vec = vec && (key_stride % 4) == 0 && tecoops::aligned(key, align);
    if (!is_neox) vec = vec && (head_size % 8) == 0 && (query_stride % 8) == 0 &&
                        (key == nullptr || (key_stride % 8) == 0);
    // NeoX with 8 pairs per lane: both halves in 16-byte words
    bool wide = is_neox && vec && (half % 8) == 0 && (head_size % 8) == 0 &&
                (query_stride % 8) == 0 && tecoops::aligned(query, 16);
    if (key != nullptr) wide = wide && (key_stride % 8) == 0 && tecoops::aligned(key, 16);
    const int vw = wide ? 2 : vec ? 1 : 0;
    const float lb = cos_sin_cache ? 0.0f : log2f(base);
    const int Hkv = key ? num_kv_heads : 0;
    using tecoops::dev::bf16;
    using tecoops::dev::f16;
    hipStream_t s = handle->stream;
    if (dataType == TECOOPS_DATA_HALF) {
        if (is_neox) launch<f16, true>(vw, num_tokens, s, positions, query, key, num_heads, Hkv,
                                       head_size, rot_dim, query_stride, key_stride,
                                       cos_sin_cache, max_position, lb);
        else launch<f16, false>(vw, num_tokens, s, positions, query, key, num_heads, Hkv,
                                head_size, rot_dim, query_stride, key_stride, cos_sin_cache,
                                max_position, lb);
    } else {
        if (is_neox) launch<bf16, true>(vw, num_tokens, s, positions, query, key, num_heads, Hkv,
                                        head_size, rot_dim, query_stride, key_stride,
                                        cos_sin_cache, max_position, lb);
        else launch<bf16, false>(vw, num_tokens, s, positions, query, key, num_heads, Hkv,
                                 head_size, rot_dim, query_stride, key_stride, cos_sin_cache,
                                 max_position, lb);
    }
    TECO_CHECK_LAUNCH("rotary_embedding");
    return TECOOPS_STATUS_SUCCESS;
}

extern "C" tecoopsStatus_t tecoopsRotaryReshapeAndCache(
    tecoopsHandle_t handle, const int64_t *positions, void *query, void *key, const void *value,
    const int64_t *slot_mapping, void *key_cache, void *value_cache, int num_tokens,
    int num_heads, int num_kv_heads, int head_size, int rot_dim, long long query_stride,
    long long key_stride, long long value_stride, const float *cos_sin_cache, int max_position,
    float base, int is_neox, int num_blocks, int block_size, int write_key,
    tecoopsDataType_t dataType) {
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (positions == nullptr || query == nullptr || key == nullptr || value == nullptr ||
        slot_mapping == nullptr || key_cache == nullptr || value_cache == nullptr)
        return TECOOPS_STATUS_BAD_PARAM;
    if (num_tokens <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_size <= 0 ||
        num_blocks <= 0 || block_size <= 0)
        return TECOOPS_STATUS_BAD_PARAM;
    if (rot_dim <= 0 || (rot_dim & 1) || rot_dim > head_size || rot_dim / 2 > kMaxHalf)
        return TECOOPS_STATUS_BAD_PARAM;
    if (query_stride < static_cast<long long>(num_heads) * head_size ||
        key_stride < static_cast<long long>(num_kv_heads) * head_size ||
        value_stride < static_cast<long long>(num_kv_heads) * head_size)
        return TECOOPS_STATUS_BAD_PARAM;
    if (cos_sin_cache != nullptr && max_position <= 0) return TECOOPS_STATUS_BAD_PARAM;
    if (cos_sin_cache == nullptr && !(base > 0.0f)) return TECOOPS_STATUS_BAD_PARAM;
    if (!tecoops::is_16bit_float(dataType)) return TECOOPS_STATUS_BAD_PARAM;
    const long long capacity = static_cast<long long>(num_blocks) * block_size;
    if (capacity >= (1ll << 31)) return TECOOPS_STATUS_NOT_SUPPORTED;
    FusedArgs a{};
    a.positions = positions;
    a.query = static_cast<uint16_t *>(query);
    a.key = static_cast<uint16_t *>(key);
    a.value = static_cast<const uint16_t *>(value);
    a.slots = slot_mapping;
    a.kcache = static_cast<uint16_t *>(key_cache);
    a.vcache = static_cast<uint16_t *>(value_cache);
    a.num_tokens = num_tokens;
    a.num_heads = num_heads;
    a.num_kv_heads = num_kv_heads;
    a.head_size = head_size;
    a.rot_dim = rot_dim;
    a.q_stride = query_stride;
    a.k_stride = key_stride;
    a.v_stride = value_stride;
    a.cos_sin_cache = cos_sin_cache;
    a.max_position = max_position;
    a.log2_base = cos_sin_cache ? 0.0f : log2f(base);
    a.block_size = block_size;
    a.lbs = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
    a.capacity = capacity;
    a.write_key = write_key;
    // Vector path: 4 (or 8) pairs per rotation task and 16-byte value / tail
    // copies, all naturally aligned.
    const int half = rot_dim / 2;
    const size_t ra = is_neox ? 8 : 16;
    bool vec = (half % 4) == 0 && (head_size % 8) == 0 && ((head_size - rot_dim) % 8) == 0 &&
               (query_stride % 8) == 0 && (key_stride % 8) == 0 && (value_stride % 8) == 0 &&
               tecoops::aligned(query, ra) && tecoops::aligned(key, ra) &&
               tecoops::aligned(value, 16) && tecoops::aligned(key_cache, 16) &&
               tecoops::aligned(value_cache, 16);
    // NeoX with 8 pairs per lane: both halves in 16-byte words
    const bool wide = is_neox && vec && (half % 8) == 0 && tecoops::aligned(query, 16) &&
                      tecoops::aligned(key, 16);
    const unsigned grid = tecoops::ceil_div(num_tokens, kTokensPerBlock);
    using tecoops::dev::bf16;
    using tecoops::dev::f16;
    hipStream_t s = handle->stream;
    const bool h16 = dataType == TECOOPS_DATA_HALF;
#define TECO_ROT_CACHE(TT, NX, VV) \
    hipLaunchKernelGGL((rotary_cache_kernel<TT, NX, VV>), dim3(grid), dim3(kThreads), 0, s, a)
    if (h16) {
        if (is_neox) {
            if (wide) TECO_ROT_CACHE(f16, true, 2);
            else if (vec) TECO_ROT_CACHE(f16, true, 1);
            else TECO_ROT_CACHE(f16, true, 0);
        } else {
            if (vec) TECO_ROT_CACHE(f16, false, 1); else TECO_ROT_CACHE(f16, false, 0);
        }
    } else {
        if (is_neox) {
            if (wide) TECO_ROT_CACHE(bf16, true, 2);
            else if (vec) TECO_ROT_CACHE(bf16, true, 1);
            else TECO_ROT_CACHE(bf16, true, 0);
        } else {
            if (vec) TECO_ROT_CACHE(bf16, false, 1); else TECO_ROT_CACHE(bf16, false, 0);
        }
    }
#undef TECO_ROT_CACHE
    TECO_CHECK_LAUNCH("rotary_reshape_and_cache");
    return TECOOPS_STATUS_SUCCESS;
}
