// rotary.hip — in-place rotary position embedding on query and key.
//
// No reference implementation: rotary is absent from the reference library.
// The signature mirrors the vLLM-style rotary_embedding(positions, query, key,
// head_size, cos_sin_cache, is_neox) that the reference's other ops follow.
// theta_i = pos * base^(-2i/rot_dim); NeoX pairs (i, i + rot_dim/2), GPT-J
// pairs (2i, 2i+1):  o1 = x1 cos - x2 sin,  o2 = x2 cos + x1 sin  (fp32 math).
//
// gfx950 design: one workgroup per 4 tokens.  The rot_dim/2 (cos, sin) pairs
// of each token are computed once (accurate sincosf, or read from the cache)
// into LDS and shared by all H + Hkv heads; each lane then rotates 4 pairs
// per task with 8-byte (NeoX) or 16-byte (GPT-J) loads and stores.  HBM-bound: every byte
// of q and k is read once and written once.
#include "common.h"
#include "device.h"

namespace {

using namespace tecoops::dev;

constexpr int kThreads = 256;
constexpr int kMaxHalf = 256;  // rot_dim <= 512

constexpr int kTokensPerBlock = 4;

template <typename T, bool NEOX, bool VEC>
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
    constexpr int P = VEC ? 4 : 1;  // pairs per lane-task
    const int tasks_per_head = half / P;
    const int heads = num_heads + (key ? num_kv_heads : 0);
    const int per_token = heads * tasks_per_head;
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
            if (VEC) {
                uint2 *p1 = reinterpret_cast<uint2 *>(row + i0);
                uint2 *p2 = reinterpret_cast<uint2 *>(row + half + i0);
                uint2 a = *p1, b = *p2;
                const uint32_t *pa = reinterpret_cast<const uint32_t *>(&a);
                const uint32_t *pb = reinterpret_cast<const uint32_t *>(&b);
                uint2 oa, ob;
                uint32_t *qa = reinterpret_cast<uint32_t *>(&oa);
                uint32_t *qb = reinterpret_cast<uint32_t *>(&ob);
#pragma unroll
                for (int w = 0; w < 2; ++w) {
                    const float2 c0 = c[i0 + 2 * w], c1 = c[i0 + 2 * w + 1];
                    const float x10 = lo<T>(pa[w]), x11 = hi<T>(pa[w]);
                    const float x20 = lo<T>(pb[w]), x21 = hi<T>(pb[w]);
                    qa[w] = pack<T>(x10 * c0.x - x20 * c0.y, x11 * c1.x - x21 * c1.y);
                    qb[w] = pack<T>(x20 * c0.x + x10 * c0.y, x21 * c1.x + x11 * c1.y);
                }
                *p1 = oa;
                *p2 = ob;
            } else {
                const float2 cc = c[i0];
                const float x1 = Cvt<T>::to(row[i0]), x2 = Cvt<T>::to(row[half + i0]);
                row[i0] = Cvt<T>::from(x1 * cc.x - x2 * cc.y);
                row[half + i0] = Cvt<T>::from(x2 * cc.x + x1 * cc.y);
            }
        } else {
            if (VEC) {
                uint4 *p = reinterpret_cast<uint4 *>(row + 2 * i0);
                uint4 a = *p;
                uint32_t *pa = reinterpret_cast<uint32_t *>(&a);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const float2 cc = c[i0 + w];
                    const float x1 = lo<T>(pa[w]), x2 = hi<T>(pa[w]);
                    pa[w] = pack<T>(x1 * cc.x - x2 * cc.y, x2 * cc.x + x1 * cc.y);
                }
                *p = a;
            } else {
                const float2 cc = c[i0];
                const float x1 = Cvt<T>::to(row[2 * i0]), x2 = Cvt<T>::to(row[2 * i0 + 1]);
                row[2 * i0] = Cvt<T>::from(x1 * cc.x - x2 * cc.y);
                row[2 * i0 + 1] = Cvt<T>::from(x2 * cc.x + x1 * cc.y);
            }
        }
    }
}

template <typename T, bool NEOX>
void launch(bool vec, int T_, hipStream_t s, const int64_t *pos, void *q, void *k, int H,
            int Hkv, int D, int rot, long long qs, long long ks, const float *cache, int maxpos,
            float lb) {
    const unsigned grid = tecoops::ceil_div(T_, kTokensPerBlock);
    if (vec)
        hipLaunchKernelGGL((rotary_kernel<T, NEOX, true>), dim3(grid), dim3(kThreads), 0, s, pos,
                           static_cast<uint16_t *>(q), static_cast<uint16_t *>(k), T_, H, Hkv, D,
                           rot, qs, ks, cache, maxpos, lb);
    else
        hipLaunchKernelGGL((rotary_kernel<T, NEOX, false>), dim3(grid), dim3(kThreads), 0, s, pos,
                           static_cast<uint16_t *>(q), static_cast<uint16_t *>(k), T_, H, Hkv, D,
                           rot, qs, ks, cache, maxpos, lb);
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
    // Vector path: 4 pairs per lane with naturally aligned 8 / 16 byte accesses.
    const size_t align = is_neox ? 8 : 16;
    bool vec = (half % 4) == 0 && (head_size % 4) == 0 && (query_stride % 4) == 0 &&
               tecoops::aligned(query, align);
    if (key != nullptr) vec = vec && (key_stride % 4) == 0 && tecoops::aligned(key, align);
    if (!is_neox) vec = vec && (head_size % 8) == 0 && (query_stride % 8) == 0 &&
                        (key == nullptr || (key_stride % 8) == 0);
    const float lb = cos_sin_cache ? 0.0f : log2f(base);
    const int Hkv = key ? num_kv_heads : 0;
    using tecoops::dev::bf16;
    using tecoops::dev::f16;
    hipStream_t s = handle->stream;
    if (dataType == TECOOPS_DATA_HALF) {
        if (is_neox) launch<f16, true>(vec, num_tokens, s, positions, query, key, num_heads, Hkv,
                                       head_size, rot_dim, query_stride, key_stride,
                                       cos_sin_cache, max_position, lb);
        else launch<f16, false>(vec, num_tokens, s, positions, query, key, num_heads, Hkv,
                                head_size, rot_dim, query_stride, key_stride, cos_sin_cache,
                                max_position, lb);
    } else {
        if (is_neox) launch<bf16, true>(vec, num_tokens, s, positions, query, key, num_heads, Hkv,
                                        head_size, rot_dim, query_stride, key_stride,
                                        cos_sin_cache, max_position, lb);
        else launch<bf16, false>(vec, num_tokens, s, positions, query, key, num_heads, Hkv,
                                 head_size, rot_dim, query_stride, key_stride, cos_sin_cache,
                                 max_position, lb);
    }
    TECO_CHECK_LAUNCH("rotary_embedding");
    return TECOOPS_STATUS_SUCCESS;
}
