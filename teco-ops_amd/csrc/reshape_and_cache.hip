// reshape_and_cache.hip — scatter key/value rows into the paged KV cache.
//
// Semantics (teco/interface/ops/reshape_and_cache.cpp:64-105,
// teco/ual/kernel/reshape_and_cache/reshape_and_cache_fp16.scpp:47-96,
// doc/op_docs/reshape_and_cache.md:13-22): for every token t with
// slot = slot_mapping[t] >= 0, blk = slot / block_size, off = slot % block_size,
//   key_cache[blk][h][off][:] = key[t][h][:]   (and value likewise)
// for every kv head h.  The copy is bit-exact.
//
// gfx950 design: one lane per 16-byte chunk of a (token, head) row; a wave
// covers 1 KiB of contiguous key (and value) bytes, so reads are fully
// coalesced and every destination run is a whole head_size row.  Each lane
// moves its key and its value chunk, i.e. 32 B in flight per lane.  HBM-bound:
// algorithmic bytes = 4 * num_tokens * H * D * 2 + 8 * num_tokens.
#include "common.h"

namespace {

template <typename V>
__global__ void __launch_bounds__(256)
reshape_and_cache_kernel(const V *__restrict__ key, const V *__restrict__ value,
                         const int64_t *__restrict__ slot_mapping, V *__restrict__ key_cache,
                         V *__restrict__ value_cache, long long total, int heads, int vec_per_row,
                         int block_size, long long capacity) {
    const long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (i >= total) return;
    const int per_token = heads * vec_per_row;
    const long long t = i / per_token;
    const int rem = static_cast<int>(i - t * per_token);
    const int64_t slot = slot_mapping[t];
    if (slot < 0 || slot >= capacity) return;
    const int h = rem / vec_per_row;
    const int c = rem - h * vec_per_row;
    const long long blk = slot / block_size;
    const long long off = slot - blk * block_size;
    const long long dst = ((blk * heads + h) * block_size + off) * vec_per_row + c;
    const V k = key[i];
    const V v = value[i];
    key_cache[dst] = k;
    value_cache[dst] = v;
}

template <typename V>
tecoopsStatus_t launch(tecoopsHandle_t handle, const void *key, const void *value,
                       const int64_t *slot_mapping, void *key_cache, void *value_cache,
                       int num_tokens, int heads, int vec_per_row, int num_blocks,
                       int block_size) {
    const long long total = static_cast<long long>(num_tokens) * heads * vec_per_row;
    const long long capacity = static_cast<long long>(num_blocks) * block_size;
    hipLaunchKernelGGL(reshape_and_cache_kernel<V>, dim3(tecoops::ceil_div(total, 256)),
                       dim3(256), 0, handle->stream, static_cast<const V *>(key),
                       static_cast<const V *>(value), slot_mapping, static_cast<V *>(key_cache),
                       static_cast<V *>(value_cache), total, heads, vec_per_row, block_size,
                       capacity);
    TECO_CHECK_LAUNCH("reshape_and_cache");
    return TECOOPS_STATUS_SUCCESS;
}

}  // namespace

extern "C" tecoopsStatus_t tecoopsReshapeAndCacheEx(tecoopsHandle_t handle, const void *key,
                                                    const void *value,
                                                    const int64_t *slot_mapping,
                                                    void *key_cache, void *value_cache,
                                                    int num_tokens, int num_kv_heads,
                                                    int head_size, int num_blocks,
                                                    int block_size,
                                                    tecoopsDataType_t dataType) {
    // Argument checks of reference reshape_and_cache.cpp:39-62.
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (key == nullptr || value == nullptr || slot_mapping == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    if (key_cache == nullptr || value_cache == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    if (num_kv_heads <= 0 || head_size <= 0 || num_tokens <= 0 || num_blocks <= 0 ||
        block_size <= 0)
        return TECOOPS_STATUS_BAD_PARAM;
    if (!tecoops::is_16bit_float(dataType)) return TECOOPS_STATUS_BAD_PARAM;
    const void *ptrs[4] = {key, value, key_cache, value_cache};
    bool a16 = (head_size % 8) == 0, a4 = (head_size % 2) == 0;
    for (const void *p : ptrs) {
        a16 = a16 && tecoops::aligned(p, 16);
        a4 = a4 && tecoops::aligned(p, 4);
    }
    if (a16)
        return launch<uint4>(handle, key, value, slot_mapping, key_cache, value_cache, num_tokens,
                             num_kv_heads, head_size / 8, num_blocks, block_size);
    if (a4)
        return launch<uint32_t>(handle, key, value, slot_mapping, key_cache, value_cache,
                                num_tokens, num_kv_heads, head_size / 2, num_blocks, block_size);
    return launch<uint16_t>(handle, key, value, slot_mapping, key_cache, value_cache, num_tokens,
                            num_kv_heads, head_size, num_blocks, block_size);
}

extern "C" tecoopsStatus_t tecoopsReshapeAndCache(tecoopsHandle_t handle, const void *key,
                                                  const void *value,
                                                  const int64_t *slot_mapping, void *key_cache,
                                                  void *value_cache, int num_tokens,
                                                  int num_kv_heads, int head_size,
                                                  int num_blocks, int block_size) {
    return tecoopsReshapeAndCacheEx(handle, key, value, slot_mapping, key_cache, value_cache,
                                    num_tokens, num_kv_heads, head_size, num_blocks, block_size,
                                    TECOOPS_DATA_HALF);
}
