// reshape_and_cache.hip — scatter key/value rows into the paged KV cache.
//
// Semantics (teco/interface/ops/reshape_and_cache.cpp:64-105,
// teco/ual/kernel/reshape_and_cache/reshape_and_cache_fp16.scpp:47-96,
// doc/op_docs/reshape_and_cache.md:13-22): for every token t with
// slot = slot_mapping[t] >= 0, blk = slot / block_size, off = slot % block_size,
//   key_cache[blk][h][off][:] = key[t][h][:]   (and value likewise)
// for every kv head h.  The copy is bit-exact.
//
// gfx950 design: 16-byte chunks of (token, head) rows; each load instruction
// of a wave covers 1 KiB of contiguous key (and value) bytes, so reads are
// fully coalesced and every destination run is a whole head_size row.  Each
// lane moves 4 key and 4 value chunks with every load in flight before the
// first store (non-temporal, read and written once).
// HBM-bound: algorithmic bytes = 4 * num_tokens * H * D * 2 + 8 * num_tokens.
#include "common.h"
#include "device.h"


namespace {

// Each lane moves U chunks (16 bytes when aligned) of (token, head) rows, key
// and value, spaced 256 chunks apart over a 1-D grid of num_tokens * per_token
// chunks (per launch slice), so every lane moves data whatever heads *
// head_size is; all U key / value / slot loads are issued before the
// scattered stores.  Slot arithmetic is 32-bit (slots < 2^31 after the range
// check), with a shift / mask when block_size is a power of two.  Key and
// value are streamed (non-temporal).
template <typename V, bool POW2, int U>
__global__ void __launch_bounds__(256)
reshape_and_cache_kernel(const V *__restrict__ key, const V *__restrict__ value,
                         const int64_t *__restrict__ slot_mapping, V *__restrict__ key_cache,
                         V *__restrict__ value_cache, int heads, int vec_per_row, int block_size,
                         int lbs, long long capacity, int total) {
    const int per_token = heads * vec_per_row;
    const int g0 = blockIdx.x * (256 * U) + threadIdx.x;
    V kv[U], vv[U];
    int64_t slot[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int gid = g0 + 256 * u;
        if (gid < total) {
            kv[u] = tecoops::dev::ld_stream(key + gid);
            vv[u] = tecoops::dev::ld_stream(value + gid);
            slot[u] = slot_mapping[gid / per_token];
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int gid = g0 + 256 * u;
        if (gid >= total || slot[u] < 0 || slot[u] >= capacity) continue;
        const int t = gid / per_token;
        const int rem = gid - t * per_token;
        const int s32 = static_cast<int>(slot[u]);
        int blk, off;
        if (POW2) {
            blk = s32 >> lbs;
            off = s32 & (block_size - 1);
        } else {
            blk = s32 / block_size;
            off = s32 - blk * block_size;
        }
        const int h = rem / vec_per_row;
        const int c = rem - h * vec_per_row;
        const long long dst =
            ((static_cast<long long>(blk) * heads + h) * block_size + off) * vec_per_row + c;
        tecoops::dev::st_stream(key_cache + dst, kv[u]);
        tecoops::dev::st_stream(value_cache + dst, vv[u]);
    }
}

template <typename V>
tecoopsStatus_t launch(tecoopsHandle_t handle, const void *key, const void *value,
                       const int64_t *slot_mapping, void *key_cache, void *value_cache,
                       int num_tokens, int heads, int vec_per_row, int num_blocks,
                       int block_size) {
    const long long per_token = static_cast<long long>(heads) * vec_per_row;
    const long long capacity = static_cast<long long>(num_blocks) * block_size;
    if (capacity >= (1ll << 31) || per_token >= (1ll << 30)) {
        TECO_ERROR("reshape_and_cache: sizes beyond the supported index range");
        return TECOOPS_STATUS_NOT_SUPPORTED;
    }
    const int lbs = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
    // 4 chunks per lane, all loaded before the scattered stores: 12.2 us at
    // 8192 tokens x 8 heads x 128 (2 / 8 / 16 chunks: 13.6 / 12.3 / 13.5 us;
    // plain instead of non-temporal stores: 12.8 us)
    constexpr int U = 4;
    auto *kern = lbs >= 0 ? &reshape_and_cache_kernel<V, true, U> : &reshape_and_cache_kernel<V, false, U>;
    // lane indices are 32-bit: tokens run in slices of fewer than 2^30 lanes
    const int slice = static_cast<int>((1ll << 30) / per_token);
    for (int t0 = 0; t0 < num_tokens; t0 += slice) {
        const int nt = num_tokens - t0 < slice ? num_tokens - t0 : slice;
        const int total = static_cast<int>(per_token * nt);
        const long long src0 = static_cast<long long>(t0) * per_token;
        hipLaunchKernelGGL(kern, dim3(tecoops::ceil_div(total, 256 * U)), dim3(256), 0, handle->stream,
                           static_cast<const V *>(key) + src0, static_cast<const V *>(value) + src0,
                           slot_mapping + t0, static_cast<V *>(key_cache),
                           static_cast<V *>(value_cache), heads, vec_per_row, block_size, lbs,
                           capacity, total);
        TECO_CHECK_LAUNCH("reshape_and_cache");
    }
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
