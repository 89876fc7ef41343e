// fa_noalloc.hip — tecoopsFlashAttentionNoAlloc, the flash-attention entry
// point that allocates nothing (no counterpart in the reference), and the
// static device array its split-KV decode partials live in.
//
// The array is in a code object of its own, apart from the attention
// kernels: the HIP runtime loads a code object (and allocates its device
// variables) when it is first used, so a process that never calls this entry
// point does not hold the array.
#include <mutex>

#include "common.h"
#include "flash_attention.h"

namespace {

// Split-KV partials of tecoopsFlashAttentionNoAlloc.  Each GPU the entry
// point runs on holds its own copy, at its own address, until the process
// ends.  Every call on a GPU shares that GPU's copy.
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

// Device address of this GPU's copy of `scratch`, looked up once per device
// with that device current.  In host code the array's name is only a
// host-side stand-in; kernels must get this address instead.
tecoopsStatus_t static_scratch(void **out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void *addr[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return TECOOPS_STATUS_INTERNAL_ERROR;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (addr[dev] == nullptr) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            TECO_ERROR("flash_attention: cannot get the static scratch address on device %d", dev);
            return TECOOPS_STATUS_INTERNAL_ERROR;
        }
        addr[dev] = p;
    }
    *out = addr[dev];
    return TECOOPS_STATUS_SUCCESS;
}

}  // namespace

extern "C" tecoopsStatus_t tecoopsFlashAttentionNoAlloc(
    tecoopsHandle_t handle, int max_seqlen_q, int max_seqlen_k, const int *q_seq_lens,
    const int *cu_seqlens_q, const int *kv_seq_lens, const tecoopsTensorDescriptor_t btDesc,
    const void *blockTable, const tecoopsTensorDescriptor_t qDesc, const void *qData,
    const tecoopsTensorDescriptor_t kDesc, const void *kCache,
    const tecoopsTensorDescriptor_t vDesc, const void *vCache,
    const tecoopsTensorDescriptor_t oDesc, void *oData, float softmax_scale, int causal) {
    tecoops::fa::FaCall c;
    tecoopsStatus_t st = tecoops::fa::prepare(handle, max_seqlen_q, max_seqlen_k, q_seq_lens,
                                              cu_seqlens_q, kv_seq_lens, btDesc, blockTable, qDesc,
                                              qData, kDesc, kCache, vDesc, vCache, oDesc, oData,
                                              softmax_scale, causal, false, c);
    if (st != TECOOPS_STATUS_SUCCESS) return st;
    void *ws = nullptr;
    // With one split per sequence the decode kernel reads no partials.
    if (c.pl.decode && c.pl.max_splits > 1) {
        const size_t need = tecoops::fa::workspace_bytes(c);
        TECO_RETURN_IF(need > kStaticScratchBytes, TECOOPS_STATUS_BAD_PARAM,
                       "tecoopsFlashAttentionNoAlloc: split-KV decode needs %zu bytes of scratch, "
                       "more than the static %zu (use tecoopsFlashAttentionEx)",
                       need, kStaticScratchBytes);
        st = static_scratch(&ws);
        if (st != TECOOPS_STATUS_SUCCESS) return st;
    }
    // Every partial the combine kernel reads is written by the same call's
    // decode kernel first, so the scratch needs no clearing.
    return tecoops::fa::launch(handle->stream, c, ws);
}
