// flash_attention.h — host-side types of the flash-attention entry points,
// shared by flash_attention.hip (kernels, planning, the C entry points) and
// fa_noalloc.hip (the allocation-free entry point and its static scratch).
#pragma once

#include <cstddef>
#include <cstdint>

#include "common.h"

namespace tecoops {
namespace fa {

// Kernel parameters (passed by value to every flash-attention kernel).
struct FaParams {
    const uint16_t *q;
    const uint16_t *kc;
    const uint16_t *vc;
    uint16_t *o;
    const int *bt;
    long long bt_stride;
    const int *q_lens;   // per-sequence q lengths, or NULL
    const int *cu_q;     // cumulative q offsets [batch+1], used when q_lens is NULL
    const int *kv_lens;
    int batch, H, Hkv, G, bs, lbs, num_blocks;  // lbs = log2(bs) when bs is a power of 2
    int kv_cap;          // block-table width * block_size: kv lengths are clamped to it
    long long page_stride;                      // Hkv * bs * D elements per cache block
    float scale_log2;    // softmax_scale * log2(e)
    float inv_scale_log2;  // 1 / scale_log2: the rescale test compares raw scores
    int causal;
    long long total_q;   // rows of q and of the output (q's descriptor)
    // split-KV decode
    float *ws_o;         // [B][Hkv][max_splits][ncols][D]
    float *ws_ml;        // [B][Hkv][max_splits][ncols][2]
    int split_len, max_splits, rq, ncols;
};

// Launch shape.  rq is the host's bound on q_len (routing and grid height),
// rk its bound on kv_len (prefill routing), split_len / max_splits the
// split-KV plan from rk.  Neither bound changes the output (the kernels also
// cover longer sequences), only the speed.
struct Plan {
    bool decode;
    int rq, rk, ncols, split_len, max_splits;
};

// A validated call: kernel parameters, launch shape and element type.
struct FaCall {
    FaParams p;
    Plan pl;
    int D;
    bool bf16;
};

// Argument checks of reference flash_attention.cpp:44-69 and the launch plan
// (fixed_hints: the hints as given, for a workspace sized from them).
tecoopsStatus_t prepare(tecoopsHandle_t handle, int max_seqlen_q, int max_seqlen_k,
                        const int *q_seq_lens, const int *cu_seqlens_q, const int *kv_seq_lens,
                        const tecoopsTensorDescriptor_t btDesc, const void *blockTable,
                        const tecoopsTensorDescriptor_t qDesc, const void *qData,
                        const tecoopsTensorDescriptor_t kDesc, const void *kCache,
                        const tecoopsTensorDescriptor_t vDesc, const void *vCache,
                        const tecoopsTensorDescriptor_t oDesc, void *oData, float softmax_scale,
                        int causal, bool fixed_hints, FaCall &c);

// Bytes of split-KV partials the call needs (0 for prefill).
size_t workspace_bytes(const FaCall &c);

// Enqueues the call on stream s, its split-KV partials in ws.
tecoopsStatus_t launch(hipStream_t s, FaCall &c, void *ws);

}  // namespace fa
}  // namespace tecoops
