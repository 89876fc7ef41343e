/*
 * tecoops.h — C ABI of the MI355X (gfx950) LLM-inference operator library.
 *
 * Drop-in for the reference interface teco/interface/include/tecoops.h:37-188.
 * Every enum value, handle/descriptor function and op signature of the
 * reference is kept; the only type change is the stream: sdaaStream_t
 * (reference tecoops.h:92-93) becomes hipStream_t.  All tensors are device
 * pointers owned by the caller; every entry point validates its arguments
 * before any device work, enqueues on the handle's stream and returns without
 * synchronising.
 *
 * Entry points below the "Extensions" banner have no counterpart in the
 * reference header.  They are additive: bf16 through a dataType argument,
 * rotary embedding, GEMV (fp16 / int8 weights), causal_conv1d with bias and
 * arbitrary strides, flash attention with cumulative query offsets and an
 * explicit softmax scale.
 */
#ifndef TECOOPS_INCLUDE_TECOOPS_H_
#define TECOOPS_INCLUDE_TECOOPS_H_

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference tecoops.h:37 */
#define TECOOPS_DIM_MAX 8

/* reference tecoops.h:39-47 — values are part of the ABI. */
typedef enum {
    TECOOPS_STATUS_SUCCESS = 0,
    TECOOPS_STATUS_NOT_INITIALIZED = 1,
    TECOOPS_STATUS_ALLOC_FAILED = 2,
    TECOOPS_STATUS_BAD_PARAM = 3,
    TECOOPS_STATUS_INTERNAL_ERROR = 4,
    TECOOPS_STATUS_INVALID_VALUE = 5,
    TECOOPS_STATUS_NOT_SUPPORTED = 6,
} tecoopsStatus_t;

/* reference tecoops.h:49-58 */
typedef enum {
    TECOOPS_TENSOR_NCHW = 0,
    TECOOPS_TENSOR_NHWC = 1,
    TECOOPS_TENSOR_CHWN = 2,
    TECOOPS_TENSOR_NWHC = 3,
    TECOOPS_TENSOR_NCDHW = 4,
    TECOOPS_TENSOR_NDHWC = 5,
    TECOOPS_TENSOR_CDHWN = 6,
} tecoopsTensorFormat_t;

/* reference tecoops.h:60-71 */
typedef enum {
    TECOOPS_ALGO_0 = 0,
    TECOOPS_ALGO_1,
    TECOOPS_ALGO_2,
    TECOOPS_ALGO_3,
    TECOOPS_ALGO_4,
    TECOOPS_ALGO_5,
    TECOOPS_ALGO_6,
    TECOOPS_ALGO_7,
    TECOOPS_ALGO_8,
    TECOOPS_ALGO_9,
} tecoopsAlgo_t;

/* reference tecoops.h:73-85 */
typedef enum {
    TECOOPS_DATA_FLOAT = 0,
    TECOOPS_DATA_HALF = 1,
    TECOOPS_DATA_INT8 = 2,
    TECOOPS_DATA_INT16 = 3,
    TECOOPS_DATA_INT32 = 4,
    TECOOPS_DATA_INT64 = 5,
    TECOOPS_DATA_UINT8 = 6,
    TECOOPS_DATA_BOOL = 7,
    TECOOPS_DATA_DOUBLE = 8,
    TECOOPS_DATA_BFLOAT16 = 9,
    TECOOPS_DATA_COMPLEX_FLOAT = 10,
} tecoopsDataType_t;

/* reference tecoops.h:87-88 */
typedef struct tecoopsContext *tecoopsHandle_t;
typedef struct tecoopsTensorStruct *tecoopsTensorDescriptor_t;

/* ---- handle (reference tecoops.h:90-94; impl tecoops.cpp:38-68, :239-258) ---- */
tecoopsStatus_t tecoopsCreate(tecoopsHandle_t *handle);
tecoopsStatus_t tecoopsDestroy(tecoopsHandle_t handle);
tecoopsStatus_t tecoopsSetStream(tecoopsHandle_t handle, hipStream_t stream);
tecoopsStatus_t tecoopsGetStream(tecoopsHandle_t handle, hipStream_t *stream);
const char *tecoopsGetErrorString(tecoopsStatus_t status);

/* ---- tensor descriptors (reference tecoops.h:96-123; impl tecoops.cpp:70-237) ---- */
tecoopsStatus_t tecoopsCreateTensorDescriptor(tecoopsTensorDescriptor_t *tensorDesc);
tecoopsStatus_t tecoopsSetTensor4dDescriptor(tecoopsTensorDescriptor_t tensorDesc,
                                             tecoopsTensorFormat_t format,
                                             tecoopsDataType_t dataType,
                                             int n, int c, int h, int w);
tecoopsStatus_t tecoopsGetTensor4dDescriptor(const tecoopsTensorDescriptor_t tensorDesc,
                                             tecoopsDataType_t *dataType,
                                             int *n, int *c, int *h, int *w,
                                             int *nStride, int *cStride, int *hStride,
                                             int *wStride);
tecoopsStatus_t tecoopsSetTensorNdDescriptor(tecoopsTensorDescriptor_t tensorDesc,
                                             tecoopsDataType_t dataType, int nbDims,
                                             const int dimA[], const int strideA[]);
tecoopsStatus_t tecoopsGetTensorNdDescriptor(const tecoopsTensorDescriptor_t tensorDesc,
                                             int nbDimsRequested, tecoopsDataType_t *dataType,
                                             int *nbDims, int dimA[], int strideA[]);
tecoopsStatus_t tecoopsDestroyTensorDescriptor(tecoopsTensorDescriptor_t tensorDesc);

/* ---- ops outside the LLM path (reference tecoops.h:125-126, :139-145).
 *      Exported for ABI completeness; they return TECOOPS_STATUS_NOT_SUPPORTED
 *      after argument validation. ---- */
tecoopsStatus_t tecoopsFlattenRays(tecoopsHandle_t handle, const int *rays, uint32_t N, uint32_t M,
                                   int *res, tecoopsAlgo_t algo);
tecoopsStatus_t tecoopsReduceVariance(const tecoopsHandle_t handle, int axis, int correction,
                                      const tecoopsTensorDescriptor_t xDesc, const void *x,
                                      const tecoopsTensorDescriptor_t yDesc, void *y);
tecoopsStatus_t tecoopsMorton3DInvert(tecoopsHandle_t handle, const int *indices, uint32_t N,
                                      int *coords);

/* ---- memset (reference tecoops.h:128; impl ops/memset.cpp:52-67).
 *      Fills `size` bytes at x with (uint8_t)value. ---- */
tecoopsStatus_t tecoopsMemset(tecoopsHandle_t handle, void *x, const int value, size_t size);

/* ---- reshape_and_cache (reference tecoops.h:130-137; impl ops/reshape_and_cache.cpp:64-105).
 *      key/value fp16 [num_tokens, num_kv_heads, head_size];
 *      caches fp16 [num_blocks, num_kv_heads, block_size, head_size];
 *      slot_mapping int64 [num_tokens]; slot < 0 is skipped.  Slots at or beyond
 *      num_blocks*block_size are also skipped (the reference would write out of
 *      bounds there). ---- */
tecoopsStatus_t tecoopsReshapeAndCache(tecoopsHandle_t handle,
                                       const void *key, const void *value,
                                       const int64_t *slot_mapping,
                                       void *key_cache, void *value_cache,
                                       int num_tokens, int num_kv_heads, int head_size,
                                       int num_blocks, int block_size);

/* ---- rms_norm (reference tecoops.h:147-156; impl ops/rms_norm.cpp:64-100).
 *      fp16 [num_tokens, hidden_size].  residual != NULL selects the fused
 *      add variant and then requires residual_out. ---- */
tecoopsStatus_t tecoopsRmsNorm(tecoopsHandle_t handle,
                               const void *input, const void *weight, const void *residual,
                               void *output, void *residual_out,
                               int num_tokens, int hidden_size, float eps);

/* ---- flash_attention (reference tecoops.h:158-169; impl ops/flash_attention.cpp:71-119).
 *      Paged, varlen, bottom-right causal, GQA.  q [sum(q_seq_lens), H, D];
 *      caches [num_blocks, Hkv, block_size, D]; blockTable int32
 *      [batch, max_blocks_per_seq]; q_seq_lens / kv_seq_lens int32 [batch]
 *      (device).  Scale is 1/sqrt(D).  Element type comes from the
 *      descriptors: TECOOPS_DATA_HALF or TECOOPS_DATA_BFLOAT16 (q, caches and
 *      output must agree).  D in {32, 64, 96, 128, 160, 192}; any
 *      block_size >= 1.  As in the reference, the results do not depend on
 *      max_seqlen_q / max_seqlen_k (any value, also <= 0, is accepted): they
 *      only shape the launch, and a bound that holds makes it fastest.
 *      kv lengths past block_table_dim * block_size (the reference's
 *      precondition) are clamped to it.  max_block_num and workspace are
 *      accepted and ignored, as in the reference (flash_attention.cpp:110):
 *      the split-KV partials of decode live in the handle's scratch, one
 *      buffer per stream the handle runs on. ---- */
tecoopsStatus_t tecoopsFlashAttention(tecoopsHandle_t handle,
                                      int max_seqlen_q, int max_seqlen_k,
                                      int max_block_num, const int *q_seq_lens,
                                      const int *kv_seq_lens,
                                      const tecoopsTensorDescriptor_t blockTableDesc,
                                      const void *blockTable,
                                      const tecoopsTensorDescriptor_t qDataDesc,
                                      const void *qData,
                                      const tecoopsTensorDescriptor_t kCacheDesc,
                                      const void *kCache,
                                      const tecoopsTensorDescriptor_t vCacheDesc,
                                      const void *vCache,
                                      const tecoopsTensorDescriptor_t oDataDesc,
                                      void *oData, void *workspace);

/* ---- causal_conv1d (reference tecoops.h:171-188; impl ops/causal_conv1d.cpp:56-105).
 *      x/out fp16 [totalSeqLen, dim] with token strides xSeqStride/outSeqStride;
 *      weight fp16 [width, dim]; convState fp16 [entries, width-1, dim] with
 *      entry stride convStateStride.  SiLU is always applied (actMode is
 *      ignored, as in the reference).  queryStartLoc NULL means one token per
 *      sequence; convStateIndices NULL means the identity. width in [2, 4]. ---- */
tecoopsStatus_t tecoopsCausalConv1d(tecoopsHandle_t handle,
                                    int batch, int totalSeqLen, int dim, int width,
                                    int convStateStride, int xSeqStride, int outSeqStride,
                                    int padSlotId, int api_mode, int actMode,
                                    const void *x, void *convState, const void *weight,
                                    void *out,
                                    const int *queryStartLoc,
                                    const int *convStateIndices,
                                    const int8_t *hasInitialState);

/* ======================== Extensions (no reference counterpart) ======================== */

/* rms_norm with an explicit element type (TECOOPS_DATA_HALF or
 * TECOOPS_DATA_BFLOAT16); otherwise identical to tecoopsRmsNorm. */
tecoopsStatus_t tecoopsRmsNormEx(tecoopsHandle_t handle,
                                 const void *input, const void *weight, const void *residual,
                                 void *output, void *residual_out,
                                 int num_tokens, int hidden_size, float eps,
                                 tecoopsDataType_t dataType);

/* reshape_and_cache for any 2-byte element type (HALF / BFLOAT16): the copy is
 * bit-exact, so only the element size matters. */
tecoopsStatus_t tecoopsReshapeAndCacheEx(tecoopsHandle_t handle,
                                         const void *key, const void *value,
                                         const int64_t *slot_mapping,
                                         void *key_cache, void *value_cache,
                                         int num_tokens, int num_kv_heads, int head_size,
                                         int num_blocks, int block_size,
                                         tecoopsDataType_t dataType);

/* Flash attention with the arguments the reference's torch wrapper accepts but
 * drops (api/torch_ext.cpp:99-165): cu_seqlens_q int32 [batch+1] (device) is
 * used when q_seq_lens is NULL, so callers need no host synchronisation;
 * softmax_scale > 0 overrides 1/sqrt(D); causal = 0 disables the mask.
 * With cu_seqlens_q, output rows past cu_seqlens_q[batch] (rows of no
 * sequence, e.g. a graph's padding) are written as zeros, as the reference
 * torch wrapper zeroes its output first (api/torch_ext.cpp:128-132).
 * workspace NULL uses the handle's scratch for a split-KV decode; on a stream
 * being captured into a graph that call returns TECOOPS_STATUS_NOT_SUPPORTED
 * (a later call may free the scratch the graph would keep): pass a workspace
 * or call tecoopsFlashAttentionNoAlloc there.  A workspace must hold
 * tecoopsGetFlashAttentionWorkspaceSize() bytes for the same batch, heads,
 * head size, max_seqlen_q and max_seqlen_k, and max_seqlen_k must then be > 0
 * (it sizes the split-KV partials). */
tecoopsStatus_t tecoopsFlashAttentionEx(tecoopsHandle_t handle,
                                        int max_seqlen_q, int max_seqlen_k,
                                        const int *q_seq_lens, const int *cu_seqlens_q,
                                        const int *kv_seq_lens,
                                        const tecoopsTensorDescriptor_t blockTableDesc,
                                        const void *blockTable,
                                        const tecoopsTensorDescriptor_t qDataDesc,
                                        const void *qData,
                                        const tecoopsTensorDescriptor_t kCacheDesc,
                                        const void *kCache,
                                        const tecoopsTensorDescriptor_t vCacheDesc,
                                        const void *vCache,
                                        const tecoopsTensorDescriptor_t oDataDesc,
                                        void *oData, float softmax_scale, int causal,
                                        void *workspace);

/* Flash attention that allocates nothing, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  Arguments and
 * results are those of tecoopsFlashAttentionEx without a workspace: the
 * split-KV partials of decode go to a static device array of 64 MiB per GPU
 * (held until the process ends) instead of the handle's scratch, and a call
 * whose decode plan needs more returns TECOOPS_STATUS_BAD_PARAM.  Every call
 * on a GPU shares that array: calls that overlap on one GPU (different
 * streams, threads or handles) race and must be ordered by the caller. */
tecoopsStatus_t tecoopsFlashAttentionNoAlloc(tecoopsHandle_t handle,
                                             int max_seqlen_q, int max_seqlen_k,
                                             const int *q_seq_lens, const int *cu_seqlens_q,
                                             const int *kv_seq_lens,
                                             const tecoopsTensorDescriptor_t blockTableDesc,
                                             const void *blockTable,
                                             const tecoopsTensorDescriptor_t qDataDesc,
                                             const void *qData,
                                             const tecoopsTensorDescriptor_t kCacheDesc,
                                             const void *kCache,
                                             const tecoopsTensorDescriptor_t vCacheDesc,
                                             const void *vCache,
                                             const tecoopsTensorDescriptor_t oDataDesc,
                                             void *oData, float softmax_scale, int causal);

/* Bytes of caller workspace tecoopsFlashAttentionEx needs for these sizes
 * (max_seqlen_k > 0; max_seqlen_q <= 0 sizes for the longest q length the
 * split-KV decode route takes). */
tecoopsStatus_t tecoopsGetFlashAttentionWorkspaceSize(int batch, int num_heads,
                                                      int head_size, int max_seqlen_q,
                                                      int max_seqlen_k, size_t *bytes);

/* causal_conv1d with bias and general strides.
 *   element (b, t, d) of x lives at
 *     x + b*xBatchStride + t*xSeqStride + d*xDimStride     when queryStartLoc == NULL
 *     x + (queryStartLoc[b] + t)*xSeqStride + d*xDimStride  otherwise;
 *   out likewise.  With queryStartLoc == NULL every sequence has seqLen tokens.
 *   weight element (d, k) at weight + d*wDimStride + k*wWidthStride.
 *   bias fp16 [dim] or NULL; silu != 0 applies SiLU.  State semantics are
 *   those of tecoopsCausalConv1d.  The [batch, dim, seqlen] layout of
 *   BASELINE-style callers is xBatchStride = dim*seqlen, xDimStride = seqlen,
 *   xSeqStride = 1. */
tecoopsStatus_t tecoopsCausalConv1dEx(tecoopsHandle_t handle,
                                      int batch, int seqLen, int dim, int width,
                                      const void *x, long long xBatchStride,
                                      long long xSeqStride, long long xDimStride,
                                      void *out, long long outBatchStride,
                                      long long outSeqStride, long long outDimStride,
                                      const void *weight, int wDimStride, int wWidthStride,
                                      const void *bias,
                                      void *convState, int convStateStride,
                                      const int *queryStartLoc,
                                      const int *convStateIndices,
                                      const int8_t *hasInitialState,
                                      int padSlotId, int api_mode, int silu);

/* Rotary position embedding, in place on query [num_tokens, num_heads, head_size]
 * and key [num_tokens, num_kv_heads, head_size] (token strides query_stride /
 * key_stride in elements; key may be NULL).  The first rot_dim dims of each
 * head rotate by theta_i = pos * base^(-2i/rot_dim), i < rot_dim/2.
 * is_neox != 0 pairs (i, i + rot_dim/2); otherwise (2i, 2i+1).
 * cos_sin_cache (float32 [max_position, rot_dim]: cos then sin) may be NULL,
 * in which case the angles are computed from base.  dataType HALF or
 * BFLOAT16.  Positions outside [0, max_position) with a cache are skipped. */
tecoopsStatus_t tecoopsRotaryEmbedding(tecoopsHandle_t handle, const int64_t *positions,
                                       void *query, void *key,
                                       int num_tokens, int num_heads, int num_kv_heads,
                                       int head_size, int rot_dim,
                                       long long query_stride, long long key_stride,
                                       const float *cos_sin_cache, int max_position,
                                       float base, int is_neox, tecoopsDataType_t dataType);

/* Fused decode step over the paged KV cache: rotary embedding on query (in
 * place) and key as tecoopsRotaryEmbedding, then the rotated key and value
 * [num_tokens, num_kv_heads, head_size] (token stride value_stride) stored at
 * slot_mapping[t] of key_cache / value_cache [num_blocks, num_kv_heads,
 * block_size, head_size] as tecoopsReshapeAndCache (slots < 0 or past the
 * cache are not stored).  write_key != 0 also writes the rotated key back in
 * place.  The cached values are bit-identical to those two calls in sequence. */
tecoopsStatus_t tecoopsRotaryReshapeAndCache(tecoopsHandle_t handle, const int64_t *positions,
                                             void *query, void *key, const void *value,
                                             const int64_t *slot_mapping,
                                             void *key_cache, void *value_cache,
                                             int num_tokens, int num_heads, int num_kv_heads,
                                             int head_size, int rot_dim,
                                             long long query_stride, long long key_stride,
                                             long long value_stride,
                                             const float *cos_sin_cache, int max_position,
                                             float base, int is_neox,
                                             int num_blocks, int block_size, int write_key,
                                             tecoopsDataType_t dataType);

/* y[b, n] = sum_k W[n, k] * x[b, k], fp32 accumulation.
 * W [n, k] row-major, x [batch, k], y [batch, n]; dataType HALF or BFLOAT16. */
tecoopsStatus_t tecoopsGemv(tecoopsHandle_t handle, const void *weight, const void *x, void *y,
                            int batch, int n, int k, tecoopsDataType_t dataType);

/* y[b, n] = scales[n] * sum_k float(Wq[n, k]) * x[b, k], fp32 accumulation.
 * Wq int8 [n, k] row-major, scales fp16 [n], x / y fp16. */
tecoopsStatus_t tecoopsGemvInt8(tecoopsHandle_t handle, const int8_t *weight,
                                const void *scales, const void *x, void *y,
                                int batch, int n, int k);

#ifdef __cplusplus
}
#endif

#endif  /* TECOOPS_INCLUDE_TECOOPS_H_ */
