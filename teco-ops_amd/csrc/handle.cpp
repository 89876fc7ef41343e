// handle.cpp — handle, stream, tensor descriptor and status functions.
//
// Behaviour follows teco/interface/common/tecoops.cpp:38-258: the same
// NULL-argument statuses, the same row-major default strides in
// SetTensorNdDescriptor and the same format-to-stride table in
// SetTensor4dDescriptor.  Differences: the handle owns a scratch buffer per
// stream it runs split-KV attention on, and descriptors free their >8-dim
// arrays.  Create/Destroy of a handle that never
// ran an op make no HIP call.
#include <mutex>

#include "common.h"

#include <cstdlib>

extern "C" {

tecoopsStatus_t tecoopsCreate(tecoopsHandle_t *handle) {
    if (handle == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    tecoopsContext *ctx = new (std::nothrow) tecoopsContext();
    if (ctx == nullptr) return TECOOPS_STATUS_ALLOC_FAILED;
    ctx->stream = nullptr;  // the default stream until SetStream
    *handle = ctx;
    return TECOOPS_STATUS_SUCCESS;
}

tecoopsStatus_t tecoopsDestroy(tecoopsHandle_t handle) {
    if (handle == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    // hipFree synchronises the device first: enqueued work that still reads
    // a buffer finishes before it is freed.
    for (ScratchSlot &sl : handle->scratch)
        if (sl.ptr != nullptr) (void)hipFree(sl.ptr);
    delete handle;
    return TECOOPS_STATUS_SUCCESS;
}

tecoopsStatus_t tecoopsSetStream(tecoopsHandle_t handle, hipStream_t stream) {
    if (handle == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    handle->stream = stream;
    return TECOOPS_STATUS_SUCCESS;
}

tecoopsStatus_t tecoopsGetStream(tecoopsHandle_t handle, hipStream_t *stream) {
    if (handle == nullptr || stream == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    *stream = handle->stream;
    return TECOOPS_STATUS_SUCCESS;
}

const char *tecoopsGetErrorString(tecoopsStatus_t status) {
    switch (status) {
        case TECOOPS_STATUS_SUCCESS: return "TECOOPS_STATUS_SUCCESS";
        case TECOOPS_STATUS_NOT_INITIALIZED: return "TECOOPS_STATUS_NOT_INITIALIZED";
        case TECOOPS_STATUS_ALLOC_FAILED: return "TECOOPS_STATUS_ALLOC_FAILED";
        case TECOOPS_STATUS_BAD_PARAM: return "TECOOPS_STATUS_BAD_PARAM";
        case TECOOPS_STATUS_INTERNAL_ERROR: return "TECOOPS_STATUS_INTERNAL_ERROR";
        case TECOOPS_STATUS_INVALID_VALUE: return "TECOOPS_STATUS_INVALID_VALUE";
        case TECOOPS_STATUS_NOT_SUPPORTED: return "TECOOPS_STATUS_NOT_SUPPORTED";
        default: return "UNKNOWN_ERROR";
    }
}

tecoopsStatus_t tecoopsCreateTensorDescriptor(tecoopsTensorDescriptor_t *tensorDesc) {
    if (tensorDesc == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    tecoopsTensorStruct *d = new (std::nothrow) tecoopsTensorStruct();
    if (d == nullptr) return TECOOPS_STATUS_ALLOC_FAILED;
    *tensorDesc = d;
    return TECOOPS_STATUS_SUCCESS;
}

static void release_expanded(tecoopsTensorStruct *d) {
    std::free(d->expand_dims);
    std::free(d->expand_strides);
    d->expand_dims = d->expand_strides = nullptr;
    d->dimA = d->dims_inline;
    d->strideA = d->strides_inline;
}

tecoopsStatus_t tecoopsSetTensor4dDescriptor(tecoopsTensorDescriptor_t d,
                                             tecoopsTensorFormat_t format,
                                             tecoopsDataType_t dataType, int n, int c, int h,
                                             int w) {
    if (d == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    int ns, cs, hs, ws;
    switch (format) {  // reference tecoops.cpp:85-110
        case TECOOPS_TENSOR_NCHW: ns = c * h * w; cs = h * w; hs = w; ws = 1; break;
        case TECOOPS_TENSOR_NHWC: ns = h * w * c; cs = 1; hs = w * c; ws = c; break;
        case TECOOPS_TENSOR_CHWN: ns = 1; cs = h * w * n; hs = w * n; ws = n; break;
        case TECOOPS_TENSOR_NWHC: ns = w * h * c; cs = 1; hs = c; ws = h * c; break;
        default: return TECOOPS_STATUS_BAD_PARAM;
    }
    release_expanded(d);
    d->format = format;
    d->dataType = dataType;
    d->nbDims = 4;
    d->dimA[0] = n; d->dimA[1] = c; d->dimA[2] = h; d->dimA[3] = w;
    d->strideA[0] = ns; d->strideA[1] = cs; d->strideA[2] = hs; d->strideA[3] = ws;
    return TECOOPS_STATUS_SUCCESS;
}

tecoopsStatus_t tecoopsGetTensor4dDescriptor(const tecoopsTensorDescriptor_t d,
                                             tecoopsDataType_t *dataType, int *n, int *c,
                                             int *h, int *w, int *nStride, int *cStride,
                                             int *hStride, int *wStride) {
    if (d == nullptr || d->nbDims != 4) return TECOOPS_STATUS_BAD_PARAM;
    if (dataType) *dataType = d->dataType;
    if (n) *n = d->dimA[0];
    if (c) *c = d->dimA[1];
    if (h) *h = d->dimA[2];
    if (w) *w = d->dimA[3];
    if (nStride) *nStride = d->strideA[0];
    if (cStride) *cStride = d->strideA[1];
    if (hStride) *hStride = d->strideA[2];
    if (wStride) *wStride = d->strideA[3];
    return TECOOPS_STATUS_SUCCESS;
}

tecoopsStatus_t tecoopsSetTensorNdDescriptor(tecoopsTensorDescriptor_t d,
                                             tecoopsDataType_t dataType, int nbDims,
                                             const int dimA[], const int strideA[]) {
    if (d == nullptr || nbDims <= 0 || dimA == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    release_expanded(d);
    if (nbDims > TECOOPS_DIM_MAX) {
        d->expand_dims = static_cast<int *>(std::malloc(sizeof(int) * nbDims));
        d->expand_strides = static_cast<int *>(std::malloc(sizeof(int) * nbDims));
        if (!d->expand_dims || !d->expand_strides) {
            release_expanded(d);
            return TECOOPS_STATUS_ALLOC_FAILED;
        }
        d->dimA = d->expand_dims;
        d->strideA = d->expand_strides;
    }
    d->dataType = dataType;
    d->format = TECOOPS_TENSOR_NCHW;
    d->nbDims = nbDims;
    std::memcpy(d->dimA, dimA, sizeof(int) * nbDims);
    if (strideA != nullptr) {
        std::memcpy(d->strideA, strideA, sizeof(int) * nbDims);
    } else {  // row-major, reference tecoops.cpp:197-202
        d->strideA[nbDims - 1] = 1;
        for (int i = nbDims - 2; i >= 0; --i) d->strideA[i] = d->strideA[i + 1] * dimA[i + 1];
    }
    return TECOOPS_STATUS_SUCCESS;
}

tecoopsStatus_t tecoopsGetTensorNdDescriptor(const tecoopsTensorDescriptor_t d,
                                             int nbDimsRequested, tecoopsDataType_t *dataType,
                                             int *nbDims, int dimA[], int strideA[]) {
    if (d == nullptr || nbDimsRequested <= 0) return TECOOPS_STATUS_BAD_PARAM;
    if (dataType) *dataType = d->dataType;
    int n = d->nbDims;
    if (nbDims) *nbDims = d->nbDims;
    if (n > nbDimsRequested) n = nbDimsRequested;
    if (dimA) std::memcpy(dimA, d->dimA, sizeof(int) * n);
    if (strideA) std::memcpy(strideA, d->strideA, sizeof(int) * n);
    return TECOOPS_STATUS_SUCCESS;
}

tecoopsStatus_t tecoopsDestroyTensorDescriptor(tecoopsTensorDescriptor_t d) {
    if (d != nullptr) {
        release_expanded(d);
        delete d;
    }
    return TECOOPS_STATUS_SUCCESS;
}

// Ops of the reference that are not on the LLM-inference path.
tecoopsStatus_t tecoopsFlattenRays(tecoopsHandle_t handle, const int *rays, uint32_t, uint32_t,
                                   int *res, tecoopsAlgo_t) {
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (rays == nullptr || res == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    return TECOOPS_STATUS_NOT_SUPPORTED;
}

tecoopsStatus_t tecoopsReduceVariance(const tecoopsHandle_t handle, int, int,
                                      const tecoopsTensorDescriptor_t xDesc, const void *x,
                                      const tecoopsTensorDescriptor_t yDesc, void *y) {
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (!xDesc || !x || !yDesc || !y) return TECOOPS_STATUS_BAD_PARAM;
    return TECOOPS_STATUS_NOT_SUPPORTED;
}

tecoopsStatus_t tecoopsMorton3DInvert(tecoopsHandle_t handle, const int *indices, uint32_t,
                                      int *coords) {
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (indices == nullptr || coords == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    return TECOOPS_STATUS_NOT_SUPPORTED;
}

}  // extern "C"

namespace tecoops {

// The largest size set for each kernel so far is kept in a fixed table (no
// heap allocation, so the allocation-free entry points can use it too): the
// attribute is set again only when a launch needs more than that (the GEMV
// kernels' LDS grows with K), and past the table's capacity on every launch.
bool reserve_lds(const void *kernel, size_t bytes) {
    static std::mutex mu;
    static const void *kern[256];
    static size_t size[256];
    static int n = 0;
    if (bytes <= kLdsDefault) return true;
    if (bytes > kLdsMax) {
        TECO_ERROR("a kernel asks for %zu bytes of LDS, more than the %zu a workgroup can hold",
                   bytes, kLdsMax);
        return false;
    }
    std::lock_guard<std::mutex> lock(mu);
    int i = 0;
    while (i < n && kern[i] != kernel) ++i;
    if (i < n && size[i] >= bytes) return true;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(bytes)) != hipSuccess) {
        (void)hipGetLastError();
        TECO_ERROR("cannot reserve %zu bytes of LDS for a kernel", bytes);
        return false;
    }
    if (i < n) {
        size[i] = bytes;
    } else if (n < 256) {
        kern[n] = kernel;
        size[n++] = bytes;
    }
    return true;
}

tecoopsStatus_t handle_scratch(tecoopsHandle_t handle, size_t bytes, void **out) {
    // A graph captured from this stream would keep the slot's address, and a
    // later call may free the slot (a larger plan grows it, a ninth stream
    // takes it over), leaving the graph writing freed memory.  Under capture
    // the caller passes a workspace or uses the allocation-free entry point.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(handle->stream, &cs) != hipSuccess) {
        (void)hipGetLastError();
        cs = hipStreamCaptureStatusNone;
    }
    if (cs != hipStreamCaptureStatusNone) {
        TECO_ERROR("the handle's split-KV scratch cannot be used while its stream is captured: "
                   "pass a workspace (tecoopsFlashAttentionEx) or call "
                   "tecoopsFlashAttentionNoAlloc");
        return TECOOPS_STATUS_NOT_SUPPORTED;
    }
    if (bytes == 0) bytes = 256;
    ScratchSlot *slot = nullptr;
    for (ScratchSlot &sl : handle->scratch)
        if (sl.ptr != nullptr && sl.stream == handle->stream) slot = &sl;
    if (slot == nullptr) {  // a free slot, else the least recently used one
        slot = &handle->scratch[0];
        for (ScratchSlot &sl : handle->scratch) {
            if (sl.ptr == nullptr) {
                slot = &sl;
                break;
            }
            if (sl.last_use < slot->last_use) slot = &sl;
        }
        // A buffer taken over from another stream may still be read by work
        // enqueued there: free it (hipFree waits for the device) and let the
        // allocation below start afresh.
        if (slot->ptr != nullptr) {
            const hipError_t e = hipFree(slot->ptr);
            *slot = ScratchSlot{};
            if (e != hipSuccess) {
                (void)hipGetLastError();
                return TECOOPS_STATUS_INTERNAL_ERROR;
            }
        }
        slot->stream = handle->stream;
    }
    if (slot->bytes < bytes) {
        // hipFree synchronises the device, so work still reading the old
        // buffer (on this slot's stream) has finished.
        if (slot->ptr != nullptr && hipFree(slot->ptr) != hipSuccess) {
            (void)hipGetLastError();
            *slot = ScratchSlot{};
            return TECOOPS_STATUS_INTERNAL_ERROR;
        }
        *slot = ScratchSlot{};
        const size_t grow = bytes + bytes / 4;
        void *p = nullptr;
        if (hipMalloc(&p, grow) != hipSuccess) {
            (void)hipGetLastError();
            return TECOOPS_STATUS_ALLOC_FAILED;
        }
        slot->stream = handle->stream;
        slot->ptr = p;
        slot->bytes = grow;
    }
    slot->last_use = ++handle->uses;
    *out = slot->ptr;
    return TECOOPS_STATUS_SUCCESS;
}

}  // namespace tecoops
