// common.h — host-side internals shared by the tecoops library sources.
//
// The handle replaces the reference's tecoopsContext{spa_num, spe_num,
// spm_size, stream} (teco/interface/include/builtin_type.h:33-38): on gfx950
// there is no SPA/SPE/SPM to describe, so the handle holds the HIP stream and
// the device scratch used by split-KV flash attention when the caller passes
// no workspace.  The scratch is kept per stream (up to kScratchSlots streams,
// least recently used replaced first): work on one stream is ordered by the
// stream, and calls on different streams never share a buffer, so no event or
// wait is needed.  Each buffer grows on demand on the device current at the
// op, and a slot taken over from another stream gets a new buffer; hipFree
// synchronises the device first, so a buffer still read by enqueued work is
// never freed or reused under it.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdint>
#include <atomic>
#include <cstring>

#include "tecoops.h"

constexpr int kScratchSlots = 8;

struct ScratchSlot {
    hipStream_t stream = nullptr;
    void *ptr = nullptr;
    size_t bytes = 0;
    unsigned long long last_use = 0;
};

struct tecoopsContext {
    hipStream_t stream = nullptr;
    ScratchSlot scratch[kScratchSlots];
    unsigned long long uses = 0;
};

// Descriptor: same fields and stride rules as the reference
// (teco/interface/common/tensor.h; tecoops.cpp:70-237).  Dims beyond
// TECOOPS_DIM_MAX live in heap arrays owned (and freed) by the descriptor.
struct tecoopsTensorStruct {
    tecoopsDataType_t dataType = TECOOPS_DATA_FLOAT;
    tecoopsTensorFormat_t format = TECOOPS_TENSOR_NCHW;
    int nbDims = 0;
    int dims_inline[TECOOPS_DIM_MAX] = {0};
    int strides_inline[TECOOPS_DIM_MAX] = {0};
    int *dimA = dims_inline;
    int *strideA = strides_inline;
    int *expand_dims = nullptr;
    int *expand_strides = nullptr;
};

namespace tecoops {

#define TECO_ERROR(...)                                        \
    do {                                                       \
        std::fprintf(stderr, "[tecoops] error: " __VA_ARGS__); \
        std::fputc('\n', stderr);                              \
    } while (0)

// Checks the launch that was just enqueued; the reference returns SUCCESS
// unconditionally after its launch (teco/ual/ops/base_op.hpp:72-73), this
// library maps a launch failure to TECOOPS_STATUS_INTERNAL_ERROR.
#define TECO_CHECK_LAUNCH(what)                                                   \
    do {                                                                          \
        hipError_t _e = hipGetLastError();                                        \
        if (_e != hipSuccess) {                                                   \
            TECO_ERROR("%s launch failed: %s", what, hipGetErrorString(_e));      \
            return TECOOPS_STATUS_INTERNAL_ERROR;                                 \
        }                                                                         \
    } while (0)

#define TECO_RETURN_IF(cond, status, ...) \
    do {                                  \
        if (cond) {                       \
            TECO_ERROR(__VA_ARGS__);      \
            return status;                \
        }                                 \
    } while (0)

inline bool is_16bit_float(tecoopsDataType_t t) {
    return t == TECOOPS_DATA_HALF || t == TECOOPS_DATA_BFLOAT16;
}

__host__ __device__ inline bool aligned(const void *p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

inline unsigned ceil_div(long long a, long long b) {
    return static_cast<unsigned>((a + b - 1) / b);
}

// Dynamic LDS a workgroup may hold on gfx950, and the amount a kernel gets
// without raising its limit.
constexpr size_t kLdsMax = 160 * 1024;
constexpr size_t kLdsDefault = 64 * 1024;

// Sets a kernel's dynamic-LDS attribute to `bytes` (above kLdsDefault) when
// that is more than any size set for it before; false (with the HIP error
// cleared) above kLdsMax or if refused.  HIP documents that AMD devices may
// ignore this attribute (hipFuncAttribute in hip_runtime_api.h); the launch
// itself then checks the dynamic LDS against the workgroup limit, kLdsMax on
// gfx950.  It is set anyway, for a runtime that does enforce it.
bool reserve_lds(const void *kernel, size_t bytes);

// Compute units of the current device, queried once per device (256 on
// MI355X; 256 is also the answer when the query fails).
inline int device_cus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            v <= 0)
            v = 256;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// Returns a device buffer of at least `bytes` owned by the handle for the
// handle's current stream, for an op about to be enqueued there.
tecoopsStatus_t handle_scratch(tecoopsHandle_t handle, size_t bytes, void **out);

}  // namespace tecoops
