// memset.hip — tecoopsMemset: byte fill of a device buffer.
//
// Semantics of teco/interface/ops/memset.cpp:52-67 and
// teco/ual/kernel/memset/memset_4B_align.scpp:79-140: `size` bytes at x are
// set to (uint8_t)value.  The plugins zero whole outputs with it.
//
// gfx950 design: the aligned body is written with 16-byte stores, one per
// lane per grid-stride step (HBM-bound, 1 byte written per byte of size);
// the unaligned head and tail bytes are written by the first block.  A kernel
// rather than hipMemsetAsync, so that the op is safe inside captured graphs.
#include "common.h"

namespace {

__global__ void __launch_bounds__(256) memset_kernel(uint8_t *x, uint32_t word, size_t head,
                                                     size_t nvec, size_t tail_begin,
                                                     size_t size) {
    const size_t tid = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    uint4 v = make_uint4(word, word, word, word);
    uint4 *body = reinterpret_cast<uint4 *>(x + head);
    for (size_t i = tid; i < nvec; i += stride) body[i] = v;
    if (blockIdx.x == 0) {
        const uint8_t b = static_cast<uint8_t>(word);
        if (threadIdx.x < head) x[threadIdx.x] = b;
        if (tail_begin + threadIdx.x < size) x[tail_begin + threadIdx.x] = b;
    }
}

}  // namespace

extern "C" tecoopsStatus_t tecoopsMemset(tecoopsHandle_t handle, void *x, const int value,
                                         size_t size) {
    // reference memset.cpp:37-45 returns BAD_PARAM for a NULL handle.
    if (handle == nullptr || x == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    if (size == 0) return TECOOPS_STATUS_SUCCESS;
    uint8_t *p = static_cast<uint8_t *>(x);
    size_t head = (16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15;
    if (head > size) head = size;
    const size_t nvec = (size - head) / 16;
    const size_t tail_begin = head + nvec * 16;  // < 16 bytes remain after this
    const uint32_t b = static_cast<uint8_t>(value);
    const uint32_t word = b * 0x01010101u;
    size_t blocks = (nvec + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(memset_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       handle->stream, p, word, head, nvec, tail_begin, size);
    TECO_CHECK_LAUNCH("memset");
    return TECOOPS_STATUS_SUCCESS;
}
