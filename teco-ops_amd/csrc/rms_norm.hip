// rms_norm.hip — RMS normalisation with optional fused residual add.
//
// Semantics (teco/ual/kernel/rms_norm/rms_norm_fp16.scpp:52-235, CPU baseline
// test/zoo/teco/rms_norm/rms_norm.cpp:195-234):
//   pure: rstd = 1/sqrt(sum(x^2)/D + eps);  y = T(x * rstd * w)
//   add:  v = x + r in fp32; residual_out = T(v); rstd from sum(v^2) of the
//         unrounded v; y = T(float(T(v)) * rstd * w)
// fp32 accumulation throughout.
//
// gfx950 design: rows up to 8192 elements (16-byte aligned, D % 8 == 0) run
// one wave per row: each lane keeps its chunks of the row in registers
// between the reduction and the output pass, so x (and r) are read from HBM
// exactly once and the sum of squares is a wave-wide xor-shuffle reduction
// (no LDS, no barrier).  Rows up to 16384 use a 256-lane workgroup per row
// with an LDS reduction across its 4 waves.  Other rows (D % 8 != 0,
// misaligned, wider) take a two-pass element loop (second read hits L2).  HBM-bound:
// algorithmic bytes = 2*N*D*2 + 2*D (+ 2*N*D*2 for the add variant).
#include "common.h"
#include "device.h"

namespace {

using namespace tecoops::dev;

constexpr int kThreads = 256;

__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nwaves = (blockDim.x + 63) >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nwaves; ++i) s += red[i];
    return s;
}

template <typename T, int VPT, bool ADD>
__global__ void __launch_bounds__(kThreads)
rms_norm_vec(const uint4 *__restrict__ x, const uint4 *__restrict__ w, const uint4 *__restrict__ r,
             uint4 *__restrict__ y, uint4 *__restrict__ r_out, int vec_per_row, int hidden,
             float eps) {
    __shared__ float red[kThreads / 64];
    const long long row = blockIdx.x;
    const uint4 *xr = x + row * vec_per_row;
    uint4 v[VPT];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c = threadIdx.x + j * blockDim.x;
        if (c < vec_per_row) {
            uint4 a = xr[c];
            if (ADD) {
                const uint4 b = r[row * vec_per_row + c];
                uint32_t *pa = reinterpret_cast<uint32_t *>(&a);
                const uint32_t *pb = reinterpret_cast<const uint32_t *>(&b);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float s0 = lo<T>(pa[q]) + lo<T>(pb[q]);
                    const float s1 = hi<T>(pa[q]) + hi<T>(pb[q]);
                    ss += s0 * s0;
                    ss += s1 * s1;
                    pa[q] = pack<T>(s0, s1);
                }
                r_out[row * vec_per_row + c] = a;
            } else {
                const uint32_t *pa = reinterpret_cast<const uint32_t *>(&a);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float s0 = lo<T>(pa[q]), s1 = hi<T>(pa[q]);
                    ss += s0 * s0;
                    ss += s1 * s1;
                }
            }
            v[j] = a;
        }
    }
    const float total = block_sum(ss, red);
    const float rstd = 1.0f / sqrtf(total / static_cast<float>(hidden) + eps);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c = threadIdx.x + j * blockDim.x;
        if (c < vec_per_row) {
            const uint4 wv = w[c];
            const uint32_t *pa = reinterpret_cast<const uint32_t *>(&v[j]);
            const uint32_t *pw = reinterpret_cast<const uint32_t *>(&wv);
            uint4 o;
            uint32_t *po = reinterpret_cast<uint32_t *>(&o);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                po[q] = pack<T>(lo<T>(pa[q]) * rstd * lo<T>(pw[q]),
                                hi<T>(pa[q]) * rstd * hi<T>(pw[q]));
            y[row * vec_per_row + c] = o;
        }
    }
}

// One wave per row: each lane holds VPT 16-byte chunks of its row in
// registers, so the row is read once and the sum of squares needs only a wave
// reduction (no LDS, no barrier).  4 independent rows per workgroup.
template <typename T, int VPT, bool ADD>
__global__ void __launch_bounds__(256)
rms_norm_wave(const uint4 *__restrict__ x, const uint4 *__restrict__ w, const uint4 *__restrict__ r,
              uint4 *__restrict__ y, uint4 *__restrict__ r_out, int rows, int vec_per_row,
              int hidden, float eps) {
    const int lane = threadIdx.x & 63;
    const long long row = static_cast<long long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint4 *xr = x + row * vec_per_row;
    uint4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c = lane + 64 * j;
        if (c < vec_per_row) v[j] = ld_stream(xr + c);
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c = lane + 64 * j;
        if (c < vec_per_row) {
            uint32_t *pa = reinterpret_cast<uint32_t *>(&v[j]);
            if (ADD) {
                const uint4 b = ld_stream(r + row * vec_per_row + c);
                const uint32_t *pb = reinterpret_cast<const uint32_t *>(&b);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float s0 = lo<T>(pa[q]) + lo<T>(pb[q]);
                    const float s1 = hi<T>(pa[q]) + hi<T>(pb[q]);
                    ss += s0 * s0;
                    ss += s1 * s1;
                    pa[q] = pack<T>(s0, s1);
                }
                st_stream(r_out + row * vec_per_row + c, v[j]);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float s0 = lo<T>(pa[q]), s1 = hi<T>(pa[q]);
                    ss += s0 * s0;
                    ss += s1 * s1;
                }
            }
        }
    }
    const float total = wave_sum(ss);
    const float rstd = 1.0f / sqrtf(total / static_cast<float>(hidden) + eps);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c = lane + 64 * j;
        if (c < vec_per_row) {
            const uint4 wv = w[c];
            const uint32_t *pa = reinterpret_cast<const uint32_t *>(&v[j]);
            const uint32_t *pw = reinterpret_cast<const uint32_t *>(&wv);
            uint4 o;
            uint32_t *po = reinterpret_cast<uint32_t *>(&o);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                po[q] = pack<T>(lo<T>(pa[q]) * rstd * lo<T>(pw[q]),
                                hi<T>(pa[q]) * rstd * hi<T>(pw[q]));
            st_stream(y + row * vec_per_row + c, o);
        }
    }
}

// Generic path: any hidden size, element-wise, two passes over the row.
template <typename T, bool ADD>
__global__ void __launch_bounds__(kThreads)
rms_norm_scalar(const uint16_t *__restrict__ x, const uint16_t *__restrict__ w,
                const uint16_t *__restrict__ r, uint16_t *__restrict__ y,
                uint16_t *__restrict__ r_out, int hidden, float eps) {
    __shared__ float red[kThreads / 64];
    const long long base = static_cast<long long>(blockIdx.x) * hidden;
    float ss = 0.0f;
    for (int d = threadIdx.x; d < hidden; d += blockDim.x) {
        float v = Cvt<T>::to(x[base + d]);
        if (ADD) {
            v += Cvt<T>::to(r[base + d]);
            r_out[base + d] = Cvt<T>::from(v);
        }
        ss += v * v;
    }
    const float total = block_sum(ss, red);
    const float rstd = 1.0f / sqrtf(total / static_cast<float>(hidden) + eps);
    // r_out written above by this same lane is re-read (same thread, same
    // address: ordered by program order).
    for (int d = threadIdx.x; d < hidden; d += blockDim.x) {
        const float v = ADD ? Cvt<T>::to(r_out[base + d]) : Cvt<T>::to(x[base + d]);
        y[base + d] = Cvt<T>::from(v * rstd * Cvt<T>::to(w[d]));
    }
}

template <typename T, int VPT, bool ADD>
void launch_wave(const void *x, const void *w, const void *r, void *y, void *ro, int rows,
                 int hidden, float eps, hipStream_t s) {
    hipLaunchKernelGGL((rms_norm_wave<T, VPT, ADD>), dim3(tecoops::ceil_div(rows, 4)), dim3(256),
                       0, s, static_cast<const uint4 *>(x), static_cast<const uint4 *>(w),
                       static_cast<const uint4 *>(r), static_cast<uint4 *>(y),
                       static_cast<uint4 *>(ro), rows, hidden / 8, hidden, eps);
}

template <typename T, int VPT, bool ADD>
void launch_vec(int threads, const void *x, const void *w, const void *r, void *y, void *ro,
                int rows, int hidden, float eps, hipStream_t s) {
    hipLaunchKernelGGL((rms_norm_vec<T, VPT, ADD>), dim3(rows), dim3(threads), 0, s,
                       static_cast<const uint4 *>(x), static_cast<const uint4 *>(w),
                       static_cast<const uint4 *>(r), static_cast<uint4 *>(y),
                       static_cast<uint4 *>(ro), hidden / 8, hidden, eps);
}

template <typename T, bool ADD>
tecoopsStatus_t dispatch(tecoopsHandle_t handle, const void *x, const void *w, const void *r,
                         void *y, void *ro, int rows, int hidden, float eps) {
    hipStream_t s = handle->stream;
    bool vec = (hidden % 8) == 0;
    for (const void *p : {x, w, r, static_cast<const void *>(y), static_cast<const void *>(ro)})
        if (p != nullptr) vec = vec && tecoops::aligned(p, 16);
    const int nvec = hidden / 8;
    if (vec && nvec <= 64 * 16) {
        // up to 16 chunks (8 KiB of fp16 row at 4096 hidden = 8 chunks) per lane
        const int vpt = (nvec + 63) / 64;
        if (vpt <= 1) launch_wave<T, 1, ADD>(x, w, r, y, ro, rows, hidden, eps, s);
        else if (vpt <= 2) launch_wave<T, 2, ADD>(x, w, r, y, ro, rows, hidden, eps, s);
        else if (vpt <= 4) launch_wave<T, 4, ADD>(x, w, r, y, ro, rows, hidden, eps, s);
        else if (vpt <= 8) launch_wave<T, 8, ADD>(x, w, r, y, ro, rows, hidden, eps, s);
        else launch_wave<T, 16, ADD>(x, w, r, y, ro, rows, hidden, eps, s);
    } else if (vec && nvec <= kThreads * 8) {
        // Narrow rows use one wave; wide rows 256 lanes with up to 8 chunks each.
        const int threads = nvec <= 64 ? 64 : (nvec <= 128 ? 128 : kThreads);
        const int vpt = (nvec + threads - 1) / threads;
        if (vpt <= 1) launch_vec<T, 1, ADD>(threads, x, w, r, y, ro, rows, hidden, eps, s);
        else if (vpt <= 2) launch_vec<T, 2, ADD>(threads, x, w, r, y, ro, rows, hidden, eps, s);
        else if (vpt <= 4) launch_vec<T, 4, ADD>(threads, x, w, r, y, ro, rows, hidden, eps, s);
        else launch_vec<T, 8, ADD>(threads, x, w, r, y, ro, rows, hidden, eps, s);
    } else {
        hipLaunchKernelGGL((rms_norm_scalar<T, ADD>), dim3(rows), dim3(kThreads), 0, s,
                           static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(w),
                           static_cast<const uint16_t *>(r), static_cast<uint16_t *>(y),
                           static_cast<uint16_t *>(ro), hidden, eps);
    }
    TECO_CHECK_LAUNCH("rms_norm");
    return TECOOPS_STATUS_SUCCESS;
}

}  // namespace

extern "C" tecoopsStatus_t tecoopsRmsNormEx(tecoopsHandle_t handle, const void *input,
                                            const void *weight, const void *residual,
                                            void *output, void *residual_out, int num_tokens,
                                            int hidden_size, float eps,
                                            tecoopsDataType_t dataType) {
    // Argument checks of reference rms_norm.cpp:41-62.
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (input == nullptr || weight == nullptr || output == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    if (residual != nullptr && residual_out == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    if (num_tokens <= 0 || hidden_size <= 0) return TECOOPS_STATUS_BAD_PARAM;
    if (!tecoops::is_16bit_float(dataType)) return TECOOPS_STATUS_BAD_PARAM;
    using tecoops::dev::bf16;
    using tecoops::dev::f16;
    const bool add = residual != nullptr;  // reference find_rms_norm.cpp:35-42
    if (dataType == TECOOPS_DATA_HALF)
        return add ? dispatch<f16, true>(handle, input, weight, residual, output, residual_out,
                                         num_tokens, hidden_size, eps)
                   : dispatch<f16, false>(handle, input, weight, nullptr, output, nullptr,
                                          num_tokens, hidden_size, eps);
    return add ? dispatch<bf16, true>(handle, input, weight, residual, output, residual_out,
                                      num_tokens, hidden_size, eps)
               : dispatch<bf16, false>(handle, input, weight, nullptr, output, nullptr,
                                       num_tokens, hidden_size, eps);
}

extern "C" tecoopsStatus_t tecoopsRmsNorm(tecoopsHandle_t handle, const void *input,
                                          const void *weight, const void *residual, void *output,
                                          void *residual_out, int num_tokens, int hidden_size,
                                          float eps) {
    return tecoopsRmsNormEx(handle, input, weight, residual, output, residual_out, num_tokens,
                            hidden_size, eps, TECOOPS_DATA_HALF);
}
