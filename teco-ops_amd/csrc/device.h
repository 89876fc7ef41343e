// device.h — gfx950 device helpers shared by the kernels: 16-bit float
// element types, conversions, 128-bit vector access and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tecoops {
namespace dev {

// Element tags: the kernels move 16-bit floats as raw bits and convert to fp32
// for arithmetic.
struct f16 {};
struct bf16 {};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return static_cast<float>(v);
}

__device__ __forceinline__ uint16_t f2h(float f) {
    _Float16 v = static_cast<_Float16>(f);  // v_cvt_f16_f32, round to nearest even
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

__device__ __forceinline__ float b2f(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f2b(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

template <typename T> struct Cvt;
template <> struct Cvt<f16> {
    static __device__ __forceinline__ float to(uint16_t v) { return h2f(v); }
    static __device__ __forceinline__ uint16_t from(float f) { return f2h(f); }
};
template <> struct Cvt<bf16> {
    static __device__ __forceinline__ float to(uint16_t v) { return b2f(v); }
    static __device__ __forceinline__ uint16_t from(float f) { return f2b(f); }
};

// Low / high 16-bit halves of a packed dword as fp32.
template <typename T>
__device__ __forceinline__ float lo(uint32_t w) { return Cvt<T>::to(static_cast<uint16_t>(w)); }
template <typename T>
__device__ __forceinline__ float hi(uint32_t w) { return Cvt<T>::to(static_cast<uint16_t>(w >> 16)); }

template <typename T>
__device__ __forceinline__ uint32_t pack(float a, float b) {
    return static_cast<uint32_t>(Cvt<T>::from(a)) | (static_cast<uint32_t>(Cvt<T>::from(b)) << 16);
}

// Streaming 128-bit access for tensors touched once per launch: the
// non-temporal policy keeps them from displacing reused data (weights, block
// tables) in L2 / MALL.
typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
template <typename V>
__device__ __forceinline__ V ld_stream(const V *p) {
    if constexpr (sizeof(V) == 16)
        return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt *>(p)));
    else
        return __builtin_nontemporal_load(p);
}
template <typename V>
__device__ __forceinline__ void st_stream(V *p, const V &v) {
    if constexpr (sizeof(V) == 16)
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4_nt, v), reinterpret_cast<u32x4_nt *>(p));
    else
        __builtin_nontemporal_store(v, p);
}

// Value of lane l ^ 32 combined with lane l's own, through v_permlane32_swap
// (a VALU lane-half swap on gfx950, no LDS round trip).  With both operands
// equal to x, the swap returns {x[l], x[l + 32]} in lanes 0-31 and
// {x[l - 32], x[l]} in lanes 32-63.
__device__ __forceinline__ float half_swap_max(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(r[0])),
                 __builtin_bit_cast(float, static_cast<uint32_t>(r[1])));
}

__device__ __forceinline__ float half_swap_sum(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) +
           __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}

// Lane l combined with the lane that dpp_ctrl CTRL selects within its row of
// 16 (a DPP operand of the VALU op, no LDS round trip).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane 7 - l within each 8 lanes
constexpr int kDppMirror = 0x140;      // lane 15 - l within each 16 lanes
constexpr int kDppRor4 = 0x124;        // rotation by 4 lanes within each 16
constexpr int kDppRor8 = 0x128;        // rotation by 8 lanes within each 16

// Rows 2i and 2i + 1 (16 lanes each) combined through v_permlane16_swap: with
// both operands equal to x, the two results hold row 2i and row 2i + 1 of x in
// both rows of the pair.
__device__ __forceinline__ float row_swap_sum(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, static_cast<uint32_t>(r[0])) +
           __builtin_bit_cast(float, static_cast<uint32_t>(r[1]));
}
__device__ __forceinline__ float row_swap_max(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return fmaxf(__builtin_bit_cast(float, static_cast<uint32_t>(r[0])),
                 __builtin_bit_cast(float, static_cast<uint32_t>(r[1])));
}

// Sum over the 64 lanes, in every lane, without LDS: pairs, quads, halves and
// rows through DPP, then row pairs and wave halves through the permlane swaps.
// Every step adds two operands that the partner lane adds too, so all lanes
// end with the same bits.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    v = row_swap_sum(v);
    return half_swap_sum(v);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppMirror>(v));
    v = row_swap_max(v);
    return half_swap_max(v);
}

}  // namespace dev
}  // namespace tecoops
