// causal_conv1d.hip — depthwise causal 1-D convolution (+bias, SiLU) with
// conv-state carry.
//
// Semantics (teco/ual/kernel/causal_conv1d/causal_conv1d.scpp:56-116 and the
// CPU baseline test/zoo/teco/causal_conv1d/causal_conv1d.py:44-122):
//   per sequence b with cache index c = cache_indices[b] (identity if NULL),
//   skipped when c == pad_slot_id or its length is 0;
//   full_x = [prefix (W-1 values), x_b],  prefix = conv_state[c] when
//   api_mode == 1 or has_initial_state[b] != 0, else zeros;
//   out[t, d] = act(sum_k full_x[t + k, d] * w[k, d] + bias[d])   (fp32 acc)
//   conv_state[c] = last W-1 entries of full_x.
// act is SiLU (v / (1 + exp(-v))); the reference always applies it.
//
// gfx950 design: every lane holds a chunk of consecutive tokens in registers
// with the W-1 inputs before it (a sliding window), so each input is fetched
// from HBM once.  Three mappings:
//   token stride 1 (e.g. [batch, dim, seqlen], the reference's [dim, tokens]):
//     a wave streams whole rows, lanes on consecutive 8-token chunks ->
//     16-byte loads / stores, the W-1 overlap passed between lanes in
//     registers (conv1d_rows_kernel);
//   channel stride 1 with dim % 8 == 0 (the reference C layout [tokens, dim]):
//     a lane owns 8 consecutive channels (one 16-byte vector per token) of a
//     16-token chunk of the global token axis; the W-1 rows before the chunk
//     are re-read from L2 (conv1d_tokens_kernel);
//   otherwise: consecutive lanes take consecutive channels of one 16-token
//     chunk with 2-byte accesses (conv1d_kernel).
// Only one lane of a (sequence, channel) touches conv_state, reading the old
// state before writing the new one, so there is no cross-lane race.
// HBM-bound: algorithmic bytes = 2 * (x + out) + weights + bias + state.
#include "common.h"
#include "device.h"

namespace {

using namespace tecoops::dev;

struct ConvArgs {
    int batch, seq_len, dim;
    const uint16_t *x;
    long long xb, xs, xd;
    uint16_t *out;
    long long ob, os, od;
    const uint16_t *w;
    int wd, ww;
    const uint16_t *bias;
    uint16_t *state;
    int state_stride;
    const int *qsl;
    const int *cidx;
    const int8_t *hinit;
    int pad_slot_id, api_mode, silu;
    int nchunks;
};

// SiLU v / (1 + e^-v) with the hardware exp2 and reciprocal (about 1 ulp
// each); saturates correctly to 0 / v for large |v|.  A template flag, so
// the kernels carry no per-element select for it.  (Folding -log2(e) into
// the weights saves one multiply per element but measured no faster: these
// kernels wait on memory, not on the VALU.)
template <bool SILU>
__device__ __forceinline__ float act(float v) {
    if (!SILU) return v;
    const float e = __builtin_amdgcn_exp2f(-v * 1.4426950408889634f);
    return v * __builtin_amdgcn_rcpf(1.0f + e);
}

// Two floats rounded to fp16 (round to nearest even) and packed, as one
// packed conversion.
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, half2_t));
}

template <int W, bool SEQ_CONTIG, int CH, bool SILU>
__device__ __forceinline__ void conv1d_body(const ConvArgs &a, int b, int d, int c) {
    long long len, xoff, ooff;
    if (a.qsl != nullptr) {
        const long long s = a.qsl[b];
        len = a.qsl[b + 1] - s;
        xoff = s * a.xs;
        ooff = s * a.os;
    } else {
        len = a.seq_len;
        xoff = b * a.xb;
        ooff = b * a.ob;
    }
    const int cidx = a.cidx ? a.cidx[b] : b;
    if (cidx == a.pad_slot_id) return;
    const long long t0 = static_cast<long long>(c) * CH;
    if (t0 >= len) return;
    const uint16_t *xr = a.x + xoff + d * a.xd;
    uint16_t *outr = a.out + ooff + d * a.od;
    const bool use_state =
        a.state != nullptr && (a.api_mode == 1 || (a.hinit != nullptr && a.hinit[b] != 0));
    uint16_t *st = a.state ? a.state + static_cast<long long>(cidx) * a.state_stride + d : nullptr;

    float wv[W];
#pragma unroll
    for (int k = 0; k < W; ++k)
        wv[k] = h2f(a.w[static_cast<long long>(d) * a.wd + k * a.ww]);
    const float bv = a.bias ? h2f(a.bias[d]) : 0.0f;

    // win[k] = full_x value at sequence position t0 - (W-1) + k
    float win[W - 1 + CH];
    uint16_t prefix[W - 1];  // old state values, used when t0 == 0
#pragma unroll
    for (int k = 0; k < W - 1; ++k)
        prefix[k] = (t0 == 0 && use_state) ? st[static_cast<long long>(k) * a.dim] : 0;
#pragma unroll
    for (int k = 0; k < W - 1; ++k) {
        const long long tt = t0 - (W - 1) + k;
        win[k] = tt >= 0 ? h2f(xr[tt * a.xs]) : h2f(prefix[k]);
    }
    const bool full = t0 + CH <= len;
    if (SEQ_CONTIG && full && tecoops::aligned(xr + t0, 16)) {
#pragma unroll
        for (int v = 0; v < CH / 8; ++v) {
            const uint4 q = *reinterpret_cast<const uint4 *>(xr + t0 + 8 * v);
            const uint32_t *pq = reinterpret_cast<const uint32_t *>(&q);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                win[W - 1 + 8 * v + 2 * j] = lo<f16>(pq[j]);
                win[W - 1 + 8 * v + 2 * j + 1] = hi<f16>(pq[j]);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < CH; ++j)
            win[W - 1 + j] = (t0 + j < len) ? h2f(xr[(t0 + j) * a.xs]) : 0.0f;
    }

    float o[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < W; ++k) acc += win[j + k] * wv[k];
        o[j] = act<SILU>(acc + bv);
    }
    if (SEQ_CONTIG && full && tecoops::aligned(outr + t0, 16)) {
#pragma unroll
        for (int v = 0; v < CH / 8; ++v) {
            uint4 q;
            uint32_t *pq = reinterpret_cast<uint32_t *>(&q);
#pragma unroll
            for (int j = 0; j < 4; ++j) pq[j] = pack_h2(o[8 * v + 2 * j], o[8 * v + 2 * j + 1]);
            *reinterpret_cast<uint4 *>(outr + t0 + 8 * v) = q;
        }
    } else {
#pragma unroll
        for (int j = 0; j < CH; ++j)
            if (t0 + j < len) outr[(t0 + j) * a.os] = f2h(o[j]);
    }

    if (c == 0 && st != nullptr) {
        uint16_t ns[W - 1];
#pragma unroll
        for (int k = 0; k < W - 1; ++k) {
            const long long src = len - (W - 1) + k;
            ns[k] = src >= 0 ? xr[src * a.xs] : prefix[W - 1 + src];
        }
#pragma unroll
        for (int k = 0; k < W - 1; ++k) st[static_cast<long long>(k) * a.dim] = ns[k];
    }
}

// Token-contiguous rows ([batch, dim, seqlen] and the reference's
// [dim, tokens]): one wave streams whole (sequence, channel) rows.  The row is
// cut into segments of 512 tokens, lane l owning tokens [8l, 8l + 8) of a
// segment as one 16-byte vector; the loads of up to kSegs segments are issued
// together, so every lane keeps kSegs vectors in flight.  The W-1 inputs
// before a lane's tokens are the last values of lane l-1's vector (a lane
// shuffle), of lane 63 of the previous segment (a readlane) for lane 0, and
// the carried last values of the previous group of segments, or the prefix
// (old conv state or zeros), at the start of a row.  A workgroup of 4 waves
// takes 4 * kRowsPerWave consecutive rows.  Token stride is 1 (x and out).
// One row per wave: at [8, 4096, 2048] that is 32768 short-lived waves, which
// keep reads and writes of different waves overlapped (47.5 us); 4 rows per
// wave made the resident waves load, compute and store in lockstep (58.3 us).
constexpr int kSegs = 4;
constexpr int kRowsPerWave = 1;

template <int W, bool SILU>
__global__ void __launch_bounds__(256) conv1d_rows_kernel(ConvArgs a) {
    constexpr int CH = 8, SEG = 64 * CH;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const long long nrows = static_cast<long long>(a.batch) * a.dim;
    const long long r0 = (static_cast<long long>(blockIdx.x) * 4 + wave) * kRowsPerWave;
    for (int rr = 0; rr < kRowsPerWave; ++rr) {
        const long long r = r0 + rr;
        if (r >= nrows) return;
        const int b = static_cast<int>(r / a.dim), d = static_cast<int>(r % a.dim);
        long long len, xoff, ooff;
        if (a.qsl != nullptr) {
            const long long s0 = a.qsl[b];
            len = a.qsl[b + 1] - s0;
            xoff = s0 * a.xs;
            ooff = s0 * a.os;
        } else {
            len = a.seq_len;
            xoff = b * a.xb;
            ooff = b * a.ob;
        }
        const int cidx = a.cidx ? a.cidx[b] : b;
        if (cidx == a.pad_slot_id || len <= 0) continue;
        const uint16_t *xr = a.x + xoff + d * a.xd;
        uint16_t *outr = a.out + ooff + d * a.od;
        const bool use_state =
            a.state != nullptr && (a.api_mode == 1 || (a.hinit != nullptr && a.hinit[b] != 0));
        uint16_t *st = a.state ? a.state + static_cast<long long>(cidx) * a.state_stride + d : nullptr;
        const bool vec_row = tecoops::aligned(xr, 16) && tecoops::aligned(outr, 16);
        float wv[W];
#pragma unroll
        for (int k = 0; k < W; ++k)
            wv[k] = h2f(a.w[static_cast<long long>(d) * a.wd + k * a.ww]);
        const float bv = a.bias ? h2f(a.bias[d]) : 0.0f;
        // prefix[k]: full_x at position k - (W-1), the old state or zeros
        uint16_t prefix[W - 1];
#pragma unroll
        for (int k = 0; k < W - 1; ++k) prefix[k] = use_state ? st[static_cast<long long>(k) * a.dim] : 0;
        // carry[k]: full_x at position g0 - 3 + k for the current group start g0
        float carry[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < W - 1; ++k) carry[3 - (W - 1) + k] = h2f(prefix[k]);

        for (long long g0 = 0; g0 < len; g0 += kSegs * SEG) {
            const int nseg = static_cast<int>(min<long long>(kSegs, (len - g0 + SEG - 1) / SEG));
            uint32_t dw[kSegs][4];
#pragma unroll
            for (int u = 0; u < kSegs; ++u) {
                if (u >= nseg) break;
                const long long t0 = g0 + u * SEG + lane * CH;
                if (vec_row && t0 + CH <= len) {
                    const uint4 q = ld_stream(reinterpret_cast<const uint4 *>(xr + t0));
                    dw[u][0] = q.x; dw[u][1] = q.y; dw[u][2] = q.z; dw[u][3] = q.w;
                } else {
                    uint16_t e[CH];
#pragma unroll
                    for (int j = 0; j < CH; ++j) e[j] = (t0 + j < len) ? xr[t0 + j] : 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        dw[u][j] = e[2 * j] | (static_cast<uint32_t>(e[2 * j + 1]) << 16);
                }
            }
#pragma unroll
            for (int u = 0; u < kSegs; ++u) {
                if (u >= nseg) break;
                const long long t0 = g0 + u * SEG + lane * CH;
                // tokens t0-3 .. t0-1: lane-1's last three, or for lane 0 the
                // previous segment's lane 63 (the carry for the first segment)
                const uint32_t p2 = __shfl_up(dw[u][2], 1, 64);
                const uint32_t p3 = __shfl_up(dw[u][3], 1, 64);
                float prev[3] = {hi<f16>(p2), lo<f16>(p3), hi<f16>(p3)};
                if (lane == 0) {
                    if (u == 0) {
                        prev[0] = carry[0]; prev[1] = carry[1]; prev[2] = carry[2];
                    } else {
                        const uint32_t q2 = __builtin_amdgcn_readlane(dw[u - 1][2], 63);
                        const uint32_t q3 = __builtin_amdgcn_readlane(dw[u - 1][3], 63);
                        prev[0] = hi<f16>(q2); prev[1] = lo<f16>(q3); prev[2] = hi<f16>(q3);
                    }
                }
                float win[W - 1 + CH];
#pragma unroll
                for (int k = 0; k < W - 1; ++k) win[k] = prev[3 - (W - 1) + k];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    win[W - 1 + 2 * j] = lo<f16>(dw[u][j]);
                    win[W - 1 + 2 * j + 1] = hi<f16>(dw[u][j]);
                }
                float o[CH];
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    float acc = 0.0f;
#pragma unroll
                    for (int k = 0; k < W; ++k) acc += win[j + k] * wv[k];
                    o[j] = act<SILU>(acc + bv);
                }
                if (vec_row && t0 + CH <= len) {
                    uint4 q;
                    q.x = pack_h2(o[0], o[1]);
                    q.y = pack_h2(o[2], o[3]);
                    q.z = pack_h2(o[4], o[5]);
                    q.w = pack_h2(o[6], o[7]);
                    st_stream(reinterpret_cast<uint4 *>(outr + t0), q);
                } else {
#pragma unroll
                    for (int j = 0; j < CH; ++j)
                        if (t0 + j < len) outr[t0 + j] = f2h(o[j]);
                }
            }
            // the next group starts at g0 + kSegs * SEG only when this group was
            // full, and then its last three tokens are lane 63's of segment kSegs-1
            const uint32_t c2 = __builtin_amdgcn_readlane(dw[kSegs - 1][2], 63);
            const uint32_t c3 = __builtin_amdgcn_readlane(dw[kSegs - 1][3], 63);
            carry[0] = hi<f16>(c2); carry[1] = lo<f16>(c3); carry[2] = hi<f16>(c3);
        }
        if (lane == 0 && st != nullptr) {
            uint16_t ns[W - 1];
#pragma unroll
            for (int k = 0; k < W - 1; ++k) {
                const long long src = len - (W - 1) + k;
                uint16_t old = 0;  // prefix[W - 1 + src] without a dynamic index
#pragma unroll
                for (int m = 0; m < W - 1; ++m)
                    if (m == W - 1 + src) old = prefix[m];
                ns[k] = src >= 0 ? xr[src] : old;
            }
#pragma unroll
            for (int k = 0; k < W - 1; ++k) st[static_cast<long long>(k) * a.dim] = ns[k];
        }
    }
}

// --------------------------------------------------- short rows, grouped

// Token-contiguous rows of a few hundred tokens at most: the wave's 64 lanes
// hold 64 / G rows side by side, G lanes per row (segments of 8G tokens), so
// that a wave is not mostly idle on a short row.  Within each group of G
// lanes this is conv1d_rows_kernel: the W-1 inputs before a lane's tokens
// come from lane l-1 of its group (a shuffle of width G), from the group's
// last lane in the previous segment, or from the carried values / the prefix
// at the start of the row.  Rows of one wave can differ in length (varlen
// batches): the wave walks the longest and every lane guards its own tokens.
template <int W, bool SILU, int G>
__global__ void __launch_bounds__(256) conv1d_rows_group_kernel(ConvArgs a) {
    constexpr int CH = 8, SEG = G * CH, R = 64 / G;
    const int lane = threadIdx.x & 63, gl = lane % G;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const long long nrows = static_cast<long long>(a.batch) * a.dim;
    const long long r = (static_cast<long long>(blockIdx.x) * 4 + wave) * R + lane / G;
    int b = 0, d = 0, cidx = 0;
    long long len = 0, xoff = 0, ooff = 0;
    if (r < nrows) {
        b = static_cast<int>(r / a.dim);
        d = static_cast<int>(r % a.dim);
        if (a.qsl != nullptr) {
            const long long s0 = a.qsl[b];
            len = a.qsl[b + 1] - s0;
            xoff = s0 * a.xs;
            ooff = s0 * a.os;
        } else {
            len = a.seq_len;
            xoff = b * a.xb;
            ooff = b * a.ob;
        }
        cidx = a.cidx ? a.cidx[b] : b;
        if (cidx == a.pad_slot_id || len < 0) len = 0;
    }
    long long mlen = len;  // the wave's longest row
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mlen = max(mlen, static_cast<long long>(__shfl_xor(mlen, o, 64)));
    if (mlen <= 0) return;
    const uint16_t *xr = a.x + xoff + d * a.xd;
    uint16_t *outr = a.out + ooff + d * a.od;
    const bool use_state = len > 0 && a.state != nullptr &&
                           (a.api_mode == 1 || (a.hinit != nullptr && a.hinit[b] != 0));
    uint16_t *st = len > 0 && a.state ? a.state + static_cast<long long>(cidx) * a.state_stride + d
                                      : nullptr;
    const bool vec_row = tecoops::aligned(xr, 16) && tecoops::aligned(outr, 16);
    float wv[W];
#pragma unroll
    for (int k = 0; k < W; ++k) wv[k] = h2f(a.w[static_cast<long long>(d) * a.wd + k * a.ww]);
    const float bv = a.bias ? h2f(a.bias[d]) : 0.0f;
    uint16_t prefix[W - 1];
#pragma unroll
    for (int k = 0; k < W - 1; ++k) prefix[k] = use_state ? st[static_cast<long long>(k) * a.dim] : 0;
    float carry[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < W - 1; ++k) carry[3 - (W - 1) + k] = h2f(prefix[k]);

    for (long long g0 = 0; g0 < mlen; g0 += kSegs * SEG) {
        uint32_t dw[kSegs][4];
#pragma unroll
        for (int u = 0; u < kSegs; ++u) {
            const long long t0 = g0 + u * SEG + gl * CH;
            if (vec_row && t0 + CH <= len) {
                const uint4 q = ld_stream(reinterpret_cast<const uint4 *>(xr + t0));
                dw[u][0] = q.x; dw[u][1] = q.y; dw[u][2] = q.z; dw[u][3] = q.w;
            } else {
                uint16_t e[CH];
#pragma unroll
                for (int j = 0; j < CH; ++j) e[j] = (t0 + j < len) ? xr[t0 + j] : 0;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    dw[u][j] = e[2 * j] | (static_cast<uint32_t>(e[2 * j + 1]) << 16);
            }
        }
#pragma unroll
        for (int u = 0; u < kSegs; ++u) {
            const long long t0 = g0 + u * SEG + gl * CH;
            // all lanes take part in the shuffles; the group's first lane then
            // takes the previous segment's last lane, or the carry
            const uint32_t p2 = __shfl_up(dw[u][2], 1, G);
            const uint32_t p3 = __shfl_up(dw[u][3], 1, G);
            const uint32_t q2 = u > 0 ? __shfl(dw[u > 0 ? u - 1 : 0][2], G - 1, G) : 0u;
            const uint32_t q3 = u > 0 ? __shfl(dw[u > 0 ? u - 1 : 0][3], G - 1, G) : 0u;
            float prev[3] = {hi<f16>(p2), lo<f16>(p3), hi<f16>(p3)};
            if (gl == 0) {
                if (u == 0) {
                    prev[0] = carry[0]; prev[1] = carry[1]; prev[2] = carry[2];
                } else {
                    prev[0] = hi<f16>(q2); prev[1] = lo<f16>(q3); prev[2] = hi<f16>(q3);
                }
            }
            if (t0 >= len) continue;
            float win[W - 1 + CH];
#pragma unroll
            for (int k = 0; k < W - 1; ++k) win[k] = prev[3 - (W - 1) + k];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                win[W - 1 + 2 * j] = lo<f16>(dw[u][j]);
                win[W - 1 + 2 * j + 1] = hi<f16>(dw[u][j]);
            }
            float o[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                float acc = 0.0f;
#pragma unroll
                for (int k = 0; k < W; ++k) acc += win[j + k] * wv[k];
                o[j] = act<SILU>(acc + bv);
            }
            if (vec_row && t0 + CH <= len) {
                uint4 q;
                q.x = pack_h2(o[0], o[1]);
                q.y = pack_h2(o[2], o[3]);
                q.z = pack_h2(o[4], o[5]);
                q.w = pack_h2(o[6], o[7]);
                st_stream(reinterpret_cast<uint4 *>(outr + t0), q);
            } else {
#pragma unroll
                for (int j = 0; j < CH; ++j)
                    if (t0 + j < len) outr[t0 + j] = f2h(o[j]);
            }
        }
        // the next group of segments starts at g0 + kSegs * SEG only where this
        // one was full, and then its last three tokens are the group's last lane's
        const uint32_t c2 = __shfl(dw[kSegs - 1][2], G - 1, G);
        const uint32_t c3 = __shfl(dw[kSegs - 1][3], G - 1, G);
        carry[0] = hi<f16>(c2); carry[1] = lo<f16>(c3); carry[2] = hi<f16>(c3);
    }
    if (gl == 0 && st != nullptr) {
        uint16_t ns[W - 1];
#pragma unroll
        for (int k = 0; k < W - 1; ++k) {
            const long long src = len - (W - 1) + k;
            uint16_t old = 0;  // prefix[W - 1 + src] without a dynamic index
#pragma unroll
            for (int m = 0; m < W - 1; ++m)
                if (m == W - 1 + src) old = prefix[m];
            ns[k] = src >= 0 ? xr[src] : old;
        }
#pragma unroll
        for (int k = 0; k < W - 1; ++k) st[static_cast<long long>(k) * a.dim] = ns[k];
    }
}

// ------------------------------------------------------- short sequences

// Decode steps and short chunks (a few tokens per sequence): one thread per
// (sequence, channel), channels fastest, so that the conv-state rows and a
// [tokens, dim] x are read and written coalesced; the thread walks its
// sequence's tokens with the window in registers.  Same arithmetic order as
// the other kernels (oldest window element first, bias, then the activation).
template <int W, bool SILU>
__global__ void __launch_bounds__(256) conv1d_short_kernel(ConvArgs a) {
    const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= static_cast<long long>(a.batch) * a.dim) return;
    const int b = static_cast<int>(i / a.dim), d = static_cast<int>(i % a.dim);
    long long len, xoff, ooff;
    if (a.qsl != nullptr) {
        const long long s0 = a.qsl[b];
        len = a.qsl[b + 1] - s0;
        xoff = s0 * a.xs;
        ooff = s0 * a.os;
    } else {
        len = a.seq_len;
        xoff = b * a.xb;
        ooff = b * a.ob;
    }
    const int cidx = a.cidx ? a.cidx[b] : b;
    if (cidx == a.pad_slot_id || len <= 0) return;
    const uint16_t *xr = a.x + xoff + d * a.xd;
    uint16_t *outr = a.out + ooff + d * a.od;
    const bool use_state =
        a.state != nullptr && (a.api_mode == 1 || (a.hinit != nullptr && a.hinit[b] != 0));
    uint16_t *st = a.state ? a.state + static_cast<long long>(cidx) * a.state_stride + d : nullptr;
    float wv[W];
#pragma unroll
    for (int k = 0; k < W; ++k) wv[k] = h2f(a.w[static_cast<long long>(d) * a.wd + k * a.ww]);
    const float bv = a.bias ? h2f(a.bias[d]) : 0.0f;
    uint16_t raw[W - 1];  // the last W-1 inputs (state or zeros before the first token)
#pragma unroll
    for (int k = 0; k < W - 1; ++k) raw[k] = use_state ? st[static_cast<long long>(k) * a.dim] : 0;
    for (long long t = 0; t < len; ++t) {
        const uint16_t xv = xr[t * a.xs];
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < W - 1; ++k) acc += h2f(raw[k]) * wv[k];
        acc += h2f(xv) * wv[W - 1];
        outr[t * a.os] = f2h(act<SILU>(acc + bv));
#pragma unroll
        for (int k = 0; k < W - 2; ++k) raw[k] = raw[k + 1];
        raw[W - 2] = xv;
    }
    if (st != nullptr) {
#pragma unroll
        for (int k = 0; k < W - 1; ++k) st[static_cast<long long>(k) * a.dim] = raw[k];
    }
}

// ------------------------------------------------ channel-contiguous tokens

constexpr int kTokChunk = 8;    // tokens per lane (4 measured alike, 16 slower)
constexpr int kTokSlab = 512;   // channels per wave (64 lanes x 8)
// Waves per workgroup, each its own 512-channel slab.  [16384, 4096] µs, 1 /
// 2 / 4 waves: 49.1-49.3 / 49.2-49.3 / 49.6-49.8 (three alternating runs).
constexpr int kTokWaves = 1;

// A sequence of the global token axis: index b, tokens [s, e); b < 0 when the
// token lies in no sequence.
struct SeqSpan {
    int b;
    long long s, e;
};

// The sequence holding global token t.  With query_start_loc, the largest b
// with qsl[b] <= t (empty sequences before it share its start); otherwise
// sequence t / seq_len.
__device__ __forceinline__ SeqSpan seq_of(const ConvArgs &a, long long t) {
    SeqSpan r{-1, 0, 0};
    if (a.qsl == nullptr) {
        const long long b = t / a.seq_len;
        if (t < 0 || b >= a.batch) return r;
        r.b = static_cast<int>(b);
        r.s = b * a.seq_len;
        r.e = r.s + a.seq_len;
        return r;
    }
    if (t < a.qsl[0] || t >= a.qsl[a.batch]) return r;
    int lo = 0, hi = a.batch - 1;  // qsl[lo] <= t
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.qsl[mid] <= t) lo = mid; else hi = mid - 1;
    }
    r.b = lo;
    r.s = a.qsl[lo];
    r.e = a.qsl[lo + 1];
    return r;
}

// Element offsets of token t of sequence sp in x and out.
__device__ __forceinline__ long long x_off(const ConvArgs &a, const SeqSpan &sp, long long t) {
    return a.qsl ? t * a.xs : sp.b * a.xb + (t - sp.s) * a.xs;
}
__device__ __forceinline__ long long o_off(const ConvArgs &a, const SeqSpan &sp, long long t) {
    return a.qsl ? t * a.os : sp.b * a.ob + (t - sp.s) * a.os;
}

__device__ __forceinline__ void unpack8(const uint4 &q, float (&v)[8]) {
    v[0] = lo<f16>(q.x); v[1] = hi<f16>(q.x); v[2] = lo<f16>(q.y); v[3] = hi<f16>(q.y);
    v[4] = lo<f16>(q.z); v[5] = hi<f16>(q.z); v[6] = lo<f16>(q.w); v[7] = hi<f16>(q.w);
}

// Conv state row r (0 .. W-2: full_x position r - (W-1)) of the 8 channels at
// d0 for cache entry cidx.
__device__ __forceinline__ uint4 *state_row(const ConvArgs &a, int cidx, int r, int d0) {
    return reinterpret_cast<uint4 *>(a.state + static_cast<long long>(cidx) * a.state_stride +
                                     static_cast<long long>(r) * a.dim + d0);
}

// Output row of token t (sequence sp) for the 8 channels at d0, its window
// read from x and, for positions before the sequence start, from the old
// state (or zeros).  The boundary path of conv1d_tokens_kernel.
template <int W, bool SILU>
__device__ __forceinline__ void token_row(const ConvArgs &a, const SeqSpan &sp, int cidx,
                                          bool use_state, long long t, int d0,
                                          const float (&wv)[W][8], const float (&bv)[8]) {
    float acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = bv[c];
#pragma unroll
    for (int k = 0; k < W; ++k) {
        const long long pos = t - (W - 1) + k;
        uint4 q = {0u, 0u, 0u, 0u};
        if (pos >= sp.s)
            q = *reinterpret_cast<const uint4 *>(a.x + x_off(a, sp, pos) + d0);
        else if (use_state)
            q = *state_row(a, cidx, static_cast<int>(pos - sp.s + (W - 1)), d0);
        float v[8];
        unpack8(q, v);
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] += v[c] * wv[k][c];
    }
    uint4 o;
    o.x = pack_h2(act<SILU>(acc[0]), act<SILU>(acc[1]));
    o.y = pack_h2(act<SILU>(acc[2]), act<SILU>(acc[3]));
    o.z = pack_h2(act<SILU>(acc[4]), act<SILU>(acc[5]));
    o.w = pack_h2(act<SILU>(acc[6]), act<SILU>(acc[7]));
    *reinterpret_cast<uint4 *>(a.out + o_off(a, sp, t) + d0) = o;
}

// Channel-contiguous layout ([tokens, dim] rows, dim % 8 == 0, 16-byte
// aligned rows): work item (chunk, slab) covers tokens [8 chunk, +8) of the
// global token axis and channels [512 kTokWaves slab, +512 kTokWaves), wave
// w and lane l channels [512 (kTokWaves slab + w) + 8 l, +8) as one 16-byte
// vector per token.
// Work items are dealt to the 8 XCDs in contiguous ranges (workgroup n runs
// on XCD n % 8), so the W-1 rows before a chunk, which the previous chunk
// loaded, are L2 hits.
//
// A chunk inside one sequence and at least W-1 tokens past its start loads
// its W-1 + 8 rows at once and convolves them in registers.  Rows that no
// other chunk reads go through the non-temporal path; the window (the W-1
// rows before the chunk, read last here) and the chunk's last W-1 rows (the
// next chunk's window) stay in L2.  Measured at the BASELINE shape: 48.9 us,
// against 55.6 us with every load plain, 57.6 us with every load
// non-temporal (the next chunk's window then misses L2) and 52.8 us with
// the window non-temporal too; passing the window between the waves of a
// workgroup through LDS instead of L2 cost a barrier and ran 49.5 us.
//
// Other chunks take their tokens one at a time (token_row), by this
// ownership rule: a token within W-1 of its sequence's start belongs to the
// chunk holding that start (even past the chunk's end), every other token to
// the chunk holding it.  Only the chunk holding a sequence's start then reads
// the sequence's old conv state, and it writes the new state after its
// tokens, so no lane reads a state another lane writes.
template <int W, bool SILU>
__global__ void __launch_bounds__(kTokWaves * 64) conv1d_tokens_kernel(ConvArgs a, long long nitems,
                                                            long long per_xcd, int nslabs) {
    constexpr int CH = kTokChunk;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const long long item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (item >= nitems) return;
    const long long t0 = (item / nslabs) * CH;
    const int d0 = static_cast<int>(item % nslabs) * (kTokWaves * kTokSlab) + wave * kTokSlab + lane * 8;
    if (d0 >= a.dim) return;
    const SeqSpan sp = seq_of(a, t0);
    if (sp.b < 0 && t0 >= (a.qsl ? a.qsl[a.batch] : static_cast<long long>(a.batch) * a.seq_len))
        return;  // past the last sequence

    float wv[W][8], bv[8];
    if (a.wd == 1 && a.ww % 8 == 0 && tecoops::aligned(a.w, 16)) {
        // channel-contiguous weight ([width, dim], the reference layout)
#pragma unroll
        for (int k = 0; k < W; ++k)
            unpack8(*reinterpret_cast<const uint4 *>(a.w + static_cast<long long>(k) * a.ww + d0),
                    wv[k]);
    } else {
#pragma unroll
        for (int k = 0; k < W; ++k)
#pragma unroll
            for (int c = 0; c < 8; ++c)
                wv[k][c] = h2f(a.w[static_cast<long long>(d0 + c) * a.wd + k * a.ww]);
    }
    if (a.bias != nullptr && tecoops::aligned(a.bias, 16)) {
        unpack8(*reinterpret_cast<const uint4 *>(a.bias + d0), bv);
    } else {
#pragma unroll
        for (int c = 0; c < 8; ++c) bv[c] = a.bias ? h2f(a.bias[d0 + c]) : 0.0f;
    }

    const int cidx0 = sp.b >= 0 ? (a.cidx ? a.cidx[sp.b] : sp.b) : 0;
    if (sp.b >= 0 && t0 - sp.s >= W - 1 && t0 + CH <= sp.e) {
        if (cidx0 == a.pad_slot_id) return;
        // rows t0 - (W-1) .. t0 + CH - 1, all inside the sequence
        const uint16_t *xr = a.x + x_off(a, sp, t0 - (W - 1)) + d0;
        uint4 raw[W - 1 + CH];
#pragma unroll
        for (int j = 0; j < W - 1 + CH; ++j) {
            const uint4 *p = reinterpret_cast<const uint4 *>(xr + j * a.xs);
            raw[j] = (j >= W - 1 && j < CH) ? ld_stream(p) : *p;
        }
        float win[W][8];
#pragma unroll
        for (int k = 0; k < W - 1; ++k) unpack8(raw[k], win[k + 1]);
        uint16_t *outr = a.out + o_off(a, sp, t0) + d0;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
#pragma unroll
            for (int k = 0; k < W - 1; ++k)
#pragma unroll
                for (int c = 0; c < 8; ++c) win[k][c] = win[k + 1][c];
            unpack8(raw[W - 1 + j], win[W - 1]);
            float o[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                float acc = bv[c];
#pragma unroll
                for (int k = 0; k < W; ++k) acc += win[k][c] * wv[k][c];
                o[c] = act<SILU>(acc);
            }
            uint4 q;
            q.x = pack_h2(o[0], o[1]);
            q.y = pack_h2(o[2], o[3]);
            q.z = pack_h2(o[4], o[5]);
            q.w = pack_h2(o[6], o[7]);
            st_stream(reinterpret_cast<uint4 *>(outr + j * a.os), q);
        }
        return;
    }

    // Boundary chunk: its tokens one at a time, by the ownership rule.
    SeqSpan cur = sp;
    for (long long t = t0; t < t0 + CH + W - 2; ++t) {
        if (cur.b < 0 || t >= cur.e) cur = seq_of(a, t);
        if (cur.b < 0) continue;
        const bool owned = t - cur.s >= W - 1 ? t < t0 + CH : (cur.s >= t0 && cur.s < t0 + CH);
        if (!owned) continue;
        const int cidx = a.cidx ? a.cidx[cur.b] : cur.b;
        if (cidx == a.pad_slot_id) continue;
        const bool use_state = a.state != nullptr &&
                               (a.api_mode == 1 || (a.hinit != nullptr && a.hinit[cur.b] != 0));
        token_row<W, SILU>(a, cur, cidx, use_state, t, d0, wv, bv);
    }
    // New conv states of the (non-empty) sequences that start in this chunk:
    // the last W-1 entries of full_x, read (x, or the old state for short
    // sequences) before any is written.
    if (a.state == nullptr) return;
    int b = sp.b >= 0 ? sp.b : 0;
    if (sp.b >= 0 && sp.s < t0) ++b;
    for (; b < a.batch; ++b) {
        SeqSpan q;
        q.b = b;
        q.s = a.qsl ? a.qsl[b] : static_cast<long long>(b) * a.seq_len;
        q.e = a.qsl ? a.qsl[b + 1] : q.s + a.seq_len;
        if (q.s >= t0 + CH) break;
        if (q.s < t0 || q.e <= q.s) continue;
        const int cidx = a.cidx ? a.cidx[b] : b;
        if (cidx == a.pad_slot_id) continue;
        const bool use_state = a.api_mode == 1 || (a.hinit != nullptr && a.hinit[b] != 0);
        uint4 ns[W - 1];
#pragma unroll
        for (int k = 0; k < W - 1; ++k) {
            const long long pos = q.e - (W - 1) + k;
            uint4 v = {0u, 0u, 0u, 0u};
            if (pos >= q.s)
                v = *reinterpret_cast<const uint4 *>(a.x + x_off(a, q, pos) + d0);
            else if (use_state)
                v = *state_row(a, cidx, static_cast<int>(pos - q.s + (W - 1)), d0);
            ns[k] = v;
        }
#pragma unroll
        for (int k = 0; k < W - 1; ++k) *state_row(a, cidx, k, d0) = ns[k];
    }
}

template <int W, bool SEQ_CONTIG, int CH, bool SILU>
__global__ void __launch_bounds__(256) conv1d_kernel(ConvArgs a) {
    // SEQ_CONTIG: grid (chunk blocks, channels, batch), chunk fastest;
    // otherwise: grid (channel blocks, chunks, batch), channel fastest.
    const int b = blockIdx.z;
    const int lin = blockIdx.x * blockDim.x + threadIdx.x;
    for (int y = blockIdx.y; y < (SEQ_CONTIG ? a.dim : a.nchunks); y += gridDim.y) {
        const int c = SEQ_CONTIG ? lin : y;
        const int d = SEQ_CONTIG ? y : lin;
        if ((SEQ_CONTIG ? c >= a.nchunks : d >= a.dim)) return;
        conv1d_body<W, SEQ_CONTIG, CH, SILU>(a, b, d, c);
    }
}

// The channel-contiguous kernel's preconditions: channel stride 1 in x and
// out, 8-channel vectors 16-byte aligned everywhere they are read or written.
bool tokens_layout(const ConvArgs &a) {
    using tecoops::aligned;
    if (a.xd != 1 || a.od != 1 || a.dim % 8 != 0) return false;
    if (!aligned(a.x, 16) || !aligned(a.out, 16) || a.xs % 8 || a.os % 8) return false;
    if (a.qsl == nullptr && (a.xb % 8 || a.ob % 8)) return false;
    if (a.state != nullptr && (!aligned(a.state, 16) || a.state_stride % 8)) return false;
    return true;
}

// Mean sequence length up to which conv1d_short_kernel runs rather than the
// grouped-row kernel: its per-thread token walk is one dependent round trip
// per token, and coalesced only when neighbouring channels are close in
// memory.  dim 4096, 64 sequences, short / 16 rows per wave: [B, dim, L]
// with 8 tokens 8.4 / 12.4 us, 12 tokens 10.5 / 15.0 us; [dim, tokens]
// (channels a whole token axis apart) with 4 tokens 10.8 / 10.7 us, 8 tokens
// 18.3 / 15.7 us.  One token: 8 us against 134 us with one row per wave.
constexpr long long kShortLenNear = 12, kShortLenFar = 4;

template <int W, bool SILU>
void launch(const ConvArgs &a0, bool seq_contig, long long max_len, hipStream_t s) {
    ConvArgs a = a0;
    if (!seq_contig && tokens_layout(a)) {
        // global token axis: sum of lengths bounded by max_len with
        // query_start_loc, batch * seq_len without
        const long long tokens = a.qsl ? max_len : static_cast<long long>(a.batch) * a.seq_len;
        const long long chunks = (tokens + kTokChunk - 1) / kTokChunk;
        const int nslabs = static_cast<int>(tecoops::ceil_div(a.dim, kTokWaves * kTokSlab));
        const long long nitems = chunks * nslabs;
        const long long per_xcd = (nitems + 7) / 8;
        hipLaunchKernelGGL((conv1d_tokens_kernel<W, SILU>), dim3(static_cast<unsigned>(8 * per_xcd)),
                           dim3(kTokWaves * 64), 0, s, a, nitems, per_xcd, nslabs);
        return;
    }
    // mean tokens per sequence: the whole axis over the batch with
    // query_start_loc, seq_len without
    const long long mean_len = a.qsl ? (max_len + a.batch - 1) / a.batch : a.seq_len;
    if (mean_len <= (a.xd <= 64 ? kShortLenNear : kShortLenFar)) {
        const unsigned grid =
            static_cast<unsigned>(tecoops::ceil_div(static_cast<long long>(a.batch) * a.dim, 256));
        hipLaunchKernelGGL((conv1d_short_kernel<W, SILU>), dim3(grid), dim3(256), 0, s, a);
        return;
    }
    if (seq_contig && mean_len <= 256) {
        // short rows: 16, 8, 4 or 2 rows per wave (segments of 32, 64, 128
        // and 256 tokens)
        const long long rows = static_cast<long long>(a.batch) * a.dim;
        const int rpw = mean_len <= 32 ? 16 : mean_len <= 64 ? 8 : mean_len <= 128 ? 4 : 2;
        const unsigned grid = static_cast<unsigned>(tecoops::ceil_div(rows, 4LL * rpw));
        if (rpw == 16)
            hipLaunchKernelGGL((conv1d_rows_group_kernel<W, SILU, 4>), dim3(grid), dim3(256), 0, s, a);
        else if (rpw == 8)
            hipLaunchKernelGGL((conv1d_rows_group_kernel<W, SILU, 8>), dim3(grid), dim3(256), 0, s, a);
        else if (rpw == 4)
            hipLaunchKernelGGL((conv1d_rows_group_kernel<W, SILU, 16>), dim3(grid), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((conv1d_rows_group_kernel<W, SILU, 32>), dim3(grid), dim3(256), 0, s, a);
        return;
    }
    if (seq_contig) {
        (void)max_len;
        const long long rows = static_cast<long long>(a.batch) * a.dim;
        const unsigned grid = static_cast<unsigned>(tecoops::ceil_div(rows, 4LL * kRowsPerWave));
        hipLaunchKernelGGL((conv1d_rows_kernel<W, SILU>), dim3(grid), dim3(256), 0, s, a);
    } else {
        constexpr int CH = 16;
        a.nchunks = static_cast<int>((max_len + CH - 1) / CH);
        dim3 grid(tecoops::ceil_div(a.dim, 256), a.nchunks < 65535 ? a.nchunks : 65535, a.batch);
        hipLaunchKernelGGL((conv1d_kernel<W, false, CH, SILU>), grid, dim3(256), 0, s, a);
    }
}

}  // namespace

extern "C" tecoopsStatus_t tecoopsCausalConv1dEx(
    tecoopsHandle_t handle, int batch, int seqLen, int dim, int width, const void *x,
    long long xBatchStride, long long xSeqStride, long long xDimStride, void *out,
    long long outBatchStride, long long outSeqStride, long long outDimStride, const void *weight,
    int wDimStride, int wWidthStride, const void *bias, void *convState, int convStateStride,
    const int *queryStartLoc, const int *convStateIndices, const int8_t *hasInitialState,
    int padSlotId, int api_mode, int silu) {
    // Argument checks of reference causal_conv1d.cpp:39-54, plus the width
    // range this library supports and a usable sequence-length bound.
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (x == nullptr || weight == nullptr || out == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    if (batch <= 0 || seqLen <= 0 || dim <= 0 || width <= 0) return TECOOPS_STATUS_BAD_PARAM;
    if (batch > 65535) return TECOOPS_STATUS_NOT_SUPPORTED;  // grid z limit
    if (width < 2 || width > 4) {
        TECO_ERROR("causal_conv1d: width %d not supported (2..4)", width);
        return TECOOPS_STATUS_NOT_SUPPORTED;
    }
    ConvArgs a{};
    a.batch = batch;
    a.seq_len = seqLen;
    a.dim = dim;
    a.x = static_cast<const uint16_t *>(x);
    a.xb = xBatchStride; a.xs = xSeqStride; a.xd = xDimStride;
    a.out = static_cast<uint16_t *>(out);
    a.ob = outBatchStride; a.os = outSeqStride; a.od = outDimStride;
    a.w = static_cast<const uint16_t *>(weight);
    a.wd = wDimStride; a.ww = wWidthStride;
    a.bias = static_cast<const uint16_t *>(bias);
    a.state = static_cast<uint16_t *>(convState);
    a.state_stride = convStateStride;
    a.qsl = queryStartLoc;
    a.cidx = convStateIndices;
    a.hinit = hasInitialState;
    a.pad_slot_id = padSlotId;
    a.api_mode = api_mode;
    a.silu = silu != 0;
    const bool seq_contig = xSeqStride == 1 && outSeqStride == 1;
    hipStream_t st = handle->stream;
    switch (width * 2 + (a.silu ? 1 : 0)) {
        case 4: launch<2, false>(a, seq_contig, seqLen, st); break;
        case 5: launch<2, true>(a, seq_contig, seqLen, st); break;
        case 6: launch<3, false>(a, seq_contig, seqLen, st); break;
        case 7: launch<3, true>(a, seq_contig, seqLen, st); break;
        case 8: launch<4, false>(a, seq_contig, seqLen, st); break;
        default: launch<4, true>(a, seq_contig, seqLen, st); break;
    }
    TECO_CHECK_LAUNCH("causal_conv1d");
    return TECOOPS_STATUS_SUCCESS;
}

extern "C" tecoopsStatus_t tecoopsCausalConv1d(
    tecoopsHandle_t handle, int batch, int totalSeqLen, int dim, int width, int convStateStride,
    int xSeqStride, int outSeqStride, int padSlotId, int api_mode, int actMode, const void *x,
    void *convState, const void *weight, void *out, const int *queryStartLoc,
    const int *convStateIndices, const int8_t *hasInitialState) {
    (void)actMode;  // ignored: SiLU always applied (reference causal_conv1d.scpp:110)
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (x == nullptr || weight == nullptr || out == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    if (batch <= 0 || totalSeqLen <= 0 || dim <= 0 || width <= 0) return TECOOPS_STATUS_BAD_PARAM;
    // Layout [totalSeqLen, dim]; without queryStartLoc sequence b is the single
    // token at row b (reference causal_conv1d.scpp:58-60).
    const int seq_len_bound = queryStartLoc ? totalSeqLen : 1;
    return tecoopsCausalConv1dEx(handle, batch, seq_len_bound, dim, width, x, xSeqStride,
                                 xSeqStride, 1, out, outSeqStride, outSeqStride, 1, weight, 1,
                                 dim, nullptr, convState, convStateStride, queryStartLoc,
                                 convStateIndices, hasInitialState, padSlotId, api_mode, 1);
}
