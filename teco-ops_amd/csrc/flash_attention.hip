// flash_attention.hip — paged, varlen, causal, GQA attention on gfx950 MFMA.
//
// Semantics (teco/interface/ops/flash_attention.cpp:71-119,
// teco/ual/kernel/flash_attention/flash_attention.scpp:179-416, CPU baseline
// test/zoo/teco/flash_attention/flash_attention.py:79-140):
//   for sequence b with q_len L and kv_len S, query row i (0-based in its
//   chunk) sits at causal position q_start + i, q_start = max(S - L, 0)
//   (bottom-right alignment) and sees keys j <= q_start + i, j < S.  Head h
//   reads kv head h / (H / Hkv).  O = softmax(scale * Q K^T + mask) V with an
//   fp32 online softmax whose running max is clamped at >= 0 (scpp:149), P
//   rounded to the element type before the PV product (scpp:316-329), and
//   rows with no visible key written as 0 (scpp:388).
//   K/V are read from the paged caches [num_blocks, Hkv, block_size, D]
//   through block_table[b][j / block_size].
//
// gfx950 design (one wave = 64 lanes; v_mfma_f32_32x32x16_{bf16,f16}):
//   * Scores are computed transposed, S^T = K Q^T, so each lane owns one query
//     column (lane % 32) and 16 key rows per 32x32 block: the row max / sum of
//     the online softmax is a lane-local reduction plus one exchange with the
//     other half-wave.  P^T stays in registers and is directly the B operand
//     of O^T += V^T P^T (the key order inside an MFMA k-step is permuted
//     consistently on both operands).
//   * Prefill with D = 128 and a paged cache (block_size a multiple of 8):
//     K and V tiles go from HBM straight into LDS (global_load_lds_dwordx4,
//     no registers), two tiles ahead in a ring of three buffers, in a layout
//     of 4-row blocks (rows chunk-major, 64-byte pad per block) on which the
//     128-bit K reads and the transposing V reads (ds_read_b64_tr_b16, the A
//     operand of the PV product) are conflict-free.  Decode with D = 128
//     stages K and V row-major through registers (16- and 32-byte row pads),
//     with the same transposing V reads.  The other loaders stage K row-major
//     (16-byte pad) and V transposed (V^T[d][key], 4-element pad, two plain
//     64-bit reads).  Global -> register prefetch of the next tile overlaps
//     the current tile's MFMA work.
//   * Prefill (D = 128, block_size a multiple of 8): a workgroup of 12 waves
//     (3 per SIMD) shares each 96-key K/V tile among up to 4 query heads of
//     one GQA group (HW heads x (12/HW) row blocks of 32); other shapes use 4
//     waves and 64-key tiles.  The grid walks query tiles heaviest-first and
//     keeps all tiles of one (batch, kv head) on the same XCD (workgroup index
//     % 8 depends only on (b, kv head) when B*Hkv*groups is a multiple of 8),
//     so K/V are re-read from that XCD's L2.  MFMA-bound: 4*D*visible(q, k)
//     FLOP per (q row, head).  A wave issues MFMA and VALU work serially, so
//     the MFMA pipe is kept busy by the other waves of its SIMD: occupancy
//     (waves per SIMD) is the main lever.
//   * Decode (G * q_len <= 32): the 32 MFMA columns hold every (head, row) of
//     a GQA group; 4 waves split each 128-key tile and the key range is split
//     across workgroups (split-KV), partial (m, l, O) merged first in LDS and
//     then by a combine kernel.  HBM-bound: every cached K/V byte is read
//     once.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>

#include "common.h"
#include "device.h"
#include "flash_attention.h"

namespace {

using namespace tecoops::dev;
using tecoops::fa::FaCall;
using tecoops::fa::FaParams;
using tecoops::fa::Plan;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

template <typename T> struct Mma;
template <> struct Mma<bf16> {
    static __device__ __forceinline__ f32x16_t run(const u32x4 &a, const u32x4 &b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float a, float b) {
        float2_t v = {a, b};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf162_t));
    }
};
template <> struct Mma<f16> {
    static __device__ __forceinline__ f32x16_t run(const u32x4 &a, const u32x4 &b, f32x16_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                      __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float a, float b) {
        float2_t v = {a, b};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, half2_t));
    }
};

constexpr float kNegInf = -INFINITY;


// P values are computed against a running max that is only raised when a
// tile's max exceeds it by more than this (log2 domain), so that the O / l
// rescale runs rarely; P <= 2^kRescaleSlack stays exact in fp32 and keeps
// its relative precision in 16 bit.
constexpr float kRescaleSlack = 8.0f;

// Pad (elements) of a row-major V row in LDS: each 16-lane group of the PV
// product's transposing reads takes 4 key rows x 8 dwords, which a row pitch
// of 72 dwords puts on distinct banks (measured against pads of 8 and 32:
// prefill 547 vs 554 and 550 us at B4 x 4096).
constexpr int kVRowPad = 16;

// With q_lens the offset is the sum of the lengths before b, taken by the 64
// lanes of the wave in parallel (called by every lane of every wave).
__device__ __forceinline__ void seq_info(const FaParams &p, int b, long long &q_off, int &L) {
    if (p.q_lens == nullptr) {
        q_off = p.cu_q[b];
        L = p.cu_q[b + 1] - p.cu_q[b];
    } else {
        long long off = 0;
        for (int i = threadIdx.x & 63; i < b; i += 64) off += p.q_lens[i];
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) off += __shfl_xor(off, d, 64);
        q_off = off;
        L = p.q_lens[b];
    }
}

// kv length of sequence b.  The reference reads block_table[b][j / block_size]
// for every key j < kv_len from a row of block_table_dim entries
// (flash_attention.scpp:190, :206), so kv_len <= block_table_dim * block_size
// is its precondition; clamping to that keeps every block-table read inside
// the row.  A negative length counts as 0.
__device__ __forceinline__ int kv_len(const FaParams &p, int b) {
    return min(max(p.kv_lens[b], 0), p.kv_cap);
}

// Output rows past cu_seqlens_q[batch] belong to no sequence (padding of a
// captured graph, say).  With cumulative offsets they are written as zeros,
// as the reference torch wrapper zeroes its whole output before the call
// (api/torch_ext.cpp:128-132); the rows of the sequences are all written by
// the attention kernels, so only this tail needs it.  One workgroup, 16-byte
// stores; in the usual case the offsets cover every row and nothing is done.
__device__ __forceinline__ void zero_tail_rows(const FaParams &p, int D) {
    if (p.cu_q == nullptr) return;
    const long long end = max(p.cu_q[p.batch], 0);
    if (end >= p.total_q) return;
    const long long chunks = static_cast<long long>(p.H) * D / 8;  // per row
    u32x4 *o = reinterpret_cast<u32x4 *>(p.o);
    const u32x4 zero = {0u, 0u, 0u, 0u};
    for (long long c = end * chunks + threadIdx.x; c < p.total_q * chunks; c += blockDim.x) o[c] = zero;
}

// 16-byte K/V load; STREAM selects the non-temporal policy for data read once.
template <bool STREAM>
__device__ __forceinline__ u32x4 load16(const uint16_t *p) {
    if constexpr (STREAM)
        return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    else
        return *reinterpret_cast<const u32x4 *>(p);
}

// Element offset of key row `kv` of the (sequence, kv head) whose block-table
// row is bt_row and whose head offset inside a block is head_off.  Rows at or
// beyond kv_limit, and rows whose page id is out of range, are redirected to
// a row that exists and reported through ok = false; the caller zeroes V for
// them and masks K.
// Block-size modes of the loaders (a template argument, so that the power
// of two case keeps its shift): 0 any block_size (one block-table lookup per
// key row), 1 a power of two >= 8, 2 another multiple of 8.  Cache block of
// key row kv: a shift in mode 1, a division otherwise.
template <int BSM>
__device__ __forceinline__ int block_of(const FaParams &p, int kv) {
    return BSM == 1 ? kv >> p.lbs : kv / p.bs;
}

template <int D, int BSM>
__device__ __forceinline__ long long row_offset(const FaParams &p, const int *bt_row,
                                                long long head_off, int kv, int kv_limit,
                                                bool &ok) {
    ok = kv < kv_limit;
    const int kvs = ok ? kv : 0;
    int blk, off;
    if (BSM == 1) {
        blk = kvs >> p.lbs;
        off = kvs & (p.bs - 1);
    } else {
        blk = kvs / p.bs;
        off = kvs - blk * p.bs;
    }
    int page = bt_row[blk];
    ok = ok && page >= 0 && page < p.num_blocks;
    page = ok ? page : 0;
    return static_cast<long long>(page) * p.page_stride + head_off + static_cast<long long>(off) * D;
}

// Cooperative global -> register -> LDS staging of one TILE-key K/V tile by NT
// threads, for any head size D that is a multiple of 32.  K is stored
// row-major [TILE][D + 8]; V transposed [D][TILE + 4].  The TILE * D/8
// 16-byte chunks of K are dealt to the threads in order (chunk tid + i*NT is
// row / column (tid + i*NT) / (D/8), % (D/8)); each thread also owns VPT
// (4-row x 8-column) blocks of V.
template <int D, int TILE, int NT, int BSM, bool STREAM = false>
struct TileLoader {
    static constexpr int KP = D + 8;
    static constexpr int VP = TILE + 4;
    static constexpr int VR = 0;
    static constexpr int VOFF = TILE * KP;  // V region of a tile buffer
    static constexpr bool DMA = false;
    static constexpr int STAGES = 2;  // tile buffers in LDS
    static constexpr int ELEMS = TILE * KP + D * VP;  // one K + V^T buffer
    static constexpr int CPR = D / 8;                  // 16-byte chunks per row
    static constexpr int KTASKS = TILE * CPR;
    static constexpr int KCH = (KTASKS + NT - 1) / NT;
    static constexpr int VTASKS = (TILE / 4) * CPR;
    static constexpr int VPT = (VTASKS + NT - 1) / NT;
    static_assert(D % 32 == 0 && TILE % 4 == 0, "whole 32-column slabs and 4-row V blocks");
    u32x4 k[KCH];
    u32x4 v[VPT][4];
    uint32_t vok;  // bit 4i+r: V row of v[i][r] is valid (below kv_limit, page in range)

    __device__ __forceinline__ void prefetch(const FaParams &, const int *, int, int) {}

    __device__ __forceinline__ void load(const FaParams &p, const int *bt_row, long long head_off,
                                         int j0, int kv_limit) {
        const int tid = threadIdx.x;
        // All page lookups first, then all K/V loads: a load whose address
        // waits on a block-table read interleaved with the K/V loads would
        // wait for every K/V load issued before it (loads complete in order),
        // one round trip per row.
        long long ko[KCH], vo[VPT][4];
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int task = tid + i * NT;
            if (KTASKS % NT != 0 && task >= KTASKS) continue;
            bool ok;
            ko[i] = row_offset<D, BSM>(p, bt_row, head_off, j0 + task / CPR, kv_limit, ok);
        }
        // Invalid V rows are zeroed in store(), so the wave does not wait for
        // the loads here.
        vok = 0;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int task = tid + i * NT;
            if (VTASKS % NT != 0 && task >= VTASKS) continue;
            const int rg = task % (TILE / 4);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                bool ok;
                vo[i][r] = row_offset<D, BSM>(p, bt_row, head_off, j0 + 4 * rg + r, kv_limit, ok);
                vok |= (ok ? 1u : 0u) << (4 * i + r);
            }
        }
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            if (KTASKS % NT != 0 && tid + i * NT >= KTASKS) continue;
            k[i] = load16<STREAM>(p.kc + ko[i] + ((tid + i * NT) % CPR) * 8);
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int task = tid + i * NT;
            if (VTASKS % NT != 0 && task >= VTASKS) continue;
            const int cg = task / (TILE / 4);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[i][r] = load16<STREAM>(p.vc + vo[i][r] + cg * 8);
        }
    }

    __device__ __forceinline__ void store(uint16_t *buf) const {
        uint16_t *Ks = buf;
        uint16_t *Vt = buf + TILE * KP;
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int task = tid + i * NT;
            if (KTASKS % NT != 0 && task >= KTASKS) continue;
            *reinterpret_cast<u32x4 *>(Ks + (task / CPR) * KP + (task % CPR) * 8) = k[i];
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int task = tid + i * NT;
            if (VTASKS % NT != 0 && task >= VTASKS) continue;
            const int rg = task % (TILE / 4), cg = task / (TILE / 4);
            const u32x4 zero = {0u, 0u, 0u, 0u};
            const u32x4 a = (vok >> (4 * i)) & 1u ? v[i][0] : zero;
            const u32x4 b = (vok >> (4 * i + 1)) & 1u ? v[i][1] : zero;
            const u32x4 c = (vok >> (4 * i + 2)) & 1u ? v[i][2] : zero;
            const u32x4 d = (vok >> (4 * i + 3)) & 1u ? v[i][3] : zero;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                // columns d = 8cg + 2w (low halves) and 8cg + 2w + 1 (high halves)
                u32x2 lo2, hi2;
                lo2.x = __builtin_amdgcn_perm(b[w], a[w], 0x05040100u);
                lo2.y = __builtin_amdgcn_perm(d[w], c[w], 0x05040100u);
                hi2.x = __builtin_amdgcn_perm(b[w], a[w], 0x07060302u);
                hi2.y = __builtin_amdgcn_perm(d[w], c[w], 0x07060302u);
                *reinterpret_cast<u32x2 *>(Vt + (8 * cg + 2 * w) * VP + 4 * rg) = lo2;
                *reinterpret_cast<u32x2 *>(Vt + (8 * cg + 2 * w + 1) * VP + 4 * rg) = hi2;
            }
        }
    }
};

// Block id of the aligned row group (a multiple of 4 rows inside one cache
// block) starting at `row0` (wave-uniform), or 0 past kv_limit.  The block
// table is read-only for the launch: read through the constant address space,
// the wave-uniform entry is always a scalar load, so waiting for it never
// waits for the K/V vector loads in flight (a vector load here would, under
// s_waitcnt vmcnt).
template <int BSM>
__device__ __forceinline__ int uniform_group_page(const FaParams &p, const int *bt_row, int row0,
                                                  int kv_limit) {
    row0 = __builtin_amdgcn_readfirstlane(row0);
    const auto *bt4 = (const __attribute__((address_space(4))) int *)(bt_row);
    return row0 < kv_limit ? bt4[block_of<BSM>(p, row0)] : 0;
}

// Element offset of such a group's first row (page 0 when its id is out of
// range).
template <int D, int BSM>
__device__ __forceinline__ long long uniform_group_base(const FaParams &p, long long head_off,
                                                        int row0, int page) {
    if (page < 0 || page >= p.num_blocks) page = 0;
    return static_cast<long long>(page) * p.page_stride + head_off +
           static_cast<long long>(BSM == 1 ? row0 & (p.bs - 1)
                                            : row0 - block_of<BSM>(p, row0) * p.bs) * D;
}

// Loader for D = 128 and a block_size that is a multiple of 8.  Wave w stages rows
// [w*RW, (w+1)*RW) of the tile.  Each K load instruction covers 4 aligned rows
// (16 lanes x 16 bytes per row) and each V load instruction 8 aligned rows
// (lane l: rows 2*(l%4) + {0,1}, column block l/4), so the cache block
// holding an instruction's rows is the same for the whole wave: its id is a
// scalar, read from the block table one load() call ahead (prefetch), so the
// global loads never wait for it.  K and V are both stored row-major, [TILE]
// [D + 8] and [TILE][D + kVRowPad] (VP = 0, VR = row pitch tells wave_attend
// so): V is not transposed on the way in, the PV product reads it with
// transposing LDS reads.  load() must be
// called for consecutive tiles after one prefetch() of the first.
template <int TILE, int W, int BSM, bool STREAM = false>
struct PagedLoader128 {
    static constexpr int D = 128;
    static constexpr int KP = D + 8;
    static constexpr int VP = 0;
    static constexpr int VR = D + kVRowPad;
    static constexpr int VOFF = TILE * KP;
    static constexpr bool DMA = false;
    static constexpr int STAGES = 2;  // tile buffers in LDS
    static constexpr int ELEMS = TILE * (KP + VR);
    static constexpr int RW = TILE / W;     // rows per wave
    static constexpr int KI = RW / 4;       // K load instructions per wave
    static constexpr int VI = RW / 8;       // V load instruction pairs per wave
    static_assert(RW % 8 == 0, "each wave stages whole 8-row groups");
    u32x4 k[KI];
    u32x4 v[VI][2];
    uint32_t vok;     // bit 2i+j: V row of v[i][j] is below kv_limit
    int pg[KI + VI];  // cache block ids of the next load()'s row groups (uniform)

    static __device__ __forceinline__ int group_page(const FaParams &p, const int *bt_row,
                                                     int row0, int kv_limit) {
        return uniform_group_page<BSM>(p, bt_row, row0, kv_limit);
    }
    static __device__ __forceinline__ long long group_base(const FaParams &p, long long head_off,
                                                           int row0, int page) {
        return uniform_group_base<D, BSM>(p, head_off, row0, page);
    }

    __device__ __forceinline__ void prefetch(const FaParams &p, const int *bt_row, int j0,
                                             int kv_limit) {
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int i = 0; i < KI; ++i) pg[i] = group_page(p, bt_row, j0 + w * RW + 4 * i, kv_limit);
#pragma unroll
        for (int i = 0; i < VI; ++i)
            pg[KI + i] = group_page(p, bt_row, j0 + w * RW + 8 * i, kv_limit);
    }

    __device__ __forceinline__ void load(const FaParams &p, const int *bt_row, long long head_off,
                                         int j0, int kv_limit) {
        const int lane = threadIdx.x & 63;
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int kr = lane >> 4, kc = lane & 15;          // K: row in group of 4, chunk
        const int vr = 2 * (lane & 3), vc = lane >> 2;     // V: row pair, column block
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int row0 = j0 + w * RW + 4 * i;
            const long long base = group_base(p, head_off, row0, pg[i]);
            k[i] = load16<STREAM>(p.kc + base + kr * D + kc * 8);
        }
        // V rows at or past kv_limit are zeroed in store(), not here: a select
        // on the loaded value would make the wave wait for the load at once.
        vok = 0;
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int row0 = j0 + w * RW + 8 * i;
            const long long base = group_base(p, head_off, row0, pg[KI + i]);
            const uint16_t *src = p.vc + base + vr * D + vc * 8;
            v[i][0] = load16<STREAM>(src);
            v[i][1] = load16<STREAM>(src + D);
            vok |= (row0 + vr < kv_limit ? 1u : 0u) << (2 * i);
            vok |= (row0 + vr + 1 < kv_limit ? 1u : 0u) << (2 * i + 1);
        }
        prefetch(p, bt_row, j0 + TILE, kv_limit);
    }

    __device__ __forceinline__ void store(uint16_t *buf) const {
        uint16_t *Ks = buf;
        uint16_t *Vs = buf + TILE * KP;
        const int lane = threadIdx.x & 63;
        const int w = threadIdx.x >> 6;
        const int kr = lane >> 4, kc = lane & 15;
        const int vr = 2 * (lane & 3), vc = lane >> 2;
#pragma unroll
        for (int i = 0; i < KI; ++i)
            *reinterpret_cast<u32x4 *>(Ks + (w * RW + 4 * i + kr) * KP + kc * 8) = k[i];
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int r = w * RW + 8 * i + vr;
            const u32x4 zero = {0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4 *>(Vs + r * VR + vc * 8) = (vok >> (2 * i)) & 1u ? v[i][0] : zero;
            *reinterpret_cast<u32x4 *>(Vs + (r + 1) * VR + vc * 8) =
                (vok >> (2 * i + 1)) & 1u ? v[i][1] : zero;
        }
    }
};

// Bytes of one 4-row block of the prefill's D = 128 DMA tile layout: 4 key
// rows of 256 bytes stored chunk-major (16-byte chunk c of row j at 64c +
// 16j), then a 64-byte pad.  One global_load_lds_dwordx4 fills a block (lane
// l's 16 bytes land at 16l), the 128-bit K reads of 16 consecutive rows and
// the transposing V reads of each half-wave fall on distinct banks, and the
// fragment offsets stay additive (instruction offsets).
constexpr int kLdsBlockBytes = 1088;

// 16 zero bytes: the source of V rows past the end of a sequence.
__device__ __attribute__((aligned(16))) const uint32_t kZero16[4] = {0u, 0u, 0u, 0u};

// HBM -> LDS with no register staging: 16 bytes per lane into
// dst + 16 * lane (dst wave-uniform, in M0).  Inline assembly on purpose:
// through the builtin the compiler treats every transposing LDS read as
// possibly reading the copy's destination and waits for all copies in flight
// before each one, which serialises the next tile's copy with this tile's
// work.  Here the copies are ordered by wait_dma() and the workgroup barrier
// after it.  No other code of these kernels uses M0.
__device__ __forceinline__ void dma16(const void *src, void *dst) {
    const uint32_t lds = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void *)(dst)));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
                 : "memory");
}

// Prefill loader for D = 128 and a block_size that is a multiple of 8: K and
// V go from the paged caches straight into LDS (global_load_lds_dwordx4), in
// the 4-row block layout above, so the tile costs no registers and no LDS
// stores.  Wave w stages rows [w*RW, (w+1)*RW) of the tile, 4 aligned rows
// per instruction (lane l: row l % 4, chunk l / 4), whose cache block is the
// same for the whole wave: its id is a scalar, read from the block table one
// load() ahead.  V rows at or past kv_limit are read from kZero16; K rows
// there are read from some cache row and masked in the softmax.  load()
// issues the copies into a tile buffer, wait_tiles() waits for them (the
// caller's barrier then publishes the tile).
template <int TILE, int W, int BSM>
struct PagedLoaderDma128 {
    static constexpr int D = 128;
    static constexpr bool DMA = true;
    static constexpr int KP = 0, VP = 0, VR = 0;      // the block layout
    static constexpr int VOFF = TILE / 4 * kLdsBlockBytes / 2;  // elements
    static constexpr int ELEMS = 2 * VOFF;
    static constexpr int RW = TILE / W;  // rows per wave
    static constexpr int KI = RW / 4;    // 4-row blocks per wave
    static constexpr int STAGES = 3;     // tile buffers: copies run two tiles ahead
    static constexpr int PER_TILE = 2 * KI;  // copy instructions per tile and lane
    static_assert(RW % 4 == 0, "each wave stages whole 4-row blocks");
    static_assert(PER_TILE < 16, "vmcnt immediate");
    int pg[KI];  // cache block ids of the next load()'s row groups (uniform)

    __device__ __forceinline__ void prefetch(const FaParams &p, const int *bt_row, int j0,
                                             int kv_limit) {
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int i = 0; i < KI; ++i)
            pg[i] = uniform_group_page<BSM>(p, bt_row, j0 + w * RW + 4 * i, kv_limit);
    }

    __device__ __forceinline__ void load(const FaParams &p, const int *bt_row, long long head_off,
                                         int j0, int kv_limit, uint16_t *dst) {
        const int lane = threadIdx.x & 63;
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int r = lane & 3, c = lane >> 2;
        char *kd = reinterpret_cast<char *>(dst) + w * KI * kLdsBlockBytes;
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int row0 = j0 + w * RW + 4 * i;
            const long long off =
                uniform_group_base<D, BSM>(p, head_off, row0, pg[i]) + r * D + c * 8;
            dma16(p.kc + off, kd + i * kLdsBlockBytes);
            dma16(row0 + r < kv_limit ? static_cast<const void *>(p.vc + off)
                                      : static_cast<const void *>(kZero16),
                  kd + 2 * VOFF + i * kLdsBlockBytes);
        }
        prefetch(p, bt_row, j0 + TILE, kv_limit);
    }

    // Waits until this wave has at most NEWER tiles' copies in flight, i.e.
    // the tile issued before them has landed (vector memory counter; no
    // other vector loads are in flight in the tile loop).
    template <int NEWER>
    static __device__ __forceinline__ void wait_tiles() {
        __builtin_amdgcn_s_waitcnt(0x0F70 | (NEWER * PER_TILE));
    }
};

// The same scheme for D = 64: each K load instruction covers 8 aligned rows
// (8 lanes x 16 bytes per row); each V instruction covers two 8-row groups,
// one per half-wave (lane l: rows 8*(l/32) + 2*(l%4) + {0,1}, column block
// (l/4)%8), whose cache blocks are looked up separately, so block sizes of 8
// work too.
template <int TILE, int W, int BSM, bool STREAM = false>
struct PagedLoader64 {
    static constexpr int D = 64;
    static constexpr int KP = D + 8;
    static constexpr int VP = TILE + 4;
    static constexpr int VR = 0;
    static constexpr int VOFF = TILE * KP;  // V region of a tile buffer
    static constexpr bool DMA = false;
    static constexpr int STAGES = 2;  // tile buffers in LDS
    static constexpr int ELEMS = TILE * KP + D * VP;
    static constexpr int RW = TILE / W;     // rows per wave
    static constexpr int KI = RW / 8;       // K load instructions per wave
    static constexpr int VI = RW / 16;      // V load instruction pairs per wave
    static_assert(RW % 16 == 0, "each wave stages whole 16-row groups");
    u32x4 k[KI];
    u32x4 v[VI][2];
    uint32_t vok;            // bit 2i+j: V row of v[i][j] is below kv_limit
    int pg[KI + 2 * VI];     // cache block ids of the next load()'s 8-row groups (uniform)

    __device__ __forceinline__ void prefetch(const FaParams &p, const int *bt_row, int j0,
                                             int kv_limit) {
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int i = 0; i < KI; ++i)
            pg[i] = uniform_group_page<BSM>(p, bt_row, j0 + w * RW + 8 * i, kv_limit);
#pragma unroll
        for (int i = 0; i < 2 * VI; ++i)
            pg[KI + i] = uniform_group_page<BSM>(p, bt_row, j0 + w * RW + 8 * i, kv_limit);
    }

    static __device__ __forceinline__ long long group_base(const FaParams &p, long long head_off,
                                                           int row0, int page) {
        if (page < 0 || page >= p.num_blocks) page = 0;
        return static_cast<long long>(page) * p.page_stride + head_off +
               static_cast<long long>(BSM == 1 ? row0 & (p.bs - 1)
                                                : row0 - block_of<BSM>(p, row0) * p.bs) * D;
    }

    __device__ __forceinline__ void load(const FaParams &p, const int *bt_row, long long head_off,
                                         int j0, int kv_limit) {
        const int lane = threadIdx.x & 63;
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int kr = lane >> 3, kc = lane & 7;                            // K: row of 8, chunk
        const int vb = lane >> 5, vr = 2 * (lane & 3), vc = (lane >> 2) & 7;  // V: group, pair, block
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int row0 = j0 + w * RW + 8 * i;
            k[i] = load16<STREAM>(p.kc + group_base(p, head_off, row0, pg[i]) + kr * D + kc * 8);
        }
        vok = 0;
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int row0 = j0 + w * RW + 16 * i;
            const long long b0 = group_base(p, head_off, row0, pg[KI + 2 * i]);
            const long long b1 = group_base(p, head_off, row0 + 8, pg[KI + 2 * i + 1]);
            const uint16_t *src = p.vc + (vb ? b1 : b0) + vr * D + vc * 8;
            v[i][0] = load16<STREAM>(src);
            v[i][1] = load16<STREAM>(src + D);
            const int r = row0 + 8 * vb + vr;
            vok |= (r < kv_limit ? 1u : 0u) << (2 * i);
            vok |= (r + 1 < kv_limit ? 1u : 0u) << (2 * i + 1);
        }
        prefetch(p, bt_row, j0 + TILE, kv_limit);
    }

    __device__ __forceinline__ void store(uint16_t *buf) const {
        uint16_t *Ks = buf;
        uint16_t *Vt = buf + TILE * KP;
        const int lane = threadIdx.x & 63;
        const int w = threadIdx.x >> 6;
        const int kr = lane >> 3, kc = lane & 7;
        const int vb = lane >> 5, vr = 2 * (lane & 3), vc = (lane >> 2) & 7;
#pragma unroll
        for (int i = 0; i < KI; ++i)
            *reinterpret_cast<u32x4 *>(Ks + (w * RW + 8 * i + kr) * KP + kc * 8) = k[i];
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int r = w * RW + 16 * i + 8 * vb + vr;
            const u32x4 zero = {0u, 0u, 0u, 0u};
            const u32x4 a = (vok >> (2 * i)) & 1u ? v[i][0] : zero;
            const u32x4 b = (vok >> (2 * i + 1)) & 1u ? v[i][1] : zero;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = __builtin_amdgcn_perm(b[e], a[e], 0x05040100u);
                const uint32_t hi = __builtin_amdgcn_perm(b[e], a[e], 0x07060302u);
                *reinterpret_cast<uint32_t *>(Vt + (8 * vc + 2 * e) * VP + r) = lo;
                *reinterpret_cast<uint32_t *>(Vt + (8 * vc + 2 * e + 1) * VP + r) = hi;
            }
        }
    }
};

// The same scheme for D = 96 (12 chunks of 16 bytes per row): a K load
// instruction covers 4 aligned rows on lanes 0-47 and a V instruction 8
// aligned rows (lane l: rows 2*(l%4) + {0,1}, column block l/4) on lanes
// 0-47; lanes 48-63 repeat lane 47's load and store nothing.
template <int TILE, int W, int BSM, bool STREAM = false>
struct PagedLoader96 {
    static constexpr int D = 96;
    static constexpr int KP = D + 8;
    static constexpr int VP = TILE + 4;
    static constexpr int VR = 0;
    static constexpr int VOFF = TILE * KP;  // V region of a tile buffer
    static constexpr bool DMA = false;
    static constexpr int STAGES = 2;  // tile buffers in LDS
    static constexpr int ELEMS = TILE * KP + D * VP;
    static constexpr int RW = TILE / W;     // rows per wave
    static constexpr int KI = RW / 4;       // K load instructions per wave
    static constexpr int VI = RW / 8;       // V load instruction pairs per wave
    static_assert(RW % 8 == 0, "each wave stages whole 8-row groups");
    u32x4 k[KI];
    u32x4 v[VI][2];
    uint32_t vok;     // bit 2i+j: V row of v[i][j] is below kv_limit
    int pg[KI + VI];  // cache block ids of the next load()'s row groups (uniform)

    __device__ __forceinline__ void prefetch(const FaParams &p, const int *bt_row, int j0,
                                             int kv_limit) {
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int i = 0; i < KI; ++i)
            pg[i] = uniform_group_page<BSM>(p, bt_row, j0 + w * RW + 4 * i, kv_limit);
#pragma unroll
        for (int i = 0; i < VI; ++i)
            pg[KI + i] = uniform_group_page<BSM>(p, bt_row, j0 + w * RW + 8 * i, kv_limit);
    }

    static __device__ __forceinline__ long long group_base(const FaParams &p, long long head_off,
                                                           int row0, int page) {
        if (page < 0 || page >= p.num_blocks) page = 0;
        return static_cast<long long>(page) * p.page_stride + head_off +
               static_cast<long long>(BSM == 1 ? row0 & (p.bs - 1)
                                                : row0 - block_of<BSM>(p, row0) * p.bs) * D;
    }

    __device__ __forceinline__ void load(const FaParams &p, const int *bt_row, long long head_off,
                                         int j0, int kv_limit) {
        const int lane = min(static_cast<int>(threadIdx.x & 63), 47);
        const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int kr = lane / 12, kc = lane % 12;          // K: row in group of 4, chunk
        const int vr = 2 * (lane & 3), vc = lane >> 2;     // V: row pair, column block
#pragma unroll
        for (int i = 0; i < KI; ++i) {
            const int row0 = j0 + w * RW + 4 * i;
            k[i] = load16<STREAM>(p.kc + group_base(p, head_off, row0, pg[i]) + kr * D + kc * 8);
        }
        vok = 0;
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int row0 = j0 + w * RW + 8 * i;
            const uint16_t *src = p.vc + group_base(p, head_off, row0, pg[KI + i]) + vr * D + vc * 8;
            v[i][0] = load16<STREAM>(src);
            v[i][1] = load16<STREAM>(src + D);
            vok |= (row0 + vr < kv_limit ? 1u : 0u) << (2 * i);
            vok |= (row0 + vr + 1 < kv_limit ? 1u : 0u) << (2 * i + 1);
        }
        prefetch(p, bt_row, j0 + TILE, kv_limit);
    }

    __device__ __forceinline__ void store(uint16_t *buf) const {
        const int lane = threadIdx.x & 63;
        if (lane >= 48) return;
        uint16_t *Ks = buf;
        uint16_t *Vt = buf + TILE * KP;
        const int w = threadIdx.x >> 6;
        const int kr = lane / 12, kc = lane % 12;
        const int vr = 2 * (lane & 3), vc = lane >> 2;
#pragma unroll
        for (int i = 0; i < KI; ++i)
            *reinterpret_cast<u32x4 *>(Ks + (w * RW + 4 * i + kr) * KP + kc * 8) = k[i];
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int r = w * RW + 8 * i + vr;
            const u32x4 zero = {0u, 0u, 0u, 0u};
            const u32x4 a = (vok >> (2 * i)) & 1u ? v[i][0] : zero;
            const u32x4 b = (vok >> (2 * i + 1)) & 1u ? v[i][1] : zero;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = __builtin_amdgcn_perm(b[e], a[e], 0x05040100u);
                const uint32_t hi = __builtin_amdgcn_perm(b[e], a[e], 0x07060302u);
                *reinterpret_cast<uint32_t *>(Vt + (8 * vc + 2 * e) * VP + r) = lo;
                *reinterpret_cast<uint32_t *>(Vt + (8 * vc + 2 * e + 1) * VP + r) = hi;
            }
        }
    }
};

// Loader choice: the uniform-page loader when it applies, else TileLoader.
// STREAM marks K/V read once per launch (decode): non-temporal loads.
template <int D, int TILE, int W, int BSM, bool STREAM = false>
struct LoaderSel {
    using type = TileLoader<D, TILE, W * 64, BSM, STREAM>;
};
template <int TILE, int W, bool STREAM>
struct LoaderSel<128, TILE, W, 1, STREAM> {
    using type = PagedLoader128<TILE, W, 1, STREAM>;
};
template <int TILE, int W, bool STREAM>
struct LoaderSel<128, TILE, W, 2, STREAM> {
    using type = PagedLoader128<TILE, W, 2, STREAM>;
};
// prefill (K/V re-read from L2 by every query tile): LDS DMA, no registers
template <int TILE, int W>
struct LoaderSel<128, TILE, W, 1, false> {
    using type = PagedLoaderDma128<TILE, W, 1>;
};
template <int TILE, int W>
struct LoaderSel<128, TILE, W, 2, false> {
    using type = PagedLoaderDma128<TILE, W, 2>;
};
template <int TILE, int W, bool STREAM>
struct LoaderSel<64, TILE, W, 1, STREAM> {
    using type = PagedLoader64<TILE, W, 1, STREAM>;
};
template <int TILE, int W, bool STREAM>
struct LoaderSel<64, TILE, W, 2, STREAM> {
    using type = PagedLoader64<TILE, W, 2, STREAM>;
};
template <int TILE, int W, bool STREAM>
struct LoaderSel<96, TILE, W, 1, STREAM> {
    using type = PagedLoader96<TILE, W, 1, STREAM>;
};
template <int TILE, int W, bool STREAM>
struct LoaderSel<96, TILE, W, 2, STREAM> {
    using type = PagedLoader96<TILE, W, 2, STREAM>;
};

template <typename T> struct Ones2;
template <> struct Ones2<bf16> {
    static __device__ __forceinline__ float dot(uint32_t a, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf162_t, a),
                                               __builtin_bit_cast(bf162_t, 0x3f803f80u), c, false);
    }
};
template <> struct Ones2<f16> {
    static __device__ __forceinline__ float dot(uint32_t a, float c) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a),
                                      __builtin_bit_cast(half2_t, 0x3c003c00u), c, false);
    }
};

// ds_read_b64_tr_b16: 8 bytes per lane, transposed within each 16-lane group
// (see the row-major V read in wave_attend).
__device__ __forceinline__ u32x2 tr_b16_b64(const uint16_t *p) {
    typedef short i16x4_t __attribute__((ext_vector_type(4)));
    const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4_t *)(p));
    return __builtin_bit_cast(u32x2, v);
}

// Max of one lane's 16 scores as a tree of three-input maxima (v_max3_f32):
// 8 instructions, 3 deep.
__device__ __forceinline__ float max16(const f32x16_t &s) {
    const auto m3 = [](float a, float b, float c) { return fmaxf(fmaxf(a, b), c); };
    const float a0 = m3(s[0], s[1], s[2]), a1 = m3(s[3], s[4], s[5]), a2 = m3(s[6], s[7], s[8]);
    const float a3 = m3(s[9], s[10], s[11]), a4 = m3(s[12], s[13], s[14]);
    return fmaxf(m3(a0, a1, a2), m3(a3, a4, s[15]));
}

// One wave's online-softmax attention over NKB 32-key blocks staged in LDS at
// rows [kv_row0, kv_row0 + 32*NKB).  Lane l owns query column (l % 32) of each
// of its QSUB column blocks.
//   qf:   Q^T B-operand fragments (8 x 16-bit per lane per 16-dim k-step)
//   oacc: O^T accumulators, element v of block db is d = 32db + 8(v/4) + 4(l/32) + v%4
//   m:    running max (log2 domain, >= 0), lsum: this half-wave's partial sum of P
//   lim:  key r (0-based in the staged rows, r = 32kb + 8(v/4) + 4(l/32) + v%4)
//         is visible when r - 4(l/32) < lim[qs]
template <typename T, int D, int KP, int VP, int VR, int NKB, int QSUB, bool MASK>
__device__ __forceinline__ void wave_attend(const uint16_t *Ks, const uint16_t *Vt, int kv_row0,
                                            const u32x4 (&qf)[QSUB][D / 16],
                                            f32x16_t (&oacc)[QSUB][D / 32], float (&m)[QSUB],
                                            float (&lsum)[QSUB], const int (&lim)[QSUB],
                                            float scale_log2, float inv_scale_log2,
                                            bool mask = MASK) {
    const float slack_raw = kRescaleSlack * inv_scale_log2;
    // row-major V (pitch VR): this lane's element offset for the transposing
    // reads, key 4g + s / 4 and head dim 16 (G % 2) + 4 (s % 4) of a 16-key,
    // 32-dim block (G = lane / 16, s = lane % 16)
    const int vlane = (4 * (threadIdx.x >> 5 & 1) + ((threadIdx.x & 15) >> 2)) * VR +
                      16 * (threadIdx.x >> 4 & 1) + 4 * (threadIdx.x & 3);
    const int lane = threadIdx.x & 63;
    const int g = lane >> 5, r32 = lane & 31;
    // the 4-row block layout (KP == 0), byte offsets of this lane: K row r32,
    // chunk g; V (transposing reads as above) key 4g + s / 4, head dims 16 (G
    // % 2) + 4 (s % 4) .. +3
    const int kblane = (r32 >> 2) * kLdsBlockBytes + 16 * (r32 & 3) + 64 * g;
    const int vblane = g * kLdsBlockBytes + 16 * ((lane & 15) >> 2) + 128 * (lane >> 4 & 1) +
                       64 * (lane >> 1 & 1) + 8 * (lane & 1);
    const char *Kb = reinterpret_cast<const char *>(Ks) + (kv_row0 >> 2) * kLdsBlockBytes;
    const char *Vb = reinterpret_cast<const char *>(Vt) + (kv_row0 >> 2) * kLdsBlockBytes;
    f32x16_t s[NKB][QSUB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int qs = 0; qs < QSUB; ++qs)
#pragma unroll
            for (int v = 0; v < 16; ++v) s[kb][qs][v] = 0.0f;
    // Issue priority by phase: the QK product highest, the PV product next,
    // the softmax lowest, so that when waves of a SIMD compete the ones with
    // matrix work issue first and the softmax fills the matrix core's gaps
    // (BASELINE prefill 513 -> 493 us; the same three levels with the softmax
    // at the PV level: 512, QK and PV equal: 505, PV raised alone: 502,
    // softmax raised: 532 us).
    __builtin_amdgcn_s_setprio(2);
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            const u32x4 a =
                KP == 0 ? *reinterpret_cast<const u32x4 *>(Kb + kblane + 8 * kb * kLdsBlockBytes +
                                                           128 * ks)
                        : *reinterpret_cast<const u32x4 *>(
                              Ks + (kv_row0 + 32 * kb + r32) * KP + 16 * ks + 8 * g);
#pragma unroll
            for (int qs = 0; qs < QSUB; ++qs) s[kb][qs] = Mma<T>::run(a, qf[qs][ks], s[kb][qs]);
        }
    }
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int qs = 0; qs < QSUB; ++qs) {
        // masked scores, then their max as a tree (short dependency chain)
        if (MASK && mask) {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    float x = s[kb][qs][v];
                    if (!(32 * kb + 8 * (v >> 2) + (v & 3) < lim[qs])) x = kNegInf;
                    s[kb][qs][v] = x;
                }
        }
        // The rescale test runs on this half-wave's raw scores: every lane's
        // max of its 16 keys is within the slack exactly when every query
        // column's max over all 32 keys is, so the exchange with the other
        // half-wave and the scaling are only needed when the max is raised.
        // (The test's rounding can differ from that of the scaled max by an
        // ulp; either outcome is exact, see kRescaleSlack.)
        float mx = max16(s[0][qs]);
#pragma unroll
        for (int kb = 1; kb < NKB; ++kb) mx = fmaxf(mx, max16(s[kb][qs]));
        if (!__all(mx <= fmaf(m[qs], inv_scale_log2, slack_raw))) {
            mx = half_swap_max(mx) * scale_log2;
            const float m_new = fmaxf(m[qs], mx);  // m >= 0 keeps the reference clamp
            const float alpha = __builtin_amdgcn_exp2f(m[qs] - m_new);
            m[qs] = m_new;
            lsum[qs] *= alpha;
#pragma unroll
            for (int db = 0; db < D / 32; ++db)
#pragma unroll
                for (int v = 0; v < 16; ++v) oacc[qs][db][v] *= alpha;
        }
        const float mneg = -m[qs];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int v = 0; v < 16; ++v)
                s[kb][qs][v] = __builtin_amdgcn_exp2f(fmaf(s[kb][qs][v], scale_log2, mneg));
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int t = 0; t < 2 * NKB; ++t) {
        const int kb = t >> 1, o = 8 * (t & 1);
        u32x4 pf[QSUB];
#pragma unroll
        for (int qs = 0; qs < QSUB; ++qs) {
            pf[qs].x = Mma<T>::pack2(s[kb][qs][o + 0], s[kb][qs][o + 1]);
            pf[qs].y = Mma<T>::pack2(s[kb][qs][o + 2], s[kb][qs][o + 3]);
            pf[qs].z = Mma<T>::pack2(s[kb][qs][o + 4], s[kb][qs][o + 5]);
            pf[qs].w = Mma<T>::pack2(s[kb][qs][o + 6], s[kb][qs][o + 7]);
            float l = lsum[qs];
            l = Ones2<T>::dot(pf[qs].x, l);
            l = Ones2<T>::dot(pf[qs].y, l);
            l = Ones2<T>::dot(pf[qs].z, l);
            l = Ones2<T>::dot(pf[qs].w, l);
            lsum[qs] = l;
        }
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
            u32x4 a;
            if constexpr (KP == 0) {
                const char *vb = Vb + vblane + 4 * t * kLdsBlockBytes + 256 * db;
                const u32x2 lo2 = tr_b16_b64(reinterpret_cast<const uint16_t *>(vb));
                const u32x2 hi2 =
                    tr_b16_b64(reinterpret_cast<const uint16_t *>(vb + 2 * kLdsBlockBytes));
                a = u32x4{lo2.x, lo2.y, hi2.x, hi2.y};
            } else if constexpr (VR > 0) {
                // V row-major [key][VR]: each 16-lane group of a
                // ds_read_b64_tr_b16 hands lane i value i % 4 of the group's
                // lanes i / 4 + {0, 4, 8, 12}; lane s points at key s / 4 and
                // head dims 4 (s % 4) .. +3 of its group's 16, so lane i gets
                // head dim d0 + i of 4 consecutive keys (the A operand's k
                // order of the V^T layout below)
                const uint16_t *vb = Vt + (kv_row0 + 16 * t) * VR + 32 * db + vlane;
                const u32x2 lo2 = tr_b16_b64(vb);
                const u32x2 hi2 = tr_b16_b64(vb + 8 * VR);
                a = u32x4{lo2.x, lo2.y, hi2.x, hi2.y};
            } else {
                const uint16_t *vr = Vt + (32 * db + r32) * VP + kv_row0 + 16 * t + 4 * g;
                const u32x2 lo2 = *reinterpret_cast<const u32x2 *>(vr);
                const u32x2 hi2 = *reinterpret_cast<const u32x2 *>(vr + 8);
                a = u32x4{lo2.x, lo2.y, hi2.x, hi2.y};
            }
#pragma unroll
            for (int qs = 0; qs < QSUB; ++qs) oacc[qs][db] = Mma<T>::run(a, pf[qs], oacc[qs][db]);
        }
    }
}

template <typename T>
__device__ __forceinline__ void store_row4(uint16_t *dst, float a, float b, float c, float d) {
    uint2 w;
    w.x = Mma<T>::pack2(a, b);
    w.y = Mma<T>::pack2(c, d);
    *reinterpret_cast<uint2 *>(dst) = w;
}

// ---------------------------------------------------------------- prefill

// Elements of one staged K/V tile of TILE keys: K [TILE][D + 8] and V either
// transposed [D][TILE + 4] or row-major [TILE][D + kVRowPad], whichever the
// loader uses (the larger of the two).
template <int D, int TILE>
constexpr size_t kv_tile_elems() {
    constexpr size_t vt = static_cast<size_t>(D) * (TILE + 4),
                     vr = static_cast<size_t>(TILE) * (D + kVRowPad);
    return static_cast<size_t>(TILE) * (D + 8) + (vt > vr ? vt : vr);
}

// Padded LDS row of the staged O rows of a prefill workgroup (HW heads x D
// values): the pad spreads the 8-byte fragment writes of consecutive rows
// over the banks.
template <int D, int HW>
constexpr int o_row() {
    return HW * D + 8;
}

// LDS of a prefill workgroup: the loader's K/V tile buffers, which the
// staged O rows ([32*QSUB*(W/HW)][o_row]) reuse at the end of the tile.
template <int D, int TILE, int W, int HW, int QSUB, int BSM>
constexpr size_t prefill_lds_bytes() {
    using Loader = typename LoaderSel<D, TILE, W, BSM>::type;
    constexpr size_t kv = static_cast<size_t>(Loader::STAGES) * Loader::ELEMS;
    constexpr size_t o = static_cast<size_t>(32 * QSUB * (W / HW)) * o_row<D, HW>();
    return sizeof(uint16_t) * (kv > o ? kv : o);
}

// One query tile [q0, q0 + QT) of workgroup (b, kv head kvh, head group hg):
// the body of fa_prefill_kernel.  Ends with a barrier, so the LDS tile
// buffers can be refilled by the next call.
template <typename T, int D, int W, int HW, int QSUB, int BSM, int TILE>
__device__ __forceinline__ void prefill_tile(const FaParams &p, uint16_t *lds, int b, int kvh,
                                             int hg, long long q_off, int L, int S, int q0) {
    constexpr int NKB = TILE % 64 == 0 ? 2 : 1;
    constexpr int KB = 32 * NKB;
    using Loader = typename LoaderSel<D, TILE, W, BSM>::type;
    constexpr int KP = Loader::KP, VP = Loader::VP, VR = Loader::VR;
    constexpr int WROWS = 32 * QSUB;
    constexpr int QT = WROWS * (W / HW);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 5, r32 = lane & 31;
    const int h = kvh * p.G + hg * HW + (wave % HW);
    const int qw0 = q0 + (wave / HW) * WROWS;
    const int q_start = p.causal ? max(S - L, 0) : 0;
    const int kv_end = p.causal ? min(S, q_start + min(q0 + QT, L)) : S;
    const int wave_kv_end =
        __builtin_amdgcn_readfirstlane(p.causal ? min(S, q_start + min(qw0 + WROWS, L)) : S);
    const int wave_min_vis = __builtin_amdgcn_readfirstlane(p.causal ? min(S, q_start + qw0 + 1) : S);
    const int *bt_row = p.bt + b * p.bt_stride;
    const long long head_off = static_cast<long long>(kvh) * p.bs * D;

    u32x4 qf[QSUB][D / 16];
    int vis[QSUB];
#pragma unroll
    for (int qs = 0; qs < QSUB; ++qs) {
        const int row = qw0 + 32 * qs + r32;
        const uint16_t *src = p.q + ((q_off + min(row, L - 1)) * p.H + h) * D;
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
            const u32x4 x = *reinterpret_cast<const u32x4 *>(src + 16 * ks + 8 * g);
            const u32x4 zero = {0u, 0u, 0u, 0u};
            qf[qs][ks] = row < L ? x : zero;
        }
        vis[qs] = p.causal ? min(S, q_start + row + 1) : S;
    }

    float m[QSUB], lsum[QSUB];
    f32x16_t oacc[QSUB][D / 32];
#pragma unroll
    for (int qs = 0; qs < QSUB; ++qs) {
        m[qs] = 0.0f;
        lsum[qs] = 0.0f;
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
            for (int v = 0; v < 16; ++v) oacc[qs][db][v] = 0.0f;
    }

    Loader ld;
    const int ntiles = (kv_end + TILE - 1) / TILE;
    // Tile t lives in LDS buffer t % NS.  A DMA loader copies straight into
    // the buffer (NS = 3: tile t + 2 is copied while tile t is attended), the
    // others stage tile t + 1 in registers and store it after tile t (NS = 2).
    constexpr int NS = Loader::STAGES;
    // (the offset goes through readfirstlane so that it stays one scalar:
    // otherwise the compiler precomputes lane addresses for every buffer)
    auto buf = [&](int t) { return lds + __builtin_amdgcn_readfirstlane((t % NS) * Loader::ELEMS); };
    auto load = [&](int t) {
        if constexpr (Loader::DMA)
            ld.load(p, bt_row, head_off, t * TILE, S, buf(t));
        else
            ld.load(p, bt_row, head_off, t * TILE, S);
    };
    // tile t is in LDS for this wave (the barrier after it publishes it)
    auto land = [&](int t) {
        if constexpr (Loader::DMA) {
            if (NS > 2 && t + 1 < ntiles)
                Loader::template wait_tiles<1>();
            else
                Loader::template wait_tiles<0>();
        } else {
            ld.store(buf(t));
        }
    };
    if (ntiles > 0) {
        ld.prefetch(p, bt_row, 0, S);
        load(0);
        if constexpr (NS > 2)
            if (ntiles > 1) load(1);
        land(0);
    }
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
        const uint16_t *cur = buf(it);
        if (it + NS - 1 < ntiles) load(it + NS - 1);
#pragma unroll
        for (int hb = 0; hb < TILE / KB; ++hb) {
            const int j0 = it * TILE + KB * hb;
            if (j0 < wave_kv_end) {
                int lim[QSUB];
#pragma unroll
                for (int qs = 0; qs < QSUB; ++qs) lim[qs] = vis[qs] - j0 - 4 * g;
                // one copy of the block code; the mask is a uniform branch
                wave_attend<T, D, KP, VP, VR, NKB, QSUB, true>(cur, cur + Loader::VOFF, KB * hb, qf, oacc, m,
                                                           lsum, lim, p.scale_log2,
                                                           p.inv_scale_log2, j0 + KB > wave_min_vis);
            }
        }
        if (it + 1 < ntiles) land(it + 1);
        __syncthreads();
    }

    // O leaves through LDS, a row (HW heads x D values) at a time, 16 bytes
    // per lane: the O^T fragments would be stored 8 bytes per lane over 32
    // rows per instruction (prefill B = 64 x 256 rows: 155 -> 108 us, the
    // BASELINE prefill 1.5 % faster).  The tile loop ended with a barrier, so
    // the K/V buffers are free.
    constexpr int OROW = o_row<D, HW>();
    constexpr int RCH = HW * D / 8;  // 16-byte chunks per row
    constexpr int NOC = (QT * RCH + W * 64 - 1) / (W * 64);
    static_assert(NS * Loader::ELEMS * sizeof(uint16_t) <= prefill_lds_bytes<D, TILE, W, HW, QSUB, BSM>() &&
                      QT * OROW * sizeof(uint16_t) <= prefill_lds_bytes<D, TILE, W, HW, QSUB, BSM>(),
                  "K/V tiles and staged O rows fit the workgroup's LDS");
#pragma unroll
    for (int qs = 0; qs < QSUB; ++qs) {
        const float lt = half_swap_sum(lsum[qs]);
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        uint16_t *dst = lds + ((wave / HW) * WROWS + 32 * qs + r32) * OROW + (wave % HW) * D;
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                store_row4<T>(dst + 32 * db + 8 * u + 4 * g, oacc[qs][db][4 * u] * inv,
                              oacc[qs][db][4 * u + 1] * inv, oacc[qs][db][4 * u + 2] * inv,
                              oacc[qs][db][4 * u + 3] * inv);
    }
    __syncthreads();
    uint16_t *o_rows = p.o + (q_off * p.H + kvh * p.G + hg * HW) * D;
#pragma unroll
    for (int j = 0; j < NOC; ++j) {
        const int c = static_cast<int>(threadIdx.x) + j * W * 64;
        const int rr = c / RCH;
        if (c < QT * RCH && q0 + rr < L)
            *reinterpret_cast<u32x4 *>(o_rows + static_cast<long long>(q0 + rr) * p.H * D +
                                       (c - rr * RCH) * 8) =
                *reinterpret_cast<const u32x4 *>(lds + rr * OROW + (c - rr * RCH) * 8);
    }
    __syncthreads();  // the next tile of the same workgroup refills the LDS
}

// A kernel's FaParams argument where it lies, at the start of the kernel
// argument segment (constant address space): read through this pointer a
// callee gets the fields with scalar loads, and no copy of the argument is
// made on the stack.
// (The host pass only parses device code, and its target has no such
// address space.)
#if defined(__HIP_DEVICE_COMPILE__)
typedef const __attribute__((address_space(4))) FaParams KernargParams;
#else
typedef const FaParams KernargParams;
#endif

// The query tiles of (b, kv head kvh, head group hg) from first_tile on, in
// turn.  Not inlined: it runs only when max_seqlen_q understates a q length,
// and its loop keeps values live across tiles that would otherwise push the
// kernel's single-tile path past its register budget.
template <typename T, int D, int W, int HW, int QSUB, int BSM, int TILE>
__device__ __attribute__((noinline)) void prefill_rest(const KernargParams *pp, int b, int kvh,
                                                       int hg, int first_tile) {
    constexpr int QT = 32 * QSUB * (W / HW);
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    const FaParams p = *pp;
    long long q_off;
    int L;
    seq_info(p, b, q_off, L);
    const int S = kv_len(p, b);
    for (int t = first_tile; t * QT < L; ++t)
        prefill_tile<T, D, W, HW, QSUB, BSM, TILE>(p, lds, b, kvh, hg, q_off, L, S, t * QT);
}

// Workgroup (b, kv head, head group, query tile) with W waves: wave w serves
// query head hg*HW + w % HW of the GQA group and query rows
// [q0 + (w / HW) * 32*QSUB, +32*QSUB).  K/V tiles of TILE keys rotate through
// the loader's LDS buffers (three for the HBM -> LDS copy, two for register
// staging; one barrier per tile) and are attended 32 * NKB keys at a time.
// W >= 12 asks for 3 waves per SIMD (168 VGPRs); head sizes above 128 with 4
// waves one (their 4-wave tiles fill the registers), else 2.
//
// The grid's tile rows are sized from max_seqlen_q, a bound the reference
// never reads (flash_attention.cpp:98-99).  The workgroup of tile 0, which
// is dispatched last, then takes every query tile past the grid in turn;
// with a bound that holds there is none.  A prefill is one launch whatever
// the bound.
template <typename T, int D, int W, int HW, int QSUB, int BSM, int TILE>
__global__ void __launch_bounds__(W * 64, (W >= 12 || TILE == 32) ? 3 : (D > 128 && W < 8 ? 1 : 2))
fa_prefill_kernel(FaParams p) {
    constexpr int QT = 32 * QSUB * (W / HW);
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    if (blockIdx.x == 0 && blockIdx.y == 0) zero_tail_rows(p, D);
    const int ngroups = p.G / HW;
    const int hg = blockIdx.x % ngroups;
    const int kvh = (blockIdx.x / ngroups) % p.Hkv;
    const int b = blockIdx.x / ngroups / p.Hkv;
    const int rows = gridDim.y;  // tile rows sized from max_seqlen_q
    long long q_off;
    int L;
    seq_info(p, b, q_off, L);
    const int S = kv_len(p, b);
    const int tile = rows - 1 - blockIdx.y;  // heaviest causal tiles first
    if (tile * QT < L)
        prefill_tile<T, D, W, HW, QSUB, BSM, TILE>(p, lds, b, kvh, hg, q_off, L, S, tile * QT);
    if (tile == 0 && rows * QT < L)
        prefill_rest<T, D, W, HW, QSUB, BSM, TILE>(
            (const KernargParams *)(__builtin_amdgcn_kernarg_segment_ptr()), b, kvh, hg, rows);
}

// ----------------------------------------------------------------- decode

constexpr int kDecTile = 128;

template <int D>
constexpr size_t decode_lds_bytes() {
    return sizeof(uint16_t) * kv_tile_elems<D, kDecTile>();
}

// The 4 waves of a decode workgroup attend keys [kv_lo, kv_hi) of (sequence
// b, kv head kvh) for the query rows [r0, r0 + rq): column c of the MFMA tile
// is (head c / rq, row r0 + c % rq) of the GQA group and wave w takes keys
// [32w, 32w + 32) of each 128-key tile.  Leaves each wave's partial state in
// LDS, after a barrier: max lm[4][32], sum ll[4][32] and unnormalised O
// lo[4][32][D] (fp32, over the tile buffers).
template <typename T, int D, int BSM>
__device__ __forceinline__ void decode_pass(const FaParams &p, uint16_t *smem, int b, int kvh,
                                            long long q_off, int L, int S, int kv_lo, int kv_hi,
                                            int rq, int r0) {
    using Loader = typename LoaderSel<D, kDecTile, 4, BSM, true>::type;
    constexpr int KP = Loader::KP, VP = Loader::VP, VR = Loader::VR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 5, r32 = lane & 31;
    const int hl = r32 / rq, row = r0 + r32 % rq;
    const bool col_ok = hl < p.G && row < L;
    const int h = kvh * p.G + min(hl, p.G - 1);
    const int q_start = p.causal ? max(S - L, 0) : 0;
    const int *bt_row = p.bt + b * p.bt_stride;
    const long long head_off = static_cast<long long>(kvh) * p.bs * D;

    u32x4 qf[1][D / 16];
    {
        const uint16_t *src = p.q + ((q_off + min(row, L - 1)) * p.H + h) * D;
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
            const u32x4 x = *reinterpret_cast<const u32x4 *>(src + 16 * ks + 8 * g);
            const u32x4 zero = {0u, 0u, 0u, 0u};
            qf[0][ks] = col_ok ? x : zero;
        }
    }
    // keys visible to this column, and to the pass's first row (the fewest)
    const int vis = min(kv_hi, p.causal ? q_start + row + 1 : S);
    const int min_vis = min(kv_hi, p.causal ? q_start + r0 + 1 : S);

    float m[1] = {0.0f}, lsum[1] = {0.0f};
    f32x16_t oacc[1][D / 32];
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) oacc[0][db][v] = 0.0f;

    Loader ld;
    const int ntiles = (kv_hi - kv_lo + kDecTile - 1) / kDecTile;
    if (ntiles > 0) {
        ld.prefetch(p, bt_row, kv_lo, kv_hi);
        ld.load(p, bt_row, head_off, kv_lo, kv_hi);
    }
    for (int it = 0; it < ntiles; ++it) {
        const int j0 = kv_lo + it * kDecTile;
        __syncthreads();
        ld.store(smem);
        __syncthreads();
        if (it + 1 < ntiles) ld.load(p, bt_row, head_off, j0 + kDecTile, kv_hi);
        const int jw = j0 + 32 * wave;
        if (jw < kv_hi) {
            const int lim[1] = {vis - jw - 4 * g};
            if (jw + 32 > min_vis)
                wave_attend<T, D, KP, VP, VR, 1, 1, true>(smem, smem + Loader::VOFF, 32 * wave, qf,
                                                      oacc, m, lsum, lim, p.scale_log2,
                                                      p.inv_scale_log2);
            else
                wave_attend<T, D, KP, VP, VR, 1, 1, false>(smem, smem + Loader::VOFF, 32 * wave, qf,
                                                       oacc, m, lsum, lim, p.scale_log2,
                                                       p.inv_scale_log2);
        }
    }

    __syncthreads();
    float *lm = reinterpret_cast<float *>(smem);   // [4][32] max
    float *ll = lm + 4 * 32;                        // [4][32] sum
    float *lo = ll + 4 * 32;                        // [4][32][D] unnormalised O
    const float lt = half_swap_sum(lsum[0]);
    if (g == 0) {
        lm[wave * 32 + r32] = m[0];
        ll[wave * 32 + r32] = lt;
    }
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int d = 32 * db + 8 * (v >> 2) + 4 * g + (v & 3);
            lo[(wave * 32 + r32) * D + d] = oacc[0][db][v];
        }
    __syncthreads();
}

// Merges the 4 waves' partial states that decode_pass left in LDS, one thread
// per (column, d) of the first ncols columns: sink(c, d, O, m, l) receives the
// column's merged unnormalised O[d], max and sum.
template <int D, typename Sink>
__device__ __forceinline__ void merge_waves(const uint16_t *smem, int ncols, Sink sink) {
    const float *lm = reinterpret_cast<const float *>(smem);
    const float *ll = lm + 4 * 32;
    const float *lo = ll + 4 * 32;
    for (int task = threadIdx.x; task < ncols * D; task += blockDim.x) {
        const int c = task / D, d = task % D;
        float M = lm[c];
#pragma unroll
        for (int w = 1; w < 4; ++w) M = fmaxf(M, lm[w * 32 + c]);
        float acc = 0.0f, lsum_all = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = __builtin_amdgcn_exp2f(lm[w * 32 + c] - M);
            acc += f * lo[(w * 32 + c) * D + d];
            lsum_all += f * ll[w * 32 + c];
        }
        sink(c, d, acc, M, lsum_all);
    }
}

// Workgroup (b, kv head, split): keys [split*split_len, +split_len), the last
// split also every key past the splits (the host sizes the splits from
// max_seqlen_k, which the reference never reads).  Its rows' partial (m, l, O)
// go to the workspace for fa_decode_combine_kernel.
//
// The host routes to this kernel when G * max_seqlen_q <= 32 and lays the
// columns out for rq = max_seqlen_q rows.  A sequence with more rows than
// that is attended here in full by its split-0 workgroup instead, 32 / G rows
// per pass over all its keys, which writes its output rows itself; the
// combine kernel leaves it alone.  So the output never depends on the host's
// bounds, only the speed does.
// q length of sequence b.
__device__ __forceinline__ int q_len_of(const FaParams &p, int b) {
    return p.q_lens != nullptr ? p.q_lens[b] : p.cu_q[b + 1] - p.cu_q[b];
}

// Split-KV work items of a sequence with q length L and kv length S: every
// split but the last is split_len keys long; the last holds the rest (up to
// the end of the sequence).  A sequence whose q length exceeds the decode
// bound rq, or that has no keys, is one item.
__device__ __forceinline__ int decode_items(const FaParams &p, int L, int S) {
    if (L <= 0 || L > p.rq || S <= 0) return 1;
    return min((S + p.split_len - 1) / p.split_len, p.max_splits);
}

// Keys of the last item, scaled by its query passes (q lengths past rq take
// several) and capped at INT_MAX; -1 for a sequence with no queries (nothing
// to do).
__device__ __forceinline__ int decode_last_work(const FaParams &p, int L, int S) {
    if (L <= 0) return -1;
    if (L > p.rq) {
        const long long w = static_cast<long long>(S) * ((L + 32 / p.G - 1) / (32 / p.G));
        return static_cast<int>(min(w, 0x7fffffffLL));
    }
    return S - (decode_items(p, L, S) - 1) * p.split_len;
}

// Workgroup i's work item in longest-first order, for batches of up to 64
// sequences: first the full split_len items of every sequence (all the same
// size), then each (sequence, kv head) last item, longest first (ties by
// sequence).  Without the ordering the full splits of long sequences are
// dispatched last and run in the tail (equal lengths with the same total keys
// took 183 us against 201 us for lengths spread over 512..8192).  Lane t of
// wave 0 reads sequence t's lengths and leaves the choice in LDS; returns
// false for workgroups past the last item.
__device__ bool decode_item(const FaParams &p, int i, int &b, int &kvh, int &split,
                            long long &q_off, int &L, int &S) {
    __shared__ long long pick_off;
    __shared__ int pick[4];  // sequence, item code, q length, kv length
    if (threadIdx.x < 64) {
        const int t = threadIdx.x;
        if (t == 0) pick[0] = -1;
        int f = 0, w = -2, Lt = 0, St = 0;  // lanes past the batch: w = -2
        long long ot = 0;
        if (t < p.batch) {
            Lt = q_len_of(p, t);
            St = kv_len(p, t);
            if (p.q_lens == nullptr) ot = p.cu_q[t];
            f = (decode_items(p, Lt, St) - 1) * p.Hkv;  // full items
            w = decode_last_work(p, Lt, St);
        }
        int x = f;  // inclusive prefix of the full items
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int v = __shfl_up(x, d, 64);
            if (t >= d) x += v;
        }
        if (p.q_lens != nullptr) {  // q offsets: exclusive prefix of the q lengths
            long long xq = Lt;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const long long vq = __shfl_up(xq, d, 64);
                if (t >= d) xq += vq;
            }
            ot = xq - Lt;
        }
        const int pre = x - f;
        if (t < p.batch && i >= pre && i < pre + f) {
            pick[0] = t;
            pick[1] = i - pre;
            pick[2] = Lt;
            pick[3] = St;
            pick_off = ot;
        }
        const int j = i - __shfl(x, 63, 64);
        if (j >= 0 && j < p.batch * p.Hkv) {
            // last items, longest first: the rank of sequence t, from scalar
            // broadcasts (v_readlane) of every lane's work; a batch whose
            // last items are all the same size keeps sequence order
            const int rank = j / p.Hkv;
            int r = 0;
            if (__all(t >= p.batch || w == __builtin_amdgcn_readfirstlane(w))) {
                r = t;
            } else {
#pragma unroll
                for (int v = 0; v < 64; ++v) {
                    const int wu = __builtin_amdgcn_readlane(w, v);
                    r += (wu > w || (wu == w && v < t)) ? 1 : 0;
                }
            }
            if (t < p.batch && r == rank) {
                pick[0] = t;
                pick[1] = -1 - (j % p.Hkv);
                pick[2] = Lt;
                pick[3] = St;
                pick_off = ot;
            }
        }
    }
    __syncthreads();
    b = pick[0];
    if (b < 0) return false;
    const int r = pick[1];
    L = pick[2];
    S = pick[3];
    q_off = pick_off;
    if (r >= 0) {
        kvh = r % p.Hkv;
        split = r / p.Hkv;
    } else {
        kvh = -1 - r;
        split = decode_items(p, L, S) - 1;
    }
    return true;
}

template <typename T, int D, int BSM>
__global__ void __launch_bounds__(256, D > 128 ? 1 : 2) fa_decode_kernel(FaParams p) {
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    if (blockIdx.x == 0 && blockIdx.y == 0) zero_tail_rows(p, D);
    int b, kvh, split, L, S;
    long long q_off;
    if (p.batch <= 64) {
        if (!decode_item(p, blockIdx.y * gridDim.x + blockIdx.x, b, kvh, split, q_off, L, S))
            return;
    } else {
        // Larger batches keep the grid's order, (sequence, kv head) by split:
        // with hundreds of items per CU the tail is short, and a scan over
        // every sequence in each workgroup would cost more than it saves.
        b = blockIdx.x / p.Hkv;
        kvh = blockIdx.x % p.Hkv;
        split = blockIdx.y;
        seq_info(p, b, q_off, L);
        S = kv_len(p, b);
        if (split >= decode_items(p, L, S)) return;
    }
    if (L <= 0) return;
    if (L > p.rq) {
        if (split != 0) return;
        const int rq = 32 / p.G;
        for (int r0 = 0; r0 < L; r0 += rq) {
            decode_pass<T, D, BSM>(p, smem, b, kvh, q_off, L, S, 0, S, rq, r0);
            merge_waves<D>(smem, p.G * rq, [&](int c, int d, float acc, float, float l) {
                const int hl = c / rq, row = r0 + c % rq;
                if (row >= L) return;
                const int h = kvh * p.G + hl;
                p.o[((q_off + row) * p.H + h) * D + d] = Cvt<T>::from(l > 0.0f ? acc / l : 0.0f);
            });
            __syncthreads();  // the next pass refills the LDS
        }
        return;
    }
    const int kv_lo = split * p.split_len;
    const int kv_hi = split == decode_items(p, L, S) - 1 ? S : min(S, kv_lo + p.split_len);
    decode_pass<T, D, BSM>(p, smem, b, kvh, q_off, L, S, kv_lo, kv_hi, p.rq, 0);
    if (p.max_splits == 1) {
        // one split per sequence: the rows are final here, normalised with
        // the merge kernel's arithmetic (the reciprocal of l, then a product),
        // and no merge kernel runs
        merge_waves<D>(smem, p.ncols, [&](int c, int d, float acc, float, float l) {
            const int hl = c / p.rq, row = c % p.rq;
            if (hl >= p.G || row >= L) return;
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            p.o[((q_off + row) * p.H + kvh * p.G + hl) * D + d] = Cvt<T>::from(inv * acc);
        });
        return;
    }
    const long long base = ((static_cast<long long>(b) * p.Hkv + kvh) * p.max_splits + split) *
                           p.ncols;
    merge_waves<D>(smem, p.ncols, [&](int c, int d, float acc, float M, float l) {
        p.ws_o[(base + c) * D + d] = acc;
        if (d == 0) {
            p.ws_ml[(base + c) * 2] = M;
            p.ws_ml[(base + c) * 2 + 1] = l;
        }
    });
}

// Merges the split partials of (b, kv head) into the output rows.  The
// splits' (m, l) are staged in LDS once, one thread per column turns them into
// normalised weights, and each output element then sums its splits' partial
// O with independent loads.  Split counts beyond the LDS staging capacity
// take a two-pass loop over global memory instead.
constexpr int kCombineStage = 2048;  // (split, column) pairs staged in LDS

template <typename T, int D>
__global__ void __launch_bounds__(256) fa_decode_combine_kernel(FaParams p) {
    __shared__ float wgt[kCombineStage];  // [split][column]: m, then weight / total l
    __shared__ float lsp[kCombineStage];  // [split][column]: l
    const int kvh = blockIdx.x % p.Hkv;
    const int b = blockIdx.x / p.Hkv;
    long long q_off;
    int L;
    seq_info(p, b, q_off, L);
    if (L <= 0 || L > p.rq) return;  // L > rq: written by fa_decode_kernel
    const int S = kv_len(p, b);
    int nsplit = S <= 0 ? 1 : (S + p.split_len - 1) / p.split_len;
    nsplit = min(nsplit, p.max_splits);
    const long long base = (static_cast<long long>(b) * p.Hkv + kvh) * p.max_splits;
    const int nc = p.ncols;
    if (nsplit * nc <= kCombineStage) {
        // all (m, l) pairs in one round of parallel loads
        for (int i = threadIdx.x; i < nsplit * nc; i += blockDim.x) {
            const float2 ml = *reinterpret_cast<const float2 *>(p.ws_ml + (base * nc + i) * 2);
            wgt[i] = ml.x;
            lsp[i] = ml.y;
        }
        __syncthreads();
        for (int c = threadIdx.x; c < nc; c += blockDim.x) {
            float M = 0.0f;
            for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, wgt[sp * nc + c]);
            float l = 0.0f;
            for (int sp = 0; sp < nsplit; ++sp) {
                const float f = __builtin_amdgcn_exp2f(wgt[sp * nc + c] - M);
                wgt[sp * nc + c] = f;
                l += f * lsp[sp * nc + c];
            }
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            for (int sp = 0; sp < nsplit; ++sp) wgt[sp * nc + c] *= inv;
        }
        __syncthreads();
        for (int task = threadIdx.x; task < nc * D; task += blockDim.x) {
            const int c = task / D, d = task % D;
            const int hl = c / p.rq, row = c % p.rq;
            if (hl >= p.G || row >= L) continue;
            const float *src = p.ws_o + (base * nc + c) * D + d;
            const long long step = static_cast<long long>(nc) * D;
            float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f;
            int sp = 0;
            for (; sp + 4 <= nsplit; sp += 4) {
                acc0 += wgt[sp * nc + c] * src[sp * step];
                acc1 += wgt[(sp + 1) * nc + c] * src[(sp + 1) * step];
                acc2 += wgt[(sp + 2) * nc + c] * src[(sp + 2) * step];
                acc3 += wgt[(sp + 3) * nc + c] * src[(sp + 3) * step];
            }
            for (; sp < nsplit; ++sp) acc0 += wgt[sp * nc + c] * src[sp * step];
            const int h = kvh * p.G + hl;
            p.o[((q_off + row) * p.H + h) * D + d] = Cvt<T>::from((acc0 + acc1) + (acc2 + acc3));
        }
        return;
    }
    for (int task = threadIdx.x; task < nc * D; task += blockDim.x) {
        const int c = task / D, d = task % D;
        const int hl = c / p.rq, row = c % p.rq;
        if (hl >= p.G || row >= L) continue;
        float M = 0.0f;
        for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, p.ws_ml[((base + sp) * nc + c) * 2]);
        float acc = 0.0f, l = 0.0f;
        for (int sp = 0; sp < nsplit; ++sp) {
            const float f = __builtin_amdgcn_exp2f(p.ws_ml[((base + sp) * nc + c) * 2] - M);
            acc += f * p.ws_o[((base + sp) * nc + c) * D + d];
            l += f * p.ws_ml[((base + sp) * nc + c) * 2 + 1];
        }
        const float out = l > 0.0f ? acc / l : 0.0f;
        const int h = kvh * p.G + hl;
        p.o[((q_off + row) * p.H + h) * D + d] = Cvt<T>::from(out);
    }
}

// ------------------------------------------------------------------- host


Plan make_plan(int batch, int H, int Hkv, int q_hint, int k_hint) {
    Plan pl{};
    const int G = H / Hkv;
    pl.decode = q_hint >= 1 && G * q_hint <= 32;
    pl.rq = q_hint;
    pl.rk = k_hint;
    pl.ncols = G * q_hint;
    // Split the key range so that the grid has at least ~512 workgroups (one
    // per slot of the 256 CUs, two each), with splits as long as that allows:
    // from 2048 keys down to 512.  Long splits write and merge fewer
    // partials; at B=64, Hkv=8 and kv_len <= 8192, 2048-key splits ran in
    // 194 us against 217 us at 512.  Splits shorter than 512 keys cost more
    // in per-workgroup start-up and merging than they gain in parallelism:
    // one sequence of 32768 keys took 86 us with 128-key splits, 41 us with
    // 512; 8 x 4096 keys 55 against 34 us.
    const long long units = static_cast<long long>(batch) * Hkv;
    int split = 2048;
    while (split > 512 && units * ((k_hint + split - 1) / split) < 512) split >>= 1;
    pl.split_len = split;
    pl.max_splits = k_hint <= 0 ? 1 : (k_hint + split - 1) / split;
    return pl;
}

size_t workspace_bytes(const Plan &pl, int batch, int Hkv, int D) {
    if (!pl.decode) return 0;
    const size_t per = static_cast<size_t>(batch) * Hkv * pl.max_splits * pl.ncols;
    return per * D * sizeof(float) + per * 2 * sizeof(float) + 256;
}

// Prefill over a grid of ceil(q_hint / QT) query tiles per (b, kv head, head
// group); the workgroups of tile 0 cover any tiles past them.
template <typename T, int D, int W, int HW, int QSUB, int BSM, int TILE>
tecoopsStatus_t launch_prefill(const FaParams &p, const Plan &pl, hipStream_t s) {
    constexpr int QT = 32 * QSUB * (W / HW);
    auto *kern = &fa_prefill_kernel<T, D, W, HW, QSUB, BSM, TILE>;
    const size_t lds = prefill_lds_bytes<D, TILE, W, HW, QSUB, BSM>();
    if (!tecoops::reserve_lds(reinterpret_cast<const void *>(kern), lds))
        return TECOOPS_STATUS_INTERNAL_ERROR;
    const int units = p.batch * p.Hkv * (p.G / HW);
    const int tiles = (pl.rq + QT - 1) / QT;
    hipLaunchKernelGGL(kern, dim3(units, tiles), dim3(W * 64), lds, s, p);
    TECO_CHECK_LAUNCH("flash_attention prefill");
    return TECOOPS_STATUS_SUCCESS;
}

template <typename T, int D, int W, int QSUB, int BSM, int TILE = 64>
tecoopsStatus_t prefill_hw(const FaParams &p, const Plan &pl, hipStream_t s) {
    const int G = p.G;
    if (G % 4 == 0) return launch_prefill<T, D, W, 4, QSUB, BSM, TILE>(p, pl, s);
    if (G % 2 == 0) return launch_prefill<T, D, W, 2, QSUB, BSM, TILE>(p, pl, s);
    return launch_prefill<T, D, W, 1, QSUB, BSM, TILE>(p, pl, s);
}

// D = 128 prefill route for a query bound of at most 1024 rows: true takes
// the 12-wave kernel (96-row tiles, one workgroup per CU), false the 4-wave
// kernel over 32-row tiles (three per CU).  Over a long cached context the
// 12-wave kernel is ~10 % faster per row and key (each K/V tile serves
// three times the rows), but it pads rows to 96 and has a third of the
// workgroup slots.  So it is taken when the context is long (keys at least
// 4x the rows, or 2x and 2048 or more), its grid covers most CUs (160
// workgroups on 256 CUs), and it needs no more dispatch rounds (workgroups
// over slots, rounded up) than the 32-row kernel.  bf16 H32 Hkv8 causal
// block 16, µs 32-row / 12-wave (batch x query rows / keys):
//   taken: 64 x 64 / 4096 409 / 387, 64 x 96 / 4096 590 / 417, 16 x 256 /
//     4096 354 / 325, 8 x 512 / 4096 323 / 293, 16 x 512 / 2048 291 / 267,
//     8 x 1024 / 2048 246 / 219, 8 x 1024 / 4096 547 / 471, 2 x 1024 /
//     16384 (176 workgroups) 585 / 551, 32 x 256 / 1024 168 / 163, 12 x 700
//     / 4096 605 / 509, 40 x 160 / 4096 594 / 530
//   more rounds: 24 x 250 / 1000 (3 against 2) 120 / 135, 64 x 128 / 1024
//     196 / 222, 64 x 16 / 4096 205 / 358
//   short context: 32 x 256 / 512 88 / 99, 64 x 96 / 192 40 / 42, 64 x 256
//     / 256 105 / 118, 32 x 512 / 512 129 / 152, 16 x 1024 / 1024 191 / 190
//   under 160 workgroups: 4 x 256 / 16384 (96) 434 / 510, 16 x 64 / 16384
//     (128) 443 / 521, 3 x 1024 / 16384 (2 rounds against 1) 830 / 1118
//   where the rule misses: 48 x 200 / 2000 (5 rounds against 4) 482 / 454,
//     6 x 256 / 16384 (144 workgroups) 528 / 516, 16 x 512 / 1024 137 / 135
bool prefill_wide(const FaParams &p, const Plan &pl) {
    const long long q = pl.rq, k = pl.rk;
    if (k < 2 * q || (k < 4 * q && k < 2048)) return false;
    const int hw = p.G % 4 == 0 ? 4 : (p.G % 2 == 0 ? 2 : 1);
    const long long units = static_cast<long long>(p.batch) * p.Hkv * (p.G / hw);
    const long long n12 = units * ((q + 95) / 96), n4 = units * ((q + 31) / 32);
    const long long cus = tecoops::device_cus();
    if (n12 * 256 < 160 * cus) return false;
    return (n12 + cus - 1) / cus <= (n4 + 3 * cus - 1) / (3 * cus);
}

template <typename T, int D>
tecoopsStatus_t run(hipStream_t s, const FaParams &p, const Plan &pl) {
    // Block-size mode (block_of): the uniform-page loaders take block sizes
    // that are multiples of 8 (their 4- and 8-row groups start at multiples
    // of 8, so none crosses a cache block), powers of two with a shift
    const int bsm = p.lbs >= 3 ? 1 : (p.bs % 8 == 0 ? 2 : 0);
    if (pl.decode) {
        const size_t lds = decode_lds_bytes<D>();
        // mode 2 only where a uniform-page loader exists (else mode 0)
        auto *kern = bsm == 1 ? &fa_decode_kernel<T, D, 1> : &fa_decode_kernel<T, D, 0>;
        if constexpr (D == 64 || D == 96 || D == 128)
            if (bsm == 2) kern = &fa_decode_kernel<T, D, 2>;
        if (!tecoops::reserve_lds(reinterpret_cast<const void *>(kern), lds)) return TECOOPS_STATUS_INTERNAL_ERROR;
        dim3 grid(p.batch * p.Hkv, pl.max_splits);
        hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, p);
        TECO_CHECK_LAUNCH("flash_attention decode");
        if (pl.max_splits > 1) {
            hipLaunchKernelGGL((fa_decode_combine_kernel<T, D>), dim3(p.batch * p.Hkv), dim3(256),
                               0, s, p);
            TECO_CHECK_LAUNCH("flash_attention combine");
        }
        return TECOOPS_STATUS_SUCCESS;
    }
    if constexpr (D == 128) {
        // the uniform-page loader.  Long query ranges: 12 waves (3 per SIMD)
        // over 96 query rows and 96-key tiles.  Up to 1024 query rows (short
        // prompts, chunks over a cached context): 4 waves over 32 rows and
        // 32-key tiles, three workgroups per CU, which wastes fewer masked
        // rows and hides each workgroup's start-up behind the others, unless
        // prefill_wide finds a long cached context and a full grid.  bf16
        // H32 Hkv8, µs 12-wave / 4-wave: 4 x 4096 643 / 689, 1 x 16384
        // 2162 / 2370.
        const bool wide = pl.rq > 1024 || prefill_wide(p, pl);
        if (bsm == 1) {
            if (!wide) return prefill_hw<T, D, 4, 1, 1, 32>(p, pl, s);
            return prefill_hw<T, D, 12, 1, 1, 96>(p, pl, s);
        }
        if (bsm == 2) {  // block 24, µs mode 0 / 2: B4 S4096 606 / 587, B16 S1024 244 / 208
            if (!wide) return prefill_hw<T, D, 4, 1, 2, 32>(p, pl, s);
            return prefill_hw<T, D, 12, 1, 2, 96>(p, pl, s);
        }
        // other block sizes (the generic loader): the 12-wave kernel above
        // 1024 query rows too.  Block 24, µs 4-wave 64-key / 12-wave: B4
        // S4096 771 / 610, B1 S16384 2868-2883 / 2264-2269 (up to 1024 rows
        // the 4-wave 32-key kernel with this loader lost: 64 x 16 rows over
        // 4096 keys 262 / 342 us)
        if (pl.rq > 1024) return prefill_hw<T, D, 12, 1, 0, 96>(p, pl, s);
    }
    if constexpr (D == 64) {
        // long query ranges: 12 waves over 192-key tiles (3 per SIMD, 136
        // VGPRs).  bf16 H32 Hkv8 causal, µs 4-wave 64-key / 12-wave: B4 S4096
        // 371-376 / 335, B1 S16384 1417-1421 / 1276, B2 S8192 718-733 / 654,
        // B8 S2048 197-201 / 190; 8 waves over 128 keys 362 / 1374 / 701 / 204
        // and 16 over 256 (128 VGPRs, spills) 342 / 1290 / 657 / 192.
        if (bsm == 1 && pl.rq > 1024) return prefill_hw<T, D, 12, 1, 1, 192>(p, pl, s);
        // other block sizes, generic loader: block 24, B4 S4096 433 -> 354 us
        if (pl.rq > 1024) return prefill_hw<T, D, 12, 1, 0, 192>(p, pl, s);
    }
    if constexpr (D == 96) {
        // long query ranges: 12 waves over 96-key tiles (142 VGPRs).  µs
        // 4-wave 64-key / 12-wave 96-key / 12-wave 192-key: B4 S4096 598 /
        // 472 / 486, B1 S16384 2196 / 1771 / 1828, B8 S2048 316 / 267 / 278
        if (bsm == 1 && pl.rq > 1024) return prefill_hw<T, D, 12, 1, 1, 96>(p, pl, s);
        // other block sizes, generic loader: block 24, B4 S4096 648 -> 494 us
        if (pl.rq > 1024) return prefill_hw<T, D, 12, 1, 0, 96>(p, pl, s);
    }
    if constexpr (D == 32) {
        // long query ranges: 8 waves over 128-key tiles.  µs 4-wave 64-key /
        // 12-wave 192-key / 8-wave 128-key: B4 S4096 256 / 245 / 233, B1
        // S16384 986 / 904 / 883, B8 S2048 139 / 142 / 126
        if (pl.rq > 1024)
            return bsm == 1 ? prefill_hw<T, D, 8, 1, 1, 128>(p, pl, s)
                            : prefill_hw<T, D, 8, 1, 0, 128>(p, pl, s);
    }
    if constexpr (D > 128) {
        // 8 waves (2 per SIMD, 234 / 252 VGPRs) over 64-key tiles instead of
        // 4 waves at one per SIMD.  µs, 4 / 8 waves: D = 192 B4 S4096 2078 /
        // 938, B16 S1024 631 / 311, 16 x 256 rows over 4096 keys 1081 / 488,
        // 64 x 16 over 4096 566 / 489; D = 160 1410 / 854, 443 / 284, 691 /
        // 458, and 378 / 477 at 64 x 16 over 4096, where 4 waves stay.
        if (D == 192 || pl.rq > 16)
            return bsm == 1 ? prefill_hw<T, D, 8, 1, 1, 64>(p, pl, s)
                            : prefill_hw<T, D, 8, 1, 0, 64>(p, pl, s);
    }
    return bsm == 1 ? prefill_hw<T, D, 4, 1, 1>(p, pl, s) : prefill_hw<T, D, 4, 1, 0>(p, pl, s);
}

// Head sizes the kernels are built for: the reference takes the head size as
// its K-dimension tile (BK = size_per_head, flash_attention.scpp:188, looped
// at :347-348) in 32-column slabs, bounded by its on-chip buffers.
constexpr int kHeadSizes[] = {32, 64, 96, 128, 160, 192};

bool head_size_supported(int D) {
    for (int d : kHeadSizes)
        if (d == D) return true;
    return false;
}

template <typename T>
tecoopsStatus_t run_d(hipStream_t s, const FaParams &p, const Plan &pl, int D) {
    switch (D) {
        case 32: return run<T, 32>(s, p, pl);
        case 64: return run<T, 64>(s, p, pl);
        case 96: return run<T, 96>(s, p, pl);
        case 128: return run<T, 128>(s, p, pl);
        case 160: return run<T, 160>(s, p, pl);
        case 192: return run<T, 192>(s, p, pl);
        default: return TECOOPS_STATUS_NOT_SUPPORTED;
    }
}

bool is_packed_rowmajor(const tecoopsTensorStruct *d) {
    int expect = 1;
    for (int i = d->nbDims - 1; i >= 0; --i) {
        if (d->dimA[i] > 1 && d->strideA[i] != expect) return false;
        expect *= d->dimA[i];
    }
    return true;
}


// Argument checks of reference flash_attention.cpp:44-69, extended to bf16 and
// to the shape facts the kernels rely on; fills everything but the split-KV
// workspace.  max_seqlen_q / max_seqlen_k are launch-shape hints only: any
// value is accepted (the reference never reads them).  The q hint is raised to
// the mean q length (sum(q) / batch from q's descriptor) and the k hint
// capped by the block-table width * block_size, or taken as that width when
// <= 0.  fixed_hints keeps both as given (a q hint <= 0 becoming the mean),
// for a caller workspace sized by tecoopsGetFlashAttentionWorkspaceSize.
tecoopsStatus_t fa_prepare(tecoopsHandle_t handle, int max_seqlen_q, int max_seqlen_k,
                           const int *q_seq_lens, const int *cu_seqlens_q, const int *kv_seq_lens,
                           const tecoopsTensorDescriptor_t btDesc, const void *blockTable,
                           const tecoopsTensorDescriptor_t qDesc, const void *qData,
                           const tecoopsTensorDescriptor_t kDesc, const void *kCache,
                           const tecoopsTensorDescriptor_t vDesc, const void *vCache,
                           const tecoopsTensorDescriptor_t oDesc, void *oData, float softmax_scale,
                           int causal, bool fixed_hints, FaCall &c) {
    if (handle == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (!btDesc || !qDesc || !kDesc || !vDesc || !oDesc) return TECOOPS_STATUS_BAD_PARAM;
    if (!blockTable || !qData || !kCache || !vCache || !oData || !kv_seq_lens)
        return TECOOPS_STATUS_BAD_PARAM;
    if (q_seq_lens == nullptr && cu_seqlens_q == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    TECO_RETURN_IF(kDesc->dataType != vDesc->dataType, TECOOPS_STATUS_BAD_PARAM,
                   "k_cache data_type must be equal to v_cache data_type");
    TECO_RETURN_IF(!tecoops::is_16bit_float(kDesc->dataType), TECOOPS_STATUS_BAD_PARAM,
                   "k/v cache must be TECOOPS_DATA_HALF or TECOOPS_DATA_BFLOAT16");
    TECO_RETURN_IF(qDesc->dataType != kDesc->dataType || oDesc->dataType != kDesc->dataType,
                   TECOOPS_STATUS_BAD_PARAM, "q, k/v cache and output types must agree");
    TECO_RETURN_IF(kDesc->nbDims != 4 || vDesc->nbDims != 4 || qDesc->nbDims != 3 ||
                   oDesc->nbDims != 3 || btDesc->nbDims != 2,
                   TECOOPS_STATUS_BAD_PARAM, "flash_attention: unexpected tensor ranks");
    for (int i = 0; i < 4; ++i)
        TECO_RETURN_IF(kDesc->dimA[i] != vDesc->dimA[i], TECOOPS_STATUS_BAD_PARAM,
                       "shape of k v cache is not equal");
    for (int i = 0; i < 3; ++i)
        TECO_RETURN_IF(qDesc->dimA[i] != oDesc->dimA[i], TECOOPS_STATUS_BAD_PARAM,
                       "q and output shapes differ");
    const int total_q = qDesc->dimA[0], H = qDesc->dimA[1], D = qDesc->dimA[2];
    const int num_blocks = kDesc->dimA[0], Hkv = kDesc->dimA[1], bs = kDesc->dimA[2];
    const int batch = btDesc->dimA[0], bt_cols = btDesc->dimA[1];
    TECO_RETURN_IF(kDesc->dimA[3] != D, TECOOPS_STATUS_BAD_PARAM, "head_size mismatch");
    TECO_RETURN_IF(!head_size_supported(D), TECOOPS_STATUS_NOT_SUPPORTED,
                   "flash_attention: head_size %d not supported (32, 64, 96, 128, 160, 192)", D);
    TECO_RETURN_IF(H <= 0 || Hkv <= 0 || H % Hkv != 0, TECOOPS_STATUS_BAD_PARAM,
                   "num_heads must be a multiple of num_kv_heads");
    TECO_RETURN_IF(bs <= 0 || num_blocks <= 0 || batch <= 0 || total_q < 0 || bt_cols < 0,
                   TECOOPS_STATUS_BAD_PARAM, "empty cache or batch");
    TECO_RETURN_IF(fixed_hints && max_seqlen_k <= 0, TECOOPS_STATUS_BAD_PARAM,
                   "flash_attention: a caller workspace needs the max_seqlen_k it was sized for");
    TECO_RETURN_IF(!is_packed_rowmajor(qDesc) || !is_packed_rowmajor(oDesc) ||
                   !is_packed_rowmajor(kDesc) || !is_packed_rowmajor(vDesc) ||
                   btDesc->strideA[1] != 1,
                   TECOOPS_STATUS_NOT_SUPPORTED, "flash_attention: tensors must be row-major");
    for (const void *ptr : {qData, kCache, vCache, static_cast<const void *>(oData)})
        TECO_RETURN_IF(!tecoops::aligned(ptr, 16), TECOOPS_STATUS_BAD_PARAM,
                       "flash_attention: tensors must be 16-byte aligned");

    FaParams &p = c.p;
    p = FaParams{};
    p.q = static_cast<const uint16_t *>(qData);
    p.kc = static_cast<const uint16_t *>(kCache);
    p.vc = static_cast<const uint16_t *>(vCache);
    p.o = static_cast<uint16_t *>(oData);
    p.bt = static_cast<const int *>(blockTable);
    p.bt_stride = btDesc->strideA[0];
    p.q_lens = q_seq_lens;
    p.cu_q = cu_seqlens_q;
    p.kv_lens = kv_seq_lens;
    p.batch = batch;
    p.H = H;
    p.Hkv = Hkv;
    p.G = H / Hkv;
    p.bs = bs;
    p.lbs = (bs & (bs - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(bs)) : -1;
    p.num_blocks = num_blocks;
    const long long cap = static_cast<long long>(bt_cols) * bs;
    p.kv_cap = cap > 0x7fffffffLL ? 0x7fffffff : static_cast<int>(cap);
    p.page_stride = static_cast<long long>(Hkv) * bs * D;
    const float scale = softmax_scale > 0.0f ? softmax_scale : 1.0f / std::sqrt(static_cast<float>(D));
    p.scale_log2 = scale * 1.4426950408889634f;
    p.inv_scale_log2 = 1.0f / p.scale_log2;
    p.causal = causal != 0;

    // The q bound routes the call (decode or prefill) and sizes the prefill
    // grid.  It is raised to the mean q length, which the host knows: a bound
    // that is too small (the reference never reads it) would otherwise send a
    // prefill down the decode route, correct but many times slower.  A caller
    // workspace was sized for the bounds as given, so they are kept then.
    const int q_mean = std::max(1, (total_q + batch - 1) / batch);
    const int q_hint = fixed_hints ? (max_seqlen_q > 0 ? max_seqlen_q : q_mean)
                                    : std::max(max_seqlen_q, q_mean);
    int k_hint = max_seqlen_k;
    if (!fixed_hints) k_hint = max_seqlen_k > 0 ? std::min(max_seqlen_k, p.kv_cap) : p.kv_cap;
    c.pl = make_plan(batch, H, Hkv, q_hint, k_hint);
    p.total_q = total_q;
    if (c.pl.decode) {
        p.rq = c.pl.rq;
        p.ncols = c.pl.ncols;
        p.split_len = c.pl.split_len;
        p.max_splits = c.pl.max_splits;
    } else {
        p.rq = 0x7fffffff;
    }
    c.D = D;
    c.bf16 = kDesc->dataType == TECOOPS_DATA_BFLOAT16;
    return TECOOPS_STATUS_SUCCESS;
}

size_t fa_workspace_bytes(const FaCall &c) {
    return workspace_bytes(c.pl, c.p.batch, c.p.Hkv, c.D);
}

// Enqueues the call on stream s with its split-KV partials in ws (at least
// fa_workspace_bytes(c) bytes; unused by prefill).
tecoopsStatus_t fa_launch(hipStream_t s, FaCall &c, void *ws) {
    if (c.pl.decode) {
        const size_t per = static_cast<size_t>(c.p.batch) * c.p.Hkv * c.pl.max_splits * c.pl.ncols;
        c.p.ws_o = static_cast<float *>(ws);
        c.p.ws_ml = c.p.ws_o + per * c.D;
    }
    using tecoops::dev::bf16;
    using tecoops::dev::f16;
    return c.bf16 ? run_d<bf16>(s, c.p, c.pl, c.D) : run_d<f16>(s, c.p, c.pl, c.D);
}

}  // namespace

namespace tecoops {
namespace fa {

tecoopsStatus_t prepare(tecoopsHandle_t handle, int max_seqlen_q, int max_seqlen_k,
                        const int *q_seq_lens, const int *cu_seqlens_q, const int *kv_seq_lens,
                        const tecoopsTensorDescriptor_t btDesc, const void *blockTable,
                        const tecoopsTensorDescriptor_t qDesc, const void *qData,
                        const tecoopsTensorDescriptor_t kDesc, const void *kCache,
                        const tecoopsTensorDescriptor_t vDesc, const void *vCache,
                        const tecoopsTensorDescriptor_t oDesc, void *oData, float softmax_scale,
                        int causal, bool fixed_hints, FaCall &c) {
    return fa_prepare(handle, max_seqlen_q, max_seqlen_k, q_seq_lens, cu_seqlens_q, kv_seq_lens,
                      btDesc, blockTable, qDesc, qData, kDesc, kCache, vDesc, vCache, oDesc, oData,
                      softmax_scale, causal, fixed_hints, c);
}

size_t workspace_bytes(const FaCall &c) { return fa_workspace_bytes(c); }

tecoopsStatus_t launch(hipStream_t s, FaCall &c, void *ws) { return fa_launch(s, c, ws); }

}  // namespace fa
}  // namespace tecoops

extern "C" tecoopsStatus_t tecoopsGetFlashAttentionWorkspaceSize(int batch, int num_heads,
                                                                 int head_size, int max_seqlen_q,
                                                                 int max_seqlen_k, size_t *bytes) {
    if (bytes == nullptr || batch <= 0 || num_heads <= 0 || head_size <= 0 || max_seqlen_k <= 0)
        return TECOOPS_STATUS_BAD_PARAM;
    // Worst case over kv-head counts; max_seqlen_q <= 0 takes the longest q
    // length the decode route admits (32 / G rows).
    size_t worst = 0;
    for (int hkv = 1; hkv <= num_heads; ++hkv) {
        if (num_heads % hkv) continue;
        const int G = num_heads / hkv;
        const int q_hint = max_seqlen_q > 0 ? max_seqlen_q : std::max(1, 32 / G);
        const Plan pl = make_plan(batch, num_heads, hkv, q_hint, max_seqlen_k);
        const size_t b = workspace_bytes(pl, batch, hkv, head_size);
        if (b > worst) worst = b;
    }
    *bytes = worst;
    return TECOOPS_STATUS_SUCCESS;
}

extern "C" tecoopsStatus_t tecoopsFlashAttentionEx(
    tecoopsHandle_t handle, int max_seqlen_q, int max_seqlen_k, const int *q_seq_lens,
    const int *cu_seqlens_q, const int *kv_seq_lens, const tecoopsTensorDescriptor_t btDesc,
    const void *blockTable, const tecoopsTensorDescriptor_t qDesc, const void *qData,
    const tecoopsTensorDescriptor_t kDesc, const void *kCache,
    const tecoopsTensorDescriptor_t vDesc, const void *vCache,
    const tecoopsTensorDescriptor_t oDesc, void *oData, float softmax_scale, int causal,
    void *workspace) {
    FaCall c;
    tecoopsStatus_t st = fa_prepare(handle, max_seqlen_q, max_seqlen_k, q_seq_lens, cu_seqlens_q,
                                    kv_seq_lens, btDesc, blockTable, qDesc, qData, kDesc, kCache,
                                    vDesc, vCache, oDesc, oData, softmax_scale, causal,
                                    workspace != nullptr, c);
    if (st != TECOOPS_STATUS_SUCCESS) return st;
    void *ws = workspace;
    // With one split per sequence the decode kernel writes the output rows
    // itself and reads no partials: no scratch is needed then.
    if (c.pl.decode && c.pl.max_splits > 1 && ws == nullptr) {
        st = tecoops::handle_scratch(handle, fa_workspace_bytes(c), &ws);
        if (st != TECOOPS_STATUS_SUCCESS) return st;
    }
    return fa_launch(handle->stream, c, ws);
}

extern "C" tecoopsStatus_t tecoopsFlashAttention(
    tecoopsHandle_t handle, int max_seqlen_q, int max_seqlen_k, int max_block_num,
    const int *q_seq_lens, const int *kv_seq_lens, const tecoopsTensorDescriptor_t blockTableDesc,
    const void *blockTable, const tecoopsTensorDescriptor_t qDataDesc, const void *qData,
    const tecoopsTensorDescriptor_t kCacheDesc, const void *kCache,
    const tecoopsTensorDescriptor_t vCacheDesc, const void *vCache,
    const tecoopsTensorDescriptor_t oDataDesc, void *oData, void *workspace) {
    // The reference accepts workspace and never reads it
    // (flash_attention.cpp:110), and takes the block count from kCacheDesc:
    // both are ignored here too, so a caller's unrelated buffer is never
    // written.  The split-KV partials live in the handle's scratch.
    (void)max_block_num;
    (void)workspace;
    if (q_seq_lens == nullptr) return handle ? TECOOPS_STATUS_BAD_PARAM : TECOOPS_STATUS_NOT_INITIALIZED;
    return tecoopsFlashAttentionEx(handle, max_seqlen_q, max_seqlen_k, q_seq_lens, nullptr,
                                   kv_seq_lens, blockTableDesc, blockTable, qDataDesc, qData,
                                   kCacheDesc, kCache, vCacheDesc, vCache, oDataDesc, oData,
                                   -1.0f, 1, nullptr);
}

