/*
 * oracle.c — CPU restatement of the reference's LLM-inference operator path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP kernels and the CPU
 * baseline timed by bench.py.  Never linked into the product library.
 *
 * What each function restates, and what pins it (the checks live in
 * tests/test_oracle.py):
 *   orc_f2h / orc_h2f   RNE fp16 conversion as in the reference harness
 *                       (test/zoo/teco/rms_norm/rms_norm.cpp:120-193).  Pinned by
 *                       exhaustive comparison with numpy's float16 over all 2^16
 *                       patterns and over float32 boundary/tie cases.
 *   orc_f2b / orc_b2f   bfloat16 RNE.  Pinned against a bit-level numpy RNE and
 *                       torch.bfloat16 casts.
 *   orc_reshape_and_cache  test/zoo/teco/reshape_and_cache/reshape_and_cache.cpp:
 *                       116-148 and doc/op_docs/reshape_and_cache.md:13-22.  Pinned
 *                       by the doc example (slots [0,1,3,6], block 2,
 *                       reshape_and_cache.md:137-146), brute force on tiny inputs,
 *                       and the permutation invariants (each slot written once,
 *                       untouched slots keep their contents, slot < 0 no-op).
 *   orc_rms_norm        rms_norm.cpp:195-234 (pure and fused-add rounding order:
 *                       sum of unrounded (x+r)^2, normalise half(x+r)).  Pinned by
 *                       closed forms (constant row -> w/sqrt(1+eps/c^2), zero row
 *                       -> 0), scale invariance, and the reference python tests'
 *                       formulas (python_api_test/test_rms_norm.py:31-43).
 *   orc_flash_attention test/zoo/teco/flash_attention/flash_attention.py:79-140
 *                       (paged gather, bottom-right causal mask, GQA by
 *                       repeat_interleave) with the kernel's q_start clamp
 *                       (flash_attention.scpp:75-76) and l == 0 -> 0 rule (:388).
 *                       Pinned by kv_len = 1 -> O = V0, constant K -> mean of V,
 *                       decode row = last row of the full prefill, a numpy
 *                       float64 dense softmax on small shapes, and GQA head
 *                       permutation equivariance.
 *   orc_causal_conv1d   test/zoo/teco/causal_conv1d/causal_conv1d.py:44-122 and
 *                       teco/ual/kernel/causal_conv1d/causal_conv1d.scpp:56-116
 *                       (pad slot skip, api_mode override, state = last width-1
 *                       inputs).  Pinned by w = e_last -> silu(x), zero initial
 *                       state == has_init 0, chunked-sequence composition through
 *                       the state, and numpy np.convolve per channel.
 *   orc_rotary_embedding  no reference implementation (rotary is absent from the
 *                       reference).  Closed form of NeoX / GPT-J rotary.  Pinned
 *                       by: position 0 is the identity, per-pair norm
 *                       preservation, composition p then -p is the identity, and
 *                       an independent numpy complex-multiplication formulation.
 *   orc_gemv / orc_gemv_int8  no reference implementation.  fp64 dot products.
 *                       Pinned against numpy matmul in float64 and exact integer
 *                       sums for integer-valued inputs.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ threads */

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------- conversions */

static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return bits_f(sign | 0x7f800000u | (m << 13) | (m ? 0x400000u : 0));
    if (e != 0) return bits_f(sign | ((e + 112u) << 23) | (m << 13));
    /* zero or subnormal: m * 2^-24 is exact in float */
    float v = (float)m * (1.0f / 16777216.0f);
    return sign ? -v : v;
}

uint16_t orc_f2h(float f) {
    uint32_t x = f_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return sign | 0x7c00u;   /* >= 65520 rounds to inf */
    if (ax <= 0x33000000u) return sign;             /* <= 2^-25 rounds to 0 */
    uint32_t e = ax >> 23;
    uint32_t mant = ax & 0x7fffffu;
    if (e >= 113) {                                 /* normal half */
        uint32_t r = ((e - 112u) << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    /* subnormal half: value = M * 2^(e-150); in units of 2^-24 shift by 126-e */
    uint32_t M = mant | 0x800000u;
    uint32_t s = 126u - e;
    uint32_t q = M >> s;
    uint32_t rem = M & ((1u << s) - 1u);
    uint32_t half = 1u << (s - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float orc_b2f(uint16_t b) { return bits_f((uint32_t)b << 16); }

uint16_t orc_f2b(float f) {
    uint32_t u = f_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_to_f(uint16_t v, int dtype) { return dtype == 9 ? orc_b2f(v) : orc_h2f(v); }
uint16_t orc_from_f(float f, int dtype) { return dtype == 9 ? orc_f2b(f) : orc_f2h(f); }

void orc_to_f_array(const uint16_t *src, float *dst, size_t n, int dtype) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) dst[i] = orc_to_f(src[i], dtype);
}

void orc_from_f_array(const float *src, uint16_t *dst, size_t n, int dtype) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) dst[i] = orc_from_f(src[i], dtype);
}

/* ------------------------------------------------------------------ memset */

/* teco/ual/kernel/memset/memset_4B_align.scpp:79-140: byte fill, value
 * truncated to uint8. */
void orc_memset(void *x, int value, size_t size) { memset(x, (uint8_t)value, size); }

/* ------------------------------------------------------- reshape_and_cache */

/* reshape_and_cache.cpp:116-148; cache layout [num_blocks, H, block_size, D]. */
void orc_reshape_and_cache(const uint16_t *key, const uint16_t *value,
                           const int64_t *slot_mapping,
                           uint16_t *key_cache, uint16_t *value_cache,
                           int num_tokens, int num_kv_heads, int head_size,
                           int num_blocks, int block_size) {
    const int64_t capacity = (int64_t)num_blocks * block_size;
    for (int t = 0; t < num_tokens; ++t) {
        int64_t slot = slot_mapping[t];
        if (slot < 0 || slot >= capacity) continue;
        int64_t blk = slot / block_size;
        int64_t off = slot % block_size;
        for (int h = 0; h < num_kv_heads; ++h) {
            size_t src = ((size_t)t * num_kv_heads + h) * head_size;
            size_t dst = (((size_t)blk * num_kv_heads + h) * block_size + off) * head_size;
            memcpy(key_cache + dst, key + src, sizeof(uint16_t) * head_size);
            memcpy(value_cache + dst, value + src, sizeof(uint16_t) * head_size);
        }
    }
}

/* ---------------------------------------------------------------- rms_norm */

/* rms_norm.cpp:195-234.  Per row, fp32 running sum in index order. */
void orc_rms_norm(const uint16_t *input, const uint16_t *weight, const uint16_t *residual,
                  uint16_t *output, uint16_t *residual_out,
                  int num_tokens, int hidden_size, float eps, int dtype) {
    const int D = hidden_size;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < num_tokens; ++r) {
        const uint16_t *xr = input + (size_t)r * D;
        uint16_t *yr = output + (size_t)r * D;
        float sum_sq = 0.0f;
        if (residual) {
            const uint16_t *rr = residual + (size_t)r * D;
            uint16_t *ro = residual_out + (size_t)r * D;
            for (int d = 0; d < D; ++d) {
                float v = orc_to_f(xr[d], dtype) + orc_to_f(rr[d], dtype);
                sum_sq += v * v;
                ro[d] = orc_from_f(v, dtype);
            }
            float rstd = 1.0f / sqrtf(sum_sq / (float)D + eps);
            for (int d = 0; d < D; ++d) {
                float v = orc_to_f(ro[d], dtype) * rstd * orc_to_f(weight[d], dtype);
                yr[d] = orc_from_f(v, dtype);
            }
        } else {
            for (int d = 0; d < D; ++d) {
                float v = orc_to_f(xr[d], dtype);
                sum_sq += v * v;
            }
            float rstd = 1.0f / sqrtf(sum_sq / (float)D + eps);
            for (int d = 0; d < D; ++d) {
                float v = orc_to_f(xr[d], dtype) * rstd * orc_to_f(weight[d], dtype);
                yr[d] = orc_from_f(v, dtype);
            }
        }
    }
}

/* --------------------------------------------------------- flash_attention */

/* flash_attention.py:79-140.  For sequence b (q_len L, kv_len S), query row i
 * is at causal position S - L + i (clamped so that a chunk longer than its KV
 * sees keys <= i, flash_attention.scpp:75-76) and attends keys j <= that
 * position; all of [0, S) without the mask.  GQA: head h reads kv head
 * h / (H / Hkv).  fp32 softmax; rows with no visible key produce 0. */
void orc_flash_attention_heads(const uint16_t *q, const uint16_t *k_cache,
                               const uint16_t *v_cache, const int32_t *block_table,
                               int block_table_stride, const int32_t *q_seq_lens,
                               const int32_t *kv_seq_lens, int batch, int num_heads,
                               int num_kv_heads, int head_size, int block_size,
                               float softmax_scale, int causal, int dtype,
                               int b_only, int h_begin, int h_end, float *out) {
    const int H = num_heads, Hkv = num_kv_heads, D = head_size;
    const int group = H / Hkv;
    long long q_off = 0;
    for (int b = 0; b < batch; ++b) {
        const int L = q_seq_lens[b];
        const int S = kv_seq_lens[b];
        const long long qb = q_off;
        q_off += L;
        if (b_only >= 0 && b != b_only) continue;
        if (L <= 0) continue;
        int q_start = causal ? S - L : 0;
        if (q_start < 0) q_start = 0;
        int hb = h_begin < 0 ? 0 : h_begin;
        int he = h_end < 0 ? H : h_end;
        for (int kvh = hb / group; kvh <= (he - 1) / group; ++kvh) {
            /* gather this (b, kv head) slice of K and V as fp32 [S][D] */
            float *kf = (float *)malloc(sizeof(float) * (size_t)(S > 0 ? S : 1) * D);
            float *vf = (float *)malloc(sizeof(float) * (size_t)(S > 0 ? S : 1) * D);
#pragma omp parallel for schedule(static)
            for (int j = 0; j < S; ++j) {
                int64_t page = block_table[(size_t)b * block_table_stride + j / block_size];
                size_t base = (((size_t)page * Hkv + kvh) * block_size + j % block_size) * D;
                for (int d = 0; d < D; ++d) {
                    kf[(size_t)j * D + d] = orc_to_f(k_cache[base + d], dtype);
                    vf[(size_t)j * D + d] = orc_to_f(v_cache[base + d], dtype);
                }
            }
            int h0 = kvh * group > hb ? kvh * group : hb;
            int h1 = (kvh + 1) * group < he ? (kvh + 1) * group : he;
            const int rows = (h1 - h0) * L;
#pragma omp parallel
            {
                float *p = (float *)malloc(sizeof(float) * (size_t)(S > 0 ? S : 1));
                float *qf = (float *)malloc(sizeof(float) * (size_t)D);
                float *acc = (float *)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(dynamic, 16)
                for (int task = 0; task < rows; ++task) {
                    const int h = h0 + task / L;
                    const int i = task % L;
                    const uint16_t *qr = q + ((size_t)(qb + i) * H + h) * D;
                    float *orow = out + ((size_t)(qb + i) * H + h) * D;
                    for (int d = 0; d < D; ++d) qf[d] = orc_to_f(qr[d], dtype);
                    int visible = causal ? q_start + i + 1 : S;
                    if (visible > S) visible = S;
                    if (visible <= 0) {
                        for (int d = 0; d < D; ++d) orow[d] = 0.0f;
                        continue;
                    }
                    float m = -INFINITY;
                    for (int j = 0; j < visible; ++j) {
                        const float *kr = kf + (size_t)j * D;
                        float s = 0.0f;
                        for (int d = 0; d < D; ++d) s += qf[d] * kr[d];
                        s *= softmax_scale;
                        p[j] = s;
                        if (s > m) m = s;
                    }
                    float l = 0.0f;
                    for (int j = 0; j < visible; ++j) {
                        p[j] = expf(p[j] - m);
                        l += p[j];
                    }
                    for (int d = 0; d < D; ++d) acc[d] = 0.0f;
                    for (int j = 0; j < visible; ++j) {
                        const float *vr = vf + (size_t)j * D;
                        const float pj = p[j];
                        for (int d = 0; d < D; ++d) acc[d] += pj * vr[d];
                    }
                    const float inv = 1.0f / l;
                    for (int d = 0; d < D; ++d) orow[d] = acc[d] * inv;
                }
                free(p);
                free(qf);
                free(acc);
            }
            free(kf);
            free(vf);
        }
    }
}

void orc_flash_attention(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                         const int32_t *block_table, int block_table_stride,
                         const int32_t *q_seq_lens, const int32_t *kv_seq_lens,
                         int batch, int num_heads, int num_kv_heads, int head_size,
                         int block_size, float softmax_scale, int causal, int dtype,
                         float *out) {
    orc_flash_attention_heads(q, k_cache, v_cache, block_table, block_table_stride,
                              q_seq_lens, kv_seq_lens, batch, num_heads, num_kv_heads,
                              head_size, block_size, softmax_scale, causal, dtype,
                              -1, -1, -1, out);
}

/* ----------------------------------------------------------- causal_conv1d */

static inline float silu_f(float v) { return v / (1.0f + expf(-v)); }

/* causal_conv1d.py:44-122 / causal_conv1d.scpp:56-116, generalised to any
 * width, optional bias and strided addressing (see tecoopsCausalConv1dEx). */
void orc_causal_conv1d(int batch, int seq_len, int dim, int width,
                       const uint16_t *x, long long x_batch_stride, long long x_seq_stride,
                       long long x_dim_stride,
                       float *out, long long out_batch_stride, long long out_seq_stride,
                       long long out_dim_stride,
                       const uint16_t *weight, int w_dim_stride, int w_width_stride,
                       const uint16_t *bias, uint16_t *conv_state, int conv_state_stride,
                       const int32_t *query_start_loc, const int32_t *cache_indices,
                       const int8_t *has_initial_state, int pad_slot_id, int api_mode,
                       int silu) {
    const int W = width;
    for (int b = 0; b < batch; ++b) {
        long long start, len, xb, ob;
        if (query_start_loc) {
            start = query_start_loc[b];
            len = query_start_loc[b + 1] - query_start_loc[b];
            xb = start * x_seq_stride;
            ob = start * out_seq_stride;
        } else {
            start = 0;
            len = seq_len;
            xb = (long long)b * x_batch_stride;
            ob = (long long)b * out_batch_stride;
        }
        const int cidx = cache_indices ? cache_indices[b] : b;
        if (cidx == pad_slot_id) continue;
        if (len <= 0) continue;
        const int use_state = conv_state &&
            (api_mode == 1 || (has_initial_state ? has_initial_state[b] != 0 : 0));
        uint16_t *st = conv_state ? conv_state + (size_t)cidx * conv_state_stride : NULL;
#pragma omp parallel for schedule(static)
        for (int d = 0; d < dim; ++d) {
            float wv[8];
            for (int k = 0; k < W; ++k)
                wv[k] = orc_h2f(weight[(size_t)d * w_dim_stride + (size_t)k * w_width_stride]);
            const float bv = bias ? orc_h2f(bias[d]) : 0.0f;
            /* full_x = [prefix (W-1 values), seq]; prefix is state or zeros */
            uint16_t prefix[8];
            for (int k = 0; k < W - 1; ++k)
                prefix[k] = use_state ? st[(size_t)k * dim + d] : 0;
            for (long long t = 0; t < len; ++t) {
                float acc = 0.0f;
                for (int k = 0; k < W; ++k) {
                    long long src = t - (W - 1) + k;   /* index into seq; < 0 is prefix */
                    uint16_t xv = src >= 0
                        ? x[xb + src * x_seq_stride + (long long)d * x_dim_stride]
                        : prefix[W - 1 + src];
                    acc += orc_h2f(xv) * wv[k];
                }
                acc += bv;
                out[ob + t * out_seq_stride + (long long)d * out_dim_stride] =
                    silu ? silu_f(acc) : acc;
            }
            if (st) {
                /* new state = last W-1 entries of full_x */
                for (int k = 0; k < W - 1; ++k) {
                    long long src = len - (W - 1) + k;
                    uint16_t v = src >= 0
                        ? x[xb + src * x_seq_stride + (long long)d * x_dim_stride]
                        : prefix[W - 1 + src];
                    st[(size_t)k * dim + d] = v;
                }
            }
        }
    }
}

/* -------------------------------------------------------- rotary embedding */

/* No reference implementation exists.  NeoX: (x[i], x[i+rot/2]) rotates by
 * theta_i; GPT-J: (x[2i], x[2i+1]).  theta_i = pos * base^(-2i/rot_dim),
 * evaluated in double; or cos/sin read from cos_sin_cache. */
void orc_rotary_embedding(const int64_t *positions, const uint16_t *query, const uint16_t *key,
                          float *query_out, float *key_out,
                          int num_tokens, int num_heads, int num_kv_heads, int head_size,
                          int rot_dim, long long query_stride, long long key_stride,
                          const float *cos_sin_cache, int max_position, float base,
                          int is_neox, int dtype) {
    const int half = rot_dim / 2;
#pragma omp parallel for schedule(static)
    for (int t = 0; t < num_tokens; ++t) {
        const int64_t pos = positions[t];
        const int valid = cos_sin_cache ? (pos >= 0 && pos < max_position) : 1;
        double cs[512], sn[512];
        for (int i = 0; i < half && i < 512; ++i) {
            if (cos_sin_cache) {
                if (valid) {
                    cs[i] = cos_sin_cache[(size_t)pos * rot_dim + i];
                    sn[i] = cos_sin_cache[(size_t)pos * rot_dim + half + i];
                }
            } else {
                double inv_freq = pow((double)base, -2.0 * i / (double)rot_dim);
                double th = (double)pos * inv_freq;
                cs[i] = cos(th);
                sn[i] = sin(th);
            }
        }
        for (int which = 0; which < 2; ++which) {
            const uint16_t *src = which ? key : query;
            float *dst = which ? key_out : query_out;
            const int nh = which ? num_kv_heads : num_heads;
            const long long ts = which ? key_stride : query_stride;
            if (!src) continue;
            for (int h = 0; h < nh; ++h) {
                const uint16_t *xr = src + (size_t)t * ts + (size_t)h * head_size;
                float *yr = dst + (size_t)t * ts + (size_t)h * head_size;
                for (int d = 0; d < head_size; ++d) yr[d] = orc_to_f(xr[d], dtype);
                if (!valid) continue;
                for (int i = 0; i < half; ++i) {
                    int i1 = is_neox ? i : 2 * i;
                    int i2 = is_neox ? i + half : 2 * i + 1;
                    double x1 = orc_to_f(xr[i1], dtype), x2 = orc_to_f(xr[i2], dtype);
                    yr[i1] = (float)(x1 * cs[i] - x2 * sn[i]);
                    yr[i2] = (float)(x2 * cs[i] + x1 * sn[i]);
                }
            }
        }
    }
}

/* -------------------------------------------------------------------- GEMV */

/* No reference implementation exists.  y[b,n] = sum_k W[n,k] x[b,k] in fp64. */
void orc_gemv(const uint16_t *weight, const uint16_t *x, float *y,
              int batch, int n, int k, int dtype) {
    float *xf = (float *)malloc(sizeof(float) * (size_t)batch * k);
    for (size_t i = 0; i < (size_t)batch * k; ++i) xf[i] = orc_to_f(x[i], dtype);
#pragma omp parallel
    {
        float *wf = (float *)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(static)
        for (int r = 0; r < n; ++r) {
            const uint16_t *wr = weight + (size_t)r * k;
            for (int c = 0; c < k; ++c) wf[c] = orc_to_f(wr[c], dtype);
            for (int b = 0; b < batch; ++b) {
                const float *xr = xf + (size_t)b * k;
                double acc = 0.0;
                for (int c = 0; c < k; ++c) acc += (double)wf[c] * (double)xr[c];
                y[(size_t)b * n + r] = (float)acc;
            }
        }
        free(wf);
    }
    free(xf);
}

/* y[b,n] = s[n] * sum_k Wq[n,k] x[b,k] in fp64; s and x fp16. */
void orc_gemv_int8(const int8_t *weight, const uint16_t *scales, const uint16_t *x, float *y,
                   int batch, int n, int k) {
    float *xf = (float *)malloc(sizeof(float) * (size_t)batch * k);
    for (size_t i = 0; i < (size_t)batch * k; ++i) xf[i] = orc_h2f(x[i]);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < n; ++r) {
        const int8_t *wr = weight + (size_t)r * k;
        const double s = orc_h2f(scales[r]);
        for (int b = 0; b < batch; ++b) {
            const float *xr = xf + (size_t)b * k;
            double acc = 0.0;
            for (int c = 0; c < k; ++c) acc += (double)wr[c] * (double)xr[c];
            y[(size_t)b * n + r] = (float)(s * acc);
        }
    }
    free(xf);
}

/* ------------------------------------------------- reference harness RNG
 * libstdc++ semantics restated (pb_tools.h:123-200): minstd_rand0 seeded with
 * s mod m (1 when that is 0); generate_canonical<double, 53> with
 * R = max - min + 1 = 2^31 - 2 takes ceil(53 / floor(log2 R)) = 2 draws:
 * (u1 - 1 + (u2 - 1) R) / R^2, clamped below 1; uniform = c (b - a) + a;
 * normal = Marsaglia polar pairs (second value cached) scaled by sigma, plus mu.
 * Pinned by the C++ standard's minstd_rand0 check value and by exact rational
 * evaluation of the canonical formula in tests/test_harness_rng.py. */

#define ORC_MINSTD_M 2147483647ull

static uint64_t minstd_seed(long long s) {
    /* result_type is unsigned long: a negative seed wraps before the modulo */
    const uint64_t u = (uint64_t)s % ORC_MINSTD_M;
    return u == 0 ? 1 : u;
}

static inline uint64_t minstd_next(uint64_t *x) {
    *x = (*x * 16807ull) % ORC_MINSTD_M;
    return *x;
}

static inline double canon53(uint64_t *x) {
    const double r = 2147483646.0;
    double sum = 0.0, tmp = 1.0;
    for (int k = 0; k < 2; ++k) {
        sum += (double)(minstd_next(x) - 1) * tmp;
        tmp *= r;
    }
    double ret = sum / tmp;
    if (ret >= 1.0) ret = nextafter(1.0, 0.0);
    return ret;
}

uint32_t orc_minstd_nth(long long seed, size_t n) {
    uint64_t x = minstd_seed(seed);
    for (size_t i = 0; i < n; ++i) minstd_next(&x);
    return (uint32_t)x;
}

void orc_harness_uniform(long long seed, size_t n, double lo, double hi, double *out) {
    uint64_t x = minstd_seed(seed);
    for (size_t i = 0; i < n; ++i) out[i] = canon53(&x) * (hi - lo) + lo;
}

void orc_harness_normal(long long seed, size_t n, double mu, double sigma, double *out) {
    uint64_t x = minstd_seed(seed);
    int saved_ok = 0;
    double saved = 0.0;
    for (size_t i = 0; i < n; ++i) {
        double v;
        if (saved_ok) {
            saved_ok = 0;
            v = saved;
        } else {
            double a, b, r2;
            do {
                a = 2.0 * canon53(&x) - 1.0;
                b = 2.0 * canon53(&x) - 1.0;
                r2 = a * a + b * b;
            } while (r2 > 1.0 || r2 == 0.0);
            const double mult = sqrt(-2 * log(r2) / r2);
            saved = a * mult;
            saved_ok = 1;
            v = b * mult;
        }
        out[i] = v * sigma + mu;
    }
}

void orc_harness_uniform_f32(long long seed, size_t n, float lo, float hi, float *out) {
    uint64_t x = minstd_seed(seed);
    /* generate_canonical<float, 24>: one draw; R rounds to 2^31 in float */
    const float r = (float)2147483646.0;
    for (size_t i = 0; i < n; ++i) {
        float ret = (float)(minstd_next(&x) - 1) / r;
        if (ret >= 1.0f) ret = nextafterf(1.0f, 0.0f);
        out[i] = ret * (hi - lo) + lo;
    }
}
