/*
 * oracle.h — CPU restatement of the reference's LLM-inference operator path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * kernels and the CPU baseline timed by bench.py.  Only tests/, the smoke()
 * entry of __graft_entry__.py and bench.py's cpu_baseline leg may load it; the
 * product library (libtecoops.so) never links or calls it.
 *
 * 16-bit element buffers are passed as uint16_t bit patterns; `dtype` selects
 * their meaning: 1 = IEEE fp16 (TECOOPS_DATA_HALF), 9 = bfloat16
 * (TECOOPS_DATA_BFLOAT16).  Conversions round to nearest even.
 *
 * Pinning status of every function is listed in the header of oracle.c.
 */
#ifndef TECOOPS_ORACLE_H_
#define TECOOPS_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void orc_set_threads(int n);
int orc_get_threads(void);

float orc_h2f(uint16_t h);
uint16_t orc_f2h(float f);
float orc_b2f(uint16_t b);
uint16_t orc_f2b(float f);
float orc_to_f(uint16_t v, int dtype);
uint16_t orc_from_f(float f, int dtype);
void orc_to_f_array(const uint16_t *src, float *dst, size_t n, int dtype);
void orc_from_f_array(const float *src, uint16_t *dst, size_t n, int dtype);

void orc_memset(void *x, int value, size_t size);

void orc_reshape_and_cache(const uint16_t *key, const uint16_t *value,
                           const int64_t *slot_mapping,
                           uint16_t *key_cache, uint16_t *value_cache,
                           int num_tokens, int num_kv_heads, int head_size,
                           int num_blocks, int block_size);

void orc_rms_norm(const uint16_t *input, const uint16_t *weight, const uint16_t *residual,
                  uint16_t *output, uint16_t *residual_out,
                  int num_tokens, int hidden_size, float eps, int dtype);

void orc_flash_attention(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                         const int32_t *block_table, int block_table_stride,
                         const int32_t *q_seq_lens, const int32_t *kv_seq_lens,
                         int batch, int num_heads, int num_kv_heads, int head_size,
                         int block_size, float softmax_scale, int causal, int dtype,
                         float *out);

void orc_flash_attention_heads(const uint16_t *q, const uint16_t *k_cache,
                               const uint16_t *v_cache, const int32_t *block_table,
                               int block_table_stride, const int32_t *q_seq_lens,
                               const int32_t *kv_seq_lens, int batch, int num_heads,
                               int num_kv_heads, int head_size, int block_size,
                               float softmax_scale, int causal, int dtype,
                               int b_only, int h_begin, int h_end, float *out);

void orc_causal_conv1d(int batch, int seq_len, int dim, int width,
                       const uint16_t *x, long long x_batch_stride, long long x_seq_stride,
                       long long x_dim_stride,
                       float *out, long long out_batch_stride, long long out_seq_stride,
                       long long out_dim_stride,
                       const uint16_t *weight, int w_dim_stride, int w_width_stride,
                       const uint16_t *bias, uint16_t *conv_state, int conv_state_stride,
                       const int32_t *query_start_loc, const int32_t *cache_indices,
                       const int8_t *has_initial_state, int pad_slot_id, int api_mode,
                       int silu);

void orc_rotary_embedding(const int64_t *positions, const uint16_t *query, const uint16_t *key,
                          float *query_out, float *key_out,
                          int num_tokens, int num_heads, int num_kv_heads, int head_size,
                          int rot_dim, long long query_stride, long long key_stride,
                          const float *cos_sin_cache, int max_position, float base,
                          int is_neox, int dtype);

void orc_gemv(const uint16_t *weight, const uint16_t *x, float *y,
              int batch, int n, int k, int dtype);

void orc_gemv_int8(const int8_t *weight, const uint16_t *scales, const uint16_t *x, float *y,
                   int batch, int n, int k);

/* Input generation of the reference's C++ op tests
 * (test/src/case/pb_tools.h:123-200, pb_tools.cpp:854-900): libstdc++'s
 * std::default_random_engine (minstd_rand0: x <- 16807 x mod 2^31-1) driving
 * uniform_real_distribution<double> and normal_distribution<double> (both
 * through generate_canonical<double, 53>: two draws per canonical value) or,
 * for bf16 tensors, uniform_real_distribution<float> (one draw).  One call
 * is one serial chunk with its own seed. */
uint32_t orc_minstd_nth(long long seed, size_t n);
void orc_harness_uniform(long long seed, size_t n, double lo, double hi, double *out);
void orc_harness_normal(long long seed, size_t n, double mu, double sigma, double *out);
void orc_harness_uniform_f32(long long seed, size_t n, float lo, float hi, float *out);

#ifdef __cplusplus
}
#endif

#endif  /* TECOOPS_ORACLE_H_ */
