/*
 * oracle.h -- CPU restatement of RustLLM's memory-bound tensor ops.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP
 * library's results are compared against.  Only tests/, the smoke() entry of
 * __graft_entry__.py and the cpu_baseline leg of bench.py may load it; the
 * product (rustllm_amd/) never links, loads or falls back to it.
 *
 * Each function restates the scalar semantics of one reference kernel
 * (kernels/<op>.metal in Lee-Dongwook/RustLLM) and cites the file:line it
 * follows.  Element-wise arithmetic is done in float32 in the same operation
 * order as the reference, with FMA contraction disabled at build time, so the
 * single-rounding ops (add, mul, cast, scale/mask, RoPE) are exact
 * restatements.  Row reductions (RMSNorm sum of squares, softmax sum) are
 * accumulated in double: the reference sums float partials in a 256-way
 * shared-memory tree whose order no scalar loop reproduces, so the oracle
 * uses the exact-sum limit and the tests apply the stated tolerance.
 *
 * f16 values are passed as their IEEE binary16 bit patterns (uint16_t).
 */
#ifndef RUSTLLM_ORACLE_H
#define RUSTLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32.  f32->f16 rounds to nearest, ties to even,
 * keeps subnormals, saturates to +-inf on overflow and keeps NaN a NaN. */
uint16_t oracle_f32_to_f16(float value);
float oracle_f16_to_f32(uint16_t bits);
void oracle_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void oracle_f16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* Threads used by the loops below (1 = the literal scalar restatement). */
void oracle_set_threads(int threads);
int oracle_get_threads(void);

void oracle_add_f32(const float* a, const float* b, float* out, size_t n);
void oracle_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t n);
void oracle_mul_f32(const float* a, const float* b, float* out, size_t n);
void oracle_mul_f16(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t n);
void oracle_silu_f32(const float* in, float* out, size_t n);
void oracle_silu_f16(const uint16_t* in, uint16_t* out, size_t n);
void oracle_swiglu_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n);
void oracle_swiglu_f32(const float* gate, const float* up, float* out, size_t n);
void oracle_cast_f32_to_f16(const float* in, uint16_t* out, size_t n);
void oracle_cast_f16_to_f32(const uint16_t* in, float* out, size_t n);
void oracle_add_broadcast_f32(const float* x, const float* bias, float* out, size_t rows,
                              size_t cols);
void oracle_add_broadcast_f16(const uint16_t* x, const uint16_t* bias, uint16_t* out,
                              size_t rows, size_t cols);

/* Strided gather of element_size-byte elements: dst[i] = src[sum coord_d * stride_d]. */
void oracle_contiguous(const void* src, void* dst, const uint64_t* dims, const uint64_t* strides,
                       uint32_t rank, size_t element_size);
void oracle_repeat_kv(const void* in, void* out, size_t batch, size_t kv_heads, size_t seq_len,
                      size_t head_dim, size_t repeats, size_t element_size);

void oracle_rmsnorm_f32(const float* in, const float* weight, float* out, size_t rows,
                        size_t hidden, float eps);
void oracle_rmsnorm_f16(const uint16_t* in, const uint16_t* weight, uint16_t* out, size_t rows,
                        size_t hidden, float eps);
/* The reference test's own CPU oracle, literally: float accumulation in index order. */
void oracle_cpu_rmsnorm_literal(const float* in, const float* weight, float* out, size_t rows,
                                size_t hidden, float eps);
void oracle_add_rmsnorm_f32(const float* x, const float* residual, const float* weight,
                            float* sum_out, float* norm_out, size_t rows, size_t hidden,
                            float eps);
void oracle_add_rmsnorm_f16(const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                            uint16_t* sum_out, uint16_t* norm_out, size_t rows, size_t hidden,
                            float eps);

void oracle_softmax_f32(const float* in, float* out, size_t rows, size_t width);
void oracle_softmax_f16(const uint16_t* in, uint16_t* out, size_t rows, size_t width);
void oracle_scale_mask_f32(const float* in, float* out, size_t numel, float scale,
                           size_t query_len, size_t key_len, size_t start);
void oracle_scale_mask_f16(const uint16_t* in, uint16_t* out, size_t numel, float scale,
                           size_t query_len, size_t key_len, size_t start);

void oracle_rope_f32(const float* in, const float* cos_table, const float* sin_table, float* out,
                     size_t numel, size_t seq_len, size_t head_dim, size_t start);
void oracle_rope_f16(const uint16_t* in, const float* cos_table, const float* sin_table,
                     uint16_t* out, size_t numel, size_t seq_len, size_t head_dim, size_t start);
void oracle_rope_table(size_t head_dim, size_t max_seq_len, float theta, float* cos_table,
                       float* sin_table);

/* Row gather out[t, :] = weight[ids[t], :] and KV-cache scatter. */
void oracle_embedding(const void* weight, const uint32_t* ids, void* out, size_t tokens,
                      size_t hidden, size_t element_size);
void oracle_kv_cache_write(void* cache, const void* src, size_t heads, size_t src_seq,
                           size_t max_seq, size_t head_dim, size_t start, size_t element_size);

/* Grouped-query matmuls of the attention core.  q and probs are contiguous
 * [B, QH, Q, D] / [B, QH, Q, K]; k and v hold kv_capacity rows per KV head
 * ([B, KVH, kv_capacity, D], the first kv_len used); query head h reads KV
 * head h / (QH / KVH).  Sums run in float32 in index order. */
void oracle_gqa_qk_f32(const float* q, const float* k, float* out, size_t batch,
                       size_t q_heads, size_t kv_heads, size_t q_len, size_t kv_len,
                       size_t head_dim, size_t kv_capacity);
void oracle_gqa_qk_f16(const uint16_t* q, const uint16_t* k, uint16_t* out, size_t batch,
                       size_t q_heads, size_t kv_heads, size_t q_len, size_t kv_len,
                       size_t head_dim, size_t kv_capacity);
void oracle_gqa_pv_f32(const float* probs, const float* v, float* out, size_t batch,
                       size_t q_heads, size_t kv_heads, size_t q_len, size_t kv_len,
                       size_t head_dim, size_t kv_capacity);
void oracle_gqa_pv_f16(const uint16_t* probs, const uint16_t* v, uint16_t* out, size_t batch,
                       size_t q_heads, size_t kv_heads, size_t q_len, size_t kv_len,
                       size_t head_dim, size_t kv_capacity);

#ifdef __cplusplus
}
#endif

#endif
