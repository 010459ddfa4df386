/*
 * oracle.c -- scalar CPU restatement of RustLLM's memory-bound tensor ops.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Built by oracle/Makefile with
 * -ffp-contract=off so that a*b-c is two roundings, as in the reference
 * shaders' float expressions.
 *
 * Reference files followed (paths relative to the Lee-Dongwook/RustLLM root):
 *   kernels/vector_add.metal, mul.metal, silu.metal, cast.metal,
 *   contiguous.metal, repeat_kv.metal, rmsnorm.metal, softmax.metal,
 *   attention_scale_mask.metal, rope.metal, embedding.metal,
 *   kv_cache_write.metal; src/nn/rope.rs (cos/sin table);
 *   src/ops/rmsnorm.rs (the test's cpu_rmsnorm).
 */
#include "oracle.h"

#include <math.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void oracle_set_threads(int threads) { g_threads = threads < 1 ? 1 : threads; }
int oracle_get_threads(void) { return g_threads; }

#define PAR_FOR _Pragma("omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)")

/* ---------------------------------------------------------------- f16 <-> f32 */

/* IEEE 754 binary32 -> binary16, round to nearest, ties to even.  The MSL
 * conversion half(float) used by cast.metal:10 and every f16 kernel rounds
 * this way; the Rust side uses half 2.7.1 f16::from_f32, also RNE. */
uint16_t oracle_f32_to_f16(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof x);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;

    if (exp == 0xffu) {
        if (mant == 0) return (uint16_t)(sign | 0x7c00u);          /* +-inf */
        return (uint16_t)(sign | 0x7e00u | (mant >> 13));          /* quiet NaN */
    }
    int e = (int)exp - 112; /* rebias 127 -> 15 */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);                /* overflow */
    if (e <= 0) {
        /* binary16 subnormal (or zero): value = full * 2^(exp-150), and one
         * subnormal ulp is 2^-24, so the quotient is full >> (126 - exp). */
        if (exp == 0) return (uint16_t)sign; /* f32 zero/subnormal < 2^-126 */
        uint32_t full = mant | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        if (shift > 24) return (uint16_t)sign;
        uint32_t q = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u; /* may carry to inf */
    return (uint16_t)(sign | q);
}

float oracle_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)bits >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)bits & 0x3ffu;
    uint32_t out;
    if (exp == 0) {
        if (mant == 0) {
            out = sign;
        } else {
            float v = (float)mant * 5.9604644775390625e-8f; /* 2^-24, exact */
            memcpy(&out, &v, sizeof out);
            out |= sign;
        }
    } else if (exp == 31) {
        out = sign | 0x7f800000u | (mant << 13);
    } else {
        out = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &out, sizeof f);
    return f;
}

void oracle_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
    PAR_FOR
    for (size_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

void oracle_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    PAR_FOR
    for (size_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}

#define H2F(v) oracle_f16_to_f32(v)
#define F2H(v) oracle_f32_to_f16(v)

/* ----------------------------------------------------------- element-wise */

/* vector_add.metal:5-12 */
void oracle_add_f32(const float* a, const float* b, float* out, size_t n) {
    PAR_FOR
    for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* vector_add.metal:14-21: half(float(a) + float(b)) */
void oracle_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t n) {
    PAR_FOR
    for (size_t i = 0; i < n; ++i) out[i] = F2H(H2F(a[i]) + H2F(b[i]));
}

/* mul.metal:5-20 */
void oracle_mul_f32(const float* a, const float* b, float* out, size_t n) {
    PAR_FOR
    for (size_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}

/* mul.metal:22-36: half(float(a) * float(b)) */
void oracle_mul_f16(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t n) {
    PAR_FOR
    for (size_t i = 0; i < n; ++i) out[i] = F2H(H2F(a[i]) * H2F(b[i]));
}

/* silu.metal:17-23: sigmoid = 1/(1+exp(-x)); out = x * sigmoid */
static inline float silu_f32_expr(float x) {
    float sigmoid = 1.0f / (1.0f + expf(-x));
    return x * sigmoid;
}

/* silu.metal:31-35 (f16 kernel uses a different formula): x / (1 + exp(-x)) */
static inline float silu_f16_expr(float x) { return x / (1.0f + expf(-x)); }

void oracle_silu_f32(const float* in, float* out, size_t n) {
    PAR_FOR
    for (size_t i = 0; i < n; ++i) out[i] = silu_f32_expr(in[i]);
}

void oracle_silu_f16(const uint16_t* in, uint16_t* out, size_t n) {
    PAR_FOR
    for (size_t i = 0; i < n; ++i) out[i] = F2H(silu_f16_expr(H2F(in[i])));
}

/* silu.metal:38-46: half((x / (1 + exp(-x))) * float(up)), one rounding */
void oracle_swiglu_f16(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n) {
    PAR_FOR
    for (size_t i = 0; i < n; ++i) out[i] = F2H(silu_f16_expr(H2F(gate[i])) * H2F(up[i]));
}

/* src/nn/swiglu.rs:15-37, F32 branch: silu_f32 then mul_f32 (float intermediate). */
void oracle_swiglu_f32(const float* gate, const float* up, float* out, size_t n) {
    PAR_FOR
    for (size_t i = 0; i < n; ++i) out[i] = silu_f32_expr(gate[i]) * up[i];
}

/* cast.metal:5-11 */
void oracle_cast_f32_to_f16(const float* in, uint16_t* out, size_t n) {
    oracle_f32_to_f16_array(in, out, n);
}

/* cast.metal:13-19 */
void oracle_cast_f16_to_f32(const uint16_t* in, float* out, size_t n) {
    oracle_f16_to_f32_array(in, out, n);
}

/* A [cols] bias broadcast over rows through a stride-0 view: the reference
 * semantics are contiguous.metal:21-34 on the view (stride 0 repeats the
 * bias) followed by vector_add.metal. */
void oracle_add_broadcast_f32(const float* x, const float* bias, float* out, size_t rows,
                              size_t cols) {
    PAR_FOR
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) out[r * cols + c] = x[r * cols + c] + bias[c];
}

void oracle_add_broadcast_f16(const uint16_t* x, const uint16_t* bias, uint16_t* out,
                              size_t rows, size_t cols) {
    PAR_FOR
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c)
            out[r * cols + c] = F2H(H2F(x[r * cols + c]) + H2F(bias[c]));
}

/* ------------------------------------------------------------ data movement */

/* contiguous.metal:21-34: peel coordinates from the last dimension. */
void oracle_contiguous(const void* src, void* dst, const uint64_t* dims, const uint64_t* strides,
                       uint32_t rank, size_t element_size) {
    size_t numel = 1;
    for (uint32_t d = 0; d < rank; ++d) numel *= (size_t)dims[d];
    const unsigned char* s = (const unsigned char*)src;
    unsigned char* o = (unsigned char*)dst;
    PAR_FOR
    for (size_t id = 0; id < numel; ++id) {
        size_t remaining = id;
        size_t source_index = 0;
        for (int d = (int)rank - 1; d >= 0; --d) {
            size_t coord = remaining % (size_t)dims[d];
            remaining /= (size_t)dims[d];
            source_index += coord * (size_t)strides[d];
        }
        memcpy(o + id * element_size, s + source_index * element_size, element_size);
    }
}

/* repeat_kv.metal:16-30: out[b, h, s, d] = in[b, h / repeats, s, d]. */
void oracle_repeat_kv(const void* in, void* out, size_t batch, size_t kv_heads, size_t seq_len,
                      size_t head_dim, size_t repeats, size_t element_size) {
    size_t query_heads = kv_heads * repeats;
    size_t numel = batch * query_heads * seq_len * head_dim;
    const unsigned char* s = (const unsigned char*)in;
    unsigned char* o = (unsigned char*)out;
    PAR_FOR
    for (size_t index = 0; index < numel; ++index) {
        size_t d = index % head_dim;
        size_t temp = index / head_dim;
        size_t seq = temp % seq_len;
        temp /= seq_len;
        size_t query_head = temp % query_heads;
        size_t b = temp / query_heads;
        size_t kv_head = query_head / repeats;
        size_t input_index = ((b * kv_heads + kv_head) * seq_len + seq) * head_dim + d;
        memcpy(o + index * element_size, s + input_index * element_size, element_size);
    }
}

/* embedding.metal:5-34: out[t, h] = weight[ids[t], h]. */
void oracle_embedding(const void* weight, const uint32_t* ids, void* out, size_t tokens,
                      size_t hidden, size_t element_size) {
    const unsigned char* w = (const unsigned char*)weight;
    unsigned char* o = (unsigned char*)out;
    PAR_FOR
    for (size_t t = 0; t < tokens; ++t)
        memcpy(o + t * hidden * element_size, w + (size_t)ids[t] * hidden * element_size,
               hidden * element_size);
}

/* kv_cache_write.metal:4-19: cache[(head*max_seq + start + seq)*D + d] = src[id]. */
void oracle_kv_cache_write(void* cache, const void* src, size_t heads, size_t src_seq,
                           size_t max_seq, size_t head_dim, size_t start, size_t element_size) {
    const unsigned char* s = (const unsigned char*)src;
    unsigned char* c = (unsigned char*)cache;
    size_t rows = heads * src_seq;
    PAR_FOR
    for (size_t row = 0; row < rows; ++row) {
        size_t seq = row % src_seq;
        size_t head = row / src_seq;
        memcpy(c + ((head * max_seq + start + seq) * head_dim) * element_size,
               s + row * head_dim * element_size, head_dim * element_size);
    }
}

/* ---------------------------------------------------------------- RMSNorm */

/* rmsnorm.metal:20-68 (f32) and :84-125 (f16): mean_square = sum(x^2)/h,
 * inv = rsqrt(mean_square + eps), y = x * inv * w.  The sum and inv are
 * formed in double and inv is rounded to float once. */
static inline float rms_inverse(double sum_sq, size_t hidden, float eps) {
    double mean_square = sum_sq / (double)hidden;
    return (float)(1.0 / sqrt(mean_square + (double)eps));
}

void oracle_rmsnorm_f32(const float* in, const float* weight, float* out, size_t rows,
                        size_t hidden, float eps) {
    PAR_FOR
    for (size_t r = 0; r < rows; ++r) {
        const float* x = in + r * hidden;
        double acc = 0.0;
        for (size_t i = 0; i < hidden; ++i) acc += (double)x[i] * (double)x[i];
        float inv = rms_inverse(acc, hidden, eps);
        for (size_t i = 0; i < hidden; ++i) out[r * hidden + i] = x[i] * inv * weight[i];
    }
}

void oracle_rmsnorm_f16(const uint16_t* in, const uint16_t* weight, uint16_t* out, size_t rows,
                        size_t hidden, float eps) {
    PAR_FOR
    for (size_t r = 0; r < rows; ++r) {
        const uint16_t* x = in + r * hidden;
        double acc = 0.0;
        for (size_t i = 0; i < hidden; ++i) {
            double v = (double)H2F(x[i]);
            acc += v * v;
        }
        float inv = rms_inverse(acc, hidden, eps);
        for (size_t i = 0; i < hidden; ++i)
            out[r * hidden + i] = F2H(H2F(x[i]) * inv * H2F(weight[i]));
    }
}

/* src/ops/rmsnorm.rs:286-319 (cpu_rmsnorm in the reference's tests), literally:
 * float sum in index order, 1/sqrt(mean + eps), input * inv * weight. */
void oracle_cpu_rmsnorm_literal(const float* in, const float* weight, float* out, size_t rows,
                                size_t hidden, float eps) {
    for (size_t r = 0; r < rows; ++r) {
        const float* x = in + r * hidden;
        float sum = 0.0f;
        for (size_t i = 0; i < hidden; ++i) sum += x[i] * x[i];
        float mean_square = sum / (float)hidden;
        float inv_rms = 1.0f / sqrtf(mean_square + eps);
        for (size_t i = 0; i < hidden; ++i) out[r * hidden + i] = x[i] * inv_rms * weight[i];
    }
}

/* Residual add then RMSNorm, as the two adjacent calls in
 * src/nn/transformer_block.rs:148-152 (add_encode, then rmsnorm on the sum). */
void oracle_add_rmsnorm_f32(const float* x, const float* residual, const float* weight,
                            float* sum_out, float* norm_out, size_t rows, size_t hidden,
                            float eps) {
    oracle_add_f32(x, residual, sum_out, rows * hidden);
    oracle_rmsnorm_f32(sum_out, weight, norm_out, rows, hidden, eps);
}

void oracle_add_rmsnorm_f16(const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                            uint16_t* sum_out, uint16_t* norm_out, size_t rows, size_t hidden,
                            float eps) {
    oracle_add_f16(x, residual, sum_out, rows * hidden);
    oracle_rmsnorm_f16(sum_out, weight, norm_out, rows, hidden, eps);
}

/* ---------------------------------------------------------------- softmax */

/* softmax.metal:25-131: row max (fmax semantics), sum of exp(x - max),
 * out = exp(x - max) / sum.  A row whose max is -inf therefore yields NaN
 * in f32, exactly as the reference kernel (no guard in the f32 kernel). */
void oracle_softmax_f32(const float* in, float* out, size_t rows, size_t width) {
    PAR_FOR
    for (size_t r = 0; r < rows; ++r) {
        const float* x = in + r * width;
        float m = -INFINITY;
        for (size_t i = 0; i < width; ++i) m = fmaxf(m, x[i]);
        double sum = 0.0;
        for (size_t i = 0; i < width; ++i) sum += (double)expf(x[i] - m);
        for (size_t i = 0; i < width; ++i)
            out[r * width + i] = (float)((double)expf(x[i] - m) / sum);
    }
}

/* softmax.metal:147-194: as f32 on the widened values, but a row whose max is
 * -inf is written as zeros (:166-173). */
void oracle_softmax_f16(const uint16_t* in, uint16_t* out, size_t rows, size_t width) {
    PAR_FOR
    for (size_t r = 0; r < rows; ++r) {
        const uint16_t* x = in + r * width;
        float m = -INFINITY;
        for (size_t i = 0; i < width; ++i) m = fmaxf(m, H2F(x[i]));
        if (isinf(m) && m < 0.0f) {
            for (size_t i = 0; i < width; ++i) out[r * width + i] = 0;
            continue;
        }
        double sum = 0.0;
        for (size_t i = 0; i < width; ++i) sum += (double)expf(H2F(x[i]) - m);
        for (size_t i = 0; i < width; ++i)
            out[r * width + i] = F2H((float)((double)expf(H2F(x[i]) - m) / sum));
    }
}

/* attention_scale_mask.metal:21-41 (f32) and :62-70 (f16): a key past the
 * query's absolute position is -inf, everything else is x * scale in f32. */
void oracle_scale_mask_f32(const float* in, float* out, size_t numel, float scale,
                           size_t query_len, size_t key_len, size_t start) {
    PAR_FOR
    for (size_t id = 0; id < numel; ++id) {
        size_t key_index = id % key_len;
        size_t query_index = (id / key_len) % query_len;
        out[id] = key_index > start + query_index ? -INFINITY : in[id] * scale;
    }
}

void oracle_scale_mask_f16(const uint16_t* in, uint16_t* out, size_t numel, float scale,
                           size_t query_len, size_t key_len, size_t start) {
    PAR_FOR
    for (size_t id = 0; id < numel; ++id) {
        size_t key_index = id % key_len;
        size_t query_index = (id / key_len) % query_len;
        out[id] = key_index > start + query_index ? (uint16_t)0xfc00u : F2H(H2F(in[id]) * scale);
    }
}

/* ------------------------------------------------------------------- RoPE */

/* rope.metal:23-63 (f32) and :82-96 (f16): for pair (i, i + D/2) of row r,
 * position = r % seq_len + start, (a, b) -> (a*c - b*s, b*c + a*s). */
void oracle_rope_f32(const float* in, const float* cos_table, const float* sin_table, float* out,
                     size_t numel, size_t seq_len, size_t head_dim, size_t start) {
    size_t half_dim = head_dim / 2;
    size_t total_pairs = numel / head_dim * half_dim;
    PAR_FOR
    for (size_t id = 0; id < total_pairs; ++id) {
        size_t pair_index = id % half_dim;
        size_t row = id / half_dim;
        size_t position = row % seq_len;
        size_t base = row * head_dim;
        size_t table_index = (start + position) * half_dim + pair_index;
        float c = cos_table[table_index], s = sin_table[table_index];
        float first = in[base + pair_index], second = in[base + half_dim + pair_index];
        out[base + pair_index] = first * c - second * s;
        out[base + half_dim + pair_index] = second * c + first * s;
    }
}

void oracle_rope_f16(const uint16_t* in, const float* cos_table, const float* sin_table,
                     uint16_t* out, size_t numel, size_t seq_len, size_t head_dim, size_t start) {
    size_t half_dim = head_dim / 2;
    size_t total_pairs = numel / head_dim * half_dim;
    PAR_FOR
    for (size_t id = 0; id < total_pairs; ++id) {
        size_t pair_index = id % half_dim;
        size_t row = id / half_dim;
        size_t position = row % seq_len;
        size_t base = row * head_dim;
        size_t table_index = (start + position) * half_dim + pair_index;
        float c = cos_table[table_index], s = sin_table[table_index];
        float first = H2F(in[base + pair_index]), second = H2F(in[base + half_dim + pair_index]);
        out[base + pair_index] = F2H(first * c - second * s);
        out[base + half_dim + pair_index] = F2H(second * c + first * s);
    }
}

/* src/nn/rope.rs:44-62, in float: exponent = (2i)/D, inv = 1/theta^exponent,
 * angle = position * inv, table = cos/sin(angle). */
void oracle_rope_table(size_t head_dim, size_t max_seq_len, float theta, float* cos_table,
                       float* sin_table) {
    size_t half_dim = head_dim / 2;
    for (size_t position = 0; position < max_seq_len; ++position) {
        for (size_t i = 0; i < half_dim; ++i) {
            float exponent = (float)(2 * i) / (float)head_dim;
            float inverse_frequency = 1.0f / powf(theta, exponent);
            float angle = (float)position * inverse_frequency;
            cos_table[position * half_dim + i] = cosf(angle);
            sin_table[position * half_dim + i] = sinf(angle);
        }
    }
}

/* ------------------------------------------------------ GQA attention core */

/* gqa_matmul.metal:7-161 (f32) and :163-322 (f16): one thread per score;
 * kv_head = q_head / (q_heads / kv_heads) (:25-38); K rows of a head are
 * kv_capacity apart (:59-65); the dot product runs over d in order (16-wide
 * tiles, each summed in order, :75-140) in float32, f16 products widened first
 * (:287-295), and the f16 score is rounded once at the store (:319). */
void oracle_gqa_qk_f32(const float* q, const float* k, float* out, size_t batch,
                       size_t q_heads, size_t kv_heads, size_t q_len, size_t kv_len,
                       size_t head_dim, size_t kv_capacity) {
    size_t groups = q_heads / kv_heads;
    size_t rows = batch * q_heads * q_len;
    PAR_FOR
    for (size_t row = 0; row < rows; ++row) {
        size_t flat_head = row / q_len, query = row % q_len;
        size_t b = flat_head / q_heads, kv_head = (flat_head % q_heads) / groups;
        const float* qr = q + (flat_head * q_len + query) * head_dim;
        const float* kh = k + (b * kv_heads + kv_head) * kv_capacity * head_dim;
        for (size_t key = 0; key < kv_len; ++key) {
            float sum = 0.0f;
            for (size_t d = 0; d < head_dim; ++d) sum += qr[d] * kh[key * head_dim + d];
            out[row * kv_len + key] = sum;
        }
    }
}

void oracle_gqa_qk_f16(const uint16_t* q, const uint16_t* k, uint16_t* out, size_t batch,
                       size_t q_heads, size_t kv_heads, size_t q_len, size_t kv_len,
                       size_t head_dim, size_t kv_capacity) {
    size_t groups = q_heads / kv_heads;
    size_t rows = batch * q_heads * q_len;
    PAR_FOR
    for (size_t row = 0; row < rows; ++row) {
        size_t flat_head = row / q_len, query = row % q_len;
        size_t b = flat_head / q_heads, kv_head = (flat_head % q_heads) / groups;
        const uint16_t* qr = q + (flat_head * q_len + query) * head_dim;
        const uint16_t* kh = k + (b * kv_heads + kv_head) * kv_capacity * head_dim;
        for (size_t key = 0; key < kv_len; ++key) {
            float sum = 0.0f;
            for (size_t d = 0; d < head_dim; ++d) sum += H2F(qr[d]) * H2F(kh[key * head_dim + d]);
            out[row * kv_len + key] = F2H(sum);
        }
    }
}

/* gqa_matmul.metal:323-474 (f32) and :475-629 (f16): out[b,h,i,d] =
 * sum over keys j in order of p[b,h,i,j] * v[b,h/g,j,d] in float32, V rows
 * kv_capacity apart per head (:372-378); f16 rounded once at the store. */
void oracle_gqa_pv_f32(const float* probs, const float* v, float* out, size_t batch,
                       size_t q_heads, size_t kv_heads, size_t q_len, size_t kv_len,
                       size_t head_dim, size_t kv_capacity) {
    size_t groups = q_heads / kv_heads;
    size_t rows = batch * q_heads * q_len;
    PAR_FOR
    for (size_t row = 0; row < rows; ++row) {
        size_t flat_head = row / q_len;
        size_t b = flat_head / q_heads, kv_head = (flat_head % q_heads) / groups;
        const float* pr = probs + row * kv_len;
        const float* vh = v + (b * kv_heads + kv_head) * kv_capacity * head_dim;
        for (size_t d = 0; d < head_dim; ++d) {
            float sum = 0.0f;
            for (size_t key = 0; key < kv_len; ++key) sum += pr[key] * vh[key * head_dim + d];
            out[row * head_dim + d] = sum;
        }
    }
}

void oracle_gqa_pv_f16(const uint16_t* probs, const uint16_t* v, uint16_t* out, size_t batch,
                       size_t q_heads, size_t kv_heads, size_t q_len, size_t kv_len,
                       size_t head_dim, size_t kv_capacity) {
    size_t groups = q_heads / kv_heads;
    size_t rows = batch * q_heads * q_len;
    PAR_FOR
    for (size_t row = 0; row < rows; ++row) {
        size_t flat_head = row / q_len;
        size_t b = flat_head / q_heads, kv_head = (flat_head % q_heads) / groups;
        const uint16_t* pr = probs + row * kv_len;
        const uint16_t* vh = v + (b * kv_heads + kv_head) * kv_capacity * head_dim;
        for (size_t d = 0; d < head_dim; ++d) {
            float sum = 0.0f;
            for (size_t key = 0; key < kv_len; ++key)
                sum += H2F(pr[key]) * H2F(vh[key * head_dim + d]);
            out[row * head_dim + d] = F2H(sum);
        }
    }
}
