/*
 * rustllm_hip.h -- C ABI of the MI355X (gfx950) tensor-op library.
 *
 * This is the drop-in boundary under RustLLM's `src/ops` / `src/tensor`
 * API: every entry point below replaces one Metal-side item of
 * Lee-Dongwook/RustLLM, cited as file:line relative to that repository.
 * The Rust side binds these with an `extern "C"` block and keeps its public
 * signatures; the C++ mirror in rustllm_amd/host/ is the same layer
 * restated in C++.
 *
 * Conventions
 *  - Every fallible call returns an rl_status (0 = RL_OK).  The codes map
 *    one-to-one onto the TinyError variants the op layer can raise
 *    (src/error.rs:4-43); RL_ERR_DEVICE stands in for TinyError::Metal.
 *    rl_last_error_message() returns the thread's message for the last
 *    failure.
 *  - Validation runs before anything is enqueued and has no side effects,
 *    in the reference's order (e.g. src/ops/softmax.rs:91-108).  An op called
 *    with ctx == NULL validates its arguments and then returns
 *    RL_ERR_DEVICE, so argument checking is testable without a GPU.
 *  - Ops are the `_encode` twins: they enqueue on the context's stream and
 *    return without waiting.  rl_execution_finish() is the commit + wait of
 *    MetalExecution::finish (src/metal/execution.rs:30-36).  The synchronous
 *    reference ops (e.g. ops::add_f32, src/ops/add.rs:8-16) are
 *    begin + op + finish.
 *  - Output buffers are passed in by the caller, allocated with
 *    rl_buffer_empty() exactly where the reference calls MetalBuffer::empty /
 *    empty_with_element_size (src/metal/buffer.rs:111-142).  Each op checks
 *    the output's len and byte_len.  The reference always writes a fresh
 *    buffer; here an output may also be the very buffer of an input (same
 *    data pointer and length) for add, mul, SiLU, SwiGLU, the bias add,
 *    RMSNorm and add + RMSNorm, softmax, scale/mask and the fused scale/mask
 *    + softmax, and RoPE -- each reads all it writes first.  For every other
 *    op, and for outputs that overlap an input only in part, the output must
 *    not overlap the inputs.
 *  - f16 is IEEE binary16.  All arithmetic is float32; f16 results are
 *    rounded to nearest even.
 *  - One context per thread; a context is not thread-safe (MetalContext is
 *    !Sync, src/metal/context.rs:14-17).  All work of a context runs in
 *    order on its one stream.
 */
#ifndef RUSTLLM_HIP_H
#define RUSTLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ status codes */
typedef int32_t rl_status;
#define RL_OK 0
#define RL_ERR_INVALID_ARGUMENT 1      /* TinyError::InvalidArgument      src/error.rs:5   */
#define RL_ERR_INVALID_SHAPE 2         /* TinyError::InvalidShape         src/error.rs:6   */
#define RL_ERR_SHAPE_MISMATCH 3        /* TinyError::ShapeMismatch        src/error.rs:7-10 */
#define RL_ERR_INVALID_DIMENSION 4     /* TinyError::InvalidDimension     src/error.rs:11  */
#define RL_ERR_UNSUPPORTED_DTYPE 5     /* TinyError::UnsupportedDType     src/error.rs:18  */
#define RL_ERR_NON_CONTIGUOUS 6        /* TinyError::NonContiguousTensor  src/error.rs:19  */
#define RL_ERR_POSITION_OUT_OF_RANGE 7 /* TinyError::PositionOutOfRange   src/error.rs:20-24 */
#define RL_ERR_MODEL_FORMAT 8          /* TinyError::ModelFormat          src/error.rs:32  */
#define RL_ERR_DEVICE 9                /* TinyError::Metal                src/error.rs:38  */
#define RL_ERR_INVALID_TOKEN_ID 10     /* TinyError::InvalidTokenId       src/error.rs:13-16 */

/* --------------------------------------------------------------- handles */
typedef struct rl_context rl_context; /* MetalContext   src/metal/context.rs:10-18 */
typedef struct rl_graph rl_graph;     /* a recorded command buffer, replayable */
typedef struct rl_event rl_event;     /* a stream timestamp */

/* A device buffer.  Same three fields as MetalBuffer (src/metal/buffer.rs:8-12):
 * `len` is the element count, `byte_len` the size in bytes. */
typedef struct rl_buffer {
    void* data;
    uint64_t len;
    uint64_t byte_len;
} rl_buffer;

/* Submission counters: MetalDecodeProfile, src/profile.rs:7-16. */
typedef struct rl_profile {
    uint64_t command_buffers;
    uint64_t compute_encoders;
    uint64_t kernel_dispatches;
    uint64_t commits;
    uint64_t waits;
    uint64_t buffer_allocations;
    uint64_t allocated_bytes;
} rl_profile;

/* ---------------------------------------------------------------- errors */
/* Message of the calling thread's last failure ("" if none). */
const char* rl_last_error_message(void);

/* The integer fields of the TinyError variants that carry data
 * (src/error.rs:7-24), for the calling thread's last failure.  `code` is
 * that failure's status (RL_OK if none) and selects which fields are set;
 * the others are zero.
 *  - RL_ERR_SHAPE_MISMATCH: TinyError::ShapeMismatch { left, right }
 *    (raised by the buffer ops as in src/tensor/elementwise.rs:119-124 and
 *    src/ops/rmsnorm.rs:232-237): left_rank/left and right_rank/right.
 *  - RL_ERR_POSITION_OUT_OF_RANGE: TinyError::PositionOutOfRange
 *    { start_pos, seq_len, max_seq_len } (src/ops/kv_cache_write.rs:101-110).
 *  - RL_ERR_INVALID_TOKEN_ID: TinyError::InvalidTokenId { token_id,
 *    vocab_size } (src/ops/embedding.rs:129-136).
 * Shapes of more than RL_ERROR_MAX_RANK dims keep their first
 * RL_ERROR_MAX_RANK dims; the rank fields hold the full rank. */
#define RL_ERROR_MAX_RANK 16
typedef struct rl_error_payload {
    rl_status code;
    uint32_t left_rank;
    uint32_t right_rank;
    uint32_t token_id;
    uint64_t left[RL_ERROR_MAX_RANK];
    uint64_t right[RL_ERROR_MAX_RANK];
    uint64_t start_pos;
    uint64_t seq_len;
    uint64_t max_seq_len;
    uint64_t vocab_size;
} rl_error_payload;
/* Copies the calling thread's last failure payload to *out and returns its
 * code (RL_OK if the thread has no failure recorded, or out is NULL). */
rl_status rl_last_error_payload(rl_error_payload* out);
/* Library version string. */
const char* rl_version(void);

/* --------------------------------------------------------------- context */
/* MetalContext::new (src/metal/context.rs:27-44): opens `device` and makes one
 * in-order stream at the default priority. */
rl_status rl_context_create(int32_t device, rl_context** out);
/* As rl_context_create, but enqueues on an existing HIP stream (hipStream_t
 * passed as void*).  The stream stays owned by the caller. */
rl_status rl_context_create_on_stream(int32_t device, void* stream, rl_context** out);
/* Frees pooled memory and the stream; buffers still held become invalid. */
void rl_context_destroy(rl_context* ctx);
/* The hipStream_t the context enqueues on. */
void* rl_context_stream(const rl_context* ctx);
/* Number of visible devices (0 when no GPU is present). */
int32_t rl_device_count(void);

/* ---------------------------------------------------------------- buffers */
/* MetalBuffer::empty_with_element_size (src/metal/buffer.rs:127-142): `len`
 * elements of `element_size` bytes from the context's stream-ordered pool.
 * Contents are undefined.  len and element_size must be > 0. */
rl_status rl_buffer_empty(rl_context* ctx, uint64_t len, uint64_t element_size, rl_buffer* out);
/* MetalBuffer::from_slice / from_f16_slice (src/metal/buffer.rs:15-34,57-73):
 * allocate and copy `len` elements from host memory; returns after the copy. */
rl_status rl_buffer_from_host(rl_context* ctx, const void* host, uint64_t len,
                              uint64_t element_size, rl_buffer* out);
/* MetalBuffer::as_slice / as_f16_slice (src/metal/buffer.rs:160-169): waits for
 * the stream, then copies `byte_len` bytes to host memory. */
rl_status rl_buffer_to_host(rl_context* ctx, const rl_buffer* buffer, void* host,
                            uint64_t byte_len);
/* Stream-ordered copy of `byte_len` bytes between device buffers. */
rl_status rl_buffer_copy(rl_context* ctx, const rl_buffer* src, const rl_buffer* dst,
                         uint64_t byte_len);
/* Drop of MetalBuffer: returns the block to the pool (stream-ordered reuse)
 * and zeroes *buffer. */
void rl_buffer_release(rl_context* ctx, rl_buffer* buffer);
/* Returns unused pooled blocks to the device. */
rl_status rl_context_trim(rl_context* ctx);

/* ------------------------------------------------------------- execution */
/* MetalExecution::new (src/metal/execution.rs:11-20): opens a batch; ops
 * enqueued until finish form one submission. */
rl_status rl_execution_begin(rl_context* ctx);
/* MetalExecution::finish (src/metal/execution.rs:30-36): waits for every
 * enqueued op and reports any device error (the reference never checks). */
rl_status rl_execution_finish(rl_context* ctx);

/* Records the ops enqueued between begin and end as a replayable graph (the
 * HIP counterpart of re-encoding one command buffer).  Buffers used while
 * recording must stay allocated while the graph is replayed.  While
 * recording, consecutive streaming ops (add, mul, SiLU, SwiGLU, casts, bias
 * add) that touch disjoint bytes or only read the same ones are recorded as
 * one kernel (each computing exactly what its own launch does), as the
 * encoders of one Metal command buffer may overlap. */
rl_status rl_graph_capture_begin(rl_context* ctx);
/* No counterpart in the reference: turns that fusion of recorded streaming
 * ops off (enabled = 0) or on (the default), for callers that time or
 * inspect the ops of a graph one by one. */
rl_status rl_context_set_fusion(rl_context* ctx, int32_t enabled);
rl_status rl_graph_capture_end(rl_context* ctx, rl_graph** out);
rl_status rl_graph_launch(rl_context* ctx, rl_graph* graph);
void rl_graph_destroy(rl_graph* graph);

/* Stream timestamps for measuring device time, and cross-stream ordering:
 * rl_event_wait makes later work of `ctx` wait for `event` (recorded on
 * another context's stream), which also forks and joins a graph recording
 * across contexts so that independent ops become parallel branches. */
rl_status rl_event_create(rl_context* ctx, rl_event** out);
rl_status rl_event_record(rl_context* ctx, rl_event* event);
rl_status rl_event_wait(rl_context* ctx, rl_event* event);
rl_status rl_event_elapsed_ms(rl_event* start, rl_event* end, float* ms);
void rl_event_destroy(rl_event* event);
/* The next kernel this context launches records its own start and end
 * timestamps in `start` and `stop` (the device time of that one kernel). */
rl_status rl_event_time_next_kernel(rl_context* ctx, rl_event* start, rl_event* stop);

/* ----------------------------------------------------------- profiling */
/* MetalContext::begin_decode_submission_profile (src/metal/context.rs:48-50). */
void rl_profile_begin(rl_context* ctx);
/* MetalContext::take_decode_submission_profile (src/metal/context.rs:52-54):
 * returns 1 and fills *out if profiling was active, else 0. */
int32_t rl_profile_take(rl_context* ctx, rl_profile* out);
/* Dispatch count of one kernel family by name (e.g. "add_f32") in the active
 * profile: MetalDecodeProfile::kernel_dispatches_by_name (src/profile.rs:15). */
uint64_t rl_profile_dispatches(const rl_context* ctx, const char* kernel_name);

/* =========================================================== element-wise */
/* ops::add_f32_encode (src/ops/add.rs:18-49): out = a + b. */
rl_status rl_add_f32(rl_context* ctx, const rl_buffer* a, const rl_buffer* b,
                     const rl_buffer* out);
/* ops::add_f16_encode (src/ops/add.rs:61-101): out = half(float(a) + float(b)). */
rl_status rl_add_f16(rl_context* ctx, const rl_buffer* a, const rl_buffer* b,
                     const rl_buffer* out);
/* ops::mul_f32_encode (src/ops/mul.rs:20-68). */
rl_status rl_mul_f32(rl_context* ctx, const rl_buffer* a, const rl_buffer* b,
                     const rl_buffer* out);
/* ops::mul_f16_encode (src/ops/mul.rs:80-119). */
rl_status rl_mul_f16(rl_context* ctx, const rl_buffer* a, const rl_buffer* b,
                     const rl_buffer* out);
/* ops::silu_f32_encode (src/ops/silu.rs:20-63): x * (1 / (1 + exp(-x))). */
rl_status rl_silu_f32(rl_context* ctx, const rl_buffer* input, const rl_buffer* out);
/* ops::silu_f16_encode (src/ops/silu.rs:75-109): half(x / (1 + exp(-x))). */
rl_status rl_silu_f16(rl_context* ctx, const rl_buffer* input, const rl_buffer* out);
/* ops::swiglu_f16_encode (src/ops/swiglu.rs:8-34): half(silu(gate) * up), one rounding. */
rl_status rl_swiglu_f16(rl_context* ctx, const rl_buffer* gate, const rl_buffer* up,
                        const rl_buffer* out);
/* SwiGlu::forward_encode F32 branch (src/nn/swiglu.rs:15-37: silu_f32 then mul_f32)
 * fused into one pass; bit-identical to the two-kernel composition. */
rl_status rl_swiglu_f32(rl_context* ctx, const rl_buffer* gate, const rl_buffer* up,
                        const rl_buffer* out);
/* ops::cast F32 -> F16 (src/ops/cast.rs:10-83, kernels/cast.metal:5-11), RNE. */
rl_status rl_cast_f32_to_f16(rl_context* ctx, const rl_buffer* input, const rl_buffer* out);
/* ops::cast F16 -> F32 (src/ops/cast.rs:10-83, kernels/cast.metal:13-19), exact. */
rl_status rl_cast_f16_to_f32(rl_context* ctx, const rl_buffer* input, const rl_buffer* out);
/* Tensor::add with a row-broadcast right operand (a [cols] bias seen through a
 * stride-0 view): the reference materialises the view with contiguous.metal
 * and adds (src/tensor/elementwise.rs:108-132); this is that composition in
 * one pass.  out[r, c] = x[r, c] + bias[c]. */
rl_status rl_add_broadcast_f32(rl_context* ctx, const rl_buffer* x, const rl_buffer* bias,
                               uint64_t rows, uint64_t cols, const rl_buffer* out);
rl_status rl_add_broadcast_f16(rl_context* ctx, const rl_buffer* x, const rl_buffer* bias,
                               uint64_t rows, uint64_t cols, const rl_buffer* out);

/* ========================================================== data movement */
/* ops::materialize_contiguous_f32_encode (src/ops/contiguous.rs:28-44,85-154):
 * out[i] = src[sum_d coord_d(i) * strides[d]] for the `rank`-dim view `dims`.
 * Strides may be 0 (broadcast). */
rl_status rl_contiguous_f32(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                            const uint64_t* strides, uint32_t rank, const rl_buffer* out);
/* ops::materialize_contiguous_f16_encode (src/ops/contiguous.rs:67-83). */
rl_status rl_contiguous_f16(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                            const uint64_t* strides, uint32_t rank, const rl_buffer* out);
/* tensor::repeat_kv dispatch (src/tensor/repeat_kv.rs:13-130): contiguous
 * [batch, kv_heads, seq, head_dim] -> [batch, kv_heads*repeats, seq, head_dim],
 * out[b, h] = in[b, h / repeats].  repeats must be >= 1 (the Tensor layer
 * returns its input unchanged for 1). */
rl_status rl_repeat_kv_f32(rl_context* ctx, const rl_buffer* input, uint64_t batch,
                           uint64_t kv_heads, uint64_t seq_len, uint64_t head_dim,
                           uint64_t repeats, const rl_buffer* out);
rl_status rl_repeat_kv_f16(rl_context* ctx, const rl_buffer* input, uint64_t batch,
                           uint64_t kv_heads, uint64_t seq_len, uint64_t head_dim,
                           uint64_t repeats, const rl_buffer* out);

/* ============================================================= reductions */
/* ops::rmsnorm_f32_encode (src/ops/rmsnorm.rs:38-116): per row of `hidden`,
 * y = x * rsqrt(mean(x^2) + eps) * w. */
rl_status rl_rmsnorm_f32(rl_context* ctx, const rl_buffer* input, const rl_buffer* weight,
                         uint64_t rows, uint64_t hidden, float eps, const rl_buffer* out);
/* ops::rmsnorm_f16_encode (src/ops/rmsnorm.rs:142-206). */
rl_status rl_rmsnorm_f16(rl_context* ctx, const rl_buffer* input, const rl_buffer* weight,
                         uint64_t rows, uint64_t hidden, float eps, const rl_buffer* out);
/* Residual add then RMSNorm, the adjacent calls of src/nn/transformer_block.rs:148-152
 * fused: sum_out = x + residual (rounded to the dtype), norm_out = RMSNorm(sum_out) * w. */
rl_status rl_add_rmsnorm_f32(rl_context* ctx, const rl_buffer* x, const rl_buffer* residual,
                             const rl_buffer* weight, uint64_t rows, uint64_t hidden, float eps,
                             const rl_buffer* sum_out, const rl_buffer* norm_out);
rl_status rl_add_rmsnorm_f16(rl_context* ctx, const rl_buffer* x, const rl_buffer* residual,
                             const rl_buffer* weight, uint64_t rows, uint64_t hidden, float eps,
                             const rl_buffer* sum_out, const rl_buffer* norm_out);

/* ops::softmax_f32_encode (src/ops/softmax.rs:27-49): row softmax over `width`;
 * a row whose max is -inf yields NaN, as kernels/softmax.metal:7-132. */
rl_status rl_softmax_f32(rl_context* ctx, const rl_buffer* input, uint64_t rows, uint64_t width,
                         const rl_buffer* out);
/* ops::softmax_f16_encode (src/ops/softmax.rs:67-89): a row whose max is -inf
 * is written as zeros (kernels/softmax.metal:166-173). */
rl_status rl_softmax_f16(rl_context* ctx, const rl_buffer* input, uint64_t rows, uint64_t width,
                         const rl_buffer* out);

/* ops::attention_scale_mask_f32_encode (src/ops/attention_scale_mask.rs:35-58):
 * on [..., query_len, key_len] scores, out = key > start + q ? -inf : x * scale. */
rl_status rl_attention_scale_mask_f32(rl_context* ctx, const rl_buffer* input, float scale,
                                      uint64_t query_len, uint64_t key_len,
                                      uint64_t query_start_pos, const rl_buffer* out);
/* ops::attention_scale_mask_f16_encode (src/ops/attention_scale_mask.rs:92-116). */
rl_status rl_attention_scale_mask_f16(rl_context* ctx, const rl_buffer* input, float scale,
                                      uint64_t query_len, uint64_t key_len,
                                      uint64_t query_start_pos, const rl_buffer* out);
/* attention_scale_mask then softmax_last_dim, the adjacent calls of
 * src/nn/attention.rs:233-240, in one pass: masked keys are never read and
 * come out as exact zeros.  Same validation as the scale/mask op; results
 * equal the two-op composition (f16: the scaled score is rounded to f16
 * before the softmax, as the composition does). */
rl_status rl_attention_softmax_f32(rl_context* ctx, const rl_buffer* input, float scale,
                                   uint64_t query_len, uint64_t key_len,
                                   uint64_t query_start_pos, const rl_buffer* out);
rl_status rl_attention_softmax_f16(rl_context* ctx, const rl_buffer* input, float scale,
                                   uint64_t query_len, uint64_t key_len,
                                   uint64_t query_start_pos, const rl_buffer* out);

/* ================================================================== RoPE */
/* ops::rope_f32_encode (src/ops/rope.rs:38-151): contiguous [..., seq_len,
 * head_dim] input, f32 [table_rows, head_dim/2] cos/sin tables; position of
 * row r is r % seq_len + start_pos. */
rl_status rl_rope_f32(rl_context* ctx, const rl_buffer* input, const rl_buffer* cos_table,
                      const rl_buffer* sin_table, uint64_t seq_len, uint64_t head_dim,
                      uint64_t start_pos, const rl_buffer* out);
/* ops::rope_f16_encode (src/ops/rope.rs:177-277); tables stay f32. */
rl_status rl_rope_f16(rl_context* ctx, const rl_buffer* input, const rl_buffer* cos_table,
                      const rl_buffer* sin_table, uint64_t seq_len, uint64_t head_dim,
                      uint64_t start_pos, const rl_buffer* out);
/* ops::rope_encode on a strided view (src/ops/rope.rs:303-370): the
 * contiguous_encode gather of :345 and the rotation in one pass.  The view is
 * `dims`/`strides` of rank >= 2 with strides[rank-1] == 1; the output is the
 * contiguous [dims] tensor; `table_rows` is the cos/sin row count. */
rl_status rl_rope_strided_f32(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                              const uint64_t* strides, uint32_t rank, const rl_buffer* cos_table,
                              const rl_buffer* sin_table, uint64_t table_rows,
                              uint64_t start_pos, const rl_buffer* out);
rl_status rl_rope_strided_f16(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                              const uint64_t* strides, uint32_t rank, const rl_buffer* cos_table,
                              const rl_buffer* sin_table, uint64_t table_rows,
                              uint64_t start_pos, const rl_buffer* out);

/* ======================================================== KV cache writes */
/* ops::kv_cache_write_f32_encode (src/ops/kv_cache_write.rs:24-41,71-141):
 * a contiguous [1, kv_heads, seq_len, head_dim] source into rows
 * start .. start + seq_len of each head of the [1, kv_heads, max_seq, head_dim]
 * cache (written in place).  start + seq_len > max_seq is
 * RL_ERR_POSITION_OUT_OF_RANGE. */
rl_status rl_kv_cache_write_f32(rl_context* ctx, const rl_buffer* cache, uint64_t kv_heads,
                                uint64_t max_seq, uint64_t head_dim, const rl_buffer* source,
                                uint64_t seq_len, uint64_t start);
/* ops::kv_cache_write_f16_encode (src/ops/kv_cache_write.rs:54-69). */
rl_status rl_kv_cache_write_f16(rl_context* ctx, const rl_buffer* cache, uint64_t kv_heads,
                                uint64_t max_seq, uint64_t head_dim, const rl_buffer* source,
                                uint64_t seq_len, uint64_t start);
/* LayerKvCache::append_encode's contiguous_encode + kv_cache_write of one
 * tensor (src/model/kv_cache.rs:123-137) in one pass: `src` is a rank-4
 * [1, kv_heads, seq_len, head_dim] view (dims/strides, any strides) written
 * into the cache as above. */
rl_status rl_kv_cache_write_strided_f32(rl_context* ctx, const rl_buffer* src,
                                        const uint64_t* dims, const uint64_t* strides,
                                        uint32_t rank, const rl_buffer* cache, uint64_t max_seq,
                                        uint64_t start);
rl_status rl_kv_cache_write_strided_f16(rl_context* ctx, const rl_buffer* src,
                                        const uint64_t* dims, const uint64_t* strides,
                                        uint32_t rank, const rl_buffer* cache, uint64_t max_seq,
                                        uint64_t start);
/* RotaryEmbedding::forward_encode of the key view then its append into the
 * cache (src/nn/attention.rs:202-207, src/model/kv_cache.rs:112-142) in one
 * pass: the [1, kv_heads, seq_len, head_dim] view (unit innermost stride) is
 * rotated at positions start_pos .. start_pos + seq_len and written to the
 * same rows of the [1, kv_heads, max_seq, head_dim] cache.  RoPE's checks
 * come first, then the cache write's. */
rl_status rl_rope_kv_cache_write_f32(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                                     const uint64_t* strides, uint32_t rank,
                                     const rl_buffer* cos_table, const rl_buffer* sin_table,
                                     uint64_t table_rows, uint64_t start_pos,
                                     const rl_buffer* cache, uint64_t max_seq);
rl_status rl_rope_kv_cache_write_f16(rl_context* ctx, const rl_buffer* src, const uint64_t* dims,
                                     const uint64_t* strides, uint32_t rank,
                                     const rl_buffer* cos_table, const rl_buffer* sin_table,
                                     uint64_t table_rows, uint64_t start_pos,
                                     const rl_buffer* cache, uint64_t max_seq);

/* The non-GEMM part of the attention's projection step as one launch:
 * RotaryEmbedding::forward_encode of Q and of K at start_pos
 * (src/nn/attention.rs:202-207) and LayerKvCache::append_encode of K and V at
 * the same position (src/model/kv_cache.rs:112-142, called with
 * cache.len() == start_pos at src/nn/attention.rs:304-307).  q/k/v are rank-4
 * [1, H, S, D] views with unit innermost strides (the permutes of the
 * [1, S, H*D] projections); Q (QH heads) is written rotated to the contiguous
 * q_out, K rotated and V as is to rows start_pos .. start_pos + S of the
 * [1, KVH, max_seq, D] caches.  Checks in the reference's order (RoPE on Q,
 * RoPE on K, the append's K/V shape check as RL_ERR_MODEL_FORMAT, the two
 * cache writes). */
rl_status rl_qkv_rope_kv_append_f32(rl_context* ctx, const rl_buffer* q_src,
                                    const uint64_t* q_dims, const uint64_t* q_strides,
                                    const rl_buffer* k_src, const uint64_t* k_dims,
                                    const uint64_t* k_strides, const rl_buffer* v_src,
                                    const uint64_t* v_dims, const uint64_t* v_strides,
                                    const rl_buffer* cos_table, const rl_buffer* sin_table,
                                    uint64_t table_rows, uint64_t start_pos,
                                    const rl_buffer* q_out, const rl_buffer* k_cache,
                                    const rl_buffer* v_cache, uint64_t max_seq);
rl_status rl_qkv_rope_kv_append_f16(rl_context* ctx, const rl_buffer* q_src,
                                    const uint64_t* q_dims, const uint64_t* q_strides,
                                    const rl_buffer* k_src, const uint64_t* k_dims,
                                    const uint64_t* k_strides, const rl_buffer* v_src,
                                    const uint64_t* v_dims, const uint64_t* v_strides,
                                    const rl_buffer* cos_table, const rl_buffer* sin_table,
                                    uint64_t table_rows, uint64_t start_pos,
                                    const rl_buffer* q_out, const rl_buffer* k_cache,
                                    const rl_buffer* v_cache, uint64_t max_seq);

/* rl_qkv_rope_kv_append_* followed, in the same launch, by
 * tensor::repeat_kv (src/tensor/repeat_kv.rs:13-130) of the two caches'
 * prefixes after the append -- the [1, KVH, start_pos + S, D] key() and
 * value() views (src/model/kv_cache.rs:87-99) -- into the contiguous
 * [1, KVH * n_rep, start_pos + S, D] k_rep and v_rep: the C5 layer chain's
 * "RoPE(Q, K) -> repeat_kv(K, V)" prologue, which the reference runs as
 * separate calls.  Checks: those of rl_qkv_rope_kv_append_*, then
 * repeat_kv's (n_rep == 0 and a head-count overflow are
 * RL_ERR_MODEL_FORMAT), then the output sizes.  With n_rep == 1 the outputs
 * are copies of the prefixes (repeat_kv returns its input there). */
rl_status rl_qkv_rope_kv_append_repeat_f32(
    rl_context* ctx, const rl_buffer* q_src, const uint64_t* q_dims, const uint64_t* q_strides,
    const rl_buffer* k_src, const uint64_t* k_dims, const uint64_t* k_strides,
    const rl_buffer* v_src, const uint64_t* v_dims, const uint64_t* v_strides,
    const rl_buffer* cos_table, const rl_buffer* sin_table, uint64_t table_rows,
    uint64_t start_pos, const rl_buffer* q_out, const rl_buffer* k_cache,
    const rl_buffer* v_cache, uint64_t max_seq, uint64_t n_rep, const rl_buffer* k_rep,
    const rl_buffer* v_rep);
rl_status rl_qkv_rope_kv_append_repeat_f16(
    rl_context* ctx, const rl_buffer* q_src, const uint64_t* q_dims, const uint64_t* q_strides,
    const rl_buffer* k_src, const uint64_t* k_dims, const uint64_t* k_strides,
    const rl_buffer* v_src, const uint64_t* v_dims, const uint64_t* v_strides,
    const rl_buffer* cos_table, const rl_buffer* sin_table, uint64_t table_rows,
    uint64_t start_pos, const rl_buffer* q_out, const rl_buffer* k_cache,
    const rl_buffer* v_cache, uint64_t max_seq, uint64_t n_rep, const rl_buffer* k_rep,
    const rl_buffer* v_rep);

/* ============================================================= embedding */
/* ops::embedding_f32_encode (src/ops/embedding.rs:32-57,119-193):
 * out[t, :] = weight[token_ids[t], :] for a [vocab_size, hidden_size] weight.
 * token_ids is host memory (n_tokens values), checked against vocab_size
 * (RL_ERR_INVALID_TOKEN_ID) and copied to the device in stream order; it may
 * be reused as soon as the call returns.  Not allowed while recording a
 * graph. */
rl_status rl_embedding_f32(rl_context* ctx, const rl_buffer* weight, uint64_t vocab_size,
                           uint64_t hidden_size, const uint32_t* token_ids, uint64_t n_tokens,
                           const rl_buffer* out);
/* ops::embedding_f16_encode (src/ops/embedding.rs:81-106). */
rl_status rl_embedding_f16(rl_context* ctx, const rl_buffer* weight, uint64_t vocab_size,
                           uint64_t hidden_size, const uint32_t* token_ids, uint64_t n_tokens,
                           const rl_buffer* out);

/* ============================================================= attention */
/* SelfAttention::attention_core_encode (src/nn/attention.rs:216-247) as one
 * pass: scores = Q K^T (Tensor::gqa_qk_matmul_encode,
 * src/tensor/gqa_matmul.rs:23-61, or batched_matmul when q_heads ==
 * kv_heads), attention_scale_mask(scale, query_start_pos), softmax over the
 * keys, then P V (gqa_pv_matmul_encode, :72-110); the [B, QH, Q, K] scores
 * are never written.
 *   q:    contiguous [batch, q_heads, q_len, head_dim]
 *   k, v: [batch, kv_heads, kv_capacity, head_dim]; the first kv_len rows of
 *         each head are used (a LayerKvCache's buffers with kv_capacity =
 *         max_seq, or contiguous tensors with kv_capacity = kv_len); query
 *         head h reads KV head h / (q_heads / kv_heads)
 *   out:  contiguous [batch, q_heads, q_len, head_dim]
 * Key j is masked for query i when j > query_start_pos + i.  Checks in the
 * reference's order (head groups as RL_ERR_MODEL_FORMAT, the u32 limits,
 * the scale/mask checks); also rejected: kv_capacity < kv_len and
 * head_dim > 512 when the matrix-core path (f16, head_dim 32/64/96/128)
 * does not apply.  Results differ from the four separate calls by their
 * intermediate roundings: scores and probabilities stay in f32 here.  f16
 * launches with few 128-query tiles and long key ranges (a prefill after
 * cached keys) split each tile's keys over workgroups: f32 partials in a
 * pool block, merged by a second kernel (not while a graph records, where
 * the one-pass kernels run). */
rl_status rl_attention_f32(rl_context* ctx, const rl_buffer* q, const rl_buffer* k,
                           const rl_buffer* v, uint64_t batch, uint64_t q_heads,
                           uint64_t kv_heads, uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                           uint64_t kv_capacity, float scale, uint64_t query_start_pos,
                           const rl_buffer* out);
rl_status rl_attention_f16(rl_context* ctx, const rl_buffer* q, const rl_buffer* k,
                           const rl_buffer* v, uint64_t batch, uint64_t q_heads,
                           uint64_t kv_heads, uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                           uint64_t kv_capacity, float scale, uint64_t query_start_pos,
                           const rl_buffer* out);

/* No counterpart in the reference.  rl_attention_f16 for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): same arguments, checks and results, but
 * the decode path (few query rows per KV head, >= 512 visible keys) keeps
 * its per-split partials and hand-off counters in a file-scope device array
 * of 8 MiB (256 KiB of counters, the rest partials) that each GPU holds from
 * the library's load until the process ends, instead of a pool block and
 * the context's counters; the other paths allocate nothing anyway.  A decode
 * shape needing more -- batch*q_heads*q_len * ceil(keys/256) * (head_dim+2)
 * floats above 8 MiB - 256 KiB, or more than 1024 batch*kv_heads counters --
 * is RL_ERR_INVALID_SHAPE.  Every call on one GPU shares that array: calls
 * that overlap on one GPU (other streams, other threads) race.  Allowed
 * while recording a graph. */
rl_status rl_attention_f16_noalloc(rl_context* ctx, const rl_buffer* q, const rl_buffer* k,
                                   const rl_buffer* v, uint64_t batch, uint64_t q_heads,
                                   uint64_t kv_heads, uint64_t q_len, uint64_t kv_len,
                                   uint64_t head_dim, uint64_t kv_capacity, float scale,
                                   uint64_t query_start_pos, const rl_buffer* out);

/* Tensor::gqa_qk_matmul_encode (src/tensor/gqa_matmul.rs:23-61, kernels
 * gqa_qk_f32/f16, kernels/gqa_matmul.metal:7-322): scores [batch, q_heads,
 * q_len, kv_len] = Q K^T without repeating the KV heads; query head h reads
 * KV head h / (q_heads / kv_heads).  q: contiguous [batch, q_heads, q_len,
 * head_dim]; k: [batch, kv_heads, kv_capacity, head_dim], first kv_len rows
 * per head used (the reference passes kv_capacity from K's head stride,
 * :54-59).  f32 accumulation; the f16 score is rounded once.  Checks: head
 * groups (RL_ERR_MODEL_FORMAT), the u32 limits of :192-212, kv_capacity >=
 * kv_len, exact buffer lengths. */
rl_status rl_gqa_qk_matmul_f32(rl_context* ctx, const rl_buffer* q, const rl_buffer* k,
                               uint64_t batch, uint64_t q_heads, uint64_t kv_heads,
                               uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                               uint64_t kv_capacity, const rl_buffer* out);
rl_status rl_gqa_qk_matmul_f16(rl_context* ctx, const rl_buffer* q, const rl_buffer* k,
                               uint64_t batch, uint64_t q_heads, uint64_t kv_heads,
                               uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                               uint64_t kv_capacity, const rl_buffer* out);
/* Tensor::gqa_pv_matmul_encode (src/tensor/gqa_matmul.rs:72-110, kernels
 * gqa_pv_f32/f16, kernels/gqa_matmul.metal:323-629): out [batch, q_heads,
 * q_len, head_dim] = P V for probabilities P [batch, q_heads, q_len, kv_len]
 * (contiguous) and V [batch, kv_heads, kv_capacity, head_dim] (first kv_len
 * rows per head).  Same checks as rl_gqa_qk_matmul_*. */
rl_status rl_gqa_pv_matmul_f32(rl_context* ctx, const rl_buffer* probs, const rl_buffer* v,
                               uint64_t batch, uint64_t q_heads, uint64_t kv_heads,
                               uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                               uint64_t kv_capacity, const rl_buffer* out);
rl_status rl_gqa_pv_matmul_f16(rl_context* ctx, const rl_buffer* probs, const rl_buffer* v,
                               uint64_t batch, uint64_t q_heads, uint64_t kv_heads,
                               uint64_t q_len, uint64_t kv_len, uint64_t head_dim,
                               uint64_t kv_capacity, const rl_buffer* out);

#ifdef __cplusplus
}
#endif

#endif /* RUSTLLM_HIP_H */
