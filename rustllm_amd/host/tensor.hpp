// tensor.hpp -- C++ restatement of RustLLM's host-side tensor layer over the
// gfx950 C ABI (include/rustllm_hip.h).
//
// This is the layer the Rust crate keeps above the FFI line: `Tensor` with
// Shape / Strides / DType / shared Storage and zero-copy views
// (src/tensor/tensor.rs), the buffer-level ops (src/ops/mod.rs:20-53), the
// context / buffer / execution handles (src/metal/{context,buffer,
// execution}.rs) and the three nn wrappers on the hot path
// (src/nn/{rmsnorm,rope,swiglu}.rs).  Names, argument meaning, validation
// order and error kinds follow the reference; `Result<T>` becomes a thrown
// `TinyError` carrying the same kind.
//
// As in the reference, `*_encode` functions enqueue into the current
// execution and return at once; the plain functions open an Execution,
// encode, and finish (commit + wait).
#pragma once

#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "rustllm_hip.h"

namespace rustllm {

// ------------------------------------------------------------------ errors

// src/error.rs:4-43 (the variants the op layer raises; Device = Metal).
class TinyError : public std::runtime_error {
   public:
    enum class Kind {
        InvalidArgument,
        InvalidShape,
        ShapeMismatch,
        InvalidDimension,
        UnsupportedDType,
        NonContiguousTensor,
        PositionOutOfRange,
        ModelFormat,
        Device,
        InvalidTokenId,
    };
    TinyError(Kind kind, const std::string& message);
    Kind kind() const { return kind_; }
    // The library's failure as the variant it names, with the payload of
    // ShapeMismatch / PositionOutOfRange / InvalidTokenId (rl_last_error_payload).
    static TinyError from_status(rl_status status);
    // The variants that carry data (src/error.rs:7-24), with the reference's
    // Display text as the message.
    static TinyError shape_mismatch(std::vector<size_t> left, std::vector<size_t> right);
    static TinyError position_out_of_range(size_t start_pos, size_t seq_len, size_t max_seq_len);
    static TinyError invalid_token_id(uint32_t token_id, size_t vocab_size);

    // ShapeMismatch { left, right }
    std::vector<size_t> left, right;
    // PositionOutOfRange { start_pos, seq_len, max_seq_len }
    size_t start_pos = 0, seq_len = 0, max_seq_len = 0;
    // InvalidTokenId { token_id, vocab_size }
    uint32_t token_id = 0;
    size_t vocab_size = 0;

   private:
    Kind kind_;
};

const char* kind_name(TinyError::Kind kind);

// ------------------------------------------------------------- dtype/shape

// src/tensor/dtype.rs:1-14
enum class DType { F32, F16 };
size_t size_in_bytes(DType dtype);
const char* dtype_name(DType dtype);

// half::f16::from_f32 / to_f32 (round to nearest even), as used by
// Tensor::from_f16_slice callers and to_f32_vec (tensor.rs:337-346).
uint16_t f16_from_f32(float value);
float f16_to_f32(uint16_t bits);

// src/tensor/shape.rs:9-45
class Shape {
   public:
    static Shape create(const std::vector<size_t>& dims);  // rejects rank 0 and zero dims
    const std::vector<size_t>& dims() const { return dims_; }
    size_t rank() const { return dims_.size(); }
    size_t numel() const;
    size_t dim(size_t index) const;
    bool operator==(const Shape& o) const { return dims_ == o.dims_; }
    bool operator!=(const Shape& o) const { return dims_ != o.dims_; }

   private:
    std::vector<size_t> dims_;
};

// src/tensor/strides.rs:9-35
class Strides {
   public:
    static Strides contiguous(const Shape& shape);
    static Strides from_values(std::vector<size_t> values);
    const std::vector<size_t>& values() const { return values_; }
    std::optional<size_t> get(size_t index) const;
    bool operator==(const Strides& o) const { return values_ == o.values_; }

   private:
    std::vector<size_t> values_;
};

// ------------------------------------------------------------ GPU runtime

// MetalDecodeProfile (src/profile.rs:7-16)
struct DecodeProfile {
    uint64_t command_buffers = 0, compute_encoders = 0, kernel_dispatches = 0, commits = 0,
             waits = 0, buffer_allocations = 0, allocated_bytes = 0;
};

// MetalContext (src/metal/context.rs:10-139): one device, one in-order stream.
class Context {
   public:
    static Context create(int device = 0);  // MetalContext::new
    rl_context* raw() const { return handle_.get(); }
    void begin_decode_submission_profile();
    std::optional<DecodeProfile> take_decode_submission_profile();
    uint64_t dispatches(const std::string& kernel_name) const;

   private:
    std::shared_ptr<rl_context> handle_;
};

// MetalBuffer (src/metal/buffer.rs:8-169): owns a pooled device buffer.
class Buffer {
   public:
    Buffer() = default;
    Buffer(const Context& ctx, rl_buffer raw);
    ~Buffer();
    Buffer(Buffer&& other) noexcept;
    Buffer& operator=(Buffer&& other) noexcept;
    Buffer(const Buffer&) = delete;
    Buffer& operator=(const Buffer&) = delete;

    static Buffer from_slice(const Context& ctx, const std::vector<float>& data);
    static Buffer from_f16_slice(const Context& ctx, const std::vector<uint16_t>& data);
    static Buffer empty(const Context& ctx, size_t len);  // f32-sized
    static Buffer empty_with_element_size(const Context& ctx, size_t len, size_t element_size);

    size_t len() const { return size_t(raw_.len); }
    size_t byte_len() const { return size_t(raw_.byte_len); }
    bool is_empty() const { return raw_.len == 0; }
    const rl_buffer* raw() const { return &raw_; }
    // Host copies (the reference borrows shared memory; HBM needs a copy).
    std::vector<float> as_slice() const;
    std::vector<uint16_t> as_f16_slice() const;

   private:
    Context ctx_;
    rl_buffer raw_{nullptr, 0, 0};
};

// MetalExecution (src/metal/execution.rs:5-36)
class Execution {
   public:
    explicit Execution(const Context& ctx);
    ~Execution();  // an unfinished execution still waits, so buffers stay valid
    void finish();
    const Context& context() const { return ctx_; }

   private:
    Context ctx_;
    bool finished_ = false;
};

// ----------------------------------------------------------------- tensor

// src/tensor/storage.rs:1-51
struct Storage {
    Buffer buffer;
};

// src/tensor/tensor.rs:15-21
class Tensor {
   public:
    static Tensor from_f32_slice(const Context& ctx, const std::vector<float>& data,
                                 const std::vector<size_t>& dims);
    static Tensor from_f16_slice(const Context& ctx, const std::vector<uint16_t>& data,
                                 const std::vector<size_t>& dims);
    static Tensor empty(const Context& ctx, const std::vector<size_t>& dims, DType dtype);
    static Tensor zeros(const Context& ctx, const std::vector<size_t>& dims);
    static Tensor from_buffer(Buffer buffer, const std::vector<size_t>& dims, DType dtype);

    const Shape& shape() const { return shape_; }
    const Strides& strides() const { return strides_; }
    DType dtype() const { return dtype_; }
    size_t rank() const { return shape_.rank(); }
    size_t numel() const { return shape_.numel(); }
    size_t len() const { return numel(); }
    size_t byte_len() const { return numel() * size_in_bytes(dtype_); }
    size_t dim(size_t index) const { return shape_.dim(index); }
    bool is_contiguous() const;  // strict stride equality (tensor.rs:251-253)
    const Buffer& buffer() const { return storage_->buffer; }
    bool shares_storage_with(const Tensor& o) const { return storage_ == o.storage_; }

    // Zero-copy views (tensor.rs:137-306) plus `expand` (stride-0 broadcast).
    Tensor transpose(size_t dim_a, size_t dim_b) const;
    Tensor permute(const std::vector<size_t>& order) const;
    Tensor reshape(const std::vector<size_t>& dims) const;
    Tensor narrow(size_t dim, size_t start, size_t len) const;
    Tensor expand(const std::vector<size_t>& dims) const;

    Tensor contiguous(const Context& ctx) const;
    Tensor contiguous_encode(const Context& ctx) const;
    std::vector<float> to_f32_vec() const;
    Tensor to_dtype(const Context& ctx, DType dtype) const;

    Tensor add(const Context& ctx, const Tensor& rhs) const;
    Tensor mul(const Context& ctx, const Tensor& rhs) const;
    Tensor silu(const Context& ctx) const;
    Tensor add_encode(const Context& ctx, const Tensor& rhs) const;
    Tensor mul_encode(const Context& ctx, const Tensor& rhs) const;
    Tensor silu_encode(const Context& ctx) const;
    Tensor softmax_last_dim(const Context& ctx) const;
    Tensor softmax_last_dim_encode(const Context& ctx) const;
    Tensor attention_scale_mask(const Context& ctx, float scale, size_t query_start_pos) const;
    Tensor attention_scale_mask_encode(const Context& ctx, float scale,
                                       size_t query_start_pos) const;
    // attention_scale_mask then softmax_last_dim in one pass (new).
    Tensor attention_softmax_encode(const Context& ctx, float scale,
                                    size_t query_start_pos) const;
    Tensor repeat_kv(const Context& ctx, size_t repeats) const;
    // src/tensor/gqa_matmul.rs:16-110: Q [B, QH, Q, D] x K^T without
    // repeating the KV heads, and P [B, QH, Q, K] x V.  A one-query Q (and the
    // K / V it meets) is used in place -- a KV-cache view included -- as the
    // reference does; otherwise the operands are made contiguous first.
    Tensor gqa_qk_matmul(const Context& ctx, const Tensor& key) const;
    Tensor gqa_qk_matmul_encode(const Context& ctx, const Tensor& key) const;
    Tensor gqa_pv_matmul(const Context& ctx, const Tensor& value) const;
    Tensor gqa_pv_matmul_encode(const Context& ctx, const Tensor& value) const;

   private:
    Tensor(std::shared_ptr<Storage> storage, Shape shape, Strides strides, DType dtype);
    Tensor binary_elementwise(const Context& ctx, const Tensor& rhs, bool is_add) const;
    Tensor binary_elementwise_encode(const Context& ctx, const Tensor& rhs, bool is_add) const;

    std::shared_ptr<Storage> storage_;
    Shape shape_;
    Strides strides_;
    DType dtype_;
};

// -------------------------------------------------------------------- ops

// Buffer-level ops (src/ops/mod.rs:20-53).  Plain versions wait; _encode
// versions enqueue into the current execution.
namespace ops {
Buffer add_f32(const Context& ctx, const Buffer& a, const Buffer& b);
Buffer add_f16(const Context& ctx, const Buffer& a, const Buffer& b);
Buffer add_f32_encode(const Context& ctx, const Buffer& a, const Buffer& b);
Buffer add_f16_encode(const Context& ctx, const Buffer& a, const Buffer& b);
Buffer mul_f32(const Context& ctx, const Buffer& a, const Buffer& b);
Buffer mul_f16(const Context& ctx, const Buffer& a, const Buffer& b);
Buffer mul_f32_encode(const Context& ctx, const Buffer& a, const Buffer& b);
Buffer mul_f16_encode(const Context& ctx, const Buffer& a, const Buffer& b);
Buffer silu_f32(const Context& ctx, const Buffer& input);
Buffer silu_f16(const Context& ctx, const Buffer& input);
Buffer silu_f32_encode(const Context& ctx, const Buffer& input);
Buffer silu_f16_encode(const Context& ctx, const Buffer& input);
Buffer swiglu_f16(const Context& ctx, const Buffer& gate, const Buffer& up);
Buffer swiglu_f16_encode(const Context& ctx, const Buffer& gate, const Buffer& up);
Buffer swiglu_f32_encode(const Context& ctx, const Buffer& gate, const Buffer& up);
Tensor cast(const Context& ctx, const Tensor& input, DType dtype);
Buffer materialize_contiguous_f32(const Context& ctx, const Buffer& source,
                                  const std::vector<size_t>& dims,
                                  const std::vector<size_t>& strides);
Buffer materialize_contiguous_f16(const Context& ctx, const Buffer& source,
                                  const std::vector<size_t>& dims,
                                  const std::vector<size_t>& strides);
Buffer materialize_contiguous_f32_encode(const Context& ctx, const Buffer& source,
                                         const std::vector<size_t>& dims,
                                         const std::vector<size_t>& strides);
Buffer materialize_contiguous_f16_encode(const Context& ctx, const Buffer& source,
                                         const std::vector<size_t>& dims,
                                         const std::vector<size_t>& strides);
Buffer rmsnorm_f32(const Context& ctx, const Buffer& input, const Buffer& weight, size_t rows,
                   size_t hidden_size, float epsilon);
Buffer rmsnorm_f16(const Context& ctx, const Buffer& input, const Buffer& weight, size_t rows,
                   size_t hidden_size, float epsilon);
Buffer rmsnorm_f32_encode(const Context& ctx, const Buffer& input, const Buffer& weight,
                          size_t rows, size_t hidden_size, float epsilon);
Buffer rmsnorm_f16_encode(const Context& ctx, const Buffer& input, const Buffer& weight,
                          size_t rows, size_t hidden_size, float epsilon);
Tensor rmsnorm(const Context& ctx, const Tensor& input, const Tensor& weight, float epsilon);
Buffer softmax_f32(const Context& ctx, const Buffer& input, size_t rows, size_t width);
Buffer softmax_f16(const Context& ctx, const Buffer& input, size_t rows, size_t width);
Buffer softmax_f32_encode(const Context& ctx, const Buffer& input, size_t rows, size_t width);
Buffer softmax_f16_encode(const Context& ctx, const Buffer& input, size_t rows, size_t width);
Buffer attention_scale_mask_f32(const Context& ctx, const Buffer& input, float scale,
                                size_t query_len, size_t key_len, size_t query_start_pos);
Buffer attention_scale_mask_f16(const Context& ctx, const Buffer& input, float scale,
                                size_t query_len, size_t key_len, size_t query_start_pos);
Buffer attention_scale_mask_f32_encode(const Context& ctx, const Buffer& input, float scale,
                                       size_t query_len, size_t key_len, size_t query_start_pos);
Buffer attention_scale_mask_f16_encode(const Context& ctx, const Buffer& input, float scale,
                                       size_t query_len, size_t key_len, size_t query_start_pos);
Buffer rope_f32(const Context& ctx, const Buffer& input, const Buffer& cos_table,
                const Buffer& sin_table, size_t seq_len, size_t head_dim, size_t start_pos);
Buffer rope_f16(const Context& ctx, const Buffer& input, const Buffer& cos_table,
                const Buffer& sin_table, size_t seq_len, size_t head_dim, size_t start_pos);
Tensor rope(const Context& ctx, const Tensor& input, const Tensor& cos, const Tensor& sin,
            size_t start_pos);
Tensor rope_encode(const Context& ctx, const Tensor& input, const Tensor& cos, const Tensor& sin,
                   size_t start_pos);
void validate_rope(const Tensor& input, const Tensor& cos, const Tensor& sin, size_t start_pos);
// Residual add + RMSNorm fused (nn/transformer_block.rs:148-152); returns {sum, norm}.
std::pair<Tensor, Tensor> add_rmsnorm_encode(const Context& ctx, const Tensor& x,
                                             const Tensor& residual, const Tensor& weight,
                                             float epsilon);
// src/ops/embedding.rs:10-193: rows of a [vocab_size, hidden_size] weight.
Buffer embedding_f32(const Context& ctx, const Buffer& weight,
                     const std::vector<uint32_t>& token_ids, size_t vocab_size,
                     size_t hidden_size);
Buffer embedding_f16(const Context& ctx, const Buffer& weight,
                     const std::vector<uint32_t>& token_ids, size_t vocab_size,
                     size_t hidden_size);
Buffer embedding_f32_encode(const Context& ctx, const Buffer& weight,
                            const std::vector<uint32_t>& token_ids, size_t vocab_size,
                            size_t hidden_size);
Buffer embedding_f16_encode(const Context& ctx, const Buffer& weight,
                            const std::vector<uint32_t>& token_ids, size_t vocab_size,
                            size_t hidden_size);
// src/ops/kv_cache_write.rs:9-141: source [1, H, S, D] into cache [1, H, max, D] at start.
void kv_cache_write_f32(const Context& ctx, const Tensor& cache, const Tensor& source,
                        size_t start);
void kv_cache_write_f16(const Context& ctx, const Tensor& cache, const Tensor& source,
                        size_t start);
void kv_cache_write_f32_encode(const Context& ctx, const Tensor& cache, const Tensor& source,
                               size_t start);
void kv_cache_write_f16_encode(const Context& ctx, const Tensor& cache, const Tensor& source,
                               size_t start);
}  // namespace ops

// --------------------------------------------------------------------- nn

namespace nn {

// src/nn/rmsnorm.rs
class RmsNorm {
   public:
    RmsNorm(Tensor weight, float epsilon);
    size_t hidden_size() const { return hidden_size_; }
    float epsilon() const { return epsilon_; }
    const Tensor& weight() const { return weight_; }
    DType dtype() const { return weight_.dtype(); }
    Tensor forward(const Context& ctx, const Tensor& input) const;
    Tensor forward_encode(const Context& ctx, const Tensor& input) const;
    RmsNorm to_dtype(const Context& ctx, DType dtype) const;

   private:
    Tensor weight_;
    size_t hidden_size_;
    float epsilon_;
};

// src/nn/rope.rs:9-152: f32 cos/sin tables [max_seq_len, head_dim/2] built on the host.
class RotaryEmbedding {
   public:
    RotaryEmbedding(const Context& ctx, size_t head_dim, size_t max_seq_len, float theta);
    size_t head_dim() const { return head_dim_; }
    size_t max_seq_len() const { return max_seq_len_; }
    float theta() const { return theta_; }
    const Tensor& cos_table() const { return cos_; }
    const Tensor& sin_table() const { return sin_; }
    Tensor forward(const Context& ctx, const Tensor& input, size_t start_pos) const;
    Tensor forward_encode(const Context& ctx, const Tensor& input, size_t start_pos) const;

   private:
    Tensor cos_, sin_;
    size_t head_dim_, max_seq_len_;
    float theta_;
};

// src/nn/swiglu.rs:7-37
struct SwiGlu {
    static Tensor forward(const Context& ctx, const Tensor& gate, const Tensor& up);
    static Tensor forward_encode(const Context& ctx, const Tensor& gate, const Tensor& up);
};

// SelfAttention::attention_core_encode (src/nn/attention.rs:216-247) in one
// pass: QK^T, scale/mask(scale, start_pos), softmax, PV, the scores never
// written.  q [B, QH, Q, D]; key / value [B, KVH, K, D] (contiguous, or the
// narrowed views of a LayerKvCache, read in place).  Checks of the four
// calls it replaces, in their order.
Tensor attention_core_encode(const Context& ctx, const Tensor& q, const Tensor& key,
                             const Tensor& value, float scale, size_t start_pos);

}  // namespace nn

// ------------------------------------------------------------------ model

namespace model {

// src/model/kv_cache.rs:9-142: one layer's [1, kv_heads, max, dim] key and
// value caches and the logical length.
class LayerKvCache {
   public:
    LayerKvCache(const Context& ctx, size_t num_kv_heads, size_t max, size_t dim, DType dtype);
    size_t len() const { return len_; }
    bool is_empty() const { return len_ == 0; }
    size_t capacity() const { return max_seq_len_; }
    size_t storage_bytes() const;
    void reset() { len_ = 0; }
    DType dtype() const { return key_.dtype(); }
    Tensor key() const;    // narrow(2, 0, len)
    Tensor value() const;  // narrow(2, 0, len)
    void append(const Context& ctx, const Tensor& key, const Tensor& value);
    // Gathers strided key/value views straight into the cache (the
    // contiguous_encode + kv_cache_write of the reference in one pass each).
    void append_encode(const Context& ctx, const Tensor& key, const Tensor& value);
    // RotaryEmbedding::forward_encode(key, len()) then append_encode, with the
    // rotated key written straight into the cache (nn/attention.rs:202-207,306-307).
    void append_rotated_encode(const Context& ctx, const nn::RotaryEmbedding& rope,
                               const Tensor& key, const Tensor& value);
    // The attention step's Q and K rotation at len() and the K/V append
    // (nn/attention.rs:196-207, 304-307) in one launch; returns the rotated,
    // contiguous Q.
    Tensor rotate_query_and_append_encode(const Context& ctx, const nn::RotaryEmbedding& rope,
                                          const Tensor& query, const Tensor& key,
                                          const Tensor& value);

   private:
    void validate_append(const Tensor& key, const Tensor& value) const;
    Tensor key_, value_;
    size_t len_ = 0, max_seq_len_, num_kv_heads_, head_dim_;
};

}  // namespace model
}  // namespace rustllm
