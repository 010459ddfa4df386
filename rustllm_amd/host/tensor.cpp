// tensor.cpp -- the host tensor layer over the gfx950 C ABI (see tensor.hpp).
// Every function cites the reference item it restates.
#include "tensor.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <sstream>

namespace rustllm {

// ------------------------------------------------------------------ errors

static const char* const kKindNames[] = {
    "InvalidArgument", "InvalidShape", "ShapeMismatch",      "InvalidDimension", "UnsupportedDType",
    "NonContiguousTensor", "PositionOutOfRange", "ModelFormat", "Device", "InvalidTokenId",
};

const char* kind_name(TinyError::Kind kind) { return kKindNames[int(kind)]; }

TinyError::TinyError(Kind kind, const std::string& message)
    : std::runtime_error(std::string(kind_name(kind)) + ": " + message), kind_(kind) {}

TinyError TinyError::from_status(rl_status status) {
    Kind kind = (status >= 1 && status <= 10) ? Kind(status - 1) : Kind::Device;
    TinyError e(kind, rl_last_error_message());
    rl_error_payload p{};
    if (rl_last_error_payload(&p) != status) return e;
    if (kind == Kind::ShapeMismatch) {
        e.left.assign(p.left, p.left + std::min<uint32_t>(p.left_rank, RL_ERROR_MAX_RANK));
        e.right.assign(p.right, p.right + std::min<uint32_t>(p.right_rank, RL_ERROR_MAX_RANK));
    } else if (kind == Kind::PositionOutOfRange) {
        e.start_pos = p.start_pos;
        e.seq_len = p.seq_len;
        e.max_seq_len = p.max_seq_len;
    } else if (kind == Kind::InvalidTokenId) {
        e.token_id = p.token_id;
        e.vocab_size = p.vocab_size;
    }
    return e;
}

static void check(rl_status status) {
    if (status != RL_OK) throw TinyError::from_status(status);
}

static std::string dims_str(const std::vector<size_t>& dims) {
    std::ostringstream os;
    os << "[";
    for (size_t i = 0; i < dims.size(); ++i) os << (i ? ", " : "") << dims[i];
    os << "]";
    return os.str();
}

TinyError TinyError::shape_mismatch(std::vector<size_t> left, std::vector<size_t> right) {
    TinyError e(Kind::ShapeMismatch, "left=" + dims_str(left) + ", right=" + dims_str(right));
    e.left = std::move(left);
    e.right = std::move(right);
    return e;
}

TinyError TinyError::position_out_of_range(size_t start_pos, size_t seq_len, size_t max_seq_len) {
    TinyError e(Kind::PositionOutOfRange,
                "position range [" + std::to_string(start_pos) + ", " +
                    std::to_string(start_pos + seq_len) + ") exceeds max sequence length " +
                    std::to_string(max_seq_len));
    e.start_pos = start_pos;
    e.seq_len = seq_len;
    e.max_seq_len = max_seq_len;
    return e;
}

TinyError TinyError::invalid_token_id(uint32_t token_id, size_t vocab_size) {
    TinyError e(Kind::InvalidTokenId, "invalid token id " + std::to_string(token_id) +
                                          ": vocabulary size is " + std::to_string(vocab_size));
    e.token_id = token_id;
    e.vocab_size = vocab_size;
    return e;
}

static TinyError shape_mismatch(const std::vector<size_t>& left, const std::vector<size_t>& right) {
    return TinyError::shape_mismatch(left, right);
}

// ------------------------------------------------------------- dtype/shape

size_t size_in_bytes(DType dtype) { return dtype == DType::F32 ? 4 : 2; }
const char* dtype_name(DType dtype) { return dtype == DType::F32 ? "F32" : "F16"; }

uint16_t f16_from_f32(float value) {
    uint32_t x;
    std::memcpy(&x, &value, 4);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    const uint32_t abs = x & 0x7fffffffu;
    if (abs >= 0x7f800000u)  // inf, NaN (quieted)
        return uint16_t(sign | 0x7c00u | (abs > 0x7f800000u ? 0x0200u | ((abs >> 13) & 0x3ffu) : 0));
    if (abs >= 0x477ff000u) return uint16_t(sign | 0x7c00u);  // >= 65520 rounds to inf
    if (abs < 0x38800000u) {
        // Below the smallest normal half: scale to units of 2^-24 and round.
        if (abs < 0x33000000u) return sign;  // <= 2^-25 rounds to zero (tie to even)
        const uint32_t e = abs >> 23;
        const uint32_t m = (abs & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;  // 14 .. 24
        uint32_t q = m >> shift;
        const uint32_t rest = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        q += (rest > half || (rest == half && (q & 1u))) ? 1u : 0u;
        return uint16_t(sign | q);
    }
    // Normal: rebias and round the 13 dropped bits to nearest even.
    const uint32_t r = abs - 0x38000000u;  // exponent 127 -> 15
    uint32_t q = r >> 13;
    const uint32_t rest = r & 0x1fffu;
    q += (rest > 0x1000u || (rest == 0x1000u && (q & 1u))) ? 1u : 0u;
    return uint16_t(sign | q);
}

float f16_to_f32(uint16_t bits) {
    const uint32_t sign = uint32_t(bits & 0x8000u) << 16;
    const uint32_t e = (bits >> 10) & 0x1fu, m = bits & 0x3ffu;
    uint32_t out;
    if (e == 31) {
        out = sign | 0x7f800000u | (m << 13);
    } else if (e == 0) {
        float v = std::ldexp(float(m), -24);
        std::memcpy(&out, &v, 4);
        out |= sign;
    } else {
        out = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &out, 4);
    return f;
}

// src/tensor/shape.rs:9-23
Shape Shape::create(const std::vector<size_t>& dims) {
    if (dims.empty()) throw TinyError(TinyError::Kind::InvalidShape, "shape cannot be empty");
    for (size_t d : dims)
        if (d == 0)
            throw TinyError(TinyError::Kind::InvalidShape,
                            "shape dimensions must be greater than zero");
    Shape s;
    s.dims_ = dims;
    return s;
}

size_t Shape::numel() const {
    size_t n = 1;
    for (size_t d : dims_) n *= d;
    return n;
}

// src/tensor/shape.rs:37-44
size_t Shape::dim(size_t index) const {
    if (index >= dims_.size())
        throw TinyError(TinyError::Kind::InvalidDimension,
                        "dimension " + std::to_string(index) + " does not exist for shape " +
                            dims_str(dims_));
    return dims_[index];
}

// src/tensor/strides.rs:9-22
Strides Strides::contiguous(const Shape& shape) {
    const auto& dims = shape.dims();
    Strides s;
    s.values_.assign(dims.size(), 0);
    size_t stride = 1;
    for (size_t i = dims.size(); i-- > 0;) {
        s.values_[i] = stride;
        stride *= dims[i];
    }
    return s;
}

Strides Strides::from_values(std::vector<size_t> values) {
    Strides s;
    s.values_ = std::move(values);
    return s;
}

std::optional<size_t> Strides::get(size_t index) const {
    if (index >= values_.size()) return std::nullopt;
    return values_[index];
}

// ---------------------------------------------------------------- runtime

Context Context::create(int device) {
    rl_context* raw = nullptr;
    check(rl_context_create(device, &raw));
    Context c;
    c.handle_ = std::shared_ptr<rl_context>(raw, [](rl_context* p) { rl_context_destroy(p); });
    return c;
}

void Context::begin_decode_submission_profile() { rl_profile_begin(raw()); }

std::optional<DecodeProfile> Context::take_decode_submission_profile() {
    rl_profile p{};
    if (!rl_profile_take(raw(), &p)) return std::nullopt;
    DecodeProfile d;
    d.command_buffers = p.command_buffers;
    d.compute_encoders = p.compute_encoders;
    d.kernel_dispatches = p.kernel_dispatches;
    d.commits = p.commits;
    d.waits = p.waits;
    d.buffer_allocations = p.buffer_allocations;
    d.allocated_bytes = p.allocated_bytes;
    return d;
}

uint64_t Context::dispatches(const std::string& kernel_name) const {
    return rl_profile_dispatches(raw(), kernel_name.c_str());
}

Buffer::Buffer(const Context& ctx, rl_buffer raw) : ctx_(ctx), raw_(raw) {}

Buffer::~Buffer() {
    if (raw_.data && ctx_.raw()) rl_buffer_release(ctx_.raw(), &raw_);
}

Buffer::Buffer(Buffer&& other) noexcept : ctx_(other.ctx_), raw_(other.raw_) {
    other.raw_ = rl_buffer{nullptr, 0, 0};
}

Buffer& Buffer::operator=(Buffer&& other) noexcept {
    if (this != &other) {
        if (raw_.data && ctx_.raw()) rl_buffer_release(ctx_.raw(), &raw_);
        ctx_ = other.ctx_;
        raw_ = other.raw_;
        other.raw_ = rl_buffer{nullptr, 0, 0};
    }
    return *this;
}

// src/metal/buffer.rs:15-34 (the reference asserts non-empty data)
Buffer Buffer::from_slice(const Context& ctx, const std::vector<float>& data) {
    rl_buffer raw{};
    check(rl_buffer_from_host(ctx.raw(), data.data(), data.size(), 4, &raw));
    return Buffer(ctx, raw);
}

// src/metal/buffer.rs:57-73
Buffer Buffer::from_f16_slice(const Context& ctx, const std::vector<uint16_t>& data) {
    rl_buffer raw{};
    check(rl_buffer_from_host(ctx.raw(), data.data(), data.size(), 2, &raw));
    return Buffer(ctx, raw);
}

// src/metal/buffer.rs:111-126
Buffer Buffer::empty(const Context& ctx, size_t len) { return empty_with_element_size(ctx, len, 4); }

// src/metal/buffer.rs:128-142
Buffer Buffer::empty_with_element_size(const Context& ctx, size_t len, size_t element_size) {
    rl_buffer raw{};
    check(rl_buffer_empty(ctx.raw(), len, element_size, &raw));
    return Buffer(ctx, raw);
}

std::vector<float> Buffer::as_slice() const {
    std::vector<float> out(len());
    check(rl_buffer_to_host(ctx_.raw(), &raw_, out.data(), out.size() * 4));
    return out;
}

std::vector<uint16_t> Buffer::as_f16_slice() const {
    std::vector<uint16_t> out(len());
    check(rl_buffer_to_host(ctx_.raw(), &raw_, out.data(), out.size() * 2));
    return out;
}

// src/metal/execution.rs:11-20
Execution::Execution(const Context& ctx) : ctx_(ctx) { check(rl_execution_begin(ctx.raw())); }

// src/metal/execution.rs:30-36
void Execution::finish() {
    if (finished_) return;
    finished_ = true;
    check(rl_execution_finish(ctx_.raw()));
}

Execution::~Execution() {
    if (!finished_) (void)rl_execution_finish(ctx_.raw());
}

// ----------------------------------------------------------------- tensor

Tensor::Tensor(std::shared_ptr<Storage> storage, Shape shape, Strides strides, DType dtype)
    : storage_(std::move(storage)), shape_(std::move(shape)), strides_(std::move(strides)),
      dtype_(dtype) {}

static std::shared_ptr<Storage> make_storage(Buffer buffer) {
    auto s = std::make_shared<Storage>();
    s->buffer = std::move(buffer);
    return s;
}

// src/tensor/tensor.rs:24-46
Tensor Tensor::from_f32_slice(const Context& ctx, const std::vector<float>& data,
                              const std::vector<size_t>& dims) {
    Shape shape = Shape::create(dims);
    if (data.size() != shape.numel())
        throw TinyError(TinyError::Kind::InvalidShape,
                        "shape " + dims_str(dims) + " requires " + std::to_string(shape.numel()) +
                            " elements, but " + std::to_string(data.size()) + " were provided");
    Strides strides = Strides::contiguous(shape);
    return Tensor(make_storage(Buffer::from_slice(ctx, data)), shape, strides, DType::F32);
}

// src/tensor/tensor.rs:48-68
Tensor Tensor::from_f16_slice(const Context& ctx, const std::vector<uint16_t>& data,
                              const std::vector<size_t>& dims) {
    Shape shape = Shape::create(dims);
    if (data.size() != shape.numel())
        throw TinyError(TinyError::Kind::InvalidShape,
                        "shape " + dims_str(dims) + " requires " + std::to_string(shape.numel()) +
                            " elements, but " + std::to_string(data.size()) + " were provided");
    Strides strides = Strides::contiguous(shape);
    return Tensor(make_storage(Buffer::from_f16_slice(ctx, data)), shape, strides, DType::F16);
}

// src/tensor/tensor.rs:670-684
Tensor Tensor::empty(const Context& ctx, const std::vector<size_t>& dims, DType dtype) {
    Shape shape = Shape::create(dims);
    Strides strides = Strides::contiguous(shape);
    return Tensor(
        make_storage(Buffer::empty_with_element_size(ctx, shape.numel(), size_in_bytes(dtype))),
        shape, strides, dtype);
}

// src/tensor/tensor.rs:203-209
Tensor Tensor::zeros(const Context& ctx, const std::vector<size_t>& dims) {
    Shape shape = Shape::create(dims);
    return from_f32_slice(ctx, std::vector<float>(shape.numel(), 0.0f), dims);
}

// src/tensor/tensor.rs:360-387 (from_metal_buffer)
Tensor Tensor::from_buffer(Buffer buffer, const std::vector<size_t>& dims, DType dtype) {
    Shape shape = Shape::create(dims);
    if (buffer.len() != shape.numel() || buffer.byte_len() != shape.numel() * size_in_bytes(dtype))
        throw TinyError(TinyError::Kind::InvalidShape,
                        "buffer has " + std::to_string(buffer.len()) + " elements, but shape " +
                            dims_str(dims) + " requires " + std::to_string(shape.numel()));
    Strides strides = Strides::contiguous(shape);
    return Tensor(make_storage(std::move(buffer)), shape, strides, dtype);
}

// src/tensor/tensor.rs:251-253
bool Tensor::is_contiguous() const { return strides_ == Strides::contiguous(shape_); }

// src/tensor/tensor.rs:137-157
Tensor Tensor::transpose(size_t dim_a, size_t dim_b) const {
    const size_t r = rank();
    for (size_t d : {dim_a, dim_b})
        if (d >= r)
            throw TinyError(TinyError::Kind::InvalidDimension,
                            "dimension " + std::to_string(d) + " does not exist for rank " +
                                std::to_string(r));
    std::vector<size_t> order(r);
    for (size_t i = 0; i < r; ++i) order[i] = i;
    std::swap(order[dim_a], order[dim_b]);
    return permute(order);
}

// src/tensor/tensor.rs:159-201
Tensor Tensor::permute(const std::vector<size_t>& order) const {
    const size_t r = rank();
    if (order.size() != r)
        throw TinyError(TinyError::Kind::InvalidDimension,
                        "permute order length " + std::to_string(order.size()) +
                            " does not match tensor rank " + std::to_string(r));
    std::vector<bool> seen(r, false);
    for (size_t d : order) {
        if (d >= r)
            throw TinyError(TinyError::Kind::InvalidDimension,
                            "dimension " + std::to_string(d) + " does not exist for rank " +
                                std::to_string(r));
        if (seen[d])
            throw TinyError(TinyError::Kind::InvalidDimension,
                            "dimension " + std::to_string(d) + " appears more than once in permutation");
        seen[d] = true;
    }
    std::vector<size_t> dims(r), strides(r);
    for (size_t i = 0; i < r; ++i) {
        dims[i] = shape_.dims()[order[i]];
        strides[i] = strides_.values()[order[i]];
    }
    return Tensor(storage_, Shape::create(dims), Strides::from_values(strides), dtype_);
}

// src/tensor/tensor.rs:255-280
Tensor Tensor::reshape(const std::vector<size_t>& dims) const {
    Shape shape = Shape::create(dims);
    if (shape.numel() != numel())
        throw TinyError(TinyError::Kind::InvalidShape,
                        "cannot reshape " + dims_str(shape_.dims()) + " into " + dims_str(dims) +
                            ": element count differs");
    if (!is_contiguous())
        throw TinyError(TinyError::Kind::InvalidShape,
                        "cannot reshape a non-contiguous tensor without copying");
    return Tensor(storage_, shape, Strides::contiguous(shape), dtype_);
}

// src/tensor/tensor.rs:283-306: start must be 0 and the parent strides are kept.
Tensor Tensor::narrow(size_t dim, size_t start, size_t len) const {
    if (dim >= rank() || start + len < start || start + len > shape_.dims()[dim])
        throw TinyError(TinyError::Kind::InvalidDimension, "tensor narrow range is out of bounds");
    if (start != 0)
        throw TinyError(TinyError::Kind::InvalidDimension,
                        "tensor narrow currently supports ranges starting at zero");
    std::vector<size_t> dims = shape_.dims();
    dims[dim] = len;
    return Tensor(storage_, Shape::create(dims), strides_, dtype_);
}

// Additive API: a stride-0 broadcast view (numpy rules: size-1 dims stretch,
// missing leading dims are added).  The reference exposes no way to build
// stride 0 (Strides::from_values is crate-private, strides.rs:24).
Tensor Tensor::expand(const std::vector<size_t>& dims) const {
    const size_t r = rank();
    if (dims.size() < r)
        throw TinyError(TinyError::Kind::InvalidShape,
                        "cannot expand " + dims_str(shape_.dims()) + " to " + dims_str(dims));
    const size_t lead = dims.size() - r;
    std::vector<size_t> strides(dims.size(), 0);
    for (size_t i = 0; i < r; ++i) {
        const size_t have = shape_.dims()[i], want = dims[lead + i];
        if (have == want)
            strides[lead + i] = strides_.values()[i];
        else if (have == 1)
            strides[lead + i] = 0;
        else
            throw TinyError(TinyError::Kind::InvalidShape,
                            "cannot expand " + dims_str(shape_.dims()) + " to " + dims_str(dims));
    }
    return Tensor(storage_, Shape::create(dims), Strides::from_values(strides), dtype_);
}

// src/tensor/tensor.rs:70-100
Tensor Tensor::contiguous(const Context& ctx) const {
    if (is_contiguous()) return *this;
    Buffer b = dtype_ == DType::F32
                   ? ops::materialize_contiguous_f32(ctx, buffer(), shape_.dims(), strides_.values())
                   : ops::materialize_contiguous_f16(ctx, buffer(), shape_.dims(), strides_.values());
    return from_buffer(std::move(b), shape_.dims(), dtype_);
}

// src/tensor/tensor.rs:102-135
Tensor Tensor::contiguous_encode(const Context& ctx) const {
    if (is_contiguous()) return *this;
    Buffer b = dtype_ == DType::F32
                   ? ops::materialize_contiguous_f32_encode(ctx, buffer(), shape_.dims(),
                                                            strides_.values())
                   : ops::materialize_contiguous_f16_encode(ctx, buffer(), shape_.dims(),
                                                            strides_.values());
    return from_buffer(std::move(b), shape_.dims(), dtype_);
}

// src/tensor/tensor.rs:308-346 (as_f32_slice / as_f16_slice / to_f32_vec)
std::vector<float> Tensor::to_f32_vec() const {
    if (!is_contiguous())
        throw TinyError(TinyError::Kind::NonContiguousTensor, "shape=" + dims_str(shape_.dims()));
    if (dtype_ == DType::F32) {
        auto v = buffer().as_slice();
        v.resize(numel());
        return v;
    }
    auto h = buffer().as_f16_slice();
    std::vector<float> out(numel());
    for (size_t i = 0; i < out.size(); ++i) out[i] = f16_to_f32(h[i]);
    return out;
}

// src/tensor/tensor.rs:352-354
Tensor Tensor::to_dtype(const Context& ctx, DType dtype) const { return ops::cast(ctx, *this, dtype); }

// A right operand that is a [cols] row seen through stride-0 leading dims.
static bool is_row_broadcast(const Tensor& t) {
    const auto& st = t.strides().values();
    if (st.empty() || st.back() != 1) return false;
    for (size_t i = 0; i + 1 < st.size(); ++i)
        if (st[i] != 0) return false;
    return t.rank() >= 2;
}

static Buffer add_broadcast_encode(const Context& ctx, const Tensor& x, const Tensor& row) {
    const size_t cols = row.shape().dims().back();
    const size_t rows = x.numel() / cols;
    const size_t es = size_in_bytes(x.dtype());
    Buffer out = Buffer::empty_with_element_size(ctx, x.numel(), es);
    rl_buffer bias = *row.buffer().raw();
    bias.len = cols;  // the row is the first `cols` elements of its storage
    bias.byte_len = cols * es;
    check(x.dtype() == DType::F32
              ? rl_add_broadcast_f32(ctx.raw(), x.buffer().raw(), &bias, rows, cols, out.raw())
              : rl_add_broadcast_f16(ctx.raw(), x.buffer().raw(), &bias, rows, cols, out.raw()));
    return out;
}

// src/tensor/elementwise.rs:108-132
Tensor Tensor::binary_elementwise(const Context& ctx, const Tensor& rhs, bool is_add) const {
    if (shape_ != rhs.shape_) throw shape_mismatch(shape_.dims(), rhs.shape_.dims());
    if (is_add && is_contiguous() && is_row_broadcast(rhs)) {
        // contiguous(rhs) then add, in one pass: same values, no materialised copy.
        Execution e(ctx);
        Buffer out = add_broadcast_encode(ctx, *this, rhs);
        e.finish();
        return from_buffer(std::move(out), shape_.dims(), dtype_);
    }
    Tensor lhs = contiguous(ctx);
    Tensor r = rhs.contiguous(ctx);
    Buffer out = dtype_ == DType::F32
                     ? (is_add ? ops::add_f32(ctx, lhs.buffer(), r.buffer())
                               : ops::mul_f32(ctx, lhs.buffer(), r.buffer()))
                     : (is_add ? ops::add_f16(ctx, lhs.buffer(), r.buffer())
                               : ops::mul_f16(ctx, lhs.buffer(), r.buffer()));
    return from_buffer(std::move(out), shape_.dims(), dtype_);
}

// src/tensor/elementwise.rs:61-75
Tensor Tensor::add(const Context& ctx, const Tensor& rhs) const {
    if (dtype_ != rhs.dtype_)
        throw TinyError(TinyError::Kind::UnsupportedDType,
                        std::string("add dtype mismatch: ") + dtype_name(dtype_) + " vs " +
                            dtype_name(rhs.dtype_));
    return binary_elementwise(ctx, rhs, true);
}

// src/tensor/elementwise.rs:76-89
Tensor Tensor::mul(const Context& ctx, const Tensor& rhs) const {
    if (dtype_ != rhs.dtype_)
        throw TinyError(TinyError::Kind::UnsupportedDType,
                        std::string("mul dtype mismatch: ") + dtype_name(dtype_) + " vs " +
                            dtype_name(rhs.dtype_));
    return binary_elementwise(ctx, rhs, false);
}

// src/tensor/elementwise.rs:91-106
Tensor Tensor::silu(const Context& ctx) const {
    Tensor input = contiguous(ctx);
    Buffer out = dtype_ == DType::F32 ? ops::silu_f32(ctx, input.buffer())
                                      : ops::silu_f16(ctx, input.buffer());
    return from_buffer(std::move(out), shape_.dims(), dtype_);
}

// src/tensor/elementwise.rs:134-185
Tensor Tensor::binary_elementwise_encode(const Context& ctx, const Tensor& rhs, bool is_add) const {
    if (dtype_ != rhs.dtype_)
        throw TinyError(TinyError::Kind::UnsupportedDType,
                        std::string("elementwise dtype mismatch: ") + dtype_name(dtype_) + " vs " +
                            dtype_name(rhs.dtype_));
    if (shape_ != rhs.shape_) throw shape_mismatch(shape_.dims(), rhs.shape_.dims());
    if (is_add && is_contiguous() && is_row_broadcast(rhs))
        return from_buffer(add_broadcast_encode(ctx, *this, rhs), shape_.dims(), dtype_);
    if (!is_contiguous() || !rhs.is_contiguous())
        throw TinyError(TinyError::Kind::ModelFormat,
                        "batched elementwise operation requires contiguous tensors");
    Buffer out = dtype_ == DType::F32
                     ? (is_add ? ops::add_f32_encode(ctx, buffer(), rhs.buffer())
                               : ops::mul_f32_encode(ctx, buffer(), rhs.buffer()))
                     : (is_add ? ops::add_f16_encode(ctx, buffer(), rhs.buffer())
                               : ops::mul_f16_encode(ctx, buffer(), rhs.buffer()));
    return from_buffer(std::move(out), shape_.dims(), dtype_);
}

// src/tensor/elementwise.rs:11-26
Tensor Tensor::add_encode(const Context& ctx, const Tensor& rhs) const {
    return binary_elementwise_encode(ctx, rhs, true);
}

// src/tensor/elementwise.rs:27-39
Tensor Tensor::mul_encode(const Context& ctx, const Tensor& rhs) const {
    return binary_elementwise_encode(ctx, rhs, false);
}

// src/tensor/elementwise.rs:41-60
Tensor Tensor::silu_encode(const Context& ctx) const {
    if (!is_contiguous())
        throw TinyError(TinyError::Kind::ModelFormat, "batched SiLU requires a contiguous tensor");
    Buffer out = dtype_ == DType::F32 ? ops::silu_f32_encode(ctx, buffer())
                                      : ops::silu_f16_encode(ctx, buffer());
    return from_buffer(std::move(out), shape_.dims(), dtype_);
}

// src/tensor/tensor.rs:458-466
Tensor Tensor::softmax_last_dim(const Context& ctx) const {
    Execution e(ctx);
    Tensor out = softmax_last_dim_encode(ctx);
    e.finish();
    return out;
}

// src/tensor/tensor.rs:468-495
Tensor Tensor::softmax_last_dim_encode(const Context& ctx) const {
    if (rank() == 0)
        throw TinyError(TinyError::Kind::InvalidDimension, "Softmax requires at least one dimension");
    Tensor input = contiguous_encode(ctx);
    const size_t width = input.dim(input.rank() - 1);
    const size_t rows = input.numel() / width;
    Buffer out = dtype_ == DType::F32 ? ops::softmax_f32_encode(ctx, input.buffer(), rows, width)
                                      : ops::softmax_f16_encode(ctx, input.buffer(), rows, width);
    return from_buffer(std::move(out), input.shape().dims(), dtype_);
}

// src/tensor/tensor.rs:604-622
Tensor Tensor::attention_scale_mask(const Context& ctx, float scale, size_t query_start_pos) const {
    Execution e(ctx);
    Tensor out = attention_scale_mask_encode(ctx, scale, query_start_pos);
    e.finish();
    return out;
}

// src/tensor/tensor.rs:624-668
Tensor Tensor::attention_scale_mask_encode(const Context& ctx, float scale,
                                           size_t query_start_pos) const {
    if (rank() < 2)
        throw TinyError(TinyError::Kind::InvalidDimension,
                        "attention scores require rank >= 2, got rank " + std::to_string(rank()));
    const size_t query_len = dim(rank() - 2), key_len = dim(rank() - 1);
    Tensor input = contiguous_encode(ctx);
    Buffer out = dtype_ == DType::F32
                     ? ops::attention_scale_mask_f32_encode(ctx, input.buffer(), scale, query_len,
                                                            key_len, query_start_pos)
                     : ops::attention_scale_mask_f16_encode(ctx, input.buffer(), scale, query_len,
                                                            key_len, query_start_pos);
    return from_buffer(std::move(out), input.shape().dims(), dtype_);
}

// The two adjacent calls of src/nn/attention.rs:233-240 in one kernel.
Tensor Tensor::attention_softmax_encode(const Context& ctx, float scale,
                                        size_t query_start_pos) const {
    if (rank() < 2)
        throw TinyError(TinyError::Kind::InvalidDimension,
                        "attention scores require rank >= 2, got rank " + std::to_string(rank()));
    const size_t query_len = dim(rank() - 2), key_len = dim(rank() - 1);
    Tensor input = contiguous_encode(ctx);
    const size_t es = size_in_bytes(dtype_);
    Buffer out = Buffer::empty_with_element_size(ctx, input.numel(), es);
    check(dtype_ == DType::F32
              ? rl_attention_softmax_f32(ctx.raw(), input.buffer().raw(), scale, query_len, key_len,
                                         query_start_pos, out.raw())
              : rl_attention_softmax_f16(ctx.raw(), input.buffer().raw(), scale, query_len, key_len,
                                         query_start_pos, out.raw()));
    return from_buffer(std::move(out), input.shape().dims(), dtype_);
}

// src/tensor/repeat_kv.rs:13-81 (the reference submits and waits on its own).
Tensor Tensor::repeat_kv(const Context& ctx, size_t repeats) const {
    if (rank() != 4)
        throw TinyError(TinyError::Kind::ModelFormat,
                        "repeat_kv expects [B, KVH, S, D], got " + dims_str(shape_.dims()));
    if (repeats == 0)
        throw TinyError(TinyError::Kind::ModelFormat, "repeat_kv repeats must be greater than zero");
    if (repeats == 1) return *this;
    Tensor input = is_contiguous() ? *this : contiguous(ctx);
    const size_t batch = input.dim(0), kv_heads = input.dim(1), seq = input.dim(2),
                 head_dim = input.dim(3);
    if (kv_heads > SIZE_MAX / repeats)
        throw TinyError(TinyError::Kind::ModelFormat, "repeat_kv head count overflow");
    Tensor output = Tensor::empty(ctx, {batch, kv_heads * repeats, seq, head_dim}, dtype_);
    Execution e(ctx);
    check(dtype_ == DType::F32
              ? rl_repeat_kv_f32(ctx.raw(), input.buffer().raw(), batch, kv_heads, seq, head_dim,
                                 repeats, output.buffer().raw())
              : rl_repeat_kv_f16(ctx.raw(), input.buffer().raw(), batch, kv_heads, seq, head_dim,
                                 repeats, output.buffer().raw()));
    e.finish();
    return output;
}

// src/tensor/gqa_matmul.rs:135-182 (validate_qk / validate_pv and their helpers).
static void validate_gqa(const Tensor& left, const Tensor& right, const char* op,
                         const char* expected) {
    if (left.dtype() != right.dtype())
        throw TinyError(TinyError::Kind::UnsupportedDType,
                        std::string("GQA ") + op + " dtype mismatch: " + dtype_name(left.dtype()) +
                            " vs " + dtype_name(right.dtype()));
    if (left.rank() != 4 || right.rank() != 4)
        throw TinyError(TinyError::Kind::ModelFormat,
                        std::string("GQA ") + op + " expects " + expected + ", got " +
                            dims_str(left.shape().dims()) + " and " + dims_str(right.shape().dims()));
}

static void validate_head_groups(size_t q_heads, size_t kv_heads) {
    if (kv_heads == 0 || q_heads % kv_heads != 0)
        throw TinyError(TinyError::Kind::ModelFormat,
                        "Q heads " + std::to_string(q_heads) +
                            " must be divisible by non-zero KV heads " + std::to_string(kv_heads));
}

// A one-query [B, H, 1, D] view whose elements lie as in the contiguous
// tensor (the head permutation of a [B, 1, H * D] projection).
static bool one_query_in_place(const Tensor& q) {
    const auto& st = q.strides().values();
    return q.dim(2) == 1 && st[3] == 1 && st[1] == q.dim(3) &&
           (q.dim(0) == 1 || st[0] == q.dim(1) * q.dim(3)) && q.buffer().len() == q.numel();
}

// A [B, H, S, D] operand the kernels can read in place: contiguous, or rows of
// D elements with unit stride laid out as whole heads of `capacity` rows
// (a narrowed LayerKvCache view).  Returns the capacity, 0 if not.
static size_t rows_in_place(const Tensor& t) {
    const auto& st = t.strides().values();
    const size_t heads = t.dim(1), d = t.dim(3);
    if (st[3] != 1 || st[2] != d || st[1] % d != 0) return 0;
    const size_t capacity = st[1] / d;
    if (capacity < t.dim(2) || (t.dim(0) > 1 && st[0] != heads * st[1])) return 0;
    if (t.buffer().len() != t.dim(0) * heads * capacity * d) return 0;
    return capacity;
}

Tensor Tensor::gqa_qk_matmul(const Context& ctx, const Tensor& key) const {
    Execution e(ctx);
    Tensor out = gqa_qk_matmul_encode(ctx, key);
    e.finish();
    return out;
}

// src/tensor/gqa_matmul.rs:23-61
Tensor Tensor::gqa_qk_matmul_encode(const Context& ctx, const Tensor& key) const {
    validate_gqa(*this, key, "QK", "Q [B,QH,Q,D] and K [B,KVH,K,D]");
    const size_t batch = dim(0), q_heads = dim(1), q_len = dim(2), head_dim = dim(3);
    if (batch != key.dim(0) || head_dim != key.dim(3))
        throw shape_mismatch(shape_.dims(), key.shape().dims());
    const size_t kv_heads = key.dim(1), kv_len = key.dim(2);
    validate_head_groups(q_heads, kv_heads);
    // A one-query head permutation is layout-equivalent to the contiguous
    // tensor on device (gqa_matmul.rs:31-42); prefill makes both contiguous.
    const bool one = q_len == 1;
    const Tensor q = is_contiguous() || one_query_in_place(*this) ? *this : contiguous_encode(ctx);
    size_t capacity = one ? rows_in_place(key) : 0;
    const Tensor k = capacity ? key : key.contiguous_encode(ctx);
    if (!capacity) capacity = kv_len;
    Tensor out = Tensor::empty(ctx, {batch, q_heads, q_len, kv_len}, dtype_);
    check(dtype_ == DType::F32
              ? rl_gqa_qk_matmul_f32(ctx.raw(), q.buffer().raw(), k.buffer().raw(), batch, q_heads,
                                     kv_heads, q_len, kv_len, head_dim, capacity,
                                     out.buffer().raw())
              : rl_gqa_qk_matmul_f16(ctx.raw(), q.buffer().raw(), k.buffer().raw(), batch, q_heads,
                                     kv_heads, q_len, kv_len, head_dim, capacity,
                                     out.buffer().raw()));
    return out;
}

Tensor Tensor::gqa_pv_matmul(const Context& ctx, const Tensor& value) const {
    Execution e(ctx);
    Tensor out = gqa_pv_matmul_encode(ctx, value);
    e.finish();
    return out;
}

// src/tensor/gqa_matmul.rs:72-110
Tensor Tensor::gqa_pv_matmul_encode(const Context& ctx, const Tensor& value) const {
    validate_gqa(*this, value, "PV", "P [B,QH,Q,K] and V [B,KVH,K,D]");
    const size_t batch = dim(0), q_heads = dim(1), q_len = dim(2), kv_len = dim(3);
    if (batch != value.dim(0) || kv_len != value.dim(2))
        throw shape_mismatch(shape_.dims(), value.shape().dims());
    const size_t kv_heads = value.dim(1), head_dim = value.dim(3);
    validate_head_groups(q_heads, kv_heads);
    const Tensor probs = is_contiguous() ? *this : contiguous_encode(ctx);
    size_t capacity = q_len == 1 ? rows_in_place(value) : 0;
    const Tensor v = capacity ? value : value.contiguous_encode(ctx);
    if (!capacity) capacity = kv_len;
    Tensor out = Tensor::empty(ctx, {batch, q_heads, q_len, head_dim}, dtype_);
    check(dtype_ == DType::F32
              ? rl_gqa_pv_matmul_f32(ctx.raw(), probs.buffer().raw(), v.buffer().raw(), batch,
                                     q_heads, kv_heads, q_len, kv_len, head_dim, capacity,
                                     out.buffer().raw())
              : rl_gqa_pv_matmul_f16(ctx.raw(), probs.buffer().raw(), v.buffer().raw(), batch,
                                     q_heads, kv_heads, q_len, kv_len, head_dim, capacity,
                                     out.buffer().raw()));
    return out;
}

// -------------------------------------------------------------------- ops

namespace ops {

template <typename Fn>
static Buffer synced(const Context& ctx, Fn fn) {
    Execution e(ctx);
    Buffer out = fn();
    e.finish();
    return out;
}

static Buffer binary(const Context& ctx, const Buffer& a, size_t es,
                     rl_status (*op)(rl_context*, const rl_buffer*, const rl_buffer*,
                                     const rl_buffer*),
                     const Buffer& b) {
    Buffer out = Buffer::empty_with_element_size(ctx, a.len(), es);
    check(op(ctx.raw(), a.raw(), b.raw(), out.raw()));
    return out;
}

// src/ops/add.rs:18-101, src/ops/mul.rs:20-119
Buffer add_f32_encode(const Context& ctx, const Buffer& a, const Buffer& b) {
    return binary(ctx, a, 4, rl_add_f32, b);
}
Buffer add_f16_encode(const Context& ctx, const Buffer& a, const Buffer& b) {
    return binary(ctx, a, 2, rl_add_f16, b);
}
Buffer mul_f32_encode(const Context& ctx, const Buffer& a, const Buffer& b) {
    return binary(ctx, a, 4, rl_mul_f32, b);
}
Buffer mul_f16_encode(const Context& ctx, const Buffer& a, const Buffer& b) {
    return binary(ctx, a, 2, rl_mul_f16, b);
}
Buffer add_f32(const Context& ctx, const Buffer& a, const Buffer& b) {
    return synced(ctx, [&] { return add_f32_encode(ctx, a, b); });
}
Buffer add_f16(const Context& ctx, const Buffer& a, const Buffer& b) {
    return synced(ctx, [&] { return add_f16_encode(ctx, a, b); });
}
Buffer mul_f32(const Context& ctx, const Buffer& a, const Buffer& b) {
    return synced(ctx, [&] { return mul_f32_encode(ctx, a, b); });
}
Buffer mul_f16(const Context& ctx, const Buffer& a, const Buffer& b) {
    return synced(ctx, [&] { return mul_f16_encode(ctx, a, b); });
}

// src/ops/silu.rs:20-109 (the reference rejects an empty input; an empty
// output buffer cannot even be allocated, so the check comes first here)
static Buffer unary(const Context& ctx, const Buffer& input, size_t es,
                    rl_status (*op)(rl_context*, const rl_buffer*, const rl_buffer*)) {
    if (input.is_empty())
        throw TinyError(TinyError::Kind::InvalidShape, "SiLU input cannot be empty");
    Buffer out = Buffer::empty_with_element_size(ctx, input.len(), es);
    check(op(ctx.raw(), input.raw(), out.raw()));
    return out;
}
Buffer silu_f32_encode(const Context& ctx, const Buffer& input) {
    return unary(ctx, input, 4, rl_silu_f32);
}
Buffer silu_f16_encode(const Context& ctx, const Buffer& input) {
    return unary(ctx, input, 2, rl_silu_f16);
}
Buffer silu_f32(const Context& ctx, const Buffer& input) {
    return synced(ctx, [&] { return silu_f32_encode(ctx, input); });
}
Buffer silu_f16(const Context& ctx, const Buffer& input) {
    return synced(ctx, [&] { return silu_f16_encode(ctx, input); });
}

// src/ops/swiglu.rs:8-45
Buffer swiglu_f16_encode(const Context& ctx, const Buffer& gate, const Buffer& up) {
    return binary(ctx, gate, 2, rl_swiglu_f16, up);
}
Buffer swiglu_f16(const Context& ctx, const Buffer& gate, const Buffer& up) {
    return synced(ctx, [&] { return swiglu_f16_encode(ctx, gate, up); });
}
Buffer swiglu_f32_encode(const Context& ctx, const Buffer& gate, const Buffer& up) {
    return binary(ctx, gate, 4, rl_swiglu_f32, up);
}

// src/ops/cast.rs:10-83
Tensor cast(const Context& ctx, const Tensor& input, DType dtype) {
    if (input.dtype() == dtype) return input;
    Tensor src = input.is_contiguous() ? input : input.contiguous(ctx);
    Tensor output = Tensor::empty(ctx, src.shape().dims(), dtype);
    Execution e(ctx);
    check(dtype == DType::F16 ? rl_cast_f32_to_f16(ctx.raw(), src.buffer().raw(), output.buffer().raw())
                              : rl_cast_f16_to_f32(ctx.raw(), src.buffer().raw(), output.buffer().raw()));
    e.finish();
    return output;
}

// src/ops/contiguous.rs:85-154
static Buffer contiguous_encode(const Context& ctx, const Buffer& source,
                                const std::vector<size_t>& dims, const std::vector<size_t>& strides,
                                size_t es) {
    if (dims.size() != strides.size())
        throw TinyError(TinyError::Kind::InvalidShape, "shape rank and strides rank differ");
    size_t numel = 1;
    for (size_t d : dims) numel *= d;
    Buffer out = Buffer::empty_with_element_size(ctx, numel, es);
    std::vector<uint64_t> d64(dims.begin(), dims.end()), s64(strides.begin(), strides.end());
    check(es == 4 ? rl_contiguous_f32(ctx.raw(), source.raw(), d64.data(), s64.data(),
                                      uint32_t(dims.size()), out.raw())
                  : rl_contiguous_f16(ctx.raw(), source.raw(), d64.data(), s64.data(),
                                      uint32_t(dims.size()), out.raw()));
    return out;
}
Buffer materialize_contiguous_f32_encode(const Context& ctx, const Buffer& source,
                                         const std::vector<size_t>& dims,
                                         const std::vector<size_t>& strides) {
    return contiguous_encode(ctx, source, dims, strides, 4);
}
Buffer materialize_contiguous_f16_encode(const Context& ctx, const Buffer& source,
                                         const std::vector<size_t>& dims,
                                         const std::vector<size_t>& strides) {
    return contiguous_encode(ctx, source, dims, strides, 2);
}
Buffer materialize_contiguous_f32(const Context& ctx, const Buffer& source,
                                  const std::vector<size_t>& dims,
                                  const std::vector<size_t>& strides) {
    return synced(ctx, [&] { return contiguous_encode(ctx, source, dims, strides, 4); });
}
Buffer materialize_contiguous_f16(const Context& ctx, const Buffer& source,
                                  const std::vector<size_t>& dims,
                                  const std::vector<size_t>& strides) {
    return synced(ctx, [&] { return contiguous_encode(ctx, source, dims, strides, 2); });
}

// src/ops/rmsnorm.rs:38-206
static Buffer rmsnorm_encode(const Context& ctx, const Buffer& input, const Buffer& weight,
                             size_t rows, size_t hidden, float eps, size_t es) {
    Buffer out = Buffer::empty_with_element_size(ctx, input.len() ? input.len() : 1, es);
    if (input.len() == 0) throw TinyError(TinyError::Kind::InvalidShape, "RMSNorm input is empty");
    check(es == 4 ? rl_rmsnorm_f32(ctx.raw(), input.raw(), weight.raw(), rows, hidden, eps, out.raw())
                  : rl_rmsnorm_f16(ctx.raw(), input.raw(), weight.raw(), rows, hidden, eps,
                                   out.raw()));
    return out;
}
Buffer rmsnorm_f32_encode(const Context& ctx, const Buffer& input, const Buffer& weight,
                          size_t rows, size_t hidden_size, float epsilon) {
    return rmsnorm_encode(ctx, input, weight, rows, hidden_size, epsilon, 4);
}
Buffer rmsnorm_f16_encode(const Context& ctx, const Buffer& input, const Buffer& weight,
                          size_t rows, size_t hidden_size, float epsilon) {
    return rmsnorm_encode(ctx, input, weight, rows, hidden_size, epsilon, 2);
}
Buffer rmsnorm_f32(const Context& ctx, const Buffer& input, const Buffer& weight, size_t rows,
                   size_t hidden_size, float epsilon) {
    return synced(ctx, [&] { return rmsnorm_encode(ctx, input, weight, rows, hidden_size, epsilon, 4); });
}
Buffer rmsnorm_f16(const Context& ctx, const Buffer& input, const Buffer& weight, size_t rows,
                   size_t hidden_size, float epsilon) {
    return synced(ctx, [&] { return rmsnorm_encode(ctx, input, weight, rows, hidden_size, epsilon, 2); });
}

// src/ops/rmsnorm.rs:208-272
Tensor rmsnorm(const Context& ctx, const Tensor& input, const Tensor& weight, float epsilon) {
    if (input.dtype() != weight.dtype())
        throw TinyError(TinyError::Kind::UnsupportedDType,
                        std::string("RMSNorm dtype mismatch: input ") + dtype_name(input.dtype()) +
                            ", weight " + dtype_name(weight.dtype()));
    if (input.rank() == 0)
        throw TinyError(TinyError::Kind::InvalidDimension,
                        "RMSNorm input must have at least one dimension");
    if (!std::isfinite(epsilon) || epsilon <= 0.0f)
        throw TinyError(TinyError::Kind::InvalidShape,
                        "RMSNorm epsilon must be positive and finite, got " + std::to_string(epsilon));
    const size_t hidden = input.dim(input.rank() - 1);
    if (weight.rank() != 1 || weight.numel() != hidden)
        throw shape_mismatch(input.shape().dims(), weight.shape().dims());
    if (input.dtype() == DType::F16 && (!input.is_contiguous() || !weight.is_contiguous()))
        throw TinyError(TinyError::Kind::NonContiguousTensor,
                        "F16 RMSNorm currently requires contiguous input and weight");
    Tensor in = input.contiguous(ctx);
    Tensor w = weight.contiguous(ctx);
    const size_t rows = in.numel() / hidden;
    Buffer out = input.dtype() == DType::F32
                     ? rmsnorm_f32(ctx, in.buffer(), w.buffer(), rows, hidden, epsilon)
                     : rmsnorm_f16(ctx, in.buffer(), w.buffer(), rows, hidden, epsilon);
    return Tensor::from_buffer(std::move(out), in.shape().dims(), in.dtype());
}

// src/ops/softmax.rs:27-89
Buffer softmax_f32_encode(const Context& ctx, const Buffer& input, size_t rows, size_t width) {
    Buffer out = Buffer::empty_with_element_size(ctx, input.len() ? input.len() : 1, 4);
    check(rl_softmax_f32(ctx.raw(), input.raw(), rows, width, out.raw()));
    return out;
}
Buffer softmax_f16_encode(const Context& ctx, const Buffer& input, size_t rows, size_t width) {
    Buffer out = Buffer::empty_with_element_size(ctx, input.len() ? input.len() : 1, 2);
    check(rl_softmax_f16(ctx.raw(), input.raw(), rows, width, out.raw()));
    return out;
}
Buffer softmax_f32(const Context& ctx, const Buffer& input, size_t rows, size_t width) {
    return synced(ctx, [&] { return softmax_f32_encode(ctx, input, rows, width); });
}
Buffer softmax_f16(const Context& ctx, const Buffer& input, size_t rows, size_t width) {
    return synced(ctx, [&] { return softmax_f16_encode(ctx, input, rows, width); });
}

// src/ops/attention_scale_mask.rs:35-116
Buffer attention_scale_mask_f32_encode(const Context& ctx, const Buffer& input, float scale,
                                       size_t query_len, size_t key_len, size_t query_start_pos) {
    Buffer out = Buffer::empty_with_element_size(ctx, input.len() ? input.len() : 1, 4);
    check(rl_attention_scale_mask_f32(ctx.raw(), input.raw(), scale, query_len, key_len,
                                      query_start_pos, out.raw()));
    return out;
}
Buffer attention_scale_mask_f16_encode(const Context& ctx, const Buffer& input, float scale,
                                       size_t query_len, size_t key_len, size_t query_start_pos) {
    Buffer out = Buffer::empty_with_element_size(ctx, input.len() ? input.len() : 1, 2);
    check(rl_attention_scale_mask_f16(ctx.raw(), input.raw(), scale, query_len, key_len,
                                      query_start_pos, out.raw()));
    return out;
}
Buffer attention_scale_mask_f32(const Context& ctx, const Buffer& input, float scale,
                                size_t query_len, size_t key_len, size_t query_start_pos) {
    return synced(ctx, [&] {
        return attention_scale_mask_f32_encode(ctx, input, scale, query_len, key_len,
                                               query_start_pos);
    });
}
Buffer attention_scale_mask_f16(const Context& ctx, const Buffer& input, float scale,
                                size_t query_len, size_t key_len, size_t query_start_pos) {
    return synced(ctx, [&] {
        return attention_scale_mask_f16_encode(ctx, input, scale, query_len, key_len,
                                               query_start_pos);
    });
}

// src/ops/rope.rs:11-277
static Buffer rope_buffer_encode(const Context& ctx, const Buffer& input, const Buffer& cos,
                                 const Buffer& sin, size_t seq_len, size_t head_dim, size_t start,
                                 size_t es) {
    Buffer out = Buffer::empty_with_element_size(ctx, input.len() ? input.len() : 1, es);
    check(es == 4 ? rl_rope_f32(ctx.raw(), input.raw(), cos.raw(), sin.raw(), seq_len, head_dim,
                                start, out.raw())
                  : rl_rope_f16(ctx.raw(), input.raw(), cos.raw(), sin.raw(), seq_len, head_dim,
                                start, out.raw()));
    return out;
}
Buffer rope_f32(const Context& ctx, const Buffer& input, const Buffer& cos_table,
                const Buffer& sin_table, size_t seq_len, size_t head_dim, size_t start_pos) {
    return synced(ctx, [&] {
        return rope_buffer_encode(ctx, input, cos_table, sin_table, seq_len, head_dim, start_pos, 4);
    });
}
Buffer rope_f16(const Context& ctx, const Buffer& input, const Buffer& cos_table,
                const Buffer& sin_table, size_t seq_len, size_t head_dim, size_t start_pos) {
    return synced(ctx, [&] {
        return rope_buffer_encode(ctx, input, cos_table, sin_table, seq_len, head_dim, start_pos, 2);
    });
}

// src/ops/rope.rs:279-300
Tensor rope(const Context& ctx, const Tensor& input, const Tensor& cos, const Tensor& sin,
            size_t start_pos) {
    Execution e(ctx);
    Tensor out = rope_encode(ctx, input, cos, sin, start_pos);
    e.finish();
    return out;
}

// src/ops/rope.rs:303-370.  A strided input with a unit innermost stride is
// gathered and rotated by one kernel instead of contiguous_encode + rope.
// ops::rope_encode's checks (src/ops/rope.rs:303-343) in order.
void validate_rope(const Tensor& input, const Tensor& cos, const Tensor& sin, size_t start_pos) {
    if (cos.dtype() != DType::F32 || sin.dtype() != DType::F32)
        throw TinyError(TinyError::Kind::UnsupportedDType, "RoPE requires F32 cos/sin tables");
    if (input.rank() < 2)
        throw TinyError(TinyError::Kind::InvalidDimension,
                        "RoPE expects [..., sequence, head_dim], got rank " +
                            std::to_string(input.rank()));
    const size_t seq_len = input.dim(input.rank() - 2), head_dim = input.dim(input.rank() - 1);
    if (head_dim == 0 || head_dim % 2 != 0)
        throw TinyError(TinyError::Kind::InvalidShape,
                        "RoPE head dimension must be positive and even, got " +
                            std::to_string(head_dim));
    if (cos.rank() != 2 || sin.rank() != 2 || cos.shape() != sin.shape())
        throw TinyError(TinyError::Kind::InvalidShape,
                        "RoPE cos/sin tables must have equal rank-2 shapes");
    const size_t table_rows = cos.dim(0);
    if (cos.dim(1) != head_dim / 2 || start_pos + seq_len < start_pos ||
        start_pos + seq_len > table_rows)
        throw TinyError(TinyError::Kind::InvalidShape,
                        "RoPE cos/sin table shape or position range is invalid");
}

Tensor rope_encode(const Context& ctx, const Tensor& input, const Tensor& cos, const Tensor& sin,
                   size_t start_pos) {
    validate_rope(input, cos, sin, start_pos);
    const size_t seq_len = input.dim(input.rank() - 2), head_dim = input.dim(input.rank() - 1);
    const size_t table_rows = cos.dim(0);
    const size_t es = size_in_bytes(input.dtype());
    if (!input.is_contiguous() && input.strides().values().back() == 1) {
        Buffer out = Buffer::empty_with_element_size(ctx, input.numel(), es);
        std::vector<uint64_t> d(input.shape().dims().begin(), input.shape().dims().end());
        std::vector<uint64_t> s(input.strides().values().begin(), input.strides().values().end());
        check(input.dtype() == DType::F32
                  ? rl_rope_strided_f32(ctx.raw(), input.buffer().raw(), d.data(), s.data(),
                                        uint32_t(d.size()), cos.buffer().raw(), sin.buffer().raw(),
                                        table_rows, start_pos, out.raw())
                  : rl_rope_strided_f16(ctx.raw(), input.buffer().raw(), d.data(), s.data(),
                                        uint32_t(d.size()), cos.buffer().raw(), sin.buffer().raw(),
                                        table_rows, start_pos, out.raw()));
        return Tensor::from_buffer(std::move(out), input.shape().dims(), input.dtype());
    }
    Tensor in = input.contiguous_encode(ctx);
    Buffer out = rope_buffer_encode(ctx, in.buffer(), cos.buffer(), sin.buffer(), seq_len, head_dim,
                                    start_pos, es);
    return Tensor::from_buffer(std::move(out), in.shape().dims(), in.dtype());
}

std::pair<Tensor, Tensor> add_rmsnorm_encode(const Context& ctx, const Tensor& x,
                                             const Tensor& residual, const Tensor& weight,
                                             float epsilon) {
    if (x.dtype() != residual.dtype() || x.dtype() != weight.dtype())
        throw TinyError(TinyError::Kind::UnsupportedDType, "add + RMSNorm dtype mismatch");
    if (x.shape() != residual.shape()) throw shape_mismatch(x.shape().dims(), residual.shape().dims());
    if (x.rank() != 2 || !x.is_contiguous() || !residual.is_contiguous() || !weight.is_contiguous())
        throw TinyError(TinyError::Kind::ModelFormat, "invalid batched RMSNorm input");
    const size_t rows = x.dim(0), hidden = x.dim(1);
    const size_t es = size_in_bytes(x.dtype());
    Buffer sum = Buffer::empty_with_element_size(ctx, x.numel(), es);
    Buffer norm = Buffer::empty_with_element_size(ctx, x.numel(), es);
    check(es == 4 ? rl_add_rmsnorm_f32(ctx.raw(), x.buffer().raw(), residual.buffer().raw(),
                                       weight.buffer().raw(), rows, hidden, epsilon, sum.raw(),
                                       norm.raw())
                  : rl_add_rmsnorm_f16(ctx.raw(), x.buffer().raw(), residual.buffer().raw(),
                                       weight.buffer().raw(), rows, hidden, epsilon, sum.raw(),
                                       norm.raw()));
    return {Tensor::from_buffer(std::move(sum), x.shape().dims(), x.dtype()),
            Tensor::from_buffer(std::move(norm), x.shape().dims(), x.dtype())};
}

// src/ops/embedding.rs:10-193.  The library validates the ids and copies
// them to the device in stream order.
static Buffer embedding_encode(const Context& ctx, const Buffer& weight,
                               const std::vector<uint32_t>& token_ids, size_t vocab_size,
                               size_t hidden_size, DType dtype) {
    const size_t es = size_in_bytes(dtype);
    Buffer out;
    if (token_ids.empty()) {  // the library reports the reference's error
        const rl_buffer none{nullptr, 0, 0};
        check(dtype == DType::F32
                  ? rl_embedding_f32(ctx.raw(), weight.raw(), vocab_size, hidden_size,
                                     token_ids.data(), 0, &none)
                  : rl_embedding_f16(ctx.raw(), weight.raw(), vocab_size, hidden_size,
                                     token_ids.data(), 0, &none));
    }
    out = Buffer::empty_with_element_size(ctx, token_ids.size() * hidden_size, es);
    check(dtype == DType::F32
              ? rl_embedding_f32(ctx.raw(), weight.raw(), vocab_size, hidden_size,
                                 token_ids.data(), token_ids.size(), out.raw())
              : rl_embedding_f16(ctx.raw(), weight.raw(), vocab_size, hidden_size,
                                 token_ids.data(), token_ids.size(), out.raw()));
    return out;
}

Buffer embedding_f32_encode(const Context& ctx, const Buffer& weight,
                            const std::vector<uint32_t>& token_ids, size_t vocab_size,
                            size_t hidden_size) {
    return embedding_encode(ctx, weight, token_ids, vocab_size, hidden_size, DType::F32);
}

Buffer embedding_f16_encode(const Context& ctx, const Buffer& weight,
                            const std::vector<uint32_t>& token_ids, size_t vocab_size,
                            size_t hidden_size) {
    return embedding_encode(ctx, weight, token_ids, vocab_size, hidden_size, DType::F16);
}

Buffer embedding_f32(const Context& ctx, const Buffer& weight,
                     const std::vector<uint32_t>& token_ids, size_t vocab_size,
                     size_t hidden_size) {
    Execution exe(ctx);
    Buffer out = embedding_f32_encode(ctx, weight, token_ids, vocab_size, hidden_size);
    exe.finish();
    return out;
}

Buffer embedding_f16(const Context& ctx, const Buffer& weight,
                     const std::vector<uint32_t>& token_ids, size_t vocab_size,
                     size_t hidden_size) {
    Execution exe(ctx);
    Buffer out = embedding_f16_encode(ctx, weight, token_ids, vocab_size, hidden_size);
    exe.finish();
    return out;
}

// kv_cache_write_encode (src/ops/kv_cache_write.rs:71-141), Tensor-level
// checks in order; the buffer-level ones are repeated by the library.
static void kv_cache_write_tensor_encode(const Context& ctx, const Tensor& cache,
                                         const Tensor& source, size_t start, DType dtype,
                                         const char* kernel_name) {
    if (cache.dtype() != dtype || source.dtype() != dtype)
        throw TinyError(TinyError::Kind::UnsupportedDType,
                        std::string(kernel_name) + " expects " + dtype_name(dtype) +
                            " cache and source, got " + dtype_name(cache.dtype()) + " and " +
                            dtype_name(source.dtype()));
    if (cache.rank() != 4 || source.rank() != 4 || cache.dim(0) != 1 || source.dim(0) != 1 ||
        cache.dim(1) != source.dim(1) || cache.dim(3) != source.dim(3))
        throw TinyError(TinyError::Kind::InvalidShape, "invalid KV cache write shape");
    const size_t seq = source.dim(2), max_seq = cache.dim(2);
    if (start + seq < start || start + seq > max_seq)
        throw TinyError::position_out_of_range(start, seq, max_seq);
    if (!source.is_contiguous())
        throw TinyError(TinyError::Kind::NonContiguousTensor,
                        "batched KV cache write requires a contiguous source");
    check(dtype == DType::F32
              ? rl_kv_cache_write_f32(ctx.raw(), cache.buffer().raw(), cache.dim(1), max_seq,
                                      cache.dim(3), source.buffer().raw(), seq, start)
              : rl_kv_cache_write_f16(ctx.raw(), cache.buffer().raw(), cache.dim(1), max_seq,
                                      cache.dim(3), source.buffer().raw(), seq, start));
}

void kv_cache_write_f32_encode(const Context& ctx, const Tensor& cache, const Tensor& source,
                               size_t start) {
    kv_cache_write_tensor_encode(ctx, cache, source, start, DType::F32, "kv_cache_write_f32");
}

void kv_cache_write_f16_encode(const Context& ctx, const Tensor& cache, const Tensor& source,
                               size_t start) {
    kv_cache_write_tensor_encode(ctx, cache, source, start, DType::F16, "kv_cache_write_f16");
}

void kv_cache_write_f32(const Context& ctx, const Tensor& cache, const Tensor& source,
                        size_t start) {  // kv_cache_write.rs:9-20
    Execution exe(ctx);
    Tensor src = source.contiguous_encode(ctx);
    kv_cache_write_f32_encode(ctx, cache, src, start);
    exe.finish();
}

void kv_cache_write_f16(const Context& ctx, const Tensor& cache, const Tensor& source,
                        size_t start) {  // kv_cache_write.rs:43-54
    Execution exe(ctx);
    Tensor src = source.contiguous_encode(ctx);
    kv_cache_write_f16_encode(ctx, cache, src, start);
    exe.finish();
}

}  // namespace ops

// --------------------------------------------------------------------- nn

namespace nn {

// src/nn/rmsnorm.rs:15-41
RmsNorm::RmsNorm(Tensor weight, float epsilon)
    : weight_(std::move(weight)), hidden_size_(0), epsilon_(epsilon) {
    if (weight_.rank() != 1)
        throw TinyError(TinyError::Kind::InvalidDimension,
                        "RMSNorm weight must have rank 1, got rank " + std::to_string(weight_.rank()));
    if (!std::isfinite(epsilon) || epsilon <= 0.0f)
        throw TinyError(TinyError::Kind::InvalidShape,
                        "RMSNorm epsilon must be positive, got " + std::to_string(epsilon));
    hidden_size_ = weight_.dim(0);
}

// src/nn/rmsnorm.rs:56-66
Tensor RmsNorm::forward(const Context& ctx, const Tensor& input) const {
    if (input.dtype() != weight_.dtype())
        throw TinyError(TinyError::Kind::UnsupportedDType,
                        std::string("RMSNorm input dtype ") + dtype_name(input.dtype()) +
                            " does not match weight dtype " + dtype_name(weight_.dtype()));
    return ops::rmsnorm(ctx, input, weight_, epsilon_);
}

// src/nn/rmsnorm.rs:68-105
Tensor RmsNorm::forward_encode(const Context& ctx, const Tensor& input) const {
    if (input.dtype() != weight_.dtype() || input.rank() != 2 || input.dim(1) != hidden_size_ ||
        !input.is_contiguous())
        throw TinyError(TinyError::Kind::ModelFormat, "invalid batched RMSNorm input");
    const size_t rows = input.dim(0);
    Buffer out = input.dtype() == DType::F32
                     ? ops::rmsnorm_f32_encode(ctx, input.buffer(), weight_.buffer(), rows,
                                               hidden_size_, epsilon_)
                     : ops::rmsnorm_f16_encode(ctx, input.buffer(), weight_.buffer(), rows,
                                               hidden_size_, epsilon_);
    return Tensor::from_buffer(std::move(out), input.shape().dims(), input.dtype());
}

// src/nn/rmsnorm.rs:107-114
RmsNorm RmsNorm::to_dtype(const Context& ctx, DType dtype) const {
    return RmsNorm(weight_.to_dtype(ctx, dtype), epsilon_);
}

static Tensor table(const Context& ctx, size_t head_dim, size_t max_seq_len, float theta, bool sine) {
    const size_t half = head_dim / 2;
    std::vector<float> values;
    values.reserve(max_seq_len * half);
    for (size_t position = 0; position < max_seq_len; ++position) {
        for (size_t i = 0; i < half; ++i) {
            const float exponent = float(2 * i) / float(head_dim);
            const float inverse_frequency = 1.0f / std::pow(theta, exponent);
            const float angle = float(position) * inverse_frequency;
            values.push_back(sine ? std::sin(angle) : std::cos(angle));
        }
    }
    return Tensor::from_f32_slice(ctx, values, {max_seq_len, half});
}

// src/nn/rope.rs:20-75: tables built in float on the host, uploaded once.
RotaryEmbedding::RotaryEmbedding(const Context& ctx, size_t head_dim, size_t max_seq_len,
                                 float theta)
    : cos_(head_dim == 0 || head_dim % 2 != 0
               ? throw TinyError(TinyError::Kind::InvalidShape,
                                 "RoPE head dimension must be positive and even, got " +
                                     std::to_string(head_dim))
           : max_seq_len == 0
               ? throw TinyError(TinyError::Kind::InvalidShape,
                                 "RoPE max sequence length cannot be zero")
           : !(theta > 0.0f)
               ? throw TinyError(TinyError::Kind::InvalidShape,
                                 "RoPE theta must be positive, got " + std::to_string(theta))
               : table(ctx, head_dim, max_seq_len, theta, false)),
      sin_(table(ctx, head_dim, max_seq_len, theta, true)),
      head_dim_(head_dim),
      max_seq_len_(max_seq_len),
      theta_(theta) {}

// src/nn/rope.rs:89-130
Tensor RotaryEmbedding::forward(const Context& ctx, const Tensor& input, size_t start_pos) const {
    if (input.rank() < 2)
        throw TinyError(TinyError::Kind::InvalidDimension,
                        "RoPE expects [..., sequence, head_dim], got rank " +
                            std::to_string(input.rank()));
    const size_t seq_len = input.dim(input.rank() - 2);
    const size_t input_head_dim = input.dim(input.rank() - 1);
    if (input_head_dim != head_dim_)
        throw TinyError(TinyError::Kind::InvalidShape,
                        "RoPE expected head dimension " + std::to_string(head_dim_) + ", got " +
                            std::to_string(input_head_dim));
    if (start_pos + seq_len < start_pos)
        throw TinyError(TinyError::Kind::InvalidShape, "RoPE position overflow");
    if (start_pos + seq_len > max_seq_len_)
        throw TinyError::position_out_of_range(start_pos, seq_len, max_seq_len_);
    return ops::rope(ctx, input, cos_, sin_, start_pos);
}

// src/nn/rope.rs:132-151
Tensor RotaryEmbedding::forward_encode(const Context& ctx, const Tensor& input,
                                       size_t start_pos) const {
    return ops::rope_encode(ctx, input, cos_, sin_, start_pos);
}

// src/nn/swiglu.rs:9-13: silu then mul, synchronously, even for F16.
Tensor SwiGlu::forward(const Context& ctx, const Tensor& gate, const Tensor& up) {
    return gate.silu(ctx).mul(ctx, up);
}

// src/nn/swiglu.rs:15-37: an F16 gate with contiguous inputs of equal shape
// takes the fused kernel, whose buffer check rejects an up that is not F16
// (InvalidShape "SwiGLU requires equal F16 buffers", ops/swiglu.rs:14-19).
// Otherwise silu then mul; for two contiguous F32 tensors of equal shape
// that pair runs as one launch (swiglu_f32: silu_f32(g) * u, the same
// values as the two ops).
Tensor SwiGlu::forward_encode(const Context& ctx, const Tensor& gate, const Tensor& up) {
    const bool fusable = gate.is_contiguous() && up.is_contiguous() && gate.shape() == up.shape();
    if (gate.dtype() == DType::F16 && fusable) {
        Buffer out = ops::swiglu_f16_encode(ctx, gate.buffer(), up.buffer());
        return Tensor::from_buffer(std::move(out), gate.shape().dims(), DType::F16);
    }
    if (gate.dtype() == DType::F32 && up.dtype() == DType::F32 && fusable) {
        Buffer out = ops::swiglu_f32_encode(ctx, gate.buffer(), up.buffer());
        return Tensor::from_buffer(std::move(out), gate.shape().dims(), DType::F32);
    }
    return gate.silu_encode(ctx).mul_encode(ctx, up);
}

// src/nn/attention.rs:216-247 as one pass.  The checks of gqa_qk_matmul
// (dtype, rank 4, batch and head size, head groups), then those of
// attention_scale_mask (query range within the keys), then gqa_pv_matmul's
// (value shape).  Key and value are read in place when they are contiguous
// or the narrowed views of one LayerKvCache (same capacity); otherwise they
// are made contiguous first.
Tensor attention_core_encode(const Context& ctx, const Tensor& q, const Tensor& key,
                             const Tensor& value, float scale, size_t start_pos) {
    validate_gqa(q, key, "QK", "Q [B,QH,Q,D] and K [B,KVH,K,D]");
    const size_t batch = q.dim(0), q_heads = q.dim(1), q_len = q.dim(2), head_dim = q.dim(3);
    if (batch != key.dim(0) || head_dim != key.dim(3))
        throw shape_mismatch(q.shape().dims(), key.shape().dims());
    const size_t kv_heads = key.dim(1), kv_len = key.dim(2);
    validate_head_groups(q_heads, kv_heads);
    validate_gqa(q, value, "PV", "P [B,QH,Q,K] and V [B,KVH,K,D]");
    if (value.dim(0) != batch || value.dim(1) != kv_heads || value.dim(2) != kv_len ||
        value.dim(3) != head_dim)
        throw shape_mismatch(key.shape().dims(), value.shape().dims());
    const Tensor qc = q.is_contiguous() || one_query_in_place(q) ? q : q.contiguous_encode(ctx);
    size_t capacity = rows_in_place(key);
    Tensor k = key, v = value;
    if (capacity == 0 || rows_in_place(value) != capacity) {
        k = key.contiguous_encode(ctx);
        v = value.contiguous_encode(ctx);
        capacity = kv_len;
    }
    Tensor out = Tensor::empty(ctx, {batch, q_heads, q_len, head_dim}, q.dtype());
    check(q.dtype() == DType::F32
              ? rl_attention_f32(ctx.raw(), qc.buffer().raw(), k.buffer().raw(), v.buffer().raw(),
                                 batch, q_heads, kv_heads, q_len, kv_len, head_dim, capacity, scale,
                                 start_pos, out.buffer().raw())
              : rl_attention_f16(ctx.raw(), qc.buffer().raw(), k.buffer().raw(), v.buffer().raw(),
                                 batch, q_heads, kv_heads, q_len, kv_len, head_dim, capacity, scale,
                                 start_pos, out.buffer().raw()));
    return out;
}

}  // namespace nn
// ------------------------------------------------------------------ model

namespace model {

// LayerKvCache::new (src/model/kv_cache.rs:53-74)
LayerKvCache::LayerKvCache(const Context& ctx, size_t num_kv_heads, size_t max, size_t dim,
                           DType dtype)
    : key_(Tensor::empty(ctx, {1, num_kv_heads ? num_kv_heads : 1, max ? max : 1, dim ? dim : 1},
                         dtype)),
      value_(Tensor::empty(ctx, {1, num_kv_heads ? num_kv_heads : 1, max ? max : 1, dim ? dim : 1},
                           dtype)),
      max_seq_len_(max),
      num_kv_heads_(num_kv_heads),
      head_dim_(dim) {
    if (num_kv_heads == 0 || max == 0 || dim == 0)
        throw TinyError(TinyError::Kind::InvalidShape, "KV cache dimensions must be positive");
}

size_t LayerKvCache::storage_bytes() const {  // kv_cache.rs:86-89
    return 2 * num_kv_heads_ * max_seq_len_ * head_dim_ * size_in_bytes(dtype());
}

Tensor LayerKvCache::key() const { return key_.narrow(2, 0, len_); }
Tensor LayerKvCache::value() const { return value_.narrow(2, 0, len_); }

// kv_cache.rs:18-52
void LayerKvCache::validate_append(const Tensor& key, const Tensor& value) const {
    if (key.dtype() != key_.dtype() || value.dtype() != value_.dtype())
        throw TinyError(TinyError::Kind::UnsupportedDType,
                        std::string("KV cache dtype mismatch: cache=") + dtype_name(key_.dtype()) +
                            "/" + dtype_name(value_.dtype()) + ", input=" +
                            dtype_name(key.dtype()) + "/" + dtype_name(value.dtype()));
    if (key.shape() != value.shape() || key.rank() != 4 || key.dim(0) != 1 ||
        key.dim(1) != num_kv_heads_ || key.dim(3) != head_dim_)
        throw TinyError(TinyError::Kind::ModelFormat,
                        "KV cache write shape does not match this layer: cache has " +
                            std::to_string(num_kv_heads_) + " KV heads, input has " +
                            std::to_string(key.dim(1)) + " heads");
    const size_t seq = key.dim(2);
    if (len_ + seq < len_ || len_ + seq > max_seq_len_)
        throw TinyError::position_out_of_range(len_, seq, max_seq_len_);
}

// One tensor of append_encode (kv_cache.rs:123-137): contiguous_encode then
// kv_cache_write, or both at once for a strided view.
static void write_into(const Context& ctx, const Tensor& cache, const Tensor& src, size_t start) {
    if (src.is_contiguous()) {
        if (cache.dtype() == DType::F32)
            ops::kv_cache_write_f32_encode(ctx, cache, src, start);
        else
            ops::kv_cache_write_f16_encode(ctx, cache, src, start);
        return;
    }
    std::vector<uint64_t> d(src.shape().dims().begin(), src.shape().dims().end());
    std::vector<uint64_t> s(src.strides().values().begin(), src.strides().values().end());
    check(cache.dtype() == DType::F32
              ? rl_kv_cache_write_strided_f32(ctx.raw(), src.buffer().raw(), d.data(), s.data(),
                                              uint32_t(d.size()), cache.buffer().raw(),
                                              cache.dim(2), start)
              : rl_kv_cache_write_strided_f16(ctx.raw(), src.buffer().raw(), d.data(), s.data(),
                                              uint32_t(d.size()), cache.buffer().raw(),
                                              cache.dim(2), start));
}

void LayerKvCache::append_encode(const Context& ctx, const Tensor& key, const Tensor& value) {
    validate_append(key, value);
    const size_t start = len_, seq = key.dim(2);
    write_into(ctx, key_, key, start);
    write_into(ctx, value_, value, start);
    len_ = start + seq;
}

void LayerKvCache::append(const Context& ctx, const Tensor& key, const Tensor& value) {
    Execution exe(ctx);  // kv_cache.rs:104-111
    append_encode(ctx, key, value);
    exe.finish();
}

void LayerKvCache::append_rotated_encode(const Context& ctx, const nn::RotaryEmbedding& rope,
                                         const Tensor& key, const Tensor& value) {
    if (key.rank() == 4 && key.strides().values().back() == 1 && key.dtype() == key_.dtype()) {
        ops::validate_rope(key, rope.cos_table(), rope.sin_table(), len_);  // forward_encode first
        validate_append(key, value);
        const size_t start = len_, seq = key.dim(2);
        std::vector<uint64_t> d(key.shape().dims().begin(), key.shape().dims().end());
        std::vector<uint64_t> s(key.strides().values().begin(), key.strides().values().end());
        const Tensor& c = rope.cos_table();
        const Tensor& sn = rope.sin_table();
        check(key_.dtype() == DType::F32
                  ? rl_rope_kv_cache_write_f32(ctx.raw(), key.buffer().raw(), d.data(), s.data(),
                                               4, c.buffer().raw(), sn.buffer().raw(), c.dim(0),
                                               start, key_.buffer().raw(), max_seq_len_)
                  : rl_rope_kv_cache_write_f16(ctx.raw(), key.buffer().raw(), d.data(), s.data(),
                                               4, c.buffer().raw(), sn.buffer().raw(), c.dim(0),
                                               start, key_.buffer().raw(), max_seq_len_));
        write_into(ctx, value_, value, start);
        len_ = start + seq;
        return;
    }
    // Anything else takes the two-step path (and raises its errors).
    append_encode(ctx, rope.forward_encode(ctx, key, len_), value);
}

Tensor LayerKvCache::rotate_query_and_append_encode(const Context& ctx,
                                                    const nn::RotaryEmbedding& rope,
                                                    const Tensor& query, const Tensor& key,
                                                    const Tensor& value) {
    auto fusable = [&](const Tensor& t) {
        return t.rank() == 4 && t.strides().values().back() == 1 && t.dtype() == key_.dtype();
    };
    if (!(fusable(query) && fusable(key) && fusable(value) && query.dim(2) == key.dim(2))) {
        Tensor q = rope.forward_encode(ctx, query, len_);  // the unfused order and errors
        append_rotated_encode(ctx, rope, key, value);
        return q;
    }
    ops::validate_rope(query, rope.cos_table(), rope.sin_table(), len_);
    ops::validate_rope(key, rope.cos_table(), rope.sin_table(), len_);
    validate_append(key, value);
    const size_t start = len_, seq = key.dim(2);
    auto dims = [](const Tensor& t) {
        return std::vector<uint64_t>(t.shape().dims().begin(), t.shape().dims().end());
    };
    auto strides = [](const Tensor& t) {
        return std::vector<uint64_t>(t.strides().values().begin(), t.strides().values().end());
    };
    const auto qd = dims(query), kd = dims(key), vd = dims(value);
    const auto qs = strides(query), ks = strides(key), vs = strides(value);
    Buffer out = Buffer::empty_with_element_size(ctx, query.numel(), size_in_bytes(key_.dtype()));
    const Tensor& c = rope.cos_table();
    const Tensor& sn = rope.sin_table();
    check(key_.dtype() == DType::F32
              ? rl_qkv_rope_kv_append_f32(ctx.raw(), query.buffer().raw(), qd.data(), qs.data(),
                                          key.buffer().raw(), kd.data(), ks.data(),
                                          value.buffer().raw(), vd.data(), vs.data(),
                                          c.buffer().raw(), sn.buffer().raw(), c.dim(0), start,
                                          out.raw(), key_.buffer().raw(), value_.buffer().raw(),
                                          max_seq_len_)
              : rl_qkv_rope_kv_append_f16(ctx.raw(), query.buffer().raw(), qd.data(), qs.data(),
                                          key.buffer().raw(), kd.data(), ks.data(),
                                          value.buffer().raw(), vd.data(), vs.data(),
                                          c.buffer().raw(), sn.buffer().raw(), c.dim(0), start,
                                          out.raw(), key_.buffer().raw(), value_.buffer().raw(),
                                          max_seq_len_));
    len_ = start + seq;
    return Tensor::from_buffer(std::move(out), query.shape().dims(), key_.dtype());
}

}  // namespace model
}  // namespace rustllm
