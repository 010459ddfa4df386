// tensor_tests.cpp -- the reference's own unit tests for the hot path,
// restated in C++ against the host mirror (rustllm_amd/host/tensor.hpp) on
// the gfx950 library.  Each TEST cites the Rust test it restates; values and
// tolerances are the reference's.  Further tests cover the additive pieces
// (expand, fused RoPE gather, fused SwiGLU/softmax) against the unfused path.
//
//   tests/cpp/tensor_tests.bin [name-substring]   (exit status = failures)
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <limits>
#include <string>
#include <vector>

#include "tensor.hpp"

using namespace rustllm;

namespace {

struct Failure {
    std::string what;
};

struct Case {
    const char* name;
    void (*fn)(const Context&);
};

std::vector<Case>& registry() {
    static std::vector<Case> cases;
    return cases;
}

struct Registrar {
    Registrar(const char* name, void (*fn)(const Context&)) { registry().push_back({name, fn}); }
};

#define TEST(name)                                        \
    static void name(const Context& context);             \
    static Registrar registrar_##name(#name, name);       \
    static void name(const Context& context)

#define CHECK(cond)                                                                       \
    do {                                                                                  \
        if (!(cond))                                                                      \
            throw Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " #cond}; \
    } while (0)

template <typename Fn>
TinyError catch_error(Fn fn) {
    try {
        fn();
    } catch (const TinyError& e) {
        return e;
    }
    throw Failure{"expected a TinyError"};
}

template <typename Fn>
TinyError::Kind expect_error(Fn fn) {
    try {
        fn();
    } catch (const TinyError& e) {
        return e.kind();
    }
    throw Failure{"expected a TinyError"};
}

void assert_close(const std::vector<float>& actual, const std::vector<float>& expected,
                  float tolerance, bool strict = false) {
    CHECK(actual.size() == expected.size());
    for (size_t i = 0; i < actual.size(); ++i) {
        float error = std::fabs(actual[i] - expected[i]);
        bool ok = strict ? error < tolerance : error <= tolerance;
        if (!ok)
            throw Failure{"value " + std::to_string(i) + " differs by " + std::to_string(error) +
                          ": actual=" + std::to_string(actual[i]) +
                          " expected=" + std::to_string(expected[i])};
    }
}

std::vector<uint16_t> to_f16(const std::vector<float>& v) {
    std::vector<uint16_t> out(v.size());
    for (size_t i = 0; i < v.size(); ++i) out[i] = f16_from_f32(v[i]);
    return out;
}

const float kNegInf = -std::numeric_limits<float>::infinity();

// ---------------------------------------------------- src/tensor/tensor.rs

// tensor.rs:790-818
TEST(repeat_kv_repeats_each_kv_head_for_f32_and_f16) {
    auto input = Tensor::from_f32_slice(context, {1, 2, 3, 4, 10, 20, 30, 40}, {1, 2, 2, 2});
    std::vector<float> expected = {1,  2,  3,  4,  1,  2,  3,  4,  1,  2,  3,  4,
                                   10, 20, 30, 40, 10, 20, 30, 40, 10, 20, 30, 40};
    auto output = input.repeat_kv(context, 3);
    CHECK((output.shape().dims() == std::vector<size_t>{1, 6, 2, 2}));
    CHECK(output.to_f32_vec() == expected);
    auto output_f16 = input.to_dtype(context, DType::F16).repeat_kv(context, 3);
    CHECK(output_f16.dtype() == DType::F16);
    CHECK((output_f16.shape().dims() == std::vector<size_t>{1, 6, 2, 2}));
    CHECK(output_f16.to_f32_vec() == expected);
}

// tensor.rs:820-831
TEST(repeat_kv_with_one_returns_the_original_tensor) {
    auto input = Tensor::from_f32_slice(context, {1, 2, 3, 4}, {1, 1, 2, 2});
    auto output = input.repeat_kv(context, 1);
    CHECK(output.shape() == input.shape());
    CHECK(output.to_f32_vec() == input.to_f32_vec());
    CHECK(output.shares_storage_with(input));
}

// tensor.rs:932-949
TEST(f16_add_uses_f16_storage_and_matches_expected_values) {
    auto left = Tensor::from_f32_slice(context, {1.0, 2.0, 3.0, 4.0}, {2, 2})
                    .to_dtype(context, DType::F16);
    auto right = Tensor::from_f32_slice(context, {0.5, 1.5, -1.0, 2.0}, {2, 2})
                     .to_dtype(context, DType::F16);
    auto output = left.add(context, right);
    CHECK(output.dtype() == DType::F16);
    CHECK((output.to_f32_vec() == std::vector<float>{1.5, 3.5, 2.0, 6.0}));
}

void assert_scale_mask_close(const Tensor& expected, const Tensor& actual) {
    CHECK(actual.dtype() == DType::F16);
    auto e = expected.to_f32_vec(), a = actual.to_f32_vec();
    for (size_t i = 0; i < e.size(); ++i) {
        if (std::isinf(e[i])) {
            CHECK(std::isinf(a[i]));
            CHECK(std::signbit(e[i]) == std::signbit(a[i]));
            continue;
        }
        CHECK(std::fabs(e[i] - a[i]) < 0.01f);
    }
}

// tensor.rs:984-1004
TEST(f16_attention_scale_mask_matches_f32_prefill) {
    auto scores = Tensor::from_f32_slice(context, {1, 2, 3, 4, 5, 6, 7, 8, 9}, {1, 1, 3, 3});
    auto expected = scores.attention_scale_mask(context, 0.5f, 0);
    auto actual = scores.to_dtype(context, DType::F16).attention_scale_mask(context, 0.5f, 0);
    assert_scale_mask_close(expected, actual);
}

// tensor.rs:1006-1019
TEST(f16_attention_scale_mask_keeps_all_keys_at_decode_position) {
    auto scores =
        Tensor::from_f32_slice(context, {1, 2, 3, 4}, {1, 1, 1, 4}).to_dtype(context, DType::F16);
    auto actual = scores.attention_scale_mask(context, 0.5f, 3);
    CHECK(actual.dtype() == DType::F16);
    CHECK((actual.to_f32_vec() == std::vector<float>{0.5, 1.0, 1.5, 2.0}));
}

// tensor.rs:1021-1035
TEST(f16_attention_scale_mask_masks_future_key_at_intermediate_position) {
    auto scores =
        Tensor::from_f32_slice(context, {1, 2, 3, 4}, {1, 1, 1, 4}).to_dtype(context, DType::F16);
    auto values = scores.attention_scale_mask(context, 0.5f, 2).to_f32_vec();
    CHECK((std::vector<float>(values.begin(), values.begin() + 3) ==
           std::vector<float>{0.5, 1.0, 1.5}));
    CHECK(std::isinf(values[3]) && std::signbit(values[3]));
}

// tensor.rs:1037-1057
TEST(f16_softmax_last_dim_matches_f32_and_normalizes_each_row) {
    auto input = Tensor::from_f32_slice(context, {1, 2, 3, 4, 5, 6}, {2, 3});
    auto expected = input.softmax_last_dim(context);
    auto actual = input.to_dtype(context, DType::F16).softmax_last_dim(context);
    CHECK(actual.dtype() == DType::F16);
    assert_close(actual.to_f32_vec(), expected.to_f32_vec(), 0.01f, true);
    auto v = actual.to_f32_vec();
    for (size_t r = 0; r < 2; ++r) {
        float sum = v[3 * r] + v[3 * r + 1] + v[3 * r + 2];
        CHECK(std::fabs(sum - 1.0f) < 0.01f);
    }
}

// tensor.rs:1059-1089
TEST(f16_attention_mask_and_softmax_match_f32_and_zero_masked_probabilities) {
    auto scores = Tensor::from_f32_slice(context, {1, 2, 3, 4, 5, 6, 7, 8, 9}, {1, 1, 3, 3});
    auto expected = scores.attention_scale_mask(context, 0.5f, 0).softmax_last_dim(context);
    auto actual = scores.to_dtype(context, DType::F16)
                      .attention_scale_mask(context, 0.5f, 0)
                      .softmax_last_dim(context);
    assert_close(actual.to_f32_vec(), expected.to_f32_vec(), 0.01f, true);
    auto values = actual.to_f32_vec();
    CHECK(values[1] == 0.0f && values[2] == 0.0f && values[5] == 0.0f);
}

// --------------------------------------------------------------- src/ops

// ops/add.rs:113-168
TEST(batches_two_f16_adds_in_one_command_buffer) {
    auto a = Tensor::from_f16_slice(context, to_f16({1.0, 2.0}), {2});
    auto b = Tensor::from_f16_slice(context, to_f16({10.0, 20.0}), {2});
    auto c = Tensor::from_f16_slice(context, to_f16({100.0, 200.0}), {2});
    Execution execution(context);
    Buffer first = ops::add_f16_encode(context, a.buffer(), b.buffer());
    Buffer second = ops::add_f16_encode(context, first, c.buffer());
    // No wait has happened yet.
    execution.finish();
    auto values = Tensor::from_buffer(std::move(second), {2}, DType::F16).to_f32_vec();
    CHECK(std::fabs(values[0] - 111.0f) < 0.01f);
    CHECK(std::fabs(values[1] - 222.0f) < 0.01f);
}

// ops/mul.rs:132-203
TEST(batches_add_then_mul_in_one_command_buffer) {
    auto a = Tensor::from_f16_slice(context, to_f16({1.0, 2.0}), {2});
    auto b = Tensor::from_f16_slice(context, to_f16({10.0, 20.0}), {2});
    auto c = Tensor::from_f16_slice(context, to_f16({2.0, 3.0}), {2});
    Execution execution(context);
    Buffer added = ops::add_f16_encode(context, a.buffer(), b.buffer());
    Buffer multiplied = ops::mul_f16_encode(context, added, c.buffer());
    execution.finish();
    auto values = Tensor::from_buffer(std::move(multiplied), {2}, DType::F16).to_f32_vec();
    CHECK(std::fabs(values[0] - 22.0f) < 0.01f);
    CHECK(std::fabs(values[1] - 66.0f) < 0.01f);
}

// ops/silu.rs:122-167
TEST(batches_silu_then_mul_in_one_command_buffer) {
    auto gate = Tensor::from_f16_slice(context, to_f16({1.0, -1.0}), {2});
    auto up = Tensor::from_f16_slice(context, to_f16({2.0, 3.0}), {2});
    Execution execution(context);
    Buffer activated = ops::silu_f16_encode(context, gate.buffer());
    Buffer multiplied = ops::mul_f16_encode(context, activated, up.buffer());
    execution.finish();
    auto values = Tensor::from_buffer(std::move(multiplied), {2}, DType::F16).to_f32_vec();
    CHECK(std::fabs(values[0] - 1.4621172f) < 0.02f);
    CHECK(std::fabs(values[1] + 0.8068242f) < 0.02f);
}

// nn/swiglu.rs:15-37 with ops/swiglu.rs:14-19: an F16 gate with contiguous
// equal-shape inputs takes the fused F16 kernel, whose buffer check rejects
// an F32 up; an F32 gate falls through to silu then mul, which rejects the
// dtype pair there.
TEST(swiglu_encode_dispatch_follows_the_gate_dtype) {
    auto gate16 = Tensor::from_f16_slice(context, to_f16({1.0, -1.0}), {2});
    auto up16 = Tensor::from_f16_slice(context, to_f16({2.0, 3.0}), {2});
    auto gate32 = Tensor::from_f32_slice(context, {1.0f, -1.0f}, {2});
    auto up32 = Tensor::from_f32_slice(context, {2.0f, 3.0f}, {2});
    {
        TinyError e = catch_error([&] {
            Execution execution(context);
            nn::SwiGlu::forward_encode(context, gate16, up32);
            execution.finish();
        });
        CHECK(e.kind() == TinyError::Kind::InvalidShape);
        CHECK(std::string(e.what()).find("SwiGLU requires equal F16 buffers") != std::string::npos);
    }
    CHECK(expect_error([&] {
              Execution execution(context);
              nn::SwiGlu::forward_encode(context, gate32, up16);
              execution.finish();
          }) == TinyError::Kind::UnsupportedDType);
    Execution execution(context);
    Tensor fused = nn::SwiGlu::forward_encode(context, gate16, up16);
    Tensor fused32 = nn::SwiGlu::forward_encode(context, gate32, up32);
    execution.finish();
    CHECK(fused.dtype() == DType::F16 && fused32.dtype() == DType::F32);
    auto values = fused.to_f32_vec();
    CHECK(std::fabs(values[0] - 1.4621172f) < 0.02f);
    CHECK(std::fabs(values[1] + 0.8068242f) < 0.02f);
    auto values32 = fused32.to_f32_vec();
    CHECK(std::fabs(values32[0] - 1.4621172f) < 1e-5f);
    CHECK(std::fabs(values32[1] + 0.8068242f) < 1e-5f);
}

// ops/rmsnorm.rs:286-319: the reference test's own CPU implementation.
std::vector<float> cpu_rmsnorm(const std::vector<float>& input, const std::vector<float>& weight,
                               size_t rows, size_t hidden_size, float epsilon) {
    std::vector<float> output(input.size());
    for (size_t row = 0; row < rows; ++row) {
        float sum = 0.0f;
        for (size_t i = 0; i < hidden_size; ++i) sum += input[row * hidden_size + i] * input[row * hidden_size + i];
        float mean_square = sum / float(hidden_size);
        float inv_rms = 1.0f / std::sqrt(mean_square + epsilon);
        for (size_t c = 0; c < hidden_size; ++c)
            output[row * hidden_size + c] = input[row * hidden_size + c] * inv_rms * weight[c];
    }
    return output;
}

const std::vector<float> kRmsInput = {1.0, 2.0, 3.0, 4.0, -1.0, 0.5, -0.5, 2.0};
const std::vector<float> kRmsWeight = {1.0, 1.5, 0.5, 2.0};

// ops/rmsnorm.rs:341-386
TEST(rmsnorm_f32_matches_cpu_reference) {
    auto input = Tensor::from_f32_slice(context, kRmsInput, {2, 4});
    auto weight = Tensor::from_f32_slice(context, kRmsWeight, {4});
    auto expected = cpu_rmsnorm(kRmsInput, kRmsWeight, 2, 4, 1e-5f);
    Buffer out = ops::rmsnorm_f32(context, input.buffer(), weight.buffer(), 2, 4, 1e-5f);
    auto actual = Tensor::from_buffer(std::move(out), {2, 4}, DType::F32).to_f32_vec();
    assert_close(actual, expected, 1e-4f);
}

// ops/rmsnorm.rs:388-440
TEST(rmsnorm_f16_matches_cpu_reference) {
    auto input = Tensor::from_f16_slice(context, to_f16(kRmsInput), {2, 4});
    auto weight = Tensor::from_f16_slice(context, to_f16(kRmsWeight), {4});
    auto expected = cpu_rmsnorm(kRmsInput, kRmsWeight, 2, 4, 1e-5f);
    Buffer out = ops::rmsnorm_f16(context, input.buffer(), weight.buffer(), 2, 4, 1e-5f);
    auto output = Tensor::from_buffer(std::move(out), {2, 4}, DType::F16);
    CHECK(output.dtype() == DType::F16);
    assert_close(output.to_f32_vec(), expected, 0.02f);
}

// ops/rmsnorm.rs:442-530
TEST(batches_rmsnorm_then_add_in_one_command_buffer) {
    auto input = Tensor::from_f16_slice(context, to_f16(kRmsInput), {2, 4});
    auto weight = Tensor::from_f16_slice(context, to_f16(kRmsWeight), {4});
    auto zeros = Tensor::from_f16_slice(context, to_f16(std::vector<float>(8, 0.0f)), {2, 4});
    auto expected = cpu_rmsnorm(kRmsInput, kRmsWeight, 2, 4, 1e-5f);
    Execution execution(context);
    Buffer normalized =
        ops::rmsnorm_f16_encode(context, input.buffer(), weight.buffer(), 2, 4, 1e-5f);
    Buffer added = ops::add_f16_encode(context, normalized, zeros.buffer());
    execution.finish();
    auto actual = Tensor::from_buffer(std::move(added), {2, 4}, DType::F16).to_f32_vec();
    assert_close(actual, expected, 0.02f);
}

// ops::rmsnorm error paths (ops/rmsnorm.rs:208-246)
TEST(rmsnorm_tensor_validation_matches_reference_errors) {
    auto x = Tensor::from_f32_slice(context, kRmsInput, {2, 4});
    auto w = Tensor::from_f32_slice(context, kRmsWeight, {4});
    auto w16 = w.to_dtype(context, DType::F16);
    CHECK(expect_error([&] { ops::rmsnorm(context, x, w16, 1e-5f); }) ==
          TinyError::Kind::UnsupportedDType);
    CHECK(expect_error([&] { ops::rmsnorm(context, x, w, 0.0f); }) ==
          TinyError::Kind::InvalidShape);
    auto w3 = Tensor::from_f32_slice(context, {1, 2, 3}, {3});
    const TinyError mismatch = catch_error([&] { ops::rmsnorm(context, x, w3, 1e-5f); });
    CHECK(mismatch.kind() == TinyError::Kind::ShapeMismatch);
    CHECK((mismatch.left == std::vector<size_t>{2, 4}));  // ops/rmsnorm.rs:232-237
    CHECK((mismatch.right == std::vector<size_t>{3}));
    // F16 RMSNorm rejects a strided view (ops/rmsnorm.rs:240-246)
    auto x16t = x.to_dtype(context, DType::F16).transpose(0, 1);
    auto w16_2 = Tensor::from_f32_slice(context, {1, 1}, {2}).to_dtype(context, DType::F16);
    CHECK(expect_error([&] { ops::rmsnorm(context, x16t, w16_2, 1e-5f); }) ==
          TinyError::Kind::NonContiguousTensor);
}

// ------------------------------------------------------------- src/nn

// nn/rmsnorm.rs:153-178
TEST(f16_rmsnorm_stays_close_to_f32_and_returns_f16) {
    auto input =
        Tensor::from_f32_slice(context, {0.125, -1.25, 2.5, 3.75, -0.5, 1.5, -2.25, 4.0}, {2, 4});
    auto weight = Tensor::from_f32_slice(context, {1.0, 0.5, 1.25, 0.75}, {4});
    nn::RmsNorm norm(weight, 1e-5f);
    auto output_f32 = norm.forward(context, input).to_f32_vec();
    auto norm_f16 = norm.to_dtype(context, DType::F16);
    auto output_f16 = norm_f16.forward(context, input.to_dtype(context, DType::F16));
    CHECK(norm_f16.dtype() == DType::F16);
    CHECK(output_f16.dtype() == DType::F16);
    assert_close(output_f16.to_f32_vec(), output_f32, 0.01f);
}

// nn/rope.rs:186-208
TEST(f16_rope_stays_close_to_f32_and_returns_f16) {
    nn::RotaryEmbedding rope(context, 4, 8, 10000.0f);
    auto input = Tensor::from_f32_slice(context, {0.125, -1.25, 2.5, 3.75, -0.5, 1.5, -2.25, 4.0},
                                        {1, 1, 2, 4});
    auto output_f32 = rope.forward(context, input, 1).to_f32_vec();
    auto output_f16 = rope.forward(context, input.to_dtype(context, DType::F16), 1);
    CHECK(output_f16.dtype() == DType::F16);
    assert_close(output_f16.to_f32_vec(), output_f32, 0.01f);
}

// nn/rope.rs:211-233
TEST(f16_rope_materializes_non_contiguous_input) {
    nn::RotaryEmbedding rope(context, 4, 8, 10000.0f);
    auto input = Tensor::from_f32_slice(context, {1, 2, 3, 4, 5, 6, 7, 8}, {1, 2, 1, 4})
                     .to_dtype(context, DType::F16)
                     .permute({0, 2, 1, 3});
    CHECK(!input.is_contiguous());
    auto output = rope.forward(context, input, 0);
    CHECK(output.dtype() == DType::F16);
    CHECK(output.is_contiguous());
    // and it equals rotating the materialised copy
    auto reference = rope.forward(context, input.contiguous(context), 0);
    CHECK(output.to_f32_vec() == reference.to_f32_vec());
}

// RotaryEmbedding::forward position check (nn/rope.rs:117-127)
TEST(rope_rejects_positions_past_the_table) {
    nn::RotaryEmbedding rope(context, 4, 8, 10000.0f);
    auto input = Tensor::from_f32_slice(context, std::vector<float>(8, 1.0f), {1, 1, 2, 4});
    CHECK(expect_error([&] { rope.forward(context, input, 7); }) ==
          TinyError::Kind::PositionOutOfRange);
    auto wrong = Tensor::from_f32_slice(context, std::vector<float>(12, 1.0f), {1, 1, 2, 6});
    CHECK(expect_error([&] { rope.forward(context, wrong, 0); }) == TinyError::Kind::InvalidShape);
    CHECK(expect_error([&] { nn::RotaryEmbedding(context, 3, 8, 10000.0f); }) ==
          TinyError::Kind::InvalidShape);
}

// model/kv_cache.rs:213-258: a narrowed cache view keeps the parent strides
// and materialises in sequence order.
TEST(f16_cache_narrow_view_materialises_in_order) {
    std::vector<float> cache(1 * 2 * 8 * 4, 0.0f);
    const float appended[2][8] = {{1, 2, 3, 4, 5, 6, 7, 8}, {9, 10, 11, 12, 13, 14, 15, 16}};
    for (int pos = 0; pos < 2; ++pos)
        for (int head = 0; head < 2; ++head)
            for (int d = 0; d < 4; ++d) cache[(head * 8 + pos) * 4 + d] = appended[pos][head * 4 + d];
    auto key = Tensor::from_f32_slice(context, cache, {1, 2, 8, 4}).to_dtype(context, DType::F16);
    auto view = key.narrow(2, 0, 2);
    CHECK((view.shape().dims() == std::vector<size_t>{1, 2, 2, 4}));
    CHECK(!view.is_contiguous());
    CHECK((view.contiguous(context).to_f32_vec() ==
           std::vector<float>{1, 2, 3, 4, 9, 10, 11, 12, 5, 6, 7, 8, 13, 14, 15, 16}));
}

// ------------------------------------------------- src/model/kv_cache.rs

Tensor f16_tensor(const Context& context, const std::vector<float>& data,
                  const std::vector<size_t>& dims) {
    return Tensor::from_f32_slice(context, data, dims).to_dtype(context, DType::F16);
}

// kv_cache.rs:213-258
TEST(f16_cache_appends_decode_tokens_and_returns_f16_prefix) {
    model::LayerKvCache cache(context, 2, 8, 4, DType::F16);
    CHECK(cache.dtype() == DType::F16);
    CHECK(cache.len() == 0);
    cache.append(context, f16_tensor(context, {1, 2, 3, 4, 5, 6, 7, 8}, {1, 2, 1, 4}),
                 f16_tensor(context, {10, 20, 30, 40, 50, 60, 70, 80}, {1, 2, 1, 4}));
    cache.append(context, f16_tensor(context, {9, 10, 11, 12, 13, 14, 15, 16}, {1, 2, 1, 4}),
                 f16_tensor(context, {90, 100, 110, 120, 130, 140, 150, 160}, {1, 2, 1, 4}));
    CHECK(cache.len() == 2);
    auto cached_key = cache.key();
    auto cached_value = cache.value();
    CHECK((cached_key.shape().dims() == std::vector<size_t>{1, 2, 2, 4}));
    CHECK(cached_key.dtype() == DType::F16);
    CHECK(cached_value.dtype() == DType::F16);
    CHECK((cached_key.contiguous(context).to_f32_vec() ==
           std::vector<float>{1, 2, 3, 4, 9, 10, 11, 12, 5, 6, 7, 8, 13, 14, 15, 16}));
    CHECK((cached_value.contiguous(context).to_f32_vec() ==
           std::vector<float>{10, 20, 30, 40, 90, 100, 110, 120, 50, 60, 70, 80, 130, 140, 150,
                              160}));
}

// kv_cache.rs:260-273
TEST(f16_cache_appends_prefill_sequence) {
    model::LayerKvCache cache(context, 2, 8, 4, DType::F16);
    cache.append(context, f16_tensor(context, std::vector<float>(24, 1.0f), {1, 2, 3, 4}),
                 f16_tensor(context, std::vector<float>(24, 2.0f), {1, 2, 3, 4}));
    CHECK(cache.len() == 3);
    CHECK((cache.key().shape().dims() == std::vector<size_t>{1, 2, 3, 4}));
}

// kv_cache.rs:275-295
TEST(append_encode_updates_the_logical_prefix_after_submission) {
    model::LayerKvCache cache(context, 2, 8, 2, DType::F16);
    auto key = f16_tensor(context, std::vector<float>(4, 1.0f), {1, 2, 1, 2});
    auto value = f16_tensor(context, std::vector<float>(4, 2.0f), {1, 2, 1, 2});
    Execution execution(context);
    cache.append_encode(context, key, value);
    execution.finish();
    CHECK(cache.len() == 1);
    CHECK((cache.key().shape().dims() == std::vector<size_t>{1, 2, 1, 2}));
    CHECK((cache.value().shape().dims() == std::vector<size_t>{1, 2, 1, 2}));
}

// kv_cache.rs:297-309
TEST(f16_cache_rejects_f32_inputs_without_casting) {
    model::LayerKvCache cache(context, 2, 8, 4, DType::F16);
    auto key = Tensor::from_f32_slice(context, std::vector<float>(8, 1.0f), {1, 2, 1, 4});
    auto value = Tensor::from_f32_slice(context, std::vector<float>(8, 2.0f), {1, 2, 1, 4});
    CHECK(expect_error([&] { cache.append(context, key, value); }) ==
          TinyError::Kind::UnsupportedDType);
    CHECK(cache.len() == 0);
}

// kv_cache.rs:31-50: wrong head count, then a write past max_seq_len.
TEST(cache_rejects_foreign_shapes_and_overflow) {
    model::LayerKvCache cache(context, 2, 4, 4, DType::F32);
    auto three_heads = Tensor::from_f32_slice(context, std::vector<float>(12, 1.0f), {1, 3, 1, 4});
    CHECK(expect_error([&] { cache.append(context, three_heads, three_heads); }) ==
          TinyError::Kind::ModelFormat);
    auto five = Tensor::from_f32_slice(context, std::vector<float>(40, 1.0f), {1, 2, 5, 4});
    CHECK(expect_error([&] { cache.append(context, five, five); }) ==
          TinyError::Kind::PositionOutOfRange);
    CHECK(expect_error([&] { model::LayerKvCache(context, 0, 4, 4, DType::F32); }) ==
          TinyError::Kind::InvalidShape);
    CHECK(cache.storage_bytes() == 2 * 2 * 4 * 4 * 4);
}

// The attention path (nn/attention.rs:196-207, 306-307): K and V come as
// [1, H, S, D] permutes of the [1, S, H*D] projections; K is rotated at the
// cache's length.  Appending the views (gather + write in one pass) and the
// rotated key (rotation + write in one pass) equals contiguous -> rope ->
// append of the materialised tensors, bit for bit.
TEST(fused_append_of_projection_views_equals_the_unfused_path) {
    const size_t seq = 3, heads = 2, hd = 8, max = 8;
    nn::RotaryEmbedding rope(context, hd, max, 10000.0f);
    std::vector<float> kd(seq * heads * hd), vd(seq * heads * hd);
    for (size_t i = 0; i < kd.size(); ++i) {
        kd[i] = std::sin(0.37f * float(i)) * 3.0f;
        vd[i] = std::cos(0.11f * float(i)) * 2.0f;
    }
    for (DType dtype : {DType::F32, DType::F16}) {
        auto k = Tensor::from_f32_slice(context, kd, {1, seq, heads, hd}).to_dtype(context, dtype);
        auto v = Tensor::from_f32_slice(context, vd, {1, seq, heads, hd}).to_dtype(context, dtype);
        auto k_view = k.permute({0, 2, 1, 3});
        auto v_view = v.permute({0, 2, 1, 3});
        CHECK(!k_view.is_contiguous());
        model::LayerKvCache fused(context, heads, max, hd, dtype);
        model::LayerKvCache plain(context, heads, max, hd, dtype);
        for (size_t round = 0; round < 2; ++round) {  // second append at start = 3
            Execution a(context);
            fused.append_rotated_encode(context, rope, k_view, v_view);
            a.finish();
            Execution b(context);
            auto k_rot = rope.forward_encode(context, k_view.contiguous_encode(context),
                                             plain.len());
            plain.append_encode(context, k_rot, v_view.contiguous_encode(context));
            b.finish();
        }
        CHECK(fused.len() == 2 * seq && plain.len() == 2 * seq);
        CHECK(fused.key().contiguous(context).to_f32_vec() ==
              plain.key().contiguous(context).to_f32_vec());
        CHECK(fused.value().contiguous(context).to_f32_vec() ==
              plain.value().contiguous(context).to_f32_vec());
    }
}

// The same with Q: its rotation and the K/V append in one launch equals
// rope(Q), rope(K), append of the materialised tensors.
TEST(one_launch_query_rotation_and_append_equals_the_unfused_path) {
    const size_t seq = 3, qheads = 4, heads = 2, hd = 8, max = 8;
    nn::RotaryEmbedding rope(context, hd, max, 10000.0f);
    std::vector<float> qd(seq * qheads * hd), kd(seq * heads * hd), vd(seq * heads * hd);
    for (size_t i = 0; i < qd.size(); ++i) qd[i] = std::cos(0.23f * float(i)) * 2.5f;
    for (size_t i = 0; i < kd.size(); ++i) {
        kd[i] = std::sin(0.37f * float(i)) * 3.0f;
        vd[i] = std::cos(0.11f * float(i)) * 2.0f;
    }
    for (DType dtype : {DType::F32, DType::F16}) {
        auto q = Tensor::from_f32_slice(context, qd, {1, seq, qheads, hd}).to_dtype(context, dtype)
                     .permute({0, 2, 1, 3});
        auto k = Tensor::from_f32_slice(context, kd, {1, seq, heads, hd}).to_dtype(context, dtype)
                     .permute({0, 2, 1, 3});
        auto v = Tensor::from_f32_slice(context, vd, {1, seq, heads, hd}).to_dtype(context, dtype)
                     .permute({0, 2, 1, 3});
        model::LayerKvCache fused(context, heads, max, hd, dtype);
        model::LayerKvCache plain(context, heads, max, hd, dtype);
        for (size_t round = 0; round < 2; ++round) {
            Execution a(context);
            auto q_fused = fused.rotate_query_and_append_encode(context, rope, q, k, v);
            a.finish();
            Execution b(context);
            auto q_plain = rope.forward_encode(context, q, plain.len());
            auto k_rot = rope.forward_encode(context, k, plain.len());
            plain.append_encode(context, k_rot, v);
            b.finish();
            CHECK(q_fused.is_contiguous());
            CHECK(q_fused.to_f32_vec() == q_plain.to_f32_vec());
        }
        CHECK(fused.len() == 2 * seq);
        CHECK(fused.key().contiguous(context).to_f32_vec() ==
              plain.key().contiguous(context).to_f32_vec());
        CHECK(fused.value().contiguous(context).to_f32_vec() ==
              plain.value().contiguous(context).to_f32_vec());
    }
}

// ---------------------------------------------------- src/nn/attention.rs

// nn/attention.rs:590-668 (batched_attention_core_matches_op_by_op_submission):
// the attention core in one pass equals QK^T, scale/mask, softmax and PV
// issued one by one, within 1e-5, for (2, 2) and (3, 1) heads, head size 4,
// 3 new positions after 2 cached.  (For equal head counts the reference's
// op-by-op side uses batched_matmul over K^T; gqa_qk_matmul with one query
// head per KV head computes the same sums.)
TEST(batched_attention_core_matches_op_by_op_submission) {
    for (auto heads : {std::pair<size_t, size_t>{2, 2}, {3, 1}}) {
        const size_t num_heads = heads.first, num_kv_heads = heads.second;
        const size_t head_dim = 4, seq_len = 3, start_pos = 2;
        std::vector<float> query(num_heads * seq_len * head_dim);
        for (size_t i = 0; i < query.size(); ++i) query[i] = std::fmod(float(i), 5.0f) - 2.0f;
        std::vector<float> cached(num_kv_heads * (start_pos + seq_len) * head_dim);
        for (size_t i = 0; i < cached.size(); ++i) cached[i] = std::fmod(float(i), 3.0f) - 1.0f;
        auto q = Tensor::from_f32_slice(context, query, {1, num_heads, seq_len, head_dim});
        auto key = Tensor::from_f32_slice(context, cached,
                                          {1, num_kv_heads, start_pos + seq_len, head_dim});
        auto value = key;
        const float scale = 1.0f / std::sqrt(float(head_dim));
        auto scores = q.gqa_qk_matmul(context, key);
        scores = scores.attention_scale_mask(context, scale, start_pos);
        auto probabilities = scores.softmax_last_dim(context);
        auto expected = probabilities.gqa_pv_matmul(context, value);

        Execution execution(context);
        auto actual = nn::attention_core_encode(context, q, key, value, scale, start_pos);
        execution.finish();
        CHECK(actual.shape() == expected.shape());
        assert_close(actual.to_f32_vec(), expected.to_f32_vec(), 1e-5f, true);
    }
}

// gqa_matmul.rs:31-42 and :79-83: a decode step reads the narrowed KV-cache
// views in place; the result equals the same step on contiguous copies.
TEST(decode_attention_reads_cache_views_in_place) {
    const size_t q_heads = 6, kv_heads = 2, hd = 64, max = 1024, len = 700;
    for (DType dtype : {DType::F32, DType::F16}) {
        model::LayerKvCache cache(context, kv_heads, max, hd, dtype);
        std::vector<float> kd(len * kv_heads * hd), vd(len * kv_heads * hd), qd(q_heads * hd);
        for (size_t i = 0; i < kd.size(); ++i) {
            kd[i] = std::sin(0.013f * float(i)) * 2.0f;
            vd[i] = std::cos(0.007f * float(i));
        }
        for (size_t i = 0; i < qd.size(); ++i) qd[i] = std::cos(0.31f * float(i));
        auto k = Tensor::from_f32_slice(context, kd, {1, kv_heads, len, hd}).to_dtype(context, dtype);
        auto v = Tensor::from_f32_slice(context, vd, {1, kv_heads, len, hd}).to_dtype(context, dtype);
        cache.append(context, k, v);
        auto q = Tensor::from_f32_slice(context, qd, {1, q_heads, 1, hd}).to_dtype(context, dtype);
        CHECK(!cache.key().is_contiguous());
        Execution a(context);
        auto in_place = nn::attention_core_encode(context, q, cache.key(), cache.value(), 0.125f,
                                                  len - 1);
        auto scores = q.gqa_qk_matmul_encode(context, cache.key());
        a.finish();
        Execution b(context);
        auto copied = nn::attention_core_encode(context, q, cache.key().contiguous_encode(context),
                                                cache.value().contiguous_encode(context), 0.125f,
                                                len - 1);
        auto scores_copied = q.gqa_qk_matmul_encode(context, k);
        b.finish();
        assert_close(in_place.to_f32_vec(), copied.to_f32_vec(), 0.0f);
        assert_close(scores.to_f32_vec(), scores_copied.to_f32_vec(), 0.0f);
    }
}

// gqa_matmul.rs:135-182: dtype, rank, batch/head size, head groups -- in that order.
TEST(gqa_matmuls_validate_like_the_reference) {
    auto q = Tensor::zeros(context, {1, 6, 3, 8});
    auto k = Tensor::zeros(context, {1, 2, 5, 8});
    CHECK(expect_error([&] { q.gqa_qk_matmul(context, k.to_dtype(context, DType::F16)); }) ==
          TinyError::Kind::UnsupportedDType);
    CHECK(expect_error([&] { q.gqa_qk_matmul(context, Tensor::zeros(context, {2, 5, 8})); }) ==
          TinyError::Kind::ModelFormat);
    CHECK(expect_error([&] { q.gqa_qk_matmul(context, Tensor::zeros(context, {2, 2, 5, 8})); }) ==
          TinyError::Kind::ShapeMismatch);
    CHECK(expect_error([&] { q.gqa_qk_matmul(context, Tensor::zeros(context, {1, 4, 5, 8})); }) ==
          TinyError::Kind::ModelFormat);
    auto p = Tensor::zeros(context, {1, 6, 3, 5});
    CHECK(expect_error([&] { p.gqa_pv_matmul(context, Tensor::zeros(context, {1, 2, 4, 8})); }) ==
          TinyError::Kind::ShapeMismatch);
    CHECK((q.gqa_qk_matmul(context, k).shape().dims() == std::vector<size_t>{1, 6, 3, 5}));
    CHECK((p.gqa_pv_matmul(context, k).shape().dims() == std::vector<size_t>{1, 6, 3, 8}));
    // the attention core's own scale/mask check: queries past the keys
    CHECK(expect_error([&] { nn::attention_core_encode(context, q, k, k, 0.5f, 3); }) ==
          TinyError::Kind::InvalidShape);
}

// ---------------------------------------------------- src/ops/embedding.rs

// ops/embedding.rs:119-149: rows of the weight, token ids checked against the vocabulary.
TEST(embedding_gathers_rows_and_rejects_bad_ids) {
    const size_t vocab = 5, hidden = 3;
    std::vector<float> w(vocab * hidden);
    for (size_t i = 0; i < w.size(); ++i) w[i] = float(i) * 0.5f;
    auto weight = Buffer::from_slice(context, w);
    auto out = ops::embedding_f32(context, weight, {4, 0, 4, 2}, vocab, hidden);
    std::vector<float> expected;
    for (uint32_t id : {4u, 0u, 4u, 2u})
        for (size_t h = 0; h < hidden; ++h) expected.push_back(w[id * hidden + h]);
    CHECK(out.as_slice() == expected);
    auto weight16 = Buffer::from_f16_slice(context, to_f16(w));
    auto out16 = ops::embedding_f16(context, weight16, {1, 3}, vocab, hidden);
    CHECK((out16.as_f16_slice() ==
           std::vector<uint16_t>{to_f16(w)[3], to_f16(w)[4], to_f16(w)[5], to_f16(w)[9],
                                 to_f16(w)[10], to_f16(w)[11]}));
    // raised by the library (ops/embedding.rs:129-136), payload carried across the ABI
    const TinyError bad_id =
        catch_error([&] { ops::embedding_f32(context, weight, {1, 7}, vocab, hidden); });
    CHECK(bad_id.kind() == TinyError::Kind::InvalidTokenId);
    CHECK(bad_id.token_id == 7 && bad_id.vocab_size == vocab);
    CHECK(expect_error([&] { ops::embedding_f32(context, weight, {}, vocab, hidden); }) ==
          TinyError::Kind::InvalidShape);
    CHECK(expect_error([&] { ops::embedding_f32(context, weight, {1}, vocab, hidden + 1); }) ==
          TinyError::Kind::InvalidShape);
}

// Submission counters (nn/attention.rs:562-588 style): a batch of encoded
// ops is one command buffer, one commit and one wait.
TEST(one_execution_is_one_submission) {
    auto x = Tensor::from_f32_slice(context, kRmsInput, {2, 4});
    nn::RmsNorm norm(Tensor::from_f32_slice(context, kRmsWeight, {4}), 1e-5f);
    context.raw();
    Context ctx = context;
    ctx.begin_decode_submission_profile();
    Execution execution(ctx);
    auto normed = norm.forward_encode(ctx, x);
    auto sum = x.add_encode(ctx, normed);
    auto act = nn::SwiGlu::forward_encode(ctx, sum, x);
    execution.finish();
    auto profile = ctx.take_decode_submission_profile();
    CHECK(profile.has_value());
    CHECK(profile->command_buffers == 1 && profile->commits == 1 && profile->waits == 1);
    CHECK(profile->kernel_dispatches == 3);
    CHECK(ctx.dispatches("swiglu_f32") == 1);
    CHECK(!ctx.take_decode_submission_profile().has_value());
    (void)act;
}

// ------------------------------------------------- views and additive API

TEST(views_follow_reference_rules) {
    auto t = Tensor::from_f32_slice(context, {1, 2, 3, 4, 5, 6}, {2, 3});
    CHECK(expect_error([&] { t.transpose(0, 2); }) == TinyError::Kind::InvalidDimension);
    CHECK(expect_error([&] { t.permute({0, 0}); }) == TinyError::Kind::InvalidDimension);
    CHECK(expect_error([&] { t.transpose(0, 1).reshape({6}); }) == TinyError::Kind::InvalidShape);
    CHECK(expect_error([&] { t.narrow(1, 1, 2); }) == TinyError::Kind::InvalidDimension);
    CHECK(expect_error([&] { t.narrow(1, 0, 4); }) == TinyError::Kind::InvalidDimension);
    CHECK(expect_error([&] { Tensor::from_f32_slice(context, {1, 2}, {3}); }) ==
          TinyError::Kind::InvalidShape);
    CHECK(expect_error([&] { Shape::create({}); }) == TinyError::Kind::InvalidShape);
    CHECK(expect_error([&] { t.transpose(0, 1).to_f32_vec(); }) ==
          TinyError::Kind::NonContiguousTensor);
    // strict stride equality even on size-1 dims (tensor.rs:251-253)
    auto one = Tensor::from_f32_slice(context, {1, 2, 3}, {1, 3});
    CHECK(!one.transpose(0, 1).is_contiguous());  // strides [1, 3] vs contiguous [1, 1]
    CHECK((t.transpose(0, 1).contiguous(context).to_f32_vec() ==
           std::vector<float>{1, 4, 2, 5, 3, 6}));
}

TEST(expand_broadcast_add_equals_materialised_add) {
    std::vector<float> xs(6 * 8), bs(8);
    for (size_t i = 0; i < xs.size(); ++i) xs[i] = float(i) * 0.25f - 3.0f;
    for (size_t i = 0; i < bs.size(); ++i) bs[i] = float(i) - 2.5f;
    for (DType dt : {DType::F32, DType::F16}) {
        auto x = Tensor::from_f32_slice(context, xs, {6, 8}).to_dtype(context, dt);
        auto bias = Tensor::from_f32_slice(context, bs, {8}).to_dtype(context, dt);
        auto view = bias.expand({6, 8});
        CHECK(!view.is_contiguous());
        auto fused = x.add(context, view);
        auto materialised = x.add(context, view.contiguous(context));
        CHECK(fused.to_f32_vec() == materialised.to_f32_vec());
    }
    auto bias = Tensor::from_f32_slice(context, bs, {8});
    CHECK(expect_error([&] { bias.expand({6, 4}); }) == TinyError::Kind::InvalidShape);
}

TEST(fused_swiglu_f32_is_bit_identical_to_silu_then_mul) {
    std::vector<float> g(1000), u(1000);
    for (size_t i = 0; i < g.size(); ++i) {
        g[i] = std::sin(float(i)) * 6.0f;
        u[i] = std::cos(float(i) * 0.37f) * 2.0f;
    }
    auto gate = Tensor::from_f32_slice(context, g, {10, 100});
    auto up = Tensor::from_f32_slice(context, u, {10, 100});
    Execution execution(context);
    auto fused = nn::SwiGlu::forward_encode(context, gate, up);
    execution.finish();
    auto unfused = nn::SwiGlu::forward(context, gate, up);
    CHECK(fused.to_f32_vec() == unfused.to_f32_vec());
}

TEST(fused_attention_softmax_equals_the_two_op_composition) {
    std::vector<float> s(2 * 5 * 12);
    for (size_t i = 0; i < s.size(); ++i) s[i] = std::sin(float(i) * 1.3f) * 8.0f;
    for (DType dt : {DType::F32, DType::F16}) {
        auto scores = Tensor::from_f32_slice(context, s, {2, 5, 12}).to_dtype(context, dt);
        Execution execution(context);
        auto fused = scores.attention_softmax_encode(context, 0.125f, 7);
        auto pair = scores.attention_scale_mask_encode(context, 0.125f, 7)
                        .softmax_last_dim_encode(context);
        execution.finish();
        auto a = fused.to_f32_vec(), b = pair.to_f32_vec();
        for (size_t i = 0; i < a.size(); ++i) {
            if (b[i] == 0.0f) CHECK(a[i] == 0.0f);
            CHECK(std::fabs(a[i] - b[i]) <= (dt == DType::F16 ? 2e-3f : 1e-6f) * std::fabs(b[i]) + 1e-12f);
        }
    }
}

TEST(fused_add_rmsnorm_equals_add_then_rmsnorm) {
    std::vector<float> xs(4 * 64), rs(4 * 64), ws(64);
    for (size_t i = 0; i < xs.size(); ++i) {
        xs[i] = std::sin(float(i));
        rs[i] = std::cos(float(i) * 0.5f);
    }
    for (size_t i = 0; i < ws.size(); ++i) ws[i] = 0.5f + float(i) / 64.0f;
    auto x = Tensor::from_f32_slice(context, xs, {4, 64});
    auto r = Tensor::from_f32_slice(context, rs, {4, 64});
    nn::RmsNorm norm(Tensor::from_f32_slice(context, ws, {64}), 1e-5f);
    Execution execution(context);
    auto fused = ops::add_rmsnorm_encode(context, x, r, norm.weight(), 1e-5f);
    auto sum = x.add_encode(context, r);
    auto normed = norm.forward_encode(context, sum);
    execution.finish();
    CHECK(fused.first.to_f32_vec() == sum.to_f32_vec());
    auto a = fused.second.to_f32_vec(), b = normed.to_f32_vec();
    CHECK(a == b);  // same kernel arithmetic on the same sum
}

TEST(host_f16_conversion_round_trips_every_half) {
    (void)context;
    for (uint32_t bits = 0; bits < 65536; ++bits) {
        float f = f16_to_f32(uint16_t(bits));
        if (std::isnan(f)) continue;
        CHECK(f16_from_f32(f) == uint16_t(bits));
    }
    CHECK(f16_from_f32(65520.0f) == 0x7c00);
    CHECK(f16_from_f32(65519.0f) == 0x7bff);
    CHECK(f16_from_f32(std::ldexp(1.0f, -25)) == 0x0000);
    CHECK(f16_from_f32(std::ldexp(1.5f, -25)) == 0x0001);
}

}  // namespace

int main(int argc, char** argv) {
    const char* filter = argc > 1 ? argv[1] : nullptr;
    Context context = Context::create(0);
    int failures = 0, passed = 0;
    for (const Case& c : registry()) {
        if (filter && !std::strstr(c.name, filter)) continue;
        std::printf("RUN  %s\n", c.name);
        std::fflush(stdout);
        try {
            c.fn(context);
            ++passed;
            std::printf("PASS %s\n", c.name);
        } catch (const Failure& f) {
            ++failures;
            std::printf("FAIL %s: %s\n", c.name, f.what.c_str());
        } catch (const std::exception& e) {
            ++failures;
            std::printf("FAIL %s: exception %s\n", c.name, e.what());
        }
        std::fflush(stdout);
    }
    std::printf("%d passed, %d failed\n", passed, failures);
    return failures == 0 ? 0 : 1;
}
